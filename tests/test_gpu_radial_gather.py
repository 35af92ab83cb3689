"""fu_radial_gather_fwd (the radial output layer with the gather-rotate forward in its epilogue)
against the two kernels it replaces, fu_linear_resident with the unpermuted weight followed by
fu_gather_fwd: rad and X_m0, X_m1, X_m2 bitwise equal, for both column layouts, ragged edge
counts, a row-strided h2, and panels that take the two-loop pass of split_f16.h."""
import pytest
import torch

pytestmark = pytest.mark.gpu


def _inputs(cuda, E, N, seed, ramp=None):
    g = torch.Generator().manual_seed(seed)
    C, K = 128, 128
    wide = torch.randn(E, 5 * K, generator=g, dtype=torch.float64)
    W3 = torch.randn(12 * C, K, generator=g, dtype=torch.float64) / K ** 0.5
    if ramp is not None:   # x ~ 2^t, w ~ 2^-t along K: spreads of 2^(2T) take the two-loop pass
        t = torch.linspace(-ramp, ramp, K, dtype=torch.float64)
        wide[:, 2 * K:3 * K] *= torch.exp2(t)
        W3 *= torch.exp2(-t)
    h2 = wide.float().to(cuda)[:, 2 * K:3 * K]   # a row-strided view, as the trunk's slices
    b3 = torch.randn(12 * C, generator=g).to(cuda)
    x = torch.randn(N, 9, C, generator=g).to(cuda)
    idx_i = torch.randint(0, N, (E,), generator=g).to(cuda)
    idx_j = torch.sort(torch.randint(0, N, (E,), generator=g)).values.to(cuda)
    wig = torch.randn(E, 34, generator=g).to(cuda)
    csd = torch.randn(3, C, generator=g).to(cuda)
    batch = torch.randint(0, 3, (N,), generator=g).to(cuda)
    return h2, W3.float().to(cuda), b3, x, idx_i, idx_j, wig, csd, batch


def _both(h2, W3, b3, x, idx_i, idx_j, wig, csd, batch, layout):
    from ops import gather, linear
    rad_ref = linear.gemm_resident(h2, linear.linear_weight_split(W3), W3.shape[0], b3)
    X_ref = gather.gather_fwd(x, idx_i, idx_j, wig, rad_ref, csd, batch, layout)
    perm = gather.radial_gather_perm(128, layout).to(W3.device)
    W2p = linear.linear_weight_split(W3[perm].contiguous())
    got = gather.radial_gather_fwd(h2, W2p, b3[perm].contiguous(), x, idx_i, idx_j, wig, csd, batch, layout)
    return (rad_ref, *X_ref), got


def _assert_equal(ref, got):
    for name, a, b in zip(("rad", "X_m0", "X_m1", "X_m2"), ref, got):
        assert a.shape == b.shape, name
        n_diff = (a != b).sum().item()
        assert n_diff == 0, f"{name}: {n_diff} elements differ, max abs {(a - b).abs().max().item():.3e}"


@pytest.mark.parametrize("layout", [0, 1])
@pytest.mark.parametrize("E,N", [(70000, 2400), (3001, 200), (128, 7), (1, 1)])
def test_radial_gather_bitwise(cuda, layout, E, N):
    ops = _inputs(cuda, E, N, seed=E + N + layout)
    _assert_equal(*_both(*ops, layout))


@pytest.mark.parametrize("T", [8, 12])
def test_radial_gather_two_loop_pass(cuda, T):
    ops = _inputs(cuda, 5000, 300, seed=T, ramp=T)
    ref, got = _both(*ops, 1)
    assert torch.isfinite(got[0]).all()
    _assert_equal(ref, got)


def test_radial_gather_argument_checks(cuda):
    from ops import _lib
    args = lambda C, K, layout: (None, 128, *([None] * 12), 10, 4, 1, C, K, layout, None)
    with pytest.raises(_lib.FlashUMAError, match="C=64"):
        _lib.call("fu_radial_gather_fwd", *args(64, 128, 0))
    with pytest.raises(_lib.FlashUMAError, match="K=64"):
        _lib.call("fu_radial_gather_fwd", *args(128, 64, 0))
    with pytest.raises(_lib.FlashUMAError, match="layout=2"):
        _lib.call("fu_radial_gather_fwd", *args(128, 128, 2))
    with pytest.raises(_lib.FlashUMAError, match="NULL"):
        _lib.call("fu_radial_gather_fwd", *args(128, 128, 1))


def test_model_radial_gather_matches_two_kernels(cuda, monkeypatch):
    """The model with its blocks' radial output layers fused with the gather (RADIAL_GATHER,
    the default) against the output GEMM and the gather as two kernels, on a bcc Fe cell
    (4,096 atoms, 122,880 edges): energy, forces and stress bit for bit equal, the fused kernel
    called once per block and the gather kernel not at all."""
    import escn_md
    import heads
    import systems
    from ops import _lib
    from wrapper import ZeroAllocBackbone
    bb = escn_md.eSCNMDBackbone(seed=0, num_layers=2)
    hd = heads.MLPEnergyHead(bb.sphere_channels, bb.hidden_channels, seed=1)
    model = heads.PotentialModel(ZeroAllocBackbone(bb.to(cuda)), hd.to(cuda))
    s = systems.bcc_fe(n_rep=8)
    ei, off = systems.neighbor_list(s.pos, s.cell, s.pbc, 6.0, 30)
    data = heads.make_atomic_data(s, ei, off, cuda)
    ce = model.backbone.ce
    real = _lib.call
    outs = {}
    for fused in (False, True):
        calls = []

        def spy(name, *args):
            calls.append(name)
            return real(name, *args)

        monkeypatch.setattr(ce, "RADIAL_GATHER", fused)
        monkeypatch.setattr(_lib, "call", spy)
        out = model(data, compute_forces=True, compute_stress=True)
        torch.cuda.synchronize()
        monkeypatch.setattr(_lib, "call", real)
        outs[fused] = {k: v.detach().cpu() for k, v in out.items() if torch.is_tensor(v)}
        assert calls.count("fu_radial_gather_fwd") == (2 if fused else 0)
        assert calls.count("fu_gather_fwd") == (0 if fused else 2)
    for k in ("energy", "forces", "stress"):
        assert torch.equal(outs[False][k], outs[True][k]), k


def _lmax_inputs(cuda, E, N, L, seed):
    from ops.lmax import ext_width
    g = torch.Generator().manual_seed(seed)
    C, K = 128, 128
    wide = torch.randn(E, 5 * K, generator=g)
    h2 = wide.to(cuda)[:, K:2 * K]
    W3 = (torch.randn(6 * L * C, K, generator=g) / K ** 0.5).to(cuda)
    b3 = torch.randn(6 * L * C, generator=g).to(cuda)
    x = torch.randn(N, (L + 1) ** 2, C, generator=g).to(cuda)
    idx_i = torch.randint(0, N, (E,), generator=g).to(cuda)
    idx_j = torch.sort(torch.randint(0, N, (E,), generator=g)).values.to(cuda)
    wig = torch.randn(E, 34, generator=g).to(cuda)
    ext = torch.randn(E, ext_width(L), generator=g).to(cuda)
    csd = torch.randn(2, C, generator=g).to(cuda)
    batch = torch.randint(0, 2, (N,), generator=g).to(cuda)
    return h2, W3, b3, x, idx_i, idx_j, wig, ext, csd, batch


@pytest.mark.parametrize("L", [3, 4])
@pytest.mark.parametrize("E,N", [(20000, 700), (1001, 64), (1, 1)])
def test_radial_gather_lmax_bitwise(cuda, L, E, N):
    """fu_radial_gather_fwd_lmax against fu_linear_resident (unpermuted weight) followed by
    fu_gather_fwd_lmax (edge-parallel and node-centric forms): rad and X bitwise equal."""
    from ops import linear, lmax
    h2, W3, b3, x, idx_i, idx_j, wig, ext, csd, batch = _lmax_inputs(cuda, E, N, L, seed=7 * E + N + L)
    rad_ref = linear.gemm_resident(h2, linear.linear_weight_split(W3), W3.shape[0], b3)
    perm = lmax.radial_gather_lmax_perm(128, L).to(cuda)
    got = lmax.radial_gather_lmax_fwd(h2, linear.linear_weight_split(W3[perm].contiguous()), b3[perm].contiguous(),
                                      x, idx_i, idx_j, wig, ext, csd, batch, L)
    for topology in (None,):
        X_ref = lmax.gather_lmax_fwd(x, idx_i, idx_j, wig, ext, rad_ref, csd, batch, L, topology)
        _assert_equal((rad_ref, *X_ref), got)


@pytest.mark.parametrize("L", [3, 4])
def test_model_radial_gather_lmax_matches_two_kernels(cuda, monkeypatch, L):
    """lmax 3 / 4 backbone (2 layers) on bcc Fe 6^3 (432 atoms): energy, forces and stress bit for
    bit equal with the fused radial-gather kernel on and off; the fused kernel called once per
    block and the lmax gather forward not at all."""
    import escn_md
    import heads
    import systems
    from ops import _lib
    from wrapper import ZeroAllocBackbone
    bb = escn_md.eSCNMDBackbone(num_layers=2, sphere_channels=128, hidden_channels=128, lmax=L, seed=0)
    hd = heads.MLPEnergyHead(128, 128, seed=1)
    model = heads.PotentialModel(ZeroAllocBackbone(bb.to(cuda)), hd.to(cuda))
    s = systems.bcc_fe(n_rep=6)
    ei, off = systems.neighbor_list(s.pos, s.cell, s.pbc, 6.0, 30)
    data = heads.make_atomic_data(s, ei, off, cuda)
    ce = model.backbone.ce
    real = _lib.call
    outs = {}
    for fused in (False, True):
        calls = []

        def spy(name, *args):
            calls.append(name)
            return real(name, *args)

        monkeypatch.setattr(ce, "RADIAL_GATHER", fused)
        monkeypatch.setattr(_lib, "call", spy)
        out = model(data, compute_forces=True, compute_stress=True)
        torch.cuda.synchronize()
        monkeypatch.setattr(_lib, "call", real)
        outs[fused] = {k: v.detach().cpu() for k, v in out.items() if torch.is_tensor(v)}
        assert calls.count("fu_radial_gather_fwd_lmax") == (2 if fused else 0)
        assert calls.count("fu_gather_fwd_lmax") == (0 if fused else 2)
    for k in ("energy", "forces", "stress"):
        assert torch.equal(outs[False][k], outs[True][k]), k


def test_radial_gather_with_recomputed_radial_outputs(cuda, monkeypatch):
    """The large-graph path that keeps each block's (E, C) radial source and recomputes the
    radial output in the backward (RAD_RECOMPUTE_MIN_EDGES) together with the fused forward:
    the recomputed output (fu_linear_resident, unpermuted weight) is the one the fused kernel
    wrote, so energy, forces and stress are bit for bit those of the path that keeps it."""
    import escn_md
    import heads
    import systems
    from wrapper import ZeroAllocBackbone
    bb = escn_md.eSCNMDBackbone(seed=0, num_layers=2)
    hd = heads.MLPEnergyHead(bb.sphere_channels, bb.hidden_channels, seed=1)
    model = heads.PotentialModel(ZeroAllocBackbone(bb.to(cuda)), hd.to(cuda))
    s = systems.bcc_fe(n_rep=6)
    ei, off = systems.neighbor_list(s.pos, s.cell, s.pbc, 6.0, 30)
    data = heads.make_atomic_data(s, ei, off, cuda)
    ce = model.backbone.ce
    assert ce.RADIAL_GATHER
    outs = []
    for threshold in (ce.RAD_RECOMPUTE_MIN_EDGES, 0):
        monkeypatch.setattr(ce, "RAD_RECOMPUTE_MIN_EDGES", threshold)
        out = model(data, compute_forces=True, compute_stress=True)
        outs.append({k: v.detach().cpu() for k, v in out.items() if torch.is_tensor(v)})
    for k in ("energy", "forces", "stress"):
        assert torch.equal(outs[0][k], outs[1][k]), k
