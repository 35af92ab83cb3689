"""Tall split-fp16 GEMMs reading pre-split weight fragments (the W2 argument of fu_linear,
fu_linear_gate, fu_linear_gate_bwd and fu_linear_dgrad_ln_silu_bwd): the products keep the bars
of the tiled split GEMM against float64 and the fp32 MFMA (tests/test_gpu_ops.py), on the model's
shapes and on the window cases of split_f16.h, and the model's users of W2 (the conv pair and the
radial bank) agree with the same computation without it to fp32 rounding."""
import pytest
import torch

pytestmark = pytest.mark.gpu

M_TALL = 70000   # >= 65,536 rows: tall tiles, where W2 is read


def _ops():
    from ops import _lib, linear
    return _lib, linear


def _fp32_mfma(x, W):
    _lib, linear = _ops()
    with _lib.matmul_mode(_lib.MATMUL_FP32):
        return linear.gemm(x, W)


def _with_w2(x, W):
    _lib, linear = _ops()
    return linear.gemm(x, W, W2=linear.linear_weight_split(W))


@pytest.mark.parametrize("N,K", [(640, 768), (768, 640), (384, 384), (128, 1536), (200, 64)])
def test_weight_fragments_accuracy(cuda, N, K):
    g = torch.Generator().manual_seed(N + K)
    x = torch.randn(M_TALL, K, generator=g).to(cuda)
    W = (torch.randn(N, K, generator=g) / K ** 0.5).to(cuda)
    ref = x.double() @ W.double().T
    err = {}
    for k, y in (("w2", _with_w2(x, W)), ("fp32", _fp32_mfma(x, W))):
        d = y.double() - ref
        err[k] = (d.norm().item() / ref.norm().item(), d.abs().max().item() / ref.abs().max().item())
    print(f"W2 {N}x{K}: rms {err['w2'][0]:.2e} max {err['w2'][1]:.2e}; fp32 MFMA rms {err['fp32'][0]:.2e} "
          f"max {err['fp32'][1]:.2e}")
    assert err["w2"][0] < 1e-6
    assert err["w2"][0] <= 1.1 * err["fp32"][0] and err["w2"][1] <= 1.5 * err["fp32"][1], err


@pytest.mark.parametrize("T", [4, 8, 12])
@pytest.mark.parametrize("orient", [1, -1], ids=["max_last", "max_first"])
def test_weight_fragments_anticorrelated_range(cuda, T, orient):
    """x ~ 2^t N(0,1), w ~ 2^-t N(0,1), t ramping over [-T, T] along K: the weight's side of the
    window rule comes from its precomputed column flags."""
    N, K = 256, 768
    g = torch.Generator().manual_seed(31 * T + orient)
    t = torch.linspace(-T, T, K, dtype=torch.float64) * orient
    x = (torch.randn(M_TALL, K, generator=g, dtype=torch.float64) * torch.exp2(t)).float().to(cuda)
    W = (torch.randn(N, K, generator=g, dtype=torch.float64) * torch.exp2(-t) / K ** 0.5).float().to(cuda)
    ref = x.double() @ W.double().T
    rn = ref.norm(dim=1).clamp_min(1e-300)
    y = _with_w2(x, W)
    assert torch.isfinite(y).all()
    w_res = ((y.double() - ref).norm(dim=1) / rn).max().item()
    w_f = ((_fp32_mfma(x, W).double() - ref).norm(dim=1) / rn).max().item()
    print(f"W2 anticorrelated +-2^{T} orient {orient}: worst row {w_res:.2e}, fp32 MFMA {w_f:.2e}")
    assert w_res <= 1.5 * w_f + 1e-7


@pytest.mark.parametrize("s", [16, 26])
def test_weight_fragments_small_entries_elementwise(cuda, s):
    N, K = 256, 768
    g = torch.Generator().manual_seed(200 + s)
    x = torch.randn(M_TALL, K, generator=g, dtype=torch.float64)
    x[:, 16:] *= 2.0 ** -s
    W = torch.randn(N, K, generator=g, dtype=torch.float64) / K ** 0.5
    W[:, :16] = 0.0
    x, W = x.float().to(cuda), W.float().to(cuda)
    ref = x.double() @ W.double().T
    scale = (x.double().abs() @ W.double().abs().T).clamp_min(1e-300)
    w_res = ((_with_w2(x, W).double() - ref).abs() / scale).max().item()
    w_f = ((_fp32_mfma(x, W).double() - ref).abs() / scale).max().item()
    print(f"W2 small entries 2^-{s}: worst element {w_res:.2e}, fp32 MFMA {w_f:.2e}")
    assert w_res <= 1.5 * w_f + 2.0 ** -22


def test_weight_fragments_dynamic_range(cuda):
    """Rows at 2^+-40, zero and 1e-20 rows, weight columns at 2^+-30 and a zero column."""
    N, K = 256, 384
    g = torch.Generator().manual_seed(5)
    x = torch.randn(M_TALL, K, generator=g, dtype=torch.float64)
    x[0::7] *= 2.0 ** 40
    x[1::7] *= 2.0 ** -40
    x[2::7] = 0.0
    x[3::7] *= 1e-20
    W = torch.randn(N, K, generator=g, dtype=torch.float64) / K ** 0.5
    W[0::5] *= 2.0 ** 30
    W[1::5] *= 2.0 ** -30
    W[7] = 0.0
    x, W = x.float().to(cuda), W.float().to(cuda)
    ref = x.double() @ W.double().T
    rn = ref.norm(dim=1).clamp_min(1e-300)
    y = _with_w2(x, W)
    assert torch.isfinite(y).all() and (y[2::7] == 0.0).all() and (y[:, 7] == 0.0).all()
    w_res = ((y.double() - ref).norm(dim=1) / rn).max().item()
    w_f = ((_fp32_mfma(x, W).double() - ref).norm(dim=1) / rn).max().item()
    print(f"W2 dynamic range: worst row {w_res:.2e}, fp32 MFMA {w_f:.2e}")
    assert w_res <= 1.5 * w_f + 1e-7


def test_w2_not_read_below_tall_tiles(cuda):
    """Below 65,536 rows (128-row tiles) and outside the split-fp16 mode W2 is not read: the
    result is the plain path's, bit for bit."""
    _lib, linear = _ops()
    g = torch.Generator().manual_seed(9)
    x = torch.randn(3000, 384, generator=g).to(cuda)
    W = (torch.randn(256, 384, generator=g) / 384 ** 0.5).to(cuda)
    W2 = linear.linear_weight_split(W)
    assert torch.equal(linear.gemm(x, W, W2=W2), linear.gemm(x, W))
    xt = torch.randn(M_TALL, 384, generator=g).to(cuda)
    with _lib.matmul_mode(_lib.MATMUL_SPLIT_BF16):
        assert torch.equal(linear.gemm(xt, W, W2=W2), linear.gemm(xt, W))


def _normwise(a, b):
    return ((a.double() - b.double()).norm() / b.double().norm()).item()


def test_conv_pair_with_weight_fragments(cuda):
    """conv1 + gate + conv2 and its backward at a tall size (C = 128, lmax 2) with the m = 0
    weights pre-split (fu_linear_gate, fu_linear, fu_linear_gate_bwd read W2) against the same
    with the complex splits only: outputs and input gradients agree normwise to 2e-6, and the
    forward's first 2,048 rows match float64 at the op bar."""
    from ops import gating
    from ops.linear import complex_weight_split, linear_weight_split
    from oracle import ops_ref as R
    C, L, M = 128, 2, M_TALL
    g = torch.Generator().manual_seed(11)
    r = lambda *s: torch.randn(*s, generator=g)
    X = [r(M, 2 * (L + 1) * C), r(M, 4 * L * C), r(M, 4 * (L - 1) * C)]
    W0, b0 = r((2 * L + 1) * C, 2 * (L + 1) * C) / (2 * (L + 1) * C) ** 0.5, r((2 * L + 1) * C) * 0.3
    R1, I1 = r(L * C, 2 * L * C) / (2 * L * C) ** 0.5, r(L * C, 2 * L * C) / (2 * L * C) ** 0.5
    n2 = (L - 1) * C
    R2, I2 = r(n2, 2 * n2) / (2 * n2) ** 0.5, r(n2, 2 * n2) / (2 * n2) ** 0.5
    V0, c0 = r((L + 1) * C, (L + 1) * C) / ((L + 1) * C) ** 0.5, r((L + 1) * C) * 0.3
    S1, T1 = r(L * C, L * C) / (L * C) ** 0.5, r(L * C, L * C) / (L * C) ** 0.5
    S2, T2 = r(n2, n2) / n2 ** 0.5, r(n2, n2) / n2 ** 0.5
    rows = gating.gate_paired_rows(C, L)
    dv = lambda t: t.contiguous().to(cuda)
    W0p = W0[rows]
    conv1 = [dv(W0p), dv(b0[rows]), dv(W0p.t()), dv(R1), dv(I1), dv(R1.t()), dv(-I1.t()), dv(R2), dv(I2), dv(R2.t()),
             dv(-I2.t())]
    conv2 = [dv(V0), dv(c0), dv(V0.t()), dv(S1), dv(T1), dv(S1.t()), dv(-T1.t()), dv(S2), dv(T2), dv(S2.t()),
             dv(-T2.t())]
    pairs = [conv1[3:5], conv1[5:7], conv1[7:9], conv1[9:11], conv2[3:5], conv2[5:7], conv2[7:9], conv2[9:11]]
    csplits = tuple(complex_weight_split(P, Q) for P, Q in pairs)
    rsplits = tuple(linear_weight_split(w) for w in (conv1[0], conv1[2], conv2[0], conv2[2]))
    cot = [r(M, (L + 1) * C), r(M, 2 * L * C), r(M, 2 * (L - 1) * C)]
    res = {}
    for tag, sp in (("w2", csplits + rsplits), ("plain", csplits)):
        Xg = [x.to(cuda).requires_grad_(True) for x in X]
        Zo = gating.conv1_gate_conv2(*Xg, conv1, conv2, C, sp)
        gx = torch.autograd.grad(Zo, Xg, [c.to(cuda) for c in cot])
        res[tag] = ([z.detach() for z in Zo], gx)
    for a, b in zip(res["w2"][0] + list(res["w2"][1]), res["plain"][0] + list(res["plain"][1])):
        assert _normwise(a, b) <= 2e-6, _normwise(a, b)
    n = 2048
    y0 = X[0][:n].double() @ W0.double().T + b0.double()
    y1 = X[1][:n].double() @ R.pack_so2(R1.double(), I1.double()).T
    y2 = X[2][:n].double() @ R.pack_so2(R2.double(), I2.double()).T
    z0, z1, z2 = R.gating(y0, y1, y2, C)
    ref = (z0 @ V0.double().T + c0.double(), z1 @ R.pack_so2(S1.double(), T1.double()).T,
           z2 @ R.pack_so2(S2.double(), T2.double()).T)
    for z, rr in zip(res["w2"][0], ref):
        d = (z[:n].double().cpu() - rr).abs().max().item() / rr.abs().max().item()
        assert d <= 2e-5, d


def test_radial_bank_backward_with_weight_fragments(cuda, monkeypatch):
    """The radial bank's input-gradient GEMMs (fu_linear_dgrad_ln_silu_bwd with W3^T, the trunk's
    Gaussian gradient with W1g^T) with their pre-split weights against the same without them:
    the Gaussian gradient agrees normwise to 2e-6."""
    import escn_md
    from ops.radial import RadialBank
    from wrapper import ZeroAllocBackbone
    bb = escn_md.eSCNMDBackbone(seed=0, num_layers=2).to(cuda)
    bank = ZeroAllocBackbone(bb).ce.radial_bank
    E = M_TALL
    g = torch.Generator(device=cuda).manual_seed(3)
    gauss = torch.rand(E, bank.B, device=cuda, generator=g)
    Z = torch.full((100,), 26, dtype=torch.long, device=cuda)
    ii = torch.randint(0, 100, (E,), device=cuda, generator=g)
    jj = torch.randint(0, 100, (E,), device=cuda, generator=g)
    cots = None
    res = {}
    for tag in ("w2", "plain"):
        if tag == "plain":
            monkeypatch.setattr(RadialBank, "out_t_split", lambda self, k: None)
            monkeypatch.setattr(RadialBank, "_split", lambda self, name, ok: None)
        gg = gauss.clone().requires_grad_(True)
        outs = bank(gg, Z, ii, jj)
        if cots is None:
            cots = [torch.randn(o.shape, device=cuda, generator=g) for o in outs]
        (res[tag],) = torch.autograd.grad(outs, [gg], cots)
    assert _normwise(res["w2"], res["plain"]) <= 2e-6, _normwise(res["w2"], res["plain"])
