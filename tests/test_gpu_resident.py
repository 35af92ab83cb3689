"""fu_linear_resident (the radial output layers' GEMM with each workgroup's rows of A resident in
LDS, split-fp16 products at exact row scales) against float64 and against the fp32 MFMA on the
same operands, with the bars of the tiled split GEMM (tests/test_gpu_ops.py): rms within 1.1x
and max within 1.5x the fp32 MFMA's on Gaussian operands, every row within 1.5x the fp32
MFMA's worst row (+1e-7) on the window cases, and the model routing its output layers here."""
import pytest
import torch

pytestmark = pytest.mark.gpu


def _ops():
    from ops import _lib, linear
    return _lib, linear


def _fp32_mfma(x, W, bias=None):
    """The same product on the fp32 MFMA (fu_linear takes N % 4 == 0: W padded with zero rows)."""
    _lib, linear = _ops()
    N = W.shape[0]
    pad = (-N) % 4
    if pad:
        W = torch.cat([W, W.new_zeros(pad, W.shape[1])])
        bias = None if bias is None else torch.cat([bias, bias.new_zeros(pad)])
    with _lib.matmul_mode(_lib.MATMUL_FP32):
        return linear.gemm(x, W, bias)[:, :N]


@pytest.mark.parametrize("M,N,K", [(70000, 1536, 128), (3001, 384, 128), (1000, 200, 64), (513, 32, 16),
                                   (257, 100, 48), (130, 3072, 128), (300, 90, 32)])
@pytest.mark.parametrize("with_bias", [True, False], ids=["bias", "nobias"])
def test_resident_accuracy(cuda, M, N, K, with_bias):
    _lib, linear = _ops()
    g = torch.Generator().manual_seed(M + N + K)
    x = torch.randn(M, K, generator=g).to(cuda)
    W = (torch.randn(N, K, generator=g) / K ** 0.5).to(cuda)
    b = torch.randn(N, generator=g).to(cuda) if with_bias else None
    W2 = linear.linear_weight_split(W)
    y = linear.gemm_resident(x, W2, N, b)
    ref = x.double() @ W.double().T + (b.double() if with_bias else 0.0)
    yf = _fp32_mfma(x, W, b)
    err = {}
    for k, v in (("res", y), ("fp32", yf)):
        d = v.double() - ref
        err[k] = (d.norm().item() / ref.norm().item(), d.abs().max().item() / ref.abs().max().item())
    print(f"resident {M}x{N}x{K}: rms {err['res'][0]:.2e} max {err['res'][1]:.2e}; "
          f"fp32 MFMA rms {err['fp32'][0]:.2e} max {err['fp32'][1]:.2e}")
    assert err["res"][0] < 1e-6
    # at K = 16 both errors are a few fp32 roundings of the output: one rounding (2^-24) of slack
    slack = 2.0 ** -24
    assert err["res"][0] <= 1.1 * err["fp32"][0] + slack and err["res"][1] <= 1.5 * err["fp32"][1] + slack, err


def test_resident_strided_input_and_untouched_padding(cuda):
    """A row-strided view of a wider buffer as A (the radial trunk's per-block slices), an output
    with ldy > N inside a larger buffer: columns past N and rows past M keep their contents, and
    two calls give the same bits."""
    _lib, linear = _ops()
    M, N, K = 1000, 384, 128
    g = torch.Generator().manual_seed(7)
    wide = torch.randn(M, 5 * K, generator=g).to(cuda)
    x = wide[:, 2 * K:3 * K]
    W = (torch.randn(N, K, generator=g) / K ** 0.5).to(cuda)
    b = torch.randn(N, generator=g).to(cuda)
    W2 = linear.linear_weight_split(W)
    buf = torch.full((M + 7, N + 12), 12345.0, device=cuda)
    out = buf[:M, :N]
    _lib.call("fu_linear_resident", x.data_ptr(), x.stride(0), W2.data_ptr(), b.data_ptr(), out.data_ptr(),
              out.stride(0), M, N, K, _lib.stream_ptr(x.device))
    assert (buf[:, N:] == 12345.0).all() and (buf[M:] == 12345.0).all()
    ref = x.contiguous().double() @ W.double().T + b.double()
    assert ((out.double() - ref).norm() / ref.norm()).item() < 1e-6
    again = linear.gemm_resident(x, W2, N, b)
    assert torch.equal(again, out)


def _ramp(K, T, orient):
    return torch.linspace(-T, T, K, dtype=torch.float64) * orient


@pytest.mark.parametrize("M", [70000, 3000], ids=["m70000", "m3000"])
@pytest.mark.parametrize("T", [4, 8, 12])
@pytest.mark.parametrize("orient", [1, -1], ids=["max_last", "max_first"])
def test_resident_anticorrelated_range(cuda, M, T, orient):
    """x ~ 2^t N(0,1) and w ~ 2^-t N(0,1) with t ramping over [-T, T] along K: every k
    contributes comparably, so the small pieces of each row matter; spreads of 2^24 take the
    two-loop pass (split_f16.h)."""
    _lib, linear = _ops()
    N, K = 384, 128
    g = torch.Generator().manual_seed(M + 31 * T + orient)
    t = _ramp(K, T, orient)
    x = (torch.randn(M, K, generator=g, dtype=torch.float64) * torch.exp2(t)).float().to(cuda)
    W = (torch.randn(N, K, generator=g, dtype=torch.float64) * torch.exp2(-t) / K ** 0.5).float().to(cuda)
    ref = x.double() @ W.double().T
    rn = ref.norm(dim=1).clamp_min(1e-300)
    y = linear.gemm_resident(x, linear.linear_weight_split(W), N)
    assert torch.isfinite(y).all()
    w_res = ((y.double() - ref).norm(dim=1) / rn).max().item()
    w_f = ((_fp32_mfma(x, W).double() - ref).norm(dim=1) / rn).max().item()
    print(f"resident anticorrelated +-2^{T} orient {orient} M {M}: worst row {w_res:.2e}, fp32 MFMA {w_f:.2e}")
    assert w_res <= 1.5 * w_f + 1e-7


@pytest.mark.parametrize("s", [16, 20, 26])
def test_resident_small_entries_elementwise(cuda, s):
    """Each row's first chunk is O(1) and meets zero weights, the rest is 2^-s smaller and meets
    O(1) weights: error per element against sum_k |x_ik| |w_jk|, worst element within 1.5x the
    fp32 MFMA's plus 2^-22."""
    _lib, linear = _ops()
    M, N, K = 3000, 384, 128
    g = torch.Generator().manual_seed(100 + s)
    x = torch.randn(M, K, generator=g, dtype=torch.float64)
    x[:, 16:] *= 2.0 ** -s
    W = torch.randn(N, K, generator=g, dtype=torch.float64) / K ** 0.5
    W[:, :16] = 0.0
    x, W = x.float().to(cuda), W.float().to(cuda)
    ref = x.double() @ W.double().T
    scale = (x.double().abs() @ W.double().abs().T).clamp_min(1e-300)
    y = linear.gemm_resident(x, linear.linear_weight_split(W), N)
    w_res = ((y.double() - ref).abs() / scale).max().item()
    w_f = ((_fp32_mfma(x, W).double() - ref).abs() / scale).max().item()
    print(f"resident small entries 2^-{s}: worst element {w_res:.2e}, fp32 MFMA {w_f:.2e}")
    assert w_res <= 1.5 * w_f + 2.0 ** -22


def test_resident_dynamic_range(cuda):
    """Rows scaled by 2^+-40, zero rows, 1e-20 rows and columns scaled by 2^+-30: every row's
    error relative to its norm within 1.5x the fp32 MFMA's worst row plus 1e-7, and finite."""
    _lib, linear = _ops()
    M, N, K = 3000, 256, 128
    g = torch.Generator().manual_seed(3)
    x = torch.randn(M, K, generator=g, dtype=torch.float64)
    x[0::7] *= 2.0 ** 40
    x[1::7] *= 2.0 ** -40
    x[2::7] = 0.0
    x[3::7] *= 1e-20
    W = torch.randn(N, K, generator=g, dtype=torch.float64) / K ** 0.5
    W[0::5] *= 2.0 ** 30
    W[1::5] *= 2.0 ** -30
    x, W = x.float().to(cuda), W.float().to(cuda)
    ref = x.double() @ W.double().T
    rn = ref.norm(dim=1).clamp_min(1e-300)
    y = linear.gemm_resident(x, linear.linear_weight_split(W), N)
    assert torch.isfinite(y).all()
    assert (y[2::7] == 0.0).all()
    w_res = ((y.double() - ref).norm(dim=1) / rn).max().item()
    w_f = ((_fp32_mfma(x, W).double() - ref).norm(dim=1) / rn).max().item()
    print(f"resident dynamic range: worst row {w_res:.2e}, fp32 MFMA {w_f:.2e}")
    assert w_res <= 1.5 * w_f + 1e-7


def test_resident_rejects_bad_shapes(cuda):
    _lib, linear = _ops()
    lib = _lib.load()
    for N, K in ((0, 128), (64, 8), (64, 100)):
        assert lib.fu_linear_weight_split_bytes(N, K) < 0, (N, K)
    # the split serves any K % 16 == 0 (the tall GEMMs' W2); the resident GEMM takes K <= 128
    W144 = linear.linear_weight_split(torch.randn(64, 144, device=cuda))
    x144 = torch.randn(10, 144, device=cuda)
    with pytest.raises(_lib.FlashUMAError):
        linear.gemm_resident(x144, W144, 64)
    W = torch.randn(64, 100, device=cuda)
    with pytest.raises(_lib.FlashUMAError):
        linear.linear_weight_split(W)
    W2 = linear.linear_weight_split(torch.randn(64, 128, device=cuda))
    x = torch.randn(10, 128, device=cuda)
    y = torch.empty(10, 64, device=cuda)
    with pytest.raises(_lib.FlashUMAError):   # ldy < N
        _lib.call("fu_linear_resident", x.data_ptr(), 128, W2.data_ptr(), None, y.data_ptr(), 32, 10, 64, 128,
                  _lib.stream_ptr(x.device))
    with pytest.raises(_lib.FlashUMAError):   # lda not a multiple of 4
        _lib.call("fu_linear_resident", x.data_ptr(), 129, W2.data_ptr(), None, y.data_ptr(), 64, 9, 64, 128,
                  _lib.stream_ptr(x.device))


def test_model_output_layers_use_resident_kernel(cuda, monkeypatch):
    """In the default (split-fp16) mode the radial bank's output layers run on
    fu_linear_resident or, for the blocks' layers (RADIAL_GATHER), fu_radial_gather_fwd (one
    launch per MLP in the forward), in the other modes on fu_linear."""
    import escn_md
    import heads
    import systems
    from ops import _lib
    from wrapper import ZeroAllocBackbone
    bb = escn_md.eSCNMDBackbone(seed=0, num_layers=2)
    hd = heads.MLPEnergyHead(bb.sphere_channels, bb.hidden_channels, seed=1)
    model = heads.PotentialModel(ZeroAllocBackbone(bb.to(cuda)), hd.to(cuda))
    s = systems.cu_slab_co()
    ei, off = systems.neighbor_list(s.pos, s.cell, s.pbc, bb.cutoff, bb.max_neighbors)
    real = _lib.call
    for mode, want, fused in ((_lib.MATMUL_SPLIT_F16, 1, 2), (_lib.MATMUL_SPLIT_BF16, 0, 0)):
        calls = []

        def spy(name, *args):
            calls.append(name)
            return real(name, *args)

        monkeypatch.setattr(_lib, "call", spy)
        with _lib.matmul_mode(mode):
            out = model(heads.make_atomic_data(s, ei, off, cuda), compute_forces=True, compute_stress=True)
            torch.cuda.synchronize()
        monkeypatch.setattr(_lib, "call", real)
        assert calls.count("fu_linear_resident") == want, (mode, calls.count("fu_linear_resident"))
        assert calls.count("fu_radial_gather_fwd") == fused, (mode, calls.count("fu_radial_gather_fwd"))
        assert torch.isfinite(out["forces"]).all()
