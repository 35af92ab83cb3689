"""Algorithmic traffic and work of every C-ABI entry point, from its call arguments.

Bytes count each tensor the kernel must touch exactly once (reads + writes, fp32 features,
int64 graph indices, int32 CSR arrays); node-sized tables are counted once per launch.
GEMMs count 2*M*N*K flops; the complex layer counts the 6*M*Nc*Kc flops of its three real
products.  These are the denominators of the roofline fractions:
achieved = algorithmic bytes (flops) / measured kernel time.

Matrix-core kernels run in one of three modes (fu_set_matmul_mode).  fp32 mode executes the
fp32 flops on v_mfma_f32_32x32x2_f32 (peak 157.3 TFLOP/s).  The split-bf16 mode executes each
fp32 product as six bf16 products of the operands' exact three-way bf16 splits; the split-fp16
mode as three fp16 products of two-way fp16 splits of power-of-two-scaled operands.  The
matrix cores then execute 6x (3x) the fp32 flops at the dense bf16 (fp16) peak of 2.5 PFLOP/s;
the roofline is that executed work against 2.5 PFLOP/s, with the fp32-equivalent rate alongside.
fu_gather_linear_gate keeps the bf16 split in both split modes.

Per-unit figures at C = 128, B = 64 (bytes per edge + bytes per node):
  gating fwd 10240 / bwd 15872; gather fwd 15512 + 4616, bwd 21784 + 9232;
  radial output layer + gather fwd (fu_radial_gather_fwd, K = 128) 16,024 + 4,616, with
  2 * 12C * K flops per edge on the matrix cores (HBM-bound: 3.9 GB against 0.29 PFLOP
  executed per launch at bcc Fe);
  scatter fwd 4752 + 9220, bwd 9504 + 4608; init scatter fwd 1576 + 5640, bwd 3256 + 4608;
  geom fwd 1448 (+ 1024 with embeddings) + 20, bwd 436 + 12; ln_silu 1032 / 1544 per row
  (grouped: per row and group, plus 16 B of edge ids per row when the tables are used).
"""
from __future__ import annotations

HBM_PEAK_GBS = 8000.0        # MI355X HBM3E
FP32_MFMA_PEAK_TFLOPS = 157.3  # MI355X dense fp32 matrix
BF16_MFMA_PEAK_TFLOPS = 2500.0  # MI355X dense bf16 matrix
SPLIT_PRODUCTS = 6              # bf16 products per fp32 product in the split-bf16 mode
F16_PRODUCTS = 3                # fp16 products per fp32 product in the split-fp16 mode
MATMUL_SPLIT_BF16, MATMUL_FP32, MATMUL_SPLIT_F16 = 0, 1, 2


def _products(name: str, matmul_mode: int) -> tuple[int, str]:
    """Matrix-core products per fp32 product of entry `name` in `matmul_mode`, and their kind."""
    if name == "fu_linear_resident":   # split-fp16 in every mode
        return F16_PRODUCTS, "fp16 mfma, 3 products per fp32 product"
    if matmul_mode == MATMUL_FP32:
        return 1, "fp32 mfma"
    if matmul_mode == MATMUL_SPLIT_F16 and name != "fu_gather_linear_gate":
        return F16_PRODUCTS, "fp16 mfma, 3 products per fp32 product"
    return SPLIT_PRODUCTS, "bf16 mfma, 6 products per fp32 product"


def _gating_fwd(a):
    E, C = a[6], a[7]
    return E * C * 20 * 4, 0


def _gating_bwd(a):
    E, C = a[9], a[10]
    return E * C * 31 * 4, 0


def _gather_fwd(a):
    # rad (12C) read and X (18C) written per edge; without X_m0 (conv1 m = 0 gathers its own
    # operand) 6C fewer of each
    E, N, C = a[10], a[11], a[13]
    per_edge = 30 * C if a[7] is not None else 18 * C
    return E * (per_edge * 4 + 34 * 4 + 16) + N * (9 * C * 4 + 8), 0


def _acc_read(E, acc, wig, env=1):
    """Bytes an accumulating call reads back: the Wigner rows (bit 0) and envelope (bit 1)."""
    return E * ((wig * 4 if acc & 1 else 0) + (env * 4 if acc & 2 else 0))


def _gather_bwd(a):
    E, N, C = a[18], a[19], a[21]
    return E * (42 * C * 4 + 2 * 34 * 4 + 8) + N * (2 * 9 * C * 4 + 16) + _acc_read(E, a[23], 34, 0), 0


def _scatter_fwd(a):
    N, E, C = a[9], a[10], a[11]
    return E * (9 * C * 4 + 34 * 4 + 4 + 4) + N * (2 * 9 * C * 4 + 4), 0


def _scatter_bwd(a):
    E, N, C = a[12], a[13], a[14]
    return E * (2 * 9 * C * 4 + 2 * 34 * 4 + 8 + 8) + N * 9 * C * 4 + _acc_read(E, a[15], 34), 0


def _init_fwd(a):
    N, E, C = a[10], a[11], a[14]
    return E * (3 * C * 4 + 8 * 4 + 4 + 4) + N * (9 * C * 4 + 2 * C * 4 + 16), 0


def _init_bwd(a):
    E, N, C = a[8], a[9], a[10]
    return E * (2 * 3 * C * 4 + 8 * 4 + 34 * 4 + 8 + 8) + N * 9 * C * 4 + _acc_read(E, a[11], 8), 0


def _geom_fwd(a):
    E, N, B, C = a[12], a[13], a[14], a[15]
    width = B + 2 * C if a[5] is not None else B
    return E * (16 + 12 + width * 4 + 34 * 4 + 4) + N * 20, 0


def _geom_bwd(a):
    E, N, B = a[10], a[11], a[12]
    gx = B * 4 if a[5] is not None else 0
    return E * (16 + 12 + gx + 34 * 4 + 4 + 12) + N * 12, 0


def _edge_vec(a):
    N, E = a[6], a[7]
    return E * (12 + 4 + 4) + N * (12 + 8), 0


def _ln_fwd(a):
    M, D = a[6], a[7]
    return M * (2 * D * 4 + 8), 0


def _ln_bwd(a):
    M, D = a[7], a[8]
    return M * (3 * D * 4 + 8), 0


def _linear_gate_bwd(a):
    # g_Z never stored: reads Y0 ((2L+1)C: values and gate pre-activations), P1 (LC),
    # P2 ((L-1)C); writes gY0 ((2L+1)C)
    M, C, K, L = a[12], a[13], a[14], a[15]
    N = (L + 1) * C
    return 4 * (M * K + N * K + (6 * L + 1) * M * C), 2 * M * N * K


def _complex_linear_gate_bwd(a):
    # reads F (2 Nc) and the gate columns of Y0 (Nc), writes gY (2 Nc) and the gate sums (Nc)
    M, Nc, Kc = a[19], a[20], a[21]
    return 4 * (2 * M * Kc + 2 * Nc * Kc + 6 * M * Nc), 6 * M * Nc * Kc


# lmax-general entry points: K = (L+1)^2 node rows, 34 + ext Wigner scalars, X 10L-2 and rad
# 6L blocks per edge, Y 6L-1 and Z 5L-1 blocks (the lmax = 2 formulas above at L = 2).
def _ext(L):
    return {2: 0, 3: 35, 4: 80}[L]


def _gather_fwd_l(a):
    E, N, C, L = a[15], a[16], a[18], a[19]
    return E * ((16 * L - 2) * C * 4 + (34 + _ext(L)) * 4 + 16) + N * ((L + 1) ** 2 * C * 4 + 8), 0


def _gather_bwd_l(a):
    E, N, C, L = a[18], a[19], a[21], a[22]
    return (E * ((22 * L - 2) * C * 4 + 2 * (34 + _ext(L)) * 4 + 8) + N * (2 * (L + 1) ** 2 * C * 4 + 16)
            + _acc_read(E, a[23], 34 + _ext(L), 0)), 0


def _scatter_fwd_l(a):
    N, E, C, L = a[10], a[11], a[12], a[13]
    return E * ((5 * L - 1) * C * 4 + (34 + _ext(L)) * 4 + 8) + N * (2 * (L + 1) ** 2 * C * 4 + 4), 0


def _scatter_bwd_l(a):
    E, N, C, L = a[14], a[15], a[16], a[17]
    return (E * (2 * (5 * L - 1) * C * 4 + 2 * (34 + _ext(L)) * 4 + 16) + N * (L + 1) ** 2 * C * 4
            + _acc_read(E, a[18], 34 + _ext(L))), 0


def _init_fwd_l(a):
    N, E, C, L = a[11], a[12], a[15], a[16]
    return E * ((L + 1) * C * 4 + ((L + 1) ** 2 - 1) * 4 + 8) + N * ((L + 1) ** 2 * C * 4 + 2 * C * 4 + 16), 0


def _init_bwd_l(a):
    E, N, C, L = a[10], a[11], a[12], a[13]
    return (E * (2 * (L + 1) * C * 4 + ((L + 1) ** 2 - 1) * 4 + (34 + _ext(L)) * 4 + 16) + N * (L + 1) ** 2 * C * 4
            + _acc_read(E, a[14], (L + 1) ** 2 - 1)), 0


def _gating_fwd_l(a):
    E, C, L = a[6], a[7], a[8]
    return E * C * (11 * L - 2) * 4, 0


def _gating_bwd_l(a):
    E, C, L = a[9], a[10], a[11]
    return E * C * (17 * L - 3) * 4, 0


def _radial_gather(a):
    # the radial output layer fused with the gather: h2 (E, K) read, rad (12C) and X (18C)
    # written per edge, the edge's two ids and 34 Wigner scalars read, the weight once, the node
    # rows counted once per launch (as the gather's)
    E, N, C, K = a[14], a[15], a[17], a[18]
    return E * ((K + 30 * C + 34) * 4 + 16) + N * (9 * C * 4 + 8) + 12 * C * K * 4, 2 * E * 12 * C * K


def _radial_gather_l(a):
    # lmax 3, 4: h2 read, rad (6L C) and X (2(5L - 1) C) written per edge, the ids, the 34 + ext
    # Wigner scalars read, the weight once, the node rows once per launch
    E, N, C, K, L = a[15], a[16], a[18], a[19], a[20]
    per_edge = (K + 6 * L * C + 2 * (5 * L - 1) * C + 34 + _ext(L)) * 4 + 16
    return E * per_edge + N * ((L + 1) ** 2 * C * 4 + 8) + 6 * L * C * K * 4, 2 * E * 6 * L * C * K


def _wig_ext_fwd(a):
    E, L = a[2], a[3]
    return E * (34 + _ext(L)) * 4, 0


def _wig_ext_bwd(a):
    E, L = a[3], a[4]
    return E * (2 * 34 + _ext(L)) * 4, 0


def _linear(a):
    M, N, K = a[7], a[8], a[9]
    return 4 * (M * K + M * N + N * K), 2 * M * N * K


def _linear_resident(a):
    M, N, K = a[6], a[7], a[8]
    return 4 * (M * K + M * N + N * K), 2 * M * N * K


def _linear_batched(a):
    M, N, K, B = a[15], a[16], a[17], a[18]
    r = M * N if a[9] else 0   # the residual, read once
    return 4 * B * (M * K + M * N + N * K + r), 2 * B * M * N * K


def _linear_ln_silu(a):
    # the GEMM (batch B) plus the LayerNorm epilogue: Y written once (pre too when stored),
    # the statistics, and with tables two int64 edge ids per row (tables L2-resident)
    M, N, K, B, G = a[15], a[16], a[17], a[18], a[30]
    pre = B * M * N if a[12] else 0
    tab = M * 16 if a[19] else 0
    return 4 * (B * (M * K + M * N + N * K) + pre) + 8 * M * G + tab, 2 * B * M * N * K


def _linear_ln_silu_bwd(a):
    # the recomputed GEMM plus the LayerNorm backward epilogue: g_out read, g_x written
    M, N, K, G = a[6], a[7], a[8], a[22]
    tab = M * 16 if a[11] else 0
    return 4 * (M * K + N * K + 2 * M * N) + 8 * M * G + tab, 2 * M * N * K


def _linear_dgrad_ln_silu_bwd(a):
    # the output-layer input-gradient GEMM (N = 128) plus the LayerNorm backward epilogue:
    # the LayerNorm input x read, g_x written, the row statistics read
    M, K, N = a[6], a[7], 128
    return 4 * (M * K + N * K + 2 * M * N) + 8 * M, 2 * M * N * K


def _complex_linear(a):
    # three real (M x Kc) x (Kc x Nc) products (the packed real form of the reference would be
    # four; so is the split path without a pre-split weight, which executes 4/3 of this)
    M, Nc, Kc = a[10], a[11], a[12]
    return 4 * (2 * M * Kc + 2 * M * Nc + 2 * Nc * Kc), 6 * M * Nc * Kc


def _linear_gate(a):
    # N = (2L+1)C outputs Y plus the gated / SiLU copies Z ((L+1)C) (and the sigmoids S (LC)
    # when requested)
    M, C, K, L = a[11], a[12], a[13], a[14]
    N = (2 * L + 1) * C
    zs = (2 * L + 1) if a[9] is not None else (L + 1)
    return 4 * (M * K + N * K + M * N + zs * M * C), 2 * M * N * K


def _gather_linear_gate(a):
    # conv1 m = 0 with its operand gathered: the m = 0 radial blocks (6C), the edge's two ids
    # and 8 Wigner scalars read, Y (5C) and Z (3C) written, W once (the node rows are the
    # gather's per-node bytes, L2-resident across a node's edges, and not counted)
    E, C = a[14], a[15]
    return 4 * E * (6 * C + 5 * C + 3 * C + 8) + 16 * E + 4 * 30 * C * C, 2 * E * 5 * C * 6 * C


def _complex_linear_gate(a):
    # complex product plus the gate columns of Y0 read (Nc) and the gated copies Z_r, Z_i (2 Nc)
    M, Nc, Kc = a[17], a[18], a[19]
    return 4 * (2 * M * Kc + 2 * M * Nc + 2 * Nc * Kc + 3 * M * Nc), 6 * M * Nc * Kc


def _ln_grouped_fwd(a):
    # x read + out written per row and group, mean/rstd; with tables: two int64 edge ids per
    # row and the (L2-resident) 100-row tables once per launch
    M, G, D = a[15], a[16], a[17]
    tab = (M * 16 + 2 * 100 * G * D * 4) if a[2] is not None else 0
    return M * G * (2 * D * 4 + 8) + tab, 0


def _ln_grouped_bwd(a):
    M, G, D = a[17], a[18], a[19]
    tab = (M * 16 + 2 * 100 * G * D * 4) if a[2] is not None else 0
    return M * G * (3 * D * 4 + 8) + tab, 0


WORK = {
    "fu_gating_fwd": _gating_fwd,
    "fu_gating_bwd": _gating_bwd,
    "fu_gather_fwd": _gather_fwd,
    "fu_gather_bwd": _gather_bwd,
    "fu_scatter_fwd": _scatter_fwd,
    "fu_scatter_bwd": _scatter_bwd,
    "fu_init_scatter_fwd": _init_fwd,
    "fu_init_scatter_bwd": _init_bwd,
    "fu_geom_fwd": _geom_fwd,
    "fu_geom_bwd": _geom_bwd,
    "fu_edge_vec_reduce": _edge_vec,
    "fu_ln_silu_fwd": _ln_fwd,
    "fu_ln_silu_bwd": _ln_bwd,
    "fu_ln_silu_grouped_fwd": _ln_grouped_fwd,
    "fu_ln_silu_grouped_bwd": _ln_grouped_bwd,
    "fu_linear": _linear,
    "fu_linear_batched": _linear_batched,
    "fu_linear_resident": _linear_resident,
    "fu_radial_gather_fwd": _radial_gather,
    "fu_radial_gather_fwd_lmax": _radial_gather_l,
    "fu_linear_ln_silu": _linear_ln_silu,
    "fu_linear_ln_silu_bwd": _linear_ln_silu_bwd,
    "fu_linear_dgrad_ln_silu_bwd": _linear_dgrad_ln_silu_bwd,
    "fu_complex_linear": _complex_linear,
    "fu_linear_gate": _linear_gate,
    "fu_gather_linear_gate": _gather_linear_gate,
    "fu_linear_gate_bwd": _linear_gate_bwd,
    "fu_complex_linear_gate_bwd": _complex_linear_gate_bwd,
    "fu_gather_fwd_lmax": _gather_fwd_l,
    "fu_gather_bwd_lmax": _gather_bwd_l,
    "fu_scatter_fwd_lmax": _scatter_fwd_l,
    "fu_scatter_bwd_lmax": _scatter_bwd_l,
    "fu_init_scatter_fwd_lmax": _init_fwd_l,
    "fu_init_scatter_bwd_lmax": _init_bwd_l,
    "fu_gating_fwd_lmax": _gating_fwd_l,
    "fu_gating_bwd_lmax": _gating_bwd_l,
    "fu_wigner_ext_fwd": _wig_ext_fwd,
    "fu_wigner_ext_bwd": _wig_ext_bwd,
    "fu_complex_linear_gate": _complex_linear_gate,
}

MFMA_BOUND = {"fu_linear", "fu_linear_batched", "fu_complex_linear", "fu_linear_gate", "fu_complex_linear_gate",
              "fu_linear_gate_bwd", "fu_complex_linear_gate_bwd", "fu_linear_ln_silu", "fu_linear_ln_silu_bwd",
              "fu_linear_dgrad_ln_silu_bwd", "fu_gather_linear_gate", "fu_linear_resident"}


def summarize(durations, matmul_mode: int = MATMUL_SPLIT_F16) -> dict:
    """Per entry point: calls, total/avg ms, algorithmic bytes/flops per launch and the
    achieved fraction of the bounding roofline (matrix-core kernels in `matmul_mode`).

    For the matrix-core entry points `frac` is the executed rate against the matrix peak.
    `roofline_frac` is the standard roofline reading: the sum over launches of
    max(executed flops / matrix peak, algorithmic bytes / HBM peak) over the measured time,
    which differs from `frac` where a launch's arithmetic intensity puts it under the HBM
    slope (the K = 128 shapes, whose operands and output are as large as their work);
    `hbm_bound_launches` counts those launches."""
    mpeak = FP32_MFMA_PEAK_TFLOPS if matmul_mode == MATMUL_FP32 else BF16_MFMA_PEAK_TFLOPS
    agg: dict = {}
    for name, args, ms in durations:
        if name not in WORK:
            continue
        nbytes, flops = WORK[name](args)
        a = agg.setdefault(name, {"calls": 0, "ms": 0.0, "bytes": 0, "flops": 0, "ideal_s": 0.0, "hbm_bound": 0})
        a["calls"] += 1
        a["ms"] += ms
        a["bytes"] += nbytes
        a["flops"] += flops
        if name in MFMA_BOUND:
            mul = _products(name, matmul_mode)[0]
            t_mfma, t_hbm = mul * flops / (mpeak * 1e12), nbytes / (HBM_PEAK_GBS * 1e9)
            a["ideal_s"] += max(t_mfma, t_hbm)
            a["hbm_bound"] += int(t_hbm > t_mfma)
    out = {}
    for name, a in agg.items():
        sec = a["ms"] / 1e3
        rec = {"calls": a["calls"], "total_ms": round(a["ms"], 4), "avg_us": round(1e3 * a["ms"] / a["calls"], 2)}
        if name in MFMA_BOUND:
            fp32_rate = a["flops"] / sec / 1e12 if sec > 0 else 0.0
            mul, op = _products(name, matmul_mode)
            ach, peak = mul * fp32_rate, mpeak
            rec.update(bound="mfma", unit="TFLOP/s", achieved=round(ach, 2), peak=peak, frac=round(ach / peak, 4),
                       matrix_op=op, fp32_tflops=round(fp32_rate, 2), flops_per_launch=a["flops"] // a["calls"],
                       hbm_gbs=round(a["bytes"] / sec / 1e9, 1) if sec > 0 else 0.0,
                       roofline_frac=round(a["ideal_s"] / sec, 4) if sec > 0 else 0.0,
                       hbm_bound_launches=a["hbm_bound"])
        else:
            ach = a["bytes"] / sec / 1e9 if sec > 0 else 0.0
            rec.update(bound="hbm", unit="GB/s", achieved=round(ach, 1), peak=HBM_PEAK_GBS,
                       frac=round(ach / HBM_PEAK_GBS, 4), bytes_per_launch=a["bytes"] // a["calls"])
        out[name] = rec
    return out
