"""The roofline accounting reads each entry point's sizes from the right argument positions:
for every entry point with a work function, the size parameters are located by name in
include/flashuma.h and the work computed from a call with distinct sizes is checked against
the formula stated for it."""
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "flashuma.h")


def _params(name):
    text = re.sub(r"/\*.*?\*/", "", open(HEADER).read(), flags=re.S)
    m = re.search(r"\b" + name + r"\s*\(([^)]*)\)\s*;", text)
    assert m, name
    return [p.split()[-1].lstrip("*") for p in m.group(1).split(",")]


def _args(name, **sizes):
    params = _params(name)
    args = [0] * len(params)
    for key, val in sizes.items():
        args[params.index(key)] = val
    return tuple(args)


GEMMS = {
    # entry point: (sizes, algorithmic flops)
    "fu_linear": (dict(M=1000, N=384, K=640), 2 * 1000 * 384 * 640),
    "fu_linear_batched": (dict(M=1000, N=128, K=256, batch=5), 2 * 5 * 1000 * 128 * 256),
    "fu_linear_gate": (dict(M=1000, C=128, K=768, lmax=2), 2 * 1000 * 640 * 768),
    "fu_linear_gate_bwd": (dict(M=1000, C=128, K=384, lmax=2), 2 * 1000 * 384 * 384),
    "fu_complex_linear": (dict(M=1000, Nc=256, Kc=512), 6 * 1000 * 256 * 512),
    "fu_complex_linear_gate": (dict(M=1000, Nc=256, Kc=512), 6 * 1000 * 256 * 512),
    "fu_complex_linear_gate_bwd": (dict(M=1000, Nc=128, Kc=256), 6 * 1000 * 128 * 256),
    "fu_linear_ln_silu": (dict(M=1000, N=128, K=128, batch=5, G=5), 2 * 5 * 1000 * 128 * 128),
    "fu_linear_ln_silu_bwd": (dict(M=1000, N=640, K=64, G=5), 2 * 1000 * 640 * 64),
    "fu_linear_dgrad_ln_silu_bwd": (dict(M=1000, K=1536, G=5, group=2), 2 * 1000 * 128 * 1536),
    "fu_gather_linear_gate": (dict(E=1000, C=128), 2 * 1000 * 640 * 768),
}


@pytest.mark.parametrize("name", sorted(GEMMS))
def test_gemm_work_reads_the_size_arguments(name):
    import roofline
    sizes, flops = GEMMS[name]
    nbytes, got = roofline.WORK[name](_args(name, **sizes))
    assert got == flops
    assert nbytes > 0


def test_every_work_function_names_a_declared_entry_point():
    import roofline
    text = open(HEADER).read()
    for name in roofline.WORK:
        assert re.search(r"\b" + name + r"\s*\(", text), name


def test_split_mode_accounting():
    import roofline
    args = _args("fu_linear", M=1000, N=384, K=640)
    flops = 2 * 1000 * 384 * 640
    ms = 1.0
    split = roofline.summarize([("fu_linear", args, ms)], roofline.MATMUL_SPLIT_BF16)["fu_linear"]
    fp32 = roofline.summarize([("fu_linear", args, ms)], roofline.MATMUL_FP32)["fu_linear"]
    f16 = roofline.summarize([("fu_linear", args, ms)], roofline.MATMUL_SPLIT_F16)["fu_linear"]
    rate = flops / 1e-3 / 1e12
    assert fp32["peak"] == 157.3 and abs(fp32["achieved"] - rate) < 0.01
    assert split["peak"] == 2500.0 and abs(split["achieved"] - 6 * rate) < 0.05
    assert f16["peak"] == 2500.0 and abs(f16["achieved"] - 3 * rate) < 0.05 and "fp16" in f16["matrix_op"]
    assert abs(split["fp32_tflops"] - rate) < 0.01 and abs(f16["fp32_tflops"] - rate) < 0.01
    # the gathered conv1 loader keeps the bf16 split in both split modes
    g = _args("fu_gather_linear_gate", E=1000, C=128)
    gf = roofline.summarize([("fu_gather_linear_gate", g, ms)], roofline.MATMUL_SPLIT_F16)["fu_gather_linear_gate"]
    assert "bf16" in gf["matrix_op"]


def test_roofline_frac_takes_the_larger_of_the_two_bounds():
    """roofline_frac = sum over launches of max(executed flops / matrix peak, bytes / HBM peak)
    over the measured time: equal to frac for a high-intensity GEMM, larger where the launch
    sits under the HBM slope (K = 128 with as many output columns as input)."""
    import roofline
    big = _args("fu_linear", M=245760, N=640, K=768)
    small = _args("fu_linear_batched", M=245760, N=128, K=128, batch=5)
    ms = 1.0
    r = roofline.summarize([("fu_linear", big, ms)])["fu_linear"]
    assert r["hbm_bound_launches"] == 0 and abs(r["roofline_frac"] - r["frac"]) < 1e-3
    nbytes, flops = roofline.WORK["fu_linear_batched"](small)
    t_hbm = nbytes / (roofline.HBM_PEAK_GBS * 1e9)
    t_mfma = 6 * flops / (roofline.BF16_MFMA_PEAK_TFLOPS * 1e12)
    assert t_hbm > t_mfma
    r = roofline.summarize([("fu_linear_batched", small, ms)])["fu_linear_batched"]
    assert r["hbm_bound_launches"] == 1 and abs(r["roofline_frac"] - t_hbm / 1e-3) < 1e-3


@pytest.mark.parametrize("name,sizes,per_edge", [
    ("fu_scatter_bwd", dict(E=1000, N=50, C=128), (34 + 1) * 4),
    ("fu_init_scatter_bwd", dict(E=1000, N=50, C=128), (8 + 1) * 4),
    ("fu_gather_bwd", dict(E=1000, N=50, C=128), 34 * 4),
])
def test_accumulating_calls_count_the_read_back(name, sizes, per_edge):
    import roofline
    b0, _ = roofline.WORK[name](_args(name, **sizes, accumulate=0))
    b3, _ = roofline.WORK[name](_args(name, **sizes, accumulate=3))
    assert b3 - b0 == sizes["E"] * per_edge
