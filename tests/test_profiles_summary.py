"""profiles_summary.py: every kernel of the library maps to the C-ABI entry point that launches
it, and the summaries are rebuilt from rocprofv3-shaped CSV files (CPU only)."""
import csv
import os
import re

import profiles_summary as ps

CSRC = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "flash-uma_amd", "csrc")


def _kernels():
    names = set()
    for f in os.listdir(CSRC):
        if f.endswith(".hip"):
            src = open(os.path.join(CSRC, f)).read()
            names |= set(re.findall(r"__global__[^;{]*?\bvoid\s+(\w+)\s*\(", src, re.S))
    return names


def test_every_kernel_has_an_entry_point():
    names = _kernels()
    assert len(names) > 40
    missing = sorted(n for n in names if n not in ("linear_mfma_kernel", "complex_linear_kernel")
                     and n not in ps.KERNEL_ENTRY)
    assert not missing, missing


def test_template_instances_map_to_their_entry_points():
    e = ps.kernel_entry
    assert e("void fu::linear_mfma_kernel<0, true, false, true, false, true>(float const*)") == "fu_linear"
    assert e("void fu::linear_mfma_kernel<0, true, false, true, false, true>(float const*)", 3) == "fu_linear_batched"
    assert e("void fu::linear_mfma_kernel<1, true, false, true, true, false>(x)") == "fu_gather_linear_gate"
    assert e("void fu::linear_mfma_kernel<1, true, false, true, false, true>(x)") == "fu_linear_gate"
    assert e("void fu::linear_mfma_kernel<5, true, false, true, false, true>(x)") == "fu_linear_dgrad_ln_silu_bwd"
    assert e("void fu::complex_linear_kernel<2, 3, false>(x)") == "fu_complex_linear_gate_bwd"
    assert e("void fu::gather_fwd_pair_kernel<1, true>(float const*)") == "fu_gather_fwd"
    assert e("void fu::lm::gather_bwd_lmax_kernel<2, 4>(x)") == "fu_gather_bwd_lmax"
    assert e("void at::native::vectorized_elementwise_kernel<4>(x)") is None


def _trace(path, rows):
    keys = ["Dispatch_Id", "Kernel_Name", "Start_Timestamp", "End_Timestamp", "Grid_Size_Y", "Stream_Id"][:len(rows[0])]
    with open(path, "w", newline="") as f:
        w = csv.DictWriter(f, keys)
        w.writeheader()
        for r in rows:
            w.writerow(dict(zip(keys, r)))


def test_timed_table_from_a_trace(tmp_path):
    rows, t = [], 0
    for step in range(3):   # one warm-up, two timed steps
        for name, us, gy in (("void fu::geom_fwd_kernel(x)", 40, 1),
                             ("void fu::linear_mfma_kernel<0, true, false, true, false, true>(x)", 500, 1),
                             ("void fu::linear_mfma_kernel<0, true, false, true, false, true>(x)", 30, 4)):
            rows.append((len(rows), name, t, t + us * 1000, gy))
            t += us * 1000 + 1000
    tr = tmp_path / "t.csv"
    _trace(tr, rows)
    out = tmp_path / "t.md"
    ps.timed(str(tr), 1, 2, "test", "cmd", str(out))
    text = out.read_text()
    assert "| fu_linear | 1.0 | 500.0 | 0.500 |" in text
    assert "| fu_linear_batched | 1.0 | 30.0 | 0.030 |" in text
    assert "Kernel time 0.57 ms/step" in text


def test_profiled_pass_table_from_a_trace(tmp_path):
    """--pass profiled: the table comes from the steps after the timed ones (bench.py's per-kernel
    profiling pass, one stream); the header gives the timed pass's wall time and stream count."""
    rows, t = [], 0
    for step in range(5):   # one warm-up, two timed steps on two streams, two profiled steps on one
        timed_pass = 1 <= step <= 2
        for name, us, gy, sid in (("void fu::geom_fwd_kernel(x)", 40, 1, 0),
                                  ("void fu::complex_linear_kernel<0, 3, false>(x)", 400 if timed_pass else 420, 1, 0),
                                  ("void fu::complex_linear_kernel<0, 3, false>(x)", 150, 1, 1 if timed_pass else 0)):
            rows.append((len(rows), name, t, t + us * 1000, gy, sid))
            t += us * 1000 + 1000
    tr = tmp_path / "t.csv"
    _trace(tr, rows)
    out = tmp_path / "t.md"
    ps.timed(str(tr), 1, 2, "test", "cmd", str(out), which="profiled")
    text = out.read_text()
    assert "| fu_complex_linear | 2.0 | 285.0 | 0.570 |" in text
    assert "kernels on 2 streams" in text
    assert "first dispatch to last completion 0.59 ms/step. The table" in text
