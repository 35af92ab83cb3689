"""Summaries of rocprofv3 CSV output as the Markdown tables kept under profiles/.

Every table there is rebuilt by one of these commands from the CSV files of the rocprofv3
command named in its header (run from the repository root on one MI355X):

  timed   per-kernel time over the timed steps of a bench.py kernel trace
          (--trace <dir>/<name>_kernel_trace.csv --warmup W --steps S)
  pmc     HBM bytes per launch from two counter passes, FETCH_SIZE and WRITE_SIZE, each run
          with --kernel-trace, scaled by what the counters read for the plain 256 MiB copy
          that bench.py --pmc-calibration dispatches first; also writes profiles/pmc_traffic.json
  sq      MFMA-pipe occupancy and LDS bank conflicts per launch from one SQ counter pass

Kernels are mapped to the C-ABI entry point that launches them (KERNEL_ENTRY, kernel_entry);
fu_linear and fu_linear_batched share one kernel instance and are told apart by the launch's
grid (a batched launch has grid y > 1), which the kernel trace records.
"""
from __future__ import annotations

import argparse
import collections
import csv
import json
import os

# kernel (namespace-stripped name, template arguments removed) -> entry point
KERNEL_ENTRY = {
    "geom_fwd_kernel": "fu_geom_fwd", "geom_bwd_kernel": "fu_geom_bwd", "edge_vec_reduce_kernel": "fu_edge_vec_reduce",
    "gather_fwd_kernel": "fu_gather_fwd", "gather_fwd_pair_kernel": "fu_gather_fwd",
    "gather_bwd_kernel": "fu_gather_bwd", "add_inplace_kernel": "fu_gather_bwd(add)",
    "gating_fwd_kernel": "fu_gating_fwd", "gating_bwd_kernel": "fu_gating_bwd",
    "scatter_fwd_kernel": "fu_scatter_fwd", "scatter_bwd_kernel": "fu_scatter_bwd",
    "init_scatter_fwd_kernel": "fu_init_scatter_fwd", "init_scatter_bwd_kernel": "fu_init_scatter_bwd",
    "ln_silu_fwd_kernel": "fu_ln_silu_grouped_fwd", "ln_silu_bwd_kernel": "fu_ln_silu_grouped_bwd",
    "complex_weight_scale_kernel": "fu_complex_weight_split", "complex_weight_split_kernel": "fu_complex_weight_split",
    "resident_weight_scale_kernel": "fu_linear_weight_split", "resident_weight_summary_kernel": "fu_linear_weight_split",
    "resident_weight_split_kernel": "fu_linear_weight_split", "linear_resident_kernel": "fu_linear_resident",
    "radial_gather_kernel": "fu_radial_gather_fwd", "radial_gather_lmax_kernel": "fu_radial_gather_fwd_lmax",
    "rms_norm_fwd_kernel": "fu_rms_norm_sh_fwd", "rms_norm_bwd_kernel": "fu_rms_norm_sh_bwd",
    "gate_fwd_kernel": "fu_gate_act_fwd", "gate_bwd_kernel": "fu_gate_act_bwd",
    "gather_rows_kernel": "fu_gather_rows", "scatter_rows_kernel": "fu_scatter_rows",
    "edge_shifts_kernel": "fu_edge_shifts", "outer_sum3_stage1": "fu_outer_sum3", "outer_sum3_stage2": "fu_outer_sum3",
    "balance_sums_kernel": "fu_balance_channels", "balance_apply_kernel": "fu_balance_channels",
    "morton_keys_kernel": "fu_morton_keys", "invert_perm_kernel": "fu_invert_perm", "take_i64_kernel": "fu_take_i64",
    "csr_row_ptr_kernel": "fu_csr_row_ptr", "narrow_kernel": "fu_narrow_i64_i32",
    "nlist_bin_kernel": "fu_nlist_bin", "nlist_search_kernel": "fu_nlist_search", "nlist_scan_kernel": "fu_nlist_scan",
    "nlist_emit_kernel": "fu_nlist_emit",
    "wigner_ext_fwd_kernel": "fu_wigner_ext_fwd", "wigner_ext_bwd_kernel": "fu_wigner_ext_bwd",
    "gather_fwd_lmax_kernel": "fu_gather_fwd_lmax", "gather_fwd_node_lmax_kernel": "fu_gather_fwd_lmax",
    "gather_bwd_lmax_kernel": "fu_gather_bwd_lmax",
    "add_rows_kernel": "fu_gather_bwd_lmax(add)",
    "scatter_fwd_lmax_kernel": "fu_scatter_fwd_lmax", "scatter_bwd_lmax_kernel": "fu_scatter_bwd_lmax",
    "init_scatter_fwd_lmax_kernel": "fu_init_scatter_fwd_lmax", "init_scatter_bwd_lmax_kernel": "fu_init_scatter_bwd_lmax",
    "gating_fwd_lmax_kernel": "fu_gating_fwd_lmax", "gating_bwd_lmax_kernel": "fu_gating_bwd_lmax",
}
# linear_mfma_kernel<MODE, SPLIT, KTAIL, TALL, GATHER, F16>: MODE -> entry point (MODE 1 with
# GATHER: fu_gather_linear_gate); complex_linear_kernel<MODE, PATH, KTAIL>
LINEAR_MODE = {"0": "fu_linear", "1": "fu_linear_gate", "2": "fu_linear_gate_bwd", "3": "fu_linear_ln_silu",
               "4": "fu_linear_ln_silu_bwd", "5": "fu_linear_dgrad_ln_silu_bwd"}
COMPLEX_MODE = {"0": "fu_complex_linear", "1": "fu_complex_linear_gate", "2": "fu_complex_linear_gate_bwd"}


def short_name(kernel_name: str) -> str:
    """The kernel's name without its argument list and leading 'void '."""
    return kernel_name.split("(")[0].replace("void ", "").strip()


def kernel_entry(kernel_name: str, grid_y: int = 1) -> str | None:
    """Entry point that launched a kernel (None for kernels that are not the library's)."""
    head = short_name(kernel_name)
    base = head.split("<")[0].split("::")[-1]
    targs = [t.strip() for t in head.split("<", 1)[1].rstrip(">").split(",")] if "<" in head else []
    if base == "linear_mfma_kernel":
        if len(targs) > 4 and targs[4] == "true" and targs[0] == "1":
            return "fu_gather_linear_gate"
        ent = LINEAR_MODE.get(targs[0] if targs else "0", "fu_linear")
        if ent == "fu_linear" and grid_y > 1:
            return "fu_linear_batched"
        return ent
    if base == "complex_linear_kernel":
        return COMPLEX_MODE.get(targs[0] if targs else "0")
    return KERNEL_ENTRY.get(base)


def _read(path: str) -> list[dict]:
    with open(path) as f:
        return list(csv.DictReader(f))


def _grid_y(row: dict) -> int:
    return int(row.get("Grid_Size_Y", 1) or 1)


def _steps(rows: list[dict], marker: str = "geom_fwd_kernel") -> list[int]:
    return [i for i, r in enumerate(rows) if marker in r["Kernel_Name"]]


def _streams(rows: list[dict]) -> int:
    return len({r.get("Stream_Id", "0") for r in rows})


def timed(trace: str, warmup: int, steps: int, title: str, command: str, out: str, top: int = 40,
          which: str = "timed") -> None:
    """Kernel time per step over the timed steps of a kernel trace: a step starts at its
    geom_fwd_kernel dispatch, the first `warmup` steps are left out.  which="profiled": the
    trace also holds bench.py's per-kernel profiling pass (the same number of steps after the
    timed ones, every call on one stream with the HIP-event profiler on); the table is built
    from that pass, whose kernel durations are those of bench.py's roofline figures, and the
    header gives the timed pass's wall time beside it."""
    rows = sorted(_read(trace), key=lambda r: int(r["Start_Timestamp"]))
    starts = _steps(rows)
    n_pass = 2 if which == "profiled" else 1
    if len(starts) != warmup + n_pass * steps:
        raise SystemExit(f"{trace}: {len(starts)} steps found, expected {warmup} + {n_pass} x {steps}")
    timed_rows = rows[starts[warmup]:starts[warmup + steps]] if n_pass == 2 else rows[starts[warmup]:]
    sel = rows[starts[warmup + steps]:] if n_pass == 2 else timed_rows
    w0, w1 = int(timed_rows[0]["Start_Timestamp"]), max(int(r["End_Timestamp"]) for r in timed_rows)
    t0, t1 = int(sel[0]["Start_Timestamp"]), max(int(r["End_Timestamp"]) for r in sel)
    agg = collections.defaultdict(lambda: [0, 0])
    for r in sel:
        key = (short_name(r["Kernel_Name"])[:90], kernel_entry(r["Kernel_Name"], _grid_y(r)))
        agg[key][0] += 1
        agg[key][1] += int(r["End_Timestamp"]) - int(r["Start_Timestamp"])
    tot = sum(v[1] for v in agg.values())
    lines = [f"# Kernel time per step — {title}", "", "Command (run from the repository root on one MI355X):", "",
             "```", command, "```", ""]
    if n_pass == 1:
        nst = _streams(sel)
        lines += [f"rocprofv3 kernel trace, the {steps} timed steps only (each step starts at its `geom_fwd_kernel` "
                  f"dispatch; the {warmup} warm-up steps are left out). Kernel time {tot / 1e6 / steps:.2f} ms/step; "
                  f"first dispatch to last completion {(t1 - t0) / 1e6 / steps:.2f} ms/step. Kernels ran on {nst} "
                  f"stream{'s' if nst > 1 else ''}. Summarised by `python flash-uma_amd/profiles_summary.py timed`.",
                  ""]
    else:
        nst = _streams(timed_rows)
        lines += [f"rocprofv3 kernel trace of bench.py's two passes (each step starts at its `geom_fwd_kernel` "
                  f"dispatch; the {warmup} warm-up steps are left out). Timed pass ({steps} steps, kernels on {nst} "
                  f"stream{'s' if nst > 1 else ''}): first dispatch to last completion {(w1 - w0) / 1e6 / steps:.2f} "
                  f"ms/step. The table is the per-kernel profiling pass ({steps} steps, every kernel on one stream, "
                  f"HIP events around each call: the durations behind bench.py's roofline figures): kernel time "
                  f"{tot / 1e6 / steps:.2f} ms/step, first dispatch to last completion "
                  f"{(t1 - t0) / 1e6 / steps:.2f} ms/step. Summarised by "
                  f"`python flash-uma_amd/profiles_summary.py timed --pass profiled`.", ""]
    lines += ["| ms/step | calls/step | avg us | share | kernel | entry point |", "|---:|---:|---:|---:|---|---|"]
    for (nm, ent), (n, t) in sorted(agg.items(), key=lambda kv: -kv[1][1])[:top]:
        lines.append(f"| {t / 1e6 / steps:.3f} | {n / steps:.1f} | {t / n / 1e3:.1f} | {100 * t / tot:.1f}% | `{nm}` | "
                     f"{ent or '(torch / rocBLAS)'} |")
    by_entry = collections.defaultdict(lambda: [0, 0])
    for (nm, ent), (n, t) in agg.items():
        if ent:
            by_entry[ent][0] += n
            by_entry[ent][1] += t
    lines += ["", "Per entry point (every kernel it launches):", "",
              "| entry point | calls/step | avg us | ms/step |", "|---|---:|---:|---:|"]
    for ent, (n, t) in sorted(by_entry.items(), key=lambda kv: -kv[1][1]):
        lines.append(f"| {ent} | {n / steps:.1f} | {t / n / 1e3:.1f} | {t / 1e6 / steps:.3f} |")
    _write(out, lines)


def _joined(counters: str, trace: str) -> list[tuple[dict, int]]:
    """Counter rows with the grid y of the same dispatch from the run's kernel trace."""
    gy = {r["Dispatch_Id"]: _grid_y(r) for r in _read(trace)}
    return [(r, gy.get(r["Dispatch_Id"], 1)) for r in _read(counters)]


def _calibration(rows: list[tuple[dict, int]]) -> float:
    """Counter value (KiB) of the 256 MiB copy kernel bench.py --pmc-calibration dispatches: the
    largest reading among the copy kernels of its grid (model set-up copies smaller buffers with
    the same grid)."""
    vals = [float(r["Counter_Value"]) for r, _ in rows
            if "copyBuffer" in r["Kernel_Name"] and int(r["Grid_Size"]) == 131072]
    if not vals:
        raise SystemExit("no 256 MiB copy kernel in the counter file: run bench.py with --pmc-calibration")
    return max(vals)


def _in_steps(rows: list[tuple[dict, int]]) -> list[tuple[dict, str]]:
    """(row, entry point) of the library's launches from the first step on (set-up launches
    before it are left out)."""
    rows = sorted(rows, key=lambda rg: int(rg[0]["Dispatch_Id"]))
    out, started = [], False
    for r, gy in rows:
        if "geom_fwd_kernel" in r["Kernel_Name"]:
            started = True
        ent = kernel_entry(r["Kernel_Name"], gy)
        if started and ent:
            out.append((r, ent))
    return out


def pmc(fetch: str, fetch_trace: str, write: str, write_trace: str, config: str, cmd_fetch: str, cmd_write: str,
        out: str, out_json: str, commit: str) -> None:
    """HBM traffic per launch: FETCH_SIZE and WRITE_SIZE (KiB per dispatch) scaled by the
    copy kernel's reading of 256 MiB read and 256 MiB written."""
    f, w = _joined(fetch, fetch_trace), _joined(write, write_trace)
    sf, sw = 262144.0 / _calibration(f), 262144.0 / _calibration(w)
    agg = collections.defaultdict(lambda: [0, 0.0, 0.0])
    for r, e in _in_steps(f):
        agg[e][0] += 1
        agg[e][1] += float(r["Counter_Value"]) * sf * 1024
    for r, e in _in_steps(w):
        agg[e][2] += float(r["Counter_Value"]) * sw * 1024
    js = {}
    lines = [f"# HBM traffic per launch — {config}", "", "Two counter passes (one counter group each):", "", "```",
             cmd_fetch, cmd_write, "```", "",
             f"Scale factors from the plain 256 MiB copy kernel dispatched by `--pmc-calibration` (262144 KiB read "
             f"and written): FETCH_SIZE x{sf:.4f}, WRITE_SIZE x{sw:.4f}. Launches of the warm-up and the timed step "
             f"are averaged; measured at commit {commit}. Summarised by "
             "`python flash-uma_amd/profiles_summary.py pmc`.", "",
             "| entry point | launches | fetch MB/launch | write MB/launch | traffic MB/launch |",
             "|---|---:|---:|---:|---:|"]
    for e, (n, fb, wb) in sorted(agg.items(), key=lambda kv: -(kv[1][1] + kv[1][2])):
        t = (fb + wb) / n
        js[e] = round(t)
        lines.append(f"| `{e}` | {n} | {fb / n / 1e6:.1f} | {wb / n / 1e6:.1f} | {t / 1e6:.1f} |")
    _write(out, lines)
    old = {}
    if os.path.exists(out_json):
        with open(out_json) as fh:
            old = json.load(fh)
    old[config] = js
    old["measured_at"] = commit
    with open(out_json, "w") as fh:
        json.dump(old, fh, indent=1)
        fh.write("\n")


def sq(counters: str, trace: str, title: str, command: str, out: str) -> None:
    """MFMA busy = SQ_VALU_MFMA_BUSY_CYCLES / (128 SIMDs x GRBM_GUI_ACTIVE): GRBM_GUI_ACTIVE sums
    the active cycles of the 8 XCDs of 128 SIMDs each.  LDS conflict = SQ_LDS_BANK_CONFLICT
    cycles per SQ_INSTS_LDS instruction."""
    gy = {r["Dispatch_Id"]: _grid_y(r) for r in _read(trace)}
    by = collections.defaultdict(dict)
    name = {}
    for r in _read(counters):
        d = int(r["Dispatch_Id"])
        by[d][r["Counter_Name"]] = float(r["Counter_Value"])
        name[d] = r["Kernel_Name"]
    agg = collections.defaultdict(lambda: collections.defaultdict(float))
    started = False
    for d in sorted(by):
        nm = name[d]
        if "geom_fwd_kernel" in nm:
            started = True
        e = kernel_entry(nm, gy.get(str(d), 1))
        if not started or e is None:
            continue
        key = (e, short_name(nm)[:70])
        agg[key]["n"] += 1
        for c, v in by[d].items():
            agg[key][c] += v
    lines = [f"# Matrix-core occupancy and LDS bank conflicts per launch — {title}", "", "Command:", "", "```",
             command, "```", "",
             "MFMA busy = SQ_VALU_MFMA_BUSY_CYCLES / (128 SIMDs x GRBM_GUI_ACTIVE), where GRBM_GUI_ACTIVE sums the "
             "active cycles of the 8 XCDs; SQ_VALU_MFMA_BUSY_CYCLES counts 32 cycles per v_mfma_f32_32x32x16_bf16 or "
             "_f16 issued. LDS conflict = SQ_LDS_BANK_CONFLICT cycles per SQ_INSTS_LDS instruction. Clock = "
             "GRBM_GUI_ACTIVE / 8 XCDs / kernel duration. The warm-up and the timed step are both included. "
             "Summarised by `python flash-uma_amd/profiles_summary.py sq`.", "",
             "| entry point | kernel | launches | MFMA busy | LDS conflict cycles / LDS instr | waves / launch | "
             "clock GHz |", "|---|---|---:|---:|---:|---:|---:|"]
    dur = {}
    for r in _read(trace):
        dur[r["Dispatch_Id"]] = int(r["End_Timestamp"]) - int(r["Start_Timestamp"])
    clk = collections.defaultdict(lambda: [0.0, 0.0])
    for d in by:
        e = kernel_entry(name[d], gy.get(str(d), 1))
        if e and str(d) in dur:
            k = (e, short_name(name[d])[:70])
            clk[k][0] += by[d].get("GRBM_GUI_ACTIVE", 0.0) / 8
            clk[k][1] += dur[str(d)]
    for (e, nm), a in sorted(agg.items(), key=lambda kv: -kv[1]["SQ_VALU_MFMA_BUSY_CYCLES"]):
        if a["SQ_VALU_MFMA_BUSY_CYCLES"] == 0:
            continue
        busy = a["SQ_VALU_MFMA_BUSY_CYCLES"] / (128 * a["GRBM_GUI_ACTIVE"])
        conf = a["SQ_LDS_BANK_CONFLICT"] / max(a["SQ_INSTS_LDS"], 1)
        cy, ns = clk[(e, nm)]
        ghz = cy / ns if ns else float("nan")
        lines.append(f"| `{e}` | `{nm}` | {int(a['n'])} | {busy:.3f} | {conf:.3f} | {a['SQ_WAVES'] / a['n']:.0f} | "
                     f"{ghz:.2f} |")
    _write(out, lines)


def _write(path: str, lines: list[str]) -> None:
    with open(path, "w") as f:
        f.write("\n".join(lines) + "\n")


def main(argv=None) -> None:
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    sub = ap.add_subparsers(dest="cmd", required=True)
    t = sub.add_parser("timed")
    t.add_argument("--trace", required=True)
    t.add_argument("--warmup", type=int, required=True)
    t.add_argument("--steps", type=int, required=True)
    t.add_argument("--title", required=True)
    t.add_argument("--command", required=True)
    t.add_argument("--out", required=True)
    t.add_argument("--pass", dest="which", choices=("timed", "profiled"), default="timed")
    p = sub.add_parser("pmc")
    for k in ("fetch", "fetch-trace", "write", "write-trace", "config", "cmd-fetch", "cmd-write", "out", "commit"):
        p.add_argument(f"--{k}", required=True)
    p.add_argument("--json", default=os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))),
                                                  "profiles", "pmc_traffic.json"))
    q = sub.add_parser("sq")
    for k in ("counters", "trace", "title", "command", "out"):
        q.add_argument(f"--{k}", required=True)
    a = ap.parse_args(argv)
    if a.cmd == "timed":
        timed(a.trace, a.warmup, a.steps, a.title, a.command, a.out, which=a.which)
    elif a.cmd == "pmc":
        pmc(a.fetch, a.fetch_trace, a.write, a.write_trace, a.config, a.cmd_fetch, a.cmd_write, a.out, a.json,
            a.commit)
    else:
        sq(a.counters, a.trace, a.title, a.command, a.out)


if __name__ == "__main__":
    main()
