"""Benchmark of the FlashUMA ZeroAllocBackbone hot path on one MI355X.

A step is one energy + forces + stress evaluation (backbone forward through the HIP kernels,
energy head, autograd backward to positions and cell) of the headline workload: bcc Fe
16x16x16 conventional cells (8,192 atoms, 245,760 edges, cutoff 6 A, max 30 neighbours),
UMA-s-shaped random-init weights (lmax = mmax = 2, 4 layers, C = 128, 64 Gaussians), fp32.
The graph is built once on the host and its topology is cached (as across MD steps);
all inputs are resident in HBM before the timed region.

Prints one JSON line: atom-steps/s, ms/step, the roofline of the dominant kernel measured
with HIP events on the launch stream during the timed steps, a per-kernel breakdown and the
CPU baseline (the float32 torch-CPU oracle on a bounded sample of the same workload).

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--config bcc_fe] [--no-cpu-baseline]

--config bcc_fe_lmax4 runs the lmax-4 workload instead (same input, lmax = 4, 8 layers, E+F).
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
PKG = os.path.join(ROOT, "flash-uma_amd")
sys.path[:0] = [ROOT, PKG]

METRIC = "atom-steps/sec (energy+forces) on 1 MI355X; % HBM roofline per kernel"
MATMUL_TEXT = {
    0: "fp32 operands split exactly into three bf16 planes, six bf16 MFMA products, fp32 accumulation",
    1: "fp32 MFMA",
    2: "fp32 operands scaled by per-row powers of two and split into two fp16 planes, three fp16 MFMA "
       "products, fp32 accumulation; tiles whose rows leave the fp16 window rerun at exact scales (two "
       "loops when needed); row-norm-relative error against float64 within 1.1x (rms) / 1.5x (max) of "
       "the fp32 MFMA's on the tested shapes, including anti-correlated operand ramps up to 2^+-12 "
       "(tests/test_gpu_ops.py::test_split_gemm_accuracy, test_f16_split_anticorrelated_range, "
       "test_f16_complex_anticorrelated_range)",
}


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


# backbone shape per workload: the UMA-s-shaped headline model, and the lmax-4 workload
# (lmax = 4, 8 layers, E+F) on the same bcc Fe input
MODELS = {"bcc_fe_lmax4": dict(lmax=4, num_layers=8)}


def make_system(config: str):
    import systems
    if config == "bcc_fe":
        return systems.bcc_fe(n_rep=16), True, "bcc_fe_16x16x16"
    if config == "bcc_fe_lmax4":
        return systems.bcc_fe(n_rep=16), False, "bcc_fe_16x16x16_lmax4"
    if config == "water_box":
        return systems.water_box(), False, "water_box_333"
    if config == "amorphous":
        return systems.amorphous(), False, "amorphous_50k"
    if config == "cu_slab_co":
        return systems.cu_slab_co(), False, "cu_slab_co"
    if config in ("sweep_1000x30", "sweep_2000x50"):
        # the reference's own sweep workloads (examples/sweep.py:33-81, E+F+S), explicit edges
        n, deg = (int(v) for v in config.split("_")[1].split("x"))
        system, ei, off = systems.sweep_graph(n, deg)
        system.info["edges"] = (ei, off)
        return system, True, f"random_{n}_atoms_{deg}_edges_per_atom"
    raise SystemExit(f"unknown config {config}")


def cpu_baseline(budget_s: float = 30.0, model_kw: dict | None = None, stress: bool = True, n_rep: int = 16,
                 min_steps: int = 3) -> dict:
    """float32 torch-CPU oracle (reference-algorithm restatement) on a bcc Fe n_rep^3 cell, E+F+S:
    by default the headline cell itself (8,192 atoms, ~35 s per step on 16 EPYC cores, ~70 GB of
    host memory), the median of min_steps steps (more, up to 5, while within budget_s) after a
    warm-up on a 4^3 cell.
    The oracle's cost per atom grows with the cell (its eager element-wise passes leave the
    caches: 16 cores ran 128 atoms at 520-590 atom-steps/s, 432 at 364, 1,024 at 273 and 3,456 at
    241), so a small cell would overstate it.  With less free host memory than the cell needs,
    the largest of 12^3 / 8^3 that fits is timed instead (the sample field says which)."""
    import torch
    import escn_md
    import heads
    import systems
    from oracle.model_ref import energy_forces_stress

    # the threads of the host share this process may use: the harness states it in
    # OMP_NUM_THREADS (16 per GPU on the MI355X boxes, whatever the affinity mask shows);
    # without it, every core of the affinity mask
    affinity = len(os.sched_getaffinity(0))
    cores = min(affinity, int(os.environ.get("OMP_NUM_THREADS", affinity)))
    torch.set_num_threads(cores)
    try:
        import psutil
        avail = psutil.virtual_memory().available
    except ImportError:
        avail = float("inf")
    # ~9 MB of host memory per atom at lmax 2 (measured: 10.2 GB at 1,024 atoms, 29.6 at 3,456)
    per_atom = 9e6 * (1 if not model_kw else 6)
    for cand in (n_rep, 12, 8, 6, 4):
        if cand <= n_rep and 2 * cand ** 3 * per_atom * 1.5 <= avail:
            n_rep = cand
            break
    else:
        n_rep = 4
    bb = escn_md.eSCNMDBackbone(seed=0, **(model_kw or {}))
    hd = heads.MLPEnergyHead(bb.sphere_channels, bb.hidden_channels, seed=1)
    w = systems.bcc_fe(n_rep=4)
    wei, woff = systems.neighbor_list(w.pos, w.cell, w.pbc, bb.cutoff, bb.max_neighbors)
    energy_forces_stress(bb, hd, w.pos, w.Z, w.cell, wei, woff, dtype=torch.float32, stress=stress)   # warm-up
    s = systems.bcc_fe(n_rep=n_rep)
    ei, off = systems.neighbor_list(s.pos, s.cell, s.pbc, bb.cutoff, bb.max_neighbors)
    # the median of at least min_steps steps (more, up to 5, while within budget_s)
    times = []
    t_start = time.perf_counter()
    while len(times) < 5 and (len(times) < min_steps or time.perf_counter() - t_start < budget_s):
        t0 = time.perf_counter()
        energy_forces_stress(bb, hd, s.pos, s.Z, s.cell, ei, off, dtype=torch.float32, stress=stress)
        times.append(time.perf_counter() - t0)
        log(f"[bench] CPU baseline step {len(times)}: {times[-1]:.1f} s")
    times.sort()
    med = times[len(times) // 2]
    model = "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {"value": round(s.n_atoms / med, 2), "unit": "atom-steps/s", "cores": cores, "kind": "port",
            "sample": f"bcc Fe {n_rep}x{n_rep}x{n_rep} ({s.n_atoms} atoms, {ei.shape[1]} edges), "
                      f"{'E+F+S' if stress else 'E+F'}, "
                      f"lmax={bb.lmax}, {bb.num_layers} layers, float32 torch-CPU oracle "
                      f"(oracle/model_ref.py), median of {len(times)} step(s) after a 4x4x4 warm-up; CPU: {model}"}


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--config", default="bcc_fe")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-kernel-profile", action="store_true")
    ap.add_argument("--graph", action="store_true",
                    help="time the step captured once in a HIP graph and replayed (captured.py); "
                         "the per-kernel profile is not available then")
    ap.add_argument("--matmul", choices=["split_f16", "split_bf16", "fp32"], default="split_f16",
                    help="matrix-core mode of the fp32 contractions: power-of-two row scales with a two-way "
                         "fp16 split and three fp16 MFMA products (default), exact three-way bf16 split with "
                         "six bf16 MFMA products, or fp32 MFMA; fp32 accumulation in all three")
    ap.add_argument("--pmc-calibration", action="store_true",
                    help="first copy a 256 MiB buffer (a plain copy kernel of known size, the scale "
                         "reference for rocprofv3 FETCH_SIZE / WRITE_SIZE counters)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (this build has no multi-GPU path); got --gpus {args.gpus}",
              file=sys.stderr)
        raise SystemExit(2)

    import numpy as np
    import torch
    import escn_md
    import heads
    import roofline
    import systems
    from ops import _lib
    from wrapper import ZeroAllocBackbone

    dev = torch.device("cuda:0")
    _lib.load()
    mm_mode = _lib.MATMUL_MODES[args.matmul]
    _lib.set_matmul_mode(mm_mode)
    system, with_stress, wl_name = make_system(args.config)
    model_kw = MODELS.get(args.config, {})
    bb = escn_md.eSCNMDBackbone(seed=0, **model_kw)
    hd = heads.MLPEnergyHead(bb.sphere_channels, bb.hidden_channels, seed=1)
    t0 = time.perf_counter()
    if "edges" in system.info:
        ei, off = system.info["edges"]
    else:
        ei, off = systems.neighbor_list(system.pos, system.cell, system.pbc, bb.cutoff, bb.max_neighbors)
    log(f"[bench] {wl_name}: {system.n_atoms} atoms, {ei.shape[1]} edges (graph {time.perf_counter() - t0:.1f}s)")
    model = heads.PotentialModel(ZeroAllocBackbone(bb.to(dev)), hd.to(dev))
    data = heads.make_atomic_data(system, ei, off, dev)

    if args.pmc_calibration:
        src_buf = torch.ones(64 * 1024 * 1024, device=dev)
        dst_buf = torch.empty_like(src_buf)
        dst_buf.copy_(src_buf)
        torch.cuda.synchronize()
        del src_buf, dst_buf

    def step():
        return model(data, compute_forces=True, compute_stress=with_stress)

    if args.graph:
        from captured import CapturedStep
        cap = CapturedStep(model, data, compute_stress=with_stress)
        pos0 = data.pos.detach().clone()
        args.no_kernel_profile = True

        def step():   # noqa: F811 -- one replay of the whole E+F(+S) step on the same inputs
            return cap(pos0)

    for k in range(args.warmup):
        out = step()
        torch.cuda.synchronize()
        log(f"[bench] warm-up {k + 1}/{args.warmup}: E = {out['energy'].item():.6f}")
    # the timed steps run without instrumentation; the per-kernel roofline comes from a
    # separate pass over the same number of steps with HIP events around every library call
    torch.cuda.synchronize()
    torch.cuda.reset_peak_memory_stats(dev)
    t0 = time.perf_counter()
    for _ in range(args.steps):
        out = step()
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    peak_mib = torch.cuda.max_memory_allocated(dev) / 2**20
    ms = 1e3 * elapsed / args.steps
    value = system.n_atoms / (elapsed / args.steps)
    log(f"[bench] timed {args.steps} steps: {ms:.3f} ms/step, {value:.1f} atom-steps/s")
    prof = None
    if not args.no_kernel_profile:
        prof = _lib.KernelProfiler()
        _lib.set_profiler(prof)
        for _ in range(args.steps):
            step()
        torch.cuda.synchronize()
        _lib.set_profiler(None)
        log(f"[bench] profiled {args.steps} more steps for the per-kernel roofline")

    kernels = roofline.summarize(prof.durations(), mm_mode) if prof else {}
    for rec in kernels.values():
        rec["ms_per_step"] = round(rec["total_ms"] / args.steps, 4)
    rl = None
    if kernels:
        dom = max(kernels, key=lambda k: kernels[k]["total_ms"])
        d = kernels[dom]
        rl = {"kernel": dom, "bound": d["bound"], "achieved": d["achieved"], "peak": d["peak"], "unit": d["unit"],
              "frac": d["frac"], "traffic": None}
        if "matrix_op" in d:
            rl.update(matrix_op=d["matrix_op"], fp32_tflops=d["fp32_tflops"], roofline_frac=d["roofline_frac"])
        # HBM bytes per launch of the dominant kernel from two rocprofv3 counter passes
        # (FETCH_SIZE, WRITE_SIZE; profiles/<config>_pmc_traffic.md), labelled with the
        # commit they were measured at: counters cannot be read inside this process
        pmc = os.path.join(ROOT, "profiles", "pmc_traffic.json")
        if os.path.exists(pmc):
            with open(pmc) as f:
                js = json.load(f)
            tr = js.get(args.config, {}).get(dom)
            if tr is not None:
                rl["traffic"] = tr
                rl["traffic_source"] = (f"rocprofv3 --pmc FETCH_SIZE / WRITE_SIZE, profiles/{args.config}_pmc_traffic.md, "
                                        f"measured at commit {js.get('measured_at', 'unrecorded')}")

    cpu = None
    if not args.no_cpu_baseline:
        log("[bench] CPU baseline (float32 torch-CPU oracle) ...")
        # lmax 4 with 8 layers costs ~10x more per atom on the CPU: a 6^3 cell there
        cpu = cpu_baseline(model_kw=model_kw, stress=with_stress, n_rep=6 if model_kw else 16)
        log(f"[bench] CPU baseline: {cpu['value']} atom-steps/s on {cpu['cores']} cores")

    rec = {
        "metric": METRIC, "value": round(value, 2), "unit": "atom-steps/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "f32", "data": "synthetic",
        "config": {"workload": f"{wl_name}: {system.n_atoms} atoms, {ei.shape[1]} edges, "
                               f"{'E+F+S' if with_stress else 'E+F'}, UMA-s-shaped random-init eSCN-MD "
                               f"(lmax={bb.lmax}, mmax=2, {bb.num_layers} layers, C=128, B=64, cutoff 6, "
                               + ("every pair within the cutoff, no per-atom cap)" if "edges" in system.info
                                  else "max_neighbors 30)"),
                   "atoms": system.n_atoms, "edges": int(ei.shape[1]), "parallelism": "single GPU",
                   "execution": "hip graph replay" if args.graph else "eager",
                   "matmul": MATMUL_TEXT[mm_mode]},
        "roofline": rl, "cpu_baseline": cpu, "kernels": kernels,
        "peak_memory_mib": round(peak_mib, 1),   # torch allocator peak over the timed steps
        "energy": round(float(out["energy"].item()), 8),
    }
    print(json.dumps(rec), flush=True)


if __name__ == "__main__":
    main()
