"""Write golden vectors from the reference's own op kernels (build container only, CPU).

This script imports the reference's `ops/{geom,gather,gating,scatter,ln_silu}.py` from a
checkout of ArcelliEmanuele/flash-uma (default /root/reference) and runs its Triton kernels
under Triton's CPU interpreter (TRITON_INTERPRET=1) on tiny seeded inputs. It stores the
inputs, the forward outputs and the gradients of the reference's hand-written backward
kernels in tests/golden/ref_ops_fixtures.npz. The fixture is data only: no reference source
travels with it, and this script itself never runs on a GPU box (it is listed in
.gpurunignore; the tests read only the .npz).

What these vectors pin that the mathematics alone does not: which rotated coefficient is
multiplied by which radial block in the gather (ops/gather.py:132-154), which gate scales
which block (ops/gating.py:63-103), where the scatter places each Z block
(ops/scatter.py:104-127) and the init scatter's radial blocks (ops/scatter.py:409-411),
and the hand-derived geometry VJP (ops/geom.py:313-493).

Interpreter adjustments (none changes arithmetic):
* `torch.cuda.synchronize` (called after the autotune warm-ups at ops/geom.py:568 and
  ops/gather.py:472,500) becomes a no-op: there is no device.
* every `triton.autotune` kernel keeps one configuration, chosen below, so the autotuner
  runs nothing extra. Block sizes are chosen smaller than the inputs so masked tails and
  several channel blocks are exercised.

Run from the repository root:  python tests/golden/make_ref_fixtures.py [--reference PATH]
"""
from __future__ import annotations

import argparse
import os
import sys

os.environ["TRITON_INTERPRET"] = "1"

import numpy as np  # noqa: E402
import torch  # noqa: E402

OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "ref_ops_fixtures.npz")

# sizes: N atoms, E edges, C channels, B Gaussians, S systems, M/D for LayerNorm-SiLU
N, E, C, B, S = 14, 45, 64, 8, 2
NUM_Z = 100
CUTOFF = 6.0
LN_SHAPES = ((37, 64), (21, 128))

# one autotune configuration per kernel (meta-parameters only; see module docstring)
CHOICE = {"BLOCK_E": 16, "BLOCK_C": 16, "BLOCK_NB": 16}


def _load_reference(path: str):
    # nothing may be written into the read-only reference tree (no __pycache__ there)
    sys.dont_write_bytecode = True
    sys.path.insert(0, path)
    torch.cuda.synchronize = lambda *a, **k: None
    import triton
    from triton.runtime.autotuner import Autotuner
    from ops import gather, gating, geom, ln_silu, scatter  # reference modules
    mods = dict(geom=geom, gather=gather, gating=gating, scatter=scatter, ln_silu=ln_silu)
    for mod in mods.values():
        for name in dir(mod):
            obj = getattr(mod, name)
            if isinstance(obj, Autotuner):
                keep = [c for c in obj.configs
                        if all(c.kwargs.get(k, v) == v for k, v in CHOICE.items())
                        and c.num_warps == 4 and c.num_stages == 1]
                if not keep:
                    raise RuntimeError(f"no matching autotune config for {name}")
                obj.configs = keep[:1]
    return mods, triton.__version__


def _graph(rng):
    """Random directed multigraph over N atoms, two systems, skewed degrees, two atoms
    without edges, and five special edges: along +y, -y, +x, -z and one beyond the cutoff."""
    pos = rng.uniform(0.0, 5.0, size=(N, 3)).astype(np.float32)
    Z = rng.integers(1, 90, size=N).astype(np.int64)
    batch = np.repeat(np.arange(S), [N // 2, N - N // 2]).astype(np.int64)
    n_act = N - 2
    w = rng.gamma(0.7, size=n_act)
    w /= w.sum()
    src = rng.choice(n_act, size=E, p=w)
    dst = rng.integers(0, n_act, size=E)
    same = src == dst
    dst[same] = (dst[same] + 1) % n_act
    shifts = (rng.integers(-1, 2, size=(E, 3)) * 0.5).astype(np.float32)
    special = [(0.0, 1.7, 0.0), (0.0, -2.1, 0.0), (1.3, 0.0, 0.0), (0.0, 0.0, -0.9), (4.0, 4.0, 3.0)]
    for k, v in enumerate(special):
        shifts[k] = (np.array(v) - (pos[src[k]].astype(np.float64) - pos[dst[k]])).astype(np.float32)
    idx_i = src.astype(np.int64)
    idx_j = dst.astype(np.int64)
    col_idx = np.argsort(idx_j, kind="stable").astype(np.int32)
    row_ptr = np.zeros(N + 1, dtype=np.int32)
    row_ptr[1:] = np.cumsum(np.bincount(idx_j, minlength=N))
    return dict(pos=pos, Z=Z, batch=batch, idx_i=idx_i, idx_j=idx_j, shifts=shifts,
                row_ptr=row_ptr, col_idx=col_idx)


def _t(a):
    return torch.from_numpy(np.ascontiguousarray(a))


def _randn(rng, *shape):
    return rng.standard_normal(shape).astype(np.float32)


def main() -> None:
    ap = argparse.ArgumentParser()
    ap.add_argument("--reference", default="/root/reference")
    args = ap.parse_args()
    mods, triton_version = _load_reference(args.reference)
    rng = np.random.default_rng(20261202)
    g = _graph(rng)
    out = {f"graph.{k}": v for k, v in g.items()}
    out["meta.sizes"] = np.array([N, E, C, B, S], dtype=np.int64)
    pos, Z, batch = _t(g["pos"]), _t(g["Z"]), _t(g["batch"])
    idx_i, idx_j, shifts = _t(g["idx_i"]), _t(g["idx_j"]), _t(g["shifts"])
    row_ptr, col_idx = _t(g["row_ptr"]), _t(g["col_idx"])

    # geometry (ops/geom.py:496-592): forward, then the hand-written VJP kernel
    W_src, W_tgt = _randn(rng, NUM_Z, C), _randn(rng, NUM_Z, C)
    offset_g = np.linspace(0.0, CUTOFF, B).astype(np.float32)
    coeff_g = -0.5 / float(offset_g[1] - offset_g[0]) ** 2
    p = _t(pos.numpy().copy()).requires_grad_(True)
    sh = _t(shifts.numpy().copy()).requires_grad_(True)
    xe, wig, env = mods["geom"].precompute_geometry(p, Z, idx_i, idx_j, sh, _t(W_src), _t(W_tgt),
                                                   _t(offset_g), coeff_g, CUTOFF)
    g_xe, g_wig, g_env = _randn(rng, E, B + 2 * C), _randn(rng, E, 34), _randn(rng, E)
    torch.autograd.backward([xe, wig, env], [_t(g_xe), _t(g_wig), _t(g_env)])
    out.update({"geom.W_src": W_src, "geom.W_tgt": W_tgt, "geom.offset_g": offset_g,
                "geom.coeff_g": np.float64(coeff_g), "geom.cutoff": np.float64(CUTOFF),
                "geom.x_edge_raw": xe.detach().numpy(), "geom.wigner": wig.detach().numpy(),
                "geom.env": env.detach().numpy(), "geom.g_x_edge_raw": g_xe, "geom.g_wigner": g_wig,
                "geom.g_env": g_env, "geom.g_pos": p.grad.numpy(), "geom.g_shifts": sh.grad.numpy()})

    # gather (ops/gather.py:408-514) with a general (not orthogonal) 34-entry wigner, so
    # every entry's position in the rotation is visible in the outputs
    x = _t(_randn(rng, N, 9, C)).requires_grad_(True)
    wg = _t(_randn(rng, E, 34)).requires_grad_(True)
    rad = _t(_randn(rng, E, 12 * C)).requires_grad_(True)
    csd = _randn(rng, S, C)
    X0, X1, X2 = mods["gather"].gather_wigner_split(x, idx_i, idx_j, wg, rad, _t(csd), batch)
    gX0, gX1, gX2 = _randn(rng, E, 6 * C), _randn(rng, E, 8 * C), _randn(rng, E, 4 * C)
    torch.autograd.backward([X0, X1, X2], [_t(gX0), _t(gX1), _t(gX2)])
    out.update({"gather.x": x.detach().numpy(), "gather.wigner": wg.detach().numpy(),
                "gather.rad": rad.detach().numpy(), "gather.csd": csd,
                "gather.X_m0": X0.detach().numpy(), "gather.X_m1": X1.detach().numpy(),
                "gather.X_m2": X2.detach().numpy(), "gather.g_X_m0": gX0, "gather.g_X_m1": gX1,
                "gather.g_X_m2": gX2, "gather.g_x": x.grad.numpy(), "gather.g_wigner": wg.grad.numpy(),
                "gather.g_rad": rad.grad.numpy()})

    # gating (ops/gating.py:186-236)
    Y = [_t(_randn(rng, E, k * C)).requires_grad_(True) for k in (5, 4, 2)]
    Zs = mods["gating"].fused_gating_split(Y[0], Y[1], Y[2], C)
    gZ = [_randn(rng, E, k * C) for k in (3, 4, 2)]
    torch.autograd.backward(list(Zs), [_t(a) for a in gZ])
    for k in range(3):
        out[f"gating.Y_m{k}"] = Y[k].detach().numpy()
        out[f"gating.Z_m{k}"] = Zs[k].detach().numpy()
        out[f"gating.g_Z_m{k}"] = gZ[k]
        out[f"gating.g_Y_m{k}"] = Y[k].grad.numpy()

    # rotate-scatter (ops/scatter.py:295-354)
    Zm = [_t(_randn(rng, E, k * C)).requires_grad_(True) for k in (3, 4, 2)]
    wg = _t(_randn(rng, E, 34)).requires_grad_(True)
    ev = _t(rng.uniform(0.1, 1.0, size=E).astype(np.float32)).requires_grad_(True)
    xr = _t(_randn(rng, N, 9, C)).requires_grad_(True)
    xo = mods["scatter"].rotate_scatter_split(Zm[0], Zm[1], Zm[2], wg, ev, xr, idx_j, row_ptr, col_idx, N)
    g_out = _randn(rng, N, 9, C)
    xo.backward(_t(g_out))
    for k in range(3):
        out[f"scatter.Z_m{k}"] = Zm[k].detach().numpy()
        out[f"scatter.g_Z_m{k}"] = Zm[k].grad.numpy()
    out.update({"scatter.wigner": wg.detach().numpy(), "scatter.env": ev.detach().numpy(),
                "scatter.x_res": xr.detach().numpy(), "scatter.x_out": xo.detach().numpy(),
                "scatter.g_out": g_out, "scatter.g_wigner": wg.grad.numpy(), "scatter.g_env": ev.grad.numpy(),
                "scatter.g_x_res": xr.grad.numpy()})

    # init scatter (ops/scatter.py:484-527)
    rad = _t(_randn(rng, E, 3 * C)).requires_grad_(True)
    wg = _t(_randn(rng, E, 34)).requires_grad_(True)
    ev = _t(rng.uniform(0.1, 1.0, size=E).astype(np.float32)).requires_grad_(True)
    W_sphere = _t(_randn(rng, NUM_Z, C)).requires_grad_(True)
    csd = _t(_randn(rng, S, C)).requires_grad_(True)
    x0 = mods["scatter"].init_node_scatter(rad, wg, ev, Z, batch, W_sphere, csd, idx_j, row_ptr, col_idx, N)
    g_out = _randn(rng, N, 9, C)
    x0.backward(_t(g_out))
    out.update({"init.rad": rad.detach().numpy(), "init.wigner": wg.detach().numpy(),
                "init.env": ev.detach().numpy(), "init.W_sphere": W_sphere.detach().numpy(),
                "init.csd": csd.detach().numpy(), "init.x_out": x0.detach().numpy(), "init.g_out": g_out,
                "init.g_rad": rad.grad.numpy(), "init.g_wigner": wg.grad.numpy(), "init.g_env": ev.grad.numpy(),
                "init.g_W_sphere": W_sphere.grad.numpy(), "init.g_csd": csd.grad.numpy()})

    # LayerNorm-SiLU (ops/ln_silu.py:126-185), eps 1e-7 (the reference default)
    for t, (M, D) in enumerate(LN_SHAPES):
        xl = _t(_randn(rng, M, D) * 2.0 + 0.5).requires_grad_(True)
        gam = (1.0 + 0.3 * rng.standard_normal(D)).astype(np.float32)
        bet = (0.2 * rng.standard_normal(D)).astype(np.float32)
        yl = mods["ln_silu"].layer_norm_silu(xl, _t(gam), _t(bet))
        g_y = _randn(rng, M, D)
        yl.backward(_t(g_y))
        out.update({f"ln{t}.x": xl.detach().numpy(), f"ln{t}.gamma": gam, f"ln{t}.beta": bet,
                    f"ln{t}.out": yl.detach().numpy(), f"ln{t}.g_out": g_y, f"ln{t}.g_x": xl.grad.numpy()})

    out["meta.triton_version"] = np.array(triton_version)
    np.savez_compressed(OUT, **out)
    print(f"wrote {OUT}: {len(out)} arrays, triton {triton_version} interpreter")


if __name__ == "__main__":
    main()
