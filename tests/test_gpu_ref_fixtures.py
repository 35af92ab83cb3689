"""The HIP ops (reference layout) against golden vectors from the reference's own kernels.

Same fixture as test_ref_fixtures.py (tests/golden/ref_ops_fixtures.npz, written by the
reference's ops/*.py under Triton's CPU interpreter). Each op is called through the
product's autograd Functions and the C-ABI, with the fixture's inputs and output
cotangents, and every forward output and gradient must match the reference kernels to
scale-relative 2e-5 (both sides compute in fp32; the order of the fp32 reductions
differs)."""
from __future__ import annotations

import os

import numpy as np
import pytest
import torch

FIX = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "ref_ops_fixtures.npz")
TOL = 2e-5

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def fx():
    with np.load(FIX, allow_pickle=False) as d:
        return {k: d[k] for k in d.files}


def rel(a, b) -> float:
    a = a.detach().double().cpu().numpy()
    b = np.asarray(b, np.float64)
    return float(np.abs(a - b).max() / max(np.abs(b).max(), 1e-30))


def check(pairs):
    errs = {k: rel(a, b) for k, (a, b) in pairs.items()}
    bad = {k: v for k, v in errs.items() if not v <= TOL}
    assert not bad, f"HIP op vs reference kernels: {bad} (all: {errs})"


def G(fx, cuda):
    def to(key, grad=False):
        t = torch.from_numpy(np.ascontiguousarray(fx[key])).to(cuda)
        return t.requires_grad_(True) if grad else t
    return to


def test_geometry_vs_reference(fx, cuda):
    from ops.geom import precompute_geometry
    to = G(fx, cuda)
    pos, sh = to("graph.pos", True), to("graph.shifts", True)
    xe, wig, env = precompute_geometry(pos, to("graph.Z"), to("graph.idx_i"), to("graph.idx_j"), sh,
                                       to("geom.W_src"), to("geom.W_tgt"), to("geom.offset_g"),
                                       float(fx["geom.coeff_g"]), float(fx["geom.cutoff"]))
    torch.autograd.backward([xe, wig, env], [to("geom.g_x_edge_raw"), to("geom.g_wigner"), to("geom.g_env")])
    check({"x_edge_raw": (xe, fx["geom.x_edge_raw"]), "wigner": (wig, fx["geom.wigner"]),
           "env": (env, fx["geom.env"]), "g_pos": (pos.grad, fx["geom.g_pos"]),
           "g_shifts": (sh.grad, fx["geom.g_shifts"])})


def test_gather_vs_reference(fx, cuda):
    from ops.gather import gather_wigner_split
    to = G(fx, cuda)
    x, wg, rad = to("gather.x", True), to("gather.wigner", True), to("gather.rad", True)
    Xs = gather_wigner_split(x, to("graph.idx_i"), to("graph.idx_j"), wg, rad, to("gather.csd"), to("graph.batch"))
    torch.autograd.backward(list(Xs), [to(f"gather.g_X_m{k}") for k in range(3)])
    pairs = {f"X_m{k}": (Xs[k], fx[f"gather.X_m{k}"]) for k in range(3)}
    pairs.update({"g_x": (x.grad, fx["gather.g_x"]), "g_wigner": (wg.grad, fx["gather.g_wigner"]),
                  "g_rad": (rad.grad, fx["gather.g_rad"])})
    check(pairs)


def test_gating_vs_reference(fx, cuda):
    from ops.gating import fused_gating_split
    to = G(fx, cuda)
    C = int(fx["meta.sizes"][2])
    Y = [to(f"gating.Y_m{k}", True) for k in range(3)]
    Zs = fused_gating_split(Y[0], Y[1], Y[2], C)
    torch.autograd.backward(list(Zs), [to(f"gating.g_Z_m{k}") for k in range(3)])
    pairs = {f"Z_m{k}": (Zs[k], fx[f"gating.Z_m{k}"]) for k in range(3)}
    pairs.update({f"g_Y_m{k}": (Y[k].grad, fx[f"gating.g_Y_m{k}"]) for k in range(3)})
    check(pairs)


def test_rotate_scatter_vs_reference(fx, cuda):
    from ops.scatter import rotate_scatter_split
    to = G(fx, cuda)
    N = int(fx["meta.sizes"][0])
    Zm = [to(f"scatter.Z_m{k}", True) for k in range(3)]
    wg, ev, xr = to("scatter.wigner", True), to("scatter.env", True), to("scatter.x_res", True)
    xo = rotate_scatter_split(Zm[0], Zm[1], Zm[2], wg, ev, xr, to("graph.idx_j"), to("graph.row_ptr"),
                              to("graph.col_idx"), N)
    xo.backward(to("scatter.g_out"))
    pairs = {"x_out": (xo, fx["scatter.x_out"]), "g_wigner": (wg.grad, fx["scatter.g_wigner"]),
             "g_env": (ev.grad, fx["scatter.g_env"]), "g_x_res": (xr.grad, fx["scatter.g_x_res"])}
    pairs.update({f"g_Z_m{k}": (Zm[k].grad, fx[f"scatter.g_Z_m{k}"]) for k in range(3)})
    check(pairs)


def test_init_scatter_vs_reference(fx, cuda):
    from ops.scatter import init_node_scatter
    to = G(fx, cuda)
    N = int(fx["meta.sizes"][0])
    rad, wg, ev = to("init.rad", True), to("init.wigner", True), to("init.env", True)
    Ws, csd = to("init.W_sphere", True), to("init.csd", True)
    x0 = init_node_scatter(rad, wg, ev, to("graph.Z"), to("graph.batch"), Ws, csd, to("graph.idx_j"),
                           to("graph.row_ptr"), to("graph.col_idx"), N)
    x0.backward(to("init.g_out"))
    check({"x_out": (x0, fx["init.x_out"]), "g_rad": (rad.grad, fx["init.g_rad"]),
           "g_wigner": (wg.grad, fx["init.g_wigner"]), "g_env": (ev.grad, fx["init.g_env"]),
           "g_W_sphere": (Ws.grad, fx["init.g_W_sphere"]), "g_csd": (csd.grad, fx["init.g_csd"])})


@pytest.mark.parametrize("t", [0, 1])
def test_ln_silu_vs_reference(fx, cuda, t):
    from ops.ln_silu import layer_norm_silu
    to = G(fx, cuda)
    x = to(f"ln{t}.x", True)
    y = layer_norm_silu(x, to(f"ln{t}.gamma"), to(f"ln{t}.beta"), 1e-7)
    y.backward(to(f"ln{t}.g_out"))
    check({"out": (y, fx[f"ln{t}.out"]), "g_x": (x.grad, fx[f"ln{t}.g_x"])})
