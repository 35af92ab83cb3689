"""The oracle against golden vectors written by the reference's own op kernels.

tests/golden/ref_ops_fixtures.npz holds inputs, forward outputs and hand-written-backward
gradients of the reference's geometry, gather, gating, rotate-scatter, init-scatter and
LayerNorm-SiLU kernels (ops/*.py run under Triton's CPU interpreter by
tests/golden/make_ref_fixtures.py). The float64 oracle must reproduce every array to
scale-relative 1e-6 (the reference computes in fp32). This pins the slot, gate and
radial-block layouts (ops/gather.py:132-154, ops/gating.py:63-103,
ops/scatter.py:104-127,409-411) and the geometry VJP (ops/geom.py:313-493), which the
mathematical checks in test_oracle_pins.py leave open.

The planted-mistake tests swap one layout entry of the oracle (on the CPU) and show that
the fixture comparison fails."""
from __future__ import annotations

import os

import numpy as np
import pytest
import torch

from oracle import ops_ref

FIX = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "ref_ops_fixtures.npz")
TOL = 1e-6
# The envelope 1 - 21u^5 + 35u^6 - 15u^7 (ops/geom.py) is evaluated in fp32 by the reference:
# its terms reach 35x the result near the cutoff, so fp32 rounding alone gives up to
# ~35 * 2^-24 * (a few) = 4e-6 absolute.
TOL_KEY = {"env": 5e-6}


@pytest.fixture(scope="module")
def fx():
    with np.load(FIX, allow_pickle=False) as d:
        return {k: d[k] for k in d.files}


def T(a, grad=False):
    t = torch.from_numpy(np.array(a))
    if t.is_floating_point():
        t = t.double()
    return t.requires_grad_(grad) if grad else t


def rel(a, b) -> float:
    a = a.detach().double().numpy() if torch.is_tensor(a) else np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.abs(a - b).max() / max(np.abs(b).max(), 1e-30))


def check(pairs):
    errs = {k: rel(a, b) for k, (a, b) in pairs.items()}
    bad = {k: v for k, v in errs.items() if not v <= TOL_KEY.get(k, TOL)}
    assert not bad, f"oracle vs reference kernels: {bad} (all: {errs})"
    return errs


def graph(fx):
    return {k.split(".", 1)[1]: T(v) for k, v in fx.items() if k.startswith("graph.")}


def run_geometry(fx):
    g = graph(fx)
    pos, sh = T(fx["graph.pos"], True), T(fx["graph.shifts"], True)
    xe, wig, env = ops_ref.edge_geometry(pos, g["Z"], g["idx_i"], g["idx_j"], sh, T(fx["geom.W_src"]),
                                         T(fx["geom.W_tgt"]), T(fx["geom.offset_g"]),
                                         float(fx["geom.coeff_g"]), float(fx["geom.cutoff"]))
    torch.autograd.backward([xe, wig, env], [T(fx["geom.g_x_edge_raw"]), T(fx["geom.g_wigner"]),
                                             T(fx["geom.g_env"])])
    return {"x_edge_raw": (xe, fx["geom.x_edge_raw"]), "wigner": (wig, fx["geom.wigner"]),
            "env": (env, fx["geom.env"]), "g_pos": (pos.grad, fx["geom.g_pos"]),
            "g_shifts": (sh.grad, fx["geom.g_shifts"])}


def run_gather(fx, fn=None):
    g = graph(fx)
    x, wg, rad = T(fx["gather.x"], True), T(fx["gather.wigner"], True), T(fx["gather.rad"], True)
    Xs = (fn or ops_ref.gather_rotate)(x, g["idx_i"], g["idx_j"], wg, rad, T(fx["gather.csd"]), g["batch"])
    torch.autograd.backward(list(Xs), [T(fx[f"gather.g_X_m{k}"]) for k in range(3)])
    out = {f"X_m{k}": (Xs[k], fx[f"gather.X_m{k}"]) for k in range(3)}
    out.update({"g_x": (x.grad, fx["gather.g_x"]), "g_wigner": (wg.grad, fx["gather.g_wigner"]),
                "g_rad": (rad.grad, fx["gather.g_rad"])})
    return out


def run_gating(fx, fn=None):
    C = int(fx["meta.sizes"][2])
    Y = [T(fx[f"gating.Y_m{k}"], True) for k in range(3)]
    Zs = (fn or ops_ref.gating)(Y[0], Y[1], Y[2], C)
    torch.autograd.backward(list(Zs), [T(fx[f"gating.g_Z_m{k}"]) for k in range(3)])
    out = {f"Z_m{k}": (Zs[k], fx[f"gating.Z_m{k}"]) for k in range(3)}
    out.update({f"g_Y_m{k}": (Y[k].grad, fx[f"gating.g_Y_m{k}"]) for k in range(3)})
    return out


def run_scatter(fx, fn=None):
    g = graph(fx)
    N = int(fx["meta.sizes"][0])
    Zm = [T(fx[f"scatter.Z_m{k}"], True) for k in range(3)]
    wg, ev, xr = T(fx["scatter.wigner"], True), T(fx["scatter.env"], True), T(fx["scatter.x_res"], True)
    xo = (fn or ops_ref.rotate_scatter)(Zm[0], Zm[1], Zm[2], wg, ev, xr, g["idx_j"], N)
    xo.backward(T(fx["scatter.g_out"]))
    out = {"x_out": (xo, fx["scatter.x_out"]), "g_wigner": (wg.grad, fx["scatter.g_wigner"]),
           "g_env": (ev.grad, fx["scatter.g_env"]), "g_x_res": (xr.grad, fx["scatter.g_x_res"])}
    out.update({f"g_Z_m{k}": (Zm[k].grad, fx[f"scatter.g_Z_m{k}"]) for k in range(3)})
    return out


def run_init(fx, fn=None):
    g = graph(fx)
    N = int(fx["meta.sizes"][0])
    rad, wg, ev = T(fx["init.rad"], True), T(fx["init.wigner"], True), T(fx["init.env"], True)
    Ws, csd = T(fx["init.W_sphere"], True), T(fx["init.csd"], True)
    x0 = (fn or ops_ref.init_scatter)(rad, wg, ev, g["Z"], g["batch"], Ws, csd, g["idx_j"], N)
    x0.backward(T(fx["init.g_out"]))
    return {"x_out": (x0, fx["init.x_out"]), "g_rad": (rad.grad, fx["init.g_rad"]),
            "g_wigner": (wg.grad, fx["init.g_wigner"]), "g_env": (ev.grad, fx["init.g_env"]),
            "g_W_sphere": (Ws.grad, fx["init.g_W_sphere"]), "g_csd": (csd.grad, fx["init.g_csd"])}


def run_ln(fx, t):
    x = T(fx[f"ln{t}.x"], True)
    y = ops_ref.layer_norm_silu(x, T(fx[f"ln{t}.gamma"]), T(fx[f"ln{t}.beta"]), eps=1e-7)
    y.backward(T(fx[f"ln{t}.g_out"]))
    return {"out": (y, fx[f"ln{t}.out"]), "g_x": (x.grad, fx[f"ln{t}.g_x"])}


def test_fixture_shapes(fx):
    N, E, C, B, S = (int(v) for v in fx["meta.sizes"])
    assert fx["geom.x_edge_raw"].shape == (E, B + 2 * C)
    assert fx["geom.wigner"].shape == (E, 34)
    assert fx["gather.X_m0"].shape == (E, 6 * C) and fx["gather.X_m1"].shape == (E, 8 * C)
    assert fx["gather.X_m2"].shape == (E, 4 * C) and fx["gather.g_rad"].shape == (E, 12 * C)
    assert fx["scatter.x_out"].shape == (N, 9, C) and fx["init.x_out"].shape == (N, 9, C)
    # the graph exercises empty receiver segments and an edge beyond the cutoff
    assert (np.diff(fx["graph.row_ptr"]) == 0).any()
    assert (fx["geom.env"] == 0).any()


def test_geometry_matches_reference_kernels(fx):
    check(run_geometry(fx))


def test_gather_matches_reference_kernels(fx):
    check(run_gather(fx))


def test_gating_matches_reference_kernels(fx):
    check(run_gating(fx))


def test_rotate_scatter_matches_reference_kernels(fx):
    check(run_scatter(fx))


def test_init_scatter_matches_reference_kernels(fx):
    check(run_init(fx))


@pytest.mark.parametrize("t", [0, 1])
def test_ln_silu_matches_reference_kernels(fx, t):
    check(run_ln(fx, t))


# ---- planted mistakes: each plausible layout slip must fail the fixture comparison ----

def _fails(pairs) -> bool:
    return any(not rel(a, b) <= TOL for a, b in pairs.values())


def test_planted_gather_radial_swap_fails(fx, monkeypatch):
    """r6 <-> r8 in X_m1 keeps the m-structure (and equivariance) but not the reference."""
    monkeypatch.setattr(ops_ref, "X_M1_RAD", [8, 7, 6, 9, 8, 7, 6, 9])
    assert _fails(run_gather(fx))


def test_planted_gather_side_swap_fails(fx, monkeypatch):
    """sender/receiver radial blocks exchanged in X_m2."""
    monkeypatch.setattr(ops_ref, "X_M2_RAD", [11, 10, 11, 10])
    assert _fails(run_gather(fx))


def test_planted_m1_coefficient_swap_fails(fx, monkeypatch):
    """R and I coefficients of the l=1, m=1 pair exchanged (k3 <-> k1)."""
    monkeypatch.setattr(ops_ref, "M1_COEF", [1, 7, 3, 5])
    assert _fails(run_gather(fx))
    assert _fails(run_scatter(fx))


def test_planted_gate_swap_fails(fx):
    """Z_m2 gated by g1 instead of g2."""
    def wrong(Y_m0, Y_m1, Y_m2, C):
        Z0, Z1, _ = ops_ref.gating(Y_m0, Y_m1, Y_m2, C)
        g1 = torch.sigmoid(Y_m0[:, 0:C])
        return Z0, Z1, torch.cat([Y_m2[:, 0:C] * g1, Y_m2[:, C:2 * C] * g1], 1)
    assert _fails(run_gating(fx, wrong))


def test_planted_init_block_swap_fails(fx):
    """init scatter with the l=1 and l=2 radial blocks exchanged."""
    def wrong(rad, *a):
        C = rad.shape[1] // 3
        return ops_ref.init_scatter(torch.cat([rad[:, :C], rad[:, 2 * C:], rad[:, C:2 * C]], 1), *a)
    assert _fails(run_init(fx, wrong))


def test_planted_wigner_transpose_fails(fx):
    """scatter with D instead of D^T."""
    def wrong(Z_m0, Z_m1, Z_m2, wigner, *a):
        E = wigner.shape[0]
        w = torch.cat([wigner[:, :9].reshape(E, 3, 3).transpose(1, 2).reshape(E, 9),
                       wigner[:, 9:].reshape(E, 5, 5).transpose(1, 2).reshape(E, 25)], 1)
        return ops_ref.rotate_scatter(Z_m0, Z_m1, Z_m2, w, *a)
    assert _fails(run_scatter(fx, wrong))
