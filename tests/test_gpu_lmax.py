"""GPU parity of the lmax = 3, 4 path (the bcc Fe lmax-4 benchmark workload; the reference rejects lmax != 2).

Op level: every lmax-general entry point (Wigner extension, gather, gate, scatter, edge-degree
scatter; forward and backward) against the float64 oracle restatements (oracle/ops_ref.py
*_lmax, oracle/sh_ref.py), with the same scale-relative tolerance as the lmax = 2 ops.  At
lmax = 2 the same kernels are held to the reference-pinned oracle functions.

Model level: ZeroAllocBackbone at lmax = 3 and 4 against the float64 whole-model oracle
(energy per atom rel 1e-6, forces and stress max-abs 1e-4), and the full config-5 workload
(bcc Fe 16^3, lmax = 4, 8 layers) through size-independent invariants: zero net force,
rotation covariance, bitwise reproducibility.
"""
import importlib.util
import pathlib

import numpy as np
import pytest
import torch

from _helpers import assert_close, random_graph
from oracle import ops_ref as R
from oracle import sh_ref as S

pytestmark = pytest.mark.gpu
TOL = 2e-5
ROOT = pathlib.Path(__file__).resolve().parents[1]


def _vjp(fn, inputs, cot):
    ins = [t.detach().double().clone().requires_grad_(True) if t.is_floating_point() else t for t in inputs]
    outs = fn(*ins)
    if not isinstance(outs, tuple):
        outs = (outs,)
    s = sum((o * c.double()).sum() for o, c in zip(outs, cot))
    grads = torch.autograd.grad(s, [t for t in ins if t.is_floating_point() and t.requires_grad], allow_unused=True)
    return outs, grads


def _wigner(E, seed):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(E, 4, generator=g, dtype=torch.float64)
    q = q / q.norm(dim=1, keepdim=True)
    Rm = R.rotation_from_quaternion(q)
    wig = torch.cat([Rm.reshape(E, 9), R.wigner_l2_from_quaternion(q).reshape(E, 25)], 1)
    return wig, Rm


def _tables():
    spec = importlib.util.spec_from_file_location("gen_wigner_tables",
                                                  ROOT / "flash-uma_amd" / "csrc" / "gen_wigner_tables.py")
    G = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(G)
    return torch.tensor(G.coupling(3)), torch.tensor(G.coupling(4))


def _ext_from_blocks(wig, L, U3, U4):
    """Oracle of fu_wigner_ext_fwd as a function of the 34 scalars (D^1, D^2 independent
    inputs), for the VJP check: rows |m| <= 2 of D^3 = U3^T (D2 (x) D1) U3, D^4 likewise."""
    E = wig.shape[0]
    R1 = wig[:, :9].reshape(E, 3, 3)
    D2 = wig[:, 9:].reshape(E, 5, 5)
    D3 = U3.T @ torch.einsum("eab,eij->eaibj", D2, R1).reshape(E, 15, 15) @ U3
    parts = [D3[:, 1:6].reshape(E, -1)]
    if L >= 4:
        D4 = U4.T @ torch.einsum("eab,eij->eaibj", D3, R1).reshape(E, 21, 21) @ U4
        parts.append(D4[:, 2:7].reshape(E, -1))
    return torch.cat(parts, 1)


@pytest.mark.parametrize("L", [3, 4])
def test_wigner_extend(cuda, L):
    from ops.lmax import wigner_extend
    E = 500
    wig, Rm = _wigner(E, 1)
    wg = wig.float().to(cuda).requires_grad_(True)
    ext = wigner_extend(wg, L)
    # forward against the tensor-power formula (independent of the recursion)
    assert_close(ext, S.wigner_ext(Rm, L), 1e-5, "wigner ext fwd")
    U3, U4 = _tables()
    g = torch.Generator().manual_seed(2)
    cot = torch.randn(ext.shape, generator=g)
    (ref,), (gref,) = _vjp(lambda w: _ext_from_blocks(w, L, U3.double(), U4.double()), [wig.float()], [cot])
    assert_close(ext, ref, 1e-5, "wigner ext fwd (recursion)")
    (gw,) = torch.autograd.grad(ext, wg, cot.to(cuda))
    assert_close(gw, gref, 1e-5, "wigner ext bwd")


def _inputs(L, seed=4, N=40, E=300, C=128):
    pos, Z, ei, shifts = random_graph(N, E, seed=seed)
    wig, Rm = _wigner(E, seed)
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(N, (L + 1) ** 2, C, generator=g)
    rad = torch.randn(E, 6 * L * C, generator=g)
    csd = torch.randn(1, C, generator=g)
    batch = torch.zeros(N, dtype=torch.long)
    ext = S.wigner_ext(Rm, L).float() if L > 2 else torch.zeros(E, 0)
    return x, torch.from_numpy(ei), wig.float(), ext, rad, csd, batch


@pytest.mark.parametrize("L,C", [(2, 128), (3, 64), (4, 128)])
def test_gather_lmax(cuda, L, C):
    from ops.lmax import gather_rotate_lmax
    x, ei, wig, ext, rad, csd, batch = _inputs(L, C=C)
    xg, wg, eg, rg = (t.to(cuda).requires_grad_(True) for t in (x, wig, ext, rad))
    X = gather_rotate_lmax(xg, ei[0].to(cuda), ei[1].to(cuda), wg, eg, rg, csd.to(cuda), batch.to(cuda), None, L)
    g = torch.Generator().manual_seed(5)
    cot = [torch.randn(t.shape, generator=g) for t in X]
    if L == 2:   # the reference-pinned restatement
        ref, gref = _vjp(lambda a, w, r: R.gather_rotate(a, ei[0], ei[1], w, r, csd.double(), batch), [x, wig, rad],
                         cot)
        grads = torch.autograd.grad(X, (xg, wg, rg), [c.to(cuda) for c in cot])
    else:
        ref, gref = _vjp(lambda a, w, e, r: R.gather_rotate_lmax(a, ei[0], ei[1], w, e, r, csd.double(), batch, L),
                         [x, wig, ext, rad], cot)
        grads = torch.autograd.grad(X, (xg, wg, eg, rg), [c.to(cuda) for c in cot])
    for a, b in zip(X, ref):
        assert_close(a, b, TOL, "gather fwd")
    for a, b in zip(grads, gref):
        assert_close(a, b, TOL, "gather bwd")


@pytest.mark.parametrize("L,C", [(2, 128), (3, 64), (4, 128)])
def test_gather_lmax_node_and_edge_forms(cuda, L, C):
    """fu_gather_fwd_lmax with the graph's CSRs (each node's receiver and sender segments, node
    rows read once per side) and without them (edge-parallel): bitwise equal outputs, both
    equal to the float64 oracle.  The graph has nodes without incoming or outgoing edges."""
    from ops import _lib
    from ops.lmax import _csrs, _ext_ptr
    x, ei, wig, ext, rad, csd, batch = _inputs(L, C=C, N=60, E=250)
    xg, wg, eg, rg, cg, bg = (t.to(cuda) for t in (x, wig, ext, rad, csd, batch))
    ii, jj = ei[0].to(cuda), ei[1].to(cuda)
    N, E = x.shape[0], ii.shape[0]
    assert (torch.bincount(ei[0], minlength=N) == 0).any() and (torch.bincount(ei[1], minlength=N) == 0).any()
    rptr, ridx, sptr, sidx = _csrs(None, ii, jj, N, E)
    outs = []
    for csr in (True, False):
        X = [torch.full((E, w * C), float("nan"), device=cuda) for w in (2 * (L + 1), 4 * L, 4 * (L - 1))]
        p = [t.data_ptr() for t in (rptr, ridx, sptr, sidx)] if csr else [None] * 4
        _lib.call("fu_gather_fwd_lmax", xg.data_ptr(), ii.data_ptr(), jj.data_ptr(), wg.data_ptr(), _ext_ptr(eg),
                  rg.data_ptr(), cg.data_ptr(), bg.data_ptr(), *p, X[0].data_ptr(), X[1].data_ptr(), X[2].data_ptr(),
                  E, N, 1, C, L, _lib.stream_ptr(cuda))
        outs.append([t.cpu() for t in X])
    ref = R.gather_rotate_lmax(x.double(), ei[0], ei[1], wig.double(), ext.double(), rad.double(), csd.double(),
                               batch, L)
    for a, b, r in zip(*outs, ref):
        assert torch.equal(a, b)
        assert_close(a, r, TOL, "gather fwd (node-centric)")


@pytest.mark.parametrize("L", [2, 3, 4])
def test_gating_lmax(cuda, L):
    from ops.lmax import gating_lmax
    C, E = 128, 257
    g = torch.Generator().manual_seed(6)
    Y = [torch.randn(E, k * C, generator=g) for k in (2 * L + 1, 2 * L, 2 * (L - 1))]
    Yg = [t.to(cuda).requires_grad_(True) for t in Y]
    Z = gating_lmax(*Yg, C, L)
    cot = [torch.randn(t.shape, generator=g) for t in Z]
    fn = (lambda a, b, c: R.gating(a, b, c, C)) if L == 2 else (lambda a, b, c: R.gating_lmax(a, b, c, C, L))
    ref, gref = _vjp(fn, Y, cot)
    for a, b in zip(Z, ref):
        assert_close(a, b, TOL, "gating fwd")
    for a, b in zip(torch.autograd.grad(Z, Yg, [c.to(cuda) for c in cot]), gref):
        assert_close(a, b, TOL, "gating bwd")


@pytest.mark.parametrize("L", [2, 3, 4])
def test_scatter_lmax(cuda, L):
    from ops.lmax import rotate_scatter_lmax
    from ops import topology
    C = 128
    x, ei, wig, ext, _, _, _ = _inputs(L, seed=8, C=C)
    N, E = x.shape[0], ei.shape[1]
    g = torch.Generator().manual_seed(9)
    Zs = [torch.randn(E, k * C, generator=g) for k in (L + 1, 2 * L, 2 * (L - 1))]
    env = torch.rand(E, generator=g)
    idx_j = ei[1].to(cuda)
    row_ptr, col_idx = topology.receiver_csr(idx_j, N)
    Zg = [z.to(cuda).requires_grad_(True) for z in Zs]
    wg, xg, eg, envg = (t.to(cuda).requires_grad_(True) for t in (wig, x, ext, env))
    out = rotate_scatter_lmax(*Zg, wg, eg, envg, xg, idx_j, row_ptr, col_idx, N, L)
    cot = [torch.randn(out.shape, generator=g)]
    (ref,), gref = _vjp(lambda a, b, c, w, e, en, xr: R.rotate_scatter_lmax(a, b, c, w, e, en, xr, ei[1], N, L),
                        [*Zs, wig, ext, env, x], cot)
    assert_close(out, ref, TOL, "scatter fwd")
    grads = torch.autograd.grad(out, (*Zg, wg) + ((eg,) if L > 2 else ()) + (envg, xg), cot[0].to(cuda))
    gref = [t for t in gref if t is not None]
    for a, b in zip(grads, gref):
        assert_close(a, b, TOL, "scatter bwd")


@pytest.mark.parametrize("L", [2, 3, 4])
def test_init_scatter_lmax(cuda, L):
    from ops.lmax import init_node_scatter_lmax
    from ops import topology
    C = 128
    x, ei, wig, ext, _, _, _ = _inputs(L, seed=10, C=C)
    N, E = x.shape[0], ei.shape[1]
    g = torch.Generator().manual_seed(11)
    rad = torch.randn(E, (L + 1) * C, generator=g)
    Zn = torch.randint(1, 90, (N,), generator=g)
    W_sphere = torch.randn(100, C, generator=g)
    csd = torch.randn(1, C, generator=g)
    batch = torch.zeros(N, dtype=torch.long)
    env = torch.rand(E, generator=g)
    idx_j = ei[1].to(cuda)
    row_ptr, col_idx = topology.receiver_csr(idx_j, N)
    rg, wg, eg, envg = (t.to(cuda).requires_grad_(True) for t in (rad, wig, ext, env))
    out = init_node_scatter_lmax(rg, wg, eg, envg, Zn.to(cuda), batch.to(cuda), W_sphere.to(cuda), csd.to(cuda),
                                 idx_j, row_ptr, col_idx, N, L)
    cot = [torch.randn(out.shape, generator=g)]
    (ref,), gref = _vjp(lambda r, w, e, en: R.init_scatter_lmax(r, w, e, en, Zn, batch, W_sphere.double(),
                                                                csd.double(), ei[1], N, L), [rad, wig, ext, env], cot)
    assert_close(out, ref, TOL, "init scatter fwd")
    grads = torch.autograd.grad(out, (rg, wg) + ((eg,) if L > 2 else ()) + (envg,), cot[0].to(cuda))
    gref = [t for t in gref if t is not None]
    for a, b in zip(grads, gref):
        assert_close(a, b, TOL, "init scatter bwd")


def test_node_modules_lmax4(cuda):
    from ops.node import rms_norm_sh
    import escn_md
    from oracle import model_ref as M
    g = torch.Generator().manual_seed(20)
    N, C, L = 37, 128, 4
    x = torch.randn(N, 25, C, generator=g) * 2 + 0.3
    w = torch.rand(L + 1, C, generator=g) + 0.5
    b = torch.randn(C, generator=g)
    xg = x.to(cuda).requires_grad_(True)
    out = rms_norm_sh(xg, w.to(cuda), b.to(cuda), L, 1e-5)
    cot = torch.randn(N, 25, C, generator=g)
    (ref,), (gref,) = _vjp(lambda a: M.rms_norm_sh(a, w.double(), b.double(), L, 1e-5), [x], [cot])
    assert_close(out, ref, TOL, "rms norm fwd")
    assert_close(torch.autograd.grad(out, xg, cot.to(cuda))[0], gref, 1e-4, "rms norm bwd")
    mod = escn_md.SpectralAtomwise(C, C, L, generator=g)
    P = {"m." + k: v.double() for k, v in mod.state_dict().items()}
    xg = x.to(cuda).requires_grad_(True)
    out = mod.to(cuda)(xg)
    (ref,), (gref,) = _vjp(lambda a: M.spectral_atomwise(a, P, "m.", L, C), [x], [cot])
    assert_close(out, ref, TOL, "atom-wise fwd")
    assert_close(torch.autograd.grad(out, xg, cot.to(cuda))[0], gref, 1e-4, "atom-wise bwd")


def _model(cuda, L, layers, C=128, seed=0):
    import escn_md
    import heads
    from wrapper import ZeroAllocBackbone
    bb = escn_md.eSCNMDBackbone(num_layers=layers, sphere_channels=C, hidden_channels=C, lmax=L, seed=seed)
    hd = heads.MLPEnergyHead(C, C, seed=seed + 1)
    model = heads.PotentialModel(ZeroAllocBackbone(bb.to(cuda)), hd.to(cuda))
    return bb, hd, model


def _run(model, system, ei, off, cuda, stress=True):
    import heads
    data = heads.make_atomic_data(system, ei, off, cuda)
    out = model(data, compute_forces=True, compute_stress=stress)
    return {k: (v.detach().cpu() if torch.is_tensor(v) else v) for k, v in out.items()}


@pytest.mark.parametrize("L,layers", [(3, 2), (4, 2)])
def test_model_lmax_parity(cuda, L, layers):
    import systems
    from oracle.model_ref import energy_forces_stress
    bb, hd, model = _model(cuda, L, layers)
    s = systems.cu_slab_co()
    ei, off = systems.neighbor_list(s.pos, s.cell, s.pbc, bb.cutoff, bb.max_neighbors)
    out = _run(model, s, ei, off, cuda)
    ref = energy_forces_stress(bb.cpu(), hd.cpu(), s.pos, s.Z, s.cell, ei, off, dtype=torch.float64)
    assert out["node_embedding"].shape[1] == (L + 1) ** 2
    e_rel = abs(out["energy"].double().item() - ref["energy"].item()) / abs(ref["energy"].item())
    f_err = (out["forces"].double() - ref["forces"]).abs().max().item()
    s_err = (out["stress"].double() - ref["stress"]).abs().max().item()
    print(f"lmax={L}: E rel {e_rel:.2e}, F max-abs {f_err:.2e}, S max-abs {s_err:.2e}")
    assert e_rel <= 1e-6 and f_err <= 1e-4 and s_err <= 1e-4


def test_config5_model_on_fe54_fixture(cuda):
    """The lmax-4 benchmark workload's backbone (lmax = 4, mmax = 2, 8 layers, C = 128) on bcc Fe 3x3x3
    (54 atoms, 30 edges per atom, E+F+S) against the committed float64 oracle fixture
    (tests/golden/fe54_lmax4_oracle.npz).  Bars as for lmax = 2; per-atom contributions rel
    1e-5 (a float32 oracle run is 1.6e-6 from float64 here)."""
    import os
    import systems
    g = np.load(os.path.join(os.path.dirname(__file__), "golden", "fe54_lmax4_oracle.npz"))
    bb, hd, model = _model(cuda, 4, 8)
    s = systems.AtomicSystem("fe54", g["pos"], g["Z"].astype(np.int64), g["cell"])
    out = _run(model, s, g["edge_index"].astype(np.int64), g["cell_offsets"].astype(np.float32), cuda)
    e_rel = abs(out["energy"].double().item() - g["energy"][0]) / abs(g["energy"][0])
    f_err = np.abs(out["forces"].double().numpy() - g["forces"]).max()
    s_err = np.abs(out["stress"].double().numpy() - g["stress"]).max()
    a_rel = (np.abs(out["atom_energy"].double().numpy() - g["atom_energy"]) /
             np.maximum(np.abs(g["atom_energy"]), 1e-3)).max()
    print(f"fe54 lmax4: E rel {e_rel:.2e}, F {f_err:.2e}, S {s_err:.2e}, per-atom {a_rel:.2e}")
    assert e_rel <= 1e-6 and f_err <= 1e-4 and s_err <= 1e-4 and a_rel <= 1e-5


def test_config5_bcc_fe_lmax4_invariants(cuda):
    """The lmax-4 benchmark workload at full size: bcc Fe 16^3 (8,192 atoms), lmax = 4, 8 layers, C = 128,
    energy + forces.  No CPU oracle finishes at this size; checked through invariants."""
    import systems
    bb, hd, model = _model(cuda, 4, 8)
    s = systems.bcc_fe(16)
    ei, off = systems.neighbor_list(s.pos, s.cell, s.pbc, bb.cutoff, bb.max_neighbors)
    a = _run(model, s, ei, off, cuda, stress=False)
    assert torch.isfinite(a["energy"]).all() and torch.isfinite(a["forces"]).all()
    fmax = a["forces"].abs().max().item()
    net = a["forces"].double().sum(0).abs().max().item()
    print(f"config 5: E = {a['energy'].item():.6f}, max |F| = {fmax:.3e}, |sum F| = {net:.2e}")
    assert net < 1e-5 * s.n_atoms * max(fmax, 1e-3)
    b = _run(model, s, ei, off, cuda, stress=False)
    assert torch.equal(a["energy"], b["energy"]) and torch.equal(a["forces"], b["forces"])
    # rotate the whole periodic system: same graph, energy unchanged, forces rotated
    ang = 0.61
    Rm = np.array([[np.cos(ang), 0, np.sin(ang)], [0, 1, 0], [-np.sin(ang), 0, np.cos(ang)]]) @ \
        np.array([[1, 0, 0], [0, np.cos(0.3), -np.sin(0.3)], [0, np.sin(0.3), np.cos(0.3)]])
    r = systems.AtomicSystem("fe_rot", (s.pos.astype(np.float64) @ Rm.T).astype(np.float32), s.Z,
                             (np.asarray(s.cell, dtype=np.float64) @ Rm.T).astype(np.float32))
    c = _run(model, r, ei, off, cuda, stress=False)
    e_rel = abs(c["energy"].double().item() - a["energy"].double().item()) / abs(a["energy"].double().item())
    f_err = (c["forces"].double() - a["forces"].double() @ torch.tensor(Rm).T).abs().max().item()
    print(f"config 5 rotated: E rel {e_rel:.2e}, F max-abs {f_err:.2e}")
    assert e_rel < 1e-6 and f_err < 1e-4
