"""Pins of the lmax = 3, 4 oracle (the reference stops at lmax = 2, wrapper.py:105-118, so the
degree-3/4 blocks and slot maps are pinned by mathematics and by physical invariants of the
whole model, never by reference outputs).

  * the real-SH basis reproduces the reference's l = 1 and l = 2 bases and is orthonormal and
    traceless for l = 3, 4; D^l is orthogonal and a homomorphism;
  * rotations about the polar axis y act on every (m, -m) pair of every degree as the same
    planar rotation by m * angle (the property the SO(2) layers rely on);
  * the recursion tables the GPU kernel uses agree with the tensor-power formula;
  * at lmax = 2 the general gather / gate / scatter / init restatements equal the
    reference-pinned ones exactly;
  * the lmax = 4 model is rotation-equivariant, translation-invariant and its forces match
    finite differences; a planted slot mistake breaks equivariance.
"""
import importlib.util
import math
import re
import pathlib

import numpy as np
import pytest
import torch

import escn_md
import heads
import systems
from oracle import model_ref as M
from oracle import ops_ref as R
from oracle import sh_ref as S

DT = torch.float64
ROOT = pathlib.Path(__file__).resolve().parents[1]


def _unit_q(n, seed):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(n, 4, generator=g, dtype=DT)
    return q / q.norm(dim=1, keepdim=True)


def test_basis_reproduces_reference_l1_l2():
    assert (S.sh_basis(1) - torch.eye(3, dtype=DT)).abs().max() == 0
    assert (S.sh_basis(2) - R._l2_basis()).abs().max() < 1e-15
    q = _unit_q(200, 0)
    Rm = R.rotation_from_quaternion(q)
    assert (S.wigner_from_rotation(Rm, 2) - R.wigner_l2_from_quaternion(q)).abs().max() < 1e-13


@pytest.mark.parametrize("l", [3, 4])
def test_basis_orthonormal_traceless_and_representation(l):
    B = S.sh_basis(l)
    n = 2 * l + 1
    Bf = B.reshape(n, -1)
    assert (Bf @ Bf.T - torch.eye(n, dtype=DT)).abs().max() < 1e-14
    # traceless over every index pair and symmetric under index swaps
    for i in range(l):
        for j in range(i + 1, l):
            assert B.diagonal(dim1=1 + i, dim2=1 + j).sum(-1).abs().max() < 1e-14
            assert (B - B.transpose(1 + i, 1 + j)).abs().max() < 1e-15
    q1, q2 = _unit_q(300, 1), _unit_q(300, 2)
    R1, R2 = R.rotation_from_quaternion(q1), R.rotation_from_quaternion(q2)
    D1, D2, D12 = S.wigner_from_rotation(R1, l), S.wigner_from_rotation(R2, l), S.wigner_from_rotation(R1 @ R2, l)
    assert (D1 @ D1.transpose(1, 2) - torch.eye(n, dtype=DT)).abs().max() < 1e-13
    assert (D1 @ D2 - D12).abs().max() < 1e-13
    assert (torch.linalg.det(D1) - 1).abs().max() < 1e-11


def test_polar_rotation_acts_on_m_pairs_alike_for_every_degree():
    a = 0.83
    for l in range(1, 5):
        D = S.wigner_from_rotation(S.rotation_about_y(a), l)
        assert abs(D[l, l].item() - 1.0) < 1e-14          # m = 0 is invariant
        for m in range(1, l + 1):
            blk = D[[l + m, l - m]][:, [l + m, l - m]]
            want = torch.tensor([[math.cos(m * a), -math.sin(m * a)], [math.sin(m * a), math.cos(m * a)]], dtype=DT)
            assert (blk - want).abs().max() < 1e-13, (l, m)
            # and nothing else couples to this pair
            assert D[l + m].abs().sum() - blk[0].abs().sum() < 1e-13


def test_gpu_recursion_tables_match_tensor_formula():
    spec = importlib.util.spec_from_file_location("gen_wigner_tables",
                                                  ROOT / "flash-uma_amd" / "csrc" / "gen_wigner_tables.py")
    G = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(G)
    U3, U4 = torch.tensor(G.coupling(3)), torch.tensor(G.coupling(4))
    q = _unit_q(100, 4)
    Rm = R.rotation_from_quaternion(q)
    D2 = R.wigner_l2_from_quaternion(q)
    D3 = U3.T @ torch.einsum("eab,eij->eaibj", D2, Rm).reshape(-1, 15, 15) @ U3
    D4 = U4.T @ torch.einsum("eab,eij->eaibj", D3, Rm).reshape(-1, 21, 21) @ U4
    assert (D3 - S.wigner_from_rotation(Rm, 3)).abs().max() < 1e-13
    assert (D4 - S.wigner_from_rotation(Rm, 4)).abs().max() < 1e-13
    # the committed header holds the same numbers
    text = (ROOT / "flash-uma_amd" / "csrc" / "wigner_tables.h").read_text()
    for name, U in (("kU3", G.coupling(3)), ("kU4", G.coupling(4))):
        body = text.split(name)[1].split("=", 1)[1].split("};")[0]
        vals = [float(v) for v in re.findall(r"-?\d+\.\d+(?:e[-+]\d+)?", body)]
        assert np.allclose(np.array(vals).reshape(U.shape), U, atol=1e-9)


def test_general_ops_equal_reference_ops_at_lmax2():
    g = torch.Generator().manual_seed(5)
    N, E, C = 9, 40, 4
    x = torch.randn(N, 9, C, generator=g, dtype=DT)
    ii, jj = torch.randint(0, N, (E,), generator=g), torch.randint(0, N, (E,), generator=g)
    q = _unit_q(E, 6)
    w = torch.cat([R.rotation_from_quaternion(q).reshape(E, 9), R.wigner_l2_from_quaternion(q).reshape(E, 25)], 1)
    ext = torch.zeros(E, 0, dtype=DT)
    rad = torch.randn(E, 12 * C, generator=g, dtype=DT)
    csd = torch.randn(2, C, generator=g, dtype=DT)
    b = torch.randint(0, 2, (N,), generator=g)
    for p, r in zip(R.gather_rotate(x, ii, jj, w, rad, csd, b), R.gather_rotate_lmax(x, ii, jj, w, ext, rad, csd, b, 2)):
        assert torch.equal(p, r)
    Y = [torch.randn(E, k * C, generator=g, dtype=DT) for k in (5, 4, 2)]
    for p, r in zip(R.gating(*Y, C), R.gating_lmax(*Y, C, 2)):
        assert torch.equal(p, r)
    Zs = [torch.randn(E, k * C, generator=g, dtype=DT) for k in (3, 4, 2)]
    env = torch.rand(E, generator=g, dtype=DT)
    assert torch.equal(R.rotate_scatter(*Zs, w, env, x, jj, N), R.rotate_scatter_lmax(*Zs, w, ext, env, x, jj, N, 2))


def test_gather_lmax4_rotated_frame_is_explicit_rotation():
    """Each X block is (D v)[k] * rad for the slot's coefficient k, D the full rotation."""
    g = torch.Generator().manual_seed(7)
    L, N, E, C = 4, 6, 15, 3
    x = torch.randn(N, 25, C, generator=g, dtype=DT)
    ii, jj = torch.randint(0, N, (E,), generator=g), torch.randint(0, N, (E,), generator=g)
    q = _unit_q(E, 8)
    Rm = R.rotation_from_quaternion(q)
    w = torch.cat([Rm.reshape(E, 9), R.wigner_l2_from_quaternion(q).reshape(E, 25)], 1)
    ext = S.wigner_ext(Rm, L)
    rad = torch.randn(E, 6 * L * C, generator=g, dtype=DT)
    csd = torch.zeros(1, C, dtype=DT)
    b = torch.zeros(N, dtype=torch.long)
    X0, X1, X2 = R.gather_rotate_lmax(x, ii, jj, w, ext, rad, csd, b, L)
    full = torch.zeros(E, 25, 25, dtype=DT)
    for l in range(L + 1):
        full[:, l * l:(l + 1) ** 2, l * l:(l + 1) ** 2] = S.wigner_from_rotation(Rm, l)
    rs = torch.einsum("eab,ebc->eac", full, x[ii])
    r = rad.reshape(E, 6 * L, C)
    # (l = 3, m = -2) of the sender: X_m2 imaginary half, block 2 (L - 1 + 3 - 2) + 0; rad 4L + 2 + 2
    k = 9 + 3 - 2
    assert (X2.reshape(E, -1, C)[:, 2 * (L - 1 + 1)] - rs[:, k] * r[:, 4 * L + 2 + 2]).abs().max() < 1e-13
    # (l = 4, m = +1) of the sender: X_m1 block 2 (4 - 1); rad 2 (L + 1) + 2 (4 - 1)
    k = 16 + 4 + 1
    assert (X1.reshape(E, -1, C)[:, 6] - rs[:, k] * r[:, 2 * (L + 1) + 6]).abs().max() < 1e-13


@pytest.fixture(scope="module")
def small_l4():
    bb = escn_md.eSCNMDBackbone(num_layers=1, sphere_channels=16, hidden_channels=16, num_distance_basis=8, lmax=4,
                                seed=0)
    hd = heads.MLPEnergyHead(16, 16, seed=1)
    s = systems.cu_slab_co()
    ei, off = systems.neighbor_list(s.pos, s.cell, s.pbc, bb.cutoff, bb.max_neighbors)
    ref = M.energy_forces_stress(bb, hd, s.pos, s.Z, s.cell, ei, off)
    return bb, hd, s, ei, off, ref


def _rot(a, b, c):
    ca, sa, cb, sb, cc, sc = np.cos(a), np.sin(a), np.cos(b), np.sin(b), np.cos(c), np.sin(c)
    Rz = np.array([[ca, -sa, 0], [sa, ca, 0], [0, 0, 1]])
    Ry = np.array([[cb, 0, sb], [0, 1, 0], [-sb, 0, cb]])
    Rx = np.array([[1, 0, 0], [0, cc, -sc], [0, sc, cc]])
    return torch.tensor(Rz @ Ry @ Rx)


def test_lmax4_model_rotation_equivariance(small_l4):
    bb, hd, s, ei, off, ref = small_l4
    assert ref["node_embedding"].shape[1] == 25
    Rm = _rot(0.7, -0.4, 1.1)
    out = M.energy_forces_stress(bb, hd, torch.tensor(s.pos, dtype=DT) @ Rm.T, s.Z,
                                 torch.tensor(s.cell, dtype=DT) @ Rm.T, ei, off)
    assert abs(out["energy"].item() - ref["energy"].item()) < 1e-7 * abs(ref["energy"].item()) + 1e-9
    assert (out["forces"] - ref["forces"] @ Rm.T).abs().max() < 1e-7
    assert (out["stress"][0] - Rm @ ref["stress"][0] @ Rm.T).abs().max() < 1e-8


def test_lmax4_planted_slot_mistake_breaks_equivariance(small_l4, monkeypatch):
    bb, hd, s, ei, off, ref = small_l4
    real = R.slot_maps

    def wrong(L):
        m0, m1, m2, r0, r1, r2 = real(L)
        m2 = list(m2)
        m2[-1], m2[-2] = m2[-2], m2[-1]      # swap the (3, -2) and (4, -2) slots
        return m0, m1, m2, r0, r1, r2

    monkeypatch.setattr(R, "slot_maps", wrong)
    Rm = _rot(0.3, 0.9, -0.5)
    a = M.energy_forces_stress(bb, hd, s.pos, s.Z, s.cell, ei, off, stress=False)
    b = M.energy_forces_stress(bb, hd, torch.tensor(s.pos, dtype=DT) @ Rm.T, s.Z, torch.tensor(s.cell, dtype=DT) @ Rm.T,
                               ei, off, stress=False)
    assert abs(a["energy"].item() - b["energy"].item()) > 1e-6 * abs(a["energy"].item())


def test_lmax4_planted_basis_sign_breaks_equivariance(small_l4, monkeypatch):
    """Flipping the sign of one order -m basis function of degree 3 (so that rotations about
    the polar axis turn its (m, -m) pair the other way) must be caught."""
    bb, hd, s, ei, off, ref = small_l4
    real = S.sh_basis

    def flipped(l, dtype=DT):
        B = real(l, dtype)
        if l == 3:
            B = B.clone()
            B[3 - 1] = -B[3 - 1]
        return B

    monkeypatch.setattr(S, "sh_basis", flipped)
    Rm = _rot(-0.6, 0.2, 0.8)
    a = M.energy_forces_stress(bb, hd, s.pos, s.Z, s.cell, ei, off, stress=False)
    b = M.energy_forces_stress(bb, hd, torch.tensor(s.pos, dtype=DT) @ Rm.T, s.Z, torch.tensor(s.cell, dtype=DT) @ Rm.T,
                               ei, off, stress=False)
    assert abs(a["energy"].item() - b["energy"].item()) > 1e-6 * abs(a["energy"].item())


def test_lmax4_forces_match_finite_differences(small_l4):
    bb, hd, s, ei, off, ref = small_l4
    assert ref["forces"].sum(0).abs().max() < 1e-12
    h = 1e-5
    for atom, ax in [(3, 0), (28, 1)]:
        p = torch.tensor(s.pos, dtype=DT)
        pp, pm = p.clone(), p.clone()
        pp[atom, ax] += h
        pm[atom, ax] -= h
        ep = M.energy_forces_stress(bb, hd, pp, s.Z, s.cell, ei, off, stress=False)["energy"].item()
        em = M.energy_forces_stress(bb, hd, pm, s.Z, s.cell, ei, off, stress=False)["energy"].item()
        assert abs(-(ep - em) / (2 * h) - ref["forces"][atom, ax].item()) < 1e-6
