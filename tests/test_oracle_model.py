"""Physical invariants of the whole-model oracle (these pin the slot maps, the SO(2) packing
and the gate wiring together: a wrong slot, sign or transposed block breaks rotation
equivariance), plus force/stress consistency with finite differences.

A small model (C = 64, 2 layers, 16 Gaussians) keeps the CPU suite fast; the structure is
the same as the UMA-s-shaped headline model."""
import copy

import numpy as np
import pytest
import torch

import escn_md
import heads
import systems
from oracle import model_ref as M
from oracle import ops_ref as R


@pytest.fixture(scope="module")
def small():
    bb = escn_md.eSCNMDBackbone(num_layers=2, sphere_channels=64, hidden_channels=64, num_distance_basis=16, seed=0)
    hd = heads.MLPEnergyHead(64, 64, seed=1)
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


def test_rotation_equivariance(small):
    bb, hd, s, ei, off, ref = small
    Rm = _rot(0.7, -0.4, 1.1)
    pos = torch.tensor(s.pos, dtype=torch.float64) @ Rm.T
    cell = torch.tensor(s.cell, dtype=torch.float64) @ Rm.T
    out = M.energy_forces_stress(bb, hd, pos, s.Z, cell, ei, off)
    # invariance holds up to the 1e-7 regularisers inside the edge-frame normalisation
    assert abs(out["energy"].item() - ref["energy"].item()) < 1e-7 * abs(ref["energy"].item()) + 1e-9
    assert (out["forces"] - ref["forces"] @ Rm.T).abs().max() < 1e-7
    assert (out["stress"][0] - Rm @ ref["stress"][0] @ Rm.T).abs().max() < 1e-8


def test_planted_slot_mistake_breaks_equivariance(small, monkeypatch):
    """Swapping two rotated-frame slots in a copy of the oracle must be caught."""
    bb, hd, s, ei, off, ref = small
    monkeypatch.setattr(R, "M1_COEF", [3, 7, 5, 1])   # swap the two imaginary m=1 slots
    Rm = _rot(0.3, 0.9, -0.5)
    a = M.energy_forces_stress(bb, hd, s.pos, s.Z, s.cell, ei, off, stress=False)
    b = M.energy_forces_stress(bb, hd, torch.tensor(s.pos, dtype=torch.float64) @ Rm.T, s.Z,
                               torch.tensor(s.cell, dtype=torch.float64) @ Rm.T, ei, off, stress=False)
    assert abs(a["energy"].item() - b["energy"].item()) > 1e-5 * abs(a["energy"].item())


def test_translation_and_permutation_invariance(small):
    bb, hd, s, ei, off, ref = small
    out = M.energy_forces_stress(bb, hd, torch.tensor(s.pos, dtype=torch.float64) + torch.tensor([0.3, -1.2, 2.0]),
                                 s.Z, s.cell, ei, off)
    assert abs(out["energy"].item() - ref["energy"].item()) < 1e-12 * max(1, abs(ref["energy"].item()))
    perm = np.random.default_rng(0).permutation(s.n_atoms)
    inv = np.argsort(perm)
    out = M.energy_forces_stress(bb, hd, s.pos[perm], s.Z[perm], s.cell, inv[ei], off)
    assert abs(out["energy"].item() - ref["energy"].item()) < 1e-12 * max(1, abs(ref["energy"].item()))
    assert (out["forces"] - ref["forces"][perm]).abs().max() < 1e-12


def test_forces_sum_to_zero_and_match_finite_differences(small):
    bb, hd, s, ei, off, ref = small
    assert ref["forces"].sum(0).abs().max() < 1e-12
    h = 1e-5
    for atom, ax in [(3, 0), (27, 2), (28, 1)]:
        p = torch.tensor(s.pos, dtype=torch.float64)
        pp, pm = p.clone(), p.clone()
        pp[atom, ax] += h
        pm[atom, ax] -= h
        ep = M.energy_forces_stress(bb, hd, pp, s.Z, s.cell, ei, off, stress=False)["energy"].item()
        em = M.energy_forces_stress(bb, hd, pm, s.Z, s.cell, ei, off, stress=False)["energy"].item()
        fd = -(ep - em) / (2 * h)
        assert abs(fd - ref["forces"][atom, ax].item()) < 1e-7


def test_stress_matches_strain_derivative_and_virial(small):
    bb, hd, s, ei, off, ref = small
    pos = torch.tensor(s.pos, dtype=torch.float64)
    cell = torch.tensor(s.cell, dtype=torch.float64)
    vol = abs(torch.linalg.det(cell).item())
    h = 1e-6
    for a, b in [(0, 0), (1, 2), (2, 1)]:
        eps = torch.zeros(3, 3, dtype=torch.float64)
        eps[a, b] = h
        F = torch.eye(3, dtype=torch.float64) + eps
        ep = M.energy_forces_stress(bb, hd, pos @ F, s.Z, cell @ F, ei, off, stress=False)["energy"].item()
        F = torch.eye(3, dtype=torch.float64) - eps
        em = M.energy_forces_stress(bb, hd, pos @ F, s.Z, cell @ F, ei, off, stress=False)["energy"].item()
        assert abs((ep - em) / (2 * h) / vol - ref["stress"][0, a, b].item()) < 1e-8
    # symmetric up to the frame regulariser
    st = ref["stress"][0]
    assert (st - st.T).abs().max() < 1e-9


def test_sweep_fixture_graph_is_reproducible():
    """systems.sweep_graph(200, 100) still builds the graph stored in the committed fixture
    (the GPU parity test reads the fixture; this pins the generator the bench uses)."""
    import os
    import numpy as np
    import systems
    g = np.load(os.path.join(os.path.dirname(__file__), "golden", "sweep200_oracle.npz"))
    s, ei, off = systems.sweep_graph(200, 100)
    assert np.array_equal(s.pos, g["pos"]) and np.array_equal(s.Z, g["Z"].astype(np.int64))
    assert np.array_equal(ei, g["edge_index"].astype(np.int64))
    assert np.array_equal(off, g["cell_offsets"].astype(np.float32))
