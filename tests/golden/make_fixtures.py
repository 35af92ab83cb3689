"""Write the float64 oracle fixtures used by the GPU parity tests.

Run from the repository root:  python tests/golden/make_fixtures.py
Fixture water64_oracle.npz: a 64-molecule periodic water box (seed 3, L = 12.42 A), its
capped radius graph, and the oracle's energy, per-atom energies, forces and stress for the
seed-0 UMA-s-shaped random-init backbone and the seed-1 energy head.
Fixture sweep200_oracle.npz: systems.sweep_graph(200, 100) (the reference's benchmark graph
construction: every pair within the cutoff, no per-receiver cap, up to 171 edges per atom,
unit cell, random cell offsets) with the same backbone, head and oracle outputs.
Fixture fe432_oracle.npz: bcc Fe 6x6x6 (432 atoms, 12,960 edges; the headline workload's
local structure) with the same backbone and head.
Fixture fe54_lmax4_oracle.npz: bcc Fe 3x3x3 with the lmax-4 benchmark workload's backbone (lmax = 4,
8 layers)."""
import os
import sys

import numpy as np
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path[:0] = [ROOT, os.path.join(ROOT, "flash-uma_amd")]

import escn_md  # noqa: E402
import heads  # noqa: E402
import systems  # noqa: E402
from oracle.model_ref import energy_forces_stress  # noqa: E402


def water64():
    bb = escn_md.eSCNMDBackbone(seed=0)
    hd = heads.MLPEnergyHead(bb.sphere_channels, bb.hidden_channels, seed=1)
    s = systems.water_box(n_mol=64, L=12.42, seed=3)
    ei, off = systems.neighbor_list(s.pos, s.cell, s.pbc, bb.cutoff, bb.max_neighbors)
    ref = energy_forces_stress(bb, hd, s.pos, s.Z, s.cell, ei, off, dtype=torch.float64)
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "water64_oracle.npz")
    np.savez_compressed(path, pos=s.pos, Z=s.Z, cell=s.cell, edge_index=ei, cell_offsets=off,
                        energy=ref["energy"].numpy(), atom_energy=ref["atom_energy"].numpy(),
                        forces=ref["forces"].numpy(), stress=ref["stress"].numpy())
    print(f"wrote {path}: N={s.n_atoms} E={ei.shape[1]} energy={ref['energy'].item():.10f}")


def sweep200():
    bb = escn_md.eSCNMDBackbone(seed=0)
    hd = heads.MLPEnergyHead(bb.sphere_channels, bb.hidden_channels, seed=1)
    s, ei, off = systems.sweep_graph(200, 100)
    ref = energy_forces_stress(bb, hd, s.pos, s.Z, s.cell, ei, off, dtype=torch.float64)
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "sweep200_oracle.npz")
    np.savez_compressed(path, pos=s.pos, Z=s.Z.astype(np.int8), cell=s.cell, edge_index=ei.astype(np.int16),
                        cell_offsets=off.astype(np.int8), energy=ref["energy"].numpy(),
                        atom_energy=ref["atom_energy"].numpy(), forces=ref["forces"].numpy(),
                        stress=ref["stress"].numpy())
    print(f"wrote {path}: N={s.n_atoms} E={ei.shape[1]} energy={ref['energy'].item():.10f}")


def _fe(n_rep: int, name: str, **model_kw):
    bb = escn_md.eSCNMDBackbone(seed=0, **model_kw)
    hd = heads.MLPEnergyHead(bb.sphere_channels, bb.hidden_channels, seed=1)
    s = systems.bcc_fe(n_rep=n_rep)
    ei, off = systems.neighbor_list(s.pos, s.cell, s.pbc, bb.cutoff, bb.max_neighbors)
    ref = energy_forces_stress(bb, hd, s.pos, s.Z, s.cell, ei, off, dtype=torch.float64)
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), name)
    np.savez_compressed(path, pos=s.pos, Z=s.Z.astype(np.int8), cell=s.cell, edge_index=ei.astype(np.int32),
                        cell_offsets=off.astype(np.int8), energy=ref["energy"].numpy(),
                        atom_energy=ref["atom_energy"].numpy(), forces=ref["forces"].numpy(),
                        stress=ref["stress"].numpy())
    print(f"wrote {path}: N={s.n_atoms} E={ei.shape[1]} energy={ref['energy'].item():.10f}")


def fe432():
    """The headline workload's local structure at a size the float64 oracle finishes: bcc Fe
    6x6x6 (432 atoms, 30 edges per atom), UMA-s-shaped backbone, E+F+S."""
    _fe(6, "fe432_oracle.npz")


def fe54_lmax4():
    """The lmax-4 benchmark workload's model (lmax = 4, 8 layers) on bcc Fe 3x3x3 (54 atoms), E+F+S."""
    _fe(3, "fe54_lmax4_oracle.npz", lmax=4, num_layers=8)


if __name__ == "__main__":
    which = sys.argv[1:] or ["water64", "sweep200", "fe432", "fe54_lmax4"]
    for name in which:
        globals()[name]()
