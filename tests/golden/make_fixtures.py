"""Write the float64 oracle fixtures used by the GPU parity tests.

Run from the repository root:  python tests/golden/make_fixtures.py
Fixture water64_oracle.npz: a 64-molecule periodic water box (seed 3, L = 12.42 A), its
capped radius graph, and the oracle's energy, per-atom energies, forces and stress for the
seed-0 UMA-s-shaped random-init backbone and the seed-1 energy head."""
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


if __name__ == "__main__":
    water64()
