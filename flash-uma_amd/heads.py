"""Energy / force / stress head above the backbone boundary, and the model container.

The reference leaves the head to FAIRChem (`HydraModel` + the MLP energy head; the
backbone returns only {"node_embedding", "batch"}, wrapper.py:212).  FAIRChem is absent, so
this module provides the equivalent conservative head: per-atom energy from the l=0
channels by an MLP, per-system sum, forces = -dE/dpos and stress from the pos/cell
gradients, all through torch autograd (which runs the HIP backward kernels of ops/*).

Stress: for strain eps applied to positions and cell, dE/deps_ab =
sum_i pos_ia dE/dpos_ib + sum_k cell_ka dE/dcell_kb, and stress = (1/V) dE/deps, V = |det cell|.
"""
from __future__ import annotations

import math
from types import SimpleNamespace

import numpy as np
import torch
import torch.nn as nn
import torch.nn.functional as F


class MLPEnergyHead(nn.Module):
    """E_atom = MLP(node_embedding[:, 0, :]); E_system = sum over the system's atoms."""

    def __init__(self, sphere_channels: int, hidden_channels: int, seed: int = 1):
        super().__init__()
        g = torch.Generator().manual_seed(seed)
        dims = [sphere_channels, hidden_channels, hidden_channels, 1]
        self.layers = nn.ModuleList()
        for a, b in zip(dims[:-1], dims[1:]):
            lin = nn.Linear(a, b)
            bound = 1.0 / math.sqrt(a)
            with torch.no_grad():
                lin.weight.uniform_(-bound, bound, generator=g)
                lin.bias.uniform_(-bound, bound, generator=g)
            self.layers.append(lin)

    def atom_energy(self, node_embedding: torch.Tensor) -> torch.Tensor:
        h = node_embedding[:, 0, :]
        for k, lin in enumerate(self.layers):
            h = lin(h)
            if k < len(self.layers) - 1:
                h = F.silu(h)
        return h.squeeze(-1)


def system_sum(values: torch.Tensor, natoms: list) -> torch.Tensor:
    """Per-system sum over the leading (atom) dimension; systems are contiguous runs of
    natoms[s] atoms (FAIRChem batches).  One fixed-order reduction per system, no atomics."""
    if len(natoms) == 1:
        return values.sum(0, keepdim=True)
    return torch.stack([v.sum(0) for v in values.split(natoms)])


class PotentialModel(nn.Module):
    """backbone (ZeroAllocBackbone) + energy head, returning energy, forces and stress."""

    def __init__(self, backbone: nn.Module, head: MLPEnergyHead):
        super().__init__()
        self.backbone = backbone
        self.head = head
        for p in self.head.parameters():
            p.requires_grad_(False)

    def forward(self, data, compute_forces: bool = True, compute_stress: bool = False, natoms=None) -> dict:
        """natoms: atoms per system as a host list.  When omitted it is the atom count for a
        single system (known on the host) and data.natoms read back otherwise; that read is a
        device-to-host copy, which stalls the launch queue mid-step and which graph capture
        forbids, so batched callers on a hot loop pass natoms."""
        emb = self.backbone(data)
        e_atom = self.head.atom_energy(emb["node_embedding"])
        if natoms is None:
            if data.natoms.numel() == 1:
                natoms = [int(data.pos.shape[0])]
            else:
                natoms = [int(n) for n in data.natoms.tolist()]
        energy = system_sum(e_atom, natoms)
        out = {"energy": energy, "atom_energy": e_atom, "node_embedding": emb["node_embedding"]}
        if compute_forces or compute_stress:
            inputs = [data.pos] + ([data.cell] if compute_stress else [])
            grads = torch.autograd.grad(energy.sum(), inputs, allow_unused=True)
            g_pos = grads[0] if grads[0] is not None else torch.zeros_like(data.pos)
            out["forces"] = -g_pos
            if compute_stress:
                g_cell = grads[1] if grads[1] is not None else torch.zeros_like(data.cell)
                out["stress"] = stress_from_gradients(data.pos, data.cell, g_pos, g_cell, natoms)
        return out


def stress_from_gradients(pos, cell, g_pos, g_cell, natoms: list):
    """(1/V) (sum_i pos_i^T g_pos_i + cell^T g_cell) per system, (S, 3, 3)."""
    n_sys = len(natoms)
    pos = pos.detach()
    cell = cell.detach().reshape(n_sys, 3, 3)
    g_cell = g_cell.reshape(n_sys, 3, 3)
    w = system_sum(pos[:, :, None] * g_pos[:, None, :], natoms)
    w = w + cell.transpose(1, 2) @ g_cell
    # |det cell| as the triple product a . (b x c) (elementwise, no solver call)
    vol = (cell[:, 0] * torch.linalg.cross(cell[:, 1], cell[:, 2])).sum(-1).abs().reshape(n_sys, 1, 1)
    return w / vol


def make_atomic_data(system, edge_index, cell_offsets, device, dtype=torch.float32,
                     charge: int = 0, spin: int = 0):
    """Data object with the attribute names of FAIRChem's AtomicData that the backbone reads
    (wrapper.py:173-210): one system, batch = 0."""
    n = system.n_atoms
    E = edge_index.shape[1]
    return SimpleNamespace(
        pos=torch.as_tensor(system.pos, dtype=dtype, device=device).clone(),
        atomic_numbers=torch.as_tensor(system.Z, dtype=torch.long, device=device),
        cell=torch.as_tensor(system.cell, dtype=dtype, device=device).reshape(1, 3, 3).clone(),
        pbc=torch.as_tensor(system.pbc, device=device).reshape(1, 3),
        natoms=torch.tensor([n], dtype=torch.long, device=device),
        edge_index=torch.as_tensor(edge_index, dtype=torch.long, device=device),
        cell_offsets=torch.as_tensor(cell_offsets, dtype=dtype, device=device),
        nedges=torch.tensor([E], dtype=torch.long, device=device),
        charge=torch.tensor([charge], dtype=torch.long, device=device),
        spin=torch.tensor([spin], dtype=torch.long, device=device),
        batch=torch.zeros(n, dtype=torch.long, device=device),
    )


def make_batch_data(items, device, dtype=torch.float32):
    """One FAIRChem-style batch of several systems: items = [(system, edge_index,
    cell_offsets, charge, spin), ...].  Atoms and edges are concatenated system by system,
    edge indices offset by the atoms before, batch / natoms / nedges / cell / charge / spin
    per system (the layout wrapper.py:173-210 reads)."""
    pos, Z, cells, ei, off, batch, natoms, nedges, chg, spn = [], [], [], [], [], [], [], [], [], []
    base = 0
    for s, (system, edge_index, cell_offsets, charge, spin) in enumerate(items):
        n = system.n_atoms
        pos.append(np.asarray(system.pos, dtype=np.float32))
        Z.append(np.asarray(system.Z, dtype=np.int64))
        cells.append(np.asarray(system.cell, dtype=np.float32).reshape(1, 3, 3))
        ei.append(np.asarray(edge_index, dtype=np.int64) + base)
        off.append(np.asarray(cell_offsets, dtype=np.float32))
        batch.append(np.full(n, s, dtype=np.int64))
        natoms.append(n)
        nedges.append(np.asarray(edge_index).shape[1])
        chg.append(charge)
        spn.append(spin)
        base += n
    t = lambda a, dt: torch.as_tensor(a, dtype=dt, device=device)
    return SimpleNamespace(
        pos=t(np.concatenate(pos), dtype).clone(), atomic_numbers=t(np.concatenate(Z), torch.long),
        cell=t(np.concatenate(cells), dtype).clone(), natoms=t(natoms, torch.long),
        edge_index=t(np.concatenate(ei, axis=1), torch.long), cell_offsets=t(np.concatenate(off), dtype),
        nedges=t(nedges, torch.long), charge=t(chg, torch.long), spin=t(spn, torch.long),
        batch=t(np.concatenate(batch), torch.long), pbc=t(np.ones((len(items), 3), dtype=bool), torch.bool))
