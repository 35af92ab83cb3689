"""One energy + forces (+ stress) step captured in a HIP graph and replayed with new positions.

For MD and other loops that evaluate the same graph many times (the water-box workload
holds its step-0 graph for 100 steps): after capture, each step is one graph launch instead
of several hundred kernel launches plus the Python that issues them, which dominates small
systems (a 29-atom cell spends ~3.9 ms per eager step, almost all of it launch and host
work).  The reference has no counterpart; its CSR cache only removes the graph preprocessing.

Held fixed by a capture: the atoms (N, Z, batch, charge, spin), edge_index, cell_offsets,
the device buffers of data.pos / data.cell and the returned output tensors.  New positions
(and cells) are copied into those buffers before each replay; the outputs are overwritten
in place by every replay (clone them to keep a step's result).  When the graph changes
(neighbour-list rebuild), make a new CapturedStep.

The step contains no hipMemsetAsync (fills are kernels) and no host synchronisation; the
replay results equal the eager results bitwise (tests/test_gpu_captured.py).
"""
from __future__ import annotations

import torch


class CapturedStep:
    def __init__(self, model, data, compute_stress: bool = False, warmup: int = 2):
        """model: heads.PotentialModel (ZeroAllocBackbone + energy head) on the GPU; data:
        its AtomicData-like input, whose pos / cell tensors become the replay inputs."""
        self.model, self.data, self.compute_stress = model, data, bool(compute_stress)
        self.natoms = [int(n) for n in data.natoms.tolist()]
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            # eager warm-up on the capture stream: builds and caches the topology, checks
            # the atoms, and lets the allocator settle
            for _ in range(max(1, warmup)):
                model(data, compute_forces=True, compute_stress=self.compute_stress, natoms=self.natoms)
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph):
            self.out = model(data, compute_forces=True, compute_stress=self.compute_stress, natoms=self.natoms)

    @torch.no_grad()
    def __call__(self, pos: torch.Tensor, cell: torch.Tensor | None = None) -> dict:
        """Copy pos (N, 3) (and cell) into the captured buffers and replay; returns the
        captured output dict (energy, atom_energy, node_embedding, forces[, stress])."""
        self.data.pos.copy_(pos)
        if cell is not None:
            self.data.cell.copy_(cell.reshape(self.data.cell.shape))
        self.graph.replay()
        return self.out
