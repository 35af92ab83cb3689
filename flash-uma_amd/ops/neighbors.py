"""Capped periodic radius graph on the GPU (the graph FAIRChem's a2g hands the reference,
readme.md:34), bit-identical to the host builder `systems.neighbor_list`.

radius_graph(pos, cell, pbc, cutoff, max_neighbors) -> (edge_index (2, E) int64,
cell_offsets (E, 3) float32), both on the positions' device; definition in csrc/nlist.hip.

NeighborList adds the MD-side policy.  With skin = 0 (default) it rebuilds on every call,
which reproduces the capped host graph of the current positions.  With skin > 0 it builds an
uncapped graph at cutoff + skin and keeps it (and so the cached topology) while no atom has
moved more than skin / 2 and the cell and periodicity are unchanged: every pair within the
cutoff of the current positions is then still in the graph, and the extra pairs lie at or
beyond the cutoff, where the envelope and its derivative vanish, so energies and forces
equal those of a fresh uncapped graph.  A per-receiver cap cannot be kept under reuse (the
nearest-K set changes as atoms move), so skin > 0 refuses max_neighbors."""
from __future__ import annotations

import math

import numpy as np
import torch

from . import _lib
from .topology import csr_from_keys

NL_CAP = 512      # within-cutoff candidates held per receiver (csrc/nlist.hip)
_MAX_WRAP = 60    # |floor(fractional coordinate)| allowed (offsets are encoded in 8 bits)


def _geometry(cell, pbc, cutoff: float):
    cell64 = np.asarray(cell, dtype=np.float32).astype(np.float64).reshape(3, 3)
    inv = np.linalg.inv(cell64)
    nb, reach = [], []
    for ax in range(3):
        if pbc[ax]:
            a, b = cell64[(ax + 1) % 3], cell64[(ax + 2) % 3]
            normal = np.cross(a, b)
            width = abs(float(np.dot(cell64[ax], normal))) / float(np.linalg.norm(normal))
            n = max(1, int(math.floor(width / (cutoff + 1e-3))))
            nb.append(n)
            reach.append(int(math.ceil((cutoff + 1e-3) / (width / n))))
        else:
            nb.append(1)
            reach.append(0)
    arr = lambda v, t: np.ascontiguousarray(np.asarray(v, dtype=t))
    return (arr(cell64.ravel(), np.float64), arr(inv.ravel(), np.float64), arr(nb, np.int32), arr(reach, np.int32),
            arr([1 if p else 0 for p in pbc], np.int32))


def radius_graph(pos: torch.Tensor, cell, pbc, cutoff: float, max_neighbors: int):
    """Receivers ascending; per receiver the max_neighbors nearest (i, o) by
    (|d|^2, i, o0, o1, o2) with |d| < cutoff; float64 distances as in systems.neighbor_list."""
    pos = _lib.require(pos.detach(), torch.float32, "pos")
    N = pos.shape[0]
    dev = pos.device
    st = _lib.stream_ptr(dev)
    if N == 0:
        return (torch.zeros(2, 0, dtype=torch.int64, device=dev), torch.zeros(0, 3, dtype=torch.float32, device=dev))
    cell_h, inv_h, nb_h, reach_h, pbc_h = _geometry(cell, pbc, float(cutoff))
    ptr = lambda a: a.ctypes.data
    key = torch.empty(N, dtype=torch.int64, device=dev)
    wrap = torch.empty(N, 3, dtype=torch.int32, device=dev)
    _lib.call("fu_nlist_bin", pos.data_ptr(), N, ptr(cell_h), ptr(inv_h), ptr(nb_h), ptr(reach_h), ptr(pbc_h),
              key.data_ptr(), wrap.data_ptr(), st)
    if int(wrap.abs().max().item()) > _MAX_WRAP:
        raise _lib.FlashUMAError("radius_graph: positions lie too far outside the cell; wrap them first")
    nbins = int(np.prod(nb_h))
    bin_ptr, atoms, sorted_keys = csr_from_keys(key, nbins)
    K = int(max_neighbors)
    sender = torch.empty(N, K, dtype=torch.int32, device=dev)
    off = torch.empty(N, K, 3, dtype=torch.int32, device=dev)
    count = torch.empty(N, dtype=torch.int32, device=dev)
    nout = torch.empty(N, dtype=torch.int32, device=dev)
    _lib.call("fu_nlist_search", pos.data_ptr(), atoms.data_ptr(), bin_ptr.data_ptr(), wrap.data_ptr(),
              key.data_ptr(), N, ptr(cell_h), ptr(inv_h), ptr(nb_h), ptr(reach_h), ptr(pbc_h), float(cutoff), K,
              sender.data_ptr(), off.data_ptr(), count.data_ptr(), nout.data_ptr(), st)
    row_ptr = torch.empty(N + 1, dtype=torch.int64, device=dev)
    _lib.call("fu_nlist_scan", nout.data_ptr(), row_ptr.data_ptr(), N, st)
    E = int(row_ptr[N].item())
    if int(count.max().item()) > NL_CAP:
        raise _lib.FlashUMAError(f"radius_graph: more than {NL_CAP} atoms within the cutoff of one receiver")
    edge_index = torch.empty(2, E, dtype=torch.int64, device=dev)
    cell_offsets = torch.empty(E, 3, dtype=torch.float32, device=dev)
    _lib.call("fu_nlist_emit", sender.data_ptr(), off.data_ptr(), nout.data_ptr(), row_ptr.data_ptr(), N, K,
              edge_index.data_ptr(), cell_offsets.data_ptr(), E, st)
    return edge_index, cell_offsets


class NeighborList:
    """Graph holder for MD.

    skin = 0: radius_graph(pos, cell, pbc, cutoff, max_neighbors) on every call.
    skin > 0 (max_neighbors must be None): an uncapped graph at cutoff + skin, rebuilt when
    some atom has moved more than skin / 2 since the last build or when the cell or the
    periodic axes change; otherwise the same edge_index tensor is returned, so the
    backbone's topology cache (keyed on that tensor) is reused."""

    def __init__(self, cutoff: float, max_neighbors: int | None, skin: float = 0.0):
        if skin < 0.0:
            raise ValueError("skin must be >= 0")
        if skin > 0.0 and max_neighbors is not None:
            raise ValueError("a neighbour cap cannot be kept while a graph is reused: NeighborList with "
                             "skin > 0 needs max_neighbors=None (uncapped)")
        if skin == 0.0 and max_neighbors is None:
            max_neighbors = NL_CAP
        self.cutoff, self.skin = float(cutoff), float(skin)
        self.max_neighbors = NL_CAP if max_neighbors is None else int(max_neighbors)
        self._ref_pos = None
        self._ref_cell = None
        self._ref_pbc = None
        self._graph = None
        self.builds = 0

    def __call__(self, pos: torch.Tensor, cell, pbc):
        pos = pos.detach()
        cell64 = np.asarray(cell, dtype=np.float64).reshape(3, 3)
        pbc_t = tuple(bool(p) for p in pbc)
        if (self._graph is not None and self.skin > 0.0 and pbc_t == self._ref_pbc
                and np.array_equal(cell64, self._ref_cell) and pos.shape == self._ref_pos.shape):
            moved = (pos - self._ref_pos).norm(dim=1).max().item() if pos.shape[0] else 0.0
            if moved <= 0.5 * self.skin:
                return self._graph
        self._graph = radius_graph(pos, cell, pbc, self.cutoff + self.skin, self.max_neighbors)
        self._ref_pos = pos.clone()
        self._ref_cell = cell64.copy()
        self._ref_pbc = pbc_t
        self.builds += 1
        return self._graph
