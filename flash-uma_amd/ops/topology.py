"""Graph topology on the GPU: Morton atom order, receiver-sorted edge order and the
receiver and sender CSRs (model.py:17-74, plus the sender CSR the deterministic backward
needs).  Everything integer is computed by the C-ABI kernels and is bit-exact.

Edge order.  The reference keeps edges in input order and reaches a receiver's edges
through col_idx = stable argsort(idx_j) (model.py:20-26).  Here the edges are permuted once
into exactly that order, so the receiver CSR becomes (row_ptr, arange(E)): every per-edge
array is then read contiguously by the segment kernels.  Within each receiver segment the
edges keep their input order (stable sort), so every floating-point sum runs in the same
order as the reference's CSR walk and the results do not depend on the Morton permutation.
"""
from __future__ import annotations

from collections import OrderedDict
from dataclasses import dataclass

import torch

from . import _lib


@dataclass
class GraphTopology:
    N: int
    E: int
    perm: torch.Tensor          # (N,) int64: Morton order -> input atom index
    inv_perm: torch.Tensor      # (N,) int64: input atom index -> Morton position
    edge_perm: torch.Tensor     # (E,) int64: sorted edge position -> input edge index
    idx_i: torch.Tensor         # (E,) int64 senders, Morton atom ids, sorted edge order
    idx_j: torch.Tensor         # (E,) int64 receivers (non-decreasing)
    recv_ptr: torch.Tensor      # (N+1,) int32
    recv_idx: torch.Tensor      # (E,) int32 = arange(E)
    send_ptr: torch.Tensor      # (N+1,) int32
    send_idx: torch.Tensor      # (E,) int32: sorted edge positions grouped by sender
    source: torch.Tensor | None = None  # the edge_index this was built from (kept alive)


def _bits_for(n: int) -> int:
    return max(1, int(n - 1).bit_length()) if n > 1 else 1


def sort_pairs(keys: torch.Tensor, vals: torch.Tensor, end_bit: int):
    """Stable GPU radix sort of int64 (key, value) pairs on bits [0, end_bit)."""
    n = keys.numel()
    dev = keys.device
    keys_out = torch.empty_like(keys)
    vals_out = torch.empty_like(vals)
    import ctypes
    ws = ctypes.c_size_t(0)
    st = _lib.stream_ptr(dev)
    _lib.call("fu_sort_pairs_i64", keys.data_ptr(), keys_out.data_ptr(), vals.data_ptr(), vals_out.data_ptr(),
              n, 0, end_bit, None, ctypes.byref(ws), st)
    workspace = torch.empty(max(int(ws.value), 1), dtype=torch.uint8, device=dev)
    _lib.call("fu_sort_pairs_i64", keys.data_ptr(), keys_out.data_ptr(), vals.data_ptr(), vals_out.data_ptr(),
              n, 0, end_bit, workspace.data_ptr(), ctypes.byref(ws), st)
    return keys_out, vals_out


def morton_permutation(pos: torch.Tensor, batch: torch.Tensor):
    """(perm, inv_perm) of reorder_graph_morton (model.py:60-72), stable."""
    pos = _lib.require(pos.detach(), torch.float32, "pos")
    batch = _lib.require(batch, torch.int64, "batch")
    N = pos.shape[0]
    dev = pos.device
    st = _lib.stream_ptr(dev)
    keys = torch.empty(N, dtype=torch.int64, device=dev)
    _lib.call("fu_morton_keys", pos.data_ptr(), batch.data_ptr(), keys.data_ptr(), N, st)
    n_sys = int(batch.max().item()) + 1 if N > 0 else 1
    end_bit = 31 if n_sys == 1 else 32 + _bits_for(n_sys)   # Morton codes occupy bits 1..30
    ar = torch.arange(N, dtype=torch.int64, device=dev)
    _, perm = sort_pairs(keys, ar, end_bit)
    inv = torch.empty_like(perm)
    _lib.call("fu_invert_perm", perm.data_ptr(), inv.data_ptr(), N, st)
    return perm, inv


def take(table: torch.Tensor, idx: torch.Tensor) -> torch.Tensor:
    out = torch.empty_like(idx)
    _lib.call("fu_take_i64", table.data_ptr(), table.numel(), idx.data_ptr(), out.data_ptr(), idx.numel(),
              _lib.stream_ptr(idx.device))
    return out


def csr_from_keys(keys: torch.Tensor, N: int):
    """(row_ptr int32, order int64, sorted keys) for a stable sort of edge keys in [0, N)."""
    E = keys.numel()
    dev = keys.device
    ar = torch.arange(E, dtype=torch.int64, device=dev)
    sk, order = sort_pairs(keys, ar, _bits_for(N))
    row_ptr = torch.empty(N + 1, dtype=torch.int32, device=dev)
    _lib.call("fu_csr_row_ptr", sk.data_ptr(), E, row_ptr.data_ptr(), N, _lib.stream_ptr(dev))
    return row_ptr, order, sk


def narrow32(t: torch.Tensor) -> torch.Tensor:
    out = torch.empty(t.shape, dtype=torch.int32, device=t.device)
    _lib.call("fu_narrow_i64_i32", t.data_ptr(), out.data_ptr(), t.numel(), _lib.stream_ptr(t.device))
    return out


def check_indices(edge_index: torch.Tensor, N: int) -> None:
    if edge_index.numel() == 0:
        return
    lo, hi = int(edge_index.min().item()), int(edge_index.max().item())
    if lo < 0 or hi >= N:
        raise _lib.FlashUMAError(f"edge_index holds atom ids in [{lo}, {hi}], outside [0, {N})")
    if edge_index.shape[1] >= 2**31:
        raise _lib.FlashUMAError("more than 2^31 - 1 edges are not supported (int32 CSR)")


def build_topology(pos: torch.Tensor, batch: torch.Tensor, edge_index: torch.Tensor) -> GraphTopology:
    # the cache keys on the caller's tensor, so that tensor (not a converted copy) is the
    # one kept alive in the entry
    source = edge_index
    edge_index = _lib.require(edge_index, torch.int64, "edge_index")
    batch = _lib.require(batch, torch.int64, "batch")
    N = pos.shape[0]
    E = edge_index.shape[1]
    check_indices(edge_index, N)
    dev = pos.device
    perm, inv = morton_permutation(pos, batch)
    idx_i_m = take(inv, edge_index[0].contiguous())
    idx_j_m = take(inv, edge_index[1].contiguous())
    recv_ptr, edge_perm, idx_j_sorted = csr_from_keys(idx_j_m, N)
    idx_i_sorted = take(idx_i_m, edge_perm)
    send_ptr, send_order, _ = csr_from_keys(idx_i_sorted, N)
    recv_idx = torch.arange(E, dtype=torch.int32, device=dev)
    return GraphTopology(N=N, E=E, perm=perm, inv_perm=inv, edge_perm=edge_perm, idx_i=idx_i_sorted,
                         idx_j=idx_j_sorted, recv_ptr=recv_ptr, recv_idx=recv_idx, send_ptr=send_ptr,
                         send_idx=narrow32(send_order), source=source)


_TOPO_CAPACITY = 8
_topo_cache: "OrderedDict[tuple, GraphTopology]" = OrderedDict()
_topo_stats = {"hits": 0, "builds": 0}


def get_topology(pos: torch.Tensor, batch: torch.Tensor, edge_index: torch.Tensor) -> GraphTopology:
    """Topology cached across calls (MD steps with a fixed graph).

    Key: (edge_index storage address, its in-place version counter, shape, N, device).  The
    cache entry keeps edge_index alive, so its address cannot be recycled for another graph
    while the entry exists; an in-place edit bumps the version and forces a rebuild.  The
    Morton order is frozen at build time: it only decides memory placement, never results."""
    key = (edge_index.data_ptr(), edge_index._version, tuple(edge_index.shape), pos.shape[0],
           pos.device.index)
    hit = _topo_cache.get(key)
    if hit is not None:
        _topo_cache.move_to_end(key)
        _topo_stats["hits"] += 1
        return hit
    topo = build_topology(pos, batch, edge_index)
    _topo_stats["builds"] += 1
    _topo_cache[key] = topo
    if len(_topo_cache) > _TOPO_CAPACITY:
        _topo_cache.popitem(last=False)
    return topo


def clear_topology_cache() -> None:
    _topo_cache.clear()
    _topo_stats["hits"] = _topo_stats["builds"] = 0


def topology_cache_stats() -> dict:
    """{'entries', 'hits', 'builds'} since the last clear_topology_cache()."""
    return {"entries": len(_topo_cache), **_topo_stats}


def sender_csr(idx_i: torch.Tensor, N: int):
    """(send_ptr, send_idx int32) over an arbitrary edge order."""
    ptr, order, _ = csr_from_keys(_lib.require(idx_i, torch.int64, "idx_i"), N)
    return ptr, narrow32(order)


def receiver_csr(idx_j: torch.Tensor, N: int):
    """(row_ptr, col_idx int32) over an arbitrary edge order (model.py:20-26)."""
    ptr, order, _ = csr_from_keys(_lib.require(idx_j, torch.int64, "idx_j"), N)
    return ptr, narrow32(order)
