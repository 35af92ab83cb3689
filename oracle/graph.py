"""Integer graph preprocessing, restated in numpy — test infrastructure only.

Restates model.py:17-74 (Morton reorder, receiver CSR) and defines the neighbour list the
build uses in place of FAIRChem's a2g (absent from the reference tree).

Pins:
  - expand_bits_loop / morton_code_loop: a per-bit loop, independent of the magic-mask
    restatement (morton_code) — checked equal on every 10-bit value.
  - csr: numpy stable argsort + bincount (model.py:20-26), checked against a pure-Python
    segment construction on small inputs.
  - neighbor_list_bruteforce: all pairs x all periodic images, exact fp64 ordering — the
    reference for the product's cell-list neighbour list.
"""
from __future__ import annotations

import itertools

import numpy as np


def expand_bits(v: np.ndarray) -> np.ndarray:
    """Spread the low 10 bits of v, bit k -> bit 3k + 1 (model.py:48-54: the four mask steps of
    the usual 3k spread, then a fifth that lifts every bit by one)."""
    v = v.astype(np.int64)
    v = (v | (v << 16)) & 0x030000FF
    v = (v | (v << 8)) & 0x0300F00F
    v = (v | (v << 4)) & 0x030C30C3
    v = (v | (v << 2)) & 0x09249249
    v = (v | (v << 1)) & 0x12492492
    return v


def expand_bits_loop(v: int) -> int:
    """Same map as expand_bits by an explicit bit loop: bit k of v -> bit 3k + 1."""
    out = 0
    for k in range(10):
        if (v >> k) & 1:
            out |= 1 << (3 * k + 1)
    return out


def morton_code(ix: np.ndarray, iy: np.ndarray, iz: np.ndarray) -> np.ndarray:
    """x -> bit 3k+1, y -> bit 3k+2, z -> bit 3k+3 (model.py:56-58)."""
    return expand_bits(ix) | (expand_bits(iy) << 1) | (expand_bits(iz) << 2)


def morton_code_loop(ix: int, iy: int, iz: int) -> int:
    return expand_bits_loop(ix) | (expand_bits_loop(iy) << 1) | (expand_bits_loop(iz) << 2)


def morton_keys(pos: np.ndarray, batch: np.ndarray) -> np.ndarray:
    """Sort keys of reorder_graph_morton (model.py:61-68) with the reference's fp32
    arithmetic: scale = 1023 / max(max - min, 1e-5), q = int32((pos - min) * scale)."""
    pos = np.asarray(pos, dtype=np.float32)
    pmin = pos.min(axis=0)
    pmax = pos.max(axis=0)
    rng = np.maximum(pmax - pmin, np.float32(1e-5)).astype(np.float32)
    scale = (np.float32(1023.0) / rng).astype(np.float32)
    q = ((pos - pmin).astype(np.float32) * scale).astype(np.float32).astype(np.int32)
    code = morton_code(q[:, 0], q[:, 1], q[:, 2]).astype(np.int64)
    return code | (np.asarray(batch, dtype=np.int64) << 32)


def reorder_graph_morton(pos, Z, batch, idx_i, idx_j):
    """model.py:60-74 with a stable sort (the reference's argsort is unstable; keys of
    min-separated atoms are unique, so the permutation is the same)."""
    keys = morton_keys(pos, batch)
    perm = np.argsort(keys, kind="stable")
    inv = np.empty_like(perm)
    inv[perm] = np.arange(len(perm))
    return (np.asarray(pos)[perm], np.asarray(Z)[perm], np.asarray(batch)[perm],
            inv[idx_i], inv[idx_j], perm, inv)


def csr(keys: np.ndarray, n: int):
    """_build_csr_uncached (model.py:20-26): col_idx = stable argsort(keys) as int32,
    row_ptr = [0, cumsum(bincount(keys, n))] as int32."""
    keys = np.asarray(keys, dtype=np.int64)
    col = np.argsort(keys, kind="stable").astype(np.int32)
    counts = np.bincount(keys, minlength=n)
    row_ptr = np.zeros(n + 1, dtype=np.int32)
    row_ptr[1:] = np.cumsum(counts)
    return row_ptr, col


def csr_loop(keys, n):
    """Pure-Python segment construction, for checking csr() on small inputs."""
    segs = [[] for _ in range(n)]
    for e, k in enumerate(keys):
        segs[int(k)].append(e)
    row_ptr = [0]
    col = []
    for s in segs:
        col.extend(s)
        row_ptr.append(len(col))
    return np.asarray(row_ptr, dtype=np.int32), np.asarray(col, dtype=np.int32)


def neighbor_list_bruteforce(pos, cell, pbc, cutoff: float, max_neighbors: int):
    """Radius graph with a per-receiver cap, by brute force over all pairs and images.

    Definition (the build's stand-in for FAIRChem a2g): for receiver j, candidates are
    (i, o) with o an integer cell offset (zero on non-periodic axes), (i, o) != (j, 0),
    d = (pos_i - pos_j) + o @ cell evaluated in float64 from the float32 inputs as
    dx = (x_i - x_j) + ((o0 c0x + o1 c1x) + o2 c2x), and |d|^2 = (dx dx + dy dy) + dz dz
    < cutoff^2.  Candidates are ordered by (|d|^2, i, o0, o1, o2) and the first
    max_neighbors are kept.  Edges are grouped by receiver (ascending), in that order.
    Returns edge_index (2, E) int64 [sender; receiver] and cell_offsets (E, 3) float32.
    """
    pos = np.asarray(pos, dtype=np.float32).astype(np.float64)
    cell = np.asarray(cell, dtype=np.float32).astype(np.float64)
    n = pos.shape[0]
    reps = []
    for ax in range(3):
        if pbc[ax]:
            # perpendicular width of the cell along axis ax
            other = [cell[(ax + 1) % 3], cell[(ax + 2) % 3]]
            normal = np.cross(other[0], other[1])
            width = abs(np.dot(cell[ax], normal)) / np.linalg.norm(normal)
            reps.append(int(np.ceil(cutoff / width)) + 1)
        else:
            reps.append(0)
    offsets = np.array(list(itertools.product(*[range(-r, r + 1) for r in reps])), dtype=np.int64)
    cut2 = float(cutoff) * float(cutoff)
    senders, receivers, offs = [], [], []
    for j in range(n):
        cand = []
        for o in offsets:
            sh = (o[0] * cell[0] + o[1] * cell[1]) + o[2] * cell[2]
            d = (pos - pos[j]) + sh
            d2 = (d[:, 0] * d[:, 0] + d[:, 1] * d[:, 1]) + d[:, 2] * d[:, 2]
            ok = np.nonzero(d2 < cut2)[0]
            for i in ok:
                if i == j and not o.any():
                    continue
                cand.append((d2[i], int(i), int(o[0]), int(o[1]), int(o[2])))
        cand.sort()
        for c in cand[:max_neighbors]:
            senders.append(c[1])
            receivers.append(j)
            offs.append(c[2:])
    edge_index = np.array([senders, receivers], dtype=np.int64).reshape(2, -1)
    cell_offsets = np.array(offs, dtype=np.float32).reshape(-1, 3)
    return edge_index, cell_offsets
