"""Synthetic atomic systems and the radius graph that feeds the backbone.

The reference takes its graph from FAIRChem's a2g (pymatgen, CPU) outside the backbone
(readme.md:34); neither is in the reference tree.  This module builds the five benchmark
systems (seeded numpy PCG64, float64 generation, float32 output) and their neighbour list
on the host, before any timed region:

  neighbor_list(): for receiver j, candidates (i, o) with o an integer cell offset (zero on
  non-periodic axes), (i, o) != (j, 0) and
      d = (pos_i - pos_j) + ((o0 c0 + o1 c1) + o2 c2)        in float64 from float32 input,
      |d|^2 = (dx dx + dy dy) + dz dz  <  cutoff^2,
  ordered by (|d|^2, i, o0, o1, o2); the first max_neighbors are kept.  Edges are grouped by
  receiver in ascending order.  edge_index = [sender; receiver] (int64), cell_offsets (E, 3).
"""
from __future__ import annotations

import itertools
import math
from dataclasses import dataclass, field

import numpy as np

# Element symbols used by the configs.
Z_OF = {"H": 1, "C": 6, "N": 7, "O": 8, "Si": 14, "Fe": 26, "Cu": 29, "Pt": 78}


@dataclass
class AtomicSystem:
    """One periodic structure: float32 positions (N, 3), int64 atomic numbers, float32 cell
    (3, 3) with lattice vectors as rows, and per-axis periodicity."""
    name: str
    pos: np.ndarray
    Z: np.ndarray
    cell: np.ndarray
    pbc: tuple = (True, True, True)
    info: dict = field(default_factory=dict)

    @property
    def n_atoms(self) -> int:
        return int(self.pos.shape[0])


def _wrap(pos: np.ndarray, L: np.ndarray) -> np.ndarray:
    return pos - np.floor(pos / L) * L


def cu_slab_co(seed: int = 0, jitter: float = 0.02) -> AtomicSystem:
    """Config 1: 3x3x3 Cu fcc(100) slab (a = 3.61 A, 8 A vacuum on each side, periodic)
    with CO at a bridge site, C 2.0 A above the top layer and O 1.13 A above C."""
    a = 3.61
    d = a / math.sqrt(2.0)           # in-plane nearest-neighbour spacing of fcc(100)
    nx = ny = nl = 3
    vac = 8.0
    Lx, Ly = nx * d, ny * d
    Lz = 2 * vac + (nl - 1) * a / 2.0
    pos = []
    for layer in range(nl):
        shift = 0.5 * (layer % 2)
        z = vac + layer * a / 2.0
        for ix in range(nx):
            for iy in range(ny):
                pos.append([(ix + shift) * d, (iy + shift) * d, z])
    top = vac + (nl - 1) * a / 2.0
    top_shift = 0.5 * ((nl - 1) % 2)
    bridge = [(top_shift + 0.5) * d, (top_shift) * d]   # midway between two top-layer atoms
    pos.append([bridge[0], bridge[1], top + 2.0])
    pos.append([bridge[0], bridge[1], top + 2.0 + 1.13])
    pos = np.array(pos, dtype=np.float64)
    rng = np.random.default_rng(seed)
    pos = pos + rng.normal(0.0, jitter, size=pos.shape)
    Z = np.array([Z_OF["Cu"]] * (nx * ny * nl) + [Z_OF["C"], Z_OF["O"]], dtype=np.int64)
    cell = np.diag([Lx, Ly, Lz])
    return AtomicSystem("cu_slab_co", pos.astype(np.float32), Z, cell.astype(np.float32))


def _random_unit(rng, n):
    v = rng.normal(size=(n, 3))
    return v / np.linalg.norm(v, axis=1, keepdims=True)


def _rsa(rng, n: int, L: float, dmin: float) -> np.ndarray:
    """Random sequential addition of n points in a periodic cube of side L with minimum
    pairwise (minimum-image) distance dmin, accelerated by a grid of cell >= dmin."""
    nb = max(1, int(L // dmin))
    h = L / nb
    grid: dict = {}
    out = np.empty((n, 3))
    k = 0
    d2 = dmin * dmin
    while k < n:
        p = rng.uniform(0.0, L, size=3)
        c = tuple((p // h).astype(int) % nb)
        ok = True
        for dc in itertools.product((-1, 0, 1), repeat=3):
            cc = ((c[0] + dc[0]) % nb, (c[1] + dc[1]) % nb, (c[2] + dc[2]) % nb)
            for q in grid.get(cc, ()):
                dv = p - out[q]
                dv -= L * np.round(dv / L)
                if dv @ dv < d2:
                    ok = False
                    break
            if not ok:
                break
        if ok:
            out[k] = p
            grid.setdefault(c, []).append(k)
            k += 1
    return out


def water_box(n_mol: int = 333, L: float = 21.5, seed: int = 0) -> AtomicSystem:
    """Config 2: periodic liquid-water box; O by random sequential addition (min O-O 2.6 A),
    H at 0.96 A with H-O-H 104.5 deg in a random orientation."""
    rng = np.random.default_rng(seed)
    O = _rsa(rng, n_mol, L, 2.6)
    half = math.radians(104.5) / 2.0
    pos = []
    Z = []
    for k in range(n_mol):
        u = _random_unit(rng, 1)[0]               # bisector direction
        w = _random_unit(rng, 1)[0]
        w = w - (w @ u) * u
        w /= np.linalg.norm(w)                    # in-plane perpendicular
        h1 = O[k] + 0.96 * (math.cos(half) * u + math.sin(half) * w)
        h2 = O[k] + 0.96 * (math.cos(half) * u - math.sin(half) * w)
        pos += [O[k], h1, h2]
        Z += [Z_OF["O"], Z_OF["H"], Z_OF["H"]]
    pos = _wrap(np.array(pos), L)
    return AtomicSystem("water_box", pos.astype(np.float32), np.array(Z, dtype=np.int64),
                        np.diag([L, L, L]).astype(np.float32))


def bcc_fe(n_rep: int = 16, a: float = 2.87, jitter: float = 0.05, seed: int = 0) -> AtomicSystem:
    """Config 3/5: bcc Fe supercell of n_rep^3 conventional cells with Gaussian jitter."""
    rng = np.random.default_rng(seed)
    g = np.arange(n_rep, dtype=np.float64)
    base = np.stack(np.meshgrid(g, g, g, indexing="ij"), -1).reshape(-1, 3)
    pos = np.concatenate([base, base + 0.5], 0) * a
    # interleave the two basis atoms per conventional cell
    pos = pos.reshape(2, -1, 3).transpose(1, 0, 2).reshape(-1, 3)
    pos = pos + rng.normal(0.0, jitter, size=pos.shape)
    L = n_rep * a
    pos = _wrap(pos, L)
    Z = np.full(pos.shape[0], Z_OF["Fe"], dtype=np.int64)
    return AtomicSystem(f"bcc_fe_{n_rep}", pos.astype(np.float32), Z,
                        np.diag([L, L, L]).astype(np.float32))


def amorphous(n_atoms: int = 50000, density: float = 0.08, dmin: float = 1.2,
              seed: int = 0) -> AtomicSystem:
    """Config 4: amorphous 8-element system (Z in {1,6,7,8,14,26,29,78}, equal fractions,
    shuffled), uniform random positions at the given density with minimum separation."""
    rng = np.random.default_rng(seed)
    L = (n_atoms / density) ** (1.0 / 3.0)
    pos = _rsa(rng, n_atoms, L, dmin)
    elems = np.array([1, 6, 7, 8, 14, 26, 29, 78], dtype=np.int64)
    Z = np.repeat(elems, int(math.ceil(n_atoms / len(elems))))[:n_atoms]
    rng.shuffle(Z)
    return AtomicSystem("amorphous", pos.astype(np.float32), Z,
                        np.diag([L, L, L]).astype(np.float32))


def sweep_graph(n_atoms: int, degree: int, cutoff: float = 6.0, seed: int = 0):
    """The synthetic graphs of the reference's own benchmark sweep (examples/sweep.py:33-81),
    generated here with numpy: uniform random positions in a cube scaled so that about
    n_atoms * degree ordered pairs lie within the cutoff, every such pair an edge (no
    per-receiver cap), random elements 1..99, a unit cell without periodicity and random
    cell offsets in {-1, 0, 1} per edge (shift vectors of up to 1 A per axis).  Returns the
    system and its explicit (edge_index, cell_offsets)."""
    rng = np.random.default_rng(seed)
    p = rng.random((n_atoms, 3))
    d = np.linalg.norm(p[:, None, :] - p[None, :, :], axis=-1)
    k = min(n_atoms * degree + n_atoms, n_atoms * n_atoms)   # the diagonal's n zeros first
    kth = np.partition(d.ravel(), k - 1)[k - 1]
    scale = (cutoff - 1e-4) / kth
    pos = (p * scale).astype(np.float32)
    Z = rng.integers(1, 100, n_atoms).astype(np.int64)
    within = (d * scale < cutoff) & ~np.eye(n_atoms, dtype=bool)
    send, recv = np.nonzero(within)   # row-major: sender-major, as the reference's pair list
    ei = np.stack([send, recv]).astype(np.int64)
    off = rng.integers(-1, 2, (ei.shape[1], 3)).astype(np.float32)
    system = AtomicSystem(f"sweep_{n_atoms}x{degree}", pos, Z, np.eye(3, dtype=np.float32),
                          pbc=(False, False, False))
    return system, ei, off


def _image_reps(cell: np.ndarray, pbc, cutoff: float):
    reps = []
    for ax in range(3):
        if pbc[ax]:
            other = [cell[(ax + 1) % 3], cell[(ax + 2) % 3]]
            normal = np.cross(other[0], other[1])
            width = abs(np.dot(cell[ax], normal)) / np.linalg.norm(normal)
            reps.append(int(math.ceil(cutoff / width)) + 1)
        else:
            reps.append(0)
    return reps


def neighbor_list(pos, cell, pbc, cutoff: float, max_neighbors: int):
    """Capped radius graph (see the module docstring for the exact definition).

    Candidate pairs come from a k-d tree over all periodic images within cutoff + 1e-3;
    the exact float64 test, ordering and cap are then applied per receiver."""
    from scipy.spatial import cKDTree

    pos32 = np.asarray(pos, dtype=np.float32)
    pos64 = pos32.astype(np.float64)
    cell64 = np.asarray(cell, dtype=np.float32).astype(np.float64)
    n = pos64.shape[0]
    reps = _image_reps(cell64, pbc, cutoff)
    offsets = np.array(list(itertools.product(*[range(-r, r + 1) for r in reps])), dtype=np.int64)
    shifts = np.array([(o[0] * cell64[0] + o[1] * cell64[1]) + o[2] * cell64[2] for o in offsets])
    # keep only images that can reach the primary cell's bounding box
    lo, hi = pos64.min(0) - cutoff, pos64.max(0) + cutoff
    img_pos = pos64[None, :, :] + shifts[:, None, :]
    img_keep = ((img_pos >= lo) & (img_pos <= hi)).all(-1)
    img_o, img_i = np.nonzero(img_keep)
    tree = cKDTree(img_pos[img_o, img_i])
    cand = tree.query_ball_point(pos64, r=cutoff + 1e-3, return_sorted=False)
    cut2 = float(cutoff) * float(cutoff)
    send, recv, offs = [], [], []
    for j in range(n):
        k = np.asarray(cand[j], dtype=np.int64)
        if k.size == 0:
            continue
        oi, ii = img_o[k], img_i[k]
        o = offsets[oi]
        d = (pos64[ii] - pos64[j]) + shifts[oi]
        d2 = (d[:, 0] * d[:, 0] + d[:, 1] * d[:, 1]) + d[:, 2] * d[:, 2]
        ok = (d2 < cut2) & ~((ii == j) & ~o.any(1))
        d2, ii, o = d2[ok], ii[ok], o[ok]
        order = np.lexsort((o[:, 2], o[:, 1], o[:, 0], ii, d2))[:max_neighbors]
        send.append(ii[order])
        recv.append(np.full(order.size, j, dtype=np.int64))
        offs.append(o[order])
    if send:
        edge_index = np.stack([np.concatenate(send), np.concatenate(recv)]).astype(np.int64)
        cell_offsets = np.concatenate(offs).astype(np.float32)
    else:
        edge_index = np.zeros((2, 0), dtype=np.int64)
        cell_offsets = np.zeros((0, 3), dtype=np.float32)
    return edge_index, cell_offsets


CONFIGS = {
    "cu_slab_co": dict(builder=cu_slab_co, lmax=2, layers=4, stress=False),
    "water_box": dict(builder=water_box, lmax=2, layers=4, stress=False),
    "bcc_fe": dict(builder=bcc_fe, lmax=2, layers=4, stress=True),
    "amorphous": dict(builder=amorphous, lmax=2, layers=4, stress=False),
    "bcc_fe_lmax4": dict(builder=bcc_fe, lmax=4, layers=8, stress=False),
}
