"""Shared test utilities: seeded random graphs and comparison helpers."""
from __future__ import annotations

import numpy as np
import torch


def random_graph(N: int = 40, E: int = 300, seed: int = 0, box: float = 6.0, isolated: int = 2):
    """Random directed multigraph with varied degrees; atoms [N-isolated, N) have no edges.

    Returns numpy arrays: pos (N,3) f32, Z (N,) i64, edge_index (2,E) i64, shifts (E,3) f32."""
    rng = np.random.default_rng(seed)
    pos = rng.uniform(0.0, box, size=(N, 3)).astype(np.float32)
    Z = rng.integers(1, 90, size=N).astype(np.int64)
    n_act = N - isolated
    # skewed receiver/sender degrees
    w = rng.gamma(0.7, size=n_act)
    w /= w.sum()
    src = rng.choice(n_act, size=E, p=w)
    dst = rng.integers(0, n_act, size=E)
    same = src == dst
    dst[same] = (dst[same] + 1) % n_act
    shifts = rng.integers(-1, 2, size=(E, 3)).astype(np.float32) * 0.5
    ei = np.stack([src, dst]).astype(np.int64)
    return pos, Z, ei, shifts


def axis_aligned_edges(pos, ei, shifts):
    """Overwrite the first edges so their vectors point exactly along +y, -y and x, and
    one lies beyond a 6 A cutoff (edge-frame clamp branches and env = 0)."""
    pos = pos.copy()
    shifts = shifts.copy()
    special = [np.array([0.0, 1.7, 0.0]), np.array([0.0, -2.1, 0.0]), np.array([1.3, 0.0, 0.0]),
               np.array([0.0, 0.0, -0.9]), np.array([4.0, 4.0, 3.0])]
    for k, v in enumerate(special):
        i, j = ei[0, k], ei[1, k]
        shifts[k] = (v - (pos[i].astype(np.float64) - pos[j])).astype(np.float32)
    return pos, shifts


def max_rel(a: torch.Tensor, b: torch.Tensor) -> float:
    """max |a - b| / max |b| (scale-relative error)."""
    a = a.detach().double().cpu()
    b = b.detach().double().cpu()
    den = max(b.abs().max().item(), 1e-30)
    return (a - b).abs().max().item() / den


def assert_close(a, b, tol: float, what: str = ""):
    err = max_rel(a, b)
    assert err <= tol, f"{what}: scale-relative error {err:.3e} > {tol:.1e}"
