"""Real spherical-harmonic bases and Wigner blocks for any degree l — test infrastructure only.

The reference handles lmax = 2 only (wrapper.py:105-118 rejects anything else; its 34 Wigner
scalars are the L=1 3x3 and L=2 5x5 blocks, ops/geom.py:137-178).  Generalising to lmax = 4
needs the l = 3 and l = 4 blocks in the same convention, which this module defines from the
mathematics alone:

  * y is the polar axis and the azimuth runs in the (z, x) plane (the reference's l = 1
    block is the rotation matrix in (x, y, z) order with m = -1, 0, +1 <-> x, y, z; its
    l = 2 basis is xz, xy, 3y^2 - r^2, yz, z^2 - x^2, oracle.ops_ref._l2_basis);
  * the degree-l harmonic of order m >= 0 is Re((z + i x)^m) Q_l^m(y, r^2) and of order -m
    Im((z + i x)^m) Q_l^m(y, r^2), with Q_l^m the homogenised m-th derivative of the
    Legendre polynomial P_l, r^l P_l^m(y / r) = rho^m Q_l^m (no Condon-Shortley phase);
  * coefficient (l, m) sits at index l^2 + l + m;
  * each harmonic polynomial p is represented by its symmetric traceless tensor
    T = (1/l!) d^l p (p(v) = T(v, ..., v)), normalised in the Frobenius norm, and
    D^l[a][b] = <B_a, R^{(x)l} B_b>, the matrix of p -> p o R^T in that basis.

For l = 1, 2 this reproduces the reference's blocks exactly (tests/test_oracle_pins.py).
Pins for l = 3, 4: orthonormality and tracelessness of the basis, the homomorphism
D(R1 R2) = D(R1) D(R2), orthogonality, and rotations about y acting on every (m, -m) pair
as the same planar rotation by m * angle (the property the SO(2) convolution relies on).
"""
from __future__ import annotations

import itertools
import math

import torch


def _legendre_q(l: int, m: int) -> list[tuple[float, int, int]]:
    """Q_l^m as a list of (coefficient, power of y, power of r^2)."""
    out = []
    for k in range((l - m) // 2 + 1):
        c = (-1) ** k * math.comb(l, k) * math.comb(2 * l - 2 * k, l) * math.factorial(l - 2 * k) / \
            math.factorial(l - 2 * k - m) / 2 ** l
        out.append((c, l - 2 * k - m, k))
    return out


def _poly_mul(a: dict, b: dict) -> dict:
    out: dict = {}
    for ea, ca in a.items():
        for eb, cb in b.items():
            e = tuple(x + y for x, y in zip(ea, eb))
            out[e] = out.get(e, 0.0) + ca * cb
    return out


def _harmonic_poly(l: int, m: int) -> dict:
    """Polynomial {(px, py, pz): coefficient} of the (l, m) harmonic described above."""
    am = abs(m)
    # (z + i x)^am = sum_k C(am, k) z^(am-k) (i x)^k; real part: k even, imaginary: k odd
    zx: dict = {}
    for k in range(am + 1):
        if (k % 2 == 0) != (m >= 0):
            continue
        sign = (-1) ** (k // 2)
        zx[(k, 0, am - k)] = zx.get((k, 0, am - k), 0.0) + sign * math.comb(am, k)
    q: dict = {}
    for c, py, pr in _legendre_q(l, am):
        # r^(2 pr) = (x^2 + y^2 + z^2)^pr
        for ks in itertools.product(range(3), repeat=pr):
            e = [0, py, 0]
            for axis in ks:
                e[axis] += 2
            q[tuple(e)] = q.get(tuple(e), 0.0) + c
    return _poly_mul(zx, q)


def _poly_to_tensor(p: dict, l: int, dtype) -> torch.Tensor:
    """Symmetric tensor T with T(v, ..., v) = p(v)."""
    T = torch.zeros((3,) * l, dtype=dtype)
    for idx in itertools.product(range(3), repeat=l):
        e = tuple(idx.count(a) for a in range(3))
        c = p.get(e, 0.0)
        if c != 0.0:
            mult = math.factorial(l) // (math.factorial(e[0]) * math.factorial(e[1]) * math.factorial(e[2]))
            T[idx] = c / mult
    return T


def sh_basis(l: int, dtype=torch.float64) -> torch.Tensor:
    """(2l+1, 3, ..., 3) Frobenius-orthonormal symmetric traceless tensors, row l + m = order m."""
    if l == 0:
        return torch.ones(1, dtype=dtype)
    out = []
    for m in range(-l, l + 1):
        T = _poly_to_tensor(_harmonic_poly(l, m), l, dtype)
        out.append(T / T.pow(2).sum().sqrt())
    return torch.stack(out)


def wigner_from_rotation(R: torch.Tensor, l: int) -> torch.Tensor:
    """D^l (..., 2l+1, 2l+1) of the rotation R (..., 3, 3): D[a][b] = <B_a, R^(x)l B_b>."""
    batch = R.shape[:-2]
    Rb = R.reshape(-1, 3, 3)
    E = Rb.shape[0]
    if l == 0:
        return torch.ones(*batch, 1, 1, dtype=R.dtype)
    B = sh_basis(l, R.dtype)
    n = B.shape[0]
    T = B.unsqueeze(0).expand(E, *B.shape).clone()
    for ax in range(l):
        # T'[.., i, ..] = sum_j R[i, j] T[.., j, ..] along tensor axis ax
        T = torch.movedim(T, 1 + 1 + ax, -1)
        shp = T.shape
        T = (T.reshape(E, -1, 3) @ Rb.transpose(1, 2)).reshape(shp)
        T = torch.movedim(T, -1, 1 + 1 + ax)
    D = torch.einsum("ak,ebk->eab", B.reshape(n, -1), T.reshape(E, n, -1))
    return D.reshape(*batch, n, n)


def wigner_rows(l: int) -> list[int]:
    """Rows of D^l the eSCN edge frame uses (|m| <= 2)."""
    return [l + m for m in range(-min(l, 2), min(l, 2) + 1)]


def wigner_ext_width(lmax: int) -> int:
    """Scalars per edge beyond the reference's 34: rows |m| <= 2 of D^3, D^4, ..."""
    return sum(len(wigner_rows(l)) * (2 * l + 1) for l in range(3, lmax + 1))


def wigner_ext(R: torch.Tensor, lmax: int) -> torch.Tensor:
    """(E, wigner_ext_width) : for l = 3..lmax the rows |m| <= 2 of D^l, row-major."""
    parts = [wigner_from_rotation(R, l)[:, wigner_rows(l)].reshape(R.shape[0], -1) for l in range(3, lmax + 1)]
    if not parts:
        return torch.zeros(R.shape[0], 0, dtype=R.dtype)
    return torch.cat(parts, 1)


def rotation_about_y(angle: float, dtype=torch.float64) -> torch.Tensor:
    c, s = math.cos(angle), math.sin(angle)
    return torch.tensor([[c, 0.0, s], [0.0, 1.0, 0.0], [-s, 0.0, c]], dtype=dtype)
