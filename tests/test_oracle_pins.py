"""Pins of the CPU oracle against mathematics (the reference ships no golden vectors or
known-answer tests, so every function is checked against a closed form, an independent
derivation, an invariant or brute force)."""
import math

import numpy as np
import pytest
import torch

from oracle import graph as G
from oracle import ops_ref as R

DT = torch.float64


def _unit_q(n, seed):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(n, 4, generator=g, dtype=DT)
    return q / q.norm(dim=1, keepdim=True)


# --- geometry -------------------------------------------------------------------------

def test_l2_table_equals_symmetric_tensor_representation():
    """The 25 quartic polynomials restated from ops/geom.py:154-178 equal <B_a, R B_b R^T>."""
    q = _unit_q(2000, 0)
    d_poly = R.wigner_l2_from_quaternion(q)
    d_rep = R.wigner_l2_from_rotation(R.rotation_from_quaternion(q))
    assert (d_poly - d_rep).abs().max() < 1e-13


def test_wigner_blocks_orthogonal_and_homomorphic():
    q1, q2 = _unit_q(500, 1), _unit_q(500, 2)
    w, x, y, z = q1.unbind(1)
    a, b, c, d = q2.unbind(1)
    prod = torch.stack([w * a - x * b - y * c - z * d, w * b + x * a + y * d - z * c,
                        w * c - x * d + y * a + z * b, w * d + x * c - y * b + z * a], 1)
    for f in (R.rotation_from_quaternion, R.wigner_l2_from_quaternion):
        D1, D2, D12 = f(q1), f(q2), f(prod)
        n = D1.shape[-1]
        assert (D1 @ D1.transpose(1, 2) - torch.eye(n, dtype=DT)).abs().max() < 1e-13
        assert (D1 @ D2 - D12).abs().max() < 1e-13
        assert (torch.linalg.det(D1) - 1).abs().max() < 1e-12


def test_edge_frame_maps_edge_to_y():
    g = torch.Generator().manual_seed(3)
    e = torch.randn(4000, 3, generator=g, dtype=DT)
    e = torch.cat([e, torch.tensor([[0.0, 1.0, 0.0], [0.0, -1.0, 0.0], [1.0, 0, 0], [0, 0, -1.0]], dtype=DT)])
    e = e / e.norm(dim=1, keepdim=True)
    q = R.edge_frame_quaternion(e[:, 0], e[:, 1], e[:, 2])
    Rm = R.rotation_from_quaternion(q)
    ye = torch.einsum("eij,ej->ei", Rm, e)
    # exact up to the 1e-7 regulariser inside the reference's normalisations
    assert (ye - torch.tensor([0.0, 1.0, 0.0], dtype=DT)).abs().max() < 1e-6
    # L1 row 1 (the m=0 row) is the edge direction itself
    assert (Rm[:, 1, :] - e).abs().max() < 1e-6


def test_envelope_closed_form():
    c = 6.0
    d = torch.tensor([0.0, c, 2.5], dtype=DT, requires_grad=True)
    env = R.envelope(d, c)
    assert env[0].item() == 1.0 and env[1].item() == 0.0
    u = 2.5 / c
    assert abs(env[2].item() - (1 - 21 * u ** 5 + 35 * u ** 6 - 15 * u ** 7)) < 1e-15
    # C^2 continuity at the cutoff: derivative of the polynomial branch vanishes there
    dc = torch.tensor([c - 1e-9], dtype=DT, requires_grad=True)
    u = dc / c
    poly = 1.0 + u ** 5 * (-21.0 + u * (35.0 - 15.0 * u))
    (g1,) = torch.autograd.grad(poly.sum(), dc, create_graph=True)
    (g2,) = torch.autograd.grad(g1.sum(), dc)
    assert abs(g1.item()) < 1e-12 and abs(g2.item()) < 1e-6


def test_gaussian_basis():
    pos = torch.tensor([[0.0, 0.0, 0.0], [1.5, 0.0, 0.0]], dtype=DT)
    off = torch.linspace(0, 6.0, 64, dtype=DT)
    coeff = -0.5 / (2.0 * (off[1] - off[0])) ** 2
    xe, _, _ = R.edge_geometry(pos, torch.tensor([1, 2]), torch.tensor([1]), torch.tensor([0]), torch.zeros(1, 3, dtype=DT),
                               torch.zeros(100, 4, dtype=DT), torch.zeros(100, 4, dtype=DT), off, float(coeff), 6.0)
    ref = torch.exp(coeff * (1.5 - off) ** 2)
    assert (xe[0, :64] - ref).abs().max() < 1e-15


# --- rotated-frame maps -----------------------------------------------------------------

def _random_frames(E, seed):
    q = _unit_q(E, seed)
    return torch.cat([R.rotation_from_quaternion(q).reshape(E, 9), R.wigner_l2_from_quaternion(q).reshape(E, 25)], 1)


def test_scatter_is_adjoint_of_receiver_rotation():
    """<rotate(v), z> over the receiver slots == <v, scatter(z)>: the gather slot map and the
    scatter slot map are transposes of each other."""
    E, N, C = 50, 7, 3
    g = torch.Generator().manual_seed(4)
    wig = _random_frames(E, 5)
    x = torch.randn(N, 9, C, generator=g, dtype=DT)
    idx_i = torch.randint(0, N, (E,), generator=g)
    idx_j = torch.randint(0, N, (E,), generator=g)
    rad = torch.zeros(E, 12 * C, dtype=DT)
    # receiver (t) slots only: odd radial blocks = 1
    for b in (1, 3, 5, 7, 9, 11):
        rad[:, b * C:(b + 1) * C] = 1.0
    X0, X1, X2 = R.gather_rotate(x, idx_i, idx_j, wig, rad, torch.zeros(1, C, dtype=DT), torch.zeros(N, dtype=torch.long))
    Z0 = torch.randn(E, 3 * C, generator=g, dtype=DT)
    Z1 = torch.randn(E, 4 * C, generator=g, dtype=DT)
    Z2 = torch.randn(E, 2 * C, generator=g, dtype=DT)

    def t_slots(X, n):
        return X.reshape(E, n, C)[:, 1::2].reshape(E, -1)
    lhs = (t_slots(X0, 6) * Z0).sum() + (t_slots(X1, 8) * Z1).sum() + (t_slots(X2, 4) * Z2).sum()
    out = R.rotate_scatter(Z0, Z1, Z2, wig, torch.ones(E, dtype=DT), torch.zeros(N, 9, C, dtype=DT), idx_j, N)
    rhs = (out * x).sum()
    assert abs(lhs.item() - rhs.item()) < 1e-10 * max(1.0, abs(lhs.item()))


def test_gating_closed_form():
    C = 2
    Y0 = torch.tensor([[0.0, 0.0, 1.0, 1.0, 2.0, 2.0, 3.0, 3.0, 4.0, 4.0]], dtype=DT)
    Y1 = torch.ones(1, 4 * C, dtype=DT)
    Y2 = torch.full((1, 2 * C), 2.0, dtype=DT)
    Z0, Z1, Z2 = R.gating(Y0, Y1, Y2, C)
    s1 = 1 / (1 + math.exp(-1.0))
    silu2 = 2.0 / (1 + math.exp(-2.0))
    # Y_m0 blocks: gate_l1 = 0, gate_l2 = 1, y_l0 = 2, y_l1m0 = 3, y_l2m0 = 4
    assert torch.allclose(Z0, torch.tensor([[silu2, silu2, 1.5, 1.5, 4 * s1, 4 * s1]], dtype=DT))
    assert torch.allclose(Z1, torch.tensor([[0.5, 0.5, s1, s1, 0.5, 0.5, s1, s1]], dtype=DT))
    assert torch.allclose(Z2, torch.full((1, 4), 2 * s1, dtype=DT))


def test_ln_silu_closed_form():
    x = torch.tensor([[1.0, 2.0, 3.0, 6.0]], dtype=DT)
    out = R.layer_norm_silu(x, torch.ones(4, dtype=DT), torch.zeros(4, dtype=DT), 1e-7)
    m, v = 3.0, (4 + 1 + 0 + 9) / 4
    xh = (x - m) / math.sqrt(v + 1e-7)
    assert (out - xh * torch.sigmoid(xh)).abs().max() < 1e-14


def test_so2_packing_is_complex_product():
    g = torch.Generator().manual_seed(6)
    Rr, Ii = torch.randn(3, 5, generator=g, dtype=DT), torch.randn(3, 5, generator=g, dtype=DT)
    a, b = torch.randn(5, generator=g, dtype=DT), torch.randn(5, generator=g, dtype=DT)
    W = R.pack_so2(Rr, Ii)
    y = W @ torch.cat([a, b])
    z = torch.complex(Rr, Ii) @ torch.complex(a, b)
    assert torch.allclose(y[:3], z.real) and torch.allclose(y[3:], z.imag)


# --- integer graph ----------------------------------------------------------------------

def test_morton_bit_interleave_all_values():
    v = np.arange(1024)
    fast = G.expand_bits(v)
    loop = np.array([G.expand_bits_loop(int(k)) for k in v])
    assert np.array_equal(fast, loop)
    g = np.random.default_rng(7)
    for ix, iy, iz in g.integers(0, 1024, size=(500, 3)):
        assert int(G.morton_code(np.array([ix]), np.array([iy]), np.array([iz]))[0]) == G.morton_code_loop(ix, iy, iz)
    # known answers: the reference's keys start at bit 1 (x), 2 (y), 3 (z) and end at bit 30
    one = lambda a, b, c: int(G.morton_code(np.array([a]), np.array([b]), np.array([c]))[0])
    assert (one(1, 0, 0), one(0, 1, 0), one(0, 0, 1), one(2, 0, 0)) == (2, 4, 8, 16)
    assert one(1023, 1023, 1023) == 2**31 - 2


def test_csr_matches_loop():
    g = np.random.default_rng(8)
    keys = g.integers(0, 17, size=400)
    keys[keys == 5] = 6            # an empty segment
    a = G.csr(keys, 20)
    b = G.csr_loop(keys, 20)
    assert np.array_equal(a[0], b[0]) and np.array_equal(a[1], b[1])


def test_neighbor_list_product_matches_bruteforce():
    import systems
    for s in (systems.cu_slab_co(), systems.water_box(n_mol=30, L=9.7, seed=2)):
        a = systems.neighbor_list(s.pos, s.cell, s.pbc, 6.0, 30)
        b = G.neighbor_list_bruteforce(s.pos, s.cell, s.pbc, 6.0, 30)
        assert np.array_equal(a[0], b[0]) and np.array_equal(a[1], b[1])
        # cap and grouping: every receiver has <= 30 edges, receivers ascending
        assert np.all(np.diff(a[0][1]) >= 0) and np.bincount(a[0][1]).max() <= 30
