"""GPU integer graph preprocessing is bit-exact against the numpy oracle (model.py:17-74)."""
import numpy as np
import pytest
import torch

from oracle import graph as G

pytestmark = pytest.mark.gpu


def test_morton_and_csr_bit_exact(cuda):
    import systems
    from ops import topology
    s = systems.bcc_fe(n_rep=6)
    ei, off = systems.neighbor_list(s.pos, s.cell, s.pbc, 6.0, 30)
    N = s.n_atoms
    pos = torch.from_numpy(s.pos).to(cuda)
    batch = torch.zeros(N, dtype=torch.long, device=cuda)
    keys = torch.empty(N, dtype=torch.long, device=cuda)
    from ops import _lib
    _lib.call("fu_morton_keys", pos.data_ptr(), batch.data_ptr(), keys.data_ptr(), N, _lib.stream_ptr(cuda))
    ref_keys = G.morton_keys(s.pos, np.zeros(N, dtype=np.int64))
    assert np.array_equal(keys.cpu().numpy(), ref_keys)
    perm, inv = topology.morton_permutation(pos, batch)
    _, _, _, ii, jj, rperm, rinv = G.reorder_graph_morton(s.pos, s.Z, np.zeros(N, dtype=np.int64), ei[0], ei[1])
    assert np.array_equal(perm.cpu().numpy(), rperm)
    assert np.array_equal(inv.cpu().numpy(), rinv)
    row_ptr, col = topology.receiver_csr(torch.from_numpy(jj).to(cuda), N)
    rrow, rcol = G.csr(jj, N)
    assert np.array_equal(row_ptr.cpu().numpy(), rrow)
    assert np.array_equal(col.cpu().numpy(), rcol)


def test_topology_consistency(cuda):
    """Sorted edge order = the reference CSR order; sender CSR covers every edge once."""
    import systems
    from ops import topology
    s = systems.water_box(n_mol=40, L=10.5, seed=1)
    ei, _ = systems.neighbor_list(s.pos, s.cell, s.pbc, 6.0, 30)
    N = s.n_atoms
    topo = topology.build_topology(torch.from_numpy(s.pos).to(cuda), torch.zeros(N, dtype=torch.long, device=cuda),
                                   torch.from_numpy(ei).to(cuda))
    _, _, _, ii, jj, rperm, rinv = G.reorder_graph_morton(s.pos, s.Z, np.zeros(N, dtype=np.int64), ei[0], ei[1])
    rrow, rcol = G.csr(jj, N)
    assert np.array_equal(topo.edge_perm.cpu().numpy(), rcol.astype(np.int64))
    assert np.array_equal(topo.recv_ptr.cpu().numpy(), rrow)
    assert np.array_equal(topo.idx_j.cpu().numpy(), jj[rcol])
    assert np.array_equal(topo.idx_i.cpu().numpy(), ii[rcol])
    sptr, sidx = G.csr(ii[rcol], N)
    assert np.array_equal(topo.send_ptr.cpu().numpy(), sptr)
    assert np.array_equal(topo.send_idx.cpu().numpy(), sidx)


def _triclinic(n=300, seed=5, outside=0.02):
    import systems
    g = np.random.default_rng(seed)
    cell = np.array([[14.0, 0.0, 0.0], [3.1, 13.2, 0.0], [-2.4, 1.7, 12.5]])
    frac = g.uniform(-outside, 1.0 + outside, size=(n, 3))
    pos = (frac @ cell).astype(np.float32)
    Z = g.choice([1, 6, 8, 26], size=n).astype(np.int64)
    return systems.AtomicSystem("triclinic", pos, Z, cell.astype(np.float32))


def _graph_cases():
    import systems
    return {
        "cu_slab": (systems.cu_slab_co, 30),
        "water999": (lambda: systems.water_box(n_mol=333, L=21.5, seed=0), 30),
        "bcc_fe_8192": (lambda: systems.bcc_fe(16), 30),
        "amorphous_50k": (systems.amorphous, 30),
        "triclinic": (_triclinic, 30),
        "triclinic_cap8": (_triclinic, 8),
        "slab_open_z": (lambda: _open_z(), 30),
    }


def _open_z():
    import systems
    s = _triclinic(n=200, seed=9, outside=0.0)
    return systems.AtomicSystem("open_z", s.pos, s.Z, s.cell, pbc=(True, True, False))


@pytest.mark.parametrize("case", ["cu_slab", "water999", "bcc_fe_8192", "amorphous_50k", "triclinic", "triclinic_cap8",
                                  "slab_open_z"])
def test_radius_graph_bit_exact(cuda, case):
    """GPU radius graph == host builder (edge order, senders, receivers, offsets), including
    a triclinic cell with atoms slightly outside it, a small cap and a non-periodic axis."""
    import systems
    from ops.neighbors import radius_graph
    build, K = _graph_cases()[case]
    s = build()
    ei, off = systems.neighbor_list(s.pos, s.cell, s.pbc, 6.0, K)
    gei, goff = radius_graph(torch.from_numpy(np.asarray(s.pos)).to(cuda), s.cell, s.pbc, 6.0, K)
    print(case, s.n_atoms, "atoms", ei.shape[1], "edges", flush=True)
    assert gei.shape == ei.shape and np.array_equal(gei.cpu().numpy(), ei)
    assert np.array_equal(goff.cpu().numpy(), off)


def test_radius_graph_brute_force(cuda):
    """Against the oracle's all-pairs, all-images enumeration."""
    from oracle.graph import neighbor_list_bruteforce
    from ops.neighbors import radius_graph
    s = _triclinic(n=120, seed=11)
    ref_ei, ref_off = neighbor_list_bruteforce(s.pos, s.cell, s.pbc, 6.0, 30)
    pos = torch.from_numpy(s.pos).to(cuda)
    gei, goff = radius_graph(pos, s.cell, s.pbc, 6.0, 30)
    assert np.array_equal(gei.cpu().numpy(), ref_ei) and np.array_equal(goff.cpu().numpy(), ref_off)


def _pairs_within(ei, off, pos, cell, cutoff):
    """{(sender, receiver, o0, o1, o2)} of the edges shorter than cutoff (float64)."""
    ei, off = ei.cpu().numpy(), off.cpu().numpy()
    p = pos.detach().cpu().numpy().astype(np.float64)
    d = p[ei[0]] - p[ei[1]] + off.astype(np.float64) @ np.asarray(cell, np.float64)
    keep = np.sqrt((d * d).sum(1)) < cutoff
    return set(map(tuple, np.concatenate([ei.T, off.astype(np.int64)], 1)[keep].tolist()))


def test_neighbor_list_skin_reuse(cuda):
    """NeighborList(skin): the reused graph holds every pair within the cutoff of the moved
    positions (the same set as a fresh uncapped graph), energies and forces through the
    model equal those of the fresh graph, and a move beyond skin / 2 or a cell change
    rebuilds; a cap together with a skin is refused."""
    import heads
    import systems
    from ops.neighbors import NL_CAP, NeighborList, radius_graph
    with pytest.raises(ValueError):
        NeighborList(6.0, 30, skin=0.5)
    s = systems.water_box(n_mol=40, L=10.5, seed=1)
    pos0 = torch.from_numpy(s.pos).to(cuda)
    nl = NeighborList(6.0, None, skin=0.6)
    g0 = nl(pos0, s.cell, s.pbc)
    rng = np.random.default_rng(3)
    step = rng.normal(size=s.pos.shape)
    step *= 0.29 / np.linalg.norm(step, axis=1).max()          # largest move 0.29 < skin / 2
    pos1 = pos0 + torch.from_numpy(step.astype(np.float32)).to(cuda)
    g1 = nl(pos1, s.cell, s.pbc)
    assert g1[0] is g0[0] and nl.builds == 1
    fresh = radius_graph(pos1, s.cell, s.pbc, 6.0, NL_CAP)
    assert _pairs_within(*g1, pos1, s.cell, 6.0) == _pairs_within(*fresh, pos1, s.cell, 6.0)
    assert g1[0].shape[1] > fresh[0].shape[1]          # the reused graph carries extra pairs

    from test_gpu_model import _build
    _, _, model = _build(cuda)
    moved = systems.AtomicSystem("water_moved", pos1.cpu().numpy(), s.Z, s.cell, s.pbc)
    outs = []
    for ei, off in (g1, fresh):
        data = heads.make_atomic_data(moved, ei.cpu().numpy(), off.cpu().numpy(), cuda)
        out = model(data, compute_forces=True, compute_stress=False)
        outs.append({k: v.detach().double().cpu() for k, v in out.items() if torch.is_tensor(v)})
    e_rel = abs(outs[0]["energy"].item() - outs[1]["energy"].item()) / abs(outs[1]["energy"].item())
    f_err = (outs[0]["forces"] - outs[1]["forces"]).abs().max().item()
    print(f"reused vs fresh graph: E rel {e_rel:.2e}, F max-abs {f_err:.2e}")
    assert e_rel <= 1e-6 and f_err <= 1e-4

    nl(pos0 + 0.31 * torch.tensor([1.0, 0.0, 0.0], device=cuda), s.cell, s.pbc)   # 0.31 > skin / 2
    assert nl.builds == 2
    cell2 = np.asarray(s.cell, np.float64) * 1.001
    nl(pos0 + 0.31 * torch.tensor([1.0, 0.0, 0.0], device=cuda), cell2, s.pbc)
    assert nl.builds == 3
