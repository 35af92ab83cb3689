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
