"""The HIP-graph-captured step (flash-uma_amd/captured.py) against eager evaluation: several
replays with new positions (and a strained cell), eager work and synchronisations between
them, every replay compared with the eager result of the same inputs (bitwise: the same
kernels run in the same order)."""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _setup(cuda, system):
    import escn_md
    import heads
    import systems
    from wrapper import ZeroAllocBackbone
    bb = escn_md.eSCNMDBackbone(seed=0)
    hd = heads.MLPEnergyHead(bb.sphere_channels, bb.hidden_channels, seed=1)
    model = heads.PotentialModel(ZeroAllocBackbone(bb.to(cuda)), hd.to(cuda))
    ei, off = systems.neighbor_list(system.pos, system.cell, system.pbc, bb.cutoff, bb.max_neighbors)
    return model, ei, off


@pytest.mark.parametrize("name", ["water64", "cu_slab", "water333"])
def test_captured_step_equals_eager(cuda, name):
    """Three graph sizes: 192, 29 and 999 atoms (5,760, 859 and 29,970 edges)."""
    import heads
    import systems
    from captured import CapturedStep
    s = {"water64": lambda: systems.water_box(n_mol=64, L=12.42, seed=3), "cu_slab": systems.cu_slab_co,
         "water333": systems.water_box}[name]()
    model, ei, off = _setup(cuda, s)
    data_c = heads.make_atomic_data(s, ei, off, cuda)
    cap = CapturedStep(model, data_c, compute_stress=True)
    rng = np.random.default_rng(0)
    for k in range(4):
        pos = torch.tensor(s.pos + rng.normal(0.0, 0.01, s.pos.shape), dtype=torch.float32, device=cuda)
        strain = torch.eye(3, dtype=torch.float32) + (0.002 * k) * torch.tensor([[1.0, 0.3, 0.0], [0.3, -0.5, 0.1],
                                                                                  [0.0, 0.1, 0.2]])
        cell = torch.tensor(s.cell, dtype=torch.float32) @ strain
        out = {key: v.detach().clone() for key, v in cap(pos, cell.to(cuda)).items()}
        # eager reference on the same edge_index tensor, hence the same cached topology
        # (Morton order), so the same summation orders
        data_e = heads.make_atomic_data(s, ei, off, cuda)
        data_e.edge_index = data_c.edge_index
        with torch.no_grad():
            data_e.pos.copy_(pos)
            data_e.cell.copy_(cell.reshape(1, 3, 3))
        ref = model(data_e, compute_forces=True, compute_stress=True)
        torch.cuda.synchronize()
        for key in ("energy", "forces", "stress", "atom_energy"):
            assert torch.equal(out[key], ref[key].detach()), f"replay {k}: {key} differs"
