"""The host interface mirrors the reference's wrapper module (wrapper.py:7-212): the same
public names, and the hooks FAIRChem's predict unit calls behave as the reference's do
(no GPU needed)."""
import types

import pytest


def test_module_names_match_reference():
    import wrapper
    for name in ("ZeroAllocBackbone", "transfer_weights", "validate_atoms_data", "on_predict_check",
                 "prepare_for_inference"):
        assert callable(getattr(wrapper, name)), name
    for name in ("validate_atoms_data", "on_predict_check", "prepare_for_inference", "csd_embedding", "forward"):
        assert callable(getattr(wrapper.ZeroAllocBackbone, name)), name


@pytest.mark.parametrize("task,spin", [("omol", 1), ("omat", 0), ("oc20", 0)])
def test_validate_atoms_data_defaults(task, spin):
    """Missing charge and spin default to 0 and (1 for omol, else 0); given values stay."""
    import wrapper
    atoms = types.SimpleNamespace(info={})
    for fn in (wrapper.validate_atoms_data, wrapper.ZeroAllocBackbone.validate_atoms_data):
        atoms.info = {}
        fn(None, atoms, task)
        assert atoms.info == {"charge": 0, "spin": spin}
        atoms.info = {"charge": -2, "spin": 3}
        fn(None, atoms, task)
        assert atoms.info == {"charge": -2, "spin": 3}


def test_prepare_for_inference_returns_self_and_check_is_bypassed():
    import wrapper
    obj = object()
    assert wrapper.prepare_for_inference(obj, None, None) is obj
    assert wrapper.on_predict_check(obj, None) is None


def test_model_module_names_match_reference():
    import model
    for name in ("build_csr_cached", "clear_csr_cache", "expand_bits_torch", "morton3d_torch",
                 "reorder_graph_morton", "Packed_eSCN_Layer", "eSCN_Inference_Model"):
        assert callable(getattr(model, name)), name


def test_morton_helpers_equal_oracle_keys():
    """model.morton3d_torch gives the reference's codes: equal to the oracle's restatement of
    model.py:48-58 on every 10-bit value per axis and on random triples."""
    import numpy as np
    import torch
    import model
    from oracle import graph as G
    v = torch.arange(1024, dtype=torch.int32)
    assert np.array_equal(model.expand_bits_torch(v).numpy(), G.expand_bits(v.numpy()))
    g = np.random.default_rng(3)
    ijk = g.integers(0, 1024, size=(2000, 3)).astype(np.int32)
    t = torch.from_numpy(ijk)
    got = model.morton3d_torch(t[:, 0], t[:, 1], t[:, 2]).numpy()
    assert np.array_equal(got, G.morton_code(ijk[:, 0], ijk[:, 1], ijk[:, 2]))


def test_constants_names_match_reference():
    """ops/constants.py names of the reference: Wigner scalar offsets W<row><col> (rows and
    columns 1-3 for L = 1, 4-8 for L = 2) and the m-block widths."""
    from ops import constants as K
    assert (K.W11, K.W13, K.W21, K.W33, K.W44, K.W48, K.W54, K.W88) == (0, 2, 3, 8, 9, 13, 14, 33)
    assert (K.X_M0_MULT, K.Y_M0_MULT, K.Z_M0_MULT, K.TRUNC_Y_M0_MULT, K.TRUNC_Z_M0_MULT) == (6, 5, 3, 5, 3)
    assert abs(K.S3X4 - 8 * 3 ** 0.5) < 1e-12 and abs(K.S3 - 2 * 3 ** 0.5) < 1e-12


def test_atom_range_check_is_not_skipped_for_a_new_tensor():
    """The host range check of atomic numbers and batch ids runs again for a new tensor even
    when it reuses the address of a freed, already-checked one, and after an in-place edit."""
    import torch
    import model
    m = model.eSCN_Inference_Model(num_layers=1, sphere_channels=8, num_distance_basis=4)
    batch = torch.zeros(64, dtype=torch.long)
    Z = torch.full((64,), 26, dtype=torch.long)
    m._check_atoms(Z, batch, 1)
    m._check_atoms(Z, batch, 1)                 # same tensors: cached
    del Z
    for _ in range(4):                          # likely to land on the freed address
        Z_bad = torch.full((64,), 26, dtype=torch.long)
        Z_bad[5] = 250
        with pytest.raises(ValueError):
            m._check_atoms(Z_bad, batch, 1)
        del Z_bad
    Z = torch.full((64,), 8, dtype=torch.long)
    m._check_atoms(Z, batch, 1)
    Z[3] = -1                                   # in-place edit bumps the version
    with pytest.raises(ValueError):
        m._check_atoms(Z, batch, 1)
    with pytest.raises(ValueError):
        m._check_atoms(torch.full((64,), 8, dtype=torch.long), batch, 0)   # batch id 0 >= 0 systems
