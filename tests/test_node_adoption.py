"""transfer_weights rebuilds FAIRChem's node modules on the HIP node kernels by parameter name
(CPU only: module construction, parameter copies and the plain-torch double's numerics).

tests/_fairchem_like.py holds plain-PyTorch modules with FAIRChem's names; the first tests pin
their forward against the float64 oracle (itself pinned in test_oracle_node_pins.py), so that
the GPU test that wraps a backbone carrying them (test_gpu_model.py) compares like with like."""
import warnings

import pytest
import torch

import _fairchem_like as fc


def _rand_(mod, seed):
    g = torch.Generator().manual_seed(seed)
    with torch.no_grad():
        for p in mod.parameters():
            p.copy_(torch.randn(p.shape, generator=g, dtype=torch.float64).to(p.dtype))
    return mod


@pytest.mark.parametrize("lmax", [2, 3, 4])
def test_plain_norm_equals_oracle(lmax):
    from oracle.model_ref import rms_norm_sh
    C = 16
    m = _rand_(fc.FCRMSNorm(lmax, C), lmax).double()
    x = torch.randn(7, (lmax + 1) ** 2, C, dtype=torch.float64, generator=torch.Generator().manual_seed(1))
    x[:, 0] += 3.0                                  # a large l = 0 mean, removed by the centring
    ref = rms_norm_sh(x, m.affine_weight.detach(), m.affine_bias.detach(), lmax, 1e-5)
    assert torch.allclose(m(x), ref, rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("lmax,H", [(2, 8), (3, 12), (4, 8)])
def test_plain_atom_wise_equals_oracle(lmax, H):
    from oracle.model_ref import spectral_atomwise
    C = 16
    m = _rand_(fc.FCSpectralAtomwise(C, H, lmax), 10 + lmax).double()
    x = torch.randn(5, (lmax + 1) ** 2, C, dtype=torch.float64, generator=torch.Generator().manual_seed(2))
    P = {k: v.detach() for k, v in m.state_dict().items()}
    ref = spectral_atomwise(x, P, "", lmax, H)
    assert torch.allclose(m(x), ref, rtol=1e-12, atol=1e-12)


def _wrap_cpu(bb):
    import model
    import wrapper
    cust = model.eSCN_Inference_Model(num_layers=bb.num_layers, sphere_channels=bb.sphere_channels,
                                      num_distance_basis=bb.num_distance_basis, lmax=bb.lmax)
    wrapper.transfer_weights(bb, cust)
    return cust


@pytest.mark.parametrize("lmax", [2, 4])
def test_transfer_weights_adopts_fairchem_named_modules(lmax):
    import escn_md
    import node_layers as nl
    bb = escn_md.eSCNMDBackbone(seed=3, num_layers=2, lmax=lmax, hidden_channels=64)
    want = {k: v.clone() for k, v in bb.state_dict().items()}
    foreign = fc.fairchem_like(escn_md.eSCNMDBackbone(seed=3, num_layers=2, lmax=lmax, hidden_channels=64))
    # the double carries the stand-in's parameter names, so the oracle reads both alike
    assert set(foreign.state_dict()) == set(want)
    with warnings.catch_warnings():
        warnings.simplefilter("error")
        cust = _wrap_cpu(foreign)
    for i, layer in enumerate(cust.layers):
        assert type(layer.norm_1) is nl.EquivariantRMSNormArraySphericalHarmonicsV2
        assert type(layer.norm_2) is nl.EquivariantRMSNormArraySphericalHarmonicsV2
        assert type(layer.atom_wise) is nl.SpectralAtomwise
        for name in ("norm_1", "norm_2", "atom_wise"):
            for k, v in getattr(layer, name).state_dict().items():
                assert torch.equal(v, want[f"blocks.{i}.{name}.{k}"]), (i, name, k)
    assert type(cust.final_norm) is nl.EquivariantRMSNormArraySphericalHarmonicsV2
    assert torch.equal(cust.final_norm.affine_weight, want["norm.affine_weight"])
    assert cust.final_norm.eps == 1e-5


def test_own_modules_are_attached_unchanged():
    import escn_md
    bb = escn_md.eSCNMDBackbone(seed=0, num_layers=1)
    cust = _wrap_cpu(bb)
    assert cust.layers[0].norm_1 is bb.blocks[0].norm_1
    assert cust.layers[0].atom_wise is bb.blocks[0].atom_wise
    assert cust.final_norm is bb.norm


def test_norm_eps_is_carried():
    import node_layers as nl
    m = fc.FCRMSNorm(2, 8, eps=1e-7)
    new = nl.adopt_rms_norm(m, 2, 8)
    assert type(new) is nl.EquivariantRMSNormArraySphericalHarmonicsV2 and new.eps == 1e-7


@pytest.mark.parametrize("case", ["no_centering", "other_normalization", "wrong_shape", "gelu", "no_bias",
                                  "other_balance"])
def test_other_modules_are_kept_with_a_warning(case):
    """A module whose configuration the kernels do not compute stays attached as given."""
    import node_layers as nl
    L, C = 2, 8
    if case in ("no_centering", "other_normalization", "wrong_shape", "other_balance"):
        m = fc.FCRMSNorm(L, C, centering=case != "no_centering")
        if case == "other_normalization":
            m.normalization = "norm"
        if case == "wrong_shape":
            m.affine_weight = torch.nn.Parameter(torch.ones(L, C))
        if case == "other_balance":
            m.balance_degree_weight.fill_(1.0 / 9)
        adopt = nl.adopt_rms_norm
    else:
        m = fc.FCSpectralAtomwise(C, 4, L, act=torch.nn.GELU if case == "gelu" else torch.nn.SiLU)
        if case == "no_bias":
            m.so3_linear_2.bias = None
        adopt = nl.adopt_atom_wise
    with pytest.warns(UserWarning, match="kept as given"):
        assert adopt(m, L, C) is m
