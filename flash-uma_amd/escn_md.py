"""Random-init stand-in for FAIRChem's UMA eSCN-MD backbone and its node-level modules.

The reference wraps an official `eSCNMDBackbone` (fairchem.core.models.uma.escn_md) and
copies its weights (wrapper.py:22-85); FAIRChem is not in the reference tree and cannot be
installed offline.  This module provides an object with exactly the attributes
`transfer_weights` and `ZeroAllocBackbone.__init__` read (wrapper.py:28-146), shaped like
UMA-s, with seeded random weights, plus the node modules the reference attaches by
reference (norm_1, norm_2, atom_wise, final norm, charge/spin embeddings).

The node modules are the HIP-backed ones of node_layers.py, which restate the published
FAIRChem eSCN-MD designs (no FAIRChem code or fixtures exist here).  Their GPU forward and
backward are checked against the CPU oracle's restatement, which is itself checked against the
library routines the modules reduce to at lmax = 0 (LayerNorm, Linear, a Linear-SiLU-Linear
MLP), hand-derived known answers and equivariance; like the rest of the backbone they need GPU
tensors.

Initialisation (seeded CPU torch.Generator, fixed creation order): nn.Linear default
(kaiming-uniform weights, uniform bias), nn.Embedding N(0, 1), LayerNorm/affine weights 1,
biases 0.
"""
from __future__ import annotations

from types import SimpleNamespace

import torch
import torch.nn as nn

from node_layers import (EquivariantRMSNormArraySphericalHarmonicsV2, GateActivation, SO3_Linear,  # noqa: F401
                         SpectralAtomwise, _linear, degree_index, num_coefficients)


def _embedding(n: int, d: int, generator) -> nn.Embedding:
    emb = nn.Embedding(n, d)
    with torch.no_grad():
        emb.weight.normal_(0.0, 1.0, generator=generator)
    return emb


class RadialFunction(nn.Module):
    """Radial MLP: net = [Linear, LayerNorm, SiLU, Linear, LayerNorm, SiLU, Linear]; the
    Sequential indices 0/1/3/4/6 are the ones transfer_weights reads (wrapper.py:33-55)."""

    def __init__(self, channels: list[int], generator=None):
        super().__init__()
        layers: list[nn.Module] = []
        for k in range(len(channels) - 1):
            layers.append(_linear(channels[k], channels[k + 1], True, generator))
            if k < len(channels) - 2:
                layers.append(nn.LayerNorm(channels[k + 1]))
                layers.append(nn.SiLU())
        self.net = nn.Sequential(*layers)

    def forward(self, x):
        return self.net(x)


class SO2_m_Convolution(nn.Module):
    def __init__(self, in_ch: int, out_ch: int, generator=None):
        super().__init__()
        # rows [:out] are the real part R, rows [out:] the imaginary part I (wrapper.py:57-71)
        self.fc = _linear(in_ch, 2 * out_ch, False, generator)


class SO2_Convolution(nn.Module):
    """Parameter container of FAIRChem's SO2_Convolution for mmax = 2."""

    def __init__(self, C: int, lmax: int, in_mult: int, out_mult_m0: int, out_mult_m: list[int],
                 rad_channels: list[int] | None, generator=None):
        super().__init__()
        self.rad_func = RadialFunction(rad_channels, generator) if rad_channels else None
        m0_in = in_mult * (lmax + 1) * C
        self.fc_m0 = _linear(m0_in, out_mult_m0 * C, True, generator)
        self.so2_m_conv = nn.ModuleList()
        for m in (1, 2):
            n_l = lmax + 1 - m
            self.so2_m_conv.append(SO2_m_Convolution(in_mult * n_l * C, out_mult_m[m - 1] * C, generator))


class Edgewise(nn.Module):
    def __init__(self, C: int, B: int, lmax: int, generator=None):
        super().__init__()
        rad = [B + 2 * C, C, C, 6 * lmax * C]
        # conv1: inputs are (sender, receiver) pairs -> in_mult 2; m0 output carries the
        # (lmax+1)C values plus lmax*C gate scalars; m>0 outputs n_l * C per part.
        self.so2_conv_1 = SO2_Convolution(C, lmax, 2, 2 * lmax + 1, [lmax, lmax - 1], rad, generator)
        self.so2_conv_2 = SO2_Convolution(C, lmax, 1, lmax + 1, [lmax, lmax - 1], None, generator)


class eSCNMD_Block(nn.Module):
    def __init__(self, C: int, H: int, B: int, lmax: int, generator=None):
        super().__init__()
        self.norm_1 = EquivariantRMSNormArraySphericalHarmonicsV2(lmax, C)
        self.edge_wise = Edgewise(C, B, lmax, generator)
        self.norm_2 = EquivariantRMSNormArraySphericalHarmonicsV2(lmax, C)
        self.atom_wise = SpectralAtomwise(C, H, lmax, generator)


class ChgSpinEmbedding(nn.Module):
    """Learned table indexed by the integer charge (offset 100) or spin multiplicity."""

    def __init__(self, C: int, offset: int, size: int, generator=None):
        super().__init__()
        self.offset = offset
        self.table = _embedding(size, C, generator)

    def forward(self, v: torch.Tensor) -> torch.Tensor:
        return self.table(v.long() + self.offset)


class EdgeDegreeEmbedding(nn.Module):
    def __init__(self, C: int, B: int, lmax: int, generator=None):
        super().__init__()
        self.rad_func = RadialFunction([B + 2 * C, C, C, (lmax + 1) * C], generator)
        self.rescale_factor = 5.0


class eSCNMDBackbone(nn.Module):
    """UMA-s-shaped eSCN-MD backbone with seeded random weights (parameters only; the
    forward pass is the ZeroAllocBackbone's)."""

    def __init__(self, num_layers: int = 4, sphere_channels: int = 128, hidden_channels: int = 128,
                 lmax: int = 2, mmax: int = 2, num_distance_basis: int = 64, cutoff: float = 6.0,
                 max_neighbors: int = 30, max_num_elements: int = 100, seed: int = 0,
                 charge_channels: tuple = (0, 0), spin_channels: tuple = (0, 0)):
        super().__init__()
        if mmax != 2:
            raise ValueError("only mmax = 2 is modelled")
        g = torch.Generator().manual_seed(seed)
        C = sphere_channels
        self.lmax, self.mmax = lmax, mmax
        self.num_layers = num_layers
        self.sphere_channels = C
        self.edge_channels = C
        self.hidden_channels = hidden_channels
        self.num_distance_basis = num_distance_basis
        self.cutoff = cutoff
        self.max_neighbors = max_neighbors
        self.sphere_embedding = _embedding(max_num_elements, C, g)
        self.source_embedding = _embedding(max_num_elements, C, g)
        self.target_embedding = _embedding(max_num_elements, C, g)
        self.edge_degree_embedding = EdgeDegreeEmbedding(C, num_distance_basis, lmax, g)
        self.blocks = nn.ModuleList(
            [eSCNMD_Block(C, hidden_channels, num_distance_basis, lmax, g) for _ in range(num_layers)])
        self.norm = EquivariantRMSNormArraySphericalHarmonicsV2(lmax, C)
        self.charge_embedding = ChgSpinEmbedding(C, 100, 201, g)
        self.spin_embedding = ChgSpinEmbedding(C, 0, 101, g)
        self.dataset_embedding = None
        self.use_dataset_embedding = False
        self.mix_csd = _linear(2 * C, C, True, g)
        # l = 0 channel ranges balanced to the system charge / spin after every block
        self.charge_channel_start, self.charge_channel_end = (int(v) for v in charge_channels)
        self.spin_channel_start, self.spin_channel_end = (int(v) for v in spin_channels)
        self.regress_config = SimpleNamespace(forces=True, stress=True, direct_forces=False)
