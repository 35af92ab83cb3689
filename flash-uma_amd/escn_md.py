"""Random-init stand-in for FAIRChem's UMA eSCN-MD backbone and its node-level modules.

The reference wraps an official `eSCNMDBackbone` (fairchem.core.models.uma.escn_md) and
copies its weights (wrapper.py:22-85); FAIRChem is not in the reference tree and cannot be
installed offline.  This module provides an object with exactly the attributes
`transfer_weights` and `ZeroAllocBackbone.__init__` read (wrapper.py:28-146), shaped like
UMA-s, with seeded random weights, plus the node modules the reference attaches by
reference (norm_1, norm_2, atom_wise, final norm, charge/spin embeddings).

The node modules restate the published FAIRChem eSCN-MD designs (no FAIRChem code or
fixtures exist here).  Their GPU forward and backward are checked against the CPU oracle's
restatement, which is itself checked against the library routines the modules reduce to at
lmax = 0 (LayerNorm, Linear, a Linear-SiLU-Linear MLP), hand-derived known answers and
equivariance.  Their forward passes run on the gfx950 node kernels
(ops/node.py: RMS norm, batched per-degree MFMA GEMM, gate activation); like the rest of
the backbone they need GPU tensors.

Initialisation (seeded CPU torch.Generator, fixed creation order): nn.Linear default
(kaiming-uniform weights, uniform bias), nn.Embedding N(0, 1), LayerNorm/affine weights 1,
biases 0.
"""
from __future__ import annotations

import math
from types import SimpleNamespace

import torch
import torch.nn as nn
import torch.nn.functional as F

from ops.linear import linear
from ops.node import (gate_act, rms_norm_sh, rms_norm_sh_residual, scalar_gemm_so3, so3_linear,
                      so3_linear_residual)


def num_coefficients(lmax: int) -> int:
    return (lmax + 1) ** 2


def degree_index(lmax: int) -> torch.Tensor:
    """Degree l of every SH coefficient k (k = l^2 + l + m)."""
    return torch.cat([torch.full((2 * l + 1,), l, dtype=torch.long) for l in range(lmax + 1)])


class EquivariantRMSNormArraySphericalHarmonicsV2(nn.Module):
    """Equivariant RMS norm over SH coefficients (FAIRChem's "rms_norm_sh" layer, recalled):
    subtract the channel mean of l=0, scale every coefficient by
    (mean_c sum_l w_l mean_{m} x_{lm,c}^2 + eps)^(-1/2) with degree-balanced weights
    w_l = 1/(lmax+1), apply a per-(l, c) affine weight and an l=0 bias."""

    def __init__(self, lmax: int, num_channels: int, eps: float = 1e-5):
        super().__init__()
        self.lmax = lmax
        self.num_channels = num_channels
        self.eps = eps
        self.affine_weight = nn.Parameter(torch.ones(lmax + 1, num_channels))
        self.affine_bias = nn.Parameter(torch.zeros(num_channels))
        self.register_buffer("expand_index", degree_index(lmax), persistent=False)
        bal = torch.zeros(num_coefficients(lmax), 1)
        for l in range(lmax + 1):
            bal[l * l:(l + 1) * (l + 1)] = 1.0 / (2 * l + 1)
        self.register_buffer("balance_degree_weight", bal / (lmax + 1), persistent=False)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return rms_norm_sh(x, self.affine_weight, self.affine_bias, self.lmax, self.eps)

    def forward_with_residual(self, x: torch.Tensor):
        """(norm(x), x) for an x that also feeds a residual skip; the backward sums the two
        gradients inside the norm's backward kernel."""
        return rms_norm_sh_residual(x, self.affine_weight, self.affine_bias, self.lmax, self.eps)


class SO3_Linear(nn.Module):
    """Per-degree linear map: coefficient (l, m) of the output is W_l x_(l, m); l=0 has a bias."""

    def __init__(self, in_features: int, out_features: int, lmax: int, generator=None):
        super().__init__()
        self.lmax = lmax
        bound = 1.0 / math.sqrt(in_features)
        self.weight = nn.Parameter(torch.empty(lmax + 1, out_features, in_features).uniform_(
            -bound, bound, generator=generator))
        self.bias = nn.Parameter(torch.empty(out_features).uniform_(-bound, bound, generator=generator))
        self.register_buffer("expand_index", degree_index(lmax), persistent=False)

    def per_coefficient_weights(self):
        """(W_k, W_k^T) stacked over the (lmax+1)^2 coefficients (weights are frozen)."""
        w = self.weight.detach().index_select(0, self.expand_index).contiguous()
        return w, w.transpose(1, 2).contiguous()

    def weights(self, device) -> tuple:
        """(W_k, W_k^T, bias) on `device`, built once per device (weights are frozen)."""
        if getattr(self, "_wk", None) is None or self._wk[0].device != device:
            self._wk = self.per_coefficient_weights()
        return self._wk[0], self._wk[1], self.bias.detach()

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return so3_linear(x, *self.weights(x.device))


class GateActivation(nn.Module):
    """l=0 -> SiLU; coefficients of degree l>0 scaled by sigmoid(gate_l) per channel."""

    def __init__(self, lmax: int, num_channels: int):
        super().__init__()
        self.lmax = lmax
        self.num_channels = num_channels
        self.register_buffer("gate_index", (degree_index(lmax)[1:] - 1), persistent=False)

    def forward(self, pre: torch.Tensor, x: torch.Tensor) -> torch.Tensor:
        """pre: the scalar MLP's pre-activation (N, lmax * H); the gate is
        sigmoid(silu(pre)) per degree (FAIRChem applies SiLU in the scalar MLP and the
        sigmoid here)."""
        return gate_act(pre, x, self.lmax)


class SpectralAtomwise(nn.Module):
    """Per-node gated SO(3) feed-forward block (FAIRChem's spectral atom-wise FFN, recalled)."""

    def __init__(self, sphere_channels: int, hidden_channels: int, lmax: int, generator=None):
        super().__init__()
        self.scalar_mlp = nn.Sequential(_linear(sphere_channels, lmax * hidden_channels, True, generator), nn.SiLU())
        self.so3_linear_1 = SO3_Linear(sphere_channels, hidden_channels, lmax, generator)
        self.act = GateActivation(lmax, hidden_channels)
        self.so3_linear_2 = SO3_Linear(hidden_channels, sphere_channels, lmax, generator)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        lin = self.scalar_mlp[0]
        if getattr(self, "_wt", None) is None or self._wt.device != x.device:
            self._wt = lin.weight.detach().t().contiguous()
        pre = linear(x[:, 0, :], lin.weight.detach(), lin.bias.detach(), self._wt)
        h = self.so3_linear_1(x)
        h = self.act(pre, h)
        return self.so3_linear_2(h)

    def forward_residual(self, x: torch.Tensor, skip: torch.Tensor) -> torch.Tensor:
        """forward(x) + skip with no node-sized elementwise pass: the scalar and SO(3) reads of
        x share one backward, and skip is added in the last GEMM's epilogue."""
        lin = self.scalar_mlp[0]
        if getattr(self, "_wt", None) is None or self._wt.device != x.device:
            self._wt = lin.weight.detach().t().contiguous()
        pre, h = scalar_gemm_so3(x, lin.weight.detach(), lin.bias.detach(), self._wt,
                                 *self.so3_linear_1.weights(x.device))
        h = self.act(pre, h)
        return so3_linear_residual(h, *self.so3_linear_2.weights(x.device), skip)


def _linear(i: int, o: int, bias: bool, generator) -> nn.Linear:
    lin = nn.Linear(i, o, bias=bias)
    bound = 1.0 / math.sqrt(i)
    with torch.no_grad():
        lin.weight.uniform_(-bound, bound, generator=generator)
        if bias:
            lin.bias.uniform_(-bound, bound, generator=generator)
    return lin


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
