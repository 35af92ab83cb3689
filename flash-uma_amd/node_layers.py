"""Node-level modules of the eSCN-MD block on the gfx950 node kernels (ops/node.py).

FAIRChem's block applies, per node, an equivariant RMS norm over the spherical-harmonic
coefficients ("rms_norm_sh", EquivariantRMSNormArraySphericalHarmonicsV2) before the edge-wise
convolution and before a gated SO(3) feed-forward block (SpectralAtomwise: a scalar MLP giving
per-degree gates, SO3_Linear, GateActivation, SO3_Linear); the reference attaches the official
modules as they are (wrapper.py:74-79) and calls them from its block (model.py:145 and
model.py:156-157).  The classes here compute the same functions with the HIP kernels: the norm's
forward and backward are one kernel each, the atom-wise block is two batched per-degree GEMMs
and the gate kernel, with the skip connections added inside the kernels.

`adopt_rms_norm` and `adopt_atom_wise` build these modules from any module that carries
FAIRChem's parameter names (affine_weight, affine_bias; scalar_mlp.0, so3_linear_1,
so3_linear_2) and the configuration the kernels compute; a module that does not is kept and
called as given, with a warning.
"""
from __future__ import annotations

import math
import warnings

import torch
import torch.nn as nn

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


def _shape(t, shape) -> bool:
    return torch.is_tensor(t) and t.is_floating_point() and tuple(t.shape) == tuple(shape)


def _norm_mismatch(mod, lmax: int, C: int) -> str | None:
    """Why `mod` is not the norm the kernels compute (None if it is).  FAIRChem's
    configuration attributes are checked when present; without them the module is taken to
    have the defaults of the "rms_norm_sh" layer (component normalisation, l = 0 centring,
    degree-balanced mean, affine)."""
    if not _shape(getattr(mod, "affine_weight", None), (lmax + 1, C)):
        return f"no affine_weight of shape ({lmax + 1}, {C})"
    if not _shape(getattr(mod, "affine_bias", None), (C,)):
        return f"no affine_bias of shape ({C},)"
    for name, want in (("lmax", lmax), ("num_channels", C), ("affine", True), ("centering", True),
                       ("std_balance_degrees", True), ("normalization", "component")):
        if hasattr(mod, name) and getattr(mod, name) != want:
            return f"{name} = {getattr(mod, name)!r}, the kernels compute {name} = {want!r}"
    bal = getattr(mod, "balance_degree_weight", None)
    if bal is not None:
        want = EquivariantRMSNormArraySphericalHarmonicsV2(lmax, C).balance_degree_weight
        if tuple(bal.shape) != tuple(want.shape) or not torch.allclose(bal.detach().cpu().float(), want):
            return "balance_degree_weight differs from 1 / ((2l + 1)(lmax + 1))"
    return None


@torch.no_grad()
def adopt_rms_norm(mod: nn.Module, lmax: int, C: int) -> nn.Module:
    """The HIP-backed norm with the parameters (affine_weight, affine_bias, eps) of `mod`,
    on its device; `mod` itself if it is one already or does not carry them."""
    if isinstance(mod, EquivariantRMSNormArraySphericalHarmonicsV2):
        return mod
    why = _norm_mismatch(mod, lmax, C)
    if why is not None:
        warnings.warn(f"{type(mod).__name__} kept as given (not on the HIP node kernels): {why}")
        return mod
    new = EquivariantRMSNormArraySphericalHarmonicsV2(lmax, C, eps=float(getattr(mod, "eps", 1e-5)))
    new.affine_weight.copy_(mod.affine_weight)
    new.affine_bias.copy_(mod.affine_bias)
    return new.to(mod.affine_weight.device)


def _atom_wise_mismatch(mod, lmax: int, C: int) -> str | None:
    """Why `mod` is not the gated SO(3) feed-forward block the kernels compute (None if it is)."""
    mlp = getattr(mod, "scalar_mlp", None)
    l1, l2 = getattr(mod, "so3_linear_1", None), getattr(mod, "so3_linear_2", None)
    if mlp is None or l1 is None or l2 is None:
        return "no scalar_mlp, so3_linear_1 and so3_linear_2"
    w1 = getattr(l1, "weight", None)
    if not torch.is_tensor(w1) or w1.dim() != 3:
        return "so3_linear_1.weight is not (lmax + 1, hidden, channels)"
    H = w1.shape[1]
    try:
        lin = mlp[0]
        acts = list(mlp)[1:]
    except (TypeError, IndexError):
        return "scalar_mlp is not a sequence starting with a Linear"
    if not _shape(getattr(lin, "weight", None), (lmax * H, C)) or not _shape(getattr(lin, "bias", None), (lmax * H,)):
        return f"scalar_mlp.0 is not a Linear {C} -> {lmax * H} with bias"
    if len(acts) != 1 or type(acts[0]) is not nn.SiLU:
        return "scalar_mlp is not Linear followed by SiLU"
    for name, l, o, i in (("so3_linear_1", l1, H, C), ("so3_linear_2", l2, C, H)):
        if not _shape(getattr(l, "weight", None), (lmax + 1, o, i)) or not _shape(getattr(l, "bias", None), (o,)):
            return f"{name} is not a per-degree map {i} -> {o} with an l = 0 bias"
        if hasattr(l, "lmax") and l.lmax != lmax:
            return f"{name}.lmax = {l.lmax}"
    act = getattr(mod, "act", None)
    if act is not None:
        for name, cls in (("gate_act", nn.Sigmoid), ("scalar_act", nn.SiLU)):
            if hasattr(act, name) and type(getattr(act, name)) is not cls:
                return f"act.{name} is not {cls.__name__}"
    return None


@torch.no_grad()
def adopt_atom_wise(mod: nn.Module, lmax: int, C: int) -> nn.Module:
    """The HIP-backed SpectralAtomwise with the parameters (scalar_mlp.0, so3_linear_1,
    so3_linear_2) of `mod`, on its device; `mod` itself if it is one already or does not carry
    them."""
    if isinstance(mod, SpectralAtomwise):
        return mod
    why = _atom_wise_mismatch(mod, lmax, C)
    if why is not None:
        warnings.warn(f"{type(mod).__name__} kept as given (not on the HIP node kernels): {why}")
        return mod
    H = mod.so3_linear_1.weight.shape[1]
    new = SpectralAtomwise(C, H, lmax)
    new.scalar_mlp[0].weight.copy_(mod.scalar_mlp[0].weight)
    new.scalar_mlp[0].bias.copy_(mod.scalar_mlp[0].bias)
    for name in ("so3_linear_1", "so3_linear_2"):
        getattr(new, name).weight.copy_(getattr(mod, name).weight)
        getattr(new, name).bias.copy_(getattr(mod, name).bias)
    return new.to(mod.so3_linear_1.weight.device)
