"""Plain-PyTorch node modules with FAIRChem's parameter and attribute names, as a FAIRChem
backbone carries them (EquivariantRMSNormArraySphericalHarmonicsV2, SO3_Linear,
GateActivation, SpectralAtomwise of fairchem.core.models.uma; FAIRChem is not installed here).
Their forward passes are the published ones written with torch tensor ops: a backbone that
carries these is what transfer_weights meets in practice, and nothing here calls the HIP
library.  tests/test_node_adoption.py pins them against the float64 oracle."""
from __future__ import annotations

import torch
import torch.nn as nn


def _degree_index(lmax: int) -> torch.Tensor:
    return torch.cat([torch.full((2 * l + 1,), l, dtype=torch.long) for l in range(lmax + 1)])


class FCRMSNorm(nn.Module):
    def __init__(self, lmax: int, num_channels: int, eps: float = 1e-5, centering: bool = True):
        super().__init__()
        self.lmax, self.num_channels, self.eps = lmax, num_channels, eps
        self.affine, self.centering, self.std_balance_degrees = True, centering, True
        self.normalization = "component"
        self.affine_weight = nn.Parameter(torch.ones(lmax + 1, num_channels))
        self.affine_bias = nn.Parameter(torch.zeros(num_channels))
        self.register_buffer("expand_index", _degree_index(lmax), persistent=False)
        w = torch.zeros((lmax + 1) ** 2, 1, dtype=torch.float64)   # exact in the float64 pins
        for l in range(lmax + 1):
            w[l * l:(l + 1) ** 2] = 1.0 / (2 * l + 1)
        self.register_buffer("balance_degree_weight", w / (lmax + 1), persistent=False)

    def forward(self, x):
        f = x
        if self.centering:
            f0 = f.narrow(1, 0, 1)
            f = torch.cat((f0 - f0.mean(dim=2, keepdim=True), f.narrow(1, 1, f.shape[1] - 1)), dim=1)
        norm = torch.einsum("nic,ia->nac", f.pow(2), self.balance_degree_weight.to(f.dtype))
        norm = (norm.mean(dim=2, keepdim=True) + self.eps).pow(-0.5)
        w = self.affine_weight.view(1, self.lmax + 1, self.num_channels).index_select(1, self.expand_index)
        out = f * (norm * w)
        if self.centering:
            out = torch.cat((out.narrow(1, 0, 1) + self.affine_bias.view(1, 1, -1), out.narrow(1, 1, out.shape[1] - 1)),
                            dim=1)
        return out


class FCSO3Linear(nn.Module):
    def __init__(self, in_features: int, out_features: int, lmax: int):
        super().__init__()
        self.in_features, self.out_features, self.lmax = in_features, out_features, lmax
        self.weight = nn.Parameter(torch.zeros(lmax + 1, out_features, in_features))
        self.bias = nn.Parameter(torch.zeros(out_features))
        self.register_buffer("expand_index", _degree_index(lmax), persistent=False)

    def forward(self, x):
        w = self.weight.index_select(0, self.expand_index)
        out = torch.einsum("bmi,moi->bmo", x, w)
        return torch.cat((out.narrow(1, 0, 1) + self.bias.view(1, 1, -1), out.narrow(1, 1, out.shape[1] - 1)), dim=1)


class FCGateActivation(nn.Module):
    def __init__(self, lmax: int, num_channels: int):
        super().__init__()
        self.lmax, self.num_channels = lmax, num_channels
        self.scalar_act = nn.SiLU()
        self.gate_act = nn.Sigmoid()
        self.register_buffer("expand_index", _degree_index(lmax)[1:] - 1, persistent=False)

    def forward(self, gating_scalars, x):
        g = self.gate_act(gating_scalars).reshape(x.shape[0], self.lmax, self.num_channels)
        g = g.index_select(1, self.expand_index)
        return torch.cat((self.scalar_act(x.narrow(1, 0, 1)), x.narrow(1, 1, x.shape[1] - 1) * g), dim=1)


class FCSpectralAtomwise(nn.Module):
    def __init__(self, sphere_channels: int, hidden_channels: int, lmax: int, act=nn.SiLU):
        super().__init__()
        self.scalar_mlp = nn.Sequential(nn.Linear(sphere_channels, lmax * hidden_channels, bias=True), act())
        self.so3_linear_1 = FCSO3Linear(sphere_channels, hidden_channels, lmax)
        self.act = FCGateActivation(lmax, hidden_channels)
        self.so3_linear_2 = FCSO3Linear(hidden_channels, sphere_channels, lmax)

    def forward(self, x):
        gates = self.scalar_mlp(x.narrow(1, 0, 1))
        return self.so3_linear_2(self.act(gates, self.so3_linear_1(x)))


@torch.no_grad()
def fairchem_like(bb):
    """Replace every node module of the stand-in backbone `bb` (in place) by one of the classes
    above carrying the same parameter values; returns bb."""
    L, C = bb.lmax, bb.sphere_channels

    def norm(src):
        m = FCRMSNorm(L, C)
        m.affine_weight.copy_(src.affine_weight); m.affine_bias.copy_(src.affine_bias)
        return m.to(src.affine_weight.device)

    def ffn(src):
        H = src.so3_linear_1.weight.shape[1]
        m = FCSpectralAtomwise(C, H, L)
        m.load_state_dict(src.state_dict())
        return m.to(src.so3_linear_1.weight.device)

    for blk in bb.blocks:
        blk.norm_1, blk.norm_2, blk.atom_wise = norm(blk.norm_1), norm(blk.norm_2), ffn(blk.atom_wise)
    bb.norm = norm(bb.norm)
    return bb
