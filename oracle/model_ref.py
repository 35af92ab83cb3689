"""Whole-backbone CPU oracle: eSCN_Inference_Model.forward (model.py:187-221), the wrapper's
system embedding and shifts (wrapper.py:163-197), the node modules and the energy head,
with forces and stress from torch autograd — test infrastructure only.

Inputs are the parameters of the FAIRChem-shaped backbone object (read by name, the way
transfer_weights reads them, wrapper.py:22-85) and of the energy head.  All arithmetic is
in the requested dtype (float64 for parity references) on the CPU, in input atom and edge
order; the Morton permutation and edge sorting of the GPU path only change memory order.

Node modules (rms_norm_sh, so3_linear, spectral atom-wise FFN, energy head) restate the
published FAIRChem eSCN-MD modules (fairchem-core, which the reference's setup.sh clones at
git main) that the reference calls at model.py:145,157,218; no FAIRChem code or fixtures
exist in the reference tree.  tests/test_oracle_node_pins.py pins them against the library
routines they reduce to at lmax = 0 (LayerNorm, Linear, a Linear-SiLU-Linear MLP),
hand-derived known answers, per-module equivariance and the gate wiring; the head through
finite differences of the energy.
"""
from __future__ import annotations

import torch
import torch.nn.functional as F

from . import ops_ref as R
from . import sh_ref


def _p(t: torch.Tensor, dtype) -> torch.Tensor:
    return t.detach().to("cpu", dtype)


def degree_index(lmax: int) -> torch.Tensor:
    return torch.cat([torch.full((2 * l + 1,), l, dtype=torch.long) for l in range(lmax + 1)])


def rms_norm_sh(x, weight, bias, lmax: int, eps: float):
    """Equivariant RMS norm (flash-uma_amd/node_layers.py): centre l=0 over channels, scale
    by the degree-balanced mean square, per-(l, c) weight, l=0 bias."""
    l0 = x[:, :1] - x[:, :1].mean(dim=2, keepdim=True)
    feat = torch.cat([l0, x[:, 1:]], 1)
    deg = degree_index(lmax)
    w_deg = torch.tensor([1.0 / ((2 * l + 1) * (lmax + 1)) for l in deg.tolist()], dtype=x.dtype)
    ms = (feat.pow(2) * w_deg[None, :, None]).sum(1, keepdim=True).mean(2, keepdim=True)
    out = feat * (ms + eps).pow(-0.5) * weight[deg][None]
    return out + torch.cat([bias[None, None], torch.zeros(1, x.shape[1] - 1, x.shape[2], dtype=x.dtype)], 1)


def so3_linear(x, weight, bias, lmax: int):
    deg = degree_index(lmax)
    out = torch.einsum("nki,koi->nko", x, weight[deg])
    return torch.cat([out[:, :1] + bias[None, None], out[:, 1:]], 1)


def spectral_atomwise(x, P: dict, prefix: str, lmax: int, H: int):
    gates = F.silu(x[:, 0] @ P[prefix + "scalar_mlp.0.weight"].T + P[prefix + "scalar_mlp.0.bias"])
    h = so3_linear(x, P[prefix + "so3_linear_1.weight"], P[prefix + "so3_linear_1.bias"], lmax)
    g = torch.sigmoid(gates).view(-1, lmax, H)[:, degree_index(lmax)[1:] - 1]
    h = torch.cat([F.silu(h[:, :1]), h[:, 1:] * g], 1)
    return so3_linear(h, P[prefix + "so3_linear_2.weight"], P[prefix + "so3_linear_2.bias"], lmax)


def radial_mlp(x, P: dict, prefix: str):
    """Linear -> LN+SiLU -> Linear -> LN+SiLU -> Linear with the reference's LN eps = 1e-7
    (ops/ln_silu.py:180; model.py:147-149)."""
    h = R.layer_norm_silu(x @ P[prefix + "0.weight"].T + P[prefix + "0.bias"], P[prefix + "1.weight"],
                          P[prefix + "1.bias"], 1e-7)
    h = R.layer_norm_silu(h @ P[prefix + "3.weight"].T + P[prefix + "3.bias"], P[prefix + "4.weight"],
                          P[prefix + "4.bias"], 1e-7)
    return h @ P[prefix + "6.weight"].T + P[prefix + "6.bias"]


def energy_forces_stress(backbone, head, pos, Z, cell, edge_index, cell_offsets, charge: int = 0, spin: int = 0,
                         dtype=torch.float64, stress: bool = True):
    """Returns dict(energy (1,), atom_energy (N,), forces (N, 3), stress (1, 3, 3) or None,
    node_embedding (N, (lmax+1)^2, C)) computed on the CPU in `dtype`."""
    P = {k: _p(v, dtype) for k, v in backbone.state_dict().items()}
    H = {k: _p(v, dtype) for k, v in head.state_dict().items()}
    lmax = backbone.lmax
    C = backbone.sphere_channels
    Hc = backbone.hidden_channels
    B = backbone.num_distance_basis
    cutoff = float(backbone.cutoff)
    offset_g = torch.linspace(0.0, cutoff, B)
    coeff_g = float(-0.5 / (2.0 * (offset_g[1] - offset_g[0])) ** 2)   # wrapper.py:122-125
    offset_g = offset_g.to(dtype)

    pos = torch.as_tensor(pos).to(dtype).clone().requires_grad_(True)
    cell = torch.as_tensor(cell).to(dtype).reshape(3, 3).clone().requires_grad_(stress)
    Z = torch.as_tensor(Z, dtype=torch.long)
    ei = torch.as_tensor(edge_index, dtype=torch.long)
    idx_i, idx_j = ei[0], ei[1]
    N = pos.shape[0]
    batch = torch.zeros(N, dtype=torch.long)

    # system (charge/spin) embedding, wrapper.py:163-169
    chg = P["charge_embedding.table.weight"][torch.tensor([charge + 100])]
    spn = P["spin_embedding.table.weight"][torch.tensor([spin])]
    csd = F.silu(torch.cat([chg, spn], 1) @ P["mix_csd.weight"].T + P["mix_csd.bias"])

    shifts = torch.as_tensor(cell_offsets).to(dtype) @ cell          # wrapper.py:193-194
    x_edge_raw, wigner, env = R.edge_geometry(pos, Z, idx_i, idx_j, shifts, P["source_embedding.weight"],
                                              P["target_embedding.weight"], offset_g, coeff_g, cutoff)
    L = lmax
    # lmax > 2: rows |m| <= 2 of D^3, D^4 from the rotation D^1 (tensor representation)
    wig_ext = sh_ref.wigner_ext(wigner[:, :9].reshape(-1, 3, 3), L) if L > 2 else None
    rad0 = radial_mlp(x_edge_raw, P, "edge_degree_embedding.rad_func.net.")
    if L == 2:
        x = R.init_scatter(rad0, wigner, env, Z, batch, P["sphere_embedding.weight"], csd, idx_j, N)
    else:
        x = R.init_scatter_lmax(rad0, wigner, wig_ext, env, Z, batch, P["sphere_embedding.weight"], csd, idx_j, N, L)
    for l in range(backbone.num_layers):
        pre = f"blocks.{l}."
        c1 = pre + "edge_wise.so2_conv_1."
        c2 = pre + "edge_wise.so2_conv_2."
        xn = rms_norm_sh(x, P[pre + "norm_1.affine_weight"], P[pre + "norm_1.affine_bias"], lmax, 1e-5)
        rad = radial_mlp(x_edge_raw, P, c1 + "rad_func.net.")
        if L == 2:
            X0, X1, X2 = R.gather_rotate(xn, idx_i, idx_j, wigner, rad, csd, batch)
        else:
            X0, X1, X2 = R.gather_rotate_lmax(xn, idx_i, idx_j, wigner, wig_ext, rad, csd, batch, L)
        # SO(2) m > 0 weights: rows [:n C] are R, [n C:] are I, n = L (m = 1) or L - 1 (m = 2)
        w1 = P[c1 + "so2_m_conv.0.fc.weight"]
        w2 = P[c1 + "so2_m_conv.1.fc.weight"]
        W1_m1 = R.pack_so2(w1[:L * C], w1[L * C:])
        W1_m2 = R.pack_so2(w2[:(L - 1) * C], w2[(L - 1) * C:])
        Y0 = X0 @ P[c1 + "fc_m0.weight"].T + P[c1 + "fc_m0.bias"]
        Y1 = X1 @ W1_m1.T
        Y2 = X2 @ W1_m2.T
        Z0, Z1, Z2 = R.gating(Y0, Y1, Y2, C) if L == 2 else R.gating_lmax(Y0, Y1, Y2, C, L)
        v1 = P[c2 + "so2_m_conv.0.fc.weight"]
        v2 = P[c2 + "so2_m_conv.1.fc.weight"]
        Zo0 = Z0 @ P[c2 + "fc_m0.weight"].T + P[c2 + "fc_m0.bias"]
        Zo1 = Z1 @ R.pack_so2(v1[:L * C], v1[L * C:]).T
        Zo2 = Z2 @ R.pack_so2(v2[:(L - 1) * C], v2[(L - 1) * C:]).T
        if L == 2:
            x_mid = R.rotate_scatter(Zo0, Zo1, Zo2, wigner, env, x, idx_j, N)
        else:
            x_mid = R.rotate_scatter_lmax(Zo0, Zo1, Zo2, wigner, wig_ext, env, x, idx_j, N, L)
        h = rms_norm_sh(x_mid, P[pre + "norm_2.affine_weight"], P[pre + "norm_2.affine_bias"], lmax, 1e-5)
        x = spectral_atomwise(h, P, pre + "atom_wise.", lmax, Hc) + x_mid
        # charge / spin channel balancing after every block (model.py:213-216)
        if backbone.charge_channel_end > backbone.charge_channel_start:
            x = R.balance_channels(x, torch.tensor([charge]), batch, 1, backbone.charge_channel_start,
                                   backbone.charge_channel_end, 0.0)
        if backbone.spin_channel_end > backbone.spin_channel_start:
            x = R.balance_channels(x, torch.tensor([spin]), batch, 1, backbone.spin_channel_start,
                                   backbone.spin_channel_end, 1.0)
    x = rms_norm_sh(x, P["norm.affine_weight"], P["norm.affine_bias"], lmax, 1e-5)

    h = x[:, 0]
    n_lin = len([k for k in H if k.endswith(".weight")])
    for k in range(n_lin):
        h = h @ H[f"layers.{k}.weight"].T + H[f"layers.{k}.bias"]
        if k < n_lin - 1:
            h = F.silu(h)
    e_atom = h.squeeze(-1)
    energy = e_atom.sum().reshape(1)
    inputs = [pos] + ([cell] if stress else [])
    grads = torch.autograd.grad(energy.sum(), inputs, allow_unused=True)
    g_pos = grads[0]
    out = {"energy": energy.detach(), "atom_energy": e_atom.detach(), "forces": (-g_pos).detach(),
           "node_embedding": x.detach(), "stress": None}
    if stress:
        g_cell = grads[1] if grads[1] is not None else torch.zeros_like(cell)
        w = pos.detach().T @ g_pos + cell.detach().T @ g_cell
        out["stress"] = (w / torch.linalg.det(cell.detach()).abs()).reshape(1, 3, 3).detach()
    return out
