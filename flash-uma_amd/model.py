"""eSCN-MD inference model on the gfx950 kernels (mirrors the reference model.py).

Public names and signatures follow the reference: reorder_graph_morton, build_csr_cached,
clear_csr_cache (model.py:17-74), Packed_eSCN_Layer (model.py:81-157) and
eSCN_Inference_Model (model.py:160-221).  Every per-edge and per-CSR operation runs in
libflashuma_hip.so; the node-level modules set by transfer_weights (norm_1, norm_2,
atom_wise, final_norm) are the HIP-backed ones of node_layers.py, rebuilt from FAIRChem's
modules by parameter name (a module without FAIRChem's parameters is called as given).

Differences in mechanism (not in results):
  - the graph topology (Morton order, receiver-sorted edge order, receiver and sender CSRs)
    is built once per edge_index on the GPU and cached (ops/topology.py);
  - dense layers use the fp32 MFMA GEMM with pre-transposed frozen weights for the input
    gradient (ops/linear.py);
  - the m = 1, 2 SO(2) layers keep their weights as complex pairs (R, I) and run the
    three-product complex layer instead of the packed [[R, -I], [I, R]] GEMM: the same
    product, one quarter fewer flops.

lmax: the reference builds lmax = 2 only (wrapper.py:105-118).  Here lmax = 3 and 4 are
supported too (mmax = 2): the per-edge blocks grow degree by degree in the reference's order
(ops/lmax.py), the Wigner rows of degree 3 and 4 come from fu_wigner_ext_fwd, and the layer
runs the same fused conv1 + gate + conv2 as lmax = 2 (gate-paired conv1 m = 0 rows); only
lmax = 2 also permutes the gather blocks side-major.
"""
from __future__ import annotations

from collections import OrderedDict

import torch
import torch.nn as nn

from ops.gather import LAYOUT1_PERM, block_permutation
from ops.gating import edge_block, gate_paired_rows
from ops.edge_grad import EdgeGradSink
from ops.geom import precompute_geometry
from ops.linear import complex_linear, complex_weight_split, linear, linear_weight_split
from ops.lmax import init_node_scatter_lmax, rotate_scatter_lmax, wigner_extend
from ops.ln_silu import layer_norm_silu
from ops.node import balance_channels_batched, permute_rows, system_ptr
from ops.radial import RadialBank
from ops.scatter import init_node_scatter, rotate_scatter_split
from ops.topology import (clear_topology_cache, get_topology, morton_permutation, receiver_csr, take)

# ==============================================================================
# 1. GRAPH PREPROCESSING (MORTON & CSR CACHING)
# ==============================================================================

_CSR_CACHE_CAPACITY = 8
_csr_cache: "OrderedDict[tuple, tuple]" = OrderedDict()


def build_csr_cached(idx_j: torch.Tensor, N: int):
    """Receiver CSR (row_ptr int32 (N+1), col_idx int32 (E)) with an LRU cache (model.py:28-44).

    The entry keeps idx_j alive, so the (data_ptr, _version) key cannot be matched by a
    different tensor that reuses a freed address."""
    key = (idx_j.data_ptr(), idx_j._version, idx_j.numel(), N,
           idx_j.device.index if idx_j.device.type == "cuda" else -1)
    hit = _csr_cache.get(key)
    if hit is not None:
        _csr_cache.move_to_end(key)
        return hit[0], hit[1]
    row_ptr, col_idx = receiver_csr(idx_j, N)
    _csr_cache[key] = (row_ptr, col_idx, idx_j)
    if len(_csr_cache) > _CSR_CACHE_CAPACITY:
        _csr_cache.popitem(last=False)
    return row_ptr, col_idx


def clear_csr_cache():
    _csr_cache.clear()
    clear_topology_cache()


def expand_bits_torch(v: torch.Tensor) -> torch.Tensor:
    """Bit k (k < 10) of the integer tensor v moved to bit 3k + 1 (model.py:48-54)."""
    out = torch.zeros_like(v)
    for k in range(10):
        out |= ((v >> k) & 1) << (3 * k + 1)
    return out


def morton3d_torch(x: torch.Tensor, y: torch.Tensor, z: torch.Tensor) -> torch.Tensor:
    """Morton code of 10-bit cell indices: x on bits 3k+1, y on 3k+2, z on 3k+3
    (model.py:56-58).  The model computes its sort keys with fu_morton_keys on the GPU; this
    is the reference's public helper, for callers that build keys themselves."""
    return expand_bits_torch(x) | (expand_bits_torch(y) << 1) | (expand_bits_torch(z) << 2)


def reorder_graph_morton(pos, Z, batch, idx_i, idx_j):
    """Morton Z-order of the atoms and remapped edge endpoints (model.py:60-74).
    Returns (pos[perm], Z[perm], batch[perm], inv[idx_i], inv[idx_j], perm, inv)."""
    perm, inv = morton_permutation(pos, batch)
    return (pos[perm], Z[perm], batch[perm], take(inv, idx_i.contiguous()), take(inv, idx_j.contiguous()),
            perm, inv)


# ==============================================================================
# 2. MODEL DEFINITIONS
# ==============================================================================


def _frozen(t: torch.Tensor) -> torch.Tensor:
    return t.detach().clone().contiguous()


class Packed_eSCN_Layer(nn.Module):
    """One eSCN-MD message-passing block (model.py:81-157)."""

    def __init__(self, C: int, B: int, lmax: int = 2):
        super().__init__()
        if lmax not in (2, 3, 4):
            raise ValueError(f"lmax={lmax} unsupported (2, 3 or 4)")
        self.C, self.lmax = C, lmax
        L = lmax
        z = torch.zeros
        self.W_rad1_1 = nn.Parameter(z(C, B + 2 * C)); self.b_rad1_1 = nn.Parameter(z(C))
        self.gamma_rad1_1 = nn.Parameter(torch.ones(C)); self.beta_rad1_1 = nn.Parameter(z(C))
        self.W_rad1_2 = nn.Parameter(z(C, C)); self.b_rad1_2 = nn.Parameter(z(C))
        self.gamma_rad1_2 = nn.Parameter(torch.ones(C)); self.beta_rad1_2 = nn.Parameter(z(C))
        self.W_rad1_3 = nn.Parameter(z(6 * L * C, C)); self.b_rad1_3 = nn.Parameter(z(6 * L * C))

        # m = 0: (L+1) degrees x (sender, receiver) in, L gates + (L+1) values out; m = 1, 2:
        # complex maps over the n = L + 1 - m degrees that carry order m
        self.W1_m0 = nn.Parameter(z((2 * L + 1) * C, 2 * (L + 1) * C)); self.b1_m0 = nn.Parameter(z((2 * L + 1) * C))
        self.W1_m1_R = nn.Parameter(z(L * C, 2 * L * C)); self.W1_m1_I = nn.Parameter(z(L * C, 2 * L * C))
        self.W1_m2_R = nn.Parameter(z((L - 1) * C, 2 * (L - 1) * C))
        self.W1_m2_I = nn.Parameter(z((L - 1) * C, 2 * (L - 1) * C))

        self.W2_m0 = nn.Parameter(z((L + 1) * C, (L + 1) * C)); self.b2_m0 = nn.Parameter(z((L + 1) * C))
        self.W2_m1_R = nn.Parameter(z(L * C, L * C)); self.W2_m1_I = nn.Parameter(z(L * C, L * C))
        self.W2_m2_R = nn.Parameter(z((L - 1) * C, (L - 1) * C)); self.W2_m2_I = nn.Parameter(z((L - 1) * C, (L - 1) * C))

        self.norm_1 = None; self.norm_2 = None; self.atom_wise = None
        self.prepared = False
        self.layout = 0  # gather slot layout; 1 after prepare_for_inference

    def _register(self, name: str, W: torch.Tensor, dtype) -> None:
        W = W.to(dtype).contiguous()
        self._splits_dev = None  # pre-split copies are rebuilt from the new buffers on next use
        self.register_buffer(name, W)
        self.register_buffer(name + "_t", W.t().contiguous())

    def _register_complex(self, name: str, R: torch.Tensor, I: torch.Tensor, dtype) -> None:
        # The reference packs (R + iI) on [real; imag] stacked features as the real block
        # matrix [[R, -I], [I, R]] (model.py:111-138); the complex layer takes R and I
        # themselves, plus R^T and -I^T for its input gradient.
        R = R.to(dtype).contiguous()
        I = I.to(dtype).contiguous()
        self._splits_dev = None  # pre-split copies are rebuilt from the new buffers on next use
        self.register_buffer(name + "_R", R)
        self.register_buffer(name + "_I", I)
        self.register_buffer(name + "_Rt", R.t().contiguous())
        self.register_buffer(name + "_It_neg", (-I).t().contiguous())

    def _complex(self, x: torch.Tensor, name: str) -> torch.Tensor:
        k = 2 * self._COMPLEX.index(name)
        sp = self._complex_splits(x.device)[k:k + 2]
        return complex_linear(x, getattr(self, name + "_R"), getattr(self, name + "_I"), getattr(self, name + "_Rt"),
                              getattr(self, name + "_It_neg"), *sp)

    _COMPLEX = ("W_conv1_m1", "W_conv1_m2", "W_conv2_m1", "W_conv2_m2")

    # The pre-split weights select the three-product (Gauss) complex kernel: y_i = T3 - T1 - T2
    # loses relative accuracy when y_i is much smaller than T1 = x_r P^T, which needs one of P, Q
    # to dominate the other.  A weight whose parts differ in Frobenius norm by more than this
    # factor keeps the four-product kernel (no pre-split copy).
    GAUSS_MAX_NORM_RATIO = 10.0

    # the real m = 0 weights whose tall GEMMs read pre-split fragments (linear_weight_split), in
    # the order conv1_gate_conv2 takes them after the complex splits
    _REAL = ("W_conv1_m0", "W_conv1_m0_t", "W_conv2_m0", "W_conv2_m0_t")

    def _complex_splits(self, dev: torch.device) -> tuple:
        """complex_weight_split of each frozen complex weight and of its transpose pair, in the
        order conv1_gate_conv2 takes them, then linear_weight_split of the m = 0 weights and
        their transposes; built on first use on a device (the weights are frozen), not part of
        the state dict.  None (four-product kernel) for an unbalanced complex weight, and for a
        real weight whose K is not a multiple of 16."""
        if getattr(self, "_splits_dev", None) != dev:
            sp = []
            for name in self._COMPLEX:
                R, I = getattr(self, name + "_R"), getattr(self, name + "_I")
                nr, ni = R.norm().item(), I.norm().item()
                r = self.GAUSS_MAX_NORM_RATIO
                if not (nr <= r * ni and ni <= r * nr):
                    sp += [None, None]
                    continue
                sp.append(complex_weight_split(R, I))
                sp.append(complex_weight_split(getattr(self, name + "_Rt"), getattr(self, name + "_It_neg")))
            for name in self._REAL:
                W = getattr(self, name)
                sp.append(linear_weight_split(W) if W.shape[1] % 16 == 0 else None)
            self._splits, self._splits_dev = tuple(sp), dev
        return self._splits

    def prepare_for_inference(self, dtype=torch.float32):
        if self.norm_1 is not None:
            for mod in (self.norm_1, self.norm_2, self.atom_wise):
                for p in mod.parameters():
                    p.requires_grad = False
        if self.lmax != 2:
            self._prepare_reference_order(dtype)
            return
        # Slot layout 1 of the gather (ops/gather.py): the radial output blocks and the conv1
        # input columns are permuted alike, so rad -> X -> conv1 computes the same products
        # while each side's share of an edge row is contiguous for the gather backward and
        # X_m1 = [x_r | x_i] for the complex layer.
        C = self.C
        dev = self.W1_m0.device
        p_rad = block_permutation(LAYOUT1_PERM["rad"], C).to(dev)
        self.W_rad1_3.data = self.W_rad1_3.data[p_rad].contiguous()
        self.b_rad1_3.data = self.b_rad1_3.data[p_rad].contiguous()
        pm1 = LAYOUT1_PERM["m1"]
        re_order, im_order = pm1[:4], [b - 4 for b in pm1[4:]]
        assert re_order == im_order, "x_r and x_i blocks must be permuted alike"
        c_m1 = block_permutation(re_order, C).to(dev)
        assert LAYOUT1_PERM["m2"] == [0, 1, 2, 3]
        for name in ("W_rad1_1", "W_rad1_2", "W_rad1_3"):
            W = getattr(self, name).data
            self.register_buffer(name + "_t", W.to(dtype).t().contiguous())
        # conv1 m = 0 output rows in the gate-paired order of the fused gate epilogue
        rows = gate_paired_rows(C).to(dev)
        self._register("W_conv1_m0", self.W1_m0.data[rows][:, block_permutation(LAYOUT1_PERM["m0"], C).to(dev)],
                       dtype)
        self.register_buffer("b_conv1_m0", _frozen(self.b1_m0.data[rows]).to(dtype))
        self._register_complex("W_conv1_m1", self.W1_m1_R.data[:, c_m1], self.W1_m1_I.data[:, c_m1], dtype)
        self._register_complex("W_conv1_m2", self.W1_m2_R.data, self.W1_m2_I.data, dtype)
        self.layout = 1
        self._register("W_conv2_m0", self.W2_m0.data, dtype)
        self.register_buffer("b_conv2_m0", _frozen(self.b2_m0.data).to(dtype))
        self._register_complex("W_conv2_m1", self.W2_m1_R.data, self.W2_m1_I.data, dtype)
        self._register_complex("W_conv2_m2", self.W2_m2_R.data, self.W2_m2_I.data, dtype)
        del self.W1_m0, self.b1_m0, self.W1_m1_R, self.W1_m1_I, self.W1_m2_R, self.W1_m2_I
        del self.W2_m0, self.b2_m0, self.W2_m1_R, self.W2_m1_I, self.W2_m2_R, self.W2_m2_I
        self.prepared = True

    def _prepare_reference_order(self, dtype):
        """lmax > 2: gather blocks in the reference's order extended by degree (ops/lmax.py);
        conv1 m = 0 rows gate-paired for the fused conv1 + gate + conv2."""
        for name in ("W_rad1_1", "W_rad1_2", "W_rad1_3"):
            W = getattr(self, name).data
            self.register_buffer(name + "_t", W.to(dtype).t().contiguous())
        # conv1 m = 0 output rows in the gate-paired order of the fused gate epilogue
        rows = gate_paired_rows(self.C, self.lmax).to(self.W1_m0.device)
        self._register("W_conv1_m0", self.W1_m0.data[rows], dtype)
        self.register_buffer("b_conv1_m0", _frozen(self.b1_m0.data[rows]).to(dtype))
        self._register_complex("W_conv1_m1", self.W1_m1_R.data, self.W1_m1_I.data, dtype)
        self._register_complex("W_conv1_m2", self.W1_m2_R.data, self.W1_m2_I.data, dtype)
        self._register("W_conv2_m0", self.W2_m0.data, dtype)
        self.register_buffer("b_conv2_m0", _frozen(self.b2_m0.data).to(dtype))
        self._register_complex("W_conv2_m1", self.W2_m1_R.data, self.W2_m1_I.data, dtype)
        self._register_complex("W_conv2_m2", self.W2_m2_R.data, self.W2_m2_I.data, dtype)
        del self.W1_m0, self.b1_m0, self.W1_m1_R, self.W1_m1_I, self.W1_m2_R, self.W1_m2_I
        del self.W2_m0, self.b2_m0, self.W2_m1_R, self.W2_m1_I, self.W2_m2_R, self.W2_m2_I
        self.layout = 0
        self.prepared = True

    def radial(self, x_edge_raw):
        h1 = layer_norm_silu(linear(x_edge_raw, self.W_rad1_1, self.b_rad1_1, self.W_rad1_1_t),
                             self.gamma_rad1_1, self.beta_rad1_1)
        h2 = layer_norm_silu(linear(h1, self.W_rad1_2, self.b_rad1_2, self.W_rad1_2_t),
                             self.gamma_rad1_2, self.beta_rad1_2)
        return linear(h2, self.W_rad1_3, self.b_rad1_3, self.W_rad1_3_t)

    def radial_mlp(self):
        """This block's radial-MLP parameters in RadialBank order."""
        return (self.W_rad1_1, self.b_rad1_1, self.gamma_rad1_1, self.beta_rad1_1, self.W_rad1_2, self.b_rad1_2,
                self.gamma_rad1_2, self.beta_rad1_2, self.W_rad1_3, self.b_rad1_3)

    def forward(self, x_in, x_edge_raw, wigner, env, idx_i, idx_j, row_ptr, col_idx, csd_emb, batch,
                topology=None, rad_out=None, wig_ext=None, rad_src=None, sink=None, gather_m0=False,
                before_ffn=None, rad_gather=None):
        """rad_out, when given, is this block's radial-MLP output (computed by the model's
        RadialBank); otherwise it is computed here from x_edge_raw (E, B+2C).  wig_ext: the
        degree-3/4 Wigner rows (ops/lmax.wigner_extend), needed for lmax > 2.  before_ffn: a
        callable run after the edge-wise part is queued, before the node-side block (the model
        queues the next block's radial output there, RadialOutputs.prelaunch).  rad_gather: a
        callable (x_norm, layout) -> (rad_out, [X_m0, X_m1, X_m2]) that makes this block's
        radial output and the gather's outputs in one kernel (RadialOutputs.get_with_gather),
        used instead of rad_out."""
        x_norm, x_skip = self._norm_skip(x_in)
        X_pre = None
        if rad_gather is not None:
            rad_out, X_pre = rad_gather(x_norm, self.layout)
        elif rad_out is None:
            rad_out = self.radial(x_edge_raw)
        # gather -> conv1 + gate -> conv2 as one node: the (E, 18C) gather output X never
        # outlives the block (model.py:150-154)
        sfx = ("_R", "_I", "_Rt", "_It_neg")
        c1 = [self.W_conv1_m0, self.b_conv1_m0, self.W_conv1_m0_t] + \
            [getattr(self, "W_conv1_m" + m + x) for m in "12" for x in sfx]
        c2 = [self.W_conv2_m0, self.b_conv2_m0, self.W_conv2_m0_t] + \
            [getattr(self, "W_conv2_m" + m + x) for m in "12" for x in sfx]
        Zo_m0, Zo_m1, Zo_m2 = edge_block(x_norm, wigner, wig_ext, rad_out, idx_i, idx_j, csd_emb, batch, topology,
                                         self.layout, self.lmax, c1, c2, self.C, self._complex_splits(x_norm.device),
                                         rad_src, sink, gather_m0, X_pre)
        del rad_out
        if self.lmax == 2:
            x_mid = rotate_scatter_split(Zo_m0, Zo_m1, Zo_m2, wigner, env, x_skip, idx_j, row_ptr, col_idx,
                                         x_skip.shape[0], sink)
        else:
            x_mid = rotate_scatter_lmax(Zo_m0, Zo_m1, Zo_m2, wigner, wig_ext, env, x_skip, idx_j, row_ptr, col_idx,
                                        x_skip.shape[0], self.lmax, sink)
        if before_ffn is not None:
            before_ffn()
        return self._ffn_residual(x_mid)

    def _norm_skip(self, x_in):
        """(norm_1(x_in), x_in): with this build's norm the second is a view whose gradient the
        norm's backward kernel adds (model.py:145 and the x_in skip of model.py:155)."""
        if hasattr(self.norm_1, "forward_with_residual"):
            return self.norm_1.forward_with_residual(x_in)
        return self.norm_1(x_in), x_in

    def _ffn_residual(self, x_mid):
        """atom_wise(norm_2(x_mid)) + x_mid (model.py:157); with this build's modules the skip
        is added in the atom-wise block's last GEMM and its gradient in norm_2's backward."""
        if hasattr(self.norm_2, "forward_with_residual") and hasattr(self.atom_wise, "forward_residual"):
            x_n2, skip = self.norm_2.forward_with_residual(x_mid)
            return self.atom_wise.forward_residual(x_n2, skip)
        return self.atom_wise(self.norm_2(x_mid)) + x_mid


class eSCN_Inference_Model(nn.Module):
    """eSCN-MD backbone forward (model.py:160-221)."""

    # From this many edges on, each block recomputes its radial-MLP output in the backward
    # instead of keeping it (about 100 KB per edge are held otherwise, e.g. 138 GiB at 1.5 M
    # edges; the recompute lowers that by ~22 KB per edge for ~5 % more step time).
    RAD_RECOMPUTE_MIN_EDGES = 1_000_000
    # The blocks' backward kernels add dE/dwigner, dE/dwig_ext and dE/denv into one buffer
    # each (ops/edge_grad.py); False returns per-block gradients for autograd to sum instead
    # (the same values up to the order of the fp32 additions).
    SUM_EDGE_GRADS_IN_PLACE = True
    # conv1 m = 0 gathers its operand in the GEMM loader (fu_gather_linear_gate; lmax 2, a
    # split matrix-core mode, with the bf16 split in both) instead of reading the gather's
    # X_m0.  Off by default: at bcc Fe the fused GEMM costs more than the gather traffic it
    # removes (each rotated element is produced once per 128-column tile of the 640 outputs).
    GATHER_IN_CONV1 = False
    # C = 128, split-fp16 mode: each block's radial output layer writes the gather's outputs
    # from its GEMM epilogue (fu_radial_gather_fwd, lmax 2; fu_radial_gather_fwd_lmax, lmax 3,
    # 4: the separate gather kernel and its read of the radial output are gone; X bitwise as
    # before).  False runs the output GEMM and the gather as two kernels (the output GEMM then
    # queued early on the side stream).
    RADIAL_GATHER = True

    def __init__(self, num_layers=4, sphere_channels=128, edge_channels=128, num_distance_basis=32, cutoff=5.0,
                 coeff_g=-0.5, lmax=2):
        super().__init__()
        self.C, self.cutoff, self.coeff_g, self.B = sphere_channels, cutoff, coeff_g, num_distance_basis
        self.lmax = lmax
        C, B = self.C, self.B
        self.W_sphere = nn.Parameter(torch.zeros(100, C))
        self.W_src = nn.Parameter(torch.zeros(100, C)); self.W_tgt = nn.Parameter(torch.zeros(100, C))
        self.offset_g = nn.Parameter(torch.linspace(0, cutoff, B))

        self.W_rad1_1 = nn.Parameter(torch.zeros(C, B + 2 * C)); self.b_rad1_1 = nn.Parameter(torch.zeros(C))
        self.gamma_rad1_1 = nn.Parameter(torch.ones(C)); self.beta_rad1_1 = nn.Parameter(torch.zeros(C))
        self.W_rad1_2 = nn.Parameter(torch.zeros(C, C)); self.b_rad1_2 = nn.Parameter(torch.zeros(C))
        self.gamma_rad1_2 = nn.Parameter(torch.ones(C)); self.beta_rad1_2 = nn.Parameter(torch.zeros(C))
        self.W_rad1_3 = nn.Parameter(torch.zeros((lmax + 1) * C, C))
        self.b_rad1_3 = nn.Parameter(torch.zeros((lmax + 1) * C))

        self.layers = nn.ModuleList([Packed_eSCN_Layer(C, B, lmax) for _ in range(num_layers)])
        self.final_norm = None
        self.charge_start = 0; self.charge_end = 0; self.spin_start = 0; self.spin_end = 0

    def prepare_for_inference(self, dtype=torch.float32):
        self.eval()
        for p in self.parameters():
            p.requires_grad = False
        if self.final_norm is not None:
            for p in self.final_norm.parameters():
                p.requires_grad = False
        for name in ("W_rad1_1", "W_rad1_2", "W_rad1_3"):
            self.register_buffer(name + "_t", getattr(self, name).data.to(dtype).t().contiguous())
        for layer in self.layers:
            layer.prepare_for_inference(dtype)
        mlps = [(self.W_rad1_1, self.b_rad1_1, self.gamma_rad1_1, self.beta_rad1_1, self.W_rad1_2, self.b_rad1_2,
                 self.gamma_rad1_2, self.beta_rad1_2, self.W_rad1_3, self.b_rad1_3)]
        mlps += [layer.radial_mlp() for layer in self.layers]
        self.radial_bank = RadialBank([tuple(t.data for t in m) for m in mlps], self.W_src.data, self.W_tgt.data,
                                      self.B, dtype=dtype)
        self.to(dtype)

    def radial(self, x_edge_raw):
        h1 = layer_norm_silu(linear(x_edge_raw, self.W_rad1_1, self.b_rad1_1, self.W_rad1_1_t),
                             self.gamma_rad1_1, self.beta_rad1_1)
        h2 = layer_norm_silu(linear(h1, self.W_rad1_2, self.b_rad1_2, self.W_rad1_2_t),
                             self.gamma_rad1_2, self.beta_rad1_2)
        return linear(h2, self.W_rad1_3, self.b_rad1_3, self.W_rad1_3_t)

    def _radial_gather(self, layer, k: int) -> bool:
        """Whether block `layer` (radial output k of the bank) makes its radial output and its
        gather's outputs in one kernel (RADIAL_GATHER)."""
        if not self.RADIAL_GATHER or (self.lmax == 2 and self.GATHER_IN_CONV1):
            return False
        layouts = (0, 1) if self.lmax == 2 else (0,)
        return layer.layout in layouts and self.radial_bank.gather_ok(k, self.lmax)

    def _radial_gather_next(self, k: int) -> bool:
        """The same for the block that reads radial output k (False past the last block)."""
        return 1 <= k <= len(self.layers) and self._radial_gather(self.layers[k - 1], k)

    def _check_atoms(self, Z, batch, n_systems: int) -> None:
        """Atomic numbers index the 100-row element tables and batch ids the per-system
        embedding inside the kernels, so both are range-checked on the host (once per pair
        of tensors: an MD loop passes the same ones every step).  The checked tensors are
        held, and matched by identity and in-place version, so a new tensor that reuses a
        freed address is checked again."""
        prev = getattr(self, "_checked_atoms", None)
        if (prev is not None and prev[0] is Z and prev[1] is batch
                and prev[2] == (Z._version, batch._version, n_systems)):
            return
        n_el = self.W_sphere.shape[0]
        if Z.numel():
            zlo, zhi = (int(v) for v in torch.aminmax(Z))
            blo, bhi = (int(v) for v in torch.aminmax(batch))
            if zlo < 0 or zhi >= n_el:
                raise ValueError(f"atomic numbers must lie in [0, {n_el}); got [{zlo}, {zhi}]")
            if blo < 0 or bhi >= n_systems:
                raise ValueError(f"batch ids must lie in [0, {n_systems}); got [{blo}, {bhi}]")
        self._checked_atoms = (Z, batch, (Z._version, batch._version, n_systems))

    def forward(self, pos, Z, batch, edge_index, shifts, csd_emb, charge=None, spin=None, natoms=None):
        self._check_atoms(Z, batch, csd_emb.shape[0])
        # 1. Topology (Morton order + receiver-sorted edges + both CSRs), cached per graph
        topo = get_topology(pos, batch, edge_index)
        pos_s = permute_rows(pos, topo.perm)
        Z_s = take(Z.contiguous(), topo.perm)
        batch_s = take(batch.contiguous(), topo.perm)
        shifts_s = permute_rows(shifts, topo.edge_perm)
        idx_i_s, idx_j_s = topo.idx_i, topo.idx_j
        row_ptr, col_idx = topo.recv_ptr, topo.recv_idx
        N = pos_s.shape[0]

        # 2. Per-edge geometry: Gaussians, Wigner blocks, envelope.  The element-embedding
        #    columns of x_edge_raw are folded into the radial bank's per-element tables.
        # Every block's backward adds its dE/dwigner and dE/denv into one accumulator each
        # (ops/edge_grad.py) instead of autograd summing per-block gradients with add kernels.
        sink = EdgeGradSink() if torch.is_grad_enabled() and self.SUM_EDGE_GRADS_IN_PLACE else None
        gauss, wigner, env = precompute_geometry(pos_s, Z_s, idx_i_s, idx_j_s, shifts_s, self.W_src, self.W_tgt,
                                                 self.offset_g, self.coeff_g, self.cutoff, topo, False, sink)
        # 3. Every radial MLP (edge-degree embedding + one per block) as one bank.  On large
        #    graphs the blocks keep each radial output's (E, C) source instead of the (E, 12C)
        #    output and recompute it in their backward (one GEMM per block, ~5 % of the step,
        #    for ~22 KB less per edge held through the step).
        #    Each block's output layer is made when the block runs (its GEMM queued on the
        #    side stream during the previous block's node-side work, ops/radial.RadialOutputs).
        recompute = idx_i_s.shape[0] >= self.RAD_RECOMPUTE_MIN_EDGES
        rads = self.radial_bank(gauss, Z_s, idx_i_s, idx_j_s, lazy=True)
        rad = rads.get(0)
        if not self._radial_gather_next(1):
            rads.prelaunch(1)
        # 4. Edge-degree embedding (lmax > 2: with the degree-3/4 Wigner rows)
        wig_ext = None
        if self.lmax == 2:
            x_node_s = init_node_scatter(rad, wigner, env, Z_s, batch_s, self.W_sphere, csd_emb, idx_j_s,
                                         row_ptr, col_idx, N, sink)
        else:
            wig_ext = wigner_extend(wigner, self.lmax, sink)
            x_node_s = init_node_scatter_lmax(rad, wigner, wig_ext, env, Z_s, batch_s, self.W_sphere, csd_emb,
                                              idx_j_s, row_ptr, col_idx, N, self.lmax, sink)
        del rad
        # 5. Message-passing blocks, each followed by the charge / spin channel balancing when
        #    the backbone reserves channels for them (model.py:213-216)
        balance = self.charge_end > self.charge_start or self.spin_end > self.spin_start
        sys_ptr = system_ptr(batch_s, csd_emb.shape[0]) if balance else None   # batch_s is sorted
        for k, layer in enumerate(self.layers):
            if self._radial_gather(layer, k + 1):
                rad, before = None, None
                rg = lambda xn, lay, n=k + 1: rads.get_with_gather(n, xn, idx_i_s, idx_j_s, wigner, csd_emb, batch_s,
                                                                  lay, self.lmax, wig_ext)
            else:
                rad, rg = rads.get(k + 1), None
                before = None if self._radial_gather_next(k + 2) else (lambda n=k + 2: rads.prelaunch(n))
            x_node_s = layer(x_node_s, None, wigner, env, idx_i_s, idx_j_s, row_ptr, col_idx, csd_emb,
                             batch_s, topo, rad_out=rad, wig_ext=wig_ext,
                             rad_src=rads.source(k + 1) if recompute else None, sink=sink,
                             gather_m0=self.GATHER_IN_CONV1, before_ffn=before, rad_gather=rg)
            del rad, rg
            if self.charge_end > self.charge_start:
                x_node_s = balance_channels_batched(x_node_s, charge, natoms, batch_s, self.charge_start,
                                                    self.charge_end, 0.0, sys_ptr)
            if self.spin_end > self.spin_start:
                x_node_s = balance_channels_batched(x_node_s, spin, natoms, batch_s, self.spin_start, self.spin_end,
                                                    1.0, sys_ptr)
        x_node_s = self.final_norm(x_node_s)
        # 6. Back to the input atom order
        return permute_rows(x_node_s, topo.inv_perm)
