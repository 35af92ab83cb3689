"""rotate_scatter_split and init_node_scatter (ops/scatter.py:295-527) on the gfx950
scatter kernels (fp64 CSR accumulation, no atomics)."""
from __future__ import annotations

import torch

from . import _lib, edge_grad
from .constants import INIT_RAD_MULT, Z_M0_MULT
from .edge_grad import ENV, WIGNER


class RotateScatterSplit(torch.autograd.Function):
    @staticmethod
    def forward(ctx, Z_m0, Z_m1, Z_m2, wigner, env, x_res, idx_j, row_ptr, col_idx, N, sink=None):
        Z_m0 = _lib.require(Z_m0, torch.float32, "Z_m0")
        Z_m1 = _lib.require(Z_m1, torch.float32, "Z_m1")
        Z_m2 = _lib.require(Z_m2, torch.float32, "Z_m2")
        wigner = _lib.require(wigner, torch.float32, "wigner")
        env = _lib.require(env, torch.float32, "env")
        x_res = _lib.require(x_res, torch.float32, "x_res")
        row_ptr = _lib.require(row_ptr, torch.int32, "row_ptr")
        col_idx = _lib.require(col_idx, torch.int32, "col_idx")
        E = Z_m0.shape[0]
        C = Z_m0.shape[1] // Z_M0_MULT
        x_out = torch.empty(N, 9, C, device=Z_m0.device, dtype=torch.float32)
        _lib.call("fu_scatter_fwd", row_ptr.data_ptr(), col_idx.data_ptr(), Z_m0.data_ptr(), Z_m1.data_ptr(),
                  Z_m2.data_ptr(), wigner.data_ptr(), env.data_ptr(), x_res.data_ptr(), x_out.data_ptr(), N, E, C,
                  _lib.stream_ptr(Z_m0.device))
        ctx.save_for_backward(Z_m0, Z_m1, Z_m2, wigner, env, _lib.require(idx_j, torch.int64, "idx_j"))
        ctx.C, ctx.N, ctx.sink = C, N, sink
        return x_out

    @staticmethod
    def backward(ctx, g_out):
        Z_m0, Z_m1, Z_m2, wigner, env, idx_j = ctx.saved_tensors
        E, C, N = Z_m0.shape[0], ctx.C, ctx.N
        g_out = g_out.contiguous()
        g_Z_m0 = torch.empty_like(Z_m0)
        g_Z_m1 = torch.empty_like(Z_m1)
        g_Z_m2 = torch.empty_like(Z_m2)
        # with a sink (the model's path) the Wigner and envelope gradients are added to its
        # accumulators and not returned
        bufs, acc = edge_grad.outputs(ctx.sink, {WIGNER: wigner, ENV: env})
        _lib.call("fu_scatter_bwd", g_out.data_ptr(), idx_j.data_ptr(), Z_m0.data_ptr(), Z_m1.data_ptr(),
                  Z_m2.data_ptr(), wigner.data_ptr(), env.data_ptr(), g_Z_m0.data_ptr(), g_Z_m1.data_ptr(),
                  g_Z_m2.data_ptr(), bufs[WIGNER].data_ptr(), bufs[ENV].data_ptr(), E, N, C, acc,
                  _lib.stream_ptr(g_out.device))
        g_wigner, g_env = (None, None) if ctx.sink is not None else (bufs[WIGNER], bufs[ENV])
        return g_Z_m0, g_Z_m1, g_Z_m2, g_wigner, g_env, g_out, None, None, None, None, None


rotate_scatter_split = RotateScatterSplit.apply


class InitNodeScatter(torch.autograd.Function):
    @staticmethod
    def forward(ctx, rad_out, wigner, env, Z, batch, W_sphere, csd_emb, idx_j, row_ptr, col_idx, N, sink=None):
        rad_out = _lib.require(rad_out, torch.float32, "rad_out")
        wigner = _lib.require(wigner, torch.float32, "wigner")
        env = _lib.require(env, torch.float32, "env")
        Z = _lib.require(Z, torch.int64, "Z")
        batch = _lib.require(batch, torch.int64, "batch")
        W_sphere = _lib.require(W_sphere, torch.float32, "W_sphere")
        csd_emb = _lib.require(csd_emb, torch.float32, "csd_emb")
        row_ptr = _lib.require(row_ptr, torch.int32, "row_ptr")
        col_idx = _lib.require(col_idx, torch.int32, "col_idx")
        E = rad_out.shape[0]
        C = rad_out.shape[1] // INIT_RAD_MULT
        x_out = torch.empty(N, 9, C, device=rad_out.device, dtype=torch.float32)
        _lib.call("fu_init_scatter_fwd", row_ptr.data_ptr(), col_idx.data_ptr(), rad_out.data_ptr(),
                  wigner.data_ptr(), env.data_ptr(), Z.data_ptr(), batch.data_ptr(), W_sphere.data_ptr(),
                  csd_emb.data_ptr(), x_out.data_ptr(), N, E, W_sphere.shape[0], csd_emb.shape[0], C,
                  _lib.stream_ptr(rad_out.device))
        ctx.save_for_backward(rad_out, wigner, env, _lib.require(idx_j, torch.int64, "idx_j"), Z, batch)
        ctx.C, ctx.N, ctx.sink = C, N, sink
        ctx.num_z, ctx.num_batches = W_sphere.shape[0], csd_emb.shape[0]
        return x_out

    @staticmethod
    def backward(ctx, g_out):
        rad_out, wigner, env, idx_j, Z, batch = ctx.saved_tensors
        E, C, N = rad_out.shape[0], ctx.C, ctx.N
        g_out = g_out.contiguous()
        g_rad = torch.empty_like(rad_out)
        bufs, acc = edge_grad.outputs(ctx.sink, {WIGNER: wigner, ENV: env})
        _lib.call("fu_init_scatter_bwd", g_out.data_ptr(), idx_j.data_ptr(), rad_out.data_ptr(), wigner.data_ptr(),
                  env.data_ptr(), g_rad.data_ptr(), bufs[WIGNER].data_ptr(), bufs[ENV].data_ptr(), E, N, C, acc,
                  _lib.stream_ptr(g_out.device))
        g_wigner, g_env = (None, None) if ctx.sink is not None else (bufs[WIGNER], bufs[ENV])
        g_W_sphere = g_csd = None
        if ctx.needs_input_grad[5] or ctx.needs_input_grad[6]:
            # parameter-side gradients (ops/scatter.py:519-523); not on the force path
            g_l0 = g_out[:, 0, :]
            if ctx.needs_input_grad[5]:
                g_W_sphere = torch.zeros(ctx.num_z, C, device=g_out.device).index_add_(0, Z, g_l0)
            if ctx.needs_input_grad[6]:
                g_csd = torch.zeros(ctx.num_batches, C, device=g_out.device).index_add_(0, batch, g_l0)
        return g_rad, g_wigner, g_env, None, None, g_W_sphere, g_csd, None, None, None, None, None


init_node_scatter = InitNodeScatter.apply
