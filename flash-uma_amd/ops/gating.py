"""fused_gating_split (ops/gating.py:188-236) on the gfx950 gate kernels."""
from __future__ import annotations

import torch

from . import _lib
from .constants import Z_M0_MULT, Z_M1_MULT, Z_M2_MULT


class FusedGatingSplit(torch.autograd.Function):
    @staticmethod
    def forward(ctx, Y_m0, Y_m1, Y_m2, C):
        Y_m0 = _lib.require(Y_m0, torch.float32, "Y_m0")
        Y_m1 = _lib.require(Y_m1, torch.float32, "Y_m1")
        Y_m2 = _lib.require(Y_m2, torch.float32, "Y_m2")
        E = Y_m0.shape[0]
        dev = Y_m0.device
        Z_m0 = torch.empty((E, Z_M0_MULT * C), device=dev, dtype=torch.float32)
        Z_m1 = torch.empty((E, Z_M1_MULT * C), device=dev, dtype=torch.float32)
        Z_m2 = torch.empty((E, Z_M2_MULT * C), device=dev, dtype=torch.float32)
        _lib.call("fu_gating_fwd", Y_m0.data_ptr(), Y_m1.data_ptr(), Y_m2.data_ptr(), Z_m0.data_ptr(),
                  Z_m1.data_ptr(), Z_m2.data_ptr(), E, C, _lib.stream_ptr(dev))
        ctx.save_for_backward(Y_m0, Y_m1, Y_m2)
        ctx.C = C
        return Z_m0, Z_m1, Z_m2

    @staticmethod
    def backward(ctx, g_z_m0, g_z_m1, g_z_m2):
        Y_m0, Y_m1, Y_m2 = ctx.saved_tensors
        E, C = Y_m0.shape[0], ctx.C
        g_z_m0 = torch.zeros_like(Y_m0[:, : 3 * C]) if g_z_m0 is None else g_z_m0.contiguous()
        g_z_m1 = torch.zeros_like(Y_m1) if g_z_m1 is None else g_z_m1.contiguous()
        g_z_m2 = torch.zeros_like(Y_m2) if g_z_m2 is None else g_z_m2.contiguous()
        g_y_m0 = torch.empty_like(Y_m0)
        g_y_m1 = torch.empty_like(Y_m1)
        g_y_m2 = torch.empty_like(Y_m2)
        _lib.call("fu_gating_bwd", g_z_m0.data_ptr(), g_z_m1.data_ptr(), g_z_m2.data_ptr(), Y_m0.data_ptr(),
                  Y_m1.data_ptr(), Y_m2.data_ptr(), g_y_m0.data_ptr(), g_y_m1.data_ptr(), g_y_m2.data_ptr(), E, C,
                  _lib.stream_ptr(Y_m0.device))
        return g_y_m0, g_y_m1, g_y_m2, None


fused_gating_split = FusedGatingSplit.apply
