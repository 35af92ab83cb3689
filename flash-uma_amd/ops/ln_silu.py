"""layer_norm_silu (ops/ln_silu.py:126-185) on the gfx950 row kernels.

gamma and beta are frozen (inference): the backward returns the input gradient only."""
from __future__ import annotations

import torch

from . import _lib
from .constants import LN_EPS


class _LayerNormSiLUFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, gamma, beta, eps):
        x = _lib.require(x, torch.float32, "x")
        gamma = _lib.require(gamma, torch.float32, "gamma")
        beta = _lib.require(beta, torch.float32, "beta")
        M, D = x.shape
        out = torch.empty_like(x)
        mean = torch.empty(M, device=x.device, dtype=torch.float32)
        rstd = torch.empty(M, device=x.device, dtype=torch.float32)
        _lib.call("fu_ln_silu_fwd", x.data_ptr(), gamma.data_ptr(), beta.data_ptr(), out.data_ptr(),
                  mean.data_ptr(), rstd.data_ptr(), M, D, float(eps), _lib.stream_ptr(x.device))
        ctx.save_for_backward(x, gamma, beta, mean, rstd)
        return out

    @staticmethod
    def backward(ctx, g_out):
        x, gamma, beta, mean, rstd = ctx.saved_tensors
        M, D = x.shape
        g_out = g_out.contiguous()
        g_x = torch.empty_like(x)
        _lib.call("fu_ln_silu_bwd", x.data_ptr(), gamma.data_ptr(), beta.data_ptr(), mean.data_ptr(),
                  rstd.data_ptr(), g_out.data_ptr(), g_x.data_ptr(), M, D, _lib.stream_ptr(x.device))
        return g_x, None, None, None


def layer_norm_silu(x, gamma, beta, eps=LN_EPS):
    """Fused LayerNorm + SiLU over rows of x (M, D)."""
    return _LayerNormSiLUFn.apply(x, gamma, beta, eps)
