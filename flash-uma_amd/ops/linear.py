"""Dense layers on the gfx950 fp32 MFMA GEMM (replaces torch F.linear at model.py:147-154,203-205).

y = x W^T + b.  Weights are frozen; the backward returns the input gradient
g_x = g_y W, computed by the same kernel against the pre-transposed weight W^T."""
from __future__ import annotations

import torch

from . import _lib


def gemm(x: torch.Tensor, W: torch.Tensor, bias: torch.Tensor | None = None,
         out: torch.Tensor | None = None) -> torch.Tensor:
    """out[M, N] = x[M, K] @ W[N, K]^T (+ bias).  x may be a row-strided view."""
    if x.stride(-1) != 1:
        x = x.contiguous()
    M, K = x.shape
    N = W.shape[0]
    if W.shape[1] != K:
        raise _lib.FlashUMAError(f"gemm: x has K={K} but W is {tuple(W.shape)}")
    if out is None:
        out = torch.empty((M, N), device=x.device, dtype=torch.float32)
    _lib.call("fu_linear", x.data_ptr(), x.stride(0), W.data_ptr(), W.stride(0),
              None if bias is None else bias.data_ptr(), out.data_ptr(), out.stride(0), M, N, K,
              _lib.stream_ptr(x.device))
    return out


class _LinearFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, W, bias, Wt):
        x = _lib.require(x, torch.float32, "x")
        ctx.save_for_backward(Wt)
        return gemm(x, W, bias)

    @staticmethod
    def backward(ctx, g_y):
        (Wt,) = ctx.saved_tensors
        return gemm(g_y.contiguous(), Wt), None, None, None


def linear(x: torch.Tensor, W: torch.Tensor, bias: torch.Tensor | None, Wt: torch.Tensor) -> torch.Tensor:
    """x W^T + b with a frozen weight; Wt must be W.t().contiguous()."""
    return _LinearFn.apply(x, W, bias, Wt)
