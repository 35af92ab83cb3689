"""Dense layers on the gfx950 matrix cores (replaces torch F.linear at model.py:147-154,203-205).

y = x W^T + b.  Weights are frozen; the backward returns the input gradient
g_x = g_y W, computed by the same kernel against the pre-transposed weight W^T."""
from __future__ import annotations

import torch

from . import _lib


def gemm(x: torch.Tensor, W: torch.Tensor, bias: torch.Tensor | None = None,
         out: torch.Tensor | None = None, W2: torch.Tensor | None = None) -> torch.Tensor:
    """out[M, N] = x[M, K] @ W[N, K]^T (+ bias).  x may be a row-strided view.  W2: W pre-split by
    linear_weight_split, read instead of W where fu_linear can (split-fp16 mode, tall tiles)."""
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
              _lib.ptr(W2), _lib.stream_ptr(x.device))
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


def resident_ok(K: int) -> bool:
    """fu_linear_resident takes K in 16..128, a multiple of 16."""
    return 16 <= K <= 128 and K % 16 == 0


def linear_weight_split(W: torch.Tensor) -> torch.Tensor:
    """The frozen weight W (N, K) pre-split for fu_linear_resident: fp16 hi, lo and 2^11 lo
    planes of the columns at their exact power-of-two scales in MFMA-fragment order, the unscale
    factors and the window flags."""
    W = _lib.require(W, torch.float32, "W")
    N, K = W.shape
    nbytes = _lib.load().fu_linear_weight_split_bytes(N, K)
    if nbytes < 0:
        raise _lib.FlashUMAError(f"linear_weight_split: bad shape {(N, K)} (16 <= K <= 128, K % 16 == 0)")
    W2 = torch.empty(nbytes // 16, 4, device=W.device, dtype=torch.int32)
    _lib.call("fu_linear_weight_split", W.data_ptr(), W.stride(0), N, K, W2.data_ptr(), _lib.stream_ptr(W.device))
    return W2


def gemm_resident(x: torch.Tensor, W2: torch.Tensor, N: int, bias: torch.Tensor | None = None,
                  out: torch.Tensor | None = None) -> torch.Tensor:
    """out[M, N] = x[M, K] @ W^T (+ bias) for K <= 128 with W pre-split by linear_weight_split
    (fu_linear_resident: split-fp16 products, each workgroup's rows of x resident in LDS across
    all N).  x may be a row-strided view with 16-byte aligned rows."""
    M, K = x.shape
    if x.stride(-1) != 1 or x.stride(0) % 4 != 0 or x.data_ptr() % 16 != 0:
        x = x.contiguous()
    if out is None:
        out = torch.empty((M, N), device=x.device, dtype=torch.float32)
    _lib.call("fu_linear_resident", x.data_ptr(), x.stride(0), W2.data_ptr(), _lib.ptr(bias), out.data_ptr(),
              out.stride(0), M, N, K, _lib.stream_ptr(x.device))
    return out


def complex_weight_split(P: torch.Tensor, Q: torch.Tensor) -> torch.Tensor:
    """The frozen complex weight P + iQ (Nc, Kc each) pre-split for fu_complex_linear's W3
    argument: exact three-way bf16 splits of P, Q and P + Q in MFMA-fragment order, then their
    two-way fp16 splits with power-of-two column scales and the columns' unscale factors (one
    buffer for both split modes)."""
    P = _lib.require(P, torch.float32, "P")
    Q = _lib.require(Q, torch.float32, "Q")
    Nc, Kc = P.shape
    if Q.shape != P.shape:
        raise _lib.FlashUMAError(f"complex_weight_split: P {tuple(P.shape)} vs Q {tuple(Q.shape)}")
    nbytes = _lib.load().fu_complex_weight_split_bytes(Nc, Kc)
    if nbytes < 0:
        raise _lib.FlashUMAError(f"complex_weight_split: bad shape {(Nc, Kc)}")
    W3 = torch.empty(nbytes // 16, 4, device=P.device, dtype=torch.int32)
    _lib.call("fu_complex_weight_split", P.data_ptr(), Q.data_ptr(), P.stride(0), Nc, Kc, W3.data_ptr(),
              _lib.stream_ptr(P.device))
    return W3


def complex_gemm(x: torch.Tensor, P: torch.Tensor, Q: torch.Tensor, W3: torch.Tensor | None = None,
                 out: torch.Tensor | None = None) -> torch.Tensor:
    """[y_r | y_i] = complex product of x = [x_r | x_i] (M, 2 Kc) with (P + iQ)^T, P, Q (Nc, Kc):
    y_r = x_r P^T - x_i Q^T, y_i = x_r Q^T + x_i P^T (fu_complex_linear; W3 = complex_weight_split(P, Q)
    or None; out: an (M, 2 Nc) float32 array with unit column stride to write, or None)."""
    if x.stride(-1) != 1:
        x = x.contiguous()
    M = x.shape[0]
    Nc, Kc = P.shape
    if x.shape[1] != 2 * Kc or Q.shape != P.shape:
        raise _lib.FlashUMAError(f"complex_gemm: x {tuple(x.shape)} vs P {tuple(P.shape)}, Q {tuple(Q.shape)}")
    if out is not None and (out.shape != (M, 2 * Nc) or out.dtype != torch.float32 or out.stride(-1) != 1):
        raise _lib.FlashUMAError(f"complex_gemm: out {tuple(out.shape)} {out.dtype}, expected ({M}, {2 * Nc}) float32")
    y = torch.empty((M, 2 * Nc), device=x.device, dtype=torch.float32) if out is None else out
    _lib.call("fu_complex_linear", x.data_ptr(), x[:, Kc:].data_ptr(), x.stride(0), P.data_ptr(), Q.data_ptr(),
              P.stride(0), _lib.ptr(W3), y.data_ptr(), y[:, Nc:].data_ptr(), y.stride(0), M, Nc, Kc, _lib.stream_ptr(x.device))
    return y


class _ComplexLinearFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, P, Q, Pt, Qt_neg, W3, W3t):
        x = _lib.require(x, torch.float32, "x")
        ctx.save_for_backward(Pt, Qt_neg)
        ctx.W3t = W3t
        return complex_gemm(x, P, Q, W3)

    @staticmethod
    def backward(ctx, g_y):
        Pt, Qt_neg = ctx.saved_tensors
        return complex_gemm(g_y.contiguous(), Pt, Qt_neg, ctx.W3t), None, None, None, None, None, None


def complex_linear(x: torch.Tensor, P: torch.Tensor, Q: torch.Tensor, Pt: torch.Tensor,
                   Qt_neg: torch.Tensor, W3: torch.Tensor | None = None,
                   W3t: torch.Tensor | None = None) -> torch.Tensor:
    """Frozen complex layer: equals x @ [[P, -Q], [Q, P]]^T (the reference's packed SO(2)
    weight, model.py:108-138).  Pt = P^T and Qt_neg = -Q^T (contiguous) give the input
    gradient through the same kernel: g_x_r = g_r P + g_i Q, g_x_i = g_i P - g_r Q.  W3, W3t:
    optional complex_weight_split of (P, Q) and (Pt, Qt_neg)."""
    return _ComplexLinearFn.apply(x, P, Q, Pt, Qt_neg, W3, W3t)
