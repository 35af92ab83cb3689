"""fused_gating_split (ops/gating.py:188-236) on the gfx950 gate kernels, and conv1_gate:
the SO(2) conv1 of a block (model.py:152) with the gate activation (model.py:153) in the
GEMM epilogues, so the gated features are written once and the gating pass over Y is gone.

layout 1 of Y_m0 is the gate-paired column order (gate_paired_rows): 64-column pairs
[32 gate_l channels | the 32 y_lm0 channels they gate] for l = 1..lmax, then y_l0; the
conv1 m = 0 weight rows are permuted to it at freeze time.  conv1_gate_conv2 handles lmax
2, 3 and 4 (the degree count is read from the conv1 m = 0 weight)."""
from __future__ import annotations

import torch

from . import _lib
from .constants import Z_M0_MULT, Z_M1_MULT, Z_M2_MULT
from .linear import complex_gemm, gemm


def gate_paired_rows(C: int, lmax: int = 2) -> torch.Tensor:
    """Reference column of Y_m0 (= [gate_1 .. gate_L, y_0, y_1m0 .. y_Lm0], C each, L = lmax)
    for each column of the gate-paired order: 64-column pairs [gate_l | y_lm0] x C/32 for
    l = 1..L, then y_0."""
    L, n1 = lmax, C // 32
    cols = []
    for p in range((2 * L + 1) * C // 64):
        for h in range(2):
            for c in range(32):
                if p < L * n1:
                    l, q = p // n1 + 1, p % n1
                    cols.append(((l - 1) * C if h == 0 else (L + l) * C) + 32 * q + c)
                else:
                    cols.append(L * C + 64 * (p - L * n1) + 32 * h + c)
    return torch.tensor(cols, dtype=torch.long)


def _degrees(W0: torch.Tensor, C: int) -> int:
    """lmax from the conv1 m = 0 weight ((2 lmax + 1) C rows)."""
    return (W0.shape[0] // C - 1) // 2


class FusedGatingSplit(torch.autograd.Function):
    @staticmethod
    def forward(ctx, Y_m0, Y_m1, Y_m2, C, layout=0):
        Y_m0 = _lib.require(Y_m0, torch.float32, "Y_m0")
        Y_m1 = _lib.require(Y_m1, torch.float32, "Y_m1")
        Y_m2 = _lib.require(Y_m2, torch.float32, "Y_m2")
        E = Y_m0.shape[0]
        dev = Y_m0.device
        Z_m0 = torch.empty((E, Z_M0_MULT * C), device=dev, dtype=torch.float32)
        Z_m1 = torch.empty((E, Z_M1_MULT * C), device=dev, dtype=torch.float32)
        Z_m2 = torch.empty((E, Z_M2_MULT * C), device=dev, dtype=torch.float32)
        _lib.call("fu_gating_fwd", Y_m0.data_ptr(), Y_m1.data_ptr(), Y_m2.data_ptr(), Z_m0.data_ptr(),
                  Z_m1.data_ptr(), Z_m2.data_ptr(), E, C, int(layout), _lib.stream_ptr(dev))
        ctx.save_for_backward(Y_m0, Y_m1, Y_m2)
        ctx.C, ctx.layout = C, int(layout)
        return Z_m0, Z_m1, Z_m2

    @staticmethod
    def backward(ctx, g_z_m0, g_z_m1, g_z_m2):
        Y_m0, Y_m1, Y_m2 = ctx.saved_tensors
        return _gating_bwd(Y_m0, Y_m1, Y_m2, g_z_m0, g_z_m1, g_z_m2, ctx.C, ctx.layout) + (None, None)


def _gating_bwd(Y_m0, Y_m1, Y_m2, g_z_m0, g_z_m1, g_z_m2, C, layout):
    E = Y_m0.shape[0]
    g_z_m0 = torch.zeros(E, 3 * C, device=Y_m0.device) if g_z_m0 is None else g_z_m0.contiguous()
    g_z_m1 = torch.zeros_like(Y_m1) if g_z_m1 is None else g_z_m1.contiguous()
    g_z_m2 = torch.zeros_like(Y_m2) if g_z_m2 is None else g_z_m2.contiguous()
    g_y_m0 = torch.empty_like(Y_m0)
    g_y_m1 = torch.empty_like(Y_m1)
    g_y_m2 = torch.empty_like(Y_m2)
    _lib.call("fu_gating_bwd", g_z_m0.data_ptr(), g_z_m1.data_ptr(), g_z_m2.data_ptr(), Y_m0.data_ptr(),
              Y_m1.data_ptr(), Y_m2.data_ptr(), g_y_m0.data_ptr(), g_y_m1.data_ptr(), g_y_m2.data_ptr(), E, C,
              int(layout), _lib.stream_ptr(Y_m0.device))
    return g_y_m0, g_y_m1, g_y_m2


def fused_gating_split(Y_m0, Y_m1, Y_m2, C, layout=0):
    return FusedGatingSplit.apply(Y_m0, Y_m1, Y_m2, C, layout)


class Conv1Gate(torch.autograd.Function):
    """X_m0, X_m1, X_m2 -> Z_m0, Z_m1, Z_m2: conv1 m = 0 (W0 rows and b0 in the gate-paired
    order, W0t = W0^T) and the complex m = 1, 2 layers (P + iQ, with Pt = P^T, Qtn = -Q^T for
    the input gradient), gated in their epilogues.  Saves Y (pre-activation) for the gate
    backward, which runs as the separate kernel before the input-gradient GEMMs."""

    @staticmethod
    def forward(ctx, X0, X1, X2, W0, b0, W0t, P1, Q1, P1t, Q1tn, P2, Q2, P2t, Q2tn, C, splits):
        X0 = _lib.require(X0, torch.float32, "X_m0")
        X1 = _lib.require(X1, torch.float32, "X_m1")
        X2 = _lib.require(X2, torch.float32, "X_m2")
        E = X0.shape[0]
        dev = X0.device
        st = _lib.stream_ptr(dev)
        f = lambda *s: torch.empty(*s, device=dev, dtype=torch.float32)
        L = _degrees(W0, C)
        Y0, Z0, S = f(E, (2 * L + 1) * C), f(E, (L + 1) * C), f(E, L * C)
        _lib.call("fu_linear_gate", X0.data_ptr(), X0.stride(0), W0.data_ptr(), W0.stride(0), _lib.ptr(b0),
                  Y0.data_ptr(), Y0.stride(0), Z0.data_ptr(), Z0.stride(0), S.data_ptr(), S.stride(0), E, C,
                  W0.shape[1], L, st)
        sp = splits or (None,) * 4
        outs = []
        for X, P, Q, W3, s_off in ((X1, P1, Q1, sp[0], 0), (X2, P2, Q2, sp[2], C)):
            Nc, Kc = P.shape
            Y, Z = f(E, 2 * Nc), f(E, 2 * Nc)
            _lib.call("fu_complex_linear_gate", X.data_ptr(), X[:, Kc:].data_ptr(), X.stride(0), P.data_ptr(),
                      Q.data_ptr(), P.stride(0), _lib.ptr(W3), Y.data_ptr(), Y[:, Nc:].data_ptr(), Y.stride(0),
                      Z.data_ptr(), Z[:, Nc:].data_ptr(), Z.stride(0), S.data_ptr(), S.stride(0), s_off, E, Nc, Kc,
                      st)
            outs += [Y, Z]
        Y1, Z1, Y2, Z2 = outs
        if L != 2:
            raise _lib.FlashUMAError("conv1_gate: lmax 2 only (use conv1_gate_conv2 for lmax 3, 4)")
        ctx.save_for_backward(Y0, Y1, Y2, W0t, P1t, Q1tn, P2t, Q2tn)
        ctx.C, ctx.sp = C, sp
        return Z0, Z1, Z2

    @staticmethod
    def backward(ctx, g_z0, g_z1, g_z2):
        Y0, Y1, Y2, W0t, P1t, Q1tn, P2t, Q2tn = ctx.saved_tensors
        sp = ctx.sp
        g_y0, g_y1, g_y2 = _gating_bwd(Y0, Y1, Y2, g_z0, g_z1, g_z2, ctx.C, 1)
        return ((gemm(g_y0, W0t), complex_gemm(g_y1, P1t, Q1tn, sp[1]), complex_gemm(g_y2, P2t, Q2tn, sp[3])) +
                (None,) * 13)


def conv1_gate(X0, X1, X2, W0, b0, W0t, P1, Q1, P1t, Q1tn, P2, Q2, P2t, Q2tn, C, splits=None):
    """splits: None or complex_weight_split of (P1, Q1), (P1t, Q1tn), (P2, Q2), (P2t, Q2tn)."""
    return Conv1Gate.apply(X0, X1, X2, W0, b0, W0t, P1, Q1, P1t, Q1tn, P2, Q2, P2t, Q2tn, C, splits)


class Conv1GateConv2(torch.autograd.Function):
    """The edge-wise SO(2) pair of a block (model.py:152-154): conv1 + gate as in Conv1Gate,
    then conv2 (m = 0 real with bias V0 / c0, m = 1, 2 complex R + iI).  Its backward fuses the
    gate backward into the conv2 input-gradient epilogues: the m = 1, 2 complex GEMMs write
    g_Y = g_Z s and their gate sums, then the m = 0 GEMM finishes g_Y_m0 (gate-paired) with
    the gate gradients; g_Z is never stored and no separate gating pass runs."""

    @staticmethod
    def forward(ctx, X0, X1, X2, W0, b0, W0t, P1, Q1, P1t, Q1tn, P2, Q2, P2t, Q2tn, V0, c0, V0t, R1, I1, R1t, I1tn, R2,
                I2, R2t, I2tn, C, splits):
        X0 = _lib.require(X0, torch.float32, "X_m0")
        X1 = _lib.require(X1, torch.float32, "X_m1")
        X2 = _lib.require(X2, torch.float32, "X_m2")
        E = X0.shape[0]
        dev = X0.device
        st = _lib.stream_ptr(dev)
        f = lambda *s: torch.empty(*s, device=dev, dtype=torch.float32)
        L = _degrees(W0, C)
        Y0, Z0, S = f(E, (2 * L + 1) * C), f(E, (L + 1) * C), f(E, L * C)
        _lib.call("fu_linear_gate", X0.data_ptr(), X0.stride(0), W0.data_ptr(), W0.stride(0), _lib.ptr(b0),
                  Y0.data_ptr(), Y0.stride(0), Z0.data_ptr(), Z0.stride(0), S.data_ptr(), S.stride(0), E, C,
                  W0.shape[1], L, st)
        sp = splits or (None,) * 8
        outs = []
        for X, P, Q, W3, s_off in ((X1, P1, Q1, sp[0], 0), (X2, P2, Q2, sp[2], C)):
            Nc, Kc = P.shape
            Y, Z = f(E, 2 * Nc), f(E, 2 * Nc)
            _lib.call("fu_complex_linear_gate", X.data_ptr(), X[:, Kc:].data_ptr(), X.stride(0), P.data_ptr(),
                      Q.data_ptr(), P.stride(0), _lib.ptr(W3), Y.data_ptr(), Y[:, Nc:].data_ptr(), Y.stride(0),
                      Z.data_ptr(), Z[:, Nc:].data_ptr(), Z.stride(0), S.data_ptr(), S.stride(0), s_off, E, Nc, Kc,
                      st)
            outs += [Y, Z]
        Y1, Z1, Y2, Z2 = outs
        Zo0 = gemm(Z0, V0, c0)
        Zo1 = complex_gemm(Z1, R1, I1, sp[4])
        Zo2 = complex_gemm(Z2, R2, I2, sp[6])
        ctx.save_for_backward(Y0, Y1, Y2, S, W0t, P1t, Q1tn, P2t, Q2tn, V0t, R1t, I1tn, R2t, I2tn)
        ctx.C, ctx.L, ctx.sp = C, L, sp
        return Zo0, Zo1, Zo2

    @staticmethod
    def backward(ctx, g0, g1, g2):
        Y0, Y1, Y2, S, W0t, P1t, Q1tn, P2t, Q2tn, V0t, R1t, I1tn, R2t, I2tn = ctx.saved_tensors
        C, L = ctx.C, ctx.L
        E = Y0.shape[0]
        dev = Y0.device
        st = _lib.stream_ptr(dev)
        f = lambda *s: torch.empty(*s, device=dev, dtype=torch.float32)
        g0 = torch.zeros(E, (L + 1) * C, device=dev) if g0 is None else g0.contiguous()
        g1 = torch.zeros(E, 2 * L * C, device=dev) if g1 is None else g1.contiguous()
        g2 = torch.zeros(E, 2 * (L - 1) * C, device=dev) if g2 is None else g2.contiguous()
        sp = ctx.sp
        gys, psums = [], []
        for g, Rt, Itn, W3, F, s_off in ((g1, R1t, I1tn, sp[5], Y1, 0), (g2, R2t, I2tn, sp[7], Y2, C)):
            Nc, Kc = Rt.shape
            gy, ps = f(E, 2 * Nc), f(E, Nc)
            _lib.call("fu_complex_linear_gate_bwd", g.data_ptr(), g[:, Kc:].data_ptr(), g.stride(0), Rt.data_ptr(),
                      Itn.data_ptr(), Rt.stride(0), _lib.ptr(W3), gy.data_ptr(), gy[:, Nc:].data_ptr(),
                      gy.stride(0), F.data_ptr(), F[:, Nc:].data_ptr(), F.stride(0), S.data_ptr(), S.stride(0),
                      s_off, ps.data_ptr(), ps.stride(0), E, Nc, Kc, st)
            gys.append(gy)
            psums.append(ps)
        gy0 = f(E, (2 * L + 1) * C)
        _lib.call("fu_linear_gate_bwd", g0.data_ptr(), g0.stride(0), V0t.data_ptr(), V0t.stride(0), Y0.data_ptr(),
                  Y0.stride(0), S.data_ptr(), S.stride(0), psums[0].data_ptr(), psums[0].stride(0),
                  psums[1].data_ptr(), psums[1].stride(0), gy0.data_ptr(), gy0.stride(0), E, C, V0t.shape[1], L,
                  st)
        return ((gemm(gy0, W0t), complex_gemm(gys[0], P1t, Q1tn, sp[1]), complex_gemm(gys[1], P2t, Q2tn, sp[3])) +
                (None,) * 24)


def conv1_gate_conv2(X0, X1, X2, conv1, conv2, C, splits=None):
    """conv1 = (W0, b0, W0t, P1, Q1, P1t, Q1tn, P2, Q2, P2t, Q2tn) as for conv1_gate; conv2 =
    (V0, c0, V0t, R1, I1, R1t, I1tn, R2, I2, R2t, I2tn) (m = 0 weight, bias and transpose; the
    complex m = 1, 2 weights with R^T and -I^T).  splits: None or the complex_weight_split of
    (P1, Q1), (P1t, Q1tn), (P2, Q2), (P2t, Q2tn), (R1, I1), (R1t, I1tn), (R2, I2), (R2t, I2tn).
    Returns Zout_m0, Zout_m1, Zout_m2."""
    return Conv1GateConv2.apply(X0, X1, X2, *conv1, *conv2, C, splits)
