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


def _gather_conv1_gate_m0(ops, W0, b0, C, st):
    """fu_gather_linear_gate: (Y0, Z0) of conv1 m = 0 with X_m0 gathered in the GEMM loader
    from the gather operands (x, idx_i, idx_j, wigner, rad, csd, batch; layout 1, lmax 2)."""
    x, idx_i, idx_j, wigner, rad, csd, batch = ops
    E = idx_i.shape[0]
    Y0 = torch.empty(E, 5 * C, device=x.device, dtype=torch.float32)
    Z0 = torch.empty(E, 3 * C, device=x.device, dtype=torch.float32)
    _lib.call("fu_gather_linear_gate", x.data_ptr(), idx_i.data_ptr(), idx_j.data_ptr(), wigner.data_ptr(),
              rad.data_ptr(), csd.data_ptr(), batch.data_ptr(), W0.data_ptr(), W0.stride(0), _lib.ptr(b0),
              Y0.data_ptr(), Y0.stride(0), Z0.data_ptr(), Z0.stride(0), E, C, st)
    return Y0, Z0


def _conv1_gate_m0(X0, W0, b0, C, L, st, W2=None):
    """fu_linear_gate: Y0 (gate-paired pre-activations, kept for the backward) and Z0; W2: W0
    pre-split (linear_weight_split) or None."""
    E = X0.shape[0]
    Y0 = torch.empty(E, (2 * L + 1) * C, device=X0.device, dtype=torch.float32)
    Z0 = torch.empty(E, (L + 1) * C, device=X0.device, dtype=torch.float32)
    _lib.call("fu_linear_gate", X0.data_ptr(), X0.stride(0), W0.data_ptr(), W0.stride(0), _lib.ptr(b0),
              Y0.data_ptr(), Y0.stride(0), Z0.data_ptr(), Z0.stride(0), None, 0, E, C, W0.shape[1], L, _lib.ptr(W2),
              st)
    return Y0, Z0


def _conv1_gate_mc(X, P, Q, W3, Y0, s_off, C, Y, Z):
    """fu_complex_linear_gate for m = 1 (gates of degrees 1..L, s_off 0) or m = 2 (degrees
    2..L, s_off C) into Y, Z (E, 2 Nc), the sigmoids recomputed from the gate columns of Y0;
    on torch's current stream."""
    E = X.shape[0]
    Nc, Kc = P.shape
    _lib.call("fu_complex_linear_gate", X.data_ptr(), X[:, Kc:].data_ptr(), X.stride(0), P.data_ptr(),
              Q.data_ptr(), P.stride(0), _lib.ptr(W3), Y.data_ptr(), Y[:, Nc:].data_ptr(), Y.stride(0),
              Z.data_ptr(), Z[:, Nc:].data_ptr(), Z.stride(0), Y0.data_ptr(), Y0.stride(0), s_off, C, E, Nc,
              Kc, _lib.stream_ptr(X.device))


def _conv1_gate_m12(X1, X2, P1, Q1, P2, Q2, W3_1, W3_2, Y0, C):
    """Both complex conv1 GEMMs with their gates: (Y1, Z1, Y2, Z2)."""
    outs = []
    for X, P, Q, W3, s_off in ((X1, P1, Q1, W3_1, 0), (X2, P2, Q2, W3_2, C)):
        Y = torch.empty(X.shape[0], 2 * P.shape[0], device=X.device, dtype=torch.float32)
        Z = torch.empty_like(Y)
        _conv1_gate_mc(X, P, Q, W3, Y0, s_off, C, Y, Z)
        outs += [Y, Z]
    return tuple(outs)


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
        Y0, Z0 = _conv1_gate_m0(X0, W0, b0, C, L, st)
        sp = splits or (None,) * 4
        Y1, Z1, Y2, Z2 = _conv1_gate_m12(X1, X2, P1, Q1, P2, Q2, sp[0], sp[2], Y0, C)
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


def _conv2_gate_bwd_mc(gz, Rt, Itn, W3, F, Y0, s_off, C, gy, ps):
    """fu_complex_linear_gate_bwd of conv2 m = 1 (s_off 0) or m = 2 (s_off C): g_Y = g_Z s into
    gy (E, 2 Nc) and the per-degree gate sums into ps (E, Nc); on torch's current stream."""
    E = gz.shape[0]
    Nc, Kc = Rt.shape
    _lib.call("fu_complex_linear_gate_bwd", gz.data_ptr(), gz[:, Kc:].data_ptr(), gz.stride(0), Rt.data_ptr(),
              Itn.data_ptr(), Rt.stride(0), _lib.ptr(W3), gy.data_ptr(), gy[:, Nc:].data_ptr(), gy.stride(0),
              F.data_ptr(), F[:, Nc:].data_ptr(), F.stride(0), Y0.data_ptr(), Y0.stride(0), s_off, C,
              ps.data_ptr(), ps.stride(0), E, Nc, Kc, _lib.stream_ptr(gz.device))


def _splits12(splits):
    """The 12 pre-split weights of a conv pair: the complex W3 of conv1 m = 1, 2 and conv2
    m = 1, 2 with their transpose pairs, then linear_weight_split of W0, W0t, V0, V0t (None
    where absent)."""
    sp = tuple(splits) if splits else ()
    return sp + (None,) * (12 - len(sp))


def conv_pair_fwd(X: list, conv1, conv2, C: int, splits, m0=None):
    """conv1 + gate + conv2 of one block on X = [X_m0, X_m1, X_m2].  Each entry of X is set
    to None once its GEMM has read it, so a caller that hands over its only references
    frees the (E, 18C) gather output while the block runs.  m0: None, or conv1 m = 0's
    (Y0, Z0) computed already (X_m0 is then None).  Returns (Zo0, Zo1, Zo2) and the
    pre-activations (Y0, Y1, Y2) the backward needs.

    After conv1 m = 0 (whose gate columns the complex gate epilogues read), conv1 m = 1 and
    conv2 m = 1 run on the current stream while conv1 m = 2, conv2 m = 2 and conv2 m = 0 run
    on the device's side stream (_lib.side_stream; one stream when it is off): they are
    independent, and each kernel's tail overlaps the other stream's work."""
    W0, b0, W0t, P1, Q1, P1t, Q1tn, P2, Q2, P2t, Q2tn = conv1
    V0, c0, V0t, R1, I1, R1t, I1tn, R2, I2, R2t, I2tn = conv2
    dev = X[1].device
    L = _degrees(W0, C)
    sp = _splits12(splits)
    if m0 is None:
        Y0, Z0 = _conv1_gate_m0(_lib.require(X[0], torch.float32, "X_m0"), W0, b0, C, L, _lib.stream_ptr(dev),
                                sp[8])
    else:
        Y0, Z0 = m0
    X[0] = None
    X1, X2 = _lib.require(X[1], torch.float32, "X_m1"), _lib.require(X[2], torch.float32, "X_m2")
    X[1] = X[2] = None
    E = X1.shape[0]
    f = lambda n: torch.empty(E, n, device=dev, dtype=torch.float32)
    # the side stream's outputs, allocated on the current stream; its operands stay referenced
    # until the join
    Y2, Z2, Zo2, Zo0 = f(2 * P2.shape[0]), f(2 * P2.shape[0]), f(2 * R2.shape[0]), f(V0.shape[0])
    side = _lib.side_stream(dev)
    with _lib.on_side(side):
        _conv1_gate_mc(X2, P2, Q2, sp[2], Y0, C, C, Y2, Z2)
        complex_gemm(Z2, R2, I2, sp[6], out=Zo2)
        gemm(Z0, V0, c0, out=Zo0, W2=sp[10])
    Y1, Z1 = f(2 * P1.shape[0]), f(2 * P1.shape[0])
    _conv1_gate_mc(X1, P1, Q1, sp[0], Y0, 0, C, Y1, Z1)
    del X1
    Zo1 = complex_gemm(Z1, R1, I1, sp[4])
    del Z1
    _lib.join(side)
    del X2, Z2, Z0
    return (Zo0, Zo1, Zo2), (Y0, Y1, Y2)


def conv_pair_bwd(Y, conv1, conv2, C: int, splits, g: list):
    """Input gradient of conv_pair_fwd: g = [g_Zo0, g_Zo1, g_Zo2] -> (g_X0, g_X1, g_X2).  The
    gate backward runs in the conv2 input-gradient epilogues (the m = 1, 2 complex GEMMs write
    g_Y = g_Z s and their gate sums, then the m = 0 GEMM finishes the gate-paired g_Y_m0 with
    the gate gradients, s recomputed from Y0); g_Z is never stored.  The entries of g are
    released once read.  The m = 2 gate backward and the m = 1 conv1 input gradient run on the
    device's side stream beside the independent calls on the current stream (as in
    conv_pair_fwd)."""
    Y0, Y1, Y2 = Y
    W0, b0, W0t, P1, Q1, P1t, Q1tn, P2, Q2, P2t, Q2tn = conv1
    V0, c0, V0t, R1, I1, R1t, I1tn, R2, I2, R2t, I2tn = conv2
    L = _degrees(W0, C)
    E = Y0.shape[0]
    dev = Y0.device
    st = _lib.stream_ptr(dev)
    f = lambda *s: torch.empty(*s, device=dev, dtype=torch.float32)
    sp = _splits12(splits)
    g0 = torch.zeros(E, (L + 1) * C, device=dev) if g[0] is None else g[0].contiguous()
    g1 = torch.zeros(E, 2 * L * C, device=dev) if g[1] is None else g[1].contiguous()
    g2 = torch.zeros(E, 2 * (L - 1) * C, device=dev) if g[2] is None else g[2].contiguous()
    g[0] = g[1] = g[2] = None
    gy1, ps1 = f(E, 2 * R1t.shape[0]), f(E, R1t.shape[0])
    gy2, ps2 = f(E, 2 * R2t.shape[0]), f(E, R2t.shape[0])
    side = _lib.side_stream(dev)
    with _lib.on_side(side):
        _conv2_gate_bwd_mc(g2, R2t, I2tn, sp[7], Y2, Y0, C, C, gy2, ps2)
    _conv2_gate_bwd_mc(g1, R1t, I1tn, sp[5], Y1, Y0, 0, C, gy1, ps1)
    _lib.join(side)
    del g1, g2
    gy0 = f(E, (2 * L + 1) * C)
    _lib.call("fu_linear_gate_bwd", g0.data_ptr(), g0.stride(0), V0t.data_ptr(), V0t.stride(0), Y0.data_ptr(),
              Y0.stride(0), ps1.data_ptr(), ps1.stride(0), ps2.data_ptr(), ps2.stride(0),
              gy0.data_ptr(), gy0.stride(0), E, C, V0t.shape[1], L, _lib.ptr(sp[11]), st)
    # release each intermediate as soon as it is consumed: the backward of a block runs near
    # the step's memory peak (every earlier layer's saved tensors are still alive)
    del ps1, ps2, g0
    g_x1 = f(E, 2 * P1t.shape[0])
    with _lib.on_side(side):
        complex_gemm(gy1, P1t, Q1tn, sp[1], out=g_x1)
    g_x0 = gemm(gy0, W0t, W2=sp[9])
    del gy0
    g_x2 = complex_gemm(gy2, P2t, Q2tn, sp[3])
    del gy2
    _lib.join(side)
    del gy1
    return g_x0, g_x1, g_x2


class Conv1GateConv2(torch.autograd.Function):
    """The edge-wise SO(2) pair of a block (model.py:152-154): conv1 + gate as in Conv1Gate,
    then conv2 (m = 0 real with bias V0 / c0, m = 1, 2 complex R + iI); see conv_pair_fwd and
    conv_pair_bwd."""

    @staticmethod
    def forward(ctx, X0, X1, X2, W0, b0, W0t, P1, Q1, P1t, Q1tn, P2, Q2, P2t, Q2tn, V0, c0, V0t, R1, I1, R1t, I1tn, R2,
                I2, R2t, I2tn, C, splits):
        conv1 = (W0, b0, W0t, P1, Q1, P1t, Q1tn, P2, Q2, P2t, Q2tn)
        conv2 = (V0, c0, V0t, R1, I1, R1t, I1tn, R2, I2, R2t, I2tn)
        Zo, Y = conv_pair_fwd([X0, X1, X2], conv1, conv2, C, splits)
        ctx.save_for_backward(*Y)
        ctx.conv1, ctx.conv2, ctx.C, ctx.sp = conv1, conv2, C, splits
        return Zo

    @staticmethod
    def backward(ctx, g0, g1, g2):
        gx = conv_pair_bwd(ctx.saved_tensors, ctx.conv1, ctx.conv2, ctx.C, ctx.sp, [g0, g1, g2])
        return tuple(gx) + (None,) * 24


def conv1_gate_conv2(X0, X1, X2, conv1, conv2, C, splits=None):
    """conv1 = (W0, b0, W0t, P1, Q1, P1t, Q1tn, P2, Q2, P2t, Q2tn) as for conv1_gate; conv2 =
    (V0, c0, V0t, R1, I1, R1t, I1tn, R2, I2, R2t, I2tn) (m = 0 weight, bias and transpose; the
    complex m = 1, 2 weights with R^T and -I^T).  splits: None or the complex_weight_split of
    (P1, Q1), (P1t, Q1tn), (P2, Q2), (P2t, Q2tn), (R1, I1), (R1t, I1tn), (R2, I2), (R2t, I2tn).
    Returns Zout_m0, Zout_m1, Zout_m2."""
    return Conv1GateConv2.apply(X0, X1, X2, *conv1, *conv2, C, splits)


class EdgeBlock(torch.autograd.Function):
    """One block's edge-wise path as one autograd node: gather-rotate (ops/gather.py), conv1 +
    gate + conv2 (model.py:150-154).  The (E, 18C) gather output X lives only inside the
    forward (each part freed after its GEMM) and its gradient only inside the backward, which
    runs conv_pair_bwd and then the node-centric gather backward.  lmax = 2 (layout 0 or 1) or
    lmax = 3, 4 (reference block order with the degree-3/4 Wigner rows wig_ext).  gather_m0
    (lmax 2, layout 1, a split matrix-core mode): conv1 m = 0 gathers its operand in the GEMM
    loader (fu_gather_linear_gate, bf16 split) and the gather forms X_m1, X_m2 only."""

    @staticmethod
    def forward(ctx, x_in, wigner, wig_ext, rad_out, idx_i, idx_j, csd_emb, batch, topology, layout, lmax, conv1,
                conv2, C, splits, rad_src, sink=None, gather_m0=False, X_pre=None):
        from .gather import gather_fwd, gather_operands
        from .lmax import gather_lmax_fwd, gather_lmax_operands
        L = int(lmax)
        m0 = None
        if L == 2:
            ops = gather_operands(x_in, idx_i, idx_j, wigner, rad_out, csd_emb, batch)
            fuse = gather_m0 and X_pre is None and int(layout) == 1 and _lib.get_matmul_mode() != _lib.MATMUL_FP32
            if X_pre is not None:
                # take over the caller's references, so that each part is freed after its GEMM
                X = list(X_pre)
                X_pre.clear()
            else:
                X = list(gather_fwd(*ops, layout, skip_m0=fuse))
            if fuse:
                m0 = _gather_conv1_gate_m0(ops, conv1[0], conv1[1], C, _lib.stream_ptr(x_in.device))
        else:
            ops = gather_lmax_operands(x_in, idx_i, idx_j, wigner, wig_ext, rad_out, csd_emb, batch, L)
            if X_pre is not None:
                X = list(X_pre)
                X_pre.clear()
            else:
                X = list(gather_lmax_fwd(*ops, L, topology))
        Zo, Y = conv_pair_fwd(X, conv1, conv2, C, splits, m0)
        r = 4 if L == 2 else 5   # position of rad_out among the gather operands
        if rad_src is not None:
            # keep the (E, C) source of the radial output instead of the (E, 6 L C) output
            ops = ops[:r] + (rad_src[0],) + ops[r + 1:]
            ctx.rad_w = rad_src[1:]
        else:
            ctx.rad_w = None
        ctx.save_for_backward(*ops, *Y)
        ctx.n_ops, ctx.r, ctx.topology, ctx.layout, ctx.L = len(ops), r, topology, int(layout), L
        ctx.conv1, ctx.conv2, ctx.C, ctx.sp, ctx.sink = conv1, conv2, C, splits, sink
        return Zo

    @staticmethod
    def backward(ctx, g0, g1, g2):
        from .gather import gather_bwd
        from .lmax import gather_lmax_bwd
        from .radial import recompute_output
        saved = ctx.saved_tensors
        ops, Y = list(saved[:ctx.n_ops]), saved[ctx.n_ops:]
        if ctx.rad_w is not None:
            ops[ctx.r] = recompute_output((ops[ctx.r],) + tuple(ctx.rad_w))
        gz = [g0, g1, g2]
        gx = list(conv_pair_bwd(Y, ctx.conv1, ctx.conv2, ctx.C, ctx.sp, list(gz)))
        # The incoming gradients are the rotate-scatter backward's fresh g_Zout buffers, read
        # only by conv_pair_bwd above.  The autograd engine keeps its references until this
        # function returns, through the gather backward below, where the step's memory peaks;
        # their device memory is handed back now (queued after the kernels that read it).
        for t in gz:
            if t is not None and t.is_contiguous() and t._base is None:
                t.untyped_storage().resize_(0)
        del g0, g1, g2, gz
        if ctx.L == 2:
            g_x, g_w, g_rad = gather_bwd(*ops, ctx.topology, ctx.layout, *gx, sink=ctx.sink)
            g_ext = None
        else:
            g_x, g_w, g_ext, g_rad = gather_lmax_bwd(*ops, ctx.topology, ctx.L, *gx, sink=ctx.sink)
        return (g_x, g_w, g_ext, g_rad, None, None, None, None, None, None, None, None, None, None, None, None,
                None, None, None)


def edge_block(x_in, wigner, wig_ext, rad_out, idx_i, idx_j, csd_emb, batch, topology, layout, lmax, conv1, conv2, C,
               splits=None, rad_src=None, sink=None, gather_m0=False, X_pre=None):
    """gather_wigner_split (or gather_rotate_lmax) followed by conv1_gate_conv2, as one node
    whose gather output never outlives the block: returns (Zout_m0, Zout_m1, Zout_m2).
    rad_src: None, or the radial bank's (h2_k, W3_k, b3_k) source of rad_out; the backward
    then recomputes rad_out from it instead of keeping it (memory for one extra GEMM).
    sink: accumulators of the Wigner-row gradients (ops/edge_grad.py) or None.  gather_m0: conv1
    m = 0 gathers its own operand (see EdgeBlock).  X_pre: a list of the gather's
    [X_m0, X_m1, X_m2] already formed from these operands (ops/radial.RadialOutputs.
    get_with_gather), emptied here; the forward then skips the gather kernel, the backward is the
    same."""
    return EdgeBlock.apply(x_in, wigner, wig_ext, rad_out, idx_i, idx_j, csd_emb, batch, topology, layout, lmax,
                           tuple(conv1), tuple(conv2), C, splits, rad_src, sink, gather_m0, X_pre)
