"""Edge ops for lmax = 3 or 4 (mmax = 2) on the gfx950 kernels of csrc/edge_lmax.hip and
csrc/wigner_hi.hip.

The reference supports lmax = 2 only (wrapper.py:105-118); these autograd functions extend
its ops degree by degree with the same meaning and the reference's column-block order
continued over the degrees (the lmax = 2 calls of the same functions reproduce
gather_wigner_split / fused_gating_split / rotate_scatter_split / init_node_scatter with
layout 0 exactly in shape and order):

  wigner_extend(wigner, lmax)                -> wig_ext (E, 35 | 80): rows m = -2..2 of D^3, D^4
  gather_rotate_lmax(x, ..., wig_ext, ...)   -> X_m0 (E, 2(L+1)C), X_m1 (E, 4LC), X_m2 (E, 4(L-1)C)
  gating_lmax(Y_m0, Y_m1, Y_m2, C, lmax)     -> Z_m0 (E, (L+1)C), Z_m1 (E, 2LC), Z_m2 (E, 2(L-1)C)
  rotate_scatter_lmax(Z..., wig_ext, ...)    -> x_out (N, (L+1)^2, C)
  init_node_scatter_lmax(rad (E, (L+1)C), ...) -> x0 (N, (L+1)^2, C)
"""
from __future__ import annotations

import torch

from . import _lib, edge_grad
from .edge_grad import ENV, WIG_EXT, WIGNER
from .topology import receiver_csr, sender_csr


def ext_width(lmax: int) -> int:
    return {2: 0, 3: 35, 4: 80}[int(lmax)]


def _ext_ptr(t):
    return 0 if t is None or t.numel() == 0 else t.data_ptr()


class WignerExtend(torch.autograd.Function):
    @staticmethod
    def forward(ctx, wigner, lmax, sink=None):
        wigner = _lib.require(wigner, torch.float32, "wigner")
        E = wigner.shape[0]
        ext = torch.empty(E, ext_width(lmax), device=wigner.device, dtype=torch.float32)
        _lib.call("fu_wigner_ext_fwd", wigner.data_ptr(), ext.data_ptr(), E, int(lmax), _lib.stream_ptr(wigner.device))
        ctx.save_for_backward(wigner)
        ctx.lmax, ctx.sink = int(lmax), sink
        ctx.set_materialize_grads(False)   # g_ext stays None when every reader used the sink
        return ext

    @staticmethod
    def backward(ctx, g_ext):
        (wigner,) = ctx.saved_tensors
        g_ext = edge_grad.merge(ctx.sink, WIG_EXT, g_ext)
        if g_ext is None:
            return None, None, None
        E = wigner.shape[0]
        g_w = torch.empty_like(wigner)
        _lib.call("fu_wigner_ext_bwd", wigner.data_ptr(), g_ext.contiguous().data_ptr(), g_w.data_ptr(), E, ctx.lmax,
                  _lib.stream_ptr(wigner.device))
        return g_w, None, None


def wigner_extend(wigner, lmax: int, sink=None):
    return WignerExtend.apply(wigner, int(lmax), sink)


def _csrs(topology, idx_i, idx_j, N, E):
    if topology is not None and topology.E == E and topology.N == N:
        return topology.recv_ptr, topology.recv_idx, topology.send_ptr, topology.send_idx
    rptr, ridx = receiver_csr(idx_j, N)
    sptr, sidx = sender_csr(idx_i, N)
    return rptr, ridx, sptr, sidx


def gather_lmax_operands(x_in, idx_i, idx_j, wigner, wig_ext, rad_out, csd_emb, batch, L):
    ops = (_lib.require(x_in, torch.float32, "x_in"), _lib.require(idx_i, torch.int64, "idx_i"),
           _lib.require(idx_j, torch.int64, "idx_j"), _lib.require(wigner, torch.float32, "wigner"),
           _lib.require(wig_ext, torch.float32, "wig_ext"), _lib.require(rad_out, torch.float32, "rad_out"),
           _lib.require(csd_emb, torch.float32, "csd_emb"), _lib.require(batch, torch.int64, "batch"))
    N, K, C = ops[0].shape
    E = ops[1].shape[0]
    if K != (L + 1) ** 2 or ops[5].shape != (E, 6 * L * C) or ops[4].shape != (E, ext_width(L)):
        raise _lib.FlashUMAError(f"gather_rotate_lmax: shapes do not match lmax={L}")
    return ops


def radial_gather_lmax_perm(C: int, L: int) -> torch.Tensor:
    """(6 L C,) int64 on the host: row p of the weight that radial_gather_lmax_fwd takes is row
    perm[p] of the radial output layer's weight (fu_radial_gather_perm_lmax)."""
    import ctypes
    buf = (ctypes.c_int32 * (6 * L * C))()
    _lib.call("fu_radial_gather_perm_lmax", C, int(L), ctypes.addressof(buf))
    return torch.tensor(list(buf), dtype=torch.int64)


def radial_gather_lmax_fwd(h2, W2p, bias_p, x_in, idx_i, idx_j, wigner, wig_ext, csd_emb, batch, L):
    """fu_radial_gather_fwd_lmax: the radial output layer and the lmax 3 / 4 gather's
    (X_m0, X_m1, X_m2) from it in one kernel; returns (rad, X_m0, X_m1, X_m2).  W2p / bias_p:
    the weight with its rows permuted by radial_gather_lmax_perm, pre-split by
    linear_weight_split, and the bias permuted the same way."""
    E, K = h2.shape
    N, _, C = x_in.shape
    if h2.stride(-1) != 1 or h2.stride(0) % 4 != 0 or h2.data_ptr() % 16 != 0:
        h2 = h2.contiguous()
    dev = x_in.device
    rad = torch.empty(E, 6 * L * C, device=dev)
    X_m0 = torch.empty(E, 2 * (L + 1) * C, device=dev)
    X_m1 = torch.empty(E, 4 * L * C, device=dev)
    X_m2 = torch.empty(E, 4 * (L - 1) * C, device=dev)
    _lib.call("fu_radial_gather_fwd_lmax", h2.data_ptr(), h2.stride(0), W2p.data_ptr(), _lib.ptr(bias_p),
              x_in.data_ptr(), idx_i.data_ptr(), idx_j.data_ptr(), wigner.data_ptr(), wig_ext.data_ptr(),
              csd_emb.data_ptr(), batch.data_ptr(), rad.data_ptr(), X_m0.data_ptr(), X_m1.data_ptr(),
              X_m2.data_ptr(), E, N, csd_emb.shape[0], C, K, int(L), _lib.stream_ptr(dev))
    return rad, X_m0, X_m1, X_m2


def gather_lmax_fwd(x_in, idx_i, idx_j, wigner, wig_ext, rad_out, csd_emb, batch, L, topology=None):
    """fu_gather_fwd_lmax: (X_m0, X_m1, X_m2) for operands from gather_lmax_operands.  The kernel
    walks each node's receiver and sender CSR segments (from the topology, or built here), so
    every node row is read once per side."""
    N, _, C = x_in.shape
    E = idx_i.shape[0]
    dev = x_in.device
    X_m0 = torch.empty(E, 2 * (L + 1) * C, device=dev)
    X_m1 = torch.empty(E, 4 * L * C, device=dev)
    X_m2 = torch.empty(E, 4 * (L - 1) * C, device=dev)
    rptr, ridx, sptr, sidx = _csrs(topology, idx_i, idx_j, N, E)
    _lib.call("fu_gather_fwd_lmax", x_in.data_ptr(), idx_i.data_ptr(), idx_j.data_ptr(), wigner.data_ptr(),
              _ext_ptr(wig_ext), rad_out.data_ptr(), csd_emb.data_ptr(), batch.data_ptr(), rptr.data_ptr(),
              ridx.data_ptr(), sptr.data_ptr(), sidx.data_ptr(), X_m0.data_ptr(), X_m1.data_ptr(), X_m2.data_ptr(),
              E, N, csd_emb.shape[0], C, L, _lib.stream_ptr(dev))
    return X_m0, X_m1, X_m2


def gather_lmax_bwd(x_in, idx_i, idx_j, wigner, wig_ext, rad_out, csd_emb, batch, topology, L, g0, g1, g2,
                    sink=None):
    """fu_gather_bwd_lmax: (g_x, g_wigner, g_wig_ext, g_rad); with a sink (ops/edge_grad.py) the
    Wigner gradients are added to its accumulators and None is returned for them."""
    N, _, C = x_in.shape
    E = idx_i.shape[0]
    dev = x_in.device
    g0 = torch.zeros(E, 2 * (L + 1) * C, device=dev) if g0 is None else g0.contiguous()
    g1 = torch.zeros(E, 4 * L * C, device=dev) if g1 is None else g1.contiguous()
    g2 = torch.zeros(E, 4 * (L - 1) * C, device=dev) if g2 is None else g2.contiguous()
    rptr, ridx, sptr, sidx = _csrs(topology, idx_i, idx_j, N, E)
    g_x = torch.empty_like(x_in)
    bufs, acc = edge_grad.outputs(sink, {WIGNER: wigner, WIG_EXT: wig_ext})
    g_rad = torch.empty_like(rad_out)
    ws = torch.empty(E * (34 + ext_width(L)), device=dev)
    _lib.call("fu_gather_bwd_lmax", g0.data_ptr(), g1.data_ptr(), g2.data_ptr(), x_in.data_ptr(),
              wigner.data_ptr(), _ext_ptr(wig_ext), rad_out.data_ptr(), csd_emb.data_ptr(), batch.data_ptr(),
              rptr.data_ptr(), ridx.data_ptr(), sptr.data_ptr(), sidx.data_ptr(), g_x.data_ptr(),
              bufs[WIGNER].data_ptr(), _ext_ptr(bufs[WIG_EXT]), g_rad.data_ptr(), ws.data_ptr(), E, N,
              csd_emb.shape[0], C, L, acc, _lib.stream_ptr(dev))
    if sink is not None:
        return g_x, None, None, g_rad
    return g_x, bufs[WIGNER], bufs[WIG_EXT], g_rad


class GatherRotateLmax(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x_in, idx_i, idx_j, wigner, wig_ext, rad_out, csd_emb, batch, topology, lmax):
        L = int(lmax)
        ops = gather_lmax_operands(x_in, idx_i, idx_j, wigner, wig_ext, rad_out, csd_emb, batch, L)
        X = gather_lmax_fwd(*ops, L, topology)
        ctx.save_for_backward(*ops)
        ctx.topology, ctx.lmax = topology, L
        return X

    @staticmethod
    def backward(ctx, g0, g1, g2):
        g_x, g_w, g_ext, g_rad = gather_lmax_bwd(*ctx.saved_tensors, ctx.topology, ctx.lmax, g0, g1, g2)
        return g_x, None, None, g_w, g_ext, g_rad, None, None, None, None


def gather_rotate_lmax(x_in, idx_i, idx_j, wigner, wig_ext, rad_out, csd_emb, batch, topology=None, lmax=2):
    return GatherRotateLmax.apply(x_in, idx_i, idx_j, wigner, wig_ext, rad_out, csd_emb, batch, topology, int(lmax))


class GatingLmax(torch.autograd.Function):
    @staticmethod
    def forward(ctx, Y_m0, Y_m1, Y_m2, C, lmax):
        L = int(lmax)
        Y_m0 = _lib.require(Y_m0, torch.float32, "Y_m0")
        Y_m1 = _lib.require(Y_m1, torch.float32, "Y_m1")
        Y_m2 = _lib.require(Y_m2, torch.float32, "Y_m2")
        E = Y_m0.shape[0]
        dev = Y_m0.device
        Z_m0 = torch.empty(E, (L + 1) * C, device=dev)
        Z_m1 = torch.empty(E, 2 * L * C, device=dev)
        Z_m2 = torch.empty(E, 2 * (L - 1) * C, device=dev)
        _lib.call("fu_gating_fwd_lmax", Y_m0.data_ptr(), Y_m1.data_ptr(), Y_m2.data_ptr(), Z_m0.data_ptr(),
                  Z_m1.data_ptr(), Z_m2.data_ptr(), E, C, L, _lib.stream_ptr(dev))
        ctx.save_for_backward(Y_m0, Y_m1, Y_m2)
        ctx.C, ctx.lmax = C, L
        return Z_m0, Z_m1, Z_m2

    @staticmethod
    def backward(ctx, g0, g1, g2):
        Y_m0, Y_m1, Y_m2 = ctx.saved_tensors
        C, L = ctx.C, ctx.lmax
        E = Y_m0.shape[0]
        dev = Y_m0.device
        g0 = torch.zeros(E, (L + 1) * C, device=dev) if g0 is None else g0.contiguous()
        g1 = torch.zeros(E, 2 * L * C, device=dev) if g1 is None else g1.contiguous()
        g2 = torch.zeros(E, 2 * (L - 1) * C, device=dev) if g2 is None else g2.contiguous()
        gY0, gY1, gY2 = torch.empty_like(Y_m0), torch.empty_like(Y_m1), torch.empty_like(Y_m2)
        _lib.call("fu_gating_bwd_lmax", g0.data_ptr(), g1.data_ptr(), g2.data_ptr(), Y_m0.data_ptr(), Y_m1.data_ptr(),
                  Y_m2.data_ptr(), gY0.data_ptr(), gY1.data_ptr(), gY2.data_ptr(), E, C, L, _lib.stream_ptr(dev))
        return gY0, gY1, gY2, None, None


def gating_lmax(Y_m0, Y_m1, Y_m2, C: int, lmax: int):
    return GatingLmax.apply(Y_m0, Y_m1, Y_m2, int(C), int(lmax))


class RotateScatterLmax(torch.autograd.Function):
    @staticmethod
    def forward(ctx, Z_m0, Z_m1, Z_m2, wigner, wig_ext, env, x_res, idx_j, row_ptr, col_idx, N, lmax, sink=None):
        L = int(lmax)
        Z_m0 = _lib.require(Z_m0, torch.float32, "Z_m0")
        Z_m1 = _lib.require(Z_m1, torch.float32, "Z_m1")
        Z_m2 = _lib.require(Z_m2, torch.float32, "Z_m2")
        wigner = _lib.require(wigner, torch.float32, "wigner")
        wig_ext = _lib.require(wig_ext, torch.float32, "wig_ext")
        env = _lib.require(env, torch.float32, "env")
        x_res = _lib.require(x_res, torch.float32, "x_res")
        row_ptr = _lib.require(row_ptr, torch.int32, "row_ptr")
        col_idx = _lib.require(col_idx, torch.int32, "col_idx")
        E = Z_m0.shape[0]
        C = Z_m0.shape[1] // (L + 1)
        if x_res.shape != (N, (L + 1) ** 2, C):
            raise _lib.FlashUMAError(f"rotate_scatter_lmax: x_res must be ({N}, {(L + 1) ** 2}, {C})")
        x_out = torch.empty_like(x_res)
        _lib.call("fu_scatter_fwd_lmax", row_ptr.data_ptr(), col_idx.data_ptr(), Z_m0.data_ptr(), Z_m1.data_ptr(),
                  Z_m2.data_ptr(), wigner.data_ptr(), _ext_ptr(wig_ext), env.data_ptr(), x_res.data_ptr(),
                  x_out.data_ptr(), N, E, C, L, _lib.stream_ptr(Z_m0.device))
        ctx.save_for_backward(Z_m0, Z_m1, Z_m2, wigner, wig_ext, env, _lib.require(idx_j, torch.int64, "idx_j"))
        ctx.C, ctx.N, ctx.lmax, ctx.sink = C, N, L, sink
        return x_out

    @staticmethod
    def backward(ctx, g_out):
        Z_m0, Z_m1, Z_m2, wigner, wig_ext, env, idx_j = ctx.saved_tensors
        E, C, N, L = Z_m0.shape[0], ctx.C, ctx.N, ctx.lmax
        g_out = g_out.contiguous()
        gZ0, gZ1, gZ2 = torch.empty_like(Z_m0), torch.empty_like(Z_m1), torch.empty_like(Z_m2)
        bufs, acc = edge_grad.outputs(ctx.sink, {WIGNER: wigner, WIG_EXT: wig_ext, ENV: env})
        _lib.call("fu_scatter_bwd_lmax", g_out.data_ptr(), idx_j.data_ptr(), Z_m0.data_ptr(), Z_m1.data_ptr(),
                  Z_m2.data_ptr(), wigner.data_ptr(), _ext_ptr(wig_ext), env.data_ptr(), gZ0.data_ptr(),
                  gZ1.data_ptr(), gZ2.data_ptr(), bufs[WIGNER].data_ptr(), _ext_ptr(bufs[WIG_EXT]),
                  bufs[ENV].data_ptr(), E, N, C, L, acc, _lib.stream_ptr(g_out.device))
        g_w, g_ext, g_env = (None,) * 3 if ctx.sink is not None else (bufs[WIGNER], bufs[WIG_EXT], bufs[ENV])
        return gZ0, gZ1, gZ2, g_w, g_ext, g_env, g_out, None, None, None, None, None, None


def rotate_scatter_lmax(Z_m0, Z_m1, Z_m2, wigner, wig_ext, env, x_res, idx_j, row_ptr, col_idx, N, lmax, sink=None):
    return RotateScatterLmax.apply(Z_m0, Z_m1, Z_m2, wigner, wig_ext, env, x_res, idx_j, row_ptr, col_idx, N,
                                   int(lmax), sink)


class InitNodeScatterLmax(torch.autograd.Function):
    @staticmethod
    def forward(ctx, rad_out, wigner, wig_ext, env, Z, batch, W_sphere, csd_emb, idx_j, row_ptr, col_idx, N, lmax,
                sink=None):
        L = int(lmax)
        rad_out = _lib.require(rad_out, torch.float32, "rad_out")
        wigner = _lib.require(wigner, torch.float32, "wigner")
        wig_ext = _lib.require(wig_ext, torch.float32, "wig_ext")
        env = _lib.require(env, torch.float32, "env")
        Z = _lib.require(Z, torch.int64, "Z")
        batch = _lib.require(batch, torch.int64, "batch")
        W_sphere = _lib.require(W_sphere, torch.float32, "W_sphere")
        csd_emb = _lib.require(csd_emb, torch.float32, "csd_emb")
        row_ptr = _lib.require(row_ptr, torch.int32, "row_ptr")
        col_idx = _lib.require(col_idx, torch.int32, "col_idx")
        E = rad_out.shape[0]
        C = rad_out.shape[1] // (L + 1)
        x_out = torch.empty(N, (L + 1) ** 2, C, device=rad_out.device)
        _lib.call("fu_init_scatter_fwd_lmax", row_ptr.data_ptr(), col_idx.data_ptr(), rad_out.data_ptr(),
                  wigner.data_ptr(), _ext_ptr(wig_ext), env.data_ptr(), Z.data_ptr(), batch.data_ptr(),
                  W_sphere.data_ptr(), csd_emb.data_ptr(), x_out.data_ptr(), N, E, W_sphere.shape[0],
                  csd_emb.shape[0], C, L, _lib.stream_ptr(rad_out.device))
        ctx.save_for_backward(rad_out, wigner, wig_ext, env, _lib.require(idx_j, torch.int64, "idx_j"))
        ctx.C, ctx.N, ctx.lmax, ctx.sink = C, N, L, sink
        return x_out

    @staticmethod
    def backward(ctx, g_out):
        rad_out, wigner, wig_ext, env, idx_j = ctx.saved_tensors
        E, C, N, L = rad_out.shape[0], ctx.C, ctx.N, ctx.lmax
        g_out = g_out.contiguous()
        g_rad = torch.empty_like(rad_out)
        bufs, acc = edge_grad.outputs(ctx.sink, {WIGNER: wigner, WIG_EXT: wig_ext, ENV: env})
        _lib.call("fu_init_scatter_bwd_lmax", g_out.data_ptr(), idx_j.data_ptr(), rad_out.data_ptr(),
                  wigner.data_ptr(), _ext_ptr(wig_ext), env.data_ptr(), g_rad.data_ptr(), bufs[WIGNER].data_ptr(),
                  _ext_ptr(bufs[WIG_EXT]), bufs[ENV].data_ptr(), E, N, C, L, acc, _lib.stream_ptr(g_out.device))
        g_w, g_ext, g_env = (None,) * 3 if ctx.sink is not None else (bufs[WIGNER], bufs[WIG_EXT], bufs[ENV])
        return g_rad, g_w, g_ext, g_env, None, None, None, None, None, None, None, None, None, None


def init_node_scatter_lmax(rad_out, wigner, wig_ext, env, Z, batch, W_sphere, csd_emb, idx_j, row_ptr, col_idx, N,
                           lmax, sink=None):
    return InitNodeScatterLmax.apply(rad_out, wigner, wig_ext, env, Z, batch, W_sphere, csd_emb, idx_j, row_ptr,
                                     col_idx, N, int(lmax), sink)
