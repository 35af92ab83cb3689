"""precompute_geometry (ops/geom.py:496-592) on the gfx950 geometry kernels.

Backward: the per-edge VJP kernel writes dE/dd (which is also dE/dshifts, ops/geom.py:490-493);
dE/dpos is then reduced per atom over the sender and receiver CSRs in a fixed order
instead of the reference's atomics (ops/geom.py:483-488)."""
from __future__ import annotations

import torch

from . import _lib, edge_grad
from .edge_grad import ENV, WIGNER
from .topology import receiver_csr, sender_csr


class PrecomputeGeometry(torch.autograd.Function):
    @staticmethod
    def forward(ctx, pos, Z, idx_i, idx_j, shifts, W_src, W_tgt, offset_g, coeff_g, cutoff, topology=None,
                embeddings=True, sink=None):
        pos = _lib.require(pos, torch.float32, "pos")
        shifts = _lib.require(shifts, torch.float32, "shifts")
        Z = _lib.require(Z, torch.int64, "Z")
        idx_i = _lib.require(idx_i, torch.int64, "idx_i")
        idx_j = _lib.require(idx_j, torch.int64, "idx_j")
        offset_g = _lib.require(offset_g, torch.float32, "offset_g")
        E = idx_i.shape[0]
        N = pos.shape[0]
        B = offset_g.shape[0]
        C = W_src.shape[1]
        dev = pos.device
        width = B + 2 * C if embeddings else B
        x_edge_raw = torch.empty(E, width, device=dev, dtype=torch.float32)
        wigner = torch.empty(E, 34, device=dev, dtype=torch.float32)
        env = torch.empty(E, device=dev, dtype=torch.float32)
        Ws = _lib.require(W_src, torch.float32, "W_src") if embeddings else None
        Wt = _lib.require(W_tgt, torch.float32, "W_tgt") if embeddings else None
        _lib.call("fu_geom_fwd", pos.data_ptr(), Z.data_ptr(), idx_i.data_ptr(), idx_j.data_ptr(), shifts.data_ptr(),
                  _lib.ptr(Ws), _lib.ptr(Wt), offset_g.data_ptr(), x_edge_raw.data_ptr(), width,
                  wigner.data_ptr(), env.data_ptr(), E, N, B, C, float(cutoff), float(coeff_g),
                  _lib.stream_ptr(dev))
        ctx.save_for_backward(pos, idx_i, idx_j, shifts, offset_g)
        ctx.cutoff, ctx.coeff_g, ctx.B = float(cutoff), float(coeff_g), B
        ctx.topology, ctx.sink = topology, sink
        # outputs whose readers all add into the sink receive no gradient from autograd: keep
        # those None instead of zero-filled arrays
        ctx.set_materialize_grads(False)
        return x_edge_raw, wigner, env

    @staticmethod
    def backward(ctx, g_x_edge_raw, g_wigner, g_env):
        pos, idx_i, idx_j, shifts, offset_g = ctx.saved_tensors
        E, N, B = idx_i.shape[0], pos.shape[0], ctx.B
        dev = pos.device
        st = _lib.stream_ptr(dev)
        # the readers that took part in the sink (ops/edge_grad.py) added their gradients there
        g_wigner = edge_grad.merge(ctx.sink, WIGNER, g_wigner)
        g_env = edge_grad.merge(ctx.sink, ENV, g_env)
        gxe = None if g_x_edge_raw is None else g_x_edge_raw.contiguous()
        gw = None if g_wigner is None else g_wigner.contiguous()
        ge = None if g_env is None else g_env.contiguous()
        g_d = torch.empty(E, 3, device=dev, dtype=torch.float32)
        _lib.call("fu_geom_bwd", pos.data_ptr(), idx_i.data_ptr(), idx_j.data_ptr(), shifts.data_ptr(),
                  offset_g.data_ptr(), _lib.ptr(gxe), 0 if gxe is None else gxe.stride(0), _lib.ptr(gw),
                  _lib.ptr(ge), g_d.data_ptr(), E, N, B, ctx.cutoff, ctx.coeff_g, st)
        g_pos = None
        if ctx.needs_input_grad[0]:
            topo = ctx.topology
            if topo is not None and topo.E == E and topo.N == N:
                rptr, ridx, sptr, sidx = topo.recv_ptr, topo.recv_idx, topo.send_ptr, topo.send_idx
            else:
                rptr, ridx = receiver_csr(idx_j, N)
                sptr, sidx = sender_csr(idx_i, N)
            g_pos = torch.empty(N, 3, device=dev, dtype=torch.float32)
            _lib.call("fu_edge_vec_reduce", g_d.data_ptr(), rptr.data_ptr(), ridx.data_ptr(), sptr.data_ptr(),
                      sidx.data_ptr(), g_pos.data_ptr(), N, E, st)
        g_shifts = g_d if ctx.needs_input_grad[4] else None
        return g_pos, None, None, None, g_shifts, None, None, None, None, None, None, None, None


def precompute_geometry(pos, Z, idx_i, idx_j, shifts, W_src, W_tgt, offset_g, coeff_g, cutoff, topology=None,
                        embeddings=True, sink=None):
    """Returns (x_edge_raw (E, B+2C), wigner (E, 34), env (E)); with embeddings=False the
    element-embedding columns are left out and x_edge_raw is (E, B).  sink: the readers'
    accumulators of dE/dwigner and dE/denv (ops/edge_grad.py), taken in the backward."""
    return PrecomputeGeometry.apply(pos, Z, idx_i, idx_j, shifts, W_src, W_tgt, offset_g, coeff_g, cutoff,
                                    topology, embeddings, sink)
