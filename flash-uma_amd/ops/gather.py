"""gather_wigner_split (ops/gather.py:408-516) on the gfx950 gather kernels.

The backward is node-centric over the receiver and sender CSRs (no atomics, bitwise
reproducible); it needs both CSRs, taken from the cached topology when given.

layout 0 keeps the reference's column-block order of X_m* and rad_out (sender/receiver
slots interleaved, ops/gather.py:132-154).  layout 1 (LAYOUT1_PERM below) stores X_m0 and
rad side-major (sender blocks, then receiver blocks), X_m1 as [real half | imaginary half]
with each half side-major, and X_m2 in reference order; the model uses it with conv1 and
radial weights permuted to match, which leaves every product unchanged, gives each side of
the backward contiguous runs, and hands the complex m = 1, 2 layers contiguous x_r, x_i."""
from __future__ import annotations

import torch

from . import _lib, edge_grad
from .constants import RAD_MULT, X_M0_MULT, X_M1_MULT, X_M2_MULT
from .edge_grad import WIGNER
from .topology import receiver_csr, sender_csr


# Column-block permutation of layout 1: new block b holds reference block perm[b].
LAYOUT1_PERM = {
    "m0": [0, 2, 4, 1, 3, 5],
    "m1": [0, 2, 1, 3, 4, 6, 5, 7],
    "m2": [0, 1, 2, 3],
    "rad": [0, 2, 4, 6, 8, 10, 1, 3, 5, 7, 9, 11],
}


def block_permutation(perm, C: int) -> torch.Tensor:
    """Column index map (len(perm) * C) of a block permutation with blocks of C columns."""
    return torch.cat([torch.arange(p * C, (p + 1) * C) for p in perm])


def gather_fwd(x_in, idx_i, idx_j, wigner, rad_out, csd_emb, batch, layout, skip_m0=False):
    """fu_gather_fwd: (X_m0, X_m1, X_m2) for contiguous, correctly typed operands; with
    skip_m0, X_m0 is None (not formed: conv1 m = 0 gathers it, fu_gather_linear_gate)."""
    N, _, C = x_in.shape
    E = idx_i.shape[0]
    if rad_out.shape != (E, RAD_MULT * C):
        raise _lib.FlashUMAError(f"rad_out must be ({E}, {RAD_MULT * C}), got {tuple(rad_out.shape)}")
    dev = x_in.device
    X_m0 = None if skip_m0 else torch.empty((E, X_M0_MULT * C), device=dev, dtype=torch.float32)
    X_m1 = torch.empty((E, X_M1_MULT * C), device=dev, dtype=torch.float32)
    X_m2 = torch.empty((E, X_M2_MULT * C), device=dev, dtype=torch.float32)
    _lib.call("fu_gather_fwd", x_in.data_ptr(), idx_i.data_ptr(), idx_j.data_ptr(), wigner.data_ptr(),
              rad_out.data_ptr(), csd_emb.data_ptr(), batch.data_ptr(), _lib.ptr(X_m0), X_m1.data_ptr(),
              X_m2.data_ptr(), E, N, csd_emb.shape[0], C, int(layout), _lib.stream_ptr(dev))
    return X_m0, X_m1, X_m2


def gather_bwd(x_in, idx_i, idx_j, wigner, rad_out, csd_emb, batch, topology, layout, g_x_m0, g_x_m1, g_x_m2,
               sink=None):
    """fu_gather_bwd (node-centric over both CSRs): (g_x, g_wigner, g_rad); with a sink
    (ops/edge_grad.py) g_wigner is added to its accumulator and None is returned for it."""
    N, _, C = x_in.shape
    E = idx_i.shape[0]
    dev = x_in.device
    g_x_m0 = torch.zeros(E, X_M0_MULT * C, device=dev) if g_x_m0 is None else g_x_m0.contiguous()
    g_x_m1 = torch.zeros(E, X_M1_MULT * C, device=dev) if g_x_m1 is None else g_x_m1.contiguous()
    g_x_m2 = torch.zeros(E, X_M2_MULT * C, device=dev) if g_x_m2 is None else g_x_m2.contiguous()
    topo = topology
    if topo is not None and topo.E == E and topo.N == N:
        rptr, ridx, sptr, sidx = topo.recv_ptr, topo.recv_idx, topo.send_ptr, topo.send_idx
    else:
        rptr, ridx = receiver_csr(idx_j, N)
        sptr, sidx = sender_csr(idx_i, N)
    g_x = torch.empty_like(x_in)
    bufs, acc = edge_grad.outputs(sink, {WIGNER: wigner})
    g_rad = torch.empty_like(rad_out)
    ws = torch.empty_like(wigner)
    _lib.call("fu_gather_bwd", g_x_m0.data_ptr(), g_x_m1.data_ptr(), g_x_m2.data_ptr(), x_in.data_ptr(),
              idx_i.data_ptr(), idx_j.data_ptr(), wigner.data_ptr(), rad_out.data_ptr(), csd_emb.data_ptr(),
              batch.data_ptr(), rptr.data_ptr(), ridx.data_ptr(), sptr.data_ptr(), sidx.data_ptr(),
              g_x.data_ptr(), bufs[WIGNER].data_ptr(), g_rad.data_ptr(), ws.data_ptr(), E, N, csd_emb.shape[0], C,
              int(layout), acc, _lib.stream_ptr(dev))
    return g_x, (None if sink is not None else bufs[WIGNER]), g_rad


def radial_gather_perm(C: int, layout: int) -> torch.Tensor:
    """(12C,) int64 on the host: row p of the weight that radial_gather_fwd takes is row perm[p]
    of the radial output layer's weight (fu_radial_gather_perm)."""
    import ctypes
    buf = (ctypes.c_int32 * (RAD_MULT * C))()
    _lib.call("fu_radial_gather_perm", C, int(layout), ctypes.addressof(buf))
    return torch.tensor(list(buf), dtype=torch.int64)


def radial_gather_fwd(h2, W2p, bias_p, x_in, idx_i, idx_j, wigner, csd_emb, batch, layout):
    """fu_radial_gather_fwd: the radial output layer rad = h2 W3^T + b3 and the gather's
    (X_m0, X_m1, X_m2) from it in one kernel; returns (rad, X_m0, X_m1, X_m2).  W2p / bias_p:
    the weight with its rows permuted by radial_gather_perm, pre-split by linear_weight_split,
    and the bias permuted the same way.  h2 may be a row-strided view with 16-byte aligned rows."""
    E, K = h2.shape
    N, _, C = x_in.shape
    if h2.stride(-1) != 1 or h2.stride(0) % 4 != 0 or h2.data_ptr() % 16 != 0:
        h2 = h2.contiguous()
    dev = x_in.device
    rad = torch.empty((E, RAD_MULT * C), device=dev, dtype=torch.float32)
    X_m0 = torch.empty((E, X_M0_MULT * C), device=dev, dtype=torch.float32)
    X_m1 = torch.empty((E, X_M1_MULT * C), device=dev, dtype=torch.float32)
    X_m2 = torch.empty((E, X_M2_MULT * C), device=dev, dtype=torch.float32)
    _lib.call("fu_radial_gather_fwd", h2.data_ptr(), h2.stride(0), W2p.data_ptr(), _lib.ptr(bias_p), x_in.data_ptr(),
              idx_i.data_ptr(), idx_j.data_ptr(), wigner.data_ptr(), csd_emb.data_ptr(), batch.data_ptr(),
              rad.data_ptr(), X_m0.data_ptr(), X_m1.data_ptr(), X_m2.data_ptr(), E, N, csd_emb.shape[0], C, K,
              int(layout), _lib.stream_ptr(dev))
    return rad, X_m0, X_m1, X_m2


def gather_operands(x_in, idx_i, idx_j, wigner, rad_out, csd_emb, batch):
    """The gather's operands as contiguous tensors of the kernel's types."""
    return (_lib.require(x_in, torch.float32, "x_in"), _lib.require(idx_i, torch.int64, "idx_i"),
            _lib.require(idx_j, torch.int64, "idx_j"), _lib.require(wigner, torch.float32, "wigner"),
            _lib.require(rad_out, torch.float32, "rad_out"), _lib.require(csd_emb, torch.float32, "csd_emb"),
            _lib.require(batch, torch.int64, "batch"))


class GatherWignerSplit(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x_in, idx_i, idx_j, wigner, rad_out, csd_emb, batch, topology=None, layout=0):
        ops = gather_operands(x_in, idx_i, idx_j, wigner, rad_out, csd_emb, batch)
        X = gather_fwd(*ops, layout)
        ctx.save_for_backward(*ops)
        ctx.topology, ctx.layout = topology, int(layout)
        return X

    @staticmethod
    def backward(ctx, g_x_m0, g_x_m1, g_x_m2):
        g_x, g_wigner, g_rad = gather_bwd(*ctx.saved_tensors, ctx.topology, ctx.layout, g_x_m0, g_x_m1, g_x_m2)
        # no gradient for csd_emb or batch (ops/gather.py:513-514)
        return g_x, None, None, g_wigner, g_rad, None, None, None, None


def gather_wigner_split(x_in, idx_i, idx_j, wigner, rad_out, csd_emb, batch, topology=None, layout=0):
    return GatherWignerSplit.apply(x_in, idx_i, idx_j, wigner, rad_out, csd_emb, batch, topology, layout)
