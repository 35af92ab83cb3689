"""Node-level ops on the gfx950 kernels: the equivariant RMS norm over SH coefficients, the
per-degree SO(3) linear and the gate activation of the atom-wise FFN (the FAIRChem modules
the reference attaches to each block, model.py:145,157,218), plus row permutations and the
PBC shift product used around the hot path (model.py:72-74,221; wrapper.py:193-194).

All parameters are frozen: backward passes return input gradients only."""
from __future__ import annotations

import torch

from . import _lib


class RmsNormSH(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, weight, bias, lmax, eps):
        x = _lib.require(x, torch.float32, "x")
        weight = _lib.require(weight, torch.float32, "weight")
        bias = _lib.require(bias, torch.float32, "bias")
        N, _, C = x.shape
        out = torch.empty_like(x)
        inv = torch.empty(N, device=x.device, dtype=torch.float32)
        _lib.call("fu_rms_norm_sh_fwd", x.data_ptr(), weight.data_ptr(), bias.data_ptr(), out.data_ptr(),
                  inv.data_ptr(), N, C, lmax, float(eps), _lib.stream_ptr(x.device))
        ctx.save_for_backward(x, weight, inv)
        ctx.lmax = lmax
        return out

    @staticmethod
    def backward(ctx, g_out):
        x, weight, inv = ctx.saved_tensors
        return _rms_norm_bwd(x, weight, inv, g_out, None, ctx.lmax), None, None, None, None


def _rms_norm_bwd(x, weight, inv, g_out, g_res, lmax):
    N, _, C = x.shape
    g_x = torch.empty_like(x)
    if g_out is None:
        g_out = torch.zeros_like(x)
    g_out = g_out.contiguous()
    g_res = None if g_res is None else g_res.contiguous()
    _lib.call("fu_rms_norm_sh_bwd", x.data_ptr(), weight.data_ptr(), inv.data_ptr(), g_out.data_ptr(),
              _lib.ptr(g_res), g_x.data_ptr(), N, C, lmax, _lib.stream_ptr(x.device))
    return g_x


def rms_norm_sh(x, weight, bias, lmax: int, eps: float):
    return RmsNormSH.apply(x, weight, bias, lmax, eps)


class RmsNormSHResidual(torch.autograd.Function):
    """(norm(x), x) for an x that also feeds a residual skip: the second output is x itself
    (a new view), and the backward returns norm^T g_norm + g_skip from one kernel, so autograd
    never sums the two node-sized gradients."""

    @staticmethod
    def forward(ctx, x, weight, bias, lmax, eps):
        out = RmsNormSH.forward(ctx, x, weight, bias, lmax, eps)
        return out, x.view_as(x)

    @staticmethod
    def backward(ctx, g_out, g_skip):
        x, weight, inv = ctx.saved_tensors
        if g_out is None and g_skip is None:
            return None, None, None, None, None
        return _rms_norm_bwd(x, weight, inv, g_out, g_skip, ctx.lmax), None, None, None, None


def rms_norm_sh_residual(x, weight, bias, lmax: int, eps: float):
    return RmsNormSHResidual.apply(x, weight, bias, lmax, eps)


def _so3_apply(x: torch.Tensor, Wk: torch.Tensor, bias: torch.Tensor | None,
               res: torch.Tensor | None = None) -> torch.Tensor:
    """y[:, k] = x[:, k] @ Wk[k]^T (+ bias on k = 0) (+ res) as one batched MFMA GEMM over k."""
    N, K9, Cin = x.shape
    Cout = Wk.shape[1]
    y = torch.empty(N, K9, Cout, device=x.device, dtype=torch.float32)
    if res is not None:
        res = _lib.require(res, torch.float32, "res")
    _lib.call("fu_linear_batched", x.data_ptr(), K9 * Cin, Cin, Wk.data_ptr(), Cin, Cout * Cin,
              None if bias is None else bias.data_ptr(), 0, 1, _lib.ptr(res), K9 * Cout, Cout, y.data_ptr(),
              K9 * Cout, Cout, N, Cout, Cin, K9, _lib.stream_ptr(x.device))
    return y


class So3Linear(torch.autograd.Function):
    """x (N, K, Cin) -> (N, K, Cout) with a weight per coefficient k: W_k (Cout, Cin)
    (the weight of k's degree), bias on k = 0.  Wt_k = W_k^T for the input gradient."""

    @staticmethod
    def forward(ctx, x, Wk, Wtk, bias):
        x = _lib.require(x, torch.float32, "x")
        ctx.save_for_backward(Wtk)
        return _so3_apply(x, Wk, bias)

    @staticmethod
    def backward(ctx, g_y):
        (Wtk,) = ctx.saved_tensors
        return _so3_apply(g_y.contiguous(), Wtk, None), None, None, None


def so3_linear(x, Wk, Wtk, bias):
    return So3Linear.apply(x, Wk, Wtk, bias)


class So3LinearResidual(torch.autograd.Function):
    """so3_linear(x) + res with the residual added in the GEMM epilogue; the residual's
    gradient is the output gradient itself (no copy, no add)."""

    @staticmethod
    def forward(ctx, x, Wk, Wtk, bias, res):
        x = _lib.require(x, torch.float32, "x")
        ctx.save_for_backward(Wtk)
        return _so3_apply(x, Wk, bias, res)

    @staticmethod
    def backward(ctx, g_y):
        (Wtk,) = ctx.saved_tensors
        g_y = g_y.contiguous()
        return _so3_apply(g_y, Wtk, None), None, None, None, g_y


def so3_linear_residual(x, Wk, Wtk, bias, res):
    return So3LinearResidual.apply(x, Wk, Wtk, bias, res)


class ScalarGemmSo3(torch.autograd.Function):
    """(pre, h) = (x[:, 0] @ W^T + b, so3_linear(x)) for the atom-wise block's two reads of x:
    the backward adds the scalar branch's (N, C) gradient into the l = 0 rows of the SO(3)
    branch's gradient in place, instead of autograd zero-filling an (N, K, C) tensor for the
    slice and summing two node-sized gradients."""

    @staticmethod
    def forward(ctx, x, W, b, Wt, Wk, Wtk, bias):
        from .linear import gemm
        x = _lib.require(x, torch.float32, "x")
        pre = gemm(x[:, 0, :], W, b)
        h = _so3_apply(x, Wk, bias)
        ctx.save_for_backward(Wt, Wtk)
        return pre, h

    @staticmethod
    def backward(ctx, g_pre, g_h):
        from .linear import gemm
        Wt, Wtk = ctx.saved_tensors
        g_x = _so3_apply(g_h.contiguous(), Wtk, None)
        if g_pre is not None:
            g_x[:, 0, :] += gemm(g_pre.contiguous(), Wt)
        return g_x, None, None, None, None, None, None


def scalar_gemm_so3(x, W, b, Wt, Wk, Wtk, bias):
    return ScalarGemmSo3.apply(x, W, b, Wt, Wk, Wtk, bias)


class GateAct(torch.autograd.Function):
    """gate_l = sigmoid(silu(pre_l)); out_0 = silu(h_0); out_k = h_k gate_{l_k}."""

    @staticmethod
    def forward(ctx, pre, h, lmax):
        pre = _lib.require(pre, torch.float32, "pre")
        h = _lib.require(h, torch.float32, "h")
        out = torch.empty_like(h)
        N, _, H = h.shape
        _lib.call("fu_gate_act_fwd", pre.data_ptr(), h.data_ptr(), out.data_ptr(), N, H, lmax,
                  _lib.stream_ptr(h.device))
        ctx.save_for_backward(pre, h)
        ctx.lmax = lmax
        return out

    @staticmethod
    def backward(ctx, g_out):
        pre, h = ctx.saved_tensors
        N, _, H = h.shape
        g_out = g_out.contiguous()
        g_pre = torch.empty_like(pre)
        g_h = torch.empty_like(h)
        _lib.call("fu_gate_act_bwd", pre.data_ptr(), h.data_ptr(), g_out.data_ptr(), g_pre.data_ptr(), g_h.data_ptr(),
                  N, H, ctx.lmax, _lib.stream_ptr(h.device))
        return g_pre, g_h, None


def gate_act(pre, h, lmax: int):
    return GateAct.apply(pre, h, lmax)


class PermuteRows(torch.autograd.Function):
    """out[r] = src[perm[r]] for a permutation perm; the backward scatters rows back
    (each row once: no accumulation, deterministic)."""

    @staticmethod
    def forward(ctx, src, perm):
        src = _lib.require(src, torch.float32, "src")
        rows = perm.numel()
        width = src[0].numel() if src.shape[0] else 1
        out = torch.empty((rows,) + tuple(src.shape[1:]), device=src.device, dtype=torch.float32)
        _lib.call("fu_gather_rows", src.data_ptr(), perm.data_ptr(), out.data_ptr(), rows, width,
                  _lib.stream_ptr(src.device))
        ctx.save_for_backward(perm)
        ctx.width = width
        return out

    @staticmethod
    def backward(ctx, g_out):
        (perm,) = ctx.saved_tensors
        g_out = g_out.contiguous()
        g_src = torch.empty_like(g_out)
        _lib.call("fu_scatter_rows", g_out.data_ptr(), perm.data_ptr(), g_src.data_ptr(), perm.numel(), ctx.width,
                  _lib.stream_ptr(g_out.device))
        return g_src, None


def permute_rows(src, perm):
    return PermuteRows.apply(src, perm)


class EdgeShifts(torch.autograd.Function):
    """shifts = cell_offsets @ cell for one system; dE/dcell = cell_offsets^T dE/dshifts,
    reduced deterministically in fp64."""

    @staticmethod
    def forward(ctx, cell_offsets, cell):
        off = _lib.require(cell_offsets, torch.float32, "cell_offsets")
        c = _lib.require(cell.reshape(3, 3), torch.float32, "cell")
        E = off.shape[0]
        shifts = torch.empty(E, 3, device=off.device, dtype=torch.float32)
        _lib.call("fu_edge_shifts", off.data_ptr(), c.data_ptr(), None, shifts.data_ptr(), E,
                  _lib.stream_ptr(off.device))
        ctx.save_for_backward(off)
        ctx.cell_shape = cell.shape
        return shifts

    @staticmethod
    def backward(ctx, g_shifts):
        (off,) = ctx.saved_tensors
        g_shifts = g_shifts.contiguous()
        g_cell = torch.empty(3, 3, device=off.device, dtype=torch.float32)
        partial = torch.empty(256 * 9, device=off.device, dtype=torch.float64)
        _lib.call("fu_outer_sum3", off.data_ptr(), None, g_shifts.data_ptr(), g_cell.data_ptr(), partial.data_ptr(),
                  partial.numel(), off.shape[0], _lib.stream_ptr(off.device))
        return None, g_cell.reshape(ctx.cell_shape)


def edge_shifts(cell_offsets, cell):
    return EdgeShifts.apply(cell_offsets, cell)


def system_ptr(batch: torch.Tensor, n_systems: int) -> torch.Tensor:
    """(S + 1,) int32 segment pointers of a batch vector sorted ascending (atoms of system s
    are rows [ptr[s], ptr[s + 1]))."""
    batch = _lib.require(batch, torch.int64, "batch")
    ptr = torch.empty(n_systems + 1, dtype=torch.int32, device=batch.device)
    _lib.call("fu_csr_row_ptr", batch.data_ptr(), batch.numel(), ptr.data_ptr(), n_systems,
              _lib.stream_ptr(batch.device))
    return ptr


def _balance(x, batch, sys_ptr, target, offset, S, start, end):
    N, K, C = x.shape
    out = torch.empty_like(x)
    corr = torch.empty(max(S * (end - start), 1), device=x.device, dtype=torch.float32)
    _lib.call("fu_balance_channels", x.data_ptr(), out.data_ptr(), batch.data_ptr(), sys_ptr.data_ptr(),
              _lib.ptr(target), float(offset), corr.data_ptr(), corr.numel(), N, K, C, S, start, end,
              _lib.stream_ptr(x.device))
    return out


class BalanceChannels(torch.autograd.Function):
    """FAIRChem balance_channels_batched (model.py:213-216) on fu_balance_channels: the l = 0
    coefficients of channels [start, end) are shifted per system so that they sum to
    target - target_offset over the system's atoms.  Affine in x, so the input gradient
    removes the per-system mean of those channels' output gradient."""

    @staticmethod
    def forward(ctx, emb, target, batch, sys_ptr, start, end, offset):
        emb = _lib.require(emb, torch.float32, "emb")
        batch = _lib.require(batch, torch.int64, "batch")
        target = _lib.require(target.reshape(-1), torch.float32, "target")
        S = target.numel()
        ctx.save_for_backward(batch, sys_ptr)
        ctx.S, ctx.start, ctx.end = S, start, end
        return _balance(emb, batch, sys_ptr, target, offset, S, start, end)

    @staticmethod
    def backward(ctx, g_out):
        batch, sys_ptr = ctx.saved_tensors
        g = _balance(g_out.contiguous(), batch, sys_ptr, None, 0.0, ctx.S, ctx.start, ctx.end)
        return g, None, None, None, None, None, None


def balance_channels_batched(emb, target, natoms, batch, start_idx: int, end_idx: int, target_offset: float = 0.0,
                             sys_ptr=None):
    """FAIRChem's balance_channels_batched with its argument meaning (emb (N, K, C), target
    (S,) per-system charge or spin, natoms (S,) atoms per system, batch (N,) system of each
    atom).  The divisor n_s is the number of atoms of system s in batch, which equals
    natoms[s] for consistent inputs.  The kernel works on system segments of a batch sorted
    ascending; an unsorted batch (which FAIRChem's index_add form accepts) is balanced
    through a stable sort of the atoms and the result put back in the input order.
    sys_ptr: the system segments of a batch already known to be sorted (system_ptr); it is
    then trusted without a check, as the model does with its Morton-ordered systems."""
    if target is None:
        raise ValueError("balance_channels_batched: the backbone balances channels but no per-system target "
                         "(charge or spin) was given")
    S = int(target.numel())
    if natoms is not None and int(natoms.numel()) != S:
        raise ValueError(f"balance_channels_batched: {int(natoms.numel())} systems in natoms, {S} targets")
    args = (int(start_idx), int(end_idx), float(target_offset))
    if sys_ptr is None:
        batch = _lib.require(batch, torch.int64, "batch")
        if batch.numel() > 1 and bool((batch[1:] < batch[:-1]).any()):   # one host sync, public path only
            perm = torch.sort(batch, stable=True).indices
            sb = batch.index_select(0, perm)
            out = BalanceChannels.apply(emb.index_select(0, perm), target, sb, system_ptr(sb, S), *args)
            return out.index_select(0, torch.argsort(perm))
        sys_ptr = system_ptr(batch, S)
    return BalanceChannels.apply(emb, target, batch, sys_ptr, *args)
