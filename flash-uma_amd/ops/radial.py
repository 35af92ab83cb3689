"""All radial MLPs of the model as one bank (the per-block radial MLP of model.py:147-149 and
the edge-degree one of model.py:203-205, each Linear -> LNSiLU -> Linear -> LNSiLU -> Linear).

Every radial MLP reads the same edge features x_edge_raw = [g | W_src[Z_i] | W_tgt[Z_j]]
(Gaussians g (B), source and target element embeddings (C each), ops/geom.py:196-214).  Its
first linear therefore splits as

    W1 x_edge_raw + b1 = W1[:, :B] g + (W1[:, B:B+C] W_src^T)[:, Z_i] + (W1[:, B+C:] W_tgt^T)[:, Z_j] + b1

and the two element terms are tables of 100 rows per block, computed once when the model is
frozen.  The bank runs the Gaussian part of all G blocks as ONE GEMM (E x B -> E x G*C), adds
the table rows inside the grouped LayerNorm+SiLU kernel, runs the G second linears as one
batched GEMM, a second grouped LayerNorm+SiLU, then each block's output linear.  The
backward mirrors it and returns one gradient for the Gaussians: the per-block (E, B+2C)
x_edge_raw gradients and their G-way sum are never formed.  Element embeddings are frozen
and the geometry backward ignores their columns (ops/geom.py:588-589), so no gradient is
lost.  Results equal the per-block MLPs up to fp32 rounding order."""
from __future__ import annotations

import torch

from . import _lib
from .constants import LN_EPS
from .linear import gemm_resident, linear_weight_split, resident_ok


def _ln_grouped_fwd(x, tabs, z, isrc, idst, bias, gamma, beta, G, D, eps):
    M = x.shape[0]
    out = torch.empty_like(x)
    mean = torch.empty(M * G, device=x.device, dtype=torch.float32)
    rstd = torch.empty(M * G, device=x.device, dtype=torch.float32)
    ts, td = tabs if tabs is not None else (None, None)
    _lib.call("fu_ln_silu_grouped_fwd", x.data_ptr(), x.stride(0), _lib.ptr(ts), _lib.ptr(td),
              0 if ts is None else ts.stride(0), _lib.ptr(z), _lib.ptr(isrc), _lib.ptr(idst), _lib.ptr(bias),
              gamma.data_ptr(), beta.data_ptr(), out.data_ptr(), out.stride(0), mean.data_ptr(), rstd.data_ptr(),
              M, G, D, float(eps), _lib.stream_ptr(x.device))
    return out, mean, rstd


def _ln_grouped_bwd(x, tabs, z, isrc, idst, bias, gamma, beta, mean, rstd, g_out, G, D):
    M = x.shape[0]
    g_x = torch.empty_like(x)
    ts, td = tabs if tabs is not None else (None, None)
    _lib.call("fu_ln_silu_grouped_bwd", x.data_ptr(), x.stride(0), _lib.ptr(ts), _lib.ptr(td),
              0 if ts is None else ts.stride(0), _lib.ptr(z), _lib.ptr(isrc), _lib.ptr(idst), _lib.ptr(bias),
              gamma.data_ptr(), beta.data_ptr(), mean.data_ptr(), rstd.data_ptr(), g_out.data_ptr(),
              g_out.stride(0), g_x.data_ptr(), g_x.stride(0), M, G, D, _lib.stream_ptr(x.device))
    return g_x


def _batched(A, W, bias, G, C_in, C_out, out):
    """out[:, g*C_out:(g+1)*C_out] = A[:, g*C_in:(g+1)*C_in] @ W[g]^T (+ bias[g]) for all g."""
    M = A.shape[0]
    _lib.call("fu_linear_batched", A.data_ptr(), A.stride(0), C_in, W.data_ptr(), C_in, C_out * C_in,
              _lib.ptr(bias), C_out if bias is not None else 0, G if bias is not None else 0, None, 0, 0,
              out.data_ptr(),
              out.stride(0), C_out, M, C_out, C_in, G, _lib.stream_ptr(A.device))
    return out


# Channel count of the one-kernel GEMM + LayerNorm-SiLU path (one 128-column GEMM tile per
# LayerNorm group); other widths run the GEMM and the grouped LayerNorm kernel one after the other.
LN_FUSED_C = 128


def _layer1_fwd(gauss, bank, Z, idx_i, idx_j):
    """h1 = silu(LN(gauss W1g^T + tables + b1)) per group: (h1, mean1, rstd1)."""
    E, G, C = gauss.shape[0], bank.G, bank.C
    dev = gauss.device
    tabs = (bank.tab_src, bank.tab_tgt)
    if C != LN_FUSED_C:
        p1 = _gemm(gauss, bank.W1g, None, torch.empty(E, G * C, device=dev, dtype=torch.float32))
        return _ln_grouped_fwd(p1, tabs, Z, idx_i, idx_j, bank.b1, bank.gamma1, bank.beta1, G, C, bank.eps)
    h1 = torch.empty(E, G * C, device=dev, dtype=torch.float32)
    m1 = torch.empty(E * G, device=dev, dtype=torch.float32)
    r1 = torch.empty(E * G, device=dev, dtype=torch.float32)
    _lib.call("fu_linear_ln_silu", gauss.data_ptr(), gauss.stride(0), 0, bank.W1g.data_ptr(), bank.W1g.stride(0), 0,
              None, 0, 0, h1.data_ptr(), h1.stride(0), 0, None, 0, 0, E, G * C, bank.B, 1,
              bank.tab_src.data_ptr(), bank.tab_tgt.data_ptr(), bank.tab_src.stride(0), Z.data_ptr(),
              idx_i.data_ptr(), idx_j.data_ptr(), bank.b1.data_ptr(), bank.gamma1.data_ptr(), bank.beta1.data_ptr(),
              m1.data_ptr(), r1.data_ptr(), G, float(bank.eps), _lib.stream_ptr(dev))
    return h1, m1, r1


def _layer2_fwd(h1, bank):
    """p2 = h1_g W2_g^T + b2_g per group, h2 = silu(LN(p2)): (h2, mean2, rstd2, p2)."""
    E, G, C = h1.shape[0], bank.G, bank.C
    if C != LN_FUSED_C:
        p2 = _batched(h1, bank.W2, bank.b2, G, C, C, torch.empty_like(h1))
        h2, m2, r2 = _ln_grouped_fwd(p2, None, None, None, None, None, bank.gamma2, bank.beta2, G, C, bank.eps)
        return h2, m2, r2, p2
    dev = h1.device
    h2, p2 = torch.empty_like(h1), torch.empty_like(h1)
    m2 = torch.empty(E * G, device=dev, dtype=torch.float32)
    r2 = torch.empty(E * G, device=dev, dtype=torch.float32)
    _lib.call("fu_linear_ln_silu", h1.data_ptr(), h1.stride(0), C, bank.W2.data_ptr(), C, C * C, bank.b2.data_ptr(),
              C, G, h2.data_ptr(), h2.stride(0), C, p2.data_ptr(), p2.stride(0), C, E, C, C, G,
              None, None, 0, None, None, None, None, bank.gamma2.data_ptr(), bank.beta2.data_ptr(),
              m2.data_ptr(), r2.data_ptr(), G, float(bank.eps), _lib.stream_ptr(dev))
    return h2, m2, r2, p2


def _layer1_bwd(gauss, bank, Z, idx_i, idx_j, m1, r1, g_h1):
    """dL/d(first-layer LayerNorm input) from g_h1, recomputing gauss W1g^T."""
    E, G, C = gauss.shape[0], bank.G, bank.C
    dev = gauss.device
    tabs = (bank.tab_src, bank.tab_tgt)
    if C != LN_FUSED_C:
        p1 = _gemm(gauss, bank.W1g, None, torch.empty(E, G * C, device=dev, dtype=torch.float32))
        return _ln_grouped_bwd(p1, tabs, Z, idx_i, idx_j, bank.b1, bank.gamma1, bank.beta1, m1, r1, g_h1, G, C)
    g_p1 = torch.empty(E, G * C, device=dev, dtype=torch.float32)
    _lib.call("fu_linear_ln_silu_bwd", gauss.data_ptr(), gauss.stride(0), bank.W1g.data_ptr(), bank.W1g.stride(0),
              g_p1.data_ptr(), g_p1.stride(0), E, G * C, bank.B, g_h1.data_ptr(), g_h1.stride(0),
              bank.tab_src.data_ptr(), bank.tab_tgt.data_ptr(), bank.tab_src.stride(0), Z.data_ptr(),
              idx_i.data_ptr(), idx_j.data_ptr(), bank.b1.data_ptr(), bank.gamma1.data_ptr(), bank.beta1.data_ptr(),
              m1.data_ptr(), r1.data_ptr(), G, _lib.stream_ptr(dev))
    return g_p1


def _gemm(A, W, bias, out, W2=None):
    M, K = A.shape
    N = W.shape[0]
    _lib.call("fu_linear", A.data_ptr(), A.stride(0), W.data_ptr(), W.stride(0), _lib.ptr(bias), out.data_ptr(),
              out.stride(0), M, N, K, _lib.ptr(W2), _lib.stream_ptr(A.device))
    return out


def _out_gemm(A, W, bias, W2, out=None):
    """An output layer's product: in the split-fp16 mode, with the weight pre-split (W2), on
    fu_linear_resident (the (E, C) input read and split once per 128-row panel instead of once
    per 128-column tile); otherwise fu_linear.  out: the (E, n_k) result array, or None."""
    if out is None:
        out = torch.empty(A.shape[0], W.shape[0], device=A.device, dtype=torch.float32)
    if W2 is not None and _lib.get_matmul_mode() == _lib.MATMUL_SPLIT_F16:
        return gemm_resident(A, W2, W.shape[0], bias, out)
    return _gemm(A, W, bias, out)


class RadialBank(torch.nn.Module):
    """Frozen bank of G radial MLPs sharing the edge features.

    mlps: list of (W1 (C, B+2C), b1, gamma1, beta1, W2 (C, C), b2, gamma2, beta2, W3 (n_k, C), b3),
    one per block in the order their outputs are returned."""

    def __init__(self, mlps, W_src: torch.Tensor, W_tgt: torch.Tensor, B: int, eps: float = LN_EPS,
                 dtype=torch.float32):
        super().__init__()
        C = mlps[0][4].shape[0]
        self.G, self.C, self.B, self.eps = len(mlps), C, B, eps
        f64 = torch.float64
        W1g = torch.cat([m[0][:, :B] for m in mlps], 0)                                         # (G*C, B)
        tab_src = torch.cat([W_src.to(f64) @ m[0][:, B:B + C].to(f64).t() for m in mlps], 1)  # (100, G*C)
        tab_tgt = torch.cat([W_tgt.to(f64) @ m[0][:, B + C:].to(f64).t() for m in mlps], 1)
        reg = lambda n, t: self.register_buffer(n, t.detach().to(dtype).contiguous())
        reg("W1g", W1g)
        reg("W1g_t", W1g.t())
        reg("tab_src", tab_src)
        reg("tab_tgt", tab_tgt)
        reg("b1", torch.cat([m[1] for m in mlps]))
        reg("gamma1", torch.cat([m[2] for m in mlps]))
        reg("beta1", torch.cat([m[3] for m in mlps]))
        reg("W2", torch.stack([m[4] for m in mlps]))                 # (G, C, C)
        reg("W2_t", torch.stack([m[4].t() for m in mlps]))
        reg("b2", torch.cat([m[5] for m in mlps]))
        reg("gamma2", torch.cat([m[6] for m in mlps]))
        reg("beta2", torch.cat([m[7] for m in mlps]))
        for k, m in enumerate(mlps):
            reg(f"W3_{k}", m[8])
            reg(f"W3_{k}_t", m[8].t())
            reg(f"b3_{k}", m[9])

    # The output layers' GEMMs may run on a side stream (RadialOutputs), but every array they
    # write is allocated on the caller's stream and every array they read stays referenced
    # until the caller's stream waits for them: a tensor that crossed streams otherwise makes
    # the caching allocator hold its block until the other stream's events complete, and with
    # the host enqueueing steps ahead of the GPU (an MD loop without host reads) an earlier
    # side-stream version grew the reserve from 31 to 230 GB on the 8,192-atom Fe cell.

    def _split(self, name: str, ok):
        """linear_weight_split of buffer `name`, built on first use on its device (None when `ok`
        rejects its K).  Weights are frozen."""
        W = getattr(self, name)
        if not ok(W.shape[1]):
            return None
        cache = self.__dict__.setdefault("_weight_splits", {})
        if name not in cache or cache[name].device != W.device:
            cache[name] = linear_weight_split(W)
        return cache[name]

    def out_split(self, k: int):
        """Output layer k's weight pre-split for fu_linear_resident (None outside its K range)."""
        return self._split(f"W3_{k}", resident_ok)

    def out_t_split(self, k: int):
        """Output layer k's transposed weight pre-split for its input-gradient GEMM."""
        return self._split(f"W3_{k}_t", lambda K: K % 16 == 0)

    def gather_split(self, k: int, layout: int, lmax: int = 2):
        """(W2p, b3p): output layer k's weight with its rows in the column order of the fused
        kernel (lmax 2: ops/gather.radial_gather_perm for `layout`; lmax 3, 4:
        ops/lmax.radial_gather_lmax_perm), pre-split, and its bias in that order; built on first
        use on the weight's device (weights are frozen)."""
        W, b = getattr(self, f"W3_{k}"), getattr(self, f"b3_{k}")
        cache = self.__dict__.setdefault("_gather_splits", {})
        key = (k, int(layout), int(lmax))
        if key not in cache or cache[key][0].device != W.device:
            if lmax == 2:
                from .gather import radial_gather_perm
                perm = radial_gather_perm(self.C, layout)
            else:
                from .lmax import radial_gather_lmax_perm
                perm = radial_gather_lmax_perm(self.C, lmax)
            perm = perm.to(W.device)
            cache[key] = (linear_weight_split(W[perm].contiguous()), b[perm].contiguous())
        return cache[key]

    def gather_ok(self, k: int, lmax: int = 2) -> bool:
        """Whether block k's output layer can run fused with the gather (fu_radial_gather_fwd,
        lmax 2; fu_radial_gather_fwd_lmax, lmax 3, 4): C = 128 and a 6 lmax C-wide output, in the
        split-fp16 mode (the mode whose output GEMM, fu_linear_resident, the fused kernel's
        products equal bit for bit)."""
        W = getattr(self, f"W3_{k}")
        return (self.C == 128 and lmax in (2, 3, 4) and tuple(W.shape) == (6 * lmax * self.C, self.C)
                and _lib.get_matmul_mode() == _lib.MATMUL_SPLIT_F16)

    def forward(self, gauss, Z, idx_i, idx_j, with_sources: bool = False, lazy: bool = False):
        """gauss (E, B) -> tuple of G radial outputs (E, n_k).

        The trunk (first two layers of all MLPs) is one autograd node; each block's output
        layer is its own node, whose backward writes its input gradient straight into the
        trunk's gradient buffer.  with_sources: also return, per block, (h2_k, W3_k, b3_k), from
        which a consumer can recompute the output bit for bit (source(...)) instead of keeping
        it for its backward.  lazy: return the RadialOutputs instead, which create each block's
        output node when the block asks for it."""
        holder = _GradHolder()
        h2s = _RadialTrunkFn.apply(gauss, Z, idx_i, idx_j, self, holder)
        lo = RadialOutputs(self, h2s, holder)
        if lazy:
            return lo
        outs = tuple(lo.get(k) for k in range(self.G))
        srcs = tuple(lo.source(k) for k in range(self.G))
        return (outs, srcs) if with_sources else outs


class RadialOutputs:
    """The radial bank's block outputs, made on demand.  get(k) creates block k's output node
    and returns its output; creating it just before block k runs puts its backward right after
    that block's in the autograd engine's order (later-created nodes first), so the output
    layer's input gradient is formed while the next block's backward runs (the backward
    launches it on the device's side stream, ops/_lib.side_stream) instead of after all of
    them, and its (E, n_k) output gradient is released a block later instead of at the end.
    prelaunch(k) queues block k's output GEMM early on the side stream, into an array
    allocated on the current stream, so that it runs beside the previous block's node-side
    work (small GEMMs on 8,192 rows that leave most CUs idle); get(k) then waits for it."""

    def __init__(self, bank, h2s, holder):
        self.bank, self.h2s, self.holder = bank, h2s, holder
        self._pre = {}
        self._made = 0

    def _w(self, k):
        b = self.bank
        return getattr(b, f"W3_{k}"), getattr(b, f"b3_{k}"), getattr(b, f"W3_{k}_t"), b.out_split(k), b.out_t_split(k)

    def source(self, k: int):
        """(h2_k, W3_k, b3_k, split W3_k): recompute_output(source(k)) equals get(k) bit for bit."""
        W, b, _, W2, _ = self._w(k)
        return self.h2s[k].detach(), W, b, W2

    def prelaunch(self, k: int) -> None:
        if k >= self.bank.G or k in self._pre:
            return
        h2k = self.h2s[k]
        side = _lib.side_stream(h2k.device)
        if side is None:
            return
        W, b, _, W2, _ = self._w(k)
        out = torch.empty(h2k.shape[0], W.shape[0], device=h2k.device, dtype=torch.float32)
        with _lib.on_side(side):
            _out_gemm(h2k, W, b, W2, out)
        self._pre[k] = (out, side)

    def get_with_gather(self, k: int, x_in, idx_i, idx_j, wigner, csd_emb, batch, layout, lmax=2, wig_ext=None):
        """Block k's output together with the gather's (X_m0, X_m1, X_m2) of node features x_in,
        from one kernel (fu_radial_gather_fwd, or fu_radial_gather_fwd_lmax with the degree-3/4
        Wigner rows wig_ext for lmax 3, 4; bank.gather_ok(k, lmax) must hold).  The output node
        is the one get(k) makes (same backward); the X arrays carry no autograd history: the
        consumer's gather backward (ops/gating.EdgeBlock) returns the gradients of x_in, wigner,
        wig_ext and the output."""
        W, b, Wt, W2, W2t = self._w(k)
        W2p, b3p = self.bank.gather_split(k, layout, lmax)
        rq = _lib.require
        h2k = self.h2s[k].detach()
        xs = (rq(x_in.detach(), torch.float32, "x_in"), rq(idx_i, torch.int64, "idx_i"),
              rq(idx_j, torch.int64, "idx_j"), rq(wigner.detach(), torch.float32, "wigner"))
        nodes = (rq(csd_emb, torch.float32, "csd_emb"), rq(batch, torch.int64, "batch"))
        if lmax == 2:
            from .gather import radial_gather_fwd
            rad, *X = radial_gather_fwd(h2k, W2p, b3p, *xs, *nodes, layout)
        else:
            from .lmax import radial_gather_lmax_fwd
            ext = rq(wig_ext.detach(), torch.float32, "wig_ext")
            rad, *X = radial_gather_lmax_fwd(h2k, W2p, b3p, *xs, ext, *nodes, lmax)
        out = _RadialOutFn.apply(self.h2s[k], W, b, Wt, self.holder, k, W2, W2t, rad)
        self._made += 1
        if self._made == self.bank.G:
            self.holder.ln = None
        # a list, so that the consumer can drop each array once its GEMM has read it
        return out, X

    def get(self, k: int) -> torch.Tensor:
        W, b, Wt, W2, W2t = self._w(k)
        pre = self._pre.pop(k, None)
        if pre is not None:
            _lib.join(pre[1])
        out = _RadialOutFn.apply(self.h2s[k], W, b, Wt, self.holder, k, W2, W2t, None if pre is None else pre[0])
        self._made += 1
        if self._made == self.bank.G:
            self.holder.ln = None   # every output node holds what it needs
        return out


def recompute_output(src) -> torch.Tensor:
    """A block's radial output from its (h2_k, W3_k, b3_k, split W3_k) source: the forward's GEMM
    on the same operands, so bitwise the tensor the bank returned."""
    h2k, W, b, W2 = src
    return _out_gemm(h2k, W, b, W2)


class _GradHolder:
    """The (E, G*C) gradient buffer of the trunk: allocated by the first output-layer backward,
    filled slice by slice by the blocks' output-layer backwards and released by the trunk
    backward that consumes it (the holder outlives the backward inside the autograd graph,
    which the returned outputs keep referenced, so it must not keep device memory).

    At C = 128 the slices hold the gradient of the second hidden layer's LayerNorm input
    (each output-layer backward applies that layer's LayerNorm-SiLU backward for its group in
    the GEMM epilogue); otherwise the gradient of the trunk outputs.  `ln` carries the
    LayerNorm operands (p2, mean, rstd, gamma, beta, G) from the trunk's forward to the output
    layers' forwards only."""

    def __init__(self):
        self.g = None
        self.shape = None
        self.device = None
        self.ln = None
        self.side = None      # stream of the output-layer backward in flight, if any
        self.pending = ()     # the tensors it reads, kept alive until settle()

    def settle(self) -> None:
        """Make the current stream wait for the output-layer backward queued on the side stream
        and release the tensors it read."""
        if self.side is not None:
            _lib.join(self.side)
        self.side, self.pending = None, ()

    def buffer(self) -> torch.Tensor:
        if self.g is None:
            if self.shape is None:
                raise _lib.FlashUMAError("radial bank: backward through an output built without input gradients")
            self.g = torch.empty(self.shape, device=self.device, dtype=torch.float32)
        return self.g


class _RadialTrunkFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, gauss, Z, idx_i, idx_j, bank, holder):
        gauss = _lib.require(gauss, torch.float32, "gauss")
        Z = _lib.require(Z, torch.int64, "Z")
        idx_i = _lib.require(idx_i, torch.int64, "idx_i")
        idx_j = _lib.require(idx_j, torch.int64, "idx_j")
        E, G, C = gauss.shape[0], bank.G, bank.C
        dev = gauss.device
        if gauss.shape[1] != bank.B:
            raise _lib.FlashUMAError(f"radial bank: expected {bank.B} Gaussians per edge, got {gauss.shape[1]}")
        # each hidden layer is one kernel at C = 128: the GEMM's epilogue applies the
        # LayerNorm-SiLU (the first layer's (E, G*C) product is never stored)
        h1, m1, r1 = _layer1_fwd(gauss, bank, Z, idx_i, idx_j)
        h2, m2, r2, p2 = _layer2_fwd(h1, bank)
        del h1
        # the trunk gradient buffer is allocated by the first output-layer backward, not here:
        # it is not needed before the backward, and the forward's end is a memory peak
        holder.shape = tuple(p2.shape) if ctx.needs_input_grad[0] else None
        holder.device = p2.device
        ctx.dgrad_fused = C == LN_FUSED_C
        # an output without a gradient arrives as None (not a materialised zero tensor)
        ctx.set_materialize_grads(False)
        holder.ln = (p2, m2, r2, bank.gamma2, bank.beta2, G) if ctx.dgrad_fused else None
        # the first layer's product (E, G*C) is not kept: the backward recomputes it from the
        # (E, B) Gaussians with the K = B GEMM (10x fewer bytes held through the step)
        ctx.save_for_backward(gauss, m1, r1, p2, m2, r2, Z, idx_i, idx_j)
        ctx.bank, ctx.holder = bank, holder
        return tuple(h2[:, k * C:(k + 1) * C] for k in range(G))

    @staticmethod
    def backward(ctx, *g_views):
        gauss, m1, r1, p2, m2, r2, Z, idx_i, idx_j = ctx.saved_tensors
        bank, holder = ctx.bank, ctx.holder
        holder.settle()
        E, G, C = gauss.shape[0], bank.G, bank.C
        g_buf = holder.g if holder.g is not None else torch.empty_like(p2)
        holder.g = None   # a retained graph's next backward allocates a fresh buffer
        for k, gv in enumerate(g_views):
            sl = g_buf[:, k * C:(k + 1) * C]
            if gv is None:
                sl.zero_()   # zero in either meaning of the slice
            elif gv.data_ptr() != sl.data_ptr() or gv.stride() != sl.stride():
                if ctx.dgrad_fused:
                    # the views are internal to RadialBank.forward: only the output layers read them
                    raise _lib.FlashUMAError("radial bank: a trunk output has a reader besides its output layer")
                sl.copy_(gv)
        if ctx.dgrad_fused:
            g_p2 = g_buf   # the output layers' epilogues applied the LayerNorm-SiLU backward
        else:
            g_p2 = _ln_grouped_bwd(p2, None, None, None, None, None, bank.gamma2, bank.beta2, m2, r2, g_buf, G, C)
        del g_buf
        g_h1 = _batched(g_p2, bank.W2_t, None, G, C, C, torch.empty_like(g_p2))
        del g_p2
        g_p1 = _layer1_bwd(gauss, bank, Z, idx_i, idx_j, m1, r1, g_h1)
        del g_h1
        g_gauss = _gemm(g_p1, bank.W1g_t, None, torch.empty(E, bank.B, device=gauss.device, dtype=torch.float32),
                        bank._split("W1g_t", lambda K: K % 16 == 0))
        return g_gauss, None, None, None, None, None


class _RadialOutFn(torch.autograd.Function):
    """Output layer of block k: rad = h2_k W3^T + b3.  Its backward writes into the trunk's
    gradient buffer and returns that slice: at C = 128 the gradient of the LayerNorm input of
    group k of the second hidden layer (fu_linear_dgrad_ln_silu_bwd: the g_h2_k GEMM with that
    LayerNorm-SiLU backward in its epilogue, g_h2_k never stored), otherwise g_h2_k.  The
    backward runs on the device's side stream when there is one (RadialOutputs); the trunk's
    backward, which reads the buffer, waits for it.  pre: the output already computed
    (RadialOutputs.prelaunch), or None."""

    @staticmethod
    def forward(ctx, h2k, W, b, Wt, holder, k, W2=None, W2t=None, pre=None):
        ctx.holder, ctx.k, ctx.W2t = holder, k, W2t
        # (p2, mean, rstd, gamma, beta) of the trunk's forward are saved like the weight, so
        # that they are released after the backward (a plain ctx attribute would keep p2 alive
        # as long as the graph's nodes, i.e. into the next step)
        ctx.ln_groups = None if holder.ln is None else holder.ln[-1]
        ctx.save_for_backward(Wt, *(() if holder.ln is None else holder.ln[:-1]))
        return pre if pre is not None else _out_gemm(h2k, W, b, W2)

    @staticmethod
    def backward(ctx, g_rad):
        Wt, *ln = ctx.saved_tensors
        g_rad = g_rad.contiguous()
        C = Wt.shape[0]
        holder = ctx.holder
        buf = holder.buffer()
        sl = buf[:, ctx.k * C:(ctx.k + 1) * C]
        # the previous output layer's backward (a block later in the forward) is done by now;
        # its operands are released here
        holder.settle()
        side = _lib.side_stream(g_rad.device)
        with _lib.on_side(side):
            if ctx.ln_groups is None:
                _gemm(g_rad, Wt, None, sl, ctx.W2t)
            else:
                p2, m2, r2, gamma, beta = ln
                G = ctx.ln_groups
                M, K = g_rad.shape
                _lib.call("fu_linear_dgrad_ln_silu_bwd", g_rad.data_ptr(), g_rad.stride(0), Wt.data_ptr(),
                          Wt.stride(0), sl.data_ptr(), buf.stride(0), M, K, p2.data_ptr(), p2.stride(0),
                          gamma.data_ptr(), beta.data_ptr(), m2.data_ptr(), r2.data_ptr(), G, ctx.k,
                          _lib.ptr(ctx.W2t), _lib.stream_ptr(g_rad.device))
        if side is not None:
            holder.side, holder.pending = side, (g_rad, Wt, *ln)
        return sl, None, None, None, None, None, None, None, None
