"""In-place sums of the per-edge gradients dE/dwigner, dE/dwig_ext and dE/denv.

Every message-passing block reads the same Wigner rows and envelope (the gather, the scatter
and the edge-degree embedding; ops/gather.py, ops/scatter.py).  Left to autograd, each block's
backward returns its own (E, 34) / (E,) gradient and autograd sums them with one add kernel
per extra reader.  With a sink, the blocks' backward kernels add their contribution to one
buffer per tensor in place (the C-ABI `accumulate` flags: bit 0 for the Wigner rows, bit 1
for the envelope), in the fixed order autograd runs them, and return no gradient for those
inputs; the Function that produced the tensor (the geometry, the Wigner extension) takes the
sum in its backward.  Autograd still runs that producer after every reader, since each
reader's node has an edge to it."""
from __future__ import annotations

import torch

WIGNER, WIG_EXT, ENV = "wigner", "wig_ext", "env"
_BIT = {WIGNER: 1, WIG_EXT: 1, ENV: 2}


def _pass_id() -> int:
    """Id of the backward pass (autograd graph task) running on this thread; -1 outside one."""
    return torch._C._current_graph_task_id()


class EdgeGradSink:
    """Accumulators of one forward pass.  `target(name, like)` hands out the buffer the next
    contribution goes to (allocated on first use, uninitialised: the first writer overwrites)
    with its accumulate bit; `take(name)` returns the sum and forgets it.  Each buffer belongs
    to the backward pass that started it: a contribution from another pass starts afresh, and
    the producer takes only its own pass's sum.  So a backward through a retained graph that
    stopped before the producer (a gradient toward an intermediate tensor) leaves nothing that
    a later backward would add onto."""

    def __init__(self):
        self._buf = {}

    def target(self, name: str, like: torch.Tensor):
        pid = _pass_id()
        entry = self._buf.get(name)
        if entry is None or entry[1] != pid:
            t = torch.empty_like(like)
            self._buf[name] = (t, pid)
            return t, 0
        return entry[0], _BIT[name]

    def take(self, name: str):
        entry = self._buf.pop(name, None)
        if entry is None or entry[1] != _pass_id():
            return None
        return entry[0]


def outputs(sink, ctx_like: dict):
    """(buffers, accumulate flags) for a backward kernel writing the gradients of the named
    tensors ({name: tensor}): from the sink when there is one, else fresh arrays (flags 0)."""
    bufs, flags, seen = {}, 0, {}
    for name, like in ctx_like.items():
        if like is None:
            bufs[name] = None
            continue
        if sink is None:
            bufs[name] = torch.empty_like(like)
        else:
            bufs[name], bit = sink.target(name, like)
            flags |= bit
            # the Wigner rows and their extension share one flag bit: both or neither started
            if seen.setdefault(_BIT[name], bit) != bit:
                raise RuntimeError("EdgeGradSink: wigner and wig_ext accumulators out of step")
    return bufs, flags


def merge(sink, name: str, incoming):
    """The producer's view of a gradient: the sink's sum plus whatever autograd delivered
    (a reader outside the sink)."""
    acc = None if sink is None else sink.take(name)
    if acc is None:
        return incoming
    return acc if incoming is None else acc + incoming
