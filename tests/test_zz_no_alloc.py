"""fu_balance_channels_noalloc (the allocation-free variant of fu_balance_channels, with its
corrections in a library-owned device array) against fu_balance_channels, called through
the C-ABI: bitwise equal outputs on two calls in a row, the second with a smaller input,
and a clear error for a system x channel count beyond the built-in scratch."""
from __future__ import annotations

import ctypes

import pytest
import torch

pytestmark = pytest.mark.gpu

MAX_CORR = 65536   # FU_BALANCE_NOALLOC_MAX_CORR in include/flashuma.h


def _case(cuda, sizes, C, seed):
    g = torch.Generator().manual_seed(seed)
    batch = torch.repeat_interleave(torch.arange(len(sizes)), torch.tensor(sizes)).to(cuda)
    x = torch.randn(sum(sizes), 9, C, generator=g).to(cuda)
    target = torch.randint(-3, 4, (len(sizes),), generator=g).float().to(cuda)
    return x, batch, target


def _both(lib, x, batch, target, start, end, offset):
    from ops import _lib
    from ops.node import system_ptr
    N, K, C = x.shape
    S = target.numel()
    sys_ptr = system_ptr(batch, S)
    st = _lib.stream_ptr(x.device)
    ref = torch.empty_like(x)
    corr = torch.empty(max(S * (end - start), 1), device=x.device)
    assert lib.fu_balance_channels(x.data_ptr(), ref.data_ptr(), batch.data_ptr(), sys_ptr.data_ptr(),
                                   target.data_ptr(), ctypes.c_float(offset), corr.data_ptr(), corr.numel(), N, K, C,
                                   S, start, end, st) == 0
    out = torch.full_like(x, float("nan"))
    rc = lib.fu_balance_channels_noalloc(x.data_ptr(), out.data_ptr(), batch.data_ptr(), sys_ptr.data_ptr(),
                                         target.data_ptr(), ctypes.c_float(offset), N, K, C, S, start, end, st)
    assert rc == 0, lib.fu_last_error().decode()
    torch.cuda.synchronize()
    return out, ref


def test_noalloc_balance_equals_allocating_entry_point(cuda):
    from ops import _lib
    lib = _lib.load()
    # first call: 5 systems x 96 channels; second: 2 systems x 8 channels (a smaller input, so
    # the scratch still holds the first call's larger contents)
    for sizes, C, (start, end), offset, seed in (([40, 7, 130, 1, 66], 128, (16, 112), 1.0, 0),
                                                 ([9, 20], 64, (0, 8), 0.0, 1)):
        x, batch, target = _case(cuda, sizes, C, seed)
        out, ref = _both(lib, x, batch, target, start, end, offset)
        assert torch.equal(out, ref), f"noalloc differs from fu_balance_channels (sizes {sizes})"
        sums = torch.zeros(len(sizes), end - start, dtype=torch.float64, device=cuda)
        sums.index_add_(0, batch, out[:, 0, start:end].double())
        assert (sums - (target.double() - offset)[:, None]).abs().max().item() < 1e-4


def test_noalloc_balance_rejects_oversized_input(cuda):
    from ops import _lib
    lib = _lib.load()
    S, C = MAX_CORR // 64 + 1, 64
    N = S
    x = torch.zeros(N, 9, C, device=cuda)
    out = torch.empty_like(x)
    batch = torch.arange(N, device=cuda)
    sys_ptr = torch.arange(N + 1, dtype=torch.int32, device=cuda)
    target = torch.zeros(S, device=cuda)
    rc = lib.fu_balance_channels_noalloc(x.data_ptr(), out.data_ptr(), batch.data_ptr(), sys_ptr.data_ptr(),
                                         target.data_ptr(), ctypes.c_float(0.0), N, 9, C, S, 0, 64,
                                         _lib.stream_ptr(cuda))
    assert rc == -6 and b"exceeds the built-in scratch" in lib.fu_last_error()
