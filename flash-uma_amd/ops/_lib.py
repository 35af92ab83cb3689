"""ctypes binding of libflashuma_hip.so (the C-ABI declared in include/flashuma.h).

The op modules call `lib.<entry point>(...)` through `call()`, passing raw device
pointers (`tensor.data_ptr()`), sizes and the current HIP stream.  There is no fallback:
if the library is missing, or the tensors are not on a ROCm device, the call raises.
"""
from __future__ import annotations

import contextlib
import ctypes
import os
from pathlib import Path

import torch

_PKG_DIR = Path(__file__).resolve().parent.parent
LIB_PATH = Path(os.environ.get("FLASHUMA_LIB", _PKG_DIR / "libflashuma_hip.so"))

P = ctypes.c_void_p
I64 = ctypes.c_int64
I32 = ctypes.c_int32
F32 = ctypes.c_float
SZ_P = ctypes.POINTER(ctypes.c_size_t)

# fu_version() of the library these signatures describe (major*10000 + minor*100 + patch).
ABI_VERSION = 600

# Argument types of every exported entry point, in header order.
SIGNATURES: dict[str, list] = {
    "fu_version": [],
    "fu_last_error": [],
    "fu_set_matmul_mode": [I32],
    "fu_matmul_mode": [],
    "fu_geom_fwd": [P, P, P, P, P, P, P, P, P, I64, P, P, I64, I64, I32, I32, F32, F32, P],
    "fu_geom_bwd": [P, P, P, P, P, P, I64, P, P, P, I64, I64, I32, F32, F32, P],
    "fu_edge_vec_reduce": [P, P, P, P, P, P, I64, I64, P],
    "fu_gather_fwd": [P, P, P, P, P, P, P, P, P, P, I64, I64, I64, I32, I32, P],
    "fu_gather_bwd": [P, P, P, P, P, P, P, P, P, P, P, P, P, P, P, P, P, P, I64, I64, I64, I32, I32, I32, P],
    "fu_gating_fwd": [P, P, P, P, P, P, I64, I32, I32, P],
    "fu_gating_bwd": [P, P, P, P, P, P, P, P, P, I64, I32, I32, P],
    "fu_scatter_fwd": [P, P, P, P, P, P, P, P, P, I64, I64, I32, P],
    "fu_scatter_bwd": [P, P, P, P, P, P, P, P, P, P, P, P, I64, I64, I32, I32, P],
    "fu_init_scatter_fwd": [P, P, P, P, P, P, P, P, P, P, I64, I64, I64, I64, I32, P],
    "fu_init_scatter_bwd": [P, P, P, P, P, P, P, P, I64, I64, I32, I32, P],
    "fu_ln_silu_fwd": [P, P, P, P, P, P, I64, I32, F32, P],
    "fu_ln_silu_bwd": [P, P, P, P, P, P, P, I64, I32, P],
    "fu_ln_silu_grouped_fwd": [P, I64, P, P, I64, P, P, P, P, P, P, P, I64, P, P, I64, I32, I32, F32, P],
    "fu_ln_silu_grouped_bwd": [P, I64, P, P, I64, P, P, P, P, P, P, P, P, P, I64, P, I64, I64, I32, I32, P],
    "fu_linear": [P, I64, P, I64, P, P, I64, I64, I32, I32, P, P],
    "fu_linear_batched": [P, I64, I64, P, I64, I64, P, I64, I32, P, I64, I64, P, I64, I64, I64, I32, I32, I32, P],
    "fu_complex_linear": [P, P, I64, P, P, I64, P, P, P, I64, I64, I32, I32, P],
    "fu_complex_weight_split_bytes": [I32, I32],
    "fu_complex_weight_split": [P, P, I64, I32, I32, P, P],
    "fu_linear_weight_split_bytes": [I32, I32],
    "fu_linear_weight_split": [P, I64, I32, I32, P, P],
    "fu_linear_resident": [P, I64, P, P, P, I64, I64, I32, I32, P],
    "fu_radial_gather_fwd": [P, I64, P, P, P, P, P, P, P, P, P, P, P, P, I64, I64, I64, I32, I32, I32, P],
    "fu_radial_gather_perm": [I32, I32, P],
    "fu_radial_gather_fwd_lmax": [P, I64, P, P, P, P, P, P, P, P, P, P, P, P, P, I64, I64, I64, I32, I32, I32, P],
    "fu_radial_gather_perm_lmax": [I32, I32, P],
    "fu_linear_gate": [P, I64, P, I64, P, P, I64, P, I64, P, I64, I64, I32, I32, I32, P, P],
    "fu_gather_linear_gate": [P, P, P, P, P, P, P, P, I64, P, P, I64, P, I64, I64, I32, P],
    "fu_complex_linear_gate": [P, P, I64, P, P, I64, P, P, P, I64, P, P, I64, P, I64, I32, I32, I64, I32, I32, P],
    "fu_linear_gate_bwd": [P, I64, P, I64, P, I64, P, I64, P, I64, P, I64, I64, I32, I32, I32, P, P],
    "fu_linear_ln_silu": [P, I64, I64, P, I64, I64, P, I64, I32, P, I64, I64, P, I64, I64, I64, I32, I32, I32,
                          P, P, I64, P, P, P, P, P, P, P, P, I32, F32, P],
    "fu_linear_ln_silu_bwd": [P, I64, P, I64, P, I64, I64, I32, I32, P, I64, P, P, I64, P, P, P, P, P, P, P, P,
                              I32, P],
    "fu_linear_dgrad_ln_silu_bwd": [P, I64, P, I64, P, I64, I64, I32, P, I64, P, P, P, P, I32, I32, P, P],
    "fu_complex_linear_gate_bwd": [P, P, I64, P, P, I64, P, P, P, I64, P, P, I64, P, I64, I32, I32, P, I64, I64, I32, I32, P],
    "fu_rms_norm_sh_fwd": [P, P, P, P, P, I64, I32, I32, F32, P],
    "fu_rms_norm_sh_bwd": [P, P, P, P, P, P, I64, I32, I32, P],
    "fu_gate_act_fwd": [P, P, P, I64, I32, I32, P],
    "fu_gate_act_bwd": [P, P, P, P, P, I64, I32, I32, P],
    "fu_balance_channels": [P, P, P, P, P, F32, P, I64, I64, I32, I32, I32, I32, I32, P],
    "fu_balance_channels_noalloc": [P, P, P, P, P, F32, I64, I32, I32, I32, I32, I32, P],
    "fu_gather_rows": [P, P, P, I64, I32, P],
    "fu_scatter_rows": [P, P, P, I64, I32, P],
    "fu_edge_shifts": [P, P, P, P, I64, P],
    "fu_outer_sum3": [P, P, P, P, P, I64, I64, P],
    "fu_morton_keys": [P, P, P, I64, P],
    "fu_sort_pairs_i64": [P, P, P, P, I64, I32, I32, P, SZ_P, P],
    "fu_invert_perm": [P, P, I64, P],
    "fu_take_i64": [P, I64, P, P, I64, P],
    "fu_csr_row_ptr": [P, I64, P, I64, P],
    "fu_narrow_i64_i32": [P, P, I64, P],
    "fu_nlist_bin": [P, I64, P, P, P, P, P, P, P, P],
    "fu_nlist_search": [P, P, P, P, P, I64, P, P, P, P, P, ctypes.c_double, I32, P, P, P, P, P],
    "fu_nlist_scan": [P, P, I64, P],
    "fu_nlist_emit": [P, P, P, P, I64, I32, P, P, I64, P],
    "fu_wigner_ext_width": [I32],
    "fu_wigner_ext_fwd": [P, P, I64, I32, P],
    "fu_wigner_ext_bwd": [P, P, P, I64, I32, P],
    "fu_gather_fwd_lmax": [P, P, P, P, P, P, P, P, P, P, P, P, P, P, P, I64, I64, I64, I32, I32, P],
    "fu_gather_bwd_lmax": [P, P, P, P, P, P, P, P, P, P, P, P, P, P, P, P, P, P, I64, I64, I64, I32, I32, I32, P],
    "fu_scatter_fwd_lmax": [P, P, P, P, P, P, P, P, P, P, I64, I64, I32, I32, P],
    "fu_scatter_bwd_lmax": [P, P, P, P, P, P, P, P, P, P, P, P, P, P, I64, I64, I32, I32, I32, P],
    "fu_init_scatter_fwd_lmax": [P, P, P, P, P, P, P, P, P, P, P, I64, I64, I64, I64, I32, I32, P],
    "fu_init_scatter_bwd_lmax": [P, P, P, P, P, P, P, P, P, P, I64, I64, I32, I32, I32, P],
    "fu_gating_fwd_lmax": [P, P, P, P, P, P, I64, I32, I32, P],
    "fu_gating_bwd_lmax": [P, P, P, P, P, P, P, P, P, I64, I32, I32, P],
}

_lib: ctypes.CDLL | None = None


class FlashUMAError(RuntimeError):
    """A C-ABI entry point returned a negative status."""


def load() -> ctypes.CDLL:
    """Load the shared library once and attach the argument types of every entry point."""
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        raise FlashUMAError(
            f"{LIB_PATH} is missing: build it first (python flash-uma_amd/build_lib.py or "
            "__graft_entry__.build()); there is no non-HIP fallback")
    lib = ctypes.CDLL(str(LIB_PATH))
    lib.fu_version.restype = ctypes.c_int
    if lib.fu_version() != ABI_VERSION:
        raise FlashUMAError(f"{LIB_PATH} has ABI version {lib.fu_version()}, these bindings expect "
                            f"{ABI_VERSION}: rebuild the library")
    for name, argtypes in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.argtypes = argtypes
        fn.restype = (ctypes.c_char_p if name == "fu_last_error" else
                      ctypes.c_int64 if name.endswith("_bytes") else ctypes.c_int)
    _lib = lib
    return lib


def exported_symbols() -> list[str]:
    return list(SIGNATURES)


def stream_ptr(device: torch.device | None = None) -> int:
    """hipStream_t of torch's current stream on `device`."""
    return torch.cuda.current_stream(device).cuda_stream


class KernelProfiler:
    """Brackets selected entry points with HIP events on the stream they launch on (torch's
    current stream, the one every op passes to the library) and keeps (name, args, start,
    end) per call; durations are read after a synchronisation."""

    def __init__(self, names=None):
        self.names = set(names) if names else None
        self.records: list = []

    def wants(self, name: str) -> bool:
        return self.names is None or name in self.names

    def durations(self):
        """[(name, args, milliseconds)] of all recorded calls (synchronises first)."""
        torch.cuda.synchronize()
        return [(n, a, s.elapsed_time(e)) for n, a, s, e in self.records]


_profiler: KernelProfiler | None = None


def set_profiler(profiler: KernelProfiler | None) -> None:
    global _profiler
    _profiler = profiler


def call(name: str, *args) -> None:
    """Invoke entry point `name`; raise FlashUMAError with the library message on failure."""
    lib = load()
    prof = _profiler
    if prof is not None and prof.wants(name):
        start = torch.cuda.Event(enable_timing=True)
        end = torch.cuda.Event(enable_timing=True)
        start.record()
        status = getattr(lib, name)(*args)
        end.record()
        prof.records.append((name, args, start, end))
    else:
        status = getattr(lib, name)(*args)
    if status != 0:
        msg = lib.fu_last_error().decode(errors="replace")
        raise FlashUMAError(f"{name} failed with status {status}: {msg}")


# Independent library calls of one SO(2) convolution (ops/gating.py) run on a second stream of
# the device, so that each kernel's tail overlaps the next one's start.  Off under graph
# capture and while a KernelProfiler records (its per-call events would time overlapped
# kernels); set_overlap(False) turns it off.
_overlap = True
_side_streams: dict = {}


def set_overlap(on: bool) -> None:
    global _overlap
    _overlap = bool(on)


def side_stream(device: torch.device) -> torch.cuda.Stream | None:
    """The device's second stream (default priority) for calls independent of the work queued
    next on the current stream, or None when they should stay on the current stream."""
    if not _overlap or _profiler is not None or torch.cuda.is_current_stream_capturing():
        return None
    idx = torch.device(device).index
    idx = torch.cuda.current_device() if idx is None else idx
    s = _side_streams.get(idx)
    if s is None:
        s = _side_streams[idx] = torch.cuda.Stream(device=idx)
    return s


@contextlib.contextmanager
def on_side(side: torch.cuda.Stream | None):
    """Queue the enclosed calls on `side` after everything queued so far on the current stream
    (no-op for None).  The caller allocates their outputs before, keeps every tensor they touch
    alive until join(side), and allocates nothing inside (the side stream has no pool of its
    own then, and no tensor needs record_stream)."""
    if side is None:
        yield
        return
    side.wait_stream(torch.cuda.current_stream(side.device))
    with torch.cuda.stream(side):
        yield


def join(side: torch.cuda.Stream | None) -> None:
    """Make the current stream wait for the calls queued on `side`."""
    if side is not None:
        torch.cuda.current_stream(side.device).wait_stream(side)


MATMUL_SPLIT_BF16 = 0  # fp32 operands split exactly into three bf16 planes, six MFMA products
MATMUL_FP32 = 1        # v_mfma_f32_32x32x2_f32
MATMUL_SPLIT_F16 = 2   # power-of-two row scales, two fp16 planes, three MFMA products
MATMUL_MODES = {"split_bf16": MATMUL_SPLIT_BF16, "fp32": MATMUL_FP32, "split_f16": MATMUL_SPLIT_F16}


def get_matmul_mode() -> int:
    """Matrix-core mode of the library's fp32 contractions (one of MATMUL_MODES)."""
    return load().fu_matmul_mode()


def set_matmul_mode(mode: int) -> None:
    """Select the matrix-core mode of every later fp32 contraction (process-wide)."""
    call("fu_set_matmul_mode", int(mode))


@contextlib.contextmanager
def matmul_mode(mode: int):
    """Run the enclosed launches in matrix-core `mode`; restores the previous mode after."""
    prev = get_matmul_mode()
    set_matmul_mode(mode)
    try:
        yield
    finally:
        set_matmul_mode(prev)


def ptr(t: torch.Tensor | None) -> int | None:
    """Device address of a tensor (None for an absent optional operand)."""
    if t is None:
        return None
    if not t.is_cuda:
        raise FlashUMAError("FlashUMA kernels need tensors on a ROCm GPU device; got a CPU tensor")
    return t.data_ptr()


def require(t: torch.Tensor, dtype: torch.dtype, name: str) -> torch.Tensor:
    """Return `t` as a contiguous tensor of `dtype` on its GPU (copying only if needed)."""
    if not t.is_cuda:
        raise FlashUMAError(f"{name}: FlashUMA kernels need a ROCm GPU tensor, got device {t.device}")
    if t.dtype != dtype:
        t = t.to(dtype)
    return t.contiguous()
