"""The C-ABI library loads, exports every symbol include/flashuma.h declares, and rejects bad
arguments with the documented status codes before touching the GPU (no compute calls)."""
import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "flashuma.h")


def header_symbols():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(fu_[a-z0-9_]+)\s*\(", text)))


def test_header_matches_binding():
    from ops import _lib
    assert header_symbols() == sorted(_lib.exported_symbols())


def test_library_exports_all_symbols():
    from ops import _lib
    lib = _lib.load()
    for name in header_symbols():
        assert hasattr(lib, name), f"{name} not exported"
    assert lib.fu_version() == _lib.ABI_VERSION


def _status(name, *args):
    from ops import _lib
    lib = _lib.load()
    return getattr(lib, name)(*args), lib.fu_last_error().decode()


def test_error_codes():
    # FU_ERR_SHAPE = -1, UNSUPPORTED = -2, ALIGN = -3, NULL = -5, WORKSPACE = -6
    st, msg = _status("fu_gating_fwd", None, None, None, None, None, None, 10, 6, 0, None)
    assert st == -2 and "multiple of 4" in msg
    st, msg = _status("fu_gating_fwd", None, None, None, None, None, None, 10, 128, 0, None)
    assert st == -5
    st, _ = _status("fu_gating_fwd", None, None, None, None, None, None, -1, 128, 0, None)
    assert st == -1
    st, msg = _status("fu_linear", 16, 8, 16, 8, None, 16, 8, 10, 8, 6, None, None)
    assert st == -2 and "multiples of 4" in msg
    st, _ = _status("fu_linear", 3, 8, 16, 8, None, 16, 8, 10, 8, 8, None, None)
    assert st == -3
    st, _ = _status("fu_gather_fwd", *([None] * 10), 5, 5, 1, 96, 0, None)
    assert st == -2
    st, msg = _status("fu_gather_fwd", *([None] * 10), 5, 5, 1, 128, 2, None)
    assert st == -2 and "layout" in msg
    st, _ = _status("fu_ln_silu_fwd", *([None] * 6), 4, 100, ctypes.c_float(1e-7), None)
    assert st == -2
    ws = ctypes.c_size_t(0)
    st, _ = _status("fu_sort_pairs_i64", None, None, None, None, 10, 8, 8, None, ctypes.byref(ws), None)
    assert st == -1
    st, _ = _status("fu_geom_fwd", *([None] * 9), 4, None, None, 10, 5, 8, 4, ctypes.c_float(6.0),
                    ctypes.c_float(-1.0), None)
    assert st == -1  # ld_xe smaller than the embedding row width
    st, _ = _status("fu_scatter_fwd", *([None] * 9), 3, 3, 192, None)
    assert st == -2
    # LayerNorm-SiLU GEMMs: whole 128-column groups, one per N-tile or per batch
    st, msg = _status("fu_linear_ln_silu", None, 64, 0, None, 64, 0, None, 0, 0, None, 600, 0, None, 0, 0, 0, 600,
                      64, 1, *([None] * 2), 0, *([None] * 8), 5, ctypes.c_float(1e-5), None)
    assert st == -2 and "groups of 128" in msg
    st, msg = _status("fu_linear_ln_silu", None, 640, 128, None, 128, 0, None, 0, 0, None, 640, 128, None, 0, 0, 0,
                      128, 128, 4, *([None] * 2), 0, *([None] * 8), 5, ctypes.c_float(1e-5), None)
    assert st == -2 and "groups of 128" in msg
    # conv1 m = 0 with its operand gathered: C a multiple of 64, strides of whole rows
    st, msg = _status("fu_gather_linear_gate", *([None] * 7), None, 576, None, None, 480, None, 288, 0, 96, None)
    assert st == -2 and "C=96" in msg
    st, msg = _status("fu_gather_linear_gate", *([None] * 7), None, 700, None, None, 640, None, 384, 0, 128, None)
    assert st == -1 and "ldw" in msg
    # the output-layer gradient GEMM with the LayerNorm backward: one group of G
    st, msg = _status("fu_linear_dgrad_ln_silu_bwd", None, 64, None, 64, None, 640, 0, 64, None, 640, *([None] * 4),
                      5, 5, None, None)
    assert st == -1 and "group=5" in msg
    st, msg = _status("fu_linear_dgrad_ln_silu_bwd", None, 64, None, 64, None, 640, 0, 64, None, 512, *([None] * 4),
                      5, 0, None, None)
    assert st == -1 and "ldx=512" in msg
    # accumulate flags: bit 0 (wigner rows), bit 1 (env); nothing else
    for name, args in (("fu_scatter_bwd", (*([None] * 12), 0, 5, 128)),
                       ("fu_init_scatter_bwd", (*([None] * 8), 0, 5, 128)),
                       ("fu_gather_bwd", (*([None] * 18), 0, 0, 1, 128, 1)),
                       ("fu_scatter_bwd_lmax", (*([None] * 14), 0, 5, 128, 4)),
                       ("fu_init_scatter_bwd_lmax", (*([None] * 10), 0, 5, 128, 4)),
                       ("fu_gather_bwd_lmax", (*([None] * 18), 0, 0, 1, 128, 4))):
        for acc, want in ((3, 0), (4, -2), (-1, -2)):
            st, msg = _status(name, *args, acc, None)
            assert st == want, (name, acc, msg)


def test_zero_sized_calls_are_no_ops():
    # E == 0 returns before any launch
    st, _ = _status("fu_gating_fwd", 16, 16, 16, 16, 16, 16, 0, 128, 0, None)
    assert st == 0
    st, _ = _status("fu_linear", 16, 8, 16, 8, None, 16, 8, 0, 8, 8, None, None)
    assert st == 0


def test_zero_rows_accept_empty_arrays():
    """A graph without edges hands the per-edge entry points empty torch tensors, whose
    storage pointer is NULL: with zero rows every such call is a no-op returning FU_OK, while
    the shape checks still apply."""
    f = ctypes.c_float
    calls = {
        "fu_geom_fwd": (*([None] * 9), 8, None, None, 0, 5, 8, 0, f(6.0), f(-1.0), None),
        "fu_geom_bwd": (*([None] * 6), 8, None, None, None, 0, 5, 8, f(6.0), f(-1.0), None),
        "fu_gating_fwd": (*([None] * 6), 0, 128, 1, None),
        "fu_gating_bwd": (*([None] * 9), 0, 128, 1, None),
        "fu_linear": (None, 16, None, 16, None, None, 16, 0, 16, 16, None, None),
        "fu_linear_batched": (None, 640, 128, None, 128, 16384, None, 128, 5, None, 0, 0, None, 640, 128, 0, 128,
                              128, 5, None),
        "fu_linear_gate": (None, 768, None, 768, None, None, 640, None, 384, None, 256, 0, 128, 768, 2, None, None),
        "fu_linear_gate_bwd": (None, 384, None, 384, None, 640, None, 256, None, 128, None, 640, 0, 128, 384, 2,
                               None, None),
        "fu_complex_linear": (None, None, 256, None, None, 256, None, None, None, 128, 0, 128, 256, None),
        "fu_complex_linear_gate": (None, None, 256, None, None, 256, None, None, None, 128, None, None, 128, None,
                                   640, 0, 128, 0, 128, 256, None),
        "fu_complex_linear_gate_bwd": (None, None, 256, None, None, 256, None, None, None, 128, None, None, 128,
                                       None, 640, 0, 128, None, 128, 0, 128, 256, None),
        # element tables present (a weight), per-edge element ids empty
        "fu_ln_silu_grouped_fwd": (None, 640, 16, 16, 128, 16, None, None, None, None, None, None, 640, None, None, 0,
                                   5, 128, f(1e-7), None),
        "fu_ln_silu_grouped_bwd": (None, 640, 16, 16, 128, 16, None, None, None, None, None, None, None, None, 640,
                                   None, 640, 0, 5, 128, None),
        "fu_scatter_bwd": (*([None] * 12), 0, 5, 128, 0, None),
        "fu_init_scatter_bwd": (*([None] * 8), 0, 5, 128, 0, None),
        "fu_gather_fwd": (*([None] * 10), 0, 5, 1, 128, 1, None),
        "fu_edge_shifts": (None, None, None, None, 0, None),
        "fu_wigner_ext_fwd": (None, None, 0, 4, None),
        "fu_wigner_ext_bwd": (None, None, None, 0, 4, None),
        "fu_gating_fwd_lmax": (*([None] * 6), 0, 128, 4, None),
        "fu_scatter_bwd_lmax": (*([None] * 14), 0, 5, 128, 4, 0, None),
        "fu_linear_ln_silu": (None, 64, 0, None, 64, 0, None, 0, 0, None, 640, 0, None, 0, 0, 0, 640, 64, 1,
                              *([None] * 2), 0, *([None] * 8), 5, f(1e-5), None),
        "fu_linear_ln_silu_bwd": (None, 64, None, 64, None, 640, 0, 640, 64, None, 640, *([None] * 2), 0,
                                  *([None] * 8), 5, None),
        "fu_linear_dgrad_ln_silu_bwd": (None, 64, None, 64, None, 640, 0, 64, None, 640, *([None] * 4), 5, 4, None,
                                        None),
        "fu_gather_linear_gate": (*([None] * 7), None, 768, None, None, 640, None, 384, 0, 128, None),
    }
    for name, args in calls.items():
        st, msg = _status(name, *args)
        assert st == 0, (name, msg)
    # the shape checks still run with zero rows
    st, _ = _status("fu_linear", None, 16, None, 16, None, None, 16, 0, 16, 6, None, None)
    assert st == -2
    st, _ = _status("fu_complex_linear_gate", None, None, 256, None, None, 256, None, None, None, 128, None, None,
                    64, None, 640, 0, 128, 0, 128, 256, None)
    assert st == -1
    # gate columns beyond the rows of Y0
    st, _ = _status("fu_complex_linear_gate", None, None, 256, None, None, 256, None, None, None, 128, None, None,
                    128, None, 256, 0, 128, 0, 128, 256, None)
    assert st == -1


def test_product_raises_without_gpu_tensors():
    """The op layer has no CPU fallback: CPU tensors are rejected loudly."""
    import torch
    from ops import _lib
    from ops.gating import fused_gating_split
    with pytest.raises(_lib.FlashUMAError):
        fused_gating_split(torch.zeros(4, 640), torch.zeros(4, 512), torch.zeros(4, 256), 128)


@pytest.mark.parametrize("attr,value", [("lmax", 5), ("lmax", 1), ("mmax", 4)])
def test_backbone_rejects_unsupported_lmax_mmax(attr, value):
    """lmax 2, 3 and 4 are built (the reference stops at 2, wrapper.py:109-118); anything else,
    and mmax != 2, is rejected with a ValueError before any kernel runs."""
    import escn_md
    from wrapper import ZeroAllocBackbone
    bb = escn_md.eSCNMDBackbone(seed=0)
    setattr(bb, attr, value)
    with pytest.raises(ValueError, match=f"{attr}={value}"):
        ZeroAllocBackbone(bb)


def test_lmax_entry_points_reject_bad_arguments():
    """The lmax-general entry points check lmax, C and pointers on the host (no GPU needed)."""
    import ctypes
    from ops import _lib
    lib = _lib.load()
    assert lib.fu_wigner_ext_width(2) == 0 and lib.fu_wigner_ext_width(3) == 35 and lib.fu_wigner_ext_width(4) == 80
    assert lib.fu_wigner_ext_width(5) == -1
    assert lib.fu_wigner_ext_fwd(None, None, 10, 2, None) != 0      # lmax 2 needs no extension
    assert b"lmax" in lib.fu_last_error()
    assert lib.fu_gating_fwd_lmax(None, None, None, None, None, None, 10, 128, 5, None) != 0
    assert b"lmax" in lib.fu_last_error()
    assert lib.fu_scatter_fwd_lmax(None, None, None, None, None, None, None, None, None, None, 4, 8, 96, 4, None) != 0
    assert b"C=96" in lib.fu_last_error()
    assert lib.fu_gather_fwd_lmax(None, None, None, None, None, None, None, None, None, None, None, None, None, None,
                                  None, 8, 4, 1, 128, 4, None) != 0
    assert b"NULL" in lib.fu_last_error()
    # lmax 3 and 4 need the extension rows; lmax 2 accepts NULL there (checked before any launch)
    assert lib.fu_init_scatter_bwd_lmax(None, None, None, None, None, None, None, None, None, None, 0, 4, 128, 4, 0,
                                        None) == 0


def test_complex_weight_split_arguments():
    # one (32-column, 16-k) block holds 9 bf16 and 9 fp16 planes (hi, lo, lo' of P, Q, P + Q)
    # x 64 lanes x 16 B, and each 32-column block 32 column factors and 32 column flags
    # (2 x 128 B); sizes round up to whole blocks
    st, _ = _status("fu_complex_weight_split_bytes", 32, 16)
    assert st == (9 + 9) * 64 * 16 + 2 * 128
    st, _ = _status("fu_complex_weight_split_bytes", 33, 17)
    assert st == 4 * (9 + 9) * 64 * 16 + 2 * 2 * 128
    st, _ = _status("fu_complex_weight_split_bytes", 0, 16)
    assert st == -1
    st, _ = _status("fu_complex_weight_split", None, None, 16, 32, 16, None, None)
    assert st == -5
    st, msg = _status("fu_complex_weight_split", 16, 16, 8, 32, 16, 16, None)
    assert st == -1 and "ldw" in msg
    st, msg = _status("fu_complex_weight_split", 16, 16, 16, 32, 16, 8, None)
    assert st == -3 and "aligned" in msg
    # a misaligned pre-split weight is rejected before any launch
    st, msg = _status("fu_complex_linear", 16, 16, 16, 16, 16, 16, 8, 16, 16, 16, 4, 4, 16, None)
    assert st == -3 and "W3" in msg


def test_matmul_mode_rejects_unknown():
    st, msg = _status("fu_set_matmul_mode", 5)
    assert st == -2 and "mode=5" in msg
    st, _ = _status("fu_matmul_mode")
    assert st in (0, 1, 2)


def test_binding_types_match_header():
    """Every ctypes signature in ops/_lib.py has the argument count and kinds the header
    declares (pointer, int64_t, int32_t, float, double), so no argument is marshalled with
    the wrong width or register class."""
    from ops import _lib
    text = re.sub(r"/\*.*?\*/", "", open(HEADER).read(), flags=re.S)
    kinds = {"int64_t": ctypes.c_int64, "int32_t": ctypes.c_int32, "float": ctypes.c_float,
             "double": ctypes.c_double}
    checked = 0
    for m in re.finditer(r"\b(?:int|int64_t|const char\*)\s+(fu_\w+)\s*\(([^)]*)\)\s*;", text):
        name, params = m.group(1), m.group(2).strip()
        want = []
        if params and params != "void":
            for p in params.split(","):
                p = " ".join(p.split())
                if "*" in p:
                    want.append("ptr")
                else:
                    want.append(kinds[p.rsplit(" ", 1)[0].replace("const ", "")])
        got = _lib.SIGNATURES[name]
        assert len(got) == len(want), (name, len(got), len(want))
        for k, (g, w) in enumerate(zip(got, want)):
            if w == "ptr":
                assert g in (ctypes.c_void_p, _lib.SZ_P), (name, k, g)
            else:
                assert g is w, (name, k, g, w)
        checked += 1
    assert checked == len(_lib.SIGNATURES)


def test_linear_weight_split_arguments():
    # per (32-column, 16-k) block: hi, lo and lo' planes x 64 lanes x 16 B; then 32 column
    # factors and 32 column flags per block (2 x 128 B) and the 16-byte summary word
    st, _ = _status("fu_linear_weight_split_bytes", 32, 16)
    assert st == 3 * 64 * 16 + 2 * 128 + 16
    st, _ = _status("fu_linear_weight_split_bytes", 33, 768)
    assert st == 2 * 48 * 3 * 64 * 16 + 2 * 2 * 128 + 16
    for N, K in ((0, 16), (32, 8), (32, 100)):
        st, _ = _status("fu_linear_weight_split_bytes", N, K)
        assert st == -1, (N, K)
    st, _ = _status("fu_linear_weight_split", None, 16, 32, 16, None, None)
    assert st == -5
    st, msg = _status("fu_linear_weight_split", 16, 16, 32, 16, 8, None)
    assert st == -3 and "aligned" in msg
    # a misaligned W2 is rejected before any launch, by every entry point that takes one
    st, msg = _status("fu_linear", 16, 16, 16, 16, None, 16, 16, 10, 16, 16, 8, None)
    assert st == -3 and "W2" in msg
    st, msg = _status("fu_linear_gate", 16, 768, 16, 768, None, 16, 640, 16, 384, None, 256, 10, 128, 768, 2, 8,
                      None)
    assert st == -3 and "W2" in msg
    st, msg = _status("fu_linear_gate_bwd", 16, 384, 16, 384, 16, 640, 16, 256, 16, 128, 16, 640, 10, 128, 384, 2,
                      8, None)
    assert st == -3 and "W2" in msg
    st, msg = _status("fu_linear_dgrad_ln_silu_bwd", 16, 64, 16, 64, 16, 640, 10, 64, 16, 640, 16, 16, 16, 16, 5,
                      0, 8, None)
    assert st == -3 and "W2" in msg
    # the resident GEMM takes K <= 128 only
    st, msg = _status("fu_linear_resident", 16, 144, 16, None, 16, 64, 10, 64, 144, None)
    assert st == -1 and "K=144" in msg


@pytest.mark.parametrize("layout", [0, 1])
def test_radial_gather_perm(layout):
    """fu_radial_gather_perm (host only): a permutation of the 12C radial columns whose 96-column
    tiles each hold three radial blocks of one side for 32 consecutive channels, those of
    degrees 0 and 1 ((l, |m|) = (0, 0), (1, 0), (1, 1): slots 0, 1, 3) in even tiles and of
    degree 2 ((2, 0), (2, 1), (2, 2): slots 2, 4, 5) in odd ones, in the slot order of the
    gather's layout (layout 0: block 2q + side; layout 1: 6 side + q)."""
    from ops.gather import radial_gather_perm
    C = 128
    perm = radial_gather_perm(C, layout).tolist()
    assert sorted(perm) == list(range(12 * C))
    for t in range(16):
        so, cg, hq = t >> 3, (t >> 1) & 3, t & 1
        for j in range(3):
            q = ((0, 1, 3), (2, 4, 5))[hq][j]
            block = 2 * q + so if layout == 0 else 6 * so + q
            cols = perm[96 * t + 32 * j:96 * t + 32 * j + 32]
            assert cols == [block * C + 32 * cg + c for c in range(32)]
    st, msg = _status("fu_radial_gather_perm", 64, layout, None)
    assert st == -2 and "C=64" in msg
    st, msg = _status("fu_radial_gather_perm", C, 2, None)
    assert st == -2 and "layout=2" in msg
    st, msg = _status("fu_radial_gather_perm", C, layout, None)
    assert st == -5


def test_radial_gather_fwd_argument_checks():
    """Shape, layout and NULL checks of fu_radial_gather_fwd, before any launch."""
    args = lambda ldh, C, K, layout: (None, ldh, *([None] * 12), 10, 4, 1, C, K, layout, None)
    st, msg = _status("fu_radial_gather_fwd", *args(128, 64, 128, 1))
    assert st == -2 and "C=64" in msg
    st, msg = _status("fu_radial_gather_fwd", *args(128, 128, 64, 1))
    assert st == -2 and "K=64" in msg
    st, msg = _status("fu_radial_gather_fwd", *args(64, 128, 128, 1))
    assert st == -1
    st, msg = _status("fu_radial_gather_fwd", *args(128, 128, 128, 1))
    assert st == -5


@pytest.mark.parametrize("L", [3, 4])
def test_radial_gather_lmax_perm(L):
    """fu_radial_gather_perm_lmax (host only): a permutation of the 6 L C radial columns whose
    96-column tiles hold, for one side and 32 consecutive channels, the radial blocks of degrees
    0 and 1 ((l, |m|) = (0, 0), (1, 0), (1, 1)) or of one degree l >= 2 ((l, 0), (l, 1), (l, 2)),
    each block at its place in the lmax kernels' order (|m| = 0: 2l + side; 1: 2(L+1) + 2(l-1)
    + side; 2: 4L + 2 + 2(l-2) + side)."""
    from ops.lmax import radial_gather_lmax_perm
    C = 128
    perm = radial_gather_lmax_perm(C, L).tolist()
    assert sorted(perm) == list(range(6 * L * C))

    def radblk(l, am, so):
        return 2 * l + so if am == 0 else (2 * (L + 1) + 2 * (l - 1) + so if am == 1 else 4 * L + 2 + 2 * (l - 2) + so)

    for t in range(8 * L):
        g, cg, so = t % L, (t // L) % 4, t // (4 * L)
        blocks = [(0, 0), (1, 0), (1, 1)] if g == 0 else [(g + 1, 0), (g + 1, 1), (g + 1, 2)]
        for j, (l, am) in enumerate(blocks):
            cols = perm[96 * t + 32 * j:96 * t + 32 * j + 32]
            assert cols == [radblk(l, am, so) * C + 32 * cg + c for c in range(32)]
    st, msg = _status("fu_radial_gather_perm_lmax", C, 2, None)
    assert st == -2 and "lmax=2" in msg
    st, msg = _status("fu_radial_gather_perm_lmax", C, L, None)
    assert st == -5
    args = lambda C_, K_, L_: (None, 128, *([None] * 13), 10, 4, 1, C_, K_, L_, None)
    st, msg = _status("fu_radial_gather_fwd_lmax", *args(128, 128, 5))
    assert st == -2 and "lmax=5" in msg
    st, msg = _status("fu_radial_gather_fwd_lmax", *args(64, 128, L))
    assert st == -2 and "C=64" in msg
    st, msg = _status("fu_radial_gather_fwd_lmax", *args(128, 128, L))
    assert st == -5
