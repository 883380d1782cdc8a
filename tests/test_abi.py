"""The C ABI library (fast_amd/lib/libfastagg_hip.so) on the CPU: it loads, exports exactly
the entry points include/fastagg.h declares, and its host-side logic (status text, K-space
width, scratch sizes, argument validation that rejects a call before any launch) behaves
as documented. No kernel is launched here."""
import ctypes
import os
import re
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "fastagg.h")
FA_OK, FA_EINVAL, FA_EUNSUPPORTED, FA_EALIGN, FA_ESCRATCH = 0, -1, -2, -3, -4


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    text = re.sub(r"//[^\n]*", "", text)
    return sorted(set(re.findall(r"\b(fa_[a-z0-9_]+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    from fast_amd import build as fb

    path = fb.lib_path()
    if not os.path.exists(path):
        fb.build_hip_library()
    return ctypes.CDLL(path)


def test_header_declares_the_path():
    names = declared_functions()
    for must in ("fa_tgat_attn_fwd_f32", "fa_tgat_attn_bwd_f32", "fa_edge_softmax_fwd_f32",
                 "fa_edge_softmax_bwd_f32", "fa_edge_scatter_sum_f32", "fa_segment_sum_f32",
                 "fa_exclusive_sum_i32", "fa_degree_count_i32", "fa_balance_mask_i32",
                 "fa_fused_attn_fwd_f32", "fa_fused_attn_bwd_f32", "fa_group_softmax_fwd_f32",
                 "fa_head_proj_f32", "fa_head_reduce_f32", "fa_head_wgrad_f32",
                 "fa_row_group_dots_f32"):
        assert must in names


def test_every_declared_symbol_is_exported(lib):
    missing = [n for n in declared_functions() if not hasattr(lib, n)]
    assert not missing, f"declared in fastagg.h but not exported: {missing}"


def test_no_undeclared_exports():
    from fast_amd import build as fb

    out = subprocess.run(["nm", "-D", "--defined-only", fb.lib_path()], capture_output=True,
                         text=True, check=True).stdout
    exported = {ln.split()[-1] for ln in out.splitlines() if " T " in ln}
    extra = sorted(n for n in exported if n.startswith("fa_") and n not in declared_functions())
    assert not extra, f"exported but not declared: {extra}"


def test_status_strings_and_version(lib):
    lib.fa_status_string.restype = ctypes.c_char_p
    for st in (FA_OK, FA_EINVAL, FA_EUNSUPPORTED, FA_EALIGN, FA_ESCRATCH):
        assert lib.fa_status_string(st)
    assert lib.fa_status_string(FA_OK) == b"success"
    assert lib.fa_status_string(-99) == b"unknown status"
    assert lib.fa_abi_version() // 100 == 5


def test_kspace_width(lib):
    lib.fa_tgat_kspace.restype = ctypes.c_int64
    k = lambda dn, de, dt: lib.fa_tgat_kspace(ctypes.c_int32(dn), ctypes.c_int32(de),
                                              ctypes.c_int32(dt))
    # node | edge | time blocks padded to 4, then the bias column padded to a float4 chunk
    assert k(100, 172, 100) == 100 + 172 + 100 + 4
    assert k(7, 5, 3) == 8 + 8 + 4 + 4
    assert k(0, 0, 0) == 4
    assert k(413, 186, 100) == 416 + 188 + 100 + 4
    assert k(-1, 0, 0) < 0


def test_scratch_sizes(lib):
    lib.fa_tgat_attn_bwd_scratch_bytes.restype = ctypes.c_size_t
    lib.fa_exclusive_sum_scratch_bytes.restype = ctypes.c_size_t
    assert lib.fa_tgat_attn_bwd_scratch_bytes(ctypes.c_int64(1000), ctypes.c_int32(0)) == 0
    small = lib.fa_tgat_attn_bwd_scratch_bytes(ctypes.c_int64(1000), ctypes.c_int32(100))
    big = lib.fa_tgat_attn_bwd_scratch_bytes(ctypes.c_int64(10 ** 7), ctypes.c_int32(100))
    assert 0 < small <= big
    assert big <= 64 << 20  # per-workgroup partials of the time gradients: bounded
    assert lib.fa_exclusive_sum_scratch_bytes(ctypes.c_int64(10 ** 6)) >= 0
    lib.fa_head_wgrad_scratch_bytes.restype = ctypes.c_size_t
    hw = lambda n, ones: lib.fa_head_wgrad_scratch_bytes(ctypes.c_int64(n), ctypes.c_int32(50),
                                                         ctypes.c_int32(376), ctypes.c_int32(2),
                                                         ctypes.c_int32(ones))
    assert hw(0, 0) == 0
    # one [heads][j(+1)][c] partial per row chunk; the chunk count is capped
    assert hw(16, 0) == 1 * 2 * 50 * 376 * 4
    assert hw(16, 1) == 1 * 2 * 51 * 376 * 4
    assert 0 < hw(132000, 1) <= 3072 * 2 * 51 * 376 * 4


class TgatGraph(ctypes.Structure):
    _fields_ = [("n_dst", ctypes.c_int64), ("n_edges", ctypes.c_int64),
                ("rowptr", ctypes.c_void_p),
                ("node_tab", ctypes.c_void_p), ("ld_node", ctypes.c_int64),
                ("n_node", ctypes.c_int64), ("dn", ctypes.c_int32), ("node_idx", ctypes.c_void_p),
                ("node_dtype", ctypes.c_int32),
                ("edge_tab", ctypes.c_void_p), ("ld_edge", ctypes.c_int64),
                ("n_edge_rows", ctypes.c_int64), ("de", ctypes.c_int32),
                ("edge_idx", ctypes.c_void_p), ("edge_dtype", ctypes.c_int32),
                ("dt", ctypes.c_void_p), ("time_w", ctypes.c_void_p), ("time_b", ctypes.c_void_p),
                ("dt_dim", ctypes.c_int32)]


def _fwd(lib, g, heads=2, qt=None, qt_rs=0, qt_hs=0, xbar=None, xbar_rs=0, xbar_hs=0,
         scores=None, stats=None):
    return lib.fa_tgat_attn_fwd_f32(ctypes.byref(g), ctypes.c_int32(heads), ctypes.c_void_p(qt),
                                    ctypes.c_int64(qt_rs), ctypes.c_int64(qt_hs),
                                    ctypes.c_float(0.2), None, ctypes.c_uint64(0),
                                    ctypes.c_float(0.0), ctypes.c_void_p(xbar),
                                    ctypes.c_int64(xbar_rs), ctypes.c_int64(xbar_hs),
                                    ctypes.c_void_p(scores), ctypes.c_void_p(stats), None)


def test_tgat_fwd_rejects_bad_arguments(lib):
    """Argument errors come back as FA_E* codes before anything touches a device."""
    assert lib.fa_tgat_attn_fwd_f32(None, 2, None, 0, 0, ctypes.c_float(0.2), None, 0,
                                    ctypes.c_float(0.0), None, 0, 0, None, None,
                                    None) == FA_EINVAL
    g = TgatGraph(n_dst=-1)
    assert _fwd(lib, g) == FA_EINVAL
    g = TgatGraph(n_dst=4, n_edges=8, rowptr=None, dn=4, ld_node=4)
    assert _fwd(lib, g) == FA_EINVAL  # missing rowptr / tables
    g = TgatGraph(n_dst=4, n_edges=8, rowptr=16, node_tab=64, ld_node=2, n_node=10, dn=4)
    assert _fwd(lib, g, qt=64) == FA_EINVAL  # leading dimension below the row width
    g = TgatGraph(n_dst=4, n_edges=8, rowptr=16, dt_dim=4)
    assert _fwd(lib, g, qt=64) == FA_EINVAL  # time encoding without dt / w / b
    g = TgatGraph(n_dst=4, n_edges=8, rowptr=16)
    assert _fwd(lib, g, heads=0, qt=64) == FA_EINVAL


def test_noalloc_backward_rejects_bad_arguments(lib):
    """The no-allocation backward checks its arguments like the scratch-taking one, before
    it looks up its device array or launches anything (no GPU needed here)."""
    f = lib.fa_tgat_attn_bwd_noalloc_f32
    none = [None] * 25
    assert f(None, ctypes.c_int32(2), *none) == FA_EINVAL
    g = TgatGraph(n_dst=-1)
    assert f(ctypes.byref(g), ctypes.c_int32(2), *none) == FA_EINVAL
    g = TgatGraph(n_dst=4, n_edges=8, rowptr=16)
    # qt given, but neither xbar nor tdot, and no outputs
    assert f(ctypes.byref(g), ctypes.c_int32(2), ctypes.c_void_p(64), *([None] * 24)) == FA_EINVAL


def test_tgat_block_layouts_are_checked(lib):
    """Per-destination blocks: 16-byte alignment, strides in whole float4s, and output rows
    that do not overlap (destination-major or head-major); all rejected before a launch."""
    g = TgatGraph(n_dst=4, n_edges=8, rowptr=16)           # Kp = 4
    ok = dict(scores=4096, stats=8192)
    assert _fwd(lib, g, qt=68, qt_rs=8, qt_hs=4) == FA_EALIGN
    assert _fwd(lib, g, qt=64, qt_rs=6, qt_hs=4) == FA_EALIGN
    assert _fwd(lib, g, qt=64, qt_rs=-8, qt_hs=4) == FA_EINVAL
    # the two heads of a destination on top of each other, or on the next destination
    assert _fwd(lib, g, qt=64, xbar=128, xbar_rs=8, xbar_hs=0, **ok) == FA_EINVAL
    assert _fwd(lib, g, qt=64, xbar=128, xbar_rs=4, xbar_hs=4, **ok) == FA_EINVAL
    # head-major rows that run into the next head
    assert _fwd(lib, g, qt=64, xbar=128, xbar_rs=4, xbar_hs=12, **ok) == FA_EINVAL
    assert _fwd(lib, g, qt=64, xbar=132, xbar_rs=8, xbar_hs=4, **ok) == FA_EALIGN


def test_head_gemm_rejects_bad_arguments(lib):
    f = lib.fa_head_proj_f32
    i64, i32 = ctypes.c_int64, ctypes.c_int32
    # (n, j, c, groups, x, ldx, xg, w, wg, ldw, bias, bg, y, yg, ldy, stream)
    args = [i64(16), i32(50), i32(376), i32(2), ctypes.c_void_p(64), i64(100), i64(50),
            ctypes.c_void_p(128), i64(50 * 376), i64(376), None, i64(0), ctypes.c_void_p(256),
            i64(16 * 376), i64(376), None]
    bad = list(args); bad[1] = i32(65)
    assert f(*bad) == FA_EUNSUPPORTED           # J above 64
    bad = list(args); bad[5] = i64(10)
    assert f(*bad) == FA_EINVAL                 # ldx below J
    bad = list(args); bad[14] = i64(100)
    assert f(*bad) == FA_EINVAL                 # ldy below C
    bad = list(args); bad[4] = None
    assert f(*bad) == FA_EINVAL
    r = lib.fa_head_reduce_f32
    # (n, j, c, groups, y, yg, ldy, w, wg, ldw, z, ldz, zg, stream)
    assert r(i64(16), i32(70), i32(376), i32(2), ctypes.c_void_p(64), i64(0), i64(376),
             ctypes.c_void_p(128), i64(0), i64(376), ctypes.c_void_p(256), i64(140), i64(70),
             None) == FA_EUNSUPPORTED
    w = lib.fa_head_wgrad_f32
    # (n, j, c, groups, x, ldx, xg, y, yg, ldy, ones, dw, scratch, bytes, stream)
    assert w(i64(16), i32(50), i32(376), i32(2), ctypes.c_void_p(64), i64(100), i64(50),
             ctypes.c_void_p(128), i64(16 * 376), i64(376), i32(1), ctypes.c_void_p(256),
             ctypes.c_void_p(512), ctypes.c_size_t(16), None) == FA_ESCRATCH


def test_head_reduce_supported(lib):
    """The query names the head_reduce path from the same LDS rules the entry point applies:
    split-bf16 for 16-byte rows when W's three bf16 parts fit, float32 when its float32 copy
    fits, nothing beyond (or past 64 rows per head)."""
    q = lambda j, c, ld, r16: lib.fa_head_reduce_supported(ctypes.c_int32(j), ctypes.c_int32(c),
                                                           ctypes.c_int64(ld), ctypes.c_int32(r16))
    assert q(50, 376, 384, 1) == 2 and q(50, 376, 384, 0) == 1    # C3: K-space reduce
    assert q(32, 708, 736, 1) == 2                                # C5: 8 heads of 32
    assert q(64, 708, 736, 1) == 0 and q(64, 708, 736, 0) == 0    # 4 heads of 64 over Kp 708
    assert q(64, 416, 416, 1) == 1                                # bf16 parts too large
    assert q(65, 100, 100, 1) == 0 and q(0, 100, 100, 1) == 0 and q(8, 100, 50, 1) == 0


def test_softmax_rejects_bad_arguments(lib):
    f = lib.fa_edge_softmax_fwd_f32
    # (indptr, n_seg, n_edges, x, ldx, heads, y, ldy, mode, stream)
    assert f(None, ctypes.c_int64(4), ctypes.c_int64(8), None, ctypes.c_int64(2),
             ctypes.c_int32(2), None, ctypes.c_int64(2), ctypes.c_int32(0), None) == FA_EINVAL
    P = ctypes.c_void_p(16)
    call = lambda n_seg, heads, ldx, mode: f(P, ctypes.c_int64(n_seg), ctypes.c_int64(8), P,
                                             ctypes.c_int64(ldx), ctypes.c_int32(heads), P,
                                             ctypes.c_int64(2), ctypes.c_int32(mode), None)
    assert call(4, 2, 2, 2) == FA_EINVAL    # unknown mode
    assert call(4, 2, 1, 0) == FA_EINVAL    # leading dimension below the head count
    assert call(-1, 2, 2, 0) == FA_EINVAL
    assert call(4, 0, 2, 0) == FA_OK        # nothing to do: returns before any launch
    # no edges: nothing to write (with edges but no segment the output is zero-filled, a launch)
    assert f(P, ctypes.c_int64(0), ctypes.c_int64(0), P, ctypes.c_int64(2), ctypes.c_int32(2), P,
             ctypes.c_int64(2), ctypes.c_int32(0), None) == FA_OK


def test_memory_entry_points_reject_bad_arguments(lib):
    """The memory path's argument checks run before any launch (no device access)."""
    vp, c = ctypes.c_void_p, ctypes.c_int64
    one = ctypes.c_void_p(16)
    # generation 0 and negative sizes
    assert lib.fa_memory_update_f32(c(1), one, 1, one, c(4), 4, one, one, c(4), one, c(10), one,
                                    ctypes.c_uint32(0), None) == -1
    assert lib.fa_memory_update_f32(c(-1), one, 1, one, c(4), 4, one, one, c(4), one, c(10), one,
                                    ctypes.c_uint32(1), None) == -1
    # mailbox rows narrower than slots x (2m + de)
    assert lib.fa_mailbox_update_f32(c(2), one, one, 1, one, c(4), 4, None, c(0), 0, one, one,
                                     c(7), one, one, 2, c(10), one, ctypes.c_uint32(1), None) == -1
    # gru: leading dimension below 3m; missing workspace
    assert lib.fa_gru_fwd_f32(c(2), 4, one, c(11), one, c(12), None, c(0), None, None, one, c(4),
                              one, None) == -1
    assert lib.fa_gru_fwd_f32(c(2), 4, one, c(12), one, c(12), None, c(0), None, None, one, c(4),
                              None, None) == -1
    # time gradient without scratch
    assert lib.fa_time_rows_grad_f32(c(3), one, None, one, one, 8, one, c(8), one, one, None,
                                     ctypes.c_size_t(0), None) == -4
    assert lib.fa_time_rows_grad_scratch_bytes(8) >= 2 * 8 * 4
    # nothing to do is not an error
    assert lib.fa_mail_gather_f32(c(0), None, 0, c(0), None, c(0), 0, None, None, c(0), c(0), None,
                                  0, None, c(0), None, None, c(0), None, None) == 0
