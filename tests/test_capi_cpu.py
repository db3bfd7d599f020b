"""The C-ABI library (libsoinfer_hip.so) loads on a machine without a GPU and exports every
function include/soinfer_amd.h declares; argument checks return SOI_ERR_INVALID_ARGUMENT before
any HIP call (so they are safe to exercise here); status strings and workspace queries are pure host code.
"""
import ctypes as C
import re
from pathlib import Path

import pytest

REPO = Path(__file__).resolve().parent.parent
HEADER = REPO / "include" / "soinfer_amd.h"
LIB = REPO / "sparse-offload-infer_amd" / "soinfer" / "libsoinfer_hip.so"


@pytest.fixture(scope="module")
def lib():
    import torch  # noqa: F401  (same HIP runtime as the product process)

    assert LIB.exists(), "libsoinfer_hip.so not built: run __graft_entry__.build()"
    return C.CDLL(str(LIB))


def declared_functions():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(soi_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_the_hot_path():
    names = declared_functions()
    for required in ("soi_gemv_w4a16_group", "soi_gemv_w4a16_group_lop3", "soi_gemv_w8a16",
                     "soi_topk_threshold_select", "soi_gather_rows_staged", "soi_gather_rows_naive",
                     "soi_gemv_w4a16_sparse_accumulate", "soi_build_dip_descriptors", "soi_gemv_dip_fused_up",
                     "soi_gemv_dip_fused_down", "soi_decode_attention"):
        assert required in names


def test_every_declared_symbol_is_exported(lib):
    missing = [n for n in declared_functions() if not hasattr(lib, n)]
    assert not missing, f"declared but not exported: {missing}"


def test_status_strings_and_version(lib):
    lib.soi_status_string.restype = C.c_char_p
    lib.soi_version.restype = C.c_char_p
    assert lib.soi_status_string(0) == b"success"
    assert lib.soi_status_string(1) == b"invalid argument"
    assert b"gfx950" in lib.soi_version()


def test_argument_checks_return_before_launch(lib):
    lib.soi_last_error.restype = C.c_char_p
    i64 = C.c_int64
    f = lib.soi_gemv_w4a16_group_lop3
    f.argtypes = [C.c_void_p] * 4 + [i64] * 4 + [C.c_void_p]
    # group_size 7 is rejected
    assert f(None, None, None, None, 16, 256, 7, 2, None) == 1
    assert b"group_size" in lib.soi_last_error()
    # num_groups must be ceil(K/gs)
    assert f(None, None, None, None, 16, 256, 128, 3, None) == 1
    t = lib.soi_topk_threshold_select
    t.argtypes = [C.c_void_p, i64, i64, C.c_void_p, C.c_void_p, C.c_void_p]
    assert t(None, 100, 0, None, None, None) == 1  # k < 1
    assert t(None, 100, 101, None, None, None) == 1  # k > n
    a = lib.soi_decode_attention
    a.argtypes = [C.c_void_p] * 4 + [i64] * 5 + [C.c_float, C.c_void_p, C.c_size_t, C.c_void_p]
    assert a(None, None, None, None, 15, 8, 64, 128, 1, C.c_float(0.1), None, 0, None) == 1  # 15 % 8 != 0
    g = lib.soi_gather_rows_naive
    g.argtypes = [C.c_void_p, i64, i64, C.c_void_p, i64, C.c_void_p, C.c_void_p]
    idx = (C.c_int64 * 2)(0, 5)
    buf = (C.c_uint8 * 64)()
    assert g(buf, 4, 8, idx, 2, buf, None) == 1  # index 5 out of range [0, 4)
    assert b"out of range" in lib.soi_last_error()
    gr = lib.soi_gemv_w4a16_grouped
    gr.argtypes = [C.c_void_p] * 4 + [i64, C.c_void_p, C.c_void_p, C.c_void_p, i64, C.c_void_p]
    cnt, n, k = (C.c_int64 * 9)(*[1] * 9), (C.c_int64 * 9)(*[8] * 9), (C.c_int64 * 9)(*[256] * 9)
    assert gr(None, None, None, None, 9, cnt, n, k, 128, None) == 1  # more than 8 classes
    assert b"num_classes" in lib.soi_last_error()
    assert gr(None, None, None, None, 1, cnt, n, k, 12, None) == 1  # group_size not a multiple of 8
    assert gr(None, None, None, None, 0, None, None, None, 128, None) == 0  # nothing to do
    sw = lib.soi_swiglu_gate_up
    sw.argtypes = [C.c_void_p] * 4 + [i64, i64, C.c_void_p]
    assert sw(None, None, None, None, 16, 0, None) == 1  # H < 1
    assert sw(None, None, None, None, 16, 64, None) == 1  # rows to write, null pointers
    assert b"null pointer" in lib.soi_last_error()
    assert sw(None, None, None, None, 0, 64, None) == 0  # I = 0: nothing to do


def test_cached_dip_argument_checks(lib):
    """The hot-cache GEMVs reject missing sources, half-given copy arguments and oversized copied rows before any
    launch; k = 0 is a no-op for the up form."""
    lib.soi_last_error.restype = C.c_char_p
    i64, vp = C.c_int64, C.c_void_p
    up = lib.soi_gemv_dip_cached_up_silu
    up.argtypes = [vp, vp, i64, vp, vp, i64, vp, vp, i64, vp, vp, vp, i64, i64, i64, vp, i64, vp, vp]
    b = (C.c_uint8 * 4096)()
    p = C.addressof(b)
    # k > 0 with a null selection
    assert up(None, None, 0, p, p, 64, p, None, 8, p, p, p, 2048, 128, 16, None, 0, None, None) == 1
    # copy destination without a source
    assert up(None, None, 0, p, p, 64, p, p, 8, p, p, p, 2048, 128, 16, None, 1024, p, None) == 1
    assert b"copy_src and copy_dst" in lib.soi_last_error()
    # copied rows over 4096 bytes
    assert up(None, None, 0, p, p, 64, p, p, 8, p, p, p, 2048, 128, 16, p, 8192, p, None) == 1
    assert up(None, None, 0, None, None, 64, None, None, 0, None, None, None, 2048, 128, 16, None, 0, None,
              None) == 0  # k = 0
    dn = lib.soi_gemv_dip_cached_down
    dn.argtypes = [vp, vp, i64, vp, vp, i64, vp, vp, i64, vp, vp, i64, i64, i64, vp, vp, C.c_size_t, vp]
    # neither the full matrix nor staging for the misses
    assert dn(None, None, 0, None, p, 64, p, p, 8, p, p, 2048, 128, 16, None, p, 4096, None) == 1
    assert b"null pointer" in lib.soi_last_error()


def test_dip_select_gated_down_argument_checks(lib):
    """The fused selection + gated down rejects k outside [1, n], a down^T with fewer rows than channels, null
    pointers and a short workspace before any launch."""
    lib.soi_last_error.restype = C.c_char_p
    i64, vp = C.c_int64, C.c_void_p
    f = lib.soi_dip_select_gated_down
    f.argtypes = [vp, vp, i64, i64, vp, vp, i64, vp, vp, vp, i64, i64, i64, vp, C.c_size_t, vp]
    b = (C.c_uint8 * 4096)()
    p = C.addressof(b)
    assert f(p, p, 6144, 0, p, p, 6144, p, p, p, 2048, 128, 16, p, 4096, None) == 1  # k < 1
    assert f(p, p, 6144, 6145, p, p, 6144, p, p, p, 2048, 128, 16, p, 4096, None) == 1  # k > n
    assert f(p, p, 6144, 3072, p, p, 6143, p, p, p, 2048, 128, 16, p, 4096, None) == 1  # rows < channels
    assert b"fewer than" in lib.soi_last_error()
    assert f(p, None, 6144, 3072, p, p, 6144, p, p, p, 2048, 128, 16, p, 4096, None) == 1  # null up
    assert b"null pointer" in lib.soi_last_error()
    assert f(p, p, 6144, 3072, p, p, 6144, p, p, p, 2048, 128, 15, p, 4096, None) == 1  # num_groups != H/gs
    # a workspace below the partial rows' size (either path)
    assert f(p, p, 6144, 3072, p, p, 6144, p, p, p, 2048, 128, 16, p, 4096, None) == 2
    assert b"workspace" in lib.soi_last_error()


def test_workspace_queries(lib):
    lib.soi_sparse_accumulate_workspace_bytes.restype = C.c_size_t
    lib.soi_sparse_accumulate_workspace_bytes.argtypes = [C.c_int64, C.c_int64]
    w = lib.soi_sparse_accumulate_workspace_bytes(2048, 3072)
    assert w > 0 and w % 256 == 0 and w >= 16 * 2048 * 4  # partial rows of 16 row chunks + slice counters
    assert lib.soi_sparse_accumulate_workspace_bytes(2048, 0) == 0
    lib.soi_decode_attention_workspace_bytes.restype = C.c_size_t
    lib.soi_decode_attention_workspace_bytes.argtypes = [C.c_int64] * 4
    a = lib.soi_decode_attention_workspace_bytes(16, 8, 128, 2048)
    assert a >= 16 * 130 * 4 and a % 256 == 0  # split states (256-byte aligned) + arrival counters
