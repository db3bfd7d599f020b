"""numpy/ctypes front end of the CPU oracle (oracle/soi_oracle.c).

TEST INFRASTRUCTURE ONLY. Imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg, and there only as the checker / reported CPU
baseline. The product (the HIP library, soinfer._C, the soinfer package)
never imports this module.

Every function restates the reference arithmetic named in its docstring
(file:line in the reference repository). fp16 arrays are numpy float16;
they cross into C as their raw uint16 bit patterns.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess
from pathlib import Path

import numpy as np

_HERE = Path(__file__).resolve().parent
_LIB_PATH = _HERE / "_build" / "libsoi_oracle.so"
_lib = None


def build() -> Path:
    """Compile the oracle with its Makefile (gcc only)."""
    subprocess.run(["make", "-s", "-C", str(_HERE)], check=True)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not _LIB_PATH.exists():
            build()
        _lib = C.CDLL(str(_LIB_PATH))
        _declare(_lib)
    return _lib


_p = C.c_void_p
_i64 = C.c_int64


def _declare(L):
    L.soi_ref_f16_to_f32.restype = C.c_float
    L.soi_ref_f16_to_f32.argtypes = [C.c_uint16]
    L.soi_ref_f32_to_f16.restype = C.c_uint16
    L.soi_ref_f32_to_f16.argtypes = [C.c_float]
    for name in ("soi_ref_f16_to_f32_array", "soi_ref_f32_to_f16_array", "soi_ref_f64_to_f16_array"):
        getattr(L, name).argtypes = [_p, _i64, _p]
    L.soi_ref_quantize_group.argtypes = [_p, _i64, _i64, _i64, C.c_int, _p, _p]
    L.soi_ref_quantize_simple.argtypes = [_p, _i64, _i64, C.c_int, C.c_int, _p, _p]
    L.soi_ref_pack_int4.argtypes = [_p, _i64, _i64, _p]
    L.soi_ref_unpack_int4.argtypes = [_p, _i64, _i64, _p]
    L.soi_ref_gemv_w4_f64.argtypes = [_p, _p, _p, _i64, _i64, _i64, _i64, _p]
    L.soi_ref_gemv_w4_f32.argtypes = [_p, _p, _p, _i64, _i64, _i64, _i64, _p]
    L.soi_ref_gemv_w4_f64_mt.argtypes = [_p, _p, _p, _i64, _i64, _i64, _i64, _p, C.c_int]
    L.soi_ref_dequant_int4.argtypes = [_p, _p, _i64, _i64, _i64, _i64, _p]
    L.soi_ref_gemv_w8_f64.argtypes = [_p, _p, _p, _i64, _i64, _i64, _i64, _p]
    L.soi_ref_topk_tau_rule_a.restype = C.c_float
    L.soi_ref_topk_tau_rule_a.argtypes = [_p, _i64, _i64]
    L.soi_ref_topk_rule_a.restype = _i64
    L.soi_ref_topk_rule_a.argtypes = [_p, _i64, _i64, _p]
    L.soi_ref_topk_rule_b.restype = _i64
    L.soi_ref_topk_rule_b.argtypes = [_p, _i64, _i64, _p]
    L.soi_ref_gather_rows.argtypes = [_p, _p, _i64, _i64, _p]
    L.soi_ref_sparse_accumulate_f64.argtypes = [_p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _p]
    L.soi_ref_fused_up_f64.argtypes = [_p, _p, _p, _p, _p, _p, _i64, _i64, _i64, _i64, _p]
    L.soi_ref_build_dip_descriptors.restype = C.c_int32
    L.soi_ref_build_dip_descriptors.argtypes = [_p, _i64, _p, _p, _p]
    L.soi_ref_decode_attention_f64.argtypes = [_p, _p, _p, _i64, _i64, _i64, _i64, _i64, _p]


def _c(a: np.ndarray, dtype) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=dtype)


def _ptr(a: np.ndarray | None):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


# --------------------------------------------------------------------------
# fp16 helpers (IEEE-754 binary16, written from the format definition)
# --------------------------------------------------------------------------

def f16_bits_to_f32(h: np.ndarray) -> np.ndarray:
    h = _c(h, np.uint16)
    out = np.empty(h.shape, np.float32)
    lib().soi_ref_f16_to_f32_array(_ptr(h), h.size, _ptr(out))
    return out


def f32_to_f16_bits(f: np.ndarray) -> np.ndarray:
    f = _c(f, np.float32)
    out = np.empty(f.shape, np.uint16)
    lib().soi_ref_f32_to_f16_array(_ptr(f), f.size, _ptr(out))
    return out


def f64_to_f16(d: np.ndarray) -> np.ndarray:
    """binary64 -> binary16, correctly rounded (round-to-odd through binary32)."""
    d = _c(d, np.float64)
    out = np.empty(d.shape, np.uint16)
    lib().soi_ref_f64_to_f16_array(_ptr(d), d.size, _ptr(out))
    return out.view(np.float16)


# --------------------------------------------------------------------------
# R1/R2: quantizer + AWQ pack
# --------------------------------------------------------------------------

def quantize_group(w: np.ndarray, group_size: int, bits: int = 4) -> tuple[np.ndarray, np.ndarray]:
    """formats.quantize(granularity='group', scale_fn=min_max)
    (python/soinfer/quant/formats.py:55-65,77-110; calibrate.py:22-27).
    Returns (q int8 [N, ceil(K/gs)*gs], scale float32 [N, ceil(K/gs)])."""
    w = _c(w, np.float32)
    N, K = w.shape
    G = -(-K // group_size)
    q = np.empty((N, G * group_size), np.int8)
    s = np.empty((N, G), np.float32)
    lib().soi_ref_quantize_group(_ptr(w), N, K, group_size, bits, _ptr(q), _ptr(s))
    return q, s


def quantize_simple(w: np.ndarray, granularity: str, bits: int = 8) -> tuple[np.ndarray, np.ndarray]:
    """formats.quantize per_tensor / per_channel branches (formats.py:88-99).
    Returns (q int8 [N, K], scale float32 [1,1] or [N,1])."""
    w = _c(w, np.float32)
    N, K = w.shape
    g = {"per_tensor": 0, "per_channel": 1}[granularity]
    q = np.empty((N, K), np.int8)
    s = np.empty((1, 1) if g == 0 else (N, 1), np.float32)
    lib().soi_ref_quantize_simple(_ptr(w), N, K, bits, g, _ptr(q), _ptr(s))
    return q, s


def pack_int4(q: np.ndarray) -> np.ndarray:
    """pack_int4 (python/soinfer/quant/pack.py:31-49; csrc/include/layout.h:19-45)."""
    q = _c(q, np.int8)
    N, K = q.shape
    out = np.empty((N, -(-K // 8) * 4), np.uint8)
    lib().soi_ref_pack_int4(_ptr(q), N, K, _ptr(out))
    return out


def unpack_int4(packed: np.ndarray, K: int) -> np.ndarray:
    """unpack_int4 (python/soinfer/quant/pack.py:52-69)."""
    packed = _c(packed, np.uint8)
    N = packed.shape[0]
    out = np.empty((N, K), np.int8)
    lib().soi_ref_unpack_int4(_ptr(packed), N, K, _ptr(out))
    return out


def dequant_int4(Wq: np.ndarray, scale: np.ndarray, K: int, group_size: int) -> np.ndarray:
    """binary32 dequantized weights fl(q*s) (formats.dequantize, formats.py:113-123)."""
    Wq, scale = _c(Wq, np.uint8), _c(scale, np.float32)
    N, G = scale.shape
    W = np.empty((N, K), np.float32)
    lib().soi_ref_dequant_int4(_ptr(Wq), _ptr(scale), N, K, group_size, G, _ptr(W))
    return W


# --------------------------------------------------------------------------
# R4/R5: dense GEMVs
# --------------------------------------------------------------------------

def gemv_w4_f64(Wq: np.ndarray, scale: np.ndarray, x: np.ndarray, K: int, group_size: int,
                threads: int = 1) -> np.ndarray:
    """y = dequant(Wq, scale) @ x in binary64 (gemv_w4a16_group.cu:23-127 arithmetic). threads > 1 splits the rows
    over POSIX threads (same result: each row is summed by one thread in ascending k)."""
    Wq, scale = _c(Wq, np.uint8), _c(scale, np.float32)
    xb = _c(x, np.float16).view(np.uint16)
    N, G = scale.shape
    y = np.empty(N, np.float64)
    if threads > 1:
        lib().soi_ref_gemv_w4_f64_mt(_ptr(Wq), _ptr(scale), _ptr(xb), N, K, group_size, G, _ptr(y), threads)
    else:
        lib().soi_ref_gemv_w4_f64(_ptr(Wq), _ptr(scale), _ptr(xb), N, K, group_size, G, _ptr(y))
    return y


def gemv_w4_f32(Wq: np.ndarray, scale: np.ndarray, x: np.ndarray, K: int, group_size: int) -> np.ndarray:
    """Same GEMV, binary32 accumulation in ascending k (one fma per term)."""
    Wq, scale = _c(Wq, np.uint8), _c(scale, np.float32)
    xb = _c(x, np.float16).view(np.uint16)
    N, G = scale.shape
    y = np.empty(N, np.float32)
    lib().soi_ref_gemv_w4_f32(_ptr(Wq), _ptr(scale), _ptr(xb), N, K, group_size, G, _ptr(y))
    return y


def gemv_w8_f64(Wq: np.ndarray, scale: np.ndarray, x: np.ndarray, group_size: int) -> np.ndarray:
    """INT8 GEMV in binary64 (gemv_w8a16.cu:22-62). scale [N|1, G]; row stride 0 when [1, G]."""
    Wq, scale = _c(Wq, np.int8), _c(scale, np.float32)
    xb = _c(x, np.float16).view(np.uint16)
    N, K = Wq.shape
    stride = 0 if scale.shape[0] == 1 else scale.shape[1]
    y = np.empty(N, np.float64)
    lib().soi_ref_gemv_w8_f64(_ptr(Wq), _ptr(scale), _ptr(xb), N, K, group_size, stride, _ptr(y))
    return y


# --------------------------------------------------------------------------
# R7: top-k
# --------------------------------------------------------------------------

def topk_tau_rule_a(v: np.ndarray, k: int) -> np.float32:
    v = _c(v, np.float32)
    return np.float32(lib().soi_ref_topk_tau_rule_a(_ptr(v), v.size, k))


def topk_rule_a(v: np.ndarray, k: int) -> np.ndarray:
    """topk_threshold_select rule A (csrc/kernels/topk_select.cu:10-96): int32 [count]."""
    v = _c(v, np.float32)
    out = np.full(k, -1, np.int32)
    n = lib().soi_ref_topk_rule_a(_ptr(v), v.size, k, _ptr(out))
    return out[:n]


def topk_rule_b(v: np.ndarray, k: int) -> np.ndarray:
    """Exact top-k with lowest-index tie-break, ascending index order."""
    v = _c(v, np.float32)
    out = np.empty(k, np.int32)
    lib().soi_ref_topk_rule_b(_ptr(v), v.size, k, _ptr(out))
    return out


# --------------------------------------------------------------------------
# R8, R11-R14: gather, sparse down, descriptors, fused up/down
# --------------------------------------------------------------------------

def gather_rows(matrix: np.ndarray, idx: np.ndarray) -> np.ndarray:
    """gather_rows_* (csrc/kernels/gather_rows.cu:6-21)."""
    matrix = _c(matrix, np.uint8)
    idx = _c(idx, np.int64)
    out = np.empty((idx.size, matrix.shape[1]), np.uint8)
    lib().soi_ref_gather_rows(_ptr(matrix), _ptr(idx), idx.size, matrix.shape[1], _ptr(out))
    return out


def sparse_accumulate_f64(Wq_sel: np.ndarray, scale_sel: np.ndarray, h: np.ndarray, H: int, group_size: int,
                          staging_Wq: np.ndarray | None = None, staging_scale: np.ndarray | None = None,
                          desc: np.ndarray | None = None) -> np.ndarray:
    """y[H] = sum_j h_j * dequant(row_j) in binary64 (gemv_sparse_accumulate.cu:10-38; with desc, the
    fused form gemv_dip_fused.cu:116-154, rows resolved through the descriptors)."""
    Wq_sel, scale_sel = _c(Wq_sel, np.uint8), _c(scale_sel, np.float32)
    hb = _c(h, np.float16).view(np.uint16)
    G = scale_sel.shape[1]
    sW = None if staging_Wq is None else _c(staging_Wq, np.uint8)
    sS = None if staging_scale is None else _c(staging_scale, np.float32)
    d = None if desc is None else _c(desc, np.int32)
    y = np.empty(H, np.float64)
    lib().soi_ref_sparse_accumulate_f64(_ptr(Wq_sel), _ptr(scale_sel), _ptr(sW), _ptr(sS), _ptr(d), _ptr(hb),
                                        hb.size, H, group_size, G, _ptr(y))
    return y


def fused_up_f64(cache_Wq, cache_scale, staging_Wq, staging_scale, desc, x, K: int, group_size: int) -> np.ndarray:
    """gemv_dip_fused_up (gemv_dip_fused.cu:48-102) in binary64."""
    cW, cS = _c(cache_Wq, np.uint8), _c(cache_scale, np.float32)
    sW, sS = _c(staging_Wq, np.uint8), _c(staging_scale, np.float32)
    d = _c(desc, np.int32)
    xb = _c(x, np.float16).view(np.uint16)
    G = cS.shape[1] if cS.size else sS.shape[1]
    y = np.empty(d.size, np.float64)
    lib().soi_ref_fused_up_f64(_ptr(cW), _ptr(cS), _ptr(sW), _ptr(sS), _ptr(d), _ptr(xb), d.size, K, group_size, G,
                               _ptr(y))
    return y


def build_dip_descriptors(sel: np.ndarray, slot_of: np.ndarray) -> tuple[np.ndarray, np.ndarray, int]:
    """build_dip_descriptors (gemv_dip_fused.cu:17-42), misses numbered in ascending j."""
    sel, slot_of = _c(sel, np.int32), _c(slot_of, np.int32)
    desc = np.empty(sel.size, np.int32)
    miss = np.full(sel.size, -1, np.int32)
    mc = lib().soi_ref_build_dip_descriptors(_ptr(sel), sel.size, _ptr(slot_of), _ptr(desc), _ptr(miss))
    return desc, miss, int(mc)


# --------------------------------------------------------------------------
# R16: decode attention
# --------------------------------------------------------------------------

def decode_attention_f64(q: np.ndarray, k_cache: np.ndarray, v_cache: np.ndarray, cur_len: int) -> np.ndarray:
    """decode_attention (csrc/kernels/decode_attention.cu:17-55), softmax in binary64."""
    qb = _c(q, np.float16).view(np.uint16)
    kb = _c(k_cache, np.float16).view(np.uint16)
    vb = _c(v_cache, np.float16).view(np.uint16)
    NQ, hd = q.shape
    NKV, S, _ = k_cache.shape
    out = np.empty((NQ, hd), np.float64)
    lib().soi_ref_decode_attention_f64(_ptr(qb), _ptr(kb), _ptr(vb), NQ, NKV, S, hd, cur_len, _ptr(out))
    return out


def threads_used() -> int:
    """The oracle is scalar C; every function runs on one thread except gemv_w4_f64 with threads > 1."""
    return 1


if __name__ == "__main__":  # pragma: no cover
    print(build())
    print(os.path.getsize(_LIB_PATH))
