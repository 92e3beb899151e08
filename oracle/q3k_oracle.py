"""numpy front end of the CPU oracle (oracle/build/libq3k_oracle.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg, never by the product package.  Each function
returns the primary result and, when ``band`` is true, the per-element band
(lo, hi) described in q3k_oracle.h.
"""
from __future__ import annotations

import ctypes
import os

import numpy as np

ORACLE_DIR = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(ORACLE_DIR, "build", "libq3k_oracle.so")

_lib = None
_p, _i64, _i32, _f32, _int = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int32, ctypes.c_float, ctypes.c_int


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} is not built (make -C oracle)")
        L = ctypes.CDLL(LIB_PATH)
        sig = {
            "q3o_embedding": ([_p, _i64, _p, _i64, _i64, _p, _int], None),
            "q3o_add_inplace": ([_p, _p, _i64, _int], None),
            "q3o_rms_norm": ([_p, _p, _i64, _i64, _f32, _p, _p, _p, _int], None),
            "q3o_add_rms_norm": ([_p, _p, _p, _i64, _i64, _f32, _p, _p, _p, _int], None),
            "q3o_rms_norm_test_order": ([_p, _p, _i64, _i64, _f32, _p, _int], None),
            "q3o_silu_mul": ([_p, _p, _i64, _p, _p, _p, _int], None),
            "q3o_build_rope_cache": ([_i64, _i32, _f32, _p], _int),
            "q3o_rope": ([_p, _i64, _i64, _i32, _i32, _p, _i64, _i64, _p, _p, _p, _int], _int),
            "q3o_qk_norm_rope": ([_p, _p, _i64, _i64, _i32, _i32, _f32, _p, _i64, _i64, _p, _p, _p, _int], _int),
            "q3o_kv_append": ([_p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64], None),
            "q3o_gqa_attention": ([_p, _p, _p, _i64, _i64, _i32, _i32, _i32, _i64, _i64, _p, _p, _p, _i64, _p, _p, _p,
                                   _int], _int),
            "q3o_argmax": ([_p, _i64, _i64, _i64, _p], None),
            "q3o_topk_set": ([_p, _i64, _i32, _p], _i64),
            "q3o_sample_row": ([_p, _i64, _f32, _i32, _f32, ctypes.c_double], _i32),
            "q3o_compare_band": ([_p, _p, _p, _p, _i64, _p], None),
            "q3o_ulp_distance": ([ctypes.c_uint16, ctypes.c_uint16], ctypes.c_int32),
            "q3o_bf16_from_f32": ([_f32], ctypes.c_uint16),
            "q3o_f32_from_bf16": ([ctypes.c_uint16], _f32),
            "q3o_band_rel_inv": ([], ctypes.c_double),
            "q3o_band_rel_silu": ([], ctypes.c_double),
        }
        for name, (args, res) in sig.items():
            fn = getattr(L, name)
            fn.argtypes = args
            fn.restype = res
        _lib = L
    return _lib


def _a(x, dtype):
    return np.ascontiguousarray(x, dtype=dtype)


def _ptr(x):
    return None if x is None else x.ctypes.data


def default_threads() -> int:
    return max(1, min(16, os.cpu_count() or 1))


def embedding(ids, table, nthreads=None):
    ids = _a(ids, np.int32)
    table = _a(table, np.uint16)
    V, H = table.shape
    out = np.empty(ids.shape + (H,), dtype=np.uint16)
    lib().q3o_embedding(_ptr(ids), ids.size, _ptr(table), V, H, _ptr(out), nthreads or default_threads())
    return out


def add_inplace(d, s, nthreads=None):
    d = _a(d, np.uint16).copy()
    s = _a(s, np.uint16)
    lib().q3o_add_inplace(_ptr(d), _ptr(s), d.size, nthreads or default_threads())
    return d


def _bands(shape, band):
    if not band:
        return None, None
    return np.empty(shape, np.uint16), np.empty(shape, np.uint16)


def rms_norm(x, w, eps, band=True, nthreads=None):
    x = _a(x, np.uint16)
    w = _a(w, np.uint16)
    N = w.size
    y = np.empty_like(x)
    lo, hi = _bands(x.shape, band)
    lib().q3o_rms_norm(_ptr(x), _ptr(w), x.size // N, N, eps, _ptr(y), _ptr(lo), _ptr(hi),
                       nthreads or default_threads())
    return y, lo, hi


def rms_norm_test_order(x, w, eps, nthreads=None):
    """The reference test's own CPU RMSNorm (rms_norm_cuda_test.cpp:174-244):
    fp32 sum of squares in column order.  The CPU baseline of config 1."""
    x = _a(x, np.uint16)
    w = _a(w, np.uint16)
    N = w.size
    y = np.empty_like(x)
    lib().q3o_rms_norm_test_order(_ptr(x), _ptr(w), x.size // N, N, eps, _ptr(y), nthreads or default_threads())
    return y


def add_rms_norm(h, d, w, eps, band=True, nthreads=None):
    h = _a(h, np.uint16).copy()
    d = _a(d, np.uint16)
    w = _a(w, np.uint16)
    N = w.size
    y = np.empty_like(h)
    lo, hi = _bands(h.shape, band)
    lib().q3o_add_rms_norm(_ptr(h), _ptr(d), _ptr(w), h.size // N, N, eps, _ptr(y), _ptr(lo), _ptr(hi),
                           nthreads or default_threads())
    return h, y, lo, hi


def silu_mul(g, u, band=True, nthreads=None):
    g = _a(g, np.uint16)
    u = _a(u, np.uint16)
    out = np.empty_like(g)
    lo, hi = _bands(g.shape, band)
    lib().q3o_silu_mul(_ptr(g), _ptr(u), g.size, _ptr(out), _ptr(lo), _ptr(hi), nthreads or default_threads())
    return out, lo, hi


def build_rope_cache(P, D, theta):
    out = np.empty((P, D // 2, 2), dtype=np.float32)
    if lib().q3o_build_rope_cache(P, D, theta, _ptr(out)) != 0:
        raise ValueError("bad RoPE cache arguments")
    return out


def rope(x, B, S, heads, D, cache, start=0, positions=None, band=True, nthreads=None):
    x = _a(x, np.uint16).copy()
    cache = _a(cache, np.float32)
    pos = None if positions is None else _a(positions, np.int32)
    lo, hi = _bands(x.shape, band)
    st = lib().q3o_rope(_ptr(x), B, S, heads, D, _ptr(cache), cache.shape[0], start, _ptr(pos), _ptr(lo), _ptr(hi),
                        nthreads or default_threads())
    if st != 0:
        raise ValueError("bad RoPE arguments")
    return x, lo, hi


def qk_norm_rope(x, w, B, S, heads, D, eps, cache, start=0, positions=None, band=True, nthreads=None):
    x = _a(x, np.uint16).copy()
    w = _a(w, np.uint16)
    cache = _a(cache, np.float32)
    pos = None if positions is None else _a(positions, np.int32)
    lo, hi = _bands(x.shape, band)
    st = lib().q3o_qk_norm_rope(_ptr(x), _ptr(w), B, S, heads, D, eps, _ptr(cache), cache.shape[0], start, _ptr(pos),
                                _ptr(lo), _ptr(hi), nthreads or default_threads())
    if st != 0:
        raise ValueError("bad Q/K norm + RoPE arguments")
    return x, lo, hi


def kv_append(k, v, k_cache, v_cache, start):
    """k, v [B, S, row] into copies of the layer caches [batch_cap, seq_cap, row] at row `start`."""
    k = np.ascontiguousarray(k)
    v = np.ascontiguousarray(v)
    kc = np.array(k_cache, copy=True, order="C")
    vc = np.array(v_cache, copy=True, order="C")
    B, S = k.shape[0], k.shape[1]
    row_bytes = k[0, 0].nbytes
    seq_cap = kc.shape[1]
    lib().q3o_kv_append(_ptr(k), _ptr(v), _ptr(kc), _ptr(vc), B, S, row_bytes, seq_cap, start)
    return kc, vc


def gqa_attention(q, k_cache, v_cache, Hq, start, rows=None, band=True, nthreads=None):
    """q [B, S, Hq * D] bf16; k_cache / v_cache [B, cached, Hkv, D] bf16 (any strides, e.g. views of a larger
    cache).  Returns (out, lo, hi) shaped [B, S, Hq * D], or [len(rows), D] when rows is given."""
    q = _a(q, np.uint16)
    B, S = q.shape[0], q.shape[1]
    _, cached, Hkv, D = k_cache.shape
    assert k_cache.dtype == np.uint16 and v_cache.dtype == np.uint16 and v_cache.shape == k_cache.shape
    ks = np.array([st // 2 for st in k_cache.strides], np.int64)
    vs = np.array([st // 2 for st in v_cache.strides], np.int64)
    r = None if rows is None else np.ascontiguousarray(rows, np.int64)
    n = B * S * Hq if r is None else r.size
    out = np.empty((n, D), np.uint16)
    lo, hi = _bands((n, D), band)
    st = lib().q3o_gqa_attention(_ptr(q), k_cache.ctypes.data, v_cache.ctypes.data, B, S, Hq, Hkv, D, cached, start,
                                 _ptr(ks), _ptr(vs), _ptr(r), n, _ptr(out), _ptr(lo), _ptr(hi),
                                 nthreads or default_threads())
    if st != 0:
        raise ValueError("bad attention arguments")
    if r is None:
        shape = (B, S, Hq * D)
        return out.reshape(shape), None if lo is None else lo.reshape(shape), None if hi is None else hi.reshape(shape)
    return out, lo, hi


def argmax(x, search_size=0):
    """x [..., N] bf16 bits -> int32 [...]: argmax over the first search_size (0 = all) columns."""
    x = _a(x, np.uint16)
    N = x.shape[-1]
    n = search_size or N
    rows = x.size // N
    out = np.empty(x.shape[:-1], np.int32)
    lib().q3o_argmax(_ptr(x), rows, N, n, _ptr(out))
    return out


def topk_set(row, k):
    """The reference's top-k set of one bf16 row (ties at the k-th kept), ids best first; None if non-finite."""
    row = _a(row, np.uint16)
    ids = np.empty(row.size, np.int32)
    n = lib().q3o_topk_set(_ptr(row), row.size, k, _ptr(ids))
    return None if n < 0 else ids[:n].copy()


def sample_row(row, temperature, top_k, top_p, u):
    """One row of the reference sampler given its uniform draw u; -1 if non-finite."""
    row = _a(row, np.uint16)
    return int(lib().q3o_sample_row(_ptr(row), row.size, temperature, top_k, top_p, u))


def compare(got, primary, lo=None, hi=None) -> dict:
    got = _a(got, np.uint16).ravel()
    primary = _a(primary, np.uint16).ravel()
    lo = None if lo is None else _a(lo, np.uint16).ravel()
    hi = None if hi is None else _a(hi, np.uint16).ravel()
    if got.size != primary.size:
        raise ValueError("size mismatch")
    stats = np.zeros(8, dtype=np.int64)
    lib().q3o_compare_band(_ptr(got), _ptr(primary), _ptr(lo), _ptr(hi), got.size, _ptr(stats))
    return {
        "n": int(stats[0]), "fail": int(stats[1]), "first_fail": int(stats[2]), "ambiguous": int(stats[3]),
        "ulp_hist": [int(v) for v in stats[4:8]],
        "max_ulp": (3 if stats[7] else 2 if stats[6] else 1 if stats[5] else 0),
    }


def ulp_distance(a: int, b: int) -> int:
    return int(lib().q3o_ulp_distance(a, b))


def bf16(x: float) -> int:
    return int(lib().q3o_bf16_from_f32(x))
