"""Python view of the gfx950 kernel library ``lib/libq3k.so``.

The product is the C ABI in ``include/q3k_abi.h`` (plain device pointers,
sizes and a HIP stream) and the C++ ``qwen3::ops`` layer above it.  This
module binds the same entry points through ctypes for the test suite, the
benchmark and ``__graft_entry__``; each wrapper keeps the argument order of
the C function and turns a non-zero status into the exception the C++ layer
throws (``std::invalid_argument`` -> ValueError, ``std::out_of_range`` ->
IndexError, ``std::overflow_error`` -> OverflowError, HIP failures ->
RuntimeError).

There is no fallback: if the library is not built, :func:`load` raises.
Device memory comes from :mod:`.hip` (the HIP runtime the library links).
"""
from __future__ import annotations

import ctypes
import os
import re

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
REPO_DIR = os.path.dirname(PKG_DIR)
LIB_DIR = os.path.join(PKG_DIR, "lib")
LIB_PATH = os.path.join(LIB_DIR, "libq3k.so")
RUNTIME_LIB_PATH = os.path.join(LIB_DIR, "libqwen3_runtime.so")
BENCH_LIB_PATH = os.path.join(LIB_DIR, "libq3k_bench.so")
ABI_HEADERS = [os.path.join(REPO_DIR, "include", "q3k_abi.h")]
BENCH_HEADERS = [os.path.join(REPO_DIR, "include", "q3k_bench.h")]

Q3K_OK = 0
Q3K_ERR_INVALID_ARGUMENT = 1
Q3K_ERR_OUT_OF_RANGE = 2
Q3K_ERR_OVERFLOW = 3
Q3K_ERR_HIP = 4


class Q3kError(RuntimeError):
    """A non-zero q3k_status."""

    def __init__(self, status: int, message: str):
        super().__init__(message)
        self.status = status


class Q3kInvalidArgument(Q3kError, ValueError):
    pass


class Q3kOutOfRange(Q3kError, IndexError):
    pass


class Q3kOverflow(Q3kError, OverflowError):
    pass


class Q3kHipError(Q3kError):
    pass


_ERRORS = {
    Q3K_ERR_INVALID_ARGUMENT: Q3kInvalidArgument,
    Q3K_ERR_OUT_OF_RANGE: Q3kOutOfRange,
    Q3K_ERR_OVERFLOW: Q3kOverflow,
    Q3K_ERR_HIP: Q3kHipError,
}

_p = ctypes.c_void_p
_i64 = ctypes.c_int64
_i32 = ctypes.c_int32
_f32 = ctypes.c_float

# name -> argtypes, in the order of include/q3k_abi.h
SIGNATURES = {
    "q3k_embedding_bf16": [_p, _i64, _p, _i64, _i64, _p, _p],
    "q3k_rms_norm_bf16": [_p, _p, _p, _i64, _i64, _f32, _p],
    "q3k_add_rms_norm_bf16": [_p, _p, _p, _p, _i64, _i64, _f32, _p],
    "q3k_rms_norm_rows_bf16": [_p, _p, _p, _i64, _i64, _i64, _i64, _f32, _p],
    "q3k_add_rms_norm_rows_bf16": [_p, _p, _p, _p, _i64, _i64, _i64, _i64, _f32, _p],
    "q3k_embedding_rms_norm_bf16": [_p, _i64, _p, _i64, _i64, _p, _f32, _p, _p, _p],
    "q3k_add_inplace_bf16": [_p, _p, _i64, _p],
    "q3k_silu_mul_bf16": [_p, _p, _p, _i64, _p],
    "q3k_rope_bf16": [_p, _i64, _i64, _i32, _i32, _p, _i64, _i64, _p, _p],
    "q3k_rope_qk_bf16": [_p, _p, _i64, _i64, _i32, _i32, _i32, _p, _i64, _i64, _p, _p],
    "q3k_qk_norm_rope_bf16": [_p, _p, _p, _p, _i64, _i64, _i32, _i32, _i32, _f32, _p, _i64, _i64, _p, _p],
    "q3k_gqa_attention_bf16": [_p, _p, _p, _p, _i64, _i64, _i32, _i32, _i32, _i64, _i64, _p, _p, _p, _i64, _p],
    "q3k_gqa_attention_workspace_bytes": [_i64, _i64, _i32, _i32, _i32, _i64],
    "q3k_argmax_bf16": [_p, _p, _i64, _i64, _i64, _p, _i64, _p],
    "q3k_argmax_workspace_bytes": [_i64, _i64],
    "q3k_argmax_bf16_noalloc": [_p, _p, _i64, _i64, _i64, _p],
    "q3k_topk_candidates_bf16": [_p, _i64, _i64, _i64, _i32, _i32, _p, _p, _p, _p, _p, _i64, _p],
    "q3k_topk_workspace_bytes": [_i64, _i64, _i32],
    "q3k_kv_append": [_p, _p, _p, _p, _i64, _i64, _i64, _i64, _i64, _p],
    "q3k_qk_norm_rope_kv_append_bf16": [_p, _p, _p, _p, _p, _i64, _i64, _i32, _i32, _i32, _f32, _p, _i64, _i64, _p,
                                        _p, _p, _i64, _i64, _p],
    "q3k_build_rope_cache_f32": [_p, _i64, _i32, _f32],
}

_lib = None


# name -> argtypes, in the order of include/q3k_bench.h (lib/libq3k_bench.so)
BENCH_SIGNATURES = {
    "q3k_bench_copy_u128": [_p, _p, _i64, _p],
    "q3k_bench_stream_u128": [_p, _p, _p, _p, _i64, _i32, _p],
    "q3k_bench_read_rows_u128": [_p, _p, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _p, _p],
}
_bench_lib = None


def declared_symbols(headers=None) -> list[str]:
    """Function names declared in the public C headers (default: the op ABI)."""
    names = []
    for path in headers or ABI_HEADERS:
        with open(path) as f:
            text = f.read()
        names += re.findall(r"Q3K_API\s+[\w\s\*]*?\b(q3k_\w+)\s*\(", text)
    return names


def load(path: str | None = None) -> ctypes.CDLL:
    """Load libq3k.so (RTLD_GLOBAL, so that :mod:`.hip` binds the same HIP runtime)."""
    global _lib
    if _lib is not None and path is None:
        return _lib
    lib_path = path or LIB_PATH
    if not os.path.exists(lib_path):
        raise RuntimeError(
            f"{lib_path} is not built; run __graft_entry__.build() (the HIP kernels have no fallback)")
    lib = ctypes.CDLL(lib_path, mode=ctypes.RTLD_GLOBAL)
    for name, argtypes in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.argtypes = argtypes
        fn.restype = ctypes.c_int64 if name.endswith("_bytes") else ctypes.c_int
    lib.q3k_last_error_string.restype = ctypes.c_char_p
    lib.q3k_last_error_string.argtypes = []
    lib.q3k_version.restype = ctypes.c_char_p
    lib.q3k_version.argtypes = []
    if path is None:
        _lib = lib
    return lib


def load_bench() -> ctypes.CDLL:
    """Load lib/libq3k_bench.so, the benchmark's measurement kernels."""
    global _bench_lib
    if _bench_lib is None:
        load()
        if not os.path.exists(BENCH_LIB_PATH):
            raise RuntimeError(f"{BENCH_LIB_PATH} is not built; run __graft_entry__.build()")
        lib = ctypes.CDLL(BENCH_LIB_PATH)
        for name, argtypes in BENCH_SIGNATURES.items():
            fn = getattr(lib, name)
            fn.argtypes = argtypes
            fn.restype = ctypes.c_int
        lib.q3k_bench_last_error_string.restype = ctypes.c_char_p
        lib.q3k_bench_last_error_string.argtypes = []
        _bench_lib = lib
    return _bench_lib


def _check_bench(status: int) -> None:
    if status != Q3K_OK:
        msg = load_bench().q3k_bench_last_error_string().decode()
        raise _ERRORS.get(status, Q3kError)(status, msg)


def _check(status: int) -> None:
    if status != Q3K_OK:
        msg = load().q3k_last_error_string().decode()
        raise _ERRORS.get(status, Q3kError)(status, msg)


def _ptr(x):
    """Device address of a buffer object (anything with ``.ptr``) or an int."""
    if x is None:
        return None
    return getattr(x, "ptr", x)


def version() -> str:
    return load().q3k_version().decode()


def embedding(ids, T, table, V, H, out, stream=None):
    _check(load().q3k_embedding_bf16(_ptr(ids), T, _ptr(table), V, H, _ptr(out), _ptr(stream)))


def rms_norm(x, w, y, rows, N, eps, stream=None):
    _check(load().q3k_rms_norm_bf16(_ptr(x), _ptr(w), _ptr(y), rows, N, eps, _ptr(stream)))


def add_rms_norm(h, d, w, y, rows, N, eps, stream=None):
    _check(load().q3k_add_rms_norm_bf16(_ptr(h), _ptr(d), _ptr(w), _ptr(y), rows, N, eps, _ptr(stream)))


def rms_norm_rows(x, w, y, count, first_row, row_stride, N, eps, stream=None):
    _check(load().q3k_rms_norm_rows_bf16(_ptr(x), _ptr(w), _ptr(y), count, first_row, row_stride, N, eps, _ptr(stream)))


def add_rms_norm_rows(h, d, w, y, count, first_row, row_stride, N, eps, stream=None):
    _check(load().q3k_add_rms_norm_rows_bf16(_ptr(h), _ptr(d), _ptr(w), _ptr(y), count, first_row, row_stride, N, eps,
                                             _ptr(stream)))


def embedding_rms_norm(ids, T, table, V, H, w, eps, hidden, y, stream=None):
    _check(load().q3k_embedding_rms_norm_bf16(_ptr(ids), T, _ptr(table), V, H, _ptr(w), eps, _ptr(hidden), _ptr(y),
                                              _ptr(stream)))


def add_inplace(d, s, n, stream=None):
    _check(load().q3k_add_inplace_bf16(_ptr(d), _ptr(s), n, _ptr(stream)))


def silu_mul(g, u, out, n, stream=None):
    _check(load().q3k_silu_mul_bf16(_ptr(g), _ptr(u), _ptr(out), n, _ptr(stream)))


def rope(x, B, S, heads, D, cache, P, start, positions=None, stream=None):
    _check(load().q3k_rope_bf16(_ptr(x), B, S, heads, D, _ptr(cache), P, start, _ptr(positions), _ptr(stream)))


def rope_qk(q, k, B, S, Hq, Hkv, D, cache, P, start, positions=None, stream=None):
    _check(load().q3k_rope_qk_bf16(_ptr(q), _ptr(k), B, S, Hq, Hkv, D, _ptr(cache), P, start, _ptr(positions),
                                   _ptr(stream)))


def qk_norm_rope(q, k, qw, kw, B, S, Hq, Hkv, D, eps, cache, P, start, positions=None, stream=None):
    _check(load().q3k_qk_norm_rope_bf16(_ptr(q), _ptr(k), _ptr(qw), _ptr(kw), B, S, Hq, Hkv, D, eps,
                                        _ptr(cache), P, start, _ptr(positions), _ptr(stream)))


def gqa_attention(q, k_cache, v_cache, out, B, S, Hq, Hkv, D, cached, start, k_strides, v_strides, stream=None,
                  workspace=None, workspace_bytes=0):
    """k_strides / v_strides: 4 element strides (batch, position, head, dim) of the cache views."""
    ks = (ctypes.c_int64 * 4)(*[int(x) for x in k_strides])
    vs = (ctypes.c_int64 * 4)(*[int(x) for x in v_strides])
    _check(load().q3k_gqa_attention_bf16(_ptr(q), _ptr(k_cache), _ptr(v_cache), _ptr(out), B, S, Hq, Hkv, D, cached,
                                         start, ctypes.cast(ks, _p), ctypes.cast(vs, _p), _ptr(workspace),
                                         workspace_bytes, _ptr(stream)))


def gqa_attention_workspace_bytes(B, S, Hq, Hkv, D, cached):
    return int(load().q3k_gqa_attention_workspace_bytes(B, S, Hq, Hkv, D, cached))


def argmax(x, out, rows, row_stride, search_size, stream=None, workspace=None, workspace_bytes=0):
    _check(load().q3k_argmax_bf16(_ptr(x), _ptr(out), rows, row_stride, search_size, _ptr(workspace),
                                  workspace_bytes, _ptr(stream)))


def argmax_noalloc(x, out, rows, row_stride, search_size, stream=None):
    _check(load().q3k_argmax_bf16_noalloc(_ptr(x), _ptr(out), rows, row_stride, search_size, _ptr(stream)))


def argmax_workspace_bytes(rows, search_size):
    return int(load().q3k_argmax_workspace_bytes(rows, search_size))


def topk_candidates(logits, rows, row_stride, search_size, k, cap, count, cand_index, cand_logit, nonfinite,
                    stream=None, workspace=None, workspace_bytes=0):
    _check(load().q3k_topk_candidates_bf16(_ptr(logits), rows, row_stride, search_size, k, cap, _ptr(count),
                                           _ptr(cand_index), _ptr(cand_logit), _ptr(nonfinite), _ptr(workspace),
                                           workspace_bytes, _ptr(stream)))


def topk_workspace_bytes(rows, search_size, k):
    return int(load().q3k_topk_workspace_bytes(rows, search_size, k))


def kv_append(k, v, k_cache, v_cache, B, S, row_bytes, seq_cap, start, stream=None):
    _check(load().q3k_kv_append(_ptr(k), _ptr(v), _ptr(k_cache), _ptr(v_cache), B, S, row_bytes, seq_cap, start,
                                _ptr(stream)))


def qk_norm_rope_kv_append(q, k, v, qw, kw, B, S, Hq, Hkv, D, eps, cache, P, start, k_cache, v_cache, seq_cap,
                           cache_start, positions=None, stream=None):
    _check(load().q3k_qk_norm_rope_kv_append_bf16(_ptr(q), _ptr(k), _ptr(v), _ptr(qw), _ptr(kw), B, S, Hq, Hkv, D,
                                                  eps, _ptr(cache), P, start, _ptr(positions), _ptr(k_cache),
                                                  _ptr(v_cache), seq_cap, cache_start, _ptr(stream)))


def build_rope_cache(P: int, D: int, theta: float):
    """Host RoPE table [P, D/2, 2] as a float32 numpy array."""
    import numpy as np

    out = np.empty((P, D // 2, 2), dtype=np.float32)
    _check(load().q3k_build_rope_cache_f32(out.ctypes.data, P, D, theta))
    return out


def _need(buf, nbytes, what):
    """The C ABI takes bare addresses; a buffer object that knows its size is
    checked against the bytes the call will touch before anything launches."""
    have = getattr(buf, "nbytes", None)
    if buf is not None and have is not None and have < nbytes:
        raise ValueError(f"{what} holds {have} bytes, the call touches {nbytes}")


def bench_copy(src, dst, nbytes, stream=None):
    _need(src, nbytes, "bench_copy source")
    _need(dst, nbytes, "bench_copy destination")
    _check_bench(load_bench().q3k_bench_copy_u128(_ptr(src), _ptr(dst), nbytes, _ptr(stream)))


def bench_stream(in0, in1, out0, out1, nbytes, stream=None, threads=256):
    """out0 = in0 XOR in1, out1 = in0 + in1 (in1, out1 may be None) with 128-bit loads and stores, `threads`
    threads per block (q3k_bench.h)."""
    for buf, what in ((in0, "in0"), (in1, "in1"), (out0, "out0"), (out1, "out1")):
        _need(buf, nbytes, "bench_stream " + what)
    _check_bench(load_bench().q3k_bench_stream_u128(_ptr(in0), _ptr(in1), _ptr(out0), _ptr(out1), nbytes, threads,
                                                    _ptr(stream)))


def bench_read_rows(base, base2, outer, outer_stride, inner, inner_stride, rows, row_stride, row_bytes, sink,
                    stream=None):
    """Read ceiling of a strided row layout (q3k_bench.h); all sizes in bytes.  The kernel writes one 4-byte
    word per thread to sink: outer * inner * 256 words."""
    if outer > 0 and inner > 0 and rows > 0:
        last = (outer - 1) * outer_stride + (inner - 1) * inner_stride + (rows - 1) * row_stride + row_bytes
        _need(base, last, "bench_read_rows base")
        _need(base2, last, "bench_read_rows base2")
        _need(sink, outer * inner * 256 * 4, "bench_read_rows sink")
    _check_bench(load_bench().q3k_bench_read_rows_u128(_ptr(base), _ptr(base2), outer, outer_stride, inner, inner_stride, rows,
                                           row_stride, row_bytes, _ptr(sink), _ptr(stream)))
