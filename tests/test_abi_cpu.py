"""The C ABI library on the CPU: it loads, exports what the headers declare,
and rejects bad arguments with the documented status before touching the GPU.
No kernel is launched here."""
import ctypes
import subprocess

import numpy as np
import pytest


def test_library_exports_every_declared_symbol(q3k):
    lib = q3k.load()
    declared = q3k.declared_symbols()
    assert len(declared) >= 11
    for name in declared:
        assert hasattr(lib, name), f"{name} declared in include/ but not exported"
    assert set(declared) == set(q3k.SIGNATURES) | {"q3k_last_error_string", "q3k_version"}


def _exports(path):
    out = subprocess.run(["nm", "-D", "--defined-only", path], capture_output=True, text=True, check=True)
    return {line.split()[-1] for line in out.stdout.splitlines() if " T " in line}


def test_exports_are_only_the_abi(q3k):
    assert _exports(q3k.LIB_PATH) == set(q3k.declared_symbols())


def test_bench_library_exports_only_the_measurement_aids(q3k):
    """The measurement kernels live in lib/libq3k_bench.so, not in the product library."""
    declared = set(q3k.declared_symbols(q3k.BENCH_HEADERS))
    assert declared == set(q3k.BENCH_SIGNATURES) | {"q3k_bench_last_error_string"}
    assert _exports(q3k.BENCH_LIB_PATH) == declared
    assert not declared & _exports(q3k.LIB_PATH)


def test_version(q3k):
    assert q3k.version().count(".") == 2


def _expect(fn, exc, status, *args):
    with pytest.raises(exc) as info:
        fn(*args)
    assert info.value.status == status
    return str(info.value)


def test_argument_errors_without_gpu(q3k):
    IA, OR, OV = q3k.Q3K_ERR_INVALID_ARGUMENT, q3k.Q3K_ERR_OUT_OF_RANGE, q3k.Q3K_ERR_OVERFLOW
    fake = 256  # never dereferenced: every call below fails validation first
    # rms_norm: eps must be finite and positive (rms_norm.cu:209-214), N positive
    msg = _expect(q3k.rms_norm, ValueError, IA, fake, fake, fake, 4, 128, 0.0)
    assert "epsilon" in msg
    _expect(q3k.rms_norm, ValueError, IA, fake, fake, fake, 4, 128, float("nan"))
    _expect(q3k.rms_norm, ValueError, IA, fake, fake, fake, 4, 128, float("inf"))
    _expect(q3k.rms_norm, ValueError, IA, fake, fake, fake, 4, 0, 1e-6)
    _expect(q3k.rms_norm, ValueError, IA, None, fake, fake, 4, 128, 1e-6)
    _expect(q3k.rms_norm, OverflowError, OV, fake, fake, fake, 2**62, 2**10, 1e-6)
    _expect(q3k.add_rms_norm, ValueError, IA, fake, None, fake, fake, 4, 128, 1e-6)
    # elementwise
    _expect(q3k.silu_mul, ValueError, IA, fake, fake, None, 8)
    _expect(q3k.silu_mul, ValueError, IA, fake, fake, fake, -1)
    _expect(q3k.add_inplace, ValueError, IA, None, fake, 8)
    # embedding
    _expect(q3k.embedding, ValueError, IA, fake, 4, fake, 0, 8, fake)
    _expect(q3k.embedding, ValueError, IA, None, 4, fake, 10, 8, fake)
    # rope: negative start (rope.cu:190-194), range past the table (rope.cu:204-210)
    _expect(q3k.rope, ValueError, IA, fake, 1, 3, 2, 8, fake, 16, -1)
    msg = _expect(q3k.rope, IndexError, OR, fake, 1, 3, 2, 8, fake, 16, 15)
    assert "exceeds" in msg
    _expect(q3k.rope, ValueError, IA, fake, 1, 3, 0, 8, fake, 16, 0)
    _expect(q3k.rope, ValueError, IA, fake, 1, 3, 2, 7, fake, 16, 0)
    _expect(q3k.qk_norm_rope, IndexError, OR, fake, fake, fake, fake, 1, 3, 2, 1, 8, 1e-6, fake, 16, 14)
    _expect(q3k.qk_norm_rope, ValueError, IA, fake, fake, fake, fake, 1, 3, 2, 1, 8, -1.0, fake, 16, 0)
    _expect(q3k.qk_norm_rope, ValueError, IA, fake, fake, None, fake, 1, 3, 2, 1, 8, 1e-6, fake, 16, 0)
    # measurement aids
    _expect(q3k.bench_copy, ValueError, IA, fake, fake, 15)
    _expect(q3k.bench_read_rows, ValueError, IA, fake, None, 2, 4096, 2, 256, 8, 512, 24, fake)    # row not 2^k
    _expect(q3k.bench_read_rows, ValueError, IA, fake, None, 2, 4096, 2, 8, 8, 512, 256, fake)     # stride % 16
    _expect(q3k.bench_read_rows, ValueError, IA, None, None, 2, 4096, 2, 256, 8, 512, 256, fake)
    _expect(q3k.bench_read_rows, ValueError, IA, fake, None, -1, 4096, 2, 256, 8, 512, 256, fake)
    q3k.bench_read_rows(None, None, 0, 4096, 2, 256, 8, 512, 256, None)
    # grids past 2^32 - 1 work-items (256-thread blocks) are refused, not launched
    _expect(q3k.bench_copy, OverflowError, OV, fake, fake, 16 * 256 * (2**24))
    _expect(q3k.bench_stream, OverflowError, OV, fake, None, fake, None, 16 * 256 * (2**24))
    _expect(q3k.bench_stream, OverflowError, OV, fake, None, fake, None, 16 * 64 * (2**26), None, 64)
    for threads in (0, 32, 96, 2048):
        _expect(q3k.bench_stream, ValueError, IA, fake, None, fake, None, 4096, None, threads)
    q3k.bench_copy(None, None, 0)   # nothing to move: no launch
    _expect(q3k.bench_read_rows, OverflowError, OV, fake, None, 2**13, 16, 2**11, 16, 1, 16, 16, fake)


class _SizedFake:
    """A buffer object that knows its size but is never dereferenced."""

    def __init__(self, nbytes):
        self.ptr, self.nbytes = 256, nbytes


def test_bench_wrappers_refuse_buffers_smaller_than_the_call(q3k):
    """The measurement aids' C ABI takes bare addresses; the Python wrappers check a sized buffer object against
    the bytes the call reads or writes before calling it (the read kernel writes outer * inner * 256 words of
    sink)."""
    small, big = _SizedFake(1 << 20), _SizedFake(1 << 30)
    with pytest.raises(ValueError, match="sink"):
        q3k.bench_read_rows(big, None, 8, 1 << 20, 256, 256, 4, 2048, 256, small)   # 2048 views: 2 MiB of sink
    with pytest.raises(ValueError, match="base"):
        q3k.bench_read_rows(small, None, 64, 1 << 20, 8, 256, 4096, 2048, 256, big)
    with pytest.raises(ValueError, match="destination"):
        q3k.bench_copy(big, small, 1 << 21)
    with pytest.raises(ValueError, match="out1"):
        q3k.bench_stream(big, big, big, small, 1 << 21)


def test_empty_inputs_are_no_ops(q3k):
    # zero work returns OK without a launch (no GPU needed)
    q3k.rms_norm(None, None, None, 0, 128, 1e-6)
    q3k.add_rms_norm(None, None, None, None, 0, 128, 1e-6)
    q3k.silu_mul(None, None, None, 0)
    q3k.add_inplace(None, None, 0)
    q3k.embedding(None, 0, None, 10, 8, None)
    q3k.rope(None, 0, 5, 2, 8, None, 16, 0)
    q3k.qk_norm_rope(None, None, None, None, 3, 0, 2, 1, 8, 1e-6, None, 16, 0)


def test_rope_cache_builder_matches_oracle(q3k, oracle):
    for P, D, theta in ((16, 8, 1.0e6), (2048, 128, 1.0e6), (33, 64, 10000.0)):
        ours = q3k.build_rope_cache(P, D, theta)
        ref = oracle.build_rope_cache(P, D, theta)
        assert ours.shape == (P, D // 2, 2)
        assert np.array_equal(ours.view(np.uint32), ref.view(np.uint32))
    with pytest.raises(ValueError):
        q3k.build_rope_cache(0, 128, 1e6)
    with pytest.raises(ValueError):
        q3k.build_rope_cache(4, 7, 1e6)
    with pytest.raises(ValueError):
        q3k.build_rope_cache(4, 8, float("inf"))


def test_error_string_is_thread_local(q3k):
    import threading

    lib = q3k.load()
    lib.q3k_rms_norm_bf16(None, None, None, 1, 0, ctypes.c_float(1e-6), None)
    seen = {}

    def other():
        seen["msg"] = lib.q3k_last_error_string().decode()

    t = threading.Thread(target=other)
    t.start()
    t.join()
    assert seen["msg"] == "no error"
    assert "normalized size" in lib.q3k_last_error_string().decode()


def test_caller_fusion_argument_errors(q3k):
    IA, OV = q3k.Q3K_ERR_INVALID_ARGUMENT, q3k.Q3K_ERR_OVERFLOW
    fake = 256
    _expect(q3k.rms_norm_rows, ValueError, IA, fake, fake, fake, 4, -1, 8, 1024, 1e-6)
    _expect(q3k.rms_norm_rows, ValueError, IA, fake, fake, fake, 4, 0, -8, 1024, 1e-6)
    _expect(q3k.add_rms_norm_rows, OverflowError, OV, fake, fake, fake, fake, 4, 2**61, 1, 1024, 1e-6)
    _expect(q3k.add_rms_norm_rows, ValueError, IA, fake, None, fake, fake, 4, 0, 1, 1024, 1e-6)
    # the residual add writes its rows back, so they must be distinct rows
    _expect(q3k.add_rms_norm_rows, ValueError, IA, fake, fake, fake, fake, 2, 0, 0, 1024, 1e-6)
    _expect(q3k.add_rms_norm_rows, ValueError, IA, fake, fake, fake, fake, 1 << 20, 5, 0, 1024, 1e-6)
    q3k.add_rms_norm_rows(None, None, None, None, 0, 3, 0, 1024, 1e-6)
    _expect(q3k.embedding_rms_norm, ValueError, IA, fake, 4, fake, 0, 1024, fake, 1e-6, fake, fake)
    _expect(q3k.embedding_rms_norm, ValueError, IA, None, 4, fake, 10, 1024, fake, 1e-6, fake, fake)
    _expect(q3k.embedding_rms_norm, ValueError, IA, fake, 4, fake, 10, 1024, fake, 0.0, fake, fake)
    q3k.rms_norm_rows(None, None, None, 0, 0, 1, 1024, 1e-6)
    q3k.embedding_rms_norm(None, 0, None, 10, 1024, None, 1e-6, None, None)


def test_kv_and_attention_argument_errors(q3k):
    IA, OR, OV = q3k.Q3K_ERR_INVALID_ARGUMENT, q3k.Q3K_ERR_OUT_OF_RANGE, q3k.Q3K_ERR_OVERFLOW
    fake = 256
    # KV append: capacity (kv_cache.cpp:121-125), sizes, null pointers
    msg = _expect(q3k.kv_append, IndexError, OR, fake, fake, fake, fake, 2, 5, 2048, 8, 4)
    assert "capacity" in msg
    _expect(q3k.kv_append, ValueError, IA, fake, fake, fake, fake, -1, 5, 2048, 8, 0)
    _expect(q3k.kv_append, ValueError, IA, fake, fake, fake, fake, 2, 5, 0, 8, 0)
    _expect(q3k.kv_append, ValueError, IA, None, fake, fake, fake, 2, 5, 2048, 8, 0)
    _expect(q3k.kv_append, OverflowError, OV, fake, fake, fake, fake, 2**40, 1, 2**20, 2**10, 0)
    q3k.kv_append(None, None, None, None, 0, 5, 2048, 8, 0)
    # fused Q/K norm + RoPE + append: RoPE range first, then the cache capacity
    _expect(q3k.qk_norm_rope_kv_append, IndexError, OR, fake, fake, fake, fake, fake, 1, 3, 2, 1, 8, 1e-6, fake, 16, 14,
            fake, fake, 64, 0)
    _expect(q3k.qk_norm_rope_kv_append, IndexError, OR, fake, fake, fake, fake, fake, 1, 3, 2, 1, 8, 1e-6, fake, 16, 0,
            fake, fake, 4, 2)
    _expect(q3k.qk_norm_rope_kv_append, ValueError, IA, fake, fake, None, fake, fake, 1, 3, 2, 1, 8, 1e-6, fake, 16, 0,
            fake, fake, 8, 0)
    # attention (gqa_attention.cu:157-302)
    st = (64, 16, 8, 1)
    msg = _expect(q3k.gqa_attention, ValueError, IA, fake, fake, fake, fake, 1, 2, 4, 2, 8, 5, 1, st, st)
    assert "start_position + sequence_length" in msg
    _expect(q3k.gqa_attention, ValueError, IA, fake, fake, fake, fake, 1, 2, 3, 2, 8, 3, 1, st, st)
    _expect(q3k.gqa_attention, ValueError, IA, fake, fake, fake, fake, 1, 2, 4, 2, 512, 3, 1, st, st)
    _expect(q3k.gqa_attention, ValueError, IA, fake, fake, fake, fake, 1, 2, 4, 2, 8, 1, -1, st, st)
    _expect(q3k.gqa_attention, ValueError, IA, None, fake, fake, fake, 1, 2, 4, 2, 8, 3, 1, st, st)
    _expect(q3k.gqa_attention, OverflowError, OV, fake, fake, fake, fake, 2**20, 2**10, 4, 2, 8, 2**10, 0, st, st)
    q3k.gqa_attention(None, None, None, None, 0, 2, 4, 2, 8, 3, 1, st, st)


def test_argmax_argument_errors(q3k):
    IA = q3k.Q3K_ERR_INVALID_ARGUMENT
    fake = 256
    _expect(q3k.argmax, ValueError, IA, fake, fake, 2, 0, 0)
    _expect(q3k.argmax, ValueError, IA, fake, fake, 2, 2**31, 2**31)
    msg = _expect(q3k.argmax, ValueError, IA, fake, fake, 2, 100, 101)
    assert "valid reduction size" in msg
    _expect(q3k.argmax, ValueError, IA, None, fake, 2, 100, 100)
    msg = _expect(q3k.argmax, ValueError, IA, fake, fake, 2, 100, 100, None, fake, -8)
    assert "workspace" in msg
    q3k.argmax(None, None, 0, 100, 100)


def test_selection_workspace_plans(q3k):
    """Argmax and top-k ask for a workspace only when the rows are too few to fill the GPU (and, for top-k, k fits
    the bound step); the size covers one 8-byte key per slice, or a header and a list per slice."""
    V = 151936
    ws = q3k.argmax_workspace_bytes(64, V)
    assert ws > 0 and ws % (64 * 8) == 0 and 2 <= ws // (64 * 8) <= 64
    assert q3k.argmax_workspace_bytes(1, V) > 0
    assert q3k.argmax_workspace_bytes(512, V) == 0        # enough rows: one block per row
    assert q3k.argmax_workspace_bytes(4, 10000) == 0      # a row too short to cut
    assert q3k.argmax_workspace_bytes(0, V) == 0
    tk = q3k.topk_workspace_bytes(64, V, 20)
    assert tk > 0 and tk % 64 == 0
    assert q3k.topk_workspace_bytes(64, V, 1024) == tk    # the size does not depend on k up to the thread count
    assert q3k.topk_workspace_bytes(64, V, 1025) == 0     # k above the thread count: whole-row select
    assert q3k.topk_workspace_bytes(600, V, 20) == 0
    IA = q3k.Q3K_ERR_INVALID_ARGUMENT
    fake = 256
    msg = _expect(q3k.topk_candidates, ValueError, IA, fake, 2, 100, 100, 5, 8, fake, fake, fake, fake, None, fake,
                  -1)
    assert "workspace" in msg
