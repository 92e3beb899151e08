"""Fallback guards, second line: the head layouts of the Qwen3 family and of their tensor-parallel shards must run
on the fast kernels, not on the generic ones.  The launchers' decisions themselves are checked on the host,
deterministically, by tests/cpp/dispatch_cpu_test.cpp (csrc/kernels/dispatch.hpp is the only place they are made).
This file checks the same on the device through time: the generic kernels give the same results (the parity tests
cover both), but at these sizes the generic Q/K path ran 8x and the generic attention ~165x slower than the fast
ones.  The floors sit far below the fast kernels (3-6x) and far above the generic ones."""
import numpy as np
import pytest

from gpu_util import announce

D = 128
EPS = 1.0e-6
# (query heads, KV heads): Qwen3 0.6B/1.7B, 4B/8B, 14B, 32B, and one rank of 8-way tensor parallelism of each
HEADS = [(16, 8), (32, 8), (40, 8), (64, 8), (2, 1), (4, 1), (5, 1), (8, 1)]
QK_FLOOR_GBS = 1000.0      # fast: 2500-6200 GB/s here; the generic fallback: ~400
ATTN_FLOOR_TFLOPS = 20.0   # fast: 80-700 TFLOP/s here; the generic fallback: ~4


def _time_us(hip, stream, fn, calls=20, warmup=3):
    for _ in range(warmup):
        fn()
    stream.synchronize()
    e0, e1 = hip.Event(), hip.Event()
    e0.record(stream)
    for _ in range(calls):
        fn()
    e1.record(stream)
    e1.synchronize()
    return e0.elapsed_ms(e1) * 1e3 / calls


@pytest.mark.gpu
@pytest.mark.parametrize("Hq,Hkv", HEADS)
def test_qk_norm_rope_fast_path(q3k, hip, synth, Hq, Hkv):
    B, S = 4, 2048
    announce(f"qk_norm_rope path B={B} S={S} Hq={Hq} Hkv={Hkv}")
    stream = hip.Stream()
    q = hip.DeviceBuffer.from_array(synth.normal_bf16(190, Hq, (B, S, Hq * D)))
    k = hip.DeviceBuffer.from_array(synth.normal_bf16(191, Hkv, (B, S, Hkv * D)))
    qw = hip.DeviceBuffer.from_array(synth.normal_bf16(192, D, (D,), mean=1.0, std=0.1))
    kw = hip.DeviceBuffer.from_array(synth.normal_bf16(193, D, (D,), mean=1.0, std=0.1))
    cache = hip.DeviceBuffer.from_array(q3k.build_rope_cache(S, D, 1.0e6))
    us = _time_us(hip, stream, lambda: q3k.qk_norm_rope(q, k, qw, kw, B, S, Hq, Hkv, D, EPS, cache, S, 0, None,
                                                          stream))
    gbs = 2 * B * S * (Hq + Hkv) * D * 2 / (us * 1e-6) / 1e9
    print(f"[path] qk_norm_rope Hq={Hq} Hkv={Hkv}: {us:.1f} us, {gbs:.0f} GB/s", flush=True)
    for buf in (q, k, qw, kw, cache):
        buf.free()
    stream.destroy()
    assert gbs > QK_FLOOR_GBS, f"qk_norm_rope at {Hq}/{Hkv} heads ran at {gbs:.0f} GB/s: a generic fallback?"


@pytest.mark.gpu
@pytest.mark.parametrize("Hq,Hkv", HEADS)
def test_attention_prefill_fast_path(q3k, hip, synth, Hq, Hkv):
    B, S = 2, 2048
    announce(f"attention path B={B} S={S} Hq={Hq} Hkv={Hkv}")
    stream = hip.Stream()
    q = hip.DeviceBuffer.from_array(synth.normal_bf16(194, Hq, (B, S, Hq * D)))
    k = hip.DeviceBuffer.from_array(synth.normal_bf16(195, Hkv, (B, S, Hkv, D)))
    v = hip.DeviceBuffer.from_array(synth.normal_bf16(196, Hkv, (B, S, Hkv, D)))
    out = hip.DeviceBuffer(B * S * Hq * D * 2)
    st = (S * Hkv * D, Hkv * D, D, 1)
    wb = q3k.gqa_attention_workspace_bytes(B, S, Hq, Hkv, D, S)
    ws = hip.DeviceBuffer(wb) if wb else None
    us = _time_us(hip, stream, lambda: q3k.gqa_attention(q, k, v, out, B, S, Hq, Hkv, D, S, 0, st, st, stream,
                                                          workspace=ws, workspace_bytes=wb), calls=5, warmup=1)
    tflops = 4 * D * B * Hq * S * (S + 1) / 2 / (us * 1e-6) / 1e12
    print(f"[path] attention prefill Hq={Hq} Hkv={Hkv}: {us:.1f} us, {tflops:.1f} TFLOP/s", flush=True)
    got = out.download(np.uint16, (B * S * Hq * D,))
    for buf in (q, k, v, out) + ((ws,) if ws else ()):
        buf.free()
    stream.destroy()
    assert np.isfinite(synth.bf16_to_f32(got)).all()
    assert tflops > ATTN_FLOOR_TFLOPS, f"attention at {Hq}/{Hkv} heads ran at {tflops:.1f} TFLOP/s: a generic fallback?"
