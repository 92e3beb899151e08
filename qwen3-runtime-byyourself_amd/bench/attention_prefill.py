"""Causal GQA attention prefill alone, for profiling under rocprofv3: the
matrix-core path of q3k_gqa_attention_bf16 (src/ops/gqa_attention.cu:20-155 of
the reference) at Qwen3-8B heads (32 query, 8 key/value, head_dim 128) over a
synthetic [B, S] batch whose keys are the batch's own positions (start 0).

Prints one line per timed pass: microseconds per call and TFLOP/s, counting
4 * head_dim flops per visible (query, key) pair (Q K^T and P V), against the
2.5 PFLOP/s dense bf16 peak of MI355X.

Usage: python3 attention_prefill.py [--batch 4] [--seq 2048] [--calls 10] [--passes 3]
"""
import argparse
import importlib
import os
import sys

PKG_PARENT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
PEAK_BF16_TFLOPS = 2500.0
HQ, HKV, D = 32, 8, 128


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--batch", type=int, default=4)
    ap.add_argument("--seq", type=int, default=2048)
    ap.add_argument("--calls", type=int, default=10)
    ap.add_argument("--passes", type=int, default=3)
    args = ap.parse_args()
    sys.path.insert(0, PKG_PARENT)
    q3k = importlib.import_module("qwen3-runtime-byyourself_amd")
    hip = importlib.import_module("qwen3-runtime-byyourself_amd.hip")
    synth = importlib.import_module("qwen3-runtime-byyourself_amd.synth")
    q3k.load()
    B, S = args.batch, args.seq
    stream = hip.Stream()
    q = hip.DeviceBuffer.from_array(synth.normal_bf16(4, 40, (B, S, HQ * D)))
    k = hip.DeviceBuffer.from_array(synth.normal_bf16(4, 41, (B, S, HKV, D)))
    v = hip.DeviceBuffer.from_array(synth.normal_bf16(4, 42, (B, S, HKV, D)))
    out = hip.DeviceBuffer(B * S * HQ * D * 2)
    strides = (S * HKV * D, HKV * D, D, 1)

    def call():
        q3k.gqa_attention(q, k, v, out, B, S, HQ, HKV, D, S, 0, strides, strides, stream)

    flops = 4 * D * B * HQ * S * (S + 1) // 2
    for _ in range(3):
        call()
    stream.synchronize()
    for p in range(args.passes):
        e0, e1 = hip.Event(), hip.Event()
        e0.record(stream)
        for _ in range(args.calls):
            call()
        e1.record(stream)
        e1.synchronize()
        us = e0.elapsed_ms(e1) * 1e3 / args.calls
        tf = flops / (us * 1e-6) / 1e12
        print(f"attention prefill B={B} S={S} Hq={HQ} Hkv={HKV} D={D} pass {p}: {us:.1f} us/call, "
              f"{tf:.1f} TFLOP/s = {100 * tf / PEAK_BF16_TFLOPS:.2f}% of dense bf16", flush=True)
    for buf in (q, k, v, out):
        buf.free()
    stream.destroy()
    return 0


if __name__ == "__main__":
    sys.exit(main())
