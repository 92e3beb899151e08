#!/usr/bin/env python3
"""Benchmark: HBM throughput of the Qwen3 decoder layer's non-GEMM chain on
one MI355X (gfx950), through the C ABI of libq3k.so.

A step is one pass of the per-layer non-GEMM chain over one batch of
synthetic input at benchmark config 4 (Qwen3-8B prefill, T = 8192 tokens as
4 sequences x 2048, positions 0..2047 per sequence):

  add_rms_norm  h1 += d1; y1 = rmsnorm(h1)     [8192, 4096]   attention residual + post-attention norm
  qk_norm_rope  Q [8192, 32, 128], K [8192, 8, 128]           per-head norm + RoPE, in place
  add_rms_norm  h2 += d2; y2 = rmsnorm(h2)     [8192, 4096]   MLP residual + next layer's input norm
  silu_mul      o = silu(g) * u                [8192, 12288]

Every tensor of a step is distinct and the steps rotate over six full input
sets (6 x 1.31 GB; the smallest per-op cycle, 6 x 80 MB of Q/K, is still far
above the 256 MB Infinity Cache), so each launch reads its inputs from HBM.  ``value`` is the chain's algorithmic bytes (each
compulsory byte once) divided by the measured time per step, inputs already
resident in HBM.  Per-kernel durations come from back-to-back launches of
each kernel alone between one pair of HIP events, rotating over copies of
its buffers whose cycle exceeds 1.5 GiB (so none is served from the cache).

Also reported (not part of ``value``): the embedding gather and the final
RMSNorm at config 4, the same chain built from the unfused drop-in ops in
the reference's order, each op's own access-pattern ceiling at its size, a
128-bit copy ceiling, the other benchmark configs (1: RMSNorm [16, 1024];
2: the Qwen3-0.6B chain with its embedding gather; 3: the decode step; 5:
Qwen3-32B shapes), attention, token selection, weight IO, and the CPU
baseline (the oracle's restatement of the reference's CPU arithmetic, timed
on this host).

Usage: python bench.py [--gpus 1] [--steps 50] [--warmup 10] [--no-cpu-baseline]
"""
from __future__ import annotations

import argparse
import dataclasses
import importlib
import importlib.util
import json
import os
import platform
import re
import sys
import time

import numpy as np

REPO = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, REPO)
PKG = "qwen3-runtime-byyourself_amd"
METRIC = "HBM GB/s (% of peak) for RMSNorm/QK-norm+RoPE/SwiGLU at Qwen3-8B shapes"
PEAK_GBS = 8000.0
PEAK_BF16_TFLOPS = 2500.0  # MI355X dense bf16 matrix-core peak
EPS = 1e-6
D = 128


def parse_args():
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--config", default="c4")
    ap.add_argument("--sets", type=int, default=6,
                    help="rotating input sets (6: even the smallest per-op cycle, 6 x 80 MB, exceeds the 256 MB cache)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--no-extras", action="store_true", help="chain only (no embedding/final-norm/unfused/copy)")
    return ap.parse_args()


def make_chain_set(hip, synth, configs, c, q3k, seed_shift=0):
    T, H, I = c.tokens, c.hidden, c.inter
    s = c.seed
    DB = hip.DeviceBuffer.from_array
    bufs = {
        "h1": DB(synth.normal_bf16(s, configs.TID_H, (T, H))),
        "d1": DB(synth.normal_bf16(s, configs.TID_D1, (T, H))),
        "w1": DB(synth.normal_bf16(s, configs.TID_W1, (H,), mean=1.0, std=0.1)),
        "y1": hip.DeviceBuffer(T * H * 2),
        "q": DB(synth.normal_bf16(s, configs.TID_Q, (T, c.heads_q * D))),
        "k": DB(synth.normal_bf16(s, configs.TID_K, (T, c.heads_kv * D))),
        "qw": DB(synth.normal_bf16(s, configs.TID_QW, (D,), mean=1.0, std=0.1)),
        "kw": DB(synth.normal_bf16(s, configs.TID_KW, (D,), mean=1.0, std=0.1)),
        "h2": DB(synth.normal_bf16(s, configs.TID_H2, (T, H))),
        "d2": DB(synth.normal_bf16(s, configs.TID_D2, (T, H))),
        "w2": DB(synth.normal_bf16(s, configs.TID_W2, (H,), mean=1.0, std=0.1)),
        "y2": hip.DeviceBuffer(T * H * 2),
        "g": DB(synth.normal_bf16(s, configs.TID_GATE, (T, I))),
        "u": DB(synth.normal_bf16(s, configs.TID_UP, (T, I))),
        "o": hip.DeviceBuffer(T * I * 2),
        # the unfused chain's normalised Q and K (rms_norm returns new tensors, self_attention.cpp:147-149)
        "qn": hip.DeviceBuffer(T * c.heads_q * D * 2),
        "kn": hip.DeviceBuffer(T * c.heads_kv * D * 2),
        "cache": DB(q3k.build_rope_cache(c.max_pos, D, configs.THETA)),
    }
    if c.positions == "uniform":   # one position per sequence (config 3): the Int32 positions overload
        bufs["pos"] = DB(synth.uniform_positions(s, configs.TID_POS, T, c.max_pos))
    return bufs


def clone_set(hip, src):
    out = {}
    for k, b in src.items():
        nb = hip.DeviceBuffer(b.nbytes)
        nb.copy_from(b)
        out[k] = nb
    return out


def chain_ops(q3k, c, b, stream):
    T, H = c.tokens, c.hidden
    return [
        ("add_rms_norm_attn", lambda: q3k.add_rms_norm(b["h1"], b["d1"], b["w1"], b["y1"], T, H, EPS, stream)),
        ("qk_norm_rope", lambda: q3k.qk_norm_rope(b["q"], b["k"], b["qw"], b["kw"], c.batch, c.seq, c.heads_q,
                                                  c.heads_kv, D, EPS, b["cache"], c.max_pos, 0, b.get("pos"), stream)),
        ("add_rms_norm_mlp", lambda: q3k.add_rms_norm(b["h2"], b["d2"], b["w2"], b["y2"], T, H, EPS, stream)),
        ("silu_mul", lambda: q3k.silu_mul(b["g"], b["u"], b["o"], T * c.inter, stream)),
    ]


def unfused_ops(q3k, c, b, stream):
    """The same chain through the drop-in ops in the reference's order
    (decoder_layer.cpp:78->88, self_attention.cpp:147-152, mlp.cpp:111, :94->:72)."""
    T, H = c.tokens, c.hidden
    return [
        ("add_inplace", lambda: q3k.add_inplace(b["h1"], b["d1"], T * H, stream)),
        ("rms_norm", lambda: q3k.rms_norm(b["h1"], b["w1"], b["y1"], T, H, EPS, stream)),
        ("rms_norm_q", lambda: q3k.rms_norm(b["q"], b["qw"], b["qn"], T * c.heads_q, D, EPS, stream)),
        ("rms_norm_k", lambda: q3k.rms_norm(b["k"], b["kw"], b["kn"], T * c.heads_kv, D, EPS, stream)),
        # apply_rope_inplace on the normalised Q and K: one launch over both (the reference makes two,
        # rope.cu:326-332)
        ("rope", lambda: q3k.rope_qk(b["qn"], b["kn"], c.batch, c.seq, c.heads_q, c.heads_kv, D, b["cache"],
                                     c.max_pos, 0, b.get("pos"), stream)),
        ("add_inplace_2", lambda: q3k.add_inplace(b["h2"], b["d2"], T * H, stream)),
        ("rms_norm_2", lambda: q3k.rms_norm(b["h2"], b["w2"], b["y2"], T, H, EPS, stream)),
        ("silu_mul", lambda: q3k.silu_mul(b["g"], b["u"], b["o"], T * c.inter, stream)),
    ]


def time_chain(hip, stream, sets, make_ops, steps, warmup):
    """Warm up, then time `steps` passes of the op list (rotating over the
    input sets) between one pair of events; returns ms per pass."""
    per_set = [make_ops(s) for s in sets]
    for i in range(warmup):
        for _, fn in per_set[i % len(sets)]:
            fn()
    start, stop = hip.Event(), hip.Event()
    hip.synchronize()
    start.record(stream)
    for i in range(steps):
        for _, fn in per_set[i % len(sets)]:
            fn()
    stop.record(stream)
    stop.synchronize()
    hip.synchronize()
    return start.elapsed_ms(stop) / steps


def time_chain_graph(hip, stream, sets, make_ops, steps, warmup):
    """The chain over every input set captured into one HIP graph (one host
    launch per cycle of the sets, as a serving loop replays a captured decode
    step), replayed between one pair of events; returns ms per pass."""
    per_set = [make_ops(s) for s in sets]

    def record():
        for ops in per_set:
            for _, fn in ops:
                fn()

    graph = hip.Graph(stream, record)
    try:
        cycles = max(1, -(-steps // len(sets)))
        for _ in range(max(1, -(-warmup // len(sets)))):
            graph.launch(stream)
        start, stop = hip.Event(), hip.Event()
        hip.synchronize()
        start.record(stream)
        for _ in range(cycles):
            graph.launch(stream)
        stop.record(stream)
        stop.synchronize()
        hip.synchronize()
        return start.elapsed_ms(stop) / (cycles * len(sets))
    finally:
        graph.destroy()


# Buffers each chain op touches (for its own rotation when timed alone).
OP_BUFFERS = {
    "add_rms_norm_attn": ("h1", "d1", "y1"),
    "qk_norm_rope": ("q", "k"),
    "add_rms_norm_mlp": ("h2", "d2", "y2"),
    "silu_mul": ("g", "u", "o"),
}
UNFUSED_BUFFERS = {
    "add_inplace": ("h1", "d1"), "rms_norm": ("h1", "y1"), "rms_norm_q": ("q", "qn"), "rms_norm_k": ("k", "kn"),
    "rope": ("qn", "kn"), "add_inplace_2": ("h2", "d2"), "rms_norm_2": ("h2", "y2"),
    "silu_mul": ("g", "u", "o"),
}
MIN_CYCLE_BYTES = 3 << 29  # 1.5 GiB: 6x the 256 MB Infinity Cache


def op_rotation(hip, sets, keys):
    """Input sets for timing one op alone: enough copies of the op's own
    buffers that one cycle over them exceeds MIN_CYCLE_BYTES (so no launch
    finds its inputs in the Infinity Cache); other buffers are shared."""
    per_set = sum(sets[0][k].nbytes for k in keys)
    need = max(len(sets), -(-MIN_CYCLE_BYTES // per_set))
    out = list(sets)
    while len(out) < need:
        extra = dict(sets[0])
        for k in keys:
            extra[k] = hip.DeviceBuffer(sets[0][k].nbytes)
            extra[k].copy_from(sets[len(out) % len(sets)][k])
        out.append(extra)
    return out


# Block sizes the stream aid is timed at; a ceiling is the best of them (the block size alone moves a
# 2-in-1-out stream of 201 MB from 78% to 82% of peak on MI355X).
CEILING_THREADS = (64, 128, 256, 1024)


def pattern_ceiling(hip, q3k, stream, nbytes, n_in, n_out, in_place, reps):
    """GB/s of the stream aid (q3k_bench_stream_u128) with n_in input and n_out output streams of nbytes each,
    the first output written over the first input when in_place, back to back over enough buffer sets that one
    cycle exceeds MIN_CYCLE_BYTES (contents are whatever the allocations hold: nothing depends on them); the
    best over the block sizes of CEILING_THREADS.  Returns (GB/s, threads per block of the best)."""
    n_bufs = n_in + n_out - (1 if in_place else 0)
    count = max(2, -(-MIN_CYCLE_BYTES // (nbytes * n_bufs)))
    rot = []
    for _ in range(count):
        bufs = [hip.DeviceBuffer(nbytes) for _ in range(n_bufs)]
        ins = bufs[:n_in] + [None] * (2 - n_in)
        outs = ([bufs[0]] if in_place else []) + bufs[n_in:]
        outs = outs + [None] * (2 - len(outs))
        rot.append((ins[0], ins[1], outs[0], outs[1]))
    best = None
    for threads in CEILING_THREADS:
        ms = time_chain(hip, stream, rot,
                        lambda r, t=threads: [("stream", lambda: q3k.bench_stream(*r, nbytes, stream, threads=t))],
                        max(reps, len(rot)), 2)
        if best is None or ms < best[0]:
            best = (ms, threads)
    for r in rot:
        for buf in {id(x): x for x in r if x is not None}.values():
            buf.free()
    return (n_in + n_out) * nbytes / (best[0] * 1e-3) / 1e9, best[1]


def time_each_op(hip, stream, sets, make_ops, reps, warmup=2, buffers=None):
    """Per-op duration: `reps` back-to-back launches of one op, rotating over
    input sets whose cycle exceeds the Infinity Cache (so every launch reads
    from HBM), between one pair of events; returns {op: ms per launch}."""
    out = {}
    for k, (name, _) in enumerate(make_ops(sets[0])):
        rot = op_rotation(hip, sets, buffers[name]) if buffers and name in buffers else sets
        out[name] = time_chain(hip, stream, rot, lambda s, k=k: [make_ops(s)[k]], max(reps, len(rot)), warmup)
        del rot
    return out


def attention_flops(B, S, start, Hq, D):
    """Algorithmic flops of causal attention: 2 * D for Q K^T and 2 * D for P V per visible (query, key) pair."""
    pairs = B * Hq * (S * start + S * (S + 1) // 2)
    return 4 * D * pairs


def time_attention(q3k, hip, synth, c, stream):
    """Grouped-query attention over the layer's KV cache (gqa_attention.cu:304-345): prefill at the config's
    [B, S] (matrix-core bound, reported in TFLOP/s against the 2.5 PFLOP/s bf16 peak) and a batched decode step
    at 64 sequences x 4096 cached keys (HBM bound: the K/V cache is read once).  The prefill is also timed with
    Qwen3-14B's 40 query heads over 8 KV heads (a group size of 5, which does not divide a wave's 32 columns)."""
    out = {}
    print("[bench] timing attention", file=sys.stderr, flush=True)
    for name, B, S, start, Hq, Hkv in (("prefill", c.batch, c.seq, 0, c.heads_q, c.heads_kv),
                                       ("prefill_40q_8kv", c.batch, c.seq, 0, 40, 8),
                                       ("decode_b64_l4096", 64, 1, 4095, c.heads_q, c.heads_kv),
                                       ("decode_b1_l4096", 1, 1, 4095, c.heads_q, c.heads_kv)):
        L = start + S
        q = hip.DeviceBuffer.from_array(synth.normal_bf16(c.seed, 40, (B, S, Hq * D)))
        kc = hip.DeviceBuffer.from_array(synth.normal_bf16(c.seed, 41, (B, L, Hkv, D)))
        vc = hip.DeviceBuffer.from_array(synth.normal_bf16(c.seed, 42, (B, L, Hkv, D)))
        o = hip.DeviceBuffer(B * S * Hq * D * 2)
        st = (L * Hkv * D, Hkv * D, D, 1)
        wb = q3k.gqa_attention_workspace_bytes(B, S, Hq, Hkv, D, L)
        ws = hip.DeviceBuffer(wb) if wb else None   # a launch too small for the GPU splits the key range
        ms = time_chain(hip, stream, [0], lambda _: [
            ("attention", lambda: q3k.gqa_attention(q, kc, vc, o, B, S, Hq, Hkv, D, L, start, st, st,
                                                    stream, workspace=ws, workspace_bytes=wb))],
                        50, 50 if S > 1 else 5)
        flops = attention_flops(B, S, start, Hq, D)
        byts = 2 * B * L * Hkv * D * 2 + 2 * B * S * Hq * D * 2
        rec = {"ms": round(ms, 5), "B": B, "S": S, "cached": L, "heads_q": Hq, "heads_kv": Hkv, "TFLOP/s": round(flops / (ms * 1e-3) / 1e12, 1),
               "GB/s": round(byts / (ms * 1e-3) / 1e9, 1)}
        if S > 1:
            rec["pct_of_bf16_peak"] = round(100 * flops / (ms * 1e-3) / 1e12 / PEAK_BF16_TFLOPS, 2)
        else:
            rec["pct_of_hbm_peak"] = round(100 * byts / (ms * 1e-3) / 1e9 / PEAK_GBS, 2)
            if B >= 64:
                # the same K/V rows read by a kernel that only reads them: the HBM
                # ceiling of this access pattern at this grid
                sink = hip.DeviceBuffer(B * Hkv * 256 * 4)
                ms_r = time_chain(hip, stream, [0], lambda _: [("read", lambda: q3k.bench_read_rows(
                    kc, vc, B, L * Hkv * D * 2, Hkv, D * 2, L, Hkv * D * 2, D * 2, sink,
                    stream))], 50, 2)
                kv_bytes = 2 * B * L * Hkv * D * 2
                rec["read_ceiling_GB/s"] = round(kv_bytes / (ms_r * 1e-3) / 1e9, 1)
                rec["pct_of_read_ceiling"] = round(100 * ms_r / ms, 1)
                sink.free()
        rec["key_splits"] = wb > 0
        out["attention_" + name] = rec
        for buf in (q, kc, vc, o) + ((ws,) if ws else ()):
            buf.free()
    return out


def time_sampling(q3k, hip, synth, configs, c, stream):
    """Next-token selection over [B, 151936] bf16 logits of a decode step (B = 64 and 1): greedy argmax
    (argmax.cu:34-100) and the GPU top-k candidate selection of sampling (top_k 20), with the workspace the library
    asks for (rows cut into slices when they are too few to fill the GPU).  The same logits are read every launch,
    so after the first they come from the 256 MB Infinity Cache, as they would right after the LM-head GEMM that
    writes them."""
    out = {}
    print("[bench] timing argmax / top-k", file=sys.stderr, flush=True)
    V, cap, k = configs.VOCAB, 1024, 20
    for B in (64, 1):
        x = hip.DeviceBuffer.from_array(synth.normal_bf16(c.seed, 43, (B, V), std=3.0))
        ids = hip.DeviceBuffer(B * 4)
        cnt, bad = hip.DeviceBuffer(B * 4), hip.DeviceBuffer(B * 4)
        ci, cv = hip.DeviceBuffer(B * cap * 4), hip.DeviceBuffer(B * cap * 2)
        wa = q3k.argmax_workspace_bytes(B, V)
        wk = q3k.topk_workspace_bytes(B, V, k)
        ws_a = hip.DeviceBuffer(wa) if wa else None
        ws_k = hip.DeviceBuffer(wk) if wk else None
        ms_a = time_chain(hip, stream, [0], lambda _: [("argmax", lambda: q3k.argmax(
            x, ids, B, V, V, stream, workspace=ws_a, workspace_bytes=wa))], 50, 5)
        ms_k = time_chain(hip, stream, [0], lambda _: [("topk", lambda: q3k.topk_candidates(
            x, B, V, V, k, cap, cnt, ci, cv, bad, stream, workspace=ws_k, workspace_bytes=wk))], 50, 5)
        nb = B * V * 2
        out[f"argmax_b{B}_v{V}"] = {"ms": round(ms_a, 5), "bytes": nb, "GB/s": round(nb / (ms_a * 1e-3) / 1e9, 1),
                                    "sliced": wa > 0}
        out[f"topk{k}_candidates_b{B}_v{V}"] = {"ms": round(ms_k, 5), "bytes_read_2_passes": 2 * nb,
                                                "logits_GB/s": round(nb / (ms_k * 1e-3) / 1e9, 1), "sliced": wk > 0}
        for buf in (x, ids, cnt, bad, ci, cv, ws_a, ws_k):
            if buf is not None:
                buf.free()
    return out


TRAFFIC_PROFILE = os.path.join("profiles", "pmc_traffic_c4.md")


# C++ tokens for the source hash: string and character literals, comments, runs of other non-space
# characters (a slash alone, so that "a;//c" splits before the comment)
_CXX_TOKENS = re.compile(r'"(?:\\.|[^"\\\n])*"|\'(?:\\.|[^\'\\\n])*\'|//[^\n]*|/\*.*?\*/|[^\s"\'/]+|/', re.S)


def code_tokens(text):
    """The code of a C++ source without its comments, one space between tokens: edits to comments and layout
    leave it unchanged."""
    return " ".join(t for t in _CXX_TOKENS.findall(text) if not t.startswith(("//", "/*")))


def kernel_source_hash(kdir=None):
    """sha256 (first 16 hex digits) over the code of the kernel sources (comments and layout dropped), in name
    order: a rocprof summary records the hash of the sources it measured, so a line can tell whether its
    traffic figure still describes these kernels."""
    import hashlib
    kdir = kdir or os.path.join(REPO, PKG, "csrc", "kernels")
    h = hashlib.sha256()
    for name in sorted(os.listdir(kdir)):
        if name.endswith((".hip", ".hpp")):
            h.update(name.encode() + b"\0")
            with open(os.path.join(kdir, name), encoding="utf-8") as f:
                h.update(code_tokens(f.read()).encode() + b"\0")
    return h.hexdigest()[:16]


def read_traffic(kernel_key):
    """HBM bytes per launch of `kernel_key` from the committed rocprofv3 --pmc summary, and where the figure
    comes from: the file, the commit and kernel-source hash it records, and whether that hash is the one of
    the kernels this run measured (if not, the figure is stale)."""
    path = os.path.join(REPO, TRAFFIC_PROFILE)
    source = {"file": TRAFFIC_PROFILE, "commit": None, "kernel_sources": None, "current_kernel_sources":
              kernel_source_hash(), "stale": True}
    if not os.path.exists(path):
        return None, source
    value = None
    with open(path) as f:
        for line in f:
            text = line.strip()
            m = re.match(r"Generated at commit `([0-9a-f]+)`", text)
            if m:
                source["commit"] = m.group(1)
            m = re.match(r"Kernel sources sha256/16 `([0-9a-f]+)`", text)
            if m:
                source["kernel_sources"] = m.group(1)
            parts = text.strip("|").split("|")
            if len(parts) >= 2 and parts[0].strip() == kernel_key:
                try:
                    value = int(float(parts[-1].strip()))
                except ValueError:
                    pass
    source["stale"] = source["kernel_sources"] != source["current_kernel_sources"]
    return value, source


def cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return platform.processor() or platform.machine()


def cpu_threads():
    """Threads for the CPU baseline: every core this process may run on (its CPU affinity), within the job's
    CPU share when the environment states one (OMP_NUM_THREADS, set on the GPU boxes)."""
    try:
        visible = len(os.sched_getaffinity(0))
    except AttributeError:
        visible = os.cpu_count() or 1
    share = os.environ.get("OMP_NUM_THREADS", "")
    used = min(visible, int(share)) if share.isdigit() and int(share) > 0 else visible
    return max(1, used), visible


def cpu_baseline(configs, synth, seconds):
    """The oracle (a C restatement of the reference's CPU arithmetic, worker threads kept for the whole run) on
    bounded samples of the benchmark configs, on all the job's cores and on one:
      - the config-4 chain (add_rms_norm x2, qk_norm_rope on Q with q_norm and K with k_norm, silu_mul) over
        its first Ts tokens, repeated until its share of `seconds` has elapsed;
      - config 1 itself (RMSNorm [16, 1024]), with the reference test's own CPU loop
        (tests/unit/rms_norm_cuda_test.cpp:174-244)."""
    spec = importlib.util.spec_from_file_location("q3k_oracle", os.path.join(REPO, "oracle", "q3k_oracle.py"))
    oracle = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(oracle)
    c = configs.CONFIGS["c4"]
    Ts, H, I = 256, c.hidden, c.inter
    h1 = synth.normal_bf16(c.seed, configs.TID_H, (Ts, H))
    d1 = synth.normal_bf16(c.seed, configs.TID_D1, (Ts, H))
    w1 = synth.normal_bf16(c.seed, configs.TID_W1, (H,), mean=1.0, std=0.1)
    q = synth.normal_bf16(c.seed, configs.TID_Q, (1, Ts, c.heads_q * D))
    k = synth.normal_bf16(c.seed, configs.TID_K, (1, Ts, c.heads_kv * D))
    qw = synth.normal_bf16(c.seed, configs.TID_QW, (D,), mean=1.0, std=0.1)
    kw = synth.normal_bf16(c.seed, configs.TID_KW, (D,), mean=1.0, std=0.1)
    g = synth.normal_bf16(c.seed, configs.TID_GATE, (Ts, I))
    u = synth.normal_bf16(c.seed, configs.TID_UP, (Ts, I))
    cache = oracle.build_rope_cache(Ts, D, configs.THETA)
    nbytes = configs.chain_bytes(configs.Config("sample", 0, 1, Ts, H, I, c.heads_q, c.heads_kv, "range", Ts))
    c1 = configs.CONFIGS["c1"]
    x1 = synth.normal_bf16(c1.seed, configs.TID_X, (c1.seq, c1.hidden))
    wf1 = synth.normal_bf16(c1.seed, configs.TID_WF, (c1.hidden,), mean=1.0, std=0.1)
    c1_bytes = configs.bytes_rms_norm(c1.tokens, c1.hidden)

    def chain_pass(nt):
        oracle.add_rms_norm(h1, d1, w1, EPS, band=False, nthreads=nt)
        oracle.qk_norm_rope(q, qw, 1, Ts, c.heads_q, D, EPS, cache, band=False, nthreads=nt)
        oracle.qk_norm_rope(k, kw, 1, Ts, c.heads_kv, D, EPS, cache, band=False, nthreads=nt)
        oracle.add_rms_norm(h1, d1, w1, EPS, band=False, nthreads=nt)
        oracle.silu_mul(g, u, band=False, nthreads=nt)

    def c1_pass(nt):
        oracle.rms_norm_test_order(x1, wf1, EPS, nthreads=nt)

    def rate(fn, nt, budget):
        fn(nt)
        n, t0 = 0, time.perf_counter()
        while True:
            fn(nt)
            n += 1
            el = time.perf_counter() - t0
            if el >= budget:
                return el / n, n

    cores, visible = cpu_threads()
    s_multi, passes = rate(chain_pass, cores, seconds * 0.6)
    s_single, _ = rate(chain_pass, 1, seconds * 0.3)
    c1_multi, c1_n = rate(c1_pass, cores, seconds * 0.05)
    c1_single, _ = rate(c1_pass, 1, seconds * 0.05)
    return {
        "value": round(nbytes / s_multi / 1e9, 3), "unit": "GB/s", "cores": cores, "kind": "port",
        "sample": f"config-4 chain ops (add_rms_norm x2, qk_norm_rope on Q and K with their own weights, silu_mul) "
                  f"on the first {Ts} tokens ({nbytes} algorithmic bytes per pass), {passes} passes on {cores} "
                  f"threads; oracle/q3k_oracle.c (C restatement of the reference's CPU arithmetic)",
        "value_1thread": round(nbytes / s_single / 1e9, 3),
        "cpu_model": cpu_model(), "cores_visible": visible, "os_cpu_count": os.cpu_count(),
        "c1": {"what": "config 1: RMSNorm [16, 1024] with the reference test's CPU loop "
                       "(rms_norm_cuda_test.cpp:174-244)", "bytes": c1_bytes,
               "us_per_call": round(c1_multi * 1e6, 2), "GB/s": round(c1_bytes / c1_multi / 1e9, 3),
               "threads": cores, "us_per_call_1thread": round(c1_single * 1e6, 2),
               "GB/s_1thread": round(c1_bytes / c1_single / 1e9, 3), "calls": c1_n},
    }


def weight_io_extra(seconds_limit=180):
    """The safetensors weight IO measurement (bin/q3k_weight_io_bench, a child process): a synthetic file of 4
    Qwen3-8B layers (1.5 GB) in the page cache, loaded to the GPU by the loader and by the reference's staging
    scheme, beside the host-to-device DMA ceiling."""
    import subprocess
    import tempfile

    exe = os.path.join(REPO, "qwen3-runtime-byyourself_amd", "bin", "q3k_weight_io_bench")
    if not os.path.exists(exe):
        return {"error": f"{exe} is not built"}
    with tempfile.TemporaryDirectory() as d:
        try:
            proc = subprocess.run([exe, "--layers", "4", "--repeats", "3", "--dir", d], capture_output=True,
                                  text=True, timeout=seconds_limit)
        except subprocess.TimeoutExpired:
            return {"error": f"timed out after {seconds_limit} s"}
    if proc.returncode != 0 or not proc.stdout.strip():
        return {"error": f"exit {proc.returncode}: {proc.stderr.strip()[-300:]}"}
    r = json.loads(proc.stdout.strip().splitlines()[-1])
    return {"GB/s": r["loader"], "reference_scheme_GB/s": r["reference"], "dma_ceiling_GB/s": r["dma_ceiling"],
            "bytes": r["bytes"], "vs_reference_scheme": round(r["loader"] / r["reference"], 2),
            "frac_of_dma_ceiling": round(r["loader"] / r["dma_ceiling"], 3)}


def decode_select_extra(seconds_limit=120):
    """Per-token selection latency through the C++ runtime (bin/q3k_decode_select_bench, a child process):
    argmax_last_dimension, Sampler greedy and Sampler with the reference's default sampling over [B, 151936]
    logits at B = 1 and 64, microseconds per call, and the device allocations made per call once warm."""
    import subprocess

    exe = os.path.join(REPO, PKG, "bin", "q3k_decode_select_bench")
    if not os.path.exists(exe):
        return {"error": f"{exe} is not built"}
    try:
        proc = subprocess.run([exe, "--calls", "200"], capture_output=True, text=True, timeout=seconds_limit)
    except subprocess.TimeoutExpired:
        return {"error": f"timed out after {seconds_limit} s"}
    if proc.returncode != 0 or not proc.stdout.strip():
        return {"error": f"exit {proc.returncode}: {proc.stderr.strip()[-300:]}"}
    return json.loads(proc.stdout.strip().splitlines()[-1])


def c3_decode_extra(q3k, hip, synth, configs, stream):
    """Config 3 (Qwen3-8B decode step: 64 sequences x 1 token, one position per sequence): the per-layer chain
    op by op and replayed from a HIP graph (the chain of every input set captured once, one host launch per
    cycle, as a serving loop replays a decode step).  Each op is a 1-5 MB launch, so this is latency."""
    c = configs.CONFIGS["c3"]
    print("[bench] config 3 decode chain", file=sys.stderr, flush=True)
    base = make_chain_set(hip, synth, configs, c, q3k)
    sets = [base] + [clone_set(hip, base) for _ in range(5)]
    make = lambda b: chain_ops(q3k, c, b, stream)  # noqa: E731
    ms = time_chain(hip, stream, sets, make, 120, 12)
    out = {"tokens": c.tokens, "chain_bytes": configs.chain_bytes(c), "us_per_layer_op_by_op": round(ms * 1e3, 2)}
    try:
        ms_g = time_chain_graph(hip, stream, sets, make, 120, 12)
        out.update({"us_per_layer_graph_replay": round(ms_g * 1e3, 2),
                    "tokens_per_s_graph_replay": round(c.tokens / (ms_g * 1e-3), 1),
                    "GB/s_graph_replay": round(configs.chain_bytes(c) / (ms_g * 1e-3) / 1e9, 1)})
    except hip.HipRuntimeError as e:
        out["graph_error"] = str(e)
    for st in sets:
        for b in st.values():
            b.free()
    return out


def c1_extra(q3k, hip, synth, configs, stream):
    """Config 1 (RMSNorm [16, 1024], the reference test's shape, tests/unit/rms_norm_cuda_test.cpp:174-244) on the
    GPU: microseconds per call launched back to back and replayed from a HIP graph, over 8 copies of the inputs
    (a 67 KB launch: latency, not bandwidth).  The CPU baseline times the same config with the reference test's
    own loop (cpu_baseline.c1)."""
    c = configs.CONFIGS["c1"]
    T, H = c.tokens, c.hidden
    print("[bench] config 1 rms_norm", file=sys.stderr, flush=True)
    x = synth.normal_bf16(c.seed, configs.TID_X, (T, H))
    w = synth.normal_bf16(c.seed, configs.TID_WF, (H,), mean=1.0, std=0.1)
    DB = hip.DeviceBuffer.from_array
    sets = [{"x": DB(x), "w": DB(w), "y": hip.DeviceBuffer(T * H * 2)} for _ in range(8)]
    make = lambda b: [("rms_norm", lambda: q3k.rms_norm(b["x"], b["w"], b["y"], T, H, EPS, stream))]  # noqa: E731
    ms = time_chain(hip, stream, sets, make, 400, 40)
    nb = configs.bytes_rms_norm(T, H)
    out = {"shape": [T, H], "bytes": nb, "us_per_call": round(ms * 1e3, 3), "GB/s": round(nb / (ms * 1e-3) / 1e9, 2)}
    try:
        ms_g = time_chain_graph(hip, stream, sets, make, 400, 40)
        out.update({"us_per_call_graph_replay": round(ms_g * 1e3, 3),
                    "GB/s_graph_replay": round(nb / (ms_g * 1e-3) / 1e9, 2)})
    except hip.HipRuntimeError as e:
        out["graph_error"] = str(e)
    for st in sets:
        for b in st.values():
            b.free()
    return out


def c2_extra(q3k, hip, synth, configs, stream, steps):
    """Config 2 (Qwen3-0.6B, T = 512 at positions 0..511): the embedding gather (model.cpp:118) from the
    [151936, 1024] table, residual add + RMSNorm (decoder_layer.cpp:78->88), Q/K norm + RoPE
    (self_attention.cpp:147-152) and SwiGLU (mlp.cpp:111), as a chain launched op by op and replayed from a HIP
    graph, and each op alone; GB/s of algorithmic bytes and tokens/s.  Input sets are device copies of one
    generated set, each with its own token ids, enough of them that one cycle exceeds the Infinity Cache."""
    c = configs.CONFIGS["c2"]
    T, H, I = c.tokens, c.hidden, c.inter
    print("[bench] config 2 chain", file=sys.stderr, flush=True)
    DB = hip.DeviceBuffer.from_array
    table = DB(synth.normal_bf16(c.seed, configs.TID_TABLE, (configs.VOCAB, H), std=0.02))
    base = make_chain_set(hip, synth, configs, c, q3k)
    for k in ("h2", "d2", "w2", "y2", "qn", "kn"):   # the second residual add + norm is not part of config 2
        base.pop(k).free()
    shared = ("w1", "qw", "kw", "cache")
    per_set = sum(b.nbytes for k, b in base.items() if k not in shared) + T * 4
    n_sets = max(6, -(-MIN_CYCLE_BYTES // per_set))
    sets = []
    for i in range(n_sets):
        st = base if i == 0 else clone_set(hip, {k: v for k, v in base.items() if k not in shared})
        st.update({k: base[k] for k in shared})
        st["ids"] = DB(synth.token_ids(c.seed + i, configs.TID_IDS, (T,), configs.VOCAB))
        sets.append(st)

    def ops(b):
        return [
            ("embedding", lambda: q3k.embedding(b["ids"], T, table, configs.VOCAB, H, b["h1"], stream)),
            ("add_rms_norm", lambda: q3k.add_rms_norm(b["h1"], b["d1"], b["w1"], b["y1"], T, H, EPS, stream)),
            ("qk_norm_rope", lambda: q3k.qk_norm_rope(b["q"], b["k"], b["qw"], b["kw"], c.batch, c.seq, c.heads_q,
                                                      c.heads_kv, D, EPS, b["cache"], c.max_pos, 0, None, stream)),
            ("silu_mul", lambda: q3k.silu_mul(b["g"], b["u"], b["o"], T * I, stream)),
        ]

    reps = max(len(sets), steps)
    ms = time_chain(hip, stream, sets, ops, reps, 4)
    per_op = time_each_op(hip, stream, sets, ops, reps)
    op_bytes = {"embedding": configs.bytes_embedding(T, H), "add_rms_norm": configs.bytes_add_rms_norm(T, H),
                "qk_norm_rope": configs.bytes_qk_norm_rope(T, c.heads_q, c.heads_kv, D, c.distinct_positions()),
                "silu_mul": configs.bytes_silu_mul(T, I)}
    chain = configs.c2_chain_bytes(c)
    assert chain == sum(op_bytes.values())
    out = {"tokens": T, "chain": "embedding -> add_rms_norm -> qk_norm_rope -> silu_mul", "chain_bytes": chain,
           "us_per_step": round(ms * 1e3, 2), "GB/s": round(chain / (ms * 1e-3) / 1e9, 1),
           "pct_of_peak": round(100 * chain / (ms * 1e-3) / 1e9 / PEAK_GBS, 2),
           "tokens_per_s": round(T / (ms * 1e-3), 1), "input_sets": len(sets),
           "per_op": {n: {"us": round(t * 1e3, 2), "bytes": op_bytes[n],
                          "GB/s": round(op_bytes[n] / (t * 1e-3) / 1e9, 1),
                          "pct_of_peak": round(100 * op_bytes[n] / (t * 1e-3) / 1e9 / PEAK_GBS, 2)}
                      for n, t in per_op.items()}}
    try:
        ms_g = time_chain_graph(hip, stream, sets, ops, reps, 4)
        out.update({"us_per_step_graph_replay": round(ms_g * 1e3, 2),
                    "GB/s_graph_replay": round(chain / (ms_g * 1e-3) / 1e9, 1),
                    "tokens_per_s_graph_replay": round(T / (ms_g * 1e-3), 1)})
    except hip.HipRuntimeError as e:
        out["graph_error"] = str(e)
    seen = set()
    for st in sets:
        for b in st.values():
            if id(b) not in seen:
                seen.add(id(b))
                b.free()
    table.free()
    return out


def ceiling_record(hip, q3k, stream, op_gbs, nbytes, n_in, n_out, in_place, reps, note=None):
    """An op's measured GB/s beside the ceiling of its own access pattern at its size (pattern_ceiling)."""
    gbs, threads = pattern_ceiling(hip, q3k, stream, nbytes, n_in, n_out, in_place, reps)
    rec = {"streams": f"{n_in} in, {n_out} out" + (" (first in place)" if in_place else ""), "bytes_each": nbytes,
           "GB/s": round(gbs, 1), "pct_of_peak": round(100 * gbs / PEAK_GBS, 2), "threads_per_block": threads,
           "op_GB/s": round(op_gbs, 1), "op_frac": round(op_gbs / gbs, 4)}
    if note:
        rec["note"] = note
    return rec


def c5_extra(q3k, hip, synth, configs, stream, steps):
    """Config 5 (Qwen3-32B shapes, T = 16384 as 2 x 8192): the fused per-layer chain and each of its ops, plus
    the final RMSNorm [16384, 5120], in GB/s of algorithmic bytes.  Activations are a 64 MiB block of N(0, 1)
    bf16 tiled over each buffer by device copies (generating 3.8 GB per input set on the host would take
    minutes); norm weights N(1, 0.1); the RoPE table of the 8192 positions."""
    c = configs.CONFIGS["c5"]
    T, H, I = c.tokens, c.hidden, c.inter
    print("[bench] config 5 chain", file=sys.stderr, flush=True)
    block = hip.DeviceBuffer.from_array(synth.normal_bf16(c.seed, configs.TID_H, (32 << 20,)))

    def act(nbytes):
        b = hip.DeviceBuffer(nbytes)
        b.tile_from(block)
        return b

    DB = hip.DeviceBuffer.from_array
    weights = {"w1": DB(synth.normal_bf16(c.seed, configs.TID_W1, (H,), mean=1.0, std=0.1)),
               "w2": DB(synth.normal_bf16(c.seed, configs.TID_W2, (H,), mean=1.0, std=0.1)),
               "qw": DB(synth.normal_bf16(c.seed, configs.TID_QW, (D,), mean=1.0, std=0.1)),
               "kw": DB(synth.normal_bf16(c.seed, configs.TID_KW, (D,), mean=1.0, std=0.1)),
               "cache": DB(q3k.build_rope_cache(c.max_pos, D, configs.THETA))}
    sets = []
    for _ in range(2):
        st = {k: act(T * H * 2) for k in ("h1", "d1", "y1", "h2", "d2", "y2")}
        st.update({"q": act(T * c.heads_q * D * 2), "k": act(T * c.heads_kv * D * 2),
                   "g": act(T * I * 2), "u": act(T * I * 2), "o": act(T * I * 2)})
        st.update(weights)
        sets.append(st)
    block.free()
    make = lambda b: chain_ops(q3k, c, b, stream)  # noqa: E731
    ms = time_chain(hip, stream, sets, make, max(8, steps // 4), 2)
    per_op = time_each_op(hip, stream, sets, make, max(8, steps // 4), buffers=OP_BUFFERS)
    U = c.distinct_positions()
    op_bytes = {"add_rms_norm_attn": configs.bytes_add_rms_norm(T, H),
                "qk_norm_rope": configs.bytes_qk_norm_rope(T, c.heads_q, c.heads_kv, D, U),
                "add_rms_norm_mlp": configs.bytes_add_rms_norm(T, H), "silu_mul": configs.bytes_silu_mul(T, I)}
    final = time_each_op(hip, stream, sets, lambda b: [
        ("rms_norm_final", lambda: q3k.rms_norm(b["h1"], b["w1"], b["y1"], T, H, EPS, stream))],
        max(8, steps // 4), buffers={"rms_norm_final": ("h1", "y1")})
    op_bytes["rms_norm_final"] = configs.bytes_rms_norm(T, H)
    per_op.update(final)
    chain = configs.chain_bytes(c)
    out = {"tokens": T, "chain_bytes": chain, "ms_per_step": round(ms, 5),
           "GB/s": round(chain / (ms * 1e-3) / 1e9, 1), "pct_of_peak": round(100 * chain / (ms * 1e-3) / 1e9 / PEAK_GBS, 2),
           "tokens_per_s": round(T / (ms * 1e-3), 1),
           "per_op": {n: {"ms": round(t, 5), "bytes": op_bytes[n], "GB/s": round(op_bytes[n] / (t * 1e-3) / 1e9, 1),
                          "pct_of_peak": round(100 * op_bytes[n] / (t * 1e-3) / 1e9 / PEAK_GBS, 2)}
                      for n, t in per_op.items()}}
    seen = set()
    for st in sets:
        for b in st.values():
            if id(b) not in seen:
                seen.add(id(b))
                b.free()
    return out


def tp8_shard_extra(q3k, hip, synth, configs, stream, steps):
    """Config 4 at one GPU's share under 8-way tensor parallelism, the shapes the sharding plan gives each rank
    (the collectives themselves are not built): Q/K norm + RoPE on the rank's 4 query heads and 1 KV head of
    every token, SwiGLU on its 1536 of the 12288 intermediate columns, and add + RMSNorm on its 1024-token slice
    after the reduce-scatter (whole 4096-wide rows).  Per-op GB/s of algorithmic bytes, each op timed alone over
    rotating inputs, and the three ops back to back."""
    c = dataclasses.replace(configs.CONFIGS["c4"], name="c4-tp8-shard", heads_q=32 // 8, heads_kv=8 // 8,
                            inter=12288 // 8)
    T, H, I = c.tokens, c.hidden, c.inter
    Ts = T // 8
    s = c.seed
    print("[bench] config 4 at a tensor-parallel-8 shard", file=sys.stderr, flush=True)
    DB = hip.DeviceBuffer.from_array
    base = {
        "h1": DB(synth.normal_bf16(s, configs.TID_H, (Ts, H))),
        "d1": DB(synth.normal_bf16(s, configs.TID_D1, (Ts, H))),
        "w1": DB(synth.normal_bf16(s, configs.TID_W1, (H,), mean=1.0, std=0.1)),
        "y1": hip.DeviceBuffer(Ts * H * 2),
        "q": DB(synth.normal_bf16(s, configs.TID_Q, (T, c.heads_q * D))),
        "k": DB(synth.normal_bf16(s, configs.TID_K, (T, c.heads_kv * D))),
        "qw": DB(synth.normal_bf16(s, configs.TID_QW, (D,), mean=1.0, std=0.1)),
        "kw": DB(synth.normal_bf16(s, configs.TID_KW, (D,), mean=1.0, std=0.1)),
        "g": DB(synth.normal_bf16(s, configs.TID_GATE, (T, I))),
        "u": DB(synth.normal_bf16(s, configs.TID_UP, (T, I))),
        "o": hip.DeviceBuffer(T * I * 2),
        "cache": DB(q3k.build_rope_cache(c.max_pos, D, configs.THETA)),
    }
    shared = ("w1", "qw", "kw", "cache")
    sets = [base]
    for _ in range(5):
        st = clone_set(hip, {k: v for k, v in base.items() if k not in shared})
        st.update({k: base[k] for k in shared})
        sets.append(st)

    def ops(b):
        return [
            ("add_rms_norm", lambda: q3k.add_rms_norm(b["h1"], b["d1"], b["w1"], b["y1"], Ts, H, EPS, stream)),
            ("qk_norm_rope", lambda: q3k.qk_norm_rope(b["q"], b["k"], b["qw"], b["kw"], c.batch, c.seq, c.heads_q,
                                                      c.heads_kv, D, EPS, b["cache"], c.max_pos, 0, None, stream)),
            ("silu_mul", lambda: q3k.silu_mul(b["g"], b["u"], b["o"], T * I, stream)),
        ]

    reps = max(20, steps)
    ms = time_chain(hip, stream, sets, ops, reps, 2)
    per_op = time_each_op(hip, stream, sets, ops, reps,
                          buffers={"add_rms_norm": ("h1", "d1", "y1"), "qk_norm_rope": ("q", "k"),
                                   "silu_mul": ("g", "u", "o")})
    op_bytes = {"add_rms_norm": configs.bytes_add_rms_norm(Ts, H),
                "qk_norm_rope": configs.bytes_qk_norm_rope(T, c.heads_q, c.heads_kv, D, c.distinct_positions()),
                "silu_mul": configs.bytes_silu_mul(T, I)}
    chain = sum(op_bytes.values())
    for b in sets[1:]:   # the ceilings below allocate their own buffers
        for k, v in b.items():
            if k not in shared:
                v.free()
    q_bytes = T * (c.heads_q + c.heads_kv) * D * 2
    gbs = {n: op_bytes[n] / (t * 1e-3) / 1e9 for n, t in per_op.items()}
    ceilings = {"add_rms_norm": ceiling_record(hip, q3k, stream, gbs["add_rms_norm"], Ts * H * 2, 2, 2, True, reps),
                "qk_norm_rope": ceiling_record(hip, q3k, stream, gbs["qk_norm_rope"], q_bytes, 1, 1, True, reps),
                "silu_mul": ceiling_record(hip, q3k, stream, gbs["silu_mul"], T * I * 2, 2, 1, False, reps)}
    sets = sets[:1]
    out = {"shapes": {"add_rms_norm": [Ts, H], "q": [T, c.heads_q, D], "k": [T, c.heads_kv, D], "silu_mul": [T, I]},
           "pattern_ceilings": ceilings,
           "chain_bytes": chain, "chain_ms": round(ms, 5),
           "chain_GB/s": round(chain / (ms * 1e-3) / 1e9, 1),
           "chain_pct_of_peak": round(100 * chain / (ms * 1e-3) / 1e9 / PEAK_GBS, 2),
           "per_op": {n: {"ms": round(t, 5), "bytes": op_bytes[n], "GB/s": round(op_bytes[n] / (t * 1e-3) / 1e9, 1),
                          "pct_of_peak": round(100 * op_bytes[n] / (t * 1e-3) / 1e9 / PEAK_GBS, 2)}
                      for n, t in per_op.items()}}
    seen = set()
    for st in sets:
        for b in st.values():
            if id(b) not in seen:
                seen.add(id(b))
                b.free()
    return out


def main():
    args = parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(f"bench.py measures one GPU only: this build has no multi-GPU path (--gpus {args.gpus}, "
              f"WORLD_SIZE {world}); each op is token-local and would shard by tokens with no exchange.",
              file=sys.stderr)
        sys.exit(2)

    # The measurements made by child processes run first, while this process
    # has not opened the GPU: the child is then the only process on the
    # device, as a serving process would be (with a second HIP context open,
    # each synchronising call of the selection path measured ~2x slower).
    child = {}
    if not args.no_extras:
        if args.config == "c4":
            print("[bench] decode token selection", file=sys.stderr, flush=True)
            child["decode_select"] = decode_select_extra()
        print("[bench] weight IO", file=sys.stderr, flush=True)
        child["weight_io"] = weight_io_extra()

    q3k = importlib.import_module(PKG)
    hip = importlib.import_module(PKG + ".hip")
    synth = importlib.import_module(PKG + ".synth")
    configs = importlib.import_module(PKG + ".configs")
    q3k.load()
    if not hip.available():
        print("no GPU visible", file=sys.stderr)
        sys.exit(1)
    c = configs.CONFIGS[args.config]
    print(f"[bench] config {c.name}: generating inputs", file=sys.stderr, flush=True)

    stream = hip.Stream()
    base = make_chain_set(hip, synth, configs, c, q3k)
    sets = [base] + [clone_set(hip, base) for _ in range(max(1, args.sets) - 1)]
    print(f"[bench] timing chain: {args.warmup} warmup + {args.steps} steps over {len(sets)} sets",
          file=sys.stderr, flush=True)
    make_chain = lambda b: chain_ops(q3k, c, b, stream)  # noqa: E731
    ms_step = time_chain(hip, stream, sets, make_chain, args.steps, args.warmup)
    per_op = time_each_op(hip, stream, sets, make_chain, args.steps, buffers=OP_BUFFERS)

    T, H, I = c.tokens, c.hidden, c.inter
    U = c.distinct_positions()
    op_bytes = {
        "add_rms_norm_attn": configs.bytes_add_rms_norm(T, H),
        "qk_norm_rope": configs.bytes_qk_norm_rope(T, c.heads_q, c.heads_kv, D, U),
        "add_rms_norm_mlp": configs.bytes_add_rms_norm(T, H),
        "silu_mul": configs.bytes_silu_mul(T, I),
    }
    chain_bytes = sum(op_bytes.values())
    assert chain_bytes == configs.chain_bytes(c)
    value = chain_bytes / (ms_step * 1e-3) / 1e9
    ops_report = {}
    for n, ms in per_op.items():
        gbs = op_bytes[n] / (ms * 1e-3) / 1e9
        ops_report[n] = {"ms": round(ms, 5), "bytes": op_bytes[n], "GB/s": round(gbs, 1),
                         "pct_of_peak": round(100 * gbs / PEAK_GBS, 2)}
    dominant = max(per_op, key=per_op.get)
    dom_gbs = op_bytes[dominant] / (per_op[dominant] * 1e-3) / 1e9
    kernel_key = {"silu_mul": "silu_mul", "qk_norm_rope": "qk_norm_rope"}.get(dominant, "add_rms_norm")
    traffic, traffic_source = read_traffic(kernel_key)
    roofline = {"bound": "hbm", "kernel": dominant, "achieved": round(dom_gbs, 1), "peak": PEAK_GBS, "unit": "GB/s",
                "frac": round(dom_gbs / PEAK_GBS, 4), "traffic": traffic, "traffic_source": traffic_source,
                "algorithmic_bytes": op_bytes[dominant]}

    extras = {}
    # final RMSNorm (model.cpp:146) at config 4, timed like the per-op figures: back-to-back launches over
    # copies of its input and output whose cycle exceeds the Infinity Cache
    rb = configs.bytes_rms_norm(T, H)
    ms_rn = time_each_op(hip, stream, sets, lambda b: [
        ("rms_norm_final", lambda: q3k.rms_norm(b["h1"], b["w1"], b["y1"], T, H, EPS, stream))],
        args.steps, buffers={"rms_norm_final": ("h1", "y1")})["rms_norm_final"]
    extras["rms_norm_final"] = {"ms": round(ms_rn, 5), "bytes": rb, "GB/s": round(rb / (ms_rn * 1e-3) / 1e9, 1),
                                "pct_of_peak": round(100 * rb / (ms_rn * 1e-3) / 1e9 / PEAK_GBS, 2)}
    # the same chain replayed from a HIP graph: no host launch cost between ops
    # (what bounds the op-by-op loop at decode sizes)
    try:
        ms_graph = time_chain_graph(hip, stream, sets, make_chain, args.steps, args.warmup)
        extras["chain_graph_replay"] = {
            "ms_per_step": round(ms_graph, 5), "GB/s": round(chain_bytes / (ms_graph * 1e-3) / 1e9, 1),
            "pct_of_peak": round(100 * chain_bytes / (ms_graph * 1e-3) / 1e9 / PEAK_GBS, 2)}
    except hip.HipRuntimeError as e:   # a runtime without stream capture: report it, keep the bench line
        extras["chain_graph_replay"] = {"error": str(e)}
    if not args.no_extras:
        print("[bench] timing unfused chain", file=sys.stderr, flush=True)
        make_unfused = lambda b: unfused_ops(q3k, c, b, stream)  # noqa: E731
        ms_unfused = time_chain(hip, stream, sets, make_unfused, max(5, args.steps // 2), 3)
        per_unfused = time_each_op(hip, stream, sets, make_unfused, max(5, args.steps // 2), buffers=UNFUSED_BUFFERS)
        unf_bytes = configs.unfused_op_bytes(c)
        unf_chain = sum(unf_bytes.values())
        extras["unfused_chain"] = {"ms_per_step": round(ms_unfused, 5), "chain_bytes": unf_chain,
                                   "GB/s": round(unf_chain / (ms_unfused * 1e-3) / 1e9, 1),
                                   "per_op": {k: {"ms": round(v, 5), "bytes": unf_bytes[k],
                                                  "GB/s": round(unf_bytes[k] / (v * 1e-3) / 1e9, 1),
                                                  "pct_of_peak": round(100 * unf_bytes[k] / (v * 1e-3) / 1e9 / PEAK_GBS, 2)}
                                              for k, v in per_unfused.items()},
                                   "fused_speedup": round(ms_unfused / ms_step, 3)}
        # copy ceiling: 1 GiB, 128-bit loads and stores
        nb = 1 << 30
        src, dst = hip.DeviceBuffer(nb), hip.DeviceBuffer(nb)
        ms_cp = time_chain(hip, stream, [0], lambda _: [("copy", lambda: q3k.bench_copy(src, dst, nb, stream))], 10, 2)
        extras["copy_ceiling_GB/s"] = round(2 * nb / (ms_cp * 1e-3) / 1e9, 1)
        src.free()
        dst.free()
        # each fused op's own access-pattern ceiling at its size: the same 128-bit input and output streams with
        # no arithmetic (q3k_bench_stream_u128), back to back over rotating buffers like the per-op figures
        print("[bench] timing access-pattern ceilings", file=sys.stderr, flush=True)
        q_bytes = T * (c.heads_q + c.heads_kv) * D * 2
        unf = extras["unfused_chain"]["per_op"]
        patterns = {"silu_mul": (ops_report["silu_mul"]["GB/s"], T * I * 2, 2, 1, False),
                    "add_rms_norm_attn": (ops_report["add_rms_norm_attn"]["GB/s"], T * H * 2, 2, 2, True),
                    "qk_norm_rope": (ops_report["qk_norm_rope"]["GB/s"], q_bytes, 1, 1, True),
                    # the final RMSNorm (model.cpp:146) alone: 64 MB in, 64 MB out
                    "rms_norm_final": (extras["rms_norm_final"]["GB/s"], T * H * 2, 1, 1, False),
                    # the drop-in ops of the reference's order (self_attention.cpp:147-152, decoder_layer.cpp:78)
                    "unfused_rms_norm_q": (unf["rms_norm_q"]["GB/s"], T * c.heads_q * D * 2, 1, 1, False),
                    "unfused_rms_norm_k": (unf["rms_norm_k"]["GB/s"], T * c.heads_kv * D * 2, 1, 1, False),
                    "unfused_rope": (unf["rope"]["GB/s"], q_bytes, 1, 1, True),
                    "unfused_add_inplace": (unf["add_inplace"]["GB/s"], T * H * 2, 2, 1, True)}
        extras["pattern_ceilings"] = {
            name: ceiling_record(hip, q3k, stream, gbs, nb_op, n_in, n_out, in_place, args.steps)
            for name, (gbs, nb_op, n_in, n_out, in_place) in patterns.items()}
        # Q/K norm + RoPE + KV-cache append (self_attention.cpp:147-156) fused, against qk_norm_rope followed by
        # the append; the cache holds the whole sequence (capacity S), written at cached length 0
        print("[bench] timing KV append", file=sys.stderr, flush=True)
        kv_row = c.heads_kv * D * 2
        kv_set_bytes = T * c.heads_q * D * 2 + 4 * T * kv_row
        kv_sets = []
        for i in range(-(-MIN_CYCLE_BYTES // kv_set_bytes)):
            src = sets[i % len(sets)]
            e = {"q": hip.DeviceBuffer(src["q"].nbytes), "k": hip.DeviceBuffer(src["k"].nbytes),
                 "v": hip.DeviceBuffer(T * kv_row), "kc": hip.DeviceBuffer(T * kv_row), "vc": hip.DeviceBuffer(T * kv_row)}
            e["q"].copy_from(src["q"])
            e["k"].copy_from(src["k"])
            e["v"].copy_from(src["k"])
            kv_sets.append(e)
        b0 = sets[0]
        ms_kv = time_chain(hip, stream, kv_sets, lambda e: [
            ("qk_norm_rope_kv_append", lambda: q3k.qk_norm_rope_kv_append(
                e["q"], e["k"], e["v"], b0["qw"], b0["kw"], c.batch, c.seq, c.heads_q, c.heads_kv, D, EPS, b0["cache"],
                c.max_pos, 0, e["kc"], e["vc"], c.seq, 0, None, stream))], max(20, len(kv_sets)), 3)
        ms_kv_pair = time_chain(hip, stream, kv_sets, lambda e: [
            ("qk_norm_rope", lambda: q3k.qk_norm_rope(e["q"], e["k"], b0["qw"], b0["kw"], c.batch, c.seq, c.heads_q,
                                                      c.heads_kv, D, EPS, b0["cache"], c.max_pos, 0, None, stream)),
            ("kv_append", lambda: q3k.kv_append(e["k"], e["v"], e["kc"], e["vc"], c.batch, c.seq, kv_row, c.seq, 0,
                                                stream))], max(20, len(kv_sets)), 3)
        ms_append = time_chain(hip, stream, kv_sets, lambda e: [
            ("kv_append", lambda: q3k.kv_append(e["k"], e["v"], e["kc"], e["vc"], c.batch, c.seq, kv_row, c.seq, 0,
                                                stream))], max(20, len(kv_sets)), 3)
        U = c.distinct_positions()
        kvb = configs.bytes_qk_norm_rope_kv_append(T, c.heads_q, c.heads_kv, D, U)
        ab = configs.bytes_kv_append(T, c.heads_kv, D)
        extras["qk_norm_rope_kv_append"] = {"ms": round(ms_kv, 5), "bytes": kvb,
                                            "GB/s": round(kvb / (ms_kv * 1e-3) / 1e9, 1),
                                            "unfused_ms": round(ms_kv_pair, 5),
                                            "fused_speedup": round(ms_kv_pair / ms_kv, 3)}
        extras["kv_append"] = {"ms": round(ms_append, 5), "bytes": ab, "GB/s": round(ab / (ms_append * 1e-3) / 1e9, 1)}
        # K and V in, the two cache layers out (kv_cache.cpp:147-185)
        extras["pattern_ceilings"]["kv_append"] = ceiling_record(
            hip, q3k, stream, ab / (ms_append * 1e-3) / 1e9, T * kv_row, 2, 2, False, args.steps)
        for e in kv_sets:
            for buf in e.values():
                buf.free()
        extras.update(time_attention(q3k, hip, synth, c, stream))
        extras.update(time_sampling(q3k, hip, synth, configs, c, stream))
        if "embedding" in c.ops:
            print("[bench] timing embedding", file=sys.stderr, flush=True)
            for s in sets[1:]:
                for b in s.values():
                    b.free()
            table = hip.DeviceBuffer.from_array(
                synth.normal_bf16(c.seed, configs.TID_TABLE, (configs.VOCAB, H)))
            w = sets[0]["w1"]
            # Each set gathers its own T random rows and writes its own outputs; one cycle over the sets
            # moves >= MIN_CYCLE_BYTES, so neither the gathered rows nor the outputs stay in the Infinity Cache.
            per_set = 3 * T * H * 2
            emb_sets = [{"ids": hip.DeviceBuffer.from_array(
                             synth.token_ids(c.seed + k, configs.TID_IDS, (T,), configs.VOCAB)),
                         "out": hip.DeviceBuffer(T * H * 2), "y": hip.DeviceBuffer(T * H * 2)}
                        for k in range(-(-MIN_CYCLE_BYTES // per_set))]
            ms_e = time_chain(hip, stream, emb_sets, lambda e: [
                ("embedding", lambda: q3k.embedding(e["ids"], T, table, configs.VOCAB, H, e["out"], stream))],
                max(20, len(emb_sets)), 3)
            eb = configs.bytes_embedding(T, H)
            extras["embedding"] = {"ms": round(ms_e, 5), "bytes": eb, "GB/s": round(eb / (ms_e * 1e-3) / 1e9, 1)}
            # the gathered rows against a contiguous stream of the same bytes in and out
            extras["pattern_ceilings"]["embedding"] = ceiling_record(
                hip, q3k, stream, eb / (ms_e * 1e-3) / 1e9, T * H * 2, 1, 1, False, args.steps,
                note="the op reads T random 8 KB table rows; the ceiling streams the same bytes contiguously")
            # embedding + first input norm fused (model.cpp:118 -> decoder_layer.cpp:72) against the pair
            ms_en = time_chain(hip, stream, emb_sets, lambda e: [
                ("embedding_rms_norm", lambda: q3k.embedding_rms_norm(e["ids"], T, table, configs.VOCAB, H, w, EPS,
                                                                      e["out"], e["y"], stream))],
                max(20, len(emb_sets)), 3)
            ms_pair = time_chain(hip, stream, emb_sets, lambda e: [
                ("embedding", lambda: q3k.embedding(e["ids"], T, table, configs.VOCAB, H, e["out"], stream)),
                ("rms_norm", lambda: q3k.rms_norm(e["out"], w, e["y"], T, H, EPS, stream))],
                max(20, len(emb_sets)), 3)
            enb = configs.bytes_embedding_rms_norm(T, H)
            extras["embedding_rms_norm"] = {"ms": round(ms_en, 5), "bytes": enb,
                                            "GB/s": round(enb / (ms_en * 1e-3) / 1e9, 1),
                                            "unfused_ms": round(ms_pair, 5),
                                            "fused_speedup": round(ms_pair / ms_en, 3)}
            # final norm of each sequence's last token only (model.cpp:146 + lm_head.cpp:123-181): B rows,
            # a latency-bound launch, reported against the full-sequence final norm it replaces
            Bq, Sq = c.batch, c.seq
            yl = hip.DeviceBuffer(Bq * H * 2)
            e0 = emb_sets[0]
            ms_last = time_chain(hip, stream, [0], lambda _: [
                ("add_rms_norm_last_token", lambda: q3k.add_rms_norm_rows(e0["out"], e0["y"], w, yl, Bq, Sq - 1, Sq, H,
                                                                          EPS, stream))], 50, 5)
            extras["add_rms_norm_last_token"] = {"ms": round(ms_last, 5), "rows": Bq,
                                                 "full_final_norm_ms": extras["rms_norm_final"]["ms"]}
            yl.free()
            for e in emb_sets:
                for buf in e.values():
                    buf.free()

    if not args.no_extras and args.config == "c4":
        # the other benchmark configs in the same record: their input sets replace config 4's
        for st in sets:
            for b in st.values():
                b.free()
        extras["c3_decode"] = c3_decode_extra(q3k, hip, synth, configs, stream)
        extras["c5_prefill"] = c5_extra(q3k, hip, synth, configs, stream, args.steps)
        extras["tp8_shard"] = tp8_shard_extra(q3k, hip, synth, configs, stream, args.steps)
        extras["c1_rms_norm"] = c1_extra(q3k, hip, synth, configs, stream)
        extras["c2_chain"] = c2_extra(q3k, hip, synth, configs, stream, args.steps)
    extras.update(child)

    cpu = None
    if not args.no_cpu_baseline:
        print("[bench] CPU baseline", file=sys.stderr, flush=True)
        cpu = cpu_baseline(configs, synth, args.cpu_seconds)
        if "c1_rms_norm" in extras:   # config 1 on both sides: the reference test's CPU loop against the GPU
            g = extras["c1_rms_norm"]
            cpu["c1"]["gpu_us_per_call"] = g["us_per_call"]
            cpu["c1"]["gpu_speedup_vs_threads"] = round(cpu["c1"]["us_per_call"] / g["us_per_call"], 1)
            cpu["c1"]["gpu_speedup_vs_1thread"] = round(cpu["c1"]["us_per_call_1thread"] / g["us_per_call"], 1)

    line = {
        "metric": METRIC, "value": round(value, 1), "unit": "GB/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms_step, 5), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "bf16", "data": "synthetic (seeded normals at the benchmark config shapes)",
        "config": {"workload": f"{c.name}: per-layer non-GEMM chain (add_rms_norm x2, qk_norm_rope, silu_mul)",
                   "tokens": T, "hidden": H, "intermediate": I, "heads_q": c.heads_q, "heads_kv": c.heads_kv,
                   "head_dim": D, "chain_bytes": chain_bytes, "input_sets": len(sets)},
        "pct_of_peak": round(100 * value / PEAK_GBS, 2),
        "tokens_per_s": round(T / (ms_step * 1e-3), 1),
        "per_op": ops_report,
        "roofline": roofline,
        "cpu_baseline": cpu,
        "extras": extras,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
