"""HIP graph capture of the decode-step ops.

A serving loop captures one decode step into a HIP graph and replays it, so
the host issues one launch per step instead of one per op.  Every entry point
here only launches kernels on the caller's stream (no allocation, no memset,
no synchronization), so it can be captured.  Each replay must give exactly
the eager results; replays are separated by eager work and synchronizations,
and the in-place inputs are re-uploaded before each one.
"""
import numpy as np
import pytest

from gpu_util import announce

pytestmark = pytest.mark.gpu

EPS = 1e-6
D = 128


def test_graph_replay_decode_step(q3k, hip, synth):
    """The c3 decode chain (add_rms_norm, qk_norm_rope with per-sequence positions, add_rms_norm, silu_mul), a
    key-split decode attention, a sliced argmax and a sliced top-k selection, captured into one graph: three
    replays, each bit-identical to the eager launches."""
    announce("graph replay: decode step")
    B, H, I, Hq, Hkv, P = 64, 4096, 12288, 32, 8, 4096
    Bd, L, V = 4, 700, 20000   # attention over Bd sequences of L cached keys; argmax over [Bd, V]
    rng = np.random.default_rng(5)
    arrays = {
        "h1": synth.normal_bf16(31, 1, (B, H)), "d1": synth.normal_bf16(31, 2, (B, H)),
        "w1": synth.normal_bf16(31, 3, (H,), mean=1.0, std=0.1),
        "q": synth.normal_bf16(31, 4, (B, Hq * D)), "k": synth.normal_bf16(31, 5, (B, Hkv * D)),
        "qw": synth.normal_bf16(31, 6, (D,), mean=1.0, std=0.1), "kw": synth.normal_bf16(31, 7, (D,), mean=1.0, std=0.1),
        "pos": rng.integers(0, P, size=(B,), dtype=np.int32),
        "h2": synth.normal_bf16(31, 8, (B, H)), "d2": synth.normal_bf16(31, 9, (B, H)),
        "w2": synth.normal_bf16(31, 10, (H,), mean=1.0, std=0.1),
        "g": synth.normal_bf16(31, 11, (B, I)), "u": synth.normal_bf16(31, 12, (B, I)),
        "aq": synth.normal_bf16(31, 13, (Bd, 1, Hq * D)),
        "kc": synth.normal_bf16(31, 14, (Bd, L, Hkv, D)), "vc": synth.normal_bf16(31, 15, (Bd, L, Hkv, D)),
        "logits": synth.normal_bf16(31, 16, (Bd, V), std=3.0),
        "cache": q3k.build_rope_cache(P, D, 1e6),
    }
    bufs = {k: hip.DeviceBuffer.from_array(v) for k, v in arrays.items()}
    K, cap = 20, 256
    outs = {"y1": B * H * 2, "y2": B * H * 2, "o": B * I * 2, "ao": Bd * Hq * D * 2, "ids": Bd * 4,
            "cnt": Bd * 4, "bad": Bd * 4, "ci": Bd * cap * 4, "cv": Bd * cap * 2}
    bufs.update({k: hip.DeviceBuffer(n) for k, n in outs.items()})
    wa = q3k.gqa_attention_workspace_bytes(Bd, 1, Hq, Hkv, D, L)
    wm = q3k.argmax_workspace_bytes(Bd, V)
    wk = q3k.topk_workspace_bytes(Bd, V, K)
    assert wa > 0 and wm > 0 and wk > 0, "the decode shapes should take the split and sliced paths"
    ws_a, ws_m, ws_k = hip.DeviceBuffer(wa), hip.DeviceBuffer(wm), hip.DeviceBuffer(wk)
    st = (L * Hkv * D, Hkv * D, D, 1)
    stream = hip.Stream()
    b = bufs

    def step():
        q3k.add_rms_norm(b["h1"], b["d1"], b["w1"], b["y1"], B, H, EPS, stream)
        q3k.qk_norm_rope(b["q"], b["k"], b["qw"], b["kw"], B, 1, Hq, Hkv, D, EPS, b["cache"], P, 0, b["pos"], stream)
        q3k.add_rms_norm(b["h2"], b["d2"], b["w2"], b["y2"], B, H, EPS, stream)
        q3k.silu_mul(b["g"], b["u"], b["o"], B * I, stream)
        q3k.gqa_attention(b["aq"], b["kc"], b["vc"], b["ao"], Bd, 1, Hq, Hkv, D, L, L - 1, st, st, stream,
                          workspace=ws_a, workspace_bytes=wa)
        q3k.argmax(b["logits"], b["ids"], Bd, V, V, stream, workspace=ws_m, workspace_bytes=wm)
        q3k.topk_candidates(b["logits"], Bd, V, V, K, cap, b["cnt"], b["ci"], b["cv"], b["bad"], stream,
                            workspace=ws_k, workspace_bytes=wk)

    changed = ("h1", "q", "k", "h2")   # rewritten in place by the step

    def reset():
        for k in changed:
            bufs[k].upload(arrays[k])

    def results():
        shapes = {"h1": ((B, H), np.uint16), "y1": ((B, H), np.uint16), "q": ((B, Hq * D), np.uint16),
                  "k": ((B, Hkv * D), np.uint16), "h2": ((B, H), np.uint16), "y2": ((B, H), np.uint16),
                  "o": ((B, I), np.uint16), "ao": ((Bd, Hq * D), np.uint16), "ids": ((Bd,), np.int32),
                  "cnt": ((Bd,), np.int32), "bad": ((Bd,), np.int32)}
        got = {k: bufs[k].download(dt, sh) for k, (sh, dt) in shapes.items()}
        # candidates come in no particular order: compare each row's first count entries as sorted sets
        ci = bufs["ci"].download(np.int32, (Bd, cap))
        cv = bufs["cv"].download(np.uint16, (Bd, cap))
        for r in range(Bd):
            n = min(int(got["cnt"][r]), cap)
            order = np.argsort(ci[r, :n], kind="stable")
            got[f"cand{r}"] = np.concatenate([ci[r, :n][order].astype(np.int64), cv[r, :n][order].astype(np.int64)])
        return got

    step()
    stream.synchronize()
    eager = results()
    assert not np.array_equal(eager["h1"], arrays["h1"]), "the step should have updated the residual"

    reset()
    graph = hip.Graph(stream, step)
    try:
        scratch = hip.DeviceBuffer(B * I * 2)
        for replay in range(3):
            reset()
            # eager work between replays, on the same stream
            q3k.silu_mul(b["u"], b["g"], scratch, B * I, stream)
            stream.synchronize()
            graph.launch(stream)
            stream.synchronize()
            got = results()
            for k, want in eager.items():
                assert np.array_equal(got[k], want), f"replay {replay}: {k} differs from the eager step"
        scratch.free()
    finally:
        graph.destroy()
