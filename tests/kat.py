"""Known-answer inputs of the reference's GPU op tests, restated as data
generators (closed-form integer patterns, exactly representable in bf16).

Sources (reference tests/unit/):
  rms_norm_cuda_test.cpp:111-141    x[i] = ((i % 31) - 15) * 0.125, w[j] = 0.5 + (j % 17) * 0.03125
  rope_cuda_test.cpp:38-58, 210-241 v[i] = ((i + off) % 17 - 8) * 0.25, off 0 (Q) / 5 (K)
  elementwise_cuda_test.cpp:138-181 residual ((i%41)-20)/16, delta ((i%17)-8)/32,
                                    gate ((i%37)-18)/4, up ((i%23)-11)/8
  embedding_cuda_test.cpp:102-143   W[t, h] = 10 t + h, ids [[2,0,4],[1,2,3]]
"""
import numpy as np


def bf(values):
    """Exact float -> bf16 bits for values representable in bf16."""
    v = np.asarray(values, dtype=np.float32)
    b = v.view(np.uint32)
    assert np.all((b & 0xFFFF) == 0), "KAT value not exact in bf16"
    return (b >> 16).astype(np.uint16)


def rms_input(shape):
    n = int(np.prod(shape))
    i = np.arange(n)
    return bf(((i % 31) - 15) * 0.125).reshape(shape)


def rms_weight(hidden):
    j = np.arange(hidden)
    return bf(0.5 + (j % 17) * 0.03125)


def rope_values(n, offset):
    i = np.arange(n)
    return bf((((i + offset) % 17) - 8) * 0.25)


def elementwise_inputs(shape=(2, 3, 257)):
    n = int(np.prod(shape))
    i = np.arange(n)
    return (bf(((i % 41) - 20) * 0.0625).reshape(shape), bf(((i % 17) - 8) * 0.03125).reshape(shape),
            bf(((i % 37) - 18) * 0.25).reshape(shape), bf(((i % 23) - 11) * 0.125).reshape(shape))


def embedding_inputs():
    V, H = 5, 4
    t, h = np.meshgrid(np.arange(V), np.arange(H), indexing="ij")
    table = bf((t * 10 + h).astype(np.float32))
    ids = np.array([[2, 0, 4], [1, 2, 3]], dtype=np.int32)
    return table, ids


# RoPE KAT constants (rope_cuda_test.cpp:210-220)
ROPE_B, ROPE_S, ROPE_HQ, ROPE_HKV, ROPE_D, ROPE_P, ROPE_START, ROPE_THETA = 1, 3, 2, 1, 8, 16, 5, 1.0e6


# KV cache KAT (kv_cache_cuda_test.cpp:124-138): 2 layers, batch 2, capacity 5, 2 KV heads of 4
KV_LAYERS, KV_BATCH, KV_SEQ_CAP, KV_HEADS, KV_DIM = 2, 2, 5, 2, 4


def kv_values(count, start):
    """kv_cache_cuda_test.cpp:27-43: start + 0.25 i, rounded to bf16 to nearest even."""
    bits = (np.float32(start) + np.arange(count, dtype=np.float32) * np.float32(0.25)).view(np.uint32).astype(np.uint64)
    bits = bits + 0x7FFF + ((bits >> 16) & 1)
    return (bits >> 16).astype(np.uint16)


def kv_steps():
    """(start, keys, values) of the test's prefill (2 tokens) and decode (1 token) appends, as [B, S, heads * dim]."""
    P = KV_HEADS * KV_DIM
    pre = (KV_BATCH, 2, P)
    dec = (KV_BATCH, 1, P)
    return [(0, kv_values(int(np.prod(pre)), 1.0).reshape(pre), kv_values(int(np.prod(pre)), 21.0).reshape(pre)),
            (2, kv_values(int(np.prod(dec)), 41.0).reshape(dec), kv_values(int(np.prod(dec)), 61.0).reshape(dec))]


# GQA attention KAT (gqa_attention_cuda_test.cpp:259-357): B 2, S 2 at start 1 (3 cached), 4 query heads over 2 KV
# heads of dim 4; value i of each tensor is ((i + offset) % 11 - 5) * scale; tolerance 0.04 (:239-257)
ATT_B, ATT_S, ATT_START, ATT_HQ, ATT_HKV, ATT_D, ATT_TOL = 2, 2, 1, 4, 2, 4, 0.04


def att_values(count, scale, offset):
    i = np.arange(count)
    return bf((((i + offset) % 11) - 5) * scale)


def att_inputs():
    """(query [B,S,Hq*D], keys [B,3,Hkv,D], values [B,3,Hkv,D]) of the test: one history token then the 2 current."""
    B, S, P = ATT_B, ATT_S, ATT_HKV * ATT_D
    hk = att_values(B * 1 * P, 0.125, 1).reshape(B, 1, P)
    hv = att_values(B * 1 * P, 0.25, 2).reshape(B, 1, P)
    ck = att_values(B * S * P, 0.125, 3).reshape(B, S, P)
    cv = att_values(B * S * P, 0.25, 4).reshape(B, S, P)
    q = att_values(B * S * ATT_HQ * ATT_D, 0.125, 5).reshape(B, S, ATT_HQ * ATT_D)
    keys = np.concatenate([hk, ck], axis=1).reshape(B, 1 + S, ATT_HKV, ATT_D)
    vals = np.concatenate([hv, cv], axis=1).reshape(B, 1 + S, ATT_HKV, ATT_D)
    return q, keys, vals


def argmax_inputs():
    """argmax_cuda_test.cpp:60-100: [2, 513] of -8, row 0 has 12 at 512, row 1 has 9 at 17 and at 500 (the tie
    resolves to the smaller index); expected [512, 17]."""
    x = np.full((2, 513), bf([-8.0])[0], np.uint16)
    x[0, 512] = bf([12.0])[0]
    x[1, 17] = bf([9.0])[0]
    x[1, 500] = bf([9.0])[0]
    return x, np.array([512, 17], np.int32)


# Sampler KAT (sampler_cuda_test.cpp:60-160): greedy / top-1 rows and the top-k 3, top-p 0.8 row
SAMPLER_GREEDY = np.array([[-1.0, 0.0, 4.0, 2.0, -2.0], [3.0, 7.0, 7.0, 1.0, 0.0]], np.float32)
SAMPLER_GREEDY_IDS = [2, 1]
SAMPLER_TOPP_ROW = np.array([2.0, 2.0, 1.0, -10.0], np.float32)   # top_k 3, top_p 0.8, T 1: only ids 0 and 1
