"""Every op of every benchmark config at its full size (benchmark configs
2-5), through the C ABI, against the oracle on the host.

Inputs follow the configs' stated distributions (synth.py; unstated ones:
residual deltas and Q/K ~ N(0,1), norm weights ~ N(1, 0.1)).  Each test
builds only the tensors of its op.
"""
import numpy as np
import pytest

from gpu_util import Guarded, announce, check_band, check_exact

pytestmark = pytest.mark.gpu
EPS = 1e-6
D = 128


def positions_for(c, synth, configs):
    if c.positions == "range":
        return None, 0  # scalar form: position = 0 + s for every sequence
    return synth.uniform_positions(c.seed, configs.TID_POS, c.tokens, c.max_pos), 0


@pytest.mark.parametrize("cfg", ["c2", "c4"])
def test_embedding_config(q3k, hip, oracle, synth, configs, cfg):
    c = configs.CONFIGS[cfg]
    announce(f"embedding {cfg}")
    std = 0.02 if cfg == "c2" else 1.0
    table = synth.normal_bf16(c.seed, configs.TID_TABLE, (configs.VOCAB, c.hidden), std=std)
    ids = synth.token_ids(c.seed, configs.TID_IDS, (c.batch, c.seq), configs.VOCAB)
    I, Tb, O = Guarded(hip, ids), Guarded(hip, table), Guarded(hip, nbytes=ids.size * c.hidden * 2)
    q3k.embedding(I, ids.size, Tb, configs.VOCAB, c.hidden, O)
    hip.synchronize()
    got = O.get(np.uint16, (c.batch, c.seq, c.hidden))
    assert O.guards_intact()
    check_exact(f"embedding {cfg}", got, oracle.embedding(ids, table))


@pytest.mark.parametrize("cfg", ["c2", "c3", "c4", "c5"])
def test_add_rms_norm_config(q3k, hip, oracle, synth, configs, cfg):
    c = configs.CONFIGS[cfg]
    announce(f"add_rms_norm {cfg}")
    h = synth.normal_bf16(c.seed, configs.TID_H, (c.tokens, c.hidden))
    d = synth.normal_bf16(c.seed, configs.TID_D1, (c.tokens, c.hidden))
    w = synth.normal_bf16(c.seed, configs.TID_W1, (c.hidden,), mean=1.0, std=0.1)
    H, Dd, W, Y = Guarded(hip, h), Guarded(hip, d), Guarded(hip, w), Guarded(hip, nbytes=h.nbytes)
    q3k.add_rms_norm(H, Dd, W, Y, c.tokens, c.hidden, EPS)
    hip.synchronize()
    h_got, y_got = H.get(np.uint16, h.shape), Y.get(np.uint16, h.shape)
    assert all(b.guards_intact() for b in (H, Dd, W, Y))
    h_ref, prim, lo, hi = oracle.add_rms_norm(h, d, w, EPS)
    check_exact(f"add_rms_norm {cfg} residual", h_got, h_ref)
    check_band(oracle, f"add_rms_norm {cfg}", y_got, prim, lo, hi)


@pytest.mark.parametrize("cfg", ["c4", "c5"])
def test_final_rms_norm_config(q3k, hip, oracle, synth, configs, cfg):
    c = configs.CONFIGS[cfg]
    announce(f"rms_norm {cfg}")
    x = synth.normal_bf16(c.seed, configs.TID_X, (c.tokens, c.hidden))
    w = synth.normal_bf16(c.seed, configs.TID_WF, (c.hidden,), mean=1.0, std=0.1)
    X, W, Y = Guarded(hip, x), Guarded(hip, w), Guarded(hip, nbytes=x.nbytes)
    q3k.rms_norm(X, W, Y, c.tokens, c.hidden, EPS)
    hip.synchronize()
    got = Y.get(np.uint16, x.shape)
    assert Y.guards_intact()
    prim, lo, hi = oracle.rms_norm(x, w, EPS)
    check_band(oracle, f"rms_norm {cfg}", got, prim, lo, hi)


@pytest.mark.parametrize("cfg", ["c2", "c3", "c4", "c5"])
def test_qk_norm_rope_config(q3k, hip, oracle, synth, configs, cfg):
    c = configs.CONFIGS[cfg]
    announce(f"qk_norm_rope {cfg}")
    q = synth.normal_bf16(c.seed, configs.TID_Q, (c.batch, c.seq, c.heads_q * D))
    k = synth.normal_bf16(c.seed, configs.TID_K, (c.batch, c.seq, c.heads_kv * D))
    qw = synth.normal_bf16(c.seed, configs.TID_QW, (D,), mean=1.0, std=0.1)
    kw = synth.normal_bf16(c.seed, configs.TID_KW, (D,), mean=1.0, std=0.1)
    cache = q3k.build_rope_cache(c.max_pos, D, configs.THETA)
    pos, start = positions_for(c, synth, configs)
    Q, K, QW, KW, C = Guarded(hip, q), Guarded(hip, k), Guarded(hip, qw), Guarded(hip, kw), Guarded(hip, cache)
    Pz = Guarded(hip, pos) if pos is not None else None
    q3k.qk_norm_rope(Q, K, QW, KW, c.batch, c.seq, c.heads_q, c.heads_kv, D, EPS, C, c.max_pos, start, Pz)
    hip.synchronize()
    gq, gk = Q.get(np.uint16, q.shape), K.get(np.uint16, k.shape)
    assert Q.guards_intact() and K.guards_intact()
    pq, lq, hq = oracle.qk_norm_rope(q, qw, c.batch, c.seq, c.heads_q, D, EPS, cache, start, pos)
    check_band(oracle, f"qk_norm_rope {cfg} q", gq, pq, lq, hq)
    del pq, lq, hq
    pk, lk, hk = oracle.qk_norm_rope(k, kw, c.batch, c.seq, c.heads_kv, D, EPS, cache, start, pos)
    check_band(oracle, f"qk_norm_rope {cfg} k", gk, pk, lk, hk)


@pytest.mark.parametrize("cfg", ["c2", "c3", "c4", "c5"])
def test_silu_mul_config(q3k, hip, oracle, synth, configs, cfg):
    c = configs.CONFIGS[cfg]
    announce(f"silu_mul {cfg}")
    g = synth.normal_bf16(c.seed, configs.TID_GATE, (c.tokens, c.inter))
    u = synth.normal_bf16(c.seed, configs.TID_UP, (c.tokens, c.inter))
    G, U, O = Guarded(hip, g), Guarded(hip, u), Guarded(hip, nbytes=g.nbytes)
    q3k.silu_mul(G, U, O, g.size)
    hip.synchronize()
    got = O.get(np.uint16, g.shape)
    assert O.guards_intact()
    del G, U, O
    prim, lo, hi = oracle.silu_mul(g, u)
    check_band(oracle, f"silu_mul {cfg}", got, prim, lo, hi)

