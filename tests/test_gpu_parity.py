"""Parity of the gfx950 kernels (through the C ABI) with the CPU oracle.

Bar: embedding and add bit-exact; every other bf16 output inside the
oracle's band widened by 1 bf16 ulp (q3k_oracle.h), i.e. within 1 ulp of a
result the reference's fp32 arithmetic can produce.  Every device buffer
carries guard bands that must be intact afterwards (no out-of-bounds
writes).  Shapes cover the reference tests' known answers, odd sizes that
take the generic kernels, unaligned pointers, empty inputs, out-of-range ids
and positions, and small slices of every benchmark config; the full-size
configs are in test_gpu_configs.py.
"""
import numpy as np
import pytest

import kat
from gpu_util import Guarded, announce, check_band, check_exact

pytestmark = pytest.mark.gpu
EPS = 1e-6


# ---------------------------------------------------------------- runners ---

def run_rms(q3k, hip, x, w, eps=EPS, offset=0):
    N = w.size
    rows = x.size // N
    X, W, Y = Guarded(hip, x, offset=offset), Guarded(hip, w, offset=offset), Guarded(hip, nbytes=x.nbytes, offset=offset)
    q3k.rms_norm(X, W, Y, rows, N, eps)
    hip.synchronize()
    y = Y.get(np.uint16, x.shape)
    assert X.guards_intact() and W.guards_intact() and Y.guards_intact()
    assert np.array_equal(X.get(np.uint16, x.shape), x), "rms_norm modified its input"
    return y


def run_add_rms(q3k, hip, h, d, w, eps=EPS, offset=0):
    N = w.size
    rows = h.size // N
    H, D, W = Guarded(hip, h, offset=offset), Guarded(hip, d, offset=offset), Guarded(hip, w, offset=offset)
    Y = Guarded(hip, nbytes=h.nbytes, offset=offset)
    q3k.add_rms_norm(H, D, W, Y, rows, N, eps)
    hip.synchronize()
    out = H.get(np.uint16, h.shape), Y.get(np.uint16, h.shape)
    assert all(b.guards_intact() for b in (H, D, W, Y))
    return out


def run_binary(q3k, hip, op, a, b, offset=0):
    A, B = Guarded(hip, a, offset=offset), Guarded(hip, b, offset=offset)
    if op == "silu":
        O = Guarded(hip, nbytes=a.nbytes, offset=offset)
        q3k.silu_mul(A, B, O, a.size)
    else:
        O = A
        q3k.add_inplace(A, B, a.size)
    hip.synchronize()
    out = O.get(np.uint16, a.shape)
    assert A.guards_intact() and B.guards_intact() and O.guards_intact()
    return out


def run_embedding(q3k, hip, ids, table, offset=0):
    V, H = table.shape
    I, Tb = Guarded(hip, ids), Guarded(hip, table, offset=offset)
    O = Guarded(hip, nbytes=ids.size * H * 2, offset=offset)
    q3k.embedding(I, ids.size, Tb, V, H, O)
    hip.synchronize()
    out = O.get(np.uint16, ids.shape + (H,))
    assert I.guards_intact() and Tb.guards_intact() and O.guards_intact()
    return out


def run_rope(q3k, hip, x, B, S, heads, D, cache, start=0, positions=None, offset=0):
    X, C = Guarded(hip, x, offset=offset), Guarded(hip, cache)
    Pz = Guarded(hip, positions) if positions is not None else None
    q3k.rope(X, B, S, heads, D, C, cache.shape[0], start, Pz)
    hip.synchronize()
    out = X.get(np.uint16, x.shape)
    assert X.guards_intact() and C.guards_intact()
    return out


def run_qknr(q3k, hip, q, k, qw, kw, B, S, Hq, Hkv, D, cache, start=0, positions=None, eps=EPS, offset=0):
    Q, K = Guarded(hip, q, offset=offset), Guarded(hip, k, offset=offset)
    QW, KW, C = Guarded(hip, qw), Guarded(hip, kw), Guarded(hip, cache)
    Pz = Guarded(hip, positions) if positions is not None else None
    q3k.qk_norm_rope(Q, K, QW, KW, B, S, Hq, Hkv, D, eps, C, cache.shape[0], start, Pz)
    hip.synchronize()
    out = Q.get(np.uint16, q.shape), K.get(np.uint16, k.shape)
    assert all(b.guards_intact() for b in (Q, K, QW, KW, C))
    return out


# ---------------------------------------------------------------- rms_norm ---

@pytest.mark.parametrize("shape", [(2, 3, 1024), (2, 3, 4, 128)])
def test_rms_norm_kat(q3k, hip, oracle, shape):
    announce(f"rms_norm kat {shape}")
    x, w = kat.rms_input(shape), kat.rms_weight(shape[-1])
    y = run_rms(q3k, hip, x, w)
    prim, lo, hi = oracle.rms_norm(x, w, EPS)
    check_band(oracle, f"rms_norm kat {shape}", y, prim, lo, hi)


RMS_CASES = [(16, 1024, 0), (5, 2048, 0), (3, 16384, 0), (2, 16392, 0), (4, 7168, 0), (6, 768, 0), (1, 8, 0), (3, 16, 0), (5, 24, 0), (7, 64, 0), (100, 128, 0), (9, 200, 0), (4, 256, 0),
             (6, 512, 0), (3, 1000, 0), (64, 4096, 0), (17, 5120, 0), (2, 8192, 0), (3, 8200, 0), (5, 257, 0),
             (7, 1024, 2), (33, 128, 2), (1, 1, 0),
             # per-head rows in the four-rows-per-lane-group range (16384 .. 65536 rows), whole and with a partial
             # last wave; 1024-wide rows in the two-rows-per-wave range (from 4096 rows), whole and partial
             (16384, 128, 0), (65536, 128, 0), (20001, 128, 0), (4096, 1024, 0), (4099, 1024, 0), (8192, 1000, 0)]


@pytest.mark.parametrize("rows,n,offset", RMS_CASES)
def test_rms_norm_shapes(q3k, hip, oracle, synth, rows, n, offset):
    name = f"rms_norm rows={rows} N={n} offset={offset}"
    announce(name)
    x = synth.normal_bf16(100, n, (rows, n))
    w = synth.normal_bf16(101, n, (n,), mean=1.0, std=0.1)
    y = run_rms(q3k, hip, x, w, offset=offset)
    prim, lo, hi = oracle.rms_norm(x, w, EPS)
    check_band(oracle, name, y, prim, lo, hi)


def test_rms_norm_config1(q3k, hip, oracle, synth, configs):
    """Benchmark config 1: x [16, 1024] ~ N(0,1), w ~ N(1, 0.1), eps 1e-6, seed 0."""
    announce("rms_norm c1")
    c = configs.CONFIGS["c1"]
    x = synth.normal_bf16(c.seed, configs.TID_X, (c.seq, c.hidden))
    w = synth.normal_bf16(c.seed, configs.TID_WF, (c.hidden,), mean=1.0, std=0.1)
    y = run_rms(q3k, hip, x, w)
    prim, lo, hi = oracle.rms_norm(x, w, EPS)
    st = check_band(oracle, "rms_norm c1", y, prim, lo, hi)
    assert st["ulp_hist"][2] + st["ulp_hist"][3] <= st["ambiguous"]


@pytest.mark.parametrize("rows,n,offset", [(16, 1024, 0), (64, 4096, 0), (9, 5120, 0), (3, 8200, 0), (5, 257, 0),
                                           (11, 1024, 2), (40, 128, 0), (3, 2048, 0), (2, 16384, 0), (4, 768, 0),
                                           (3, 7168, 0), (5, 512, 0)])
def test_add_rms_norm(q3k, hip, oracle, synth, rows, n, offset):
    name = f"add_rms_norm rows={rows} N={n} offset={offset}"
    announce(name)
    h = synth.normal_bf16(102, n, (rows, n))
    d = synth.normal_bf16(103, n, (rows, n))
    w = synth.normal_bf16(104, n, (n,), mean=1.0, std=0.1)
    h_out, y = run_add_rms(q3k, hip, h, d, w, offset=offset)
    h_ref, prim, lo, hi = oracle.add_rms_norm(h, d, w, EPS)
    check_exact(name + " residual", h_out, h_ref)
    check_band(oracle, name, y, prim, lo, hi)


# ---------------------------------------------------------------- elementwise -

def test_elementwise_kat(q3k, hip, oracle):
    announce("elementwise kat")
    r, d, g, u = kat.elementwise_inputs()
    check_exact("add kat", run_binary(q3k, hip, "add", r, d), oracle.add_inplace(r, d))
    prim, lo, hi = oracle.silu_mul(g, u)
    check_band(oracle, "silu kat", run_binary(q3k, hip, "silu", g, u), prim, lo, hi)


@pytest.mark.parametrize("n,offset", [(1, 0), (7, 0), (8, 0), (9, 0), (1000, 0), (8191, 0), (65536 + 3, 0),
                                      (1 << 20, 0), (4097, 2), (1 << 16, 2),
                                      # 8-byte aligned: the small-launch kernel's 64-bit accesses
                                      (1001, 8), ((1 << 19) + 3, 8),
                                      # above the small-launch size (2 MiB written): the 128-bit kernels,
                                      # or the scalar kernel for pointers that are not 16-byte aligned
                                      ((1 << 20) + 3, 8), ((3 << 20) + 5, 0), ((3 << 20) + 1, 8)])
def test_elementwise_shapes(q3k, hip, oracle, synth, n, offset):
    name = f"elementwise n={n} offset={offset}"
    announce(name)
    a = synth.normal_bf16(105, n, (n,), std=3.0)
    b = synth.normal_bf16(106, n, (n,))
    check_exact("add " + name, run_binary(q3k, hip, "add", a, b, offset), oracle.add_inplace(a, b))
    prim, lo, hi = oracle.silu_mul(a, b)
    check_band(oracle, "silu " + name, run_binary(q3k, hip, "silu", a, b, offset), prim, lo, hi)


@pytest.mark.parametrize("repeats", [9, 140003])
def test_silu_extremes(q3k, hip, oracle, synth, repeats):
    """Denominators past 2^126 and infinite ones (the IEEE-divide side) mixed with ordinary values in one lane:
    144 elements (the small-launch kernel and its scalar tail) and 2.2M (the 128-bit kernel)."""
    announce(f"silu extremes x{repeats}")
    vals = np.array([-100.0, -89.0, -88.0, -87.0, -20.0, -1e-30, 0.0, 1e-30, 20.0, 88.0, 100.0, 3.0e38, -3.0e38,
                     1e-38, -1e-38, -0.0], np.float32)
    g = synth.f32_to_bf16(np.tile(vals, repeats))
    u = np.full(g.shape, 0x3F80, np.uint16)
    prim, lo, hi = oracle.silu_mul(g, u)
    check_band(oracle, "silu extremes", run_binary(q3k, hip, "silu", g, u), prim, lo, hi)


def test_silu_output_may_alias_input(q3k, hip, oracle, synth):
    announce("silu in place")
    g = synth.normal_bf16(107, 0, (4096 + 5,))
    u = synth.normal_bf16(107, 1, (4096 + 5,))
    G, U = Guarded(hip, g), Guarded(hip, u)
    q3k.silu_mul(G, U, G, g.size)
    hip.synchronize()
    prim, lo, hi = oracle.silu_mul(g, u)
    check_band(oracle, "silu in place", G.get(np.uint16, g.shape), prim, lo, hi)


# ---------------------------------------------------------------- embedding ---

def test_embedding_kat(q3k, hip, oracle):
    announce("embedding kat")
    table, ids = kat.embedding_inputs()
    check_exact("embedding kat", run_embedding(q3k, hip, ids, table), oracle.embedding(ids, table))


# one wave per token up to 128 vectors a row (H 1024), two up to 256 (H 1032, 2048), four beyond (H 4096,
# 5120 with a partial second pass, 40960); H 12 and the 2-byte offset take the scalar kernel
@pytest.mark.parametrize("V,H,T,offset", [(1000, 1024, 300, 0), (500, 4096, 77, 0), (300, 5120, 64, 0),
                                          (200, 2048, 41, 0), (100, 1032, 7, 0),
                                          (50, 8, 9, 0), (64, 12, 33, 0), (100, 1024, 10, 2), (10, 40960, 3, 0)])
def test_embedding_shapes(q3k, hip, oracle, synth, V, H, T, offset):
    name = f"embedding V={V} H={H} T={T} offset={offset}"
    announce(name)
    table = synth.normal_bf16(108, H, (V, H), std=0.02)
    ids = synth.token_ids(109, T, (T,), V)
    ids[:3] = [-1, V, V - 1][:min(3, T)]
    check_exact(name, run_embedding(q3k, hip, ids, table, offset), oracle.embedding(ids, table))


# ---------------------------------------------------------------- rope -------

def test_rope_kat(q3k, hip, oracle):
    announce("rope kat")
    B, S, Hq, Hkv, D, P, start = (kat.ROPE_B, kat.ROPE_S, kat.ROPE_HQ, kat.ROPE_HKV, kat.ROPE_D, kat.ROPE_P,
                                  kat.ROPE_START)
    cache = q3k.build_rope_cache(P, D, kat.ROPE_THETA)
    for heads, off in ((Hq, 0), (Hkv, 5)):
        v = kat.rope_values(B * S * heads * D, off).reshape(B, S, heads * D)
        prim, lo, hi = oracle.rope(v, B, S, heads, D, cache, start)
        check_band(oracle, f"rope kat heads={heads}", run_rope(q3k, hip, v, B, S, heads, D, cache, start),
                   prim, lo, hi)
    with pytest.raises(IndexError):
        X, C = Guarded(hip, v), Guarded(hip, cache)
        q3k.rope(X, B, S, Hkv, D, C, P, P - 1)


@pytest.mark.parametrize("B,S,heads,D,start,offset", [(1, 64, 16, 128, 0, 0), (2, 33, 8, 128, 100, 0),
                                                      (4, 16, 32, 128, 7, 0), (1, 5, 2, 128, 0, 0),
                                                      (2, 9, 4, 64, 3, 0), (1, 7, 8, 128, 0, 2),
                                                      (3, 4, 6, 128, 1, 0),
                                                      # head counts that are not a multiple of 4: waves span tokens,
                                                      # and the last wave is partial
                                                      (3, 7, 1, 128, 2, 0), (2, 5, 3, 128, 0, 0),
                                                      # the same at a larger size, partial last wave
                                                      (2, 9000, 3, 128, 5, 0)])
def test_rope_shapes(q3k, hip, oracle, synth, B, S, heads, D, start, offset):
    name = f"rope B={B} S={S} heads={heads} D={D} start={start} offset={offset}"
    announce(name)
    cache = q3k.build_rope_cache(start + S + 3, D, 1.0e6)
    x = synth.normal_bf16(110, heads * S, (B, S, heads * D))
    prim, lo, hi = oracle.rope(x, B, S, heads, D, cache, start)
    check_band(oracle, name, run_rope(q3k, hip, x, B, S, heads, D, cache, start, offset=offset), prim, lo, hi)


@pytest.mark.parametrize("B", [64, 2048])   # a small launch, and the large-launch instance with positions
def test_rope_positions_overload(q3k, hip, oracle, synth, B):
    announce(f"rope positions B={B}")
    S, heads, D, P = 1, 32, 128, 4096
    cache = q3k.build_rope_cache(P, D, 1.0e6)
    x = synth.normal_bf16(111, 0, (B, S, heads * D))
    pos = synth.uniform_positions(111, 1, B * S, P)
    pos[:4] = [0, P - 1, P, -5]  # the last two are outside the table: NaN heads
    prim, lo, hi = oracle.rope(x, B, S, heads, D, cache, positions=pos)
    got = run_rope(q3k, hip, x, B, S, heads, D, cache, positions=pos)
    check_band(oracle, f"rope positions B={B}", got, prim, lo, hi)
    assert np.all((got[2:4] & 0x7FFF) > 0x7F80)


@pytest.mark.parametrize("B,S,Hq,Hkv,D,start,offset,with_pos", [
    (4, 256, 32, 8, 128, 0, 0, False),   # config 4 heads: 4 heads per lane for Q, 2 for K
    (1, 512, 16, 8, 128, 0, 0, False),   # config 2 shape
    (64, 1, 32, 8, 128, 0, 0, True),     # config 3 decode: small launch, a position per sequence
    (2, 64, 64, 8, 128, 9, 0, False),    # config 5 heads
    (4, 64, 4, 1, 128, 0, 0, False),     # a tensor-parallel-8 shard: K head count not a multiple of 4
    (3, 7, 6, 2, 128, 1, 0, False),      # both head counts not multiples of 4, partial last waves
    (4, 1024, 4, 1, 128, 0, 0, False),   # a tensor-parallel-8 shard, larger
    (3, 1001, 6, 2, 128, 1, 0, False),   # rows per lane group with partial last waves, larger
    (4096, 1, 5, 3, 128, 0, 0, True),    # rows per lane group with a position per sequence
    (2, 9, 4, 4, 64, 2, 0, False),       # head_dim 64: the generic kernel, two launches
    (1, 7, 8, 8, 128, 0, 2, False)])     # unaligned: the generic kernel
def test_rope_qk_one_launch(q3k, hip, oracle, synth, B, S, Hq, Hkv, D, start, offset, with_pos):
    """apply_rope_inplace's single launch over Q and K (q3k_rope_qk_bf16): bit-equal to q3k_rope_bf16 on Q, then
    on K (the reference's two launches, rope.cu:326-332), and inside the oracle's band."""
    name = f"rope_qk B={B} S={S} Hq={Hq} Hkv={Hkv} D={D} start={start} offset={offset} pos={with_pos}"
    announce(name)
    P = 4096 if with_pos else start + S + 2
    cache = q3k.build_rope_cache(P, D, 1.0e6)
    q = synth.normal_bf16(120, Hq * S, (B, S, Hq * D))
    k = synth.normal_bf16(121, Hkv * S, (B, S, Hkv * D))
    pos = synth.uniform_positions(122, B, B * S, P) if with_pos else None
    Q, K, C = Guarded(hip, q, offset=offset), Guarded(hip, k, offset=offset), Guarded(hip, cache)
    Pz = Guarded(hip, pos) if pos is not None else None
    q3k.rope_qk(Q, K, B, S, Hq, Hkv, D, C, P, start, Pz)
    hip.synchronize()
    gq, gk = Q.get(np.uint16, q.shape), K.get(np.uint16, k.shape)
    assert all(b.guards_intact() for b in (Q, K, C))
    check_exact(name + " q vs rope", gq, run_rope(q3k, hip, q, B, S, Hq, D, cache, start, pos, offset))
    check_exact(name + " k vs rope", gk, run_rope(q3k, hip, k, B, S, Hkv, D, cache, start, pos, offset))
    pq, lq, hq = oracle.rope(q, B, S, Hq, D, cache, start, positions=pos)
    pk, lk, hk = oracle.rope(k, B, S, Hkv, D, cache, start, positions=pos)
    check_band(oracle, name + " q", gq, pq, lq, hq)
    check_band(oracle, name + " k", gk, pk, lk, hk)
    with pytest.raises(IndexError):
        q3k.rope_qk(Q, K, B, S, Hq, Hkv, D, C, P, P - S + 1)


# ---------------------------------------------------------------- qk norm + rope

@pytest.mark.parametrize("B,S,Hq,Hkv,D,start,offset", [(1, 512, 16, 8, 128, 0, 0), (4, 64, 32, 8, 128, 0, 0),
                                                       (2, 32, 64, 8, 128, 5, 0), (1, 3, 2, 1, 8, 5, 0),
                                                       (2, 5, 6, 2, 128, 0, 0), (1, 8, 4, 4, 128, 0, 2),
                                                       (1, 4, 4, 4, 64, 2, 0),
                                                       # config 4 at one rank of 8-way tensor parallelism (4 query
                                                       # heads, 1 KV head), full size; other head counts that are
                                                       # not a multiple of 4, with partial last waves
                                                       (4, 2048, 4, 1, 128, 0, 0), (3, 7, 5, 3, 128, 1, 0),
                                                       (1, 9, 4, 1, 128, 0, 0), (2, 3, 1, 1, 128, 0, 0),
                                                       (1, 11, 2, 2, 128, 4, 0), (2, 9, 6, 4, 128, 3, 0),
                                                       # the same at larger sizes, partial last waves
                                                       (2, 1500, 5, 3, 128, 0, 0), (1, 7000, 2, 1, 128, 9, 0)])
def test_qk_norm_rope_shapes(q3k, hip, oracle, synth, B, S, Hq, Hkv, D, start, offset):
    name = f"qk_norm_rope B={B} S={S} Hq={Hq} Hkv={Hkv} D={D} start={start} offset={offset}"
    announce(name)
    cache = q3k.build_rope_cache(start + S + 1, D, 1.0e6)
    q = synth.normal_bf16(112, Hq * S, (B, S, Hq * D))
    k = synth.normal_bf16(113, Hkv * S, (B, S, Hkv * D))
    qw = synth.normal_bf16(114, D, (D,), mean=1.0, std=0.1)
    kw = synth.normal_bf16(115, D, (D,), mean=1.0, std=0.1)
    gq, gk = run_qknr(q3k, hip, q, k, qw, kw, B, S, Hq, Hkv, D, cache, start, offset=offset)
    pq, lq, hq = oracle.qk_norm_rope(q, qw, B, S, Hq, D, EPS, cache, start)
    pk, lk, hk = oracle.qk_norm_rope(k, kw, B, S, Hkv, D, EPS, cache, start)
    check_band(oracle, name + " q", gq, pq, lq, hq)
    check_band(oracle, name + " k", gk, pk, lk, hk)


def test_qk_norm_rope_rows_positions(q3k, hip, oracle, synth):
    """Head counts that are not a multiple of 4 (rows per lane group) with a position per sequence (decode at a
    tensor-parallel shard of many sequences), some of them outside the table: those heads become NaN, every other
    head is inside the band."""
    B, S, Hq, Hkv, D, P = 8192, 1, 4, 1, 128, 4096
    announce("qk_norm_rope rows per lane group, positions")
    cache = q3k.build_rope_cache(P, D, 1.0e6)
    q = synth.normal_bf16(116, 1, (B, S, Hq * D))
    k = synth.normal_bf16(117, 1, (B, S, Hkv * D))
    qw = synth.normal_bf16(118, D, (D,), mean=1.0, std=0.1)
    kw = synth.normal_bf16(119, D, (D,), mean=1.0, std=0.1)
    pos = synth.uniform_positions(116, 2, B * S, P)
    pos[[5, 77, 4000]] = [P, -1, P + 100]
    gq, gk = run_qknr(q3k, hip, q, k, qw, kw, B, S, Hq, Hkv, D, cache, positions=pos)
    pq, lq, hq = oracle.qk_norm_rope(q, qw, B, S, Hq, D, EPS, cache, positions=pos)
    pk, lk, hk = oracle.qk_norm_rope(k, kw, B, S, Hkv, D, EPS, cache, positions=pos)
    check_band(oracle, "rows positions q", gq, pq, lq, hq)
    check_band(oracle, "rows positions k", gk, pk, lk, hk)
    for t in (5, 77, 4000):
        assert np.all((gq[t] & 0x7FFF) > 0x7F80) and np.all((gk[t] & 0x7FFF) > 0x7F80), t


def _special_rows(synth, rows, n, seed):
    """Rows of normal values with one special case each: +inf, -inf, NaN, values whose squares overflow fp32,
    all zeros, values near the smallest normal, and a row spanning +-3e38; the rest stay normal."""
    f = synth.bf16_to_f32(synth.normal_bf16(seed, n, (rows, n))).copy()
    special = [lambda r: r.__setitem__(3, np.inf), lambda r: r.__setitem__(n // 2, -np.inf),
               lambda r: r.__setitem__(n - 1, np.nan), lambda r: r.__setitem__(slice(None), r * 2.0e37),
               lambda r: r.__setitem__(slice(None), 0.0), lambda r: r.__setitem__(slice(None), r * 1.5e-38),
               lambda r: r.__setitem__(slice(0, 2), [3.0e38, -3.0e38])]
    for i, fn in enumerate(special[:rows]):
        fn(f[i])
    return synth.f32_to_bf16(f.astype(np.float32))


@pytest.mark.parametrize("n", [4096, 128])
def test_norms_special_values(q3k, hip, oracle, synth, n):
    """RMSNorm and add + RMSNorm on rows holding +-inf, NaN, overflowing squares, zeros and near-underflow
    values (the reference's arithmetic propagates them: an infinite sum of squares gives 1/rms = 0, so finite
    elements become 0 and infinite ones NaN): the same non-finite pattern and the same finite values, within the
    band, as the oracle."""
    rows = 9
    name = f"norm special values N={n}"
    announce(name)
    x = _special_rows(synth, rows, n, 120)
    w = synth.normal_bf16(121, n, (n,), mean=1.0, std=0.1)
    prim, lo, hi = oracle.rms_norm(x, w, EPS)
    check_band(oracle, name, run_rms(q3k, hip, x, w), prim, lo, hi)
    d = _special_rows(synth, rows, n, 122)[::-1].copy()
    h_out, y = run_add_rms(q3k, hip, x, d, w)
    h_ref, prim, lo, hi = oracle.add_rms_norm(x, d, w, EPS)
    # the residual is bit-exact except that NaN payloads may differ
    nan_got, nan_ref = np.isnan(synth.bf16_to_f32(h_out)), np.isnan(synth.bf16_to_f32(h_ref))
    assert np.array_equal(nan_got, nan_ref), "residual NaN positions differ"
    check_exact(name + " add residual", h_out[~nan_ref], h_ref[~nan_ref])
    check_band(oracle, name + " add", y, prim, lo, hi)


def test_qk_norm_rope_special_values(q3k, hip, oracle, synth):
    """Q/K norm + RoPE on heads holding +-inf, NaN, overflowing squares, zeros and near-underflow values: the
    norm's zero or NaN results pass through the rotation as in the oracle."""
    B, S, Hq, Hkv, D = 1, 3, 4, 4, 128
    announce("qk_norm_rope special values")
    cache = q3k.build_rope_cache(S + 1, D, 1.0e6)
    q = _special_rows(synth, B * S * Hq, D, 123).reshape(B, S, Hq * D)
    k = _special_rows(synth, B * S * Hkv, D, 124)[::-1].copy().reshape(B, S, Hkv * D)
    qw = synth.normal_bf16(125, D, (D,), mean=1.0, std=0.1)
    kw = synth.normal_bf16(126, D, (D,), mean=1.0, std=0.1)
    gq, gk = run_qknr(q3k, hip, q, k, qw, kw, B, S, Hq, Hkv, D, cache)
    pq, lq, hq = oracle.qk_norm_rope(q, qw, B, S, Hq, D, EPS, cache)
    pk, lk, hk = oracle.qk_norm_rope(k, kw, B, S, Hkv, D, EPS, cache)
    check_band(oracle, "qk special q", gq, pq, lq, hq)
    check_band(oracle, "qk special k", gk, pk, lk, hk)


# 64 sequences: a decode-sized (small) launch, one head per lane group; 2048: the large-launch instance (4 query
# heads per lane, 2 KV heads) with positions read from memory
@pytest.mark.parametrize("B", [64, 2048])
def test_qk_norm_rope_positions_overload(q3k, hip, oracle, synth, B):
    announce(f"qk_norm_rope positions B={B}")
    S, Hq, Hkv, D, P = 1, 32, 8, 128, 4096
    cache = q3k.build_rope_cache(P, D, 1.0e6)
    q = synth.normal_bf16(116, 0, (B, S, Hq * D))
    k = synth.normal_bf16(116, 1, (B, S, Hkv * D))
    qw = synth.normal_bf16(116, 2, (D,), mean=1.0, std=0.1)
    kw = synth.normal_bf16(116, 3, (D,), mean=1.0, std=0.1)
    pos = synth.uniform_positions(116, 4, B * S, P)
    pos[5], pos[B - 1] = P + 10, -3   # outside the table: NaN heads
    gq, gk = run_qknr(q3k, hip, q, k, qw, kw, B, S, Hq, Hkv, D, cache, positions=pos)
    pq, lq, hq = oracle.qk_norm_rope(q, qw, B, S, Hq, D, EPS, cache, positions=pos)
    pk, lk, hk = oracle.qk_norm_rope(k, kw, B, S, Hkv, D, EPS, cache, positions=pos)
    check_band(oracle, f"qknr positions q B={B}", gq, pq, lq, hq)
    check_band(oracle, f"qknr positions k B={B}", gk, pk, lk, hk)
    for t in (5, B - 1):
        assert np.all((gq[t] & 0x7FFF) > 0x7F80) and np.all((gk[t] & 0x7FFF) > 0x7F80)


def test_fused_equals_unfused_on_gpu(q3k, hip, synth):
    """The fused kernels against the drop-in ops composed in reference order
    (decoder_layer.cpp:78->88, self_attention.cpp:147-152), both on the GPU."""
    announce("fused vs unfused")
    T, H, Hq, Hkv, D = 96, 1024, 16, 8, 128
    h = synth.normal_bf16(117, 0, (T, H))
    d = synth.normal_bf16(117, 1, (T, H))
    w = synth.normal_bf16(117, 2, (H,), mean=1.0, std=0.1)
    h1, y1 = run_add_rms(q3k, hip, h, d, w)
    hb = run_binary(q3k, hip, "add", h, d)
    y2 = run_rms(q3k, hip, hb, w)
    check_exact("add_rms_norm residual vs add_inplace", h1, hb)
    check_exact("add_rms_norm vs add_inplace + rms_norm", y1, y2)

    cache = q3k.build_rope_cache(T, D, 1.0e6)
    q = synth.normal_bf16(117, 3, (1, T, Hq * D))
    k = synth.normal_bf16(117, 4, (1, T, Hkv * D))
    qw = synth.normal_bf16(117, 5, (D,), mean=1.0, std=0.1)
    kw = synth.normal_bf16(117, 6, (D,), mean=1.0, std=0.1)
    fq, fk = run_qknr(q3k, hip, q, k, qw, kw, 1, T, Hq, Hkv, D, cache)
    nq = run_rms(q3k, hip, q, qw)
    nk = run_rms(q3k, hip, k, kw)
    check_exact("qk_norm_rope vs rms_norm + rope (q)", fq, run_rope(q3k, hip, nq, 1, T, Hq, D, cache))
    check_exact("qk_norm_rope vs rms_norm + rope (k)", fk, run_rope(q3k, hip, nk, 1, T, Hkv, D, cache))


# ---------------------------------------------------------------- caller fusions

@pytest.mark.parametrize("V,H,T,offset", [(1000, 1024, 77, 0), (500, 4096, 40, 0), (300, 5120, 9, 0),
                                          (64, 8192, 5, 0), (50, 12, 7, 0), (100, 1024, 10, 2), (64, 128, 33, 0)])
def test_embedding_rms_norm(q3k, hip, oracle, synth, V, H, T, offset):
    """Gather + first input norm: model.cpp:118 -> decoder_layer.cpp:72."""
    name = f"embedding_rms_norm V={V} H={H} T={T} offset={offset}"
    announce(name)
    table = synth.normal_bf16(120, H, (V, H))
    w = synth.normal_bf16(121, H, (H,), mean=1.0, std=0.1)
    ids = synth.token_ids(122, T, (T,), V)
    ids[:2] = [-3, V][:min(2, T)]
    I, Tb, W = Guarded(hip, ids), Guarded(hip, table, offset=offset), Guarded(hip, w, offset=offset)
    Hd, Y = Guarded(hip, nbytes=T * H * 2, offset=offset), Guarded(hip, nbytes=T * H * 2, offset=offset)
    q3k.embedding_rms_norm(I, T, Tb, V, H, W, EPS, Hd, Y)
    hip.synchronize()
    assert all(b.guards_intact() for b in (I, Tb, W, Hd, Y))
    emb = oracle.embedding(ids, table)
    check_exact(name + " hidden", Hd.get(np.uint16, (T, H)), emb)
    prim, lo, hi = oracle.rms_norm(emb, w, EPS)
    check_band(oracle, name, Y.get(np.uint16, (T, H)), prim, lo, hi)


@pytest.mark.parametrize("B,S,H,add,offset", [(4, 33, 4096, True, 0), (4, 33, 4096, False, 0), (2, 17, 5120, True, 0),
                                              (3, 5, 1024, False, 0), (64, 1, 4096, True, 0), (2, 9, 257, True, 0),
                                              (3, 7, 1024, True, 2)])
def test_last_token_norm(q3k, hip, oracle, synth, B, S, H, add, offset):
    """Final norm of the last token of each sequence: model.cpp:146 + lm_head.cpp:123-181."""
    name = f"last_token_norm B={B} S={S} H={H} add={add} offset={offset}"
    announce(name)
    h = synth.normal_bf16(123, H, (B, S, H))
    d = synth.normal_bf16(124, H, (B, S, H))
    w = synth.normal_bf16(125, H, (H,), mean=1.0, std=0.1)
    Hb, Db, W = Guarded(hip, h, offset=offset), Guarded(hip, d, offset=offset), Guarded(hip, w, offset=offset)
    Y = Guarded(hip, nbytes=B * H * 2, offset=offset)
    if add:
        q3k.add_rms_norm_rows(Hb, Db, W, Y, B, S - 1, S, H, EPS)
    else:
        q3k.rms_norm_rows(Hb, W, Y, B, S - 1, S, H, EPS)
    hip.synchronize()
    assert all(b.guards_intact() for b in (Hb, Db, W, Y))
    h_got = Hb.get(np.uint16, (B, S, H))
    last_h = h[:, -1, :]
    expect_h = h.copy()
    if add:
        expect_h[:, -1, :] = oracle.add_inplace(last_h, d[:, -1, :])
        _, prim, lo, hi = oracle.add_rms_norm(last_h, d[:, -1, :], w, EPS)
    else:
        prim, lo, hi = oracle.rms_norm(last_h, w, EPS)
    check_exact(name + " residual (only last rows change)", h_got, expect_h)
    check_band(oracle, name, Y.get(np.uint16, (B, H)), prim, lo, hi)


# ---------------------------------------------------------------- KV cache

def test_kv_append_kat(q3k, hip, oracle):
    """The reference test's prefill + decode appends into both layers (kv_cache_cuda_test.cpp:124-300)."""
    announce("kv_append KAT")
    L, Bc, Sc, P = kat.KV_LAYERS, kat.KV_BATCH, kat.KV_SEQ_CAP, kat.KV_HEADS * kat.KV_DIM
    KC = Guarded(hip, np.zeros((L, Bc, Sc, P), np.uint16))
    VC = Guarded(hip, np.zeros((L, Bc, Sc, P), np.uint16))
    kc = np.zeros((L, Bc, Sc, P), np.uint16)
    vc = np.zeros_like(kc)
    layer_bytes = Bc * Sc * P * 2
    for layer in range(L):
        for start, k, v in kat.kv_steps():
            K, V = Guarded(hip, k), Guarded(hip, v)
            q3k.kv_append(K, V, KC.ptr + layer * layer_bytes, VC.ptr + layer * layer_bytes, k.shape[0], k.shape[1],
                          P * 2, Sc, start)
            kc[layer], vc[layer] = oracle.kv_append(k, v, kc[layer], vc[layer], start)
    hip.synchronize()
    assert KC.guards_intact() and VC.guards_intact()
    check_exact("kv_append KAT keys", KC.get(np.uint16, kc.shape), kc)
    check_exact("kv_append KAT values", VC.get(np.uint16, vc.shape), vc)


@pytest.mark.parametrize("B,S,row,Bc,Sc,start,dtype,offset", [
    (4, 33, 1024, 4, 64, 7, np.uint16, 0),     # Qwen3-8B KV row (8 heads x 128), prefill
    (4, 1, 1024, 8, 64, 63, np.uint16, 0),     # decode into the last slot, batch below capacity
    (2, 5, 1024, 2, 9, 4, np.float32, 0),      # fp32 cache
    (3, 6, 3, 3, 10, 2, np.uint16, 0),         # 6-byte rows: 2-byte words
    (2, 7, 1024, 2, 11, 1, np.uint16, 2),      # unaligned pointers: 2-byte words
    (2, 4, 1024, 2, 4, 0, np.float32, 4),      # fp32, 4-byte aligned: 4-byte words
    (1, 300, 256, 1, 300, 0, np.uint16, 0),    # full capacity in one append
    (3, 5, 1024, 3, 8, 2, np.uint16, 0),       # 15 tokens: not a whole number of 4-token blocks
    (5, 3, 128, 6, 7, 4, np.uint16, 0),        # S below the tokens per block: one block spans batch rows
])
def test_kv_append_shapes(q3k, hip, oracle, synth, B, S, row, Bc, Sc, start, dtype, offset):
    name = f"kv_append B={B} S={S} row={row} cap=({Bc},{Sc}) start={start} {np.dtype(dtype).name} offset={offset}"
    announce(name)
    rng = np.random.default_rng(B * 1000 + S)
    mk = (lambda shape: rng.standard_normal(shape).astype(np.float32)) if dtype == np.float32 else \
        (lambda shape: rng.integers(0, 1 << 16, shape, dtype=np.uint16))
    k, v = mk((B, S, row)), mk((B, S, row))
    kc0, vc0 = mk((Bc, Sc, row)), mk((Bc, Sc, row))
    K, V = Guarded(hip, k, offset=offset), Guarded(hip, v, offset=offset)
    KC, VC = Guarded(hip, kc0, offset=offset), Guarded(hip, vc0, offset=offset)
    q3k.kv_append(K, V, KC, VC, B, S, k[0, 0].nbytes, Sc, start)
    hip.synchronize()
    assert all(b.guards_intact() for b in (K, V, KC, VC))
    kc, vc = oracle.kv_append(k, v, kc0, vc0, start)
    view = np.uint32 if dtype == np.float32 else np.uint16
    check_exact(name + " keys", KC.get(dtype, kc.shape).view(view), kc.view(view))
    check_exact(name + " values", VC.get(dtype, vc.shape).view(view), vc.view(view))


@pytest.mark.parametrize("B,S,Hq,Hkv,D,Sc,cs,positions,offset", [
    (2, 17, 32, 8, 128, 40, 5, None, 0),       # Qwen3-8B heads, prefill at cached length 5
    (4, 1, 16, 8, 128, 64, 63, None, 0),       # decode step into the last slot
    (3, 9, 8, 4, 128, 16, 0, "random", 0),     # per-token positions, one outside the table
    (2, 12, 64, 4, 128, 12, 0, None, 0),       # Qwen3-32B shape, whole capacity
    (2, 7, 4, 2, 64, 12, 3, None, 0),          # head_dim 64: generic path
    (2, 5, 8, 4, 128, 8, 2, None, 2),          # unaligned: generic path
    (2, 17, 4, 1, 128, 40, 5, None, 0),        # one rank of 8-way tensor parallelism: 4 query heads, 1 KV head
    (3, 9, 6, 2, 128, 16, 0, "random", 0),     # 6 and 2 heads, per-token positions, one outside the table
    (2, 5, 6, 4, 128, 8, 1, None, 0),          # per-lane rows for Q only (6 heads), K (4 heads) wave-uniform
])
def test_qk_norm_rope_kv_append(q3k, hip, oracle, synth, B, S, Hq, Hkv, D, Sc, cs, positions, offset):
    """Fused Q/K norm + RoPE + KV append (self_attention.cpp:147-156) against the oracle composition, and bit for
    bit against q3k_qk_norm_rope_bf16 followed by q3k_kv_append."""
    name = f"qk_norm_rope_kv_append B={B} S={S} Hq={Hq} Hkv={Hkv} D={D} cap={Sc} cs={cs} pos={positions} off={offset}"
    announce(name)
    P = 64
    start = cs if positions is None else 0
    q = synth.normal_bf16(130, Hq, (B, S, Hq * D))
    k = synth.normal_bf16(131, Hkv, (B, S, Hkv * D))
    v = synth.normal_bf16(132, Hkv, (B, S, Hkv * D))
    qw = synth.normal_bf16(133, D, (D,), mean=1.0, std=0.1)
    kw = synth.normal_bf16(134, D, (D,), mean=1.0, std=0.1)
    kc0 = synth.normal_bf16(135, Sc, (B + 1, Sc, Hkv * D))
    vc0 = synth.normal_bf16(136, Sc, (B + 1, Sc, Hkv * D))
    table = oracle.build_rope_cache(P, D, 1.0e6)
    pos = None
    if positions == "random":
        pos = synth.uniform_positions(137, 1, B * S, P).reshape(B, S)
        pos[1, 2] = P
    Q, K, V = Guarded(hip, q, offset=offset), Guarded(hip, k, offset=offset), Guarded(hip, v, offset=offset)
    QW, KW = Guarded(hip, qw, offset=offset), Guarded(hip, kw, offset=offset)
    KC, VC = Guarded(hip, kc0, offset=offset), Guarded(hip, vc0, offset=offset)
    C = Guarded(hip, table)
    PZ = Guarded(hip, pos) if pos is not None else None
    q3k.qk_norm_rope_kv_append(Q, K, V, QW, KW, B, S, Hq, Hkv, D, EPS, C, P, start, KC, VC, Sc, cs, PZ)
    hip.synchronize()
    assert all(b.guards_intact() for b in (Q, K, V, QW, KW, KC, VC, C))
    check_exact(name + " k input unchanged", K.get(np.uint16, k.shape), k)
    check_exact(name + " v input unchanged", V.get(np.uint16, v.shape), v)
    got_q = Q.get(np.uint16, q.shape)
    got_kc, got_vc = KC.get(np.uint16, kc0.shape), VC.get(np.uint16, vc0.shape)

    prim_q, lo_q, hi_q = oracle.qk_norm_rope(q, qw, B, S, Hq, D, EPS, table, start, pos)
    check_band(oracle, name + " q", got_q, prim_q, lo_q, hi_q)
    prim_k, lo_k, hi_k = oracle.qk_norm_rope(k, kw, B, S, Hkv, D, EPS, table, start, pos)
    rows = (slice(0, B), slice(cs, cs + S))
    check_band(oracle, name + " k cache rows", got_kc[rows], prim_k, lo_k, hi_k)
    exp_kc, exp_vc = oracle.kv_append(prim_k, v, kc0, vc0, cs)
    untouched = np.ones(kc0.shape, bool)
    untouched[rows] = False
    check_exact(name + " k cache elsewhere untouched", got_kc[untouched], kc0[untouched])
    check_exact(name + " v cache", got_vc, exp_vc)

    # bit-identity with the two-step drop-in path
    Q2, K2 = Guarded(hip, q, offset=offset), Guarded(hip, k, offset=offset)
    KC2, VC2 = Guarded(hip, kc0, offset=offset), Guarded(hip, vc0, offset=offset)
    q3k.qk_norm_rope(Q2, K2, QW, KW, B, S, Hq, Hkv, D, EPS, C, P, start, PZ)
    q3k.kv_append(K2, V, KC2, VC2, B, S, Hkv * D * 2, Sc, cs)
    hip.synchronize()
    check_exact(name + " q == qk_norm_rope", got_q, Q2.get(np.uint16, q.shape))
    check_exact(name + " k cache == qk_norm_rope + kv_append", got_kc, KC2.get(np.uint16, kc0.shape))


# ---------------------------------------------------------------- attention

def run_attention(q3k, hip, q, store_k, store_v, B, S, Hq, start, offset=0, split=False):
    """q [B, S, Hq * D]; the caches are whole KvCache-like layers [Bcap, Scap, Hkv, D], read through the
    [B, start + S] view (strides of the storage), as KvCache::key_view hands them over.  With split, a workspace of
    the size the library asks for lets it split the key range."""
    _, Scap, Hkv, D = store_k.shape
    Q, K, V = Guarded(hip, q, offset=offset), Guarded(hip, store_k, offset=offset), Guarded(hip, store_v, offset=offset)
    O = Guarded(hip, nbytes=q.nbytes, offset=offset)
    st = (Scap * Hkv * D, Hkv * D, D, 1)
    ws_bytes = q3k.gqa_attention_workspace_bytes(B, S, Hq, Hkv, D, start + S) if split else 0
    if split:
        assert ws_bytes > 0, "this shape should split"
    W = Guarded(hip, nbytes=ws_bytes) if ws_bytes else None
    q3k.gqa_attention(Q, K, V, O, B, S, Hq, Hkv, D, start + S, start, st, st, workspace=W, workspace_bytes=ws_bytes)
    hip.synchronize()
    assert all(b.guards_intact() for b in (Q, K, V, O) + ((W,) if W else ()))
    assert np.array_equal(Q.get(np.uint16, q.shape), q) and np.array_equal(K.get(np.uint16, store_k.shape), store_k)
    return O.get(np.uint16, q.shape)


def test_attention_kat(q3k, hip, oracle):
    """gqa_attention_cuda_test.cpp:259-357: 1 history token + 2 current into a capacity-4 cache, 4 query heads over
    2 KV heads of dim 4, checked at the test's tolerance and against the oracle band."""
    announce("gqa_attention KAT")
    q, kc, vc = kat.att_inputs()
    B, S = kat.ATT_B, kat.ATT_S
    store_k = np.zeros((B, 4, kat.ATT_HKV, kat.ATT_D), np.uint16)
    store_v = np.zeros_like(store_k)
    store_k[:, :3], store_v[:, :3] = kc, vc
    got = run_attention(q3k, hip, q, store_k, store_v, B, S, kat.ATT_HQ, kat.ATT_START)
    prim, lo, hi = oracle.gqa_attention(q, kc, vc, kat.ATT_HQ, kat.ATT_START)
    f = lambda b: (b.astype(np.uint32) << 16).view(np.float32)  # noqa: E731
    assert np.all(np.abs(f(got) - f(prim)) <= kat.ATT_TOL)
    check_band(oracle, "gqa_attention KAT", got, prim, lo, hi)


@pytest.mark.parametrize("B,S,start,Hq,Hkv,D,cap,offset", [
    (2, 40, 0, 32, 8, 128, 64, 0),      # Qwen3-8B heads, prefill (G = 4)
    (1, 77, 13, 16, 8, 128, 100, 0),    # G = 2, partial tiles, prefix in the cache
    (8, 1, 300, 32, 8, 128, 512, 0),    # decode step
    (2, 33, 5, 8, 8, 128, 40, 0),       # G = 1
    (1, 10, 0, 64, 8, 128, 10, 0),      # Qwen3-32B grouping (G = 8)
    (1, 9, 3, 32, 2, 128, 12, 0),       # G = 16
    (1, 5, 60, 32, 1, 128, 65, 0),      # G = 32
    (2, 21, 4, 8, 2, 64, 32, 0),        # head_dim 64: generic kernel
    (1, 12, 3, 8, 2, 128, 16, 2),       # unaligned caches: generic kernel
    (1, 6, 0, 4, 4, 256, 6, 0),         # head_dim 256: generic kernel
    # prefill blocks of two wave groups (S >= 256 / G), partial last blocks
    (1, 300, 20, 8, 8, 128, 330, 0),    # G = 1
    (2, 130, 0, 16, 8, 128, 140, 0),    # G = 2
    (1, 100, 9, 32, 8, 128, 120, 0),    # G = 4, the second group partly empty
    (1, 45, 7, 64, 8, 128, 60, 0),      # G = 8
    (1, 20, 3, 32, 2, 128, 30, 0),      # G = 16
    (1, 9, 60, 32, 1, 128, 70, 0),      # G = 32
    # group sizes that do not divide 32: padding columns in every wave
    (2, 77, 13, 40, 8, 128, 100, 0),    # Qwen3-14B heads (G = 5), prefill with a cached prefix
    (8, 1, 300, 40, 8, 128, 512, 0),    # G = 5 decode step
    (1, 50, 0, 24, 8, 128, 50, 0),      # G = 3
    (2, 33, 6, 12, 2, 128, 40, 0),      # G = 6
    (1, 20, 2, 20, 1, 128, 24, 0),      # G = 20: one position per wave
])
def test_gqa_attention(q3k, hip, oracle, synth, B, S, start, Hq, Hkv, D, cap, offset):
    name = f"gqa_attention B={B} S={S} start={start} Hq={Hq} Hkv={Hkv} D={D} cap={cap} offset={offset}"
    announce(name)
    q = synth.normal_bf16(160, S, (B, S, Hq * D))
    store_k = synth.normal_bf16(161, S, (B + 1, cap, Hkv, D))
    store_v = synth.normal_bf16(162, S, (B + 1, cap, Hkv, D))
    got = run_attention(q3k, hip, q, store_k, store_v, B, S, Hq, start, offset=offset)
    prim, lo, hi = oracle.gqa_attention(q, store_k[:B, :start + S], store_v[:B, :start + S], Hq, start)
    check_band(oracle, name, got, prim, lo, hi)


@pytest.mark.parametrize("B,S,start,cap,split", [(2, 200, 100, 320, False), (1, 1, 700, 704, True),
                                                   (1, 70, 400, 480, False)])
def test_gqa_attention_score_spikes(q3k, hip, oracle, synth, B, S, start, cap, split):
    """Keys parallel to a query row raise the scores of later tiles far above the earlier ones (by 2^10 and more in
    the exponent), so the softmax reference of the kernel moves mid-sequence and the output accumulators are
    rescaled; with split, inside key slices that the merge then weighs."""
    Hq, Hkv, D = 32, 8, 128
    name = f"gqa_attention spikes B={B} S={S} start={start} split={split}"
    announce(name)
    q = synth.normal_bf16(170, S, (B, S, Hq * D))
    store_k = synth.normal_bf16(171, S, (B, cap, Hkv, D))
    store_v = synth.normal_bf16(172, S, (B, cap, Hkv, D))
    qf = (q.astype(np.uint32) << 16).view(np.float32).reshape(B, S, Hq, D)
    L = start + S
    for b in range(B):
        for n, (key, scale) in enumerate(((L // 3, 1.0), (L // 2, 1.5), (L - 2, 2.0))):
            s_ref = min(S - 1, n * S // 3)
            for kvh in range(Hkv):
                h = kvh * (Hq // Hkv) + n % (Hq // Hkv)
                store_k[b, key, kvh] = synth.f32_to_bf16(scale * qf[b, s_ref, h])
    got = run_attention(q3k, hip, q, store_k, store_v, B, S, Hq, start, split=split)
    prim, lo, hi = oracle.gqa_attention(q, store_k[:, :L], store_v[:, :L], Hq, start)
    check_band(oracle, name, got, prim, lo, hi)


def test_bench_read_rows(q3k, hip):
    """The read-ceiling aid reads exactly the rows of the views it is given: its per-thread XOR fold matches the
    same fold computed on the host (KV-cache view layout [B, L, Hkv, D] of keys and values)."""
    announce("bench_read_rows")
    B, L, Hkv, D = 3, 300, 4, 128
    rng = np.random.default_rng(7)
    k = rng.integers(0, 1 << 32, (B, L, Hkv, D // 2), dtype=np.uint32)
    v = rng.integers(0, 1 << 32, (B, L, Hkv, D // 2), dtype=np.uint32)
    K, V = Guarded(hip, k), Guarded(hip, v)
    sink = Guarded(hip, nbytes=B * Hkv * 256 * 4)
    q3k.bench_read_rows(K, V, B, L * Hkv * D * 2, Hkv, D * 2, L, Hkv * D * 2, D * 2, sink)
    hip.synchronize()
    assert K.guards_intact() and V.guards_intact() and sink.guards_intact()
    got = sink.get(np.uint32, (B * Hkv, 256))
    chunks = D * 2 // 16
    kw, vw = k.reshape(B, L, Hkv, chunks, 4), v.reshape(B, L, Hkv, chunks, 4)
    want = np.zeros((B * Hkv, 256), np.uint32)
    for view in range(B * Hkv):
        b, h = divmod(view, Hkv)
        for t in range(256):
            r_in, c = divmod(t, chunks)
            rows = np.arange(r_in, L, 256 // chunks)
            x, y = kw[b, rows, h, c], vw[b, rows, h, c]
            f = ((x[:, 0] + x[:, 3]) ^ (y[:, 1] + y[:, 2])).astype(np.uint32)
            want[view, t] = np.bitwise_xor.reduce(f) if f.size else 0
    check_exact("bench_read_rows sink", got, want)


@pytest.mark.parametrize("threads", [64, 256, 1024])
@pytest.mark.parametrize("n_in,n_out,in_place", [(2, 1, False), (2, 2, True), (1, 1, True), (1, 2, False)])
def test_bench_stream(q3k, hip, n_in, n_out, in_place, threads):
    """The access-pattern ceiling aid reads its inputs and writes exactly its outputs: out0 = in0 XOR in1,
    out1 = in0 + in1 word for word (a missing in1 reads as zero), in place over in0 when asked, over a size that
    leaves a partial last block at every block size, and nothing outside the buffers."""
    announce(f"bench_stream in={n_in} out={n_out} in_place={in_place} threads={threads}")
    n = 16 * 1000 + 16 * 37          # bytes: 1037 vectors
    rng = np.random.default_rng(11)
    a = rng.integers(0, 1 << 32, n // 4, dtype=np.uint32)
    b = rng.integers(0, 1 << 32, n // 4, dtype=np.uint32) if n_in == 2 else np.zeros(n // 4, np.uint32)
    A = Guarded(hip, a)
    B = Guarded(hip, b) if n_in == 2 else None
    O0 = A if in_place else Guarded(hip, nbytes=n)
    O1 = Guarded(hip, nbytes=n) if n_out == 2 else None
    q3k.bench_stream(A, B, O0, O1, n, threads=threads)
    hip.synchronize()
    assert all(g.guards_intact() for g in (A, B, O0, O1) if g is not None)
    check_exact("bench_stream out0", O0.get(np.uint32, (n // 4,)), a ^ b)
    if O1 is not None:
        check_exact("bench_stream out1", O1.get(np.uint32, (n // 4,)), (a + b).astype(np.uint32))
    if B is not None:
        check_exact("bench_stream in1 unchanged", B.get(np.uint32, (n // 4,)), b)


@pytest.mark.parametrize("B,S,Hq,Hkv,nrows", [(4, 2048, 32, 8, 384), (1, 4096, 32, 8, 128), (1, 8192, 64, 8, 192),
                                               (2, 2048, 40, 8, 192)])
def test_gqa_attention_prefill_sampled(q3k, hip, oracle, synth, B, S, Hq, Hkv, nrows):
    """Benchmark-size prefill (config 4 shape, a 4096-token sequence, and one 8192-token sequence of the config-5
    model's 64 query heads over 8 KV heads): every row computed on the GPU, a seeded sample of rows (always
    including the last positions, the longest contexts) checked against the oracle."""
    D = 128
    name = f"gqa_attention prefill B={B} S={S} Hq={Hq} Hkv={Hkv} rows={nrows}"
    announce(name)
    q = synth.normal_bf16(163, S, (B, S, Hq * D))
    store_k = synth.normal_bf16(164, S, (B, S, Hkv, D))
    store_v = synth.normal_bf16(165, S, (B, S, Hkv, D))
    got = run_attention(q3k, hip, q, store_k, store_v, B, S, Hq, 0)
    rng = np.random.default_rng(S)
    total = B * S * Hq
    rows = np.unique(np.concatenate([rng.integers(0, total, nrows - 2 * Hq),
                                     np.arange(total - Hq, total), np.arange(S * Hq - Hq, S * Hq)]))
    prim, lo, hi = oracle.gqa_attention(q, store_k, store_v, Hq, 0, rows=rows)
    check_band(oracle, name, got.reshape(-1, D)[rows], prim, lo, hi)
    assert np.isfinite(synth.bf16_to_f32(got)).all()


# ---------------------------------------------------------------- argmax


def _split_cases(cases, plan):
    """Each case whole (no workspace), and sliced too where the library's plan slices it (its workspace query,
    a host-only function, returns a non-zero size), so that no parametrization exists only to be skipped."""
    try:
        import importlib
        lib = importlib.import_module("qwen3-runtime-byyourself_amd")
        sliced = [plan(lib, *c) > 0 for c in cases]
    except Exception:   # library not built: list every variant, the tests then fail on the missing library
        sliced = [True] * len(cases)
    out = []
    for c, sl in zip(cases, sliced):
        tag = "-".join(str(v) for v in c)
        out.append(pytest.param(*c, False, id=f"{tag}-whole"))
        if sl:
            out.append(pytest.param(*c, True, id=f"{tag}-sliced"))
    return out


ARGMAX_CASES = [(2, 513, 0, 0), (37, 1000, 0, 0), (64, 151936, 0, 0), (1, 151936, 151669, 0), (5, 1003, 0, 2),
                (3, 4096, 77, 2), (700, 64, 0, 0), (9, 40000, 0, 0), (2, 70001, 0, 2)]
ARGMAX_TIE_CASES = [(1, 151936, 3), (7, 50000, 2), (33, 20000, 5), (2, 151936, 256)]
TOPK_CASES = [(8, 151936, 0, 20), (4, 151936, 151669, 1), (2, 151936, 0, 1024), (3, 5000, 0, 64), (2, 513, 500, 3),
              (2, 600, 0, 100),      # fewer than k threads hold logits: all listed
              (2, 20000, 0, 1500),   # k above the thread count: whole-row select
              (1, 151936, 151669, 50), (6, 40000, 0, 700)]
TOPK_TIE_CASES = [(1, 151936, 50, 16), (3, 50000, 7, 4), (17, 16385, 1, 64), (2, 151936, 300, 2048),
                  (5, 40001, 700, 32)]


@pytest.mark.parametrize("rows,N,search,offset,split", _split_cases(
    ARGMAX_CASES, lambda lib, rows, N, search, offset: lib.argmax_workspace_bytes(rows, search or N)))
def test_argmax(q3k, hip, oracle, synth, rows, N, search, offset, split):
    """argmax_last_dimension (argmax.cu:34-100): bit-exact indices, including NaN rows, ties (also across slices),
    +-0, +-inf and a valid-vocabulary prefix of padded logits; with the workspace the library asks for, few rows
    are cut into slices searched by separate blocks, with the same result."""
    ws_bytes = q3k.argmax_workspace_bytes(rows, search or N) if split else 0
    assert ws_bytes > 0 or not split, "the plan no longer slices this shape"
    name = f"argmax rows={rows} N={N} search={search} offset={offset} split={split}"
    announce(name)
    if (rows, N) == (2, 513):
        x, _ = kat.argmax_inputs()
    else:
        x = synth.normal_bf16(171, N, (rows, N), std=4.0)
        if rows > 6:
            x[1, :] = 0xff80
            x[2, N // 3] = 0x7fc0
            x[3, :] = 0x8000
            x[3, N - 1] = 0
            x[4, 5] = x[4, N - 2] = 0x7f80
            x[5, :] = 0x7fc0
            x[6, 9] = x[6, 3] = synth.f32_to_bf16(np.array([50.0], np.float32))[0]
        if rows > 7:
            x[7, N // 2] = x[7, N - 1] = synth.f32_to_bf16(np.array([60.0], np.float32))[0]
    X = Guarded(hip, x, offset=offset)
    O = Guarded(hip, nbytes=rows * 4)
    W = Guarded(hip, nbytes=ws_bytes) if ws_bytes else None
    q3k.argmax(X, O, rows, N, search or N, workspace=W, workspace_bytes=ws_bytes)
    hip.synchronize()
    assert X.guards_intact() and O.guards_intact() and (W is None or W.guards_intact())
    check_exact(name, O.get(np.int32, (rows,)).view(np.uint32), oracle.argmax(x, search).view(np.uint32))


@pytest.mark.parametrize("rows,N,levels,split", _split_cases(
    ARGMAX_TIE_CASES, lambda lib, rows, N, levels: lib.argmax_workspace_bytes(rows, N)))
def test_argmax_ties(q3k, hip, oracle, synth, rows, N, levels, split):
    """Logits quantised to a few values, so the maximum is tied in many slices: the first index still wins."""
    ws_bytes = q3k.argmax_workspace_bytes(rows, N) if split else 0
    assert ws_bytes > 0 or not split, "the plan no longer slices this shape"
    name = f"argmax ties rows={rows} N={N} levels={levels} split={split}"
    announce(name)
    rng = np.random.default_rng(rows * 100 + levels)
    vals = synth.f32_to_bf16(np.linspace(-3.0, 3.0, levels).astype(np.float32))
    x = vals[rng.integers(0, levels, size=(rows, N))].astype(np.uint16)
    x[0, : N // 2] = vals[0]   # row 0: the maximum appears only in the second half
    X = Guarded(hip, x)
    O = Guarded(hip, nbytes=rows * 4)
    W = Guarded(hip, nbytes=ws_bytes) if ws_bytes else None
    q3k.argmax(X, O, rows, N, N, workspace=W, workspace_bytes=ws_bytes)
    hip.synchronize()
    assert X.guards_intact() and O.guards_intact() and (W is None or W.guards_intact())
    check_exact(name, O.get(np.int32, (rows,)).view(np.uint32), oracle.argmax(x).view(np.uint32))


# ---------------------------------------------------------------- sampling: top-k candidates

@pytest.mark.parametrize("rows,N,valid,k,split", _split_cases(
    TOPK_CASES, lambda lib, rows, N, valid, k: lib.topk_workspace_bytes(rows, valid or N, k)))
def test_topk_candidates(q3k, hip, oracle, synth, rows, N, valid, k, split):
    """GPU top-k selection (the reference sampler's top-k rule, sampler.cpp:160-190): the candidate set equals the
    oracle's exactly, ties at the k-th included; non-finite rows flagged.  With the workspace the library asks for,
    few rows are cut into slices (tied and non-finite rows then take the whole-row select), same set."""
    n = valid or N
    ws_bytes = q3k.topk_workspace_bytes(rows, n, k) if split else 0
    assert ws_bytes > 0 or not split, "the plan no longer slices this shape"
    name = f"topk_candidates rows={rows} N={N} valid={valid} k={k} split={split}"
    announce(name)
    cap = 1024
    x = synth.normal_bf16(174, N, (rows, N), std=3.0)
    x[0, 5] = x[0, 9] = x[0, 200] = x[0, 3]                     # ties
    x[0, 3] = synth.f32_to_bf16(np.array([40.0], np.float32))[0]
    if rows > 2:
        x[2, :] = synth.f32_to_bf16(np.array([1.5], np.float32))[0]   # all tied: count = n (> cap for large n)
        x[2, 0] = 0x8000
        x[2, 1] = 0x0000
    if rows > 3:
        x[3, n - 1] = 0x7f80                                     # non-finite inside the valid prefix
        x[3, N - 1] = 0x7fc0 if n < N else x[3, N - 1]
    if rows > 4:
        x[4, :] = synth.f32_to_bf16(np.array([-2.0], np.float32))[0]
        x[4, n - 3 * k:n] = synth.normal_bf16(175, N, (3 * k,), std=1.0)   # the top k all in the last slice
    if rows > 5:
        x[5, ::997] = synth.f32_to_bf16(np.array([9.0], np.float32))[0]   # ties at the k-th spread over slices
    X = Guarded(hip, x)
    C, F = Guarded(hip, nbytes=rows * 4), Guarded(hip, nbytes=rows * 4)
    I, V = Guarded(hip, nbytes=rows * cap * 4), Guarded(hip, nbytes=rows * cap * 2)
    W = Guarded(hip, nbytes=ws_bytes) if ws_bytes else None
    q3k.topk_candidates(X, rows, N, n, k, cap, C, I, V, F, workspace=W, workspace_bytes=ws_bytes)
    hip.synchronize()
    assert all(b.guards_intact() for b in (X, C, F, I, V) + ((W,) if W is not None else ()))
    counts, flags = C.get(np.int32, (rows,)), F.get(np.int32, (rows,))
    ids, vals = I.get(np.int32, (rows, cap)), V.get(np.uint16, (rows, cap))
    for r in range(rows):
        want = oracle.topk_set(x[r, :n], k)
        if want is None:
            assert flags[r] != 0, f"row {r}: non-finite not flagged"
            continue
        assert flags[r] == 0
        assert counts[r] == want.size, (r, counts[r], want.size)
        if want.size <= cap:
            got = ids[r, :want.size]
            check_exact(f"{name} row {r} ids", np.sort(got), np.sort(want))
            check_exact(f"{name} row {r} logits", vals[r, :want.size], x[r, got])


@pytest.mark.parametrize("rows,N,k,levels,split", _split_cases(
    TOPK_TIE_CASES, lambda lib, rows, N, k, levels: lib.topk_workspace_bytes(rows, N, k)))
def test_topk_candidates_ties(q3k, hip, oracle, synth, rows, N, k, levels, split):
    """Logits quantised to a few distinct values, so the k-th largest is tied many times over and the ties fall in
    every slice: the candidate count and set equal the oracle's (a count above the capacity is reported as is)."""
    n = N
    ws_bytes = q3k.topk_workspace_bytes(rows, n, k) if split else 0
    assert ws_bytes > 0 or not split, "the plan no longer slices this shape"
    name = f"topk ties rows={rows} N={N} k={k} levels={levels} split={split}"
    announce(name)
    cap = 1024
    rng = np.random.default_rng(rows * 1000 + k)
    vals = synth.f32_to_bf16(np.linspace(-4.0, 4.0, levels).astype(np.float32))
    x = vals[rng.integers(0, levels, size=(rows, N))].astype(np.uint16)
    X = Guarded(hip, x)
    C, F = Guarded(hip, nbytes=rows * 4), Guarded(hip, nbytes=rows * 4)
    I, V = Guarded(hip, nbytes=rows * cap * 4), Guarded(hip, nbytes=rows * cap * 2)
    W = Guarded(hip, nbytes=ws_bytes) if ws_bytes else None
    q3k.topk_candidates(X, rows, N, n, k, cap, C, I, V, F, workspace=W, workspace_bytes=ws_bytes)
    hip.synchronize()
    assert all(b.guards_intact() for b in (X, C, F, I, V) + ((W,) if W is not None else ()))
    counts, flags = C.get(np.int32, (rows,)), F.get(np.int32, (rows,))
    ids, cv = I.get(np.int32, (rows, cap)), V.get(np.uint16, (rows, cap))
    for r in range(rows):
        want = oracle.topk_set(x[r], k)
        assert flags[r] == 0 and counts[r] == want.size, (r, counts[r], want.size)
        if want.size <= cap:
            got = ids[r, :want.size]
            check_exact(f"{name} row {r} ids", np.sort(got), np.sort(want))
            check_exact(f"{name} row {r} logits", cv[r, :want.size], x[r, got])


@pytest.mark.parametrize("B,S,start,Hq,Hkv,cap", [(1, 1, 4095, 32, 8, 4096), (2, 5, 700, 32, 8, 800),
                                                 (1, 1, 300, 64, 8, 320), (1, 3, 400, 16, 8, 420),
                                                 (4, 1, 1000, 32, 8, 1100), (1, 1, 1000, 8, 8, 1100),
                                                 (1, 1, 500, 16, 8, 512), (2, 1, 900, 32, 2, 1000),
                                                 (1, 1, 2000, 32, 1, 2100), (3, 1, 129, 32, 8, 200),
                                                 (1, 1, 4095, 40, 8, 4096), (2, 3, 600, 40, 8, 700)])
def test_gqa_attention_split_keys(q3k, hip, oracle, synth, B, S, start, Hq, Hkv, cap):
    """Decode with few sequences: the key range is split across blocks (the workspace the library asks for) and the
    slices merged; same band as the single-pass kernel.  Decode steps whose slices hold one or two tiles run as
    one-wave blocks: covered for every group size G = Hq / Hkv from 1 to 32, and a cache of 130 keys (two slices,
    the second a partial tile)."""
    D = 128
    name = f"gqa_attention split B={B} S={S} start={start} Hq={Hq} Hkv={Hkv}"
    announce(name)
    q = synth.normal_bf16(166, S, (B, S, Hq * D))
    store_k = synth.normal_bf16(167, S, (B, cap, Hkv, D))
    store_v = synth.normal_bf16(168, S, (B, cap, Hkv, D))
    got = run_attention(q3k, hip, q, store_k, store_v, B, S, Hq, start, split=True)
    prim, lo, hi = oracle.gqa_attention(q, store_k[:, :start + S], store_v[:, :start + S], Hq, start)
    check_band(oracle, name, got, prim, lo, hi)
    whole = run_attention(q3k, hip, q, store_k, store_v, B, S, Hq, start)
    check_band(oracle, name + " (not split)", whole, prim, lo, hi)


def test_prefill_then_decode_matches_one_shot(q3k, hip, oracle, synth):
    """The reference's end-to-end check of one-shot prefill against prefill + decode
    (tests/integration/model_real_smoke.cu:101-170), on this library's layer pieces: Q/K norm + RoPE + KV append
    (self_attention.cpp:147-156) and attention over the cache view.  A prefill of P tokens followed by decode steps
    of one token each (key-split attention with the workspace the library asks for) leaves the KV cache and the
    roped queries bit for bit as one prefill of all the tokens does; the prefix rows of attention are bit-identical
    too (a row's result does not depend on how many positions follow it), and each decode output lies in the
    oracle's band, as the one-shot rows for the same positions do."""
    B, P, steps, Hq, Hkv, D = 2, 700, 4, 32, 8, 128
    T, cap, table_rows = P + steps, P + steps + 20, P + steps + 20
    name = f"prefill {P} + {steps} decode steps vs one-shot prefill B={B} Hq={Hq} Hkv={Hkv}"
    announce(name)
    q = synth.normal_bf16(171, T, (B, T, Hq * D))
    k = synth.normal_bf16(172, T, (B, T, Hkv * D))
    v = synth.normal_bf16(173, T, (B, T, Hkv * D))
    qw = synth.normal_bf16(174, D, (D,), mean=1.0, std=0.1)
    kw = synth.normal_bf16(175, D, (D,), mean=1.0, std=0.1)
    table = oracle.build_rope_cache(table_rows, D, 1.0e6)
    QW, KW, C = Guarded(hip, qw), Guarded(hip, kw), Guarded(hip, table)
    st = (cap * Hkv * D, Hkv * D, D, 1)
    empty = np.zeros((B, cap, Hkv * D), np.uint16)

    def append(Qb, q_part, k_part, v_part, KC, VC, at):
        Kb, Vb = Guarded(hip, k_part), Guarded(hip, v_part)
        q3k.qk_norm_rope_kv_append(Qb, Kb, Vb, QW, KW, B, q_part.shape[1], Hq, Hkv, D, EPS, C, table_rows, at, KC,
                                   VC, cap, at, None)

    def attend(Qb, KC, VC, S, start, split):
        O = Guarded(hip, nbytes=B * S * Hq * D * 2)
        ws = q3k.gqa_attention_workspace_bytes(B, S, Hq, Hkv, D, start + S) if split else 0
        assert not split or ws > 0, "a decode step over this cache should split the key range"
        W = Guarded(hip, nbytes=ws) if ws else None
        q3k.gqa_attention(Qb, KC, VC, O, B, S, Hq, Hkv, D, start + S, start, st, st, workspace=W, workspace_bytes=ws)
        hip.synchronize()
        assert O.guards_intact() and (W is None or W.guards_intact())
        return O.get(np.uint16, (B, S, Hq * D))

    # one prefill of all T tokens
    Q1, KC1, VC1 = Guarded(hip, q), Guarded(hip, empty), Guarded(hip, empty)
    append(Q1, q, k, v, KC1, VC1, 0)
    one_shot = attend(Q1, KC1, VC1, T, 0, False)
    q1 = Q1.get(np.uint16, q.shape)

    # prefill of P tokens, then one token per step
    KC2, VC2 = Guarded(hip, empty), Guarded(hip, empty)
    Qp = Guarded(hip, np.ascontiguousarray(q[:, :P]))
    append(Qp, q[:, :P], np.ascontiguousarray(k[:, :P]), np.ascontiguousarray(v[:, :P]), KC2, VC2, 0)
    prefix = attend(Qp, KC2, VC2, P, 0, False)
    check_exact(name + " prefix queries", Qp.get(np.uint16, (B, P, Hq * D)), q1[:, :P])
    decoded = []
    for s in range(P, T):
        Qd = Guarded(hip, np.ascontiguousarray(q[:, s:s + 1]))
        append(Qd, q[:, s:s + 1], np.ascontiguousarray(k[:, s:s + 1]), np.ascontiguousarray(v[:, s:s + 1]), KC2,
               VC2, s)
        decoded.append(attend(Qd, KC2, VC2, 1, s, True))
        check_exact(f"{name} step {s} query", Qd.get(np.uint16, (B, 1, Hq * D)), q1[:, s:s + 1])
    assert all(g.guards_intact() for g in (Q1, KC1, VC1, KC2, VC2, QW, KW, C))
    check_exact(name + " K cache", KC2.get(np.uint16, empty.shape), KC1.get(np.uint16, empty.shape))
    check_exact(name + " V cache", VC2.get(np.uint16, empty.shape), VC1.get(np.uint16, empty.shape))
    check_exact(name + " prefix attention rows", prefix, one_shot[:, :P])

    # the decode rows and the one-shot rows of the same positions, against the oracle on the roped inputs
    kc = KC1.get(np.uint16, empty.shape)[:, :T].reshape(B, T, Hkv, D)
    vc = VC1.get(np.uint16, empty.shape)[:, :T].reshape(B, T, Hkv, D)
    rows = np.array([(b * T + s) * Hq + h for b in range(B) for s in range(P, T) for h in range(Hq)])
    prim, lo, hi = oracle.gqa_attention(q1, kc, vc, Hq, 0, rows=rows)
    step_rows = np.stack(decoded, axis=1).reshape(-1, D)   # [B, steps, Hq * D] in (b, s, h) order
    check_band(oracle, name + " decode rows", step_rows, prim, lo, hi)
    check_band(oracle, name + " one-shot rows", one_shot.reshape(-1, D)[rows], prim, lo, hi)
