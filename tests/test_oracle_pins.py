"""Pins of the CPU oracle (CPU only).

The oracle restates the reference's arithmetic; these tests check it against
what does not depend on the oracle itself:
  * the reference tests' known-answer inputs and tolerances (kat.py);
  * closed forms evaluated in float64 / complex128;
  * an independent implementation: PyTorch CPU in the Hugging Face Qwen3
    order (RMSNorm rounds to bf16 before the weight, silu in fp32 then bf16,
    rotate_half RoPE);
  * invariants (identity at position 0, scale invariance, norm preservation).
Where an exact fp32 result of the reference cannot be known (CUDA rsqrtf /
expf / contraction), a disagreement is only allowed on elements the oracle
marks ambiguous (lo != hi); everywhere else the primary result must match
bit for bit.  That is what makes a dropped rounding step or a wrong pair
index fail here.
"""
import numpy as np
import pytest
import torch

import kat


def t_bf16(a):
    return torch.from_numpy(np.ascontiguousarray(a).astype(np.int16)).view(torch.bfloat16)


def np_bits(t):
    return t.contiguous().view(torch.int16).numpy().astype(np.uint16)


def f32(b):
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def assert_matches_where_unambiguous(primary, lo, hi, other, name, min_exact=0.995):
    primary, lo, hi, other = (np.asarray(a).ravel() for a in (primary, lo, hi, other))
    diff = primary != other
    ambiguous = lo != hi
    # Disagreements are allowed only inside the band of ambiguous elements.
    bad = diff & ~ambiguous
    assert not bad.any(), f"{name}: {bad.sum()} unambiguous mismatches, first at {np.argmax(bad)}"

    def ordv(b):
        b = b.astype(np.int32)
        return np.where(b & 0x8000, -(b & 0x7FFF), b)

    inside = (ordv(other) >= ordv(lo)) & (ordv(other) <= ordv(hi))
    assert inside.all(), f"{name}: independent result outside the band at {np.argmin(inside)}"
    assert (1.0 - diff.mean()) >= min_exact, f"{name}: only {1 - diff.mean():.5f} exact"


# ---------------------------------------------------------------- bf16 --------

def test_bf16_rounding_matches_torch(oracle, synth):
    rng = np.random.default_rng(0)
    bits = rng.integers(0, 2**32, size=200_000, dtype=np.uint64).astype(np.uint32)
    specials = np.array([0x3F808000, 0x3F818000, 0x3F80FFFF, 0x7F7FFFFF, 0x00000001, 0x80000000, 0x00008000,
                         0x7F800000, 0xFF800000, 0x3F7FFFFF], dtype=np.uint32)
    bits = np.concatenate([bits, specials])
    x = bits.view(np.float32)
    finite = np.isfinite(x) | np.isinf(x)
    ours = np.array([oracle.bf16(float(v)) for v in x[:2000]], dtype=np.uint16)
    ref = np_bits(torch.from_numpy(x[:2000]).to(torch.bfloat16))
    keep = finite[:2000]
    assert np.array_equal(ours[keep], ref[keep])
    # the numpy generator uses the same rule on the whole sample
    npr = synth.f32_to_bf16(x)
    tr = np_bits(torch.from_numpy(x).to(torch.bfloat16))
    assert np.array_equal(npr[finite], tr[finite])
    # ties to even, overflow to inf
    assert oracle.bf16(float(np.uint32(0x3F808000).view(np.float32))) == 0x3F80
    assert oracle.bf16(float(np.uint32(0x3F818000).view(np.float32))) == 0x3F82
    assert oracle.bf16(float(np.uint32(0x7F7FFFFF).view(np.float32))) == 0x7F80


def test_ulp_distance_and_compare(oracle):
    assert oracle.ulp_distance(0x3F80, 0x3F81) == 1
    assert oracle.ulp_distance(0x0000, 0x8000) == 0
    assert oracle.ulp_distance(0x0001, 0x8001) == 2
    assert oracle.ulp_distance(0x7FC0, 0x7FC1) == 0
    assert oracle.ulp_distance(0x7FC0, 0x3F80) > 1000
    prim = np.array([0x3F80, 0x3F80, 0x3F80, 0x3F80, 0x7FC0], np.uint16)
    lo = np.array([0x3F80, 0x3F80, 0x3F7F, 0x3F80, 0x7FC0], np.uint16)
    hi = np.array([0x3F80, 0x3F80, 0x3F81, 0x3F80, 0x7FC0], np.uint16)
    got = np.array([0x3F81, 0x3F82, 0x3F7E, 0x3F80, 0x7FC0], np.uint16)
    st = oracle.compare(got, prim, lo, hi)
    assert st["fail"] == 1 and st["first_fail"] == 1
    assert st["ambiguous"] == 1
    assert st["ulp_hist"] == [2, 1, 2, 0]


# ---------------------------------------------------------------- embedding ---

def test_embedding_kat(oracle):
    table, ids = kat.embedding_inputs()
    out = oracle.embedding(ids, table)
    assert out.shape == (2, 3, 4)
    expected = (ids[..., None] * 10 + np.arange(4)).astype(np.float32)
    assert np.all(np.abs(f32(out) - expected) < 0.001)  # embedding_cuda_test.cpp:204-208


def test_embedding_random_and_out_of_range(oracle, synth):
    table = synth.normal_bf16(11, 0, (97, 24))
    ids = np.array([0, 96, 5, -1, 97, 2**31 - 1, -(2**31), 40], dtype=np.int32)
    out = oracle.embedding(ids, table)
    for t, i in enumerate(ids):
        if 0 <= i < 97:
            assert np.array_equal(out[t], table[i])
        else:
            assert np.all(out[t] == 0)  # embedding.cu:38-45: +0.0 rows


# ---------------------------------------------------------------- add --------

def test_add_matches_fp32_add(oracle, synth):
    a = synth.normal_bf16(12, 0, (4, 3, 257))
    b = synth.normal_bf16(12, 1, (4, 3, 257), std=0.5)
    ours = oracle.add_inplace(a, b)
    ref = np_bits((t_bf16(a).float() + t_bf16(b).float()).to(torch.bfloat16))
    assert np.array_equal(ours, ref)


def test_add_kat(oracle):
    r, d, _, _ = kat.elementwise_inputs()
    out = oracle.add_inplace(r, d)
    expected = f32(r) + f32(d)  # every KAT sum is exact in bf16
    assert np.all(np.abs(f32(out) - expected) < 0.001)  # elementwise_cuda_test.cpp:231-234


# ---------------------------------------------------------------- rms_norm ---

def hf_rms_norm(x_bits, w_bits, eps):
    """transformers Qwen3RMSNorm.forward, on the CPU."""
    hs = t_bf16(x_bits).float()
    var = hs.pow(2).mean(-1, keepdim=True)
    hs = hs * torch.rsqrt(var + eps)
    return np_bits(t_bf16(w_bits) * hs.to(torch.bfloat16))


@pytest.mark.parametrize("shape", [(2, 3, 1024), (2, 3, 4, 128)])
def test_rms_norm_kat(oracle, shape):
    x = kat.rms_input(shape)
    w = kat.rms_weight(shape[-1])
    y, lo, hi = oracle.rms_norm(x, w, 1e-6)
    xf = f32(x).astype(np.float64).reshape(-1, shape[-1])
    inv = 1.0 / np.sqrt((xf**2).mean(axis=1, keepdims=True) + 1e-6)
    expected = (xf * inv * f32(w)).reshape(shape)
    tol = 0.02 + 0.01 * np.abs(expected)  # rms_norm_cuda_test.cpp:232-235
    assert np.all(np.abs(f32(y) - expected) <= tol)
    assert np.all(f32(lo) <= f32(y)) and np.all(f32(y) <= f32(hi))


@pytest.mark.parametrize("rows,n", [(64, 1024), (32, 4096), (16, 5120), (512, 128), (8, 257)])
def test_rms_norm_matches_hf_torch(oracle, synth, rows, n):
    x = synth.normal_bf16(13, n, (rows, n))
    w = synth.normal_bf16(13, n + 1, (n,), mean=1.0, std=0.1)
    y, lo, hi = oracle.rms_norm(x, w, 1e-6)
    ref = hf_rms_norm(x, w, 1e-6)
    assert_matches_where_unambiguous(y, lo, hi, ref, f"rms_norm[{rows},{n}]")


def test_rms_norm_dropped_rounding_is_detected(oracle, synth):
    """A restatement that skipped RNE(x * inv) must fail the rule used above."""
    x = synth.normal_bf16(14, 0, (64, 1024))
    w = synth.normal_bf16(14, 1, (1024,), mean=1.0, std=0.1)
    y, lo, hi = oracle.rms_norm(x, w, 1e-6)
    hs = t_bf16(x).float()
    hs = hs * torch.rsqrt(hs.pow(2).mean(-1, keepdim=True) + 1e-6)
    wrong = np_bits((t_bf16(w).float() * hs).to(torch.bfloat16))  # one rounding only
    with pytest.raises(AssertionError):
        assert_matches_where_unambiguous(y, lo, hi, wrong, "planted")


@pytest.mark.parametrize("rows,n", [(16, 1024), (32, 4096), (8, 257)])
def test_rms_norm_test_order(oracle, synth, rows, n):
    """The reference test's CPU loop (column-order fp32 sum): within the KAT
    tolerance of the float64 form, equal to HF torch order where that is
    unambiguous, and inside the kernel-order oracle's band (only the sum order
    differs); identical for every thread count."""
    x = synth.normal_bf16(31, n, (rows, n))
    w = synth.normal_bf16(31, n + 1, (n,), mean=1.0, std=0.1)
    y = oracle.rms_norm_test_order(x, w, 1e-6)
    xf = f32(x).astype(np.float64)
    expected = xf / np.sqrt((xf**2).mean(axis=1, keepdims=True) + 1e-6) * f32(w)
    assert np.all(np.abs(f32(y) - expected) <= 0.02 + 0.01 * np.abs(expected))  # rms_norm_cuda_test.cpp:232-235
    k, lo, hi = oracle.rms_norm(x, w, 1e-6)
    assert_matches_where_unambiguous(k, lo, hi, y, f"test-order rms_norm[{rows},{n}]")
    assert_matches_where_unambiguous(k, lo, hi, hf_rms_norm(x, w, 1e-6), f"hf rms_norm[{rows},{n}]")
    for nt in (1, 3, 8):
        assert np.array_equal(oracle.rms_norm_test_order(x, w, 1e-6, nthreads=nt), y)


def test_rms_norm_test_order_closed_form_and_planted(oracle, synth):
    n = 1024
    x = np.full((2, n), 0x3F00, np.uint16)  # 0.5: sum 256 exactly, inv = 1/sqrt(0.25 + 1e-6)
    w = np.full((n,), 0x3F80, np.uint16)
    assert np.all(oracle.rms_norm_test_order(x, w, 1e-6) == 0x3F80)
    # a loop without the RNE(x * inv) rounding would not agree with it everywhere
    x = synth.normal_bf16(32, 0, (64, n))
    w = synth.normal_bf16(32, 1, (n,), mean=1.0, std=0.1)
    y = oracle.rms_norm_test_order(x, w, 1e-6)
    xf = f32(x)
    inv = (np.float32(1.0) / np.sqrt(np.cumsum(xf * xf, axis=1, dtype=np.float32)[:, -1:] / np.float32(n)
                                     + np.float32(1e-6))).astype(np.float32)
    one_rounding = np_bits(torch.from_numpy((xf * inv * f32(w)).astype(np.float32)).to(torch.bfloat16))
    assert not np.array_equal(one_rounding, y)


def test_rms_norm_constant_row_closed_form(oracle):
    n = 1024
    x = np.full((3, n), 0x3F00, np.uint16)  # 0.5
    w = np.full((n,), 0x3F80, np.uint16)    # 1.0
    y, _, _ = oracle.rms_norm(x, w, 1e-6)
    # inv = 1/sqrt(0.25 + 1e-6) = 1.999996; 0.5 * inv rounds to 1.0 in bf16
    assert np.all(y == 0x3F80)


def test_rms_norm_scale_invariance(oracle, synth):
    x = synth.normal_bf16(15, 0, (8, 4096))
    w = synth.normal_bf16(15, 1, (4096,), mean=1.0, std=0.1)
    x2 = (x.astype(np.uint32) + (1 << 7)).astype(np.uint16)  # exponent + 1: exactly 2x (normal values)
    assert np.allclose(f32(x2)[np.abs(f32(x)) > 1e-30], 2 * f32(x)[np.abs(f32(x)) > 1e-30])
    y1, _, _ = oracle.rms_norm(x, w, 1e-30)
    y2, _, _ = oracle.rms_norm(x2, w, 1e-30)
    assert np.array_equal(y1, y2)


def test_rms_norm_packed_heads_equal_rows(oracle, synth):
    q = synth.normal_bf16(16, 0, (5, 7, 4 * 128))
    w = synth.normal_bf16(16, 1, (128,), mean=1.0, std=0.1)
    a, _, _ = oracle.rms_norm(q, w, 1e-6)
    b, _, _ = oracle.rms_norm(q.reshape(-1, 128), w, 1e-6)
    assert np.array_equal(a.reshape(-1), b.reshape(-1))


def test_add_rms_norm_is_composition(oracle, synth):
    h = synth.normal_bf16(17, 0, (33, 1024))
    d = synth.normal_bf16(17, 1, (33, 1024))
    w = synth.normal_bf16(17, 2, (1024,), mean=1.0, std=0.1)
    h2, y, lo, hi = oracle.add_rms_norm(h, d, w, 1e-6)
    assert np.array_equal(h2, oracle.add_inplace(h, d))
    y_ref, lo_ref, hi_ref = oracle.rms_norm(h2, w, 1e-6)
    assert np.array_equal(y, y_ref) and np.array_equal(lo, lo_ref) and np.array_equal(hi, hi_ref)
    # decoder_layer.cpp:78->88 in torch: add in bf16, then the HF norm of the rounded sum
    hs = np_bits((t_bf16(h).float() + t_bf16(d).float()).to(torch.bfloat16))
    assert_matches_where_unambiguous(y, lo, hi, hf_rms_norm(hs, w, 1e-6), "add_rms_norm")


# ---------------------------------------------------------------- silu -------

def test_silu_mul_matches_hf_torch(oracle, synth):
    g = synth.normal_bf16(18, 0, (512, 3072))
    u = synth.normal_bf16(18, 1, (512, 3072))
    out, lo, hi = oracle.silu_mul(g, u)
    act = torch.nn.functional.silu(t_bf16(g).float()).to(torch.bfloat16)  # silu(gate) in bf16
    ref = np_bits(act * t_bf16(u))
    assert_matches_where_unambiguous(out, lo, hi, ref, "silu_mul")


def test_silu_mul_closed_form(oracle, synth):
    g = synth.normal_bf16(19, 0, (100_000,), std=4.0)
    u = synth.normal_bf16(19, 1, (100_000,))
    out, lo, hi = oracle.silu_mul(g, u)
    gd = f32(g).astype(np.float64)
    s = gd / (1.0 + np.exp(-gd))
    n = synth.f32_to_bf16(s.astype(np.float32))
    exact = synth.f32_to_bf16(f32(n) * f32(u))
    assert_matches_where_unambiguous(out, lo, hi, exact, "silu closed form")


def test_silu_mul_kat_and_extremes(oracle):
    _, _, g, u = kat.elementwise_inputs()
    out, _, _ = oracle.silu_mul(g, u)
    gf, uf = f32(g).astype(np.float64), f32(u).astype(np.float64)
    expected = gf / (1 + np.exp(-gf)) * uf
    assert np.all(np.abs(f32(out) - expected) <= 0.02 + 0.01 * np.abs(expected))  # :294-303
    # exp(-g) overflows fp32 for g < -88.7: silu is a signed zero, as expf gives inf
    g2 = kat.bf(np.array([-100.0, -89.0, 100.0, 0.0], np.float32))
    u2 = kat.bf(np.array([1.0, 1.0, 1.0, 1.0], np.float32))
    o2, _, _ = oracle.silu_mul(g2, u2)
    assert list(f32(o2)) == [0.0, 0.0, 100.0, 0.0]


# ---------------------------------------------------------------- rope -------

def test_rope_cache_closed_form(oracle):
    P, D, theta = 64, 128, 1.0e6
    cache = oracle.build_rope_cache(P, D, theta)
    p = np.arange(P)[:, None].astype(np.float64)
    i = np.arange(D // 2)[None, :].astype(np.float64)
    ang = p * theta ** (-(2.0 * i) / D)
    assert np.array_equal(cache[..., 0], np.cos(ang).astype(np.float32))
    assert np.array_equal(cache[..., 1], np.sin(ang).astype(np.float32))
    assert np.all(cache[0, :, 0] == 1.0) and np.all(cache[0, :, 1] == 0.0)


def hf_rope(x_bits, heads, D, cache, pos):
    """transformers apply_rotary_pos_emb with rotate_half, fp32 table, on the CPU."""
    x = t_bf16(x_bits).float().reshape(len(pos), heads, D)
    cs = torch.from_numpy(cache[pos])  # [T, D/2, 2]
    cos = torch.cat([cs[..., 0], cs[..., 0]], -1)[:, None, :]
    sin = torch.cat([cs[..., 1], cs[..., 1]], -1)[:, None, :]
    rot = torch.cat([-x[..., D // 2:], x[..., : D // 2]], -1)
    return np_bits((x * cos + rot * sin).to(torch.bfloat16)).reshape(x_bits.shape)


def test_rope_kat(oracle):
    B, S, Hq, Hkv, D, P, start, theta = (kat.ROPE_B, kat.ROPE_S, kat.ROPE_HQ, kat.ROPE_HKV, kat.ROPE_D, kat.ROPE_P,
                                         kat.ROPE_START, kat.ROPE_THETA)
    cache = oracle.build_rope_cache(P, D, theta)
    for heads, off in ((Hq, 0), (Hkv, 5)):
        v = kat.rope_values(B * S * heads * D, off).reshape(B, S, heads * D)
        out, _, _ = oracle.rope(v, B, S, heads, D, cache, start)
        x = f32(v).astype(np.float64).reshape(B, S, heads, D)
        z = x[..., : D // 2] + 1j * x[..., D // 2:]
        pos = start + np.arange(S)
        ang = pos[:, None] * theta ** (-(2.0 * np.arange(D // 2)) / D)
        r = z * np.exp(1j * ang)[None, :, None, :]
        expected = np.concatenate([r.real, r.imag], -1).reshape(B, S, heads * D)
        assert np.all(np.abs(f32(out) - expected) <= 0.03)  # rope_cuda_test.cpp:325-335
    with pytest.raises(ValueError):
        oracle.rope(v, B, S, Hkv, D, cache, P - 1)  # rope_cuda_test.cpp:337-358


@pytest.mark.parametrize("heads,S,start", [(16, 64, 0), (8, 33, 100), (32, 8, 4000)])
def test_rope_matches_rotate_half(oracle, synth, heads, S, start):
    D, P = 128, 4096 + 64
    cache = oracle.build_rope_cache(P, D, 1.0e6)
    x = synth.normal_bf16(20, heads, (2, S, heads * D))
    out, lo, hi = oracle.rope(x, 2, S, heads, D, cache, start)
    pos = np.tile(start + np.arange(S), 2)
    ref = hf_rope(x.reshape(2 * S, heads * D), heads, D, cache, pos).reshape(x.shape)
    assert_matches_where_unambiguous(out, lo, hi, ref, "rope")


def test_rope_complex_closed_form_and_identity(oracle, synth):
    D, heads, S = 128, 4, 40
    cache = oracle.build_rope_cache(64, D, 1.0e6)
    x = synth.normal_bf16(21, 0, (1, S, heads * D))
    out, lo, hi = oracle.rope(x, 1, S, heads, D, cache, 0)
    # position 0 is the identity: cos = 1, sin = 0 exactly
    assert np.array_equal(out[0, 0], x[0, 0])
    xf = f32(x).astype(np.float64).reshape(S, heads, D)
    c = cache[:S, :, 0].astype(np.float64)[:, None, :]
    s = cache[:S, :, 1].astype(np.float64)[:, None, :]
    z = (xf[..., : D // 2] + 1j * xf[..., D // 2:]) * (c + 1j * s)
    exact = np.concatenate([z.real, z.imag], -1).astype(np.float32).reshape(x.shape)
    assert_matches_where_unambiguous(out, lo, hi, synth.f32_to_bf16(exact), "rope complex")
    # rotation preserves each pair's norm up to bf16 rounding
    a = f32(out).astype(np.float64).reshape(S, heads, D)
    n0 = xf[..., : D // 2] ** 2 + xf[..., D // 2:] ** 2
    n1 = a[..., : D // 2] ** 2 + a[..., D // 2:] ** 2
    assert np.allclose(n1, n0, rtol=2e-2, atol=1e-6)


def test_rope_positions_and_out_of_range(oracle, synth):
    D, heads = 128, 8
    cache = oracle.build_rope_cache(100, D, 1.0e6)
    x = synth.normal_bf16(22, 0, (3, 1, heads * D))
    pos = np.array([7, 99, 100], np.int32)
    out, _, _ = oracle.rope(x, 3, 1, heads, D, cache, positions=pos)
    for b in range(2):
        one, _, _ = oracle.rope(x[b:b + 1], 1, 1, heads, D, cache, start=int(pos[b]))
        assert np.array_equal(out[b], one[0])
    assert np.all(out[2] == 0x7FC0)  # position outside the table: NaN row


def test_qk_norm_rope_is_composition(oracle, synth):
    D, heads, B, S = 128, 8, 2, 24
    cache = oracle.build_rope_cache(64, D, 1.0e6)
    x = synth.normal_bf16(23, 0, (B, S, heads * D))
    w = synth.normal_bf16(23, 1, (D,), mean=1.0, std=0.1)
    fused, lo, hi = oracle.qk_norm_rope(x, w, B, S, heads, D, 1e-6, cache, start=3)
    normed, _, _ = oracle.rms_norm(x, w, 1e-6)
    roped, _, _ = oracle.rope(normed, B, S, heads, D, cache, start=3)
    assert np.array_equal(fused, roped)
    # self_attention.cpp:147-152 in torch: HF q_norm, then rotate_half RoPE
    normed_t = hf_rms_norm(x.reshape(-1, D), w, 1e-6).reshape(B * S, heads * D)
    pos = np.tile(3 + np.arange(S), B)
    ref = hf_rope(normed_t, heads, D, cache, pos).reshape(x.shape)
    assert_matches_where_unambiguous(fused, lo, hi, ref, "qk_norm_rope", min_exact=0.99)


# ---------------------------------------------------------------- KV cache

def test_kv_append_kat(oracle):
    """The reference test's scenario (kv_cache_cuda_test.cpp:124-300): prefill of 2 tokens and a decode step into
    both layers; every slot checked with the test's own index formula (verify_slice, :61-113), the rest stays 0."""
    L, Bc, Sc, P = kat.KV_LAYERS, kat.KV_BATCH, kat.KV_SEQ_CAP, kat.KV_HEADS * kat.KV_DIM
    kc = np.zeros((L, Bc, Sc, P), np.uint16)
    vc = np.zeros_like(kc)
    steps = kat.kv_steps()
    for layer in range(L):
        for start, k, v in steps:
            kc[layer], vc[layer] = oracle.kv_append(k, v, kc[layer], vc[layer], start)
    flat_k, flat_v = kc.reshape(-1), vc.reshape(-1)
    written = np.zeros(flat_k.size, bool)
    for layer in range(L):
        for start, k, v in steps:
            S = k.shape[1]
            for b in range(Bc):
                for t in range(S):
                    for col in range(P):
                        dst = ((layer * Bc + b) * Sc + start + t) * P + col
                        src = (b * S + t) * P + col
                        assert flat_k[dst] == k.reshape(-1)[src] and flat_v[dst] == v.reshape(-1)[src]
                        written[dst] = True
    assert not flat_k[~written].any() and not flat_v[~written].any()
    # the decode values of the test include one that bf16 must round: 61 + 0.25 * 15 = 64.75 -> 64.5 or 65
    assert kat.kv_values(16, 61.0)[15] == oracle.bf16(64.75)


def test_kv_append_fp32_rows_and_bytes(oracle, synth):
    """Bytes are copied unchanged whatever the element type (the reference cache also takes Float32)."""
    rng = np.random.default_rng(7)
    k = rng.standard_normal((3, 4, 24)).astype(np.float32)
    v = rng.standard_normal((3, 4, 24)).astype(np.float32)
    kc = np.full((4, 9, 24), np.nan, np.float32)
    vc = np.full((4, 9, 24), np.nan, np.float32)
    kc2, vc2 = oracle.kv_append(k, v, kc, vc, 5)
    assert np.array_equal(kc2[:3, 5:9].view(np.uint32), k.view(np.uint32))
    assert np.array_equal(vc2[:3, 5:9].view(np.uint32), v.view(np.uint32))
    assert np.isnan(kc2[3]).all() and np.isnan(kc2[:, :5]).all() and np.isnan(vc2[:, :5]).all()


# ---------------------------------------------------------------- attention

def _attn_f64(q, kc, vc, Hq, start):
    """Causal GQA attention in float64 with torch SDPA (head h reads KV head h // G, as HF Qwen3 repeat_kv)."""
    B, S = q.shape[:2]
    _, L, Hkv, D = kc.shape
    G = Hq // Hkv
    f = lambda b: torch.from_numpy((b.astype(np.uint32) << 16).view(np.float32).astype(np.float64))  # noqa: E731
    qt = f(np.ascontiguousarray(q)).reshape(B, S, Hq, D).transpose(1, 2)
    kt = f(np.ascontiguousarray(kc)).transpose(1, 2).repeat_interleave(G, dim=1)
    vt = f(np.ascontiguousarray(vc)).transpose(1, 2).repeat_interleave(G, dim=1)
    pos_q = start + torch.arange(S)[:, None]
    mask = torch.arange(L)[None, :] <= pos_q
    o = torch.nn.functional.scaled_dot_product_attention(qt, kt, vt, attn_mask=mask,
                                                         scale=float(np.float32(1.0) / np.sqrt(np.float32(D))))
    return o.transpose(1, 2).reshape(B, S, Hq * D).numpy()


def test_attention_kat(oracle):
    """The reference test's case and its tolerance; its own expected values are a two-pass fp32 softmax
    (gqa_attention_cuda_test.cpp:117-236), restated here in numpy."""
    q, kc, vc = kat.att_inputs()
    prim, lo, hi = oracle.gqa_attention(q, kc, vc, kat.ATT_HQ, kat.ATT_START)
    f = lambda b: (b.astype(np.uint32) << 16).view(np.float32)  # noqa: E731
    B, S, Hq, Hkv, D = kat.ATT_B, kat.ATT_S, kat.ATT_HQ, kat.ATT_HKV, kat.ATT_D
    qf, kf, vf = f(q).reshape(B, S, Hq, D), f(kc), f(vc)
    scale = np.float32(1.0) / np.sqrt(np.float32(D))
    for b in range(B):
        for s in range(S):
            vis = kat.ATT_START + s + 1
            for h in range(Hq):
                g = h // (Hq // Hkv)
                scores = np.array([np.float32(np.sum(qf[b, s, h] * kf[b, j, g], dtype=np.float32)) * scale
                                   for j in range(vis)], np.float32)
                w = np.exp(scores - scores.max()).astype(np.float32)
                ref = (w[:, None] / w.sum(dtype=np.float32) * vf[b, :vis, g]).sum(axis=0, dtype=np.float32)
                got = f(prim[b, s, h * D:(h + 1) * D])
                assert np.all(np.abs(got - ref) <= kat.ATT_TOL), (b, s, h, got, ref)
    assert oracle.compare(prim, prim, lo, hi)["fail"] == 0


def test_attention_matches_float64_sdpa(oracle, synth):
    """An independent implementation (torch SDPA in float64): its rounded values lie in the band, and the primary
    result is within one ulp of them; GQA head grouping, causal offset and strided cache views included."""
    B, S, Hq, Hkv, D, start, cap = 2, 24, 8, 2, 128, 40, 80
    q = synth.normal_bf16(140, 1, (B, S, Hq * D))
    store_k = synth.normal_bf16(141, 1, (B + 1, cap, Hkv, D))
    store_v = synth.normal_bf16(142, 1, (B + 1, cap, Hkv, D))
    kc, vc = store_k[:B, :start + S], store_v[:B, :start + S]  # strided views, as KvCache::key_view
    prim, lo, hi = oracle.gqa_attention(q, kc, vc, Hq, start)
    ref = synth.f32_to_bf16(_attn_f64(q, kc, vc, Hq, start).astype(np.float32))
    st = oracle.compare(ref, prim, lo, hi)
    assert st["fail"] == 0, st
    st2 = oracle.compare(prim, ref)
    assert st2["fail"] == 0 and st2["n"] == prim.size, st2  # primary within 1 ulp of the float64 result
    assert st["ambiguous"] <= 0.12 * prim.size, st          # the band stays narrow


def test_attention_closed_forms(oracle, synth):
    D, Hq, Hkv = 128, 4, 2
    # one visible key (start 0, position 0): the output is that value row, bit for bit
    q = synth.normal_bf16(143, 1, (1, 1, Hq * D))
    kc = synth.normal_bf16(144, 1, (1, 1, Hkv, D))
    vc = synth.normal_bf16(145, 1, (1, 1, Hkv, D))
    prim, _, _ = oracle.gqa_attention(q, kc, vc, Hq, 0)
    assert np.array_equal(prim.reshape(Hq, D), vc[0, 0, np.arange(Hq) // 2])
    # identical keys: uniform weights, the output is the mean of the visible values
    L = 37
    k1 = np.broadcast_to(synth.normal_bf16(146, 1, (1, 1, Hkv, D)), (1, L, Hkv, D)).copy()
    vL = synth.normal_bf16(147, 1, (1, L, Hkv, D))
    qL = synth.normal_bf16(148, 1, (1, 1, Hq * D))
    prim, lo, hi = oracle.gqa_attention(qL, k1, vL, Hq, L - 1)
    mean = synth.bf16_to_f32(vL).astype(np.float64).mean(axis=1)[0]          # [Hkv, D]
    want = synth.f32_to_bf16(mean[np.arange(Hq) // 2].reshape(1, 1, Hq * D).astype(np.float32))
    assert oracle.compare(want, prim, lo, hi)["fail"] == 0
    # one dominant key: weight 1 on it (others underflow), the output is its value row
    kd = synth.normal_bf16(149, 1, (1, L, Hkv, D))
    qd = np.full((1, 1, Hq * D), synth.f32_to_bf16(np.array([2.0], np.float32))[0], np.uint16)
    kd[0, 11] = synth.f32_to_bf16(np.array([8.0], np.float32))[0]
    prim, _, _ = oracle.gqa_attention(qd, kd, vL, Hq, L - 1)
    assert np.array_equal(prim.reshape(Hq, D), vL[0, 11, np.arange(Hq) // 2])


def test_attention_row_subset_and_planted_mistake(oracle, synth):
    B, S, Hq, Hkv, D = 1, 16, 8, 2, 128
    q = synth.normal_bf16(150, 1, (B, S, Hq * D))
    kc = synth.normal_bf16(151, 1, (B, S, Hkv, D))
    vc = synth.normal_bf16(152, 1, (B, S, Hkv, D))
    full, lo, hi = oracle.gqa_attention(q, kc, vc, Hq, 0)
    rows = np.array([0, 5, 77, 127])
    sub, slo, shi = oracle.gqa_attention(q, kc, vc, Hq, 0, rows=rows)
    assert np.array_equal(sub, full.reshape(-1, D)[rows])
    # a restatement that maps query head h to KV head h % Hkv (instead of h // G) is rejected by the rule
    f = lambda b: (b.astype(np.uint32) << 16).view(np.float32).astype(np.float64)  # noqa: E731
    qf = f(q).reshape(S, Hq, D)
    out = np.empty((S, Hq, D))
    for s in range(S):
        for h in range(Hq):
            g = h % Hkv
            sc = (f(kc[0, :s + 1, g]) @ qf[s, h]) * float(np.float32(1) / np.sqrt(np.float32(D)))
            w = np.exp(sc - sc.max())
            out[s, h] = (w / w.sum()) @ f(vc[0, :s + 1, g])
    wrong = synth.f32_to_bf16(out.astype(np.float32)).reshape(B, S, Hq * D)
    assert oracle.compare(wrong, full, lo, hi)["fail"] > 0


@pytest.mark.parametrize("S", [512, 1024])
def test_attention_band_separates_weight_roundings(oracle, synth, S):
    """The band decides how many bits the matrix-core kernel must keep of each softmax weight p (the reference
    multiplies fp32 p by v).  Emulated in float64 on sampled rows of the later half of the sequence (long key
    ranges): p as a bf16 high part plus a bf16 remainder (the kernel's two P V products, ~16 bits) stays inside the
    band everywhere; one bf16 rounding of p (8 bits) and one fp16 rounding (11 bits) are rejected."""
    B, Hq, Hkv, D = 1, 8, 2, 128
    G = Hq // Hkv
    q = synth.normal_bf16(160, S, (B, S, Hq * D))
    kc = synth.normal_bf16(161, S, (B, S, Hkv, D))
    vc = synth.normal_bf16(162, S, (B, S, Hkv, D))
    rng = np.random.default_rng(S)
    rows = np.unique(np.concatenate([rng.integers(S * Hq // 2, S * Hq, 512), np.arange(S * Hq - Hq, S * Hq)]))
    prim, lo, hi = oracle.gqa_attention(q, kc, vc, Hq, 0, rows=rows)

    def bf16_rne(x):
        return f32(synth.f32_to_bf16(np.asarray(x, np.float32)))

    def e4m3_scaled(x):
        """OCP fp8 e4m3 (3 mantissa bits, subnormal step 2^-9, max 448, ties to even) with a power-of-two scale
        per 32 consecutive elements of the last axis (zero-padded to a multiple of 32), as block-scaled fp8 MFMA
        operands carry it."""
        n = x.shape[-1]
        xp = np.zeros(x.shape[:-1] + (-(-n // 32) * 32,))
        xp[..., :n] = x
        xb = xp.reshape(x.shape[:-1] + (-1, 32))
        m = np.abs(xb).max(axis=-1, keepdims=True)
        scale = np.exp2(np.floor(np.log2(448.0 / np.where(m > 0, m, 448.0))))
        a = np.abs(xb) * scale
        step = np.exp2(np.maximum(np.floor(np.log2(np.where(a > 0, a, 1.0))), -6) - 3)
        r = np.sign(xb) * np.minimum(np.round(a / step) * step, 448.0)
        return (r / scale).reshape(xp.shape)[..., :n]

    # e4m3 known values (block max 448, so scale 1): ties to even, the subnormal step, flush below half of it
    kv = np.array([448.0, 1.0625, 1.1, 0.3, 2.0 ** -9, 1.5 * 2.0 ** -10, 2.0 ** -11, -3.3])
    assert np.array_equal(e4m3_scaled(kv), [448.0, 1.0, 1.125, 0.3125, 2.0 ** -9, 2.0 ** -9, 0.0, -3.25])

    qf = f32(q).astype(np.float64).reshape(S, Hq, D)
    kf = f32(kc)[0].astype(np.float64)
    vf = f32(vc)[0].astype(np.float64)
    scale2 = np.float32(np.float32(1) / np.sqrt(np.float32(D))) * np.float32(1.4426950408889634)
    outs = {"bf16 high + bf16 remainder": [], "fp16 high + fp8 remainder": [], "bf16": [], "fp16": []}
    for r in rows:
        s, h = divmod(int(r), Hq)
        g = h // G
        x = (kf[:s + 1, g] @ qf[s, h]).astype(np.float32) * scale2
        p = np.exp2(x - x.max()).astype(np.float32)
        l = p.astype(np.float64).sum()
        ph = bf16_rne(p)
        p16 = p.astype(np.float16).astype(np.float32)
        v = vf[:s + 1, g]
        sums = [(ph.astype(np.float64) + bf16_rne(p - ph)) @ v,
                p16.astype(np.float64) @ v + e4m3_scaled((p - p16).astype(np.float64)) @ e4m3_scaled(v.T).T,
                ph.astype(np.float64) @ v, p16.astype(np.float64) @ v]
        for key, o in zip(outs, sums):
            outs[key].append(synth.f32_to_bf16((o / l).astype(np.float32)))
    fails = {key: oracle.compare(np.stack(o), prim, lo, hi)["fail"] for key, o in outs.items()}
    n = rows.size * D
    assert fails["bf16 high + bf16 remainder"] == 0, fails
    assert fails["fp16 high + fp8 remainder"] == 0, fails
    assert fails["bf16"] > 0.03 * n, fails
    assert fails["fp16"] > 0, fails


# ---------------------------------------------------------------- argmax

def test_argmax_kat(oracle):
    x, want = kat.argmax_inputs()
    assert np.array_equal(oracle.argmax(x), want)


def test_argmax_matches_numpy_and_edge_cases(oracle, synth):
    """numpy's argmax returns the first maximum, as the reference's tie rule; NaN must first become -inf (numpy would
    return the NaN's index).  Also: +0 and -0 compare equal, all -inf gives 0, the valid-size prefix."""
    x = synth.normal_bf16(170, 1, (37, 1000), std=3.0)
    x[3, 100] = 0x7fc0                      # NaN ignored
    x[4, :] = 0xff80                        # all -inf -> 0
    x[5, :] = 0x8000                        # -0 everywhere ...
    x[5, 7] = 0x0000                        # ... and one +0: equal, the first index wins
    x[6, 10] = x[6, 20] = 0x7f80            # two +inf: the first
    f = synth.bf16_to_f32(x).astype(np.float64)
    f[np.isnan(f)] = -np.inf
    assert np.array_equal(oracle.argmax(x), np.argmax(f, axis=1).astype(np.int32))
    assert oracle.argmax(x)[5] == 0 and oracle.argmax(x)[4] == 0 and oracle.argmax(x)[6] == 10
    assert np.array_equal(oracle.argmax(x, 500), np.argmax(f[:, :500], axis=1).astype(np.int32))


# ---------------------------------------------------------------- sampling

def test_mt19937_64_check_value():
    """[rand.predef]: the 10000th output of a default-constructed mt19937_64 is 9981545732273789042."""
    from mt64 import MT19937_64
    g = MT19937_64()
    for _ in range(9999):
        g()
    assert g() == 9981545732273789042


def test_sampler_kat(oracle):
    """sampler_cuda_test.cpp:100-175: top_k = 1 with seed 122 gives [2, 1] (row 1 ties 7 and 7: top-k keeps both,
    and the seed's second draw picks the smaller id); top_k 3 / top_p 0.8 only ever draws ids 0 or 1."""
    from mt64 import MT19937_64
    rows = kat.bf(kat.SAMPLER_GREEDY)
    g = MT19937_64(122)
    assert [oracle.sample_row(rows[i], 0.6, 1, 1.0, g.uniform()) for i in range(2)] == kat.SAMPLER_GREEDY_IDS
    assert oracle.sample_row(rows[0], 0.6, 1, 1.0, 0.99) == 2                 # a unique maximum ignores the draw
    g = MT19937_64(42)
    for _ in range(16):
        assert oracle.sample_row(kat.bf(kat.SAMPLER_TOPP_ROW), 1.0, 3, 0.8, g.uniform()) in (0, 1)
    # the top-p cut: weights 1, 1, e^-1 (total 2.368); 0.8 * total is reached after two tokens
    assert oracle.sample_row(kat.bf(kat.SAMPLER_TOPP_ROW), 1.0, 3, 0.8, 0.49) == 0
    assert oracle.sample_row(kat.bf(kat.SAMPLER_TOPP_ROW), 1.0, 3, 0.8, 0.51) == 1
    assert oracle.sample_row(kat.bf(np.array([1.0, np.inf], np.float32)), 1.0, 0, 1.0, 0.5) == -1


def test_sampler_inverse_cdf_closed_form(oracle, synth):
    """Without top-k / top-p the draw is the inverse CDF of softmax(logit / T) over tokens ordered by (score desc,
    id asc): recomputed with numpy's lexsort and cumsum."""
    row = synth.normal_bf16(172, 1, (1000,), std=2.0)
    row[10] = row[20]                                            # a tie in score
    T = 0.7
    s = synth.bf16_to_f32(row).astype(np.float64) / np.float64(np.float32(T))
    order = np.lexsort((np.arange(s.size), -s))
    w = np.exp(s[order] - s[order[0]])
    cdf = np.cumsum(w) / w.sum()
    for u in np.random.default_rng(3).random(300):
        want = order[min(np.searchsorted(cdf, u, side="right"), s.size - 1)]
        assert oracle.sample_row(row, T, 0, 1.0, float(u)) == want
    # top-k: the draw never leaves the k best (ties at the k-th included)
    top = set(oracle.topk_set(row, 50).tolist())
    assert all(oracle.sample_row(row, T, 50, 0.9, float(u)) in top for u in np.linspace(0, 0.999, 50))


def test_topk_set_keeps_ties(oracle, synth):
    row = synth.normal_bf16(173, 1, (5000,))
    f = synth.bf16_to_f32(row)
    for k in (1, 7, 64, 4999, 5000):
        kth = np.sort(f)[::-1][k - 1]
        want = np.flatnonzero(f >= kth)
        got = oracle.topk_set(row, k)
        assert np.array_equal(np.sort(got), want) and got.size >= k
    tied = np.full(100, kat.bf([1.0])[0], np.uint16)
    tied[:10] = kat.bf([3.0])[0]
    assert oracle.topk_set(tied, 12).size == 100                  # the 12th ties with 89 others: all kept
