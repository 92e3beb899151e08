"""Sizes past the 32-bit range: every op family on tensors of more than 2^31
elements, or with element offsets past 2^31 (an MI355X holds 288 GB, so a
single activation or cache can be that large).  The ABI takes 64-bit sizes;
these cases check that no index inside a kernel wraps.

Inputs are built on the device by doubling copies of one random block whose
length is not a power of two, so element p holds block[p % len]: a wrapped
index would read a different value.  Outputs are checked against the oracle
on windows at the start, around element 2^31 and at the end.
"""
import numpy as np
import pytest

from gpu_util import announce, check_band, check_exact

pytestmark = pytest.mark.gpu
EPS = 1e-6
BLOCK = 3 * (1 << 21) + 7            # block length in elements (odd)
TWO31 = 1 << 31


@pytest.fixture(scope="module")
def block(synth):
    return synth.normal_bf16(77, 1, (BLOCK,))


def need_free(hip, nbytes):
    free, _ = hip.mem_info()
    if free < nbytes + (2 << 30):
        pytest.skip(f"needs {nbytes / 2**30:.1f} GiB of free device memory, {free / 2**30:.1f} GiB free")


def tiled(hip, block, n, shift=0):
    """A device buffer of n bf16 elements, element p = block[(p + shift) % BLOCK]."""
    buf = hip.DeviceBuffer(2 * n)
    src = np.roll(block, -shift)
    first = min(n, BLOCK)
    buf.upload(src[:first])
    rt = hip.runtime()
    filled = first
    while filled < n:
        step = min(filled, n - filled)
        hip.check(rt.hipMemcpy(buf.ptr + 2 * filled, buf.ptr, 2 * step, hip.HIP_MEMCPY_D2D), "hipMemcpy D2D")
        filled += step   # every copy starts at a multiple of BLOCK, so the period holds
    return buf


def host_elems(block, idx, shift=0):
    return block[(np.asarray(idx, np.int64) + shift) % BLOCK]


def windows(n, width):
    """Element windows [start, end) at the beginning, around 2^31 and at the end of n elements."""
    out = [(0, width)]
    if n > TWO31 + width:
        out.append((TWO31 - width, TWO31 + width))
    out.append((n - width, n))
    return out


def test_elementwise_past_int32(q3k, hip, oracle, block):
    n = TWO31 + 8 * 3 + 5                      # ragged tail past 2^31
    need_free(hip, 3 * 2 * n)
    announce(f"silu_mul / add_inplace n={n}")
    g, u = tiled(hip, block, n, 0), tiled(hip, block, n, 12345)
    out = hip.DeviceBuffer(2 * n)
    try:
        q3k.silu_mul(g, u, out, n)
        q3k.add_inplace(g, u, n)
        hip.synchronize()
        for a, b in windows(n, 4096):
            idx = np.arange(a, b)
            gh, uh = host_elems(block, idx), host_elems(block, idx, 12345)
            prim, lo, hi = oracle.silu_mul(gh, uh)
            check_band(oracle, f"silu_mul [{a}, {b})", out.download(np.uint16, (b - a,), 2 * a), prim, lo, hi)
            check_exact(f"add_inplace [{a}, {b})", g.download(np.uint16, (b - a,), 2 * a), oracle.add_inplace(gh, uh))
    finally:
        for b_ in (g, u, out):
            b_.free()


def pick_rows(rows, N):
    """Rows at the start, the row that holds element 2^31 and its neighbours, and the last rows."""
    mid = TWO31 // N
    return sorted(r for r in {0, 1, mid - 1, mid, mid + 1, rows - 2, rows - 1} if 0 <= r < rows)


def test_rms_norms_past_int32(q3k, hip, oracle, synth, block):
    N = 4096
    rows = (1 << 19) + 3                       # rows * N > 2^31
    n = rows * N
    need_free(hip, 3 * 2 * n)
    announce(f"rms_norm / add_rms_norm rows={rows} N={N}")
    w = synth.normal_bf16(78, 2, (N,), mean=1.0, std=0.1)
    W = hip.DeviceBuffer.from_array(w)
    x, d, y = tiled(hip, block, n, 0), tiled(hip, block, n, 999), hip.DeviceBuffer(2 * n)
    try:
        sel = pick_rows(rows, N)
        idx = (np.array(sel, np.int64)[:, None] * N + np.arange(N)[None, :])
        xh, dh = host_elems(block, idx), host_elems(block, idx, 999)
        q3k.rms_norm(x, W, y, rows, N, EPS)
        hip.synchronize()
        got = np.stack([y.download(np.uint16, (N,), 2 * r * N) for r in sel])
        prim, lo, hi = oracle.rms_norm(xh, w, EPS)
        check_band(oracle, f"rms_norm rows {sel}", got, prim, lo, hi)
        q3k.add_rms_norm(x, d, W, y, rows, N, EPS)
        hip.synchronize()
        got_h = np.stack([x.download(np.uint16, (N,), 2 * r * N) for r in sel])
        got_y = np.stack([y.download(np.uint16, (N,), 2 * r * N) for r in sel])
        h_ref, prim, lo, hi = oracle.add_rms_norm(xh, dh, w, EPS)
        check_exact(f"add_rms_norm residual rows {sel}", got_h, h_ref)
        check_band(oracle, f"add_rms_norm rows {sel}", got_y, prim, lo, hi)
    finally:
        for b_ in (W, x, d, y):
            b_.free()


def test_embedding_past_int32(q3k, hip, oracle, synth):
    V, H = 1000, 4096
    T = (1 << 19) + 3                          # T * H > 2^31 output elements
    need_free(hip, 2 * T * H)
    announce(f"embedding T={T} H={H}")
    table = synth.normal_bf16(79, 1, (V, H))
    ids = synth.token_ids(79, 2, (T,), V)
    Tb, I, out = hip.DeviceBuffer.from_array(table), hip.DeviceBuffer.from_array(ids), hip.DeviceBuffer(2 * T * H)
    try:
        q3k.embedding(I, T, Tb, V, H, out)
        hip.synchronize()
        sel = pick_rows(T, H)
        got = np.stack([out.download(np.uint16, (H,), 2 * t * H) for t in sel])
        check_exact(f"embedding tokens {sel}", got, oracle.embedding(ids[sel], table))
    finally:
        for b_ in (Tb, I, out):
            b_.free()


def test_qk_norm_rope_past_int32(q3k, hip, oracle, synth, block):
    Hq, Hkv, D, P = 32, 8, 128, 4096
    S = (1 << 19) + 1                          # S * Hq * D > 2^31 query elements
    nq, nk = S * Hq * D, S * Hkv * D
    need_free(hip, 2 * (nq + nk))
    announce(f"qk_norm_rope S={S} Hq={Hq} Hkv={Hkv}")
    cache = q3k.build_rope_cache(P, D, 1e6)
    pos = synth.uniform_positions(80, 1, S, P)
    qw = synth.normal_bf16(80, 2, (D,), mean=1.0, std=0.1)
    kw = synth.normal_bf16(80, 3, (D,), mean=1.0, std=0.1)
    q, k = tiled(hip, block, nq, 0), tiled(hip, block, nk, 4321)
    C, Pb = hip.DeviceBuffer.from_array(cache), hip.DeviceBuffer.from_array(pos)
    QW, KW = hip.DeviceBuffer.from_array(qw), hip.DeviceBuffer.from_array(kw)
    try:
        q3k.qk_norm_rope(q, k, QW, KW, 1, S, Hq, Hkv, D, EPS, C, P, 0, Pb)
        hip.synchronize()
        sel = pick_rows(S, Hq * D)
        for name, buf, heads, w, shift in (("q", q, Hq, qw, 0), ("k", k, Hkv, kw, 4321)):
            row = heads * D
            idx = np.array(sel, np.int64)[:, None] * row + np.arange(row)[None, :]
            xh = host_elems(block, idx, shift).reshape(1, len(sel), row)
            prim, lo, hi = oracle.qk_norm_rope(xh, w, 1, len(sel), heads, D, EPS, cache, 0, pos[sel])
            got = np.stack([buf.download(np.uint16, (row,), 2 * t * row) for t in sel]).reshape(1, len(sel), row)
            check_band(oracle, f"qk_norm_rope {name} tokens {sel}", got, prim, lo, hi)
    finally:
        for b_ in (q, k, C, Pb, QW, KW):
            b_.free()


def test_argmax_past_int32(q3k, hip, oracle, block):
    rows, N = 16384, 151936                    # rows * N > 2^31
    n = rows * N
    need_free(hip, 2 * n)
    announce(f"argmax rows={rows} N={N}")
    x = tiled(hip, block, n, 0)
    out = hip.DeviceBuffer(4 * rows)
    try:
        q3k.argmax(x, out, rows, N, N)
        hip.synchronize()
        got = out.download(np.int32, (rows,))
        sel = pick_rows(rows, N)
        idx = np.array(sel, np.int64)[:, None] * N + np.arange(N)[None, :]
        want = oracle.argmax(host_elems(block, idx))
        check_exact(f"argmax rows {sel}", got[sel], want)
    finally:
        x.free()
        out.free()


@pytest.mark.parametrize("S,cached,start", [(1, 4096, 4095), (64, 64, 0)])
def test_attention_cache_offsets_past_int32(q3k, hip, oracle, synth, S, cached, start):
    """Batch 4 of a [5, 2^19, 8, 128] cache starts at element 2^31: decode (key-range split) and prefill."""
    B, Hq, Hkv, D, seq_cap = 5, 32, 8, 128, 1 << 19
    row = Hkv * D
    n = B * seq_cap * row
    need_free(hip, 2 * 2 * n)
    announce(f"attention B={B} S={S} cached={cached} cache elements={n}")
    q = synth.normal_bf16(81, S, (B, S, Hq * D))
    kh = synth.normal_bf16(82, S, (B, cached, Hkv, D))
    vh = synth.normal_bf16(83, S, (B, cached, Hkv, D))
    K, Vb = hip.DeviceBuffer(2 * n), hip.DeviceBuffer(2 * n)
    Q, O = hip.DeviceBuffer.from_array(q), hip.DeviceBuffer(2 * B * S * Hq * D)
    ws_bytes = q3k.gqa_attention_workspace_bytes(B, S, Hq, Hkv, D, cached)
    ws = hip.DeviceBuffer(ws_bytes) if ws_bytes else None
    try:
        for b in range(B):
            K.upload(kh[b], 2 * b * seq_cap * row)
            Vb.upload(vh[b], 2 * b * seq_cap * row)
        st = (seq_cap * row, row, D, 1)
        q3k.gqa_attention(Q, K, Vb, O, B, S, Hq, Hkv, D, cached, start, st, st, workspace=ws, workspace_bytes=ws_bytes)
        hip.synchronize()
        got = O.download(np.uint16, (B, S, Hq * D))
        prim, lo, hi = oracle.gqa_attention(q, kh, vh, Hq, start)
        check_band(oracle, f"attention S={S} cached={cached}", got, prim, lo, hi)
    finally:
        for b_ in (K, Vb, Q, O) + ((ws,) if ws is not None else ()):
            b_.free()


def test_kv_append_past_int32(q3k, hip, synth):
    """Rows appended at the end of a [5, 2^19, 1024] bf16 cache: the last batch's rows lie past element 2^31."""
    B, seq_cap, row, S = 5, 1 << 19, 1024, 16
    n = B * seq_cap * row
    need_free(hip, 2 * 2 * n)
    start = seq_cap - S
    announce(f"kv_append B={B} seq_cap={seq_cap} start={start}")
    k = synth.normal_bf16(84, 1, (B, S, row))
    v = synth.normal_bf16(84, 2, (B, S, row))
    Kc, Vc = hip.DeviceBuffer(2 * n), hip.DeviceBuffer(2 * n)
    Kb, Vb = hip.DeviceBuffer.from_array(k), hip.DeviceBuffer.from_array(v)
    try:
        q3k.kv_append(Kb, Vb, Kc, Vc, B, S, 2 * row, seq_cap, start)
        hip.synchronize()
        for b in range(B):
            off = 2 * (b * seq_cap + start) * row
            check_exact(f"kv_append k batch {b}", Kc.download(np.uint16, (S, row), off), k[b])
            check_exact(f"kv_append v batch {b}", Vc.download(np.uint16, (S, row), off), v[b])
    finally:
        for b_ in (Kc, Vc, Kb, Vb):
            b_.free()
