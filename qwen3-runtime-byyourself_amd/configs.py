"""The five workload configurations of the benchmark, with their shapes and
the algorithmic (compulsory) HBM bytes of each op.

Model shapes come from the reference's config fixtures
(tests/fixtures/qwen3_0_6b.json, tests/fixtures/qwen3_8b.json) and, for the
32B-shaped config, the stated hidden 5120 / intermediate 25600 / 64 query
heads.  head_dim 128, 8 KV heads, vocab 151936, eps 1e-6, rope theta 1e6.

Byte formulas (each byte counted once; bf16 = 2 bytes):
  embedding      4T + 2*T*H*2
  rms_norm       2*T*H*2 + 2H
  add_inplace    3*T*H*2
  add_rms_norm   4*T*H*2 + 2H
  qk_norm_rope   2*T*(Hq+Hkv)*D*2 + U*(D/2)*2*4 + 2*2*D   (U = distinct positions)
  silu_mul       3*T*I*2
"""
from __future__ import annotations

from dataclasses import dataclass, field

VOCAB = 151936
HEAD_DIM = 128
EPS = 1e-6
THETA = 1.0e6


@dataclass(frozen=True)
class Config:
    name: str
    seed: int
    batch: int
    seq: int
    hidden: int
    inter: int
    heads_q: int
    heads_kv: int
    positions: str  # "range" (start 0, per sequence) or "uniform" (random per sequence)
    max_pos: int    # table rows
    ops: tuple = field(default_factory=tuple)

    @property
    def tokens(self) -> int:
        return self.batch * self.seq

    def distinct_positions(self) -> int:
        if self.positions == "range":
            return self.seq
        return min(self.tokens, self.max_pos)  # upper bound for random positions


def bytes_embedding(T, H):
    return 4 * T + 2 * T * H * 2


def bytes_rms_norm(T, H):
    return 2 * T * H * 2 + 2 * H


def bytes_embedding_rms_norm(T, H):
    """ids + gathered rows in, hidden and normalized rows out, plus the weight."""
    return 4 * T + 3 * T * H * 2 + 2 * H


def bytes_add_inplace(T, H):
    return 3 * T * H * 2


def bytes_add_rms_norm(T, H):
    return 4 * T * H * 2 + 2 * H


def bytes_qk_norm_rope(T, Hq, Hkv, D, U):
    return 2 * T * (Hq + Hkv) * D * 2 + U * (D // 2) * 2 * 4 + 2 * 2 * D


def bytes_kv_append(T, Hkv, D):
    """K and V rows read once and written once into the cache."""
    return 2 * 2 * T * Hkv * D * 2


def bytes_qk_norm_rope_kv_append(T, Hq, Hkv, D, U):
    """Q in place; K read and written to the cache; V read and copied; table and weights once."""
    return 2 * T * (Hq + 2 * Hkv) * D * 2 + U * (D // 2) * 2 * 4 + 2 * 2 * D


def bytes_silu_mul(T, I):
    return 3 * T * I * 2


def bytes_rope(T, Hq, Hkv, D, U):
    """apply_rope_inplace on Q and K: both read and written once, the table rows of the U positions once."""
    return 2 * T * (Hq + Hkv) * D * 2 + U * (D // 2) * 2 * 4


def unfused_op_bytes(c: Config, U: int | None = None) -> dict:
    """The reference-order chain's ops (decoder_layer.cpp:78->88, self_attention.cpp:147-152, mlp.cpp:111,
    :94->:72), each byte counted once per op."""
    T, H = c.tokens, c.hidden
    U = c.distinct_positions() if U is None else U
    return {"add_inplace": bytes_add_inplace(T, H), "rms_norm": bytes_rms_norm(T, H),
            "rms_norm_q": bytes_rms_norm(T * c.heads_q, HEAD_DIM), "rms_norm_k": bytes_rms_norm(T * c.heads_kv, HEAD_DIM),
            "rope": bytes_rope(T, c.heads_q, c.heads_kv, HEAD_DIM, U), "add_inplace_2": bytes_add_inplace(T, H),
            "rms_norm_2": bytes_rms_norm(T, H), "silu_mul": bytes_silu_mul(T, c.inter)}


def c2_chain_bytes(c: Config) -> int:
    """Benchmark config 2's chain: embedding gather, residual add + RMSNorm, Q/K norm + RoPE, SwiGLU."""
    T = c.tokens
    return (bytes_embedding(T, c.hidden) + bytes_add_rms_norm(T, c.hidden)
            + bytes_qk_norm_rope(T, c.heads_q, c.heads_kv, HEAD_DIM, c.distinct_positions())
            + bytes_silu_mul(T, c.inter))


def chain_bytes(c: Config, U: int | None = None) -> int:
    """Per-layer non-GEMM chain, fused: 2 x add_rms_norm + qk_norm_rope + silu_mul."""
    T = c.tokens
    U = c.distinct_positions() if U is None else U
    return (2 * bytes_add_rms_norm(T, c.hidden) + bytes_qk_norm_rope(T, c.heads_q, c.heads_kv, HEAD_DIM, U)
            + bytes_silu_mul(T, c.inter))


CONFIGS = {
    "c1": Config("c1-qwen3-0.6b-rmsnorm-T16", 0, 1, 16, 1024, 3072, 16, 8, "range", 16, ("rms_norm",)),
    "c2": Config("c2-qwen3-0.6b-layer-T512", 1, 1, 512, 1024, 3072, 16, 8, "range", 512,
                 ("embedding", "add_rms_norm", "qk_norm_rope", "silu_mul")),
    "c3": Config("c3-qwen3-8b-decode-B64", 2, 64, 1, 4096, 12288, 32, 8, "uniform", 4096,
                 ("add_rms_norm", "qk_norm_rope", "silu_mul")),
    "c4": Config("c4-qwen3-8b-prefill-T8192", 3, 4, 2048, 4096, 12288, 32, 8, "range", 2048,
                 ("embedding", "add_rms_norm", "qk_norm_rope", "silu_mul", "rms_norm")),
    "c5": Config("c5-qwen3-32b-shape-prefill-T16384", 4, 2, 8192, 5120, 25600, 64, 8, "range", 8192,
                 ("add_rms_norm", "qk_norm_rope", "silu_mul", "rms_norm")),
}

# Tensor ids of the synthetic streams (with the config seed they key the RNG).
TID_TABLE, TID_IDS, TID_H, TID_D1, TID_W1, TID_Q, TID_K, TID_QW, TID_KW = range(9)
TID_H2, TID_D2, TID_W2, TID_GATE, TID_UP, TID_POS, TID_X, TID_WF = range(9, 17)
