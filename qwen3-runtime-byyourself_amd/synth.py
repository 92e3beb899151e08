"""Seeded synthetic inputs for the benchmark configurations.

The reference ships no data for this path, so every tensor is generated on
the host: a PCG64 stream keyed by (config seed, tensor id), float32 standard
normals scaled to the stated mean/std, then rounded to bf16 (nearest-even).
Generation is chunked at fixed 2^24-element boundaries, so a tensor's bytes
depend only on (seed, tensor id, size, mean, std), on any machine with the
same numpy.  Token ids are uniform integers from the same kind of stream.
"""
from __future__ import annotations

import numpy as np

_CHUNK = 1 << 24


def f32_to_bf16(x: np.ndarray) -> np.ndarray:
    """Round float32 to bf16 bit patterns (nearest-even; NaN -> quiet NaN)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    b = x.view(np.uint32)
    nan = (b & 0x7FFFFFFF) > 0x7F800000
    r = ((b + (0x7FFF + ((b >> 16) & 1))) >> 16).astype(np.uint16)
    if nan.any():
        r[nan] = ((b[nan] >> 16) | 0x40).astype(np.uint16)
    return r


def bf16_to_f32(b: np.ndarray) -> np.ndarray:
    b = np.ascontiguousarray(b, dtype=np.uint16)
    return (b.astype(np.uint32) << 16).view(np.float32)


def _rng(seed: int, tensor_id: int) -> np.random.Generator:
    return np.random.Generator(np.random.PCG64(np.random.SeedSequence([int(seed), int(tensor_id)])))


def normal_bf16(seed: int, tensor_id: int, shape, mean: float = 0.0, std: float = 1.0) -> np.ndarray:
    shape = tuple(int(s) for s in (shape if isinstance(shape, (tuple, list)) else (shape,)))
    n = int(np.prod(shape, dtype=np.int64)) if shape else 1
    rng = _rng(seed, tensor_id)
    out = np.empty(n, dtype=np.uint16)
    m, s = np.float32(mean), np.float32(std)
    for start in range(0, n, _CHUNK):
        stop = min(n, start + _CHUNK)
        z = rng.standard_normal(stop - start, dtype=np.float32)
        out[start:stop] = f32_to_bf16(m + s * z)
    return out.reshape(shape)


def token_ids(seed: int, tensor_id: int, shape, vocab: int) -> np.ndarray:
    shape = tuple(int(s) for s in (shape if isinstance(shape, (tuple, list)) else (shape,)))
    return _rng(seed, tensor_id).integers(0, vocab, size=shape, dtype=np.int64).astype(np.int32)


def uniform_positions(seed: int, tensor_id: int, n: int, high: int) -> np.ndarray:
    return _rng(seed, tensor_id).integers(0, high, size=(int(n),), dtype=np.int64).astype(np.int32)
