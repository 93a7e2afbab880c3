"""Synthetic inputs for the benchmark configurations (seeded numpy), quantized to
GGUF Q4_0 / Q8_0 blocks in the reference's byte layout.

The quantizers are ggml's textbook ones (the reference has no GGUF quantizer; the
benchmark configurations name them):
  Q4_0: max = signed value of largest |x| (first on ties); d = max / -8;
        id = 1/d (0 if d == 0); q = min(15, trunc(x*id + 8.5)); scale = fp16(d)
  Q8_0: d = amax / 127; id = 1/d (0 if d == 0); q = round_half_away(x*id)
  Q4_1: m = min, d = (max - min) / 15 (both through fp16); id = 1/d (0 if d == 0);
        q = min(15, trunc((x - m)*id + 0.5)); value q * d + m
Q4_0 / Q4_1 codes are packed in the reference nibble order: element 2j in the high
nibble of byte j (openmini-server/src/model/inference/quant.rs:179-188, :243-253).
All arithmetic is float32 with separate multiply and add, like the C oracle.
"""
from __future__ import annotations

import numpy as np

QK = 32
Q4_0, Q4_1, Q8_0 = 2, 3, 7


def normal(seed: int, shape, sigma: float) -> np.ndarray:
    rng = np.random.default_rng(seed)
    return (rng.standard_normal(size=shape, dtype=np.float32) * np.float32(sigma)).astype(np.float32)


def quantize_q4_0(x: np.ndarray) -> np.ndarray:
    v = np.ascontiguousarray(x, dtype=np.float32).reshape(-1, QK)
    a = np.abs(v)
    idx = np.argmax(a, axis=1)
    mx = v[np.arange(v.shape[0]), idx]
    mx = np.where(a[np.arange(v.shape[0]), idx] == 0, np.float32(0.0), mx).astype(np.float32)
    d = (mx / np.float32(-8.0)).astype(np.float32)
    with np.errstate(divide="ignore"):
        inv = np.where(d != 0, np.float32(1.0) / d, np.float32(0.0)).astype(np.float32)
    t = (v * inv[:, None]).astype(np.float32) + np.float32(8.5)
    q = np.minimum(t.astype(np.int8).astype(np.int32), 15).astype(np.uint8)
    out = np.empty((v.shape[0], 18), dtype=np.uint8)
    out[:, 0:2] = d.astype(np.float16).view(np.uint8).reshape(-1, 2)
    out[:, 2:] = (q[:, 0::2] << 4) | q[:, 1::2]
    return out.ravel()


def _round_half_away(t: np.ndarray) -> np.ndarray:
    r = np.trunc(t)
    frac = t - r
    return r + np.where(np.abs(frac) >= np.float32(0.5), np.sign(t), np.float32(0.0))


def quantize_q8_0(x: np.ndarray) -> np.ndarray:
    v = np.ascontiguousarray(x, dtype=np.float32).reshape(-1, QK)
    amax = np.max(np.abs(v), axis=1)
    d = (amax / np.float32(127.0)).astype(np.float32)
    with np.errstate(divide="ignore"):
        inv = np.where(d != 0, np.float32(1.0) / d, np.float32(0.0)).astype(np.float32)
    t = (v * inv[:, None]).astype(np.float32)
    q = _round_half_away(t).astype(np.int8)
    out = np.empty((v.shape[0], 34), dtype=np.uint8)
    out[:, 0:2] = d.astype(np.float16).view(np.uint8).reshape(-1, 2)
    out[:, 2:] = q.view(np.uint8)
    return out.ravel()


def quantize_q4_1(x: np.ndarray) -> np.ndarray:
    v = np.ascontiguousarray(x, dtype=np.float32).reshape(-1, QK)
    lo, hi = v.min(axis=1), v.max(axis=1)
    m16 = lo.astype(np.float16)
    d16 = ((hi - lo) / np.float32(15.0)).astype(np.float32).astype(np.float16)
    m, d = m16.astype(np.float32), d16.astype(np.float32)
    with np.errstate(divide="ignore"):
        inv = np.where(d != 0, np.float32(1.0) / d, np.float32(0.0)).astype(np.float32)
    t = ((v - m[:, None]).astype(np.float32) * inv[:, None]).astype(np.float32) + np.float32(0.5)
    q = np.clip(np.trunc(t), 0, 15).astype(np.uint8)
    out = np.empty((v.shape[0], 20), dtype=np.uint8)
    out[:, 0:2] = d16.view(np.uint8).reshape(-1, 2)
    out[:, 2:4] = m16.view(np.uint8).reshape(-1, 2)
    out[:, 4:] = (q[:, 0::2] << 4) | q[:, 1::2]
    return out.ravel()


def quantize(qtype: int, x: np.ndarray) -> np.ndarray:
    if qtype == Q4_1:
        return quantize_q4_1(x)
    return quantize_q4_0(x) if qtype == Q4_0 else quantize_q8_0(x)


def to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """float32 -> bfloat16 bits, round to nearest even (NaN kept quiet)."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    r = ((u + np.uint32(0x7FFF) + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    return np.where(nan, ((u >> 16) | 0x40).astype(np.uint16), r)


def bf16_bits_to_f32(b: np.ndarray) -> np.ndarray:
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def weight_blocks(qtype: int, n_rows: int, k_cols: int, seed: int, sigma: float = 0.02) -> np.ndarray:
    """GGUF blocks of W[n_rows, k_cols] ~ N(0, sigma), row-major (row n = K/32 blocks)."""
    return quantize(qtype, normal(seed, (n_rows, k_cols), sigma))


Q4_K, Q5_K, Q6_K, Q8_K = 12, 13, 14, 15


def kquant_blocks(qtype: int, n_rows: int, k_cols: int, seed: int) -> np.ndarray:
    """Random GGUF Q4_K (144 B) / Q5_K (176 B) / Q6_K (210 B) / Q8_K (258 B) super-blocks
    of W[n_rows, k_cols], row n = k_cols / 256 super-blocks, with finite fp16 d (and
    dmin) of weight-like size (values up to ~0.05).  The reference has no K-quant
    quantizer; these blocks exercise its reading of the layouts (quant.rs:338-410,
    433-505, 515-600, 768-800): every code, scale and minimum byte is random, d and dmin
    are drawn small and positive or negative."""
    assert k_cols % 256 == 0
    rng = np.random.default_rng(seed)
    nblk = n_rows * (k_cols // 256)
    bpb = {Q4_K: 144, Q5_K: 176, Q6_K: 210, Q8_K: 258}[qtype]
    raw = rng.integers(0, 256, size=(nblk, bpb), dtype=np.uint8)
    sign = np.where(rng.random(nblk) < 0.5, -1.0, 1.0)
    if qtype == Q5_K:
        d = (sign * (rng.random(nblk) * 2e-5 + 5e-6)).astype(np.float16)
        dmin = (rng.standard_normal(nblk) * 1e-3).astype(np.float16)
        raw[:, 0:2] = d.view(np.uint8).reshape(-1, 2)
        raw[:, 2:4] = dmin.view(np.uint8).reshape(-1, 2)
    elif qtype == Q4_K:
        d = (sign * (rng.random(nblk) * 1e-4 + 2e-5)).astype(np.float16)
        dmin = (rng.standard_normal(nblk) * 1e-3).astype(np.float16)
        raw[:, 0:2] = d.view(np.uint8).reshape(-1, 2)
        raw[:, 2:4] = dmin.view(np.uint8).reshape(-1, 2)
    elif qtype == Q8_K:
        d = (sign * (rng.random(nblk) * 3e-4 + 1e-4)).astype(np.float16)
        raw[:, 0:2] = d.view(np.uint8).reshape(-1, 2)
    else:
        d = (sign * (rng.random(nblk) * 2e-5 + 5e-6)).astype(np.float16)
        raw[:, 0:2] = d.view(np.uint8).reshape(-1, 2)
    return raw.ravel()
