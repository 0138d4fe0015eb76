"""Seeded inputs for the BASELINE configurations and the edge cases, shared by
the GPU parity tests.  Host arrays are float32 holding values representable in
the case's dtype (bf16 cases are rounded to bf16 first), so the same arrays
feed the oracle and, converted exactly, the GPU."""
from __future__ import annotations

import math

import numpy as np

D = 128
SEED0 = 0xC3A7E000  # seed = SEED0 + config number


def rng(seed: int) -> np.random.Generator:
    return np.random.Generator(np.random.PCG64(seed))


def normal(r: np.random.Generator, shape, std: float = 1.0) -> np.ndarray:
    x = r.standard_normal(size=shape, dtype=np.float32)
    if std != 1.0:
        x *= np.float32(std)
    return x


def bf16(x: np.ndarray) -> np.ndarray:
    """Round float32 to the nearest-even bf16 value (kept as float32)."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    r = ((u + np.uint32(0x7FFF) + ((u >> np.uint32(16)) & np.uint32(1))) & np.uint32(0xFFFF0000))
    return r.view(np.float32)


def cast(x: np.ndarray, dtype: str) -> np.ndarray:
    return bf16(x) if dtype == "bf16" else np.ascontiguousarray(x, dtype=np.float32)


def scale() -> float:
    return 1.0 / math.sqrt(D)


def decode_variant(orc, Hq: int, Hkv: int, score_mode=None) -> int:
    """The oracle decode form matching a kernel call's score mode (None: the
    rule of qwen3/modeling.rs:432, grouped iff n_rep > 1)."""
    if score_mode is None:
        score_mode = "grouped" if Hq // Hkv > 1 else "standard"
    return orc.DECODE_GROUPED if score_mode == "grouped" else orc.DECODE_STANDARD


def decode_case(seed, B, Hq, Hkv, lens, cap=None, dtype="bf16", std=1.0, poison=True):
    """q [B,Hq,D], K/V caches [B,Hkv,cap,D] with rows >= lens[b] set to NaN
    (a kernel that reads past kv_len produces NaN)."""
    r = rng(seed)
    lens = np.asarray(lens, dtype=np.int32)
    cap = int(cap or max(int(lens.max()), 1))
    q = cast(normal(r, (B, Hq, D)), dtype)
    k = cast(normal(r, (B, Hkv, cap, D), std), dtype)
    v = cast(normal(r, (B, Hkv, cap, D), std), dtype)
    if poison:
        for b in range(B):
            k[b, :, lens[b]:] = np.nan
            v[b, :, lens[b]:] = np.nan
    return q, k, v, lens


def prefill_case(seed, B, S, Hq, Hkv, start, cap=None, dtype="bf16", poison=True):
    r = rng(seed)
    start = np.asarray(start, dtype=np.int32)
    L = int(start.max()) + S
    cap = int(cap or L)
    q = cast(normal(r, (B, Hq, S, D)), dtype)
    k = cast(normal(r, (B, Hkv, cap, D)), dtype)
    v = cast(normal(r, (B, Hkv, cap, D)), dtype)
    if poison:
        for b in range(B):
            k[b, :, start[b] + S:] = np.nan
            v[b, :, start[b] + S:] = np.nan
    return q, k, v, start


def c3_lengths() -> np.ndarray:
    """Config 3: 32 per-sequence lengths uniform in [512, 4096] (seeded)."""
    return rng(SEED0 + 3).integers(512, 4096, size=32, endpoint=True).astype(np.int32)


def prefill_truth(q, k, v, start, b, r0, r1, causal=True):
    """float64 softmax(q K^T / sqrt(D) + mask) V for rows [r0, r1) of sequence b,
    all heads: [r1 - r0, Hq, D]."""
    _, Hq, S, _ = q.shape
    Hkv = k.shape[1]
    L = int(start[b]) + S
    out = np.zeros((r1 - r0, Hq, D))
    for h in range(Hq):
        K = k[b, h // (Hq // Hkv), :L].astype(np.float64)
        V = v[b, h // (Hq // Hkv), :L].astype(np.float64)
        s = q[b, h, r0:r1].astype(np.float64) @ K.T * scale()
        if causal:
            pos = int(start[b]) + np.arange(r0, r1)
            s[np.arange(L)[None, :] > pos[:, None]] = -np.inf
        p = np.exp(s - s.max(1, keepdims=True))
        out[:, h] = (p / p.sum(1, keepdims=True)) @ V
    return out


def _draw_heads(r):
    n_rep = int(r.choice([1, 2, 3, 4, 5, 6, 7, 8, 16]))
    hkv = int(r.choice([1, 2, 4]))
    return n_rep * hkv, hkv


def prefill_draw(seed: int, i: int):
    """Draw i of the randomised prefill sweep at seed offset `seed`: (dtype, B,
    S, Hq, Hkv, start, causal) and its inputs (q, k, v, start array)."""
    r = rng(seed + 7300 + i)
    dtype = "f32" if i % 5 == 4 else "bf16"
    Hq, Hkv = _draw_heads(r)
    B = int(r.integers(1, 4))
    S = int(r.choice([1, 31, 64, 65, 127, 128, 129, 300, int(r.integers(1, 700))]))
    if dtype == "f32":
        S = min(S, 200)
    start = [int(r.choice([0, 0, int(r.integers(1, 400))])) for _ in range(B)]
    causal = bool(r.random() < 0.8)
    while S > 1 and B * Hq * S * (max(start) + S) > 3e7:  # keep the oracle within seconds
        S //= 2
    q, k, v, st = prefill_case(seed + 7400 + i, B, S, Hq, Hkv, start, dtype=dtype)
    return (dtype, B, S, Hq, Hkv, start, causal), (q, k, v, st)


def prefill_long_draw(seed: int, i: int):
    """Draw i of the long-row prefill sweep: chunks that continue a cache of
    900-3600 rows, so every row sees about 1000 keys or more (the prefill
    kernel's long-row arithmetic), bf16."""
    r = rng(seed + 7700 + i)
    Hq, Hkv = _draw_heads(r)
    B = int(r.integers(1, 3))
    S = int(r.choice([64, 129, 300, int(r.integers(1, 400))]))
    start = [int(r.integers(900, 3600)) for _ in range(B)]
    causal = bool(r.random() < 0.8)
    while S > 1 and B * Hq * S * (max(start) + S) > 3e7:  # keep the oracle within seconds
        S //= 2
    q, k, v, st = prefill_case(seed + 7800 + i, B, S, Hq, Hkv, start, dtype="bf16")
    return ("bf16", B, S, Hq, Hkv, start, causal), (q, k, v, st)

