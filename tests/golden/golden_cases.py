"""Case list and input construction for the golden fixtures in golden_v1.npz.

Crane's repository holds no golden vectors or known-answer tests for the
attention path, so the fixtures are written here by make_golden.py from the
oracle (the C restatement of the candle op chain).  Each was checked against a
float64 evaluation when it was written.  Inputs are not stored: they are
regenerated from the seeds below with the oracle's SplitMix64 normal
generator, whose first values are stored too (case "gen"), so the fixture
also pins the generator.
"""
from __future__ import annotations

import numpy as np

D = 128
SEED = 0xC3A7E000

# name -> spec (plain ints/strings/lists; stored in the npz as JSON)
CASES = {
    "gen": dict(kind="gen", seed=SEED, n=16, lo=512, hi=4096),
    "rope_qwen3": dict(kind="rope", theta=1e6, alpha=0.0, max_pos=32769,
                       positions=[0, 1, 2, 100, 1023, 1024, 4095, 32768]),
    "rope_hunyuan_alpha": dict(kind="rope", theta=1e4, alpha=1000.0, max_pos=4097,
                               positions=[0, 1, 7, 511, 2048, 4096]),
    "rope_qwen2_bf16": dict(kind="rope_qwen2", theta=1e6, max_pos=4097, dtype="bf16",
                            positions=[0, 1, 255, 256, 257, 1000, 4096]),
    "append_qwen3_f32": dict(kind="append", seed=SEED + 101, B=1, S=3, Hq=16, Hkv=8, cache_len=[5],
                             positions=[5], cap=9, order=0, weights=False, dtype="f32"),
    "append_hunyuan_bf16": dict(kind="append", seed=SEED + 102, B=2, S=2, Hq=4, Hkv=2, cache_len=[0, 3],
                                positions=[0, 3], cap=8, order=1, weights=True, dtype="bf16"),
    "append_qwen25_bf16": dict(kind="append", seed=SEED + 103, B=2, S=4, Hq=7, Hkv=1, cache_len=[2, 0],
                               positions=[9, 0], cap=8, order=2, weights=False, dtype="bf16"),
    "decode_f32": dict(kind="decode", seed=SEED + 201, B=2, Hq=4, Hkv=2, lens=[37, 300], cap=320, dtype="f32"),
    "decode_bf16": dict(kind="decode", seed=SEED + 202, B=3, Hq=8, Hkv=2, lens=[1, 257, 600], cap=600,
                        dtype="bf16"),
    "prefill_bf16": dict(kind="prefill", seed=SEED + 301, B=1, S=70, Hq=4, Hkv=2, start=[0], causal=1,
                         dtype="bf16"),
    "prefill_continuation_bf16": dict(kind="prefill", seed=SEED + 302, B=2, S=20, Hq=6, Hkv=3, start=[0, 50],
                                      causal=1, dtype="bf16"),
    "prefill_f32": dict(kind="prefill", seed=SEED + 303, B=1, S=33, Hq=2, Hkv=1, start=[0], causal=1,
                        dtype="f32"),
}


def _normal(orc, seed, shape, dtype):
    x = orc.gen_normal(seed, shape)
    return orc.round_bf16(x) if dtype == "bf16" else x


def inputs(orc, spec: dict) -> dict:
    """Regenerate a case's inputs with the oracle's seeded generator."""
    k = spec["kind"]
    if k == "append":
        B, S, Hq, Hkv, dt, cap = spec["B"], spec["S"], spec["Hq"], spec["Hkv"], spec["dtype"], spec["cap"]
        s = spec["seed"]
        qkv = _normal(orc, s, (B, S, (Hq + 2 * Hkv) * D), dt)
        max_pos = max(spec["positions"]) + S
        cos, sin = orc.rope_tables(D, 1e6, max_pos)
        if dt == "bf16":
            cos, sin = orc.round_bf16(cos), orc.round_bf16(sin)
        qw = kw = None
        if spec["weights"]:
            qw = orc.round_bf16(1.0 + 0.25 * orc.gen_normal(s + 1, (D,))) if dt == "bf16" else \
                1.0 + 0.25 * orc.gen_normal(s + 1, (D,))
            kw = orc.round_bf16(1.0 + 0.25 * orc.gen_normal(s + 2, (D,))) if dt == "bf16" else \
                1.0 + 0.25 * orc.gen_normal(s + 2, (D,))
        return dict(qkv=qkv, cos=cos, sin=sin, q_w=qw, k_w=kw,
                    positions=np.asarray(spec["positions"], np.int32),
                    cache_len=np.asarray(spec["cache_len"], np.int32),
                    k_cache=np.zeros((B, Hkv, cap, D), np.float32), v_cache=np.zeros((B, Hkv, cap, D), np.float32))
    if k == "decode":
        B, Hq, Hkv, cap, dt, s = spec["B"], spec["Hq"], spec["Hkv"], spec["cap"], spec["dtype"], spec["seed"]
        return dict(q=_normal(orc, s, (B, Hq, D), dt), k=_normal(orc, s + 1, (B, Hkv, cap, D), dt),
                    v=_normal(orc, s + 2, (B, Hkv, cap, D), dt), lens=np.asarray(spec["lens"], np.int32))
    if k == "prefill":
        B, S, Hq, Hkv, dt, s = spec["B"], spec["S"], spec["Hq"], spec["Hkv"], spec["dtype"], spec["seed"]
        start = np.asarray(spec["start"], np.int32)
        cap = int(start.max()) + S
        return dict(q=_normal(orc, s, (B, Hq, S, D), dt), k=_normal(orc, s + 1, (B, Hkv, cap, D), dt),
                    v=_normal(orc, s + 2, (B, Hkv, cap, D), dt), start=start)
    raise ValueError(k)


def run_oracle(orc, spec: dict) -> dict:
    """The oracle's outputs for a case (what the fixture stores)."""
    k = spec["kind"]
    if k == "gen":
        return dict(normal=orc.gen_normal(spec["seed"], (spec["n"],)),
                    uniform=orc.gen_uniform_int(spec["seed"] + 3, 32, spec["lo"], spec["hi"]))
    if k == "rope":
        c, s = orc.rope_tables(D, spec["theta"], spec["max_pos"], spec["alpha"])
        p = np.asarray(spec["positions"])
        return dict(cos=c[p], sin=s[p])
    if k == "rope_qwen2":
        c, s = orc.rope_tables_qwen2(D, spec["theta"], spec["max_pos"], spec["dtype"])
        p = np.asarray(spec["positions"])
        return dict(cos=c[p], sin=s[p])
    x = inputs(orc, spec)
    scale = 1.0 / np.sqrt(D)
    if k == "append":
        q = orc.qk_norm_rope_append(x["qkv"], spec["Hq"], spec["Hkv"], x["cos"], x["sin"], x["positions"],
                                    x["k_cache"], x["v_cache"], x["cache_len"], q_w=x["q_w"], k_w=x["k_w"],
                                    order=spec["order"], dtype=spec["dtype"])
        return dict(q_out=q, k_cache=x["k_cache"], v_cache=x["v_cache"])
    if k == "decode":
        return dict(out=orc.attn_decode(x["q"], x["k"], x["v"], x["lens"], scale, spec["dtype"]))
    if k == "prefill":
        return dict(out=orc.attn_prefill(x["q"], x["k"], x["v"], x["start"], scale, bool(spec["causal"]),
                                         spec["dtype"]))
    raise ValueError(k)
