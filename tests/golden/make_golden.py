"""Write tests/golden/golden_v1.npz from the oracle, after checking every case
against an independent float64 evaluation.

    python tests/golden/make_golden.py

The fixture holds, per case, its spec (JSON) and the oracle's outputs; inputs
are regenerated from the spec's seeds (golden_cases.inputs).
"""
from __future__ import annotations

import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)
sys.path.insert(0, HERE)

import oracle  # noqa: E402
from golden_cases import CASES, D, inputs, run_oracle  # noqa: E402

OUT = os.path.join(HERE, "golden_v1.npz")


def f64_rms_rope(x, w, cos, sin, pos, order, eps=1e-6):
    """Textbook RMSNorm over the last dim and rotate-half RoPE, float64."""
    x = x.astype(np.float64)

    def norm(y):
        r = y / np.sqrt(np.mean(y * y, axis=-1, keepdims=True) + eps)
        return r * (w.astype(np.float64) if w is not None else 1.0)

    def rope(y):
        c, s = cos[pos].astype(np.float64), sin[pos].astype(np.float64)
        h = D // 2
        return np.concatenate([y[..., :h] * c - y[..., h:] * s, y[..., h:] * c + y[..., :h] * s], axis=-1)

    if order == 0:
        return rope(norm(x))
    if order == 1:
        return norm(rope(x))
    return rope(x)


def f64_attention(q, k, v, allowed):
    s = q.astype(np.float64) @ k.astype(np.float64).T / np.sqrt(D)
    s = np.where(allowed, s, -np.inf)
    p = np.exp(s - s.max(-1, keepdims=True))
    return (p / p.sum(-1, keepdims=True)) @ v.astype(np.float64)


def check(name, spec, out):
    dt = spec.get("dtype", "f32")
    bar = 2e-2 if dt == "bf16" else 2e-5
    k = spec["kind"]
    if k == "gen":
        u = out["uniform"]
        assert u.min() >= spec["lo"] and u.max() <= spec["hi"]
        return 0.0
    if k in ("rope", "rope_qwen2"):
        # qwen3/modeling.rs:123-139: inv = 1.0f32 / (f32)(base^(2i/D)); angle = f32(p) * inv in f32
        base = spec["theta"] * (spec["alpha"] ** (D / (D - 2)) if spec.get("alpha") else 1.0)
        inv = np.array([np.float32(1.0) / np.float32(base ** (i / D)) for i in range(0, D, 2)], np.float32)
        p = np.asarray(spec["positions"], np.float32)
        if k == "rope":
            ang = (p[:, None] * inv[None, :]).astype(np.float32).astype(np.float64)
            ref = np.cos(ang)
            ulp = np.spacing(np.abs(ref).astype(np.float32)).astype(np.float64)
            assert np.all(np.abs(out["cos"] - ref) <= ulp + 1e-45), name   # libm cosf within 1 ulp
            return float(np.abs(out["cos"] - ref).max())
        # qwen2.rs:55-59: inv_freq and positions cast to bf16, the product in bf16
        ang = oracle.round_bf16((oracle.round_bf16(p)[:, None] * oracle.round_bf16(inv)[None, :]).astype(np.float32))
        ref = oracle.round_bf16(np.cos(ang.astype(np.float64)).astype(np.float32))
        err = float(np.abs(out["cos"] - ref).max())
        assert err <= 2 ** -8, (name, err)
        return err
    x = inputs(oracle, spec)
    if k == "append":
        B, S, Hq, Hkv = spec["B"], spec["S"], spec["Hq"], spec["Hkv"]
        qkv = x["qkv"].reshape(B, S, Hq + 2 * Hkv, D)
        err = 0.0
        for b in range(B):
            pos = spec["positions"][b] + np.arange(S)
            for h in range(Hq):
                ref = f64_rms_rope(qkv[b, :, h], x["q_w"], x["cos"], x["sin"], pos, spec["order"])
                err = max(err, float(np.abs(out["q_out"][b, h] - ref).max()))
            for g in range(Hkv):
                ref = f64_rms_rope(qkv[b, :, Hq + g], x["k_w"], x["cos"], x["sin"], pos, spec["order"])
                rows = spec["cache_len"][b] + np.arange(S)
                err = max(err, float(np.abs(out["k_cache"][b, g, rows] - ref).max()))
                assert np.array_equal(out["v_cache"][b, g, rows], qkv[b, :, Hq + Hkv + g])
        assert err <= (6e-2 if dt == "bf16" else 2e-5), (name, err)   # bf16: values up to ~4, a few ulps
        return err
    if k == "decode":
        B, Hq, Hkv = spec["B"], spec["Hq"], spec["Hkv"]
        err = 0.0
        for b in range(B):
            L = spec["lens"][b]
            for h in range(Hq):
                g = h // (Hq // Hkv)
                ref = f64_attention(x["q"][b, h][None], x["k"][b, g, :L], x["v"][b, g, :L], np.ones((1, L), bool))
                err = max(err, float(np.abs(out["out"][b, h * D:(h + 1) * D] - ref[0]).max()))
        assert err <= bar, (name, err)
        return err
    if k == "prefill":
        B, S, Hq, Hkv = spec["B"], spec["S"], spec["Hq"], spec["Hkv"]
        o = out["out"].reshape(B, S, Hq, D)
        err = 0.0
        for b in range(B):
            st = spec["start"][b]
            L = st + S
            allowed = np.arange(L)[None, :] <= (st + np.arange(S))[:, None]
            for h in range(Hq):
                g = h // (Hq // Hkv)
                ref = f64_attention(x["q"][b, h], x["k"][b, g, :L], x["v"][b, g, :L], allowed)
                err = max(err, float(np.abs(o[b, :, h] - ref).max()))
        assert err <= 2.5e-2 if dt == "bf16" else err <= bar, (name, err)
        return err
    raise ValueError(k)


def main():
    oracle.build()
    arrays = {}
    for name, spec in CASES.items():
        out = run_oracle(oracle, spec)
        err = check(name, spec, out)
        print(f"{name:28s} max |oracle - float64| = {err:.3e}")
        arrays[f"{name}.spec"] = np.frombuffer(json.dumps(spec, sort_keys=True).encode(), dtype=np.uint8)
        for key, val in out.items():
            arrays[f"{name}.{key}"] = np.ascontiguousarray(val)
    np.savez_compressed(OUT, **arrays)
    print(f"wrote {OUT} ({os.path.getsize(OUT)} bytes)")


if __name__ == "__main__":
    main()
