"""Randomised shapes for decode, prefill and the fused append against the
oracle: a fixed list of seeded draws over batch, head counts (every GQA group
size 1..8 and 16), lengths around the chunk and tile boundaries (including the
12288-key switch to 512-key decode chunks), continuation starts, causal and
non-causal prefill, and both dtypes.  Sizes stay small enough for the oracle
to finish in seconds.  Bars as everywhere: f32 max-abs <= 1e-4; bf16 max-abs
<= 2e-2 and mean-rel <= 1e-2.  Rows and pool entries the kernels must not
read are NaN (the case generators poison them).

The draw counts and a seed offset can be raised from the environment for a
wider sweep (CRANE_RANDOM_DECODE, CRANE_RANDOM_PREFILL, CRANE_RANDOM_APPEND,
CRANE_RANDOM_PREFILL_LONG, CRANE_RANDOM_SEED); the defaults are the committed
24 / 20 / 12 / 10 draws at offset 0."""

import os

import numpy as np
import pytest

import cases
from tolerance import assert_close, errors

pytestmark = pytest.mark.gpu

D = 128
N_DECODE = int(os.environ.get("CRANE_RANDOM_DECODE", 24))
N_PREFILL = int(os.environ.get("CRANE_RANDOM_PREFILL", 20))
N_APPEND = int(os.environ.get("CRANE_RANDOM_APPEND", 12))
N_PREFILL_LONG = int(os.environ.get("CRANE_RANDOM_PREFILL_LONG", 10))
SEED = int(os.environ.get("CRANE_RANDOM_SEED", 0))


def _heads(r):
    n_rep = int(r.choice([1, 2, 3, 4, 5, 6, 7, 8, 16]))
    hkv = int(r.choice([1, 2, 4]))
    return n_rep * hkv, hkv


def _t(x, dtype, dev):
    import torch
    t = torch.from_numpy(np.ascontiguousarray(x))
    return (t.to(torch.bfloat16) if dtype == "bf16" else t).to(dev).contiguous()


def _len(r, long_ok):
    # near a 64/256/512 boundary, or anywhere; now and then past 12288
    if long_ok and r.random() < 0.2:
        return int(r.integers(12280, 14000))
    edge = int(r.choice([64, 256, 512, 1024]))
    return max(1, int(r.choice([edge * int(r.integers(1, 5)) + int(r.integers(-2, 3)), int(r.integers(1, 2500))])))


@pytest.mark.parametrize("i", range(N_DECODE))
def test_random_decode(gpu, orc, i):
    import torch
    from crane_amd import ops
    r = cases.rng(SEED + 7100 + i)
    dtype = "f32" if i % 4 == 3 else "bf16"
    Hq, Hkv = _heads(r)
    B = int(r.integers(1, 6))
    lens = np.array([_len(r, Hq * B <= 64) for _ in range(B)], np.int32)
    if r.random() < 0.15:
        lens[int(r.integers(0, B))] = 0  # an empty sequence
    if lens.max() == 0:
        lens[0] = 1
    mode = "standard" if i % 3 == 2 else None  # every third draw takes Qwen2.5's form
    print(f"random decode {i}: B={B} Hq={Hq} Hkv={Hkv} lens={lens.tolist()} {dtype} mode={mode}", flush=True)
    q, k, v, lens = cases.decode_case(SEED + 7200 + i, B, Hq, Hkv, lens, dtype=dtype)
    out = ops.attention_decode(_t(q, dtype, gpu), _t(k, dtype, gpu), _t(v, dtype, gpu),
                               torch.as_tensor(lens, device=gpu), int(lens.max()), cases.scale(), score_mode=mode)
    torch.cuda.synchronize()
    got = out.float().cpu().numpy().reshape(B, Hq * D)
    ref = orc.attn_decode(q, k, v, lens, cases.scale(), dtype, cases.decode_variant(orc, Hq, Hkv, mode))
    for b in range(B):
        if lens[b] == 0:
            assert np.all(got[b] == 0), "an empty sequence's row is zero"
    keep = lens > 0
    print(f"  errors {errors(got[keep], ref[keep])}", flush=True)
    assert_close(got[keep], ref[keep], dtype, f"random decode {i}")


@pytest.mark.parametrize("i", range(N_PREFILL))
def test_random_prefill(gpu, orc, i):
    _prefill_draw(gpu, orc, SEED, i)


# Draws of the seed-offset-10000 sweep on which a kernel without candle's
# second score rounding and its bf16 softmax of few-key rows missed the 2e-2
# bar by one bf16 ulp at |x| >= 2 (rows with 2-8 keys, and one row of the
# key-split variant).  Kept as fixed cases.
@pytest.mark.parametrize("i", [7, 28, 70, 102])
def test_prefill_rounding_tail_draws(gpu, orc, i):
    _prefill_draw(gpu, orc, 10000, i)


# Continuation chunks over caches of 900-3600 rows: the workgroups whose rows
# see at least 1024 keys keep candle's first score rounding only.
@pytest.mark.parametrize("i", range(N_PREFILL_LONG))
def test_random_prefill_long_rows(gpu, orc, i):
    _prefill_draw(gpu, orc, SEED, i, cases.prefill_long_draw)


def _prefill_draw(gpu, orc, seed, i, draw=cases.prefill_draw):
    import torch
    from crane_amd import ops
    (dtype, B, S, Hq, Hkv, start, causal), (q, k, v, st) = draw(seed, i)
    print(f"random prefill {i}: B={B} S={S} Hq={Hq} Hkv={Hkv} start={start} causal={causal} {dtype}", flush=True)
    out = ops.attention_prefill(_t(q, dtype, gpu), _t(k, dtype, gpu), _t(v, dtype, gpu),
                                torch.as_tensor(st, device=gpu), int(st.max()), cases.scale(), causal)
    torch.cuda.synchronize()
    got = out.float().cpu().numpy()
    ref = orc.attn_prefill(q, k, v, st, cases.scale(), causal, dtype)
    print(f"  errors {errors(got, ref)}", flush=True)
    assert_close(got, ref, dtype, f"random prefill {i}")


@pytest.mark.parametrize("i", range(N_APPEND))
def test_random_append(gpu, orc, i):
    """Fused append at random shapes, orders, positions and cache lengths:
    q and the written K rows ulp-close to the oracle, V rows copied exactly,
    every other cache row untouched."""
    import torch
    from crane_amd import ops
    from tolerance import assert_ulp_close
    r = cases.rng(SEED + 7500 + i)
    dtype = "f32" if i % 4 == 3 else "bf16"
    Hq, Hkv = _heads(r)
    B = int(r.integers(1, 5))
    S = int(r.choice([1, 1, 7, 64, int(r.integers(1, 300))]))
    order = int(r.integers(0, 3))
    clen = [int(r.integers(0, 200)) for _ in range(B)]
    posn = [c + int(r.integers(0, 50)) for c in clen]
    cap = max(clen) + S + int(r.integers(0, 20))
    print(f"random append {i}: B={B} S={S} Hq={Hq} Hkv={Hkv} order={order} clen={clen} pos={posn} {dtype}",
          flush=True)
    qkv = cases.cast(cases.normal(r, (B, S, (Hq + 2 * Hkv) * D)), dtype)
    qw = cases.cast(1 + 0.1 * cases.normal(r, (D,)), dtype) if order != 2 else None
    kw = cases.cast(1 + 0.1 * cases.normal(r, (D,)), dtype) if order != 2 else None
    cos, sin = (cases.cast(t, dtype) for t in orc.rope_tables(D, 1e6, 1024))  # covers every position drawn
    kc = np.full((B, Hkv, cap, D), 3.0, np.float32)
    vc = np.full((B, Hkv, cap, D), 3.0, np.float32)
    kd, vd = _t(kc, dtype, gpu), _t(vc, dtype, gpu)
    q = ops.qk_norm_rope_append(_t(qkv, dtype, gpu), _t(cos, dtype, gpu), _t(sin, dtype, gpu),
                                torch.as_tensor(np.array(posn, np.int32), device=gpu), kd, vd,
                                torch.as_tensor(np.array(clen, np.int32), device=gpu), max(clen) + S, Hq, Hkv,
                                None if qw is None else _t(qw, dtype, gpu), None if kw is None else _t(kw, dtype, gpu),
                                1e-6, ["norm_then_rope", "rope_then_norm", "rope_only"][order])
    torch.cuda.synchronize()
    q_ref = orc.qk_norm_rope_append(qkv, Hq, Hkv, cos, sin, np.array(posn, np.int32), kc, vc,
                                    np.array(clen, np.int32), qw, kw, 1e-6, order, dtype)
    assert_ulp_close(q.float().cpu().numpy(), q_ref, dtype, f"random append {i} q")
    assert_ulp_close(kd.float().cpu().numpy(), kc, dtype, f"random append {i} k")
    assert np.array_equal(vd.float().cpu().numpy(), vc), "value rows are copies; other rows untouched"
