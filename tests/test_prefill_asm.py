"""The generated assembly of the bf16 prefill's key loop (prefill_step.inc),
executed on the CPU by the asm_sim interpreter inside a numpy restatement of
the kernel around it (prefill_asm_harness), against the model of the kernel's
arithmetic (test_prefill_rounding.kernel_model) and candle's chain (the
oracle).  These run without a GPU: they pin the assembly's data flow (the
register map, the fragment ring, the lazy rescale and its redo, the masks,
the flags of each step) before any GPU run; the GPU tests compare the kernel
itself with the same model."""
from __future__ import annotations

import numpy as np
import pytest

import cases
import prefill_asm_harness as harness
import test_prefill_rounding as rounding
from tolerance import BF16_MAX_ABS, BF16_MEAN_REL

# (B, S, Hq, Hkv, starts, causal, cus, q_gain, one_rounding)
CASES = [
    (1, 192, 2, 1, (0,), True, 256, 4.0, False),        # causal from 0, GQA 2:1, diagonal tiles
    (1, 160, 1, 1, (70,), True, 1, 4.0, False),         # key split between two wave groups, ragged start
    (2, 96, 2, 2, (0, 37), True, 256, 1.0, False),      # two sequences at different starts
    (1, 100, 1, 1, (30,), False, 256, 4.0, False),      # non-causal, partial last tile
    (1, 128, 1, 1, (0,), True, 256, 16.0, False),       # large scores: the redo path runs often
    (1, 64, 1, 1, (1040,), True, 256, 1.0, True),       # long rows, first rounding only (N(0, 1) scores)
    (1, 64, 1, 1, (1040,), True, 256, 4.0, False),      # the same rows with both roundings
]


def _draw(B, S, Hq, Hkv, starts, q_gain, seed):
    rng = np.random.default_rng(seed)
    L = max(starts) + S
    q = cases.bf16(q_gain * rng.standard_normal((B, Hq, S, 128), dtype=np.float32))
    k = cases.bf16(rng.standard_normal((B, Hkv, L, 128), dtype=np.float32))
    v = cases.bf16(rng.standard_normal((B, Hkv, L, 128), dtype=np.float32))
    return q, k, v, np.asarray(starts, np.int32)


@pytest.mark.parametrize("case", range(len(CASES)))
def test_assembly_is_the_model(orc, case):
    B, S, Hq, Hkv, starts, causal, cus, q_gain, one_rounding = CASES[case]
    q, k, v, st = _draw(B, S, Hq, Hkv, starts, q_gain, seed=100 + case)
    with np.errstate(invalid="ignore", over="ignore"):
        got = harness.simulate(q, k, v, st, causal, one_rounding=one_rounding, cus=cus)
    old = rounding.CUS
    rounding.CUS = cus
    try:
        model = rounding.kernel_model(q, k, v, st, causal,
                                      long_row_keys=rounding.LONG_ROW_KEYS if one_rounding else None)
    finally:
        rounding.CUS = old
    d = np.abs(got.astype(np.float64) - model)
    # the model sums in another order than the lanes do: a few f32 ties round apart
    assert float(np.mean(got == model)) >= 0.99 and np.all(d <= 2.0 ** -6), (case, float(d.max()))
    ref = orc.attn_prefill(q, k, v, st, cases.scale(), causal=causal, dtype="bf16")
    dr = np.abs(got.astype(np.float64) - ref)
    assert dr.max() <= BF16_MAX_ABS and dr.mean() / np.abs(ref).mean() <= BF16_MEAN_REL


def test_one_rounding_switch_changes_long_rows_only(orc):
    """The long-row switch is in effect only where the rows see at least
    kLongRowKeys keys: a short-row draw is the same with and without it."""
    q, k, v, st = _draw(1, 128, 1, 1, (0,), 4.0, seed=7)
    with np.errstate(invalid="ignore", over="ignore"):
        a = harness.simulate(q, k, v, st, True, one_rounding=False)
        b = harness.simulate(q, k, v, st, True, one_rounding=True)
    np.testing.assert_array_equal(a, b)
    q, k, v, st = _draw(1, 64, 1, 1, (1040,), 4.0, seed=8)
    with np.errstate(invalid="ignore", over="ignore"):
        a = harness.simulate(q, k, v, st, True, one_rounding=False)
        b = harness.simulate(q, k, v, st, True, one_rounding=True)
    assert np.any(a != b)
