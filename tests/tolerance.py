"""Parity bars of the north star: f32 max-abs <= 1e-4; bf16 (f32 accumulation)
max-abs <= 2e-2 and mean-relative <= 1e-2, mean-relative = mean|x-ref| / mean|ref|."""
import numpy as np

F32_MAX_ABS = 1e-4
BF16_MAX_ABS = 2e-2
BF16_MEAN_REL = 1e-2


def errors(x, ref):
    x = np.asarray(x, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    assert x.shape == ref.shape, (x.shape, ref.shape)
    d = np.abs(x - ref)
    max_abs = float(d.max()) if d.size else 0.0
    denom = float(np.abs(ref).mean()) if ref.size else 1.0
    mean_rel = float(d.mean() / denom) if denom > 0 else float(d.mean())
    return max_abs, mean_rel


def assert_close(x, ref, dtype: str, what: str = ""):
    max_abs, mean_rel = errors(x, ref)
    assert np.all(np.isfinite(np.asarray(x, dtype=np.float64))), f"{what}: non-finite output"
    if dtype == "f32":
        assert max_abs <= F32_MAX_ABS, f"{what}: f32 max-abs {max_abs:.3e} > {F32_MAX_ABS}"
    else:
        assert max_abs <= BF16_MAX_ABS and mean_rel <= BF16_MEAN_REL, (
            f"{what}: bf16 max-abs {max_abs:.3e} (<= {BF16_MAX_ABS}), mean-rel {mean_rel:.3e} "
            f"(<= {BF16_MEAN_REL})")
    return max_abs, mean_rel


def bf16_ulp(x):
    """Spacing of bf16 values at |x| (2^(e-7) for x in [2^e, 2^(e+1)))."""
    a = np.abs(np.asarray(x, dtype=np.float32))
    e = np.floor(np.log2(np.maximum(a, np.float32(2.0 ** -126))))
    return np.exp2(e - 7)


def assert_ulp_close(x, ref, dtype: str, what: str = "", min_exact: float = 0.9999):
    """Element-wise parity for the fused append, which reproduces candle's
    rounding points: bf16 bit-identical almost everywhere (the f32 sum of
    squares is summed in another order, which can move a normalised value by
    one ulp; RoPE then carries that ulp, of a value below 16, into the output),
    so a differing element may be off by at most one bf16 ulp at 8 (2^-4); f32
    within the f32 parity bar.  The bit-identical share is min_exact, or all
    but two head rows of 128 elements when that is less strict: where candle
    rounds the row's RMS to bf16 (the Hunyuan order, and Qwen3 decode), a
    different summation order now and then moves that rounded value by one
    ulp, and then many of the row's outputs by one ulp (a tensor of a few
    hundred rows cannot hold 99.99% then: 31 of 66560 K elements in one seeded
    draw of 520 rows)."""
    x = np.asarray(x, dtype=np.float32)
    ref = np.asarray(ref, dtype=np.float32)
    assert np.all(np.isfinite(x)), f"{what}: non-finite output"
    exact = float(np.mean(x == ref))
    if dtype == "f32":
        assert float(np.abs(x - ref).max()) <= F32_MAX_ABS, what
    else:
        d = np.abs(x.astype(np.float64) - ref)
        assert np.all(d <= bf16_ulp(np.maximum(np.abs(ref), 8.0))), f"{what}: differs by more than 2^-4"
        allowed = max((1.0 - min_exact) * x.size, 2 * 128)
        assert float(np.sum(x != ref)) <= allowed, f"{what}: only {exact:.5f} of elements bit-identical"
    return exact
