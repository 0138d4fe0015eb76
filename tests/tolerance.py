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
