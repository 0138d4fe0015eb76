"""Decoder-layer row kernels (include/crane_layer.h): RmsNorm, residual add +
RmsNorm, SiLU(gate) * up, residual add -- the candle ops and Crane fused ops
around the attention block (qwen3/modeling.rs:655-673, crane-core/src/fused_ops).

CPU: the oracle's new functions are pinned to torch (float64) and to exact
rounding bounds, and the launchers' argument checks return the documented
codes.  GPU: each kernel against the oracle on the hidden/intermediate sizes of
the supported models."""
import ctypes

import numpy as np
import pytest

import cases
from tolerance import BF16_MEAN_REL, assert_close, assert_ulp_close, bf16_ulp, errors

# (rows, cols): Qwen3-8B decode batch, Qwen2.5-7B, Qwen2.5-72B, Qwen3-0.6B, tiny rows
# (rows, cols): fewer than 1024 rows take a workgroup per row, more a wave per row
NORM_SHAPES = [(32, 4096), (257, 3584), (4, 8192), (1031, 2048), (3, 1024), (5, 8)]
# (rows, intermediate): Qwen3-8B, Qwen2.5-7B, tiny
MLP_SHAPES = [(32, 12288), (9, 18944), (3, 8)]


def _gen(seed, shape, std=1.0, dtype="bf16"):
    return cases.cast(cases.normal(cases.rng(seed), shape, std), dtype)


# ------------------------------------------------------------------ CPU: oracle pins

def test_silu_mul_oracle_vs_torch_float64(orc):
    """Both oracle forms lie within half a bf16 ulp (one rounding) of torch's
    float64 silu(g) * u, the f64 form exactly so; swapping gate and up, or
    sigmoid for silu, would fail."""
    import torch
    gu = _gen(1, (64, 2 * 512), 3.0)
    g, u = gu[:, :512].astype(np.float64), gu[:, 512:].astype(np.float64)
    exact = (torch.nn.functional.silu(torch.from_numpy(g)) * torch.from_numpy(u)).numpy()
    half_ulp = 0.5 * bf16_ulp(exact)
    f64 = orc.silu_mul(gu, True, "bf16")
    f32 = orc.silu_mul(gu, False, "bf16")
    assert np.all(np.abs(f64 - exact) <= half_ulp * (1 + 1e-12))
    assert np.all(np.abs(f32 - exact) <= half_ulp * 1.001 + 1e-30)
    assert np.mean(f32 == f64) > 0.999
    assert np.array_equal(f64, orc.round_bf16(f64))
    swapped = (torch.nn.functional.silu(torch.from_numpy(u)) * torch.from_numpy(g)).numpy()
    assert np.mean(np.abs(f64 - swapped) > half_ulp) > 0.5
    # f32 forms agree with the float64 value to f32 precision
    e32 = orc.silu_mul(gu, False, "f32")
    assert np.max(np.abs(e32 - exact) / np.maximum(np.abs(exact), 1e-30)) < 1e-6


def test_silu_mul_oracle_special_values(orc):
    g = np.array([0.0, -0.0, 40.0, -200.0, 1.0, -1.0, 88.0, -88.0], np.float32)
    u = np.array([3.0, 3.0, 0.5, 7.0, 2.0, 2.0, 1.0, 1.0], np.float32)
    gu = np.concatenate([g, u])[None]
    for f64 in (False, True):
        y = orc.silu_mul(gu, f64, "f32")[0]
        assert y[0] == 0.0 and y[1] == 0.0                      # silu(0) = 0
        assert y[2] == 20.0 and y[6] == 88.0                    # silu(x) = x for large x
        assert y[3] == 0.0 and abs(y[7]) < 1e-30                # silu(x) -> 0 for very negative x
        assert abs((y[4] - y[5]) / 2.0 - 1.0) < 1e-6            # silu(x) - silu(-x) = x


def test_residual_add_oracle(orc):
    r = _gen(2, (7, 3584), 4.0)
    h = _gen(3, (7, 3584), 4.0)
    np.testing.assert_array_equal(orc.residual_add(r, h, "bf16"), cases.bf16(r + h))
    np.testing.assert_array_equal(orc.residual_add(r, h, "f32"), r + h)
    # with hidden = 0 the pair reduces to RmsNorm of the residual
    new_r, y = orc.add_rms_norm(r, np.zeros_like(r), None, 1e-6, "bf16")
    np.testing.assert_array_equal(new_r, r)
    np.testing.assert_array_equal(y, orc.rms_norm(r, None, 1e-6, True, "bf16"))


def test_rms_norm_oracle_hidden_sizes(orc):
    """The norm at hidden sizes (4096 and 8192 wide rows) stays within the
    candle bound of the float64 formula (m rounded to bf16, then x/m and the
    weight product rounded)."""
    for cols in (4096, 8192):
        x = _gen(4, (8, cols), 2.0)
        w = _gen(5, (cols,), 0.5) + np.float32(1.0)
        w = cases.bf16(w)
        y = orc.rms_norm(x, w, 1e-6, True, "bf16")
        x64 = x.astype(np.float64)
        ref = x64 / np.sqrt((x64 ** 2).mean(-1, keepdims=True) + 1e-6) * w
        assert np.all(np.abs(y - ref) <= 3 * bf16_ulp(ref) + 1e-30)


# ------------------------------------------------------------------ CPU: launcher checks

def test_layer_argument_checks():
    from crane_amd import _lib
    L = _lib.lib()
    assert L.crane_hip_rms_norm(16, None, 32, 4, 4096, 1e-6, 3, None) == _lib.E_DTYPE
    assert L.crane_hip_rms_norm(16, None, 32, 4, 4100, 1e-6, 1, None) == _lib.E_ALIGN      # not 8 | cols
    assert L.crane_hip_rms_norm(16, None, 32, 4, 8200, 1e-6, 1, None) == _lib.E_INVALID    # > max cols
    assert L.crane_hip_rms_norm(None, None, 32, 4, 4096, 1e-6, 1, None) == _lib.E_INVALID
    assert L.crane_hip_rms_norm(8, None, 32, 4, 4096, 1e-6, 1, None) == _lib.E_ALIGN
    assert L.crane_hip_rms_norm(16, None, 32, 0, 4096, 1e-6, 1, None) == _lib.OK           # no rows
    assert L.crane_hip_rms_norm(16, None, 32, 4, 4096, -1.0, 1, None) == _lib.E_INVALID    # eps
    assert L.crane_hip_add_rms_norm(16, 48, None, 16, 4, 4096, 1e-6, 1, None) == _lib.E_INVALID  # out aliases
    assert L.crane_hip_silu_mul(16, 32, 4, 12, 1, None) == _lib.E_ALIGN
    assert L.crane_hip_silu_mul(16, 32, 4, 0, 1, None) == _lib.E_INVALID
    assert L.crane_hip_silu_mul(16, 32, 4, 10, 0, None) == _lib.E_ALIGN                   # f32: 4 | inter
    assert L.crane_hip_silu_mul(16, 32, 0, 16, 1, None) == _lib.OK                      # no rows
    assert L.crane_hip_residual_add(16, 32, 12, 1, None) == _lib.E_ALIGN
    assert L.crane_hip_residual_add(16, 32, -8, 1, None) == _lib.E_INVALID
    assert L.crane_hip_residual_add(16, 32, 0, 1, None) == _lib.OK


# ------------------------------------------------------------------ GPU

def _t(x, dtype, dev):
    import torch
    t = torch.from_numpy(np.ascontiguousarray(x))
    return (t.to(torch.bfloat16) if dtype == "bf16" else t).to(dev)


def _np(t):
    return t.float().cpu().numpy()


def _norm_bar(got, ref, dtype, what):
    """The norms' bar besides assert_ulp_close (one bf16 ulp at max(|ref|, 8)
    per element, 99.9% bit-identical): f32 max-abs, bf16 mean-relative.  The
    bf16 max-abs 2e-2 does not apply: a normed row reaches |v| >= 4, where one
    ulp is 2^-5 > 2e-2, and the f32 sum of squares (summed in another order
    than the oracle's) can move a row's norm, hence all of its values, by an
    ulp."""
    if dtype == "f32":
        assert_close(got, ref, dtype, what)
    else:
        assert errors(got, ref)[1] <= BF16_MEAN_REL, what


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", ["bf16", "f32"])
@pytest.mark.parametrize("rows,cols", NORM_SHAPES)
def test_rms_norm_parity(gpu, orc, dtype, rows, cols):
    from crane_amd import ops
    print(f"rms_norm {dtype} {rows}x{cols}", flush=True)
    x = _gen(100 + cols, (rows, cols), 2.0, dtype)
    w = cases.cast(_gen(101 + cols, (cols,), 0.3, "f32") + np.float32(1.0), dtype)
    got = _np(ops.rms_norm(_t(x, dtype, gpu), _t(w, dtype, gpu)))
    ref = orc.rms_norm(x, w, 1e-6, True, dtype)
    assert_ulp_close(got, ref, dtype, f"rms_norm {rows}x{cols}", min_exact=0.999)
    _norm_bar(got, ref, dtype, f"rms_norm {rows}x{cols}")
    got1 = _np(ops.rms_norm(_t(x, dtype, gpu)))                          # no weight = weight 1
    assert_ulp_close(got1, orc.rms_norm(x, None, 1e-6, True, dtype), dtype, "rms_norm w=1", min_exact=0.999)


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", ["bf16", "f32"])
@pytest.mark.parametrize("rows,cols,splits", [(32, 4096, 4), (3, 1024, 2), (1, 8192, 8), (5, 2560, 3)])
def test_add_rms_norm_parts_parity(gpu, orc, dtype, rows, cols, splits):
    """add_rms_norm of split-K partial products (ops.PartialProduct): the
    residual becomes T(residual + T(sum of the splits in split order)), bit
    for bit, and the norm is the oracle's add + norm of that rounded sum."""
    import torch
    from crane_amd import ops
    print(f"add_rms_norm of {splits} partial products, {dtype} {rows}x{cols}", flush=True)
    r = _gen(300 + cols, (rows, cols), 3.0, dtype)
    parts = _gen(301 + cols, (splits, rows, cols), 0.5, "f32")
    w = cases.cast(_gen(302 + cols, (cols,), 0.3, "f32") + np.float32(1.0), dtype)
    acc = np.zeros((rows, cols), np.float32)
    for p in parts:
        acc = (acc + p).astype(np.float32)
    h = cases.cast(acc, dtype)
    rt = _t(r, dtype, gpu)
    pp = ops.PartialProduct(torch.from_numpy(parts).to(gpu), torch.bfloat16 if dtype == "bf16" else torch.float32)
    got = _np(ops.add_rms_norm(rt, pp, _t(w, dtype, gpu)))
    new_r, ref = orc.add_rms_norm(r, h, w, 1e-6, dtype)
    np.testing.assert_array_equal(_np(rt), new_r)
    assert_ulp_close(got, ref, dtype, f"add_rms_norm parts {rows}x{cols}", min_exact=0.999)
    _norm_bar(got, ref, dtype, f"add_rms_norm parts {rows}x{cols}")


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", ["bf16", "f32"])
@pytest.mark.parametrize("rows,cols", NORM_SHAPES[:4])
def test_add_rms_norm_parity(gpu, orc, dtype, rows, cols):
    """The residual is updated bit-exactly (rounded sum), the norm is of that
    rounded sum."""
    from crane_amd import ops
    print(f"add_rms_norm {dtype} {rows}x{cols}", flush=True)
    r = _gen(200 + cols, (rows, cols), 3.0, dtype)
    h = _gen(201 + cols, (rows, cols), 1.0, dtype)
    w = cases.cast(_gen(202 + cols, (cols,), 0.3, "f32") + np.float32(1.0), dtype)
    rt = _t(r, dtype, gpu)
    got = _np(ops.add_rms_norm(rt, _t(h, dtype, gpu), _t(w, dtype, gpu)))
    new_r, ref = orc.add_rms_norm(r, h, w, 1e-6, dtype)
    np.testing.assert_array_equal(_np(rt), new_r)
    assert_ulp_close(got, ref, dtype, f"add_rms_norm {rows}x{cols}", min_exact=0.999)
    _norm_bar(got, ref, dtype, f"add_rms_norm {rows}x{cols}")


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", ["bf16", "f32"])
@pytest.mark.parametrize("rows,inter", MLP_SHAPES)
def test_silu_mul_parity(gpu, orc, dtype, rows, inter):
    """Against the f32 formula of Crane's kernel (bit-exact up to the last-ulp
    differences of two correctly rounded-ish expf implementations) and against
    its f64 cpu_fwd (parity bar)."""
    from crane_amd import ops
    print(f"silu_mul {dtype} {rows}x{inter}", flush=True)
    gu = _gen(300 + inter, (rows, 2 * inter), 3.0, dtype)
    got = _np(ops.silu_mul(_t(gu, dtype, gpu)))
    assert_ulp_close(got, orc.silu_mul(gu, False, dtype), dtype, f"silu_mul {rows}x{inter}", min_exact=0.999)
    assert_close(got, orc.silu_mul(gu, True, dtype), dtype, f"silu_mul f64 {rows}x{inter}")


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_silu_mul_special_values(gpu, orc, dtype):
    """Zeros, large and very negative gates; in bf16 the values below -80 take
    the kernel's exact fallback (the hardware reciprocal of 1 + e^-g would
    flush to zero there)."""
    from crane_amd import ops
    g = np.array([0.0, -0.0, 40.0, -200.0, 1.0, -1.0, 88.0, -88.0], np.float32)
    u = np.array([3.0, 3.0, 0.5, 7.0, 2.0, 2.0, 1.0, 1.0], np.float32)
    gu = np.concatenate([g, u])[None]
    got = _np(ops.silu_mul(_t(gu, dtype, gpu)))
    np.testing.assert_array_equal(got, orc.silu_mul(gu, False, dtype))


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", ["bf16", "f32"])
def test_residual_add_parity(gpu, orc, dtype):
    from crane_amd import ops
    r = _gen(400, (33, 3584), 4.0, dtype)
    h = _gen(401, (33, 3584), 4.0, dtype)
    rt = _t(r, dtype, gpu)
    ops.residual_add(rt, _t(h, dtype, gpu))
    np.testing.assert_array_equal(_np(rt), orc.residual_add(r, h, dtype))
