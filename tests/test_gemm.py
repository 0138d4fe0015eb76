"""The projections of a decoder layer (include/crane_gemm.h): candle Linear
y = x W^T + b -- Crane's merged qkv_proj, whose rows feed the fused append
(qwen3/modeling.rs:382-387; with the Qwen2.5 bias, qwen25/qwen2.rs:136-138),
o_proj (:466, :502), the MLP projections and the lm_head; on hipBLASLt, or on
the per-wave ring and streaming kernels for decode-shaped bf16 products.

The oracle's linear is pinned to numpy float64 matmul (a transposed weight
fails); the GPU is held to the oracle within the rounding bound of its two
differences (f32 accumulation in another order, and one rounding of product
+ bias where candle rounds twice) and the mean-relative bar, with weights
scaled like trained ones (std 1/sqrt(K)) so outputs are O(1)."""
import math
import os

import numpy as np
import pytest

import cases
from tolerance import assert_close, assert_ulp_close, bf16_ulp


def assert_linear_close(got, x, w, bias, dtype, orc, what):
    """Two references.  Against the oracle with the GPU's rounding (product +
    bias rounded once) every element lies within the f32 accumulation bound,
    K * 2^-24 * sum|x||w| (any summation order) plus one ulp, and at least 99%
    of them are bit-identical.  Against candle's (product rounded, then the
    sum) the two roundings differ by at most half an ulp at |p| plus an ulp at
    |y|: elements within 1.5 ulp of max(|y|, |p|, |b|) plus the accumulation
    bound, and the mean-relative bar.  f32: the f32 bar."""
    ref = orc.linear(x, w, bias, dtype)
    if dtype == "f32":
        return assert_close(got, ref, dtype, what)
    K = x.shape[-1]
    acc = (K * 2.0 ** -24) * (np.abs(x.astype(np.float64)) @ np.abs(w.astype(np.float64)).T)
    fused = orc.linear(x, w, bias, dtype, fused=True)
    d = np.abs(got.astype(np.float64) - fused)
    assert np.all(d <= acc + bf16_ulp(fused)), f"{what}: beyond the accumulation bound"
    exact = float(np.mean(got == fused))
    assert exact >= 0.99, f"{what}: only {exact:.4f} bit-identical to the fused-rounding oracle"
    b = np.zeros(ref.shape[-1], np.float32) if bias is None else bias
    scale = np.maximum(np.maximum(np.abs(ref), np.abs(ref - b)), np.abs(b))
    d2 = np.abs(got.astype(np.float64) - ref)
    assert np.all(d2 <= 1.5 * bf16_ulp(scale) + acc), f"{what}: beyond the candle rounding bound"
    from tolerance import errors, BF16_MEAN_REL
    assert errors(got, ref)[1] <= BF16_MEAN_REL, what


def _case(seed, M, N, K, dtype, bias=True):
    r = cases.rng(seed)
    x = cases.cast(cases.normal(r, (M, K)), dtype)
    w = cases.cast(cases.normal(r, (N, K), 1.0 / math.sqrt(K)), dtype)
    b = cases.cast(cases.normal(r, (N,), 0.5), dtype) if bias else None
    return x, w, b


# ------------------------------------------------------------------ CPU

def test_linear_oracle_vs_numpy_float64(orc):
    x, w, b = _case(1, 37, 96, 640, "bf16")
    exact = x.astype(np.float64) @ w.astype(np.float64).T
    y32 = orc.linear(x, w, None, "f32")
    assert np.max(np.abs(y32 - exact) / np.maximum(np.abs(exact), 1e-6)) < 1.5e-7
    yb = orc.linear(x, w, None, "bf16")
    assert np.all(np.abs(yb - exact) <= 0.5 * bf16_ulp(exact) * (1 + 1e-9))   # one rounding
    ybb = orc.linear(x, w, b, "bf16")
    np.testing.assert_array_equal(ybb, cases.bf16(yb + b[None, :]))          # then the bias in T
    wrong = orc.linear(x, np.ascontiguousarray(w[:, ::-1]), None, "f32")      # a planted mistake
    assert np.max(np.abs(wrong - exact)) > 0.5
    fb = orc.linear(x, w, b, "bf16", fused=True)                               # epilogue rounding
    assert np.all(np.abs(fb - (exact + b)) <= 0.5 * bf16_ulp(exact + b) * (1 + 1e-9))


def test_gemm_null_context():
    from crane_amd import _lib
    assert _lib.lib().crane_gemm_linear(None, 16, 16, None, 16, 4, 4, 4, 1, None) == _lib.E_INVALID


def test_gated_shape_query():
    """Which shapes the one-launch gate_up + SiLU*mul takes (host logic, no
    GPU): bf16, at most 32 token rows, K <= 8192, inter > 4096 with inter a
    multiple of 48 (K of 512) or of 32 (K of 1024)."""
    from crane_amd import _lib
    q = _lib.lib().crane_gemm_silu_mul_supported
    BF16, F32 = 1, 0
    assert q(32, 12288, 4096, BF16) == 1      # Qwen3-8B decode gate_up
    assert q(1, 12288, 512, BF16) == 1
    assert q(3, 4160, 1024, BF16) == 1        # 32-feature pairs
    assert q(3, 4160, 512, BF16) == 0         # ... which need K % 1024
    assert q(33, 12288, 4096, BF16) == 0      # more token rows than the kernel takes
    assert q(0, 12288, 4096, BF16) == 0
    assert q(32, 4096, 4096, BF16) == 0       # narrow: the two-call path
    assert q(32, 12288, 4096, F32) == 0
    assert q(32, 12296, 4096, BF16) == 0      # inter a multiple of neither 48 nor 32
    assert q(32, 12288, 12288, BF16) == 0     # K past the ring kernel's limit
    assert _lib.lib().crane_gemm_linear_silu_mul(None, 16, 16, 16, 4, 12288, 4096, BF16, None) == _lib.E_INVALID


# ------------------------------------------------------------------ GPU

def _t(x, dtype, dev):
    import torch
    t = torch.from_numpy(np.ascontiguousarray(x))
    return (t.to(torch.bfloat16) if dtype == "bf16" else t).to(dev)


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", ["bf16", "f32"])
@pytest.mark.parametrize("M,N,K,bias", [
    (64, 4608, 3584, True),    # Qwen2.5-7B qkv_proj (28 q + 2 x 4 kv heads), with bias
    (32, 6144, 4096, False),   # Qwen3-8B qkv_proj at the c3 decode batch
    (300, 3584, 3584, False),  # Qwen2.5-7B o_proj
    (5, 136, 72, True),        # odd small shape
])
def test_linear_parity(gpu, orc, dtype, M, N, K, bias):
    from crane_amd import ops
    print(f"linear {dtype} M={M} N={N} K={K} bias={bias}", flush=True)
    x, w, b = _case(500 + N, M, N, K, dtype, bias)
    got = ops.linear(_t(x, dtype, gpu), _t(w, dtype, gpu), _t(b, dtype, gpu) if bias else None)
    assert_linear_close(got.float().cpu().numpy(), x, w, b, dtype, orc, f"linear {M}x{N}x{K}")
    # twice: the cached plan gives the same bits
    got2 = ops.linear(_t(x, dtype, gpu), _t(w, dtype, gpu), _t(b, dtype, gpu) if bias else None)
    assert bool((got == got2).all())


@pytest.mark.gpu
@pytest.mark.parametrize("M,N,K,bias", [
    (32, 16384, 1152, False),  # the decode batch of config 3; 9 stages of 128
    (17, 16448, 384, True),    # a partial second token group; 3 stages; 257 workgroups
    (8, 16384, 640, True),     # 5 stages: the unrolled-by-three loop's remainder of 2
    (1, 16384, 256, True),     # one token row; 2 stages
    (3, 20480, 128, False),    # one stage
])
def test_linear_streaming_parity(gpu, orc, M, N, K, bias):
    """Wide bf16 products with few token rows run the streaming kernel
    (M <= 32, N >= 16384, K a multiple of 128) when K is not a whole number of
    the per-wave ring kernel's pipelines (K % 1024 != 0 here); same bar as
    the library path."""
    from crane_amd import ops
    print(f"linear (streaming) M={M} N={N} K={K} bias={bias}", flush=True)
    x, w, b = _case(900 + M + K, M, N, K, "bf16", bias)
    got = ops.linear(_t(x, "bf16", gpu), _t(w, "bf16", gpu), _t(b, "bf16", gpu) if bias else None)
    assert_linear_close(got.float().cpu().numpy(), x, w, b, "bf16", orc, f"streaming linear {M}x{N}x{K}")
    got2 = ops.linear(_t(x, "bf16", gpu), _t(w, "bf16", gpu), _t(b, "bf16", gpu) if bias else None)
    assert bool((got == got2).all())


@pytest.mark.gpu
@pytest.mark.parametrize("M,N,K,bias", [
    (32, 4096, 4096, False),   # o_proj at the c3 decode batch: 16 features x 4 waves, 2 stages ahead
    (5, 4096, 2048, True),     # one token group; each wave's 4 stages fill the ring once (no loop trip)
    (3, 2048, 6144, True),     # 128 workgroups; 12 stages a wave
    (32, 6144, 4096, True),    # qkv_proj at c3: 32 features x 2 waves, rotated k walk (16 stages)
    (17, 8192, 1024, False),   # a partial second token group; 4 stages a wave, rotation over 4
    (32, 24576, 1024, True),   # gate_up's N: 96 features x 2 waves (256 workgroups), rotated k walk
    (32, 24576, 1536, False),  # ... K a multiple of 512, not of 1024: still 96 features (6 stages a wave)
    (32, 16384, 2048, True),   # 64 features x 4 waves (256 workgroups)
    (9, 9072, 1024, False),    # N a multiple of 48, not of 64: 48 features
    (1, 12288, 2048, False),   # one token row, wide (48 features: 256 workgroups)
    (32, 4096, 12288, False),  # down_proj's shape: K past the ring kernel's limit, hipBLASLt
])
def test_linear_ring_parity(gpu, orc, M, N, K, bias):
    """bf16 products with M <= 32 token rows, N a multiple of the workgroup's
    16/32 or 48/64/96 features (N <= 4096 / <= 8192 / wider) and K <= 8192 a
    whole number of the per-wave rings (K % 2048 == 0 for the narrowest, 1024
    or 512 for the others) run the per-wave ring kernel: the decode step's qkv_proj,
    o_proj, gate_up and lm_head.  Same bar as the library path, and a second
    call repeats the bits (the waves' partial products are added in a fixed
    order)."""
    from crane_amd import ops
    print(f"linear (ring) M={M} N={N} K={K} bias={bias}", flush=True)
    x, w, b = _case(1300 + M + N // 64 + K, M, N, K, "bf16", bias)
    got = ops.linear(_t(x, "bf16", gpu), _t(w, "bf16", gpu), _t(b, "bf16", gpu) if bias else None)
    assert_linear_close(got.float().cpu().numpy(), x, w, b, "bf16", orc, f"ring linear {M}x{N}x{K}")
    got2 = ops.linear(_t(x, "bf16", gpu), _t(w, "bf16", gpu), _t(b, "bf16", gpu) if bias else None)
    assert bool((got == got2).all())


def test_split_shape_query():
    """Which shapes the split-K partial products take (host logic, no GPU):
    bf16, at most 32 token rows, N a multiple of 32 or 48, K a multiple of the
    splits with a share of at most 32768 that is a multiple of 512 (of 256
    from 3072 up: one wave a workgroup), 2 to 16 splits."""
    from crane_amd import _lib
    q = _lib.lib().crane_gemm_split_supported
    BF16, F32 = 1, 0
    assert q(32, 4096, 4096, 4, BF16) == 1    # Qwen3-8B decode o_proj
    assert q(32, 4096, 12288, 4, BF16) == 1   # ... and down_proj
    assert q(1, 64, 2048, 2, BF16) == 1
    assert q(32, 6144, 4096, 2, BF16) == 1    # ... and qkv_proj
    assert q(32, 4096, 4096, 3, BF16) == 0    # K not a multiple of the splits
    assert q(32, 4096, 2048, 4, BF16) == 1    # 512 per split: one ring turn of 2 waves
    assert q(32, 4096, 1024, 4, BF16) == 0    # 256 per split: less than a ring turn
    assert q(32, 4096, 3840, 2, BF16) == 0    # 1920 per split (2 waves): not a multiple of 512
    assert q(32, 4096, 6656, 2, BF16) == 1    # 3328 per split (1 wave): a multiple of 256
    assert q(33, 4096, 4096, 4, BF16) == 0    # more token rows than the kernel takes
    assert q(32, 4100, 4096, 4, BF16) == 0    # N not a multiple of 32 or 48
    assert q(32, 4112, 4096, 4, BF16) == 0    # ... nor of 48
    assert q(32, 144, 4096, 4, BF16) == 1     # 3 tiles of 48 features
    assert q(32, 4096, 4096, 1, BF16) == 0    # no split
    assert q(32, 4096, 4096, 4, F32) == 0
    assert q(32, 4096, 65536, 2, BF16) == 1   # 32768 per split: the limit
    assert q(32, 4096, 131072, 2, BF16) == 0  # ... past it
    assert _lib.lib().crane_gemm_linear_split(None, 16, 16, 16, 4, 4096, 4096, 4, BF16, None) == _lib.E_INVALID


@pytest.mark.gpu
@pytest.mark.parametrize("M,N,K,splits", [
    (32, 4096, 4096, 4),    # o_proj at the c3 decode batch: 64 workgroups of 64 features x 4 splits, 2 waves
    (32, 4096, 12288, 4),   # down_proj at c3: 1 wave, 24 stages through a ring of 3
    (32, 6144, 4096, 2),    # qkv_proj at c3: 128 workgroups of 48 features x 2 splits
    (5, 1024, 2048, 2),     # one token group, 32 features a workgroup; one ring turn a wave
    (17, 256, 8192, 8),     # a partial second token group, 8 splits
    (1, 640, 3072, 3),      # one token row, 3 splits
    (9, 512, 6144, 2),      # one token group, 1 wave, ring of 3
    (20, 320, 9216, 3),     # a partial second token group, 10 feature tiles, 1 wave, ring of 3
    (11, 336, 3072, 2),     # 48 features, 2 waves, ring of 3
    (24, 48, 8192, 2),      # one 48-feature tile, 1 wave, ring of 2
])
def test_linear_split_parity(gpu, orc, M, N, K, splits):
    """The f32 partial products of crane_gemm_linear_split, summed in split
    order and rounded once, are the product at the library path's bar; a
    second call repeats the bits."""
    import torch
    from crane_amd import _lib, ops
    print(f"linear split M={M} N={N} K={K} splits={splits}", flush=True)
    x, w, _ = _case(1700 + M + N // 64 + K, M, N, K, "bf16", False)
    xd, wd = _t(x, "bf16", gpu), _t(w, "bf16", gpu)
    outs = []
    for _ in range(2):
        parts = torch.empty((splits, M, N), dtype=torch.float32, device=gpu)
        assert _lib.lib().crane_gemm_linear_split(ops._gemm(gpu)._h, xd.data_ptr(), wd.data_ptr(), parts.data_ptr(),
                                                  M, N, K, splits, _lib.BF16, ops._stream(gpu)) == 0
        outs.append(parts.cpu().numpy())
    assert np.array_equal(outs[0], outs[1])
    acc = np.zeros((M, N), np.float32)
    for p in outs[0]:
        acc = (acc + p).astype(np.float32)
    assert_linear_close(cases.bf16(acc), x, w, None, "bf16", orc, f"split linear {M}x{N}x{K}/{splits}")


def _silu_mul_bound(x, w, orc):
    """The oracle chain of the gated product and a per-element bound for the
    GPU: each projection lies within the f32 accumulation bound plus one ulp
    of its rounding; out = silu(g) u moves by at most |u| |silu'(g)| <= 1.1 |u|
    per unit of g and |silu(g)| per unit of u, plus two ulps (its own rounding
    and the f32 exp)."""
    K = x.shape[-1]
    gu = orc.linear(x, w, None, "bf16", fused=True)
    acc = (K * 2.0 ** -24) * (np.abs(x.astype(np.float64)) @ np.abs(w.astype(np.float64)).T)
    dgu = acc + bf16_ulp(gu)
    inter = w.shape[0] // 2
    g, u = gu[:, :inter].astype(np.float64), gu[:, inter:].astype(np.float64)
    silu = g / (1.0 + np.exp(-g))
    ref = orc.silu_mul(gu, False, "bf16")
    bound = 1.1 * np.abs(u) * dgu[:, :inter] + np.abs(silu) * dgu[:, inter:] + 2 * bf16_ulp(ref)
    return ref, bound


@pytest.mark.gpu
@pytest.mark.parametrize("M,inter,K", [
    (32, 12288, 4096),  # Qwen3-8B decode: 48 gate + 48 up features a workgroup, 256 workgroups
    (17, 9216, 1024),   # partial second token group
    (1, 12288, 512),    # one token row; each wave's two stages fill the ring once
    (3, 4160, 1024),    # inter a multiple of 32, not 48: 32 + 32 features, one token group
    (24, 4160, 2048),   # the same with two token groups
])
def test_linear_silu_mul_parity(gpu, orc, M, inter, K):
    """crane_gemm_linear_silu_mul (one launch) against the oracle chain
    linear -> silu_mul (candle's Mlp at qwen3/modeling.rs:573-585 with Crane's
    fused_silu_mul): every element within the propagated accumulation bound,
    at least 98% bit-identical, the mean-relative bar, and a second call
    repeats the bits.  The two-call GPU path (ops.linear + ops.silu_mul) lies
    within the same bound."""
    from crane_amd import _lib, ops
    from tolerance import errors, BF16_MEAN_REL
    assert _lib.lib().crane_gemm_silu_mul_supported(M, inter, K, 1) == 1
    print(f"linear_silu_mul M={M} inter={inter} K={K}", flush=True)
    x, w, _ = _case(1700 + M + inter // 64 + K, M, 2 * inter, K, "bf16", False)
    ref, bound = _silu_mul_bound(x, w, orc)
    xt, wt = _t(x, "bf16", gpu), _t(w, "bf16", gpu)
    got = ops.linear_silu_mul(xt, wt)
    g = got.float().cpu().numpy()
    assert g.shape == (M, inter)
    d = np.abs(g.astype(np.float64) - ref)
    assert np.all(d <= bound), f"gated {M}x{inter}x{K}: beyond the bound by {float((d - bound).max())}"
    exact = float(np.mean(g == ref))
    assert exact >= 0.98, f"gated {M}x{inter}x{K}: only {exact:.4f} bit-identical"
    assert errors(g, ref)[1] <= BF16_MEAN_REL
    assert bool((ops.linear_silu_mul(xt, wt) == got).all())
    two = ops.silu_mul(ops.linear(xt, wt)).float().cpu().numpy()
    assert np.all(np.abs(two.astype(np.float64) - ref) <= bound)


N_RANDOM = int(os.environ.get("CRANE_RANDOM_GEMM", 12))
SEED = int(os.environ.get("CRANE_RANDOM_SEED", 0))


def linear_draw(seed: int, i: int):
    """Draw i of the randomised decode-projection sweep: (M, N, K, bias) with
    1-32 token rows, cycling over the shapes each path takes -- the ring
    kernel's three configurations (N <= 4096, <= 8192, wider), the streaming
    kernel (N >= 16384, K not a multiple of 1024) and hipBLASLt (anything
    else) -- and M N K at most 1.5e9 so the oracle finishes in seconds."""
    r = cases.rng(seed + 9100 + i)
    M = int(r.integers(1, 33))
    kind = i % 5
    if kind == 0:
        N, K = 16 * int(r.integers(1, 257)), 2048 * int(r.integers(1, 5))
    elif kind == 1:
        N, K = 32 * int(r.integers(129, 257)), 1024 * int(r.integers(1, 9))
    elif kind == 2:
        N, K = 64 * int(r.integers(129, 1025)), 1024 * int(r.integers(1, 5))
    elif kind == 3:
        N, K = 64 * int(r.integers(256, 513)), 128 * int(r.choice([1, 3, 5, 7, 9, 11, 13]))
    else:
        N, K = int(r.integers(1, 3000)), int(r.integers(1, 1500))
    while M * N * K > 1.5e9 and K > 1024:
        K -= 1024
    return M, N, K, bool(r.random() < 0.5)


@pytest.mark.gpu
@pytest.mark.parametrize("i", range(N_RANDOM))
def test_random_decode_linear(gpu, orc, i):
    """Random decode-shaped bf16 products against the oracle (same bar as the
    fixed shapes), each repeated for identical bits."""
    from crane_amd import ops
    M, N, K, bias = linear_draw(SEED, i)
    print(f"random linear {i} (seed {SEED}): M={M} N={N} K={K} bias={bias}", flush=True)
    x, w, b = _case(SEED + 9200 + i, M, N, K, "bf16", bias)
    got = ops.linear(_t(x, "bf16", gpu), _t(w, "bf16", gpu), _t(b, "bf16", gpu) if bias else None)
    assert_linear_close(got.float().cpu().numpy(), x, w, b, "bf16", orc, f"random linear {M}x{N}x{K}")
    got2 = ops.linear(_t(x, "bf16", gpu), _t(w, "bf16", gpu), _t(b, "bf16", gpu) if bias else None)
    assert bool((got == got2).all())


def split_draw(seed: int, i: int):
    """Draw i of the randomised split-K sweep: (M, N, K, splits) that
    crane_gemm_split_supported takes, cycling over the feature widths (N a
    multiple of 64, of 48, of 32) and the two wave counts (a share of K below
    3072, a multiple of 512, takes 2 waves; from 3072, a multiple of 256, 1),
    with M N K at most 1.5e9."""
    r = cases.rng(seed + 9700 + i)
    M = int(r.integers(1, 33))
    splits = int(r.choice([2, 3, 4, 6, 8]))
    base = (64, 48, 32)[i % 3]
    N = base * int(r.integers(1, 129))
    share = 512 * int(r.integers(1, 6)) if (i // 3) % 2 == 0 else 256 * int(r.integers(12, 33))
    while M * N * splits * share > 1.5e9 and N > base:
        N -= base
    return M, N, splits * share, splits


@pytest.mark.gpu
@pytest.mark.parametrize("i", range(N_RANDOM))
def test_random_linear_split(gpu, orc, i):
    """Random shapes of the split-K partial products, summed in split order
    and rounded once, against the oracle at the bar of
    test_linear_split_parity; a second call repeats the bits."""
    import torch
    from crane_amd import _lib, ops
    M, N, K, splits = split_draw(SEED, i)
    print(f"random linear split {i} (seed {SEED}): M={M} N={N} K={K} splits={splits}", flush=True)
    assert _lib.lib().crane_gemm_split_supported(M, N, K, splits, _lib.BF16) == 1
    x, w, _ = _case(SEED + 9800 + i, M, N, K, "bf16", False)
    xd, wd = _t(x, "bf16", gpu), _t(w, "bf16", gpu)
    outs = []
    for _ in range(2):
        parts = torch.empty((splits, M, N), dtype=torch.float32, device=gpu)
        assert _lib.lib().crane_gemm_linear_split(ops._gemm(gpu)._h, xd.data_ptr(), wd.data_ptr(), parts.data_ptr(),
                                                  M, N, K, splits, _lib.BF16, ops._stream(gpu)) == 0
        outs.append(parts.cpu().numpy())
    assert np.array_equal(outs[0], outs[1])
    acc = np.zeros((M, N), np.float32)
    for p in outs[0]:
        acc = (acc + p).astype(np.float32)
    assert_linear_close(cases.bf16(acc), x, w, None, "bf16", orc, f"random split linear {M}x{N}x{K}/{splits}")


def silu_mul_draw(seed: int, i: int):
    """Draw i of the randomised one-launch gate_up + SiLU*mul sweep: (M, inter,
    K) that crane_gemm_silu_mul_supported takes -- inter a multiple of 48
    with K of 512, or of 32 with K of 1024 -- with M * 2 inter * K <= 1.5e9."""
    r = cases.rng(seed + 9500 + i)
    M = int(r.integers(1, 33))
    if i % 2 == 0:
        inter, K = 48 * int(r.integers(86, 300)), 512 * int(r.integers(1, 9))
    else:
        inter, K = 32 * int(r.integers(129, 400)), 1024 * int(r.integers(1, 5))
    while M * 2 * inter * K > 1.5e9 and K > 1024:
        K -= 1024
    return M, inter, K


@pytest.mark.gpu
@pytest.mark.parametrize("i", range(N_RANDOM // 2))
def test_random_linear_silu_mul(gpu, orc, i):
    """Random shapes of the one-launch gated product against the oracle chain,
    the bar of test_linear_silu_mul_parity."""
    from crane_amd import _lib, ops
    M, inter, K = silu_mul_draw(SEED, i)
    print(f"random linear_silu_mul {i} (seed {SEED}): M={M} inter={inter} K={K}", flush=True)
    assert _lib.lib().crane_gemm_silu_mul_supported(M, inter, K, 1) == 1
    x, w, _ = _case(SEED + 9600 + i, M, 2 * inter, K, "bf16", False)
    ref, bound = _silu_mul_bound(x, w, orc)
    got = ops.linear_silu_mul(_t(x, "bf16", gpu), _t(w, "bf16", gpu)).float().cpu().numpy()
    d = np.abs(got.astype(np.float64) - ref)
    assert np.all(d <= bound), f"random gated {M}x{inter}x{K}: beyond the bound"
    assert float(np.mean(got == ref)) >= 0.98


@pytest.mark.gpu
def test_qkv_proj_feeds_the_append(gpu, orc):
    """Hidden states -> qkv_proj (bias) -> fused QK-norm/RoPE append, against
    the oracle's Linear followed by its append."""
    import torch
    from crane_amd import ops
    B, S, H, Hq, Hkv, D = 2, 33, 512, 8, 2, 128
    W = (Hq + 2 * Hkv) * D
    x, w, b = _case(600, B * S, W, H, "bf16")
    qkv = ops.linear(_t(x, "bf16", gpu), _t(w, "bf16", gpu), _t(b, "bf16", gpu)).reshape(B, S, W)
    assert_linear_close(qkv.float().cpu().numpy().reshape(B * S, W), x, w, b, "bf16", orc, "qkv_proj")
    cos, sin = orc.rope_tables(D, 1e6, 64)
    cos, sin = orc.round_bf16(cos), orc.round_bf16(sin)
    kc = torch.zeros((B, Hkv, 64, D), dtype=torch.bfloat16, device=gpu)
    vc = torch.zeros_like(kc)
    zero = torch.zeros(B, dtype=torch.int32, device=gpu)
    q = ops.qk_norm_rope_append(qkv, _t(cos, "bf16", gpu), _t(sin, "bf16", gpu), zero, kc, vc, zero, S, Hq, Hkv,
                                order="rope_only")
    kref = np.zeros((B, Hkv, 64, D), np.float32)
    vref = np.zeros_like(kref)
    # the append is applied to the GPU's own qkv rows: this checks the hand-off
    # (layout and row stride), the append's parity is tested on its own
    qkv_np = qkv.float().cpu().numpy()
    q_ref = orc.qk_norm_rope_append(qkv_np, Hq, Hkv, cos, sin, np.zeros(B, np.int32), kref, vref,
                                    np.zeros(B, np.int32), order=orc.ROPE_ONLY, dtype="bf16")
    assert_ulp_close(q.float().cpu().numpy(), q_ref, "bf16", "q after the append", min_exact=0.999)
    assert_ulp_close(kc.float().cpu().numpy(), kref, "bf16", "k cache after the append", min_exact=0.999)
    np.testing.assert_array_equal(vc.float().cpu().numpy(), vref)


@pytest.mark.gpu
def test_linear_on_two_streams_and_threads(gpu, orc):
    """Each stream gets its own context (its own workspace), so projections on
    two streams may overlap; host threads calling into one context at once,
    while new shapes are being planned, are serialised.  Every result is
    bit-identical to the same product on the default stream."""
    import threading
    import torch
    from crane_amd import ops
    shapes = [(64 + 7 * i, 256 + 32 * i, 512) for i in range(6)]
    xs, ws, refs = [], [], []
    for i, (M, N, K) in enumerate(shapes):
        x, w, _ = _case(700 + i, M, N, K, "bf16", False)
        xs.append(_t(x, "bf16", gpu))
        ws.append(_t(w, "bf16", gpu))
    torch.cuda.synchronize()
    refs = [ops.linear(x, w) for x, w in zip(xs, ws)]
    torch.cuda.synchronize()
    print("linear: two streams", flush=True)
    s1, s2 = torch.cuda.Stream(device=gpu), torch.cuda.Stream(device=gpu)
    outs = {}
    for s in (s1, s2):
        s.wait_stream(torch.cuda.current_stream(gpu))
    with torch.cuda.stream(s1):
        outs[1] = [ops.linear(x, w) for x, w in zip(xs, ws)]
    with torch.cuda.stream(s2):
        outs[2] = [ops.linear(x, w) for x, w in reversed(list(zip(xs, ws)))][::-1]
    torch.cuda.synchronize()
    assert ops._gemm(gpu) is not None and len({k for k in ops._GEMMS if k[0] == gpu}) >= 3
    for k in (1, 2):
        for got, ref in zip(outs[k], refs):
            assert torch.equal(got, ref), "a side stream's product differs"
    for st in (s1, s2):  # retire the side streams' contexts
        ops.release_stream(gpu, st)
        assert (gpu, st.cuda_stream) not in ops._GEMMS
    assert torch.equal(ops.linear(xs[0], ws[0]), refs[0])  # the default stream's context is untouched
    print("linear: four host threads on one stream", flush=True)
    results, errors = {}, []

    def worker(j):
        try:
            new = [(40 + 3 * j + i, 192 + 64 * j, 256) for i in range(3)]  # shapes no one planned yet
            got = []
            for (M, N, K) in new:
                x, w, _ = _case(800 + 10 * j + M, M, N, K, "bf16", False)
                xt, wt = _t(x, "bf16", gpu), _t(w, "bf16", gpu)
                got.append((ops.linear(xt, wt), xt, wt))
            results[j] = got
        except Exception as e:  # reported below, in the test's thread
            errors.append(repr(e))

    threads = [threading.Thread(target=worker, args=(j,)) for j in range(4)]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    torch.cuda.synchronize()
    assert not errors, errors
    for j, got in results.items():
        for y, xt, wt in got:
            assert torch.equal(y, ops.linear(xt, wt)), f"thread {j}: product differs on a second call"
