"""Token selection (include/crane_sampling.h): Crane's gpu_argmax and
topk_indices (crane-core/src/fused_ops/cuda_impl.rs:266-545, used by
crane-serve/src/engine/sampling.rs:127-190), batched over rows.

The oracle is pinned to numpy (argmax is the first maximum, top-k a stable
descending sort) and to the reference's CPU fallback order; the GPU must return
exactly the oracle's indices, ties, -inf masks and NaN included."""
import numpy as np
import pytest

import cases

VOCAB = 151936   # Qwen3 / Qwen2.5 vocabulary


def _logits(seed, rows, n, dtype="f32", std=4.0):
    return cases.cast(cases.normal(cases.rng(seed), (rows, n), std), dtype)


# ------------------------------------------------------------------ CPU

def test_argmax_topk_oracle_vs_numpy(orc):
    x = _logits(1, 5, 3000)
    np.testing.assert_array_equal(orc.argmax(x), np.argmax(x, axis=-1))
    for k in (1, 7, 64):
        want = np.argsort(-x, axis=-1, kind="stable")[:, :k]
        np.testing.assert_array_equal(orc.topk(x, k), want)
    # ties: bf16-rounded values repeat; the first index wins, as candle's argmax and a stable sort
    xb = cases.bf16(_logits(2, 3, 5000, std=1.0))
    np.testing.assert_array_equal(orc.argmax(xb), np.argmax(xb, axis=-1))
    np.testing.assert_array_equal(orc.topk(xb, 64), np.argsort(-xb, axis=-1, kind="stable")[:, :64])
    # a planted mistake (ascending order) fails
    assert not np.array_equal(orc.topk(x, 8), np.argsort(x, axis=-1, kind="stable")[:, :8])


def test_oracle_special_values(orc):
    x = np.float32([[1, 3, 3, np.nan, -0.0, 0.0, 3, -np.inf]])
    assert orc.argmax(x)[0] == 1
    np.testing.assert_array_equal(orc.topk(x, 8)[0], [1, 2, 6, 0, 4, 5, 7, 3])
    allnan = np.full((1, 4), np.nan, np.float32)
    assert orc.argmax(allnan)[0] == 0
    np.testing.assert_array_equal(orc.topk(allnan, 3)[0], [0, 1, 2])


def test_sampling_argument_checks():
    from crane_amd import _lib
    L = _lib.lib()
    assert L.crane_hip_argmax(16, 1, 100, 3, 16, None) == _lib.E_DTYPE
    assert L.crane_hip_argmax(16, 1, 0, 1, 16, None) == _lib.E_INVALID
    assert L.crane_hip_argmax(None, 1, 100, 1, 16, None) == _lib.E_INVALID
    assert L.crane_hip_argmax(16, 0, 100, 1, 16, None) == _lib.OK
    assert L.crane_hip_topk(16, 1, 100, 65, 16, None) == _lib.E_INVALID   # k > 64
    assert L.crane_hip_topk(16, 1, 10, 11, 16, None) == _lib.E_INVALID    # k > n
    assert L.crane_hip_topk(16, 1, 100, 0, 16, None) == _lib.E_INVALID
    assert L.crane_hip_topk(None, 1, 100, 8, 16, None) == _lib.E_INVALID


# ------------------------------------------------------------------ GPU

def _t(x, dtype, dev):
    import torch
    t = torch.from_numpy(np.ascontiguousarray(x))
    return (t.to(torch.bfloat16) if dtype == "bf16" else t).to(dev)


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", ["bf16", "f32"])
@pytest.mark.parametrize("rows,n", [(1, VOCAB), (32, VOCAB), (3, 152064), (2, 4099), (4, 7)])
def test_argmax_parity(gpu, orc, dtype, rows, n):
    from crane_amd import ops
    print(f"argmax {dtype} {rows}x{n}", flush=True)
    x = _logits(10 + n, rows, n, dtype)
    got = ops.argmax(_t(x, dtype, gpu)).cpu().numpy().astype(np.uint32)
    np.testing.assert_array_equal(got, orc.argmax(x))


@pytest.mark.gpu
def test_argmax_ties_masks_and_nan(gpu, orc):
    import torch
    from crane_amd import ops
    n = 10000
    x = _logits(20, 6, n, "bf16", std=1.0)
    x[0, [17, 4000, 9999]] = 9.0          # repeated maximum: the first index
    x[1, :] = 0.5                         # all equal
    x[2, :] = -np.inf
    x[2, 5000] = -3.0                     # everything masked but one
    x[3, ::2] = np.nan                    # NaN ranks lowest
    x[4, :] = np.nan
    x[5, 123] = -0.0
    x[5, :] = 0.0                         # -0 == +0
    for dtype in ("bf16", "f32"):
        got = ops.argmax(_t(x, dtype, gpu)).cpu().numpy().astype(np.uint32)
        np.testing.assert_array_equal(got, orc.argmax(x))
    assert list(orc.argmax(x)[:3]) == [17, 0, 5000]


@pytest.mark.gpu
@pytest.mark.parametrize("rows,n,k", [(1, VOCAB, 64), (32, VOCAB, 50), (2, VOCAB, 1), (3, 4099, 7),
                                      (2, 64, 64), (1, 100, 64), (5, 9, 9)])
def test_topk_parity(gpu, orc, rows, n, k):
    from crane_amd import ops
    print(f"topk {rows}x{n} k={k}", flush=True)
    x = _logits(30 + n + k, rows, n)
    got = ops.topk_indices(_t(x, "f32", gpu), k).cpu().numpy().astype(np.uint32)
    np.testing.assert_array_equal(got, orc.topk(x, k))


@pytest.mark.gpu
def test_topk_ties_straddling_k(gpu, orc):
    """Equal values across the k-th place are taken by index (the ordered
    path), also when the whole row is equal or masked."""
    from crane_amd import ops
    n = 20000
    x = cases.bf16(_logits(40, 6, n, std=1.0))   # many exact repeats
    x[1, :] = 2.0                                 # all equal
    x[2, :] = -np.inf
    x[2, [7, 19999, 300]] = 1.0                   # fewer finite values than k
    x[3, 1000:1100] = 50.0                        # 100 equal maxima, k = 64 of them
    x[4, ::3] = np.nan
    x[5, 10:30] = 7.0
    x[5, 5] = 8.0
    for k in (64, 33, 1):
        got = ops.topk_indices(_t(x, "f32", gpu), k).cpu().numpy().astype(np.uint32)
        np.testing.assert_array_equal(got, orc.topk(x, k), err_msg=f"k={k}")
