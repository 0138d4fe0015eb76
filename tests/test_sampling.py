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


def test_split_workspace_and_checks():
    """The split path applies to few (<= 32) long (>= 32768) rows; elsewhere
    the workspace size is 0 and the _ws calls run the single-pass kernels."""
    from crane_amd import _lib
    L = _lib.lib()
    assert L.crane_hip_select_workspace_bytes(1, VOCAB) > 0
    assert L.crane_hip_select_workspace_bytes(32, VOCAB) >= 32 * L.crane_hip_select_workspace_bytes(1, VOCAB) // 2
    assert L.crane_hip_select_workspace_bytes(33, VOCAB) == 0
    assert L.crane_hip_select_workspace_bytes(1, 32767) == 0
    assert L.crane_hip_select_workspace_bytes(0, VOCAB) == 0
    need = L.crane_hip_select_workspace_bytes(2, VOCAB)
    assert L.crane_hip_argmax_ws(16, 2, VOCAB, 1, None, 0, 16, None) == _lib.E_CAPACITY
    assert L.crane_hip_argmax_ws(16, 2, VOCAB, 1, 16, need - 1, 16, None) == _lib.E_CAPACITY
    assert L.crane_hip_topk_ws(16, 2, VOCAB, 64, None, 0, 16, None) == _lib.E_CAPACITY
    assert L.crane_hip_topk_ws(16, 2, VOCAB, 65, 16, need, 16, None) == _lib.E_INVALID
    assert L.crane_hip_argmax_ws(16, 2, VOCAB, 3, 16, need, 16, None) == _lib.E_DTYPE
    assert L.crane_hip_argmax_ws(16, 0, VOCAB, 1, None, 0, 16, None) == _lib.OK


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


@pytest.mark.gpu
def test_split_rows_ties_masks_and_nan(gpu, orc):
    """The split path (few rows of the vocabulary's length, 148 workgroups a
    row) on the tie, mask and NaN rows: equal maxima in different slices, a
    row of equal values (more candidates than the list holds: the exact
    one-workgroup fallback), fewer finite values than k, NaN runs, and slices
    holding more candidates than their slots (scanned again by the last
    phase: a hundred such slices, or every slice)."""
    from crane_amd import _lib, ops
    n = VOCAB
    assert _lib.lib().crane_hip_select_workspace_bytes(10, n) > 0
    x = cases.bf16(_logits(50, 10, n, std=1.0))
    x[0, [17, 40000, 151935]] = 9.0               # equal maxima in three slices
    x[1, :] = 2.0                                 # all equal
    x[2, :] = -np.inf
    x[2, [7, 151935, 300]] = 1.0                  # fewer finite values than k
    x[3, 100000:100100] = 50.0                    # 100 equal maxima inside two slices
    x[4, ::3] = np.nan
    x[5, 10:30] = 7.0
    x[5, 5] = 8.0
    x[6, :] = np.nan
    x[7, 1000:3000] = 30.0                        # 2000 equal maxima: k of them by index
    for i in range(100):                          # 10 candidates in each of 100 slices
        x[8, i * 600 + 7 * np.arange(10)] = 20.0 + (i % 8) / 8
    x[9, ::100] = 24.0                            # 1520 equal values, 6 in every slice
    print("split rows: argmax", flush=True)
    for dtype in ("bf16", "f32"):
        got = ops.argmax(_t(x, dtype, gpu)).cpu().numpy().astype(np.uint32)
        np.testing.assert_array_equal(got, orc.argmax(x), err_msg=dtype)
    for k in (64, 33, 1):
        print(f"split rows: topk k={k}", flush=True)
        got = ops.topk_indices(_t(x, "f32", gpu), k).cpu().numpy().astype(np.uint32)
        np.testing.assert_array_equal(got, orc.topk(x, k), err_msg=f"k={k}")


@pytest.mark.gpu
def test_split_topk_crowded_values(gpu, orc):
    """Rows whose values all lie within 2^-8 of 1 (every key shares its top 16
    bits): the split top-k's threshold, a 24-bit prefix of the k-th largest
    slice maximum, still bounds the answer, and the result is the oracle's,
    at one row and at a batch."""
    from crane_amd import ops
    n = VOCAB
    rng = np.random.default_rng(77)
    x = (np.float32(1.0) + rng.uniform(0.0, 2.0 ** -8, size=(3, n)).astype(np.float32)).astype(np.float32)
    x[2, 5000:5100] = x[2, 5000]                  # and a run of equal values among them
    for rows in (1, 3):
        for k in (64, 7):
            print(f"crowded values: rows {rows} k={k}", flush=True)
            got = ops.topk_indices(_t(x[:rows], "f32", gpu), k).cpu().numpy().astype(np.uint32)
            np.testing.assert_array_equal(got, orc.topk(x[:rows], k), err_msg=f"rows={rows} k={k}")


@pytest.mark.gpu
def test_split_workspace_shared_across_calls(gpu):
    """One workspace (filled with garbage first) serves argmax and top-k calls
    of different row counts in any order: it holds nothing between calls."""
    import torch
    from crane_amd import _lib
    L = _lib.lib()
    st = torch.cuda.current_stream(gpu).cuda_stream
    wsb = L.crane_hip_select_workspace_bytes(32, VOCAB)
    ws = torch.full((wsb,), 0x5A, dtype=torch.uint8, device=gpu)
    x = _t(_logits(70, 32, VOCAB), "f32", gpu)
    for rows, k in ((1, 64), (32, 50), (7, 1), (32, 64), (2, 17), (1, 3)):
        print(f"shared workspace: rows {rows} k {k}", flush=True)
        a = torch.empty((rows, k), dtype=torch.int32, device=gpu)
        b = torch.empty((rows, k), dtype=torch.int32, device=gpu)
        assert L.crane_hip_topk_ws(x.data_ptr(), rows, VOCAB, k, ws.data_ptr(), wsb, a.data_ptr(), st) == 0
        assert L.crane_hip_topk(x.data_ptr(), rows, VOCAB, k, b.data_ptr(), st) == 0
        c = torch.empty(rows, dtype=torch.int32, device=gpu)
        d = torch.empty(rows, dtype=torch.int32, device=gpu)
        assert L.crane_hip_argmax_ws(x.data_ptr(), rows, VOCAB, 0, ws.data_ptr(), wsb, c.data_ptr(), st) == 0
        assert L.crane_hip_argmax(x.data_ptr(), rows, VOCAB, 0, d.data_ptr(), st) == 0
        assert torch.equal(a, b) and torch.equal(c, d), (rows, k)


@pytest.mark.gpu
@pytest.mark.parametrize("rows,n", [(1, VOCAB), (32, VOCAB), (3, 32768), (2, 50001), (5, 152064)])
def test_split_matches_single_pass(gpu, rows, n):
    """The _ws (split) and single-pass entry points give the same indices, bit
    for bit, at the edges of the split's range (odd n, unaligned rows, 64
    slices)."""
    import torch
    from crane_amd import _lib
    L = _lib.lib()
    print(f"split vs single pass {rows}x{n}", flush=True)
    x = _t(_logits(60 + rows + n, rows, n), "f32", gpu)
    xb = x.to(torch.bfloat16)
    wsb = L.crane_hip_select_workspace_bytes(rows, n)
    assert wsb > 0
    ws = torch.full((wsb,), 0xA5, dtype=torch.uint8, device=gpu)   # no initial value is needed
    st = torch.cuda.current_stream(gpu).cuda_stream
    for dt, t in ((0, x), (1, xb)):
        a = torch.empty(rows, dtype=torch.int32, device=gpu)
        b = torch.empty(rows, dtype=torch.int32, device=gpu)
        assert L.crane_hip_argmax(t.data_ptr(), rows, n, dt, a.data_ptr(), st) == 0
        assert L.crane_hip_argmax_ws(t.data_ptr(), rows, n, dt, ws.data_ptr(), wsb, b.data_ptr(), st) == 0
        assert torch.equal(a, b), f"argmax dtype {dt}"
    for k in (64, 5):
        a = torch.empty((rows, k), dtype=torch.int32, device=gpu)
        b = torch.empty((rows, k), dtype=torch.int32, device=gpu)
        assert L.crane_hip_topk(x.data_ptr(), rows, n, k, a.data_ptr(), st) == 0
        assert L.crane_hip_topk_ws(x.data_ptr(), rows, n, k, ws.data_ptr(), wsb, b.data_ptr(), st) == 0
        assert torch.equal(a, b), f"topk k={k}"
    # repeated calls on the same workspace keep giving the single-pass answer
    for _ in range(3):
        c = torch.empty(rows, dtype=torch.int32, device=gpu)
        assert L.crane_hip_argmax_ws(xb.data_ptr(), rows, n, 1, ws.data_ptr(), wsb, c.data_ptr(), st) == 0
        d = torch.empty((rows, 64), dtype=torch.int32, device=gpu)
        assert L.crane_hip_topk_ws(x.data_ptr(), rows, n, 64, ws.data_ptr(), wsb, d.data_ptr(), st) == 0
        e = torch.empty((rows, 64), dtype=torch.int32, device=gpu)
        assert L.crane_hip_topk(x.data_ptr(), rows, n, 64, e.data_ptr(), st) == 0
        f = torch.empty(rows, dtype=torch.int32, device=gpu)
        assert L.crane_hip_argmax(xb.data_ptr(), rows, n, 1, f.data_ptr(), st) == 0
        assert torch.equal(c, f) and torch.equal(d, e)
