"""GPU parity: every kernel through the C ABI against the CPU oracle on the
same seeded inputs, at the BASELINE configurations (full size where the
oracle finishes in seconds, sampled rows otherwise) and at the edge cases.
Bars: f32 max-abs <= 1e-4; bf16 max-abs <= 2e-2 and mean-rel <= 1e-2.
Cache rows the kernels must not read are NaN, so an out-of-range read fails."""
import math
import sys
import zlib

import numpy as np
import pytest
import torch

from tests import cases
from tests.cases import D
from tests.tolerance import assert_close, assert_ulp_close, errors

pytestmark = pytest.mark.gpu


def dev_t(x, dtype, dev):
    t = torch.from_numpy(np.ascontiguousarray(x))
    if dtype == "bf16":
        t = t.to(torch.bfloat16)
    return t.to(dev).contiguous()


def host(t):
    return t.float().cpu().numpy()


def i32(x, dev):
    return torch.as_tensor(np.asarray(x, dtype=np.int32), device=dev).contiguous()


def note(msg):
    print(msg, flush=True)
    sys.stdout.flush()


# ------------------------------------------------------------------ decode

DECODE_CASES = [
    # name, B, Hq, Hkv, lens, dtype, std, score mode (None: Qwen3/Hunyuan's rule, grouped iff n_rep > 1)
    ("c1_qwen3_0.6b_f32", 1, 16, 8, [1025], "f32", 1.0, None),
    ("c3_qwen3_8b_bf16", 32, 32, 8, None, "bf16", 1.0, None),
    ("ragged_edges_bf16", 6, 8, 2, [1, 255, 256, 257, 511, 1000], "bf16", 1.0, None),
    ("ragged_edges_f32", 5, 8, 2, [1, 2, 256, 257, 700], "f32", 1.0, None),
    ("mha_nrep1_bf16", 3, 4, 4, [17, 300, 64], "bf16", 1.0, None),
    ("mha_nrep1_f32", 2, 4, 4, [200, 700], "f32", 1.0, None),
    # Qwen2.5 (candle-transformers qwen2): always the standard SDPA
    ("qwen25_7b_gqa7_bf16", 4, 28, 4, [100, 1500, 4096, 33], "bf16", 1.0, "standard"),
    ("qwen25_ragged_standard_bf16", 6, 8, 2, [1, 255, 256, 257, 511, 1000], "bf16", 1.0, "standard"),
    ("gqa16_bf16", 2, 32, 2, [513, 2000], "bf16", 1.0, None),
    ("gqa3_f32", 2, 6, 2, [40, 900], "f32", 1.0, None),
    # max_kv past 12288: 512-key chunks and the 8-partition merge
    ("long_chunks_f32", 2, 8, 2, [13000, 20001], "f32", 1.0, None),
    ("long_chunks_ragged_bf16", 3, 16, 2, [12289, 15000, 700], "bf16", 1.0, None),
]


@pytest.mark.parametrize("name,B,Hq,Hkv,lens,dtype,std,mode", DECODE_CASES, ids=[c[0] for c in DECODE_CASES])
def test_decode_parity(gpu, orc, name, B, Hq, Hkv, lens, dtype, std, mode):
    from crane_amd import ops
    if lens is None:
        lens = cases.c3_lengths()
    note(f"decode {name}: B={B} Hq={Hq} Hkv={Hkv} dtype={dtype} max_len={max(lens)} mode={mode}")
    q, k, v, lens = cases.decode_case(cases.SEED0 + zlib.crc32(name.encode()) % 1000, B, Hq, Hkv, lens, dtype=dtype, std=std)
    cap = k.shape[2]
    out = ops.attention_decode(dev_t(q, dtype, gpu), dev_t(k, dtype, gpu), dev_t(v, dtype, gpu), i32(lens, gpu),
                               int(lens.max()), cases.scale(), score_mode=mode)
    torch.cuda.synchronize()
    ref = orc.attn_decode(q, k, v, lens, cases.scale(), dtype, cases.decode_variant(orc, Hq, Hkv, mode))
    note(f"  errors vs oracle: max-abs {errors(host(out).reshape(B, Hq * D), ref)}")
    assert_close(host(out).reshape(B, Hq * D), ref, dtype, name)
    assert cap == int(lens.max())


def test_decode_c5_long_context(gpu, orc):
    """Config 5 at full size (Qwen2.5-72B shape, B=8, 64 / 8 heads,
    32768-token cache, K/V ~ N(0, 0.5)): every sequence against the oracle."""
    from crane_amd import ops
    B, Hq, Hkv, L = 8, 64, 8, 32768
    note("decode c5: B=8 Hq=64 Hkv=8 L=32768 bf16")
    q, k, v, lens = cases.decode_case(cases.SEED0 + 5, B, Hq, Hkv, [L] * B, dtype="bf16",
                                      std=math.sqrt(0.5), poison=False)
    out = ops.attention_decode(dev_t(q, "bf16", gpu), dev_t(k, "bf16", gpu), dev_t(v, "bf16", gpu),
                               i32(lens, gpu), L, score_mode="standard")
    ref = orc.attn_decode(q, k, v, lens, cases.scale(), "bf16", orc.DECODE_STANDARD)
    assert_close(host(out).reshape(B, Hq * D), ref, "bf16", "c5")


def test_decode_zero_length_and_cap_larger_than_len(gpu, orc):
    from crane_amd import ops
    q, k, v, lens = cases.decode_case(77, 3, 8, 2, [0, 5, 300], cap=1024, dtype="bf16")
    out = host(ops.attention_decode(dev_t(q, "bf16", gpu), dev_t(k, "bf16", gpu), dev_t(v, "bf16", gpu),
                                    i32(lens, gpu), 300)).reshape(3, 8 * D)
    assert np.all(out[0] == 0.0)
    ref = orc.attn_decode(q[1:], k[1:], v[1:], lens[1:], cases.scale(), "bf16")
    assert_close(out[1:], ref, "bf16", "zero-length batch")


def test_decode_short_rows_do_not_depend_on_the_batch(gpu, orc):
    """A sequence of at most 256 keys runs candle's exact chain whatever the
    launch's max_kv (which picks 512-key chunks past 12288): its output is the
    same bits alone and beside a 13000-key sequence, within the bar of the oracle."""
    from crane_amd import ops
    q, k, v, lens = cases.decode_case(79, 2, 8, 2, [200, 13000], dtype="bf16")
    qd, kd, vd = dev_t(q, "bf16", gpu), dev_t(k, "bf16", gpu), dev_t(v, "bf16", gpu)
    both = host(ops.attention_decode(qd, kd, vd, i32(lens, gpu), 13000)).reshape(2, 8 * D)
    alone = host(ops.attention_decode(qd[:1].contiguous(), kd[:1].contiguous(), vd[:1].contiguous(),
                                      i32(lens[:1], gpu), 200)).reshape(1, 8 * D)
    assert np.array_equal(both[0], alone[0])
    ref = orc.attn_decode(q[:1], k[:1], v[:1], lens[:1], cases.scale(), "bf16", orc.DECODE_GROUPED)
    note(f"  bit-identical to the oracle {np.mean(alone == ref.reshape(1, 8 * D)):.5f}")
    assert_close(alone, ref.reshape(1, 8 * D), "bf16", "short row")


def test_decode_kv_len_clamped_to_max_kv(gpu, orc):
    """A kv_len above the host's max_kv is clamped, never read past."""
    from crane_amd import ops
    q, k, v, lens = cases.decode_case(78, 2, 8, 2, [100, 100], cap=100, dtype="bf16")
    out = host(ops.attention_decode(dev_t(q, "bf16", gpu), dev_t(k, "bf16", gpu), dev_t(v, "bf16", gpu),
                                    i32([1000, 50], gpu), 100)).reshape(2, 8 * D)
    ref = orc.attn_decode(q, k, v, np.array([100, 50], np.int32), cases.scale(), "bf16")
    assert_close(out, ref, "bf16", "clamp")


def test_decode_properties_full_c3(gpu):
    """Size-independent properties at config 3's full size: V = 1 gives 1
    (probabilities sum to one); permuting cache rows leaves the output unchanged."""
    from crane_amd import ops
    lens = cases.c3_lengths()
    B, Hq, Hkv = 32, 32, 8
    q, k, v, lens = cases.decode_case(cases.SEED0 + 31, B, Hq, Hkv, lens, dtype="bf16", poison=False)
    qd, kd = dev_t(q, "bf16", gpu), dev_t(k, "bf16", gpu)
    ones = torch.ones_like(kd)
    out = host(ops.attention_decode(qd, kd, ones, i32(lens, gpu), int(lens.max())))
    assert np.all(out == 1.0)
    vd = dev_t(v, "bf16", gpu)
    base = host(ops.attention_decode(qd, kd, vd, i32(lens, gpu), int(lens.max())))
    kp, vp = kd.clone(), vd.clone()
    g = torch.Generator().manual_seed(5)
    for b in range(B):
        perm = torch.randperm(int(lens[b]), generator=g).to(gpu)
        kp[b, :, :lens[b]] = kd[b, :, perm]
        vp[b, :, :lens[b]] = vd[b, :, perm]
    permuted = host(ops.attention_decode(qd, kp, vp, i32(lens, gpu), int(lens.max())))
    assert np.max(np.abs(permuted - base)) <= 2 ** -7 * max(1.0, np.abs(base).max())


# ------------------------------------------------------------------ append

APPEND_CASES = [
    # name, B, S, Hq, Hkv, cache_len, positions, cap, order, dtype
    ("c2_prefill_append_bf16", 1, 2048, 16, 8, [0], [0], 4096, 0, "bf16"),
    ("c1_decode_append_f32", 1, 1, 16, 8, [1024], [1024], 1025, 0, "f32"),
    ("batched_decode_append_bf16", 32, 1, 32, 8, list(range(500, 532)), list(range(700, 732)), 600, 0, "bf16"),
    ("hunyuan_order_bf16", 2, 33, 8, 2, [0, 5], [0, 5], 64, 1, "bf16"),
    ("qwen25_rope_only_bf16", 2, 70, 28, 4, [3, 0], [3, 0], 80, 2, "bf16"),
    ("hunyuan_order_f32", 2, 9, 4, 2, [1, 2], [1, 2], 16, 1, "f32"),
    ("qwen3_prefill_f32", 1, 40, 16, 8, [0], [0], 64, 0, "f32"),
]


@pytest.mark.parametrize("name,B,S,Hq,Hkv,clen,posn,cap,order,dtype", APPEND_CASES, ids=[c[0] for c in APPEND_CASES])
def test_append_parity(gpu, orc, name, B, S, Hq, Hkv, clen, posn, cap, order, dtype):
    from crane_amd import ops
    note(f"append {name}: B={B} S={S} Hq={Hq} Hkv={Hkv} order={order} dtype={dtype}")
    r = cases.rng(cases.SEED0 + 200 + len(name))
    qkv = cases.cast(cases.normal(r, (B, S, (Hq + 2 * Hkv) * D)), dtype)
    qw = cases.cast(1 + 0.1 * cases.normal(r, (D,)), dtype) if order != 2 else None
    kw = cases.cast(1 + 0.1 * cases.normal(r, (D,)), dtype) if order != 2 else None
    cos, sin = orc.rope_tables(D, 1e6, 4096)
    cos, sin = cases.cast(cos, dtype), cases.cast(sin, dtype)
    canary = np.float32(3.0)
    kc = np.full((B, Hkv, cap, D), canary, np.float32)
    vc = np.full((B, Hkv, cap, D), canary, np.float32)
    kd, vd = dev_t(kc, dtype, gpu), dev_t(vc, dtype, gpu)
    q = ops.qk_norm_rope_append(dev_t(qkv, dtype, gpu), dev_t(cos, dtype, gpu), dev_t(sin, dtype, gpu),
                                i32(posn, gpu), kd, vd, i32(clen, gpu), max(clen) + S, Hq, Hkv,
                                None if qw is None else dev_t(qw, dtype, gpu),
                                None if kw is None else dev_t(kw, dtype, gpu), 1e-6,
                                ["norm_then_rope", "rope_then_norm", "rope_only"][order])
    torch.cuda.synchronize()
    q_ref = orc.qk_norm_rope_append(qkv, Hq, Hkv, cos, sin, np.array(posn, np.int32), kc, vc,
                                    np.array(clen, np.int32), qw, kw, 1e-6, order, dtype)
    note(f"  q errors {errors(host(q), q_ref)}, bit-exact fraction {np.mean(host(q) == q_ref):.5f}")
    assert_ulp_close(host(q), q_ref, dtype, name + " q")
    kg, vg = host(kd), host(vd)
    assert np.array_equal(vg, vc), "value rows are a copy"
    assert_ulp_close(kg, kc, dtype, name + " k")
    untouched = np.ones((B, cap), bool)
    for b in range(B):
        untouched[b, clen[b]:clen[b] + S] = False
    assert np.all(kg.transpose(0, 2, 1, 3)[untouched] == canary)


@pytest.mark.parametrize("dtype", ["bf16", "f32"])
@pytest.mark.parametrize("order", ["norm_then_rope", "rope_then_norm", "rope_only"])
@pytest.mark.parametrize("splits,bias,B,S,Hq,Hkv", [(2, False, 32, 1, 32, 8), (2, True, 3, 5, 8, 2),
                                                    (4, True, 32, 1, 32, 8), (4, False, 2, 3, 28, 4)])
def test_append_parts_matches_rows(gpu, orc, splits, bias, B, S, Hq, Hkv, order, dtype):
    """The append reading split-K partial products (a decode step's qkv_proj
    as crane_gemm_linear_split writes them) gives, bit for bit, what the
    rows path gives for the rows T(sum of the splits in split order + bias):
    q, the K and V rows written and the canary rows left alone."""
    from crane_amd import ops
    note(f"append parts: {splits} splits, bias {bias}, B={B} S={S} Hq={Hq} Hkv={Hkv} {order} {dtype}")
    cap, W = 16, (Hq + 2 * Hkv) * D
    r = cases.rng(cases.SEED0 + 260 + splits + 3 * B + S)
    parts = cases.normal(r, (splits, B * S, W)).astype(np.float32)
    b = cases.cast(0.5 * cases.normal(r, (W,)), dtype) if bias else None
    acc = np.zeros((B * S, W), np.float32)
    for p in parts:
        acc = (acc + p).astype(np.float32)
    if b is not None:
        acc = (acc + b).astype(np.float32)
    qkv = cases.cast(acc, dtype).reshape(B, S, W)
    qw = cases.cast(1 + 0.1 * cases.normal(r, (D,)), dtype)
    kw = cases.cast(1 + 0.1 * cases.normal(r, (D,)), dtype)
    cos, sin = orc.rope_tables(D, 1e6, 256)
    cos, sin = cases.cast(cos, dtype), cases.cast(sin, dtype)
    clen = [(3 * i) % (cap - S) for i in range(B)]
    posn = [(5 * i + 1) % 200 for i in range(B)]
    outs = []
    for src in ("rows", "parts"):
        kd = dev_t(np.full((B, Hkv, cap, D), 3.0, np.float32), dtype, gpu)
        vd = dev_t(np.full((B, Hkv, cap, D), 3.0, np.float32), dtype, gpu)
        if src == "rows":
            x = dev_t(qkv, dtype, gpu)
        else:
            x = ops.PartialProduct(torch.from_numpy(parts).to(gpu), torch.bfloat16 if dtype == "bf16" else torch.float32,
                                   None if b is None else dev_t(b, dtype, gpu))
        q = ops.qk_norm_rope_append(x, dev_t(cos, dtype, gpu), dev_t(sin, dtype, gpu), i32(posn, gpu), kd, vd,
                                    i32(clen, gpu), max(clen) + S, Hq, Hkv, dev_t(qw, dtype, gpu),
                                    dev_t(kw, dtype, gpu), 1e-6, order)
        torch.cuda.synchronize()
        outs.append((host(q), host(kd), host(vd)))
    for name, a, c in zip(("q", "k", "v"), outs[0], outs[1]):
        assert np.array_equal(a, c), f"{name} differs between the rows and the partial products"


@pytest.mark.parametrize("dtype", ["bf16", "f32"])
def test_cla_q_only_matches_the_append(gpu, orc, dtype):
    """Hunyuan's CLA layer: q alone through rope then query_layernorm, read
    from a narrowed [B, S, Hq*D] view of a wider row, equals the q rows of the
    full append bit for bit and the oracle's q within the bar; decode over the
    anchor's cache with it matches the oracle."""
    from crane_amd import ops
    B, S, Hq, Hkv, cap = 3, 17, 8, 2, 64
    note(f"cla q-only {dtype}: B={B} S={S} Hq={Hq}")
    r = cases.rng(cases.SEED0 + 777)
    qkv = cases.cast(cases.normal(r, (B, S, (Hq + 2 * Hkv) * D)), dtype)
    qw = cases.cast(1 + 0.1 * cases.normal(r, (D,)), dtype)
    kw = cases.cast(1 + 0.1 * cases.normal(r, (D,)), dtype)
    cos, sin = (cases.cast(t, dtype) for t in orc.rope_tables(D, 1e6, 256))
    clen, posn = [0, 4, 9], [0, 4, 30]
    kc = np.zeros((B, Hkv, cap, D), np.float32)
    vc = np.zeros((B, Hkv, cap, D), np.float32)
    kd, vd = dev_t(kc, dtype, gpu), dev_t(vc, dtype, gpu)
    qkv_d = dev_t(qkv, dtype, gpu)
    cos_d, sin_d, pos_d, qw_d = dev_t(cos, dtype, gpu), dev_t(sin, dtype, gpu), i32(posn, gpu), dev_t(qw, dtype, gpu)
    q_full = ops.qk_norm_rope_append(qkv_d, cos_d, sin_d, pos_d, kd, vd, i32(clen, gpu), max(clen) + S, Hq, Hkv,
                                     qw_d, dev_t(kw, dtype, gpu), 1e-6, "rope_then_norm")
    q_only = ops.q_norm_rope(qkv_d[:, :, :Hq * D], cos_d, sin_d, pos_d, Hq, qw_d, 1e-6, "rope_then_norm")
    torch.cuda.synchronize()
    assert torch.equal(q_only, q_full)
    q_ref = orc.qk_norm_rope_append(qkv, Hq, Hkv, cos, sin, np.array(posn, np.int32), kc, vc,
                                    np.array(clen, np.int32), qw, kw, 1e-6, 1, dtype)
    assert_ulp_close(host(q_only), q_ref, dtype, "cla q")
    # a one-token CLA decode over the anchor's cache (its rows include the new tokens)
    lens = [c + S for c in clen]
    q1 = ops.q_norm_rope(qkv_d[:, S - 1:, :].contiguous()[:, :, :Hq * D], cos_d, sin_d, i32([p + S - 1 for p in posn], gpu), Hq, qw_d,
                         1e-6, "rope_then_norm")
    out = ops.attention_decode(q1.reshape(B, Hq, D), kd, vd, i32(lens, gpu), max(lens))
    torch.cuda.synchronize()
    ref = orc.attn_decode(q_ref[:, :, S - 1, :], host(kd), host(vd), np.array(lens, np.int32), 1 / math.sqrt(D),
                          dtype)
    assert_close(host(out).reshape(ref.shape), ref, dtype, "cla decode")


# ----------------------------------------------------------------- prefill

PREFILL_CASES = [
    # name, B, S, Hq, Hkv, start, causal, dtype (configs 2 and 4 at full size: the tests below)
    ("ragged_S_bf16", 2, 200, 8, 2, [0, 0], True, "bf16"),
    ("continuation_bf16", 3, 77, 6, 2, [0, 130, 1000], True, "bf16"),
    ("noncausal_bf16", 2, 96, 8, 4, [0, 40], False, "bf16"),
    ("mha_bf16", 1, 300, 4, 4, [0], True, "bf16"),
    ("tiny_S1_bf16", 2, 1, 8, 2, [0, 63], True, "bf16"),
    ("f32_small", 2, 50, 4, 2, [0, 17], True, "f32"),
    # the f32 MFMA kernel: config 2's shape, continuation chunks over longer caches, non-causal
    ("c2_shape_f32", 1, 2048, 16, 8, [0], True, "f32"),
    ("continuation_f32", 2, 300, 8, 2, [0, 700], True, "f32"),
    ("noncausal_f32", 2, 130, 4, 2, [0, 33], False, "f32"),
]


@pytest.mark.parametrize("name,B,S,Hq,Hkv,start,causal,dtype", PREFILL_CASES, ids=[c[0] for c in PREFILL_CASES])
def test_prefill_parity(gpu, orc, name, B, S, Hq, Hkv, start, causal, dtype):
    from crane_amd import ops
    note(f"prefill {name}: B={B} S={S} Hq={Hq} Hkv={Hkv} start={start} causal={causal} dtype={dtype}")
    q, k, v, st = cases.prefill_case(cases.SEED0 + 300 + len(name), B, S, Hq, Hkv, start, dtype=dtype)
    out = host(ops.attention_prefill(dev_t(q, dtype, gpu), dev_t(k, dtype, gpu), dev_t(v, dtype, gpu),
                                     i32(st, gpu), int(st.max()), cases.scale(), causal)).reshape(B, S, Hq, D)
    assert np.all(np.isfinite(out))
    ref = orc.attn_prefill(q, k, v, st, cases.scale(), causal, dtype).reshape(B, S, Hq, D)
    note(f"  errors vs oracle (max-abs, mean-rel): {errors(out, ref)}")
    assert_close(out, ref, dtype, name)


LONG_ROW_KEYS = 1024  # rows that see this many keys or more: the long rows of the one-rounding switch


def test_prefill_c4_full(gpu, orc):
    """Config 4 at full size (Qwen2.5-7B shape: 8 sequences of 4096 rows, 28 q
    / 4 kv heads, causal, bf16): every row of every sequence against the
    oracle, in the default arithmetic (both of candle's score roundings) and
    with CRANE_HIP_PREFILL_LONG_ROWS_ONE_ROUNDING.  Rows that see 1024 keys or
    more (the long rows, 75% of the output) keep their mean-relative distance
    within 0.6 of the bar in both modes."""
    from crane_amd import ops
    from tests.tolerance import BF16_MEAN_REL
    B, S, Hq, Hkv = 8, 4096, 28, 4
    note(f"prefill c4 full: B={B} S={S} Hq={Hq} Hkv={Hkv} causal bf16, all rows")
    q, k, v, st = cases.prefill_case(cases.SEED0 + 304, B, S, Hq, Hkv, [0] * B, dtype="bf16")
    qd, kd, vd, sd = dev_t(q, "bf16", gpu), dev_t(k, "bf16", gpu), dev_t(v, "bf16", gpu), i32(st, gpu)
    ref = orc.attn_prefill(q, k, v, st, cases.scale(), True, "bf16").reshape(B, S, Hq, D)
    long_rows = np.arange(S) + 1 >= LONG_ROW_KEYS
    for one_rounding in (False, True):
        out = host(ops.attention_prefill(qd, kd, vd, sd, 0, cases.scale(), True,
                                         long_rows_one_rounding=one_rounding)).reshape(B, S, Hq, D)
        mode = "one rounding on long rows" if one_rounding else "both roundings (default)"
        e_all, e_long = errors(out, ref), errors(out[:, long_rows], ref[:, long_rows])
        e_short = errors(out[:, ~long_rows], ref[:, ~long_rows])
        note(f"  {mode}: all rows (max-abs, mean-rel) {e_all}; rows < {LONG_ROW_KEYS} keys {e_short}; "
             f"long rows {e_long}")
        tru = cases.prefill_truth(q, k, v, st, 0, 2011, 2075)
        note(f"  {mode}: sequence 0 rows 2011:2075 vs float64 softmax: gpu {errors(out[0, 2011:2075], tru)}, "
             f"oracle {errors(ref[0, 2011:2075], tru)}")
        for b in range(B):
            assert_close(out[b], ref[b], "bf16", f"c4 {mode} sequence {b}")
        assert e_long[1] <= 0.6 * BF16_MEAN_REL, f"c4 {mode}: long-row mean-rel {e_long[1]:.3e}"


def test_prefill_c2_chain(gpu, orc):
    """Config 2 as Crane runs it (Qwen3-0.6B shape, one sequence of 2048 rows,
    16 q / 8 kv heads, bf16): the fused QK-RMSNorm + RoPE append of the merged
    qkv rows into an empty cache of capacity 4096, then the causal prefill over
    that cache, against the oracle's same chain; every row compared."""
    from crane_amd import ops
    B, S, Hq, Hkv, cap = 1, 2048, 16, 8, 4096
    note(f"prefill c2 chain: append into an empty cap-{cap} cache, then prefill; B={B} S={S} Hq={Hq} Hkv={Hkv}")
    r = cases.rng(cases.SEED0 + 302)
    qkv = cases.bf16(cases.normal(r, (B, S, (Hq + 2 * Hkv) * D)))
    qw = cases.bf16(1 + 0.1 * cases.normal(r, (D,)))
    kw = cases.bf16(1 + 0.1 * cases.normal(r, (D,)))
    cos, sin = (cases.bf16(t) for t in orc.rope_tables(D, 1e6, cap))
    zeros = [0] * B
    kd = torch.zeros((B, Hkv, cap, D), dtype=torch.bfloat16, device=gpu)
    vd = torch.zeros_like(kd)
    qd = ops.qk_norm_rope_append(dev_t(qkv, "bf16", gpu), dev_t(cos, "bf16", gpu), dev_t(sin, "bf16", gpu),
                                 i32(zeros, gpu), kd, vd, i32(zeros, gpu), S, Hq, Hkv, dev_t(qw, "bf16", gpu),
                                 dev_t(kw, "bf16", gpu), 1e-6, "norm_then_rope")
    out = host(ops.attention_prefill(qd, kd, vd, i32(zeros, gpu), 0, cases.scale(), True)).reshape(B, S, Hq, D)
    kc = np.zeros((B, Hkv, cap, D), np.float32)
    vc = np.zeros((B, Hkv, cap, D), np.float32)
    q_ref = orc.qk_norm_rope_append(qkv, Hq, Hkv, cos, sin, np.zeros(B, np.int32), kc, vc, np.zeros(B, np.int32),
                                    qw, kw, 1e-6, 0, "bf16")
    st = np.zeros(B, np.int32)
    ref = orc.attn_prefill(q_ref.reshape(B, Hq, S, D), kc, vc, st, cases.scale(), True, "bf16").reshape(B, S, Hq, D)
    note(f"  q bit-identical {np.mean(host(qd).reshape(q_ref.shape) == q_ref):.5f}; "
         f"k rows bit-identical {np.mean(host(kd)[:, :, :S] == kc[:, :, :S]):.5f}")
    long_rows = np.arange(S) + 1 >= LONG_ROW_KEYS
    note(f"  prefill output vs oracle chain (max-abs, mean-rel): all rows {errors(out, ref)}; "
         f"long rows {errors(out[:, long_rows], ref[:, long_rows])}")
    assert_close(out, ref, "bf16", "c2 chain")


def test_prefill_last_row_equals_decode(gpu):
    """The last prefill row equals a decode of the same query over the same rows."""
    from crane_amd import ops
    q, k, v, st = cases.prefill_case(91, 2, 333, 16, 8, [0, 0], dtype="bf16", poison=False)
    qd, kd, vd = dev_t(q, "bf16", gpu), dev_t(k, "bf16", gpu), dev_t(v, "bf16", gpu)
    pre = host(ops.attention_prefill(qd, kd, vd, i32(st, gpu), 0))
    dec = host(ops.attention_decode(qd[:, :, -1].contiguous(), kd, vd, i32([333, 333], gpu), 333))
    assert np.max(np.abs(pre[:, -1] - dec[:, 0])) <= 2e-2


def test_decode_workspace_reuse_across_shapes(gpu, orc):
    """One workspace serves successive calls of different shapes, including
    calls with more (sequence, head) rows than an earlier one and a long call
    repeated after shorter ones: no call depends on what an earlier one left."""
    from crane_amd import ops
    ws = torch.zeros(ops.decode_workspace_bytes(8, 32, 8, 3000) + 4096, dtype=torch.uint8, device=gpu)
    for i, (B, Hq, Hkv, lens) in enumerate([(8, 32, 8, [3000, 1, 700, 2999, 256, 257, 1024, 77]),
                                             (3, 8, 2, [5, 600, 2048]), (8, 32, 8, [100] * 8),
                                             (24, 16, 8, [300 + 13 * j for j in range(24)]),
                                             (8, 32, 8, [3000, 1, 700, 2999, 256, 257, 1024, 77])]):
        note(f"workspace reuse call {i}: B={B} lens={lens}")
        q, k, v, lens = cases.decode_case(400 + i, B, Hq, Hkv, lens, dtype="bf16")
        out = host(ops.attention_decode(dev_t(q, "bf16", gpu), dev_t(k, "bf16", gpu), dev_t(v, "bf16", gpu),
                                        i32(lens, gpu), int(lens.max()), workspace=ws)).reshape(B, Hq * D)
        ref = orc.attn_decode(q, k, v, lens, cases.scale(), "bf16")
        assert_close(out, ref, "bf16", f"reuse call {i}")


def test_decode_64_heads_per_kv_head(gpu, orc):
    """64 q heads on one kv head (eight 8-head groups share each K/V row) over
    1025 ragged sequences, 65600 (sequence, head) rows in all."""
    from crane_amd import ops
    B, Hq, Hkv = 1025, 64, 1
    lens = cases.rng(57).integers(0, 520, size=B).astype(np.int32)
    note(f"decode 64 heads per kv head: B={B} Hq={Hq} Hkv={Hkv} max_len={lens.max()}")
    q, k, v, lens = cases.decode_case(58, B, Hq, Hkv, lens, dtype="bf16")
    out = host(ops.attention_decode(dev_t(q, "bf16", gpu), dev_t(k, "bf16", gpu), dev_t(v, "bf16", gpu),
                                    i32(lens, gpu), int(lens.max()))).reshape(B, Hq * D)
    ref = orc.attn_decode(q, k, v, lens, cases.scale(), "bf16")
    assert_close(out, ref, "bf16", "64 heads per kv head")


def test_decode_large_batch(gpu, orc):
    """A batch of 1100 ragged sequences, some of them empty."""
    from crane_amd import ops
    B, Hq, Hkv = 1100, 4, 2
    lens = cases.rng(55).integers(0, 600, size=B).astype(np.int32)
    note(f"decode large batch: B={B} max_len={lens.max()}")
    q, k, v, lens = cases.decode_case(56, B, Hq, Hkv, lens, dtype="bf16")
    out = host(ops.attention_decode(dev_t(q, "bf16", gpu), dev_t(k, "bf16", gpu), dev_t(v, "bf16", gpu),
                                    i32(lens, gpu), int(lens.max()))).reshape(B, Hq * D)
    ref = orc.attn_decode(q, k, v, lens, cases.scale(), "bf16")
    assert np.all(out[lens == 0] == 0)
    assert_close(out, ref, "bf16", "large batch")
