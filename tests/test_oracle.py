"""Pins of the CPU oracle (oracle/oracle.c) against what mathematics and
independent libraries fix.  The reference's own tests hold no vector for this
path (no test covers RoPE, QK-norm, the KV cache or SDPA), so each oracle
function is checked here against a closed form, a float64 brute force,
torch's SDPA, transformers' Qwen3 RoPE/RMSNorm functions, or an invariant,
chosen so that a dropped term, a wrong sign or index, or a transposed
operand fails.  CPU only."""
import math

import numpy as np
import pytest
import torch

from tests.tolerance import errors

D = 128


def _rng(seed):
    return np.random.default_rng(seed)


# ------------------------------------------------------------------ tables

def test_rope_tables_closed_form(orc):
    cos, sin = orc.rope_tables(D, 1e6, 40000)
    inv = np.array([np.float32(1.0) / np.float32(1e6 ** (i / D)) for i in range(0, D, 2)], np.float32)
    pos = np.arange(40000, dtype=np.float32)
    f = (pos[:, None] * inv[None, :]).astype(np.float32)       # one f32 rounding
    ref_c = np.cos(f.astype(np.float64))
    ref_s = np.sin(f.astype(np.float64))
    # glibc cosf/sinf are within 1 ulp of the exact value of the same f32 argument
    ulp = np.spacing(np.abs(ref_c).astype(np.float32)).astype(np.float64)
    assert np.all(np.abs(cos - ref_c) <= ulp + 1e-45)
    ulp = np.spacing(np.abs(ref_s).astype(np.float32)).astype(np.float64)
    assert np.all(np.abs(sin - ref_s) <= ulp + 1e-45)
    assert np.all(cos[0] == 1.0) and np.all(sin[0] == 0.0)      # identity row
    assert cos[1, 0] == np.float32(math.cos(1.0)) or abs(cos[1, 0] - math.cos(1.0)) < 1e-7
    # frequencies decrease along the row: at position 1 every angle inv[k] is
    # below pi/2, so sin falls strictly and cos rises (to 1 in f32) pair by pair
    assert np.all(np.diff(sin[1]) < 0) and np.all(np.diff(cos[1]) >= 0) and cos[1, -1] > cos[1, 0]
    assert inv[0] == 1.0 and inv[-1] < inv[1] < inv[0]


def test_rope_tables_hunyuan_alpha(orc):
    c0, s0 = orc.rope_tables(D, 10000.0, 64)
    c1, s1 = orc.rope_tables(D, 10000.0, 64, alpha=1000.0)
    base = 10000.0 * 1000.0 ** (D / (D - 2))
    inv = np.array([np.float32(1.0) / np.float32(base ** (i / D)) for i in range(0, D, 2)], np.float32)
    f = (np.arange(64, dtype=np.float32)[:, None] * inv[None, :]).astype(np.float32)
    assert np.max(np.abs(c1 - np.cos(f.astype(np.float64)))) < 1.2e-7
    assert not np.array_equal(c0, c1)                          # alpha changes the base


def test_rope_tables_qwen2_dtype(orc):
    c, s = orc.rope_tables(D, 1e6, 3000)
    cq, sq = orc.rope_tables_qwen2(D, 1e6, 3000, "f32")
    assert np.array_equal(c, cq) and np.array_equal(s, sq)     # same formula in f32
    cb, sb = orc.rope_tables_qwen2(D, 1e6, 3000, "bf16")
    # bf16 positions: 257 rounds to 256, so rows 256 and 257 coincide
    assert np.array_equal(cb[256], cb[257]) and not np.array_equal(c[256], c[257])
    # closed form of the bf16 chain: angle = bf16(bf16(p) * bf16(inv)), value = bf16(cos(angle))
    inv = orc.round_bf16(np.array([np.float32(1.0) / np.float32(1e6 ** (i / D)) for i in range(0, D, 2)],
                                  np.float32))
    pos = orc.round_bf16(np.arange(3000, dtype=np.float32))
    ang = orc.round_bf16((pos[:, None] * inv[None, :]).astype(np.float32))
    ref = orc.round_bf16(np.cos(ang.astype(np.float64)).astype(np.float32))
    assert np.max(np.abs(cb - ref)) <= 2 ** -8                  # at most one bf16 ulp apart
    assert np.mean(cb == ref) > 0.99
    # the angle rounding is large: row 199 differs from the f32 table by far more than bf16 noise
    assert np.max(np.abs(cb[199] - c[199])) > 0.1


def test_rope_tables_qwen2_host_builder(orc):
    """ops.rope_tables_qwen2 (the tables a Qwen2.5 model hands the append,
    built by the library's crane_hip_rope_tables_qwen2 on the host) equals the
    oracle's qwen2 chain bit for bit, in bf16 and f32."""
    import torch
    from crane_amd import ops
    cb, sb = orc.rope_tables_qwen2(D, 1e6, 3000, "bf16")
    tc, ts = ops.rope_tables_qwen2(D, 1e6, 3000, device="cpu", dtype=torch.bfloat16)
    assert np.array_equal(tc.float().numpy(), cb) and np.array_equal(ts.float().numpy(), sb)
    assert torch.equal(tc[256], tc[257])                       # positions rounded to bf16
    cf, sf = orc.rope_tables_qwen2(D, 1e6, 3000, "f32")
    tc, ts = ops.rope_tables_qwen2(D, 1e6, 3000, device="cpu", dtype=torch.float32)
    assert np.array_equal(tc.numpy(), cf) and np.array_equal(ts.numpy(), sf)


@pytest.mark.parametrize("theta,alpha,max_pos", [(1e6, 0.0, 40000), (1e4, 0.0, 5000), (1e4, 1000.0, 5000),
                                                 (1e6, 2.5, 33000)])
def test_rope_tables_host_builder(orc, theta, alpha, max_pos):
    """ops.rope_tables (the tables the fused append reads: qwen3/modeling.rs:
    117-139 cast to the model dtype as :857-864 does, and Hunyuan's NTK-alpha
    base) equals the oracle bit for bit: f32 tables, and bf16 tables equal to
    the oracle's f32 tables rounded to nearest even.  Positions up to c5's
    32769 rows are covered."""
    import torch
    from crane_amd import ops
    c, s = orc.rope_tables(D, theta, max_pos, alpha=alpha)
    tc, ts = ops.rope_tables(D, theta, max_pos, alpha=alpha, device="cpu", dtype=torch.float32)
    assert np.array_equal(tc.numpy(), c) and np.array_equal(ts.numpy(), s)
    bc, bs = ops.rope_tables(D, theta, max_pos, alpha=alpha, device="cpu", dtype=torch.bfloat16)
    assert np.array_equal(bc.float().numpy(), orc.round_bf16(c)) and np.array_equal(bs.float().numpy(), orc.round_bf16(s))


def test_rope_table_builder_argument_checks():
    import ctypes
    from crane_amd import _lib
    L = _lib.lib()
    buf = (ctypes.c_float * 64)()
    assert L.crane_hip_rope_tables(D, 1e6, 0.0, 1, 2, buf, buf) == _lib.E_DTYPE
    assert L.crane_hip_rope_tables(127, 1e6, 0.0, 1, 0, buf, buf) == _lib.E_INVALID
    assert L.crane_hip_rope_tables(D, -1.0, 0.0, 1, 0, buf, buf) == _lib.E_INVALID
    assert L.crane_hip_rope_tables(D, 1e6, -2.0, 1, 0, buf, buf) == _lib.E_INVALID
    assert L.crane_hip_rope_tables(D, 1e6, 0.0, 1, 0, None, buf) == _lib.E_INVALID
    assert L.crane_hip_rope_tables(D, 1e6, 0.0, 0, 0, None, None) == _lib.OK
    assert L.crane_hip_rope_tables_qwen2(D, 0.0, 1, 1, buf, buf) == _lib.E_INVALID


# ----------------------------------------------------------------- rmsnorm

@pytest.mark.parametrize("contiguous", [True, False])
def test_rms_norm_float64(orc, contiguous):
    x = _rng(1).standard_normal((64, D)).astype(np.float32) * 3
    w = _rng(2).standard_normal(D).astype(np.float32)
    y = orc.rms_norm(x, w, 1e-6, contiguous, "f32")
    x64 = x.astype(np.float64)
    ref = x64 / np.sqrt((x64 ** 2).mean(-1, keepdims=True) + 1e-6) * w
    assert np.max(np.abs(y - ref)) < 2e-6 * np.abs(ref).max()
    # output RMS is 1 with unit weight; scale equivariance f(c x) = f(x)
    y1 = orc.rms_norm(x, None, 1e-6, contiguous, "f32")
    assert np.allclose(np.sqrt((y1.astype(np.float64) ** 2).mean(-1)), 1.0, atol=1e-5)
    y2 = orc.rms_norm(x * 4.0, None, 1e-6, contiguous, "f32")
    assert np.allclose(y1, y2, atol=1e-6)


def test_rms_norm_bf16_paths(orc):
    x = orc.round_bf16(_rng(3).standard_normal((32, D)).astype(np.float32))
    a = orc.rms_norm(x, None, 1e-6, True, "bf16")
    b = orc.rms_norm(x, None, 1e-6, False, "bf16")
    assert np.array_equal(a, orc.round_bf16(a)) and np.array_equal(b, orc.round_bf16(b))
    x64 = x.astype(np.float64)
    ref = x64 / np.sqrt((x64 ** 2).mean(-1, keepdims=True) + 1e-6)
    assert np.max(np.abs(a - ref)) <= 2 ** -7 * np.abs(ref).max()
    assert np.max(np.abs(b - ref)) <= 2 ** -8 * np.abs(ref).max()


def test_rms_norm_vs_transformers(orc):
    from transformers.models.qwen3.modeling_qwen3 import Qwen3RMSNorm
    x = _rng(4).standard_normal((16, D)).astype(np.float32)
    w = _rng(5).standard_normal(D).astype(np.float32)
    m = Qwen3RMSNorm(D, eps=1e-6)
    with torch.no_grad():
        m.weight.copy_(torch.from_numpy(w))
        ref = m(torch.from_numpy(x)).numpy()
    y = orc.rms_norm(x, w, 1e-6, False, "f32")
    assert np.max(np.abs(y - ref)) < 1e-5


# -------------------------------------------------------------------- rope

def test_rope_vs_transformers(orc):
    from transformers.models.qwen3.modeling_qwen3 import apply_rotary_pos_emb
    cos, sin = orc.rope_tables(D, 1e6, 5000)
    S = 7
    pos = np.array([0, 1, 2, 100, 999, 3000, 4999], np.int32)
    x = _rng(6).standard_normal((S, D)).astype(np.float32)
    y = orc.rope(x, cos, sin, pos, "f32")
    c = torch.from_numpy(np.concatenate([cos[pos], cos[pos]], -1))[None]
    s = torch.from_numpy(np.concatenate([sin[pos], sin[pos]], -1))[None]
    xt = torch.from_numpy(x)[None, None]
    qr, _ = apply_rotary_pos_emb(xt, xt, c, s)
    assert np.max(np.abs(y - qr[0, 0].numpy())) < 1e-6
    assert np.array_equal(y[0], x[0])                              # position 0 is the identity


def test_rope_invariants(orc):
    cos, sin = orc.rope_tables(D, 1e6, 4096)
    x = _rng(7).standard_normal((3, D)).astype(np.float32)
    p = np.array([5, 1000, 4000], np.int32)
    y = orc.rope(x, cos, sin, p, "f32")
    pair = lambda v: v[:, :D // 2] ** 2 + v[:, D // 2:] ** 2
    assert np.allclose(pair(y.astype(np.float64)), pair(x.astype(np.float64)), rtol=1e-5, atol=1e-6)
    # rotation by p1 then p2 equals rotation by p1+p2 (float64 angles)
    inv = 1.0 / (1e6 ** (np.arange(0, D, 2) / D))

    def rot(v, ang):
        c, s = np.cos(ang), np.sin(ang)
        a, b = v[:D // 2], v[D // 2:]
        return np.concatenate([a * c - b * s, a * s + b * c])
    v = x[0].astype(np.float64)
    assert np.allclose(rot(rot(v, 3 * inv), 4 * inv), rot(v, 7 * inv), atol=1e-12)
    y7 = orc.rope(x[:1], cos, sin, np.array([7], np.int32), "f32")[0]
    assert np.max(np.abs(y7 - rot(v, np.float32(7) * inv.astype(np.float32)))) < 1e-5
    # sign convention: the first half gets -x2*sin
    e = np.zeros((1, D), np.float32); e[0, D // 2] = 1.0
    ye = orc.rope(e, cos, sin, np.array([1], np.int32), "f32")[0]
    assert ye[0] == -sin[1, 0] and ye[D // 2] == cos[1, 0]


# ------------------------------------------------------------ fused append

@pytest.mark.parametrize("order", [0, 1, 2])
@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_append_composition(orc, order, dtype):
    B, S, Hq, Hkv, cap = 2, 3, 4, 2, 16
    cos, sin = orc.rope_tables(D, 1e6, 64)
    if dtype == "bf16":
        cos, sin = orc.round_bf16(cos), orc.round_bf16(sin)
    qkv = _rng(8).standard_normal((B, S, (Hq + 2 * Hkv) * D)).astype(np.float32)
    if dtype == "bf16":
        qkv = orc.round_bf16(qkv)
    qw = (1 + 0.1 * _rng(9).standard_normal(D)).astype(np.float32)
    kw = (1 + 0.1 * _rng(10).standard_normal(D)).astype(np.float32)
    if dtype == "bf16":
        qw, kw = orc.round_bf16(qw), orc.round_bf16(kw)
    kc = np.full((B, Hkv, cap, D), 7.0, np.float32)   # canary
    vc = np.full((B, Hkv, cap, D), 7.0, np.float32)
    clen = np.array([2, 9], np.int32)
    posn = np.array([2, 11], np.int32)
    q = orc.qk_norm_rope_append(qkv, Hq, Hkv, cos, sin, posn, kc, vc, clen, qw, kw, 1e-6, order, dtype)
    contiguous = S == 1
    for b in range(B):
        for s in range(S):
            row = qkv[b, s]
            pos = np.array([posn[b] + s], np.int32)
            for h in range(Hq + Hkv):
                x = row[h * D:(h + 1) * D][None]
                w = qw if h < Hq else kw
                if order == 0:
                    ref = orc.rope(orc.rms_norm(x, w, 1e-6, contiguous, dtype), cos, sin, pos, dtype)
                elif order == 1:
                    ref = orc.rms_norm(orc.rope(x, cos, sin, pos, dtype), w, 1e-6, True, dtype)
                else:
                    ref = orc.rope(x, cos, sin, pos, dtype)
                got = q[b, h, s] if h < Hq else kc[b, h - Hq, clen[b] + s]
                assert np.array_equal(got, ref[0]), (b, s, h)
            for h in range(Hkv):
                v = row[(Hq + Hkv + h) * D:(Hq + Hkv + h + 1) * D]
                assert np.array_equal(vc[b, h, clen[b] + s], v)
    # rows outside [len, len+S) untouched
    for b in range(B):
        mask = np.ones(cap, bool)
        mask[clen[b]:clen[b] + S] = False
        assert np.all(kc[b][:, mask] == 7.0) and np.all(vc[b][:, mask] == 7.0)


def test_append_capacity(orc):
    cos, sin = orc.rope_tables(D, 1e6, 64)
    qkv = np.zeros((1, 4, 4 * D), np.float32)
    kc = np.zeros((1, 1, 5, D), np.float32)
    with pytest.raises(ValueError):
        orc.qk_norm_rope_append(qkv, 2, 1, cos, sin, np.array([2], np.int32), kc, kc.copy(),
                                np.array([2], np.int32))


# ------------------------------------------------------------------ decode

def _brute_attn(q, K, V, scale, causal_upto=None):
    """float64 softmax(q K^T * scale) V for one query row."""
    s = (K.astype(np.float64) @ q.astype(np.float64)) * scale
    if causal_upto is not None:
        s[causal_upto + 1:] = -np.inf
    p = np.exp(s - s.max())
    p /= p.sum()
    return p @ V.astype(np.float64)


def _decode_inputs(seed, B, Hq, Hkv, cap, lens, dtype, std=1.0):
    r = _rng(seed)
    q = r.standard_normal((B, Hq, D)).astype(np.float32)
    k = (std * r.standard_normal((B, Hkv, cap, D))).astype(np.float32)
    v = (std * r.standard_normal((B, Hkv, cap, D))).astype(np.float32)
    if dtype == "bf16":
        import oracle
        q, k, v = oracle.round_bf16(q), oracle.round_bf16(k), oracle.round_bf16(v)
    return q, k, v, np.array(lens, np.int32)


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
@pytest.mark.parametrize("variant", [0, 1])
def test_decode_float64(orc, dtype, variant):
    B, Hq, Hkv = 3, 8, 2
    q, k, v, lens = _decode_inputs(11, B, Hq, Hkv, 300, [1, 77, 300], dtype)
    sc = 1 / math.sqrt(D)
    out = orc.attn_decode(q, k, v, lens, sc, dtype, variant).reshape(B, Hq, D)
    ref = np.stack([np.stack([_brute_attn(q[b, h], k[b, h // 4, :lens[b]], v[b, h // 4, :lens[b]], sc)
                              for h in range(Hq)]) for b in range(B)])
    ma, mr = errors(out, ref)
    if dtype == "f32":
        assert ma < 2e-6
    else:
        assert ma < 1e-2 and mr < 8e-3
    # sequence 0 has one key: the output is that V row
    assert np.allclose(out[0], np.repeat(v[0, :, 0][:, None], 4, 1).reshape(Hq, D), atol=1e-2 if dtype == "bf16" else 1e-6)


def test_decode_vs_torch_sdpa(orc):
    B, Hq, Hkv, L = 2, 16, 8, 200
    q, k, v, lens = _decode_inputs(12, B, Hq, Hkv, L, [L, L], "f32")
    out = orc.attn_decode(q, k, v, lens, 1 / math.sqrt(D))
    ref = torch.nn.functional.scaled_dot_product_attention(
        torch.from_numpy(q)[:, :, None], torch.from_numpy(k), torch.from_numpy(v), enable_gqa=True)
    assert np.max(np.abs(out - ref.reshape(B, Hq * D).numpy())) < 2e-6


def test_decode_special_cases(orc):
    B, Hq, Hkv, L = 1, 4, 1, 50
    q, k, v, lens = _decode_inputs(13, B, Hq, Hkv, L, [L], "f32")
    keq = np.repeat(k[:, :, :1], L, axis=2)               # all keys equal -> mean of V
    out = orc.attn_decode(q, keq, v, lens, 1 / math.sqrt(D)).reshape(Hq, D)
    assert np.allclose(out, v[0, 0].mean(0)[None], atol=1e-6)
    kd = k.copy()
    kd[0, 0, 17] = q[0, 0] * 100.0                          # one dominant key for head 0
    out = orc.attn_decode(q, kd, v, lens, 1 / math.sqrt(D)).reshape(Hq, D)
    assert np.allclose(out[0], v[0, 0, 17], atol=1e-5)


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_decode_padded_equals_varlen(orc, dtype):
    q, k, v, lens = _decode_inputs(14, 4, 8, 2, 130, [3, 130, 64, 65], dtype)
    a = orc.attn_decode(q, k, v, lens, 1 / math.sqrt(D), dtype)
    b = orc.attn_decode_padded(q, k, v, lens, 1 / math.sqrt(D), dtype)
    assert np.array_equal(a, b)


# ----------------------------------------------------------------- prefill

def _prefill_inputs(seed, B, S, Hq, Hkv, start, dtype):
    r = _rng(seed)
    L = max(start) + S
    q = r.standard_normal((B, Hq, S, D)).astype(np.float32)
    k = r.standard_normal((B, Hkv, L, D)).astype(np.float32)
    v = r.standard_normal((B, Hkv, L, D)).astype(np.float32)
    if dtype == "bf16":
        import oracle
        q, k, v = oracle.round_bf16(q), oracle.round_bf16(k), oracle.round_bf16(v)
    return q, k, v, np.array(start, np.int32)


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_prefill_float64(orc, dtype):
    B, S, Hq, Hkv = 2, 37, 6, 2
    q, k, v, st = _prefill_inputs(15, B, S, Hq, Hkv, [0, 9], dtype)
    sc = 1 / math.sqrt(D)
    out = orc.attn_prefill(q, k, v, st, sc, True, dtype).reshape(B, S, Hq, D)
    ref = np.zeros_like(out, dtype=np.float64)
    for b in range(B):
        for h in range(Hq):
            for i in range(S):
                L = st[b] + S
                ref[b, i, h] = _brute_attn(q[b, h, i], k[b, h // 3, :L], v[b, h // 3, :L], sc,
                                           causal_upto=st[b] + i)
    ma, mr = errors(out, ref)
    if dtype == "f32":
        assert ma < 2e-6
    else:
        assert ma < 2e-2 and mr < 8e-3
    # causal row 0 of a fresh sequence sees only key 0
    assert np.allclose(out[0, 0], np.repeat(v[0, :, 0], 3, 0), atol=1e-6 if dtype == "f32" else 1e-2)


def test_prefill_vs_torch_sdpa(orc):
    B, S, Hq, Hkv = 2, 64, 8, 2
    q, k, v, st = _prefill_inputs(16, B, S, Hq, Hkv, [0, 0], "f32")
    out = orc.attn_prefill(q, k, v, st, 1 / math.sqrt(D), True, "f32")
    ref = torch.nn.functional.scaled_dot_product_attention(
        torch.from_numpy(q), torch.from_numpy(k), torch.from_numpy(v), is_causal=True, enable_gqa=True)
    assert np.max(np.abs(out - ref.transpose(1, 2).reshape(B, S, Hq * D).numpy())) < 2e-6


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_prefill_mask_kinds_and_rows(orc, dtype):
    q, k, v, st = _prefill_inputs(17, 1, 50, 4, 2, [5], dtype)
    sc = 1 / math.sqrt(D)
    a = orc.attn_prefill(q, k, v, st, sc, True, dtype, orc.MASK_NEG_1E9)
    b = orc.attn_prefill(q, k, v, st, sc, True, dtype, orc.MASK_NEG_INF)
    assert np.array_equal(a, b)
    part = orc.attn_prefill(q, k, v, st, sc, True, dtype, rows=(10, 20), heads=(1, 3))
    a4 = a.reshape(1, 50, 4, D)
    p4 = part.reshape(1, 50, 4, D)
    assert np.array_equal(p4[:, 10:20, 1:3], a4[:, 10:20, 1:3])
    assert np.all(p4[:, :10] == 0) and np.all(p4[:, :, 0] == 0)


def test_decode_equals_last_prefill_row(orc):
    """S=1 decode of the last token == last row of a causal prefill (f32; the
    decode path pre-scales q, the prefill path post-scales the scores)."""
    B, S, Hq, Hkv = 1, 20, 4, 2
    q, k, v, st = _prefill_inputs(18, B, S, Hq, Hkv, [0], "f32")
    pre = orc.attn_prefill(q, k, v, st, 1 / math.sqrt(D), True, "f32").reshape(B, S, Hq * D)
    dec = orc.attn_decode(np.ascontiguousarray(q[:, :, -1]), k, v, np.array([S], np.int32), 1 / math.sqrt(D))
    assert np.max(np.abs(pre[:, -1] - dec)) < 1e-6


def test_generator_is_deterministic(orc):
    a = orc.gen_normal(0xC3A7E001, 10001)
    b = orc.gen_normal(0xC3A7E001, 10001)
    assert np.array_equal(a, b) and abs(a.mean()) < 0.05 and abs(a.std() - 1) < 0.05
    i = orc.gen_uniform_int(0xC3A7E003, 1000, 512, 4096)
    assert i.min() >= 512 and i.max() <= 4096 and np.array_equal(i, orc.gen_uniform_int(0xC3A7E003, 1000, 512, 4096))
