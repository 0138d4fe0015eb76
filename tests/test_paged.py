"""Paged KV cache (include/crane_hip.h paged launchers, include/crane_pkv.h).

The paged launchers run the same arithmetic as the dense ones over the same
rows, so the bar is bit-equality with the dense entry points on identical
inputs, which are themselves held to the oracle elsewhere; the manager's flows
are checked against the oracle and against exact row bookkeeping.  Pool rows
that belong to no sequence hold NaN, so a kernel that read one would show it.
The manager replaces Crane's per-round copies (setup_batch_decode /
extract_batch_kv, qwen3/modeling.rs:973-1102) and update_kv_cache's
reallocation copy (:333-355)."""
import ctypes
import math

import numpy as np
import pytest

import cases
from tolerance import assert_close

D = 128


# ------------------------------------------------------------------ CPU

def test_paged_launcher_argument_checks():
    from crane_amd import _lib
    L = _lib.lib()
    # (q, k, v, n_pages, page_rows, table, stride, kv_len, max_kv, B, Hq, Hkv, D, scale, score_mode, ws, ws_bytes,
    #  out, dt, st)
    base = [16, 16, 16, 64, 256, 16, 8, 16, 1024, 1, 32, 8, 128, 0.088, 0, 16, 1 << 30, 16, 1, None]

    def dec(**kw):
        a = list(base)
        idx = dict(n_pages=3, page_rows=4, table=5, stride=6, max_kv=8, D=12, score=14, dt=18)
        for k, v in kw.items():
            a[idx[k]] = v
        return L.crane_hip_attn_decode_paged(*a)

    assert dec(page_rows=100) == _lib.E_INVALID          # not a multiple of 256
    assert dec(page_rows=0) == _lib.E_INVALID
    assert dec(n_pages=0) == _lib.E_INVALID
    assert dec(table=None) == _lib.E_INVALID
    assert dec(stride=0) == _lib.E_INVALID
    assert dec(max_kv=8 * 256 + 1) == _lib.E_CAPACITY    # more rows than the table can map
    assert dec(D=64) == _lib.E_HEAD_DIM
    assert dec(dt=5) == _lib.E_DTYPE
    assert dec(score=2) == _lib.E_INVALID
    assert L.crane_hip_attn_prefill_paged(16, 16, 16, 64, 256, 16, 2, 16, 400, 1, 200, 32, 8, 128, 0.088, 1, 16,
                                          1, None) == _lib.E_CAPACITY  # 400 + 200 > 2 pages of 256
    assert L.crane_hip_qknorm_rope_append_paged(16, 40 * 128, None, None, 1e-6, 0, 16, 16, 64, 4096, 16, 16, 16, 16,
                                                64, 512, 16, 1, 16, 1, 513, 32, 4, 128, 1, None) == _lib.E_CAPACITY


def test_pkv_create_argument_checks():
    from crane_amd import _lib
    L = _lib.lib()
    h = ctypes.c_void_p()
    assert L.crane_pkv_create(8, 128, 1, 100, 16, 4, 4, ctypes.byref(h)) == _lib.E_INVALID  # page_rows
    assert L.crane_pkv_create(8, 64, 1, 256, 16, 4, 4, ctypes.byref(h)) == _lib.E_HEAD_DIM
    assert L.crane_pkv_create(8, 128, 3, 256, 16, 4, 4, ctypes.byref(h)) == _lib.E_DTYPE
    assert L.crane_pkv_create(8, 128, 1, 256, 0, 4, 4, ctypes.byref(h)) == _lib.E_INVALID
    assert L.crane_pkv_create(0, 128, 1, 256, 16, 4, 4, ctypes.byref(h)) == _lib.E_INVALID
    assert L.crane_pkv_create(8, 128, 1, 256, 16, 0, 4, ctypes.byref(h)) == _lib.E_INVALID
    assert L.crane_pkv_create(8, 128, 1, 256, 16, 4, 0, ctypes.byref(h)) == _lib.E_INVALID
    assert L.crane_pkv_seq_len(None, 0) == -1 and L.crane_pkv_free_pages(None) == 0


# ------------------------------------------------------------------ GPU helpers

def _t(x, dtype, dev):
    import torch
    t = torch.from_numpy(np.ascontiguousarray(x))
    return (t.to(torch.bfloat16) if dtype == "bf16" else t).to(dev)


def to_paged(k, v, rows, page_rows, seed, extra_pages=3):
    """Scatter rows [0, rows[b]) of dense caches [B, Hkv, cap, D] into pools
    [n_pages, Hkv, page_rows, D] on shuffled pages; every other pool row is NaN.
    Returns (k_pool, v_pool, table [B, stride] int32, stride)."""
    B, Hkv, _, _ = k.shape
    need = [max(1, math.ceil(int(r) / page_rows)) for r in rows]
    stride = max(need) + 1
    n_pages = sum(need) + extra_pages
    perm = cases.rng(seed).permutation(n_pages).astype(np.int32)
    kp = np.full((n_pages, Hkv, page_rows, D), np.nan, np.float32)
    vp = np.full_like(kp, np.nan)
    table = np.full((B, stride), -1, np.int32)
    nxt = 0
    for b in range(B):
        for i in range(need[b]):
            page = perm[nxt]
            nxt += 1
            table[b, i] = page
            r0, r1 = i * page_rows, min(int(rows[b]), (i + 1) * page_rows)
            if r1 > r0:
                kp[page, :, :r1 - r0] = k[b, :, r0:r1]
                vp[page, :, :r1 - r0] = v[b, :, r0:r1]
    return kp, vp, table, stride


def from_paged(pool, table, b, n, page_rows):
    """Rows [0, n) of sequence b as [Hkv, n, D] (host)."""
    out = []
    for i in range(math.ceil(n / page_rows)):
        r = min(page_rows, n - i * page_rows)
        out.append(pool[table[b, i], :, :r])
    return np.concatenate(out, axis=1) if out else pool[:0, :, :0].reshape(pool.shape[1], 0, D)


# ------------------------------------------------------------------ GPU: launchers

@pytest.mark.gpu
@pytest.mark.parametrize("dtype,page_rows,Hq,Hkv", [("bf16", 256, 32, 8), ("bf16", 512, 64, 8), ("f32", 256, 16, 8)])
def test_paged_decode_equals_dense(gpu, dtype, page_rows, Hq, Hkv):
    import torch
    from crane_amd import ops
    lens = np.array([1, 255, 256, 257, 700, 1500, 31, 1024], np.int32)
    print(f"paged decode {dtype} P={page_rows} Hq={Hq} Hkv={Hkv}", flush=True)
    q, k, v, lens = cases.decode_case(9100 + page_rows, len(lens), Hq, Hkv, lens, dtype=dtype)
    kp, vp, table, _ = to_paged(k, v, lens, page_rows, seed=17)
    kvl = torch.as_tensor(lens, device=gpu)
    want = ops.attention_decode(_t(q, dtype, gpu), _t(k, dtype, gpu), _t(v, dtype, gpu), kvl, int(lens.max()))
    got = ops.attention_decode_paged(_t(q, dtype, gpu), _t(kp, dtype, gpu), _t(vp, dtype, gpu),
                                     torch.as_tensor(table, device=gpu), kvl, int(lens.max()))
    assert not torch.isnan(got).any()
    assert torch.equal(got, want)


@pytest.mark.gpu
@pytest.mark.parametrize("page_rows", [512, 256])
def test_paged_decode_long_context(gpu, orc, page_rows):
    """Past 12288 keys the dense launcher takes 512-key chunks; so does the
    paged one when a page holds whole 512-row chunks (then the two are
    bit-equal), and 256-row pages keep 256-key chunks (checked against the
    oracle)."""
    import torch
    from crane_amd import ops
    lens = np.array([12289, 14000, 600], np.int32)
    print(f"paged decode long P={page_rows}", flush=True)
    q, k, v, lens = cases.decode_case(9300 + page_rows, len(lens), 16, 2, lens, dtype="bf16")
    kp, vp, table, _ = to_paged(k, v, lens, page_rows, seed=19)
    kvl = torch.as_tensor(lens, device=gpu)
    got = ops.attention_decode_paged(_t(q, "bf16", gpu), _t(kp, "bf16", gpu), _t(vp, "bf16", gpu),
                                     torch.as_tensor(table, device=gpu), kvl, int(lens.max()))
    assert not torch.isnan(got).any()
    if page_rows % 512 == 0:
        want = ops.attention_decode(_t(q, "bf16", gpu), _t(k, "bf16", gpu), _t(v, "bf16", gpu), kvl, int(lens.max()))
        assert torch.equal(got, want)
    ref = orc.attn_decode(q, k, v, lens, cases.scale(), "bf16")
    assert_close(got.float().cpu().numpy().reshape(ref.shape), ref, "bf16", f"paged long P={page_rows}")


@pytest.mark.gpu
@pytest.mark.parametrize("dtype,causal,start", [("bf16", True, [0, 0]), ("bf16", True, [200, 37]),
                                                ("bf16", False, [64, 300]), ("f32", True, [5, 130]),
                                                ("bf16", True, [1100, 700]), ("bf16", False, [1500, 900])])
def test_paged_prefill_equals_dense(gpu, dtype, causal, start):
    import torch
    from crane_amd import ops
    B, S, Hq, Hkv = 2, 300 if dtype == "bf16" else 70, 14, 2
    print(f"paged prefill {dtype} causal={causal} start={start}", flush=True)
    q, k, v, st = cases.prefill_case(9200 + sum(start), B, S, Hq, Hkv, start, dtype=dtype)
    rows = st + S
    kp, vp, table, _ = to_paged(k, v, rows, 256, seed=19)
    stt = torch.as_tensor(st, device=gpu)
    want = ops.attention_prefill(_t(q, dtype, gpu), _t(k, dtype, gpu), _t(v, dtype, gpu), stt, int(st.max()),
                                 causal=causal)
    got = ops.attention_prefill_paged(_t(q, dtype, gpu), _t(kp, dtype, gpu), _t(vp, dtype, gpu),
                                      torch.as_tensor(table, device=gpu), stt, int(st.max()), causal=causal)
    assert not torch.isnan(got).any()
    assert torch.equal(got, want)


@pytest.mark.gpu
@pytest.mark.parametrize("dtype,S", [("bf16", 1), ("bf16", 300), ("f32", 3)])
def test_paged_append_equals_dense(gpu, orc, dtype, S):
    """The fused append writes the same rows and q as the dense launcher; rows
    cross a page boundary, and nothing else in the pools changes."""
    import torch
    from crane_amd import ops
    B, Hq, Hkv = 3, 8, 2
    cache_len = np.array([250, 0, 511], np.int32)
    r = cases.rng(9300 + S)
    qkv = cases.cast(cases.normal(r, (B, S, (Hq + 2 * Hkv) * D)), dtype)
    cos, sin = orc.rope_tables(D, 1e6, 1024)
    cos, sin = cases.cast(cos, dtype), cases.cast(sin, dtype)
    cap = int(cache_len.max()) + S
    k0 = cases.cast(cases.normal(r, (B, Hkv, cap, D)), dtype)
    v0 = cases.cast(cases.normal(r, (B, Hkv, cap, D)), dtype)
    kp, vp, table, _ = to_paged(k0, v0, cache_len + S, 256, seed=23)
    kd, vd = _t(k0, dtype, gpu), _t(v0, dtype, gpu)
    kpt, vpt = _t(kp, dtype, gpu), _t(vp, dtype, gpu)
    before_k = kpt.clone()
    pos = torch.as_tensor(cache_len, device=gpu)
    args = (_t(qkv, dtype, gpu), _t(cos, dtype, gpu), _t(sin, dtype, gpu), pos)
    q_want = ops.qk_norm_rope_append(*args, kd, vd, pos, cap, Hq, Hkv)
    q_got = ops.qk_norm_rope_append_paged(*args, kpt, vpt, torch.as_tensor(table, device=gpu), pos, Hq)
    assert torch.equal(q_got, q_want)
    kh, vh, kdh, vdh = (x.float().cpu().numpy() for x in (kpt, vpt, kd, vd))
    for b in range(B):
        n = int(cache_len[b]) + S
        assert np.array_equal(from_paged(kh, table, b, n, 256), kdh[b, :, :n])
        assert np.array_equal(from_paged(vh, table, b, n, 256), vdh[b, :, :n])
    # pages no sequence owns are untouched (NaN stays NaN)
    owned = set(int(x) for x in table.ravel() if x >= 0)
    for p in range(kp.shape[0]):
        if p not in owned:
            assert torch.isnan(kpt[p].float()).all() and torch.equal(kpt[p].isnan(), before_k[p].isnan())


@pytest.mark.gpu
def test_invalid_page_ids_read_zero_and_are_not_written(gpu):
    """A page id outside the pool is never dereferenced: decode sees zero rows
    there, and an append aimed at it writes nothing."""
    import torch
    from crane_amd import ops
    lens = np.array([600, 300], np.int32)
    q, k, v, lens = cases.decode_case(9400, 2, 8, 2, lens, dtype="bf16")
    kp, vp, table, _ = to_paged(k, v, lens, 256, seed=29)
    table[0, 1] = 10 ** 6      # rows 256..511 of sequence 0
    table[1, 0] = -5           # rows 0..255 of sequence 1
    kz, vz = k.copy(), v.copy()
    kz[0, :, 256:512] = 0
    vz[0, :, 256:512] = 0
    kz[1, :, 0:256] = 0
    vz[1, :, 0:256] = 0
    kvl = torch.as_tensor(lens, device=gpu)
    want = ops.attention_decode(_t(q, "bf16", gpu), _t(kz, "bf16", gpu), _t(vz, "bf16", gpu), kvl, 600)
    kpt, vpt, tt = _t(kp, "bf16", gpu), _t(vp, "bf16", gpu), torch.as_tensor(table, device=gpu)
    got = ops.attention_decode_paged(_t(q, "bf16", gpu), kpt, vpt, tt, kvl, 600)
    assert torch.equal(got, want)
    before = kpt.clone()
    qkv = _t(cases.bf16(cases.normal(cases.rng(9401), (2, 1, 12 * D))), "bf16", gpu)
    cos = torch.ones((1024, 64), dtype=torch.bfloat16, device=gpu)
    ops.qk_norm_rope_append_paged(qkv, cos, torch.zeros_like(cos), torch.as_tensor([300, 100], device=gpu, dtype=torch.int32),
                                  kpt, vpt, tt, torch.as_tensor([300, 100], device=gpu, dtype=torch.int32), 8)
    torch.cuda.synchronize()
    assert torch.equal(kpt.isnan(), before.isnan()) and torch.equal(torch.nan_to_num(kpt), torch.nan_to_num(before))


# ------------------------------------------------------------------ GPU: manager

@pytest.mark.gpu
def test_pkv_batched_decode_flow(gpu, orc):
    """Sequences written, batched, grown by one-token appends across page
    boundaries, decoded (oracle), read back exactly; pages are accounted."""
    import torch
    from crane_amd import kv
    Hq, Hkv, P = 8, 2, 256
    c = kv.PagedKvCache(Hkv, n_pages=16, page_rows=P, max_seqs=4, max_pages_per_seq=6, device=gpu)
    assert c.free_pages == 16 and c.bytes == 2 * 16 * Hkv * P * D * 2
    lens = [255, 1, 512]
    g = torch.Generator(device=gpu).manual_seed(31)
    ids, rows = [], []
    for L in lens:
        sid = c.add_sequence()
        kk = torch.randn((Hkv, L, D), generator=g, device=gpu).to(torch.bfloat16)
        vv = torch.randn((Hkv, L, D), generator=g, device=gpu).to(torch.bfloat16)
        c.write_sequence(sid, kk, vv)
        ids.append(sid)
        rows.append([kk, vv])
    assert c.free_pages == 16 - (1 + 1 + 2)
    c.set_batch(ids)
    for step in range(3):
        kn = torch.randn((3, Hkv, 1, D), generator=g, device=gpu).to(torch.bfloat16)
        vn = torch.randn((3, Hkv, 1, D), generator=g, device=gpu).to(torch.bfloat16)
        c.update_kv_cache(kn, vn)
        for i in range(3):
            rows[i][0] = torch.cat([rows[i][0], kn[i]], 1)
            rows[i][1] = torch.cat([rows[i][1], vn[i]], 1)
    assert c.lengths == [L + 3 for L in lens]
    assert c.free_pages == 16 - (2 + 1 + 3)   # 255 -> 258 and 512 -> 515 each opened a page
    q = orc.round_bf16(cases.normal(cases.rng(9500), (3, Hq, D)))
    got = c.decode(_t(q, "bf16", gpu)).float().cpu().numpy().reshape(3, Hq * D)
    n = max(c.lengths)
    kn_ = np.zeros((3, Hkv, n, D), np.float32)
    vn_ = np.zeros_like(kn_)
    for i in range(3):
        kn_[i, :, :c.lengths[i]] = rows[i][0].float().cpu().numpy()
        vn_[i, :, :c.lengths[i]] = rows[i][1].float().cpu().numpy()
    ref = orc.attn_decode(q, kn_, vn_, np.array(c.lengths, np.int32), 1 / math.sqrt(D), "bf16")
    assert_close(got, ref, "bf16", "paged batched decode")
    for i, sid in enumerate(ids):
        kr, vr = c.read_sequence(sid)
        assert torch.equal(kr, rows[i][0]) and torch.equal(vr, rows[i][1])
    # a smaller batch, then releasing a sequence returns its pages for reuse
    c.set_batch([ids[2]])
    assert c.lengths == [515]
    c.set_batch([])
    c.free_sequence(ids[0])
    assert c.free_pages == 16 - (1 + 3)
    sid = c.add_sequence()
    assert sid == ids[0]
    c.write_sequence(sid, rows[1][0], rows[1][1])
    kr, _ = c.read_sequence(sid)
    assert torch.equal(kr, rows[1][0])
    c.close()


@pytest.mark.gpu
def test_pkv_prefill_and_capacity(gpu, orc):
    """A chunked prefill through the fused append and the paged prefill equals
    the dense launchers on the same rows; running out of pages is an error
    that changes nothing."""
    import torch
    from crane_amd import _lib, kv, ops
    Hq, Hkv, P = 8, 2, 256
    c = kv.PagedKvCache(Hkv, n_pages=6, page_rows=P, max_seqs=2, max_pages_per_seq=4, device=gpu)
    a, b = c.add_sequence(), c.add_sequence()
    c.set_batch([a, b])
    cos, sin = orc.rope_tables(D, 1e6, 2048)
    cos, sin = _t(orc.round_bf16(cos), "bf16", gpu), _t(orc.round_bf16(sin), "bf16", gpu)
    dense_k = torch.zeros((2, Hkv, 1024, D), dtype=torch.bfloat16, device=gpu)
    dense_v = torch.zeros_like(dense_k)
    n = 0
    for i, S in enumerate((300, 200)):
        print(f"pkv prefill chunk {i} S={S}", flush=True)
        qkv = _t(orc.round_bf16(cases.normal(cases.rng(9600 + i), (2, S, (Hq + 2 * Hkv) * D))), "bf16", gpu)
        pos = torch.full((2,), n, dtype=torch.int32, device=gpu)
        q = c.append_qkv(qkv, cos, sin, pos, Hq)
        q_dense = ops.qk_norm_rope_append(qkv, cos, sin, pos, dense_k, dense_v, pos, n + S, Hq, Hkv)
        assert torch.equal(q, q_dense)
        n += S
        got = c.prefill(q)
        want = ops.attention_prefill(q, dense_k, dense_v, torch.full((2,), n - S, dtype=torch.int32, device=gpu),
                                     n - S)
        assert torch.equal(got, want)
    assert c.lengths == [500, 500] and c.free_pages == 6 - 4
    pos = torch.full((2,), 500, dtype=torch.int32, device=gpu)
    # 300 more rows need 2 more pages per sequence, 2 are free; 600 more rows
    # exceed the 4 pages a sequence may hold: both rejected, nothing changes
    for S in (300, 600):
        qkv = torch.zeros((2, S, (Hq + 2 * Hkv) * D), dtype=torch.bfloat16, device=gpu)
        with pytest.raises(_lib.CraneHipError) as e:
            c.append_qkv(qkv, cos, sin, pos, Hq)
        assert e.value.code == _lib.E_CAPACITY
        assert c.lengths == [500, 500] and c.free_pages == 2
    # 20 more rows take the 2 free pages; the launch is rejected (eps < 0) and
    # the pages go back
    qkv = torch.zeros((2, 20, (Hq + 2 * Hkv) * D), dtype=torch.bfloat16, device=gpu)
    with pytest.raises(_lib.CraneHipError) as e:
        c.append_qkv(qkv, cos, sin, pos, Hq, eps=-1.0)
    assert e.value.code == _lib.E_INVALID
    assert c.lengths == [500, 500] and c.free_pages == 2
    q = c.append_qkv(qkv, cos, sin, pos, Hq)   # and the same call with a valid eps succeeds
    assert c.lengths == [520, 520] and c.free_pages == 0
    kr, vr = c.read_sequence(b)
    assert torch.equal(kr[:, :500], dense_k[1, :, :500]) and torch.equal(vr[:, :500], dense_v[1, :, :500])
    c.close()
