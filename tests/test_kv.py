"""Host-side KV-cache manager (include/crane_kv.h, crane_amd/kv.py): Crane's
update_kv_cache growth policy (qwen3/modeling.rs:313-370), the batched-decode
set-up / tear-down (setup_batch_decode :973-1030, extract_batch_kv
:1066-1102) without padding, and attention through the cache."""
import math

import numpy as np
import pytest

import cases
from tolerance import assert_close, assert_ulp_close

D = 128


def crane_policy(steps):
    """Capacity and length after each append, as Attention::update_kv_cache
    computes them: first use S + 256, in place while it fits, else total + 256."""
    cap, n, out = None, 0, []
    for S in steps:
        if cap is None:
            cap, n = S + 256, S
        elif n + S <= cap:
            n += S
        else:
            n += S
            cap = n + 256
        out.append((cap, n))
    return out


# ------------------------------------------------------------------ CPU

def test_grown_capacity_policy():
    from crane_amd import kv
    assert kv.grown_capacity(0, 5) == 261          # first use: S + 256
    assert kv.grown_capacity(261, 261) == 261      # fits exactly
    assert kv.grown_capacity(261, 262) == 518      # overflow: total + 256
    assert kv.grown_capacity(0, 0) == 0
    assert kv.grown_capacity(-1, 3) == -1 and kv.grown_capacity(3, -1) == -1
    rng = np.random.default_rng(3)
    steps = [int(x) for x in rng.choice([1, 1, 1, 2, 7, 100, 255, 256, 257, 600], size=200)]
    cap, n = 0, 0
    for (want_cap, want_n), S in zip(crane_policy(steps), steps):
        n += S
        cap = kv.grown_capacity(cap, n)
        assert (cap, n) == (want_cap, want_n)


def test_create_argument_checks():
    import torch
    from crane_amd import _lib, kv
    import ctypes
    h = ctypes.c_void_p()
    L = _lib.lib()
    assert L.crane_kv_create(2, 8, 64, 1, ctypes.byref(h)) == _lib.E_HEAD_DIM
    assert L.crane_kv_create(2, 8, 128, 7, ctypes.byref(h)) == _lib.E_DTYPE
    assert L.crane_kv_create(-1, 8, 128, 1, ctypes.byref(h)) == _lib.E_INVALID
    assert L.crane_kv_create(2, 0, 128, 1, ctypes.byref(h)) == _lib.E_INVALID
    c = kv.KvCache(3, 4, torch.bfloat16, device=torch.device("cpu"))
    assert c.capacity == 0 and c.lengths == [0, 0, 0] and c.bytes == 0 and c.buffers() == (None, None)
    assert L.crane_kv_update(c._h, None, None, -1, None) == _lib.E_INVALID
    assert L.crane_kv_update(c._h, None, None, 0, None) == _lib.OK      # nothing to append
    assert L.crane_kv_extract(c._h, 5, c._h, None) == _lib.E_INVALID
    c.close()


# ------------------------------------------------------------------ GPU

def _t(x, dtype, dev):
    import torch
    t = torch.from_numpy(np.ascontiguousarray(x))
    return (t.to(torch.bfloat16) if dtype == "bf16" else t).to(dev)


@pytest.mark.gpu
def test_update_kv_cache_growth(gpu):
    """A sequence of appends: capacity follows Crane's policy and the valid
    rows are exactly the concatenation of everything appended."""
    import torch
    from crane_amd import kv
    B, Hkv = 2, 4
    steps = [7, 1, 1, 250, 3, 1, 300, 1]
    c = kv.KvCache(B, Hkv, torch.bfloat16, gpu)
    g = torch.Generator(device=gpu).manual_seed(11)
    ks, vs = [], []
    for (want_cap, want_n), S in zip(crane_policy(steps), steps):
        print(f"update_kv_cache S={S}", flush=True)
        k = torch.randn((B, Hkv, S, D), generator=g, device=gpu).to(torch.bfloat16)
        v = torch.randn((B, Hkv, S, D), generator=g, device=gpu).to(torch.bfloat16)
        ks.append(k)
        vs.append(v)
        kview, vview = c.update_kv_cache(k, v)
        torch.cuda.synchronize()
        assert c.capacity == want_cap and c.lengths == [want_n] * B
        assert c.bytes == 2 * B * Hkv * want_cap * D * 2
        assert torch.equal(kview, torch.cat(ks, 2)) and torch.equal(vview, torch.cat(vs, 2))
    c.close()


@pytest.mark.gpu
def test_append_qkv_through_cache(gpu, orc):
    """Prefill then decode steps through the fused append into a growing cache
    match the oracle's append into a preallocated cache."""
    import torch
    from crane_amd import kv, ops
    B, Hq, Hkv = 2, 8, 2
    steps = [33, 1, 1, 230, 1]
    total = sum(steps)
    cos, sin = orc.rope_tables(D, 1e6, total + 8)
    cos, sin = orc.round_bf16(cos), orc.round_bf16(sin)
    ref_k = np.zeros((B, Hkv, total, D), np.float32)
    ref_v = np.zeros_like(ref_k)
    c = kv.KvCache(B, Hkv, torch.bfloat16, gpu)
    n = 0
    for i, ((want_cap, _), S) in enumerate(zip(crane_policy(steps), steps)):
        print(f"append_qkv step {i} S={S}", flush=True)
        qkv = orc.round_bf16(cases.normal(cases.rng(700 + i), (B, S, (Hq + 2 * Hkv) * D)))
        pos = np.full(B, n, np.int32)
        q = c.append_qkv(_t(qkv, "bf16", gpu), _t(cos, "bf16", gpu), _t(sin, "bf16", gpu),
                         torch.as_tensor(pos, device=gpu), Hq)
        q_ref = orc.qk_norm_rope_append(qkv, Hq, Hkv, cos, sin, pos, ref_k, ref_v, pos, dtype="bf16")
        n += S
        assert c.capacity == want_cap and c.lengths == [n] * B
        assert_ulp_close(q.float().cpu().numpy(), q_ref, "bf16", f"step {i} q", min_exact=0.999)
    kb, vb = c.get_kv_cache()
    assert_ulp_close(kb.float().cpu().numpy(), ref_k, "bf16", "cache K", min_exact=0.999)
    assert np.array_equal(vb.float().cpu().numpy(), ref_v)
    # decode through the cache = decode over the same rows by the plain entry point
    qd = _t(orc.round_bf16(cases.normal(cases.rng(799), (B, Hq, D))), "bf16", gpu)
    got = c.decode(qd)
    want = ops.attention_decode(qd, kb.contiguous(), vb.contiguous(), torch.as_tensor([n] * B, dtype=torch.int32,
                                                                                        device=gpu), n)
    assert torch.equal(got, want)
    c.close()


@pytest.mark.gpu
def test_stack_extract_and_batched_decode(gpu, orc):
    """setup_batch_decode / extract_batch_kv without padding: rows survive the
    round trip exactly, batched decode matches the oracle per sequence, and a
    decode-step append lands at each sequence's own row."""
    import torch
    from crane_amd import kv
    Hq, Hkv = 8, 2
    lens = [5, 300, 77]
    singles, rows = [], []
    g = torch.Generator(device=gpu).manual_seed(5)
    for L in lens:
        c = kv.KvCache(1, Hkv, torch.bfloat16, gpu)
        k = torch.randn((1, Hkv, L, D), generator=g, device=gpu).to(torch.bfloat16)
        v = torch.randn((1, Hkv, L, D), generator=g, device=gpu).to(torch.bfloat16)
        c.update_kv_cache(k, v)
        singles.append(c)
        rows.append((k, v))
    batch = kv.stack(singles, extra_room=4)
    torch.cuda.synchronize()
    assert batch.lengths == lens and batch.capacity == max(lens) + 4
    assert batch.bytes == 2 * 3 * Hkv * (max(lens) + 4) * D * 2
    kb, vb = batch.buffers()
    for i, (k, v) in enumerate(rows):
        assert torch.equal(kb[i, :, :lens[i]], k[0]) and torch.equal(vb[i, :, :lens[i]], v[0])
    # batched decode == oracle decode of each sequence over its own rows
    q = orc.round_bf16(cases.normal(cases.rng(811), (3, Hq, D)))
    got = batch.decode(_t(q, "bf16", gpu)).float().cpu().numpy().reshape(3, Hq * D)
    kn = kb.float().cpu().numpy()
    vn = vb.float().cpu().numpy()
    ref = orc.attn_decode(q, kn, vn, np.array(lens, np.int32), 1 / math.sqrt(D), "bf16")
    assert_close(got, ref, "bf16", "batched decode")
    # one decode step: each sequence's token lands at its own length
    cos, sin = orc.rope_tables(D, 1e6, 512)
    cos, sin = orc.round_bf16(cos), orc.round_bf16(sin)
    tok = orc.round_bf16(cases.normal(cases.rng(812), (3, 1, (Hq + 2 * Hkv) * D)))
    batch.append_qkv(_t(tok, "bf16", gpu), _t(cos, "bf16", gpu), _t(sin, "bf16", gpu),
                     torch.as_tensor(lens, dtype=torch.int32, device=gpu), Hq)
    assert batch.lengths == [L + 1 for L in lens] and batch.capacity == max(lens) + 4
    kb, vb = batch.buffers()
    for i in range(3):
        out = kv.extract(batch, i)
        torch.cuda.synchronize()
        assert out.lengths == [lens[i] + 1] and out.capacity == lens[i] + 1
        ke, ve = out.get_kv_cache()
        assert torch.equal(ke[0], kb[i, :, :lens[i] + 1]) and torch.equal(ve[0], vb[i, :, :lens[i] + 1])
        assert torch.equal(ke[0, :, :lens[i]], rows[i][0][0])           # earlier rows untouched
        # the next append grows the extracted cache by Crane's policy
        out.update_kv_cache(torch.zeros((1, Hkv, 1, D), dtype=torch.bfloat16, device=gpu),
                            torch.zeros((1, Hkv, 1, D), dtype=torch.bfloat16, device=gpu))
        assert out.capacity == lens[i] + 2 + 256
        out.close()
    for c in singles:
        c.close()
    batch.close()


@pytest.mark.gpu
def test_prefill_through_cache(gpu):
    """Prefill of the last S rows of every sequence equals the plain entry
    point with start = length - S."""
    import torch
    from crane_amd import kv, ops
    B, Hq, Hkv, S = 2, 8, 2, 20
    c = kv.KvCache(B, Hkv, torch.bfloat16, gpu)
    g = torch.Generator(device=gpu).manual_seed(9)
    for n in (40, S):
        k = torch.randn((B, Hkv, n, D), generator=g, device=gpu).to(torch.bfloat16)
        c.update_kv_cache(k, torch.randn((B, Hkv, n, D), generator=g, device=gpu).to(torch.bfloat16))
    c.set_lengths([60, 45])   # ragged starts inside the same buffer
    q = torch.randn((B, Hq, S, D), generator=g, device=gpu).to(torch.bfloat16)
    got = c.prefill(q)
    kb, vb = c.buffers()
    want = ops.attention_prefill(q, kb, vb, torch.as_tensor([40, 25], dtype=torch.int32, device=gpu), 40)
    assert torch.equal(got, want)
    c.close()
