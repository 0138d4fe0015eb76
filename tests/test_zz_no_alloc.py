"""crane_hip_attn_decode_noalloc (include/crane_hip.h): the decode entry point
that allocates nothing, its split-KV partials in the library's per-GPU device
array.  Checked through the C ABI against crane_hip_attn_decode with a
caller-provided workspace, bit for bit, on two calls in a row (the second with
smaller inputs, so it runs over what the first left in the array), and the
size limit is rejected on the host."""
import ctypes
import math

import numpy as np
import pytest

import cases

D = 128


def _lib():
    from crane_amd import _lib
    return _lib


def test_noalloc_limit_and_rejections():
    L = _lib().lib()
    limit = L.crane_hip_attn_decode_noalloc_limit()
    assert limit == 32 << 20
    # the partials of c5 (8 sequences x 64 heads, 32769 keys, bf16) fit; f32 ones do not
    assert L.crane_hip_attn_decode_workspace(8, 64, 8, D, 32769, 1) <= limit
    assert L.crane_hip_attn_decode_workspace(8, 64, 8, D, 32769, 0) > limit

    def call(**kw):
        a = dict(q=16, k=16, v=16, cap=40000, kv_len=16, max_kv=32769, B=8, Hq=64, Hkv=8, D=D,
                 scale=1 / math.sqrt(D), score=0, out=16, dtype=0, stream=None)
        a.update(kw)
        return L.crane_hip_attn_decode_noalloc(a["q"], a["k"], a["v"], a["cap"], a["kv_len"], a["max_kv"], a["B"],
                                               a["Hq"], a["Hkv"], a["D"], a["scale"], a["score"], a["out"],
                                               a["dtype"], a["stream"])
    lib = _lib()
    assert call() == lib.E_WORKSPACE                  # f32 partials beyond the array: rejected before any launch
    assert call(max_kv=50000) == lib.E_CAPACITY
    assert call(dtype=3) == lib.E_DTYPE
    assert call(D=64) == lib.E_HEAD_DIM
    assert call(B=0, dtype=1) == lib.OK               # nothing to do


@pytest.mark.gpu
def test_noalloc_decode_equals_workspace_decode(gpu, orc):
    import torch
    lib = _lib()
    L = lib.lib()

    def dev(x, dtype):
        t = torch.from_numpy(np.ascontiguousarray(x))
        return (t.to(torch.bfloat16) if dtype == "bf16" else t).to(gpu).contiguous()

    calls = [  # name, B, Hq, Hkv, lens, dtype, score mode
        ("c3 shape, grouped", 32, 32, 8, cases.c3_lengths(), "bf16", lib.SCORE_GROUPED),
        ("smaller, standard", 3, 8, 2, [5, 600, 2048], "bf16", lib.SCORE_STANDARD),
        ("smaller still, f32", 2, 4, 2, [300, 1], "f32", lib.SCORE_GROUPED),
    ]
    for name, B, Hq, Hkv, lens, dtype, mode in calls:
        print(f"noalloc decode {name}: B={B} Hq={Hq} Hkv={Hkv} max_len={max(lens)} {dtype}", flush=True)
        q, k, v, lens = cases.decode_case(900 + B, B, Hq, Hkv, lens, dtype=dtype)
        qd, kd, vd = dev(q, dtype), dev(k, dtype), dev(v, dtype)
        kvl = torch.as_tensor(lens, device=gpu)
        cap, mx = k.shape[2], int(lens.max())
        dt = lib.BF16 if dtype == "bf16" else lib.F32
        st = torch.cuda.current_stream().cuda_stream
        need = L.crane_hip_attn_decode_workspace(B, Hq, Hkv, D, mx, dt)
        ws = torch.empty(need, dtype=torch.uint8, device=gpu)
        want = torch.empty((B, 1, Hq * D), dtype=qd.dtype, device=gpu)
        got = torch.full_like(want, float("nan"))
        assert L.crane_hip_attn_decode(qd.data_ptr(), kd.data_ptr(), vd.data_ptr(), cap, kvl.data_ptr(), mx, B, Hq,
                                       Hkv, D, 1 / math.sqrt(D), mode, ws.data_ptr(), need, want.data_ptr(), dt,
                                       st) == lib.OK
        assert L.crane_hip_attn_decode_noalloc(qd.data_ptr(), kd.data_ptr(), vd.data_ptr(), cap, kvl.data_ptr(), mx,
                                               B, Hq, Hkv, D, 1 / math.sqrt(D), mode, got.data_ptr(), dt,
                                               st) == lib.OK
        torch.cuda.synchronize()
        assert torch.equal(got, want), name
        ref = orc.attn_decode(q, k, v, lens, cases.scale(), dtype,
                              orc.DECODE_GROUPED if mode == lib.SCORE_GROUPED else orc.DECODE_STANDARD)
        from tolerance import assert_close
        assert_close(got.float().cpu().numpy().reshape(B, Hq * D), ref, dtype, name)
