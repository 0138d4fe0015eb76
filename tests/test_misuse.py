"""Misuse of the Python surface is rejected on the host, before any launch:
shapes, dtypes and layouts that would make a kernel read or write past a
buffer (a q of another element size than the cache, a qkv row narrower than
the heads it names, a norm weight of the wrong length) raise CraneHipError
with the library's error code.  Needs CUDA tensors, so it runs with the GPU
tests; nothing here launches a kernel before the checks have passed."""
import pytest

pytestmark = pytest.mark.gpu

D = 128


def _bf(shape, dev, dtype=None):
    import torch
    return torch.zeros(shape, dtype=dtype or torch.bfloat16, device=dev)


def test_cache_ops_reject_bad_q(gpu):
    import torch
    from crane_amd import _lib, kv
    from crane_amd._lib import CraneHipError
    c = kv.KvCache(2, 2, dtype=torch.float32, device=gpu)
    c.update_kv_cache(_bf((2, 2, 5, D), gpu, torch.float32), _bf((2, 2, 5, D), gpu, torch.float32))
    with pytest.raises(CraneHipError) as e:      # bf16 q for an f32 cache: half the bytes the kernel would read
        c.decode(_bf((2, 4, D), gpu))
    assert e.value.code == _lib.E_DTYPE
    with pytest.raises(CraneHipError) as e:      # batch mismatch
        c.decode(_bf((3, 4, D), gpu, torch.float32))
    assert e.value.code == _lib.E_INVALID
    with pytest.raises(CraneHipError) as e:      # prefill q must be [B, Hq, S, D]
        c.prefill(_bf((2, 4, D), gpu, torch.float32))
    assert e.value.code == _lib.E_INVALID
    with pytest.raises(CraneHipError):           # a workspace on the host
        c.decode(_bf((2, 4, D), gpu, torch.float32), workspace=torch.zeros(1 << 20, dtype=torch.uint8))
    out = c.decode(_bf((2, 4, D), gpu, torch.float32))   # the well-formed call still works
    torch.cuda.synchronize()
    assert out.shape == (2, 1, 4 * D)


def test_append_rejects_narrow_rows_and_bad_weights(gpu):
    import torch
    from crane_amd import _lib, kv, ops
    from crane_amd._lib import CraneHipError
    B, S, Hq, Hkv = 2, 3, 4, 2
    cos, sin = ops.rope_tables(D, 1e6, 64, device=gpu, dtype=torch.bfloat16)
    pos = torch.zeros(B, dtype=torch.int32, device=gpu)
    c = kv.KvCache(B, Hkv, device=gpu)
    with pytest.raises(CraneHipError) as e:      # q only: the kernel would read K and V past each row
        c.append_qkv(_bf((B, S, Hq * D), gpu), cos, sin, pos, Hq)
    assert e.value.code == _lib.E_INVALID
    with pytest.raises(CraneHipError) as e:      # a 64-element norm weight
        c.append_qkv(_bf((B, S, (Hq + 2 * Hkv) * D), gpu), cos, sin, pos, Hq, q_norm_w=_bf((64,), gpu),
                     k_norm_w=_bf((D,), gpu))
    assert e.value.code == _lib.E_INVALID
    with pytest.raises(CraneHipError) as e:      # f32 tables for bf16 rows
        c.append_qkv(_bf((B, S, (Hq + 2 * Hkv) * D), gpu), cos.float(), sin.float(), pos, Hq)
    assert e.value.code == _lib.E_DTYPE
    with pytest.raises(CraneHipError) as e:      # int64 positions
        c.append_qkv(_bf((B, S, (Hq + 2 * Hkv) * D), gpu), cos, sin, pos.long(), Hq)
    assert e.value.code == _lib.E_INVALID
    assert c.lengths == [0, 0]                   # nothing was appended
    kc, vc = _bf((B, Hkv, 16, D), gpu), _bf((B, Hkv, 16, D), gpu)
    with pytest.raises(CraneHipError) as e:      # the functional op checks the weights too
        ops.qk_norm_rope_append(_bf((B, S, (Hq + 2 * Hkv) * D), gpu), cos, sin, pos, kc, vc, pos, S, Hq, Hkv,
                                q_norm_w=_bf((2 * D,), gpu), k_norm_w=_bf((D,), gpu))
    assert e.value.code == _lib.E_INVALID
    with pytest.raises(CraneHipError) as e:      # CLA q rows narrower than Hq heads
        ops.q_norm_rope(_bf((B, S, (Hq - 1) * D), gpu), cos, sin, pos, Hq)
    assert e.value.code == _lib.E_INVALID


def test_paged_ops_reject_bad_inputs(gpu):
    import torch
    from crane_amd import _lib, kv, ops
    from crane_amd._lib import CraneHipError
    Hq, Hkv = 4, 2
    p = kv.PagedKvCache(Hkv, n_pages=8, page_rows=256, max_seqs=4, max_pages_per_seq=4, device=gpu)
    ids = [p.add_sequence(), p.add_sequence()]
    p.set_batch(ids)
    cos, sin = ops.rope_tables(D, 1e6, 64, device=gpu, dtype=torch.bfloat16)
    pos = torch.zeros(2, dtype=torch.int32, device=gpu)
    with pytest.raises(CraneHipError) as e:
        p.append_qkv(_bf((2, 1, (Hq + 2 * Hkv) * D - 8), gpu), cos, sin, pos, Hq)
    assert e.value.code == _lib.E_INVALID
    with pytest.raises(CraneHipError) as e:
        p.decode(_bf((2, Hq, D), gpu, torch.float32))
    assert e.value.code == _lib.E_DTYPE
    with pytest.raises(CraneHipError) as e:
        p.prefill(_bf((1, Hq, 1, D), gpu))
    assert e.value.code == _lib.E_INVALID
    assert p.lengths == [0, 0]
