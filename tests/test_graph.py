"""A decode step -- the fused append of each sequence's new token and the
batched split-KV decode -- captured once into a HIP graph (torch.cuda.CUDAGraph)
and replayed step after step.  The launchers neither allocate nor synchronise
nor clear memory, and they read positions and lengths from device memory, so
one capture serves a whole decode loop: the host advances those tensors
between replays, and the host-side bounds (max_rows, max_kv) are captured at
the loop's final size.  Every replay is checked bit for bit against the same
step run eagerly on a twin cache, and that eager work runs between the
replays; the last step is also checked against the oracle."""
import math

import numpy as np
import pytest

import cases
from tolerance import assert_close

pytestmark = pytest.mark.gpu

D = 128


def test_decode_step_graph_replays_match_eager(gpu, orc):
    import torch
    from crane_amd import ops
    B, Hq, Hkv, steps = 8, 32, 8, 5
    W = (Hq + 2 * Hkv) * D
    print(f"graph decode step: B={B} Hq={Hq} Hkv={Hkv} steps={steps}", flush=True)
    r = cases.rng(4242)
    lens = r.integers(300, 1000, size=B).astype(np.int32)
    max_len = int(lens.max()) + steps      # the largest length the loop reaches
    cap = max_len + 8
    bf = torch.bfloat16

    def dev(x):
        return torch.from_numpy(np.ascontiguousarray(x)).to(bf).to(gpu)

    k0 = cases.bf16(cases.normal(r, (B, Hkv, cap, D)))
    v0 = cases.bf16(cases.normal(r, (B, Hkv, cap, D)))
    kc_g, vc_g = dev(k0), dev(v0)            # written by the graph's replays
    kc_e, vc_e = kc_g.clone(), vc_g.clone()  # its eager twin
    qw = dev(cases.bf16(1 + 0.1 * cases.normal(r, (D,))))
    kw = dev(cases.bf16(1 + 0.1 * cases.normal(r, (D,))))
    cos, sin = ops.rope_tables(D, 1e6, 4096, device=gpu, dtype=bf)
    ws_bytes = ops.decode_workspace_bytes(B, Hq, Hkv, max_len, bf)
    ws_g = torch.empty(ws_bytes, dtype=torch.uint8, device=gpu)
    ws_e = torch.empty(ws_bytes, dtype=torch.uint8, device=gpu)

    def step(qkv, pos, kvl, kc, vc, ws):
        q = ops.qk_norm_rope_append(qkv, cos, sin, pos, kc, vc, pos, max_len, Hq, Hkv, qw, kw)
        return ops.attention_decode(q, kc, vc, kvl, max_len, workspace=ws)

    # static inputs of the graph
    qkv_s = torch.zeros((B, 1, W), dtype=bf, device=gpu)
    pos_s = torch.zeros(B, dtype=torch.int32, device=gpu)
    kvl_s = torch.ones(B, dtype=torch.int32, device=gpu)
    # warm-up on a side stream, on scratch caches (the step writes a cache row)
    side = torch.cuda.Stream(device=gpu)
    side.wait_stream(torch.cuda.current_stream(gpu))
    with torch.cuda.stream(side):
        step(qkv_s, pos_s, kvl_s, kc_g.clone(), vc_g.clone(), ws_g)
    torch.cuda.current_stream(gpu).wait_stream(side)
    torch.cuda.synchronize()

    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out_s = step(qkv_s, pos_s, kvl_s, kc_g, vc_g, ws_g)

    qkv_last = None
    for i in range(steps):
        qkv = cases.bf16(cases.normal(r, (B, 1, W)))
        qkv_t = dev(qkv)
        qkv_s.copy_(qkv_t)
        pos_s.copy_(torch.as_tensor(lens, device=gpu))
        kvl_s.copy_(torch.as_tensor(lens + 1, device=gpu))
        graph.replay()
        out_e = step(qkv_t, torch.as_tensor(lens, device=gpu), torch.as_tensor(lens + 1, device=gpu), kc_e, vc_e,
                     ws_e)
        torch.cuda.synchronize()
        assert torch.equal(out_s, out_e), f"replay {i} differs from the eager step"
        qkv_last, lens_last = qkv, lens.copy()
        lens = lens + 1
    assert torch.equal(kc_g, kc_e) and torch.equal(vc_g, vc_e), "the replays and the eager steps wrote different rows"

    # the last step against the oracle: append into the oracle's copy of the cache, then decode
    kc = kc_e.float().cpu().numpy()
    vc = vc_e.float().cpu().numpy()
    cos_n = cos.float().cpu().numpy()
    sin_n = sin.float().cpu().numpy()
    kq, vq = kc.copy(), vc.copy()
    q_ref = orc.qk_norm_rope_append(qkv_last, Hq, Hkv, cos_n, sin_n, lens_last, kq, vq, lens_last,
                                    qw.float().cpu().numpy(), kw.float().cpu().numpy(), 1e-6, 0, "bf16")
    ref = orc.attn_decode(q_ref[:, :, 0], kq, vq, lens_last + 1, 1 / math.sqrt(D), "bf16")
    assert_close(out_s.float().cpu().numpy().reshape(ref.shape), ref, "bf16", "graph decode step vs oracle")
