"""The decoder stack (crane_amd/model.py: Qwen3Model::forward and
step_batch_decode, qwen3/modeling.rs:846-897, 1033-1063; Hunyuan's
cross-layer attention, hunyuan_dense/modeling.rs:1035-1059) on the GPU
against the same chain of oracle ops on the CPU, layer after layer: a prefill
chunk with per-sequence positions, then decode steps, then a HIP-graph replay
of the decode step checked bit for bit against the eager step.

Bar (bf16): the decoder-layer test's per-element bar, 4e-2 + 2 bf16 ulps of
|ref|, applies to one layer whose input is exact.  Over L layers the input of
each layer already carries the previous layers' error, which the layer passes
on with a gain of about one (the residual stream adds it unchanged; the
normed branches see it through unit-RMS norms and weights of unit gain), so
the bar is L times the per-layer bar, and mean-relative <= 1e-2.  A
composition error (a wrong anchor, position or cache row) moves elements by
order one."""
import math

import numpy as np
import pytest

import cases
from tolerance import bf16_ulp, errors

pytestmark = pytest.mark.gpu

D = 128
ORDER = {"qwen3": 0, "hunyuan": 1, "qwen2": 2}


def _w(r, shape, scale):
    return cases.bf16(cases.normal(r, shape, scale))


def _weights(seed, hidden, Hq, Hkv, inter, L, family, cla):
    r = cases.rng(seed)
    layers = []
    for i in range(L):
        shared = cla > 1 and i % cla != 0
        rows = (Hq if shared else Hq + 2 * Hkv) * D
        qk_norm = family != "qwen2"
        layers.append(dict(input_norm=cases.bf16(1 + 0.1 * cases.normal(r, (hidden,))),
                           qkv=_w(r, (rows, hidden), 1 / math.sqrt(hidden)),
                           o=_w(r, (hidden, Hq * D), 1 / math.sqrt(Hq * D)),
                           post_norm=cases.bf16(1 + 0.1 * cases.normal(r, (hidden,))),
                           gate_up=_w(r, (2 * inter, hidden), 1 / math.sqrt(hidden)),
                           down=_w(r, (hidden, inter), 1 / math.sqrt(inter)),
                           qkv_bias=_w(r, (rows,), 0.5) if family == "qwen2" else None,
                           q_norm=cases.bf16(1 + 0.1 * cases.normal(r, (D,))) if qk_norm else None,
                           k_norm=cases.bf16(1 + 0.1 * cases.normal(r, (D,))) if qk_norm and not shared else None))
    final_norm = cases.bf16(1 + 0.1 * cases.normal(r, (hidden,)))
    lm_head = _w(r, (1000, hidden), 1 / math.sqrt(hidden))
    return layers, final_norm, lm_head


class RefModel:
    """The oracle chain: per anchor layer a float32 K/V cache of bf16 values;
    shared (CLA) layers attend over their anchor's."""

    def __init__(self, orc, layers, final_norm, lm_head, B, Hq, Hkv, cap, family, cla, cos, sin, eps=1e-6):
        self.orc, self.layers, self.fn, self.lm = orc, layers, final_norm, lm_head
        self.Hq, self.Hkv, self.family, self.cla, self.eps = Hq, Hkv, family, cla, eps
        self.cos, self.sin = cos, sin
        L = len(layers)
        self.kc = [np.zeros((B, Hkv, cap, D), np.float32) for _ in range(L)]
        self.vc = [np.zeros((B, Hkv, cap, D), np.float32) for _ in range(L)]
        self.len = np.zeros(B, np.int32)

    def forward(self, x, positions):
        o, eps, order = self.orc, self.eps, ORDER[self.family]
        B, S, H = x.shape
        res = x.reshape(B * S, H).copy()
        scale = 1 / math.sqrt(D)
        for i, w in enumerate(self.layers):
            shared = self.cla > 1 and i % self.cla != 0
            a = i - i % self.cla if self.cla > 1 else i
            h = o.rms_norm(res, w["input_norm"], eps, True, "bf16")
            proj = o.linear(h, w["qkv"], w["qkv_bias"], "bf16", fused=True).reshape(B, S, -1)
            if shared:
                # q only: the append chain on [q | 0 | 0] rows, into scratch caches
                rows = np.concatenate([proj, np.zeros((B, S, 2 * self.Hkv * D), np.float32)], axis=2)
                scratch = np.zeros((B, self.Hkv, S, D), np.float32)
                q = o.qk_norm_rope_append(rows, self.Hq, self.Hkv, self.cos, self.sin, positions, scratch,
                                          scratch.copy(), np.zeros(B, np.int32), w["q_norm"], None, eps, order,
                                          "bf16")
            else:
                q = o.qk_norm_rope_append(proj, self.Hq, self.Hkv, self.cos, self.sin, positions, self.kc[a],
                                          self.vc[a], self.len, w["q_norm"], w["k_norm"], eps, order, "bf16")
            if S == 1:
                mode = "standard" if self.family == "qwen2" else None
                att = o.attn_decode(q[:, :, 0], self.kc[a], self.vc[a], self.len + 1, scale, "bf16",
                                    cases.decode_variant(o, self.Hq, self.Hkv, mode))
            else:
                att = o.attn_prefill(q, self.kc[a], self.vc[a], self.len, scale, True, "bf16")
            att = att.reshape(B * S, -1)
            res, h = o.add_rms_norm(res, o.linear(att, w["o"], None, "bf16", fused=True), w["post_norm"], eps,
                                    "bf16")
            act = o.silu_mul(o.linear(h, w["gate_up"], None, "bf16", fused=True), False, "bf16")
            res = o.residual_add(res, o.linear(act, w["down"], None, "bf16", fused=True), "bf16")
        self.len = self.len + S
        last = res.reshape(B, S, H)[:, S - 1]
        hn = o.rms_norm(np.ascontiguousarray(last), self.fn, eps, True, "bf16")
        return o.linear(hn, self.lm, None, "bf16", fused=True).reshape(B, 1, -1)


def _check(got, ref, L, what):
    err_abs, mean_rel = errors(got, ref)
    d = np.abs(got.astype(np.float64) - ref)
    bound = L * (4e-2 + 2 * bf16_ulp(ref))
    print(f"  {what}: max-abs {err_abs:.3e}, mean-rel {mean_rel:.3e}, worst |err|/bound "
          f"{float(np.max(d / bound)):.3f}", flush=True)
    assert np.all(np.isfinite(got)), what
    assert np.all(d <= bound), f"{what}: {int((d > bound).sum())} elements beyond the bar"
    assert mean_rel <= 1e-2, f"{what}: mean-rel {mean_rel:.3e}"


def _build(gpu, orc, family, L, cla, hidden=512, Hq=8, Hkv=2, inter=1024, B=2, cap=64, seed=5):
    import torch
    from crane_amd import decoder, model
    layers, fn, lm = _weights(seed + L + cla, hidden, Hq, Hkv, inter, L, family, cla)
    t = lambda x: None if x is None else torch.from_numpy(x).to(torch.bfloat16).to(gpu)
    cfg = model.ModelConfig(hidden=hidden, num_heads=Hq, num_kv_heads=Hkv, intermediate=inter, num_layers=L,
                            family=family, rope_theta=1e6 if family != "hunyuan" else 1e4,
                            rope_alpha=1000.0 if family == "hunyuan" else 0.0, max_position=512,
                            cla_share_factor=cla)
    m = model.DecoderModel(cfg, [decoder.LayerWeights(**{k: t(v) for k, v in w.items()}) for w in layers], t(fn),
                           t(lm), B, cap)
    cos, sin = m.cos.float().cpu().numpy(), m.sin.float().cpu().numpy()
    ref = RefModel(orc, layers, fn, lm, B, Hq, Hkv, cap, family, cla, cos, sin)
    return m, ref


@pytest.mark.parametrize("family,L,cla", [("qwen3", 3, 1), ("hunyuan", 4, 2), ("qwen2", 2, 1)])
def test_stack_prefill_then_decode(gpu, orc, family, L, cla):
    """Per-sequence positions that differ from the cache rows, as a batched
    decode step passes them (each sequence's logical position)."""
    import torch
    print(f"decoder stack {family}: {L} layers, CLA factor {cla}", flush=True)
    m, ref = _build(gpu, orc, family, L, cla)
    r = cases.rng(77 + L)
    B, H = m.batch, m.cfg.hidden
    pos = np.array([0, 7], np.int32)
    for step, S in (("prefill", 21), ("decode 1", 1), ("decode 2", 1)):
        x = cases.bf16(cases.normal(r, (B, S, H)))
        got = m.forward(torch.from_numpy(x).to(torch.bfloat16).to(gpu), torch.as_tensor(pos, device=gpu))
        torch.cuda.synchronize()
        want = ref.forward(x, pos)
        _check(got.float().cpu().numpy(), want, L, f"{family} {step} logits")
        pos = pos + S
    assert m.host_lengths.tolist() == [23, 23] and m.lengths.tolist() == [23, 23]
    # the caches hold what the oracle's hold (anchor layers)
    for i in range(L):
        if m.k[i] is not None:
            _check(m.k[i][:, :, :23].float().cpu().numpy(), ref.kc[i][:, :, :23], 1, f"layer {i} K cache")


def test_decode_graph_replays_match_eager(gpu, orc):
    """DecodeGraph: the whole stack's decode step captured once; each replay
    equals the eager step of a twin model bit for bit, and the last matches
    the oracle chain."""
    import torch
    from crane_amd import model
    L, steps = 3, 4
    print(f"decode graph: {L} layers, {steps} replays", flush=True)
    m_g, ref = _build(gpu, orc, "qwen3", L, 1, seed=9)
    m_e, _ = _build(gpu, orc, "qwen3", L, 1, seed=9)
    r = cases.rng(99)
    B, H = m_g.batch, m_g.cfg.hidden
    x0 = cases.bf16(cases.normal(r, (B, 10, H)))
    pos = np.array([3, 0], np.int32)
    for mm in (m_g, m_e):
        mm.forward(torch.from_numpy(x0).to(torch.bfloat16).to(gpu), torch.as_tensor(pos, device=gpu))
    ref.forward(x0, pos)
    pos = pos + 10
    g = model.DecodeGraph(m_g)
    for i in range(steps):
        x = cases.bf16(cases.normal(r, (B, 1, H)))
        xt = torch.from_numpy(x).to(torch.bfloat16).to(gpu)
        g.x.copy_(xt)
        g.positions.copy_(torch.as_tensor(pos, device=gpu))
        got = g.replay()
        want = m_e.step_batch_decode(xt, torch.as_tensor(pos, device=gpu))
        torch.cuda.synchronize()
        assert torch.equal(got, want), f"replay {i} differs from the eager step"
        r_out = ref.forward(x, pos)
        pos = pos + 1
    assert torch.equal(m_g.lengths, m_e.lengths) and m_g.host_lengths.tolist() == m_e.host_lengths.tolist()
    for i in range(L):
        assert torch.equal(m_g.k[i], m_e.k[i]) and torch.equal(m_g.v[i], m_e.v[i])
    _check(got.float().cpu().numpy(), r_out, L, "graph step logits vs oracle")
