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
the bar of the end-to-end test is L times the per-layer bar, and
mean-relative <= 1e-2.  A composition error (a wrong anchor, position or
cache row) moves elements by order one.  The layer-by-layer test holds each
layer to the one-layer bar instead: the oracle's layer runs on the GPU's own
input to that layer and over the GPU's cache rows, so no earlier error
reaches it and drift of a layer cannot hide behind the L-fold bar: 2e-2 + 2
ulps per element and mean-relative <= 1e-3."""
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

    def layer(self, i, res, positions, S):
        """Layer i on the residual stream res [B S, hidden] (bf16 values) over
        the caches as they stand (appending its S new rows); returns the
        layer's output, T(res + attention) + the MLP rounded to T."""
        o, eps, order = self.orc, self.eps, ORDER[self.family]
        B = len(positions)
        scale = 1 / math.sqrt(D)
        w = self.layers[i]
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
        res, h = o.add_rms_norm(res, o.linear(att, w["o"], None, "bf16", fused=True), w["post_norm"], eps, "bf16")
        act = o.silu_mul(o.linear(h, w["gate_up"], None, "bf16", fused=True), False, "bf16")
        return o.residual_add(res, o.linear(act, w["down"], None, "bf16", fused=True), "bf16")

    def head(self, res, B, S):
        """Final norm and lm_head of the last position of each sequence."""
        o = self.orc
        last = res.reshape(B, S, -1)[:, S - 1]
        hn = o.rms_norm(np.ascontiguousarray(last), self.fn, self.eps, True, "bf16")
        return o.linear(hn, self.lm, None, "bf16", fused=True).reshape(B, 1, -1)

    def forward(self, x, positions):
        B, S, H = x.shape
        res = x.reshape(B * S, H).copy()
        for i in range(len(self.layers)):
            res = self.layer(i, res, positions, S)
        self.len = self.len + S
        return self.head(res, B, S)


def _check(got, ref, L, what, abs_bar=4e-2, mean_rel_bar=1e-2):
    err_abs, mean_rel = errors(got, ref)
    d = np.abs(got.astype(np.float64) - ref)
    bound = L * (abs_bar + 2 * bf16_ulp(ref))
    print(f"  {what}: max-abs {err_abs:.3e}, mean-rel {mean_rel:.3e}, worst |err|/bound "
          f"{float(np.max(d / bound)):.3f}", flush=True)
    assert np.all(np.isfinite(got)), what
    assert np.all(d <= bound), f"{what}: {int((d > bound).sum())} elements beyond the bar"
    assert mean_rel <= mean_rel_bar, f"{what}: mean-rel {mean_rel:.3e}"


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


# One layer on its exact input: the north star's 2e-2 (plus two ulps of |ref|,
# the last-bit differences of f32 sums in another order) and a tenth of its
# mean-relative bar.
LAYER_BAR = dict(abs_bar=2e-2, mean_rel_bar=1e-3)


def _mlp_of(t):
    """The MLP output a trace entry records: the bf16 rows, or the f32 split-K
    partial products summed in split order and rounded once."""
    x = t.float().cpu().numpy()
    if x.ndim == 3:
        acc = np.zeros(x.shape[1:], np.float32)
        for p in x:
            acc = (acc + p).astype(np.float32)
        return cases.bf16(acc)
    return x


@pytest.mark.parametrize("family,L,cla,dims", [("qwen3", 3, 1, None), ("hunyuan", 4, 2, None), ("qwen2", 2, 1, None),
                                               ("qwen3", 2, 1, (2048, 16, 4, 2048)),
                                               ("qwen2", 2, 1, (2048, 16, 4, 2048))],
                         ids=["qwen3", "hunyuan", "qwen2", "qwen3-split-projections", "qwen2-split-projections"])
def test_stack_layer_by_layer(gpu, orc, family, L, cla, dims, monkeypatch):
    """Each layer of the stack at the one-layer bar: the oracle's layer i runs
    on the GPU's own input to layer i and over the GPU's cache rows of the
    earlier steps, so no earlier layer's error reaches it; then the final norm
    and lm_head on the GPU's last residual.  Prefill, then two decode steps."""
    import torch
    print(f"decoder stack layer by layer {family}: {L} layers, CLA factor {cla}, dims {dims}", flush=True)
    if dims is None:
        m, ref = _build(gpu, orc, family, L, cla)
    else:
        # qkv_proj, o_proj and down_proj all have K = 2048: decode steps take the
        # split-K projections (qkv_proj's reduced, with Qwen2.5's bias, in the append)
        hidden, Hq, Hkv, inter = dims
        m, ref = _build(gpu, orc, family, L, cla, hidden=hidden, Hq=Hq, Hkv=Hkv, inter=inter)
    from crane_amd import ops
    qkv_split = []
    real = ops.linear_for_append

    def spy(*a, **k):
        r = real(*a, **k)
        qkv_split.append(isinstance(r, ops.PartialProduct))
        return r
    monkeypatch.setattr(ops, "linear_for_append", spy)
    r = cases.rng(177 + L)
    B, H = m.batch, m.cfg.hidden
    pos = np.array([0, 7], np.int32)
    for step, S in (("prefill", 21), ("decode 1", 1), ("decode 2", 1)):
        x = cases.bf16(cases.normal(r, (B, S, H)))
        n0 = int(m.host_lengths[0])
        trace = []
        got = m.forward(torch.from_numpy(x).to(torch.bfloat16).to(gpu), torch.as_tensor(pos, device=gpu), trace)
        torch.cuda.synchronize()
        assert len(trace) == L
        if dims is not None and S == 1:
            assert all(t[1].dim() == 3 for t in trace), "the decode step's down_proj ran split"
            assert qkv_split and all(qkv_split), "the decode step's qkv_proj ran split into the append"
        qkv_split.clear()
        res_in = x.reshape(B * S, H)
        for i in range(L):
            # the oracle's cache of the layer's anchor: the GPU's rows of the
            # earlier steps (an anchor appends this step's rows itself; a CLA
            # shared layer reads the anchor's, so it gets the GPU's new rows too)
            a = i - i % cla if cla > 1 else i
            rows = n0 + S if a != i else n0
            for c_ref, c_gpu in ((ref.kc, m.k), (ref.vc, m.v)):
                c_ref[a][:, :, :rows] = c_gpu[a][:, :, :rows].float().cpu().numpy()
            want = ref.layer(i, res_in, pos, S)
            res_mid, mlp = trace[i][0].float().cpu().numpy(), _mlp_of(trace[i][1])
            out = cases.bf16(res_mid + mlp)  # the GPU layer's output: the next add's rounding of the sum
            _check(out, want, 1, f"{family} {step} layer {i} output", **LAYER_BAR)
            res_in = out
        ref.len = ref.len + S
        _check(got.float().cpu().numpy(), ref.head(res_in, B, S), 1, f"{family} {step} logits from the last layer",
               **LAYER_BAR)
        pos = pos + S
