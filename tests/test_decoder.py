"""One whole decoder layer (crane_amd/decoder.py, DecoderLayer::forward of
qwen3/modeling.rs:655-673) on the GPU against the same chain of oracle ops on
the CPU: RmsNorm, the merged qkv projection, the fused QK-norm + RoPE append,
prefill or decode attention, o_proj, residual add + RmsNorm, gate_up, SiLU*mul,
down and the residual add.  A prefill chunk is followed by a decode step over
the cache the chunk filled.

Bar (bf16): every output element within 4e-2 + 2 bf16 ulps of |ref|, and
mean-relative error <= 1e-2 (the north star's relative bar).  Attention
matches its oracle to the north-star bar (2e-2 abs) rather than bit for bit.
That error reaches the output twice, each term bounded by the attention bar:
through o_proj into the residual stream (the weights keep norms), and through
the MLP's response to the normed stream (gain about one).  The stream itself
is rounded twice more (the two residual adds).  The other ops match their
oracles within one rounding.  A broken composition (a dropped residual,
gate and up swapped, a wrong cache row) moves elements by order one.  The K
and V rows the layer appended are held to the same bar."""
import math

import numpy as np
import pytest

import cases
from tolerance import bf16_ulp, errors

pytestmark = pytest.mark.gpu

D = 128


def _w(rng, shape, scale):
    return cases.bf16(cases.normal(rng, shape, scale))


def _weights(seed, hidden, Hq, Hkv, inter, qk_norm, bias):
    r = cases.rng(seed)
    w = dict(input_norm=cases.bf16(1 + 0.1 * cases.normal(r, (hidden,))),
             qkv=_w(r, ((Hq + 2 * Hkv) * D, hidden), 1 / math.sqrt(hidden)),
             o=_w(r, (hidden, Hq * D), 1 / math.sqrt(Hq * D)),
             post_norm=cases.bf16(1 + 0.1 * cases.normal(r, (hidden,))),
             gate_up=_w(r, (2 * inter, hidden), 1 / math.sqrt(hidden)),
             down=_w(r, (hidden, inter), 1 / math.sqrt(inter)),
             qkv_bias=_w(r, ((Hq + 2 * Hkv) * D,), 0.5) if bias else None,
             q_norm=cases.bf16(1 + 0.1 * cases.normal(r, (D,))) if qk_norm else None,
             k_norm=cases.bf16(1 + 0.1 * cases.normal(r, (D,))) if qk_norm else None)
    return w


class RefLayer:
    """The oracle chain, with its own float32 K/V cache of bf16 values."""

    def __init__(self, orc, w, B, Hq, Hkv, cap, order, eps=1e-6):
        self.orc, self.w, self.Hq, self.Hkv, self.order, self.eps = orc, w, Hq, Hkv, order, eps
        self.kc = np.zeros((B, Hkv, cap, D), np.float32)
        self.vc = np.zeros((B, Hkv, cap, D), np.float32)
        self.len = np.zeros(B, np.int32)

    def forward(self, x, cos, sin, positions):
        o, w, eps = self.orc, self.w, self.eps
        B, S, H = x.shape
        res = x.reshape(B * S, H)
        h = o.rms_norm(res, w["input_norm"], eps, True, "bf16")
        qkv = o.linear(h, w["qkv"], w["qkv_bias"], "bf16", fused=True).reshape(B, S, -1)
        q = o.qk_norm_rope_append(qkv, self.Hq, self.Hkv, cos, sin, positions, self.kc, self.vc, self.len,
                                  w["q_norm"], w["k_norm"], eps, self.order, "bf16")
        scale = 1 / math.sqrt(D)
        if S == 1:
            # Qwen2.5 (rope only) decodes by the standard SDPA; Qwen3 / Hunyuan by the grouped one
            mode = "standard" if self.order == 2 else None
            a = o.attn_decode(q[:, :, 0], self.kc, self.vc, self.len + 1, scale, "bf16",
                              cases.decode_variant(o, self.Hq, self.Hkv, mode))
        else:
            a = o.attn_prefill(q, self.kc, self.vc, self.len, scale, True, "bf16")
        self.len = self.len + S
        a = a.reshape(B * S, -1)
        res, h = o.add_rms_norm(res, o.linear(a, w["o"], None, "bf16", fused=True), w["post_norm"], eps, "bf16")
        act = o.silu_mul(o.linear(h, w["gate_up"], None, "bf16", fused=True), False, "bf16")
        out = o.residual_add(res, o.linear(act, w["down"], None, "bf16", fused=True), "bf16")
        return out.reshape(B, S, H)


def _check(got, ref, what):
    err_abs, mean_rel = errors(got, ref)
    d = np.abs(got.astype(np.float64) - ref)
    bound = 4e-2 + 2 * bf16_ulp(ref)
    worst = int(np.argmax(d / bound))
    print(f"  {what}: max-abs {err_abs:.3e}, mean-rel {mean_rel:.3e}, bit-identical {np.mean(got == ref):.4f}, "
          f"worst |err| {d.flat[worst]:.3e} at |ref| {abs(ref.flat[worst]):.3f} (bound {bound.flat[worst]:.3e})",
          flush=True)
    assert np.all(np.isfinite(got)), what
    assert np.all(d <= bound), f"{what}: {int((d > bound).sum())} elements beyond 4e-2 + 2 bf16 ulps of |ref|"
    assert mean_rel <= 1e-2, f"{what}: mean-rel {mean_rel:.3e}"


@pytest.mark.parametrize("name,hidden,Hq,Hkv,inter,order,qk_norm,bias,S", [
    # Qwen3-0.6B heads and sizes, QK-norm then RoPE
    ("qwen3_0.6b", 1024, 16, 8, 3072, "norm_then_rope", True, False, 40),
    # Qwen2.5-7B heads (GQA 7) with the qkv bias, RoPE only; smaller hidden and intermediate
    ("qwen25_gqa7_bias", 1024, 28, 4, 2048, "rope_only", False, True, 33),
    # Hunyuan order: RoPE, then the norms
    ("hunyuan_order", 512, 8, 2, 1024, "rope_then_norm", True, False, 17),
    # an intermediate size whose decode step takes the one-launch gate_up + SiLU*mul
    # (crane_gemm_linear_silu_mul), and o_proj the per-wave ring kernel
    ("gated_mlp", 1024, 16, 8, 4608, "norm_then_rope", True, False, 24),
])
def test_decoder_layer_prefill_then_decode(gpu, orc, name, hidden, Hq, Hkv, inter, order, qk_norm, bias, S):
    import torch
    from crane_amd import decoder
    print(f"decoder layer {name}: hidden={hidden} Hq={Hq} Hkv={Hkv} inter={inter} S={S}", flush=True)
    B = 2
    w = _weights(11 + hidden + Hq, hidden, Hq, Hkv, inter, qk_norm, bias)
    wt = {k: (torch.from_numpy(v).to(torch.bfloat16).to(gpu) if v is not None else None) for k, v in w.items()}
    layer = decoder.DecoderLayer(decoder.LayerWeights(**wt), B, Hq, Hkv, order=order)
    ref = RefLayer(orc, w, B, Hq, Hkv, S + 8, {"norm_then_rope": 0, "rope_then_norm": 1, "rope_only": 2}[order])
    cos, sin = orc.rope_tables(D, 1e6, 256)
    cos, sin = cases.bf16(cos), cases.bf16(sin)
    cos_d = torch.from_numpy(cos).to(torch.bfloat16).to(gpu)
    sin_d = torch.from_numpy(sin).to(torch.bfloat16).to(gpu)
    r = cases.rng(900 + hidden)
    for step, s in (("prefill", S), ("decode", 1)):
        x = cases.bf16(cases.normal(r, (B, s, hidden)))
        pos = ref.len.copy()
        got = layer.forward(torch.from_numpy(x).to(torch.bfloat16).to(gpu), cos_d, sin_d,
                            torch.as_tensor(pos, device=gpu))
        torch.cuda.synchronize()
        want = ref.forward(x, cos, sin, pos)
        _check(got.float().cpu().numpy(), want, f"{name} {step}")
    # the cache the layer filled: the prefill chunk's rows and the decode step's row
    assert layer.cache.lengths == [S + 1] * B
    k, v = layer.cache.get_kv_cache()
    _check(k.float().cpu().numpy(), ref.kc[:, :, :S + 1], f"{name} K cache")
    _check(v.float().cpu().numpy(), ref.vc[:, :, :S + 1], f"{name} V cache")
