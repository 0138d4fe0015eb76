"""What the split-KV decode's bf16 partials cost, measured on a model of the
kernel's arithmetic (decode.hip, grouped score form, bf16).

For a sequence longer than 256 keys (one chunk of 256 keys; of 512 when the
launch's max_kv passes 12288) the kernel does not run candle's one softmax row (qwen3/modeling.rs:440-467: q scaled in
T, s = T(q.K^T), e = T(exp(T(s - max))), sum rounded to T, p = T(e / sum),
p V in f32).  Per chunk c it takes the chunk's max m_c, p = T(exp2(s log2 e -
m_c log2 e)), l_c = the f32 sum of those p, O_c = sum p V in f32, and stores
the partial row T(O_c / l_c) with (m_c, l_c); the merge weighs partial c by
w_c l_c / sum(w l), w_c = exp2(m_c - max m).  `decode_model` restates that
arithmetic in numpy; `partial_bf16=False` keeps the partial rows in f32.

  - the model is the kernel (GPU test): the same inputs give the model's
    values except where f32 sums in another order move a bf16 rounding;
  - the bf16 partial row is the smaller part of the kernel's distance from
    candle (CPU): against the f32-partial model the bf16 partials move an
    output by at most their own rounding (printed: ~60% of outputs identical,
    max |d| ~1e-3 at config 3), and they add under a quarter to the kernel's
    mean-relative distance from the candle oracle (printed: 0.0044 vs 0.0041);
    the rest is the per-chunk p, which differs from candle's normalised p in
    any case."""
import numpy as np
import pytest

import cases
from tolerance import bf16_ulp, errors

bf = cases.bf16
LOG2E = np.float32(1.4426950408889634)


def decode_model(q, k, v, lens, max_kv, partial_bf16=True):
    """q [B, Hq, D] bf16 values, caches [B, Hkv, cap, D]; grouped form."""
    B, Hq, D = q.shape
    Hkv = k.shape[1]
    n_rep = Hq // Hkv
    CH = 512 if max_kv > 12288 else 256
    sct = bf(np.float32([cases.scale()]))[0]
    out = np.zeros((B, Hq, D), np.float32)
    for b in range(B):
        L = int(min(lens[b], max_kv))
        if L == 0:
            continue
        for h in range(Hq):
            qg = bf(q[b, h].astype(np.float32) * sct)
            K = k[b, h // n_rep, :L].astype(np.float64)
            V = v[b, h // n_rep, :L].astype(np.float64)
            s = bf((qg.astype(np.float64) @ K.T).astype(np.float32))
            if L <= 256:  # at most kChunkShort keys: candle's chain exactly, whatever the chunk size
                mx = s.max()
                e = bf(np.exp(bf(np.float32(s - mx))).astype(np.float32))
                p = bf(e / bf(np.float32(e.sum(dtype=np.float32))))
                out[b, h] = bf((p.astype(np.float64) @ V).astype(np.float32))
                continue
            if L <= CH:  # one 512-key chunk: the split arithmetic, normalised in place
                m = np.float32(s.max() * LOG2E)
                p = bf(np.exp2((s * LOG2E - m).astype(np.float32)).astype(np.float32))
                lc = np.float32(p.sum(dtype=np.float32))
                O = (p.astype(np.float64) @ V).astype(np.float32)
                out[b, h] = bf((O / lc).astype(np.float32))
                continue
            ms, ls, parts = [], [], []
            for j0 in range(0, L, CH):
                sc = s[j0:j0 + CH]
                m = np.float32(sc.max() * LOG2E)
                p = bf(np.exp2((sc * LOG2E - m).astype(np.float32)).astype(np.float32))
                lc = np.float32(p.sum(dtype=np.float32))
                O = (p.astype(np.float64) @ V[j0:j0 + CH]).astype(np.float32)
                part = (O / lc).astype(np.float32)
                parts.append(bf(part) if partial_bf16 else part)
                ms.append(m)
                ls.append(lc)
            ms, ls = np.float32(ms), np.float32(ls)
            w = np.exp2(ms - ms.max()).astype(np.float32)
            wl = (w * ls).astype(np.float32)
            num = (wl[:, None].astype(np.float64) * np.stack(parts)).sum(0)
            out[b, h] = bf((num / np.float32(wl.sum(dtype=np.float32))).astype(np.float32))
    return out.reshape(B, Hq * D)


def _case(seed, B, Hq, Hkv, lens):
    q, k, v, lens = cases.decode_case(seed, B, Hq, Hkv, lens, dtype="bf16")
    return q, k, v, lens, int(lens.max())


SHAPES = [
    # B, Hq, Hkv, lengths: config 3's first sequences; a long ragged batch; a
    # batch of 512-key chunks (max_kv past 12288) with sequences of one chunk
    (8, 32, 8, None),
    (3, 16, 2, [700, 2049, 5000]),
    (3, 8, 2, [200, 300, 12300]),
]


def _lens(B, lens):
    return cases.c3_lengths()[:B] if lens is None else lens


def test_model_single_chunk_is_candle(orc):
    """A sequence of one chunk follows candle's chain in the model, as in the
    kernel (bit-identical to the oracle)."""
    q, k, v, lens, mk = _case(41, 3, 8, 2, [1, 100, 256])
    np.testing.assert_array_equal(decode_model(q, k, v, lens, mk),
                                  orc.attn_decode(q, k, v, lens, cases.scale(), "bf16", orc.DECODE_GROUPED))


@pytest.mark.parametrize("B,Hq,Hkv,lens", SHAPES)
def test_bf16_partials_cost(orc, B, Hq, Hkv, lens):
    q, k, v, lens, mk = _case(42 + B, B, Hq, Hkv, _lens(B, lens))
    ref = orc.attn_decode(q, k, v, lens, cases.scale(), "bf16", orc.DECODE_GROUPED)
    m16 = decode_model(q, k, v, lens, mk, partial_bf16=True)
    m32 = decode_model(q, k, v, lens, mk, partial_bf16=False)
    d = np.abs(m16.astype(np.float64) - m32)
    e16, e32 = errors(m16, ref), errors(m32, ref)
    print(f"B={B} Hq={Hq}: bf16 vs f32 partials: bit-identical {np.mean(m16 == m32):.4f}, max |d| {d.max():.2e}; "
          f"vs candle (max-abs, mean-rel): bf16 partials {e16}, f32 partials {e32}")
    # A partial row is a convex combination of V rows (|x| <= max|v| ~ 4 here)
    # rounded once (half an ulp, 2^-9 relative); the merge is a convex
    # combination of partials, so an output moves by at most 2^-9 max|partial|
    # plus its own rounding.  Partial rows of long sequences are averages of
    # many rows (|x| well below 1): the bound uses |partial| <= 1, 2^-9 + one
    # output ulp (rarely reached).
    assert float(d.max()) <= 2.0 ** -9 + 2.0 ** -8, "the bf16 partial rows move an output beyond their rounding"
    assert float(np.mean(m16 == m32)) >= 0.5
    # the kernel's distance from candle is mostly the per-chunk p's: the bf16
    # partials add at most a quarter to the mean-relative error, and no
    # max-abs
    assert e16[1] <= 1.25 * e32[1] and e16[0] <= e32[0] + 2.0 ** -9


@pytest.mark.gpu
@pytest.mark.parametrize("B,Hq,Hkv,lens", SHAPES)
def test_model_is_the_kernel(gpu, B, Hq, Hkv, lens):
    import torch
    from crane_amd import ops
    q, k, v, lens, mk = _case(42 + B, B, Hq, Hkv, _lens(B, lens))
    print(f"decode model vs kernel: B={B} Hq={Hq} Hkv={Hkv} lens={list(lens)}", flush=True)
    t = lambda x: torch.from_numpy(np.ascontiguousarray(x)).to(torch.bfloat16).to(gpu)
    out = ops.attention_decode(t(q), t(k), t(v), torch.as_tensor(lens, device=gpu), mk, cases.scale())
    torch.cuda.synchronize()
    got = out.float().cpu().numpy().reshape(B, Hq * q.shape[2])
    model = decode_model(q, k, v, lens, mk)
    ulps = np.abs(got.astype(np.float64) - model) / bf16_ulp(np.maximum(np.abs(model), 2.0 ** -8))
    same = float(np.mean(got == model))
    print(f"  bit-identical {same:.4f}, max {ulps.max():.2f} ulps", flush=True)
    assert same >= 0.95 and float(ulps.max()) <= 4.0
