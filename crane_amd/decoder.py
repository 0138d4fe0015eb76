"""One decoder layer of the Qwen3 / Qwen2.5 / Hunyuan models Crane serves,
composed from this package's kernels: DecoderLayer::forward
(qwen3/modeling.rs:655-673) around Attention::forward (:372-503) and the
merged gate_up Mlp::forward (:570-591).

    residual = x
    h   = input_layernorm(x)                        crane_hip_rms_norm
    qkv = qkv_proj(h)                               crane_gemm_linear (+ bias)
    q   = qk-norm + rope, K/V into the cache        crane_kv_append_qkv
    a   = attention over the cache                  crane_kv_prefill / crane_kv_decode
    x   = residual + o_proj(a); h = post_norm(x)    crane_gemm_linear, crane_hip_add_rms_norm
    x   = x + down(silu(gate) * up)                 crane_gemm_linear_silu_mul (decode batches;
                                                    else crane_gemm_linear, crane_hip_silu_mul),
                                                    crane_gemm_linear, crane_hip_residual_add

The layer owns its KV cache (Attention.kv_cache).  S > 1 tokens is a prefill
chunk; S == 1 a decode step over every sequence's own length."""
from __future__ import annotations

from dataclasses import dataclass
from typing import Optional

import torch

from . import ops
from ._lib import CraneHipError, E_INVALID
from .kv import KvCache


@dataclass
class LayerWeights:
    """Row-major candle Linear weights ([out, in]) and the norm weights."""
    input_norm: torch.Tensor                 # [hidden]
    qkv: torch.Tensor                        # [(Hq + 2 Hkv) D, hidden], merged q | k | v
    o: torch.Tensor                          # [hidden, Hq D]
    post_norm: torch.Tensor                  # [hidden]
    gate_up: torch.Tensor                    # [2 inter, hidden], gate | up
    down: torch.Tensor                       # [hidden, inter]
    qkv_bias: Optional[torch.Tensor] = None  # [(Hq + 2 Hkv) D], Qwen2.5
    q_norm: Optional[torch.Tensor] = None    # [D], Qwen3 / Hunyuan
    k_norm: Optional[torch.Tensor] = None    # [D]


class DecoderLayer:
    def __init__(self, weights: LayerWeights, batch: int, num_heads: int, num_kv_heads: int,
                 eps: float = 1e-6, order: str = "norm_then_rope"):
        w = weights
        self.w, self.num_heads, self.num_kv_heads, self.eps, self.order = w, num_heads, num_kv_heads, eps, order
        self.hidden = w.input_norm.shape[0]
        self.inter = w.down.shape[1]
        if w.qkv.shape != ((num_heads + 2 * num_kv_heads) * ops.HEAD_DIM, self.hidden) or \
                w.o.shape != (self.hidden, num_heads * ops.HEAD_DIM) or \
                w.gate_up.shape != (2 * self.inter, self.hidden) or w.down.shape != (self.hidden, self.inter):
            raise CraneHipError(E_INVALID, "layer weight shapes do not match the head counts and sizes")
        self.cache = KvCache(batch, num_kv_heads, dtype=w.qkv.dtype, device=w.qkv.device)
        # Decode scores follow the candle path the model takes: Qwen2.5
        # (rope only, candle-transformers qwen2) always the standard SDPA;
        # Qwen3 and Hunyuan the grouped one when n_rep > 1.
        self.score_mode = "standard" if order == "rope_only" else None

    def forward(self, x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor, positions: torch.Tensor) -> torch.Tensor:
        """x [B, S, hidden]; positions [B] int32, the rope position of each
        sequence's first new token.  Returns [B, S, hidden]; x is not modified."""
        w = self.w
        B, S, H = x.shape
        if H != self.hidden or B != self.cache.batch:
            raise CraneHipError(E_INVALID, f"x {tuple(x.shape)} does not match the layer")
        residual = x.reshape(B * S, H).clone()  # updated in place below: residual + attn, then + mlp
        h = ops.rms_norm(residual, w.input_norm, self.eps)
        qkv = ops.linear(h, w.qkv, w.qkv_bias).view(B, S, -1)
        q = self.cache.append_qkv(qkv, cos, sin, positions, self.num_heads, w.q_norm, w.k_norm, self.eps,
                                  self.order)
        if S == 1:
            attn = self.cache.decode(q.view(B, self.num_heads, ops.HEAD_DIM), score_mode=self.score_mode)
        else:
            attn = self.cache.prefill(q)
        o = ops.linear(attn.view(B * S, -1), w.o)
        h = ops.add_rms_norm(residual, o, w.post_norm, self.eps)
        act = ops.linear_silu_mul(h, w.gate_up)
        ops.residual_add(residual, ops.linear(act, w.down))
        return residual.view(B, S, H)
