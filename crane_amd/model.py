"""The decoder stack of the models Crane serves, composed from this package's
kernels: Qwen3Model::forward and step_batch_decode
(crane-core/src/models/qwen3/modeling.rs:846-897, 1033-1063), the Hunyuan-dense
model with cross-layer attention (hunyuan_dense/modeling.rs:990-1066,
1225-1259) and the Qwen2.5 model (candle-transformers qwen2, qwen25/qwen2.rs).

    x -> [layer 0 .. L-1] -> final RmsNorm -> lm_head (last position) -> logits

One set of rope tables serves every layer (Crane's single RotaryEmbedding,
qwen3/modeling.rs:117-153; Hunyuan's NTK-alpha base with `rope_alpha`).  Each
layer holds its K/V in Crane's cache layout [B, Hkv, cap, D]; the rows valid
per sequence (the same for every layer) are one device tensor `lengths`, so a
step reads and advances them on the device and can be captured in a HIP graph
(`DecodeGraph`).  Positions are per sequence, as step_batch_decode takes them
(:1042-1053): token s of sequence b is rotated by table row positions[b] + s
and lands in cache row lengths[b] + s.

Hunyuan CLA (hunyuan_dense/modeling.rs:1035-1059): with cla_share_factor f > 1,
layer i with i % f != 0 projects q only (its weight `q_only` [Hq D, hidden]),
rotates and norms it (crane_hip_qnorm_rope) and attends over the K/V its anchor
layer (i - i % f) appended in the same step; it keeps no cache of its own.

Embedding lookup is outside this driver: it takes hidden states [B, S, hidden].
"""
from __future__ import annotations

import math
from dataclasses import dataclass
from typing import List, Optional

import numpy as np
import torch

from . import ops
from ._lib import CraneHipError, E_CAPACITY, E_INVALID
from .decoder import LayerWeights

_ORDER = {"qwen3": "norm_then_rope", "hunyuan": "rope_then_norm", "qwen2": "rope_only"}


@dataclass
class ModelConfig:
    hidden: int
    num_heads: int
    num_kv_heads: int
    intermediate: int
    num_layers: int
    family: str = "qwen3"          # "qwen3" | "hunyuan" | "qwen2"
    rope_theta: float = 1e6
    rope_alpha: float = 0.0        # Hunyuan NTK-alpha (0: plain base)
    rms_norm_eps: float = 1e-6
    max_position: int = 40960
    cla_share_factor: int = 1      # Hunyuan cross-layer attention


class DecoderModel:
    """Weights: `layers` (one LayerWeights per layer; a CLA shared layer sets
    `qkv` to its q-only projection [Hq D, hidden] and no k_norm), the final
    norm weight [hidden] and an optional lm_head [vocab, hidden]."""

    def __init__(self, cfg: ModelConfig, layers: List[LayerWeights], final_norm: torch.Tensor,
                 lm_head: Optional[torch.Tensor], batch: int, capacity: int):
        if cfg.family not in _ORDER:
            raise CraneHipError(E_INVALID, f"family {cfg.family!r}")
        if len(layers) != cfg.num_layers or cfg.num_layers < 1:
            raise CraneHipError(E_INVALID, "one LayerWeights per layer")
        if cfg.num_heads % cfg.num_kv_heads != 0 or cfg.cla_share_factor < 1:
            raise CraneHipError(E_INVALID, "head counts or CLA factor")
        self.cfg, self.layers, self.final_norm, self.lm_head = cfg, layers, final_norm, lm_head
        self.batch, self.capacity = batch, capacity
        w0 = layers[0].qkv
        self.device, self.dtype = w0.device, w0.dtype
        self.order = _ORDER[cfg.family]
        D = ops.HEAD_DIM
        H, Hq, Hkv = cfg.hidden, cfg.num_heads, cfg.num_kv_heads
        # Qwen2.5 decodes by the standard SDPA (scores post-scaled); Qwen3 and
        # Hunyuan by the grouped one when n_rep > 1 (ops.score_mode_code).
        self.score_mode = "standard" if cfg.family == "qwen2" else None
        for i, w in enumerate(layers):
            want = (Hq if self.shared(i) else Hq + 2 * Hkv) * D
            if w.qkv.shape != (want, H) or w.o.shape != (H, Hq * D) or \
                    w.gate_up.shape != (2 * cfg.intermediate, H) or w.down.shape != (H, cfg.intermediate):
                raise CraneHipError(E_INVALID, f"layer {i} weight shapes do not match the config")
        if cfg.family == "qwen2":
            self.cos, self.sin = ops.rope_tables_qwen2(D, cfg.rope_theta, cfg.max_position, self.device, self.dtype)
        else:
            self.cos, self.sin = ops.rope_tables(D, cfg.rope_theta, cfg.max_position, cfg.rope_alpha, self.device,
                                                 self.dtype)
        shape = (batch, Hkv, capacity, D)
        self.k = [None if self.shared(i) else torch.zeros(shape, dtype=self.dtype, device=self.device)
                  for i in range(cfg.num_layers)]
        self.v = [None if self.shared(i) else torch.zeros(shape, dtype=self.dtype, device=self.device)
                  for i in range(cfg.num_layers)]
        self.lengths = torch.zeros(batch, dtype=torch.int32, device=self.device)   # rows valid, every layer
        self.host_lengths = np.zeros(batch, dtype=np.int64)                         # the same, on the host
        self.scale = 1.0 / math.sqrt(D)
        self.workspace = torch.empty(ops.decode_workspace_bytes(batch, Hq, Hkv, capacity, self.dtype),
                                     dtype=torch.uint8, device=self.device)

    def shared(self, i: int) -> bool:
        """Layer i reuses its anchor's K/V (Hunyuan CLA)."""
        f = self.cfg.cla_share_factor
        return f > 1 and i % f != 0

    def anchor(self, i: int) -> int:
        f = self.cfg.cla_share_factor
        return i - i % f if f > 1 else i

    def reset(self) -> None:
        """clear_kv_cache: every sequence back to zero rows."""
        self.lengths.zero_()
        self.host_lengths[:] = 0

    # ------------------------------------------------------------------ steps

    def _layer(self, i: int, residual: torch.Tensor, h: torch.Tensor, positions: torch.Tensor,
               lengths_after: torch.Tensor, S: int, bound: int, start_bound: int) -> torch.Tensor:
        """DecoderLayer::forward (qwen3/modeling.rs:655-673) over the layer's
        cache from its normed input h [B S, hidden]; the attention half is added
        into `residual` in place, and the MLP output is returned for the caller
        to add (fused with the next norm)."""
        cfg, w = self.cfg, self.layers[i]
        B = self.batch
        D, Hq, Hkv = ops.HEAD_DIM, cfg.num_heads, cfg.num_kv_heads
        eps = cfg.rms_norm_eps
        a = self.anchor(i)
        if self.shared(i):
            q = ops.linear(h, w.qkv, w.qkv_bias).view(B, S, Hq * D)
            q = ops.q_norm_rope(q, self.cos, self.sin, positions, Hq, w.q_norm, eps, self.order)
        else:
            # a decode step's qkv_proj goes to the append as split-K partial
            # products (ops.linear_for_append), reduced inside the append
            if S == 1:
                qkv = ops.linear_for_append(h, w.qkv, w.qkv_bias)
                if not isinstance(qkv, ops.PartialProduct):
                    qkv = qkv.view(B, S, -1)
            else:
                qkv = ops.linear(h, w.qkv, w.qkv_bias).view(B, S, -1)
            q = ops.qk_norm_rope_append(qkv, self.cos, self.sin, positions, self.k[a], self.v[a], self.lengths,
                                        bound, Hq, Hkv, w.q_norm, w.k_norm, eps, self.order)
        if S == 1:
            attn = ops.attention_decode(q.view(B, Hq, D), self.k[a], self.v[a], lengths_after, bound, self.scale,
                                        self.workspace, self.score_mode)
        else:
            attn = ops.attention_prefill(q, self.k[a], self.v[a], self.lengths, start_bound, self.scale, True)
        # In a decode step o_proj and down_proj feed only the adds: their split-K
        # partial products go straight into add_rms_norm (ops.linear_for_residual).
        proj = ops.linear_for_residual if S == 1 else ops.linear
        o = proj(attn.view(B * S, Hq * D), w.o)
        h2 = ops.add_rms_norm(residual, o, w.post_norm, eps)
        return proj(ops.linear_silu_mul(h2, w.gate_up), w.down)

    def _run(self, x: torch.Tensor, positions: torch.Tensor, bound: int, start_bound: int,
             trace: Optional[list] = None) -> torch.Tensor:
        B, S, H = x.shape
        if B != self.batch or H != self.cfg.hidden or x.dtype != self.dtype:
            raise CraneHipError(E_INVALID, f"x {tuple(x.shape)} {x.dtype} does not match the model")
        if positions.dtype != torch.int32 or positions.numel() != B:
            raise CraneHipError(E_INVALID, "positions must be int32 [B]")
        eps, L = self.cfg.rms_norm_eps, self.cfg.num_layers
        x = x.contiguous().clone()       # the residual stream; the caller's tensor is not modified
        residual = x.view(B * S, H)
        lengths_after = self.lengths + S
        # each layer's last residual add is fused with the next layer's input
        # norm (candle's residual add then RmsNorm, as one add + norm kernel)
        h = ops.rms_norm(residual, self.layers[0].input_norm, eps)
        for i in range(L):
            mlp = self._layer(i, residual, h, positions, lengths_after, S, bound, start_bound)
            if trace is not None:  # the layer's output is T(residual + mlp), taken by the next add
                trace.append((residual.clone(),
                              mlp.parts.clone() if isinstance(mlp, ops.PartialProduct) else mlp.clone()))
            if i + 1 < L:
                h = ops.add_rms_norm(residual, mlp, self.layers[i + 1].input_norm, eps)
        self.lengths.add_(S)             # every layer appended S rows per sequence
        if S == 1:                       # every row is a last position: add + final norm at once
            last = ops.add_rms_norm(residual, mlp, self.final_norm, eps).view(B, 1, H)
        else:
            ops.residual_add(residual, mlp)
            last = ops.rms_norm(x[:, S - 1:, :].contiguous(), self.final_norm, eps)
        return ops.linear(last, self.lm_head) if self.lm_head is not None else last

    def forward(self, x: torch.Tensor, positions: torch.Tensor, trace: Optional[list] = None) -> torch.Tensor:
        """Qwen3Model::forward over hidden states x [B, S, hidden]: a prefill
        chunk (S > 1, causal over each sequence's cached rows and the chunk) or
        a decode step (S = 1).  positions [B] int32: the rope row of each
        sequence's first new token (forward's start_pos, per sequence).
        Returns the logits of the last position [B, 1, vocab] (the final
        normed hidden state when there is no lm_head).  trace: a list that
        receives, per layer, copies of the residual stream after the
        attention half and of the MLP output ([B S, hidden] each; the layer's
        output is their sum rounded to the model dtype), or, when down_proj
        ran split (a decode step), its f32 partial products [splits, B S,
        hidden], whose sum in split order rounded to the dtype is the MLP
        output."""
        S = x.shape[1]
        top = int(self.host_lengths.max()) + S
        if top > self.capacity:
            raise CraneHipError(E_CAPACITY, f"{top} rows > capacity {self.capacity}")
        out = self._run(x, positions, top if S > 1 else self.capacity, int(self.host_lengths.max()), trace)
        self.host_lengths += S
        return out

    def step_batch_decode(self, x: torch.Tensor, positions: torch.Tensor) -> torch.Tensor:
        """Qwen3Model::step_batch_decode: one token per sequence, x [B, 1,
        hidden], rotated by its own position; every sequence attends over its
        own rows (no padding or mask).  Returns logits [B, 1, vocab]."""
        if x.shape[1] != 1:
            raise CraneHipError(E_INVALID, "a decode step takes one token per sequence")
        return self.forward(x, positions)


class DecodeGraph:
    """One decode step of the whole stack captured once in a HIP graph and
    replayed: the launchers neither allocate nor synchronise, and they read
    positions and lengths from device memory, so a replay advances `lengths`
    on the device like the eager step does.  Host-side bounds are the cache
    capacity (the kernels clamp to each sequence's own length).  Callers copy
    the step's input into `x` and its positions into `positions`, then call
    `replay()`; the logits land in `logits`.  Replays must not run past the
    capacity (each adds a row to every sequence); `steps_left` counts them."""

    def __init__(self, model: DecoderModel):
        self.model = model
        dev = model.device
        self.x = torch.zeros((model.batch, 1, model.cfg.hidden), dtype=model.dtype, device=dev)
        self.positions = torch.zeros(model.batch, dtype=torch.int32, device=dev)
        self.stream = torch.cuda.Stream(device=dev)
        snapshot = model.lengths.clone()
        # warm-up on the capture stream: GEMM plans and per-stream contexts are
        # made here, not under capture; then the lengths are put back
        self.stream.wait_stream(torch.cuda.current_stream(dev))
        with torch.cuda.stream(self.stream):
            model._run(self.x, self.positions, model.capacity, model.capacity - 1)
            model.lengths.copy_(snapshot)
        torch.cuda.current_stream(dev).wait_stream(self.stream)
        torch.cuda.synchronize(dev)
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph, stream=self.stream):
            self.logits = model._run(self.x, self.positions, model.capacity, model.capacity - 1)
        torch.cuda.synchronize(dev)
        model.lengths.copy_(snapshot)    # the capture itself advanced them once
        torch.cuda.synchronize(dev)

    @property
    def steps_left(self) -> int:
        return int(self.model.capacity - self.model.host_lengths.max())

    def replay(self) -> torch.Tensor:
        if self.steps_left < 1:
            raise CraneHipError(E_CAPACITY, "the caches are full")
        self.graph.replay()
        self.model.host_lengths += 1
        return self.logits
