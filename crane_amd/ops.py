"""Tensor-in / Tensor-out host surface of the attention path.

Mirrors the candle calls Crane makes inside Attention::forward
(crane-core/src/models/qwen3/modeling.rs:372-503) and the operator
conventions of its fused_ops plugin (crane-core/src/fused_ops/cuda_impl.rs:
a bad shape/dtype raises, outputs are freshly allocated tensors, the KV cache
is mutated in place like `slice_set`).  torch tensors on the ROCm device
stand in for candle's device Tensor; every compute call goes through the C
ABI of libcrane_hip.so.  Tensors not on a GPU are rejected: there is no CPU
fallback.
"""
from __future__ import annotations

import ctypes
import math
from typing import Optional

import torch

from . import _lib
from ._lib import CraneHipError, check

_DTYPES = {torch.float32: _lib.F32, torch.bfloat16: _lib.BF16}
_ORDERS = {"norm_then_rope": _lib.NORM_THEN_ROPE, "rope_then_norm": _lib.ROPE_THEN_NORM,
           "rope_only": _lib.ROPE_ONLY}
_SCORES = {"grouped": _lib.SCORE_GROUPED, "standard": _lib.SCORE_STANDARD}
HEAD_DIM = 128


def score_mode_code(score_mode: Optional[str], n_rep: int) -> int:
    """The candle SDPA form a decode call reproduces.  None picks the one
    Qwen3 and Hunyuan take (qwen3/modeling.rs:432 `n_rep > 1 && seq_len == 1`:
    the grouped path, q pre-scaled; otherwise the standard path, scores
    post-scaled); Qwen2.5 (candle-transformers qwen2, qwen25/qwen2.rs:196-197)
    always takes "standard"."""
    if score_mode is None:
        return _lib.SCORE_GROUPED if n_rep > 1 else _lib.SCORE_STANDARD
    try:
        return _SCORES[score_mode]
    except KeyError:
        raise CraneHipError(_lib.E_INVALID, f"score_mode {score_mode!r}") from None


def _dtype_code(t: torch.Tensor) -> int:
    return _dtype_code_of(t.dtype)


def _dtype_code_of(dtype: torch.dtype) -> int:
    try:
        return _DTYPES[dtype]
    except KeyError:
        raise CraneHipError(_lib.E_DTYPE, f"dtype {dtype}") from None


def _dev(*ts: Optional[torch.Tensor]) -> torch.device:
    dev = None
    for t in ts:
        if t is None:
            continue
        if t.device.type != "cuda":
            raise CraneHipError(_lib.E_INVALID, f"tensor on {t.device}: crane_amd runs on the GPU only")
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise CraneHipError(_lib.E_INVALID, "tensors on different devices")
    return dev


def _contig(t: torch.Tensor, name: str) -> None:
    if not t.is_contiguous():
        raise CraneHipError(_lib.E_INVALID, f"{name} must be contiguous")


def _i32(t: torch.Tensor, n: int, name: str) -> None:
    if t.dtype != torch.int32 or t.numel() != n or not t.is_contiguous():
        raise CraneHipError(_lib.E_INVALID, f"{name} must be a contiguous int32 tensor of {n} elements")


def _stream(dev: torch.device) -> int:
    return torch.cuda.current_stream(dev).cuda_stream


def _ptr(t: Optional[torch.Tensor]) -> Optional[int]:
    return None if t is None else t.data_ptr()


# ---------------------------------------------------------------- rope tables

def _host_tables(fn, args, head_dim: int, max_pos: int, device, dtype: torch.dtype):
    code = _dtype_code(torch.empty(0, dtype=dtype))
    cos = torch.empty((max_pos, head_dim // 2), dtype=dtype)
    sin = torch.empty_like(cos)
    check(fn(head_dim, *args, max_pos, code, cos.data_ptr(), sin.data_ptr()), fn.__name__)
    return cos.to(device), sin.to(device)


def rope_tables(head_dim: int, theta: float, max_pos: int, alpha: float = 0.0,
                device: torch.device | str = "cuda", dtype: torch.dtype = torch.float32):
    """cos/sin tables [max_pos, head_dim/2] in the model dtype, bit-identical to
    Crane's: qwen3/modeling.rs:117-139 (inv_freq = 1.0f32 / (f32)(base^(2i/d))
    with the power in f64, f32 products, f32 cos/sin) with the Hunyuan
    NTK-alpha base of hunyuan_dense/modeling.rs:202-219 when alpha > 0, cast to
    the model dtype as qwen3/modeling.rs:857-864 does.  Built on the host by
    crane_hip_rope_tables (the C library's cosf/sinf, which Rust's f32::cos and
    f32::sin call) once per model, then copied to `device`."""
    return _host_tables(_lib.lib().crane_hip_rope_tables, (float(theta), float(alpha or 0.0)), head_dim, max_pos,
                        device, dtype)


def rope_tables_qwen2(head_dim: int, theta: float, max_pos: int, device: torch.device | str = "cuda",
                      dtype: torch.dtype = torch.float32):
    """cos/sin tables [max_pos, head_dim/2] in candle-transformers qwen2's form
    (copy at qwen25/qwen2.rs:47-64): inv_freq and the positions are cast to the
    model dtype before the k=1 product, whose result is rounded to the model
    dtype, and cos/sin are computed in f32 and rounded.  In bf16 this rounds
    positions above 256 and the angles themselves; in f32 it equals
    rope_tables.  Built on the host (crane_hip_rope_tables_qwen2) once per
    model, then copied to `device`."""
    return _host_tables(_lib.lib().crane_hip_rope_tables_qwen2, (float(theta),), head_dim, max_pos, device, dtype)


# ------------------------------------------------------------ fused append op

def _rope_inputs(x: torch.Tensor, width: int, cos: torch.Tensor, sin: torch.Tensor, positions: torch.Tensor,
                 q_norm_w: Optional[torch.Tensor], k_norm_w: Optional[torch.Tensor], order: str, name: str = "qkv"):
    """Checks shared by every fused-rope entry point, for rows x [B, S, width]
    (the kernels read `width` elements of each row and cos/sin rows up to
    positions[b] + S - 1, bounds-checked against the table): returns (device,
    B, S)."""
    dev = _dev(x, cos, sin, positions, q_norm_w, k_norm_w)
    if x.dim() != 3:
        raise CraneHipError(_lib.E_INVALID, f"{name} must be [B, S, {width}]")
    B, S, W = x.shape
    if W != width:
        raise CraneHipError(_lib.E_INVALID, f"{name} last dim {W} != {width}")
    _dtype_code(x)
    if x.stride(2) != 1 or x.stride(0) != S * x.stride(1):
        raise CraneHipError(_lib.E_INVALID, f"{name} rows must be dense with a unit inner stride")
    _rope_tables(x.dtype, B, cos, sin, positions, q_norm_w, k_norm_w, order, name)
    return dev, B, S


def _rope_tables(dtype: torch.dtype, B: int, cos: torch.Tensor, sin: torch.Tensor, positions: torch.Tensor,
                 q_norm_w: Optional[torch.Tensor], k_norm_w: Optional[torch.Tensor], order: str, name: str):
    """The tables, norm weights, positions and order of a fused-rope call whose
    rows are in `dtype`, for B sequences."""
    for t, n in ((cos, "cos"), (sin, "sin"), (q_norm_w, "q_norm_w"), (k_norm_w, "k_norm_w")):
        if t is not None and t.dtype != dtype:
            raise CraneHipError(_lib.E_DTYPE, f"{n} dtype {t.dtype} != {name} dtype {dtype}")
    for t, n in ((q_norm_w, "q_norm_w"), (k_norm_w, "k_norm_w")):
        if t is not None and (t.numel() != HEAD_DIM or not t.is_contiguous()):
            raise CraneHipError(_lib.E_INVALID, f"{n} must be a contiguous [{HEAD_DIM}] weight")
    _contig(cos, "cos")
    _contig(sin, "sin")
    if cos.shape != sin.shape or cos.dim() != 2 or cos.shape[1] != HEAD_DIM // 2:
        raise CraneHipError(_lib.E_INVALID, "cos/sin must be [max_pos, D/2]")
    _i32(positions, B, "positions")
    if order not in _ORDERS:
        raise CraneHipError(_lib.E_INVALID, f"order {order!r}")


def qk_norm_rope_append(qkv: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor,
                        positions: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                        cache_len: torch.Tensor, max_rows: int, num_heads: int, num_kv_heads: int,
                        q_norm_w: Optional[torch.Tensor] = None,
                        k_norm_w: Optional[torch.Tensor] = None, eps: float = 1e-6,
                        order: str = "norm_then_rope") -> torch.Tensor:
    """Per-head QK-RMSNorm + RoPE, K/V written into the cache at rows
    [cache_len[b], cache_len[b]+S).  Returns q [B, Hq, S, D].

    Replaces qwen3/modeling.rs:382-423 + update_kv_cache's slice_set (:324-327);
    order "rope_then_norm" is Hunyuan's (hunyuan_dense/modeling.rs:541-555) and
    "rope_only" Qwen2.5's (qwen2.rs:75-76).  `max_rows` is a host-side bound
    on cache_len[b] + S, checked against the cache capacity.  qkv may be a
    PartialProduct of the projection (linear_for_append): its splits are
    summed (with its bias) and rounded in the same launch."""
    D = HEAD_DIM
    if isinstance(qkv, PartialProduct):
        return _qk_norm_rope_append_parts(qkv, cos, sin, positions, k_cache, v_cache, cache_len, max_rows, num_heads,
                                          num_kv_heads, q_norm_w, k_norm_w, eps, order)
    dev, B, S = _rope_inputs(qkv, (num_heads + 2 * num_kv_heads) * D, cos, sin, positions, q_norm_w, k_norm_w, order)
    _dev(qkv, k_cache, v_cache, cache_len)
    if k_cache.shape != v_cache.shape or k_cache.dim() != 4 or k_cache.shape[0] != B or \
            k_cache.shape[1] != num_kv_heads or k_cache.shape[3] != D:
        raise CraneHipError(_lib.E_INVALID, "caches must be [B, Hkv, cap, D]")
    dt = _dtype_code(qkv)
    for t, name in ((k_cache, "k_cache"), (v_cache, "v_cache")):
        if t.dtype != qkv.dtype:
            raise CraneHipError(_lib.E_DTYPE, f"{name} dtype {t.dtype} != qkv dtype {qkv.dtype}")
        _contig(t, name)
    _i32(cache_len, B, "cache_len")
    q_out = torch.empty((B, num_heads, S, D), dtype=qkv.dtype, device=dev)
    rc = _lib.lib().crane_hip_qknorm_rope_append(
        qkv.data_ptr(), qkv.stride(1), _ptr(q_norm_w), _ptr(k_norm_w), eps, _ORDERS[order],
        cos.data_ptr(), sin.data_ptr(), cos.stride(0), cos.shape[0], positions.data_ptr(),
        q_out.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(), k_cache.shape[2],
        cache_len.data_ptr(), max_rows, B, S, num_heads, num_kv_heads, D, dt, _stream(dev))
    check(rc, "qk_norm_rope_append")
    return q_out


def _qk_norm_rope_append_parts(pp: "PartialProduct", cos, sin, positions, k_cache, v_cache, cache_len, max_rows,
                               num_heads, num_kv_heads, q_norm_w, k_norm_w, eps, order) -> torch.Tensor:
    D = HEAD_DIM
    width = (num_heads + 2 * num_kv_heads) * D
    parts = pp.parts
    dev = _dev(parts, cos, sin, positions, q_norm_w, k_norm_w, k_cache, v_cache, cache_len, pp.bias)
    B = positions.numel()
    if parts.dim() != 3 or parts.dtype != torch.float32 or B < 1 or parts.shape[1] % B or parts.shape[2] != width:
        raise CraneHipError(_lib.E_INVALID, f"partial products must be f32 [splits, B*S, {width}]")
    sp, S = parts.shape[0], parts.shape[1] // B
    _contig(parts, "parts")
    dt = _dtype_code_of(pp.dtype)
    _rope_tables(pp.dtype, B, cos, sin, positions, q_norm_w, k_norm_w, order, "qkv")
    if pp.bias is not None and (pp.bias.dtype != pp.dtype or pp.bias.numel() != width or not pp.bias.is_contiguous()):
        raise CraneHipError(_lib.E_INVALID, f"bias must be a contiguous [{width}] tensor of the rows' dtype")
    if k_cache.shape != v_cache.shape or k_cache.dim() != 4 or k_cache.shape[0] != B or \
            k_cache.shape[1] != num_kv_heads or k_cache.shape[3] != D:
        raise CraneHipError(_lib.E_INVALID, "caches must be [B, Hkv, cap, D]")
    for t, name in ((k_cache, "k_cache"), (v_cache, "v_cache")):
        if t.dtype != pp.dtype:
            raise CraneHipError(_lib.E_DTYPE, f"{name} dtype {t.dtype} != qkv dtype {pp.dtype}")
        _contig(t, name)
    _i32(cache_len, B, "cache_len")
    q_out = torch.empty((B, num_heads, S, D), dtype=pp.dtype, device=dev)
    rc = _lib.lib().crane_hip_qknorm_rope_append_parts(
        parts.data_ptr(), sp, _ptr(pp.bias), _ptr(q_norm_w), _ptr(k_norm_w), eps, _ORDERS[order],
        cos.data_ptr(), sin.data_ptr(), cos.stride(0), cos.shape[0], positions.data_ptr(),
        q_out.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(), k_cache.shape[2],
        cache_len.data_ptr(), max_rows, B, S, num_heads, num_kv_heads, D, dt, _stream(dev))
    check(rc, "qk_norm_rope_append")
    return q_out


def q_norm_rope(q: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor, positions: torch.Tensor,
                num_heads: int, q_norm_w: Optional[torch.Tensor] = None, eps: float = 1e-6,
                order: str = "rope_then_norm") -> torch.Tensor:
    """RoPE and the per-head query norm of a layer that reuses another layer's
    K/V: Hunyuan's CLA path (hunyuan_dense/modeling.rs:502-514), q = rope(q)
    then query_layernorm.  q is [B, S, Hq*D] (rows may be a narrowed view with
    a unit inner stride); returns [B, Hq, S, D] for the attention ops, which
    then read the anchor layer's cache."""
    D = HEAD_DIM
    dev, B, S = _rope_inputs(q, num_heads * D, cos, sin, positions, q_norm_w, None, order, name="q")
    dt = _dtype_code(q)
    q_out = torch.empty((B, num_heads, S, D), dtype=q.dtype, device=dev)
    rc = _lib.lib().crane_hip_qnorm_rope(
        q.data_ptr(), q.stride(1), _ptr(q_norm_w), eps, _ORDERS[order], cos.data_ptr(), sin.data_ptr(),
        cos.stride(0), cos.shape[0], positions.data_ptr(), q_out.data_ptr(), B, S, num_heads, D, dt, _stream(dev))
    check(rc, "q_norm_rope")
    return q_out


# ---------------------------------------------------------------- decode op

def decode_workspace_bytes(batch: int, num_heads: int, num_kv_heads: int, max_kv: int,
                           dtype: torch.dtype = torch.bfloat16) -> int:
    return int(_lib.lib().crane_hip_attn_decode_workspace(batch, num_heads, num_kv_heads, HEAD_DIM,
                                                          max_kv, _DTYPES.get(dtype, 0)))


_WORKSPACES: dict = {}


def decode_workspace(device: torch.device, nbytes: int) -> torch.Tensor:
    """A per-(device, stream) scratch buffer for the split-KV partials, grown on
    demand; calls on one stream are ordered, so they can share it."""
    key = (device, torch.cuda.current_stream(device).cuda_stream)
    ws = _WORKSPACES.get(key)
    if ws is None or ws.numel() < nbytes:
        ws = torch.empty(max(nbytes, 256), dtype=torch.uint8, device=device)
        _WORKSPACES[key] = ws
    return ws


def attention_decode(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                     kv_len: torch.Tensor, max_kv: int, scale: Optional[float] = None,
                     workspace: Optional[torch.Tensor] = None, score_mode: Optional[str] = None) -> torch.Tensor:
    """Batched decode attention, one new token per sequence: q [B, Hq, D] (or
    [B, Hq, 1, D]) over cache rows [0, kv_len[b]).  Returns [B, 1, Hq*D].

    Replaces the GQA-grouped decode SDPA of qwen3/modeling.rs:432-467 (or, with
    score_mode "standard", the standard SDPA of :485-500 / qwen2.rs:196-201;
    see score_mode_code) and the pad + mask of the batched path (:1118-1200)."""
    dev = _dev(q, k_cache, v_cache, kv_len, workspace)
    if q.dim() == 4:
        if q.shape[2] != 1:
            raise CraneHipError(_lib.E_INVALID, "decode q must hold one token per sequence")
        q = q.reshape(q.shape[0], q.shape[1], q.shape[3])
    if q.dim() != 3 or q.shape[2] != HEAD_DIM:
        raise CraneHipError(_lib.E_HEAD_DIM if q.dim() == 3 else _lib.E_INVALID, "q must be [B, Hq, 128]")
    B, Hq, D = q.shape
    if k_cache.shape != v_cache.shape or k_cache.dim() != 4 or k_cache.shape[0] != B or k_cache.shape[3] != D:
        raise CraneHipError(_lib.E_INVALID, "caches must be [B, Hkv, cap, D]")
    Hkv = k_cache.shape[1]
    for t, name in ((q, "q"), (k_cache, "k_cache"), (v_cache, "v_cache")):
        _contig(t, name)
        if t.dtype != q.dtype:
            raise CraneHipError(_lib.E_DTYPE, f"{name} dtype {t.dtype} != {q.dtype}")
    dt = _dtype_code(q)
    _i32(kv_len, B, "kv_len")
    scale = 1.0 / math.sqrt(D) if scale is None else float(scale)
    need = decode_workspace_bytes(B, Hq, Hkv, max_kv, q.dtype)
    if workspace is None:
        workspace = decode_workspace(dev, need)
    out = torch.empty((B, 1, Hq * D), dtype=q.dtype, device=dev)
    mode = score_mode_code(score_mode, Hq // Hkv)
    rc = _lib.lib().crane_hip_attn_decode(
        q.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(), k_cache.shape[2], kv_len.data_ptr(),
        max_kv, B, Hq, Hkv, D, scale, mode, workspace.data_ptr(), workspace.numel() * workspace.element_size(),
        out.data_ptr(), dt, _stream(dev))
    check(rc, "attention_decode")
    return out


# --------------------------------------------------------------- prefill op

PREFILL_CAUSAL = 1                  # CRANE_HIP_PREFILL_CAUSAL
PREFILL_LONG_ROWS_ONE_ROUNDING = 2  # CRANE_HIP_PREFILL_LONG_ROWS_ONE_ROUNDING


def _prefill_flags(causal: bool, long_rows_one_rounding: bool) -> int:
    return (PREFILL_CAUSAL if causal else 0) | (PREFILL_LONG_ROWS_ONE_ROUNDING if long_rows_one_rounding else 0)


def attention_prefill(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                      start_pos: torch.Tensor, max_start: int, scale: Optional[float] = None,
                      causal: bool = True, long_rows_one_rounding: bool = False) -> torch.Tensor:
    """Causal GQA prefill: q [B, Hq, S, D] against cache rows [0, start_pos[b]+S).
    Returns [B, S, Hq*D].  Replaces qwen3/modeling.rs:469-502 with the mask of
    :866-884.  bf16 scores follow both of candle's roundings (:487-488);
    long_rows_one_rounding=True opts in to the first one only in query tiles
    whose rows see 1024 keys or more (CRANE_HIP_PREFILL_LONG_ROWS_ONE_ROUNDING)."""
    dev = _dev(q, k_cache, v_cache, start_pos)
    if q.dim() != 4:
        raise CraneHipError(_lib.E_INVALID, "q must be [B, Hq, S, D]")
    B, Hq, S, D = q.shape
    if D != HEAD_DIM:
        raise CraneHipError(_lib.E_HEAD_DIM, f"head_dim {D}")
    if k_cache.shape != v_cache.shape or k_cache.dim() != 4 or k_cache.shape[0] != B or k_cache.shape[3] != D:
        raise CraneHipError(_lib.E_INVALID, "caches must be [B, Hkv, cap, D]")
    for t, name in ((q, "q"), (k_cache, "k_cache"), (v_cache, "v_cache")):
        _contig(t, name)
        if t.dtype != q.dtype:
            raise CraneHipError(_lib.E_DTYPE, f"{name} dtype {t.dtype} != {q.dtype}")
    dt = _dtype_code(q)
    _i32(start_pos, B, "start_pos")
    scale = 1.0 / math.sqrt(D) if scale is None else float(scale)
    out = torch.empty((B, S, Hq * D), dtype=q.dtype, device=dev)
    rc = _lib.lib().crane_hip_attn_prefill(
        q.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(), k_cache.shape[2], start_pos.data_ptr(),
        max_start, B, S, Hq, k_cache.shape[1], D, scale, _prefill_flags(causal, long_rows_one_rounding),
        out.data_ptr(), dt, _stream(dev))
    check(rc, "attention_prefill")
    return out


# ------------------------------------------------------------- paged layout
# K and V pools [n_pages, Hkv, page_rows, D] and a block table [B, stride]
# (int32): row j of sequence b is row j % page_rows of page
# block_table[b, j // page_rows].  Same operations, same results as the dense
# entry points over the same rows (include/crane_hip.h, paged launchers).

PAGE_ALIGN = 256


def _paged_args(k_pool: torch.Tensor, v_pool: torch.Tensor, block_table: torch.Tensor, B: int,
                dtype: torch.dtype):
    if k_pool.shape != v_pool.shape or k_pool.dim() != 4 or k_pool.shape[3] != HEAD_DIM:
        raise CraneHipError(_lib.E_INVALID, "pools must be [n_pages, Hkv, page_rows, D]")
    for t, name in ((k_pool, "k_pool"), (v_pool, "v_pool")):
        _contig(t, name)
        if t.dtype != dtype:
            raise CraneHipError(_lib.E_DTYPE, f"{name} dtype {t.dtype} != {dtype}")
    if block_table.dtype != torch.int32 or block_table.dim() != 2 or block_table.shape[0] != B or \
            not block_table.is_contiguous():
        raise CraneHipError(_lib.E_INVALID, "block_table must be a contiguous int32 [B, max_pages] tensor")
    n_pages, Hkv, page_rows, _ = k_pool.shape
    return n_pages, Hkv, page_rows, block_table.shape[1]


def qk_norm_rope_append_paged(qkv: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor, positions: torch.Tensor,
                              k_pool: torch.Tensor, v_pool: torch.Tensor, block_table: torch.Tensor,
                              cache_len: torch.Tensor, num_heads: int, q_norm_w: Optional[torch.Tensor] = None,
                              k_norm_w: Optional[torch.Tensor] = None, eps: float = 1e-6,
                              order: str = "norm_then_rope") -> torch.Tensor:
    """qk_norm_rope_append into a paged cache: token s of sequence b lands in
    its row cache_len[b]+s.  Returns q [B, Hq, S, D]."""
    _dev(qkv, k_pool, v_pool, block_table, cache_len)
    if qkv.dim() != 3:
        raise CraneHipError(_lib.E_INVALID, "qkv must be [B, S, (Hq+2Hkv)*D]")
    n_pages, Hkv, page_rows, stride = _paged_args(k_pool, v_pool, block_table, qkv.shape[0], qkv.dtype)
    dev, B, S = _rope_inputs(qkv, (num_heads + 2 * Hkv) * HEAD_DIM, cos, sin, positions, q_norm_w, k_norm_w, order)
    dt = _dtype_code(qkv)
    _i32(cache_len, B, "cache_len")
    q_out = torch.empty((B, num_heads, S, HEAD_DIM), dtype=qkv.dtype, device=dev)
    rc = _lib.lib().crane_hip_qknorm_rope_append_paged(
        qkv.data_ptr(), qkv.stride(1), _ptr(q_norm_w), _ptr(k_norm_w), eps, _ORDERS[order], cos.data_ptr(),
        sin.data_ptr(), cos.stride(0), cos.shape[0], positions.data_ptr(), q_out.data_ptr(), k_pool.data_ptr(),
        v_pool.data_ptr(), n_pages, page_rows, block_table.data_ptr(), stride, cache_len.data_ptr(), B, S,
        num_heads, Hkv, HEAD_DIM, dt, _stream(dev))
    check(rc, "qk_norm_rope_append_paged")
    return q_out


def attention_decode_paged(q: torch.Tensor, k_pool: torch.Tensor, v_pool: torch.Tensor, block_table: torch.Tensor,
                           kv_len: torch.Tensor, max_kv: int, scale: Optional[float] = None,
                           workspace: Optional[torch.Tensor] = None, score_mode: Optional[str] = None) -> torch.Tensor:
    """attention_decode over a paged cache: q [B, Hq, D]; [B, 1, Hq*D]."""
    dev = _dev(q, k_pool, v_pool, block_table, kv_len, workspace)
    if q.dim() != 3 or q.shape[2] != HEAD_DIM:
        raise CraneHipError(_lib.E_INVALID, "q must be [B, Hq, 128]")
    B, Hq, D = q.shape
    n_pages, Hkv, page_rows, stride = _paged_args(k_pool, v_pool, block_table, B, q.dtype)
    _contig(q, "q")
    dt = _dtype_code(q)
    _i32(kv_len, B, "kv_len")
    scale = 1.0 / math.sqrt(D) if scale is None else float(scale)
    if workspace is None:
        workspace = decode_workspace(dev, decode_workspace_bytes(B, Hq, Hkv, max_kv, q.dtype))
    out = torch.empty((B, 1, Hq * D), dtype=q.dtype, device=dev)
    rc = _lib.lib().crane_hip_attn_decode_paged(
        q.data_ptr(), k_pool.data_ptr(), v_pool.data_ptr(), n_pages, page_rows, block_table.data_ptr(), stride,
        kv_len.data_ptr(), max_kv, B, Hq, Hkv, D, scale, score_mode_code(score_mode, Hq // Hkv), workspace.data_ptr(),
        workspace.numel() * workspace.element_size(), out.data_ptr(), dt, _stream(dev))
    check(rc, "attention_decode_paged")
    return out


def attention_prefill_paged(q: torch.Tensor, k_pool: torch.Tensor, v_pool: torch.Tensor,
                            block_table: torch.Tensor, start_pos: torch.Tensor, max_start: int,
                            scale: Optional[float] = None, causal: bool = True,
                            long_rows_one_rounding: bool = False) -> torch.Tensor:
    """attention_prefill over a paged cache: q [B, Hq, S, D]; [B, S, Hq*D]."""
    dev = _dev(q, k_pool, v_pool, block_table, start_pos)
    if q.dim() != 4 or q.shape[3] != HEAD_DIM:
        raise CraneHipError(_lib.E_INVALID, "q must be [B, Hq, S, 128]")
    B, Hq, S, D = q.shape
    n_pages, Hkv, page_rows, stride = _paged_args(k_pool, v_pool, block_table, B, q.dtype)
    _contig(q, "q")
    dt = _dtype_code(q)
    _i32(start_pos, B, "start_pos")
    scale = 1.0 / math.sqrt(D) if scale is None else float(scale)
    out = torch.empty((B, S, Hq * D), dtype=q.dtype, device=dev)
    rc = _lib.lib().crane_hip_attn_prefill_paged(
        q.data_ptr(), k_pool.data_ptr(), v_pool.data_ptr(), n_pages, page_rows, block_table.data_ptr(), stride,
        start_pos.data_ptr(), max_start, B, S, Hq, Hkv, D, scale, _prefill_flags(causal, long_rows_one_rounding),
        out.data_ptr(), dt, _stream(dev))
    check(rc, "attention_prefill_paged")
    return out


# ------------------------------------------------------- decoder-layer rows
# The row kernels either side of the attention block (include/crane_layer.h):
# RmsNorm, residual add + RmsNorm, SiLU(gate) * up, residual add
# (qwen3/modeling.rs:655-673, crane-core/src/fused_ops).

def _rows_of(t: torch.Tensor, name: str):
    _contig(t, name)
    if t.dim() < 1:
        raise CraneHipError(_lib.E_INVALID, f"{name} must have a last dimension")
    cols = t.shape[-1]
    return t.numel() // max(cols, 1), cols


def rms_norm(x: torch.Tensor, weight: Optional[torch.Tensor] = None, eps: float = 1e-6) -> torch.Tensor:
    """candle_nn::RmsNorm::forward over the last dimension of a contiguous x."""
    dev = _dev(x, weight)
    rows, cols = _rows_of(x, "x")
    dt = _dtype_code(x)
    if weight is not None and (weight.dtype != x.dtype or weight.numel() != cols or not weight.is_contiguous()):
        raise CraneHipError(_lib.E_INVALID, "weight must be a contiguous [cols] tensor of x's dtype")
    out = torch.empty_like(x)
    check(_lib.lib().crane_hip_rms_norm(x.data_ptr(), _ptr(weight), out.data_ptr(), rows, cols, eps, dt,
                                        _stream(dev)), "rms_norm")
    return out


def add_rms_norm(residual: torch.Tensor, hidden, weight: Optional[torch.Tensor] = None,
                 eps: float = 1e-6) -> torch.Tensor:
    """residual += hidden (in place, rounded to the dtype), then RmsNorm of the
    new residual (Crane's FusedAddRmsNorm::fwd).  Returns the normed rows.
    hidden may be a PartialProduct (linear_for_residual): its splits are
    summed and rounded to the dtype in the same launch."""
    if isinstance(hidden, PartialProduct):
        return _add_rms_norm_parts(residual, hidden, weight, eps)
    dev = _dev(residual, hidden, weight)
    if residual.shape != hidden.shape or residual.dtype != hidden.dtype:
        raise CraneHipError(_lib.E_INVALID, "residual and hidden must have the same shape and dtype")
    rows, cols = _rows_of(residual, "residual")
    _contig(hidden, "hidden")
    dt = _dtype_code(residual)
    if weight is not None and (weight.dtype != residual.dtype or weight.numel() != cols or
                               not weight.is_contiguous()):
        raise CraneHipError(_lib.E_INVALID, "weight must be a contiguous [cols] tensor of the rows' dtype")
    out = torch.empty_like(residual)
    check(_lib.lib().crane_hip_add_rms_norm(residual.data_ptr(), hidden.data_ptr(), _ptr(weight), out.data_ptr(),
                                            rows, cols, eps, dt, _stream(dev)), "add_rms_norm")
    return out


def silu_mul(gate_up: torch.Tensor, intermediate_size: Optional[int] = None) -> torch.Tensor:
    """Crane's fused_silu_mul: gate_up [..., 2*I] (gate || up) -> silu(gate) * up [..., I]."""
    dev = _dev(gate_up)
    rows, last = _rows_of(gate_up, "gate_up")
    inter = intermediate_size if intermediate_size is not None else last // 2
    if last != 2 * inter:
        raise CraneHipError(_lib.E_INVALID, f"last dim {last} != 2*intermediate_size {2 * inter}")
    dt = _dtype_code(gate_up)
    out = torch.empty(gate_up.shape[:-1] + (inter,), dtype=gate_up.dtype, device=dev)
    check(_lib.lib().crane_hip_silu_mul(gate_up.data_ptr(), out.data_ptr(), rows, inter, dt, _stream(dev)),
          "silu_mul")
    return out


def residual_add(residual: torch.Tensor, hidden: torch.Tensor) -> torch.Tensor:
    """residual += hidden in place (rounded to the dtype); returns residual."""
    dev = _dev(residual, hidden)
    if residual.shape != hidden.shape or residual.dtype != hidden.dtype:
        raise CraneHipError(_lib.E_INVALID, "residual and hidden must have the same shape and dtype")
    _contig(residual, "residual")
    _contig(hidden, "hidden")
    check(_lib.lib().crane_hip_residual_add(residual.data_ptr(), hidden.data_ptr(), residual.numel(),
                                            _dtype_code(residual), _stream(dev)), "residual_add")
    return residual


# ------------------------------------------------------------- projections
# candle Linear (y = x W^T + b) on hipBLASLt (include/crane_gemm.h): the merged
# qkv_proj whose output rows feed qk_norm_rope_append, and o_proj.

class _GemmContext:
    """One crane_gemm (hipBLASLt handle, workspace, per-shape plans) per
    (device, stream): calls on one stream are ordered, so they can share its
    workspace; calls on different streams may overlap and must not."""

    def __init__(self, device: torch.device):
        h = ctypes.c_void_p()
        with torch.cuda.device(device):
            check(_lib.lib().crane_gemm_create(0, ctypes.byref(h)), "crane_gemm_create")
        self._h = h
        self._destroy = _lib.lib().crane_gemm_destroy  # bound now: usable during interpreter shutdown

    def __del__(self):
        if getattr(self, "_h", None):
            self._destroy(self._h)
            self._h = None


_GEMMS: dict = {}


def _gemm(device: torch.device) -> _GemmContext:
    key = (device, torch.cuda.current_stream(device).cuda_stream)
    ctx = _GEMMS.get(key)
    if ctx is None:
        ctx = _GEMMS[key] = _GemmContext(device)
    return ctx


def release_stream(device: Optional[torch.device] = None, stream: Optional[torch.cuda.Stream] = None) -> None:
    """Drop the decode workspace and the GEMM context kept for `stream`
    (default: the current stream of `device`).  Both live as long as their
    stream is in use, one per (device, stream); a caller that retires a stream
    releases them here.  The GEMM context's destruction frees its workspace
    with hipFree, which waits for work already queued on the device."""
    dev = torch.device(device) if device is not None else torch.device("cuda", torch.cuda.current_device())
    st = stream if stream is not None else torch.cuda.current_stream(dev)
    key = (dev, st.cuda_stream)
    _WORKSPACES.pop(key, None)
    _GEMMS.pop(key, None)


class PartialProduct:
    """The f32 split-K partial products [splits, M, N] of a projection
    (crane_gemm_linear_split) whose output only feeds add_rms_norm or
    qk_norm_rope_append, which sum them in split order (adding `bias`, when
    given, for the append) and round once, as the whole product's output."""

    def __init__(self, parts: torch.Tensor, dtype: torch.dtype, bias: Optional[torch.Tensor] = None):
        self.parts, self.dtype, self.bias = parts, dtype, bias

    @property
    def shape(self):
        return self.parts.shape[1:]


_SPLITS = (4, 2)  # split counts tried, in order (4: o_proj and down_proj of a decode step)


def linear_for_residual(x: torch.Tensor, weight: torch.Tensor):
    """The projection x [M, K] W^T of a decode step whose output goes only into
    add_rms_norm (o_proj, down_proj): a PartialProduct when a split of K
    applies (bf16, M <= 32; crane_gemm_split_supported), else linear(x, weight).
    The split kernels read x fewer times per weight byte."""
    dev = _dev(x, weight)
    K = x.shape[-1]
    M = x.numel() // K
    if x.dtype == torch.bfloat16 and weight.dim() == 2 and weight.shape[1] == K and weight.dtype == x.dtype:
        N = weight.shape[0]
        for sp in _SPLITS:
            if _lib.lib().crane_gemm_split_supported(M, N, K, sp, _lib.BF16):
                _contig(x, "x")
                _contig(weight, "weight")
                parts = torch.empty((sp, M, N), dtype=torch.float32, device=dev)
                check(_lib.lib().crane_gemm_linear_split(_gemm(dev)._h, x.data_ptr(), weight.data_ptr(),
                                                         parts.data_ptr(), M, N, K, sp, _lib.BF16, _stream(dev)),
                      "linear_split")
                return PartialProduct(parts, x.dtype)
    return linear(x, weight)


def linear_for_append(x: torch.Tensor, weight: torch.Tensor, bias: Optional[torch.Tensor] = None):
    """The merged qkv projection x [M, K] W^T (+ bias) of a decode step, whose
    rows go only into qk_norm_rope_append: a PartialProduct of 2 splits when
    the split applies (bf16, M <= 32; crane_gemm_split_supported), else
    linear(x, weight, bias).  (2 splits: 10.7 us at Qwen3-8B's qkv_proj and
    32 rows, against 13.7 for linear and 11.7 with 4 splits.)"""
    dev = _dev(x, weight, bias)
    K = x.shape[-1]
    M = x.numel() // K
    if x.dtype == torch.bfloat16 and weight.dim() == 2 and weight.shape[1] == K and weight.dtype == x.dtype and \
            (bias is None or bias.dtype == x.dtype):
        N = weight.shape[0]
        if _lib.lib().crane_gemm_split_supported(M, N, K, 2, _lib.BF16):
            _contig(x, "x")
            _contig(weight, "weight")
            parts = torch.empty((2, M, N), dtype=torch.float32, device=dev)
            check(_lib.lib().crane_gemm_linear_split(_gemm(dev)._h, x.data_ptr(), weight.data_ptr(), parts.data_ptr(),
                                                     M, N, K, 2, _lib.BF16, _stream(dev)), "linear_split")
            return PartialProduct(parts, x.dtype, bias)
    return linear(x, weight, bias)


def _add_rms_norm_parts(residual: torch.Tensor, hidden: PartialProduct, weight: Optional[torch.Tensor],
                        eps: float) -> torch.Tensor:
    dev = _dev(residual, hidden.parts, weight)
    rows, cols = _rows_of(residual, "residual")
    sp = hidden.parts.shape[0]
    if hidden.dtype != residual.dtype or tuple(hidden.parts.shape) != (sp, rows, cols):
        raise CraneHipError(_lib.E_INVALID, "partial products must be [splits, rows, cols] of the residual's dtype")
    _contig(hidden.parts, "parts")
    if weight is not None and (weight.dtype != residual.dtype or weight.numel() != cols or
                               not weight.is_contiguous()):
        raise CraneHipError(_lib.E_INVALID, "weight must be a contiguous [cols] tensor of the rows' dtype")
    out = torch.empty_like(residual)
    check(_lib.lib().crane_hip_add_rms_norm_parts(residual.data_ptr(), hidden.parts.data_ptr(), sp, _ptr(weight),
                                                  out.data_ptr(), rows, cols, eps, _dtype_code(residual),
                                                  _stream(dev)), "add_rms_norm")
    return out


def linear(x: torch.Tensor, weight: torch.Tensor, bias: Optional[torch.Tensor] = None) -> torch.Tensor:
    """candle Linear::forward: x [..., K] with weight [N, K] (and bias [N]) ->
    [..., N]; f32 accumulation, the bias added in the GEMM epilogue."""
    dev = _dev(x, weight, bias)
    K = x.shape[-1]
    if weight.dim() != 2 or weight.shape[1] != K:
        raise CraneHipError(_lib.E_INVALID, f"weight must be [N, {K}]")
    N = weight.shape[0]
    for t, name in ((x, "x"), (weight, "weight"), (bias, "bias")):
        if t is not None:
            _contig(t, name)
            if t.dtype != x.dtype:
                raise CraneHipError(_lib.E_DTYPE, f"{name} dtype {t.dtype} != {x.dtype}")
    if bias is not None and bias.numel() != N:
        raise CraneHipError(_lib.E_INVALID, f"bias must have {N} elements")
    dt = _dtype_code(x)
    M = x.numel() // K
    y = torch.empty(x.shape[:-1] + (N,), dtype=x.dtype, device=dev)
    check(_lib.lib().crane_gemm_linear(_gemm(dev)._h, x.data_ptr(), weight.data_ptr(), _ptr(bias), y.data_ptr(),
                                       M, N, K, dt, _stream(dev)), "linear")
    return y


def linear_silu_mul(x: torch.Tensor, gate_up: torch.Tensor) -> torch.Tensor:
    """Crane's Mlp gate / up projections and fused_silu_mul: x [..., K] with
    the merged weight gate_up [2 I, K] (gate rows first) -> silu(gate) * up
    [..., I].  One launch where the library's gated kernel takes the shape
    (decode batches, crane_gemm_silu_mul_supported), else linear then
    silu_mul; the roundings are the same either way."""
    dev = _dev(x, gate_up)
    K = x.shape[-1]
    if gate_up.dim() != 2 or gate_up.shape[1] != K or gate_up.shape[0] % 2:
        raise CraneHipError(_lib.E_INVALID, f"gate_up must be [2 I, {K}]")
    inter = gate_up.shape[0] // 2
    M = x.numel() // K
    dt = _dtype_code(x)
    if not _lib.lib().crane_gemm_silu_mul_supported(M, inter, K, dt):
        return silu_mul(linear(x, gate_up), inter)
    _contig(x, "x")
    _contig(gate_up, "gate_up")
    if gate_up.dtype != x.dtype:
        raise CraneHipError(_lib.E_DTYPE, f"gate_up dtype {gate_up.dtype} != {x.dtype}")
    out = torch.empty(x.shape[:-1] + (inter,), dtype=x.dtype, device=dev)
    check(_lib.lib().crane_gemm_linear_silu_mul(_gemm(dev)._h, x.data_ptr(), gate_up.data_ptr(), out.data_ptr(), M,
                                                inter, K, dt, _stream(dev)), "linear_silu_mul")
    return out


# ---------------------------------------------------------------- sampling
# Token selection on the logits (include/crane_sampling.h): Crane's gpu_argmax
# (greedy) and topk_indices (top-k / top-p candidates), batched over rows.

def argmax(logits: torch.Tensor) -> torch.Tensor:
    """Index of the largest value of every row of logits [..., n] (first one
    on ties); int32 [...]."""
    dev = _dev(logits)
    _contig(logits, "logits")
    n = logits.shape[-1]
    rows = logits.numel() // max(n, 1)
    out = torch.empty(logits.shape[:-1], dtype=torch.int32, device=dev)
    ws, wsb = _select_workspace(rows, n, dev)
    check(_lib.lib().crane_hip_argmax_ws(logits.data_ptr(), rows, n, _dtype_code(logits), _ptr(ws), wsb,
                                         out.data_ptr(), _stream(dev)), "argmax")
    return out


def _select_workspace(rows: int, n: int, dev: torch.device):
    """The split-row workspace of argmax / top-k (None when the shape takes the
    single-pass kernels); it holds nothing between calls."""
    wsb = int(_lib.lib().crane_hip_select_workspace_bytes(rows, n))
    return (torch.empty(wsb, dtype=torch.uint8, device=dev) if wsb else None), wsb


def topk_indices(x: torch.Tensor, k: int) -> torch.Tensor:
    """Indices of the k largest values of every row of x [..., n] (f32),
    largest first, ties by lower index; int32 [..., k]."""
    dev = _dev(x)
    _contig(x, "x")
    if x.dtype != torch.float32:
        raise CraneHipError(_lib.E_DTYPE, "topk_indices takes f32 logits")
    n = x.shape[-1]
    rows = x.numel() // max(n, 1)
    out = torch.empty(x.shape[:-1] + (k,), dtype=torch.int32, device=dev)
    ws, wsb = _select_workspace(rows, n, dev)
    check(_lib.lib().crane_hip_topk_ws(x.data_ptr(), rows, n, k, _ptr(ws), wsb, out.data_ptr(), _stream(dev)),
          "topk_indices")
    return out
