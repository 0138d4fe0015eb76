"""Python surface of the host-side KV-cache managers (include/crane_kv.h and
include/crane_pkv.h).

`KvCache` is one attention layer's cache in Crane's layout [B, Hkv, cap, D]
with a length per sequence; it mirrors Attention.kv_cache + cache_seq_len and
update_kv_cache (qwen3/modeling.rs:313-370).  `stack` / `extract` are the
batched-decode set-up and tear-down (setup_batch_decode :973-1030,
extract_batch_kv :1066-1102) without padding: sequence i keeps its rows at
[0, len_i) and the kernels read exactly those rows.  All work happens in
libcrane_hip.so; this module only passes pointers.
"""
from __future__ import annotations

import ctypes
from typing import List, Optional, Sequence

import torch

from . import _lib
from ._lib import CraneHipError, check
from .ops import HEAD_DIM, _ORDERS, _dev, _dtype_code, _prefill_flags, _ptr, _rope_inputs, _stream

_DT = {torch.float32: _lib.F32, torch.bfloat16: _lib.BF16}


def grown_capacity(cap: int, needed: int) -> int:
    """Rows a cache of `cap` rows holds after making room for `needed` rows
    (Crane's policy: unchanged if it fits, else needed + 256)."""
    return int(_lib.lib().crane_kv_grown_capacity(cap, needed))


def _check_q(q: torch.Tensor, ndim: int, batch: int, dtype: torch.dtype, device: torch.device) -> None:
    """q for a cache's attention ops: [B, Hq, D] (decode) or [B, Hq, S, D]
    (prefill) in the cache's dtype and on its device; the library reads it
    with the cache's element size."""
    if _dev(q) != device:
        raise CraneHipError(_lib.E_INVALID, f"q on {q.device}, cache on {device}")
    if q.dtype != dtype:
        raise CraneHipError(_lib.E_DTYPE, f"q dtype {q.dtype} != cache dtype {dtype}")
    if q.dim() != ndim or q.shape[0] != batch or q.shape[-1] != HEAD_DIM:
        shape = "[B, Hq, D]" if ndim == 3 else "[B, Hq, S, D]"
        raise CraneHipError(_lib.E_INVALID, f"q must be {shape} for a batch of {batch}, D = {HEAD_DIM}")


def _check_append(qkv: torch.Tensor, cos, sin, positions, num_heads: int, num_kv_heads: int, q_norm_w, k_norm_w,
                  order: str, batch: int, dtype: torch.dtype, device: torch.device) -> None:
    _rope_inputs(qkv, (num_heads + 2 * num_kv_heads) * HEAD_DIM, cos, sin, positions, q_norm_w, k_norm_w, order)
    if qkv.device != device:
        raise CraneHipError(_lib.E_INVALID, f"qkv on {qkv.device}, cache on {device}")
    if qkv.shape[0] != batch:
        raise CraneHipError(_lib.E_INVALID, f"qkv batch {qkv.shape[0]} != {batch}")
    if qkv.dtype != dtype:
        raise CraneHipError(_lib.E_DTYPE, f"qkv dtype {qkv.dtype} != cache dtype {dtype}")


class _DeviceView:
    """__cuda_array_interface__ over memory the library owns (no copy)."""

    def __init__(self, ptr: int, shape, typestr: str):
        self.__cuda_array_interface__ = {"shape": tuple(shape), "typestr": typestr, "data": (ptr, False),
                                         "version": 2, "strides": None}


class KvCache:
    """One layer's K/V cache for `batch` sequences of `num_kv_heads` heads."""

    def __init__(self, batch: int, num_kv_heads: int, dtype: torch.dtype = torch.bfloat16,
                 device: Optional[torch.device] = None, head_dim: int = HEAD_DIM):
        if dtype not in _DT:
            raise CraneHipError(_lib.E_DTYPE, f"KV cache dtype {dtype}")
        self.batch, self.num_kv_heads, self.dtype = batch, num_kv_heads, dtype
        self.device = torch.device(device) if device is not None else torch.device("cuda", torch.cuda.current_device())
        handle = ctypes.c_void_p()
        check(_lib.lib().crane_kv_create(batch, num_kv_heads, head_dim, _DT[dtype], ctypes.byref(handle)),
              "crane_kv_create")
        self._h = handle
        self._destroy = _lib.lib().crane_kv_destroy  # bound now: usable during interpreter shutdown

    def close(self) -> None:
        if getattr(self, "_h", None):
            self._destroy(self._h)
            self._h = None

    def __del__(self):
        self.close()

    # ------------------------------------------------------------ state

    def _views(self):
        k, v, cap, dlen = ctypes.c_void_p(), ctypes.c_void_p(), ctypes.c_int64(), ctypes.c_void_p()
        lens = (ctypes.c_int64 * max(self.batch, 1))()
        check(_lib.lib().crane_kv_views(self._h, ctypes.byref(k), ctypes.byref(v), ctypes.byref(cap),
                                        ctypes.byref(dlen), lens), "crane_kv_views")
        return k.value, v.value, cap.value, dlen.value, [int(x) for x in lens[:self.batch]]

    @property
    def capacity(self) -> int:
        return self._views()[2]

    @property
    def lengths(self) -> List[int]:
        """Valid rows per sequence (Crane's cache_seq_len, per sequence)."""
        return self._views()[4]

    @property
    def bytes(self) -> int:
        """Bytes of the allocated K and V buffers (active_kv_cache_bytes)."""
        return int(_lib.lib().crane_kv_bytes(self._h))

    def buffers(self):
        """(K, V) tensors [B, Hkv, cap, D] viewing the cache buffers (valid until
        the next append that grows the cache), or (None, None) before first use."""
        k, v, cap, _, _ = self._views()
        if not k:
            return None, None
        shape = (self.batch, self.num_kv_heads, cap, HEAD_DIM)
        ts = "<f4" if self.dtype == torch.float32 else "<i2"
        out = []
        for p in (k, v):
            t = torch.as_tensor(_DeviceView(p, shape, ts), device=self.device)
            out.append(t if self.dtype == torch.float32 else t.view(torch.bfloat16))
        return tuple(out)

    def get_kv_cache(self):
        """Views of the valid rows, like get_kv_caches: (k, v) narrowed to the
        longest sequence's length (shorter sequences' rows past their length
        are unspecified)."""
        k, v = self.buffers()
        if k is None:
            return None
        n = max(self.lengths) if self.batch else 0
        return k[:, :, :n], v[:, :, :n]

    def set_lengths(self, lengths: Sequence[int]) -> None:
        arr = (ctypes.c_int64 * max(self.batch, 1))(*lengths)
        check(_lib.lib().crane_kv_set_lengths(self._h, arr, _stream(self.device)), "crane_kv_set_lengths")

    def reserve(self, rows: int) -> None:
        check(_lib.lib().crane_kv_reserve(self._h, rows, _stream(self.device)), "crane_kv_reserve")

    # ------------------------------------------------------------ ops

    def update_kv_cache(self, k: torch.Tensor, v: torch.Tensor):
        """Append k, v [B, Hkv, S, D] at every sequence's length; returns the
        views of the valid rows (Attention::update_kv_cache)."""
        if k.shape != v.shape or k.dim() != 4 or k.shape[0] != self.batch or k.shape[1] != self.num_kv_heads:
            raise CraneHipError(_lib.E_INVALID, "k, v must be [B, Hkv, S, D] matching the cache")
        if k.dtype != self.dtype or v.dtype != self.dtype:
            raise CraneHipError(_lib.E_DTYPE, f"k/v dtype {k.dtype} != cache dtype {self.dtype}")
        k, v = k.contiguous(), v.contiguous()
        check(_lib.lib().crane_kv_update(self._h, k.data_ptr(), v.data_ptr(), k.shape[2], _stream(self.device)),
              "crane_kv_update")
        return self.get_kv_cache()

    def append_qkv(self, qkv: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor, positions: torch.Tensor,
                   num_heads: int, q_norm_w: Optional[torch.Tensor] = None, k_norm_w: Optional[torch.Tensor] = None,
                   eps: float = 1e-6, order: str = "norm_then_rope") -> torch.Tensor:
        """Fused QK-norm + RoPE written into this cache at the current lengths
        (growing it as update_kv_cache would); returns q [B, Hq, S, D]."""
        _check_append(qkv, cos, sin, positions, num_heads, self.num_kv_heads, q_norm_w, k_norm_w, order,
                      self.batch, self.dtype, self.device)
        B, S, _ = qkv.shape
        q_out = torch.empty((B, num_heads, S, HEAD_DIM), dtype=qkv.dtype, device=qkv.device)
        check(_lib.lib().crane_kv_append_qkv(
            self._h, qkv.data_ptr(), qkv.stride(1), _ptr(q_norm_w), _ptr(k_norm_w), eps, _ORDERS[order],
            cos.data_ptr(), sin.data_ptr(), cos.stride(0), cos.shape[0], positions.data_ptr(), q_out.data_ptr(),
            S, num_heads, _stream(qkv.device)), "crane_kv_append_qkv")
        return q_out

    def decode(self, q: torch.Tensor, scale: Optional[float] = None,
               workspace: Optional[torch.Tensor] = None, score_mode: Optional[str] = None) -> torch.Tensor:
        """Decode attention of q [B, Hq, D] over every sequence's rows; [B, 1, Hq*D]
        (score_mode as in ops.attention_decode)."""
        from .ops import decode_workspace, score_mode_code
        _check_q(q, 3, self.batch, self.dtype, self.device)
        q = q.contiguous()
        B, Hq, D = q.shape
        max_kv = max(self.lengths)
        need = _lib.lib().crane_hip_attn_decode_workspace(B, Hq, self.num_kv_heads, D, max_kv, _dtype_code(q))
        if workspace is not None:
            _dev(q, workspace)
        ws = workspace if workspace is not None else decode_workspace(q.device, need)
        out = torch.empty((B, 1, Hq * D), dtype=q.dtype, device=q.device)
        check(_lib.lib().crane_kv_decode(self._h, q.data_ptr(), Hq, scale if scale else D ** -0.5,
                                         score_mode_code(score_mode, Hq // self.num_kv_heads), ws.data_ptr(),
                                         ws.numel() * ws.element_size(), out.data_ptr(), _stream(q.device)),
              "crane_kv_decode")
        return out

    def prefill(self, q: torch.Tensor, scale: Optional[float] = None, causal: bool = True,
                long_rows_one_rounding: bool = False) -> torch.Tensor:
        """Attention of q [B, Hq, S, D] (the last S rows of every sequence) over
        the cache; [B, S, Hq*D].  long_rows_one_rounding as in
        ops.attention_prefill."""
        _check_q(q, 4, self.batch, self.dtype, self.device)
        B, Hq, S, D = q.shape
        out = torch.empty((B, S, Hq * D), dtype=q.dtype, device=q.device)
        check(_lib.lib().crane_kv_prefill(self._h, q.contiguous().data_ptr(), Hq, S, scale if scale else D ** -0.5,
                                          _prefill_flags(causal, long_rows_one_rounding), out.data_ptr(),
                                          _stream(q.device)), "crane_kv_prefill")
        return out


def stack(caches: Sequence[KvCache], extra_room: int = 0) -> KvCache:
    """Batched-decode set-up: one cache holding every single-sequence cache's
    rows at [0, len_i) of its slot, with max(len_i) + extra_room rows."""
    first = caches[0]
    dst = KvCache(len(caches), first.num_kv_heads, first.dtype, first.device)
    arr = (ctypes.c_void_p * len(caches))(*[c._h.value for c in caches])
    check(_lib.lib().crane_kv_stack(dst._h, arr, len(caches), extra_room, _stream(first.device)), "crane_kv_stack")
    return dst


def extract(batch: KvCache, i: int, dst: Optional[KvCache] = None) -> KvCache:
    """Batched-decode tear-down: sequence i's rows as a single-sequence cache."""
    out = dst if dst is not None else KvCache(1, batch.num_kv_heads, batch.dtype, batch.device)
    check(_lib.lib().crane_kv_extract(batch._h, i, out._h, _stream(batch.device)), "crane_kv_extract")
    return out


class PagedKvCache:
    """One layer's paged K/V cache (include/crane_pkv.h): pools of `n_pages`
    pages of `page_rows` rows, up to `max_seqs` sequences of at most
    `max_pages_per_seq` pages.  Sequences are ids; a batch is a list of ids
    (set_batch) and the ops below act on it.  No KV row moves when a batch is
    set up or torn down, or when a sequence grows: Crane's pad/stack/extract
    copies (qwen3/modeling.rs:973-1102) and update_kv_cache's reallocation copy
    (:333-355) have no counterpart here."""

    def __init__(self, num_kv_heads: int, n_pages: int, dtype: torch.dtype = torch.bfloat16,
                 page_rows: int = 256, max_seqs: int = 64, max_pages_per_seq: int = 128,
                 device: Optional[torch.device] = None, head_dim: int = HEAD_DIM):
        if dtype not in _DT:
            raise CraneHipError(_lib.E_DTYPE, f"KV cache dtype {dtype}")
        self.num_kv_heads, self.dtype, self.page_rows, self.n_pages = num_kv_heads, dtype, page_rows, n_pages
        self.max_seqs, self.max_pages_per_seq = max_seqs, max_pages_per_seq
        self.device = torch.device(device) if device is not None else torch.device("cuda", torch.cuda.current_device())
        handle = ctypes.c_void_p()
        check(_lib.lib().crane_pkv_create(num_kv_heads, head_dim, _DT[dtype], page_rows, n_pages, max_seqs,
                                          max_pages_per_seq, ctypes.byref(handle)), "crane_pkv_create")
        self._h = handle
        self._destroy = _lib.lib().crane_pkv_destroy  # bound now: usable during interpreter shutdown
        self._batch: List[int] = []

    def close(self) -> None:
        if getattr(self, "_h", None):
            self._destroy(self._h)
            self._h = None

    def __del__(self):
        self.close()

    # ------------------------------------------------------------ sequences

    def add_sequence(self) -> int:
        sid = ctypes.c_int()
        check(_lib.lib().crane_pkv_seq_add(self._h, ctypes.byref(sid)), "crane_pkv_seq_add")
        return sid.value

    def free_sequence(self, sid: int) -> None:
        check(_lib.lib().crane_pkv_seq_free(self._h, sid), "crane_pkv_seq_free")

    def seq_len(self, sid: int) -> int:
        return int(_lib.lib().crane_pkv_seq_len(self._h, sid))

    @property
    def free_pages(self) -> int:
        return int(_lib.lib().crane_pkv_free_pages(self._h))

    @property
    def bytes(self) -> int:
        """Bytes of the K and V pools."""
        return int(_lib.lib().crane_pkv_bytes(self._h))

    @property
    def lengths(self) -> List[int]:
        """Valid rows of the batch sequences."""
        return [self.seq_len(s) for s in self._batch]

    def set_batch(self, ids: Sequence[int]) -> None:
        arr = (ctypes.c_int * max(len(ids), 1))(*ids)
        check(_lib.lib().crane_pkv_set_batch(self._h, arr, len(ids), _stream(self.device)), "crane_pkv_set_batch")
        self._batch = list(ids)

    # ------------------------------------------------------------ views

    def _views(self):
        k, v, tbl, dlen = ctypes.c_void_p(), ctypes.c_void_p(), ctypes.c_void_p(), ctypes.c_void_p()
        stride = ctypes.c_int64()
        check(_lib.lib().crane_pkv_views(self._h, ctypes.byref(k), ctypes.byref(v), ctypes.byref(tbl),
                                         ctypes.byref(stride), ctypes.byref(dlen)), "crane_pkv_views")
        return k.value, v.value, tbl.value, stride.value, dlen.value

    def pools(self):
        """(K, V) tensors [n_pages, Hkv, page_rows, D] viewing the pools."""
        k, v, _, _, _ = self._views()
        shape = (self.n_pages, self.num_kv_heads, self.page_rows, HEAD_DIM)
        ts = "<f4" if self.dtype == torch.float32 else "<i2"
        out = []
        for p in (k, v):
            t = torch.as_tensor(_DeviceView(p, shape, ts), device=self.device)
            out.append(t if self.dtype == torch.float32 else t.view(torch.bfloat16))
        return tuple(out)

    def block_table(self) -> torch.Tensor:
        """The batch's block table [B, max_pages_per_seq] (int32, device view)."""
        _, _, tbl, stride, _ = self._views()
        return torch.as_tensor(_DeviceView(tbl, (len(self._batch), stride), "<i4"), device=self.device)

    def device_lengths(self) -> torch.Tensor:
        _, _, _, _, dlen = self._views()
        return torch.as_tensor(_DeviceView(dlen, (len(self._batch),), "<i4"), device=self.device)

    # ------------------------------------------------------------ ops

    def update_kv_cache(self, k: torch.Tensor, v: torch.Tensor) -> None:
        """Append k, v [B, Hkv, S, D] at every batch sequence's length."""
        if k.shape != v.shape or k.dim() != 4 or k.shape[0] != len(self._batch) or k.shape[1] != self.num_kv_heads:
            raise CraneHipError(_lib.E_INVALID, "k, v must be [B, Hkv, S, D] matching the batch")
        if k.dtype != self.dtype or v.dtype != self.dtype:
            raise CraneHipError(_lib.E_DTYPE, f"k/v dtype {k.dtype} != cache dtype {self.dtype}")
        k, v = k.contiguous(), v.contiguous()
        check(_lib.lib().crane_pkv_update(self._h, k.data_ptr(), v.data_ptr(), k.shape[2], _stream(self.device)),
              "crane_pkv_update")

    def append_qkv(self, qkv: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor, positions: torch.Tensor,
                   num_heads: int, q_norm_w: Optional[torch.Tensor] = None, k_norm_w: Optional[torch.Tensor] = None,
                   eps: float = 1e-6, order: str = "norm_then_rope") -> torch.Tensor:
        """Fused QK-norm + RoPE written at the batch sequences' lengths; q [B, Hq, S, D]."""
        _check_append(qkv, cos, sin, positions, num_heads, self.num_kv_heads, q_norm_w, k_norm_w, order,
                      len(self._batch), self.dtype, self.device)
        B, S, _ = qkv.shape
        q_out = torch.empty((B, num_heads, S, HEAD_DIM), dtype=qkv.dtype, device=qkv.device)
        check(_lib.lib().crane_pkv_append_qkv(
            self._h, qkv.data_ptr(), qkv.stride(1), _ptr(q_norm_w), _ptr(k_norm_w), eps, _ORDERS[order],
            cos.data_ptr(), sin.data_ptr(), cos.stride(0), cos.shape[0], positions.data_ptr(), q_out.data_ptr(),
            S, num_heads, _stream(qkv.device)), "crane_pkv_append_qkv")
        return q_out

    def decode(self, q: torch.Tensor, scale: Optional[float] = None,
               workspace: Optional[torch.Tensor] = None, score_mode: Optional[str] = None) -> torch.Tensor:
        """Decode attention of q [B, Hq, D] over the batch's rows; [B, 1, Hq*D]
        (score_mode as in ops.attention_decode)."""
        from .ops import decode_workspace, score_mode_code
        _check_q(q, 3, len(self._batch), self.dtype, self.device)
        q = q.contiguous()
        B, Hq, D = q.shape
        need = _lib.lib().crane_hip_attn_decode_workspace(B, Hq, self.num_kv_heads, D, max(self.lengths),
                                                          _dtype_code(q))
        if workspace is not None:
            _dev(q, workspace)
        ws = workspace if workspace is not None else decode_workspace(q.device, need)
        out = torch.empty((B, 1, Hq * D), dtype=q.dtype, device=q.device)
        check(_lib.lib().crane_pkv_decode(self._h, q.data_ptr(), Hq, scale if scale else D ** -0.5,
                                          score_mode_code(score_mode, Hq // self.num_kv_heads), ws.data_ptr(),
                                          ws.numel() * ws.element_size(), out.data_ptr(), _stream(q.device)),
              "crane_pkv_decode")
        return out

    def prefill(self, q: torch.Tensor, scale: Optional[float] = None, causal: bool = True,
                long_rows_one_rounding: bool = False) -> torch.Tensor:
        """Attention of q [B, Hq, S, D] (the last S rows of every batch
        sequence) over its rows; [B, S, Hq*D].  long_rows_one_rounding as in
        ops.attention_prefill."""
        _check_q(q, 4, len(self._batch), self.dtype, self.device)
        B, Hq, S, D = q.shape
        out = torch.empty((B, S, Hq * D), dtype=q.dtype, device=q.device)
        check(_lib.lib().crane_pkv_prefill(self._h, q.contiguous().data_ptr(), Hq, S, scale if scale else D ** -0.5,
                                           _prefill_flags(causal, long_rows_one_rounding), out.data_ptr(),
                                           _stream(q.device)), "crane_pkv_prefill")
        return out

    def read_sequence(self, sid: int):
        """A sequence's rows as contiguous (k, v) [Hkv, len, D] (get_kv_caches)."""
        n = self.seq_len(sid)
        if n < 0:
            raise CraneHipError(_lib.E_INVALID, f"sequence {sid} is not live")
        k = torch.empty((self.num_kv_heads, n, HEAD_DIM), dtype=self.dtype, device=self.device)
        v = torch.empty_like(k)
        check(_lib.lib().crane_pkv_read_seq(self._h, sid, k.data_ptr() if n else None, v.data_ptr() if n else None,
                                            _stream(self.device)), "crane_pkv_read_seq")
        return k, v

    def write_sequence(self, sid: int, k: torch.Tensor, v: torch.Tensor) -> None:
        """Replace a sequence's rows by k, v [Hkv, len, D] (set_kv_caches)."""
        if k.shape != v.shape or k.dim() != 3 or k.shape[0] != self.num_kv_heads or k.shape[2] != HEAD_DIM:
            raise CraneHipError(_lib.E_INVALID, "k, v must be [Hkv, len, D]")
        if k.dtype != self.dtype or v.dtype != self.dtype:
            raise CraneHipError(_lib.E_DTYPE, f"k/v dtype {k.dtype} != cache dtype {self.dtype}")
        k, v = k.contiguous(), v.contiguous()
        n = k.shape[1]
        check(_lib.lib().crane_pkv_write_seq(self._h, sid, k.data_ptr() if n else None, v.data_ptr() if n else None,
                                             n, _stream(self.device)), "crane_pkv_write_seq")
