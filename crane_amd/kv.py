"""Python surface of the host-side KV-cache manager (include/crane_kv.h).

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
from .ops import HEAD_DIM, _ORDERS, _dtype_code, _ptr, _stream

_DT = {torch.float32: _lib.F32, torch.bfloat16: _lib.BF16}


def grown_capacity(cap: int, needed: int) -> int:
    """Rows a cache of `cap` rows holds after making room for `needed` rows
    (Crane's policy: unchanged if it fits, else needed + 256)."""
    return int(_lib.lib().crane_kv_grown_capacity(cap, needed))


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

    def close(self) -> None:
        if getattr(self, "_h", None):
            _lib.lib().crane_kv_destroy(self._h)
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
        if qkv.dim() != 3 or qkv.shape[0] != self.batch:
            raise CraneHipError(_lib.E_INVALID, "qkv must be [B, S, (Hq+2Hkv)*D]")
        if qkv.dtype != self.dtype:
            raise CraneHipError(_lib.E_DTYPE, f"qkv dtype {qkv.dtype} != cache dtype {self.dtype}")
        if order not in _ORDERS:
            raise CraneHipError(_lib.E_INVALID, f"order {order!r}")
        B, S, _ = qkv.shape
        q_out = torch.empty((B, num_heads, S, HEAD_DIM), dtype=qkv.dtype, device=qkv.device)
        check(_lib.lib().crane_kv_append_qkv(
            self._h, qkv.data_ptr(), qkv.stride(1), _ptr(q_norm_w), _ptr(k_norm_w), eps, _ORDERS[order],
            cos.data_ptr(), sin.data_ptr(), cos.stride(0), cos.shape[0], positions.data_ptr(), q_out.data_ptr(),
            S, num_heads, _stream(qkv.device)), "crane_kv_append_qkv")
        return q_out

    def decode(self, q: torch.Tensor, scale: Optional[float] = None,
               workspace: Optional[torch.Tensor] = None) -> torch.Tensor:
        """Decode attention of q [B, Hq, D] over every sequence's rows; [B, 1, Hq*D]."""
        from .ops import decode_workspace
        B, Hq, D = q.shape
        max_kv = max(self.lengths)
        need = _lib.lib().crane_hip_attn_decode_workspace(B, Hq, self.num_kv_heads, D, max_kv, _dtype_code(q))
        ws = workspace if workspace is not None else decode_workspace(q.device, need)
        out = torch.empty((B, 1, Hq * D), dtype=q.dtype, device=q.device)
        check(_lib.lib().crane_kv_decode(self._h, q.data_ptr(), Hq, scale if scale else D ** -0.5, ws.data_ptr(),
                                         ws.numel() * ws.element_size(), out.data_ptr(), _stream(q.device)),
              "crane_kv_decode")
        return out

    def prefill(self, q: torch.Tensor, scale: Optional[float] = None, causal: bool = True) -> torch.Tensor:
        """Attention of q [B, Hq, S, D] (the last S rows of every sequence) over
        the cache; [B, S, Hq*D]."""
        B, Hq, S, D = q.shape
        out = torch.empty((B, S, Hq * D), dtype=q.dtype, device=q.device)
        check(_lib.lib().crane_kv_prefill(self._h, q.contiguous().data_ptr(), Hq, S, scale if scale else D ** -0.5,
                                          int(causal), out.data_ptr(), _stream(q.device)), "crane_kv_prefill")
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
