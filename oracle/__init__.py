"""numpy front end of the CPU oracle (oracle.c).

TEST INFRASTRUCTURE ONLY: tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg import this module as the checker.  The product path
(crane_amd) never imports it and has no CPU fallback.

Arrays cross as float32; with dtype="bf16" the values are bf16-representable
floats and every candle op output is rounded to bf16 (see oracle.h).
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")
_lib = None

F32, BF16 = 0, 1
NORM_THEN_ROPE, ROPE_THEN_NORM, ROPE_ONLY = 0, 1, 2
DECODE_GROUPED, DECODE_STANDARD = 0, 1
MASK_NEG_1E9, MASK_NEG_INF = 0, 1

_fp = ctypes.POINTER(ctypes.c_float)
_ip = ctypes.POINTER(ctypes.c_int32)


def build(force: bool = False) -> str:
    """Compile oracle.c with make (gcc).  Returns the library path."""
    if force or not os.path.exists(_LIB_PATH):
        subprocess.run(["make", "-C", _HERE, "-B" if force else "all"], check=True,
                       stdout=subprocess.DEVNULL)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        L.orc_round_bf16.argtypes = [_fp, ctypes.c_size_t]
        L.orc_gen_normal.argtypes = [ctypes.c_uint64, ctypes.c_size_t, ctypes.c_double,
                                     ctypes.c_double, _fp]
        L.orc_gen_uniform_int.argtypes = [ctypes.c_uint64, ctypes.c_size_t, ctypes.c_int,
                                          ctypes.c_int, _ip]
        L.orc_rope_tables.argtypes = [ctypes.c_int, ctypes.c_double, ctypes.c_double,
                                      ctypes.c_int, _fp, _fp]
        L.orc_rope_tables_qwen2.argtypes = [ctypes.c_int, ctypes.c_double, ctypes.c_int,
                                            ctypes.c_int, _fp, _fp]
        L.orc_rms_norm.argtypes = [_fp, _fp, ctypes.c_size_t, ctypes.c_int, _fp,
                                   ctypes.c_float, ctypes.c_int, ctypes.c_int]
        L.orc_silu_mul.argtypes = [_fp, _fp, ctypes.c_size_t, ctypes.c_int, ctypes.c_int, ctypes.c_int]
        L.orc_residual_add.argtypes = [_fp, _fp, ctypes.c_size_t, ctypes.c_int]
        _up = ctypes.POINTER(ctypes.c_uint32)
        L.orc_argmax.argtypes = [_fp, ctypes.c_size_t, ctypes.c_size_t, _up]
        L.orc_topk.argtypes = [_fp, ctypes.c_size_t, ctypes.c_size_t, ctypes.c_int, _up]
        L.orc_linear.argtypes = [_fp, _fp, _fp, _fp, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                 ctypes.c_int]
        L.orc_rope.argtypes = [_fp, _fp, ctypes.c_size_t, ctypes.c_int, _fp, _fp, _ip,
                               ctypes.c_int]
        L.orc_qk_norm_rope_append.argtypes = [
            _fp, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
            _fp, _fp, ctypes.c_float, ctypes.c_int, _fp, _fp, _ip, _fp, _fp, _fp,
            ctypes.c_int, _ip, ctypes.c_int]
        L.orc_qk_norm_rope_append.restype = ctypes.c_int
        L.orc_attn_decode.argtypes = [_fp, _fp, _fp, ctypes.c_int, _ip, ctypes.c_int,
                                      ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_float,
                                      _fp, ctypes.c_int, ctypes.c_int, ctypes.c_int]
        L.orc_attn_decode_padded.argtypes = [_fp, _fp, _fp, ctypes.c_int, _ip, ctypes.c_int,
                                             ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                             ctypes.c_float, _fp, ctypes.c_int, ctypes.c_int]
        L.orc_attn_prefill.argtypes = [_fp, _fp, _fp, ctypes.c_int, _ip, ctypes.c_int,
                                       ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                       ctypes.c_float, ctypes.c_int, _fp, ctypes.c_int,
                                       ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_int,
                                       ctypes.c_int, ctypes.c_int]
        _lib = L
    return _lib


def _f(a):
    assert a.dtype == np.float32 and a.flags.c_contiguous
    return a.ctypes.data_as(_fp)


def _i(a):
    assert a.dtype == np.int32 and a.flags.c_contiguous
    return a.ctypes.data_as(_ip)


def _dt(dtype) -> int:
    return {"f32": F32, "bf16": BF16, F32: F32, BF16: BF16}[dtype]


def round_bf16(x: np.ndarray) -> np.ndarray:
    y = np.ascontiguousarray(x, dtype=np.float32).copy()
    lib().orc_round_bf16(_f(y), y.size)
    return y


def gen_normal(seed: int, shape, mean: float = 0.0, std: float = 1.0) -> np.ndarray:
    out = np.empty(int(np.prod(shape)), dtype=np.float32)
    lib().orc_gen_normal(seed & 0xFFFFFFFFFFFFFFFF, out.size, mean, std, _f(out))
    return out.reshape(shape)


def gen_uniform_int(seed: int, n: int, lo: int, hi: int) -> np.ndarray:
    out = np.empty(n, dtype=np.int32)
    lib().orc_gen_uniform_int(seed & 0xFFFFFFFFFFFFFFFF, n, lo, hi, _i(out))
    return out


def rope_tables(dim: int, theta: float, max_pos: int, alpha: float = 0.0):
    c = np.empty((max_pos, dim // 2), dtype=np.float32)
    s = np.empty_like(c)
    lib().orc_rope_tables(dim, theta, alpha, max_pos, _f(c), _f(s))
    return c, s


def rope_tables_qwen2(dim: int, theta: float, max_pos: int, dtype="f32"):
    c = np.empty((max_pos, dim // 2), dtype=np.float32)
    s = np.empty_like(c)
    lib().orc_rope_tables_qwen2(dim, theta, max_pos, _dt(dtype), _f(c), _f(s))
    return c, s


def rms_norm(x: np.ndarray, w=None, eps: float = 1e-6, contiguous: bool = True, dtype="f32"):
    x = np.ascontiguousarray(x, dtype=np.float32)
    d = x.shape[-1]
    y = np.empty_like(x)
    wp = _f(np.ascontiguousarray(w, dtype=np.float32)) if w is not None else None
    lib().orc_rms_norm(_f(x), _f(y), x.size // d, d, wp, eps, int(contiguous), _dt(dtype))
    return y


def silu_mul(gate_up: np.ndarray, f64: bool = False, dtype="f32"):
    """Crane's fused SiLU(gate) * up over gate_up [..., 2*inter] (gate || up):
    the f32 formula of its CUDA kernel, or (f64=True) its f64 cpu_fwd."""
    gu = np.ascontiguousarray(gate_up, dtype=np.float32)
    inter = gu.shape[-1] // 2
    out = np.empty(gu.shape[:-1] + (inter,), dtype=np.float32)
    lib().orc_silu_mul(_f(gu), _f(out), gu.size // (2 * inter), inter, int(f64), _dt(dtype))
    return out


def residual_add(residual: np.ndarray, hidden: np.ndarray, dtype="f32"):
    """candle's `residual + hidden` in T (a new array)."""
    r = np.ascontiguousarray(residual, dtype=np.float32).copy()
    h = np.ascontiguousarray(hidden, dtype=np.float32)
    assert r.shape == h.shape
    lib().orc_residual_add(_f(r), _f(h), r.size, _dt(dtype))
    return r


def linear(x: np.ndarray, w: np.ndarray, bias=None, dtype="f32", fused: bool = False):
    """candle Linear: x [..., K] times w [N, K]^T (+ bias [N]) -> [..., N];
    fused=True rounds product + bias once (a GEMM epilogue)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    w = np.ascontiguousarray(w, dtype=np.float32)
    N, K = w.shape
    assert x.shape[-1] == K
    M = x.size // K
    y = np.empty(x.shape[:-1] + (N,), dtype=np.float32)
    bp = _f(np.ascontiguousarray(bias, dtype=np.float32)) if bias is not None else None
    lib().orc_linear(_f(x), _f(w), bp, _f(y), M, N, K, int(fused), _dt(dtype))
    return y


def argmax(x: np.ndarray) -> np.ndarray:
    """First maximum of every row of x [..., n] (NaN lowest, -0 == +0)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    n = x.shape[-1]
    out = np.empty(x.size // n, dtype=np.uint32)
    lib().orc_argmax(_f(x), out.size, n, out.ctypes.data_as(ctypes.POINTER(ctypes.c_uint32)))
    return out.reshape(x.shape[:-1])


def topk(x: np.ndarray, k: int) -> np.ndarray:
    """Indices of the k largest of every row (value descending, index ascending)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    n = x.shape[-1]
    rows = x.size // n
    out = np.empty((rows, k), dtype=np.uint32)
    lib().orc_topk(_f(x), rows, n, k, out.ctypes.data_as(ctypes.POINTER(ctypes.c_uint32)))
    return out.reshape(x.shape[:-1] + (k,))


def add_rms_norm(residual, hidden, w=None, eps: float = 1e-6, dtype="f32"):
    """The candle pair Crane's FusedAddRmsNorm runs: (new residual, RmsNorm of it)."""
    r = residual_add(residual, hidden, dtype)
    return r, rms_norm(r, w, eps, True, dtype)


def rope(x: np.ndarray, cos: np.ndarray, sin: np.ndarray, pos: np.ndarray, dtype="f32"):
    x = np.ascontiguousarray(x, dtype=np.float32)
    d = x.shape[-1]
    y = np.empty_like(x)
    pos = np.ascontiguousarray(pos, dtype=np.int32)
    assert pos.size == x.size // d
    lib().orc_rope(_f(x), _f(y), x.size // d, d, _f(np.ascontiguousarray(cos, np.float32)),
                   _f(np.ascontiguousarray(sin, np.float32)), _i(pos), _dt(dtype))
    return y


def qk_norm_rope_append(qkv, Hq, Hkv, cos, sin, positions, k_cache, v_cache, cache_len,
                        q_w=None, k_w=None, eps=1e-6, order=NORM_THEN_ROPE, dtype="f32"):
    """qkv [B,S,(Hq+2Hkv)*D]; returns q_out [B,Hq,S,D]; caches updated in place."""
    qkv = np.ascontiguousarray(qkv, dtype=np.float32)
    B, S, W = qkv.shape
    D = W // (Hq + 2 * Hkv)
    cap = k_cache.shape[2]
    q_out = np.zeros((B, Hq, S, D), dtype=np.float32)
    qw = _f(np.ascontiguousarray(q_w, np.float32)) if q_w is not None else None
    kw = _f(np.ascontiguousarray(k_w, np.float32)) if k_w is not None else None
    rc = lib().orc_qk_norm_rope_append(
        _f(qkv), B, S, Hq, Hkv, D, qw, kw, eps, order,
        _f(np.ascontiguousarray(cos, np.float32)), _f(np.ascontiguousarray(sin, np.float32)),
        _i(np.ascontiguousarray(positions, np.int32)), _f(q_out), _f(k_cache), _f(v_cache),
        cap, _i(np.ascontiguousarray(cache_len, np.int32)), _dt(dtype))
    if rc != 0:
        raise ValueError("orc_qk_norm_rope_append: cache capacity exceeded")
    return q_out


def attn_decode(q, k_cache, v_cache, kv_len, scale, dtype="f32", variant=DECODE_GROUPED,
                nthreads=0):
    """q [B,Hq,D]; caches [B,Hkv,cap,D]; returns [B,Hq*D]."""
    q = np.ascontiguousarray(q, dtype=np.float32)
    B, Hq, D = q.shape
    _, Hkv, cap, _ = k_cache.shape
    out = np.empty((B, Hq * D), dtype=np.float32)
    lib().orc_attn_decode(_f(q), _f(k_cache), _f(v_cache), cap,
                          _i(np.ascontiguousarray(kv_len, np.int32)), B, Hq, Hkv, D, scale,
                          _f(out), _dt(dtype), variant, nthreads)
    return out


def attn_decode_padded(q, k_cache, v_cache, kv_len, scale, dtype="f32", nthreads=0):
    q = np.ascontiguousarray(q, dtype=np.float32)
    B, Hq, D = q.shape
    _, Hkv, cap, _ = k_cache.shape
    out = np.empty((B, Hq * D), dtype=np.float32)
    lib().orc_attn_decode_padded(_f(q), _f(k_cache), _f(v_cache), cap,
                                 _i(np.ascontiguousarray(kv_len, np.int32)), B, Hq, Hkv, D,
                                 scale, _f(out), _dt(dtype), nthreads)
    return out


def attn_prefill(q, k_cache, v_cache, start, scale, causal=True, dtype="bf16",
                 mask_kind=MASK_NEG_1E9, rows=None, heads=None, nthreads=0, out=None):
    """q [B,Hq,S,D]; caches [B,Hkv,cap,D]; returns out [B,S,Hq*D] (rows/heads
    outside the requested ranges are left as they were in `out`, zeros by default)."""
    q = np.ascontiguousarray(q, dtype=np.float32)
    B, Hq, S, D = q.shape
    _, Hkv, cap, _ = k_cache.shape
    if out is None:
        out = np.zeros((B, S, Hq * D), dtype=np.float32)
    r0, r1 = rows if rows is not None else (0, S)
    h0, h1 = heads if heads is not None else (0, Hq)
    lib().orc_attn_prefill(_f(q), _f(k_cache), _f(v_cache), cap,
                           _i(np.ascontiguousarray(start, np.int32)), B, S, Hq, Hkv, D, scale,
                           int(causal), _f(out), _dt(dtype), mask_kind, r0, r1, h0, h1, nthreads)
    return out
