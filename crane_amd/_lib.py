"""ctypes binding of libcrane_hip.so, the C ABI declared in include/crane_hip.h
(attention launchers, dense and paged), include/crane_layer.h (the decoder
layer's row kernels), include/crane_gemm.h (the QKV / o_proj projections), include/crane_sampling.h
(argmax, top-k), include/crane_kv.h (host-side KV-cache manager) and
include/crane_pkv.h (paged KV-cache manager).

The library is the only compute path: there is no CPU fallback.  Loading
fails loudly when the built library is missing.
"""
from __future__ import annotations

import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libcrane_hip.so")

F32, BF16 = 0, 1
NORM_THEN_ROPE, ROPE_THEN_NORM, ROPE_ONLY = 0, 1, 2
SCORE_GROUPED, SCORE_STANDARD = 0, 1

OK = 0
E_INVALID, E_DTYPE, E_HEAD_DIM, E_GQA, E_CAPACITY, E_WORKSPACE, E_LAUNCH, E_ALIGN = range(1, 9)

# Every symbol include/*.h declares, with its ctypes signature.
_vp, _i32p, _i64, _i, _f, _sz = (ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64, ctypes.c_int,
                                 ctypes.c_float, ctypes.c_size_t)
_vpp, _i64p, _u64 = ctypes.POINTER(ctypes.c_void_p), ctypes.POINTER(ctypes.c_int64), ctypes.c_uint64
_ip = ctypes.POINTER(ctypes.c_int)
SIGNATURES = {
    "crane_hip_strerror": ([_i], ctypes.c_char_p),
    "crane_hip_version": ([], ctypes.c_char_p),
    "crane_hip_qknorm_rope_append": (
        [_vp, _i64, _vp, _vp, _f, _i, _vp, _vp, _i64, _i64, _i32p, _vp, _vp, _vp, _i64, _i32p, _i64,
         _i, _i, _i, _i, _i, _i, _vp], _i),
    "crane_hip_qknorm_rope_append_parts": (
        [_vp, _i, _vp, _vp, _vp, _f, _i, _vp, _vp, _i64, _i64, _i32p, _vp, _vp, _vp, _i64, _i32p, _i64,
         _i, _i, _i, _i, _i, _i, _vp], _i),
    "crane_hip_qnorm_rope": (
        [_vp, _i64, _vp, _f, _i, _vp, _vp, _i64, _i64, _i32p, _vp, _i, _i, _i, _i, _i, _vp], _i),
    "crane_hip_rope_tables": ([_i, ctypes.c_double, ctypes.c_double, _i64, _i, _vp, _vp], _i),
    "crane_hip_rope_tables_qwen2": ([_i, ctypes.c_double, _i64, _i, _vp, _vp], _i),
    "crane_hip_attn_decode_workspace": ([_i, _i, _i, _i, _i64, _i], _sz),
    "crane_hip_attn_decode": (
        [_vp, _vp, _vp, _i64, _i32p, _i64, _i, _i, _i, _i, _f, _i, _vp, _sz, _vp, _i, _vp], _i),
    "crane_hip_attn_decode_noalloc": (
        [_vp, _vp, _vp, _i64, _i32p, _i64, _i, _i, _i, _i, _f, _i, _vp, _i, _vp], _i),
    "crane_hip_attn_decode_noalloc_limit": ([], _sz),
    "crane_hip_attn_prefill": (
        [_vp, _vp, _vp, _i64, _i32p, _i64, _i, _i, _i, _i, _i, _f, _i, _vp, _i, _vp], _i),
    # include/crane_kv.h
    "crane_kv_grown_capacity": ([_i64, _i64], _i64),
    "crane_kv_create": ([_i, _i, _i, _i, _vpp], _i),
    "crane_kv_destroy": ([_vp], None),
    "crane_kv_reserve": ([_vp, _i64, _vp], _i),
    "crane_kv_update": ([_vp, _vp, _vp, _i, _vp], _i),
    "crane_kv_append_qkv": (
        [_vp, _vp, _i64, _vp, _vp, _f, _i, _vp, _vp, _i64, _i64, _i32p, _vp, _i, _i, _vp], _i),
    "crane_kv_decode": ([_vp, _vp, _i, _f, _i, _vp, _sz, _vp, _vp], _i),
    "crane_kv_prefill": ([_vp, _vp, _i, _i, _f, _i, _vp, _vp], _i),
    "crane_kv_views": ([_vp, _vpp, _vpp, _i64p, _vpp, _i64p], _i),
    "crane_kv_set_lengths": ([_vp, _i64p, _vp], _i),
    "crane_kv_bytes": ([_vp], _u64),
    "crane_kv_stack": ([_vp, _vpp, _i, _i64, _vp], _i),
    "crane_kv_extract": ([_vp, _i, _vp, _vp], _i),
    # include/crane_hip.h, paged layout
    "crane_hip_qknorm_rope_append_paged": (
        [_vp, _i64, _vp, _vp, _f, _i, _vp, _vp, _i64, _i64, _i32p, _vp, _vp, _vp, _i64, _i, _i32p, _i64, _i32p,
         _i, _i, _i, _i, _i, _i, _vp], _i),
    "crane_hip_attn_decode_paged": (
        [_vp, _vp, _vp, _i64, _i, _i32p, _i64, _i32p, _i64, _i, _i, _i, _i, _f, _i, _vp, _sz, _vp, _i, _vp], _i),
    "crane_hip_attn_prefill_paged": (
        [_vp, _vp, _vp, _i64, _i, _i32p, _i64, _i32p, _i64, _i, _i, _i, _i, _i, _f, _i, _vp, _i, _vp], _i),
    # include/crane_layer.h
    "crane_hip_rms_norm": ([_vp, _vp, _vp, _i64, _i, _f, _i, _vp], _i),
    "crane_hip_add_rms_norm": ([_vp, _vp, _vp, _vp, _i64, _i, _f, _i, _vp], _i),
    "crane_hip_add_rms_norm_parts": ([_vp, _vp, _i, _vp, _vp, _i64, _i, _f, _i, _vp], _i),
    "crane_hip_silu_mul": ([_vp, _vp, _i64, _i, _i, _vp], _i),
    "crane_hip_residual_add": ([_vp, _vp, _i64, _i, _vp], _i),
    # include/crane_sampling.h
    "crane_hip_argmax": ([_vp, _i64, _i64, _i, _vp, _vp], _i),
    "crane_hip_topk": ([_vp, _i64, _i64, _i, _vp, _vp], _i),
    "crane_hip_select_workspace_bytes": ([_i64, _i64], _sz),
    "crane_hip_argmax_ws": ([_vp, _i64, _i64, _i, _vp, _sz, _vp, _vp], _i),
    "crane_hip_topk_ws": ([_vp, _i64, _i64, _i, _vp, _sz, _vp, _vp], _i),
    # include/crane_gemm.h
    "crane_gemm_create": ([_sz, _vpp], _i),
    "crane_gemm_destroy": ([_vp], None),
    "crane_gemm_linear": ([_vp, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i, _vp], _i),
    "crane_gemm_silu_mul_supported": ([_i64, _i64, _i64, _i], _i),
    "crane_gemm_linear_silu_mul": ([_vp, _vp, _vp, _vp, _i64, _i64, _i64, _i, _vp], _i),
    "crane_gemm_split_supported": ([_i64, _i64, _i64, _i, _i], _i),
    "crane_gemm_linear_split": ([_vp, _vp, _vp, _vp, _i64, _i64, _i64, _i, _i, _vp], _i),
    # include/crane_pkv.h
    "crane_pkv_create": ([_i, _i, _i, _i, _i64, _i, _i, _vpp], _i),
    "crane_pkv_destroy": ([_vp], None),
    "crane_pkv_seq_add": ([_vp, _ip], _i),
    "crane_pkv_seq_free": ([_vp, _i], _i),
    "crane_pkv_seq_len": ([_vp, _i], _i64),
    "crane_pkv_free_pages": ([_vp], _i64),
    "crane_pkv_bytes": ([_vp], _u64),
    "crane_pkv_set_batch": ([_vp, _ip, _i, _vp], _i),
    "crane_pkv_update": ([_vp, _vp, _vp, _i, _vp], _i),
    "crane_pkv_append_qkv": (
        [_vp, _vp, _i64, _vp, _vp, _f, _i, _vp, _vp, _i64, _i64, _i32p, _vp, _i, _i, _vp], _i),
    "crane_pkv_decode": ([_vp, _vp, _i, _f, _i, _vp, _sz, _vp, _vp], _i),
    "crane_pkv_prefill": ([_vp, _vp, _i, _i, _f, _i, _vp, _vp], _i),
    "crane_pkv_read_seq": ([_vp, _i, _vp, _vp, _vp], _i),
    "crane_pkv_write_seq": ([_vp, _i, _vp, _vp, _i64, _vp], _i),
    "crane_pkv_views": ([_vp, _vpp, _vpp, _vpp, _i64p, _vpp], _i),
}


class CraneHipError(RuntimeError):
    """A nonzero crane_hip status (the analogue of candle's `bail!`)."""

    def __init__(self, code: int, what: str):
        self.code = code
        super().__init__(f"{what}: {strerror(code)} (code {code})")


_lib = None


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(
                f"{LIB_PATH} is not built; run `python -m crane_amd.build` (hipcc, gfx950). "
                "crane_amd has no CPU fallback.")
        # One HIP runtime per process: torch carries its own libamdhip64 and
        # libhipblaslt (soname libamdhip64.so.7).  Loaded first, they satisfy
        # this library's dependencies; loaded after it, they come in beside
        # the /opt/rocm copies its runpath names, and torch's streams and
        # memory then belong to another runtime than its kernels (launch
        # failures, then crashes).
        import torch  # noqa: F401
        L = ctypes.CDLL(LIB_PATH)
        for name, (args, res) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.argtypes = args
            fn.restype = res
        _lib = L
    return _lib


def strerror(code: int) -> str:
    return lib().crane_hip_strerror(code).decode()


def check(code: int, what: str) -> None:
    if code != OK:
        raise CraneHipError(code, what)


def version() -> str:
    return lib().crane_hip_version().decode()
