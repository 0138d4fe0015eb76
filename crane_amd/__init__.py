"""crane_amd -- MI355X (gfx950) attention hot path for Crane-style models.

The compute lives in libcrane_hip.so (hand-written HIP kernels behind the C
ABI of include/crane_hip.h); `crane_amd.ops` is the Tensor-in/Tensor-out host
surface over it and `crane_amd.attention` the model-level layer (KV cache,
prefill/decode dispatch) that stands in for Crane's Attention::forward.
"""
from ._lib import CraneHipError, LIB_PATH, version  # noqa: F401

__all__ = ["CraneHipError", "LIB_PATH", "version"]
