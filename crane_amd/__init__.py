"""crane_amd -- MI355X (gfx950) attention hot path for Crane-style models.

The compute lives in libcrane_hip.so (hand-written HIP kernels behind the C
ABI of include/*.h).  `crane_amd.ops` is the Tensor-in/Tensor-out host surface
over it; `crane_amd.kv` holds the per-layer KV caches (dense and paged) that
stand in for Attention.kv_cache; `crane_amd.decoder` composes one decoder
layer from the kernels; `crane_amd.model` runs the L-layer stack (prefill
chunks, batched decode steps, and a HIP-graph replay of the decode step).
"""
from ._lib import CraneHipError, LIB_PATH, version  # noqa: F401

__all__ = ["CraneHipError", "LIB_PATH", "version"]
