"""manta_amd: MI355X (gfx950) backend for Manta's retrieval hot path.

Packed q8/q4 candidate scoring (dot / cosine / l2_distance), top-k selection
and the embed pipeline (gather -> @matmul -> masked mean_pool -> normalize),
as hand-written HIP kernels behind the C ABI of include/manta_rocm.h.
"""
from ._lib import MantaRocmError, Unsupported, load  # noqa: F401

__all__ = ["MantaRocmError", "Unsupported", "load"]
