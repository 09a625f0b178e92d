"""rocmforge_amd -- MI355X (gfx950) Q4_K / Q6_K matmul hot path of ROCmForge.

The compute lives in librocmforge_cdna4.so (HIP kernels behind the C ABI of
include/rocmforge_cdna4.h).  `ops` exposes the library's host routing
under the names of the reference's src/gpu/ops.rs dispatch functions.
"""
from ._lib import LIB_PATH, LibraryMissing, load  # noqa: F401

__all__ = ["LIB_PATH", "LibraryMissing", "load"]
