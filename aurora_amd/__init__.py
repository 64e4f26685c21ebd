"""aurora_amd — MI355X (gfx950) backend for Aurora's GEMM + causal-attention hot path.

The compute lives in libaurora_hip.so (hand-written HIP kernels behind a C ABI,
include/aurora_hip.h).  This package only binds it; importing the submodules
that issue GPU work raises if the library has not been built.
"""

__all__ = ["gpu", "build"]
