"""rte_amd — MI355X (gfx950) native implementation of the recursive_macro hot path of the
Recursive Training Engine.  Hot operators run on hand-written HIP kernels (librte_hip.so,
C ABI in include/rte_hip.h); PyTorch-ROCm provides device memory, streams, attention core
and the optimizer."""

from rte_amd.kernels.optimized import backend_status, hip_available, set_strict_cuda

__all__ = ["backend_status", "hip_available", "set_strict_cuda"]
