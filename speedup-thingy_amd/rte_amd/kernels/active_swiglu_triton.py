"""The reference's packed SwiGLU backend module (rte/kernels/active_swiglu_triton.py) on the HIP
kernels: triton_packed_swiglu_ffn keeps its name, shapes and validation; the activation runs in
the up/gate GEMM's epilogue and its derivative in the dZ GEMM's epilogue (no separate
activation launches).  Module name kept so that `from ...kernels.active_swiglu_triton import
triton_packed_swiglu_ffn` resolves unchanged."""

from __future__ import annotations

import torch

from rte_amd import _lib
from rte_amd.kernels import hip_ops


def available() -> bool:
    return _lib.device_ready()


def triton_packed_swiglu_ffn(x: torch.Tensor, wug: torch.Tensor, wdown_rows: torch.Tensor) -> torch.Tensor:
    """(up * silu(gate)) @ wdown_rows with [up ; gate] = x @ wug^T (rte/kernels/active_swiglu_triton.py:62-118).
    x [tokens, d], wug [2M, d], wdown_rows [M, d]; bf16 output as the reference under autocast."""
    if not available():
        raise RuntimeError("packed SwiGLU FFN requires the ROCm HIP backend (the reference's CUDA + Triton path)")
    if x.ndim != 2 or wug.ndim != 2 or wdown_rows.ndim != 2:
        raise ValueError("expected x [N,D], wug [2M,D], wdown_rows [M,D]")
    if wug.shape[0] % 2 != 0:
        raise ValueError("wug first dimension must be 2M")
    if wdown_rows.shape[0] != wug.shape[0] // 2:
        raise ValueError("wdown_rows first dimension must match M")
    from rte_amd.kernels.optimized import _mm_dtype

    _mm_dtype("triton_packed_swiglu_ffn", x, wug, wdown_rows)
    return hip_ops.dense_swiglu(x, wug, wdown_rows, None, wd_rows=True, out_f32=False)
