"""The reference's SVD sparse FFN device driver module (rte/kernels/svd_sparse_ffn_triton.py) on the
HIP kernels: triton_svd_sparse_ffn_forward keeps its name, arguments and validation; the
selector GEMMs, the per-token candidate union / activation / rerank and the sparse down-sum run
as the HIP SVD sparse FFN.  Module name kept for drop-in imports."""

from __future__ import annotations

import torch

from rte_amd import _lib
from rte_amd.kernels import hip_ops


def available() -> bool:
    return _lib.device_ready()


def _require_available() -> None:
    if not available():
        raise RuntimeError("SVD sparse FFN kernels require the ROCm HIP backend (the reference's CUDA + Triton path)")


def triton_svd_sparse_ffn_forward(x, w_up, w_gate, w_down, up_a, up_b, gate_a, gate_b, wd_norm, *, top_k: int,
                                  up_m: int, gate_m: int | None = None, product_m: int = 0, block_h: int = 1024,
                                  block_d: int = 64, low_launch: bool = False, selector_backend: str = "gemm",
                                  exact_candidate_activation: bool = True, candidate_strategy: str = "union"):
    """Inference forward of the SVD sparse FFN (rte/kernels/svd_sparse_ffn_triton.py:480-714).
    block_h, block_d, low_launch and selector_backend pick among the reference's Triton launch
    variants and are accepted for API parity (one HIP path serves them all)."""
    del block_h, block_d, low_launch
    _require_available()
    gate_m = up_m if gate_m is None else gate_m
    if gate_m != up_m:
        raise ValueError("Triton SVD sparse FFN currently requires gate_m == up_m")
    if product_m not in {0, up_m}:
        raise ValueError("Triton SVD sparse FFN currently requires product_m == 0 or product_m == up_m")
    if x.ndim != 2:
        raise ValueError("Triton SVD sparse FFN expects flattened x with shape [tokens, d_model]")
    if candidate_strategy not in {"union", "product"}:
        raise ValueError("candidate_strategy must be 'union' or 'product'")
    if selector_backend not in {"gemm", "triton"}:
        raise ValueError("selector_backend must be 'gemm' or 'triton'")
    if candidate_strategy == "product" and (selector_backend != "gemm" or exact_candidate_activation):
        raise ValueError("candidate_strategy='product' requires approximate GEMM selector mode")
    tensors = (x, w_up, w_gate, w_down, up_a, up_b, gate_a, gate_b, wd_norm)
    if any(not t.is_cuda for t in tensors):
        raise RuntimeError("SVD sparse FFN requires all tensors on the ROCm device")
    if torch.is_grad_enabled() and any(t.requires_grad for t in tensors):
        raise RuntimeError("Triton SVD sparse FFN is an inference/eval kernel; backward is not implemented")
    top_m = min(int(up_m), w_up.shape[0])
    if top_m <= 0:
        raise ValueError("Triton SVD sparse FFN requires up_m > 0")
    top_k = min(int(top_k), top_m * (2 + int(product_m > 0)))
    out, _, _ = hip_ops.svd_sparse_ffn(x, w_up, w_gate, w_down, up_a, up_b, gate_a, gate_b, up_m=top_m,
                                       gate_m=top_m, product_m=product_m, top_k=top_k,
                                       exact=exact_candidate_activation and candidate_strategy == "union",
                                       product_only=candidate_strategy == "product", wd_norm=wd_norm,
                                       out_dtype=x.dtype if x.dtype in (torch.float32, torch.bfloat16) else torch.float32)
    return out
