"""Kernel dispatch boundary: the k_* symbols of rte/kernels/optimized.py:58-154 with the
same names and argument meaning, bound to the gfx950 HIP library.

Symbols on the hot path run HIP kernels and never fall back: without the library or a
ROCm device they raise RuntimeError.  Symbols the reference also leaves as plain tensor
math (pack-by-recipe sort, macro Phi, audit sampling, metric reduction, grouped banked
slices) are torch ops on the caller's device; backend_status() lists which is which.
strict_cuda keeps the reference contract (rte/kernels/optimized.py:46-55): with it set,
every symbol refuses tensors that are not on the device, with "strict_cuda" in the message.
"""

from __future__ import annotations

import torch
import torch.nn.functional as F

from rte_amd import _lib
from rte_amd.kernels import hip_ops

STRICT_CUDA = False
REQUIRE_FLASH = True

# symbol -> implementation ("hip": librte_hip kernels, "torch": tensor ops on the device,
# "python": a host loop).  The torch / python ones are the symbols the reference's own optimized
# module also leaves as plain tensor code (stable sort by recipe key, its inverse, the seeded
# Bernoulli draw, the metric copy, the recurrent loop driver).
SYMBOLS: dict[str, str] = {
    "k_fused_rmsnorm": "hip",
    "k_rope_apply": "hip",
    "k_qkv_dense": "hip",
    "k_flash_causal_dense": "hip",
    "k_qkv_grouped": "hip",
    "k_flash_causal_grouped": "hip",
    "k_out_proj_grouped": "hip",
    "k_swiglu_dense": "hip",
    "k_swiglu_grouped": "hip",
    "k_pack_by_recipe": "torch",
    "k_unpack_from_recipe": "torch",
    "k_macro_phi": "hip",
    "k_recurrent_exact_loop": "python",
    "k_logits_full": "hip",
    "k_logits_shortlist": "hip",
    "k_cross_entropy_unreduced": "hip",
    "k_sample_audit_mask": "torch",
    "k_metrics_reduce": "torch",
}


def set_strict_cuda(enabled: bool, *, require_flash: bool = True) -> None:
    global STRICT_CUDA, REQUIRE_FLASH
    STRICT_CUDA = bool(enabled)
    REQUIRE_FLASH = bool(require_flash)


def hip_available() -> bool:
    return _lib.device_ready()


def triton_available() -> bool:
    """Kept for API compatibility: this build ships no Triton kernels."""
    return False


def backend_status() -> dict[str, object]:
    ready = hip_available()
    status: dict[str, object] = {
        "mode": "rocm_hip_dispatch" if ready else "hip_unavailable",
        "strict_cuda": STRICT_CUDA,
        "require_flash": REQUIRE_FLASH,
        "cuda_available": torch.cuda.is_available(),
        "triton_available": False,
        "hip_available": ready,
        "library": str(_lib.LIB_PATH),
        "library_built": _lib.LIB_PATH.exists(),
        # no symbol ever substitutes reference math for a HIP kernel; unavailable -> error
        "uses_reference_fallback": False,
        "symbols": dict(SYMBOLS),
        "torch_symbols": sorted(k for k, v in SYMBOLS.items() if v != "hip"),
    }
    if ready:
        try:
            status["device"] = _lib.device_info()
        except RuntimeError as exc:  # pragma: no cover
            status["device_error"] = str(exc)
    return status


def cuda_required() -> None:
    if not hip_available():
        raise RuntimeError("the ROCm HIP backend (librte_hip.so on a gfx950 device) is required for this kernel path")


def _require_cuda_tensor(*tensors) -> None:
    if STRICT_CUDA and any(isinstance(t, torch.Tensor) and not t.is_cuda for t in tensors):
        raise RuntimeError("strict_cuda requires ROCm device tensors in optimized hot-path kernels")
    if STRICT_CUDA and not hip_available():
        raise RuntimeError("strict_cuda requires the HIP kernels (librte_hip, gfx950); fallback is disabled")


def _hip_inputs(op: str, *tensors) -> None:
    _require_cuda_tensor(*tensors)
    _lib.require_device_tensors(op, *[t for t in tensors if isinstance(t, torch.Tensor)])


# ----------------------------------------------------------------------------- hot-path symbols (HIP)

def _mm_dtype(op: str, *tensors) -> torch.dtype:
    """The matmul symbols compute with bf16 operands and fp32 accumulation, which is what the
    reference computes under bf16 autocast (its training precision "bf16"); their result is
    bf16 as there.  Float32 operands outside a bf16 autocast region would ask for fp32 matmuls,
    which this build does not implement: refuse instead of returning bf16-accurate numbers.  Inside
    hip_ops.fp32_precision() (training.precision fp32) they compute with fp32 operands on the
    fp32 GEMM and return fp32."""
    if torch.is_autocast_enabled("cuda") and torch.get_autocast_dtype("cuda") == torch.bfloat16:
        return torch.bfloat16
    if hip_ops.fp32_active():
        return torch.float32
    floats = [t for t in tensors if isinstance(t, torch.Tensor) and t.is_floating_point()]
    if all(t.dtype == torch.bfloat16 for t in floats):
        return torch.bfloat16
    raise RuntimeError(f"{op}: the HIP matmul kernels take bf16 operands; call it under "
                       "torch.autocast('cuda', dtype=torch.bfloat16) or pass bfloat16 tensors "
                       "(fp32 matmuls are not implemented)")


def k_fused_rmsnorm(x, weight, residual=None, eps: float = 1e-5):
    """(y * rsqrt(mean(y^2) + eps) * weight, y or None) with y = x + residual
    (rte/kernels/reference.py:9-17), in the dtypes the reference returns: the normed output is
    promote(x.dtype, weight.dtype), y keeps x's dtype."""
    _hip_inputs("k_fused_rmsnorm", x, weight, residual)
    return hip_ops.fused_rmsnorm(x, weight, residual, eps)


def k_rope_apply(q, k, cos, sin):
    """Interleaved rotary embedding of q and k (rte/kernels/reference.py:20-28)."""
    _hip_inputs("k_rope_apply", q, k, cos, sin)
    return hip_ops.rope_apply(q, k, cos, sin)


def k_qkv_dense(x, wq, wk, wv):
    """x @ wq, x @ wk, x @ wv with [in, out] weights (rte/kernels/reference.py:31-37): one GEMM
    over the concatenated weights."""
    _hip_inputs("k_qkv_dense", x, wq, wk, wv)
    _mm_dtype("k_qkv_dense", x, wq, wk, wv)
    w = torch.cat([wq.t(), wk.t(), wv.t()], dim=0)  # nn.Linear layout [3*out, in]
    out = hip_ops.linear(x, w, out_f32=False)
    return out.split(wq.shape[1], dim=-1)


def k_qkv_grouped(x, wq, wk, wv, column_indices):
    """x @ w[:, columns] for w in (wq, wk, wv) (rte/kernels/reference.py:44-51): the selected
    columns of the three weights feed one GEMM."""
    _hip_inputs("k_qkv_grouped", x, wq, wk, wv, column_indices)
    _mm_dtype("k_qkv_grouped", x, wq, wk, wv)
    cols = column_indices.to(device=wq.device, dtype=torch.long)
    w = torch.cat([wq.index_select(1, cols), wk.index_select(1, cols), wv.index_select(1, cols)], dim=1).t()
    out = hip_ops.linear(x, w, out_f32=False)
    return out.split(cols.numel(), dim=-1)


def k_out_proj_grouped(x, wo, row_indices):
    """x @ wo[rows, :] (rte/kernels/reference.py:58-59): the GEMM reads wo's rows through the index
    table; the weight gradient of repeated rows adds up in a fixed order."""
    _hip_inputs("k_out_proj_grouped", x, wo, row_indices)
    _mm_dtype("k_out_proj_grouped", x, wo)
    return hip_ops.rows_linear(x, wo, row_indices, torch.bfloat16)


def k_swiglu_dense(x, wu, wg, wd):
    """(x @ wu) * silu(x @ wg) @ wd with [in, out] weights (rte/kernels/reference.py:62-68)."""
    _hip_inputs("k_swiglu_dense", x, wu, wg, wd)
    _mm_dtype("k_swiglu_dense", x, wu, wg, wd)
    wug = torch.cat([wu.t(), wg.t()], dim=0)
    return hip_ops.dense_swiglu(x, wug, wd, None, wd_rows=True, out_f32=False)


def k_swiglu_grouped(x, wu, wg, wd, slab_indices):
    """The SwiGLU of the selected slabs, (x @ wu[:, s]) * silu(x @ wg[:, s]) @ wd[s, :]
    (rte/kernels/reference.py:71-78), on the fused SwiGLU GEMMs."""
    _hip_inputs("k_swiglu_grouped", x, wu, wg, wd, slab_indices)
    _mm_dtype("k_swiglu_grouped", x, wu, wg, wd)
    sl = slab_indices.to(device=wu.device, dtype=torch.long)
    wug = torch.cat([wu.index_select(1, sl).t(), wg.index_select(1, sl).t()], dim=0)
    return hip_ops.dense_swiglu(x, wug, wd.index_select(0, sl), None, wd_rows=True, out_f32=False)


def k_macro_phi(h, h0, d_gain, v, u, bias, eps: float = 1e-5):
    """h + d_gain h + silu(z v) u + bias with z = [rmsnorm(h) | mean_s rmsnorm(h) | h0]
    (rte/kernels/reference.py:111-124).  v [3d, m] and u [m, d] shared by all samples, or per
    sample [B, 3d, m] / [B, m, d] (a grouped GEMM keyed by sample)."""
    _hip_inputs("k_macro_phi", h, h0, v, u)
    _mm_dtype("k_macro_phi", v, u)
    ones = torch.ones(h.shape[-1], device=h.device, dtype=h.dtype)
    normed, _ = hip_ops.fused_rmsnorm(h, ones, None, eps)
    pooled = normed.mean(dim=1, keepdim=True).expand_as(normed)
    z = torch.cat([normed, pooled, h0.to(normed.dtype)], dim=-1)
    B, S, _ = h.shape
    if v.ndim == 2:
        a = hip_ops.linear(z, v.t(), out_f32=False)
        low = hip_ops.linear(F.silu(a), u.t(), out_f32=True)
    else:
        keys = torch.arange(B, device=h.device, dtype=torch.int32).repeat_interleave(S)
        pk = hip_ops.group_rows(keys, B)
        a = hip_ops.grouped_linear(z, v, pk, out_f32=False)
        low = hip_ops.grouped_linear(F.silu(a), u, pk, out_f32=True)
    return h + d_gain * h + low.view_as(h).to(h.dtype) + bias


def k_logits_full(hidden, vocab_weight):
    """hidden @ vocab_weight^T (rte/kernels/reference.py:131-132), bf16 as under autocast."""
    _hip_inputs("k_logits_full", hidden, vocab_weight)
    _mm_dtype("k_logits_full", hidden, vocab_weight)
    return hip_ops.linear(hidden, vocab_weight, out_f32=False)


def k_cross_entropy_unreduced(logits, targets):
    """Per-token cross-entropy (rte/kernels/reference.py:146-147; ignore_index -100 rows give 0)
    on the fused CE kernels, fp32 as F.cross_entropy computes it."""
    _hip_inputs("k_cross_entropy_unreduced", logits, targets)
    return hip_ops.cross_entropy(logits, targets)

# ----------------------------------------------------------------------------- attention core (SDPA)

def _flash_attention(q, k, v):
    """Causal attention with the softmax scale 1/sqrt(head_dim) (the reference's
    F.scaled_dot_product_attention(q, k, v, is_causal=True)) on the HIP kernel; head_dim 32, 64 or 128."""
    _hip_inputs("k_flash_causal", q, k, v)
    return hip_ops.attention(q, k, v)


def k_flash_causal_dense(q, k, v):
    return _flash_attention(q, k, v)


def k_flash_causal_grouped(q, k, v):
    return _flash_attention(q, k, v)


# ----------------------------------------------------------------------------- glue symbols (torch)

class PackedByRecipe:
    __slots__ = ("packed", "permutation", "inverse_permutation", "keys", "offsets", "unique_keys")

    def __init__(self, packed, permutation, inverse_permutation, keys, offsets, unique_keys):
        self.packed = packed
        self.permutation = permutation
        self.inverse_permutation = inverse_permutation
        self.keys = keys
        self.offsets = offsets
        self.unique_keys = unique_keys


def k_pack_by_recipe(hidden, recipe_ids, depth_ids, audit_flags=None) -> PackedByRecipe:
    """Stable sort by recipe*1e6 + depth*10 + audit (rte/kernels/reference.py:91-104)."""
    audit = torch.zeros_like(recipe_ids) if audit_flags is None else audit_flags.long()
    keys = recipe_ids.long() * 1_000_000 + depth_ids.long() * 10 + audit
    sorted_keys, perm = torch.sort(keys, stable=True)
    inverse = torch.empty_like(perm)
    inverse[perm] = torch.arange(perm.numel(), device=perm.device)
    unique, counts = torch.unique_consecutive(sorted_keys, return_counts=True)
    offsets = torch.cat([counts.new_zeros(1), counts.cumsum(0)])
    return PackedByRecipe(hidden[perm], perm, inverse, sorted_keys, offsets, unique)


def k_unpack_from_recipe(packed, inverse_permutation):
    return packed[inverse_permutation]


def k_recurrent_exact_loop(step_fn, h, h0, depth: int, boundaries: set[int]):
    states: dict[int, torch.Tensor] = {}
    for t in range(depth):
        h = step_fn(h, h0)
        if t + 1 in boundaries:
            states[t + 1] = h
    return h, states


def k_logits_shortlist(hidden, vocab_weight, shortlist):
    """hidden . vocab_weight[shortlist] (rte/kernels/reference.py:141-143) on the shortlist kernel
    (fp32 logits from bf16 operands; the kernel's CE at position 0 is discarded here)."""
    _require_cuda_tensor(hidden, vocab_weight, shortlist)
    return hip_ops.shortlist_ce(hidden, vocab_weight, shortlist)[0]


def k_sample_audit_mask(p, seed: int):
    gen = torch.Generator(device=p.device)
    gen.manual_seed(seed)
    return torch.bernoulli(p, generator=gen).bool()


def k_metrics_reduce(values: dict[str, torch.Tensor]) -> dict[str, float]:
    """One device->host copy for the whole dict (the reference syncs once per key)."""
    if not values:
        return {}
    keys = list(values)
    stacked = torch.stack([values[k].detach().float().mean() for k in keys]).cpu().tolist()
    return dict(zip(keys, stacked))
