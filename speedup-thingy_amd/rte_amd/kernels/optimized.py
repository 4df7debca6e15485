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

# symbol -> implementation ("hip": librte_hip kernels, "torch": tensor ops on the device)
SYMBOLS: dict[str, str] = {
    "k_fused_rmsnorm": "hip",
    "k_rope_apply": "torch",
    "k_qkv_dense": "hip",
    "k_flash_causal_dense": "hip",
    "k_qkv_grouped": "torch",
    "k_flash_causal_grouped": "hip",
    "k_out_proj_grouped": "torch",
    "k_swiglu_dense": "hip",
    "k_swiglu_grouped": "torch",
    "k_pack_by_recipe": "torch",
    "k_unpack_from_recipe": "torch",
    "k_macro_phi": "torch",
    "k_recurrent_exact_loop": "python",
    "k_logits_full": "hip",
    "k_logits_shortlist": "hip",
    "k_cross_entropy_unreduced": "torch",
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

def k_fused_rmsnorm(x, weight, residual=None, eps: float = 1e-5):
    """(normed * weight, x + residual or None), normed in bf16 (rte/kernels/reference.py:9-17)."""
    _hip_inputs("k_fused_rmsnorm", x, weight, residual)
    y = x if residual is None else x + residual
    return hip_ops.rmsnorm(y, weight, eps), (y if residual is not None else None)


def k_qkv_dense(x, wq, wk, wv):
    """x @ wq, x @ wk, x @ wv with [in, out] weights (rte/kernels/reference.py:31-37)."""
    _hip_inputs("k_qkv_dense", x, wq, wk, wv)
    w = torch.cat([wq.t(), wk.t(), wv.t()], dim=0)  # nn.Linear layout [3*out, in]
    out = hip_ops.linear(x, w, out_f32=False)
    return out.split(wq.shape[1], dim=-1)


def k_swiglu_dense(x, wu, wg, wd):
    """(x @ wu) * silu(x @ wg) @ wd with [in, out] weights (rte/kernels/reference.py:62-68)."""
    _hip_inputs("k_swiglu_dense", x, wu, wg, wd)
    wug = torch.cat([wu.t(), wg.t()], dim=0)
    return hip_ops.dense_swiglu(x, wug, wd, None, wd_rows=True, out_f32=True)


def k_logits_full(hidden, vocab_weight):
    _hip_inputs("k_logits_full", hidden, vocab_weight)
    return hip_ops.linear(hidden, vocab_weight, out_f32=True)


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

def k_rope_apply(q, k, cos, sin):
    _require_cuda_tensor(q, k)

    def rotate_half(x):
        return torch.stack((-x[..., 1::2], x[..., ::2]), dim=-1).flatten(-2)

    while cos.ndim < q.ndim:
        cos, sin = cos.unsqueeze(0), sin.unsqueeze(0)
    return q * cos + rotate_half(q) * sin, k * cos + rotate_half(k) * sin


def k_qkv_grouped(x, wq, wk, wv, column_indices):
    _require_cuda_tensor(x)
    return x @ wq[:, column_indices], x @ wk[:, column_indices], x @ wv[:, column_indices]


def k_out_proj_grouped(x, wo, row_indices):
    _require_cuda_tensor(x)
    return x @ wo[row_indices, :]


def k_swiglu_grouped(x, wu, wg, wd, slab_indices):
    _require_cuda_tensor(x)
    return (x @ wu[:, slab_indices]) * F.silu(x @ wg[:, slab_indices]) @ wd[slab_indices, :]


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


def k_macro_phi(h, h0, d_gain, v, u, bias, eps: float = 1e-5):
    _require_cuda_tensor(h, h0)
    normed = h * torch.rsqrt(h.float().pow(2).mean(dim=-1, keepdim=True) + eps).to(h.dtype)
    pooled = normed.mean(dim=1, keepdim=True).expand_as(normed)
    low = F.silu(torch.cat([normed, pooled, h0], dim=-1) @ v) @ u
    return h + d_gain * h + low + bias


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


def k_cross_entropy_unreduced(logits, targets):
    return F.cross_entropy(logits.flatten(0, -2), targets.flatten(), reduction="none").view_as(targets)


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
