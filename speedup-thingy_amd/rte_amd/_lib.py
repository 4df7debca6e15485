"""ctypes binding of librte_hip.so (declarations: include/rte_hip.h).

The library is built in-tree by ``speedup-thingy_amd/build.py`` and loaded from
this directory only.  There is no fallback: if the library or a ROCm device is
missing, ``lib()`` raises and every operator that needs it fails loudly.
"""

from __future__ import annotations

import ctypes
import os
from pathlib import Path

import torch

LIB_PATH = Path(__file__).resolve().parent / "librte_hip.so"

_P = ctypes.c_void_p
_I = ctypes.c_int
_I64 = ctypes.c_int64
_F = ctypes.c_float
_SZ = ctypes.c_size_t

# name -> (restype, argtypes); mirrors include/rte_hip.h one to one.
SIGNATURES: dict[str, tuple[object, list[object]]] = {
    "rte_abi_version": (_I, []),
    "rte_last_error": (ctypes.c_char_p, []),
    "rte_device_info": (_I, [ctypes.c_char_p, _I]),
    "rte_gemm_bf16": (
        _I, [_P, _I64, _I, _P, _P, _I64, _I, _P, _P, _I64, _I, _I, _I, _I, _F, _F, _P, _I64, _P, _SZ, _P]
    ),
    "rte_gemm_workspace_bytes": (_SZ, [_I, _I, _I]),
    "rte_gemm_bf16_split": (_I, [_P, _P, _I, _P, _P, _I, _P, _I64, _I, _I, _I, _I, _F, _F, _P, _I64, _P, _SZ, _P]),
    "rte_route_topk": (_I, [_P, _I, _I, _I, _P, _P, _P]),
    "rte_route_pack_workspace_bytes": (_SZ, [_I, _I]),
    "rte_route_pack": (_I, [_P, _I, _I, _P, _I, _I, _P, _P, _P, _P, _P, _P, _P, _P, _P, _SZ, _P]),
    "rte_pack_workspace_bytes": (_SZ, [_I, _I]),
    "rte_pack_index": (_I, [_P, _I, _I, _I, _P, _P, _P, _P, _P, _P, _P, _P, _SZ, _P]),
    "rte_pack_index_noalloc_max_bytes": (_SZ, []),
    "rte_pack_index_noalloc": (_I, [_P, _I, _I, _I, _P, _P, _P, _P, _P, _P, _P, _P]),
    "rte_combine_rows": (_I, [_P, _I, _I, _I, _P, _P, _P, _P, _I, _P]),
    "rte_route_bwd": (_I, [_P, _P, _P, _P, _I, _I, _I, _P, _P, _P]),
    "rte_grouped_swiglu_fwd": (
        _I,
        [_P, _I, _I, _P, _I, _I, _I, _P, _P, _P, _P, _P, _I64, _P, _P, _P, _P],
    ),
    "rte_grouped_swiglu_bwd": (
        _I,
        [_P, _P, _I, _I, _P, _I, _I, _I, _P, _P, _P, _P, _P, _I64, _P, _P, _P, _P, _P, _P, _P, _I, _F, _P, _SZ,
         _P],
    ),
    "rte_grouped_swiglu_bwd_workspace_bytes": (_SZ, [_I, _I, _I, _I]),
    "rte_grouped_swiglu_fused_ok": (_I, [_I, _I]),
    "rte_grouped_swiglu_fused_fwd": (
        _I,
        [_P, _I, _I, _P, _I, _I, _I, _P, _P, _P, _P, _P, _I64, _P, _P, _P, _P],
    ),
    "rte_grouped_swiglu_fused_bwd": (
        _I,
        [_P, _P, _I, _I, _P, _I, _I, _I, _P, _P, _P, _P, _P, _I64, _P, _P, _P, _P, _P, _P, _P, _I, _F, _P, _SZ,
         _P],
    ),
    "rte_dense_swiglu_fwd": (_I, [_P, _I, _I, _I, _P, _P, _I, _P, _P, _P, _P, _I, _P]),
    "rte_dense_swiglu_bwd": (_I, [_P, _P, _I, _I, _I, _P, _P, _I, _P, _P, _P, _P, _P, _P, _P, _SZ, _P]),
    "rte_qkv_rope_fwd": (_I, [_P, _P, _P, _P, _I, _I, _I, _I, _P, _P, _P, _P, _SZ, _P]),
    "rte_qkv_rope_bwd": (
        _I,
        [_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _P, _P, _P, _P, _SZ, _P],
    ),
    "rte_svd_ffn_fwd": (_I, [_P, _I, _I, _I, _I, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _I, _P]),
    "rte_svd_ffn_bwd": (
        _I,
        [_P, _P, _I, _I, _I, _I, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _SZ, _P],
    ),
    "rte_svd_ffn_fused_workspace_bytes": (_SZ, [_I, _I, _I, _I]),
    "rte_svd_ffn_fused_fwd": (_I, [_P, _I, _I, _I, _I, _P, _P, _P, _P, _P, _P, _P, _P, _I, _P, _SZ, _P]),
    "rte_svd_ffn_fused_bwd": (
        _I,
        [_P, _P, _I, _I, _I, _I, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _SZ, _P],
    ),
    "rte_svd_sparse_fwd": (_I, [_P, _I, _I, _I, _I, _P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _P, _P, _P, _P,
                                _I, _P, _P, _P, _P, _P]),
    "rte_svd_sparse_bwd": (_I, [_P, _I, _I, _I, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P]),
    "rte_rmsnorm_fwd": (_I, [_P, _P, _I, _I, _F, _P, _P, _P]),
    "rte_rmsnorm_bwd_workspace_bytes": (_SZ, [_I, _I]),
    "rte_rmsnorm_bwd": (_I, [_P, _P, _P, _P, _P, _I, _I, _P, _P, _P, _I, _P, _SZ, _P]),
    "rte_fused_rmsnorm_fwd": (_I, [_P, _P, _I, _P, _I, _I, _F, _P, _P, _I, _P, _P]),
    "rte_fused_rmsnorm_bwd_workspace_bytes": (_SZ, [_I, _I]),
    "rte_fused_rmsnorm_bwd": (_I, [_P, _I, _P, _P, _I, _P, _P, _I, _I, _P, _P, _P, _SZ, _P]),
    "rte_rope_apply": (_I, [_P, _P, _I, _I64, _I, _I, _P, _P, _P, _P, _I, _I, _P]),
    "rte_route_centers": (_I, [_P, _I, _I, _P, _I, _P, _P]),
    "rte_ce_fwd": (_I, [_P, _I64, _I, _I, _P, _P, _P, _P]),
    "rte_ce_bwd": (_I, [_P, _I64, _I, _I, _P, _P, _P, _P, _P, _P]),
    "rte_ce_bwd_rows": (_I, [_P, _I64, _I, _I, _P, _P, _P, _P, _P, _I, _I, _P, _P]),
    "rte_axpy_norm_fwd": (_I, [_P, _P, _P, _P, _P, _I, _I, _I, _P, _P, _P, _F, _P, _P, _P, _P]),
    "rte_axpy_norm_bwd_workspace_bytes": (_SZ, [_I, _I]),
    "rte_axpy_norm_bwd": (_I, [_P, _P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _P, _P, _P, _P, _P, _SZ, _P]),
    "rte_adamw_chunk": (_I, []),
    "rte_adamw_workspace_bytes": (_SZ, [_I, _I, _I]),
    "rte_adamw_step": (_I, [_P, _I, _P, _P, _I, _P, _I, _P, _I, _F, _P, _P, _P, _SZ, _P]),
    "rte_macro_workspace_bytes": (_SZ, [_I, _I, _I]),
    "rte_macro_prologue_fwd": (_I, [_P, _P, _I, _I, _I, _I, _F, _P, _P, _P, _SZ, _P]),
    "rte_macro_prologue_bwd": (_I, [_P, _P, _P, _P, _I, _I, _I, _I, _P, _P, _P, _SZ, _P]),
    "rte_macro_epilogue_fwd": (_I, [_P, _P, _P, _I, _I, _I, _I, _P, _P, _P, _F, _P, _P]),
    "rte_macro_epilogue_bwd": (_I, [_P, _P, _P, _P, _I, _I, _I, _I, _P, _P, _P, _F, _P, _P, _P, _SZ, _P]),
    "rte_macro_table_grad": (_I, [_P, _I, _I, _I, _I, _P, _P, _P, _P, _P]),
    "rte_macro_fused_tiles": (_I, [_I]),
    "rte_macro_fused_fwd_workspace_bytes": (_SZ, [_I, _I, _I]),
    "rte_macro_fused_wgrad_workspace_bytes": (_SZ, [_I, _I, _I, _I]),
    "rte_macro_fused_prep": (_I, [_P, _P, _I, _I, _P, _P, _P, _P, _P, _P]),
    "rte_macro_fused_bwd_workspace_bytes": (_SZ, [_I, _I]),
    "rte_macro_fused_fwd": (_I, [_P, _P, _I, _I, _P, _I, _I, _I, _I, _F, _P, _P, _P, _P, _P, _P, _F, _P, _P, _P,
                                 _P, _P, _P, _P, _P, _P, _P, _SZ, _P]),
    "rte_macro_fused_sum": (_I, [_P, _I, _F, _P, _P]),
    "rte_macro_cons_workspace_bytes": (_SZ, [_I, _I, _I, _I]),
    "rte_macro_cons_prep": (_I, [_P, _P, _I, _I, _P, _P, _P]),
    "rte_macro_cons_fwd": (_I, [_P, _I, _I, _I, _P, _I, _P, _I, _I, _I, _I, _F] + [_P] * 7 + [_F] + [_P] * 7
                           + [_SZ, _P]),
    "rte_macro_cons_bwd": (_I, [_P, _I, _I, _I, _P, _I, _P, _I, _I, _I, _I] + [_P] * 6 + [_F] + [_P] * 4 + [_F]
                           + [_P] * 7),
    "rte_macro_fused_bwd": (_I, [_P, _P, _P, _F, _I, _I, _P, _I, _I, _P, _P, _P, _I, _P, _I, _I, _I, _I, _P, _P, _P, _P, _P,
                                 _P, _P, _P, _P, _P, _F, _P, _P, _P, _P, _P, _P, _I, _P, _I, _P, _P, _SZ, _P]),
    "rte_macro_fused_wgrad": (_I, [_P, _I, _I, _I, _I, _I, _I, _I, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P,
                                   _P, _P, _SZ, _P]),
    "rte_attention_fwd": (_I, [_P, _P, _P, _I, _I, _I, _I, _F, _P, _P, _P, _P]),
    "rte_attention_bwd": (_I, [_P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _F, _P, _P, _P, _P, _P]),
    "rte_attention_bwd_qkv": (_I, [_P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _F, _P, _P, _P, _P, _P]),
    "rte_router_pool": (_I, [_P, _I, _I, _I, _P, _P, _P]),
    "rte_router_heads_fwd": (_I, [_P, _P, _I, _I, _P, _P, _I, _P, _P, _I, _P, _I, _P, _F, _I, _I] + [_P] * 17 + [_P]),
    "rte_router_heads_bwd": (_I, [_P, _P, _P, _P, _I, _I, _I, _I, _F] + [_P] * 13 + [_P, _P, _P, _P]),
    "rte_router_mlp_bwd": (_I, [_P] * 6 + [_I, _I, _I, _I, _P, _I, _F] + [_P] * 9 + [_P]),
    "rte_router_aux_fwd": (_I, [_P, _P, _P, _I, _I, _F, _F, _F, _F, _P, _P, _P]),
    "rte_router_aux_bwd": (_I, [_P, _P, _P, _I, _I, _F, _F, _P, _P, _P]),
    "rte_audit_sample_fixed": (_I, [_P, _P, _P, _P, _I, _I, _I] + [_F] * 8 + [_P, _P, _P, _P, _P]),
    "rte_count_ema": (_I, [_P, _P, _I, _P, _I, _F, _P]),
    "rte_nonfinite": (_I, [_P, _P, _P, _P]),
    "rte_step_metrics": (_I, [_P, _P, _P, _I, _F, _F, _P, _P]),
    "rte_loss_sum": (_I, [_P, _I, _F, _P, _I, _P, _P]),
    "rte_loss_sum_bwd": (_I, [_P, _I, _F, _P, _P]),
    "rte_mse_workspace_bytes": (_SZ, [_I64]),
    "rte_mse_fwd": (_I, [_P, _P, _I64, _P, _P, _SZ, _P]),
    "rte_replay_fwd_pass": (_I, [_I] * 8 + [_P] * 7 + [_F] + [_P] * 3 + [_F] + [_P] * 2 + [_F] + [_P] * 25),
    "rte_replay_row_tiles": (_I, [_I, _I]),
    "rte_replay_bwd_prep": (_I, [_I] * 3 + [_P] * 6),
    "rte_replay_bwd_pass": (_I, [_I] * 8 + [_P] * 5 + [_F] + [_P] * 33 + [_I] + [_P] * 9),
    "rte_replay_param_reduce": (_I, [_I] * 4 + [_P] * 7),
    "rte_gemm_f32": (_I, [_P, _I64, _I, _P, _P, _P, _I64, _I, _P, _P, _P, _I64, _P, _I, _I, _I, _F, _F, _I, _I,
                          _I64, _I64, _I64, _I64, _I64, _I64, _P]),
    "rte_gemm_f32_grouped": (_I, [_I, _P, _I, _P, _I64, _I, _P, _P, _P, _I64, _I, _P, _P, _P, _I64, _I64, _P, _I64,
                                  _P, _P, _I64, _I64, _I, _I, _I, _F, _F, _P]),
    "rte_softmax_causal_f32_fwd": (_I, [_P, _I64, _I, _F, _P, _P, _P, _P]),
    "rte_softmax_causal_f32_bwd": (_I, [_P, _P, _I64, _I, _F, _P, _P, _P]),
    "rte_swiglu_f32_fwd": (_I, [_P, _I64, _I, _I64, _P, _P]),
    "rte_swiglu_f32_bwd": (_I, [_P, _P, _I64, _I, _I64, _P, _P]),
    "rte_combine_f32": (_I, [_P, _P, _P, _I, _I, _I, _P, _P, _P]),
    "rte_pair_dot_f32": (_I, [_P, _P, _P, _I64, _I, _I, _P, _P]),
    "rte_mse_bwd": (_I, [_P, _P, _I64, _P, _P, _P, _P]),
    "rte_pack_routes_workspace_bytes": (_SZ, [_I, _I]),
    "rte_pack_routes": (_I, [_P, _P, _I, _I, _P, _I, _I, _P, _I, _P, _P, _P, _P, _P, _P, _SZ, _P]),
    "rte_distill_workspace_bytes": (_SZ, [_I, _I]),
    "rte_distill_fwd": (_I, [_P, _P, _P, _I, _I, _I, _P, _P, _I, _F, _F, _P, _P, _P, _P, _SZ, _P]),
    "rte_distill_bwd": (_I, [_P, _P, _P, _I, _I, _I, _P, _P, _I, _F, _F, _P, _P, _P, _SZ, _P, _P, _P]),
    "rte_audit_correct_fwd": (_I, [_P, _P, _I, _I, _P, _I, _P, _F, _I, _P, _P, _P, _P, _P]),
    "rte_audit_correct_bwd": (_I, [_P, _I, _I, _P, _I, _P, _P, _P, _P]),
    "rte_cast_f32_bf16": (_I, [_P, _I64, _P, _P]),
    "rte_cast_many_blocks": (_I, [_I, _I64, _I64]),
    "rte_cast_many": (_I, [_P, _P, _I, _P]),
    "rte_grouped_linear_fwd": (_I, [_P, _I, _I, _P, _I, _I, _P, _P, _P, _I, _P, _I, _P]),
    "rte_grouped_linear_bwd": (_I, [_P, _P, _I, _I, _P, _I, _I, _P, _P, _P, _I, _P, _I, _P, _P, _SZ, _P]),
    "rte_grouped_linear_bwd_workspace_bytes": (_SZ, [_I, _I, _I, _I]),
    "rte_segment_reduce_workspace_bytes": (_SZ, [_I64, _I, _I]),
    "rte_segment_reduce_rows": (_I, [_P, _I64, _I, _I, _P, _P, _I, _I, _P, _I, _P, _SZ, _P]),
    "rte_shortlist_build": (_I, [_P, _P, _I, _P, _I, _I, _P, _I, _I, _I, _I, _I, _P, _P, _P]),
    "rte_shortlist_fwd": (_I, [_P, _P, _I, _I, _P, _I, _I, _P, _P, _P, _P]),
    "rte_shortlist_bwd_workspace_bytes": (_SZ, [_I, _I, _I, _I]),
    "rte_shortlist_bwd": (_I, [_P, _P, _P, _P, _I, _I, _P, _I, _I, _P, _P, _P, _P, _I, _P, _SZ, _P]),
}

_LIB: ctypes.CDLL | None = None
_LOAD_ERROR: str | None = None


def load() -> ctypes.CDLL:
    """Load the shared library (no device call); raises if it is not built."""
    global _LIB, _LOAD_ERROR
    if _LIB is not None:
        return _LIB
    if not LIB_PATH.exists():
        _LOAD_ERROR = f"{LIB_PATH} is not built; run speedup-thingy_amd/build.py (hipcc, gfx950)"
        raise RuntimeError(_LOAD_ERROR)
    try:
        lib = ctypes.CDLL(str(LIB_PATH))
    except OSError as exc:  # pragma: no cover - depends on the ROCm runtime
        _LOAD_ERROR = f"cannot load {LIB_PATH}: {exc}"
        raise RuntimeError(_LOAD_ERROR) from exc
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _LIB = lib
    return lib


def loaded() -> bool:
    try:
        load()
        return True
    except RuntimeError:
        return False


def device_ready() -> bool:
    """Library loads and a gfx950 ROCm device is visible."""
    if not loaded() or not torch.cuda.is_available() or torch.version.hip is None:
        return False
    try:
        return "gfx950" in torch.cuda.get_device_properties(0).gcnArchName
    except Exception:  # pragma: no cover
        return False


def last_error() -> str:
    msg = load().rte_last_error()
    return msg.decode() if msg else ""


def call(name: str, *args) -> int:
    rc = getattr(load(), name)(*args)
    if rc != 0:
        raise RuntimeError(f"{name} failed (code {rc}): {last_error()}")
    return rc


def stream_ptr(device: torch.device | None = None) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def device_info() -> dict[str, str]:
    buf = ctypes.create_string_buffer(512)
    call("rte_device_info", buf, len(buf))
    out = {}
    for item in buf.value.decode().split(";"):
        if "=" in item:
            k, v = item.split("=", 1)
            out[k] = v
    return out


def require_device_tensors(op: str, *tensors: torch.Tensor | None) -> None:
    """Every operand of a HIP operator must already live on the ROCm device."""
    if not device_ready():
        reason = _LOAD_ERROR or "no gfx950 ROCm device is visible"
        if loaded() and _LOAD_ERROR is None:
            reason = "no gfx950 ROCm device is visible"
        raise RuntimeError(f"{op}: the HIP backend is required and unavailable ({reason})")
    for t in tensors:
        if t is not None and not t.is_cuda:
            raise RuntimeError(f"{op}: expects ROCm device tensors, got a tensor on {t.device}")


def env_flag(name: str) -> bool:
    return os.environ.get(name, "").lower() in {"1", "true", "yes"}
