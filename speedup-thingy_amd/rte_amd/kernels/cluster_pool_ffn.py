"""The reference's cluster-pool FFN backend module (rte/kernels/cluster_pool_ffn.py) on the HIP
kernels: same function names, arguments, shapes and error conventions.

Pools are arbitrary candidate-id lists (prepare_cluster_pool_weights, :90-126); the pooled
SwiGLU runs as the grouped MFMA kernel over a deterministic stable pack of the tokens (ascending
token order inside a cluster, the slot order of build_static_pack_gather_indices, :165-189),
so no padded [C, max_count, d] copy of x is made; pool-weight gradients reach the dense rows
through a fixed-order segmented reduction (scatter_cluster_pool_grads, :218-241), which sums
the rows of overlapping pools without atomics.  There is no CPU path: without the HIP backend
every function raises.
"""

from __future__ import annotations

import torch

from rte_amd import _lib
from rte_amd.kernels import hip_ops


def available() -> bool:
    return _lib.device_ready()


def _require_available() -> None:
    if not available():
        raise RuntimeError("Cluster-pool FFN kernels require the ROCm HIP backend (librte_hip.so on a gfx950 "
                           "device), which replaces the reference's CUDA + Triton path")


def prepare_cluster_pool_weights(w_up: torch.Tensor, w_gate: torch.Tensor, w_down: torch.Tensor,
                                 candidate_ids: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Gather each cluster's candidate rows: wup_pool / wgate_pool [C, d, M], wdown_pool [C, M, d]
    (rte/kernels/cluster_pool_ffn.py:90-126).  The row gathers' backward is the deterministic
    segmented reduction (rows shared by several pools add up in a fixed order)."""
    if candidate_ids.ndim != 2:
        raise ValueError("candidate_ids must have shape [clusters, candidate_m]")
    C, M = candidate_ids.shape
    ids = candidate_ids.to(device=w_up.device, dtype=torch.long).reshape(-1)
    up = hip_ops.embedding(w_up, ids).view(C, M, w_up.shape[1])
    gate = hip_ops.embedding(w_gate, ids).view(C, M, w_gate.shape[1])
    down = hip_ops.embedding(w_down, ids).view(C, M, w_down.shape[1])
    return up.transpose(1, 2).contiguous(), gate.transpose(1, 2).contiguous(), down.contiguous()


def route_to_static_centers(x: torch.Tensor, up_a: torch.Tensor, gate_a: torch.Tensor,
                            centers: torch.Tensor) -> torch.Tensor:
    """argmax over clusters of normalize([x A_up | x A_gate]) . centers (fp32 features;
    rte/kernels/cluster_pool_ffn.py:129-140): one GEMM for both selector halves, then the
    normalise / score / argmax kernel.  Returns int64 cluster ids [T]."""
    _lib.require_device_tensors("route_to_static_centers", x, up_a, gate_a, centers)
    a = torch.cat([up_a, gate_a], dim=1)                       # [d, 2r]
    q = hip_ops.gemm(x.reshape(-1, x.shape[-1]).to(torch.bfloat16), hip_ops.cast_bf16(a.t().contiguous()),
                     out_f32=True)
    return hip_ops.route_centers(q, centers).to(torch.long).view(x.shape[:-1])


def _pack(assignments: torch.Tensor, cluster_count: int):
    cl = assignments.reshape(-1, 1).to(torch.int32)
    pk = hip_ops.pack_index(cl, cluster_count)
    rank = pk.slot_of_pair.long() - pk.offsets.long()[cl.reshape(-1).long().clamp(0, cluster_count - 1)]
    return pk, rank


def build_static_pack_gather_indices(assignments: torch.Tensor, *, cluster_count: int):
    """(pack_index [C, max_count] long, flat_gather [T] long, counts [C] long, max_count) of
    rte/kernels/cluster_pool_ffn.py:165-189: tokens of each cluster in ascending order,
    zero-padded; flat_gather[t] = cluster * max_count + rank of t in its cluster.  The sort is the
    HIP stable pack; max_count is read on the host, as in the reference."""
    if assignments.ndim != 1:
        raise ValueError("assignments must have shape [tokens]")
    _lib.require_device_tensors("build_static_pack_gather_indices", assignments)
    pk, rank = _pack(assignments, cluster_count)
    counts = (pk.offsets[1:] - pk.offsets[:-1]).long()
    max_count = int(counts.max().item()) if counts.numel() else 0
    a = assignments.long()
    pack_index = torch.zeros(cluster_count, max_count, device=a.device, dtype=torch.long)
    pack_index[a, rank] = torch.arange(a.numel(), device=a.device)
    flat_gather = a * max_count + rank
    return pack_index.contiguous(), flat_gather.contiguous(), counts, max_count


def _pool_layout(wup_pool, wgate_pool, wdown_pool):
    C, d, M = wup_pool.shape
    if wgate_pool.shape != (C, d, M) or wdown_pool.shape != (C, M, d):
        raise ValueError("cluster pools must be wup/wgate [C, d, M] and wdown [C, M, d]")
    if M % 32 != 0:
        raise ValueError(f"candidate_m = {M} must be a multiple of 32 (MFMA tile)")
    wug_t = torch.cat([wup_pool.transpose(1, 2).reshape(C * M, d), wgate_pool.transpose(1, 2).reshape(C * M, d)])
    wd_t = wdown_pool.reshape(C * M, d).t()
    return wug_t, wd_t, M


def _run(x, cl_ids, wup_pool, wgate_pool, wdown_pool):
    wug_t, wd_t, M = _pool_layout(wup_pool, wgate_pool, wdown_pool)
    T = x.shape[0]
    w = torch.ones((T, 1), device=x.device, dtype=torch.float32)
    out = hip_ops.grouped_pool_swiglu(x, cl_ids.reshape(T, 1).to(torch.int32), w, wug_t, wd_t, M)
    dt = torch.bfloat16 if (x.dtype == torch.bfloat16 or torch.is_autocast_enabled("cuda")) else out.dtype
    return out.to(dt)


def cluster_pool_ffn_forward_preindexed(x: torch.Tensor, pack_index: torch.Tensor, flat_gather: torch.Tensor,
                                        wup_pool: torch.Tensor, wgate_pool: torch.Tensor,
                                        wdown_pool: torch.Tensor) -> torch.Tensor:
    """Differentiable pooled SwiGLU for tokens pre-indexed by build_static_pack_gather_indices
    (rte/kernels/cluster_pool_ffn.py:192-215): token t runs through pool flat_gather[t] //
    max_count.  Output bf16 as the reference's bmm under autocast."""
    if x.ndim != 2:
        raise ValueError("x must have shape [tokens, d_model]")
    _lib.require_device_tensors("cluster_pool_ffn_forward_preindexed", x, pack_index, flat_gather, wup_pool,
                                wgate_pool, wdown_pool)
    max_count = pack_index.shape[1]
    if max_count == 0:
        return x.new_zeros(x.shape)
    return _run(x, torch.div(flat_gather, max_count, rounding_mode="floor"), wup_pool, wgate_pool, wdown_pool)


def scatter_cluster_pool_grads(candidate_ids: torch.Tensor, wup_pool_grad: torch.Tensor,
                               wgate_pool_grad: torch.Tensor, wdown_pool_grad: torch.Tensor, *, d_ff: int):
    """Dense row gradients of pool gradients: dense[ids[c, j]] += pool_grad row (c, j), duplicates
    summed (rte/kernels/cluster_pool_ffn.py:218-241), by the fixed-order segmented reduction."""
    if candidate_ids.ndim != 2:
        raise ValueError("candidate_ids must have shape [clusters, candidate_m]")
    ids = candidate_ids.reshape(-1).to(device=wup_pool_grad.device, dtype=torch.int32)
    d = wdown_pool_grad.shape[-1]
    dt = wup_pool_grad.dtype
    up = hip_ops.segment_reduce_rows(ids, d_ff, wup_pool_grad.transpose(1, 2).reshape(-1, d).float())
    gate = hip_ops.segment_reduce_rows(ids, d_ff, wgate_pool_grad.transpose(1, 2).reshape(-1, d).float())
    down = hip_ops.segment_reduce_rows(ids, d_ff, wdown_pool_grad.reshape(-1, d).float())
    return up.to(dt), gate.to(dt), down.to(dt)


def cluster_pool_ffn_reference(x, assignments, wup_pool, wgate_pool, wdown_pool):
    """The reference's per-cluster loop (rte/kernels/cluster_pool_ffn.py:143-162) has the same
    result as the pooled kernel over the tokens' clusters; it runs that kernel."""
    _lib.require_device_tensors("cluster_pool_ffn_reference", x, assignments, wup_pool, wgate_pool, wdown_pool)
    return _run(x, assignments, wup_pool, wgate_pool, wdown_pool).to(x.dtype)


def cluster_pool_ffn_forward_from_assignments(x, assignments, wup_pool, wgate_pool, wdown_pool, *,
                                              max_tokens_per_cluster: int | None = None, block_d: int = 64,
                                              return_overflow: bool = False):
    """Inference pooled SwiGLU from token assignments with a per-cluster capacity
    (rte/kernels/cluster_pool_ffn.py:244-330): tokens beyond a cluster's first
    max_tokens_per_cluster (in ascending token order; the reference's slot order is that of its
    atomics) output zeros and raise the overflow flag.  block_d is accepted for API parity."""
    del block_d
    if x.ndim != 2:
        raise ValueError("x must have shape [tokens, d_model]")
    if assignments.ndim != 1 or assignments.shape[0] != x.shape[0]:
        raise ValueError("assignments must have shape [tokens]")
    if wup_pool.ndim != 3 or wgate_pool.ndim != 3 or wdown_pool.ndim != 3:
        raise ValueError("cluster pools must be rank-3 tensors")
    if wup_pool.shape[0] != wgate_pool.shape[0] or wup_pool.shape[0] != wdown_pool.shape[0]:
        raise ValueError("cluster pools must have the same cluster count")
    _require_available()
    tensors = (x, assignments, wup_pool, wgate_pool, wdown_pool)
    if any(not t.is_cuda for t in tensors):
        raise RuntimeError("cluster-pool FFN device path requires all tensors on the ROCm device")
    if torch.is_grad_enabled() and any(t.requires_grad for t in tensors):
        raise RuntimeError("cluster-pool FFN device path is inference/eval only; backward is not implemented")
    C = wup_pool.shape[0]
    cap = x.shape[0] if max_tokens_per_cluster is None else max(1, int(max_tokens_per_cluster))
    _, rank = _pack(assignments, C)
    keep = rank < cap
    overflow = (~keep).any().to(torch.int32)
    ids = torch.where(keep, assignments.long(), torch.full_like(assignments.long(), -1))
    out = _run(x, ids, wup_pool, wgate_pool, wdown_pool).to(x.dtype)
    return (out, overflow) if return_overflow else out
