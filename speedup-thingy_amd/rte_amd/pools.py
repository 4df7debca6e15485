"""Static cluster-pool construction: the offline step that turns a dense model into the
`factors` / `codebook` dicts StaticClusterPoolSwiGLU (rte_amd/layers.py) takes, and the active
union of its candidate neurons (rte/cli.py:3244-3388, 4703-4782, 4915-4941).

  build_svd_factor_cache      per block, truncated SVD of the up / gate weights (float32 on the
                              host, as the reference): up_a = U S [d, r], up_b = Vh [r, F]
  fit_cluster_centers         cosine k-means on normalised selector features (evenly spaced
                              initial rows, empty clusters keep their centre)
  aggregate_cluster_scores    mean or max of the per-token neuron scores over each cluster
  svd_cluster_features_and_scores
                              selector features [x A_up | x A_gate] and the neuron scores
                              |up_hat|, |silu(gate_hat)|, |up_hat silu(gate_hat)| weighted by the
                              down-projection column norms
  build_static_svd_cluster_pool_codebook
                              calibration batches through the dense model's blocks (the HIP
                              forward, at fp32 precision as the reference's calibration runs),
                              features and scores staged in fp16 as there, then centres and the
                              top-M candidate neurons of each cluster
  active_union_ids_from_codebook
                              the sorted union of every cluster's candidates, or its cap by a
                              frequency-plus-rank score

This is a build step, run once per codebook: small tensor arithmetic stays torch on whatever
device the model lives on; the forward passes are the model's own operators.
"""

from __future__ import annotations

import torch
import torch.nn.functional as F

from rte_amd.kernels import hip_ops


@torch.no_grad()
def build_svd_factor_cache(dense, *, max_rank: int, device=None) -> list[dict[str, torch.Tensor]]:
    """rte/cli.py:3244-3261: per block {up_a, up_b, gate_a, gate_b} with A = U[:, :r] S[:r] and
    B = Vh[:r] from torch.linalg.svd of the [d, F] weight, in float32 on the host."""
    factors = []
    for block in dense.blocks:
        dev = device if device is not None else block.mlp.wug.weight.device
        w = block.mlp.wug.weight.detach().float().cpu()
        up_w, gate_w = w.chunk(2, dim=0)
        layer = {}
        for name, mat in (("up", up_w.t().contiguous()), ("gate", gate_w.t().contiguous())):
            u, s, vh = torch.linalg.svd(mat, full_matrices=False)
            r = min(int(max_rank), s.numel())
            layer[f"{name}_a"] = (u[:, :r] * s[:r]).to(device=dev)
            layer[f"{name}_b"] = vh[:r, :].to(device=dev)
        factors.append(layer)
    return factors


def _segment_sum(keys: torch.Tensor, n: int, rows: torch.Tensor) -> torch.Tensor:
    """[n, f] sums of rows by key.  Device rows go through the HIP segmented reduction (a fixed
    summation order, so rebuilding a codebook repeats it bitwise; the width is zero-padded to
    whole 8-column chunks); host rows (tests) through index_add_."""
    if not rows.is_cuda:
        return rows.new_zeros(n, rows.shape[-1]).index_add_(0, keys, rows)
    f = rows.shape[-1]
    pad = (-f) % 8
    r = F.pad(rows.float(), (0, pad)) if pad else rows.float()
    out = []
    for c0 in range(0, r.shape[1], 2048):  # the reduction's row width limit
        out.append(hip_ops.segment_reduce_rows(keys, n, r[:, c0:c0 + 2048].contiguous()))
    return torch.cat(out, dim=1)[:, :f].to(rows.dtype)


def _kmeans(x: torch.Tensor, cluster_count: int, iters: int):
    """Cosine k-means of normalised rows x (rte/cli.py:3264-3329)."""
    n = x.shape[0]
    init = torch.linspace(0, n - 1, steps=cluster_count, device=x.device).round().long()
    centers = x.index_select(0, init).contiguous()
    assignments = torch.zeros(n, device=x.device, dtype=torch.long)
    for _ in range(max(1, int(iters))):
        assignments = (x @ centers.t()).argmax(dim=-1)
        new = _segment_sum(assignments, cluster_count, x)
        counts = torch.bincount(assignments, minlength=cluster_count).to(new.dtype)
        nonempty = counts > 0
        new[nonempty] = new[nonempty] / counts[nonempty].unsqueeze(-1).clamp_min(1.0)
        new[~nonempty] = centers[~nonempty]
        centers = F.normalize(new, dim=-1)
    return assignments, centers


@torch.no_grad()
def fit_cluster_centers(features: torch.Tensor, *, cluster_count: int, iters: int):
    """(assignments [N] long, centres [C, f]) of rte/cli.py:3297-3329: C is capped at the row
    count; one cluster (or one row) gives the normalised mean as its centre."""
    n = features.shape[0]
    cluster_count = min(max(1, int(cluster_count)), max(1, n))
    x = F.normalize(features.float(), dim=-1)
    if cluster_count == 1 or n == 1:
        return torch.zeros(n, device=x.device, dtype=torch.long), F.normalize(x.mean(dim=0, keepdim=True), dim=-1)
    return _kmeans(x, cluster_count, iters)


@torch.no_grad()
def cluster_assignments_from_features(features: torch.Tensor, *, cluster_count: int, iters: int) -> torch.Tensor:
    """rte/cli.py:3264-3294 (the assignments alone; one cluster or one row gives zeros)."""
    n = features.shape[0]
    cluster_count = min(max(1, int(cluster_count)), max(1, n))
    if cluster_count == 1 or n == 1:
        return torch.zeros(n, device=features.device, dtype=torch.long)
    return _kmeans(F.normalize(features.float(), dim=-1), cluster_count, iters)[0]


@torch.no_grad()
def aggregate_cluster_scores(scores: torch.Tensor, assignments: torch.Tensor, *, cluster_count: int,
                             aggregation: str) -> torch.Tensor:
    """rte/cli.py:3332-3355: per-cluster mean (empty clusters 0) or max of the score rows."""
    C = max(1, int(cluster_count))
    if aggregation == "mean":
        agg = _segment_sum(assignments, C, scores)
        counts = torch.bincount(assignments, minlength=C).to(scores.dtype).clamp_min(1.0)
        return agg / counts.unsqueeze(-1)
    if aggregation == "max":
        out = scores.new_zeros(C, scores.shape[-1])
        idx = assignments.unsqueeze(-1).expand_as(scores)
        out.scatter_reduce_(0, idx, scores, reduce="amax", include_self=False)
        return out  # clusters without rows keep 0, as the reference's zero rows
    raise ValueError(f"unsupported cluster score aggregation: {aggregation}")


@torch.no_grad()
def svd_cluster_features_and_scores(block, normed: torch.Tensor, factors: dict, *, rank: int, score_mode: str):
    """rte/cli.py:3358-3388: (features [N, 2r], neuron scores [N, F])."""
    flat = normed.reshape(-1, normed.shape[-1]).float()
    hidden = block.mlp.wd.weight.shape[1]
    rank = min(max(1, int(rank)), factors["up_a"].shape[1], factors["gate_a"].shape[1])
    q_up = flat @ factors["up_a"][:, :rank]
    q_gate = flat @ factors["gate_a"][:, :rank]
    up_hat = q_up @ factors["up_b"][:rank, :]
    gate_act = F.silu(q_gate @ factors["gate_b"][:rank, :])
    wd_norm = block.mlp.wd.weight.detach().float().norm(dim=0).to(flat.device)
    up_s = up_hat.abs() * wd_norm
    gate_s = gate_act.abs() * wd_norm
    prod_s = (up_hat * gate_act).abs() * wd_norm
    if score_mode == "sum":
        scores = up_s + gate_s + prod_s
    elif score_mode == "upgate":
        scores = up_s + gate_s
    elif score_mode == "product":
        scores = prod_s
    else:
        raise ValueError(f"unsupported cluster pool score mode: {score_mode}")
    if scores.shape[-1] != hidden:
        raise RuntimeError("cluster score width does not match FFN hidden width")
    return torch.cat([q_up, q_gate], dim=-1), scores


@torch.no_grad()
def build_static_svd_cluster_pool_codebook(dense, svd_factors, batches, *, calibration_batches: int, device,
                                           rank: int, cluster_count: int, candidate_m: int, score_mode: str,
                                           aggregation: str, cluster_iters: int):
    """rte/cli.py:4703-4782: ([{centers, candidate_ids}] per block, calibration metrics).  Each
    calibration batch runs the dense blocks (attention, norm, FFN) at fp32 precision; every
    block's selector features and neuron scores are staged in fp16 as the reference stages them."""
    feats = [[] for _ in dense.blocks]
    scores = [[] for _ in dense.blocks]
    seen = 0
    with hip_ops.fp32_precision():
        for _ in range(calibration_batches):
            tokens, _ = next(batches)
            tokens = tokens.to(device)
            x = dense.embed(tokens).float()
            seen += int(tokens.numel())
            for i, block in enumerate(dense.blocks):
                u = block.attn(block.norm1(x), resid=x)
                normed = block.norm2(u)
                f, s = svd_cluster_features_and_scores(block, normed, svd_factors[i], rank=rank,
                                                       score_mode=score_mode)
                feats[i].append(f.to(torch.float16))
                scores[i].append(s.to(torch.float16))
                x = block.mlp(normed, resid=u)
    codebook = []
    nonempty_sum = imbalance_sum = 0.0
    for i in range(len(dense.blocks)):
        f = torch.cat(feats[i]).float()
        s = torch.cat(scores[i]).float()
        assignments, centers = fit_cluster_centers(f, cluster_count=cluster_count, iters=cluster_iters)
        C = min(max(1, int(cluster_count)), f.shape[0])
        agg = aggregate_cluster_scores(s, assignments, cluster_count=C, aggregation=aggregation)
        cand = torch.topk(agg, k=min(candidate_m, agg.shape[-1]), dim=-1).indices
        sizes = torch.bincount(assignments, minlength=C).float()
        nonempty = sizes[sizes > 0]
        nonempty_sum += float(nonempty.numel())
        imbalance_sum += float((nonempty.max() / nonempty.mean().clamp_min(1.0)).item()) if nonempty.numel() else 0.0
        codebook.append({"centers": centers.to(device=device), "candidate_ids": cand.to(device=device)})
    nb = max(1, len(dense.blocks))
    return codebook, {"calibration_tokens_seen": float(seen),
                      "calibration_avg_nonempty_clusters": nonempty_sum / nb,
                      "calibration_avg_cluster_imbalance": imbalance_sum / nb}


@torch.no_grad()
def active_union_ids_from_codebook(candidate_ids: torch.Tensor, *, hidden: int, cap: int | None = None):
    """rte/cli.py:4915-4941: the sorted union of the candidates; above `cap`, the cap neurons of
    highest frequency-plus-rank score (rank weight linear from 1 to 1/M within a cluster's list)."""
    ids = candidate_ids.to(dtype=torch.long)
    union = torch.unique(ids.reshape(-1), sorted=True)
    if cap is None or int(cap) <= 0 or union.numel() <= int(cap):
        return union
    cap = min(int(cap), hidden)
    C, M = ids.shape
    rank_w = torch.linspace(1.0, 1.0 / max(M, 1), steps=M, device=ids.device, dtype=torch.float32)
    score = torch.zeros(hidden, device=ids.device, dtype=torch.float32)
    score.index_add_(0, ids.reshape(-1), rank_w.unsqueeze(0).expand(C, M).reshape(-1))
    return torch.sort(torch.topk(score, k=cap, dim=0).indices).values
