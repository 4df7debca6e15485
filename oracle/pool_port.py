"""CPU forms of one routed cluster-pool SwiGLU layer, forward + backward (torch on the CPU,
float32) -- CPU BASELINE AND TEST INFRASTRUCTURE ONLY.

8192 tokens, d_model 256, 32 clusters x 32 neurons (d_ff 1024), router
logits x W_r, top-4 clusters per token with softmax weights over the selected logits; x ~ N(0, 1),
weights ~ N(0, 0.02), seed 0.  Both of the reference's execution forms, generalised from one
cluster per token to k (token, cluster) pairs per token:

  loop        cluster_pool_ffn_reference (rte/kernels/cluster_pool_ffn.py:143-162): a Python loop
              over the clusters, each gathering its rows and running its pool's three products
  preindexed  prepare_cluster_pool_weights (:90-126) gathers the pools from the dense weights,
              build_static_pack_gather_indices (:165-189) pads each cluster's pair list to the
              largest count, cluster_pool_ffn_forward_preindexed (:192-215) runs index_select +
              three bmm + index_select; pool gradients reach the dense rows through the
              gather's autograd (the dense form of scatter_cluster_pool_grads, :218-241)

The routing (top-k with value-descending, index-ascending order) and the weighted sum over a
token's k pairs are common to both.  tests/test_pool_port.py pins both forms against
oracle.cluster_pool.routed_fwd and against each other's gradients.
"""

from __future__ import annotations

import torch
import torch.nn.functional as F


def make_cfg1(T: int = 8192, d: int = 256, C: int = 32, n: int = 32, seed: int = 0):
    """Seeded inputs: x [T, d], w_r [d, C], w_up / w_gate / w_down [C n, d] (row = neuron)."""
    g = torch.Generator().manual_seed(seed)
    F_ = C * n
    x = torch.randn(T, d, generator=g)
    wr = torch.randn(d, C, generator=g) * 0.02
    wup = torch.randn(F_, d, generator=g) * 0.02
    wgate = torch.randn(F_, d, generator=g) * 0.02
    wdown = torch.randn(F_, d, generator=g) * 0.02
    return x, wr, wup, wgate, wdown


def route(x, wr, k: int):
    """(pair cluster ids [T, k], softmax weights [T, k]) of logits x w_r."""
    logits = x @ wr
    ids = torch.argsort(-logits.detach(), dim=-1, stable=True)[:, :k]
    return ids, logits.gather(1, ids).softmax(dim=-1)


def layer_loop(x, wr, wup, wgate, wdown, k: int, n_clusters: int):
    """The per-cluster loop form (rte/kernels/cluster_pool_ffn.py:143-162) over top-k pairs."""
    ids, w = route(x, wr, k)
    n = wup.shape[0] // n_clusters
    out = x.new_zeros(x.shape)
    for c in range(n_clusters):
        tok, slot = torch.nonzero(ids == c, as_tuple=True)
        if tok.numel() == 0:
            continue
        xc = x.index_select(0, tok)
        z = (xc @ wup[c * n:(c + 1) * n].t()) * F.silu(xc @ wgate[c * n:(c + 1) * n].t())
        out = out.index_add(0, tok, w[tok, slot].unsqueeze(1) * (z @ wdown[c * n:(c + 1) * n]))
    return out


def pack_indices(assignments, n_clusters: int):
    """build_static_pack_gather_indices (rte/kernels/cluster_pool_ffn.py:165-189): per cluster
    its items in ascending order, padded to the largest count; flat_gather[item] = its slot."""
    counts = torch.bincount(assignments, minlength=n_clusters)
    max_count = int(counts.max())
    pack = torch.zeros(n_clusters, max_count, dtype=torch.long)
    flat = torch.empty(assignments.numel(), dtype=torch.long)
    for c in range(n_clusters):
        items = torch.nonzero(assignments == c, as_tuple=False).flatten()
        if items.numel():
            pack[c, :items.numel()] = items
            flat[items] = c * max_count + torch.arange(items.numel())
    return pack, flat, max_count


def layer_preindexed(x, wr, wup, wgate, wdown, k: int, n_clusters: int):
    """The preindexed bmm form (rte/kernels/cluster_pool_ffn.py:90-126, 165-215) over top-k pairs."""
    ids, w = route(x, wr, k)
    T, d = x.shape
    n = wup.shape[0] // n_clusters
    cand = torch.arange(n_clusters * n).view(n_clusters, n)
    up_pool = wup.index_select(0, cand.reshape(-1)).view(n_clusters, n, d).transpose(1, 2)
    gate_pool = wgate.index_select(0, cand.reshape(-1)).view(n_clusters, n, d).transpose(1, 2)
    down_pool = wdown.index_select(0, cand.reshape(-1)).view(n_clusters, n, d)
    pack, flat, M = pack_indices(ids.reshape(-1), n_clusters)
    x_pad = x.index_select(0, (pack // k).reshape(-1)).view(n_clusters, M, d)
    z = torch.bmm(x_pad, up_pool) * F.silu(torch.bmm(x_pad, gate_pool))
    y = torch.bmm(z, down_pool).reshape(n_clusters * M, d).index_select(0, flat).view(T, k, d)
    return (w.unsqueeze(-1) * y).sum(dim=1)


def fwd_bwd(form, x, wr, wup, wgate, wdown, dy, k: int, n_clusters: int):
    """One forward + backward of a form; returns the output and the gradients of x and the four
    weights."""
    ts = [t.detach().clone().requires_grad_() for t in (x, wr, wup, wgate, wdown)]
    out = form(*ts, k, n_clusters)
    out.backward(dy)
    return out.detach(), [t.grad for t in ts]
