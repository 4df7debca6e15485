"""Shortlist output head (rte/output.py:13-136): per token, a fixed-width candidate list
[target, members of the top vocab clusters, hard negatives, random negatives, fillers],
first occurrences kept in order, logits only over the shortlist, target at position 0.

The cluster router runs on the MFMA GEMM, the cluster top-k on the routing kernel, the
candidate build + dedupe, the shortlist logits and their cross-entropy on the shortlist
kernels.  The random negatives stay a torch draw from a device generator seeded with
``seed`` (rte/output.py:86-94), so they follow the same RNG stream as the reference."""

from __future__ import annotations

from dataclasses import dataclass

import torch
from torch import nn

from rte_amd.config import OutputConfig
from rte_amd.kernels import hip_ops


@dataclass(slots=True)
class ShortlistResult:
    loss_per_sample: torch.Tensor
    logits: torch.Tensor
    shortlist: torch.Tensor
    target_positions: torch.Tensor
    cluster_logits: torch.Tensor
    duplicate_count: torch.Tensor
    token_loss: torch.Tensor | None = None


class ShortlistHead(nn.Module):
    def __init__(self, d_model: int, vocab_size: int, config: OutputConfig):
        super().__init__()
        self.d_model = d_model
        self.vocab_size = vocab_size
        self.config = config
        self.cluster_router = nn.Linear(d_model, config.num_clusters, bias=False)
        cluster_ids = torch.arange(vocab_size, dtype=torch.long) % config.num_clusters
        self.register_buffer("cluster_ids", cluster_ids, persistent=False)
        per = (vocab_size + config.num_clusters - 1) // config.num_clusters
        members = torch.zeros(config.num_clusters, per, dtype=torch.long)
        counts = torch.zeros(config.num_clusters, dtype=torch.long)
        for tok in range(vocab_size):  # token t belongs to cluster t mod C (rte/output.py:30-40)
            c = tok % config.num_clusters
            members[c, counts[c]] = tok
            counts[c] += 1
        self.register_buffer("cluster_members", members, persistent=False)
        self.register_buffer("cluster_counts", counts, persistent=False)
        self.register_buffer("hard_negative_cache", torch.arange(config.hard_negatives) % vocab_size, persistent=False)
        self.register_buffer("shortlist_filler", torch.arange(config.shortlist_max_tokens) % vocab_size, persistent=False)

    def cluster_logits(self, hidden: torch.Tensor) -> torch.Tensor:
        """hidden @ W_router^T in fp32 on the MFMA GEMM (rte/output.py:81).  No loss reads the
        cluster logits in the reference, so they carry no gradient here either."""
        w = self.cluster_router.weight.detach()
        C = w.shape[0]
        pad = (-C) % 8
        if pad:
            w = torch.cat([w, w.new_zeros(pad, w.shape[1])])
        with torch.no_grad():
            lg = hip_ops.linear(hidden.detach(), w, out_f32=True)
        return lg[..., :C].contiguous() if pad else lg

    def build_shortlist(self, hidden, targets, *, seed: int, random_negs=None):
        """(shortlist int64 [b, s, L], target positions (zeros), cluster logits, duplicate count)."""
        sl, cl, dup = self._build(hidden, targets, seed, random_negs)
        return sl.long(), torch.zeros_like(targets, dtype=torch.long), cl, dup.sum().float()

    def random_negatives(self, b: int, s: int, seed: int, device) -> torch.Tensor:
        """The seeded random negatives of rte/output.py:86-94 (drawable ahead of a captured step)."""
        gen = torch.Generator(device=device)
        gen.manual_seed(seed)
        return torch.randint(0, self.vocab_size, (b, s, self.config.random_negatives), device=device, generator=gen)

    def _build(self, hidden, targets, seed: int, random_negs=None):
        b, s, _ = hidden.shape
        cl = self.cluster_logits(hidden)
        k = min(self.config.shortlist_top_clusters, self.config.num_clusters)
        top, _ = hip_ops.route_topk(cl.reshape(b * s, -1), k)
        rnd = random_negs if random_negs is not None else self.random_negatives(b, s, seed, hidden.device)
        sl, dup = hip_ops.shortlist_build(targets, top, self.cluster_members, self.config.hard_negatives, rnd,
                                          self.config.shortlist_max_tokens, self.vocab_size)
        return sl, cl, dup

    def loss(self, hidden, targets, vocab_weight, *, seed: int, random_negs=None) -> ShortlistResult:
        """Per-sample CE over the shortlist logits (rte/output.py:112-136)."""
        sl, cl, dup = self._build(hidden, targets, seed, random_negs)
        logits, tok = hip_ops.shortlist_ce(hidden, vocab_weight, sl)
        return ShortlistResult(tok.sum(dim=-1), logits, sl.long(), torch.zeros_like(targets, dtype=torch.long), cl,
                               dup.sum().float(), tok)
