"""Shortlist output head (rte/output.py:13-136): per token, a fixed-width candidate list
[target, members of the top vocab clusters, hard negatives, random negatives, fillers],
first occurrences kept in order, logits only over the shortlist, target at position 0.
Torch ops on the device for now."""

from __future__ import annotations

from dataclasses import dataclass

import torch
import torch.nn.functional as F
from torch import nn

from rte_amd.config import OutputConfig
from rte_amd.kernels import optimized as K


@dataclass(slots=True)
class ShortlistResult:
    loss_per_sample: torch.Tensor
    logits: torch.Tensor
    shortlist: torch.Tensor
    target_positions: torch.Tensor
    cluster_logits: torch.Tensor
    duplicate_count: torch.Tensor


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

    def _dedupe_preserve_first(self, candidates, max_tokens):
        width = candidates.shape[-1]
        flat = candidates.reshape(-1, width).long()
        pos = torch.arange(width, device=candidates.device, dtype=torch.float32).view(1, -1)
        first = torch.full((flat.shape[0], self.vocab_size), float(width + max_tokens), dtype=torch.float32,
                           device=candidates.device)
        first.scatter_reduce_(1, flat, pos.expand_as(flat), reduce="amin", include_self=True)
        duplicate_count = (width - (first < width).sum(dim=-1)).float().sum()
        _, shortlist = first.topk(k=max_tokens, dim=-1, largest=False, sorted=True)
        return shortlist.view(*candidates.shape[:-1], max_tokens).contiguous(), duplicate_count

    def build_shortlist(self, hidden, targets, *, seed: int):
        b, s, _ = hidden.shape
        dev = hidden.device
        cluster_logits = self.cluster_router(hidden)
        top = cluster_logits.topk(k=min(self.config.shortlist_top_clusters, self.config.num_clusters), dim=-1).indices
        L = self.config.shortlist_max_tokens
        gen = torch.Generator(device=dev)
        gen.manual_seed(seed)
        rnd = torch.randint(0, self.vocab_size, (b, s, self.config.random_negatives), device=dev, generator=gen)
        members = self.cluster_members[top].flatten(start_dim=-2)
        hard = self.hard_negative_cache.view(1, 1, -1).expand(b, s, -1)
        filler = self.shortlist_filler.view(1, 1, -1).expand(b, s, -1)
        tfill = (targets.unsqueeze(-1) + torch.arange(2 * L, device=dev).view(1, 1, -1)) % self.vocab_size
        cand = torch.cat([targets.unsqueeze(-1), members, hard, rnd, filler, tfill], dim=-1)
        shortlist, dup = self._dedupe_preserve_first(cand, L)
        return shortlist, torch.zeros(b, s, dtype=torch.long, device=dev), cluster_logits, dup

    def loss(self, hidden, targets, vocab_weight, *, seed: int) -> ShortlistResult:
        shortlist, tpos, cl, dup = self.build_shortlist(hidden, targets, seed=seed)
        logits = K.k_logits_shortlist(hidden, vocab_weight, shortlist)
        tok = F.cross_entropy(logits.float().flatten(0, -2), tpos.flatten(), reduction="none").view_as(targets)
        return ShortlistResult(tok.sum(dim=-1), logits, shortlist, tpos, cl, dup)
