"""Per-sample recipe / depth router on the pooled prelude state (rte/routing.py:47-188).

The recipe and depth heads run as one HIP operator (hip_ops.router: a pooling launch, the two
layer-1 GEMMs with the bias in their epilogue and one launch for layer 2 and every head field;
backward in two launches plus the layer-1 GEMMs).  The four factor heads (attention bank, FFN
bank, head slot, FFN slot per recursive pass, rte/routing.py:94-101) run on the bias-fused GEMM
when one of their fields is first read, since the accelerated modes' losses never read them
(their values are the reference's whenever they are read).
"""

from __future__ import annotations

from dataclasses import dataclass

import torch
import torch.nn.functional as F
from torch import nn

from rte_amd.config import ModelConfig
from rte_amd.kernels import hip_ops
from rte_amd.recipes import factor_slot_counts


@dataclass
class RouterOutput:
    recipe_logits: torch.Tensor
    recipe_probs: torch.Tensor
    recipe_id: torch.Tensor
    recipe_onehot_st: torch.Tensor
    depth_logits: torch.Tensor
    depth_probs: torch.Tensor
    depth_id: torch.Tensor
    depth: torch.Tensor
    depth_onehot_st: torch.Tensor
    router_entropy: torch.Tensor
    recipe_entropy: torch.Tensor
    depth_entropy: torch.Tensor
    expected_depth: torch.Tensor
    recipe_logits_by_pass: torch.Tensor | None = None
    recipe_probs_by_pass: torch.Tensor | None = None
    recipe_id_by_pass: torch.Tensor | None = None
    recipe_onehot_st_by_pass: torch.Tensor | None = None
    fixed_depth_value: int | None = None  # every sample's depth when the router ran with a fixed depth
    _factor_fn: object = None
    _factor: dict | None = None
    _factor_src: tuple | None = None  # (router, h0, inv_t): the factor heads' inputs

    def factor(self, name: str):
        """A factor-head field (computed once, on first use)."""
        if self._factor is None:
            if self._factor_src is not None:
                router, h0, inv_t = self._factor_src
                self._factor = router._factor_heads(h0.mean(dim=1), inv_t)
            else:
                self._factor = self._factor_fn() if self._factor_fn is not None else {}
        return self._factor.get(name)

    attn_bank_logits_by_pass = property(lambda self: self.factor("attn_bank_logits_by_pass"))
    attn_bank_probs_by_pass = property(lambda self: self.factor("attn_bank_probs_by_pass"))
    attn_bank_id_by_pass = property(lambda self: self.factor("attn_bank_id_by_pass"))
    ffn_bank_logits_by_pass = property(lambda self: self.factor("ffn_bank_logits_by_pass"))
    ffn_bank_probs_by_pass = property(lambda self: self.factor("ffn_bank_probs_by_pass"))
    ffn_bank_id_by_pass = property(lambda self: self.factor("ffn_bank_id_by_pass"))
    head_slot_logits_by_pass = property(lambda self: self.factor("head_slot_logits_by_pass"))
    head_slot_probs_by_pass = property(lambda self: self.factor("head_slot_probs_by_pass"))
    head_slot_id_by_pass = property(lambda self: self.factor("head_slot_id_by_pass"))
    ffn_slot_logits_by_pass = property(lambda self: self.factor("ffn_slot_logits_by_pass"))
    ffn_slot_probs_by_pass = property(lambda self: self.factor("ffn_slot_probs_by_pass"))
    ffn_slot_id_by_pass = property(lambda self: self.factor("ffn_slot_id_by_pass"))
    factor_entropy = property(lambda self: self.factor("factor_entropy"))

    def subset(self, mask: torch.Tensor) -> "RouterSubset":
        """The decisions of rows `mask` (bool mask or indices); each field is indexed when first
        read, so an exact replay that reads only the recipe ids and depths launches no index
        kernels for the other fields."""
        return RouterSubset(self, mask)


class RouterSubset:
    """Rows of a RouterOutput with the same field names, each indexed at its first read."""

    def __init__(self, parent, mask: torch.Tensor):
        object.__setattr__(self, "_parent", parent)
        object.__setattr__(self, "_mask", mask)

    def __getattr__(self, name: str):
        if name.startswith("_"):
            raise AttributeError(name)
        v = getattr(self._parent, name)
        if isinstance(v, torch.Tensor):
            m = self._mask
            # index rows: index_select (the generic advanced-indexing kernel is several times slower)
            v = v.index_select(0, m) if m.dtype == torch.long and m.dim() == 1 else v[m]
        object.__setattr__(self, name, v)
        return v

    def subset(self, mask: torch.Tensor) -> "RouterSubset":
        return RouterSubset(self, mask)


def _entropy(p: torch.Tensor) -> torch.Tensor:
    return -(p.clamp_min(1e-9).log() * p).sum(dim=-1)


def _mlp(seq: nn.Sequential, x: torch.Tensor) -> torch.Tensor:
    """Linear -> SiLU -> Linear on the bias-fused HIP GEMM (fp32 output)."""
    a = F.silu(hip_ops.linear_bias(x, seq[0].weight, seq[0].bias))
    return hip_ops.linear_bias(a, seq[2].weight, seq[2].bias)


class Router(nn.Module):
    def __init__(self, config: ModelConfig):
        super().__init__()
        hidden = config.router_hidden or max(32, config.d_model)
        self.config = config
        self.recipe_mlp = nn.Sequential(nn.Linear(config.d_model, hidden), nn.SiLU(), nn.Linear(hidden, config.recipe_count))
        self.pass_recipe_bias = nn.Parameter(torch.zeros(config.t_max, config.recipe_count))
        head_slots, ffn_slots = factor_slot_counts(config)
        self.head_slots, self.ffn_slots = head_slots, ffn_slots
        self.factor_mlp = nn.Sequential(nn.Linear(config.d_model, hidden), nn.SiLU(), nn.Linear(hidden, hidden))
        self.pass_factor_bias = nn.Parameter(torch.zeros(config.t_max, hidden))
        self.attn_bank_head = nn.Linear(hidden, config.attn_banks)
        self.ffn_bank_head = nn.Linear(hidden, config.ffn_banks)
        self.head_slot_head = nn.Linear(hidden, head_slots)
        self.ffn_slot_head = nn.Linear(hidden, ffn_slots)
        self.depth_mlp = nn.Sequential(nn.Linear(config.d_model, hidden), nn.SiLU(), nn.Linear(hidden, len(config.depth_choices)))
        self.register_buffer("depth_values", torch.tensor(config.depth_choices, dtype=torch.long), persistent=False)

    def _factor_heads(self, pooled: torch.Tensor, inv_t: float) -> dict[str, torch.Tensor]:
        """Per-pass factor logits / probs / argmax and the mean factor entropy (rte/routing.py:94-101,
        :114-175)."""
        fh = F.silu(_mlp(self.factor_mlp, pooled).unsqueeze(1) + self.pass_factor_bias.unsqueeze(0))
        out: dict[str, torch.Tensor] = {}
        ent = 0.0
        for name, head in (("attn_bank", self.attn_bank_head), ("ffn_bank", self.ffn_bank_head),
                           ("head_slot", self.head_slot_head), ("ffn_slot", self.ffn_slot_head)):
            logits = hip_ops.linear_bias(fh, head.weight, head.bias) * inv_t
            probs = F.softmax(logits, dim=-1)
            out[f"{name}_logits_by_pass"] = logits
            out[f"{name}_probs_by_pass"] = probs
            out[f"{name}_id_by_pass"] = probs.argmax(dim=-1)
            ent = ent + _entropy(probs)
        out["factor_entropy"] = ent.mean(dim=-1)
        return out

    def forward(self, h0: torch.Tensor, *, fixed_recipe: int | None = None, fixed_depth: int | None = None,
                temperature: float = 1.0) -> RouterOutput:
        """The recipe and depth heads in one HIP operator (hip_ops.router: pooled mean, both MLPs,
        per-pass logits, softmax / argmax / straight-through one-hot / entropies / expected depth)."""
        inv_t = 1.0 / max(temperature, 1e-6)
        depth_idx = None
        if fixed_depth is not None:
            if fixed_depth not in self.config.depth_choices:
                raise ValueError(f"fixed_depth={fixed_depth} is not in depth_choices")
            depth_idx = self.config.depth_choices.index(fixed_depth)
        rm, dm = self.recipe_mlp, self.depth_mlp
        f = hip_ops.router(h0, rm[0].weight, rm[0].bias, rm[2].weight, rm[2].bias, dm[0].weight, dm[0].bias,
                           dm[2].weight, dm[2].bias, self.pass_recipe_bias, self.depth_values, inv_t=inv_t,
                           fixed_recipe=fixed_recipe, fixed_depth=depth_idx)
        return RouterOutput(**f, fixed_depth_value=fixed_depth, _factor_src=(self, h0, inv_t))
