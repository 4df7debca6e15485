"""Static recipe templates (which attention / FFN banks and head / slab groups a
sample's recursive passes touch).  Same template rule and tables as
rte/recipes.py:10-159 — the recipe ids index trained parameters, so they must
match for checkpoints and routing decisions to mean the same thing."""

from __future__ import annotations

from dataclasses import dataclass

import torch

from rte_amd.config import ModelConfig
from rte_amd.kernels import hip_ops


@dataclass(frozen=True, slots=True)
class RecipeSpec:
    recipe_id: int
    attention_banks: tuple[int, ...]
    ffn_banks: tuple[int, ...]
    head_groups: tuple[int, ...]
    ffn_groups: tuple[int, ...]
    dense_fallback: bool = False


def factor_slot_counts(config: ModelConfig) -> tuple[int, int]:
    return (
        max(1, config.head_groups // config.active_head_groups),
        max(1, config.ffn_groups // config.active_ffn_groups),
    )


class RecipeBank:
    """Recipe 0 is the dense fallback (all banks, all groups); recipe r >= 1 walks the
    (bank, slot) grid round-robin (rte/recipes.py:65-100)."""

    def __init__(self, config: ModelConfig):
        self.config = config
        self.usage_ema = torch.zeros(config.recipe_count, dtype=torch.float32)
        cfg = config
        head_slots, ffn_slots = factor_slot_counts(cfg)
        recipes = [
            RecipeSpec(0, tuple(range(cfg.attn_banks)), tuple(range(cfg.ffn_banks)),
                       tuple(range(cfg.head_groups)), tuple(range(cfg.ffn_groups)), True)
        ]
        for idx in range(cfg.recipe_count - 1):
            hs, fs = idx % head_slots, idx % ffn_slots
            ab = (idx // head_slots) % cfg.attn_banks
            fb = (idx // ffn_slots) % cfg.ffn_banks
            heads = tuple((hs * cfg.active_head_groups + j) % cfg.head_groups for j in range(cfg.active_head_groups))
            slabs = tuple((fs * cfg.active_ffn_groups + j) % cfg.ffn_groups for j in range(cfg.active_ffn_groups))
            recipes.append(RecipeSpec(idx + 1, (ab,), (fb,), heads, slabs, False))
        self.recipes = recipes
        self.active_touch_table = torch.tensor([self.active_touches_for_spec(s) for s in recipes], dtype=torch.float32)

    def active_touches_for_spec(self, spec: RecipeSpec) -> float:
        cfg = self.config
        d = cfg.d_model
        attn = len(spec.attention_banks) * 4 * d * d * len(spec.head_groups) / cfg.head_groups
        ffn = len(spec.ffn_banks) * 3 * d * cfg.d_ff * len(spec.ffn_groups) / cfg.ffn_groups
        return float(attn + ffn)

    def get_recipe(self, recipe_id):
        if isinstance(recipe_id, torch.Tensor):
            if recipe_id.ndim == 0:
                return self.recipes[int(recipe_id.item())]
            return [self.recipes[int(x)] for x in recipe_id.detach().cpu().tolist()]
        return self.recipes[int(recipe_id)]

    def update_usage(self, recipe_ids: torch.Tensor, beta: float = 0.98) -> None:
        """usage_ema = beta usage_ema + (1 - beta) bincount(ids) / max(#ids, 1) as one HIP launch
        on the ids' device with no host sync (the reference moves ids to the CPU and bincounts
        there); counts are exact integers."""
        ids = recipe_ids.detach().long().flatten()
        if self.usage_ema.device != ids.device or not self.usage_ema.is_contiguous():
            self.usage_ema = self.usage_ema.to(ids.device).contiguous()
        hip_ops.count_ema(ids, None, self.usage_ema, beta)
