"""Fairness accounting and the hot-path budget (rte/metrics.py:12-94, :127-181).

Parameter counts and the active-parameter / FLOP estimates follow the reference's formulas
term for term, so a budget set in a reference config (target_speedup_vs_dense,
max_active_param_equiv_per_token, max_hotpath_flops_per_token) admits or refuses the same
models here.  The one extension is the routed cluster-pool FFN of this build
(ffn_kind="cluster_pool"): its blocks count the router matrix in their parameters, and a
token touches only its top-k pools, so its active FFN parameters are 3 d (k d_ff / C) plus
the router's d C.
"""

from __future__ import annotations

from dataclasses import asdict, dataclass

import torch

from rte_amd.config import ModelConfig


def dense_block_param_count(config: ModelConfig) -> int:
    """Attention 4 d^2, SwiGLU 3 d d_ff and four d-vectors (rte/metrics.py:12-14); a routed
    cluster-pool block adds its router [C, d]."""
    d = config.d_model
    count = 4 * d * d + 3 * d * config.d_ff + 4 * d
    if config.ffn_kind == "cluster_pool":
        count += d * config.ffn_clusters
    return count


def active_block_param_count(config: ModelConfig) -> int:
    """Parameters one token touches in a prelude / coda block: all of them for the dense FFN
    (rte/metrics.py:86); for the routed pool, k of the C pools plus the router."""
    if config.ffn_kind != "cluster_pool":
        return dense_block_param_count(config)
    d = config.d_model
    per_token_ff = config.ffn_top_k * (config.d_ff // config.ffn_clusters)
    return 4 * d * d + 3 * d * per_token_ff + 4 * d + d * config.ffn_clusters


def dense_param_count(config: ModelConfig) -> int:
    embeddings = config.vocab_size * config.d_model
    blocks = config.n_dense_layers * dense_block_param_count(config)
    untied = 0 if config.tie_embeddings else config.vocab_size * config.d_model
    return embeddings + blocks + config.d_model + untied


def recursive_param_count(config: ModelConfig) -> int:
    """rte/metrics.py:25-41."""
    d = config.d_model
    hidden = config.router_hidden or max(32, d)
    embeddings = config.vocab_size * d
    dense_blocks = (config.n_prelude + config.n_coda) * dense_block_param_count(config)
    core = config.attn_banks * 4 * d * d + config.ffn_banks * 3 * d * config.d_ff
    if config.use_global_lowrank_corrector:
        r = config.global_corrector_rank
        core += 3 * d + config.t_max * r + 3 * d * r + config.t_max * r + config.t_max
    router = 2 * (d * hidden + hidden)
    macro = config.recipe_count * len(config.depth_choices) * macro_operator_param_count(config)
    untied = 0 if config.tie_embeddings else config.vocab_size * d
    return embeddings + dense_blocks + core + router + macro + d + untied


def macro_operator_param_count(config: ModelConfig) -> int:
    d = config.d_model
    return d + 3 * d * config.macro_rank + config.macro_rank * d + d


def dense_aligned_param_count(config: ModelConfig) -> int:
    """Parameters of the dense model with this config's sizes (rte/metrics.py:75-76)."""
    return dense_param_count(ModelConfig(**{**asdict(config), "topology": "dense"}))


def estimate_hot_active_param_equiv_per_token(config: ModelConfig, *, shortlist_size=None,
                                              include_output: bool) -> float:
    """Prelude + coda blocks, one macro operator and (optionally) the output head over the
    vocabulary or the shortlist (rte/metrics.py:79-90)."""
    active = (config.n_prelude + config.n_coda) * active_block_param_count(config)
    active += macro_operator_param_count(config)
    if include_output:
        size = config.vocab_size if shortlist_size is None else float(shortlist_size)
        active += size * config.d_model
    return float(active)


def estimate_hot_flops_per_token(active_param_equiv_per_token: float) -> float:
    return 2.0 * active_param_equiv_per_token


def active_parameter_touches(config: ModelConfig, recipe_bank, recipe_ids: torch.Tensor) -> torch.Tensor:
    del config
    return recipe_bank.active_touch_table.to(recipe_ids.device)[recipe_ids]


def hot_budget(config: ModelConfig, training, *, shortlist_size=None, include_output: bool = True) -> dict:
    """The budget check of rte/training.py:707-740: RuntimeError when the hot path's active
    parameters exceed max_active_param_equiv_per_token or dense / target_speedup_vs_dense (the
    smaller), or its FLOPs exceed max_hotpath_flops_per_token; otherwise the budget metrics."""
    active = estimate_hot_active_param_equiv_per_token(config, shortlist_size=shortlist_size,
                                                       include_output=include_output)
    flops = estimate_hot_flops_per_token(active)
    limit = training.max_active_param_equiv_per_token
    if training.target_speedup_vs_dense is not None:
        target = dense_aligned_param_count(config) / training.target_speedup_vs_dense
        limit = target if limit is None else min(limit, target)
    if limit is not None and active > limit:
        raise RuntimeError(f"recursive hot path exceeds active parameter budget: {active:.1f} > {limit:.1f}")
    if training.max_hotpath_flops_per_token is not None and flops > training.max_hotpath_flops_per_token:
        raise RuntimeError("recursive hot path exceeds FLOPs/token budget: "
                           f"{flops:.1f} > {training.max_hotpath_flops_per_token:.1f}")
    return {"active_param_equiv_per_token": active, "hotpath_flops_per_token_est": flops,
            "active_param_budget": limit if limit is not None else 0.0}


@dataclass(slots=True)
class FairnessReport:
    dense_params: int
    recursive_params: int
    relative_delta: float
    pass_param_count: bool
    same_tokenizer: bool
    same_data: bool
    same_seq_len: bool
    same_optimizer: bool
    same_objective: bool
    exact_path_available: bool

    @property
    def passed(self) -> bool:
        return all([self.pass_param_count, self.same_tokenizer, self.same_data, self.same_seq_len,
                    self.same_optimizer, self.same_objective, self.exact_path_available])


def build_fairness_report(dense_cfg: ModelConfig, rec_cfg: ModelConfig, *, tolerance: float,
                          same_tokenizer: bool = True, same_data: bool = True, same_seq_len: bool = True,
                          same_optimizer: bool = True, same_objective: bool = True,
                          exact_path_available: bool = True) -> FairnessReport:
    """Dense vs recursive parameter parity within `tolerance` plus the equal-setup flags
    (rte/metrics.py:127-181)."""
    dense = dense_param_count(dense_cfg)
    rec = recursive_param_count(rec_cfg)
    rel = abs(rec - dense) / max(dense, 1)
    return FairnessReport(dense, rec, rel, rel <= tolerance, same_tokenizer, same_data, same_seq_len,
                          same_optimizer, same_objective, exact_path_available)


def solve_banks_for_fairness(config: ModelConfig, *, max_banks: int = 256) -> tuple[int, int, float]:
    """(attn_banks, ffn_banks, relative delta) whose recursive model is closest in parameters to the
    dense model (rte/metrics.py:44-66); the count is linear in both bank numbers, so each
    attention bank count is paired with the two nearest ffn bank counts instead of a full scan."""
    target = dense_param_count(config)
    base = recursive_param_count(ModelConfig(**{**asdict(config), "attn_banks": 1, "ffn_banks": 1}))
    d = config.d_model
    per_attn, per_ffn = 4 * d * d, 3 * d * config.d_ff
    best = None
    for a in range(1, max_banks + 1):
        rest = target - (base + (a - 1) * per_attn)
        guess = 1 + rest / per_ffn
        for f in {max(1, min(max_banks, int(guess))), max(1, min(max_banks, int(guess) + 1)), 1, max_banks}:
            rel = abs(base + (a - 1) * per_attn + (f - 1) * per_ffn - target) / max(target, 1)
            if best is None or rel < best[2] or (rel == best[2] and (a, f) < best[:2]):
                best = (a, f, rel)
    return best
