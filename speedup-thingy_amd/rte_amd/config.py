"""Experiment configuration (dataclasses + YAML), key-compatible with the reference.

Field names, defaults and validation follow rte/config.py:11-449 so the
reference's YAML presets load unchanged; unknown keys are rejected
(rte/config.py:385-397).  Added, MI355X-build-specific model keys:
  ffn_kind        "dense" (reference DenseSwiGLU) | "cluster_pool" (routed top-k cluster pool)
  ffn_clusters    number of clusters of the routed pool (d_ff must divide evenly)
  ffn_top_k       clusters per token
"""

from __future__ import annotations

from dataclasses import asdict, dataclass, field, fields, is_dataclass
from pathlib import Path
from typing import Any, Literal

import yaml


@dataclass(slots=True)
class ModelConfig:
    topology: Literal["dense", "recursive"]
    vocab_size: int
    d_model: int
    n_heads: int
    d_ff: int
    n_dense_layers: int
    n_prelude: int
    n_coda: int
    t_max: int
    depth_choices: list[int]
    attn_banks: int
    ffn_banks: int
    head_groups: int
    ffn_groups: int
    active_head_groups: int
    active_ffn_groups: int
    recipe_count: int
    tie_embeddings: bool = True
    use_rope: bool = True
    use_recursive_input_skip: bool = True
    use_global_lowrank_corrector: bool = False
    global_corrector_rank: int = 16
    fairness_tolerance: float = 0.01
    macro_type: Literal["bounded_residual", "v2_delta_radius"] = "bounded_residual"
    macro_rank: int = 32
    macro_update_scale: float = 0.05
    macro_hidden_mult: int = 1
    macro_use_gated_update: bool = False
    macro_update_scale_init: float = 1.0
    macro_include_delta_to_h0: bool = False
    macro_use_delta_to_h0: bool = False
    macro_use_depth_embedding: bool = False
    macro_use_recipe_embedding: bool = False
    macro_radius_init_from_teacher: bool = False
    macro_radius_clamp_mult_min: float = 0.25
    macro_radius_clamp_mult_max: float = 4.0
    macro_decomposition: Literal["direct", "binary", "greedy", "consistency_tree"] = "direct"
    router_hidden: int | None = None
    ffn_kind: Literal["dense", "cluster_pool"] = "dense"
    ffn_clusters: int = 64
    ffn_top_k: int = 8

    def __post_init__(self) -> None:
        if self.d_model % self.n_heads != 0:
            raise ValueError("d_model must be divisible by n_heads")
        if self.n_heads % self.head_groups != 0:
            raise ValueError("n_heads must be divisible by head_groups")
        if self.d_ff % self.ffn_groups != 0:
            raise ValueError("d_ff must be divisible by ffn_groups")
        if self.active_head_groups < 1 or self.active_head_groups > self.head_groups:
            raise ValueError("active_head_groups must be in [1, head_groups]")
        if self.active_ffn_groups < 1 or self.active_ffn_groups > self.ffn_groups:
            raise ValueError("active_ffn_groups must be in [1, ffn_groups]")
        if self.recipe_count < 2:
            raise ValueError("recipe_count must include sparse recipes plus dense fallback")
        if self.t_max not in self.depth_choices:
            raise ValueError("t_max must be present in depth_choices")
        if sorted(self.depth_choices) != self.depth_choices:
            raise ValueError("depth_choices must be sorted ascending")
        if self.macro_rank < 1:
            raise ValueError("macro_rank must be positive")
        if self.global_corrector_rank < 1:
            raise ValueError("global_corrector_rank must be positive")
        if self.macro_hidden_mult < 1:
            raise ValueError("macro_hidden_mult must be positive")
        if self.macro_update_scale_init < 0:
            raise ValueError("macro_update_scale_init must be non-negative")
        if self.macro_radius_clamp_mult_min < 0:
            raise ValueError("macro_radius_clamp_mult_min must be non-negative")
        if self.macro_radius_clamp_mult_max <= 0:
            raise ValueError("macro_radius_clamp_mult_max must be positive")
        if self.macro_radius_clamp_mult_max < self.macro_radius_clamp_mult_min:
            raise ValueError("macro_radius_clamp_mult_max must be >= macro_radius_clamp_mult_min")
        if self.ffn_kind == "cluster_pool":
            if self.d_ff % self.ffn_clusters != 0:
                raise ValueError("d_ff must be divisible by ffn_clusters")
            if (self.d_ff // self.ffn_clusters) % 32 != 0:
                raise ValueError("neurons per cluster must be a multiple of 32 (MFMA tile)")
            if not 1 <= self.ffn_top_k <= min(16, self.ffn_clusters):
                raise ValueError("ffn_top_k must be in [1, min(16, ffn_clusters)]")


@dataclass(slots=True)
class TrainingConfig:
    mode: Literal[
        "dense_exact",
        "recursive_exact",
        "recursive_deferred_grouped_exact",
        "recursive_exact_route_em",
        "recursive_exact_factorized_soft",
        "recursive_exact_dense_hidden_distill",
        "recursive_sandwich_supernet",
        "recursive_macro",
        "recursive_macro_shortlist",
        "recursive_macro_distill_only",
        "recursive_macro_lm_aligned",
        "recursive_macro_shadow_coda",
    ]
    loss_normalization: Literal["token_mean", "sample_sum"] = "token_mean"
    optimizer: Literal["adamw"] = "adamw"
    lr: float = 3e-4
    lr_base: float | None = None
    lr_macro: float | None = None
    lr_coda: float | None = None
    lr_output: float | None = None
    lr_router: float | None = None
    lr_schedule: Literal["constant", "linear_decay_after"] = "constant"
    lr_decay_start_tokens: int | None = None
    lr_decay_end_tokens: int | None = None
    lr_final_scale: float = 1.0
    weight_decay: float = 0.1
    batch_size: int = 4
    seq_len: int = 32
    grad_accum_steps: int = 1
    grad_clip_norm: float | None = None
    seed: int = 1337
    precision: Literal["fp32", "bf16"] = "fp32"
    audit_p_min: float = 0.05
    audit_p_max: float = 0.25
    audit_alpha: float = 0.08
    audit_beta: float = 0.08
    audit_gamma: float = 0.08
    audit_sampler: Literal["bernoulli", "fixed_count"] = "bernoulli"
    audit_fixed_count: int | None = None
    audit_cap: int | None = None
    audit_fixed_count_per_batch: int | None = None
    audit_mode: Literal["metric_only", "gradient_corrected", "distill_only"] = "gradient_corrected"
    audit_residual_clip: float | None = None
    audit_gradient_correction: bool = True
    audit_schedule_enabled: bool = False
    audit_schedule_min_count: int | None = None
    audit_schedule_gap_threshold: float = 0.05
    audit_schedule_nll_gap_threshold: float = 0.05
    audit_schedule_hidden_cosine_threshold: float = 0.98
    audit_schedule_residual_var_threshold: float = 1.0
    audit_schedule_delta_rms_ratio_min: float = 0.9
    audit_schedule_delta_rms_ratio_max: float = 1.1
    audit_schedule_hidden_mse_threshold: float = 1.0
    audit_schedule_macro_norm_threshold: float | None = None
    audit_schedule_macro_norm_threshold_mult: float = 2.0
    audit_schedule_require_negative_mse_slope: bool = True
    audit_schedule_require_negative_norm_slope: bool = True
    target_speedup_vs_dense: float | None = None
    max_active_param_equiv_per_token: float | None = None
    max_hotpath_flops_per_token: float | None = None
    lambda_depth: float = 1e-4
    lambda_load: float = 1e-2
    lambda_cover: float = 1e-2
    lambda_router: float = 1.0
    lambda_hid: float = 1e-2
    lambda_cos: float = 1e-2
    lambda_kl: float = 1e-2
    lambda_hidden_mse: float | None = None
    lambda_hidden_cosine: float | None = None
    lambda_logit_kl: float | None = None
    lambda_dense_hidden: float = 1.0
    lambda_dense_delta: float = 0.5
    lambda_dense_kl: float = 0.25
    lambda_norm: float = 0.05
    lambda_delta_dir: float = 2.0
    lambda_delta_rms: float = 2.0
    lambda_endpoint_normed: float = 1.0
    lambda_endpoint_raw: float = 0.05
    macro_rms_trust_region: bool = False
    macro_rms_clamp_early: bool = False
    macro_rms_clamp_min: float = 0.5
    macro_rms_clamp_max: float = 2.0
    lambda_macro_rms_trust: float = 2.0
    distill_temperature: float = 2.0
    dense_distill_temperature: float = 2.0
    dense_hidden_layer_map: list[int] | None = None
    lambda_cons: float = 1e-3
    coverage_min: float = 0.01
    coverage_beta: float = 0.98
    fixed_recipe: int | None = None
    fixed_recipe_schedule: list[int] | None = None
    fixed_depth: int | None = None
    route_em_candidates: int = 4
    route_em_allow_dense_fallback: bool = False
    route_em_proposal: Literal["router", "random"] = "router"
    factorized_route_top_k: int = 4
    factorized_route_temperature: float = 1.0
    sandwich_random_paths: int = 2
    sandwich_temperature: float = 2.0
    lambda_sandwich_rand_ce: float = 0.5
    lambda_sandwich_kd: float = 1.0
    lambda_sandwich_rand_kd: float = 0.5
    lambda_sandwich_hidden: float = 0.1
    disable_router_aux: bool = False
    debug_force_full_output: bool = False
    coda_warmup_steps: int = 0
    aligned_lm_teacher_checkpoint: str | None = None
    aligned_lm_freeze_teacher: bool = True
    aligned_lm_phase_a_train: list[str] = field(default_factory=lambda: ["macro"])
    aligned_lm_phase_b_train: list[str] = field(default_factory=lambda: ["macro", "coda"])
    aligned_lm_phase_c_train: list[str] = field(default_factory=lambda: ["macro", "coda", "output"])
    unfreeze_prelude_core_after_gate: bool = True
    log_every: int = 1
    compile_model: bool = False
    compile_mode: Literal["default", "reduce-overhead", "max-autotune"] = "reduce-overhead"
    fused_optimizer: bool = True
    foreach_optimizer: bool = True
    allow_tf32: bool = True
    strict_cuda: bool = False
    require_triton: bool = False
    require_flash_attention: bool = True

    def __post_init__(self) -> None:
        if self.audit_fixed_count is not None:
            self.audit_fixed_count_per_batch = self.audit_fixed_count
        if self.audit_sampler == "fixed_count" and self.audit_fixed_count_per_batch is None:
            raise ValueError("audit_sampler='fixed_count' requires audit_fixed_count")
        if self.audit_fixed_count_per_batch is not None:
            self.audit_sampler = "fixed_count"
        if self.grad_accum_steps < 1:
            raise ValueError("grad_accum_steps must be >= 1")
        if self.lr_final_scale <= 0:
            raise ValueError("lr_final_scale must be positive")
        if self.lr_schedule == "linear_decay_after":
            if self.lr_decay_start_tokens is None or self.lr_decay_end_tokens is None:
                raise ValueError("linear_decay_after requires lr_decay_start_tokens and lr_decay_end_tokens")
            if self.lr_decay_end_tokens <= self.lr_decay_start_tokens:
                raise ValueError("lr_decay_end_tokens must be greater than lr_decay_start_tokens")
        if self.audit_cap is not None and self.audit_cap < 0:
            raise ValueError("audit_cap must be non-negative when provided")
        if self.audit_fixed_count_per_batch is not None:
            if self.audit_fixed_count_per_batch < 0:
                raise ValueError("audit_fixed_count_per_batch must be non-negative when provided")
            if self.audit_fixed_count_per_batch > self.batch_size:
                raise ValueError("audit_fixed_count_per_batch must be <= batch_size")
        if self.audit_mode == "gradient_corrected" and not self.audit_gradient_correction and self.audit_p_max > 0:
            raise ValueError(
                "audit_mode='gradient_corrected' requires audit_gradient_correction=true when audits are enabled"
            )
        if self.distill_temperature <= 0:
            raise ValueError("distill_temperature must be positive")

    @property
    def effective_lr_base(self) -> float:
        return self.lr if self.lr_base is None else self.lr_base

    @property
    def effective_lr_macro(self) -> float:
        return self.lr if self.lr_macro is None else self.lr_macro

    @property
    def effective_lr_coda(self) -> float:
        return self.lr if self.lr_coda is None else self.lr_coda

    @property
    def effective_lr_output(self) -> float:
        return self.lr if self.lr_output is None else self.lr_output

    @property
    def effective_lr_router(self) -> float:
        return self.lr if self.lr_router is None else self.lr_router

    @property
    def effective_lambda_hid(self) -> float:
        return self.lambda_hid if self.lambda_hidden_mse is None else self.lambda_hidden_mse

    @property
    def effective_lambda_cos(self) -> float:
        return self.lambda_cos if self.lambda_hidden_cosine is None else self.lambda_hidden_cosine

    @property
    def effective_lambda_kl(self) -> float:
        return self.lambda_kl if self.lambda_logit_kl is None else self.lambda_logit_kl


@dataclass(slots=True)
class OutputConfig:
    mode: Literal["full", "shortlist"] = "full"
    num_clusters: int = 64
    shortlist_top_clusters: int = 2
    shortlist_max_tokens: int = 128
    hard_negatives: int = 32
    random_negatives: int = 32


@dataclass(slots=True)
class DataConfig:
    dataset: Literal["tinystories", "wikitext103", "local", "synthetic"] = "synthetic"
    tokenizer: Literal["gpt2_bpe", "byte"] = "gpt2_bpe"
    vocab_projection: Literal["filter", "modulo"] = "filter"
    projection_lane: Literal["filter", "modulo"] | None = None
    cache_dir: str = ".cache/rte"
    local_text_path: str | None = None
    train_split: str = "train"
    eval_split: str = "validation"
    seed: int | None = None
    train_tokens: int | None = None
    max_tokens: int = 200_000
    eval_tokens: int = 20_000
    synthetic_tokens: int = 20_000

    def __post_init__(self) -> None:
        # rte/config.py:364-369: the projection lane defaults to the vocab projection and must
        # agree with it; train_tokens, when given, is the token budget
        if self.projection_lane is None:
            self.projection_lane = self.vocab_projection
        elif self.projection_lane != self.vocab_projection:
            raise ValueError("data.projection_lane and data.vocab_projection must match")
        if self.train_tokens is not None:
            self.max_tokens = self.train_tokens


@dataclass(slots=True)
class ExperimentConfig:
    model: ModelConfig
    training: TrainingConfig
    output: OutputConfig = field(default_factory=OutputConfig)
    data: DataConfig = field(default_factory=DataConfig)
    run_name: str = "rte-run"
    output_dir: str = "runs"
    allow_unknown_config_keys: bool = False


_ROOT_KEYS = ("model", "training", "output", "data", "run_name", "output_dir", "allow_unknown_config_keys")


def _known_keys(cls, raw: dict[str, Any], section: str, allow_unknown: bool) -> dict[str, Any]:
    """The keys of `raw` that are fields of `cls`; unknown keys raise unless allow_unknown, in
    which case they are dropped (rte/config.py:385-397)."""
    known = {f.name for f in fields(cls)}
    unknown = sorted(set(raw) - known)
    if unknown and not allow_unknown:
        raise ValueError("unknown config key(s): " + ", ".join(f"{section}.{k}" for k in unknown))
    return {k: v for k, v in raw.items() if k in known}


def config_from_dict(raw: dict[str, Any]) -> ExperimentConfig:
    """ExperimentConfig of a parsed YAML mapping.  With allow_unknown_config_keys: true at the
    top level, keys this build does not know are ignored instead of rejected (rte/config.py:400-449)."""
    allow = bool(raw.get("allow_unknown_config_keys", False))
    unknown = sorted(set(raw) - set(_ROOT_KEYS))
    if unknown and not allow:
        raise ValueError("unknown config key(s): " + ", ".join(unknown))
    sections = {name: _known_keys(cls, raw.get(name) or {}, name, allow)
                for name, cls in (("model", ModelConfig), ("training", TrainingConfig), ("output", OutputConfig),
                                  ("data", DataConfig))}
    return ExperimentConfig(
        model=ModelConfig(**sections["model"]),
        training=TrainingConfig(**sections["training"]),
        output=OutputConfig(**sections["output"]),
        data=DataConfig(**sections["data"]),
        run_name=raw.get("run_name", "rte-run"),
        output_dir=raw.get("output_dir", "runs"),
        allow_unknown_config_keys=allow,
    )


def load_config(path: str | Path) -> ExperimentConfig:
    with open(path, "r", encoding="utf-8") as fh:
        raw = yaml.safe_load(fh) or {}
    return config_from_dict(raw)


def config_to_dict(cfg: Any) -> Any:
    return asdict(cfg) if is_dataclass(cfg) else cfg
