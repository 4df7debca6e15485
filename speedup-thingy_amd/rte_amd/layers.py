"""Model building blocks of the recursive_macro path (rte/layers.py:26-951).

Hot modules run on the HIP kernels (rte_amd.kernels.hip_ops):
  RMSNorm                 fused norm fwd/bwd
  DenseCausalSelfAttention  fused QKV GEMM + RoPE epilogue, SDPA core, O-proj GEMM + residual
  DenseSwiGLU             SwiGLU fused into the up/gate GEMM epilogue (fwd) and dZ GEMM (bwd)
  ClusterPoolSwiGLU       routed top-k cluster-pool SwiGLU (route, pack, grouped GEMMs, combine)
  BankedAttention         per-bank QKV+RoPE / SDPA / O-proj with recipe head masks on V
  BankedSwiGLU            grouped pool kernel over (bank, slab) clusters with recipe routes
The banked recursive core keeps the reference's parameter names and shapes, so state
dicts are interchangeable; its recipe selection is device-side table lookups.
"""

from __future__ import annotations

import math
import time

import torch
import torch.nn.functional as F
from torch import nn

from rte_amd.config import ModelConfig
from rte_amd.kernels import hip_ops
from rte_amd.kernels import optimized as K
from rte_amd.recipes import RecipeBank, RecipeSpec


class RMSNorm(nn.Module):
    def __init__(self, dim: int, eps: float = 1e-5):
        super().__init__()
        self.weight = nn.Parameter(torch.ones(dim))
        self.eps = eps

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        # bf16 output for the bf16 GEMMs that consume it (the reference's autocast casts there);
        # the dtype-preserving boundary symbol is K.k_fused_rmsnorm
        return hip_ops.rmsnorm(x, self.weight, self.eps)


class Embedding(nn.Embedding):
    """nn.Embedding (same parameter and state-dict key) whose backward is the deterministic
    segmented row reduction instead of a sort + atomic scatter."""

    def forward(self, ids: torch.Tensor) -> torch.Tensor:
        return hip_ops.embedding(self.weight, ids)


class RotaryEmbedding(nn.Module):
    """cos/sin tables [max_seq_len, dim] with frequencies repeated per interleaved pair
    (rte/layers.py:36-44)."""

    def __init__(self, dim: int, max_seq_len: int = 8192, base: float = 10_000.0):
        super().__init__()
        inv_freq = 1.0 / (base ** (torch.arange(0, dim, 2).float() / dim))
        t = torch.arange(max_seq_len, dtype=torch.float32)
        emb = torch.repeat_interleave(torch.outer(t, inv_freq), 2, dim=-1)
        self.register_buffer("cos", emb.cos(), persistent=False)
        self.register_buffer("sin", emb.sin(), persistent=False)

    def forward(self, q, k):
        s = q.shape[-2]
        return K.k_rope_apply(q, k, self.cos[:s].to(q.dtype), self.sin[:s].to(q.dtype))


class DenseCausalSelfAttention(nn.Module):
    def __init__(self, config: ModelConfig):
        super().__init__()
        self.config = config
        d = config.d_model
        self.n_heads = config.n_heads
        self.head_dim = d // config.n_heads
        self.wqkv = nn.Linear(d, 3 * d, bias=False)
        self.wo = nn.Linear(d, d, bias=False)
        self.rope = RotaryEmbedding(self.head_dim) if config.use_rope else None

    def forward(self, x: torch.Tensor, resid: torch.Tensor | None = None) -> torch.Tensor:
        """Returns resid + Wo(attention(x)) in fp32 (resid optional)."""
        if self.rope is not None:
            cos, sin = self.rope.cos, self.rope.sin
        else:
            cos = torch.ones_like(self.wqkv.weight[:1, : self.head_dim].float()).expand(x.shape[1], -1)
            sin = torch.zeros_like(cos)
        # QKV + RoPE + causal attention as one node: its backward hands the QKV GEMMs their
        # packed, rotated-back input gradient directly (k_flash_causal_dense's math)
        y = hip_ops.qkv_rope_attention(x, self.wqkv.weight, cos, sin, self.n_heads)
        return hip_ops.attn_out_proj(y, self.wo.weight, resid)


class DenseSwiGLU(nn.Module):
    """wug = nn.Linear(d, 2F) with rows [up ; gate], wd = nn.Linear(F, d) (rte/layers.py:78-87)."""

    def __init__(self, config: ModelConfig):
        super().__init__()
        d = config.d_model
        self.wug = nn.Linear(d, 2 * config.d_ff, bias=False)
        self.wd = nn.Linear(config.d_ff, d, bias=False)

    def forward(self, x: torch.Tensor, resid: torch.Tensor | None = None) -> torch.Tensor:
        return hip_ops.dense_swiglu(x, self.wug.weight, self.wd.weight, resid)


class ClusterPoolSwiGLU(nn.Module):
    """Routed cluster-pool SwiGLU: d_ff neurons in `ffn_clusters` contiguous pools, each token
    routed to its top-`ffn_top_k` pools by logits x @ Wr^T, pool outputs combined with softmax
    weights over the selected logits.  Dense parameters (wug, wd) stay the source of truth as in
    StaticClusterPoolSwiGLU (rte/layers.py:119-220)."""

    def __init__(self, config: ModelConfig):
        super().__init__()
        d = config.d_model
        self.n_clusters = config.ffn_clusters
        self.top_k = config.ffn_top_k
        self.router = nn.Linear(d, config.ffn_clusters, bias=False)
        self.wug = nn.Linear(d, 2 * config.d_ff, bias=False)
        self.wd = nn.Linear(config.d_ff, d, bias=False)
        self.last_ids: torch.Tensor | None = None
        self.last_weights: torch.Tensor | None = None

    def forward(self, x: torch.Tensor, resid: torch.Tensor | None = None) -> torch.Tensor:
        out, ids, w = hip_ops.routed_cluster_pool_swiglu(
            x, self.router.weight, self.wug.weight, self.wd.weight, self.top_k, resid=resid
        )
        self.last_ids, self.last_weights = ids, w
        return out


class PackedDenseSwiGLU(nn.Module):
    """Dense SwiGLU with row-oriented W_down (rte/layers.py:90-116): wug [2F, d], wdown_rows [F, d];
    the flag use_triton_swiglu_backward is kept for API parity (both settings run the fused
    HIP SwiGLU)."""

    def __init__(self, dense: DenseSwiGLU):
        super().__init__()
        d_model, d_ff = dense.wug.in_features, dense.wd.in_features
        self.wug = nn.Linear(d_model, 2 * d_ff, bias=False)
        self.wdown_rows = nn.Parameter(torch.empty(d_ff, d_model))
        self.use_triton_swiglu_backward = False
        with torch.no_grad():
            self.wug.weight.copy_(dense.wug.weight.detach())
            self.wdown_rows.copy_(dense.wd.weight.detach().t().contiguous())

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        flat = x.reshape(-1, x.shape[-1])
        out = hip_ops.dense_swiglu(flat, self.wug.weight, self.wdown_rows, None, wd_rows=True, out_f32=False)
        return out.view(*x.shape[:-1], -1)


class StaticClusterPoolSwiGLU(nn.Module):
    """Static cluster-pool SwiGLU (rte/layers.py:119-220): tokens routed to fixed centres of their
    SVD selector features, each cluster running its candidate pool of neurons gathered from the
    dense weights every forward (the dense weights stay the source of truth).  Pools may overlap;
    their gradients reach the dense rows through the deterministic segmented reduction."""

    def __init__(self, dense: DenseSwiGLU, factors: dict, codebook: dict, *, rank: int, sparse_enabled: bool = True):
        super().__init__()
        self.wug = nn.Linear(dense.wug.in_features, dense.wug.out_features, bias=False)
        self.wd = nn.Linear(dense.wd.in_features, dense.wd.out_features, bias=False)
        self.wug.load_state_dict(dense.wug.state_dict())
        self.wd.load_state_dict(dense.wd.state_dict())
        self.rank = int(rank)
        self.sparse_enabled = bool(sparse_enabled)
        d_model = dense.wug.in_features
        self.register_buffer("up_a", torch.empty(d_model, 0), persistent=False)
        self.register_buffer("gate_a", torch.empty(d_model, 0), persistent=False)
        self.register_buffer("centers", torch.empty(0, 0), persistent=False)
        self.register_buffer("candidate_ids", torch.empty(0, 0, dtype=torch.long), persistent=False)
        self.update_codebook(factors, codebook, rank=rank)

    @torch.no_grad()
    def update_codebook(self, factors: dict, codebook: dict, *, rank: int | None = None) -> None:
        """rte/layers.py:150-181: selector factors truncated to the rank, centres, candidate ids."""
        if rank is not None:
            self.rank = int(rank)
        rank = min(max(1, self.rank), int(factors["up_a"].shape[1]), int(factors["gate_a"].shape[1]))
        self.rank = rank
        dev, dt = self.wug.weight.device, self.wug.weight.dtype
        self.up_a = factors["up_a"][:, :rank].detach().to(device=dev, dtype=dt)
        self.gate_a = factors["gate_a"][:, :rank].detach().to(device=dev, dtype=dt)
        self.centers = codebook["centers"].detach().to(device=dev, dtype=dt)
        self.candidate_ids = codebook["candidate_ids"].detach().to(device=dev, dtype=torch.long)

    def dense_forward(self, x: torch.Tensor) -> torch.Tensor:
        flat = x.reshape(-1, x.shape[-1])
        return hip_ops.dense_swiglu(flat, self.wug.weight, self.wd.weight, None, out_f32=False).view(
            *x.shape[:-1], -1)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        from rte_amd.kernels import cluster_pool_ffn as CPF

        if not self.sparse_enabled:
            return self.dense_forward(x)
        if self.candidate_ids.numel() == 0:
            raise RuntimeError("StaticClusterPoolSwiGLU has no candidate pool")
        flat = x.reshape(-1, x.shape[-1])
        assignments = CPF.route_to_static_centers(flat, self.up_a[:, : self.rank], self.gate_a[:, : self.rank],
                                                  self.centers)
        up_w, gate_w = self.wug.weight.chunk(2, dim=0)
        pools = CPF.prepare_cluster_pool_weights(up_w, gate_w, self.wd.weight.t(), self.candidate_ids)
        out = CPF._run(flat, assignments, *pools)
        return out.view(*x.shape[:-1], -1)


class ActiveUnionSwiGLU(nn.Module):
    """SwiGLU over the union of candidate neurons (rte/layers.py:223-281): the active rows of the
    dense weights (sorted unique ids) gathered per forward, one fused SwiGLU over them."""

    def __init__(self, dense: DenseSwiGLU, active_ids: torch.Tensor, *, sparse_enabled: bool = True):
        super().__init__()
        self.wug = nn.Linear(dense.wug.in_features, dense.wug.out_features, bias=False)
        self.wd = nn.Linear(dense.wd.in_features, dense.wd.out_features, bias=False)
        self.wug.load_state_dict(dense.wug.state_dict())
        self.wd.load_state_dict(dense.wd.state_dict())
        self.sparse_enabled = bool(sparse_enabled)
        self.register_buffer("active_ids", torch.empty(0, dtype=torch.long), persistent=False)
        self.update_active_ids(active_ids)

    @torch.no_grad()
    def update_active_ids(self, active_ids: torch.Tensor) -> None:
        active_ids = active_ids.reshape(-1)
        if active_ids.numel() == 0:
            raise ValueError("active union must contain at least one neuron")
        self.active_ids = torch.unique(active_ids.detach().to(device=self.wug.weight.device, dtype=torch.long),
                                       sorted=True)

    def dense_forward(self, x: torch.Tensor) -> torch.Tensor:
        flat = x.reshape(-1, x.shape[-1])
        return hip_ops.dense_swiglu(flat, self.wug.weight, self.wd.weight, None, out_f32=False).view(
            *x.shape[:-1], -1)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if not self.sparse_enabled:
            return self.dense_forward(x)
        if self.active_ids.numel() == 0:
            raise RuntimeError("ActiveUnionSwiGLU has no active neurons")
        flat = x.reshape(-1, x.shape[-1])
        ids = self.active_ids.to(flat.device)
        d_ff = self.wd.in_features
        wug = hip_ops.embedding(self.wug.weight, torch.cat([ids, ids + d_ff]))
        down_rows = hip_ops.embedding(self.wd.weight.t(), ids)
        out = hip_ops.dense_swiglu(flat, wug, down_rows, None, wd_rows=True, out_f32=False)
        return out.view(*x.shape[:-1], -1)


class PackedActiveUnionSwiGLU(nn.Module):
    """Trainable packed active-union SwiGLU (rte/layers.py:284-339): the selected up/gate rows as
    one parameter wug_active [2M, d], the selected down rows as wdown_active_rows [M, d]."""

    def __init__(self, dense: DenseSwiGLU, active_ids: torch.Tensor):
        super().__init__()
        active_ids = active_ids.reshape(-1)
        if active_ids.numel() == 0:
            raise ValueError("packed active union must contain at least one neuron")
        ids = torch.unique(active_ids.detach().to(device=dense.wug.weight.device, dtype=torch.long), sorted=True)
        d_model, m = dense.wug.in_features, int(ids.numel())
        self.d_ff_total = int(dense.wd.in_features)
        self.wug_active = nn.Linear(d_model, 2 * m, bias=False)
        self.wdown_active_rows = nn.Parameter(torch.empty(m, d_model))
        self.use_triton_swiglu_backward = False
        self.register_buffer("active_ids", ids, persistent=True)
        with torch.no_grad():
            up_w, gate_w = dense.wug.weight.detach().chunk(2, dim=0)
            self.wug_active.weight.copy_(torch.cat([up_w.index_select(0, ids), gate_w.index_select(0, ids)]))
            self.wdown_active_rows.copy_(dense.wd.weight.detach().t().index_select(0, ids).contiguous())

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        flat = x.reshape(-1, x.shape[-1])
        out = hip_ops.dense_swiglu(flat, self.wug_active.weight, self.wdown_active_rows, None, wd_rows=True,
                                   out_f32=False)
        return out.view(*x.shape[:-1], -1)

    @property
    def active_m(self) -> int:
        return int(self.active_ids.numel())


class SVDFactorSparseFFN(nn.Module):
    """Token-level sparse SwiGLU FFN with SVD factor candidate retrieval (rte/layers.py:342-643).

    The low-rank factors of W_up and W_gate (refresh_svd) give approximate activations for every
    neuron; each token's candidates are the top up_m / gate_m / product_m neurons by |up|, |silu(gate)|
    and |up silu(gate)| times ||W_down row||, evaluated exactly, reranked to top_k and summed through
    W_down.  candidate_mode "mask" and "slots" store the candidate list as a boolean mask or as
    concatenated slots; the HIP kernel computes the set as a per-token bitmap for both.  A token
    with fewer than top_k distinct candidates gets the top_k of its approximate product scores
    added, as the reference's slots mode does (rte/layers.py:522-526).  The reference's mask mode
    writes that fill into the copy that boolean indexing returns (rte/layers.py:491), so there it
    has no effect and such a token ranks non-candidates scored -inf; this build fills in both modes
    on purpose.  "triton" is the inference-only
    device driver (rte/kernels/svd_sparse_ffn_triton.py:480-714): the "product" strategy takes the
    top top_k of the approximate product scores, "union" reranks the union with exact or
    approximate activations."""

    def __init__(self, d_model: int, d_ff: int, *, rank: int, top_k: int, up_m: int, gate_m: int | None = None,
                 product_m: int = 0, candidate_mode: str = "mask", triton_exact_activation: bool = False,
                 triton_candidate_strategy: str = "product", refresh_on_init: bool = True):
        super().__init__()
        self.d_model = int(d_model)
        self.d_ff = int(d_ff)
        self.rank = min(max(1, int(rank)), self.d_model, self.d_ff)
        self.top_k = min(max(1, int(top_k)), self.d_ff)
        self.up_m = min(max(0, int(up_m)), self.d_ff)
        self.gate_m = self.up_m if gate_m is None else min(max(0, int(gate_m)), self.d_ff)
        self.product_m = min(max(0, int(product_m)), self.d_ff)
        if candidate_mode not in {"mask", "slots", "triton"}:
            raise ValueError("candidate_mode must be 'mask', 'slots', or 'triton'")
        self.candidate_mode = candidate_mode
        self.triton_exact_activation = bool(triton_exact_activation)
        if triton_candidate_strategy not in {"union", "product"}:
            raise ValueError("triton_candidate_strategy must be 'union' or 'product'")
        self.triton_candidate_strategy = triton_candidate_strategy
        self.refresh_on_init = bool(refresh_on_init)
        self.w_up = nn.Parameter(torch.empty(self.d_ff, self.d_model))
        self.w_gate = nn.Parameter(torch.empty(self.d_ff, self.d_model))
        self.w_down = nn.Parameter(torch.empty(self.d_ff, self.d_model))
        self.register_buffer("up_a", torch.empty(self.d_model, self.rank), persistent=False)
        self.register_buffer("up_b", torch.empty(self.rank, self.d_ff), persistent=False)
        self.register_buffer("gate_a", torch.empty(self.d_model, self.rank), persistent=False)
        self.register_buffer("gate_b", torch.empty(self.rank, self.d_ff), persistent=False)
        self.reset_parameters()

    def reset_parameters(self) -> None:
        scale = 1.0 / math.sqrt(self.d_model)
        for w in (self.w_up, self.w_gate, self.w_down):
            nn.init.normal_(w, std=scale)
        if self.refresh_on_init:
            self.refresh_svd()
        else:
            for b in (self.up_a, self.up_b, self.gate_a, self.gate_b):
                nn.init.normal_(b, std=scale)

    @classmethod
    def from_dense(cls, mlp: DenseSwiGLU, *, rank: int, top_k: int, up_m: int, gate_m: int | None = None,
                   product_m: int = 0, candidate_mode: str = "mask", triton_exact_activation: bool = False,
                   triton_candidate_strategy: str = "product") -> "SVDFactorSparseFFN":
        module = cls(mlp.wug.in_features, mlp.wd.in_features, rank=rank, top_k=top_k, up_m=up_m, gate_m=gate_m,
                     product_m=product_m, candidate_mode=candidate_mode,
                     triton_exact_activation=triton_exact_activation,
                     triton_candidate_strategy=triton_candidate_strategy).to(
            device=mlp.wug.weight.device, dtype=mlp.wug.weight.dtype)
        with torch.no_grad():
            up, gate = mlp.wug.weight.detach().chunk(2, dim=0)
            module.w_up.copy_(up)
            module.w_gate.copy_(gate)
            module.w_down.copy_(mlp.wd.weight.detach().t())
            module.refresh_svd()
        return module

    @torch.no_grad()
    def refresh_svd(self) -> None:
        """Rank-r factors of W_up^T and W_gate^T: a = U[:, :r] S[:r], b = Vh[:r] (an fp32 SVD on the
        host, rte/layers.py:437-444)."""
        for prefix, weight in (("up", self.w_up), ("gate", self.w_gate)):
            mat = weight.detach().float().t().cpu().contiguous()
            u, s, vh = torch.linalg.svd(mat, full_matrices=False)
            r = self.rank
            getattr(self, f"{prefix}_a").copy_((u[:, :r] * s[:r]).to(weight.device, weight.dtype))
            getattr(self, f"{prefix}_b").copy_(vh[:r, :].to(weight.device, weight.dtype))

    def forward(self, x: torch.Tensor, *, return_aux: bool = False, profile: bool = False):
        flat = x.reshape(-1, self.d_model)
        exact, product_only = True, False
        if self.candidate_mode == "triton":
            if self.training:
                raise RuntimeError("SVDFactorSparseFFN Triton mode is inference/eval only; call .eval() first")
            product_only = self.triton_candidate_strategy == "product"
            exact = self.triton_exact_activation and not product_only
        t0 = time.perf_counter() if profile else 0.0
        out, sel, ncand = hip_ops.svd_sparse_ffn(flat, self.w_up, self.w_gate, self.w_down, self.up_a, self.up_b,
                                                 self.gate_a, self.gate_b, up_m=self.up_m, gate_m=self.gate_m,
                                                 product_m=self.product_m, top_k=self.top_k, exact=exact,
                                                 product_only=product_only)
        out = out.view(*x.shape[:-1], self.d_model)
        if not return_aux:
            return out
        aux = {"selected_ids": sel, "avg_candidate_size": float(ncand.float().mean().detach().cpu()),
               "candidate_slots": float(self.top_k if product_only else self.up_m + self.gate_m + self.product_m),
               "candidate_mode": self.candidate_mode}
        if self.candidate_mode == "triton":
            aux.update(triton_exact_activation=self.triton_exact_activation,
                       triton_candidate_strategy=self.triton_candidate_strategy)
        if profile:
            torch.cuda.synchronize()
            aux["sparse_ffn_time"] = time.perf_counter() - t0
        return out, aux


def make_ffn(config: ModelConfig) -> nn.Module:
    return ClusterPoolSwiGLU(config) if config.ffn_kind == "cluster_pool" else DenseSwiGLU(config)


class TransformerBlock(nn.Module):
    """u = x + attn(norm1(x)); out = u + mlp(norm2(u)) (rte/layers.py:646-656); the residual
    adds are fused into the O-projection and FFN-combine epilogues."""

    def __init__(self, config: ModelConfig):
        super().__init__()
        self.norm1 = RMSNorm(config.d_model)
        self.attn = DenseCausalSelfAttention(config)
        self.norm2 = RMSNorm(config.d_model)
        self.mlp = make_ffn(config)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        # each norm hands its input on as the residual branch: one gradient per stream tensor
        n1, x = hip_ops.rmsnorm_resid(x.float(), self.norm1.weight, self.norm1.eps)
        u = self.attn(n1, resid=x)
        n2, u = hip_ops.rmsnorm_resid(u, self.norm2.weight, self.norm2.eps)
        return self.mlp(n2, resid=u)


# ----------------------------------------------------------------------------- banked recursive core

def _head_scale(config: ModelConfig, spec: RecipeSpec) -> torch.Tensor:
    """[attn_banks, n_heads]: 1/|banks| on the recipe's (bank, head) pairs, 0 elsewhere
    (rte/layers.py:702-728: attention over the active head groups, mean over banks)."""
    hpg = config.n_heads // config.head_groups
    m = torch.zeros(config.attn_banks, config.n_heads)
    for b in spec.attention_banks:
        for g in spec.head_groups:
            m[b, g * hpg:(g + 1) * hpg] = 1.0 / max(len(spec.attention_banks), 1)
    return m


def _ffn_route(config: ModelConfig, spec: RecipeSpec, kmax: int) -> tuple[torch.Tensor, float]:
    """Pool clusters (bank * ffn_groups + slab group) a recipe's tokens visit, -1 padded to
    kmax, and their weight 1/|banks| (rte/layers.py:744-779)."""
    ids = [b * config.ffn_groups + g for b in spec.ffn_banks for g in spec.ffn_groups]
    row = torch.full((kmax,), -1, dtype=torch.int32)
    row[: len(ids)] = torch.tensor(ids, dtype=torch.int32)
    return row, 1.0 / max(len(spec.ffn_banks), 1)


class BankedAttention(nn.Module):
    """rte/layers.py:659-728.  Every sample runs the QKV+RoPE GEMM over all heads of each bank;
    the recipe's head/bank selection (and the 1/|banks| mean) is a per-(sample, bank, head)
    scale applied to V, which zeroes the unused heads' attention output exactly before the
    O-projection.  No host read of the recipe ids is needed."""

    def __init__(self, config: ModelConfig, recipe_bank: RecipeBank):
        super().__init__()
        self.config = config
        d = config.d_model
        scale = 1.0 / math.sqrt(d)
        self.wqkv = nn.Parameter(torch.randn(config.attn_banks, d, 3 * d) * scale)
        self.wo = nn.Parameter(torch.randn(config.attn_banks, d, d) * scale)
        self.rope = RotaryEmbedding(d // config.n_heads) if config.use_rope else None
        cols = torch.zeros(config.recipe_count, d, dtype=torch.long)
        qkv_cols = torch.zeros(config.recipe_count, 3 * d, dtype=torch.long)
        for spec in recipe_bank.recipes:
            v = torch.tensor(self._cols_for_groups(spec), dtype=torch.long)
            cols[spec.recipe_id, : v.numel()] = v
            qkv_cols[spec.recipe_id, : 3 * v.numel()] = torch.cat([v, v + d, v + 2 * d])
        self.register_buffer("recipe_cols", cols, persistent=False)
        self.register_buffer("recipe_qkv_cols", qkv_cols, persistent=False)
        self.register_buffer("recipe_head_scale", torch.stack([_head_scale(config, s) for s in recipe_bank.recipes]),
                             persistent=False)

    def _cols_for_groups(self, spec: RecipeSpec) -> list[int]:
        hpg = self.config.n_heads // self.config.head_groups
        hd = self.config.d_model // self.config.n_heads
        out: list[int] = []
        for g in spec.head_groups:
            for h in range(g * hpg, (g + 1) * hpg):
                out.extend(range(h * hd, (h + 1) * hd))
        return out

    def _tables(self):
        if self.rope is not None:
            return self.rope.cos, self.rope.sin
        hd = self.config.d_model // self.config.n_heads
        cos = torch.ones(8192, hd, device=self.wqkv.device)
        return cos, torch.zeros_like(cos)

    def bank_weights(self):
        """Per-bank (Wqkv^T, Wo^T) views, split once per forward: every recursive pass then shares
        one gradient stack per parameter instead of a zero-fill and copy per use."""
        if self.wqkv.shape[0] == 1:  # one bank: plain views (no gradient stack)
            return (self.wqkv.squeeze(0).t(),), (self.wo.squeeze(0).t(),)
        return tuple(w.t() for w in self.wqkv.unbind(0)), tuple(w.t() for w in self.wo.unbind(0))

    def forward_scaled(self, x: torch.Tensor, head_scale: torch.Tensor, banks=None, wgrads=None) -> torch.Tensor:
        """x [B, S, d], head_scale [B, attn_banks, n_heads] -> fp32 [B, S, d].  wgrads (optional):
        per bank (qkv, out) hip_ops.SharedWGrad of the passes sharing these weights."""
        cos, sin = self._tables()
        H = self.config.n_heads
        wqkv_t, wo_t = banks if banks is not None else self.bank_weights()
        out = None
        for bank in range(self.config.attn_banks):
            gq, go = wgrads[bank] if wgrads is not None else (None, None)
            # the recipe's head mask (1/|banks| on its heads, 0 elsewhere: rte/layers.py:702-730 runs
            # only the active heads and averages the banks) scales each head's attention output
            y = hip_ops.qkv_rope_attention(x, wqkv_t[bank], cos, sin, H, head_scale[:, bank, :], wgrad=gq)
            out = hip_ops.attn_out_proj(y, wo_t[bank], out, wgrad=go)
        return out

    def forward(self, x: torch.Tensor, spec: RecipeSpec) -> torch.Tensor:
        """Attention of one recipe for every sample of x (the reference's per-group call)."""
        hs = _head_scale(self.config, spec).to(x.device)
        return self.forward_scaled(x, hs.unsqueeze(0).expand(x.shape[0], -1, -1))


class BankedSwiGLU(nn.Module):
    """rte/layers.py:731-779: mean over the recipe's FFN banks of the SwiGLU restricted to its
    active slabs.  Runs as the grouped pool kernel: cluster (bank, slab group) owns the slab's
    up/gate/down neurons of that bank, each token visits its recipe's clusters with weight
    1/|banks| (absent pairs are -1 and cost nothing)."""

    def __init__(self, config: ModelConfig, recipe_bank: RecipeBank):
        super().__init__()
        self.config = config
        d = config.d_model
        scale = 1.0 / math.sqrt(d)
        self.wug = nn.Parameter(torch.randn(config.ffn_banks, d, 2 * config.d_ff) * scale)
        self.wd = nn.Parameter(torch.randn(config.ffn_banks, config.d_ff, d) * scale)
        slabs = torch.zeros(config.recipe_count, config.d_ff, dtype=torch.long)
        gate_cols = torch.zeros(config.recipe_count, 2 * config.d_ff, dtype=torch.long)
        slab = config.d_ff // config.ffn_groups
        for spec in recipe_bank.recipes:
            v = torch.tensor([c for g in spec.ffn_groups for c in range(g * slab, (g + 1) * slab)], dtype=torch.long)
            slabs[spec.recipe_id, : v.numel()] = v
            gate_cols[spec.recipe_id, : 2 * v.numel()] = torch.cat([v, v + config.d_ff])
        self.register_buffer("recipe_slabs", slabs, persistent=False)
        self.register_buffer("recipe_gate_cols", gate_cols, persistent=False)
        self.kmax = max(len(s.ffn_banks) * len(s.ffn_groups) for s in recipe_bank.recipes)
        routes = [_ffn_route(config, s, self.kmax) for s in recipe_bank.recipes]
        self.register_buffer("recipe_routes", torch.stack([r for r, _ in routes]), persistent=False)
        self.register_buffer("recipe_route_w", torch.tensor([w for _, w in routes], dtype=torch.float32),
                             persistent=False)

    def pool_weights(self) -> tuple[torch.Tensor, torch.Tensor]:
        """Bank weights in the grouped kernel's layout: wug_t [2 * banks * F, d] with rows
        [up of every bank ; gate of every bank], wd_t [d, banks * F] (differentiable copies)."""
        A, d, F2 = self.wug.shape
        F_ = F2 // 2
        wug_t = self.wug.view(A, d, 2, F_).permute(2, 0, 3, 1).reshape(2 * A * F_, d)
        wd_t = self.wd.permute(2, 0, 1).reshape(d, A * F_)
        return wug_t, wd_t

    def forward_routes(self, x: torch.Tensor, ids: torch.Tensor, w: torch.Tensor, weights=None,
                       acc=None) -> torch.Tensor:
        """x [B, S, d]; ids [B*S, kmax] int32 (-1 = no pair); w [B*S, kmax] fp32 -> fp32 [B, S, d].
        acc: hip_ops.SharedGradAccum of the passes sharing the weights (optional)."""
        wug_t, wd_t = weights if weights is not None else self.pool_weights()
        slab = self.config.d_ff // self.config.ffn_groups
        return hip_ops.grouped_pool_swiglu(x, ids, w, wug_t, wd_t, slab, acc=acc)

    def pack_recipes(self, recipe_ids: torch.Tensor, seq: int, active: torch.Tensor | None = None):
        """The pool pack of samples with recipe_ids [B] (inactive samples get no pairs)."""
        slab = self.config.d_ff // self.config.ffn_groups
        clusters = self.config.ffn_banks * self.config.d_ff // slab
        return hip_ops.pack_routes(recipe_ids, self.recipe_routes, self.recipe_route_w, seq, clusters, active)

    def forward_recipes(self, x: torch.Tensor, recipe_ids: torch.Tensor, active: torch.Tensor | None = None,
                        weights=None, acc=None, pk=None) -> torch.Tensor:
        """Every sample's tokens through its recipe's clusters (inactive samples: none), packed
        straight from the recipe ids (rte_pack_routes); pk: that pack, made ahead (optional)."""
        wug_t, wd_t = weights if weights is not None else self.pool_weights()
        slab = self.config.d_ff // self.config.ffn_groups
        if pk is None:
            pk = self.pack_recipes(recipe_ids, x.shape[1], active)
        return hip_ops.grouped_pool_swiglu(x, None, None, wug_t, wd_t, slab, pk=pk, acc=acc)

    def routes_for(self, recipe_ids: torch.Tensor, seq: int, active: torch.Tensor | None = None):
        """Per-token routes of samples with recipe_ids [B] (inactive samples get none)."""
        ids = self.recipe_routes[recipe_ids]                                   # [B, kmax]
        if active is not None:
            ids = torch.where(active[:, None], ids, torch.full_like(ids, -1))
        w = self.recipe_route_w[recipe_ids][:, None].expand(-1, self.kmax)
        B = recipe_ids.shape[0]
        return (ids[:, None, :].expand(B, seq, self.kmax).reshape(B * seq, self.kmax),
                w[:, None, :].expand(B, seq, self.kmax).reshape(B * seq, self.kmax))

    def forward(self, x: torch.Tensor, spec: RecipeSpec) -> torch.Tensor:
        """SwiGLU of one recipe for every token of x (the reference's per-group call)."""
        row, wt = _ffn_route(self.config, spec, self.kmax)
        T = x.shape[0] * x.shape[1]
        ids = row.to(x.device)[None, :].expand(T, -1)
        w = torch.full((T, self.kmax), wt, dtype=torch.float32, device=x.device)
        return self.forward_routes(x, ids, w)


class BankedRecursiveCore(nn.Module):
    """rte/layers.py:806-870 (global low-rank corrector not supported: off by default).

    The exact replay of a few samples (forward_replay) runs all passes as one node on the replay
    kernels when the shape allows (one bank of heads and of slabs, head width 64, d <= 512,
    slabs of whole 32-neuron blocks, RoPE); fused_replay = False keeps it on the per-operator
    path."""

    fused_replay = True
    replay_max_rows = 2048  # the replay's few samples; larger exact batches keep the wide GEMMs

    def __init__(self, config: ModelConfig, recipe_bank: RecipeBank):
        super().__init__()
        if config.use_global_lowrank_corrector:
            raise NotImplementedError("use_global_lowrank_corrector is outside the accelerated path")
        self.config = config
        self.recipe_bank = recipe_bank
        self.norm1 = RMSNorm(config.d_model)
        self.attn = BankedAttention(config, recipe_bank)
        self.norm2 = RMSNorm(config.d_model)
        self.mlp = BankedSwiGLU(config, recipe_bank)
        t, d = config.t_max, config.d_model
        self.pass_gamma1 = nn.Parameter(torch.zeros(t, d))
        self.pass_beta1 = nn.Parameter(torch.zeros(t, d))
        self.pass_gamma2 = nn.Parameter(torch.zeros(t, d))
        self.pass_beta2 = nn.Parameter(torch.zeros(t, d))
        self.pass_attn_scale = nn.Parameter(torch.full((t,), 1.0))
        self.pass_mlp_scale = nn.Parameter(torch.full((t,), 1.0))
        self.global_corrector = None
        if config.use_recursive_input_skip:
            self.alpha_inj = nn.Parameter(torch.tensor(0.1))
        else:
            self.register_parameter("alpha_inj", None)
        self._init_replay_tables(config, recipe_bank)

    def _init_replay_tables(self, config: ModelConfig, recipe_bank: RecipeBank) -> None:
        """Per recipe: its heads and 32-neuron slab blocks, the replay kernels' selection tables
        (rte/layers.py:702-779: the recipe's head groups and FFN groups of its single bank)."""
        from rte_amd.kernels import replay_core as RC

        H, d = config.n_heads, config.d_model
        hpg = H // config.head_groups
        slab = config.d_ff // config.ffn_groups
        self._replay_shape_ok = (config.attn_banks == 1 and config.ffn_banks == 1 and config.use_rope
                                 and d // H == RC.HEAD_DIM and d % 128 == 0 and d <= RC.MAX_D
                                 and slab % RC.BLOCK == 0)
        self._replay_meta = None
        if not self._replay_shape_ok:
            return
        bps = slab // RC.BLOCK
        heads = [[g * hpg + i for g in s.head_groups for i in range(hpg)] for s in recipe_bank.recipes]
        blocks = [[g * bps + j for g in s.ffn_groups for j in range(bps)] for s in recipe_bank.recipes]
        rec = RC.build_records(heads, blocks, H, config.d_ff // RC.BLOCK)
        self.register_buffer("replay_records", rec, persistent=False)
        self._replay_meta = (H, config.d_ff // RC.BLOCK, int(rec[:, 1].max()), int(rec[:, 2].max()))

    def replay_tables(self):
        from rte_amd.kernels import replay_core as RC

        H, NB, hm, nbm = self._replay_meta
        return RC.ReplayTables(self.replay_records, H, NB, hm, nbm)

    def replay_fused_ok(self, h0: torch.Tensor) -> bool:
        """The fused replay applies: shape supported, a ROCm device, bf16 operators (not the fp32
        precision path), sequence within the rotary table."""
        return (type(self).fused_replay and self._replay_shape_ok and h0.is_cuda and not hip_ops.fp32_active()
                and h0.dim() == 3 and h0.shape[1] <= self.attn.rope.cos.shape[0]
                and h0.shape[0] * h0.shape[1] <= self.replay_max_rows)

    def forward_replay(self, h0, recipe_ids_by_pass, active_by_pass=None, keep=()):
        """All T exact passes from h0 (rte/layers.py:847-870 for t = 0 .. T-1): recipe_ids_by_pass
        [T, B], active_by_pass [T, B] bool or None.  Returns (h_T, *states of the passes in keep)."""
        from rte_amd.kernels import replay_core as RC

        cos, sin = self.attn._tables()
        outs = RC.replay_core(h0, self.pass_gamma1, self.pass_beta1, self.pass_gamma2, self.pass_beta2,
                              self.pass_attn_scale, self.pass_mlp_scale, self.alpha_inj, self.norm1.weight,
                              self.norm2.weight, self.attn.wqkv, self.attn.wo, self.mlp.wug, self.mlp.wd,
                              recipe_ids_by_pass, active_by_pass, self.replay_tables(), cos, sin, self.norm1.eps,
                              self.norm2.eps, 1.0, keep)
        return outs

    def prepare(self):
        """Per-forward views shared by every recursive pass: the pool weight layouts and the
        per-pass FiLM / scale parameters split once (one gradient stack per parameter in the
        backward instead of a zero-fill and copy per pass)."""
        per_pass = tuple(p.unbind(0) for p in (self.pass_gamma1, self.pass_beta1, self.pass_gamma2,
                                                self.pass_beta2, self.pass_attn_scale, self.pass_mlp_scale))
        # one shared weight-gradient GEMM per attention weight over every pass of this forward
        wgrads = [(hip_ops.SharedWGrad(), hip_ops.SharedWGrad()) for _ in range(self.config.attn_banks)]
        # and one pair of pool weight-gradient buffers that every pass adds into
        return {"pool": self.mlp.pool_weights(), "pass": per_pass, "attn": self.attn.bank_weights(),
                "attn_wgrad": wgrads, "pool_wgrad": hip_ops.SharedGradAccum()}

    def _step(self, h, h0, head_scale, ids, w, pass_idx: int, weights=None, active=None, recipe_ids=None):
        """One pass: three fused residual / FiLM-norm launches around attention and the pool
        FFN; samples whose `active` entry is False keep h."""
        if weights is None:
            weights = self.prepare()
        g1, b1, g2, b2, sa, sm = (p[pass_idx] for p in weights["pass"])
        h = h.float()
        h_tilde, n1 = hip_ops.axpy_norm(h, None if self.alpha_inj is None else h0.float(), self.alpha_inj,
                                        self.norm1.weight, g1, b1, self.norm1.eps)
        attn = self.attn.forward_scaled(n1, head_scale, weights.get("attn"), weights.get("attn_wgrad"))
        u, n2 = hip_ops.axpy_norm(h_tilde, attn, sa, self.norm2.weight, g2, b2, self.norm2.eps)
        if recipe_ids is not None:  # per-sample recipes: pack the routes straight from the ids
            mlp = self.mlp.forward_recipes(n2, recipe_ids, active, weights["pool"], weights.get("pool_wgrad"),
                                           weights.get("pool_pack"))
        else:
            mlp = self.mlp.forward_routes(n2, ids, w, weights["pool"], weights.get("pool_wgrad"))
        return hip_ops.axpy(u, mlp, sm, keep=h if active is not None else None, mask=active)

    def step_group(self, h, h0, spec: RecipeSpec, pass_idx: int = 0):
        """One pass of a single recipe over every sample of h (rte/layers.py:826-845)."""
        B, S, _ = h.shape
        hs = _head_scale(self.config, spec).to(h.device).unsqueeze(0).expand(B, -1, -1)
        row, wt = _ffn_route(self.config, spec, self.mlp.kmax)
        ids = row.to(h.device)[None, :].expand(B * S, -1)
        w = torch.full((B * S, self.mlp.kmax), wt, dtype=torch.float32, device=h.device)
        return self._step(h, h0, hs, ids, w, pass_idx)

    def forward_step(self, h, h0, recipe_ids, active_mask=None, pass_idx: int = 0, *, weights=None,
                     head_scale=None):
        """One exact recursive pass (rte/layers.py:847-870): every sample runs its own recipe,
        inactive samples keep h.  The recipe ids stay on the device: the head / slab selection
        is table lookups and masks, so the pass needs no host synchronisation.  head_scale
        (optional): the recipes' rows of attn.recipe_head_scale, looked up ahead."""
        rid = recipe_ids.long()
        if head_scale is None:
            head_scale = self.attn.recipe_head_scale[rid]
        return self._step(h, h0, head_scale, None, None, pass_idx, weights, active_mask, rid).to(h.dtype)
