"""Model building blocks of the recursive_macro path (rte/layers.py:26-951).

Hot modules run on the HIP kernels (rte_amd.kernels.hip_ops):
  RMSNorm                 fused norm fwd/bwd
  DenseCausalSelfAttention  fused QKV GEMM + RoPE epilogue, SDPA core, O-proj GEMM + residual
  DenseSwiGLU             SwiGLU fused into the up/gate GEMM epilogue (fwd) and dZ GEMM (bwd)
  ClusterPoolSwiGLU       routed top-k cluster-pool SwiGLU (route, pack, grouped GEMMs, combine)
The banked recursive core (exact-replay audit path, a few samples per step) is
torch glue on the device for now; parameter names/shapes follow the reference so
state dicts are interchangeable.
"""

from __future__ import annotations

import math

import torch
import torch.nn.functional as F
from torch import nn

from rte_amd.config import ModelConfig
from rte_amd.gather import gather_cols, gather_rows
from rte_amd.kernels import hip_ops
from rte_amd.kernels import optimized as K
from rte_amd.recipes import RecipeBank, RecipeSpec


class RMSNorm(nn.Module):
    def __init__(self, dim: int, eps: float = 1e-5):
        super().__init__()
        self.weight = nn.Parameter(torch.ones(dim))
        self.eps = eps

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return K.k_fused_rmsnorm(x, self.weight, eps=self.eps)[0]


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
        q, k, v = hip_ops.qkv_rope(x, self.wqkv.weight, cos, sin, self.n_heads)
        y = K.k_flash_causal_dense(q, k, v)
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
        x = x.float()
        u = self.attn(self.norm1(x), resid=x)
        return self.mlp(self.norm2(u), resid=u)


# ----------------------------------------------------------------------------- banked recursive core

class BankedAttention(nn.Module):
    """rte/layers.py:659-728."""

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

    def _cols_for_groups(self, spec: RecipeSpec) -> list[int]:
        hpg = self.config.n_heads // self.config.head_groups
        hd = self.config.d_model // self.config.n_heads
        out: list[int] = []
        for g in spec.head_groups:
            for h in range(g * hpg, (g + 1) * hpg):
                out.extend(range(h * hd, (h + 1) * hd))
        return out

    def forward(self, x: torch.Tensor, spec: RecipeSpec) -> torch.Tensor:
        b, s, d = x.shape
        hd = d // self.config.n_heads
        active_dim = len(spec.head_groups) * (self.config.n_heads // self.config.head_groups) * hd
        cols = self.recipe_cols[spec.recipe_id, :active_dim]
        qkv_cols = self.recipe_qkv_cols[spec.recipe_id, : 3 * active_dim]
        heads = active_dim // hd
        out = x.new_zeros(b, s, d)
        for bank in spec.attention_banks:
            qkv = x @ gather_cols(self.wqkv[bank], qkv_cols)
            q, k, v = (t.view(b, s, heads, hd).transpose(1, 2) for t in qkv.split(active_dim, dim=-1))
            if self.rope is not None:
                q, k = self.rope(q, k)
            y = K.k_flash_causal_grouped(q, k, v).transpose(1, 2).contiguous().view(b, s, active_dim)
            out = out + y @ gather_rows(self.wo[bank], cols)
        return out / max(len(spec.attention_banks), 1)


class BankedSwiGLU(nn.Module):
    """rte/layers.py:731-779: mean over the recipe's FFN banks of the SwiGLU restricted to
    its active slabs."""

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

    def forward(self, x: torch.Tensor, spec: RecipeSpec) -> torch.Tensor:
        slab = self.config.d_ff // self.config.ffn_groups
        active = len(spec.ffn_groups) * slab
        slabs = self.recipe_slabs[spec.recipe_id, :active]
        gate_cols = self.recipe_gate_cols[spec.recipe_id, : 2 * active]
        out = x.new_zeros(*x.shape)
        for bank in spec.ffn_banks:
            fused = x @ gather_cols(self.wug[bank], gate_cols)
            up, gate = fused.split(active, dim=-1)
            out = out + (up * F.silu(gate)) @ gather_rows(self.wd[bank], slabs)
        return out / max(len(spec.ffn_banks), 1)


class BankedRecursiveCore(nn.Module):
    """rte/layers.py:806-870 (global low-rank corrector not supported: off by default)."""

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

    def step_group(self, h, h0, spec: RecipeSpec, pass_idx: int = 0):
        h_tilde = h if self.alpha_inj is None else h + self.alpha_inj * h0
        n1 = self.norm1(h_tilde) * (1.0 + self.pass_gamma1[pass_idx]) + self.pass_beta1[pass_idx]
        u = h_tilde + self.pass_attn_scale[pass_idx] * self.attn(n1, spec)
        n2 = self.norm2(u) * (1.0 + self.pass_gamma2[pass_idx]) + self.pass_beta2[pass_idx]
        return u + self.pass_mlp_scale[pass_idx] * self.mlp(n2, spec)

    def forward_step(self, h, h0, recipe_ids, active_mask=None, pass_idx: int = 0, *, host_ids=None,
                     host_active=None):
        """One exact recursive pass, grouped by recipe (rte/layers.py:854-870).  host_ids /
        host_active (python lists) let the caller read the routing decisions once per replay
        instead of once per pass."""
        if host_ids is None:
            host_ids = recipe_ids.detach().cpu().tolist()
            host_active = ([True] * len(host_ids) if active_mask is None
                           else active_mask.detach().cpu().tolist())
        out = h.clone()
        for rid in sorted({r for r, a in zip(host_ids, host_active) if a}):
            rows = [i for i, (r, a) in enumerate(zip(host_ids, host_active)) if a and r == rid]
            spec = self.recipe_bank.get_recipe(int(rid))
            if len(rows) == h.shape[0]:
                return self.step_group(h, h0, spec, pass_idx=pass_idx).to(out.dtype)
            idx = torch.tensor(rows, device=h.device, dtype=torch.long)
            out = out.index_copy(0, idx, self.step_group(h.index_select(0, idx), h0.index_select(0, idx), spec,
                                                         pass_idx=pass_idx).to(out.dtype))
        return out
