"""Banked recursive core oracle (numpy, float64) — TEST INFRASTRUCTURE ONLY.

Restates BankedAttention / BankedSwiGLU / BankedRecursiveCore of the reference
(rte/layers.py:659-870; rte/ = src/recursive_training_engine/) per sample and per
recipe, with the recipe templates of rte/recipes.py:65-100.  A recipe is given as a
dict with keys attention_banks, ffn_banks, head_groups, ffn_groups.
"""

from __future__ import annotations

import numpy as np

from oracle.attention import rmsnorm, rope_apply
from oracle.swiglu import silu


def recipe_templates(attn_banks, ffn_banks, head_groups, ffn_groups, active_head_groups, active_ffn_groups,
                     recipe_count):
    """Recipe 0 = every bank and group; recipe r >= 1 walks (bank, slot) round-robin
    (rte/recipes.py:65-100)."""
    out = [dict(attention_banks=tuple(range(attn_banks)), ffn_banks=tuple(range(ffn_banks)),
                head_groups=tuple(range(head_groups)), ffn_groups=tuple(range(ffn_groups)))]
    head_slots = max(1, head_groups // active_head_groups)
    ffn_slots = max(1, ffn_groups // active_ffn_groups)
    for idx in range(recipe_count - 1):
        hs, fs = idx % head_slots, idx % ffn_slots
        out.append(dict(
            attention_banks=((idx // head_slots) % attn_banks,),
            ffn_banks=((idx // ffn_slots) % ffn_banks,),
            head_groups=tuple((hs * active_head_groups + j) % head_groups for j in range(active_head_groups)),
            ffn_groups=tuple((fs * active_ffn_groups + j) % ffn_groups for j in range(active_ffn_groups)),
        ))
    return out


def causal_attention(q, k, v):
    """softmax(q k^T / sqrt(hd) + causal mask) v per head; q, k, v [H, S, hd]."""
    hd = q.shape[-1]
    s = q @ k.transpose(0, 2, 1) / np.sqrt(hd)
    S = s.shape[-1]
    s = np.where(np.tril(np.ones((S, S), bool)), s, -np.inf)
    s = s - s.max(-1, keepdims=True)
    p = np.exp(s)
    p /= p.sum(-1, keepdims=True)
    return p @ v


def banked_attention(x, recipe, wqkv, wo, n_heads, head_groups, cos, sin):
    """One sample x [S, d] (rte/layers.py:702-728): for each bank of the recipe, QKV over the
    columns of its active head groups, RoPE, causal attention, O-projection over the same
    rows of wo[bank]; mean over the banks."""
    x = np.asarray(x, np.float64)
    S, d = x.shape
    hd = d // n_heads
    hpg = n_heads // head_groups
    cols = np.array([c for g in recipe["head_groups"] for h in range(g * hpg, (g + 1) * hpg)
                     for c in range(h * hd, (h + 1) * hd)])
    qkv_cols = np.concatenate([cols, cols + d, cols + 2 * d])
    a = cols.size
    out = np.zeros((S, d))
    for b in recipe["attention_banks"]:
        qkv = x @ np.asarray(wqkv, np.float64)[b][:, qkv_cols]
        q, k, v = (qkv[:, i * a:(i + 1) * a].reshape(S, a // hd, hd).transpose(1, 0, 2) for i in range(3))
        if cos is not None:
            q, k = rope_apply(q, cos[:S], sin[:S]), rope_apply(k, cos[:S], sin[:S])
        y = causal_attention(q, k, v).transpose(1, 0, 2).reshape(S, a)
        out += y @ np.asarray(wo, np.float64)[b][cols, :]
    return out / max(len(recipe["attention_banks"]), 1)


def banked_swiglu(x, recipe, wug, wd, ffn_groups):
    """One sample x [S, d] (rte/layers.py:744-779): for each bank, x @ wug[bank][:, up/gate columns
    of the active slabs], SwiGLU, @ wd[bank][slabs, :]; mean over the banks."""
    x = np.asarray(x, np.float64)
    wug = np.asarray(wug, np.float64)
    wd = np.asarray(wd, np.float64)
    F = wd.shape[1]
    slab = F // ffn_groups
    slabs = np.array([c for g in recipe["ffn_groups"] for c in range(g * slab, (g + 1) * slab)])
    gate_cols = np.concatenate([slabs, slabs + F])
    out = np.zeros_like(x)
    for b in recipe["ffn_banks"]:
        fused = x @ wug[b][:, gate_cols]
        up, gate = fused[:, :slabs.size], fused[:, slabs.size:]
        out += (up * silu(gate)) @ wd[b][slabs, :]
    return out / max(len(recipe["ffn_banks"]), 1)


def core_step(h, h0, recipe, p, pass_idx, *, n_heads, head_groups, ffn_groups, cos, sin, eps=1e-5):
    """One recursive pass of one sample (rte/layers.py:826-845).  p holds the core's parameters
    (norm1, norm2, wqkv, wo, wug, wd, pass_gamma1/beta1/gamma2/beta2, pass_attn_scale,
    pass_mlp_scale, alpha_inj or None)."""
    h = np.asarray(h, np.float64)
    ht = h if p.get("alpha_inj") is None else h + p["alpha_inj"] * np.asarray(h0, np.float64)
    n1 = rmsnorm(ht, p["norm1"], eps) * (1.0 + p["pass_gamma1"][pass_idx]) + p["pass_beta1"][pass_idx]
    u = ht + p["pass_attn_scale"][pass_idx] * banked_attention(n1, recipe, p["wqkv"], p["wo"], n_heads, head_groups,
                                                               cos, sin)
    n2 = rmsnorm(u, p["norm2"], eps) * (1.0 + p["pass_gamma2"][pass_idx]) + p["pass_beta2"][pass_idx]
    return u + p["pass_mlp_scale"][pass_idx] * banked_swiglu(n2, recipe, p["wug"], p["wd"], ffn_groups)


def core_forward_step(h, h0, recipe_ids, active, recipes, p, pass_idx, **kw):
    """rte/layers.py:847-870: samples with active[i] run their recipe's step, the rest keep h."""
    out = np.array(h, np.float64, copy=True)
    for i in range(out.shape[0]):
        if active is None or active[i]:
            out[i] = core_step(h[i], h0[i], recipes[int(recipe_ids[i])], p, pass_idx, **kw)
    return out
