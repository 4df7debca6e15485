"""RMSNorm, interleaved RoPE and fused-QKV oracle (numpy, float64).  Test infrastructure only."""

from __future__ import annotations

import numpy as np


def rmsnorm(x, w, eps: float = 1e-5):
    """x * rsqrt(mean(x^2) + eps) * w  (rte/kernels/reference.py:9-17)."""
    x = np.asarray(x, np.float64)
    return x / np.sqrt((x * x).mean(-1, keepdims=True) + eps) * np.asarray(w, np.float64)


def rmsnorm_bwd(dy, x, w, eps: float = 1e-5):
    x = np.asarray(x, np.float64)
    w = np.asarray(w, np.float64)
    dy = np.asarray(dy, np.float64)
    d = x.shape[-1]
    r = 1.0 / np.sqrt((x * x).mean(-1, keepdims=True) + eps)
    g = dy * w
    dx = r * g - x * r**3 * (g * x).sum(-1, keepdims=True) / d
    dw = (dy * x * r).reshape(-1, d).sum(0)
    return dx, dw


def rope_tables(head_dim: int, seq_len: int, base: float = 10_000.0):
    """cos/sin [S, hd] of RotaryEmbedding (rte/layers.py:36-44): frequencies repeated per pair."""
    inv = 1.0 / (base ** (np.arange(0, head_dim, 2, dtype=np.float64) / head_dim))
    freqs = np.outer(np.arange(seq_len, dtype=np.float64), inv)
    emb = np.repeat(freqs, 2, axis=-1)
    return np.cos(emb), np.sin(emb)


def rope_apply(x, cos, sin):
    """x*cos + rotate_half(x)*sin with interleaved pairs (rte/kernels/reference.py:20-28):
    rotate_half maps (x0, x1) -> (-x1, x0) for each pair (2i, 2i+1)."""
    x = np.asarray(x, np.float64)
    rot = np.empty_like(x)
    rot[..., 0::2] = -x[..., 1::2]
    rot[..., 1::2] = x[..., 0::2]
    return x * cos + rot * sin


def rope_apply_bwd(dy, cos, sin):
    """Transpose of rope_apply's Jacobian."""
    dy = np.asarray(dy, np.float64)
    dc = dy * cos
    ds = dy * sin
    dx = dc.copy()
    dx[..., 1::2] -= ds[..., 0::2]
    dx[..., 0::2] += ds[..., 1::2]
    return dx


def qkv_rope(x, wqkv, n_heads: int, cos, sin):
    """qkv = x @ Wqkv^T viewed [B, S, 3, H, hd] (rte/layers.py:64-71), RoPE on q and k."""
    x = np.asarray(x, np.float64)
    B, S, d = x.shape
    hd = d // n_heads
    qkv = (x @ np.asarray(wqkv, np.float64).T).reshape(B, S, 3, n_heads, hd)
    q, k, v = (qkv[:, :, i].transpose(0, 2, 1, 3) for i in range(3))
    return rope_apply(q, cos[:S], sin[:S]), rope_apply(k, cos[:S], sin[:S]), v


def qkv_rope_bwd(dq, dk, dv, x, wqkv, cos, sin):
    x = np.asarray(x, np.float64)
    B, S, d = x.shape
    parts = [rope_apply_bwd(dq, cos[:S], sin[:S]), rope_apply_bwd(dk, cos[:S], sin[:S]), np.asarray(dv, np.float64)]
    dqkv = np.stack([p.transpose(0, 2, 1, 3).reshape(B, S, d) for p in parts], axis=2).reshape(B * S, 3 * d)
    x2 = x.reshape(B * S, d)
    return (dqkv @ np.asarray(wqkv, np.float64)).reshape(B, S, d), dqkv.T @ x2
