"""Dense / packed SwiGLU oracle (numpy, float64).  Test infrastructure only."""

from __future__ import annotations

import numpy as np


def sigmoid(x: np.ndarray) -> np.ndarray:
    return 1.0 / (1.0 + np.exp(-x))


def silu(x: np.ndarray) -> np.ndarray:
    return x * sigmoid(x)


def dense_swiglu_fwd(x, wug, wd, *, wd_rows: bool = False):
    """y = (up * silu(gate)) @ W_down.

    wug [2F, d] with rows [up ; gate] — the chunk order of DenseSwiGLU (rte/layers.py:85-87)
    and of the packed W_ug (rte/layers.py:107-116).  wd is the nn.Linear(F, d) weight [d, F]
    (wd_rows=False) or the packed wdown_rows [F, d] (wd_rows=True).
    Returns (y, cache) where cache holds up, gate, z for the backward.
    """
    x = np.asarray(x, np.float64)
    wug = np.asarray(wug, np.float64)
    wd = np.asarray(wd, np.float64)
    F = wug.shape[0] // 2
    ug = x @ wug.T
    up, gate = ug[:, :F], ug[:, F:]
    z = up * silu(gate)
    y = z @ (wd if wd_rows else wd.T)
    return y, {"up": up, "gate": gate, "z": z}


def dense_swiglu_bwd(dy, x, wug, wd, cache, *, wd_rows: bool = False):
    """Closed-form backward of the fused SwiGLU FFN (rte/kernels/active_swiglu_triton.py:39-59,
    :87-102):  dz = dy W_down^T, dup = dz silu(g), dg = dz up s (1 + g (1 - s)),
    dx = [dup|dg] W_ug, dW_ug = [dup|dg]^T x, dW_down = z^T dy (or dy^T z for the Linear layout)."""
    dy = np.asarray(dy, np.float64)
    x = np.asarray(x, np.float64)
    wug = np.asarray(wug, np.float64)
    wd = np.asarray(wd, np.float64)
    up, gate, z = cache["up"], cache["gate"], cache["z"]
    dz = dy @ (wd.T if wd_rows else wd)
    s = sigmoid(gate)
    dup = dz * gate * s
    dgate = dz * up * s * (1.0 + gate * (1.0 - s))
    dug = np.concatenate([dup, dgate], axis=-1)
    dx = dug @ wug
    dwug = dug.T @ x
    dwd = z.T @ dy if wd_rows else dy.T @ z
    return dx, dwug, dwd
