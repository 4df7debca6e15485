"""Macro operator oracle (numpy, float64) — TEST INFRASTRUCTURE ONLY.

Restates the bounded-residual macro operator Phi_{recipe, stride} of the reference
(rte/macro.py:201-236; rte/ = src/recursive_training_engine/) per sample: the sample's
(recipe, stride) selects its low-rank matrices v [in, m], u [m, d] and its vectors
gain, bias, update_scale [d].
"""

from __future__ import annotations

import numpy as np

from oracle.swiglu import silu


def _rmsnorm(x, eps=1e-5):
    x = np.asarray(x, np.float64)
    return x / np.sqrt((x * x).mean(-1, keepdims=True) + eps)


def grouped_linear(x, w, keys):
    """y[t] = x[t] @ w[keys[t]] (the per-sample weight gather + bmm of rte/macro.py:208-221)."""
    x = np.asarray(x, np.float64)
    w = np.asarray(w, np.float64)
    return np.einsum("tk,tkn->tn", x, w[np.asarray(keys)])


def grouped_linear_bwd(dy, x, w, keys):
    """(dx, dw): dx[t] = dy[t] @ w[keys[t]]^T; dw[g] = sum over rows of group g of x^T dy."""
    dy = np.asarray(dy, np.float64)
    x = np.asarray(x, np.float64)
    w = np.asarray(w, np.float64)
    keys = np.asarray(keys)
    dx = np.einsum("tn,tkn->tk", dy, w[keys])
    dw = np.zeros_like(w)
    np.add.at(dw, keys, x[:, :, None] * dy[:, None, :])
    return dx, dw


def bounded_apply(h, h0, recipe_ids, stride_ids, p, update_scale_const, include_delta=False):
    """Phi(h) = h + c * scale * tanh(gain * h + silu(z v) u + bias) with
    z = [rmsnorm(h), mean_s rmsnorm(h), h0 (, rmsnorm(h) - rmsnorm(h0))]  (rte/macro.py:201-236).
    p holds d_gain, bias, update_scale [R, K, d], v [R, K, in, m], u [R, K, m, d], optional v2."""
    h = np.asarray(h, np.float64)
    h0 = np.asarray(h0, np.float64)
    out = np.empty_like(h)
    for b in range(h.shape[0]):
        r, k = int(recipe_ids[b]), int(stride_ids[b])
        n = _rmsnorm(h[b])
        parts = [n, np.broadcast_to(n.mean(0, keepdims=True), n.shape), h0[b]]
        if include_delta:
            parts.append(n - _rmsnorm(h0[b]))
        z = np.concatenate(parts, -1)
        low = silu(z @ p["v"][r, k])
        if p.get("v2") is not None:
            low = silu(low @ p["v2"][r, k])
        upd = p["d_gain"][r, k] * h[b] + low @ p["u"][r, k] + p["bias"][r, k]
        out[b] = h[b] + update_scale_const * p["update_scale"][r, k] * np.tanh(upd)
    return out
