"""Control-variate audit correction oracle (numpy, float64) — TEST INFRASTRUCTURE ONLY.

Restates the loss arithmetic of AuditEngine.correction (rte/audit.py:305-321; rte/ =
src/recursive_training_engine/ of the reference) over the per-sample loss of
lm_loss_per_sample (rte/models.py:73-75, a sum of token cross-entropies over the sequence).
The audited rows are given as distinct indices ``idx`` (the reference's boolean mask, in any
order), the inclusion probabilities ``p`` per sample.
"""

from __future__ import annotations

import numpy as np


def correction(hot_tok, exact_tok, idx, p, clip=None, grad_corrected=True):
    """Returns (corrected [B], exact per-sample [A], stats [4]) with stats = residual mean,
    std, var (population, before the clip: rte/audit.py:307-309) and the corrected metric
    mean(hot + clip(r) / p) (:316-317).  corrected[idx] = hot + clip(r) / p only in the
    gradient-corrected mode (:318-321)."""
    hot = np.asarray(hot_tok, np.float64).sum(-1)
    exact = np.asarray(exact_tok, np.float64).reshape(len(idx), np.shape(hot_tok)[-1]).sum(-1)
    idx = np.asarray(idx, np.int64)
    hs = hot[idx]
    r = exact - hs
    stats = np.array([r.mean(), r.std(), r.var(), 0.0]) if r.size else np.zeros(4)
    rc = r if clip is None else np.clip(r, -clip, clip)
    ps = np.maximum(np.asarray(p, np.float64)[idx], 1e-12)
    if r.size:
        stats[3] = (hs + rc / ps).mean()
    corrected = hot.copy()
    if grad_corrected:
        corrected[idx] = hs + rc / ps
    return corrected, exact, stats


def correction_bwd(g, hot_tok, exact_tok, idx, p, clip=None, grad_corrected=True):
    """Gradients of corrected w.r.t. the token losses for an upstream gradient g [B]:
    d corrected[m] / d hot_tok[m, s] = 1 - c, d corrected[idx[a]] / d exact_tok[a, s] = c, with
    c = 1 / p on audited rows whose residual lies inside the clip (clamp passes the gradient on
    the closed interval) in the gradient-corrected mode, else 0."""
    hot_tok = np.asarray(hot_tok, np.float64)
    B, S = hot_tok.shape
    idx = np.asarray(idx, np.int64)
    g = np.asarray(g, np.float64)
    exact = np.asarray(exact_tok, np.float64).reshape(len(idx), np.shape(hot_tok)[-1]).sum(-1)
    r = exact - hot_tok.sum(-1)[idx]
    inside = np.ones_like(r, bool) if clip is None else (r >= -clip) & (r <= clip)
    c = np.where(inside & grad_corrected, 1.0 / np.maximum(np.asarray(p, np.float64)[idx], 1e-12), 0.0)
    coef = np.zeros(B)
    coef[idx] = c
    dhot = np.repeat((g * (1.0 - coef))[:, None], S, axis=1)
    dexact = np.repeat((g[idx] * c)[:, None], S, axis=1)
    return dhot, dexact
