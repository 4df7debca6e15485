"""Loss oracle (numpy, float64).  Test infrastructure only."""

from __future__ import annotations

import numpy as np


def cross_entropy(logits, targets):
    """Per-token CE and its logits gradient (rte/models.py:73-75, F.cross_entropy semantics)."""
    lg = np.asarray(logits, np.float64)
    mx = lg.max(-1, keepdims=True)
    lse = mx[..., 0] + np.log(np.exp(lg - mx).sum(-1))
    tg = np.asarray(targets).astype(np.int64)
    loss = lse - np.take_along_axis(lg, tg[..., None], -1)[..., 0]
    p = np.exp(lg - lse[..., None])
    onehot = np.zeros_like(p)
    np.put_along_axis(onehot, tg[..., None], 1.0, -1)
    return loss, lse, p - onehot


def audit_corrected(hot, exact, p):
    """corrected = hot + (exact - hot) / p on audited samples (rte/audit.py:318-321)."""
    return np.asarray(hot, np.float64) + (np.asarray(exact, np.float64) - hot) / np.asarray(p, np.float64)
