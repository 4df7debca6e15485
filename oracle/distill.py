"""Audit distillation oracle (numpy, float64) — TEST INFRASTRUCTURE ONLY.

Restates macro_distill_loss with the residual origin h0 (rte/macro.py:394-471; rte/ =
src/recursive_training_engine/ of the reference) and macro_alignment_metrics
(rte/macro.py:499-546) for A audited samples of shape [S, d], and the gradient of the
losses with respect to the hot hidden states and hot logits in closed form.
"""

from __future__ import annotations

import numpy as np

LOSSES = ("delta_dir", "delta_rms", "endpoint_normed", "endpoint_raw", "rms_trust", "kl")


def _sl1(z):
    a = np.abs(z)
    return np.where(a < 1.0, 0.5 * z * z, a - 0.5)


def _rmsnorm_rows(x, eps):
    return x / np.sqrt((x * x).mean(-1, keepdims=True) + eps)


def _log_softmax(x):
    m = x.max(-1, keepdims=True)
    return x - m - np.log(np.exp(x - m).sum(-1, keepdims=True))


def _cos(x, y):
    return (x * y).sum(-1) / np.maximum(np.sqrt((x * x).sum(-1) * (y * y).sum(-1)), 1e-8)


def distill(hot, exact, h0, hot_logits=None, exact_logits=None, t=1.0, eps=1e-5):
    """(losses dict, metrics dict) of rte/macro.py:394-471 (h0 branch) and :499-546."""
    hot, exact, h0 = (np.asarray(v, np.float64) for v in (hot, exact, h0))
    A = hot.shape[0]
    dp, de = (hot - h0).reshape(A, -1), (exact - h0).reshape(A, -1)
    hf, ef = hot.reshape(A, -1), exact.reshape(A, -1)
    rms = lambda v: np.sqrt((v * v).mean(-1))  # noqa: E731
    out = {
        "delta_dir": 1.0 - _cos(dp, de).mean(),
        "delta_rms": ((np.log(np.maximum(rms(dp), 1e-8)) - np.log(np.maximum(rms(de), 1e-8))) ** 2).mean(),
        "endpoint_normed": _sl1(_rmsnorm_rows(hot, eps) - _rmsnorm_rows(exact, eps)).mean(),
        "endpoint_raw": _sl1(hot - exact).mean(),
        "rms_trust": (np.log(np.maximum(rms(hf), 1e-8) / np.maximum(rms(ef), 1e-8)) ** 2).mean(),
        "kl": 0.0,
    }
    met = {
        "hidden_cosine_exact_macro": _cos(hf, ef).mean(),
        "hidden_mse_exact_macro": ((hot - exact) ** 2).mean(),
        "macro_norm": rms(hf).mean(),
        "exact_norm": rms(ef).mean(),
    }
    met["macro_exact_norm_ratio"] = met["macro_norm"] / max(met["exact_norm"], 1e-8)
    met["delta_cosine_exact_macro"] = _cos(dp, de).mean()
    met["delta_rms_exact"], met["delta_rms_pred"] = rms(de).mean(), rms(dp).mean()
    met["delta_rms_ratio"] = met["delta_rms_pred"] / max(met["delta_rms_exact"], 1e-8)
    if hot_logits is not None and exact_logits is not None:
        hl, el = np.asarray(hot_logits, np.float64), np.asarray(exact_logits, np.float64)
        logq, logp = _log_softmax(hl / t), _log_softmax(el / t)
        p = np.exp(logp)
        rows = np.where(p > 0, p * logp, 0.0) - p * logq
        out["kl"] = rows.sum() / A * t * t
        te, th = _log_softmax(el), _log_softmax(hl)
        met["logit_kl_exact_macro"] = (np.exp(te) * (te - th)).sum(-1).mean()
    return out, met


def distill_grad(hot, exact, h0, hot_logits=None, exact_logits=None, t=1.0, eps=1e-5, g=None):
    """(d hot, d hot_logits) of sum_i g[i] * losses[i] (order LOSSES)."""
    hot, exact, h0 = (np.asarray(v, np.float64) for v in (hot, exact, h0))
    g = np.ones(6) if g is None else np.asarray(g, np.float64)
    A = hot.shape[0]
    N = hot[0].size
    dp, de = (hot - h0).reshape(A, -1), (exact - h0).reshape(A, -1)
    hf, ef = hot.reshape(A, -1), exact.reshape(A, -1)
    w12, w1, w2 = (dp * de).sum(-1), (dp * dp).sum(-1), (de * de).sum(-1)
    D = np.sqrt(w1 * w2)
    cos = w12 / np.maximum(D, 1e-8)
    out = np.zeros_like(hf)
    # delta_dir = 1 - mean cos
    out += g[0] * (-(de / np.maximum(D, 1e-8)[:, None]) + np.where(D > 1e-8, cos / w1, 0.0)[:, None] * dp) / A
    # delta_rms
    rp, re_ = np.sqrt(w1 / N), np.sqrt(w2 / N)
    lr = np.log(np.maximum(rp, 1e-8)) - np.log(np.maximum(re_, 1e-8))
    out += g[1] * np.where(rp > 1e-8, 2.0 * lr / (rp * rp * N), 0.0)[:, None] * dp / A
    # rms_trust
    rh, rx = np.sqrt((hf * hf).sum(-1) / N), np.sqrt((ef * ef).sum(-1) / N)
    lt = np.log(np.maximum(rh, 1e-8) / np.maximum(rx, 1e-8))
    out += g[4] * np.where(rh > 1e-8, 2.0 * lt / (rh * rh * N), 0.0)[:, None] * hf / A
    # endpoint_raw
    out += g[3] * np.clip(hf - ef, -1.0, 1.0) / (A * N)
    # endpoint_normed: rmsnorm backward per row
    r = 1.0 / np.sqrt((hot * hot).mean(-1, keepdims=True) + eps)
    u = g[2] * np.clip(_rmsnorm_rows(hot, eps) - _rmsnorm_rows(exact, eps), -1.0, 1.0) / (A * N)
    dn = r * u - hot * r ** 3 * (u * hot).mean(-1, keepdims=True)
    out += dn.reshape(A, -1)
    dlog = None
    if hot_logits is not None and exact_logits is not None:
        hl, el = np.asarray(hot_logits, np.float64), np.asarray(exact_logits, np.float64)
        q, p = np.exp(_log_softmax(hl / t)), np.exp(_log_softmax(el / t))
        dlog = g[5] * t / A * (q - p)
    return out.reshape(hot.shape), dlog
