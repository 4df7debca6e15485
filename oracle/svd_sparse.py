"""SVD-factor sparse SwiGLU FFN oracle (numpy) — TEST INFRASTRUCTURE ONLY.

Restates SVDFactorSparseFFN.forward (rte/layers.py:446-643; rte/ = src/recursive_training_engine/
of the reference) per token, given the selector's approximate activations up_hat, gate_hat [T, F]:
candidate views (top up_m of |up_hat| w, top gate_m of |silu(gate_hat)| w, top product_m of
|up_hat silu(gate_hat)| w, w = ||W_down row||), their union, the fill from the product view when
the union is smaller than top_k, exact activations on the candidates, the exact rerank to top_k
and the sparse down-sum; "product" strategy (rte/kernels/svd_sparse_ffn_triton.py:570-576): the
top top_k of the product scores with the approximate activations.  Ties in every top-m go to
the lower neuron id (torch.topk leaves tie order unspecified).  Selector scores are formed in
float32 (the kernel's arithmetic), activations and sums in float64.
"""

from __future__ import annotations

import numpy as np

from oracle.swiglu import sigmoid, silu


def _top(scores, m):
    """Indices of the m largest scores, ties by lower index (NaN first), ascending index order."""
    s = np.asarray(scores)
    nan = np.isnan(s)
    order = np.lexsort((np.arange(s.size), np.where(nan, 0.0, -s.astype(np.float64)), (~nan).astype(np.int8)))
    return np.sort(order[:m])


def forward(x, w_up, w_gate, w_down, up_hat, gate_hat, *, up_m, gate_m, product_m, top_k, exact=True,
            product_only=False):
    """(out [T, d], selected ids [T, top_k] ascending, u, g of the selected)."""
    x = np.asarray(x, np.float64)
    wu, wg, wdn_rows = (np.asarray(a, np.float64) for a in (w_up, w_gate, w_down))
    w = np.sqrt((wdn_rows * wdn_rows).sum(-1)).astype(np.float32)
    uh = np.asarray(up_hat, np.float32)
    gh = np.asarray(gate_hat, np.float32)
    gs = (gh * (np.float32(1.0) / (np.float32(1.0) + np.exp(-gh)))).astype(np.float32)
    T, F = uh.shape
    out = np.zeros((T, x.shape[1]))
    sel_all = np.zeros((T, top_k), np.int64)
    u_all = np.zeros((T, top_k))
    g_all = np.zeros((T, top_k))
    for t in range(T):
        views = [(np.abs(uh[t]) * w, up_m), (np.abs(gs[t]) * w, gate_m), (np.abs(uh[t] * gs[t]) * w, product_m)]
        cand = set()
        if not product_only:
            for sc, m in views:
                if m > 0:
                    cand.update(_top(sc.astype(np.float32), min(m, F)).tolist())
        if len(cand) < top_k:
            cand.update(_top(views[2][0].astype(np.float32), min(top_k, F)).tolist())
        cid = np.array(sorted(cand))
        if exact:
            u, g = x[t] @ wu[cid].T, x[t] @ wg[cid].T
        else:
            u, g = uh[t, cid].astype(np.float64), gh[t, cid].astype(np.float64)
        es = np.abs(u * silu(g)) * w[cid]
        loc = _top(es, min(top_k, cid.size))
        sel = cid[loc]
        sel_all[t] = sel
        u_all[t], g_all[t] = u[loc], g[loc]
        out[t] = (u[loc] * silu(g[loc])) @ wdn_rows[sel]
    return out, sel_all, u_all, g_all


def backward(dout, x, w_up, w_gate, w_down, sel, u, g):
    """Gradients of the sparse FFN for a fixed selection: dx, dW_up, dW_gate, dW_down (float64)."""
    dout, x = np.asarray(dout, np.float64), np.asarray(x, np.float64)
    wu, wg, wd = (np.asarray(a, np.float64) for a in (w_up, w_gate, w_down))
    dz = np.einsum("td,tkd->tk", dout, wd[sel])
    s = sigmoid(g)
    du = dz * g * s
    dg = dz * u * s * (1.0 + g * (1.0 - s))
    dx = np.einsum("tk,tkd->td", du, wu[sel]) + np.einsum("tk,tkd->td", dg, wg[sel])
    dwu, dwg, dwd = np.zeros_like(wu), np.zeros_like(wg), np.zeros_like(wd)
    np.add.at(dwu, sel.reshape(-1), (du[:, :, None] * x[:, None, :]).reshape(-1, x.shape[1]))
    np.add.at(dwg, sel.reshape(-1), (dg[:, :, None] * x[:, None, :]).reshape(-1, x.shape[1]))
    np.add.at(dwd, sel.reshape(-1), ((u * silu(g))[:, :, None] * dout[:, None, :]).reshape(-1, x.shape[1]))
    return dx, dwu, dwg, dwd
