"""Routed cluster-pool SwiGLU oracle (numpy, float64).  Test infrastructure only.

Cluster c owns neurons [c*n, (c+1)*n) of a SwiGLU with d_ff = C*n; each token is
routed to k clusters with weights w (softmax over the selected router logits) and
out[t] = resid[t] + sum_j w_tj * SwiGLU_{c_tj}(x_t).  With k = 1 this is the
reference per-cluster loop oracle cluster_pool_ffn_reference
(rte/kernels/cluster_pool_ffn.py:143-162) over pools gathered by
prepare_cluster_pool_weights (:90-126) for a partition of the neurons.
"""

from __future__ import annotations

import numpy as np

from oracle.routing import route_softmax_bwd
from oracle.swiglu import sigmoid, silu


def cluster_pool_reference_loop(x, assignments, wup_pool, wgate_pool, wdown_pool):
    """Literal restatement of cluster_pool_ffn_reference (rte/kernels/cluster_pool_ffn.py:143-162):
    pools wup/wgate [C, d, M], wdown [C, M, d]; one cluster per token."""
    x = np.asarray(x, np.float64)
    out = np.zeros_like(x)
    for c in range(wup_pool.shape[0]):
        tok = np.nonzero(assignments == c)[0]
        if tok.size == 0:
            continue
        xc = x[tok]
        up = xc @ wup_pool[c]
        gate = xc @ wgate_pool[c]
        out[tok] = (up * silu(gate)) @ wdown_pool[c]
    return out


def prepare_pools(w_up, w_gate, w_down_rows, candidate_ids):
    """prepare_cluster_pool_weights (rte/kernels/cluster_pool_ffn.py:90-126): gather candidate
    rows into [C, d, M], [C, d, M], [C, M, d]."""
    ids = np.asarray(candidate_ids).astype(np.int64)
    return (
        np.transpose(w_up[ids], (0, 2, 1)),
        np.transpose(w_gate[ids], (0, 2, 1)),
        w_down_rows[ids],
    )


def routed_fwd(x, wug, wd, ids, w, n_clusters, resid=None):
    """Forward with given routing decisions.  wug [2F, d] rows [up; gate], wd [d, F] (Linear)."""
    x = np.asarray(x, np.float64)
    wug = np.asarray(wug, np.float64)
    wd = np.asarray(wd, np.float64)
    T, d = x.shape
    F = wug.shape[0] // 2
    n = F // n_clusters
    k = ids.shape[1]
    out = np.zeros((T, d)) if resid is None else np.asarray(resid, np.float64).copy()
    flat = ids.reshape(-1)
    for c in range(n_clusters):
        pairs = np.nonzero(flat == c)[0]
        if pairs.size == 0:
            continue
        tok = pairs // k
        wt = w.reshape(-1)[pairs].astype(np.float64)
        up = x[tok] @ wug[c * n:(c + 1) * n].T
        gate = x[tok] @ wug[F + c * n:F + (c + 1) * n].T
        z = up * silu(gate)
        y = (wt[:, None] * z) @ wd[:, c * n:(c + 1) * n].T
        np.add.at(out, tok, y)
    return out


def routed_bwd(dout, x, wr, wug, wd, ids, w, n_clusters):
    """Backward of routed_fwd followed by the router softmax (weights depend on logits = x Wr^T).

    Returns dx, dwr, dwug, dwd, dw_pair (routing-weight gradient per pair)."""
    dout = np.asarray(dout, np.float64)
    x = np.asarray(x, np.float64)
    wr = np.asarray(wr, np.float64)
    wug = np.asarray(wug, np.float64)
    wd = np.asarray(wd, np.float64)
    T, d = x.shape
    F = wug.shape[0] // 2
    n = F // n_clusters
    k = ids.shape[1]
    dx = np.zeros_like(x)
    dwug = np.zeros_like(wug)
    dwd = np.zeros_like(wd)
    dw_pair = np.zeros(T * k)
    flat = ids.reshape(-1)
    wf = w.reshape(-1).astype(np.float64)
    for c in range(n_clusters):
        pairs = np.nonzero(flat == c)[0]
        if pairs.size == 0:
            continue
        tok = pairs // k
        wt = wf[pairs]
        xs = x[tok]
        wu = wug[c * n:(c + 1) * n]
        wg = wug[F + c * n:F + (c + 1) * n]
        wdc = wd[:, c * n:(c + 1) * n]
        up = xs @ wu.T
        gate = xs @ wg.T
        z = up * silu(gate)
        dzw = dout[tok] @ wdc  # gradient wrt w*z
        dw_pair[pairs] = (z * dzw).sum(-1)
        dz = wt[:, None] * dzw
        s = sigmoid(gate)
        dup = dz * gate * s
        dgate = dz * up * s * (1.0 + gate * (1.0 - s))
        np.add.at(dx, tok, dup @ wu + dgate @ wg)
        dwug[c * n:(c + 1) * n] += dup.T @ xs
        dwug[F + c * n:F + (c + 1) * n] += dgate.T @ xs
        dwd[:, c * n:(c + 1) * n] += dout[tok].T @ (wt[:, None] * z)
    dlog = route_softmax_bwd(ids, w, dw_pair.reshape(T, k), n_clusters)
    dx += dlog @ wr
    dwr = dlog.T @ x
    return dx, dwr, dwug, dwd, dw_pair
