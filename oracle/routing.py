"""Routing and packing oracle (numpy, CPU).  Test infrastructure only."""

from __future__ import annotations

import numpy as np


def route_topk(logits: np.ndarray, k: int) -> tuple[np.ndarray, np.ndarray]:
    """Per-token top-k clusters of fp32 router logits and softmax weights over them.

    Order rule: value descending, ties by ascending cluster index, NaN ranked above
    every number (torch.topk puts NaN first).  k = 1 is the argmax routing of
    route_to_static_centers (rte/kernels/cluster_pool_ffn.py:129-140); the
    softmax-over-selected weights follow the factorized top-k combine
    (rte/models.py:300-309).
    """
    lg = np.asarray(logits, dtype=np.float32)
    T, C = lg.shape
    nan = np.isnan(lg)
    # lexsort: last key is primary.  primary: not-NaN (NaN first), then -value, then index.
    vals = np.where(nan, 0.0, -lg.astype(np.float64))
    idx = np.broadcast_to(np.arange(C), (T, C))
    order = np.lexsort((idx, vals, (~nan).astype(np.int8)), axis=-1)
    ids = order[:, :k].astype(np.int32)
    sel = np.take_along_axis(lg, ids, axis=-1).astype(np.float64)
    sel = sel - sel[:, :1]
    e = np.exp(sel)
    w = (e / e.sum(axis=-1, keepdims=True)).astype(np.float32)
    return ids, w


def pack_index(cl: np.ndarray, n_clusters: int, k: int) -> dict[str, np.ndarray]:
    """Stable counting sort of pairs p = t*k + j by cluster.

    Within a cluster the slots follow ascending pair index, i.e. ascending token —
    the order the reference index builder produces with nonzero()
    (rte/kernels/cluster_pool_ffn.py:179-188).
    """
    cl = np.asarray(cl).reshape(-1)
    P = cl.size
    valid = (cl >= 0) & (cl < n_clusters)
    counts = np.bincount(cl[valid], minlength=n_clusters)
    offsets = np.zeros(n_clusters + 1, dtype=np.int64)
    offsets[1:] = np.cumsum(counts)
    pair_of_slot = np.argsort(np.where(valid, cl, n_clusters), kind="stable")[: int(offsets[-1])]
    slot_of_pair = np.full(P, -1, dtype=np.int64)
    slot_of_pair[pair_of_slot] = np.arange(pair_of_slot.size)
    return {
        "offsets": offsets.astype(np.int32),
        "pair_of_slot": pair_of_slot.astype(np.int32),
        "tok_of_slot": (pair_of_slot // k).astype(np.int32),
        "slot_of_pair": slot_of_pair.astype(np.int32),
        "invalid": int((~valid).sum()),
    }


def static_pack_gather(assignments: np.ndarray, n_clusters: int):
    """Padded index build of build_static_pack_gather_indices (rte/kernels/cluster_pool_ffn.py:165-189).

    Returns (pack_index [C, max_count] zero padded, flat_gather [T], counts [C], max_count).
    """
    a = np.asarray(assignments).astype(np.int64)
    counts = np.bincount(a, minlength=n_clusters)
    max_count = int(counts.max()) if counts.size else 0
    pack = np.zeros((n_clusters, max_count), dtype=np.int64)
    flat = np.empty(a.shape[0], dtype=np.int64)
    for c in range(n_clusters):
        tok = np.nonzero(a == c)[0]
        pack[c, : tok.size] = tok
        flat[tok] = c * max_count + np.arange(tok.size)
    return pack, flat, counts, max_count


def route_softmax_bwd(ids: np.ndarray, w: np.ndarray, dw: np.ndarray, n_clusters: int) -> np.ndarray:
    """d logits of w = softmax(logits[ids]):  w_j (dw_j - sum_i w_i dw_i) at ids, 0 elsewhere."""
    T, k = ids.shape
    w = w.astype(np.float64)
    dw = dw.astype(np.float64)
    s = (w * dw).sum(axis=-1, keepdims=True)
    g = w * (dw - s)
    out = np.zeros((T, n_clusters), dtype=np.float64)
    np.put_along_axis(out, ids.astype(np.int64), g, axis=-1)
    return out


def segment_reduce_rows(keys, n_keys, rows, w=None, row_div=1):
    """out[v] = sum over p with keys[p] = v of w[p] * rows[p // row_div] (float64); keys outside
    [0, n_keys) are skipped -- the index_add_ scatter of rte/kernels/cluster_pool_ffn.py:235-240."""
    k = np.asarray(keys, np.int64).reshape(-1)
    r = np.asarray(rows, np.float64)
    wt = np.ones(k.shape[0]) if w is None else np.asarray(w, np.float64).reshape(-1)
    out = np.zeros((n_keys, r.shape[-1]))
    ok = (k >= 0) & (k < n_keys)
    src = r[np.arange(k.shape[0]) // row_div]
    np.add.at(out, k[ok], wt[ok, None] * src[ok])
    return out


def static_centers(q, centers):
    """route_to_static_centers (rte/kernels/cluster_pool_ffn.py:129-140) on precomputed selector
    features q = [x A_up | x A_gate]: argmax_c of normalize(q) . centers[c], normalize dividing
    by max(||q||, 1e-12) as F.normalize; the first maximal index wins (torch.argmax)."""
    q = np.asarray(q, np.float64)
    nrm = np.maximum(np.sqrt((q * q).sum(-1, keepdims=True)), 1e-12)
    scores = (q / nrm) @ np.asarray(centers, np.float64).T
    return np.argmax(scores, axis=-1).astype(np.int64), scores

