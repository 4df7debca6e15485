"""Shortlist output-head oracle (numpy) — TEST INFRASTRUCTURE ONLY.

Restates rte/output.py:30-136 and rte/kernels/reference.py:141-147 (rte/ =
src/recursive_training_engine/ of the reference).  The random negatives are an input:
the reference draws them with a seeded device generator (rte/output.py:86-94), which
the oracle does not reproduce.
"""

from __future__ import annotations

import numpy as np


def cluster_member_table(vocab_size: int, num_clusters: int):
    """Padded member table: token v belongs to cluster v % C, rows padded with id 0
    (rte/output.py:30-40).  Returns (members [C, ceil(V / C)] int64, counts [C])."""
    per = (vocab_size + num_clusters - 1) // num_clusters
    members = np.zeros((num_clusters, per), np.int64)
    counts = np.zeros(num_clusters, np.int64)
    for v in range(vocab_size):
        c = v % num_clusters
        members[c, counts[c]] = v
        counts[c] += 1
    return members, counts


def build_candidates(targets, top_clusters, members, hard_negatives: int, random_negs, max_tokens: int,
                     vocab_size: int):
    """[target | members of the top clusters | arange(H) % V | random negatives |
    arange(L) % V | (target + arange(2L)) % V] per token (rte/output.py:96-106)."""
    tg = np.asarray(targets, np.int64).reshape(-1)
    T = tg.shape[0]
    top = np.asarray(top_clusters, np.int64).reshape(T, -1)
    mem = np.asarray(members, np.int64)[top].reshape(T, -1)
    hard = np.broadcast_to(np.arange(hard_negatives, dtype=np.int64) % vocab_size, (T, hard_negatives))
    rnd = np.asarray(random_negs, np.int64).reshape(T, -1)
    filler = np.broadcast_to(np.arange(max_tokens, dtype=np.int64) % vocab_size, (T, max_tokens))
    tfill = (tg[:, None] + np.arange(2 * max_tokens, dtype=np.int64)[None, :]) % vocab_size
    return np.concatenate([tg[:, None], mem, hard, rnd, filler, tfill], axis=1)


def dedupe_preserve_first(candidates, max_tokens: int):
    """First L distinct ids of each row in order of first occurrence, and the per-row
    count of repeated candidates (rte/output.py:46-70: first positions by amin, then the
    L smallest first positions in ascending order)."""
    cand = np.asarray(candidates, np.int64)
    T, width = cand.shape
    out = np.empty((T, max_tokens), np.int64)
    dup = np.empty(T, np.int64)
    for t in range(T):
        ids, first = np.unique(cand[t], return_index=True)
        order = np.argsort(first, kind="stable")
        out[t] = ids[order[:max_tokens]]
        dup[t] = width - ids.shape[0]
    return out, dup


def build_shortlist(targets, top_clusters, members, hard_negatives, random_negs, max_tokens, vocab_size):
    """ShortlistHead.build_shortlist with the cluster top-k already taken (rte/output.py:72-110).
    Returns (shortlist [T, L], dup_per_token [T]); the target position is always 0."""
    cand = build_candidates(targets, top_clusters, members, hard_negatives, random_negs, max_tokens, vocab_size)
    return dedupe_preserve_first(cand, max_tokens)


def shortlist_logits_ce(hidden, weight, shortlist):
    """logits[t, j] = hidden[t] . W[shortlist[t, j]] (rte/kernels/reference.py:141-143) and
    CE against position 0 (rte/output.py:125-129).  Returns (logits, lse, loss) in float64."""
    h = np.asarray(hidden, np.float64)
    w = np.asarray(weight, np.float64)
    sl = np.asarray(shortlist, np.int64)
    logits = np.einsum("td,tjd->tj", h, w[sl])
    mx = logits.max(-1, keepdims=True)
    lse = mx[:, 0] + np.log(np.exp(logits - mx).sum(-1))
    return logits, lse, lse - logits[:, 0]


def shortlist_logits_ce_bwd(hidden, weight, shortlist, logits, lse, dloss=None, dlogits=None):
    """Gradients of the above: g = dloss (softmax - e_0) + dlogits; dhidden = sum_j g W[sl];
    dW[v] = sum over (t, j) with sl[t, j] = v of g[t, j] hidden[t]."""
    h = np.asarray(hidden, np.float64)
    w = np.asarray(weight, np.float64)
    sl = np.asarray(shortlist, np.int64)
    lg = np.asarray(logits, np.float64)
    g = np.zeros_like(lg)
    if dloss is not None:
        p = np.exp(lg - np.asarray(lse, np.float64)[:, None])
        p[:, 0] -= 1.0
        g += np.asarray(dloss, np.float64)[:, None] * p
    if dlogits is not None:
        g += np.asarray(dlogits, np.float64)
    dh = np.einsum("tj,tjd->td", g, w[sl])
    dw = np.zeros_like(w)
    np.add.at(dw, sl.reshape(-1), (g[:, :, None] * h[:, None, :]).reshape(-1, h.shape[1]))
    return g, dh, dw
