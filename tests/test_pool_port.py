"""Pins of the CPU cluster-pool layer forms (oracle/pool_port.py) timed as the cfg1 CPU baseline:
both forms' outputs equal oracle.cluster_pool.routed_fwd (itself pinned: all clusters with
uniform weights = dense SwiGLU / C, k = 1 = the reference's per-cluster loop) on the same
routing, and the two forms' gradients agree with each other and with finite differences."""

from __future__ import annotations

import numpy as np
import torch

from oracle import cluster_pool as OCP
from oracle import pool_port as PP
from oracle import routing as OR


def _case(T=96, d=32, C=8, n=32, seed=3):
    return PP.make_cfg1(T, d, C, n, seed)


def test_forms_equal_routed_oracle():
    x, wr, wup, wgate, wdown = (t.double() for t in _case())
    k, C = 3, 8
    ids, w = PP.route(x, wr, k)
    rid, rw = OR.route_topk((x @ wr).float().numpy(), k)
    assert np.array_equal(ids.numpy(), rid)
    wug = torch.cat([wup, wgate]).numpy()
    ref = OCP.routed_fwd(x.numpy(), wug, wdown.t().numpy(), ids.numpy(), w.numpy(), C)
    for form in (PP.layer_loop, PP.layer_preindexed):
        got = form(x, wr, wup, wgate, wdown, k, C).numpy()
        assert np.allclose(got, ref, rtol=1e-12, atol=1e-12), form.__name__


def test_forms_gradients_agree():
    x, wr, wup, wgate, wdown = (t.double() for t in _case(seed=5))
    dy = torch.randn(x.shape, generator=torch.Generator().manual_seed(1), dtype=torch.float64)
    k, C = 4, 8
    o1, g1 = PP.fwd_bwd(PP.layer_loop, x, wr, wup, wgate, wdown, dy, k, C)
    o2, g2 = PP.fwd_bwd(PP.layer_preindexed, x, wr, wup, wgate, wdown, dy, k, C)
    assert torch.allclose(o1, o2, rtol=1e-12, atol=1e-13)
    for a, b in zip(g1, g2):
        assert torch.allclose(a, b, rtol=1e-10, atol=1e-12)
    # finite differences of <out, dy> on a few weight entries (routing fixed: tiny steps)
    eps = 1e-6
    for ti, i in ((1, 5), (2, 37), (3, 100), (4, 222), (0, 64)):
        ts = [t.clone() for t in (x, wr, wup, wgate, wdown)]
        vals = []
        for s in (1.0, -1.0):
            ts2 = [t.clone() for t in ts]
            ts2[ti].view(-1)[i] += s * eps
            vals.append(float((PP.layer_loop(*ts2, k, C) * dy).sum()))
        fd = (vals[0] - vals[1]) / (2 * eps)
        an = float(g1[ti].view(-1)[i])
        assert abs(fd - an) <= 1e-6 * max(1.0, abs(an)), (ti, i, fd, an)
