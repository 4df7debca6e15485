"""Static cluster-pool construction (rte_amd/pools.py, rte/cli.py:3244-3388, 4703-4782,
4915-4941) on the CPU: k-means against a brute-force loop, the score aggregations and the capped
union against explicit enumeration, the SVD factor cache by the Eckart-Young closed form."""

from __future__ import annotations

import math

import pytest
import torch

from rte_amd import pools as PL


def _brute_kmeans(feats, C, iters):
    """Cosine k-means one row / one cluster at a time in float64 (first maximal centre wins)."""
    x = [[v / math.sqrt(sum(u * u for u in f)) for v in f] for f in feats.double().tolist()]
    n = len(x)
    init = [round(i * (n - 1) / (C - 1)) for i in range(C)]
    centers = [list(x[i]) for i in init]
    assign = [0] * n
    for _ in range(iters):
        for i, xi in enumerate(x):
            best, bi = None, 0
            for c, cc in enumerate(centers):
                s = sum(a * b for a, b in zip(xi, cc))
                if best is None or s > best:
                    best, bi = s, c
            assign[i] = bi
        new = []
        for c in range(C):
            rows = [x[i] for i in range(n) if assign[i] == c]
            if rows:
                m = [sum(col) / len(rows) for col in zip(*rows)]
                norm = math.sqrt(sum(v * v for v in m)) or 1.0
                new.append([v / norm for v in m])
            else:
                new.append(centers[c])
        centers = new
    return torch.tensor(assign), torch.tensor(centers, dtype=torch.float64)


@pytest.mark.parametrize("n,f,C,iters", [(40, 6, 4, 5), (57, 10, 7, 3), (9, 4, 3, 1)])
def test_kmeans_matches_brute_force(n, f, C, iters):
    g = torch.Generator().manual_seed(n)
    # separated blobs plus noise, so no assignment sits on a tie
    centres = torch.randn(C, f, generator=g) * 3
    feats = (centres[torch.arange(n) % C] + 0.3 * torch.randn(n, f, generator=g)).double()
    a, c = PL.fit_cluster_centers(feats, cluster_count=C, iters=iters)
    ra, rc = _brute_kmeans(feats, C, iters)
    assert torch.equal(a, ra)
    assert torch.allclose(c.double(), rc, atol=1e-6)
    assert torch.equal(PL.cluster_assignments_from_features(feats, cluster_count=C, iters=iters), ra)


def test_kmeans_degenerate_counts():
    feats = torch.randn(5, 3, dtype=torch.float64)
    a, c = PL.fit_cluster_centers(feats, cluster_count=1, iters=3)
    assert torch.equal(a, torch.zeros(5, dtype=torch.long))
    m = torch.nn.functional.normalize(feats, dim=-1).mean(0)
    assert torch.allclose(c[0].double(), m / m.norm())
    a, c = PL.fit_cluster_centers(feats[:1], cluster_count=4, iters=3)  # capped at one row
    assert a.tolist() == [0] and c.shape == (1, 3)


def test_aggregate_scores_mean_and_max():
    g = torch.Generator().manual_seed(3)
    s = torch.rand(30, 12, generator=g)
    a = torch.randint(0, 5, (30,), generator=g)
    a[a == 3] = 4  # cluster 3 stays empty
    mean = PL.aggregate_cluster_scores(s, a, cluster_count=5, aggregation="mean")
    mx = PL.aggregate_cluster_scores(s, a, cluster_count=5, aggregation="max")
    for c in range(5):
        rows = [s[i] for i in range(30) if int(a[i]) == c]
        if rows:
            assert torch.allclose(mean[c], torch.stack(rows).sum(0) / len(rows))
            assert torch.equal(mx[c], torch.stack(rows).max(0).values)
        else:
            assert torch.all(mean[c] == 0) and torch.all(mx[c] == 0)
    with pytest.raises(ValueError):
        PL.aggregate_cluster_scores(s, a, cluster_count=5, aggregation="median")


def test_active_union_ids():
    cand = torch.tensor([[5, 1, 9], [9, 2, 7], [1, 5, 3]])
    assert PL.active_union_ids_from_codebook(cand, hidden=12).tolist() == [1, 2, 3, 5, 7, 9]
    assert PL.active_union_ids_from_codebook(cand, hidden=12, cap=6).tolist() == [1, 2, 3, 5, 7, 9]
    # capped: score = sum over appearances of the rank weight (1, 2/3, 1/3 for M = 3)
    w = [1.0, 2.0 / 3.0, 1.0 / 3.0]
    score = {}
    for row in cand.tolist():
        for j, v in enumerate(row):
            score[v] = score.get(v, 0.0) + w[j]
    top = sorted(sorted(score, key=lambda v: -score[v])[:3])
    assert PL.active_union_ids_from_codebook(cand, hidden=12, cap=3).tolist() == top


def test_svd_factor_cache_closed_form():
    """A B is the best rank-r approximation of W^T (d x F): full rank reconstructs it, rank r leaves
    the Frobenius error sqrt(sum of the dropped squared singular values)."""
    from rte_amd.config import ModelConfig
    from rte_amd.models import DenseModel

    cfg = ModelConfig(topology="dense", vocab_size=32, d_model=16, n_heads=2, d_ff=24, n_dense_layers=2,
                      n_prelude=1, n_coda=1, t_max=1, depth_choices=[1], attn_banks=1, ffn_banks=1, head_groups=2,
                      ffn_groups=2, active_head_groups=1, active_ffn_groups=1, recipe_count=2)
    torch.manual_seed(0)
    dense = DenseModel(cfg)
    full = PL.build_svd_factor_cache(dense, max_rank=64, device=torch.device("cpu"))
    low = PL.build_svd_factor_cache(dense, max_rank=5, device=torch.device("cpu"))
    assert len(full) == 2
    for blk, fl, lo in zip(dense.blocks, full, low):
        up_w, gate_w = blk.mlp.wug.weight.detach().chunk(2, dim=0)
        for name, w in (("up", up_w), ("gate", gate_w)):
            wt = w.t()
            assert fl[f"{name}_a"].shape == (16, 16) and lo[f"{name}_a"].shape == (16, 5)
            assert torch.allclose(fl[f"{name}_a"] @ fl[f"{name}_b"], wt, atol=1e-5)
            s = torch.linalg.svdvals(wt.double())
            err = (lo[f"{name}_a"] @ lo[f"{name}_b"] - wt).double().norm()
            assert abs(float(err) - float(s[5:].square().sum().sqrt())) < 1e-4
