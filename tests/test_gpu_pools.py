"""The static cluster-pool build (rte_amd/pools.py) end to end on the GPU: calibration batches
through a dense model's HIP blocks, factors and codebook in the shapes StaticClusterPoolSwiGLU
takes, a full-width codebook reproducing the dense SwiGLU (the reference's full pool == dense
invariant), the selector features of the calibration pass against a float64 restatement of the
block, and a rebuild giving the same codebook."""

from __future__ import annotations

import pytest
import torch

pytestmark = pytest.mark.gpu

DEV = "cuda"


@pytest.fixture(scope="module", autouse=True)
def _hip():
    from rte_amd import _lib

    if not _lib.device_ready():
        pytest.fail("HIP backend not ready on this GPU box (library or gfx950 device missing)")
    yield


def _rel(a, b):
    a, b = a.detach().double(), b.detach().double()
    return float((a - b).norm() / b.norm().clamp_min(1e-300))


def test_static_codebook_build_and_use():
    from oracle import step_port as SP
    from rte_amd import pools as PL
    from rte_amd.config import ModelConfig
    from rte_amd.kernels import hip_ops
    from rte_amd.layers import StaticClusterPoolSwiGLU
    from rte_amd.models import DenseModel

    cfg = ModelConfig(topology="dense", vocab_size=64, d_model=128, n_heads=4, d_ff=256, n_dense_layers=2,
                      n_prelude=1, n_coda=1, t_max=1, depth_choices=[1], attn_banks=1, ffn_banks=1, head_groups=4,
                      ffn_groups=4, active_head_groups=1, active_ffn_groups=1, recipe_count=2)
    torch.manual_seed(3)
    dense = DenseModel(cfg).to(DEV)
    with torch.no_grad():
        for blk in dense.blocks:
            for p in (blk.attn.wqkv.weight, blk.attn.wo.weight, blk.mlp.wug.weight, blk.mlp.wd.weight):
                p.mul_(0.5)
    g = torch.Generator().manual_seed(0)
    data = [(torch.randint(0, 64, (4, 32), generator=g), None) for _ in range(3)]
    rank, C, M = 8, 6, 64
    factors = PL.build_svd_factor_cache(dense, max_rank=16, device=torch.device(DEV))

    def build(m):
        return PL.build_static_svd_cluster_pool_codebook(
            dense, factors, iter(data), calibration_batches=2, device=torch.device(DEV), rank=rank, cluster_count=C,
            candidate_m=m, score_mode="sum", aggregation="mean", cluster_iters=4)

    codebook, metrics = build(M)
    assert metrics["calibration_tokens_seen"] == 2 * 4 * 32
    assert len(codebook) == 2
    for cb in codebook:
        assert cb["centers"].shape == (C, 2 * rank) and cb["candidate_ids"].shape == (C, M)
        assert torch.allclose(cb["centers"].norm(dim=-1), torch.ones(C, device=DEV), atol=1e-5)
        ids = cb["candidate_ids"]
        assert int(ids.min()) >= 0 and int(ids.max()) < 256
        assert all(len(set(r)) == M for r in ids.tolist())
    again, _ = build(M)
    for a, b in zip(codebook, again):
        assert torch.equal(a["candidate_ids"], b["candidate_ids"]) and torch.equal(a["centers"], b["centers"])
    # the calibration features of block 0 against a float64 restatement of the block
    tok = data[0][0].to(DEV)
    P = {n: p.detach().double() for n, p in dense.blocks[0].named_parameters()}
    x0 = dense.embed.weight.detach().double()[tok]
    cos, sin = SP.rope_tables(32, 32, torch.float64)
    u = x0 + SP.dense_attention(SP.rmsnorm(x0, P["norm1.weight"]), P["attn.wqkv.weight"], P["attn.wo.weight"], 4,
                                cos.to(DEV), sin.to(DEV))
    normed = SP.rmsnorm(u, P["norm2.weight"]).reshape(-1, 128)
    with hip_ops.fp32_precision():
        x = dense.embed(tok).float()
        blk = dense.blocks[0]
        got, _ = PL.svd_cluster_features_and_scores(blk, blk.norm2(blk.attn(blk.norm1(x), resid=x)), factors[0],
                                                    rank=rank, score_mode="sum")
    ref = torch.cat([normed @ factors[0]["up_a"][:, :rank].double(), normed @ factors[0]["gate_a"][:, :rank].double()],
                    -1)
    assert _rel(got, ref) < 1e-5
    # a full-width codebook (every neuron in every pool) reproduces the dense SwiGLU
    full, _ = build(256)
    layer = StaticClusterPoolSwiGLU(dense.blocks[0].mlp, factors[0], full[0], rank=rank).to(DEV)
    xin = torch.randn(2, 40, 128, device=DEV, generator=torch.Generator(device=DEV).manual_seed(1))
    with hip_ops.fp32_precision():
        ref_y = dense.blocks[0].mlp(xin)
    y = layer(xin.to(torch.bfloat16))
    assert _rel(y.float(), ref_y) < 2e-2
