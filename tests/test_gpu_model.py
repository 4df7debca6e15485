"""GPU tests of the model-level path: a full dense block (fused QKV + RoPE + attention +
O-proj + dense SwiGLU) against a float32 torch reference of the same
block on the CPU, and one train step of every accelerated mode."""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from helpers import BF16_RTOL, assert_rel

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _hip():
    from rte_amd import _lib

    if not _lib.device_ready():
        pytest.fail("HIP backend not ready on this GPU box")


def _model_cfg(**over):
    from rte_amd.config import ModelConfig

    base = dict(topology="recursive", vocab_size=256, d_model=128, n_heads=4, d_ff=512, n_dense_layers=2, n_prelude=1,
                n_coda=1, t_max=4, depth_choices=[1, 2, 4], attn_banks=1, ffn_banks=2, head_groups=4, ffn_groups=16,
                active_head_groups=1, active_ffn_groups=4, recipe_count=6, macro_rank=8, router_hidden=64,
                ffn_kind="cluster_pool", ffn_clusters=16, ffn_top_k=2)
    base.update(over)
    return ModelConfig(**base)


def _ref_block(block, x):
    """float32 torch math of TransformerBlock (rte/layers.py:53-87, :646-656)."""
    def rms(v, w):
        return v * torch.rsqrt(v.pow(2).mean(-1, keepdim=True) + 1e-5) * w

    b, s, d = x.shape
    H = block.attn.n_heads
    hd = d // H
    n1 = rms(x, block.norm1.weight)
    qkv = (n1 @ block.attn.wqkv.weight.t()).view(b, s, 3, H, hd)
    q, k, v = (t.transpose(1, 2) for t in qkv.unbind(2))
    cos, sin = block.attn.rope.cos[:s], block.attn.rope.sin[:s]

    def rot(t):
        return torch.stack((-t[..., 1::2], t[..., ::2]), -1).flatten(-2)

    q = q * cos + rot(q) * sin
    k = k * cos + rot(k) * sin
    att = (q @ k.transpose(-1, -2)) / math.sqrt(hd)
    att = att.masked_fill(torch.triu(torch.ones(s, s, dtype=torch.bool), 1), float("-inf")).softmax(-1)
    y = (att @ v).transpose(1, 2).reshape(b, s, d)
    u = x + y @ block.attn.wo.weight.t()
    n2 = rms(u, block.norm2.weight)
    up, gate = (n2 @ block.mlp.wug.weight.t()).chunk(2, -1)
    return u + (up * F.silu(gate)) @ block.mlp.wd.weight.t()


@pytest.mark.parametrize("B,S,d,H,F_", [(4, 32, 128, 2, 256), (128, 64, 512, 8, 2048)])
def test_dense_block_matches_fp32_reference(B, S, d, H, F_):
    from rte_amd.config import ModelConfig
    from rte_amd.layers import TransformerBlock

    cfg = ModelConfig(topology="dense", vocab_size=64, d_model=d, n_heads=H, d_ff=F_, n_dense_layers=1, n_prelude=1,
                      n_coda=1, t_max=1, depth_choices=[1], attn_banks=1, ffn_banks=1, head_groups=1, ffn_groups=1,
                      active_head_groups=1, active_ffn_groups=1, recipe_count=2)
    torch.manual_seed(0)
    block = TransformerBlock(cfg)
    with torch.no_grad():
        for p in block.parameters():
            if p.ndim == 2:
                p.normal_(0.0, 0.02)
        # weights exactly representable in bf16 so both sides see the same operands
        for p in block.parameters():
            p.copy_(p.to(torch.bfloat16).float())
    x = torch.randn(B, S, d).to(torch.bfloat16).float()
    dy = torch.randn(B, S, d)
    xr = x.clone().requires_grad_()
    ref = _ref_block(block, xr)
    ref.backward(dy)
    ref_grads = {n: p.grad.clone() for n, p in block.named_parameters()}
    block.zero_grad()
    gb = block.cuda()
    xg = x.cuda().requires_grad_()
    out = gb(xg)
    out.backward(dy.cuda())
    assert_rel(out.detach().cpu().numpy(), ref.detach().numpy(), BF16_RTOL, "block out")
    assert_rel(xg.grad.cpu().numpy(), xr.grad.numpy(), BF16_RTOL, "block dx")
    for n, p in gb.named_parameters():
        assert_rel(p.grad.cpu().numpy(), ref_grads[n].numpy(), BF16_RTOL, f"block d{n}")


def _engine(mode="recursive_macro", **mover):
    from rte_amd.config import ExperimentConfig, OutputConfig, TrainingConfig
    from rte_amd.training import TrainEngine

    topo = "dense" if mode == "dense_exact" else "recursive"
    cfg = ExperimentConfig(
        model=_model_cfg(topology=topo, **mover),
        training=TrainingConfig(mode=mode, precision="bf16", batch_size=4, seq_len=16, audit_sampler="fixed_count",
                                audit_fixed_count=1, fixed_depth=4, seed=3),
        output=OutputConfig(num_clusters=8, shortlist_max_tokens=32, hard_negatives=4, random_negatives=4),
    )
    return TrainEngine(cfg, device=torch.device("cuda"))


@pytest.mark.parametrize("mode", ["recursive_macro", "recursive_macro_shortlist", "recursive_exact", "dense_exact"])
@pytest.mark.parametrize("ffn_kind", ["cluster_pool", "dense"])
def test_train_step_every_mode(mode, ffn_kind):
    from rte_amd.training import metrics_to_host

    eng = _engine(mode, ffn_kind=ffn_kind)
    model = eng.recursive_model if eng.recursive_model is not None else eng.dense_model
    before = {n: p.detach().clone() for n, p in model.named_parameters()}
    g = torch.Generator().manual_seed(0)
    tok = torch.randint(0, 256, (4, 17), generator=g)
    res = eng.train_step((tok[:, :-1], tok[:, 1:]))
    m = metrics_to_host(res.metrics)
    assert math.isfinite(float(res.loss)), m
    changed = sum(int(not torch.equal(before[n], p.detach())) for n, p in model.named_parameters())
    assert changed > 0


def test_audit_p1_corrected_equals_exact():
    """rte tests/test_audit.py:12-37: with every sample audited at p = 1 the corrected
    per-sample loss equals the exact replay's loss."""
    from rte_amd.config import ExperimentConfig, TrainingConfig
    from rte_amd.models import RecursiveModel

    cfg = ExperimentConfig(model=_model_cfg(), training=TrainingConfig(mode="recursive_macro", audit_fixed_count=4,
                                                                       batch_size=4, seed=5))
    torch.manual_seed(0)
    model = RecursiveModel(cfg.model, cfg.output).cuda()
    from rte_amd.audit import AuditEngine

    tok = torch.randint(0, 256, (4, 17), device="cuda")
    hot = model.forward_macro(tok[:, :-1], tok[:, 1:], return_states=True, return_loss_per_sample=True, fixed_depth=4)
    res = AuditEngine(cfg.training).correction(model, tok[:, :-1], tok[:, 1:], hot, seed=1)
    assert res.exact is not None
    # the fixed-count sampler draws randperm(n)[:k] from a generator seeded with `seed`;
    # exact losses come back in that order
    chosen = torch.randperm(4, device="cuda", generator=torch.Generator(device="cuda").manual_seed(1))[:4]
    ref = torch.empty_like(res.corrected_loss_per_sample)
    ref[chosen] = res.exact.loss_per_sample.detach()
    assert int(res.audit_mask.sum()) == 4
    np.testing.assert_allclose(res.corrected_loss_per_sample.detach().cpu().numpy(), ref.cpu().numpy(),
                               rtol=1e-5, atol=1e-5)


def test_backend_status_reports_hip():
    from rte_amd.kernels import optimized

    st = optimized.backend_status()
    assert st["mode"] == "rocm_hip_dispatch"
    assert st["uses_reference_fallback"] is False
    assert "gfx950" in st["device"]["arch"]
