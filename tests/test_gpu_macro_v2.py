"""The v2_delta_radius macro operator (rte/macro.py:238-279) on the grouped HIP products: output and
every parameter gradient against a float64 torch restatement of the reference formula, at
precision fp32 (1e-5 relative) and bf16 (2e-2 relative), with the depth and recipe embeddings,
a hidden multiple of 2 and the teacher-radius clamp."""

from __future__ import annotations

import pytest
import torch
import torch.nn.functional as F

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


def _ref(P, cfg, h0, rid, sid):
    """rte/macro.py:238-279 in float64 (per-sample weight gathers and bmm, as there)."""
    def rms(x, dim):
        return x.pow(2).mean(dim=dim, keepdim=True).sqrt()

    normed = h0 * torch.rsqrt(h0.pow(2).mean(-1, keepdim=True) + 1e-5)
    pooled = normed.mean(dim=1)
    parts = [normed, pooled.unsqueeze(1).expand_as(normed), h0]
    if cfg.macro_use_delta_to_h0 or cfg.macro_include_delta_to_h0:
        parts.append(normed - normed)
    if "depth_embed" in P:
        parts.append(P["depth_embed"][sid].unsqueeze(1).expand_as(normed))
    if "recipe_embed" in P:
        parts.append(P["recipe_embed"][rid].unsqueeze(1).expand_as(normed))
    z = torch.cat(parts, dim=-1)
    raw = torch.bmm(F.silu(torch.bmm(F.silu(torch.bmm(z, P["v"][rid, sid])), P["v2"][rid, sid])), P["u"][rid, sid])
    raw = raw + P["bias"][rid, sid].unsqueeze(1)
    direction = raw / rms(raw, (1, 2)).clamp_min(1e-6)
    rho_head = torch.bmm(pooled.unsqueeze(1), P["rho_head"][rid, sid]).squeeze(-1).squeeze(-1)
    rho = F.softplus(P["rho_base_raw"][rid, sid] + rho_head)
    teacher = P["teacher_delta_rms"][rid, sid]
    if cfg.macro_radius_init_from_teacher:
        has = teacher > 0
        rho = torch.where(has, torch.clamp(rho, min=teacher * cfg.macro_radius_clamp_mult_min,
                                           max=teacher * cfg.macro_radius_clamp_mult_max), rho)
    return h0 + rho.view(-1, 1, 1) * direction


@pytest.mark.parametrize("precision", ["fp32", "bf16"])
def test_macro_v2_matches_reference(precision):
    from rte_amd.config import ModelConfig
    from rte_amd.kernels import hip_ops
    from rte_amd.macro import MacroOperators

    cfg = ModelConfig(topology="recursive", vocab_size=64, d_model=128, n_heads=2, d_ff=256, n_dense_layers=2,
                      n_prelude=1, n_coda=1, t_max=4, depth_choices=[1, 2, 4], attn_banks=1, ffn_banks=1,
                      head_groups=2, ffn_groups=8, active_head_groups=1, active_ffn_groups=2, recipe_count=5,
                      macro_rank=16, macro_type="v2_delta_radius", macro_hidden_mult=2,
                      macro_use_depth_embedding=True, macro_use_recipe_embedding=True,
                      macro_radius_init_from_teacher=True)
    torch.manual_seed(0)
    mac = MacroOperators(cfg).to(DEV)
    g = torch.Generator(device=DEV).manual_seed(1)
    with torch.no_grad():
        mac.u.mul_(100.0)
        mac.bias.add_(0.1 * torch.randn(mac.bias.shape, device=DEV, generator=g))
        mac.rho_head.add_(0.05 * torch.randn(mac.rho_head.shape, device=DEV, generator=g))
        mac.teacher_delta_rms[1, 2] = 0.3  # one key with a teacher radius: its rho is clamped
    B, S, d = 6, 20, cfg.d_model
    h0 = torch.randn(B, S, d, device=DEV, generator=g, requires_grad=True)
    rid = torch.tensor([1, 0, 4, 1, 2, 1], device=DEV)
    sid = torch.tensor([2, 0, 1, 2, 2, 0], device=DEV)
    ctx = hip_ops.fp32_precision() if precision == "fp32" else torch.autocast("cuda", dtype=torch.bfloat16)
    with ctx:
        out = mac.apply_vectorized(h0, h0, rid, sid)
    dy = torch.randn(out.shape, device=DEV, generator=g)
    out.float().backward(dy)
    P = {n: p.detach().double().requires_grad_() for n, p in mac.named_parameters()}
    P["teacher_delta_rms"] = mac.teacher_delta_rms.double()
    hd = h0.detach().double().requires_grad_()
    ref = _ref(P, cfg, hd, rid, sid)
    ref.backward(dy.double())
    tol = 1e-5 if precision == "fp32" else 2e-2
    assert _rel(out - h0, ref - hd) < tol  # the update itself (h0 dominates the sum)
    assert _rel(h0.grad, hd.grad) < tol
    for n, p in mac.named_parameters():
        if P[n].grad is None or not bool(P[n].grad.abs().max() > 0):
            assert p.grad is None or not bool(p.grad.abs().max() > 0), n
            continue
        assert _rel(p.grad, P[n].grad) < tol, (n, _rel(p.grad, P[n].grad))
