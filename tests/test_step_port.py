"""Pins of the CPU step restatement (oracle/step_port.py), the checker the GPU train step is
compared with.

1. Its loss, term by term, equals a composition of the separately pinned numpy oracle
   functions (attention / RoPE / RMSNorm, routed pool, recipe router, bounded macro operator,
   banked core, cross-entropy, audit correction, distillation) and the closed-form router
   auxiliary terms (rte/metrics.py:97-112), on a small recursive_macro model whose depths vary
   per sample (masked replay passes) and whose zero-initialised parameters are perturbed.
2. Its gradients equal central finite differences of its own loss (float64) on entries of every
   kind of parameter, with the step's discrete decisions held fixed.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import attention as OA
from oracle import audit as OAU
from oracle import banked as OB
from oracle import cluster_pool as OCP
from oracle import distill as ODI
from oracle import losses as OL
from oracle import macro as OM
from oracle import router as ORT
from oracle import routing as OR
from oracle import step_port as SP


def _config(fixed_depth=None, audit_count=2):
    from rte_amd.config import ExperimentConfig, ModelConfig, OutputConfig, TrainingConfig

    mc = ModelConfig(topology="recursive", vocab_size=50, d_model=64, n_heads=2, d_ff=256, n_dense_layers=2,
                     n_prelude=1, n_coda=1, t_max=4, depth_choices=[1, 2, 4], attn_banks=2, ffn_banks=2,
                     head_groups=2, ffn_groups=8, active_head_groups=1, active_ffn_groups=2, recipe_count=5,
                     macro_rank=4, ffn_kind="cluster_pool", ffn_clusters=8, ffn_top_k=2, router_hidden=16)
    tc = TrainingConfig(mode="recursive_macro", precision="bf16", batch_size=6, seq_len=8,
                        audit_sampler="fixed_count", audit_fixed_count=audit_count, seed=3, fixed_depth=fixed_depth,
                        audit_residual_clip=50.0, macro_rms_trust_region=True)
    return ExperimentConfig(model=mc, training=tc, output=OutputConfig())


def _model(cfg, seed=0):
    from rte_amd.models import RecursiveModel

    torch.manual_seed(seed)
    m = RecursiveModel(cfg.model, cfg.output)
    g = torch.Generator().manual_seed(seed + 1)
    with torch.no_grad():  # zero / one initialised tensors get spread so every path carries weight
        for name, p in m.named_parameters():
            if name.startswith(("core.pass_", "macro.d_gain", "macro.bias", "router.pass_recipe_bias")) or \
                    name.endswith("bias") or name.endswith("norm1.weight") or name.endswith("norm2.weight"):
                p.add_(0.2 * torch.randn(p.shape, generator=g))
        m.macro.u.mul_(200.0)   # a macro update well above rounding
        m.router.depth_mlp[2].weight.mul_(30.0)  # depths that differ between samples
    return m


def _np(t):
    return t.detach().double().numpy()


def _numpy_step(cfg, m, tok, tgt, chosen, usage):
    """The step's loss terms composed from the numpy oracle functions."""
    mc, tc = cfg.model, cfg.training
    P = {n: _np(p) for n, p in m.named_parameters()}
    P["macro.update_scale"] = _np(m.macro.update_scale)
    B, S = tok.shape
    d, H = mc.d_model, mc.n_heads
    cos, sin = OA.rope_tables(d // H, S)

    def block(x, pre):
        n1 = OA.rmsnorm(x, P[pre + "norm1.weight"])
        q, k, v = OA.qkv_rope(n1, P[pre + "attn.wqkv.weight"], H, cos, sin)
        y = np.stack([OB.causal_attention(q[b], k[b], v[b]) for b in range(x.shape[0])])
        u = x + y.transpose(0, 2, 1, 3).reshape(x.shape) @ P[pre + "attn.wo.weight"].T
        n2 = OA.rmsnorm(u, P[pre + "norm2.weight"]).reshape(-1, d)
        ids, w = OR.route_topk((n2 @ P[pre + "mlp.router.weight"].T).astype(np.float32), mc.ffn_top_k)
        y2 = OCP.routed_fwd(n2, P[pre + "mlp.wug.weight"], P[pre + "mlp.wd.weight"], ids, w, mc.ffn_clusters)
        return u + y2.reshape(u.shape)

    def coda(h):
        hid = OA.rmsnorm(block(h, "coda.0."), P["final_norm.weight"])
        return hid @ P["embed.weight"].T

    h0 = block(P["embed.weight"][tok.numpy()], "prelude.0.")
    rp = {n[len("router."):]: v for n, v in P.items() if n.startswith("router.")}
    r = ORT.router(h0, rp, mc.depth_choices)
    if tc.fixed_depth is not None:  # rte/routing.py:121-129
        r["depth_id"] = np.full(B, mc.depth_choices.index(tc.fixed_depth))
    mp = {n[len("macro."):]: v for n, v in P.items() if n.startswith("macro.")}
    c = mc.macro_update_scale
    h = OM.bounded_apply(h0, h0, r["recipe_id"], r["depth_id"], mp, c)
    logits = coda(h)
    hot_tok = OL.cross_entropy(logits, tgt.numpy())[0]
    idx = chosen.numpy()
    recipes = OB.recipe_templates(mc.attn_banks, mc.ffn_banks, mc.head_groups, mc.ffn_groups,
                                  mc.active_head_groups, mc.active_ffn_groups, mc.recipe_count)
    cp = {k[len("core."):].replace(".weight", ""): v for k, v in P.items() if k.startswith("core.")}
    cp = {k.replace("attn.", "").replace("mlp.", ""): v for k, v in cp.items()}
    depth = np.asarray(mc.depth_choices)[r["depth_id"]]
    he = h0[idx].copy()
    for t in range(mc.t_max):
        he = OB.core_forward_step(he, h0[idx], r["recipe_id_by_pass"][idx, t], depth[idx] > t, recipes, cp, t,
                                  n_heads=H, head_groups=mc.head_groups, ffn_groups=mc.ffn_groups, cos=cos, sin=sin)
    lg_e = coda(he)
    exact_tok = OL.cross_entropy(lg_e, tgt.numpy()[idx])[0]
    p = np.full(B, len(idx) / B)
    corrected, _, _ = OAU.correction(hot_tok, exact_tok, idx, p, clip=tc.audit_residual_clip)
    dl, _ = ODI.distill(h[idx], he, h0[idx], logits[idx], lg_e, t=tc.distill_temperature)
    lam = {"delta_dir": tc.lambda_delta_dir, "delta_rms": tc.lambda_delta_rms,
           "endpoint_normed": tc.lambda_endpoint_normed, "endpoint_raw": tc.lambda_endpoint_raw,
           "rms_trust": tc.lambda_macro_rms_trust, "kl": tc.effective_lambda_kl}
    macro_aux = {k: lam[k] * dl[k] for k in lam}
    pairs = [(i, mc.depth_choices.index(s * 2)) for i, s in enumerate(mc.depth_choices) if s * 2 in mc.depth_choices]
    diffs = []
    for a, b in pairs:
        src, dst = np.full(B, a), np.full(B, b)
        diffs.append(OM.bounded_apply(h0, h0, r["recipe_id"], dst, mp, c)
                     - OM.bounded_apply(OM.bounded_apply(h0, h0, r["recipe_id"], src, mp, c), h0, r["recipe_id"], src,
                                        mp, c))
    macro_aux["cons"] = tc.lambda_cons * np.mean(np.square(np.stack(diffs)))
    R = r["recipe_probs"].shape[-1]
    router_aux = {"load": tc.lambda_load * (R * np.square(r["recipe_probs"].mean(0)).sum() - 1.0),
                  "cover": tc.lambda_cover * np.square(np.maximum(tc.coverage_min - usage.numpy(), 0.0)).sum(),
                  "depth": tc.lambda_depth * r["expected_depth"].mean()}
    ce = corrected.mean() / S
    return dict(ce=ce, macro_aux=macro_aux, router_aux=router_aux,
                loss=ce + sum(macro_aux.values()) + sum(router_aux.values()), depth=depth)


@pytest.mark.parametrize("fixed_depth,audit_count", [(None, 2), (4, 1)])
def test_step_port_equals_oracle_composition(fixed_depth, audit_count):
    cfg = _config(fixed_depth, audit_count)
    m = _model(cfg)
    tok, tgt = SP.zipf_tokens(cfg.model.vocab_size, 6, 8, seed=5)
    chosen = torch.tensor([4, 1][:audit_count])
    usage = torch.tensor([0.0, 0.02, 0.005, 0.3, 0.0])
    ref = _numpy_step(cfg, m, tok, tgt, chosen, usage)
    if fixed_depth is None:
        assert len(set(ref["depth"][chosen.numpy()].tolist())) > 1 or len(set(ref["depth"].tolist())) > 1
    port = SP.StepPort(cfg, dict(m.named_parameters()), dict(m.named_buffers()), dtype=torch.float64)
    with torch.no_grad():
        got = port.loss_terms(tok, tgt, chosen=chosen, usage_ema=usage)
    rel = lambda a, b: abs(float(a) - float(b)) / max(abs(float(b)), 1e-12)  # noqa: E731
    assert rel(got["corrected_ce"], ref["ce"]) < 1e-6
    for k, v in ref["macro_aux"].items():
        assert abs(float(got["macro_aux"][k]) - v) <= 1e-6 * max(abs(v), 1e-6), k
    for k, v in ref["router_aux"].items():
        assert abs(float(got["router_aux"][k]) - v) <= 1e-9 + 1e-6 * abs(v), k
    assert rel(got["loss"], ref["loss"]) < 1e-6
    assert float(ref["macro_aux"]["cons"]) > 0 and float(ref["macro_aux"]["kl"]) > 0


def test_step_port_gradients_match_finite_differences():
    cfg = _config(None, 2)
    m = _model(cfg, seed=2)
    tok, tgt = SP.zipf_tokens(cfg.model.vocab_size, 6, 8, seed=9)
    chosen = torch.tensor([0, 3])
    usage = torch.zeros(cfg.model.recipe_count)
    port = SP.StepPort(cfg, dict(m.named_parameters()), dict(m.named_buffers()), dtype=torch.float64)
    terms, grads = port.loss_and_grads(tok, tgt, chosen=chosen, usage_ema=usage)
    r = terms["route"]
    forced = {"recipe_id": r["recipe_id"], "recipe_id_by_pass": r["recipe_id_by_pass"],
              "pool_ids": {k: [t.clone() for t in v] for k, v in terms["pool_ids"].items()},
              "frozen": terms["frozen"]}
    names = ["embed.weight", "prelude.0.attn.wqkv.weight", "prelude.0.mlp.router.weight", "prelude.0.mlp.wug.weight",
             "prelude.0.norm2.weight", "router.recipe_mlp.2.weight", "router.depth_mlp.0.bias", "core.attn.wqkv",
             "core.attn.wo", "core.mlp.wug", "core.mlp.wd", "core.pass_gamma1", "core.pass_attn_scale",
             "core.alpha_inj", "macro.v", "macro.u", "macro.d_gain", "coda.0.attn.wo.weight", "coda.0.mlp.wd.weight",
             "final_norm.weight"]
    gen = np.random.default_rng(0)
    params = port.params(False)
    eps = 1e-6
    checked = 0
    for name in names:
        g = grads[name]
        assert g is not None, name
        flat = params[name].view(-1)
        # the entries with the largest gradient and one random entry
        picks = {int(torch.argmax(g.abs())), int(gen.integers(flat.numel()))}
        for i in picks:
            old = float(flat[i])
            vals = []
            for s in (1.0, -1.0):
                flat[i] = old + s * eps
                with torch.no_grad():
                    vals.append(float(port.loss_terms(tok, tgt, chosen=chosen, usage_ema=usage, forced=forced)["loss"]))
            flat[i] = old
            fd = (vals[0] - vals[1]) / (2 * eps)
            an = float(g.view(-1)[i])
            assert abs(fd - an) <= 1e-5 * max(abs(an), 1e-3), (name, i, fd, an)
            checked += 1
    assert checked >= len(names)
    # parameters outside the step's graph (factor heads, shortlist router) get no gradient
    assert grads["router.factor_mlp.0.weight"] is None and grads["shortlist_head.cluster_router.weight"] is None
