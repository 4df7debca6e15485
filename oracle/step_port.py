"""CPU restatement of one recursive_macro training step (torch on the CPU) -- TEST INFRASTRUCTURE
AND CPU BASELINE ONLY.

Nothing in the product package imports this module.  tests/ use it as the step-level checker
(the GPU step's loss terms and every parameter gradient against this one's, from the same
weights and batch), and bench.py's cpu_baseline leg times it on the host cores.

It restates the reference's step term by term (paths relative to the reference repository,
rte/ = src/recursive_training_engine/), on a state dict keyed like the reference modules:

  step             rte/training.py:1336-1390  loss = corrected CE / S + sum(macro aux)
                                              + sum(router aux); backward; AdamW
  forward_macro    rte/models.py:681-723      prelude -> router -> Phi -> coda -> head
  block            rte/layers.py:646-656      u = x + attn(norm1 x); u + mlp(norm2 u)
  rmsnorm          rte/kernels/reference.py:9-17
  attention        rte/layers.py:53-75, RoPE rte/layers.py:36-50 + rte/kernels/reference.py:20-28
                   (interleaved pairs), causal SDPA
  dense SwiGLU     rte/layers.py:78-87        wug rows [up ; gate], wd Linear
  routed pool      (ffn_kind "cluster_pool", the build's routed pool): logits x Wr^T, top-k
                   clusters (value desc, index asc), softmax over the selected logits, pool c =
                   neurons [c n, (c+1) n) of the dense SwiGLU (rte/kernels/cluster_pool_ffn.py:
                   143-162 per pool)
  router           rte/routing.py:80-188      pooled mean, recipe / depth MLPs, per-pass bias,
                                              argmax, expected depth
  Phi              rte/macro.py:201-236, 335-354 (bounded residual, direct decomposition)
  consistency      rte/macro.py:342-359
  audit            rte/audit.py:99-115 (fixed-count sampler: p = k / n), :245-387 (correction)
  exact replay     rte/models.py:605-679, :430-450; rte/layers.py:659-870 (banked core)
  distillation     rte/macro.py:394-471 (the h0 branch; weights from the training config)
  router aux       rte/metrics.py:97-112

Decisions the GPU and the CPU may take differently on near-ties (the routed pools' top-k, the
recipe argmax) can be forced: `forced` supplies them, so that a comparison of losses and
gradients measures arithmetic, not a flipped tie (the ids themselves are checked bit-exact
elsewhere).  How this module is pinned is listed in oracle/__init__.py.
"""

from __future__ import annotations

import math

import torch
import torch.nn.functional as F

from oracle.banked import recipe_templates


# ----------------------------------------------------------------------------- operators

def rmsnorm(x, w=None, eps: float = 1e-5):
    """x * rsqrt(mean(x^2) + eps) (* w)  (rte/kernels/reference.py:9-17)."""
    y = x * torch.rsqrt(x.pow(2).mean(dim=-1, keepdim=True) + eps)
    return y if w is None else y * w


def rope_tables(head_dim: int, seq: int, dtype, base: float = 10_000.0):
    """cos / sin [S, hd] of RotaryEmbedding (rte/layers.py:36-44), made in float32 as there."""
    inv = 1.0 / (base ** (torch.arange(0, head_dim, 2).float() / head_dim))
    freqs = torch.outer(torch.arange(seq, dtype=torch.float32), inv)
    emb = torch.repeat_interleave(freqs, 2, dim=-1)
    return emb.cos().to(dtype), emb.sin().to(dtype)


def rope(x, cos, sin):
    """x cos + rotate_half(x) sin with interleaved pairs (rte/kernels/reference.py:20-28)."""
    rot = torch.stack((-x[..., 1::2], x[..., 0::2]), dim=-1).flatten(-2)
    return x * cos + rot * sin


def causal_attention(q, k, v):
    """softmax(q k^T / sqrt(hd), causal) v  (F.scaled_dot_product_attention(is_causal=True))."""
    S = q.shape[-2]
    s = q @ k.transpose(-1, -2) / math.sqrt(q.shape[-1])
    s = s.masked_fill(~torch.ones(S, S, dtype=torch.bool, device=q.device).tril(), float("-inf"))
    return s.softmax(dim=-1) @ v


def dense_attention(x, wqkv, wo, n_heads, cos, sin):
    """DenseCausalSelfAttention.forward (rte/layers.py:63-75): wqkv [3d, d], wo [d, d] (Linear)."""
    b, s, d = x.shape
    hd = d // n_heads
    q, k, v = (x @ wqkv.t()).view(b, s, 3, n_heads, hd).unbind(dim=2)
    q, k, v = q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2)
    if cos is not None:
        q, k = rope(q, cos[:s], sin[:s]), rope(k, cos[:s], sin[:s])
    y = causal_attention(q, k, v).transpose(1, 2).reshape(b, s, d)
    return y @ wo.t()


def swiglu(x, wug, wd):
    """DenseSwiGLU (rte/layers.py:78-87): up, gate = (x wug^T).chunk(2); (up silu(gate)) wd^T."""
    up, gate = (x @ wug.t()).chunk(2, dim=-1)
    return (up * F.silu(gate)) @ wd.t()


def topk_ids(logits, k: int):
    """Top-k cluster ids per row, value descending and index ascending on ties (the build's fixed
    rule; torch.topk leaves tie order unspecified)."""
    return torch.argsort(-logits.detach(), dim=-1, stable=True)[..., :k]


def routed_pool(x, wr, wug, wd, n_clusters: int, k: int, ids=None):
    """Routed cluster pool: logits = x Wr^T; the k selected clusters (given, or top-k); weights =
    softmax over their logits; out = sum_j w_j SwiGLU_{c_j}(x), pool c = neurons [c n, (c+1) n)
    of wug [2F, d] (rows [up ; gate]) and wd [d, F].  Returns (out, ids)."""
    shape = x.shape
    xt = x.reshape(-1, shape[-1])
    logits = xt @ wr.t()
    if ids is None:
        ids = topk_ids(logits, k)
    ids = ids.reshape(xt.shape[0], k).long()
    w = logits.gather(1, ids).softmax(dim=-1)
    F_ = wd.shape[1]
    n = F_ // n_clusters
    up_w, gate_w = wug[:F_], wug[F_:]
    out = torch.zeros_like(xt)
    for c in range(n_clusters):
        tok, slot = (ids == c).nonzero(as_tuple=True)
        if tok.numel() == 0:
            continue
        xc = xt[tok]
        z = (xc @ up_w[c * n:(c + 1) * n].t()) * F.silu(xc @ gate_w[c * n:(c + 1) * n].t())
        out = out.index_add(0, tok, w[tok, slot, None] * (z @ wd[:, c * n:(c + 1) * n].t()))
    return out.view(shape), ids


# ----------------------------------------------------------------------------- the step

class StepPort:
    """One recursive_macro step of the reference on the CPU.

    config:  an experiment config (attributes .model, .training as the reference's dataclasses).
    params:  {name: tensor} of the model's parameters, keyed like the reference modules (the
             named parameters of the build's RecursiveModel); these get gradients.
    buffers: {name: tensor} of buffers the step reads (macro.update_scale when it is a buffer)."""

    def __init__(self, config, params: dict, buffers: dict | None = None, *, dtype=torch.float32):
        self.mc, self.tc = config.model, config.training
        self.dtype = dtype
        self.p = {}
        self.trainable = set()
        for src, train in ((params, True), (buffers or {}, False)):
            for name, t in src.items():
                if isinstance(t, torch.Tensor) and t.is_floating_point() and name not in self.p:
                    self.p[name] = t.detach().to("cpu", dtype).clone()
                    if train:
                        self.trainable.add(name)
        mc = self.mc
        if mc.macro_type != "bounded_residual":
            raise NotImplementedError("step port: macro_type bounded_residual only")
        if mc.macro_decomposition != "direct":
            raise NotImplementedError("step port: direct macro decomposition only")
        if getattr(mc, "use_global_lowrank_corrector", False):
            raise NotImplementedError("step port: no global low-rank corrector")
        self.recipes = recipe_templates(mc.attn_banks, mc.ffn_banks, mc.head_groups, mc.ffn_groups,
                                        mc.active_head_groups, mc.active_ffn_groups, mc.recipe_count)
        self.strides = list(mc.depth_choices)
        pairs = [(i, self.strides.index(s * 2)) for i, s in enumerate(self.strides) if s * 2 in self.strides]
        self.cons_pairs = pairs                                          # rte/macro.py:128-136

    def params(self, requires_grad: bool = True) -> dict:
        """The trainable tensors (set to require gradients or not)."""
        for name in self.trainable:
            self.p[name].requires_grad_(requires_grad)
        return {n: self.p[n] for n in self.p if n in self.trainable}

    # -- modules --------------------------------------------------------------------------
    def _block(self, x, pre: str, cos, sin, ids=None):
        """TransformerBlock (rte/layers.py:646-656).  Returns (out, pool ids or None)."""
        p, mc = self.p, self.mc
        u = x + dense_attention(rmsnorm(x, p[pre + "norm1.weight"]), p[pre + "attn.wqkv.weight"],
                                p[pre + "attn.wo.weight"], mc.n_heads, cos, sin)
        n2 = rmsnorm(u, p[pre + "norm2.weight"])
        if mc.ffn_kind == "cluster_pool":
            y, ids = routed_pool(n2, p[pre + "mlp.router.weight"], p[pre + "mlp.wug.weight"],
                                 p[pre + "mlp.wd.weight"], mc.ffn_clusters, mc.ffn_top_k, ids)
            return u + y, ids
        return u + swiglu(n2, p[pre + "mlp.wug.weight"], p[pre + "mlp.wd.weight"]), None

    def _router(self, h0, forced):
        """Router.forward (rte/routing.py:80-188): the fields the step reads."""
        p, tc = self.p, self.tc
        pooled = h0.mean(dim=1)

        def mlp(name, x):
            a = F.silu(x @ p[name + ".0.weight"].t() + p[name + ".0.bias"])
            return a @ p[name + ".2.weight"].t() + p[name + ".2.bias"]

        recipe_logits = mlp("router.recipe_mlp", pooled)
        depth_logits = mlp("router.depth_mlp", pooled)
        by_pass = recipe_logits.unsqueeze(1) + p["router.pass_recipe_bias"].unsqueeze(0)
        recipe_probs = recipe_logits.softmax(dim=-1)
        depth_probs = depth_logits.softmax(dim=-1)
        B = h0.shape[0]
        if tc.fixed_recipe is None:
            rid = recipe_probs.argmax(dim=-1)
            rid_bp = by_pass.softmax(dim=-1).argmax(dim=-1)
        else:
            rid = torch.full((B,), tc.fixed_recipe, dtype=torch.long)
            rid_bp = torch.full((B, self.mc.t_max), tc.fixed_recipe, dtype=torch.long)
        if forced.get("recipe_id") is not None:
            rid = forced["recipe_id"].long().cpu()
        if forced.get("recipe_id_by_pass") is not None:
            rid_bp = forced["recipe_id_by_pass"].long().cpu()
        dv = torch.tensor(self.strides)
        depth_id = (torch.full((B,), self.strides.index(tc.fixed_depth), dtype=torch.long)
                    if tc.fixed_depth is not None else depth_probs.argmax(dim=-1))
        expected_depth = (depth_probs * dv.to(depth_probs.dtype)).sum(dim=-1)
        return dict(recipe_logits=recipe_logits, recipe_probs=recipe_probs, recipe_id=rid, recipe_id_by_pass=rid_bp,
                    depth_id=depth_id, depth=dv[depth_id], expected_depth=expected_depth)

    def phi(self, h, h0, rid, sid):
        """Bounded macro operator (rte/macro.py:201-236) per sample key (recipe, stride)."""
        p = self.p
        normed = rmsnorm(h)
        pooled = normed.mean(dim=1, keepdim=True).expand_as(normed)
        parts = [normed, pooled, h0]
        if self.mc.macro_include_delta_to_h0:
            parts.append(normed - rmsnorm(h0))
        z = torch.cat(parts, dim=-1)
        low = F.silu(torch.bmm(z, p["macro.v"][rid, sid]))
        if "macro.v2" in p:
            low = F.silu(torch.bmm(low, p["macro.v2"][rid, sid]))
        low = torch.bmm(low, p["macro.u"][rid, sid])
        upd = p["macro.d_gain"][rid, sid].unsqueeze(1) * h + low + p["macro.bias"][rid, sid].unsqueeze(1)
        scale = p["macro.update_scale"][rid, sid]
        return h + self.mc.macro_update_scale * scale.unsqueeze(1) * torch.tanh(upd)

    def consistency(self, h0, rid):
        """MSE(Phi_dst(h0), Phi_src(Phi_src(h0))) over the (stride, 2 stride) pairs (rte/macro.py:
        342-359), the pairs stacked pair-major as there."""
        if not self.cons_pairs:
            return h0.new_zeros(())
        P, B = len(self.cons_pairs), h0.shape[0]
        hr = h0.unsqueeze(0).expand(P, *h0.shape).reshape(P * B, *h0.shape[1:])
        rr = rid.unsqueeze(0).expand(P, B).reshape(-1)
        src = torch.tensor([a for a, _ in self.cons_pairs]).unsqueeze(1).expand(P, B).reshape(-1)
        dst = torch.tensor([b for _, b in self.cons_pairs]).unsqueeze(1).expand(P, B).reshape(-1)
        direct = self.phi(hr, hr, rr, dst)
        twice = self.phi(self.phi(hr, hr, rr, src), hr, rr, src)
        return F.mse_loss(direct, twice)

    def _banked_attention(self, x, spec, cos, sin):
        """BankedAttention.forward (rte/layers.py:702-728) for one recipe."""
        p, mc = self.p, self.mc
        b, s, d = x.shape
        hpg, hd = mc.n_heads // mc.head_groups, d // mc.n_heads
        cols = torch.tensor([c for g in spec["head_groups"] for h in range(g * hpg, (g + 1) * hpg)
                             for c in range(h * hd, (h + 1) * hd)])
        qkv_cols = torch.cat([cols, cols + d, cols + 2 * d])
        a = cols.numel()
        out = x.new_zeros(b, s, d)
        for bank in spec["attention_banks"]:
            q, k, v = (x @ p["core.attn.wqkv"][bank][:, qkv_cols]).split(a, dim=-1)
            q, k, v = (t.view(b, s, a // hd, hd).transpose(1, 2) for t in (q, k, v))
            if cos is not None:
                q, k = rope(q, cos[:s], sin[:s]), rope(k, cos[:s], sin[:s])
            y = causal_attention(q, k, v).transpose(1, 2).reshape(b, s, a)
            out = out + y @ p["core.attn.wo"][bank][cols, :]
        return out / max(len(spec["attention_banks"]), 1)

    def _banked_swiglu(self, x, spec):
        """BankedSwiGLU.forward (rte/layers.py:765-779) for one recipe."""
        p, mc = self.p, self.mc
        slab = mc.d_ff // mc.ffn_groups
        slabs = torch.tensor([c for g in spec["ffn_groups"] for c in range(g * slab, (g + 1) * slab)])
        gate_cols = torch.cat([slabs, slabs + mc.d_ff])
        out = torch.zeros_like(x)
        for bank in spec["ffn_banks"]:
            up, gate = (x @ p["core.mlp.wug"][bank][:, gate_cols]).split(slabs.numel(), dim=-1)
            out = out + (up * F.silu(gate)) @ p["core.mlp.wd"][bank][slabs, :]
        return out / max(len(spec["ffn_banks"]), 1)

    def _core_step(self, h, h0, spec, t, cos, sin):
        """BankedRecursiveCore.step_group (rte/layers.py:826-845)."""
        p = self.p
        ht = h if "core.alpha_inj" not in p else h + p["core.alpha_inj"] * h0
        n1 = rmsnorm(ht, p["core.norm1.weight"]) * (1.0 + p["core.pass_gamma1"][t]) + p["core.pass_beta1"][t]
        u = ht + p["core.pass_attn_scale"][t] * self._banked_attention(n1, spec, cos, sin)
        n2 = rmsnorm(u, p["core.norm2.weight"]) * (1.0 + p["core.pass_gamma2"][t]) + p["core.pass_beta2"][t]
        return u + p["core.pass_mlp_scale"][t] * self._banked_swiglu(n2, spec)

    def _coda(self, h, cos, sin, ids_list):
        pools = []
        i = 0
        while f"coda.{i}.norm1.weight" in self.p:
            h, ids = self._block(h, f"coda.{i}.", cos, sin, None if ids_list is None else ids_list[i])
            pools.append(ids)
            i += 1
        hidden = rmsnorm(h, self.p["final_norm.weight"])
        w = self.p.get("lm_head.weight", self.p["embed.weight"])
        return hidden, hidden @ w.t(), pools

    # -- forward ----------------------------------------------------------------------------
    def loss_terms(self, tokens, targets, *, chosen, usage_ema, forced: dict | None = None) -> dict:
        """Every term of the step's loss, and what the checks read.

        chosen: the fixed-count audit's rows (long [k]; rte/audit.py:99-115 draws them with a
        seeded randperm); usage_ema: the recipe bank's usage EMA before this step's update;
        forced: optional decisions {"recipe_id", "recipe_id_by_pass", "pool_ids": {"prelude": [..],
        "coda": [..], "replay_coda": [..]}} and "frozen": the distillation's detached operands
        {"exact_hidden", "h0", "exact_logits"} (a finite-difference check holds them fixed, as
        the gradient does)."""
        forced = forced or {}
        fp = forced.get("pool_ids", {})
        mc, tc, p = self.mc, self.tc, self.p
        tokens, targets = tokens.cpu().long(), targets.cpu().long()
        B, S = tokens.shape
        hd = mc.d_model // mc.n_heads
        cos, sin = rope_tables(hd, S, self.dtype) if mc.use_rope else (None, None)
        out: dict = {"pool_ids": {"prelude": [], "coda": [], "replay_coda": []}}
        # forward_macro (rte/models.py:681-723)
        h0 = p["embed.weight"][tokens]
        i = 0
        while f"prelude.{i}.norm1.weight" in p:
            pre = fp.get("prelude")
            h0, ids = self._block(h0, f"prelude.{i}.", cos, sin, None if pre is None else pre[i])
            out["pool_ids"]["prelude"].append(ids)
            i += 1
        route = self._router(h0, forced)
        sid = route["depth_id"]  # stride ids of the depths (rte/macro.py:144-146, distinct choices)
        h = self.phi(h0, h0, route["recipe_id"], sid)
        hidden, logits, pools = self._coda(h, cos, sin, fp.get("coda"))
        out["pool_ids"]["coda"] = pools
        tok = F.cross_entropy(logits.flatten(0, 1), targets.flatten(), reduction="none").view(B, S)
        lps = tok.sum(dim=-1)                                   # rte/models.py:73-75
        # audit correction (rte/audit.py:245-387), fixed-count sampler
        idx = chosen.cpu().long()
        k = idx.numel()
        p_incl = float(k) / float(B)
        corrected = lps.clone()
        zero = lps.new_zeros(())
        aux = {n: zero for n in ("hid", "cos", "kl", "norm", "cons", "delta_dir", "delta_rms", "endpoint_normed",
                                 "endpoint_raw", "rms_trust")}
        grad_corr = tc.audit_mode == "gradient_corrected"
        if k > 0:
            # exact replay of the audited rows on the cached h0 and the hot routing (rte/models.py:605-679)
            he, h0a = h0[idx], h0[idx]
            depth_a = route["depth"][idx]
            rbp = route["recipe_id_by_pass"][idx]
            with (torch.enable_grad() if grad_corr else torch.no_grad()):
                for t in range(mc.t_max):
                    new = he.clone()
                    for a in range(k):
                        if int(depth_a[a]) > t:
                            new = new.index_copy(0, torch.tensor([a]), self._core_step(
                                he[a:a + 1], h0a[a:a + 1], self.recipes[int(rbp[a, t])], t, cos, sin))
                    he = new
                _, lg_e, pools_e = self._coda(he, cos, sin, fp.get("replay_coda"))
                tok_e = F.cross_entropy(lg_e.flatten(0, 1), targets[idx].flatten(), reduction="none").view(k, S)
            out["pool_ids"]["replay_coda"] = pools_e
            lps_e = tok_e.sum(dim=-1)
            residual = lps_e - lps[idx]
            if tc.audit_residual_clip is not None:
                residual = residual.clamp(-tc.audit_residual_clip, tc.audit_residual_clip)
            if not grad_corr:
                residual = residual.detach()
            if tc.audit_mode == "gradient_corrected":
                corrected = corrected.index_put((idx,), lps[idx] + residual / max(p_incl, 1e-12))
            # distillation (rte/macro.py:394-471, h0 branch); the exact side and h0 are constants
            # of its gradient (detached there), and may be frozen at given values
            fz = forced.get("frozen")
            ex = he.detach() if fz is None else fz["exact_hidden"]
            z0 = h0[idx].detach() if fz is None else fz["h0"]
            lg_c = lg_e.detach() if fz is None else fz["exact_logits"]
            hot_end = h[idx]
            dp, de = hot_end - z0, ex - z0
            delta_dir = 1.0 - F.cosine_similarity(dp.flatten(1), de.flatten(1), dim=-1, eps=1e-8).mean()
            prms = dp.pow(2).mean(dim=(1, 2)).sqrt().clamp_min(1e-8)
            erms = de.pow(2).mean(dim=(1, 2)).sqrt().clamp_min(1e-8)
            delta_rms = (prms.log() - erms.log()).square().mean()
            endpoint_normed = F.smooth_l1_loss(rmsnorm(hot_end), rmsnorm(ex))
            endpoint_raw = F.smooth_l1_loss(hot_end, ex)
            ratio = (hot_end.pow(2).mean(dim=(1, 2)).sqrt().clamp_min(1e-8)
                     / ex.pow(2).mean(dim=(1, 2)).sqrt().clamp_min(1e-8))
            rms_trust = ratio.log().square().mean()
            temp = max(float(tc.distill_temperature), 1e-6)
            exact_logp = F.log_softmax(lg_c / temp, dim=-1)
            hot_logp = F.log_softmax(logits[idx] / temp, dim=-1)
            kl = F.kl_div(hot_logp, exact_logp.exp(), reduction="batchmean") * temp ** 2
            aux.update({"kl": tc.effective_lambda_kl * kl, "delta_dir": tc.lambda_delta_dir * delta_dir,
                        "delta_rms": tc.lambda_delta_rms * delta_rms,
                        "endpoint_normed": tc.lambda_endpoint_normed * endpoint_normed,
                        "endpoint_raw": tc.lambda_endpoint_raw * endpoint_raw,
                        "rms_trust": (tc.lambda_macro_rms_trust if tc.macro_rms_trust_region else 0.0) * rms_trust})
            out.update(exact_lps=lps_e, exact_hidden=he,
                       frozen={"exact_hidden": ex.detach(), "h0": z0.detach(), "exact_logits": lg_c.detach()})
        if tc.lambda_cons != 0.0:
            aux["cons"] = tc.lambda_cons * self.consistency(h0, route["recipe_id"])
        # router aux (rte/metrics.py:97-112)
        R = route["recipe_probs"].shape[-1]
        mean_prob = route["recipe_probs"].mean(dim=0)
        router_aux = {
            "load": tc.lambda_load * (R * mean_prob.square().sum() - 1.0),
            "cover": tc.lambda_cover * F.relu(tc.coverage_min - usage_ema.cpu().to(self.dtype)).square().sum(),
            "depth": tc.lambda_depth * route["expected_depth"].mean(),
        }
        scale = float(S) if tc.loss_normalization == "token_mean" else 1.0
        ce = corrected.mean() / scale
        loss = ce + sum(aux.values()) + sum(router_aux.values())
        out.update(loss=loss, corrected_ce=ce, macro_aux=aux, router_aux=router_aux, hot_lps=lps,
                   corrected=corrected, route=route, h0=h0, recurrent_hidden=h, logits=logits)
        return out

    def loss_and_grads(self, tokens, targets, *, chosen, usage_ema, forced=None):
        """(terms, {name: gradient or None}) of one step's loss."""
        params = self.params(True)
        for t in params.values():
            t.grad = None
        terms = self.loss_terms(tokens, targets, chosen=chosen, usage_ema=usage_ema, forced=forced)
        terms["loss"].backward()
        return terms, {n: (t.grad.detach().clone() if t.grad is not None else None) for n, t in params.items()}


# ----------------------------------------------------------------------------- CPU baseline

def param_groups(port: StepPort) -> list[dict]:
    """The reference's AdamW parameter groups (rte/training.py:300-340) over the port's tensors."""
    tc = port.tc
    groups = {"embedding": [], "prelude": [], "core": [], "macro": [], "coda": [], "output": [], "router": []}
    lrs = {"embedding": tc.effective_lr_base, "prelude": tc.effective_lr_base, "core": tc.effective_lr_base,
           "macro": tc.effective_lr_macro, "coda": tc.effective_lr_coda, "output": tc.effective_lr_output,
           "router": tc.effective_lr_router}
    for name, t in port.params(True).items():
        head = name.split(".")[0]
        g = {"embed": "embedding", "final_norm": "coda", "lm_head": "output", "shortlist_head": "output"}.get(head, head)
        groups.setdefault(g, []).append(t)
    return [{"params": v, "lr": lrs.get(k, tc.lr)} for k, v in groups.items() if v]


def train_step(port: StepPort, opt, tokens, targets, *, chosen, usage_ema) -> float:
    """One full step on the CPU: forward, backward, optional clipping, AdamW."""
    opt.zero_grad(set_to_none=True)
    terms = port.loss_terms(tokens, targets, chosen=chosen, usage_ema=usage_ema)
    terms["loss"].backward()
    if port.tc.grad_clip_norm is not None:
        torch.nn.utils.clip_grad_norm_([t for g in opt.param_groups for t in g["params"]], port.tc.grad_clip_norm)
    opt.step()
    return float(terms["loss"].detach())


def make_optimizer(port: StepPort):
    return torch.optim.AdamW(param_groups(port), weight_decay=port.tc.weight_decay)


def zipf_tokens(vocab: int, B: int, S: int, seed: int = 0):
    """Token ids ~ Zipf(1.1) over the vocabulary; targets = next token."""
    g = torch.Generator().manual_seed(seed)
    pr = (torch.arange(vocab, dtype=torch.float64) + 1.0).pow(-1.1)
    ids = torch.multinomial((pr / pr.sum()).float(), B * (S + 1), replacement=True, generator=g).view(B, S + 1)
    return ids[:, :-1].contiguous(), ids[:, 1:].contiguous()
