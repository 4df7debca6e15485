"""CPU port of one recursive_macro training step (torch on the CPU, float32) -- BASELINE /
TEST INFRASTRUCTURE ONLY.

The CPU baseline bench.py times beside the GPU step: the same workload as the GPU benchmark
(d 512, 8 heads, prelude + coda blocks with a routed cluster-pool
SwiGLU of 64 clusters x 32 neurons top-8, banked recursive core of 64 slabs x 32 with 8 active
per recipe, depth 4, tied vocab-2048 head, fixed-count audit of one sample, AdamW), restated in
plain torch ops on the host in float32 and differentiated by torch autograd.  It follows:

  step          rte/training.py:1336-1476 (loss = corrected CE / S + macro aux + router aux,
                backward, AdamW)
  forward_macro rte/models.py:681-723 (prelude -> router -> Phi -> coda -> head)
  block         rte/layers.py:646-656 (x + attn(norm1 x); + ffn(norm2 .))
  attention     rte/layers.py:53-75 (QKV, interleaved RoPE, causal softmax attention, O-proj)
  cluster pool  rte/kernels/cluster_pool_ffn.py:143-189 (top-k clusters, softmax weights,
                per-cluster SwiGLU, weighted sum)
  router        rte/routing.py:80-188 (mean-pooled h0, recipe / depth MLP heads)
  Phi           rte/macro.py:201-236 (bounded residual, z = [rmsnorm h | mean | h0])
  consistency   rte/macro.py:342-359
  replay        rte/models.py:605-679 and rte/layers.py:806-870 (exact banked passes of the
                audited sample, then coda and head)
  correction    rte/audit.py:245-387 (gradient-corrected control variate, fixed-count sampler)
  distillation  rte/macro.py:394-471 (h0-relative terms)

Nothing in the product package imports this module; bench.py's cpu_baseline leg runs it on a
bounded sample of the batch (its rows are independent, so time per token scales).
"""

from __future__ import annotations

import math

import torch
import torch.nn.functional as F

D, H, V, C, NC, TOPK = 512, 8, 2048, 64, 32, 8  # d_model, heads, vocab, clusters, neurons / cluster, top-k
FF = C * NC                                     # prelude / coda pool width
SLABS, SLAB, ACTIVE = 64, 32, 8                 # banked core: slabs of 32 neurons, 8 per recipe
RECIPES, DEPTHS, TMAX, RANK = 16, (1, 2, 4), 4, 32


def _rms(x, w=None, eps=1e-5):
    y = x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + eps)
    return y if w is None else y * w


def _rope_tables(S, hd):
    inv = 1.0 / (10_000.0 ** (torch.arange(0, hd, 2, dtype=torch.float64) / hd))
    emb = torch.outer(torch.arange(S, dtype=torch.float64), inv).repeat_interleave(2, dim=-1)
    return emb.cos().float(), emb.sin().float()


def _rope(x, cos, sin):
    rot = torch.stack([-x[..., 1::2], x[..., 0::2]], dim=-1).flatten(-2)
    return x * cos + rot * sin


def make_params(seed: int = 0) -> dict[str, torch.Tensor]:
    """Randomly initialised parameters with the cfg3 shapes (requires_grad)."""
    g = torch.Generator().manual_seed(seed)

    def rn(*shape, s):
        return (torch.randn(*shape, generator=g) * s).requires_grad_()

    def ones(*shape):
        return torch.ones(*shape).requires_grad_()

    p = {"embed": rn(V, D, s=0.02)}
    for blk in ("pre", "coda"):
        p.update({f"{blk}.n1": ones(D), f"{blk}.n2": ones(D), f"{blk}.wqkv": rn(3 * D, D, s=D ** -0.5),
                  f"{blk}.wo": rn(D, D, s=D ** -0.5), f"{blk}.wr": rn(C, D, s=D ** -0.5),
                  f"{blk}.wug": rn(2 * FF, D, s=D ** -0.5), f"{blk}.wd": rn(D, FF, s=FF ** -0.5)})
    hid = D
    p.update({"r.w1": rn(hid, D, s=D ** -0.5), "r.b1": rn(hid, s=0.0), "r.w2": rn(RECIPES, hid, s=hid ** -0.5),
              "r.b2": rn(RECIPES, s=0.0), "r.d1": rn(hid, D, s=D ** -0.5), "r.db1": rn(hid, s=0.0),
              "r.d2": rn(len(DEPTHS), hid, s=hid ** -0.5), "r.db2": rn(len(DEPTHS), s=0.0)})
    p.update({"core.n1": ones(D), "core.n2": ones(D), "core.wqkv": rn(1, D, 3 * D, s=D ** -0.5),
              "core.wo": rn(1, D, D, s=D ** -0.5), "core.wug": rn(1, D, 2 * SLABS * SLAB, s=D ** -0.5),
              "core.wd": rn(1, SLABS * SLAB, D, s=D ** -0.5), "core.g1": rn(TMAX, D, s=0.0),
              "core.b1": rn(TMAX, D, s=0.0), "core.g2": rn(TMAX, D, s=0.0), "core.b2": rn(TMAX, D, s=0.0),
              "core.sa": ones(TMAX), "core.sm": ones(TMAX), "core.alpha": rn(1, s=0.0)})
    K = len(DEPTHS)
    p.update({"m.gain": rn(RECIPES, K, D, s=0.0), "m.v": rn(RECIPES, K, 3 * D, RANK, s=(3 * D) ** -0.5),
              "m.u": rn(RECIPES, K, RANK, D, s=1e-3), "m.scale": ones(RECIPES, K, D), "m.bias": rn(RECIPES, K, D, s=0.0)})
    p["final.n"] = ones(D)
    with torch.no_grad():
        p["core.alpha"].fill_(0.1)
    return p


def _attention(x, wqkv_t, wo_t, cos, sin, head_mask=None):
    """x [B, S, D] @ wqkv_t [D, 3D] -> causal attention per head -> @ wo_t [D, D]."""
    B, S, _ = x.shape
    hd = D // H
    q, k, v = (x @ wqkv_t).view(B, S, 3, H, hd).permute(2, 0, 3, 1, 4)
    q, k = _rope(q, cos, sin), _rope(k, cos, sin)
    y = F.scaled_dot_product_attention(q, k, v, is_causal=True)
    if head_mask is not None:
        y = y * head_mask[:, :, None, None]
    return y.transpose(1, 2).reshape(B, S, D) @ wo_t


def _cluster_pool(x, wr, wug, wd):
    """Top-k routed cluster pool: weights = softmax over the k selected router logits."""
    B, S, _ = x.shape
    xt = x.reshape(-1, D)
    vals, ids = (xt @ wr.t()).topk(TOPK, dim=-1)
    w = vals.softmax(dim=-1)
    out = torch.zeros_like(xt)
    for c in range(C):
        tok, slot = (ids == c).nonzero(as_tuple=True)
        if tok.numel() == 0:
            continue
        xc = xt[tok]
        up = xc @ wug[c * NC:(c + 1) * NC].t()
        gate = xc @ wug[FF + c * NC:FF + (c + 1) * NC].t()
        out = out.index_add(0, tok, w[tok, slot, None] * ((up * F.silu(gate)) @ wd[:, c * NC:(c + 1) * NC].t()))
    return out.view(B, S, D)


def _block(x, p, blk, cos, sin):
    u = x + _attention(_rms(x, p[f"{blk}.n1"]), p[f"{blk}.wqkv"].t(), p[f"{blk}.wo"].t(), cos, sin)
    return u + _cluster_pool(_rms(u, p[f"{blk}.n2"]), p[f"{blk}.wr"], p[f"{blk}.wug"], p[f"{blk}.wd"])


def _router(h0, p):
    pooled = h0.mean(dim=1)
    rl = F.silu(pooled @ p["r.w1"].t() + p["r.b1"]) @ p["r.w2"].t() + p["r.b2"]
    dl = F.silu(pooled @ p["r.d1"].t() + p["r.db1"]) @ p["r.d2"].t() + p["r.db2"]
    return rl, dl


def _phi(h, h0, rid, sid, p, c=0.05):
    n = _rms(h)
    z = torch.cat([n, n.mean(dim=1, keepdim=True).expand_as(n), h0], dim=-1)
    g = lambda t: t[rid, sid]  # noqa: E731
    low = torch.bmm(F.silu(torch.bmm(z, g(p["m.v"]))), g(p["m.u"]))
    upd = g(p["m.gain"]).unsqueeze(1) * h + low + g(p["m.bias"]).unsqueeze(1)
    return h + c * g(p["m.scale"]).unsqueeze(1) * torch.tanh(upd)


def _recipe_groups(r):
    """Active slab groups / head mask of recipe r (recipe 0: every group; r >= 1 round-robin)."""
    if r == 0:
        return list(range(SLABS)), torch.ones(H)
    slots = SLABS // ACTIVE
    s = (r - 1) % slots
    heads = torch.zeros(H)
    hs = (r - 1) % (8 // 2)
    heads[hs * 2:(hs + 1) * 2] = 1.0
    return [(s * ACTIVE + j) % SLABS for j in range(ACTIVE)], heads


def _core_pass(h, h0, r, t, p, cos, sin):
    groups, heads = _recipe_groups(r)
    ht = h + p["core.alpha"] * h0
    n1 = _rms(ht, p["core.n1"]) * (1.0 + p["core.g1"][t]) + p["core.b1"][t]
    u = ht + p["core.sa"][t] * _attention(n1, p["core.wqkv"][0], p["core.wo"][0], cos, sin, heads[None, :])
    n2 = _rms(u, p["core.n2"]) * (1.0 + p["core.g2"][t]) + p["core.b2"][t]
    cols = torch.tensor([c for gi in groups for c in range(gi * SLAB, (gi + 1) * SLAB)])
    F2 = SLABS * SLAB
    up = n2 @ p["core.wug"][0][:, cols]
    gate = n2 @ p["core.wug"][0][:, cols + F2]
    return u + p["core.sm"][t] * ((up * F.silu(gate)) @ p["core.wd"][0][cols])


def _head_ce(hidden, p, targets):
    logits = _rms(hidden, p["final.n"]) @ p["embed"].t()
    tok = F.cross_entropy(logits.flatten(0, 1), targets.flatten(), reduction="none").view_as(targets)
    return logits, tok


def train_step(p, opt, tokens, targets, audit_row: int = 0):
    """One step: forward_macro, fixed-count audit replay of one sample, consistency loss,
    distillation and router aux terms, backward, AdamW.  Returns the loss."""
    B, S = tokens.shape
    cos, sin = _rope_tables(S, D // H)
    h0 = _block(p["embed"][tokens], p, "pre", cos, sin)
    rl, dl = _router(h0, p)
    rid = rl.argmax(dim=-1)
    sid = torch.full((B,), DEPTHS.index(4), dtype=torch.long)
    h = _phi(h0, h0, rid, sid, p)
    hid = _block(h, p, "coda", cos, sin)
    logits, tok = _head_ce(hid, p, targets)
    lps = tok.sum(dim=-1)
    # exact replay of the audited sample: 4 banked passes, coda, head
    i = audit_row
    he, h0i = h0[i:i + 1], h0[i:i + 1]
    for t in range(TMAX):
        he = _core_pass(he, h0i, int(rid[i]), t, p, cos, sin)
    lg_e, tok_e = _head_ce(_block(he, p, "coda", cos, sin), p, targets[i:i + 1])
    # gradient-corrected control variate with inclusion probability 1 / B
    pinc = 1.0 / B
    corrected = lps + (torch.arange(B) == i).float() * (tok_e.sum() - lps[i]) / pinc
    # consistency over the (1, 2), (2, 4) stride pairs
    hr = h0.repeat(2, 1, 1)
    rr = rid.repeat(2)
    src = torch.tensor([0, 1]).repeat_interleave(B)
    dst = torch.tensor([1, 2]).repeat_interleave(B)
    cons = (_phi(hr, hr, rr, dst, p) - _phi(_phi(hr, hr, rr, src, p), hr, rr, src, p)).square().mean()
    # distillation of the audited sample (h0-relative terms), exact side detached
    dp, de = h[i:i + 1] - h0i, (he - h0i).detach()
    ddir = 1.0 - F.cosine_similarity(dp.flatten(1), de.flatten(1), dim=-1).mean()
    drms = (dp.pow(2).mean().sqrt().clamp_min(1e-8).log() - de.pow(2).mean().sqrt().clamp_min(1e-8).log()).square()
    kl = F.kl_div(F.log_softmax(logits[i:i + 1], -1), F.log_softmax(lg_e, -1).detach(), log_target=True,
                  reduction="batchmean")
    # router aux: load balance of the recipe probabilities and expected depth
    probs = rl.softmax(-1)
    load = (probs.mean(0) * RECIPES).square().mean()
    depth = (dl.softmax(-1) * torch.tensor(DEPTHS, dtype=torch.float32)).sum(-1).mean()
    loss = (corrected.mean() / S + 1e-3 * cons + 2.0 * ddir + 2.0 * drms + 1e-2 * kl + 1e-2 * load
            + 1e-4 * depth)
    opt.zero_grad(set_to_none=True)
    loss.backward()
    torch.nn.utils.clip_grad_norm_(list(p.values()), 1.0)
    opt.step()
    return float(loss.detach())


def make_optimizer(p):
    return torch.optim.AdamW(list(p.values()), lr=3e-4, weight_decay=0.1)


def zipf_tokens(B: int, S: int, seed: int = 0):
    g = torch.Generator().manual_seed(seed)
    pr = (torch.arange(V, dtype=torch.float64) + 1.0).pow(-1.1)
    ids = torch.multinomial((pr / pr.sum()).float(), B * (S + 1), replacement=True, generator=g).view(B, S + 1)
    return ids[:, :-1], ids[:, 1:]


def flops_per_token() -> float:
    """Forward matmul flops per token of the main path (fwd + bwd ~ 3x), for reference."""
    blk = 2 * D * 3 * D + 2 * D * D + 2 * TOPK * (2 * D * 2 * NC) + 2 * D * C
    return 2 * blk + 2 * D * V + 2 * (3 * D * RANK + RANK * D) * 5


assert math.isfinite(flops_per_token())
