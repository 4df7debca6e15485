"""Per-sample recipe / depth router oracle (numpy, float64) — TEST INFRASTRUCTURE ONLY.

Restates Router.forward (rte/routing.py:80-188; rte/ = src/recursive_training_engine/ of the
reference): pooled = mean over the sequence of h0; recipe / depth / factor MLPs Linear -> SiLU
-> Linear; per-pass recipe logits add pass_recipe_bias; factor hidden = silu(factor MLP +
pass_factor_bias); four factor heads; softmax, argmax (first maximal index), entropies with
the 1e-9 clamp, expected depth.  p holds numpy weights keyed like the module's state dict.
"""

from __future__ import annotations

import numpy as np

from oracle.swiglu import silu


def _lin(x, p, name):
    return x @ np.asarray(p[name + ".weight"], np.float64).T + np.asarray(p[name + ".bias"], np.float64)


def _mlp(x, p, name):
    return _lin(silu(_lin(x, p, name + ".0")), p, name + ".2")


def _softmax(x):
    e = np.exp(x - x.max(-1, keepdims=True))
    return e / e.sum(-1, keepdims=True)


def _entropy(pr):
    return -(np.log(np.maximum(pr, 1e-9)) * pr).sum(-1)


def router(h0, p, depth_choices, temperature=1.0):
    h0 = np.asarray(h0, np.float64)
    pooled = h0.mean(1)
    inv = 1.0 / max(temperature, 1e-6)
    out = {"pooled": pooled}
    out["recipe_logits"] = _mlp(pooled, p, "recipe_mlp") * inv
    out["depth_logits"] = _mlp(pooled, p, "depth_mlp") * inv
    out["recipe_logits_by_pass"] = out["recipe_logits"][:, None, :] + np.asarray(p["pass_recipe_bias"]) * inv
    for k in ("recipe", "depth"):
        out[k + "_probs"] = _softmax(out[k + "_logits"])
        out[k + "_id"] = out[k + "_probs"].argmax(-1)
        out[k + "_entropy"] = _entropy(out[k + "_probs"])
    out["recipe_probs_by_pass"] = _softmax(out["recipe_logits_by_pass"])
    out["recipe_id_by_pass"] = out["recipe_probs_by_pass"].argmax(-1)
    out["expected_depth"] = (out["depth_probs"] * np.asarray(depth_choices, np.float64)).sum(-1)
    fh = silu(_mlp(pooled, p, "factor_mlp")[:, None, :] + np.asarray(p["pass_factor_bias"], np.float64))
    ent = 0.0
    for name in ("attn_bank", "ffn_bank", "head_slot", "ffn_slot"):
        lg = _lin(fh, p, name + "_head") * inv
        pr = _softmax(lg)
        out[name + "_logits_by_pass"] = lg
        out[name + "_id_by_pass"] = pr.argmax(-1)
        ent = ent + _entropy(pr)
    out["factor_entropy"] = ent.mean(-1)
    return out


def factorized_topk(attn, ffn_bank, head_slot, ffn_slot, top_k):
    """_factorized_topk_routes (rte/models.py:273-310) for one pass: scores over the outer sum of
    the four factor logits, top-k (value desc, index asc), the flat id decoded as
    ((attn * ffn_banks + ffn_bank) * head_slots + head_slot) * ffn_slots + ffn_slot, weights =
    softmax of the selected scores."""
    from oracle.routing import route_topk

    A, Fb, Hs, Fs = attn.shape[-1], ffn_bank.shape[-1], head_slot.shape[-1], ffn_slot.shape[-1]
    s = (attn[:, :, None, None, None] + ffn_bank[:, None, :, None, None] + head_slot[:, None, None, :, None]
         + ffn_slot[:, None, None, None, :])
    flat = s.reshape(s.shape[0], -1).astype(np.float32)
    k = min(max(1, int(top_k)), flat.shape[-1])
    ids, w = route_topk(flat, k)
    fs = ids % Fs
    r = ids // Fs
    hs = r % Hs
    r = r // Hs
    fb = r % Fb
    ab = r // Fb
    return np.stack([ab, fb, hs, fs], -1).astype(np.int64), w
