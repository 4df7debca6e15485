"""Dense and recursive decoders (rte/models.py:73-723) on the HIP blocks.

RecursiveModel.forward_macro (rte/models.py:681-723) is the recursive_macro hot path:
prelude blocks -> per-sample router -> macro operator Phi -> coda blocks -> logits.
forward_exact_from_h0 / forward_exact_subset replay audited samples exactly through the
banked recursive core (rte/models.py:416-512, :605-679).
"""

from __future__ import annotations

from dataclasses import dataclass

import torch
import torch.nn.functional as F
from torch import nn

from rte_amd.config import ModelConfig, OutputConfig
from rte_amd.kernels import hip_ops
from rte_amd.kernels import optimized as K
from rte_amd.layers import BankedRecursiveCore, Embedding, RMSNorm, TransformerBlock
from rte_amd.macro import MacroOperators, MacroTrace
from rte_amd.output import ShortlistHead, ShortlistResult
from rte_amd.recipes import RecipeBank
from rte_amd.routing import Router, RouterOutput


@dataclass(slots=True)
class ModelMeta:
    router: RouterOutput | None = None
    recipe_ids: torch.Tensor | None = None
    depths: torch.Tensor | None = None
    h0: torch.Tensor | None = None
    recurrent_hidden: torch.Tensor | None = None
    hidden: torch.Tensor | None = None
    logits: torch.Tensor | None = None
    states: dict[int, torch.Tensor] | None = None
    macro_trace: MacroTrace | None = None
    shortlist: ShortlistResult | None = None
    touch_table: torch.Tensor | None = None
    token_loss: torch.Tensor | None = None
    # the LM head's output these logits are rows of, when the head ran over more rows than this
    # output's (the hot path's coda call that also carries the audit replay's rows)
    logit_source: torch.Tensor | None = None

    @property
    def active_touches(self) -> torch.Tensor | None:
        """Per-sample active touches of the chosen recipes (looked up when read)."""
        if self.touch_table is None or self.recipe_ids is None:
            return None
        return self.touch_table[self.recipe_ids]


@dataclass(slots=True)
class ExactCore:
    """The exact replay of the audited samples up to its last recursive pass: their indices, the
    routing decisions and h0 rows they reuse, the final recurrent state h and the kept states."""
    idx: torch.Tensor
    route: RouterOutput
    h0: torch.Tensor
    h: torch.Tensor
    states: dict


class ModelOutput:
    """loss (the mean of the per-sample losses), loss_per_sample, logits, meta.  Given the
    per-sample losses as `mean_of`, the mean is taken when `loss` is first read (the training
    step composes its own loss from the per-sample values and never reads it)."""

    __slots__ = ("_loss", "_mean_of", "loss_per_sample", "logits", "meta")

    def __init__(self, loss, loss_per_sample, logits, meta, *, mean_of=None):
        self._loss, self._mean_of = loss, mean_of
        self.loss_per_sample, self.logits, self.meta = loss_per_sample, logits, meta

    @property
    def loss(self):
        if self._loss is None and self._mean_of is not None:
            self._loss, self._mean_of = self._mean_of.mean(), None
        return self._loss


def lm_loss_per_sample(logits: torch.Tensor, targets: torch.Tensor) -> torch.Tensor:
    """Sum over the sequence of token cross-entropy (rte/models.py:73-75)."""
    tok = F.cross_entropy(logits.float().flatten(0, -2), targets.flatten(), reduction="none")
    return tok.view_as(targets).sum(dim=-1)


def head_logits_loss(hidden, vocab_weight, targets):
    """(logits, per-sample CE, token CE) with the HIP LM-head GEMM + fused CE kernels; targets
    may be None."""
    if targets is None:
        return hip_ops.linear(hidden, vocab_weight, out_f32=True), None, None
    logits, tok = hip_ops.lm_head_ce(hidden, vocab_weight, targets)
    return logits, tok.sum(dim=-1), tok


class DenseModel(nn.Module):
    def __init__(self, config: ModelConfig):
        super().__init__()
        if config.topology != "dense":
            raise ValueError("DenseModel requires topology='dense'")
        self.config = config
        self.embed = Embedding(config.vocab_size, config.d_model)
        self.blocks = nn.Sequential(*[TransformerBlock(config) for _ in range(config.n_dense_layers)])
        self.final_norm = RMSNorm(config.d_model)
        self.lm_head = None if config.tie_embeddings else nn.Linear(config.d_model, config.vocab_size, bias=False)

    @property
    def vocab_weight(self) -> torch.Tensor:
        return self.embed.weight if self.lm_head is None else self.lm_head.weight

    def forward(self, tokens, targets=None, return_loss_per_sample=False, return_states=False) -> ModelOutput:
        x = self.embed(tokens)
        for block in self.blocks:
            x = block(x)
        hidden = self.final_norm(x)
        logits, lps, tok = head_logits_loss(hidden, self.vocab_weight, targets)
        return ModelOutput(lps.mean() if lps is not None else None, lps if return_loss_per_sample else None, logits,
                           ModelMeta(hidden=hidden, logits=logits, token_loss=tok))


class RecursiveModel(nn.Module):
    def __init__(self, config: ModelConfig, output_config: OutputConfig | None = None):
        super().__init__()
        if config.topology != "recursive":
            raise ValueError("RecursiveModel requires topology='recursive'")
        self.config = config
        self.output_config = output_config or OutputConfig()
        self.recipe_bank = RecipeBank(config)
        self.register_buffer("active_touch_table", self.recipe_bank.active_touch_table, persistent=False)
        self.register_buffer("pass_index", torch.arange(config.t_max), persistent=False)
        self.embed = Embedding(config.vocab_size, config.d_model)
        self.prelude = nn.Sequential(*[TransformerBlock(config) for _ in range(config.n_prelude)])
        self.router = Router(config)
        self.core = BankedRecursiveCore(config, self.recipe_bank)
        self.macro = MacroOperators(config)
        self.coda = nn.Sequential(*[TransformerBlock(config) for _ in range(config.n_coda)])
        self.final_norm = RMSNorm(config.d_model)
        self.lm_head = None if config.tie_embeddings else nn.Linear(config.d_model, config.vocab_size, bias=False)
        self.shortlist_head = ShortlistHead(config.d_model, config.vocab_size, self.output_config)

    @property
    def vocab_weight(self) -> torch.Tensor:
        return self.embed.weight if self.lm_head is None else self.lm_head.weight

    def _prelude(self, tokens):
        x = self.embed(tokens)
        for block in self.prelude:
            x = block(x)
        return x

    def _coda_hidden(self, h):
        for block in self.coda:
            h = block(h)
        return self.final_norm(h)

    def _coda_logits(self, h):
        hidden = self._coda_hidden(h)
        return hidden, hip_ops.linear(hidden, self.vocab_weight, out_f32=True)

    def _factorized_topk_routes(self, route: RouterOutput, *, pass_idx: int, top_k: int):
        """(factors [B, k, 4] long = (attn bank, ffn bank, head slot, ffn slot), weights [B, k]) of
        the k best factor tuples of one pass by summed factor logits (rte/models.py:273-310): the
        outer-sum scores go through the HIP top-k (value desc, flat index asc, softmax over the
        selected)."""
        req = [route.attn_bank_logits_by_pass, route.ffn_bank_logits_by_pass, route.head_slot_logits_by_pass,
               route.ffn_slot_logits_by_pass]
        if any(v is None for v in req):
            raise RuntimeError("factorized routing requires factor logits from the router")
        a, b, c, e = (v[:, pass_idx, :] for v in req)
        scores = (a[:, :, None, None, None] + b[:, None, :, None, None] + c[:, None, None, :, None]
                  + e[:, None, None, None, :]).flatten(1).float()
        k = min(max(1, int(top_k)), scores.shape[-1])
        ids, weights = hip_ops.route_topk(scores, k)
        head_slots, ffn_slots = self.router.head_slots, self.router.ffn_slots
        flat = ids.long()
        ffn_slot = flat % ffn_slots
        flat = flat // ffn_slots
        head_slot = flat % head_slots
        flat = flat // head_slots
        ffn_bank = flat % self.config.ffn_banks
        attn_bank = flat // self.config.ffn_banks
        return torch.stack([attn_bank, ffn_bank, head_slot, ffn_slot], dim=-1), weights

    def forward_exact_from_h0(self, h0, targets=None, return_states=False, return_loss_per_sample=False, *,
                              router_decisions: RouterOutput | None = None, fixed_recipe=None, fixed_depth=None):
        route = router_decisions or self.router(h0, fixed_recipe=fixed_recipe, fixed_depth=fixed_depth)
        h, states = self._exact_core(h0, route, return_states)
        hidden = self._coda_hidden(h)
        logits, lps, tok = head_logits_loss(hidden, self.vocab_weight, targets)
        return self._exact_output(route, h0, h, states, hidden, logits, lps, tok, return_states,
                                  return_loss_per_sample)

    def _exact_output(self, route, h0, h, states, hidden, logits, lps, tok, return_states, return_loss_per_sample,
                      logit_source=None):
        meta = ModelMeta(router=route, recipe_ids=route.recipe_id, depths=route.depth, h0=h0, recurrent_hidden=h,
                         hidden=hidden, logits=logits, states=states if return_states else None,
                         touch_table=self.active_touch_table, token_loss=tok, logit_source=logit_source)
        return ModelOutput(None, lps if return_loss_per_sample else None, logits, meta, mean_of=lps)

    def _exact_core(self, h0, route: RouterOutput, return_states: bool):
        """The exact recursive passes of rte/models.py:416-512 from h0: (h, kept states)."""
        h = h0
        states: dict[int, torch.Tensor] = {}
        T = self.config.t_max
        # every pass's recipe ids, active masks and head scales in one launch each
        rid_bp = route.recipe_id_by_pass
        rids = (rid_bp.t() if rid_bp is not None else route.recipe_id.reshape(1, -1).expand(T, -1)).contiguous()
        # a fixed depth of at least T (known on the host) keeps every sample active in every pass:
        # no pass masks, and with one recipe per sample every pass shares one pool pack
        fixed = getattr(route, "fixed_depth_value", None)
        all_active = fixed is not None and fixed >= T
        actives = None if all_active else self.pass_index[:T, None] < route.depth.reshape(1, -1)
        if self.core.replay_fused_ok(h0):
            # every pass as one node on the replay kernels (the few audited rows of the exact replay)
            keep = [t for t in range(T - 1) if return_states and (t + 1) in self.config.depth_choices]
            h, *kept = self.core.forward_replay(h0, rids.long(), actives, keep)
            h = h.to(h0.dtype)
            states = {t + 1: s.to(h0.dtype) for t, s in zip(keep, kept)}
            if return_states and T in self.config.depth_choices:
                states[T] = h
        else:
            weights = self.core.prepare()
            if all_active and rid_bp is None:
                weights["pool_pack"] = self.core.mlp.pack_recipes(rids[0], h0.shape[1])
            head_scales = self.core.attn.recipe_head_scale[rids.long()]
            for t in range(T):
                h = self.core.forward_step(h, h0, rids[t], None if actives is None else actives[t], pass_idx=t,
                                           weights=weights, head_scale=head_scales[t])
                if return_states and (t + 1) in self.config.depth_choices:
                    states[t + 1] = h  # every pass returns a new tensor; nothing writes h in place
        return h, states

    def forward_exact(self, tokens, targets=None, return_states=False, return_loss_per_sample=False, **kw):
        return self.forward_exact_from_h0(self._prelude(tokens), targets, return_states, return_loss_per_sample, **kw)

    def forward_exact_subset(self, tokens, targets, audit_index, *, reuse_router_decisions: RouterOutput,
                             cached_h0=None, return_states=True, return_loss_per_sample=True):
        """Exact replay of the audited samples (audit_index: long indices or a bool mask),
        reusing the hot path's routing decisions and cached prelude state (rte/models.py:605-679)."""
        idx = audit_index.nonzero(as_tuple=False).flatten() if audit_index.dtype == torch.bool else audit_index
        route = reuse_router_decisions.subset(idx)
        if cached_h0 is not None:
            h0 = hip_ops.select_rows(cached_h0, idx)
        else:
            h0 = self._prelude(tokens.index_select(0, idx))
        return self.forward_exact_from_h0(h0, targets.index_select(0, idx), return_states, return_loss_per_sample,
                                          router_decisions=route)

    def forward_exact_subset_core(self, audit_index, *, reuse_router_decisions: RouterOutput, cached_h0,
                                  return_states=True) -> ExactCore:
        """forward_exact_subset up to the last recursive pass: the coda and the head of these rows
        can then run in another call (finish_exact builds the replay's output from its rows)."""
        idx = audit_index.nonzero(as_tuple=False).flatten() if audit_index.dtype == torch.bool else audit_index
        route = reuse_router_decisions.subset(idx)
        h0 = hip_ops.select_rows(cached_h0, idx)
        h, states = self._exact_core(h0, route, return_states)
        return ExactCore(idx, route, h0, h, states)

    def finish_exact(self, core: ExactCore, hidden, logits, lps, tok, *, logit_source=None,
                     return_states=True, return_loss_per_sample=True) -> ModelOutput:
        """The replay's output from its rows of a coda / head call: hidden [A, S, d], logits
        [A, S, V], per-sample and token cross-entropy; logit_source = the head's whole output."""
        return self._exact_output(core.route, core.h0, core.h, core.states, hidden, logits, lps, tok, return_states,
                                  return_loss_per_sample, logit_source=logit_source)

    def forward_macro(self, tokens, targets=None, return_states=False, return_loss_per_sample=False, *,
                      shortlist=False, seed=0, fixed_recipe=None, fixed_depth=None,
                      shortlist_random_negs=None, on_routed=None, coda_extra=None) -> ModelOutput:
        """rte/models.py:681-723.  on_routed(h0, route), if given, runs right after routing: the
        training step uses it to start the audit replay on its own stream while the hot path runs.
        coda_extra(), if given and it returns an object (full-vocabulary head with targets), adds
        rows to the coda, final norm, head and cross-entropy call: `.rows()` -> (h [A, S, d],
        targets [A, S]), and `.done(hidden, logits, lps, tok, source)` receives their outputs
        (the audit replay's rows: one set of launches for both instead of two)."""
        h0 = self._prelude(tokens)
        route = self.router(h0, fixed_recipe=fixed_recipe, fixed_depth=fixed_depth)
        if on_routed is not None:
            on_routed(h0, route)
        # the macro strides are the depth choices: with distinct choices a depth's stride id is its
        # depth id (stride_ids_for_depths: first stride equal to the depth)
        sid = route.depth_id if len(set(self.config.depth_choices)) == len(self.config.depth_choices) else None
        h, trace = self.macro(h0, h0, route.recipe_id, route.depth, return_states=return_states, stride_ids=sid)
        sl, source = None, None
        if shortlist and targets is not None:
            hidden = self._coda_hidden(h)
            full_logits = None
            sl = self.shortlist_head.loss(hidden, targets, self.vocab_weight, seed=seed,
                                          random_negs=shortlist_random_negs)
            lps, logits, tok = sl.loss_per_sample, sl.logits, sl.token_loss
        else:
            extra = coda_extra() if coda_extra is not None and targets is not None else None
            if extra is not None:
                hx, tx = extra.rows()
                B = h.shape[0]
                hidden_all = self._coda_hidden(torch.cat([h, hx.to(h.dtype)]))
                source, lps_all, tok_all = head_logits_loss(hidden_all, self.vocab_weight, torch.cat([targets, tx]))
                hidden, full_logits, lps, tok = hidden_all[:B], source[:B], lps_all[:B], tok_all[:B]
                extra.done(hidden_all[B:], source[B:], lps_all[B:], tok_all[B:], source)
            else:
                hidden = self._coda_hidden(h)
                full_logits, lps, tok = head_logits_loss(hidden, self.vocab_weight, targets)
            logits = full_logits
        meta = ModelMeta(router=route, recipe_ids=route.recipe_id, depths=route.depth, h0=h0, recurrent_hidden=h,
                         hidden=hidden, logits=full_logits, states=trace.states if return_states else None,
                         macro_trace=trace, shortlist=sl, touch_table=self.active_touch_table,
                         token_loss=tok, logit_source=source)
        return ModelOutput(None, lps if return_loss_per_sample else None, logits, meta, mean_of=lps)
