"""Control-variate audit of the macro hot path (rte/audit.py:20-387).

A sampled subset of the batch is replayed exactly; its per-sample loss replaces the hot
loss through corrected = hot + (exact - hot) / p (gradient-corrected mode), which keeps
the loss estimate unbiased for inclusion probability p.
"""

from __future__ import annotations

from contextlib import contextmanager, nullcontext
from dataclasses import dataclass

import torch

from rte_amd.config import TrainingConfig
from rte_amd.kernels import hip_ops
from rte_amd.macro import macro_alignment_metrics, macro_distill_loss
from rte_amd.models import ModelMeta, ModelOutput, RecursiveModel


@dataclass(slots=True)
class AuditResult:
    audit_mask: torch.Tensor
    p_audit: torch.Tensor
    exact: ModelOutput | None
    corrected_loss_per_sample: torch.Tensor
    macro_aux: dict[str, torch.Tensor]
    metrics: dict[str, torch.Tensor]


class GradSink:
    """Parameter gradients of side-stream work, kept apart from the engine's accumulation and
    added to the parameters' .grad in one multi-tensor launch after the backward (flush()),
    instead of one add per parameter where the side streams join the main stream."""

    def __init__(self):
        self.entries: list = []

    def flush(self) -> None:
        have = [(p, g) for p, g in self.entries if p.grad is not None]
        if have:
            torch._foreach_add_([p.grad for p, _ in have], [g for _, g in have])
        for p, g in self.entries:
            if p.grad is None:
                p.grad = g
        self.entries.clear()


class _SinkView(torch.autograd.Function):
    """A view of parameter p whose gradient goes to a GradSink instead of p's accumulator."""

    @staticmethod
    def forward(ctx, p, sink):
        ctx.p, ctx.sink = p, sink
        return p.view_as(p)

    @staticmethod
    def backward(ctx, g):
        ctx.sink.entries.append((ctx.p, g))
        return None, None


def make_main_aliases(*modules, sink: GradSink | None = None) -> dict:
    """The views main_stream_aliases installs, made now on the current stream: the autograd nodes
    of views made early run late in the backward (the engine runs later-made nodes first), so a
    launch whose compute is issued later can still join its parameter gradients at the end.
    With a sink the views' gradients go to it (GradSink.flush adds them after the backward)."""
    alias: dict[int, torch.Tensor] = {}
    if torch.is_grad_enabled():
        for mod in modules:
            for p in mod.parameters():
                if p.requires_grad and id(p) not in alias:
                    alias[id(p)] = _SinkView.apply(p, sink) if sink is not None else p.view_as(p)
    return alias


@contextmanager
def _aliases_installed(alias: dict, *modules):
    swaps = []
    for mod in modules:
        for m in mod.modules():
            for name, p in list(m._parameters.items()):
                if p is None or id(p) not in alias:
                    continue
                m._parameters[name] = alias[id(p)]
                swaps.append((m, name, p))
    try:
        yield
    finally:
        for m, name, p in swaps:
            m._parameters[name] = p


@contextmanager
def main_stream_aliases(*modules):
    """Inside the block every trainable parameter of `modules` reads as a view of itself made on
    the stream current at entry (one view per parameter, shared by every module holding it).

    Work issued on a side stream inside the block then differentiates into those views, whose
    backward runs on the entry stream, so each parameter's gradient accumulator is fed from that
    one stream (autograd warns, and synchronises, when a leaf's accumulator receives gradients
    produced on another stream than its own)."""
    if not torch.is_grad_enabled():
        yield
        return
    alias: dict[int, torch.Tensor] = {}
    swaps = []
    for mod in modules:
        for m in mod.modules():
            for name, p in list(m._parameters.items()):
                if p is None or not p.requires_grad:
                    continue
                a = alias.get(id(p))
                if a is None:
                    a = alias[id(p)] = p.view_as(p)
                m._parameters[name] = a
                swaps.append((m, name, p))
    try:
        yield
    finally:
        for m, name, p in swaps:
            m._parameters[name] = p


@dataclass(slots=True)
class AuditLaunch:
    """Work started right after routing: the exact replay of the audited rows and the macro
    consistency loss.  correction() joins the streams before using them.  With a deferred coda
    the replay stops after its recursive passes and the hot path's coda call runs its coda and
    head (`coda_extra`), which also builds its output."""
    chosen: torch.Tensor | None
    exact: ModelOutput | None
    cons: torch.Tensor | None
    streams: list
    coda_extra: "_CodaRows | None" = None


class _CodaRows:
    """The audited samples' final recurrent states handed to the hot path's coda call
    (RecursiveModel.forward_macro coda_extra): rows() joins the replay's stream and gives the rows
    and their targets, done() builds the replay's output from its rows of the call's outputs.  It
    holds no reference to its launch: a launch <-> rows cycle would keep the replay's autograd
    graph (and the AccumulateGrad nodes in it) alive until the cyclic collector runs."""

    def __init__(self, model: RecursiveModel, core, targets, side):
        self.model, self.core, self.targets, self.side = model, core, targets, side
        self.exact: ModelOutput | None = None

    def rows(self):
        h = self.core.h
        main = torch.cuda.current_stream(h.device)
        if self.side != main:
            main.wait_stream(self.side)
            h.record_stream(main)
        return h, self.targets.index_select(0, self.core.idx)

    def done(self, hidden, logits, lps, tok, source):
        self.exact = self.model.finish_exact(self.core, hidden, logits, lps, tok, logit_source=source)


class AuditEngine:
    def __init__(self, config: TrainingConfig):
        self.config = config
        self.recent_residual = 0.0
        self.recipe_audit_ema: torch.Tensor | None = None
        self.last_candidate_count = 0
        self.last_capped_fraction = 0.0
        self.last_sample_mode = "bernoulli"
        # False: the work begin() starts runs on the caller's stream, in order (one stream)
        self.side_streams = True
        # the consistency loss in order on the caller's stream (the replay alone on a side stream)
        self.consistency_on_main = True
        # late launch on the caller's stream: the consistency term's backward right after its
        # forward (it reads neither the replay nor the hot path), so it runs while the step waits
        # for the replay; its h0 gradient joins the step's at h0 (a hook)
        self.consistency_backward_early = True

    def state_dict(self) -> dict[str, object]:
        return {
            "recent_residual": self.recent_residual,
            "recipe_audit_ema": self.recipe_audit_ema,
            "last_candidate_count": self.last_candidate_count,
            "last_capped_fraction": self.last_capped_fraction,
            "last_sample_mode": self.last_sample_mode,
        }

    def load_state_dict(self, state: dict[str, object]) -> None:
        self.recent_residual = float(state.get("recent_residual", 0.0))
        ema = state.get("recipe_audit_ema")
        self.recipe_audit_ema = ema if isinstance(ema, torch.Tensor) else None
        self.last_candidate_count = int(state.get("last_candidate_count", 0))
        self.last_capped_fraction = float(state.get("last_capped_fraction", 0.0))
        self.last_sample_mode = str(state.get("last_sample_mode", "bernoulli"))

    def _coverage_deficit(self, recipe_ids, recipe_count):
        if self.recipe_audit_ema is None or self.recipe_audit_ema.numel() != recipe_count:
            self.recipe_audit_ema = torch.zeros(recipe_count, dtype=torch.float32, device=recipe_ids.device)
        ema = self.recipe_audit_ema.to(recipe_ids.device)
        return (self.config.coverage_min - ema[recipe_ids]).clamp_min(0.0) / max(self.config.coverage_min, 1e-12)

    def _update_coverage(self, recipe_ids, mask):
        if self.recipe_audit_ema is None:
            return
        ema = self.recipe_audit_ema.to(recipe_ids.device)
        counts = torch.zeros_like(ema).index_add_(0, recipe_ids.long(), mask.float())
        probs = counts / counts.sum().clamp_min(1.0)
        ema.mul_(self.config.coverage_beta).add_(probs, alpha=1.0 - self.config.coverage_beta)
        self.recipe_audit_ema = ema.detach()

    def compute_audit_prob(self, meta: ModelMeta) -> torch.Tensor:
        """rte/audit.py:79-97."""
        r = meta.router
        unc = r.router_entropy / (r.recipe_logits.shape[-1] + r.depth_logits.shape[-1])
        p = (self.config.audit_p_min + self.config.audit_alpha * unc
             + self.config.audit_beta * torch.full_like(unc, self.recent_residual)
             + self.config.audit_gamma * self._coverage_deficit(meta.recipe_ids, r.recipe_logits.shape[-1]))
        return p.clamp(self.config.audit_p_min, self.config.audit_p_max)

    def _zero(self, like: torch.Tensor) -> torch.Tensor:
        """A read-only zero scalar like `like`, made once per device and dtype (the auxiliary
        terms a step does not form)."""
        cache = self.__dict__.setdefault("_zeros", {})
        key = (str(like.device), like.dtype)
        if key not in cache:
            cache[key] = like.new_zeros(())
        return cache[key]

    def _side_stream(self, device, slot: int):
        if not self.side_streams:
            return torch.cuda.current_stream(device)
        streams = self.__dict__.setdefault("_streams", {})
        key = (device.index if device.index is not None else torch.cuda.current_device(), slot)
        if key not in streams:
            streams[key] = torch.cuda.Stream(device=device)  # default priority
        return streams[key]

    def begin(self, model: RecursiveModel, tokens, targets, h0, route, *, seed: int,
              chosen: torch.Tensor | None = None, defer_coda: bool = False,
              ready: torch.cuda.Event | None = None, aliases: dict | None = None) -> AuditLaunch | None:
        """Start the fixed-count audit's exact replay and the macro consistency loss as soon as h0
        and the routing decisions exist: on their own streams (side_streams), so they and their
        backward can run beside the hot path, else in order on the caller's stream.  defer_coda:
        the replay runs its recursive passes only and hands its coda and head to the hot path's
        coda call (launch.coda_extra).  ready / aliases (issued later than routing): the side
        streams wait for this event, recorded on the main stream when h0 and the routes were
        made, instead of the main stream's current work, and the parameters read through these
        views (make_main_aliases at the same point); the main-stream preparation the side streams
        read (prepare_late: the audited rows, the operator's weight copies) must precede that
        event.  Returns None when nothing can start early (Bernoulli sampler, no device)."""
        fixed = self.config.audit_fixed_count_per_batch
        if fixed is None or h0.device.type != "cuda":
            return None
        n = h0.shape[0]
        k = min(int(fixed), n)
        main = torch.cuda.current_stream(h0.device)
        launch = AuditLaunch(None, None, None, [])
        if k > 0:
            if chosen is None:
                if ready is not None:
                    raise ValueError("begin: a late launch takes the audited rows from prepare_late")
                chosen = self.fixed_count_index(n, k, seed, h0.device)
            side = self._side_stream(h0.device, 0)
            if side != main:
                side.wait_event(ready) if ready is not None else side.wait_stream(main)
            grad_corr = self.config.audit_mode == "gradient_corrected"
            with (nullcontext() if grad_corr else torch.no_grad()), \
                    (nullcontext() if side == main else
                     _aliases_installed(aliases, model) if aliases is not None else main_stream_aliases(model)):
                with torch.cuda.stream(side):
                    if defer_coda:
                        core = model.forward_exact_subset_core(chosen, reuse_router_decisions=route, cached_h0=h0)
                        launch.coda_extra = _CodaRows(model, core, targets, side)
                    else:
                        launch.exact = model.forward_exact_subset(tokens, targets, chosen,
                                                                  reuse_router_decisions=route, cached_h0=h0)
            launch.chosen = chosen
            if side != main:
                launch.streams.append(side)
        if self.config.lambda_cons != 0.0:
            side = main if self.consistency_on_main else self._side_stream(h0.device, 1)
            if ready is None:
                self._share_macro_weights(model, side)
            if side != main:
                side.wait_event(ready) if ready is not None else side.wait_stream(main)
            early = (self.consistency_backward_early and ready is not None and side == main
                     and torch.is_grad_enabled() and h0.requires_grad)
            src = h0.detach().requires_grad_() if early else h0
            with (_aliases_installed(aliases, model.macro) if aliases is not None else
                  nullcontext() if side == main else main_stream_aliases(model.macro)), torch.cuda.stream(side):
                launch.cons = model.macro.consistency_loss(src, src, route.recipe_id)
            if early:
                # the step's backward runs on loss / grad_accum_steps
                torch.autograd.backward(launch.cons * (self.config.lambda_cons / self.config.grad_accum_steps))
                launch.cons = launch.cons.detach()
                dh0 = src.grad
                if dh0 is not None:
                    h0.register_hook(lambda g, dh0=dh0: g + dh0)
            if side != main:
                launch.streams.append(side)
        return launch

    def _share_macro_weights(self, model: RecursiveModel, side) -> None:
        mac = model.macro
        if (getattr(mac, "v", None) is not None and mac._fused_bounded()
                and hip_ops.macro_fused_supported(mac.v, mac.u)):
            # one bf16 copy of the operator tables per step, shared with the hot path
            hip_ops.macro_fused_weights_share(mac.v, mac.u, side)

    def prepare_late(self, model: RecursiveModel, h0, *, seed: int, chosen: torch.Tensor | None = None):
        """The main-stream work a late begin() (ready given) reads on its side streams, issued
        before the ready event is recorded: the fixed-count audited rows (returned; None when
        nothing is audited) and the operator's shared weight copies."""
        fixed = self.config.audit_fixed_count_per_batch
        if fixed is None or h0.device.type != "cuda":
            return chosen
        n = h0.shape[0]
        k = min(int(fixed), n)
        if k > 0 and chosen is None:
            chosen = self.fixed_count_index(n, k, seed, h0.device)
        if self.config.lambda_cons != 0.0 and not self.consistency_on_main:
            self._share_macro_weights(model, self._side_stream(h0.device, 1))
        return chosen

    def _fixed_count_sample(self, meta: ModelMeta, seed: int, chosen: torch.Tensor | None):
        """compute_audit_prob followed by the fixed-count branch of sample_mask_with_prob and the
        sampler's means, as one HIP launch.  Returns (mask, inclusion p, chosen, count, stats [5])."""
        r = meta.router
        R, D = r.recipe_logits.shape[-1], r.depth_logits.shape[-1]
        ids = meta.recipe_ids
        dev = ids.device
        if self.recipe_audit_ema is None or self.recipe_audit_ema.numel() != R:
            self.recipe_audit_ema = torch.zeros(R, dtype=torch.float32, device=dev)
        self.recipe_audit_ema = self.recipe_audit_ema.to(dev).float().contiguous()
        n = ids.numel()
        k = min(int(self.config.audit_fixed_count_per_batch), n)
        self.last_sample_mode, self.last_candidate_count, self.last_capped_fraction = "fixed_count", k, 0.0
        if k > 0 and chosen is None:
            chosen = self.fixed_count_index(n, k, seed, dev)
        if k == 0:
            chosen = None
        c = self.config
        _, incl, mask, st = hip_ops.audit_sample_fixed(
            r.router_entropy, ids, self.recipe_audit_ema, chosen, denom=float(R + D), p_min=c.audit_p_min,
            p_max=c.audit_p_max, alpha=c.audit_alpha, beta=c.audit_beta, gamma=c.audit_gamma,
            residual=self.recent_residual, coverage_min=c.coverage_min)
        return mask, incl, chosen, k, st

    @staticmethod
    def fixed_count_index(n: int, k: int, seed: int, device) -> torch.Tensor:
        """The fixed-count sampler's audited rows: the first k of a seeded permutation of n
        (rte/audit.py:102-115).  Depends only on (n, k, seed), so it can be drawn ahead of a
        captured step."""
        gen = torch.Generator(device=device)
        gen.manual_seed(seed)
        return torch.randperm(n, device=device, generator=gen)[:k]

    def sample_mask_with_prob(self, p: torch.Tensor, seed: int, chosen: torch.Tensor | None = None):
        """rte/audit.py:99-132.  Returns (mask, inclusion_p, chosen_index or None, count or None);
        the fixed-count sampler knows its count on the host, so it needs no device sync.
        `chosen` supplies the fixed-count sampler's rows drawn ahead of time."""
        fixed = self.config.audit_fixed_count_per_batch
        if fixed is not None:
            n = p.numel()
            k = min(int(fixed), n)
            mask = torch.zeros_like(p, dtype=torch.bool)
            self.last_sample_mode, self.last_candidate_count, self.last_capped_fraction = "fixed_count", k, 0.0
            if k > 0 and n > 0:
                if chosen is None:
                    chosen = self.fixed_count_index(n, k, seed, p.device)
                mask.index_fill_(0, chosen, True)
                incl = torch.full_like(p, float(k) / float(n))
            else:
                chosen = None
                incl = torch.zeros_like(p)
            return mask, incl, chosen, k
        if chosen is not None:
            raise ValueError("precomputed audit rows need the fixed-count sampler")
        gen = torch.Generator(device=p.device)
        gen.manual_seed(seed)
        self.last_sample_mode = "bernoulli"
        mask = torch.bernoulli(p, generator=gen).bool()
        incl = p.clone()
        self.last_candidate_count = int(mask.sum().item())
        self.last_capped_fraction = 0.0
        cap = self.config.audit_cap
        if cap is not None and self.last_candidate_count > cap:
            sel = mask.nonzero(as_tuple=False).flatten()
            perm = torch.randperm(sel.numel(), device=p.device, generator=gen)
            capped = torch.zeros_like(mask)
            capped[sel[perm[:cap]]] = True
            self.last_capped_fraction = float((sel.numel() - cap) / max(sel.numel(), 1))
            incl = p * (float(cap) / float(sel.numel()))
            mask = capped
        return mask, incl, None, None

    def correction(self, model: RecursiveModel, tokens, targets, hot: ModelOutput, *, seed: int,
                   chosen: torch.Tensor | None = None, launch: AuditLaunch | None = None) -> AuditResult:
        """rte/audit.py:245-387.  `chosen`: fixed-count audit rows drawn ahead (captured steps);
        `launch`: the replay / consistency work begin() already started on side streams."""
        if hot.loss_per_sample is None:
            raise ValueError("hot output must include per-sample losses")
        if launch is not None:
            main = torch.cuda.current_stream(hot.loss_per_sample.device)
            for st in launch.streams:
                main.wait_stream(st)
            if launch.chosen is not None:
                chosen = launch.chosen
            if launch.exact is None and launch.coda_extra is not None:
                launch.exact = launch.coda_extra.exact  # built by the hot path's coda call
            for t in _tensors_of(launch.exact) + ([launch.cons] if launch.cons is not None else []):
                t.record_stream(main)
        if self.config.audit_fixed_count_per_batch is None:
            self.flush_pending()  # the Bernoulli sampler's probability depends on the last residual
        fused = self.config.audit_fixed_count_per_batch is not None and hot.loss_per_sample.is_cuda
        if fused:
            # requested probability, fixed-count mask, inclusion probability and their means: one launch
            mask, p, chosen, count, st = self._fixed_count_sample(hot.meta, seed, chosen)
            metrics: dict[str, torch.Tensor] = {
                name: st[i] for i, name in enumerate(("audit_probability", "audit_requested_probability",
                                                      "audit_rate", "audit_count", "audit_inclusion_prob"))}
        else:
            req = self.compute_audit_prob(hot.meta)
            mask, p, chosen, count = self.sample_mask_with_prob(req, seed=seed, chosen=chosen)
            p_mean = p.mean()
            mask_f = mask.float()
            metrics = {
                "audit_probability": p_mean,
                "audit_requested_probability": req.mean(),
                "audit_rate": mask_f.mean(),
                "audit_count": mask_f.sum(),
                "audit_inclusion_prob": p_mean,
            }
        corrected = None
        zero = self._zero(hot.loss_per_sample)
        aux = {k: zero for k in ("hid", "cos", "kl", "norm", "cons", "delta_dir", "delta_rms", "endpoint_normed",
                                 "endpoint_raw", "rms_trust")}
        if count is not None:  # fixed-count sampler: rows and count known without reading the mask
            idx, has_audit = chosen, count > 0
        else:
            idx = mask.nonzero(as_tuple=False).flatten()
            has_audit = idx.numel() > 0
        exact = None
        if has_audit:
            grad_corr = self.config.audit_mode == "gradient_corrected"
            if launch is not None and launch.exact is not None:
                exact = launch.exact
            else:
                with (nullcontext() if grad_corr else torch.no_grad()):
                    exact = model.forward_exact_subset(tokens, targets, idx, reuse_router_decisions=hot.meta.router,
                                                       cached_h0=hot.meta.h0)
            hot_tok = hot.meta.token_loss
            exact_tok = exact.meta.token_loss
            if hot_tok is None or exact_tok is None:
                raise ValueError("audit correction needs the token losses of the hot pass and of the replay")
            # one kernel: per-sample sums, residual, clip, corrected rows and residual statistics
            corrected, _, st = hip_ops.audit_correct(
                hot_tok, exact_tok if grad_corr else exact_tok.detach(), idx, p,
                clip=self.config.audit_residual_clip, grad_corrected=grad_corr)
            metrics["audit_residual_mean"] = st[0]
            metrics["audit_residual_std"] = st[1]
            metrics["audit_residual_var"] = st[2]
            metrics["corrected_metric_loss"] = st[3]
            metrics["loss_residual"] = st[0]
            hot_end = hip_ops.select_rows(hot.meta.recurrent_hidden, idx)
            # the replay already selected these h0 rows (with their gradient path when it ran with
            # gradients): reuse them instead of a second full-size selection and its backward
            h0_sub = (exact.meta.h0 if grad_corr and exact.meta.h0 is not None and exact.meta.h0.requires_grad
                      else hip_ops.select_rows(hot.meta.h0, idx))
            src = hot.meta.logit_source if hot.meta.logit_source is not None else hot.meta.logits
            hot_logits = hip_ops.select_logit_rows(src, idx) if src is not None else None
            tr = self.config
            exact_end = exact.meta.recurrent_hidden
            if h0_sub is not None and exact_end is not None:
                # fused: every distillation term and alignment metric of rte/macro.py:394-546
                lam = {"delta_dir": tr.lambda_delta_dir, "delta_rms": tr.lambda_delta_rms,
                       "endpoint_normed": tr.lambda_endpoint_normed, "endpoint_raw": tr.lambda_endpoint_raw,
                       "rms_trust": tr.lambda_macro_rms_trust if tr.macro_rms_trust_region else 0.0,
                       "kl": tr.effective_lambda_kl}
                losses, mets = hip_ops.distill(hot_end, exact_end, h0_sub, hot_logits, exact.meta.logits,
                                               temperature=tr.distill_temperature,
                                               weights=[lam[n] for n in hip_ops.DISTILL_LOSSES])
                for name, v in zip(hip_ops.DISTILL_LOSSES, losses):
                    aux[name] = v
                align = {name: mets[i] for i, name in enumerate(hip_ops.DISTILL_METRICS)}
                has_logits = (hot_logits is not None and exact.meta.logits is not None
                              and hot_logits.shape == exact.meta.logits.shape)
                if not has_logits:
                    del align["logit_kl_exact_macro"]
            else:
                aux.update(macro_distill_loss(
                    hot_end, exact_end, hot_logits, exact.meta.logits, h0=h0_sub,
                    lambda_hid=tr.effective_lambda_hid, lambda_cos=tr.effective_lambda_cos,
                    lambda_kl=tr.effective_lambda_kl, lambda_norm=tr.lambda_norm,
                    lambda_delta_dir=tr.lambda_delta_dir, lambda_delta_rms=tr.lambda_delta_rms,
                    lambda_endpoint_normed=tr.lambda_endpoint_normed, lambda_endpoint_raw=tr.lambda_endpoint_raw,
                    lambda_macro_rms_trust=tr.lambda_macro_rms_trust if tr.macro_rms_trust_region else 0.0,
                    temperature=tr.distill_temperature,
                ))
                align = macro_alignment_metrics(hot_end.detach(), exact_end, h0=h0_sub,
                                                hot_logits=None if hot_logits is None else hot_logits.detach(),
                                                exact_logits=exact.meta.logits)
            metrics.update(align)
            # recent residual feeds the next step's audit probability; kept on device
            self._pending_residual = (1.0 - align["hidden_cosine_exact_macro"]).detach().clamp_min(0)
        if corrected is None:
            corrected = hot.loss_per_sample.clone()
        if hot.meta.recipe_ids is not None:
            if fused:
                hip_ops.count_ema(hot.meta.recipe_ids, mask, self.recipe_audit_ema, self.config.coverage_beta)
            else:
                self._update_coverage(hot.meta.recipe_ids, mask)
        if launch is not None and launch.cons is not None:
            aux["cons"] = self.config.lambda_cons * launch.cons
        elif self.config.lambda_cons != 0.0 and hot.meta.h0 is not None and hot.meta.recipe_ids is not None:
            aux["cons"] = self.config.lambda_cons * model.macro.consistency_loss(hot.meta.h0, hot.meta.h0,
                                                                                 hot.meta.recipe_ids)
        return AuditResult(mask, p, exact, corrected, aux, metrics)

    def flush_pending(self) -> None:
        """Materialise the residual used by compute_audit_prob (one host read, done off the timed path)."""
        pend = getattr(self, "_pending_residual", None)
        if pend is not None:
            self.recent_residual = float(pend.item())
            self._pending_residual = None


def _tensors_of(out: ModelOutput | None) -> list[torch.Tensor]:
    """Tensors of a replay's output that the main stream reads."""
    if out is None:
        return []
    ts = [out.loss_per_sample, out.meta.recurrent_hidden, out.meta.logits, out.meta.hidden]
    return [t for t in ts if isinstance(t, torch.Tensor)]
