"""Training engine for the accelerated modes (rte/training.py:42-1701 restated for
dense_exact, recursive_exact, recursive_macro and recursive_macro_shortlist).

The step keeps the reference's loss composition (corrected CE / seq_len + macro aux +
router aux, rte/training.py:1381-1385), bf16 autocast for torch glue, fused AdamW with
the reference's parameter groups, non-finite skip, grad accumulation and clipping.
Differences that only change where numbers live: metrics stay on the device until
`metrics_to_host` (one copy instead of one sync per value), and gradient/param norms use
torch._foreach_norm.
"""

from __future__ import annotations

import dataclasses
import time
from contextlib import nullcontext
from dataclasses import dataclass
from typing import Any

import torch

from rte_amd.audit import AuditEngine, AuditResult, GradSink, make_main_aliases
from rte_amd.config import ExperimentConfig, TrainingConfig
from rte_amd.kernels import hip_ops, optimized
from rte_amd.metrics import hot_budget
from rte_amd.models import DenseModel, ModelOutput, RecursiveModel
from rte_amd.optim import FusedAdamW

ACCELERATED_MODES = {"dense_exact", "recursive_exact", "recursive_macro", "recursive_macro_shortlist"}


def set_seed(seed: int) -> None:
    import random

    import numpy as np

    random.seed(seed)
    np.random.seed(seed % (2**32))
    torch.manual_seed(seed)


def router_aux_losses(recipe_probs, expected_depth, usage_ema, tr: TrainingConfig) -> dict[str, torch.Tensor]:
    """rte/metrics.py:97-112 in torch ops (the training step runs the same formula as one HIP
    launch, hip_ops.router_aux)."""
    r = recipe_probs.shape[-1]
    mean_prob = recipe_probs.float().mean(dim=0)
    load = r * mean_prob.square().sum() - 1.0
    cover = torch.relu(tr.coverage_min - usage_ema.to(recipe_probs.device)).square().sum()
    return {
        "load": tr.lambda_load * load,
        "cover": tr.lambda_cover * cover,
        "depth": tr.lambda_depth * expected_depth.float().mean(),
    }


def _detached(obj, memo: dict | None = None):
    """obj with every tensor detached: dataclasses rebuilt field by field, containers copied,
    router subsets re-rooted, anything else (modules, numbers) kept.  A step's returned outputs
    then keep no autograd graph alive into the next step, whose leaves' gradient accumulators
    would otherwise still belong to the old graph and its streams."""
    from rte_amd.routing import RouterSubset

    memo = {} if memo is None else memo
    key = id(obj)
    if key in memo:
        return memo[key]
    if isinstance(obj, torch.Tensor):
        out = obj.detach()
    elif isinstance(obj, dict):
        out = {k: _detached(v, memo) for k, v in obj.items()}
    elif isinstance(obj, (list, tuple)):
        out = type(obj)(_detached(v, memo) for v in obj)
    elif isinstance(obj, RouterSubset):
        out = RouterSubset(_detached(obj._parent, memo), obj._mask)
    elif isinstance(obj, ModelOutput):
        out = ModelOutput(_detached(obj._loss, memo), _detached(obj.loss_per_sample, memo),
                          _detached(obj.logits, memo), _detached(obj.meta, memo),
                          mean_of=_detached(obj._mean_of, memo))
    elif dataclasses.is_dataclass(obj) and not isinstance(obj, type):
        out = dataclasses.replace(obj, **{f.name: _detached(getattr(obj, f.name), memo)
                                          for f in dataclasses.fields(obj) if f.init})
    else:
        out = obj
    memo[key] = out
    return out


@dataclass
class TrainStepResult:
    loss: torch.Tensor
    model_output: ModelOutput
    metrics: dict[str, Any]
    audit: AuditResult | None = None


class TrainEngine:
    def __init__(self, config: ExperimentConfig, *, device: torch.device | None = None,
                 dense_model: DenseModel | None = None, recursive_model: RecursiveModel | None = None):
        self.config = config
        tr = config.training
        if tr.mode not in ACCELERATED_MODES:
            raise NotImplementedError(f"mode {tr.mode!r} is outside the accelerated path ({sorted(ACCELERATED_MODES)})")
        if tr.precision not in ("bf16", "fp32"):
            raise ValueError(f"precision={tr.precision!r}: expected 'fp32' or 'bf16'")
        self.device = device or torch.device("cuda")
        set_seed(tr.seed)
        if tr.strict_cuda and self.device.type != "cuda":
            raise RuntimeError("strict_cuda requires a ROCm device")
        optimized.set_strict_cuda(tr.strict_cuda, require_flash=tr.require_flash_attention)
        if tr.allow_tf32:
            torch.backends.cuda.matmul.allow_tf32 = True
        self.dense_model = dense_model
        self.recursive_model = recursive_model
        if self.dense_model is None and config.model.topology == "dense":
            self.dense_model = DenseModel(config.model)
        if self.recursive_model is None and config.model.topology == "recursive":
            self.recursive_model = RecursiveModel(config.model, config.output)
        for m in (self.dense_model, self.recursive_model):
            if m is not None:
                m.to(self.device)
        self.optimizer = self._build_optimizer(self._param_groups())
        self.optimizer.zero_grad(set_to_none=True)
        self.audit_engine = AuditEngine(tr)
        self.global_step = 0
        self.global_micro_step = 0
        self.tokens_seen = 0
        self.last_grad_metrics: dict[str, Any] = {}
        self.aligned_lm_phase = "A"  # the lm_aligned mode's phase (rte/training.py:128); kept for checkpoints
        self._current_lr = tr.lr
        # start the audit replay and the consistency loss right after routing, on side streams;
        # graph_side_streams False: captured steps issue them in order on the step's stream (a
        # graph with parallel branches is launched node by node from the host, a one-stream graph
        # from its recorded packets, but only branches overlap on the device)
        self.audit_streams = self.device.type == "cuda"
        self.graph_side_streams = True
        # the replay's coda and head run in the hot path's coda call (its rows appended; the
        # full-vocabulary head only): one set of launches for both.  Not in captured steps with
        # side streams: there the replay's own coda overlaps the hot path instead.
        self.replay_coda_shared = True
        # with side streams and the replay's own coda: issue the replay and the consistency loss
        # after the hot path's forward (their streams still wait only for the routing point), so
        # their autograd nodes are newer than the hot path's and the backward issues their work
        # first, beside the hot path's backward rather than after it
        self.side_launch_late = True
        # late side work: its parameter gradients are added in one multi-tensor launch after the
        # backward instead of one add per parameter where the streams join
        self.side_grad_sink = True
        self._grad_sink = None
        self._capturing = False
        self._bf16 = hip_ops.Bf16Prefetch(enabled=self.device.type == "cuda" and tr.precision == "bf16")
        self._graph_enabled = False
        self._graph_keep = False
        self._gstate: dict[str, Any] | None = None
        # captured steps' "stepped" flags not yet read back (see reconcile_global_step)
        self._stepped_pending: list[torch.Tensor] = []

    # ------------------------------------------------------------------ optimizer
    def _param_groups(self) -> list[dict[str, Any]]:
        tr = self.config.training
        if self.dense_model is not None:
            return [{"params": list(self.dense_model.parameters()), "lr": tr.effective_lr_base,
                     "base_lr": tr.effective_lr_base, "name": "dense"}]
        m = self.recursive_model
        seen: set[int] = set()
        specs = [
            ("embedding", tr.effective_lr_base, list(m.embed.parameters())),
            ("prelude", tr.effective_lr_base, list(m.prelude.parameters())),
            ("core", tr.effective_lr_base, list(m.core.parameters())),
            ("macro", tr.effective_lr_macro, list(m.macro.parameters())),
            ("coda", tr.effective_lr_coda, [*m.coda.parameters(), *m.final_norm.parameters()]),
            ("output", tr.effective_lr_output,
             [*(m.lm_head.parameters() if m.lm_head is not None else []), *m.shortlist_head.parameters()]),
            ("router", tr.effective_lr_router, list(m.router.parameters())),
        ]
        groups = []
        for name, lr, params in specs:
            uniq = [p for p in params if id(p) not in seen and not seen.add(id(p))]
            if uniq:
                groups.append({"params": uniq, "lr": lr, "base_lr": lr, "name": name})
        return groups

    def _build_optimizer(self, groups):
        tr = self.config.training
        if self.device.type == "cuda" and tr.fused_optimizer:
            # HIP AdamW: clipping, update and the per-group norm metrics in three launches
            extra = []
            if self.recursive_model is not None:
                core = self.recursive_model.core
                extra = [("pass_film", [core.pass_gamma1, core.pass_beta1, core.pass_gamma2, core.pass_beta2], "core"),
                         ("pass_scale", [core.pass_attn_scale, core.pass_mlp_scale], "core")]
            return FusedAdamW(groups, weight_decay=tr.weight_decay, extra_metrics=extra,
                              clip_grad_norm=tr.grad_clip_norm)
        kw: dict[str, Any] = {"weight_decay": tr.weight_decay}
        if tr.foreach_optimizer:
            kw["foreach"] = True
        return torch.optim.AdamW(groups, **kw)

    def _autocast(self):
        """rte/training.py:356-363: bf16 autocast for precision bf16; for precision fp32 (the
        reference default) every operator computes with fp32 operands (hip_ops.fp32_precision)."""
        if self.config.training.precision != "bf16":
            return hip_ops.fp32_precision() if self.device.type == "cuda" else nullcontext()
        return torch.autocast(device_type=self.device.type, dtype=torch.bfloat16)

    def _lr_scale(self) -> float:
        """rte/training.py:470-484: constant, or linear from 1 to lr_final_scale between
        lr_decay_start_tokens and lr_decay_end_tokens of tokens seen."""
        tr = self.config.training
        if tr.lr_schedule == "constant":
            return 1.0
        if tr.lr_schedule == "linear_decay_after":
            if self.tokens_seen <= tr.lr_decay_start_tokens:
                return 1.0
            if self.tokens_seen >= tr.lr_decay_end_tokens:
                return tr.lr_final_scale
            progress = (self.tokens_seen - tr.lr_decay_start_tokens) / (
                tr.lr_decay_end_tokens - tr.lr_decay_start_tokens)
            return 1.0 + progress * (tr.lr_final_scale - 1.0)
        raise ValueError(tr.lr_schedule)

    def _apply_lr_schedule(self) -> float:
        """Scale every group's base learning rate (rte/training.py:486-490); returns the scaled
        global lr.  Runs at the start of every step, before the optimizer reads the rates."""
        scale = self._lr_scale()
        for group in self.optimizer.param_groups:
            group["lr"] = float(group.get("base_lr", self.config.training.lr)) * scale
        return self.config.training.lr * scale

    def _hot_budget(self, shortlist: bool) -> dict[str, Any]:
        """Refuse a step whose hot path exceeds the configured budget (rte/training.py:707-740,
        applied at :1389-1392); host arithmetic on the config only."""
        size = self.config.output.shortlist_max_tokens if shortlist else None
        return hot_budget(self.config.model, self.config.training, shortlist_size=size, include_output=True)

    def _loss_scale(self, targets) -> float:
        return float(targets.shape[1]) if self.config.training.loss_normalization == "token_mean" else 1.0

    # ------------------------------------------------------------------ step
    def _grad_metrics(self) -> dict[str, torch.Tensor]:
        out: dict[str, torch.Tensor] = {}
        for g in self.optimizer.param_groups:
            name = str(g.get("name", "group"))
            params = [p for p in g["params"]]
            grads = [p.grad for p in params if p.grad is not None]
            pn = torch.linalg.vector_norm(torch.stack(torch._foreach_norm([p.detach().float() for p in params])))
            gn = (torch.linalg.vector_norm(torch.stack(torch._foreach_norm([x.float() for x in grads])))
                  if grads else pn.new_zeros(()))
            out[f"grad_norm_{name}"] = gn
            out[f"update_ratio_{name}"] = float(g["lr"]) * gn / pn.clamp_min(1e-12)
        return out

    def _finish_step(self, loss: torch.Tensor, *, check_finite: bool = True) -> bool:
        """rte/training.py:445-468.  The finiteness check reads one scalar from the device."""
        tr = self.config.training
        self.last_grad_metrics = {}
        if check_finite and not bool(torch.isfinite(loss.detach()).item()):
            self._grad_sink = None
            self.optimizer.zero_grad(set_to_none=True)
            self.global_micro_step += 1
            self.last_grad_metrics = {"skipped_nonfinite_loss": 1.0}
            return False
        (loss / tr.grad_accum_steps).backward()
        self._flush_grad_sink()
        self.global_micro_step += 1
        step = self.global_micro_step % tr.grad_accum_steps == 0
        fused = isinstance(self.optimizer, FusedAdamW)
        if step and tr.grad_clip_norm is not None and not fused:
            params = [p for g in self.optimizer.param_groups for p in g["params"]]
            torch.nn.utils.clip_grad_norm_(params, tr.grad_clip_norm, foreach=True)
        self._bf16.end()  # parameters change below
        if step:
            if fused:  # clipping and metrics happen inside the fused step
                self.optimizer.step()
                self.last_grad_metrics = self.optimizer.metrics_dict()
            else:
                self.last_grad_metrics = self._grad_metrics()
                self.optimizer.step()
            self.optimizer.zero_grad(set_to_none=True)
            self.global_step += 1
        return step

    def _flush_grad_sink(self) -> None:
        """Add the side work's parameter gradients (kept by the step's GradSink) to .grad."""
        sink, self._grad_sink = self._grad_sink, None
        if sink is not None:
            sink.flush()

    def _move(self, batch):
        return batch[0].to(self.device, non_blocking=True), batch[1].to(self.device, non_blocking=True)

    def train_step(self, batch, *, check_finite: bool = True) -> TrainStepResult:
        mode = self.config.training.mode
        self._current_lr = self._apply_lr_schedule()
        if not (self._graph_enabled and mode in ("recursive_macro", "recursive_macro_shortlist")):
            self._bf16.begin()  # one bf16 copy per weight per step (the captured body opens its own)
        if mode == "dense_exact":
            return self._step_dense(batch, check_finite)
        if mode == "recursive_exact":
            return self._step_recursive_exact(batch, check_finite)
        return self._step_macro(batch, shortlist=mode == "recursive_macro_shortlist", check_finite=check_finite)

    def _step_dense(self, batch, check_finite):
        tokens, targets = self._move(batch)
        t0 = time.perf_counter()
        with self._autocast():
            out = self.dense_model(tokens, targets, return_loss_per_sample=True)
        loss = out.loss_per_sample.mean() / self._loss_scale(targets)
        stepped = self._finish_step(loss, check_finite=check_finite)
        self.tokens_seen += tokens.numel()
        loss = loss.detach()
        return TrainStepResult(loss, _detached(out), {"mode": "dense_exact", "loss": loss, "stepped": stepped,
                                                      "lr": self._current_lr, "host_time": time.perf_counter() - t0,
                                                      **self.last_grad_metrics})

    def _step_recursive_exact(self, batch, check_finite):
        tr = self.config.training
        tokens, targets = self._move(batch)
        m = self.recursive_model
        with self._autocast():
            out = m.forward_exact(tokens, targets, return_loss_per_sample=True, fixed_recipe=tr.fixed_recipe,
                                  fixed_depth=tr.fixed_depth)
            aux = self._router_aux(out)
        loss = out.loss_per_sample.mean() / self._loss_scale(targets) + sum(aux.values())
        stepped = self._finish_step(loss, check_finite=check_finite)
        m.recipe_bank.update_usage(out.meta.recipe_ids, beta=tr.coverage_beta)
        self.tokens_seen += tokens.numel()
        loss = loss.detach()
        return TrainStepResult(loss, _detached(out), {"mode": "recursive_exact", "loss": loss, "stepped": stepped,
                                                      "lr": self._current_lr, **self.last_grad_metrics})

    def _router_aux(self, out: ModelOutput) -> dict[str, torch.Tensor]:
        r = out.meta.router
        if self.config.training.disable_router_aux:
            z = r.recipe_probs.new_zeros(())
            return {"load": z, "cover": z, "depth": z}
        tr = self.config.training
        return hip_ops.router_aux(r.recipe_probs, r.expected_depth, self.recursive_model.recipe_bank.usage_ema,
                                  coverage_min=tr.coverage_min, lambda_load=tr.lambda_load,
                                  lambda_cover=tr.lambda_cover, lambda_depth=tr.lambda_depth)

    def _macro_loss(self, tokens, targets, *, shortlist: bool, chosen=None, random_negs=None):
        """Forward of the recursive_macro step (rte/training.py:1336-1385): hot path, audit
        correction, router aux; loss = corrected CE / S + macro aux + router aux.  Side work
        issued late keeps its parameter gradients in the step's GradSink: callers running the
        backward themselves call _flush_grad_sink() after it."""
        tr = self.config.training
        m = self.recursive_model
        launched = []
        audit_seed = tr.seed + 10_000 + self.global_step

        late = []

        def on_routed(h0, route):
            # the audit replay and the consistency loss need only h0 and the routing decisions
            share = self.replay_coda_shared and not shortlist and not (self._capturing and self.graph_side_streams)
            if self.side_launch_late and not share:
                rows = self.audit_engine.prepare_late(m, h0, seed=audit_seed, chosen=chosen)
                ready = torch.cuda.Event()
                ready.record(torch.cuda.current_stream(h0.device))
                sink = self._grad_sink = GradSink() if self.side_grad_sink else None
                late.append((h0, route, ready, make_main_aliases(m, sink=sink), rows))
                return
            launched.append(self.audit_engine.begin(m, tokens, targets, h0, route, seed=audit_seed, chosen=chosen,
                                                    defer_coda=share))

        def coda_extra():
            return launched[0].coda_extra if launched and launched[0] is not None else None

        with self._autocast():
            hot = m.forward_macro(tokens, targets, return_states=True, return_loss_per_sample=True,
                                  shortlist=shortlist, seed=tr.seed + self.global_step, fixed_recipe=tr.fixed_recipe,
                                  fixed_depth=tr.fixed_depth, shortlist_random_negs=random_negs,
                                  on_routed=on_routed if self.audit_streams else None, coda_extra=coda_extra)
            for h0, route, ready, aliases, rows in late:
                launched.append(self.audit_engine.begin(m, tokens, targets, h0, route, seed=audit_seed, chosen=rows,
                                                        ready=ready, aliases=aliases))
            audit = self.audit_engine.correction(m, tokens, targets, hot, seed=audit_seed, chosen=chosen,
                                                 launch=launched[0] if launched else None)
            aux = self._router_aux(hot)
            scale = self._loss_scale(targets)
            # corrected CE / S + every auxiliary term: one launch (a stacked sum for CPU tensors)
            corr = audit.corrected_loss_per_sample
            dev = corr.device
            extra = [(t if isinstance(t, torch.Tensor) else torch.tensor(float(t), device=dev)).reshape(()).float()
                     for t in (*audit.macro_aux.values(), *aux.values())]
            if corr.is_cuda:
                loss = hip_ops.loss_sum(corr, 1.0 / (corr.numel() * scale), extra)
            else:
                loss = torch.stack([corr.mean() / scale, *extra]).sum()
        return loss, hot, audit, aux, scale

    def _macro_metrics(self, loss, hot, audit, aux, scale, targets, shortlist, stepped):
        """rte/training.py:1412-1472 metric keys."""
        m = hip_ops.step_metrics(hot.loss_per_sample, audit.corrected_loss_per_sample, hot.meta.depths, scale=scale,
                                 seq=float(targets.shape[1]))
        return {
            "mode": "recursive_macro_shortlist" if shortlist else "recursive_macro",
            "loss": loss.detach(),
            "hot_lm_loss": m[0],
            "corrected_lm_loss": m[1],
            "nll_per_token": m[2],
            "avg_depth": m[3],
            "stepped": stepped,
            **{f"audit_{k}": v for k, v in audit.metrics.items()},
            **{f"macro_{k}": v.detach() for k, v in audit.macro_aux.items()},
            **{f"aux_{k}": v.detach() for k, v in aux.items()},
            **self.last_grad_metrics,
        }

    def _step_macro(self, batch, *, shortlist: bool, check_finite: bool):
        """rte/training.py:1336-1476."""
        tr = self.config.training
        m = self.recursive_model
        if shortlist and tr.debug_force_full_output:
            raise RuntimeError("debug_force_full_output forbids recursive_macro_shortlist")
        budget = self._hot_budget(shortlist)
        if self._graph_enabled:
            res = self._graph_macro_step(batch, shortlist, check_finite)
            res.metrics.update(budget, lr=self._current_lr)
            return res
        tokens, targets = self._move(batch)
        loss, hot, audit, aux, scale = self._macro_loss(tokens, targets, shortlist=shortlist)
        stepped = self._finish_step(loss, check_finite=check_finite)
        m.recipe_bank.update_usage(hot.meta.recipe_ids, beta=tr.coverage_beta)
        self.tokens_seen += tokens.numel()
        metrics = self._macro_metrics(loss, hot, audit, aux, scale, targets, shortlist, stepped)
        metrics.update(budget, lr=self._current_lr)
        memo: dict = {}
        return TrainStepResult(loss.detach(), _detached(hot, memo), metrics, _detached(audit, memo))

    # ------------------------------------------------------------------ captured step
    def enable_graph_capture(self, enabled: bool = True, *, keep_graph: bool = False) -> None:
        """Run recursive_macro(_shortlist) steps as one captured HIP graph: forward, audit
        replay, backward, gradient metrics and the fused AdamW update, replayed with one launch.

        The first two steps run eagerly (on a side stream, through the same static input
        buffers) to settle allocations and library state; the third is captured and every
        later step replays the graph.  The step's randomness (the fixed-count audit rows and
        the shortlist's random negatives) is drawn eagerly before each replay from the same
        seeds as the eager step.  The non-finite-loss skip becomes a device-side flag that
        the fused AdamW reads (found_inf): the update and its step count are skipped, and
        ``metrics["stepped"]`` is a device bool.  Tensors inside the returned model output and
        audit result are the graph's static buffers, overwritten by the next step; the loss
        and metrics are copied out.  keep_graph keeps the captured graph's nodes inspectable
        (``torch.cuda.CUDAGraph(keep_graph=True)``)."""
        tr = self.config.training
        if enabled:
            if tr.mode not in ("recursive_macro", "recursive_macro_shortlist"):
                raise ValueError("graph capture covers the recursive_macro modes")
            if tr.grad_accum_steps != 1:
                raise ValueError("graph capture needs grad_accum_steps == 1")
            if self.audit_engine.config.audit_fixed_count_per_batch is None:
                raise ValueError("graph capture needs the fixed-count audit sampler (its count is known on the host)")
            if self.device.type != "cuda" or not isinstance(self.optimizer, (FusedAdamW, torch.optim.AdamW)):
                raise ValueError("graph capture needs a ROCm device and AdamW")
            if not isinstance(self.optimizer, FusedAdamW):
                if tr.lr_schedule != "constant":
                    raise ValueError("graph capture with torch AdamW bakes the learning rate into the graph: "
                                     "use the fused optimizer for a learning-rate schedule")
                for g in self.optimizer.param_groups:
                    g["capturable"] = True
        self._graph_enabled = enabled
        self._graph_keep = keep_graph
        self._gstate = None

    def _graph_macro_step(self, batch, shortlist: bool, check_finite: bool):
        tr = self.config.training
        m = self.recursive_model
        tokens, targets = self._move(batch)
        key = (tuple(tokens.shape), tuple(targets.shape), shortlist, check_finite)
        st = self._gstate
        if st is None or st["key"] != key:
            B, S = targets.shape
            k = min(int(self.audit_engine.config.audit_fixed_count_per_batch), B)
            st = self._gstate = {
                "key": key, "graph": None, "warm": 0, "out": None,
                "tokens": torch.empty_like(tokens), "targets": torch.empty_like(targets),
                "chosen": torch.zeros((k,), dtype=torch.long, device=self.device),
                "rnd": (torch.zeros((B, S, self.config.output.random_negatives), dtype=torch.long, device=self.device)
                        if shortlist else None),
            }
        st["tokens"].copy_(tokens)
        st["targets"].copy_(targets)
        B, S = targets.shape
        if st["chosen"].numel():
            st["chosen"].copy_(self.audit_engine.fixed_count_index(B, st["chosen"].numel(),
                                                                   tr.seed + 10_000 + self.global_step, self.device))
        if shortlist:
            st["rnd"].copy_(m.shortlist_head.random_negatives(B, S, tr.seed + self.global_step, self.device))
        if st["graph"] is None and st["warm"] < 2:
            side = torch.cuda.Stream()
            side.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(side):
                out = self._graph_body(st, shortlist, check_finite)
            torch.cuda.current_stream().wait_stream(side)
            st["warm"] += 1
        else:
            if st["graph"] is None:
                self.optimizer.zero_grad(set_to_none=True)
                graph = torch.cuda.CUDAGraph(keep_graph=self._graph_keep)
                with torch.cuda.graph(graph):
                    st["out"] = self._graph_body(st, shortlist, check_finite)
                st["graph"] = graph
            if isinstance(self.optimizer, FusedAdamW):
                self.optimizer.stage_hyper()  # this step's learning rates, read by the replay
            st["graph"].replay()
            out = st["out"]
        self.global_micro_step += 1
        # Counted on the host without reading the device: reading whether the update was skipped
        # (a non-finite loss) would synchronise every captured step.  The device flag is kept and
        # reconcile_global_step() takes the skipped replays off the count (checkpoints call it, so
        # a saved global_step counts applied updates as the reference's _finish_step does); until
        # then the seeds of the following steps use the attempted-step count.
        self.global_step += 1
        self.tokens_seen += tokens.numel()
        flat = out["flat"].clone()
        metrics = dict(out["host_metrics"])
        metrics.update({name: flat[i] for i, name in enumerate(out["names"])})
        metrics["stepped"] = metrics["stepped"] > 0.5
        self._stepped_pending.append(metrics["stepped"])
        if len(self._stepped_pending) >= 1024:
            self.reconcile_global_step()
        self.last_grad_metrics = {k: metrics[k] for k in out["grad_names"]}
        return TrainStepResult(flat[out["names"].index("loss")], out["hot"], metrics, out["audit"])

    def _graph_body(self, st, shortlist: bool, check_finite: bool):
        """Device work of one captured step; everything here is replayed as recorded."""
        self._bf16.begin()
        tr = self.config.training
        m = self.recursive_model
        side, self.audit_engine.side_streams = self.audit_engine.side_streams, self.graph_side_streams
        self._capturing = True
        try:
            loss, hot, audit, aux, scale = self._macro_loss(st["tokens"], st["targets"], shortlist=shortlist,
                                                            chosen=st["chosen"] if st["chosen"].numel() else None,
                                                            random_negs=st["rnd"])
        finally:
            self.audit_engine.side_streams = side
            self._capturing = False
        if check_finite:  # skip flag and "stepped" metric in one launch, no host read
            bad, ok = hip_ops.nonfinite_flags(loss)
        else:
            bad, ok = torch.zeros((), device=loss.device), torch.ones((), device=loss.device)
        loss.backward()
        self._flush_grad_sink()
        self._bf16.end()  # parameters change below
        if isinstance(self.optimizer, FusedAdamW):
            # clipping, update (skipped on a non-finite loss) and metrics in three launches
            self.optimizer.found_inf = bad
            try:
                self.optimizer.step()
            finally:
                self.optimizer.found_inf = None
            self.last_grad_metrics = self.optimizer.metrics_dict()
        else:
            if tr.grad_clip_norm is not None:
                params = [p for g in self.optimizer.param_groups for p in g["params"]]
                torch.nn.utils.clip_grad_norm_(params, tr.grad_clip_norm, foreach=True)
            self.last_grad_metrics = self._grad_metrics()
            self.optimizer.found_inf = bad
            self.optimizer.grad_scale = None
            try:
                self.optimizer.step()
            finally:
                del self.optimizer.found_inf
                del self.optimizer.grad_scale
        self.optimizer.zero_grad(set_to_none=True)
        m.recipe_bank.update_usage(hot.meta.recipe_ids, beta=tr.coverage_beta)
        metrics = self._macro_metrics(loss, hot, audit, aux, scale, st["targets"], shortlist, ok)
        names = [k for k, v in metrics.items() if isinstance(v, torch.Tensor)]
        flat = torch.stack([metrics[k].detach().float().reshape(()) for k in names])
        memo: dict = {}
        return {"flat": flat, "names": names, "hot": _detached(hot, memo), "audit": _detached(audit, memo),
                "host_metrics": {k: v for k, v in metrics.items() if not isinstance(v, torch.Tensor)},
                "grad_names": list(self.last_grad_metrics)}

    def reconcile_global_step(self) -> int:
        """Take the captured replays whose update was skipped (their "stepped" flag False) off
        global_step, with one device read for every flag since the last call; returns the count
        of applied updates (rte/training.py:445-468 counts only those)."""
        if self._stepped_pending:
            flags = torch.stack([f.reshape(()) for f in self._stepped_pending]).cpu()
            self._stepped_pending.clear()
            self.global_step -= int((~flags).sum())
        return self.global_step

    # ------------------------------------------------------------------ checkpoint
    def save_checkpoint(self, path, *, data_cursor: int | None = None) -> None:
        """The payload of rte/training.py:1656-1676 (same keys).  The config is stored as a plain
        dict, so checkpoints written here load with torch.load(weights_only=True)."""
        from pathlib import Path

        self.reconcile_global_step()
        from rte_amd.config import config_to_dict

        model = self.dense_model if self.dense_model is not None else self.recursive_model
        payload = {
            "config": config_to_dict(self.config),
            "model": model.state_dict() if model is not None else None,
            "optimizer": self.optimizer.state_dict(),
            "global_step": self.global_step,
            "global_micro_step": self.global_micro_step,
            "tokens_seen": self.tokens_seen,
            "audit": self.audit_engine.state_dict(),
            "aligned_lm_phase": self.aligned_lm_phase,
            "data_cursor": data_cursor,
            "torch_rng_state": torch.get_rng_state(),
        }
        if torch.cuda.is_available():
            payload["cuda_rng_state_all"] = torch.cuda.get_rng_state_all()
        p = Path(path)
        p.parent.mkdir(parents=True, exist_ok=True)
        torch.save(payload, p)

    def load_checkpoint(self, path, *, trusted: bool = False) -> int | None:
        """Restore a payload with the keys of rte/training.py:1678-1701 (every key optional, as
        there); returns its data_cursor.  By default the file is read with
        torch.load(weights_only=True); a reference checkpoint, whose config is a pickled
        dataclass, needs trusted=True (full unpickling: only for files you trust)."""
        payload = torch.load(path, map_location=self.device, weights_only=not trusted)
        model = self.dense_model if self.dense_model is not None else self.recursive_model
        if model is not None and payload.get("model") is not None:
            model.load_state_dict(payload["model"])
        if payload.get("optimizer") is not None:
            try:
                self.optimizer.load_state_dict(payload["optimizer"])
            except ValueError:
                # a checkpoint of another parameter grouping: weights load, the optimizer starts fresh
                pass
        self._stepped_pending.clear()
        self.global_step = int(payload.get("global_step", 0))
        self.global_micro_step = int(payload.get("global_micro_step", 0))
        self.tokens_seen = int(payload.get("tokens_seen", 0))
        self.audit_engine.load_state_dict(payload.get("audit", {}))
        self.aligned_lm_phase = str(payload.get("aligned_lm_phase", self.aligned_lm_phase))
        if "torch_rng_state" in payload:
            torch.set_rng_state(payload["torch_rng_state"].detach().cpu())
        if torch.cuda.is_available() and "cuda_rng_state_all" in payload:
            torch.cuda.set_rng_state_all([t.detach().cpu().to(torch.uint8) for t in payload["cuda_rng_state_all"]])
        self._gstate = None  # a captured step holds the old state's buffers
        return payload.get("data_cursor")


def metrics_to_host(metrics: dict[str, Any]) -> dict[str, Any]:
    """Copy every tensor metric to the host in one transfer."""
    tens = {k: v for k, v in metrics.items() if isinstance(v, torch.Tensor)}
    host = optimized.k_metrics_reduce(tens)
    return {**{k: v for k, v in metrics.items() if not isinstance(v, torch.Tensor)}, **host}
