"""AdamW on the HIP kernels, with the trainer's per-group norm metrics computed in the same pass.

FusedAdamW keeps torch.optim.AdamW's parameter groups, hyper-parameters and state layout
('step', 'exp_avg', 'exp_avg_sq' per parameter), so state dicts move between the two.  One
step is three launches whatever the parameter count: partial norms, a one-workgroup finish
(per-tensor and per-group sums in a fixed order, optional clipping coefficient, metrics, step
counters) and the update.  `found_inf` (a device scalar set by the caller, as for torch's
fused optimizers) skips the update and the counters without a host read.

Metric groups: the optimizer groups (by their "name") plus any extra named parameter sets
given at construction, each with the group whose learning rate scales its update ratio
(rte/training.py:385-443: grad_norm_<name>, update_ratio_<name>).
"""

from __future__ import annotations

import numpy as np
import torch

from rte_amd import _lib
from rte_amd._lib import call, ptr


class FusedAdamW(torch.optim.Optimizer):
    def __init__(self, params, lr: float = 1e-3, betas=(0.9, 0.999), eps: float = 1e-8, weight_decay: float = 1e-2,
                 *, extra_metrics: list[tuple[str, list[torch.nn.Parameter], str]] | None = None,
                 clip_grad_norm: float | None = None):
        if lr < 0 or eps < 0 or weight_decay < 0 or not (0 <= betas[0] < 1 and 0 <= betas[1] < 1):
            raise ValueError("FusedAdamW: invalid hyper-parameters")
        super().__init__(params, dict(lr=lr, betas=betas, eps=eps, weight_decay=weight_decay))
        self.extra_metrics = extra_metrics or []
        self.clip_grad_norm = clip_grad_norm
        self.found_inf: torch.Tensor | None = None
        self.metric_names: list[str] = []
        self.last_metrics: torch.Tensor | None = None
        self._layout = None
        self._host_keep: list[torch.Tensor] = []  # pinned tables referenced by captured graphs
        self._eager_host: torch.Tensor | None = None
        self._eager_event = None

    # ------------------------------------------------------------------ layout
    def _params(self):
        return [p for g in self.param_groups for p in g["params"]]

    def _init_state(self):
        for p in self._params():
            st = self.state[p]
            if len(st) == 0:
                st["step"] = torch.zeros((), dtype=torch.float32, device=p.device)
                st["exp_avg"] = torch.zeros_like(p, memory_format=torch.preserve_format)
                st["exp_avg_sq"] = torch.zeros_like(p, memory_format=torch.preserve_format)

    def _build_layout(self, device):
        params = self._params()
        for p in params:
            if p.dtype != torch.float32 or not p.is_contiguous():
                raise TypeError("FusedAdamW: parameters must be contiguous float32")
        chunk = _lib.load().rte_adamw_chunk()
        blocks, first = [], [0]
        for i, p in enumerate(params):
            n = (p.numel() + chunk - 1) // chunk
            blocks.extend((i, c) for c in range(n))
            first.append(len(blocks))
        names = [str(g.get("name", f"group{gi}")) for gi, g in enumerate(self.param_groups)]
        index = {id(p): i for i, p in enumerate(params)}
        masks = [0] * len(params)
        lr_group = []
        gi_of = {}
        for gi, g in enumerate(self.param_groups):
            gi_of[names[gi]] = gi
            for p in g["params"]:
                masks[index[id(p)]] |= 1 << gi
            lr_group.append(gi)
        metric_names = list(names)
        for j, (name, ps, lr_name) in enumerate(self.extra_metrics):
            bit = len(self.param_groups) + j
            for p in ps:
                if id(p) in index:
                    masks[index[id(p)]] |= 1 << bit
            lr_group.append(gi_of.get(lr_name, 0))
            metric_names.append(name)
        if len(metric_names) > 64:
            raise ValueError("FusedAdamW: at most 64 metric groups")
        group_of = [next(gi for gi, g in enumerate(self.param_groups) if any(q is p for q in g["params"]))
                    for p in params]
        i32 = dict(dtype=torch.int32, device=device)
        self._layout = dict(
            params=params, masks=masks, group_of=group_of,
            blocks=torch.tensor(blocks if blocks else [(0, 0)], **i32).reshape(-1),
            first=torch.tensor(first, **i32), nblk=len(blocks),
            lr_group=torch.tensor(lr_group, **i32),
            ws=torch.empty((max(_lib.load().rte_adamw_workspace_bytes(len(params), len(blocks),
                                                                       len(self.param_groups)) // 4, 1),),
                           dtype=torch.float32, device=device),
            rows=torch.empty((len(params), 8), dtype=torch.int64, device=device),
            hyper=torch.empty((len(self.param_groups), 5), dtype=torch.float64, device=device),
            metrics=torch.zeros((len(metric_names), 2), dtype=torch.float32, device=device),
        )
        self.metric_names = metric_names

    def _new_host_pair(self):
        lay = self._layout
        return (torch.empty(lay["rows"].shape, dtype=torch.int64, pin_memory=True),
                torch.empty(lay["hyper"].shape, dtype=torch.float64, pin_memory=True))

    def _host_tables(self):
        """Pinned host (rows, hyper) for this step.  A captured graph copies from the pair it was
        captured with on every replay, so it takes one of the pairs allocated ahead (pinned
        allocation is not capturable) and keeps it; eager steps reuse one pair after its
        previous copy has finished."""
        lay = self._layout
        if torch.cuda.is_current_stream_capturing():
            if not lay["spares"]:
                raise RuntimeError("FusedAdamW: no pinned table left for another captured graph")
            pair = lay["spares"].pop()
            self._host_keep.extend(pair)
            return pair
        if self._eager_event is not None:
            self._eager_event.synchronize()
        if self._eager_host is None or self._eager_host[0].shape != lay["rows"].shape:
            self._eager_host = self._new_host_pair()
        return self._eager_host

    def _static_rows(self, params):
        lay = self._layout
        rows = np.zeros((len(params), 8), dtype=np.int64)
        for i, p in enumerate(params):
            st = self.state[p]
            rows[i] = (p.data_ptr(), 0, st["exp_avg"].data_ptr(), st["exp_avg_sq"].data_ptr(),
                       st["step"].data_ptr(), p.numel(), lay["group_of"][i], lay["masks"][i])
        return rows

    # ------------------------------------------------------------------ step
    @torch.no_grad()
    def step(self, closure=None):
        loss = None
        if closure is not None:
            with torch.enable_grad():
                loss = closure()
        params = self._params()
        if not params:
            return loss
        dev = params[0].device
        _lib.require_device_tensors("FusedAdamW", *params)
        self._init_state()
        if self._layout is None or len(self._layout["params"]) != len(params) or any(
                a is not b for a, b in zip(self._layout["params"], params)):
            if torch.cuda.is_current_stream_capturing():
                raise RuntimeError("FusedAdamW: run one eager step before capturing a graph")
            self._build_layout(dev)
            self._layout["static_rows"] = self._static_rows(params)
            self._layout["spares"] = [self._new_host_pair() for _ in range(4)]
            self._layout["hyper_ring"] = [(torch.empty(self._layout["hyper"].shape, dtype=torch.float64,
                                                       pin_memory=True), None) for _ in range(4)]
            self._layout["ring_i"] = 0
        lay = self._layout
        nt = len(params)
        rows_h, _ = self._host_tables()
        rows = lay["static_rows"].copy()
        for i, p in enumerate(params):
            g = p.grad
            if g is not None and (g.dtype != torch.float32 or not g.is_contiguous()):
                g = g.float().contiguous()
                p.grad = g
            rows[i, 1] = 0 if g is None else g.data_ptr()
        rows_h.numpy()[:] = rows
        lay["rows"].copy_(rows_h, non_blocking=True)
        if not torch.cuda.is_current_stream_capturing():
            # a captured step reads the hyper-parameters the caller stages before each replay
            # (stage_hyper), so a learning-rate schedule reaches every replay
            self.stage_hyper()
            self._eager_event = torch.cuda.Event()
            self._eager_event.record()
        fi = self.found_inf
        fi = None if fi is None else fi.reshape(()).to(torch.float32)
        ws = lay["ws"]
        call("rte_adamw_step", ptr(lay["rows"]), nt, ptr(lay["blocks"]), ptr(lay["first"]), lay["nblk"],
             ptr(lay["hyper"]), len(self.param_groups), ptr(lay["lr_group"]), len(self.metric_names),
             float(self.clip_grad_norm or 0.0), ptr(fi), ptr(lay["metrics"]), ptr(ws), ws.numel() * 4,
             _lib.stream_ptr())
        self.last_metrics = lay["metrics"]
        return loss

    def stage_hyper(self) -> None:
        """Copy the groups' current (lr, betas, eps, weight_decay) to the device table the update
        kernel reads, on the current stream.  Eager steps call it themselves; before replaying a
        captured step, call it so the replay uses this step's learning rates.  The pinned
        sources rotate over a ring whose entries are reused only after their copy finished."""
        lay = self._layout
        if lay is None:
            return
        ring = lay["hyper_ring"]
        i = lay["ring_i"]
        buf, ev = ring[i]
        if ev is not None:
            ev.synchronize()
        buf.numpy()[:] = np.array([[g["lr"], g["betas"][0], g["betas"][1], g["eps"], g["weight_decay"]]
                                   for g in self.param_groups], dtype=np.float64)
        lay["hyper"].copy_(buf, non_blocking=True)
        ev = torch.cuda.Event()
        ev.record()
        ring[i] = (buf, ev)
        lay["ring_i"] = (i + 1) % len(ring)

    def load_state_dict(self, state_dict):
        super().load_state_dict(state_dict)
        # the update kernel dereferences every state tensor on the device: a state loaded from a
        # CPU map_location or from torch.optim.AdamW (CPU 'step') is moved next to its parameter
        for p in self._params():
            st = self.state.get(p)
            if not st:
                continue
            if "step" in st:
                st["step"] = torch.as_tensor(st["step"]).detach().to(device=p.device, dtype=torch.float32).reshape(())
                st["step"] = st["step"].clone()
            for key in ("exp_avg", "exp_avg_sq"):
                if key not in st:
                    raise ValueError(f"FusedAdamW: optimizer state lacks {key!r}")
                t = st[key]
                if t.shape != p.shape:
                    raise ValueError(f"FusedAdamW: state {key!r} has shape {tuple(t.shape)}, parameter {tuple(p.shape)}")
                st[key] = t.detach().to(device=p.device, dtype=torch.float32).contiguous()
        self._layout = None  # state tensors were replaced: rebuild the pointer tables

    def metrics_dict(self) -> dict[str, torch.Tensor]:
        """grad_norm_<name> / update_ratio_<name> of the last step (device scalars)."""
        if self.last_metrics is None:
            return {}
        out = {}
        for j, name in enumerate(self.metric_names):
            out[f"grad_norm_{name}"] = self.last_metrics[j, 0]
            out[f"update_ratio_{name}"] = self.last_metrics[j, 1]
        return out
