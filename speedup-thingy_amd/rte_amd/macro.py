"""Macro operators Phi_{recipe, depth}: a per-sample low-rank update that stands in for
`depth` exact recursive passes (rte/macro.py:42-391), plus the distillation losses and
alignment metrics the audit uses (rte/macro.py:394-546).

Parameter shapes and initialisation order follow the reference so state dicts load.
The bounded operator's (recipe, stride)-indexed matrices run as grouped MFMA GEMMs over
the rows of all samples sharing a key; the elementwise parts are torch on the device.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch
import torch.nn.functional as F
from torch import nn

from rte_amd.config import ModelConfig
from rte_amd.gather import gather_rows
from rte_amd.kernels import hip_ops


def _rms(x, *, dim=-1, keepdim=False):
    return x.float().pow(2).mean(dim=dim, keepdim=keepdim).sqrt().to(x.dtype)


def _rmsnorm(x, eps: float = 1e-5):
    return x * torch.rsqrt(x.float().pow(2).mean(dim=-1, keepdim=True) + eps).to(x.dtype)


def _inverse_softplus(v):
    v = v.clamp_min(1e-8)
    return v + torch.log(-torch.expm1(-v))


@dataclass(slots=True)
class MacroTrace:
    states: dict[int, torch.Tensor]
    stride_sequence: list[list[int]]
    physical_passes: torch.Tensor
    decomposition_error: torch.Tensor | None = None


class MacroOperators(nn.Module):
    def __init__(self, config: ModelConfig):
        super().__init__()
        self.config = config
        self.strides = list(config.depth_choices)
        self.stride_to_idx = {s: i for i, s in enumerate(self.strides)}
        r, k, d, m = config.recipe_count, len(self.strides), config.d_model, config.macro_rank
        if config.macro_type == "v2_delta_radius":
            input_dim = 3 * d + (d if (config.macro_use_delta_to_h0 or config.macro_include_delta_to_h0) else 0)
            if config.macro_use_depth_embedding:
                input_dim += d
                self.depth_embed = nn.Parameter(torch.randn(k, d) * (1.0 / max(d, 1) ** 0.5))
            else:
                self.register_parameter("depth_embed", None)
            if config.macro_use_recipe_embedding:
                input_dim += d
                self.recipe_embed = nn.Parameter(torch.randn(r, d) * (1.0 / max(d, 1) ** 0.5))
            else:
                self.register_parameter("recipe_embed", None)
            hidden = max(m, m * config.macro_hidden_mult)
            self.v = nn.Parameter(torch.randn(r, k, input_dim, hidden) * (1.0 / input_dim**0.5))
            self.v2 = nn.Parameter(torch.randn(r, k, hidden, m) * (1.0 / hidden**0.5))
            self.u = nn.Parameter(torch.randn(r, k, m, d) * 1e-3)
            self.bias = nn.Parameter(torch.zeros(r, k, d))
            radius = max(float(config.macro_update_scale_init), float(config.macro_update_scale), 1e-3)
            self.rho_base_raw = nn.Parameter(_inverse_softplus(torch.full((r, k), radius)))
            self.rho_head = nn.Parameter(torch.zeros(r, k, d, 1))
            self.register_buffer("teacher_delta_rms", torch.zeros(r, k), persistent=True)
            for name in ("d_gain", "update_scale", "gate_v", "gate_u", "gate_bias"):
                self.register_parameter(name, None)
        else:
            input_dim = 3 * d + (d if config.macro_include_delta_to_h0 else 0)
            if config.macro_use_depth_embedding:
                input_dim += d
                self.depth_embed = nn.Parameter(torch.randn(k, d) * (1.0 / max(d, 1) ** 0.5))
            else:
                self.register_parameter("depth_embed", None)
            self.register_parameter("recipe_embed", None)
            hidden = max(m, m * config.macro_hidden_mult)
            self.d_gain = nn.Parameter(torch.zeros(r, k, d))
            self.v = nn.Parameter(torch.randn(r, k, input_dim, hidden) * (1.0 / input_dim**0.5))
            if hidden != m:
                self.v2 = nn.Parameter(torch.randn(r, k, hidden, m) * (1.0 / hidden**0.5))
            else:
                self.register_parameter("v2", None)
            self.u = nn.Parameter(torch.randn(r, k, m, d) * 1e-3)
            update_scale = torch.full((r, k, d), float(config.macro_update_scale_init))
            legacy = (
                config.macro_hidden_mult == 1
                and not config.macro_use_gated_update
                and not config.macro_include_delta_to_h0
                and not config.macro_use_depth_embedding
                and config.macro_update_scale_init == 1.0
            )
            if legacy:
                self.register_buffer("update_scale", update_scale, persistent=True)
            else:
                self.update_scale = nn.Parameter(update_scale)
            self.bias = nn.Parameter(torch.zeros(r, k, d))
            if config.macro_use_gated_update:
                self.gate_v = nn.Parameter(torch.randn(r, k, input_dim, m) * (1.0 / input_dim**0.5))
                self.gate_u = nn.Parameter(torch.randn(r, k, m, d) * 1e-3)
                self.gate_bias = nn.Parameter(torch.zeros(r, k, d))
            else:
                for name in ("gate_v", "gate_u", "gate_bias"):
                    self.register_parameter(name, None)
            self.register_parameter("rho_base_raw", None)
            self.register_parameter("rho_head", None)
            self.register_buffer("teacher_delta_rms", torch.zeros(r, k), persistent=True)
        self.register_buffer("depth_values", torch.tensor(self.strides, dtype=torch.long), persistent=False)
        pairs = [(i, self.stride_to_idx[s * 2]) for i, s in enumerate(self.strides) if s * 2 in self.stride_to_idx]
        self.register_buffer("cons_src_idx", torch.tensor([p[0] for p in pairs], dtype=torch.long), persistent=False)
        self.register_buffer("cons_dst_idx", torch.tensor([p[1] for p in pairs], dtype=torch.long), persistent=False)
        # key offsets of the consistency loss's first operator call: the sorted union of the src
        # and dst strides when each role is a run of it (chained pairs such as (1, 2), (2, 4): a
        # shared stride is applied once), else [dst strides ; src strides]
        src, dst = [p[0] for p in pairs], [p[1] for p in pairs]
        union = sorted(set(src) | set(dst))
        pos_s, pos_d = [union.index(i) for i in src], [union.index(i) for i in dst]
        run = lambda pos: pos == list(range(pos[0], pos[0] + len(pos)))  # noqa: E731
        if pairs and run(pos_s) and run(pos_d) and len(union) < 2 * len(pairs):
            first, self.cons_src_lo, self.cons_dst_lo = union, pos_s[0], pos_d[0]
        else:
            first, self.cons_src_lo, self.cons_dst_lo = dst + src, len(pairs), 0
        self.register_buffer("cons_key_idx", torch.tensor(first, dtype=torch.long), persistent=False)
        # the first call's key offsets followed by the second call's (its src blocks): one key
        # tensor holds both calls' keys back to back
        ext = first + first[self.cons_src_lo:self.cons_src_lo + len(pairs)]
        self.register_buffer("cons_key_ext", torch.tensor(ext, dtype=torch.long), persistent=False)

    def stride_ids_for_depths(self, depths: torch.Tensor) -> torch.Tensor:
        matches = depths.unsqueeze(-1) == self.depth_values.to(depths.device).unsqueeze(0)
        return matches.float().argmax(dim=-1)

    def apply_vectorized(self, h, h0, recipe_ids, stride_ids):
        if self.config.macro_type == "v2_delta_radius":
            return self._apply_v2(h, h0, recipe_ids, stride_ids)
        return self._apply_bounded(h, h0, recipe_ids, stride_ids)

    def _rows(self, table: torch.Tensor, key: torch.Tensor) -> torch.Tensor:
        """Per-sample rows of a [recipes, strides, d] table (deterministic backward)."""
        flat = table.reshape(-1, table.shape[-1])
        if isinstance(table, nn.Parameter) or table.requires_grad:
            if flat.shape[1] % 8 == 0 and flat.shape[1] <= 2048:  # the segmented-reduction backward
                return hip_ops.embedding(flat, key)
            return gather_rows(flat, key)  # narrow tables (the v2 radius): one-hot product backward
        return flat.index_select(0, key)

    def _fused_bounded(self) -> bool:
        return (self.config.macro_type != "v2_delta_radius" and self.v2 is None and self.gate_v is None
                and not self.config.macro_include_delta_to_h0 and self.depth_embed is None)

    def _apply_bounded(self, h, h0, recipe_ids, stride_ids):
        """rte/macro.py:201-236.  The (recipe, stride)-indexed low-rank matrices are applied as
        grouped GEMMs over the rows of every sample sharing a key: no per-sample copies of
        v / u are gathered, and their gradients are per-group reductions in a fixed order."""
        _, S, d = h.shape
        R, Kk = self.v.shape[0], self.v.shape[1]
        key = torch.add(stride_ids.long(), recipe_ids.long(), alpha=Kk)
        B = key.numel()  # may exceed h's samples on the fused path (repeated sources)
        if (self._fused_bounded() and B % h.shape[0] == 0
                and hip_ops.macro_fused_supported(self.v, self.u, B // h.shape[0])):
            # rank 32: one fused kernel chain per direction, no row grouping needed
            return hip_ops.macro_fused(h, h0, key, self.v, self.u, self.d_gain, self.bias, self.update_scale,
                                       self.config.macro_update_scale)
        pk = hip_ops.group_rows(key[:, None].expand(B, S), R * Kk)
        f32 = hip_ops.fp32_active()
        if self._fused_bounded() and not f32:
            # default options: fused prologue / epilogue kernels around the two grouped GEMMs
            return hip_ops.macro_bounded(h, h0, key, pk, self.v, self.u, self.d_gain, self.bias, self.update_scale,
                                         self.config.macro_update_scale)
        if h.shape[0] != B:  # repeated source batches: sample b reads h[b % B_h]
            h = h.repeat(B // h.shape[0], 1, 1)
        if h0.shape[0] != B:
            h0 = h0.repeat(B // h0.shape[0], 1, 1)
        gain = self._rows(self.d_gain, key)
        bias = self._rows(self.bias, key)
        scale = self._rows(self.update_scale, key)
        normed = _rmsnorm(h)
        parts = [normed, normed.mean(dim=1, keepdim=True).expand_as(normed), h0]
        if self.config.macro_include_delta_to_h0:
            parts.append(normed - _rmsnorm(h0))
        if self.depth_embed is not None:
            parts.append(gather_rows(self.depth_embed, stride_ids).unsqueeze(1).expand_as(normed))
        # z is a GEMM operand only: build it in bf16 (the precision autocast gives the bmm), or
        # fp32 under precision fp32
        zdt = torch.float32 if f32 else torch.bfloat16
        z = torch.cat([t.to(zdt) for t in parts], dim=-1).reshape(B * S, -1)

        def lin(x, w, out_f32=False):
            return hip_ops.grouped_linear(x, w.reshape(R * Kk, w.shape[-2], w.shape[-1]), pk, out_f32=out_f32)

        low = F.silu(lin(z, self.v))
        if self.v2 is not None:
            low = F.silu(lin(low, self.v2))
        low = lin(low, self.u, out_f32=True).view(B, S, d)
        update = gain.unsqueeze(1) * h + low + bias.unsqueeze(1)
        if self.gate_v is not None:
            gate = torch.sigmoid(lin(F.silu(lin(z, self.gate_v)), self.gate_u, out_f32=True).view(B, S, d)
                                 + self._rows(self.gate_bias, key).unsqueeze(1))
        else:
            gate = 1.0
        return h + self.config.macro_update_scale * scale.unsqueeze(1) * gate * torch.tanh(update)

    def _apply_v2(self, h, h0, recipe_ids, stride_ids):
        """rte/macro.py:238-279.  The three (recipe, stride)-indexed products run as grouped GEMMs
        over the rows of every sample sharing a key (no per-sample [B, in, hidden] copies of v /
        v2 / u), their weight gradients as per-key reductions in a fixed order; rho_head's
        per-sample dot and the normalisation are device glue."""
        B, S, d = h0.shape
        R, Kk = self.v.shape[0], self.v.shape[1]
        key = recipe_ids.long() * Kk + stride_ids.long()
        f32 = hip_ops.fp32_active()
        normed = _rmsnorm(h0)
        pooled = normed.mean(dim=1)
        parts = [normed, pooled.unsqueeze(1).expand_as(normed), h0]
        if self.config.macro_use_delta_to_h0 or self.config.macro_include_delta_to_h0:
            parts.append(normed - _rmsnorm(h0))
        if self.depth_embed is not None:
            parts.append(gather_rows(self.depth_embed, stride_ids).unsqueeze(1).expand_as(normed))
        if self.recipe_embed is not None:
            parts.append(gather_rows(self.recipe_embed, recipe_ids).unsqueeze(1).expand_as(normed))
        zdt = torch.float32 if f32 else torch.bfloat16
        z = torch.cat([t.to(zdt) for t in parts], dim=-1).reshape(B * S, -1)
        pk = hip_ops.group_rows(key[:, None].expand(B, S), R * Kk)

        def lin(x, w, out_f32=False):
            return hip_ops.grouped_linear(x.to(zdt), w.reshape(R * Kk, w.shape[-2], w.shape[-1]), pk, out_f32=out_f32)

        raw = lin(F.silu(lin(F.silu(lin(z, self.v)), self.v2)), self.u, out_f32=True).view(B, S, d).float()
        raw = raw + self._rows(self.bias, key).unsqueeze(1)
        direction = raw / _rms(raw, dim=(1, 2), keepdim=True).clamp_min(1e-6)
        # rho_head [R, K, d, 1]: the sample's row dotted with its pooled features
        rho_head = (pooled.float() * self._rows(self.rho_head.squeeze(-1), key)).sum(dim=-1)
        rho = F.softplus(self._rows(self.rho_base_raw.unsqueeze(-1), key).squeeze(-1) + rho_head)
        teacher = self.teacher_delta_rms.reshape(-1).index_select(0, key).to(rho.device)
        if self.config.macro_radius_init_from_teacher:
            has = teacher > 0
            clamped = torch.clamp(rho, min=teacher * self.config.macro_radius_clamp_mult_min,
                                  max=teacher * self.config.macro_radius_clamp_mult_max)
            rho = torch.where(has, clamped, rho)
        return h0 + rho.view(-1, 1, 1).to(direction.dtype) * direction

    def forward(self, h, h0, recipe_ids, depths, *, return_states: bool = False, stride_ids=None):
        """stride_ids (optional): stride_ids_for_depths(depths) when the caller already has it."""
        del return_states
        if self.config.macro_decomposition != "direct":
            raise NotImplementedError("only macro_decomposition='direct' is on the accelerated path")
        if stride_ids is None:
            stride_ids = self.stride_ids_for_depths(depths)
        out = self.apply_vectorized(h, h0, recipe_ids, stride_ids)
        ones, zero = self._trace_constants(depths.shape[0], h.device, h.dtype)
        trace = MacroTrace(
            states={},
            stride_sequence=[],  # filled lazily by callers that need it (avoids a host sync)
            physical_passes=ones,
            decomposition_error=zero,
        )
        return out, trace

    def _trace_constants(self, n: int, device, dtype):
        """One physical pass per sample and a zero decomposition error: made once per (n, device,
        dtype) and shared by the steps (read-only)."""
        cache = self.__dict__.setdefault("_trace_const", {})
        key = (n, str(device), dtype)
        if key not in cache:
            cache[key] = (torch.ones(n, dtype=torch.float32, device=device), torch.zeros((), dtype=dtype, device=device))
        return cache[key]

    def consistency_loss(self, h, h0, recipe_ids):
        """rte/macro.py:342-359: Phi_{2s}(h) vs Phi_s(Phi_s(h)) for every (s, 2s) stride pair."""
        if self.cons_src_idx.numel() == 0:
            return h.new_zeros(())
        pc, b = self.cons_src_idx.numel(), h.shape[0]
        nf = self.cons_key_idx.numel()
        if h is h0 and self._fused_bounded() and hip_ops.macro_fused_supported(self.v, self.u, nf):
            # both operator applications, the MSE and every backward path in the fused kernels;
            # keys[p, i] = recipe_ids[i] Kk + cons_key_ext[p] in one launch: the first call's nf key
            # blocks, then the second call's pc (adjacent: the backward's grouped reductions read
            # both without a copy)
            Kk = self.v.shape[1]
            keys = torch.add(self.cons_key_ext.unsqueeze(1), recipe_ids.long().unsqueeze(0), alpha=Kk).reshape(-1)
            return hip_ops.macro_consistency(h, keys[:nf * b], keys[nf * b:], self.v, self.u, self.d_gain, self.bias,
                                             self.update_scale, self.config.macro_update_scale,
                                             src_lo=self.cons_src_lo, dst_lo=self.cons_dst_lo)
        r_rep = recipe_ids.repeat(pc)
        src = self.cons_src_idx.repeat_interleave(b)
        dst = self.cons_dst_idx.repeat_interleave(b)
        if self._fused_bounded() and 2 * pc <= 4:
            # Phi_{2s}(h) and the first Phi_s(h) read the same source batch: one operator call
            # over the 2 pc b (sample, key) pairs; the second Phi_s reads its output with h0
            # repeated.  No copies of h / h0 are made.
            both = self._apply_bounded(h, h0, torch.cat([r_rep, r_rep]), torch.cat([dst, src]))
            direct, first = both[:pc * b], both[pc * b:]
            twice = self._apply_bounded(first, h0, r_rep, src)
            return hip_ops.mse(direct, twice)
        h_rep = h.repeat(pc, 1, 1)
        h0_rep = h0.repeat(pc, 1, 1)
        direct = self.apply_vectorized(h_rep, h0_rep, r_rep, dst)
        twice = self.apply_vectorized(self.apply_vectorized(h_rep, h0_rep, r_rep, src), h0_rep, r_rep, src)
        # F.mse_loss (mean of squares) as staged means: per row, per sample, then over samples
        return (direct - twice).square().mean(dim=-1).mean(dim=-1).mean()


def macro_distill_loss(hot_hidden, exact_hidden, hot_logits, exact_logits, *, h0=None, lambda_hid=0.0,
                       lambda_cos=0.0, lambda_kl=0.0, lambda_norm=0.0, lambda_delta_dir=0.0, lambda_delta_rms=0.0,
                       lambda_endpoint_normed=0.0, lambda_endpoint_raw=0.0, lambda_macro_rms_trust=0.0,
                       temperature=1.0):
    """rte/macro.py:394-471."""
    exact_hidden = exact_hidden.detach()
    if exact_logits is not None:
        exact_logits = exact_logits.detach()
    zero = hot_hidden.new_zeros(())
    if h0 is not None:
        h0d = h0.detach()
        dp, de = hot_hidden - h0d, exact_hidden - h0d
        delta_dir = 1.0 - F.cosine_similarity(dp.flatten(1), de.flatten(1), dim=-1, eps=1e-8).mean()
        pr = _rms(dp, dim=(1, 2)).clamp_min(1e-8)
        er = _rms(de, dim=(1, 2)).clamp_min(1e-8)
        delta_rms = (torch.log(pr) - torch.log(er)).square().mean()
        endpoint_normed = F.smooth_l1_loss(_rmsnorm(hot_hidden), _rmsnorm(exact_hidden))
        endpoint_raw = F.smooth_l1_loss(hot_hidden, exact_hidden)
        ratio = _rms(hot_hidden, dim=(1, 2)).clamp_min(1e-8) / _rms(exact_hidden, dim=(1, 2)).clamp_min(1e-8)
        rms_trust = torch.log(ratio).square().mean().to(hot_hidden.dtype)
        hid = cos = norm = zero
    else:
        hid = F.mse_loss(hot_hidden, exact_hidden)
        cos = 1.0 - F.cosine_similarity(hot_hidden.flatten(1), exact_hidden.flatten(1), dim=-1, eps=1e-8).mean()
        hr = hot_hidden.float().pow(2).mean(dim=-1).sqrt()
        er = exact_hidden.float().pow(2).mean(dim=-1).sqrt()
        norm = (hr - er).abs().mean().to(hot_hidden.dtype)
        delta_dir = delta_rms = endpoint_normed = endpoint_raw = rms_trust = zero
    if hot_logits is not None and exact_logits is not None and hot_logits.shape == exact_logits.shape:
        t = max(float(temperature), 1e-6)
        # F.kl_div(log q, p, reduction="batchmean") = sum p (log p - log q) / batch, reduced row
        # by row first (a per-row reduction keeps every partial sum inside one workgroup)
        logq = F.log_softmax(hot_logits / t, dim=-1)
        p = F.softmax(exact_logits / t, dim=-1)
        rows = (torch.xlogy(p, p) - p * logq).sum(dim=-1)
        kl = rows.reshape(rows.shape[0], -1).sum(dim=-1).sum() / hot_logits.shape[0] * (t**2)
    else:
        kl = zero
    return {
        "hid": lambda_hid * hid,
        "cos": lambda_cos * cos,
        "kl": lambda_kl * kl,
        "norm": lambda_norm * norm,
        "delta_dir": lambda_delta_dir * delta_dir,
        "delta_rms": lambda_delta_rms * delta_rms,
        "endpoint_normed": lambda_endpoint_normed * endpoint_normed,
        "endpoint_raw": lambda_endpoint_raw * endpoint_raw,
        "rms_trust": lambda_macro_rms_trust * rms_trust,
    }


def macro_alignment_metrics(hot_hidden, exact_hidden, *, h0, hot_logits=None, exact_logits=None):
    """rte/macro.py:499-546."""
    exact_hidden = exact_hidden.detach()
    m = {
        "hidden_cosine_exact_macro": F.cosine_similarity(hot_hidden.flatten(1), exact_hidden.flatten(1), dim=-1,
                                                         eps=1e-8).mean(),
        "hidden_mse_exact_macro": (hot_hidden - exact_hidden).square().mean(),
    }
    macro_norm = _rms(hot_hidden, dim=(1, 2)).mean()
    exact_norm = _rms(exact_hidden, dim=(1, 2)).mean()
    m.update(macro_norm=macro_norm, exact_norm=exact_norm, macro_exact_norm_ratio=macro_norm / exact_norm.clamp_min(1e-8))
    if h0 is not None:
        dp, de = hot_hidden - h0.detach(), exact_hidden - h0.detach()
        m["delta_cosine_exact_macro"] = F.cosine_similarity(dp.flatten(1), de.flatten(1), dim=-1, eps=1e-8).mean()
        pr, er = _rms(dp, dim=(1, 2)).mean(), _rms(de, dim=(1, 2)).mean()
        m.update(delta_rms_exact=er, delta_rms_pred=pr, delta_rms_ratio=pr / er.clamp_min(1e-8))
    if hot_logits is not None and exact_logits is not None and hot_logits.shape == exact_logits.shape:
        te = F.log_softmax(exact_logits.detach(), dim=-1)
        th = F.log_softmax(hot_logits, dim=-1)
        m["logit_kl_exact_macro"] = (te.exp() * (te - th)).sum(dim=-1).mean()
    return m
