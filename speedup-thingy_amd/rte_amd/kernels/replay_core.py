"""Exact recursive passes of the banked core for the audit replay's few samples, all T passes as
one autograd node on the HIP replay kernels (csrc/replay.hip).

Reference: BankedRecursiveCore.forward_step (rte/layers.py:806-870) applied pass by pass by
forward_exact (rte/models.py:416-512) to the audited rows (rte/audit.py:245-387).  Per pass the
forward is seven launches (residual + norm1 rows, QKV + RoPE over the recipe's heads, attention,
O-projection, residual + norm2 rows, up / gate + SwiGLU over the recipe's slabs, down-projection +
residual) and the backward seven (down + SwiGLU backward, up / gate backward, norm2 backward rows,
O-projection backward, attention backward, QKV backward, norm1 backward rows, which also form the
previous pass's down operand); the four weight gradients are one GEMM each over every pass's rows,
and the FiLM / scale / skip gradients one fixed-order reduction.  Values match the unfused pass
(the same bf16 operands, fp32 accumulation) up to summation order: the down-projection sums all
of a token's slabs in one fp32 accumulator instead of adding per-cluster bf16 rows.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

from rte_amd import _lib
from rte_amd._lib import call, ptr
from rte_amd.kernels.hip_ops import BF16, F32, _s, cast_bf16, gemm

HEAD_DIM = 64
BLOCK = 32  # neurons per slab block
MAX_D = 512


@dataclass
class ReplayTables:
    """Per-recipe records int32 [R, W], W = 4 + 2 H + 2 NB: 1 | nh | nb | 0 | heads[H] (the
    recipe's heads, ascending) | ihead[H] (slot of each head or -1) | blks[NB] (its 32-neuron
    slab blocks, ascending) | iblk[NB].  The replay gathers one per (pass, sample) and writes the
    pass's active flag into word 0."""

    records: torch.Tensor
    H: int
    NB: int
    h_max: int
    nb_max: int

    def info(self, rids: torch.Tensor, actives: torch.Tensor | None) -> torch.Tensor:
        """[T, B, W] records of the recipes rids [T, B] with the active flags."""
        info = self.records[rids]
        if actives is not None:
            info[..., 0] = actives.to(torch.int32)
        return info.contiguous()


def build_records(head_lists: list[list[int]], block_lists: list[list[int]], H: int, NB: int) -> torch.Tensor:
    """The per-recipe records of ReplayTables (CPU) from each recipe's active heads and blocks."""
    R = len(head_lists)
    W = 4 + 2 * H + 2 * NB
    rec = torch.full((R, W), -1, dtype=torch.int32)
    for r, (hl, bl) in enumerate(zip(head_lists, block_lists)):
        hl, bl = sorted(set(hl)), sorted(set(bl))
        rec[r, 0], rec[r, 1], rec[r, 2], rec[r, 3] = 1, len(hl), len(bl), 0
        for i, h in enumerate(hl):
            rec[r, 4 + i] = h
            rec[r, 4 + H + h] = i
        for i, b in enumerate(bl):
            rec[r, 4 + 2 * H + i] = b
            rec[r, 4 + 2 * H + NB + b] = i
    return rec


def _f32c(t: torch.Tensor) -> torch.Tensor:
    return t.detach().contiguous().to(F32)


class ReplayCoreFn(torch.autograd.Function):
    """(h_T, *states) = T exact passes of the banked core from h0 (fp32 [B, S, d]).

    rids [T, B] int64 recipes per pass, actives [T, B] bool (None: every sample takes every pass);
    states = the outputs of the passes listed in `keep` (each < T - 1).  Differentiable inputs:
    h0, the per-pass FiLM rows g1 / b1 / g2 / b2 [T, d], s_attn / s_mlp [T], alpha (scalar or
    None), the norm weights w1 / w2 [d] and the bank weights wqkv [1, d, 3d], wo [1, d, d],
    wug [1, d, 2F], wd [1, F, d]."""

    @staticmethod
    def forward(ctx, h0, g1, b1, g2, b2, s_attn, s_mlp, alpha, w1, w2, wqkv, wo, wug, wd, rids, actives,
                tabs: ReplayTables, cos, sin, eps1: float, eps2: float, route_w: float, keep: tuple):
        _lib.require_device_tensors("replay_core", h0, g1, b1, g2, b2, s_attn, s_mlp, alpha, w1, w2, wqkv, wo, wug,
                                    wd, rids, actives, cos, sin)
        B, S, d = h0.shape
        T = rids.shape[0]
        H, F = tabs.H, wd.shape[1]
        if d > MAX_D or d % 128 or H * HEAD_DIM != d or F != tabs.NB * BLOCK:
            raise ValueError("replay_core: d <= 512 (multiple of 128), head width 64, d_ff in 32-neuron blocks")
        if wqkv.shape[0] != 1 or wug.shape[0] != 1:
            raise ValueError("replay_core: one attention bank and one FFN bank")
        dev = h0.device
        M, Hm, NBm = B * S, tabs.h_max, tabs.nb_max
        hv = _f32c(h0)
        wqkv_t, wo_t = cast_bf16(wqkv[0].t()), cast_bf16(wo[0].t())
        wug_t, wd_t = cast_bf16(wug[0].t()), cast_bf16(wd[0].t())
        cs, sn = _f32c(cos[:S]), _f32c(sin[:S])
        info = tabs.info(rids.to(torch.int64), actives)
        meta = (B, S, d, H, F, tabs.NB, tabs.h_max, tabs.nb_max)
        vecs = [_f32c(t) for t in (g1, b1, g2, b2, s_attn, s_mlp, w1, w2)]
        g1c, b1c, g2c, b2c, sac, smc, w1c, w2c = vecs
        al = None if alpha is None else _f32c(alpha).reshape(1)

        def e(*shape, dt=F32):
            return torch.empty(shape, dtype=dt, device=dev)

        ht, attn, u, mlp = e(T, M, d), e(T, M, d), e(T, M, d), e(T, M, d)
        n1, n2, y_full = e(T, M, d, dt=BF16), e(T, M, d, dt=BF16), e(T, M, d, dt=BF16)
        rstd1, rstd2 = e(T, M), e(T, M)
        q, k, v = (e(T, B, Hm, S, HEAD_DIM, dt=BF16) for _ in range(3))
        y, lse = e(T, M, Hm * HEAD_DIM, dt=BF16), e(T, B, Hm, S)
        ug, z = e(T, M, NBm * 2 * BLOCK, dt=BF16), e(T, M, NBm * BLOCK, dt=BF16)
        z_full = e(T, M, F, dt=BF16)
        h_out = [e(B, S, d) for _ in range(T)]
        st = _s()
        for t in range(T):
            h_in = hv if t == 0 else h_out[t - 1]
            call("rte_replay_fwd_pass", *meta, ptr(info[t]), ptr(h_in), ptr(hv), ptr(al), ptr(w1c), ptr(g1c[t]),
                 ptr(b1c[t]), float(eps1), ptr(w2c), ptr(g2c[t]), ptr(b2c[t]), float(eps2), ptr(sac[t]), ptr(smc[t]), float(route_w), ptr(wqkv_t), ptr(wo_t),
                 ptr(wug_t), ptr(wd_t), ptr(cs), ptr(sn), ptr(ht[t]), ptr(n1[t]), ptr(rstd1[t]), ptr(q[t]),
                 ptr(k[t]), ptr(v[t]), ptr(y[t]), ptr(lse[t]), ptr(attn[t]), ptr(u[t]), ptr(y_full[t]), ptr(n2[t]),
                 ptr(rstd2[t]), ptr(ug[t]), ptr(z[t]), ptr(mlp[t]), ptr(h_out[t]), ptr(z_full[t]), st)
        ctx.save_for_backward(hv, info, g1c, g2c, sac, smc, al, w1c, w2c, cs, sn, ht, n1, rstd1, q, k, v, y, lse,
                              attn, u, y_full, n2, rstd2, ug, z, mlp, z_full)
        ctx.tabs, ctx.keep = tabs, tuple(keep)
        ctx.meta = (B, S, d, H, F, T, float(route_w), h0.dtype, alpha is not None)
        ctx.weights = (wqkv, wo, wug, wd)
        ctx.set_materialize_grads(False)
        return (h_out[T - 1], *[h_out[t] for t in keep])

    @staticmethod
    def backward(ctx, dhT, *dstates):
        (hv, info, g1c, g2c, sac, smc, al, w1c, w2c, cs, sn, ht, n1, rstd1, q, k, v, y, lse, attn, u, y_full, n2,
         rstd2, ug, z, mlp, z_full) = ctx.saved_tensors
        B, S, d, H, F, T, route_w, h_dt, has_alpha = ctx.meta
        tabs = ctx.tabs
        wqkv, wo, wug, wd = ctx.weights
        dev = hv.device
        M, Hm, NBm = B * S, tabs.h_max, tabs.nb_max
        nt = _lib.load().rte_replay_row_tiles(B, S)

        def e(*shape, dt=F32):
            return torch.empty(shape, dtype=dt, device=dev)

        extra = {t: g for t, g in zip(ctx.keep, dstates) if g is not None}
        dh = dhT.contiguous().to(F32) if dhT is not None else torch.zeros((B, S, d), dtype=F32, device=dev)
        wqkv_p, wo_p = cast_bf16(wqkv[0]), cast_bf16(wo[0])
        wug_p, wd_p = cast_bf16(wug[0]), cast_bf16(wd[0])
        dug, dn2, du, dn1 = e(M, NBm * 2 * BLOCK, dt=BF16), e(M, d), e(M, d), e(M, d)
        dy, dqkv = e(M, Hm * HEAD_DIM, dt=BF16), e(M, 3 * Hm * HEAD_DIM, dt=BF16)
        a_mlp, d_attn = e(T, M, d, dt=BF16), e(T, M, d, dt=BF16)
        dug_full, dqkv_full = e(T, M, 2 * F, dt=BF16), e(T, M, 3 * d, dt=BF16)
        p_film1, p_film2 = e(T, nt, 3 * d), e(T, nt, 3 * d)
        p_sa, p_alpha, p_sm = e(T, nt), e(T, nt), e(T, nt)
        bufs = [e(B, S, d), e(B, S, d)]
        dh0 = e(M, d) if has_alpha else None
        st = _s()
        fresh = True  # dh changed since the last norm1 backward formed the down operand
        for i, t in enumerate(reversed(range(T))):
            if t in extra:
                dh, fresh = dh + extra[t].to(F32), True
            dh = dh.contiguous()
            if fresh:
                call("rte_replay_bwd_prep", B, S, d, ptr(dh), ptr(mlp[t]), ptr(smc[t]), ptr(a_mlp[t]), ptr(p_sm[t]),
                     st)
            # the pass before this one gets its down operand from this call unless a state gradient lands first
            nxt = t > 0 and (t - 1) not in extra
            dh_in = bufs[i % 2]
            call("rte_replay_bwd_pass", B, S, d, H, F, tabs.NB, tabs.h_max, tabs.nb_max, ptr(info[t]), ptr(dh),
                 ptr(a_mlp[t]), ptr(wd_p), ptr(ug[t]), route_w, ptr(dug), ptr(wug_p), ptr(dn2), ptr(dug_full[t]),
                 ptr(u[t]), ptr(rstd2[t]), ptr(w2c), ptr(g2c[t]), ptr(attn[t]), ptr(sac[t]), ptr(du),
                 ptr(d_attn[t]), ptr(p_film2[t]), ptr(p_sa[t]), ptr(wo_p), ptr(dy), ptr(q[t]), ptr(k[t]), ptr(v[t]),
                 ptr(y[t]), ptr(lse[t]), ptr(cs), ptr(sn), ptr(dqkv), ptr(wqkv_p), ptr(dn1), ptr(dqkv_full[t]),
                 ptr(ht[t]), ptr(rstd1[t]), ptr(w1c), ptr(g1c[t]), ptr(hv) if has_alpha else None, ptr(al),
                 int(i > 0), ptr(dh_in), ptr(dh0), ptr(p_film1[t]), ptr(p_alpha[t]),
                 ptr(mlp[t - 1]) if nxt else None, ptr(smc[t - 1]) if nxt else None,
                 ptr(a_mlp[t - 1]) if nxt else None, ptr(p_sm[t - 1]) if nxt else None, st)
            dh, fresh = dh_in, not nxt
        red = e(T * 6 * d + 2 * d + 2 * T + 1)
        call("rte_replay_param_reduce", T, B, S, d, ptr(p_film1), ptr(p_film2), ptr(p_sa), ptr(p_sm), ptr(p_alpha),
             ptr(red), st)
        per = red[:T * 6 * d].view(T, 6 * d)
        tail = red[T * 6 * d:]
        nia = ctx.needs_input_grad
        dh0_total = dh.view(B, S, d) + dh0.view(B, S, d) if has_alpha else dh.view(B, S, d)

        def wgrad(i, a, b, shape):
            if not nia[i]:
                return None
            return gemm(a.reshape(T * M, -1), b.reshape(T * M, -1), a_t=True, b_t=True, out_f32=True).view(shape)

        return (dh0_total.to(h_dt) if nia[0] else None,
                per[:, d:2 * d] if nia[1] else None, per[:, 2 * d:3 * d] if nia[2] else None,
                per[:, 4 * d:5 * d] if nia[3] else None, per[:, 5 * d:6 * d] if nia[4] else None,
                tail[2 * d:2 * d + T] if nia[5] else None, tail[2 * d + T:2 * d + 2 * T] if nia[6] else None,
                tail[2 * d + 2 * T].reshape(()) if (has_alpha and nia[7]) else None,
                tail[:d] if nia[8] else None, tail[d:2 * d] if nia[9] else None,
                wgrad(10, n1, dqkv_full, (1, d, 3 * d)), wgrad(11, y_full, d_attn, (1, d, d)),
                wgrad(12, n2, dug_full, (1, d, 2 * F)), wgrad(13, z_full, a_mlp, (1, F, d)),
                None, None, None, None, None, None, None, None, None)


def replay_core(h0, g1, b1, g2, b2, s_attn, s_mlp, alpha, w1, w2, wqkv, wo, wug, wd, rids, actives, tabs, cos, sin,
                eps1, eps2, route_w=1.0, keep=()):
    return ReplayCoreFn.apply(h0, g1, b1, g2, b2, s_attn, s_mlp, alpha, w1, w2, wqkv, wo, wug, wd, rids, actives,
                              tabs, cos, sin, eps1, eps2, route_w, tuple(keep))
