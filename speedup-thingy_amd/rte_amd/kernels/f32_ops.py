"""fp32 operators over librte_hip: the arithmetic of training.precision = "fp32".

The reference's default precision (rte/config.py:118) runs every matmul in float32 outside an
autocast region (rte/training.py:356-363).  Here every product runs on the fp32 MFMA GEMM
(rte_gemm_f32: v_mfma_f32_32x32x2_f32, fp32 operands and accumulation) -- dense, batched (the
attention's per-(sample, head) products) and grouped (routed / banked pools, per-key macro
products and their weight gradients, each group's rows summed in a fixed order) -- and the
causal softmax, SwiGLU and pair combine run as fp32 HIP kernels.  Small per-sample arithmetic
(norm FiLM terms, router heads, the macro epilogue) is device-side torch glue on the same stream.

hip_ops dispatches here while a `hip_ops.fp32_precision()` block is active (TrainEngine opens one
for precision fp32); nothing here casts to bf16.
"""

from __future__ import annotations

import math

import torch

from rte_amd import _lib
from rte_amd._lib import call, ptr
from rte_amd.kernels import hip_ops as H

F32 = torch.float32


def _s() -> int:
    return _lib.stream_ptr()


def _c32(t: torch.Tensor) -> torch.Tensor:
    return t.contiguous() if t.dtype == F32 else t.contiguous().to(F32)


# ----------------------------------------------------------------------------- GEMM entry points

def gemm(A, lda, a_t, B, ldb, b_t, C, ldc, M, N, K, *, alpha=1.0, beta=0.0, a_rows=None, a_scale=None, b_rows=None,
         b_scale=None, c_rows=None, batch=(1, 1), sA=(0, 0), sB=(0, 0), sC=(0, 0)):
    """C(m, n) = alpha sum_k A(m, k) B(n, k) + beta C(m, n) on raw fp32 buffers (see rte_gemm_f32)."""
    call("rte_gemm_f32", ptr(A), int(lda), int(a_t), ptr(a_rows), ptr(a_scale), ptr(B), int(ldb), int(b_t), ptr(b_rows),
         ptr(b_scale), ptr(C), int(ldc), ptr(c_rows), int(M), int(N), int(K), float(alpha), float(beta), int(batch[0]),
         int(batch[1]), int(sA[0]), int(sA[1]), int(sB[0]), int(sB[1]), int(sC[0]), int(sC[1]), _s())


def gemm_grouped(mode, goff, G, A, lda, a_t, B, ldb, b_t, C, ldc, M, N, K, *, alpha=1.0, beta=0.0, a_rows=None,
                 a_scale=None, b_rows=None, b_scale=None, b_goff=None, b_gstride=0, b_rows_gstride=0, c_rows=None,
                 c_goff=None, c_gstride=0, c_rows_gstride=0):
    """mode 1: group g owns rows [goff[g], goff[g+1]); mode 2: group g reduces over that k range."""
    call("rte_gemm_f32_grouped", int(mode), ptr(goff), int(G), ptr(A), int(lda), int(a_t), ptr(a_rows), ptr(a_scale),
         ptr(B), int(ldb), int(b_t), ptr(b_rows), ptr(b_scale), ptr(b_goff), int(b_gstride), int(b_rows_gstride),
         ptr(C), int(ldc), ptr(c_rows), ptr(c_goff), int(c_gstride), int(c_rows_gstride), int(M), int(N), int(K),
         float(alpha), float(beta), _s())


def _wlayout(w: torch.Tensor):
    """(buffer, transposed, ld) of a 2-D weight read as B(n, k) = w[n, k]: a contiguous w, or a
    transposed view of a contiguous [K, N] tensor (the banked weights' layout)."""
    if w.is_contiguous():
        return w, 0, w.shape[1]
    if w.t().is_contiguous():
        return w.t(), 1, w.shape[0]
    wc = w.contiguous()
    return wc, 0, wc.shape[1]


class LinearFn(torch.autograd.Function):
    """y = x w^T (w [N, K]; a contiguous tensor or a transposed view of one), fp32."""

    @staticmethod
    def forward(ctx, x, w):
        _lib.require_device_tensors("linear_f32", x, w)
        shape = x.shape
        K = shape[-1]
        x2 = _c32(x.reshape(-1, K))
        wv = w if w.dtype == F32 else w.to(F32)
        wb, wt, ldw = _wlayout(wv)
        M, N = x2.shape[0], wv.shape[0]
        y = torch.empty((M, N), dtype=F32, device=x.device)
        gemm(x2, K, 0, wb, ldw, wt, y, N, M, N, K)
        ctx.save_for_backward(x2, wb)
        ctx.meta = (shape, wt, ldw, N, K, w.dtype, x.dtype)
        return y.view(*shape[:-1], N)

    @staticmethod
    def backward(ctx, dy):
        x2, wb = ctx.saved_tensors
        shape, wt, ldw, N, K, w_dt, x_dt = ctx.meta
        M = x2.shape[0]
        dy2 = _c32(dy.reshape(M, N))
        dx = dw = None
        if ctx.needs_input_grad[0]:
            dx = torch.empty((M, K), dtype=F32, device=x2.device)
            # dx(m, k) = sum_n dy(m, n) w(n, k): w's memory rows run over n (w contiguous) or k
            gemm(dy2, N, 0, wb, ldw, 1 - wt, dx, K, M, K, N)
            dx = dx.view(*shape[:-1], K).to(x_dt)
        if ctx.needs_input_grad[1]:
            if wt == 0:  # dw [N, K] = dy^T x
                dw = torch.empty((N, K), dtype=F32, device=x2.device)
                gemm(dy2, N, 1, x2, K, 1, dw, K, N, K, M)
            else:  # the parameter is [K, N] memory: form dW^T there and hand back its view
                dwt = torch.empty((K, N), dtype=F32, device=x2.device)
                gemm(x2, K, 1, dy2, N, 1, dwt, N, K, N, M)
                dw = dwt.t()
            dw = dw.to(w_dt)
        return dx, dw


def linear(x, w, bias=None):
    y = LinearFn.apply(x, w)
    return y if bias is None else y + bias.to(F32)


# ----------------------------------------------------------------------------- attention

class AttentionFn(torch.autograd.Function):
    """Causal attention of q, k, v [B, H, S, hd] (fp32): y [B, S, H hd] token-major for the
    output projection; P = softmax(q k^T / sqrt(hd)) with keys <= query, scaled per (b, h) by
    head_scale [B, H] when given (the banked recipe's head / bank mask)."""

    @staticmethod
    def forward(ctx, q, k, v, head_scale):
        _lib.require_device_tensors("attention_f32", q, k, v, head_scale)
        q, k, v = _c32(q), _c32(k), _c32(v)
        B, Hh, S, hd = q.shape
        dev = q.device
        scale = 1.0 / math.sqrt(hd)
        hs = None if head_scale is None else _c32(head_scale.reshape(B * Hh))
        sc = torch.empty((B, Hh, S, S), dtype=F32, device=dev)
        bst = (Hh * S * hd, S * hd)
        gemm(q, hd, 0, k, hd, 0, sc, S, S, S, hd, batch=(B, Hh), sA=bst, sB=bst, sC=(Hh * S * S, S * S))
        P = torch.empty_like(sc)
        Pm = torch.empty_like(sc) if hs is not None else P
        call("rte_softmax_causal_f32_fwd", ptr(sc), B * Hh * S, S, scale, ptr(hs), ptr(P), ptr(Pm), _s())
        y = torch.empty((B, S, Hh * hd), dtype=F32, device=dev)
        # y[b, s, h hd + j] = sum_s' Pm[b, h, s, s'] v[b, h, s', j]
        gemm(Pm, S, 0, v, hd, 1, y, Hh * hd, S, hd, S, batch=(B, Hh), sA=(Hh * S * S, S * S), sB=bst,
             sC=(S * Hh * hd, hd))
        ctx.save_for_backward(q, k, v, P, Pm, hs)
        ctx.meta = (B, Hh, S, hd, scale)
        return y

    @staticmethod
    def backward(ctx, dy):
        q, k, v, P, Pm, hs = ctx.saved_tensors
        B, Hh, S, hd, scale = ctx.meta
        dy = _c32(dy)
        dev = q.device
        bst = (Hh * S * hd, S * hd)
        sss = (Hh * S * S, S * S)
        ysd = (S * Hh * hd, hd)
        dPm = torch.empty((B, Hh, S, S), dtype=F32, device=dev)
        # dPm[s, s'] = sum_j dy[s, h hd + j] v[s', j]
        gemm(dy, Hh * hd, 0, v, hd, 0, dPm, S, S, S, hd, batch=(B, Hh), sA=ysd, sB=bst, sC=sss)
        ds = torch.empty_like(dPm)
        call("rte_softmax_causal_f32_bwd", ptr(P), ptr(dPm), B * Hh * S, S, scale, ptr(hs), ptr(ds), _s())
        dq = torch.empty_like(q)
        dk = torch.empty_like(k)
        dv = torch.empty_like(v)
        gemm(ds, S, 0, k, hd, 1, dq, hd, S, hd, S, batch=(B, Hh), sA=sss, sB=bst, sC=bst)      # ds k
        gemm(ds, S, 1, q, hd, 1, dk, hd, S, hd, S, batch=(B, Hh), sA=sss, sB=bst, sC=bst)      # ds^T q
        gemm(Pm, S, 1, dy, Hh * hd, 1, dv, hd, S, hd, S, batch=(B, Hh), sA=sss, sB=ysd, sC=bst)  # Pm^T dy
        return dq, dk, dv, None


def qkv_rope_attention(x, w, cos, sin, n_heads: int, head_scale=None):
    """qkv = x w^T viewed [B, S, 3, H, hd] (rte/layers.py:63-71), interleaved RoPE on q and k
    (the dtype-preserving HIP RoPE kernel), causal attention: y [B, S, d] fp32."""
    B, S, d = x.shape
    hd = d // n_heads
    qkv = LinearFn.apply(x, w).view(B, S, 3, n_heads, hd)
    q, k, v = (t.permute(0, 2, 1, 3) for t in qkv.unbind(dim=2))
    c, s_ = _c32(cos[:S]), _c32(sin[:S])
    if hd % 8 == 0:  # the HIP RoPE kernel
        q, k = H.RopeApplyFn.apply(q.contiguous(), k.contiguous(), c, s_)
    else:  # head widths the kernel does not tile (e.g. 4): the same rotation as device glue
        q, k = _rope_glue(q, c, s_), _rope_glue(k, c, s_)
    return AttentionFn.apply(q, k, v.contiguous(), head_scale)


def _rope_glue(x, cos, sin):
    """x cos + rotate_half(x) sin with interleaved pairs (rte/kernels/reference.py:20-28)."""
    rot = torch.stack((-x[..., 1::2], x[..., 0::2]), dim=-1).flatten(-2)
    return x * cos + rot * sin


def attn_out_proj(y, w, resid=None):
    out = LinearFn.apply(y, w)
    return out if resid is None else out + resid.to(F32)


# ----------------------------------------------------------------------------- SwiGLU

class SwiGLUFn(torch.autograd.Function):
    """z = up silu(gate) over rows [up (n) | gate (n)] of ug [..., 2n]."""

    @staticmethod
    def forward(ctx, ug):
        u2 = _c32(ug.reshape(-1, ug.shape[-1]))
        n = u2.shape[1] // 2
        z = torch.empty((u2.shape[0], n), dtype=F32, device=u2.device)
        call("rte_swiglu_f32_fwd", ptr(u2), u2.shape[0], n, u2.shape[1], ptr(z), _s())
        ctx.save_for_backward(u2)
        ctx.shape = ug.shape
        return z.view(*ug.shape[:-1], n)

    @staticmethod
    def backward(ctx, dz):
        (u2,) = ctx.saved_tensors
        n = u2.shape[1] // 2
        dug = torch.empty_like(u2)
        call("rte_swiglu_f32_bwd", ptr(u2), ptr(_c32(dz.reshape(-1, n))), u2.shape[0], n, u2.shape[1], ptr(dug), _s())
        return dug.view(ctx.shape)


def dense_swiglu(x, wug, wd, resid=None, *, wd_rows: bool = False):
    """DenseSwiGLU (rte/layers.py:78-87): wug [2F, d] rows [up ; gate], wd [d, F] (Linear) or
    wd_rows [F, d]."""
    z = SwiGLUFn.apply(LinearFn.apply(x, wug))
    y = LinearFn.apply(z, wd.t() if wd_rows else wd)
    return y if resid is None else y + resid.to(F32)


# ----------------------------------------------------------------------------- grouped pools

class GroupedPoolFn(torch.autograd.Function):
    """out[t] = sum_j w[t, j] SwiGLU_{c(t, j)}(x[t]) over a PackIndex of (token, cluster) pairs.

    wug_rows [R, d] and wd_rows [Rn, d] hold the weights row-major; cluster c's up / gate rows are
    ug_rows[c] (2n entries, up first) and its down rows dn_rows[c] (n entries).  Forward: the
    up / gate product over each cluster's slots (rows of x gathered by slot), SwiGLU, the down
    product, the fixed-order pair combine.  Backward: the same grouped products transposed, the
    weight gradients as one reduction group per cluster (its slots in order: every weight row is
    written once, so repeats are bitwise equal), the pair weights' gradient as row dots."""

    @staticmethod
    def forward(ctx, x, w, wug_rows, wd_rows, pk, ug_rows, dn_rows, n: int):
        _lib.require_device_tensors("grouped_pool_f32", x, w, wug_rows, wd_rows)
        shape = x.shape
        d = shape[-1]
        x2 = _c32(x.reshape(-1, d))
        T = x2.shape[0]
        C, k = pk.n_clusters, pk.k
        P = pk.tok_of_slot.numel()
        dev = x2.device
        wu = _c32(wug_rows)
        wdn = _c32(wd_rows)
        ug = torch.empty((P, 2 * n), dtype=F32, device=dev)
        gemm_grouped(1, pk.offsets, C, x2, d, 0, wu, d, 0, ug, 2 * n, P, 2 * n, d, a_rows=pk.tok_of_slot,
                     b_rows=ug_rows, b_rows_gstride=2 * n)
        z = torch.empty((P, n), dtype=F32, device=dev)
        call("rte_swiglu_f32_fwd", ptr(ug), P, n, 2 * n, ptr(z), _s())
        y = torch.empty((P, d), dtype=F32, device=dev)
        gemm_grouped(1, pk.offsets, C, z, n, 0, wdn, d, 1, y, d, P, d, n, b_rows=dn_rows, b_rows_gstride=n)
        wv = _c32(w.reshape(T, k))
        out = torch.empty((T, d), dtype=F32, device=dev)
        call("rte_combine_f32", ptr(y), ptr(pk.slot_of_pair), ptr(wv), T, k, d, None, ptr(out), _s())
        ctx.save_for_backward(x2, wu, wdn, ug, z, y, wv)
        ctx.meta = (shape, pk, ug_rows, dn_rows, n)
        return out.view(shape)

    @staticmethod
    def backward(ctx, dout):
        x2, wu, wdn, ug, z, y, wv = ctx.saved_tensors
        shape, pk, ug_rows, dn_rows, n = ctx.meta
        T, d = x2.shape
        C, k = pk.n_clusters, pk.k
        P = pk.tok_of_slot.numel()
        dev = x2.device
        do = _c32(dout.reshape(T, d))
        scale = pk.w_of_slot  # the slot's pair weight
        # dz[s] = (w_s dout[tok s]) wd_c^T ; dug = SwiGLU'
        dz = torch.empty((P, n), dtype=F32, device=dev)
        gemm_grouped(1, pk.offsets, C, do, d, 0, wdn, d, 0, dz, n, P, n, d, a_rows=pk.tok_of_slot, a_scale=scale,
                     b_rows=dn_rows, b_rows_gstride=n)
        dug = torch.empty_like(ug)
        call("rte_swiglu_f32_bwd", ptr(ug), ptr(dz), P, n, 2 * n, ptr(dug), _s())
        dx = None
        if ctx.needs_input_grad[0]:
            dxs = torch.empty((P, d), dtype=F32, device=dev)
            gemm_grouped(1, pk.offsets, C, dug, 2 * n, 0, wu, d, 1, dxs, d, P, d, 2 * n, b_rows=ug_rows,
                         b_rows_gstride=2 * n)
            dx = torch.empty((T, d), dtype=F32, device=dev)
            call("rte_combine_f32", ptr(dxs), ptr(pk.slot_of_pair), None, T, k, d, None, ptr(dx), _s())
            dx = dx.view(shape)
        dw = None
        if ctx.needs_input_grad[1]:
            dw = torch.empty((T, k), dtype=F32, device=dev)
            call("rte_pair_dot_f32", ptr(do), ptr(y), ptr(pk.slot_of_pair), T * k, k, d, ptr(dw), _s())
        dwu = dwd = None
        if ctx.needs_input_grad[2]:
            # rows ug_rows[c, m] of dW_ug: sum over cluster c's slots of dug[s, m] x[tok s]
            dwu = torch.zeros_like(wu)
            gemm_grouped(2, pk.offsets, C, dug, 2 * n, 1, x2, d, 1, dwu, d, 2 * n, d, P, b_rows=pk.tok_of_slot,
                         c_rows=ug_rows, c_rows_gstride=2 * n)
        if ctx.needs_input_grad[3]:
            # rows dn_rows[c, m] of dW_d: sum over the slots of z[s, m] w_s dout[tok s]
            dwd = torch.zeros_like(wdn)
            gemm_grouped(2, pk.offsets, C, z, n, 1, do, d, 1, dwd, d, n, d, P, b_rows=pk.tok_of_slot, b_scale=scale,
                         c_rows=dn_rows, c_rows_gstride=n)
        return dx, dw, dwu, dwd, None, None, None, None


_POOL_TABLES: dict = {}


def pool_tables(C: int, n: int, device):
    """(ug_rows [C, 2n], dn_rows [C, n]) int32: cluster c's up / gate rows of wug [2F, d] (rows
    [up F ; gate F], F = C n) and its neuron rows of wd^T [F, d]."""
    key = (C, n, str(device))
    if key not in _POOL_TABLES:
        F_ = C * n
        up = (torch.arange(C) * n)[:, None] + torch.arange(n)[None, :]
        _POOL_TABLES[key] = (torch.cat([up, up + F_], 1).to(torch.int32).to(device), up.to(torch.int32).to(device))
    return _POOL_TABLES[key]


def _pair_weights(pk) -> torch.Tensor:
    """[T, k] pair weights read back from a pack (0 for a dropped pair)."""
    sop = pk.slot_of_pair.long()
    w = torch.where(sop >= 0, pk.w_of_slot[sop.clamp_min(0)], torch.zeros((), device=sop.device))
    return w.view(-1, pk.k)


def grouped_pool_swiglu(x, ids, w, wug_t, wd_t, n: int, resid=None, pk=None):
    """The grouped pool in fp32 over routes ids / w [T, k] (-1 = no pair) or a ready pack: wug_t
    [2F, d] rows [up F ; gate F], wd_t [d, F], cluster c = neurons [c n, (c+1) n) (the banked
    core's (bank, slab) clusters in its pool-weight layout).  Route weights carry no gradient."""
    shape = x.shape
    d = shape[-1]
    F_ = wug_t.shape[0] // 2
    C = F_ // n
    if pk is None:
        pk = H.pack_index(ids.reshape(-1, ids.shape[-1]), C, w.reshape(-1, ids.shape[-1]))
    ug_rows, dn_rows = pool_tables(C, n, x.device)
    out = GroupedPoolFn.apply(_c32(x).reshape(-1, d), _pair_weights(pk), wug_t, wd_t.t(), pk, ug_rows, dn_rows,
                              n).view(shape)
    return out if resid is None else out + resid.to(F32)


def routed_cluster_pool_swiglu(x, wr, wug, wd, k: int, resid=None):
    """Routed cluster pool in fp32: logits x Wr^T (fp32 GEMM), top-k (value desc, index asc) on
    the HIP top-k, softmax over the selected logits (differentiable), the grouped pool, + resid.
    wug [2F, d] rows [up ; gate], wd [d, F].  Returns (out, ids int32, weights)."""
    shape = x.shape
    d = shape[-1]
    x2 = _c32(x).reshape(-1, d)
    C = wr.shape[0]
    n = wd.shape[1] // C
    logits = LinearFn.apply(x2, wr)
    ids, _ = H.route_topk(logits.detach(), k)
    w = logits.gather(1, ids.long()).softmax(dim=-1)
    pk = H.pack_index(ids, C, w.detach())
    ug_rows, dn_rows = pool_tables(C, n, x.device)
    out = GroupedPoolFn.apply(x2, w, wug, wd.t(), pk, ug_rows, dn_rows, n).view(shape)
    if resid is not None:
        out = out + resid.to(F32)
    return out, ids, w.detach()


# ----------------------------------------------------------------------------- keyed products (macro)

class GroupedLinearFn(torch.autograd.Function):
    """y[t] = x[t] w[key(t)] with the rows grouped by key in a PackIndex (hip_ops.group_rows):
    w [G, K_in, N_out].  Forward and input gradient run one group per weight block (rows gathered
    and scattered by slot); the weight gradient is one reduction group per key (its rows in slot
    order, so repeats are bitwise equal; keys without rows get zero)."""

    @staticmethod
    def forward(ctx, x, w, pk):
        _lib.require_device_tensors("grouped_linear_f32", x, w)
        x2 = _c32(x)
        G, Kin, Nout = w.shape
        wc = _c32(w)
        T = x2.shape[0]
        y = torch.zeros((T, Nout), dtype=F32, device=x2.device)  # rows of dropped keys stay 0
        gemm_grouped(1, pk.offsets, G, x2, Kin, 0, wc, Nout, 1, y, Nout, pk.tok_of_slot.numel(), Nout, Kin,
                     a_rows=pk.tok_of_slot, b_gstride=Kin * Nout, c_rows=pk.tok_of_slot)
        ctx.save_for_backward(x2, wc)
        ctx.pk = pk
        ctx.w_dtype = w.dtype
        return y

    @staticmethod
    def backward(ctx, dy):
        x2, wc = ctx.saved_tensors
        pk = ctx.pk
        G, Kin, Nout = wc.shape
        T = x2.shape[0]
        P = pk.tok_of_slot.numel()
        dy2 = _c32(dy)
        dx = dw = None
        if ctx.needs_input_grad[0]:
            dx = torch.zeros((T, Kin), dtype=F32, device=x2.device)
            gemm_grouped(1, pk.offsets, G, dy2, Nout, 0, wc, Nout, 0, dx, Kin, P, Kin, Nout, a_rows=pk.tok_of_slot,
                         b_gstride=Kin * Nout, c_rows=pk.tok_of_slot)
        if ctx.needs_input_grad[1]:
            dw = torch.empty_like(wc)
            gemm_grouped(2, pk.offsets, G, x2, Kin, 1, dy2, Nout, 1, dw, Nout, Kin, Nout, P, a_rows=pk.tok_of_slot,
                         b_rows=pk.tok_of_slot, c_gstride=Kin * Nout)
            dw = dw.to(ctx.w_dtype)
        return dx, dw, None


def grouped_linear(x, w, pk):
    return GroupedLinearFn.apply(x, w, pk)


# ----------------------------------------------------------------------------- router

def router(h0, w1r, b1r, w2r, b2r, w1d, b1d, w2d, b2d, pass_bias, depth_values, *, inv_t: float = 1.0,
           fixed_recipe=None, fixed_depth=None) -> dict:
    """Router.forward's recipe / depth fields (rte/routing.py:80-188) in fp32: the MLP products on
    the fp32 GEMM, the per-sample head arithmetic as device glue; argmax takes the first maximal
    index, as torch's does."""
    import torch.nn.functional as Fn

    pooled = _c32(h0).mean(dim=1)

    def mlp(w1, b1, w2, b2):
        return linear(Fn.silu(linear(pooled, w1, b1)), w2, b2)

    rl = mlp(w1r, b1r, w2r, b2r) * inv_t
    dl = mlp(w1d, b1d, w2d, b2d) * inv_t
    rlp = rl.unsqueeze(1) + pass_bias.to(F32).unsqueeze(0) * inv_t
    rp, dp, rpp = rl.softmax(dim=-1), dl.softmax(dim=-1), rlp.softmax(dim=-1)
    B = pooled.shape[0]
    if fixed_recipe is None:
        rid, ridp = rp.argmax(dim=-1), rpp.argmax(dim=-1)
    else:
        rid = torch.full((B,), int(fixed_recipe), dtype=torch.long, device=pooled.device)
        ridp = torch.full((B, pass_bias.shape[0]), int(fixed_recipe), dtype=torch.long, device=pooled.device)
    did = (dp.argmax(dim=-1) if fixed_depth is None
           else torch.full((B,), int(fixed_depth), dtype=torch.long, device=pooled.device))

    def st(ids, probs):
        return Fn.one_hot(ids, probs.shape[-1]).to(probs.dtype) + probs - probs.detach()

    ent = lambda p: -(p.clamp_min(1e-9).log() * p).sum(dim=-1)  # noqa: E731
    re, de = ent(rp), ent(dp)
    dv = depth_values.to(pooled.device)
    return {"recipe_logits": rl, "recipe_probs": rp, "recipe_id": rid, "recipe_onehot_st": st(rid, rp),
            "depth_logits": dl, "depth_probs": dp, "depth_id": did, "depth": dv[did],
            "depth_onehot_st": st(did, dp), "recipe_entropy": re, "depth_entropy": de, "router_entropy": re + de,
            "expected_depth": (dp * dv.to(dp.dtype)).sum(dim=-1), "recipe_logits_by_pass": rlp,
            "recipe_probs_by_pass": rpp, "recipe_id_by_pass": ridp, "recipe_onehot_st_by_pass": st(ridp, rpp)}


# ----------------------------------------------------------------------------- heads

def lm_head_ce(hidden, w, targets):
    """(logits fp32 [..., V], per-token CE) of hidden w^T on the fp32 GEMM and the HIP CE kernel."""
    logits = LinearFn.apply(hidden, w)
    return logits, H.cross_entropy(logits, targets)


class ShortlistLogitsFn(torch.autograd.Function):
    """logits[t, l] = hidden[t] . wsel[t, l] (wsel [T, L, d] the shortlisted vocabulary rows), one
    batched fp32 product per token."""

    @staticmethod
    def forward(ctx, hidden, wsel):
        h = _c32(hidden)
        ws = _c32(wsel)
        T, L, d = ws.shape
        out = torch.empty((T, L), dtype=F32, device=h.device)
        gemm(ws, d, 0, h, d, 0, out, 1, L, 1, d, batch=(T, 1), sA=(L * d, 0), sB=(d, 0), sC=(L, 0))
        ctx.save_for_backward(h, ws)
        return out

    @staticmethod
    def backward(ctx, g):
        h, ws = ctx.saved_tensors
        T, L, d = ws.shape
        g = _c32(g)
        dh = torch.empty_like(h)
        dws = torch.empty_like(ws)
        gemm(g, L, 0, ws, d, 1, dh, d, 1, d, L, batch=(T, 1), sA=(L, 0), sB=(L * d, 0), sC=(d, 0))   # g W
        gemm(g, 1, 1, h, d, 1, dws, d, L, d, 1, batch=(T, 1), sA=(L, 0), sB=(d, 0), sC=(L * d, 0))   # g^T h
        return dh, dws


def shortlist_ce(hidden, w, shortlist):
    """(logits [B, S, L], per-token CE with the target at position 0) over the shortlisted rows
    (rte/output.py:112-136): rows gathered with the deterministic embedding gather."""
    B, S, d = hidden.shape
    L = shortlist.shape[-1]
    wsel = H.embedding(w, shortlist.reshape(B * S, L))
    logits = ShortlistLogitsFn.apply(hidden.reshape(B * S, d), wsel).view(B, S, L)
    tgt = torch.zeros((B, S), dtype=torch.long, device=hidden.device)
    return logits, H.cross_entropy(logits, tgt)
