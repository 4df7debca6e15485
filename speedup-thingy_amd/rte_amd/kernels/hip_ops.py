"""Autograd operators over librte_hip (the gfx950 HIP kernels).

Every operator here launches hand-written HIP kernels through the C ABI on the
current torch stream; torch is only used to allocate outputs/workspaces.  They
raise RuntimeError when the library or a ROCm device is missing: there is no
CPU or reference-math fallback on this path.

Precision contract (mirrors bf16 autocast in the reference, rte/training.py:356-363):
activations and GEMM operands are bf16, accumulation is fp32, master weights and
their gradients are fp32, the residual stream is fp32.
"""

from __future__ import annotations

import ctypes
import math
import threading
from contextlib import contextmanager
from dataclasses import dataclass

import torch

from rte_amd import _lib
from rte_amd._lib import call, ptr

BF16 = torch.bfloat16
F32 = torch.float32

_PRECISION = threading.local()


def fp32_active() -> bool:
    """True inside a fp32_precision() block: the model's operators then compute in fp32 on the
    fp32 kernels (rte_amd.kernels.f32_ops) instead of taking bf16 GEMM operands."""
    return getattr(_PRECISION, "fp32", False)


@contextmanager
def fp32_precision(enabled: bool = True):
    """training.precision = "fp32" (the reference's default, rte/config.py:118): every operator
    called inside runs its products with fp32 operands and accumulation."""
    prev = fp32_active()
    _PRECISION.fp32 = bool(enabled)
    try:
        yield
    finally:
        _PRECISION.fp32 = prev


def _f32():
    from rte_amd.kernels import f32_ops

    return f32_ops


def _s() -> int:
    return _lib.stream_ptr()


_WS: dict[tuple[int, int], torch.Tensor] = {}


def workspace(nbytes: int, device: torch.device) -> tuple[int, int]:
    """(pointer, bytes) of a cached scratch buffer of at least nbytes, one per (device, stream).

    Launches on one stream are ordered, so they may share that stream's buffer; work issued
    on another stream gets its own."""
    if nbytes <= 0:
        return 0, 0
    idx = device.index if device.index is not None else torch.cuda.current_device()
    key = (idx, torch.cuda.current_stream(idx).cuda_stream)
    buf = _WS.get(key)
    if buf is None or buf.numel() < nbytes:
        buf = torch.empty(((nbytes + 255) // 256) * 256, dtype=torch.uint8, device=device)
        _WS[key] = buf
    return buf.data_ptr(), buf.numel()


def _gemm_ws(M: int, N: int, K: int, device) -> tuple[int, int]:
    return workspace(_lib.load().rte_gemm_workspace_bytes(M, N, K), device)


def _gemm_ws_max(device, *shapes) -> tuple[int, int]:
    """One split-K workspace for several GEMMs run in turn on one stream."""
    lib = _lib.load()
    return workspace(max(lib.rte_gemm_workspace_bytes(M, N, K) for M, N, K in shapes), device)


_BF16_CACHE: dict = {}
_BF16_CACHE_ON = [False]


def bf16_cache_begin() -> None:
    """Start of a training step: from here on the bf16 copy of a parameter (or of a view of one,
    e.g. a transposed weight) is made once and shared by every use until the next call.  The
    step's parameters must not change in place before the next call (the optimizer step comes
    last); call it at the start of every step, eager or captured."""
    _BF16_CACHE.clear()
    _BF16_CACHE_ON[0] = True


def bf16_cache_end() -> None:
    _BF16_CACHE.clear()
    _BF16_CACHE_ON[0] = False


_BF16_REC: list = [None]  # Bf16Prefetch recording the step's parameter casts


class Bf16Prefetch:
    """A training step's bf16 weight copies in one launch (rte_cast_many) instead of one cast
    per weight at first use.  The first step (eager) runs with the per-use casts and records
    which parameter views they cast on which stream; every later step makes all of them at
    begin(), into buffers kept for the session, and files them in the per-step cache under
    the keys the uses look up.  Views other than contiguous ones and 2-D transposes are left to
    the per-use path.  Use begin() / end() in place of bf16_cache_begin / bf16_cache_end."""

    def __init__(self, enabled: bool = True):
        self.enabled = enabled
        self.entries = None   # [(param, shape, stride, offset, stream or None = the step's stream)]
        self.tables = None

    def begin(self) -> None:
        bf16_cache_begin()
        _BF16_REC[0] = None
        if not self.enabled:
            return
        if self.entries is None:
            self._main = _lib.stream_ptr()
            self._rec = []
            _BF16_REC[0] = self
        elif self.entries:
            self._run()

    def end(self) -> None:
        if _BF16_REC[0] is self:
            _BF16_REC[0] = None
            if not torch.cuda.is_current_stream_capturing():
                self._build(self._rec)
            self._rec = []
        bf16_cache_end()

    def record(self, x: torch.Tensor) -> None:
        base = x._base if x._base is not None else x
        st = _lib.stream_ptr()
        self._rec.append((base, tuple(x.shape), tuple(x.stride()), x.storage_offset(),
                          None if st == self._main else torch.cuda.current_stream()))

    def _build(self, rec) -> None:
        seen, jobs, entries, outs = {}, [], [], []
        nblk = 0
        lib = _lib.load()
        for base, shape, stride, off, stream in rec:
            ident = (id(base), shape, stride, off)
            if ident not in seen:
                view = base.as_strided(shape, stride, off)
                if view.is_contiguous():
                    kind, rows, cols, ld = 0, 1, view.numel(), 0
                elif len(shape) == 2 and stride == (1, shape[0]):
                    kind, rows, cols, ld = 1, shape[0], shape[1], shape[0]
                else:
                    continue
                if view.numel() == 0:
                    continue
                dst = torch.empty(shape, dtype=BF16, device=base.device)
                nb = lib.rte_cast_many_blocks(kind, rows, cols)
                seen[ident] = len(outs)
                jobs.append([view.data_ptr(), dst.data_ptr(), rows, cols, ld, kind, nblk, 0])
                outs.append(dst)
                nblk += nb
            entries.append((base, shape, stride, off, stream, seen[ident]))
        self.entries = entries
        if not jobs:
            return
        dev = outs[0].device
        blk = torch.cat([torch.full((lib.rte_cast_many_blocks(j[5], j[2], j[3]),), i, dtype=torch.int32)
                         for i, j in enumerate(jobs)])
        self.tables = (torch.tensor(jobs, dtype=torch.int64).to(dev), blk.to(dev), nblk, outs,
                       [(e[0], e[0].data_ptr()) for e in entries])

    def _run(self) -> None:
        jobs, blk, nblk, outs, ptrs = self.tables
        if any(b.data_ptr() != pv for b, pv in ptrs):  # parameters moved: record again next step
            self.entries, self.tables = None, None
            return
        call("rte_cast_many", ptr(jobs), ptr(blk), nblk, _s())
        main = _lib.stream_ptr()
        for base, shape, stride, off, stream, j in self.entries:
            view = base.as_strided(shape, stride, off)
            st = main if stream is None else stream.cuda_stream
            _BF16_CACHE[(view.data_ptr(), shape, stride, view._version, st)] = outs[j]


def _cache_key(x: torch.Tensor):
    """Parameters (and views of them) only; keyed by the current stream as well, so a copy made
    on one stream is never read unsynchronised from another."""
    base = x._base if x._base is not None else x
    if not isinstance(base, torch.nn.Parameter):
        return None
    return (x.data_ptr(), tuple(x.shape), tuple(x.stride()), x._version, _lib.stream_ptr())


def _attach_bf16(x: torch.Tensor, xb: torch.Tensor) -> None:
    """Remember xb, the bf16 values of fp32 x written by the same kernel on the current stream,
    so cast_bf16 of x (or of a whole contiguous view of it) needs no cast launch."""
    x._rte_bf16 = (xb, x._version, _lib.stream_ptr())


def _bf16_companion(x: torch.Tensor):
    base = x._base if x._base is not None else x
    comp = getattr(base, "_rte_bf16", None)
    if comp is None:
        return None
    xb, version, stream = comp
    if (base._version != version or stream != _lib.stream_ptr() or not x.is_contiguous()
            or x.data_ptr() != base.data_ptr() or x.numel() != xb.numel()):
        return None
    return xb.view(x.shape)


def cast_bf16(x: torch.Tensor) -> torch.Tensor:
    """fp32 -> bf16 (round to nearest even) with the HIP cast kernel; parameters hit the
    per-step cache while one is open (bf16_cache_begin), and tensors whose producing kernel also
    wrote their bf16 values (_attach_bf16) return those."""
    if x.dtype == BF16:
        return x.contiguous()
    _lib.require_device_tensors("cast_bf16", x)
    comp = _bf16_companion(x)
    if comp is not None:
        return comp
    key = _cache_key(x) if _BF16_CACHE_ON[0] else None
    if key is not None:
        hit = _BF16_CACHE.get(key)
        if hit is not None:
            return hit
        if _BF16_REC[0] is not None:
            _BF16_REC[0].record(x)
    xc = x.contiguous().to(F32)
    y = torch.empty(xc.shape, dtype=BF16, device=xc.device)
    call("rte_cast_f32_bf16", ptr(xc), xc.numel(), ptr(y), _s())
    if key is not None:
        _BF16_CACHE[key] = y
    return y


# ----------------------------------------------------------------------------- GEMM

def gemm(
    a: torch.Tensor,
    b: torch.Tensor,
    *,
    a_t: bool = False,
    b_t: bool = False,
    out_f32: bool = False,
    alpha: float = 1.0,
    resid: torch.Tensor | None = None,
    out: torch.Tensor | None = None,
    beta: float = 0.0,
    b_rows: torch.Tensor | None = None,
) -> torch.Tensor:
    """C[m, n] = alpha * sum_k A(m, k) B(n, k) (+ beta C) (+ resid).

    a: [M, K] (a_t False) or [K, M] (a_t True); b: [N, K] (b_t False) or [K, N] (b_t True).
    b_rows (int32, optional): B's memory rows are b_rows[n] (b_t False) or b_rows[k] (b_t True),
    so b may hold more rows than the problem reads.  bf16 operands, fp32 accumulation.
    """
    _lib.require_device_tensors("gemm", a, b, resid, out, b_rows)
    if a.dtype != BF16 or b.dtype != BF16:
        raise TypeError("gemm operands must be bfloat16")
    a = a.contiguous()
    b = b.contiguous()
    M = a.shape[1] if a_t else a.shape[0]
    K = a.shape[0] if a_t else a.shape[1]
    N = b.shape[1] if b_t else b.shape[0]
    Kb = b.shape[0] if b_t else b.shape[1]
    if b_rows is not None:
        b_rows = b_rows.reshape(-1).contiguous().to(torch.int32)
        if b_t:
            Kb = b_rows.numel()
        else:
            N = b_rows.numel()
    if K != Kb:
        raise ValueError(f"gemm: reduction sizes differ ({K} vs {Kb})")
    if out is None:
        out = torch.empty((M, N), dtype=F32 if out_f32 else BF16, device=a.device)
    if resid is not None:
        resid = resid.contiguous().to(F32)
    wsp, wsn = _gemm_ws(M, N, K, a.device)
    call(
        "rte_gemm_bf16",
        ptr(a), a.shape[1], int(a_t), None,
        ptr(b), b.shape[1], int(b_t), ptr(b_rows),
        ptr(out), out.shape[1], int(out.dtype == F32), M, N, K,
        float(alpha), float(beta), ptr(resid), 0 if resid is None else resid.shape[1], wsp, wsn, _s(),
    )
    return out


def _token_major(y: torch.Tensor) -> bool:
    """y [B, H, S, hd] is a view of token-major [B, S, H, hd] rows (what the attention writes)."""
    B, H, S, hd = y.shape
    sb, sh, ss, sd = y.stride()
    return sd == 1 and sh == hd and ss == H * hd and (B == 1 or sb == S * ss)


def _attn_layout(y: torch.Tensor) -> tuple[list[int], int, int]:
    """Layout descriptor reading a [B, H, S, hd] tensor as rows t = b*S + s, cols c = h*hd + dim:
    plain rows for token-major memory, else a split of rows by S and columns by hd (powers of two)."""
    B, H, S, hd = y.shape
    sb, sh, ss, sd = y.stride()
    if sd != 1:
        raise ValueError("attention tensor needs a unit innermost stride")
    if _token_major(y):
        return [H * hd, 0, 0, 0, 0], B * S, H * hd
    return [ss, S, sb, hd, sh], B * S, H * hd


# ----------------------------------------------------------------------------- RMSNorm

class RMSNormFn(torch.autograd.Function):
    """bf16(x * rsqrt(mean(x^2) + eps) * w) for an fp32 residual stream (rte/kernels/reference.py:9-17)."""

    @staticmethod
    def forward(ctx, x: torch.Tensor, w: torch.Tensor, eps: float):
        _lib.require_device_tensors("rmsnorm", x, w)
        shape = x.shape
        x2 = x.reshape(-1, shape[-1]).contiguous().to(F32)
        w32 = w.contiguous().to(F32)
        T, d = x2.shape
        out = torch.empty((T, d), dtype=BF16, device=x.device)
        rstd = torch.empty((T,), dtype=F32, device=x.device)
        call("rte_rmsnorm_fwd", ptr(x2), ptr(w32), T, d, float(eps), ptr(out), ptr(rstd), _s())
        ctx.save_for_backward(x2, w32, rstd)
        ctx.shape = shape
        ctx.w_dtype = w.dtype
        return out.view(*shape[:-1], d)

    @staticmethod
    def backward(ctx, dy: torch.Tensor):
        x2, w32, rstd = ctx.saved_tensors
        T, d = x2.shape
        dy = dy.reshape(T, d).contiguous().to(BF16)
        dx = torch.empty((T, d), dtype=F32, device=x2.device)
        dw = torch.empty((d,), dtype=F32, device=x2.device)
        nbytes = _lib.load().rte_rmsnorm_bwd_workspace_bytes(T, d)
        ws = torch.empty((max(1, nbytes // 4),), dtype=F32, device=x2.device)
        dxb = torch.empty((T, d), dtype=BF16, device=x2.device)
        call("rte_rmsnorm_bwd", ptr(dy), ptr(x2), ptr(w32), ptr(rstd), None, T, d, ptr(dx), ptr(dxb), ptr(dw), 0,
             ptr(ws), nbytes, _s())
        _attach_bf16(dx, dxb)  # the next layer's GEMMs read dx in bf16
        return dx.view(ctx.shape), dw.to(ctx.w_dtype), None


def rmsnorm(x: torch.Tensor, w: torch.Tensor, eps: float = 1e-5) -> torch.Tensor:
    if fp32_active():
        return FusedRMSNormFn.apply(x.float(), w, None, eps)[0]
    return RMSNormFn.apply(x, w, eps)


class RMSNormResidFn(torch.autograd.Function):
    """(rmsnorm(x) * w, x): the norm together with its input passed on as the residual branch,
    so the backward adds the residual's gradient inside the norm-backward kernel (its dres
    input) instead of autograd adding two [T, d] gradients of x."""

    @staticmethod
    def forward(ctx, x: torch.Tensor, w: torch.Tensor, eps: float):
        _lib.require_device_tensors("rmsnorm", x, w)
        shape = x.shape
        x2 = x.reshape(-1, shape[-1]).contiguous().to(F32)
        w32 = w.contiguous().to(F32)
        T, d = x2.shape
        out = torch.empty((T, d), dtype=BF16, device=x.device)
        rstd = torch.empty((T,), dtype=F32, device=x.device)
        call("rte_rmsnorm_fwd", ptr(x2), ptr(w32), T, d, float(eps), ptr(out), ptr(rstd), _s())
        ctx.save_for_backward(x2, w32, rstd)
        ctx.shape = shape
        ctx.w_dtype = w.dtype
        ctx.x_dtype = x.dtype
        ctx.set_materialize_grads(False)
        return out.view(*shape[:-1], d), x2.view(shape)

    @staticmethod
    def backward(ctx, dy: torch.Tensor | None, dres: torch.Tensor | None):
        x2, w32, rstd = ctx.saved_tensors
        T, d = x2.shape
        if dy is None:
            return (None if dres is None else dres.to(ctx.x_dtype)), None, None
        dy = dy.reshape(T, d).contiguous().to(BF16)
        r = None if dres is None else dres.reshape(T, d).contiguous().to(F32)
        dx = torch.empty((T, d), dtype=F32, device=x2.device)
        dw = torch.empty((d,), dtype=F32, device=x2.device)
        nbytes = _lib.load().rte_rmsnorm_bwd_workspace_bytes(T, d)
        ws = torch.empty((max(1, nbytes // 4),), dtype=F32, device=x2.device)
        dxb = torch.empty((T, d), dtype=BF16, device=x2.device) if ctx.x_dtype == F32 else None
        call("rte_rmsnorm_bwd", ptr(dy), ptr(x2), ptr(w32), ptr(rstd), ptr(r), T, d, ptr(dx), ptr(dxb), ptr(dw), 0,
             ptr(ws), nbytes, _s())
        if dxb is not None:
            _attach_bf16(dx, dxb)  # the previous layer's GEMMs read dx in bf16
        return dx.view(ctx.shape).to(ctx.x_dtype), dw.to(ctx.w_dtype), None


def rmsnorm_resid(x: torch.Tensor, w: torch.Tensor, eps: float = 1e-5) -> tuple[torch.Tensor, torch.Tensor]:
    """(bf16 rmsnorm(x) * w, fp32 x for the residual add): one gradient for x."""
    if fp32_active():
        x = x.float()
        return FusedRMSNormFn.apply(x, w, None, eps)[0], x
    return RMSNormResidFn.apply(x, w, eps)


class AxpyNormFn(torch.autograd.Function):
    """x = a + c * b (c a scalar tensor, None = 1; b optional; samples whose mask is False keep
    their `keep` rows) and, when w is given, n = bf16(rmsnorm(x) * w * (1 + gamma) + beta), in
    one launch; the backward is one row kernel plus a fixed-order column sum that yields the
    gradients of w, gamma, beta and c together (rte/layers.py:826-845)."""

    @staticmethod
    def forward(ctx, a, b, c, keep, mask, w, gamma, beta, eps):
        _lib.require_device_tensors("axpy_norm", a, b, c, keep, mask, w, gamma, beta)
        shape = a.shape
        d = shape[-1]
        T = a.numel() // d
        S = 1
        if mask is not None:
            if keep is None or mask.numel() == 0 or T % mask.numel() != 0:
                raise ValueError(f"axpy_norm: a mask of {mask.numel()} samples needs keep rows and divides {T} rows")
            S = T // mask.numel()
        a2 = a.reshape(T, d).contiguous().to(F32)
        b2 = None if b is None else b.reshape(T, d).contiguous().to(F32)
        k2 = None if keep is None else keep.reshape(T, d).contiguous().to(F32)
        m = None if mask is None else mask.reshape(-1).contiguous().to(torch.bool)
        cc = None if c is None else c.reshape(()).contiguous().to(F32)
        vecs = [None if v is None else v.reshape(d).contiguous().to(F32) for v in (w, gamma, beta)]
        dev = a.device
        x = torch.empty((T, d), dtype=F32, device=dev)
        n = torch.empty((T, d) if w is not None else (0,), dtype=BF16, device=dev)
        rstd = torch.empty((T,) if w is not None else (0,), dtype=F32, device=dev)
        call("rte_axpy_norm_fwd", ptr(a2), ptr(b2), ptr(cc), ptr(k2), ptr(m), S, T, d, ptr(vecs[0]), ptr(vecs[1]),
             ptr(vecs[2]), float(eps), ptr(x), ptr(n) if w is not None else None,
             ptr(rstd) if w is not None else None, _s())
        ctx.save_for_backward(x, rstd, vecs[0], vecs[1], b2, cc, m)
        ctx.meta = (shape, T, d, S, w is not None, c.shape if c is not None else None)
        ctx.set_materialize_grads(False)  # an unused output's gradient stays None (no zero fill)
        if w is None:
            ctx.mark_non_differentiable(n)
        return x.view(shape), (n.view(shape) if w is not None else n)

    @staticmethod
    def backward(ctx, dx_ext, dn):
        x, rstd, w, gamma, b2, cc, m = ctx.saved_tensors
        shape, T, d, S, has_norm, c_shape = ctx.meta
        if dx_ext is None and (dn is None or not has_norm):
            return (None,) * 9
        dev = x.device
        dxe = None if dx_ext is None else dx_ext.reshape(T, d).contiguous().to(F32)
        dnb = None if (dn is None or not has_norm) else dn.reshape(T, d).contiguous().to(BF16)
        nia = ctx.needs_input_grad
        da = torch.empty((T, d), dtype=F32, device=dev) if nia[0] else None
        db = torch.empty((T, d), dtype=F32, device=dev) if nia[1] else None
        dk = torch.empty((T, d), dtype=F32, device=dev) if nia[3] else None
        dparams = torch.empty((3 * d + 1,), dtype=F32, device=dev)
        ws, nb = workspace(_lib.load().rte_axpy_norm_bwd_workspace_bytes(T, d), dev)
        call("rte_axpy_norm_bwd", ptr(dnb), ptr(dxe), ptr(x) if has_norm else None,
             ptr(rstd) if has_norm else None, ptr(w), ptr(gamma), ptr(b2), ptr(cc), ptr(m), S, T, d, ptr(da),
             ptr(db), ptr(dk), ptr(dparams), ws, nb, _s())
        dc = dparams[3 * d].reshape(c_shape) if (nia[2] and c_shape is not None) else None
        return (None if da is None else da.view(shape), None if db is None else db.view(shape), dc,
                None if dk is None else dk.view(shape), None,
                dparams[:d] if nia[5] else None, dparams[d:2 * d] if nia[6] else None,
                dparams[2 * d:3 * d] if nia[7] else None, None)


def _axpy_norm_f32(a, b, c, w, gamma, beta, eps, keep, mask):
    """fp32 composite of axpy_norm: x = a + c b (masked samples keep `keep`), n = rmsnorm(x) w
    (1 + gamma) + beta on the fp32 norm kernel."""
    x = a.float()
    if b is not None:
        x = x + (b.float() if c is None else c.float() * b.float())
    if mask is not None:
        m = mask.reshape(-1, *([1] * (x.dim() - 1))).to(torch.bool)
        x = torch.where(m, x, keep.float())
    if w is None:
        return x, None
    n = FusedRMSNormFn.apply(x, w, None, eps)[0]
    if gamma is not None:
        n = n * (1.0 + gamma.float())
    if beta is not None:
        n = n + beta.float()
    return x, n


def axpy_norm(a, b, c, w, gamma=None, beta=None, eps: float = 1e-5, *, keep=None, mask=None):
    """(x, n): x = a + c b (fp32), n = bf16(rmsnorm(x) w (1 + gamma) + beta)."""
    if fp32_active():
        return _axpy_norm_f32(a, b, c, w, gamma, beta, eps, keep, mask)
    return AxpyNormFn.apply(a, b, c, keep, mask, w, gamma, beta, eps)


def axpy(a, b, c, *, keep=None, mask=None):
    """x = a + c b (fp32); with mask [B], samples whose mask is False take keep's rows."""
    if fp32_active():
        return _axpy_norm_f32(a, b, c, None, None, None, 0.0, keep, mask)[0]
    return AxpyNormFn.apply(a, b, c, keep, mask, None, None, None, 0.0)[0]


def _check_rope_tables(cos: torch.Tensor, sin: torch.Tensor, S: int, hd: int) -> None:
    """The kernels read cos / sin rows 0..S-1 of width hd: refuse shorter tables (a sequence
    longer than the rotary table) before any launch, as the reference's broadcast fails."""
    if cos.ndim != 2 or cos.shape[0] < S or cos.shape[1] != hd or sin.shape != cos.shape:
        raise ValueError(f"RoPE tables of shape {tuple(cos.shape)} / {tuple(sin.shape)} do not cover "
                         f"seq_len {S} x head_dim {hd}")


# ----------------------------------------------------------------------------- fused QKV + RoPE

class QKVRopeFn(torch.autograd.Function):
    """q, k, v = split(x @ Wqkv^T) with interleaved RoPE on q, k, written as [B, H, S, hd]."""

    @staticmethod
    def forward(ctx, x: torch.Tensor, w: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor, n_heads: int):
        B, S, d = x.shape
        hd = d // n_heads
        _check_rope_tables(cos, sin, S, hd)
        _lib.require_device_tensors("qkv_rope", x, w, cos, sin)
        if w.shape != (3 * d, d):
            raise ValueError(f"wqkv must be [3d, d], got {tuple(w.shape)}")
        xb = x.contiguous().to(BF16)
        wb = cast_bf16(w)
        cos = cos[:S].contiguous().to(F32)
        sin = sin[:S].contiguous().to(F32)
        q = torch.empty((B, n_heads, S, hd), dtype=BF16, device=x.device)
        k = torch.empty_like(q)
        v = torch.empty_like(q)
        wsp, wsn = _gemm_ws(B * S, 3 * n_heads * hd, n_heads * hd, x.device)
        call("rte_qkv_rope_fwd", ptr(xb), ptr(wb), ptr(cos), ptr(sin), B, S, n_heads, hd, ptr(q), ptr(k),
             ptr(v), wsp, wsn, _s())
        ctx.save_for_backward(xb, wb, cos, sin)
        ctx.dims = (B, S, n_heads, hd)
        ctx.w_dtype = w.dtype
        return q, k, v

    @staticmethod
    def backward(ctx, dq, dk, dv):
        xb, wb, cos, sin = ctx.saved_tensors
        B, S, H, hd = ctx.dims
        d = H * hd
        grads = []
        for g in (dq, dk, dv):
            if g is None:
                g = torch.zeros((B, H, S, hd), dtype=BF16, device=xb.device)
            g = g.to(BF16)
            if g.stride(-1) != 1:
                g = g.contiguous()
            grads.append(g)
        strides = [torch.tensor(g.stride(), dtype=torch.int64) for g in grads]
        dqkv = torch.empty((B * S, 3 * d), dtype=BF16, device=xb.device)
        dx = torch.empty((B * S, d), dtype=BF16, device=xb.device)
        dw = torch.empty((3 * d, d), dtype=F32, device=xb.device)
        wsp, wsn = _gemm_ws_max(xb.device, (3 * d, d, B * S), (B * S, d, 3 * d))
        call("rte_qkv_rope_bwd", ptr(grads[0]), strides[0].data_ptr(), ptr(grads[1]), strides[1].data_ptr(),
             ptr(grads[2]), strides[2].data_ptr(), ptr(xb), ptr(wb), ptr(cos), ptr(sin), B, S, H, hd,
             ptr(dqkv), ptr(dx), ptr(dw), wsp, wsn, _s())
        return dx.view(B, S, d), dw.to(ctx.w_dtype), None, None, None


def qkv_rope(x, w, cos, sin, n_heads):
    return QKVRopeFn.apply(x, w, cos, sin, n_heads)


# ----------------------------------------------------------------------------- attention output projection

class SharedWGrad:
    """Gradient of one weight used by several calls of one forward (the recursive passes of a
    banked core): every call's backward hands over its input rows X_t and output-gradient rows
    dY_t, and the last one to arrive forms sum_t dY_t^T X_t as one GEMM over the concatenated
    rows (instead of one GEMM per call and autograd's adds); the other calls return no weight
    gradient.  The order of the rows is the order the backward calls arrive in, fixed for a
    given graph, so results repeat bitwise.  Every registered call must run its backward."""

    def __init__(self):
        self.uses = 0
        self.arrived = 0
        self.items: list[tuple[torch.Tensor, torch.Tensor]] = []

    def register(self) -> None:
        self.uses += 1

    def add(self, x2d: torch.Tensor | None, dy2d: torch.Tensor | None, transposed: bool):
        """Stores (x2d [T, K], dy2d [T, N]) (bf16; None for a call whose output got no gradient);
        returns the weight gradient fp32 ([N, K], or a transposed view of a contiguous [K, N] when
        `transposed`) once every call is in, else None."""
        self.arrived += 1
        if x2d is not None:
            self.items.append((x2d, dy2d))
        if self.arrived < self.uses:
            if self.arrived == 1:  # a backward that leaves some calls out would lose their part
                torch.autograd.Variable._execution_engine.queue_callback(self._check_drained)
            return None
        items, self.items, self.arrived = self.items, [], 0  # a second backward over the graph starts again
        if not items:
            return None
        xs = torch.cat([x for x, _ in items]) if len(items) > 1 else items[0][0]
        dys = torch.cat([dy for _, dy in items]) if len(items) > 1 else items[0][1]
        if transposed:
            return gemm(xs, dys, a_t=True, b_t=True, out_f32=True).t()
        return gemm(dys, xs, a_t=True, b_t=True, out_f32=True)

    def _check_drained(self) -> None:
        if self.arrived:
            n, self.arrived, self.items = self.arrived, 0, []
            raise RuntimeError(f"SharedWGrad: the backward reached {n} of the {self.uses} calls sharing a weight; "
                               "differentiate through every call of the forward")


class SharedGradAccum:
    """Weight gradients of several calls of one forward summed in place: the first backward call
    to arrive writes fresh buffers, every later one adds to them in its GEMM epilogue (in arrival
    order, fixed for a given graph), and the last returns them (the others return no weight
    gradient).  Every registered call must run its backward."""

    def __init__(self):
        self.uses = 0
        self.arrived = 0
        self.bufs = None

    def register(self) -> None:
        self.uses += 1

    def arrive(self, make):
        """-> (buffers, beta, last): make() allocates the buffers on the first arrival."""
        first = self.arrived == 0
        if first:
            self.bufs = make()
            if self.uses > 1:  # a backward that leaves some calls out would lose their part
                torch.autograd.Variable._execution_engine.queue_callback(self._check_drained)
        self.arrived += 1
        bufs = self.bufs
        last = self.arrived >= self.uses
        if last:
            self.arrived, self.bufs = 0, None  # a second backward over the graph starts again
        return bufs, (0.0 if first else 1.0), last

    def _check_drained(self) -> None:
        if self.arrived:
            n, self.arrived, self.bufs = self.arrived, 0, None
            raise RuntimeError(f"SharedGradAccum: the backward reached {n} of the {self.uses} calls sharing a "
                               "weight; differentiate through every call of the forward")


def _is_t_view(w: torch.Tensor) -> bool:
    """w is a 2-D transposed view of contiguous memory (its gradient is formed in that layout)."""
    return w.dim() == 2 and not w.is_contiguous() and w.t().is_contiguous()


class AttnOutProjFn(torch.autograd.Function):
    """out = resid + y @ Wo^T where y is the [B, H, S, hd] attention output (any strides)."""

    @staticmethod
    def forward(ctx, y: torch.Tensor, w: torch.Tensor, resid: torch.Tensor | None, wgrad: SharedWGrad | None = None):
        _lib.require_device_tensors("attn_out_proj", y, w, resid)
        yb = y.to(BF16)
        if yb.stride(-1) != 1:
            yb = yb.contiguous()
        B_, H_, S_, hd_ = yb.shape
        if not _token_major(yb) and (S_ & (S_ - 1) or hd_ & (hd_ - 1)):
            yb = yb.transpose(1, 2).contiguous().transpose(1, 2)  # the split layout needs powers of two
        layout, T, K = _attn_layout(yb)
        wb = cast_bf16(w)
        N = wb.shape[0]
        out = torch.empty((T, N), dtype=F32, device=y.device)
        r = None if resid is None else resid.reshape(T, N).contiguous().to(F32)
        L = torch.tensor(layout, dtype=torch.int64)
        Lw = torch.tensor([K, 0, 0, 0, 0], dtype=torch.int64)
        wsp, wsn = _gemm_ws(T, N, K, yb.device)
        call("rte_gemm_bf16_split", ptr(yb), L.data_ptr(), 0, ptr(wb), Lw.data_ptr(), 0, ptr(out), N, 1, T, N, K,
             1.0, 0.0, ptr(r), 0 if r is None else N, wsp, wsn, _s())
        ctx.save_for_backward(yb, wb)
        ctx.has_resid = resid is not None
        ctx.w_dtype = w.dtype
        ctx.w_t = _is_t_view(w)
        ctx.wgrad = wgrad if (wgrad is not None and ctx.needs_input_grad[1]) else None
        if ctx.wgrad is not None:
            ctx.wgrad.register()
        B, H, S, hd = y.shape
        return out.view(B, S, N)

    @staticmethod
    def backward(ctx, dout: torch.Tensor):
        yb, wb = ctx.saved_tensors
        B, H, S, hd = yb.shape
        T, K, N = B * S, H * hd, wb.shape[0]
        db = cast_bf16(dout.reshape(T, N))
        # dy = dout @ Wo    (B(n=c, k=o) = Wo[o][c]: layout T)
        dy = gemm(db, wb, b_t=True)
        # dWo[o, c] = sum_t dout[t, o] y[t, c]
        layout, _, _ = _attn_layout(yb)
        L = torch.tensor(layout, dtype=torch.int64)
        Ld = torch.tensor([N, 0, 0, 0, 0], dtype=torch.int64)
        dy4 = dy.view(B, S, H, hd).transpose(1, 2)
        dres = dout if ctx.has_resid else None
        if ctx.wgrad is not None:  # token-major rows of y (its memory order) for the shared gradient
            dw = ctx.wgrad.add(yb.transpose(1, 2).reshape(T, K), db, ctx.w_t)
            return dy4, (None if dw is None else dw.to(ctx.w_dtype)), dres, None
        if ctx.w_t:  # w is a transposed view: dW^T [K, N] = y^T dout, returned as its transpose
            dwt = torch.empty((K, N), dtype=F32, device=yb.device)
            wsp, wsn = _gemm_ws(K, N, T, yb.device)
            call("rte_gemm_bf16_split", ptr(yb), L.data_ptr(), 1, ptr(db), Ld.data_ptr(), 1, ptr(dwt), N, 1, K, N, T,
                 1.0, 0.0, None, 0, wsp, wsn, _s())
            dw = dwt.t()
        else:
            dw = torch.empty((N, K), dtype=F32, device=yb.device)
            wsp, wsn = _gemm_ws(N, K, T, yb.device)
            call("rte_gemm_bf16_split", ptr(db), Ld.data_ptr(), 1, ptr(yb), L.data_ptr(), 1, ptr(dw), K, 1, N, K, T,
                 1.0, 0.0, None, 0, wsp, wsn, _s())
        return dy4, dw.to(ctx.w_dtype), dres, None


def attn_out_proj(y, w, resid=None, wgrad: SharedWGrad | None = None):
    if fp32_active():
        return _f32().attn_out_proj(y, w, resid)
    return AttnOutProjFn.apply(y, w, resid, wgrad)


# ----------------------------------------------------------------------------- attention core

class AttentionFn(torch.autograd.Function):
    """Causal softmax attention, head_dim 32 / 64 / 128, softmax scale 1/sqrt(head_dim) (torch
    SDPA's default): out = head_scale[b, h] * softmax(q k^T scale, causal) v.  q, k, v [B, H, S, hd]
    (bf16 on the kernel); the output is a [B, H, S, hd] view of token-major [B, S, H, hd] memory, which the
    O-projection reads as plain rows.  head_scale (optional, [B, H], no gradient) is the banked
    attention's recipe head mask applied to v (rte/layers.py:659-730)."""

    @staticmethod
    def forward(ctx, q, k, v, head_scale):
        _lib.require_device_tensors("attention", q, k, v, head_scale)
        B, H, S, hd = q.shape
        if hd not in (32, 64, 128) or k.shape != q.shape or v.shape != q.shape:
            raise ValueError("attention: q, k, v must share the shape [B, H, S, hd], hd 32, 64 or 128")
        qb, kb, vb = (t.to(BF16).contiguous() for t in (q, k, v))
        hs = None if head_scale is None else head_scale.reshape(B * H).to(F32).contiguous()
        out = torch.empty((B, S, H, hd), dtype=BF16, device=q.device)
        lse = torch.empty((B, H, S), dtype=F32, device=q.device)
        scale = 1.0 / math.sqrt(hd)
        call("rte_attention_fwd", ptr(qb), ptr(kb), ptr(vb), B, H, S, hd, scale, ptr(hs), ptr(out), ptr(lse), _s())
        ctx.save_for_backward(qb, kb, vb, out, lse, hs)
        ctx.scale = scale
        ctx.dtypes = (q.dtype, k.dtype, v.dtype)
        return out.transpose(1, 2)

    @staticmethod
    def backward(ctx, dout):
        qb, kb, vb, out, lse, hs = ctx.saved_tensors
        B, H, S, hd = qb.shape
        dtok = dout.transpose(1, 2).to(BF16).contiguous()  # token-major [B, S, H, hd]
        dq, dk, dv = (torch.empty_like(qb) for _ in range(3))
        call("rte_attention_bwd", ptr(qb), ptr(kb), ptr(vb), ptr(out), ptr(dtok), ptr(lse), B, H, S, hd, ctx.scale,
             ptr(hs), ptr(dq), ptr(dk), ptr(dv), _s())
        qd, kd, vd = ctx.dtypes
        return dq.to(qd), dk.to(kd), dv.to(vd), None


def attention(q, k, v, head_scale=None):
    if fp32_active():  # [B, H, S, hd] view of the token-major fp32 attention output
        B, Hh, S, hd = q.shape
        return _f32().AttentionFn.apply(q, k, v, head_scale).view(B, S, Hh, hd).transpose(1, 2)
    if head_scale is not None and head_scale.requires_grad:
        raise ValueError("attention: head_scale carries no gradient")
    return AttentionFn.apply(q, k, v, head_scale)


class QKVRopeAttentionFn(torch.autograd.Function):
    """attention(qkv_rope(x, w)) as one autograd node: the attention backward writes the QKV
    projection's input gradient straight in its packed, RoPE-rotated-back layout
    (rte_attention_bwd_qkv), so the separate packing pass of the QKV backward is skipped.
    Values and gradients equal QKVRopeFn followed by AttentionFn bit for bit."""

    @staticmethod
    def forward(ctx, x, w, cos, sin, n_heads: int, head_scale, wgrad: SharedWGrad | None = None):
        B, S, d = x.shape
        hd = d // n_heads
        _check_rope_tables(cos, sin, S, hd)
        _lib.require_device_tensors("qkv_rope_attention", x, w, cos, sin, head_scale)
        if w.shape != (3 * d, d) or hd not in (32, 64, 128) or hd * n_heads != d:
            raise ValueError("qkv_rope_attention: wqkv [3d, d] and head_dim 32, 64 or 128 required")
        xb = x.contiguous().to(BF16)
        wb = cast_bf16(w)
        cs = cos[:S].contiguous().to(F32)
        sn = sin[:S].contiguous().to(F32)
        q = torch.empty((B, n_heads, S, hd), dtype=BF16, device=x.device)
        k = torch.empty_like(q)
        v = torch.empty_like(q)
        wsp, wsn = _gemm_ws(B * S, 3 * n_heads * hd, n_heads * hd, x.device)
        call("rte_qkv_rope_fwd", ptr(xb), ptr(wb), ptr(cs), ptr(sn), B, S, n_heads, hd, ptr(q), ptr(k), ptr(v), wsp,
             wsn, _s())
        hs = None if head_scale is None else head_scale.reshape(B * n_heads).to(F32).contiguous()
        out = torch.empty((B, S, n_heads, hd), dtype=BF16, device=x.device)
        lse = torch.empty((B, n_heads, S), dtype=F32, device=x.device)
        scale = 1.0 / math.sqrt(hd)
        call("rte_attention_fwd", ptr(q), ptr(k), ptr(v), B, n_heads, S, hd, scale, ptr(hs), ptr(out), ptr(lse),
             _s())
        ctx.save_for_backward(xb, wb, cs, sn, q, k, v, out, lse, hs)
        ctx.meta = (B, S, n_heads, hd, scale, x.dtype, w.dtype, _is_t_view(w))
        ctx.wgrad = wgrad if (wgrad is not None and ctx.needs_input_grad[1]) else None
        if ctx.wgrad is not None:
            ctx.wgrad.register()
        ctx.set_materialize_grads(False)
        return out.transpose(1, 2)

    @staticmethod
    def backward(ctx, dout):
        if dout is None:
            dw = ctx.wgrad.add(None, None, ctx.meta[7]) if ctx.wgrad is not None else None
            return None, (None if dw is None else dw.to(ctx.meta[6])), None, None, None, None, None
        xb, wb, cs, sn, q, k, v, out, lse, hs = ctx.saved_tensors
        B, S, H, hd, scale, x_dt, w_dt, w_t = ctx.meta
        d = H * hd
        dtok = dout.transpose(1, 2).to(BF16).contiguous()  # token-major [B, S, H, hd]
        dqkv = torch.empty((B * S, 3 * d), dtype=BF16, device=xb.device)
        call("rte_attention_bwd_qkv", ptr(q), ptr(k), ptr(v), ptr(out), ptr(dtok), ptr(lse), B, H, S, hd, scale,
             ptr(hs), ptr(cs), ptr(sn), ptr(dqkv), _s())
        dx = torch.empty((B * S, d), dtype=BF16, device=xb.device)
        shared = ctx.wgrad is not None
        dw = None if (w_t or shared) else torch.empty((3 * d, d), dtype=F32, device=xb.device)
        wsp, wsn = _gemm_ws_max(xb.device, (3 * d, d, B * S), (B * S, d, 3 * d))
        call("rte_qkv_rope_bwd", None, None, None, None, None, None, ptr(xb), ptr(wb), ptr(cs), ptr(sn), B, S, H, hd,
             ptr(dqkv), ptr(dx), ptr(dw), wsp, wsn, _s())
        if shared:
            dw = ctx.wgrad.add(xb.reshape(B * S, d), dqkv, w_t)
        elif w_t:  # w is a transposed view: dW^T [d, 3d] = x^T dqkv, returned as its transpose
            dw = gemm(xb.reshape(B * S, d), dqkv, a_t=True, b_t=True, out_f32=True).t()
        return dx.view(B, S, d).to(x_dt), (None if dw is None else dw.to(w_dt)), None, None, None, None, None


def qkv_rope_attention(x, w, cos, sin, n_heads, head_scale=None, wgrad: SharedWGrad | None = None):
    """[B, H, S, hd] view of the token-major attention output of x's fused QKV + RoPE; wgrad (optional)
    shares one weight-gradient GEMM among the calls of a forward that use w."""
    if fp32_active():
        return _f32().qkv_rope_attention(x, w, cos, sin, n_heads, head_scale)
    if head_scale is not None and head_scale.requires_grad:
        raise ValueError("qkv_rope_attention: head_scale carries no gradient")
    return QKVRopeAttentionFn.apply(x, w, cos, sin, n_heads, head_scale, wgrad)


# ----------------------------------------------------------------------------- dense SwiGLU

class DenseSwiGLUFn(torch.autograd.Function):
    """out = resid + (up * silu(gate)) @ W_down with the SwiGLU activation fused into the GEMMs.

    wug: [2F, d] rows [up ; gate] (rte/layers.py:78-87 chunk order).  wd_rows=False: wd is the
    nn.Linear(F, d) weight [d, F]; wd_rows=True: wd is [F, d] (PackedDenseSwiGLU.wdown_rows).
    """

    @staticmethod
    def forward(ctx, x, wug, wd, resid, wd_rows: bool, out_f32: bool):
        _lib.require_device_tensors("dense_swiglu", x, wug, wd, resid)
        shape = x.shape
        d = shape[-1]
        xb = x.reshape(-1, d).contiguous().to(BF16)
        T = xb.shape[0]
        F = wug.shape[0] // 2
        wugb = cast_bf16(wug)
        wdb = cast_bf16(wd)
        ug = torch.empty((T, 2 * F), dtype=BF16, device=x.device)
        z = torch.empty((T, F), dtype=BF16, device=x.device)
        out = torch.empty((T, d), dtype=F32 if out_f32 else BF16, device=x.device)
        r = None if resid is None else resid.reshape(T, d).contiguous().to(F32)
        call("rte_dense_swiglu_fwd", ptr(xb), T, d, F, ptr(wugb), ptr(wdb), int(wd_rows), ptr(r), ptr(ug), ptr(z),
             ptr(out), int(out_f32), _s())
        ctx.save_for_backward(xb, wugb, wdb, ug, z)
        ctx.meta = (shape, F, wd_rows, resid is not None, wug.dtype, wd.dtype)
        return out.view(shape)

    @staticmethod
    def backward(ctx, dout):
        xb, wugb, wdb, ug, z = ctx.saved_tensors
        shape, F, wd_rows, has_resid, wug_dtype, wd_dtype = ctx.meta
        T, d = xb.shape
        db = cast_bf16(dout.reshape(T, d)) if dout.dtype != BF16 else dout.reshape(T, d).contiguous()
        dug = torch.empty((T, 2 * F), dtype=BF16, device=xb.device)
        dx = torch.empty((T, d), dtype=BF16, device=xb.device)
        dwug = torch.empty((2 * F, d), dtype=F32, device=xb.device)
        dwd = torch.empty(wdb.shape, dtype=F32, device=xb.device)
        wsp, wsn = _gemm_ws_max(xb.device, (2 * F, d, T), (T, d, 2 * F), (d, F, T))
        call("rte_dense_swiglu_bwd", ptr(db), ptr(xb), T, d, F, ptr(wugb), ptr(wdb), int(wd_rows), ptr(ug), ptr(z),
             ptr(dug), ptr(dx), ptr(dwug), ptr(dwd), wsp, wsn, _s())
        dres = dout if has_resid else None
        return dx.view(shape), dwug.to(wug_dtype), dwd.to(wd_dtype), dres, None, None


def dense_swiglu(x, wug, wd, resid=None, *, wd_rows: bool = False, out_f32: bool = True):
    """resid + (up * silu(gate)) @ W_down; a width F that is not a multiple of 32 (the kernels'
    column block) is padded with zero neurons, which contribute nothing and get no gradient."""
    if fp32_active():
        return _f32().dense_swiglu(x, wug, wd, resid, wd_rows=wd_rows)
    F = wug.shape[0] // 2
    pad = (-F) % 32
    if pad:
        up, gate = wug[:F], wug[F:]
        zr = wug.new_zeros(pad, wug.shape[1])
        wug = torch.cat([up, zr, gate, zr])
        wd = torch.cat([wd, wd.new_zeros(pad, wd.shape[1])]) if wd_rows else torch.cat([wd, wd.new_zeros(wd.shape[0], pad)], 1)
    return DenseSwiGLUFn.apply(x, wug, wd, resid, wd_rows, out_f32)


# ----------------------------------------------------------------------------- routing / packing

@dataclass
class PackIndex:
    """Deterministic cluster packing of the T*k (token, cluster) pairs.

    offsets[C+1]: slot range of each cluster; slots inside a cluster follow ascending token.
    """

    offsets: torch.Tensor
    tok_of_slot: torch.Tensor
    pair_of_slot: torch.Tensor
    slot_of_pair: torch.Tensor
    w_of_slot: torch.Tensor
    n_clusters: int
    k: int


def route_topk(logits: torch.Tensor, k: int) -> tuple[torch.Tensor, torch.Tensor]:
    """Per-token top-k of fp32 router logits: ids int32 [T, k], softmax weights fp32 [T, k]."""
    _lib.require_device_tensors("route_topk", logits)
    lg = logits.contiguous().to(F32)
    T, C = lg.shape
    ids = torch.empty((T, k), dtype=torch.int32, device=lg.device)
    w = torch.empty((T, k), dtype=F32, device=lg.device)
    call("rte_route_topk", ptr(lg), T, C, k, ptr(ids), ptr(w), _s())
    return ids, w


def route_pack_supported(C: int, k: int, d: int) -> bool:
    """Shapes rte_route_pack takes: the router GEMM, top-k and pack in two launches."""
    return C in (32, 64, 128) and 1 <= k <= min(16, C) and d % 64 == 0


def route_pack(xb: torch.Tensor, wrb: torch.Tensor, k: int, *, with_logits: bool = False):
    """logits = xb wrb^T, ids / weights = route_topk(logits, k) and their pack, from
    rte_route_pack: (ids int32 [T, k], weights fp32 [T, k], PackIndex, logits fp32 [T, C] or None)."""
    _lib.require_device_tensors("route_pack", xb, wrb)
    T, d = xb.shape
    C = wrb.shape[0]
    dev = xb.device
    P = T * k
    ids = torch.empty((T, k), dtype=torch.int32, device=dev)
    w = torch.empty((T, k), dtype=F32, device=dev)
    offsets = torch.empty((C + 1,), dtype=torch.int32, device=dev)
    tok = torch.empty((P,), dtype=torch.int32, device=dev)
    pos = torch.empty((P,), dtype=torch.int32, device=dev)
    sop = torch.empty((P,), dtype=torch.int32, device=dev)
    wos = torch.empty((P,), dtype=F32, device=dev)
    logits = torch.empty((T, C), dtype=F32, device=dev) if with_logits else None
    wsp, wsn = workspace(_lib.load().rte_route_pack_workspace_bytes(T, C), dev)
    call("rte_route_pack", ptr(xb), T, d, ptr(wrb), C, k, ptr(ids), ptr(w), ptr(offsets), ptr(tok), ptr(pos),
         ptr(sop), ptr(wos), ptr(logits), wsp, wsn, _s())
    return ids, w, PackIndex(offsets, tok, pos, sop, wos, C, k), logits


def pack_index(ids: torch.Tensor, n_clusters: int, weights: torch.Tensor | None = None,
               invalid: torch.Tensor | None = None) -> PackIndex:
    _lib.require_device_tensors("pack_index", ids, weights, invalid)
    cl = ids.contiguous().to(torch.int32)
    k = cl.shape[-1] if cl.ndim == 2 else 1
    P = cl.numel()
    dev = cl.device
    offsets = torch.empty((n_clusters + 1,), dtype=torch.int32, device=dev)
    tok = torch.empty((P,), dtype=torch.int32, device=dev)
    pos = torch.empty((P,), dtype=torch.int32, device=dev)
    sop = torch.empty((P,), dtype=torch.int32, device=dev)
    wos = torch.empty((P,), dtype=F32, device=dev)
    nbytes = _lib.load().rte_pack_workspace_bytes(P, n_clusters)
    ws = torch.empty((max(1, nbytes // 4),), dtype=torch.int32, device=dev)
    w = None if weights is None else weights.contiguous().to(F32)
    call("rte_pack_index", ptr(cl), P, n_clusters, k, ptr(w), ptr(offsets), ptr(tok), ptr(pos), ptr(sop), ptr(wos),
         ptr(invalid), ptr(ws), nbytes, _s())
    return PackIndex(offsets, tok, pos, sop, wos, n_clusters, k)


def pack_routes(recipe_ids: torch.Tensor, routes: torch.Tensor, route_w: torch.Tensor | None, seq: int,
                n_clusters: int, active: torch.Tensor | None = None) -> PackIndex:
    """Pack of per-sample route lists: every token of sample b visits clusters
    routes[recipe_ids[b]] (-1 = none) with weight route_w[recipe_ids[b]]; samples with active
    False visit none.  The same slots as pack_index on the expanded [B*seq, kmax] ids, in two
    launches instead of the expansion, copies and three counting-sort launches."""
    _lib.require_device_tensors("pack_routes", recipe_ids, routes, route_w, active)
    rid = recipe_ids.reshape(-1).contiguous().to(torch.int64)
    rt = routes.contiguous().to(torch.int32)
    R, kmax = rt.shape
    B = rid.numel()
    P = B * seq * kmax
    dev = rid.device
    offsets = torch.empty((n_clusters + 1,), dtype=torch.int32, device=dev)
    tok = torch.empty((P,), dtype=torch.int32, device=dev)
    pos = torch.empty((P,), dtype=torch.int32, device=dev)
    sop = torch.empty((P,), dtype=torch.int32, device=dev)
    wos = torch.empty((P,), dtype=F32, device=dev)
    nbytes = _lib.load().rte_pack_routes_workspace_bytes(B, kmax)
    ws = torch.empty((max(1, nbytes // 4),), dtype=torch.int32, device=dev)
    act = None
    if active is not None:  # a bool mask is read as bytes in place
        act = active.reshape(-1).contiguous()
        act = act.view(torch.uint8) if act.dtype == torch.bool else act.to(torch.uint8)
    rw = None if route_w is None else route_w.contiguous().to(F32)
    call("rte_pack_routes", ptr(rid), ptr(act), B, seq, ptr(rt), R, kmax, ptr(rw), n_clusters, ptr(offsets), ptr(tok),
         ptr(pos), ptr(sop), ptr(wos), ptr(ws), nbytes, _s())
    return PackIndex(offsets, tok, pos, sop, wos, n_clusters, kmax)


def combine_rows(rows: torch.Tensor, T: int, k: int, *, extra=None, resid=None, out_f32=True,
                 slot_of_pair=None) -> torch.Tensor:
    """out[t] = resid[t] + extra[t] + sum_j rows[t*k + j]; pairs whose slot_of_pair is -1 are skipped."""
    _lib.require_device_tensors("combine_rows", rows, extra, resid, slot_of_pair)
    d = rows.shape[-1]
    out = torch.empty((T, d), dtype=F32 if out_f32 else BF16, device=rows.device)
    r = None if resid is None else resid.reshape(T, d).contiguous().to(F32)
    e = None if extra is None else extra.reshape(T, d).contiguous().to(BF16)
    call("rte_combine_rows", ptr(rows.contiguous()), T, k, d, ptr(slot_of_pair), ptr(e), ptr(r), ptr(out),
         int(out_f32), _s())
    return out


# ----------------------------------------------------------------------------- routed cluster-pool SwiGLU

# 32-neuron clusters at d 128 / 256 / 512 run the fused per-cluster kernels (one launch per direction
# for the two products and the SwiGLU; rte_grouped_swiglu_fused_*); [False] selects the two-GEMM form
POOL_FUSED = [True]


def _pool_entry(name: str, n: int, d: int) -> str:
    if POOL_FUSED[0] and _lib.load().rte_grouped_swiglu_fused_ok(n, d):
        return name.replace("rte_grouped_swiglu_", "rte_grouped_swiglu_fused_")
    return name


def _pool_fwd(xb, ids, w, wugb, wdb, C: int, n: int, resid, masked: bool, pk: PackIndex | None = None):
    """Grouped pool forward over the (token, cluster) pairs of ids [T, k] (id -1 = no pair), or
    of a prebuilt pack pk.  wugb [2F, d] rows [up F ; gate F], wdb [d, F]; cluster g owns
    neurons [g*n, (g+1)*n)."""
    T, d = xb.shape
    k = ids.shape[1] if pk is None else pk.k
    F = C * n
    if pk is None:
        pk = pack_index(ids, C, w)
    P = T * k
    ug = torch.empty((P, 2 * n), dtype=BF16, device=xb.device)
    zw = torch.empty((P, n), dtype=BF16, device=xb.device)
    yp = torch.empty((P, d), dtype=BF16, device=xb.device)
    call(_pool_entry("rte_grouped_swiglu_fwd", n, d), ptr(xb), T, d, ptr(pk.offsets), C, n, P, ptr(pk.tok_of_slot),
         ptr(pk.pair_of_slot), ptr(pk.w_of_slot), ptr(wugb), ptr(wdb), F, ptr(ug), ptr(zw), ptr(yp), _s())
    out = combine_rows(yp, T, k, resid=resid, out_f32=True, slot_of_pair=pk.slot_of_pair if masked else None)
    return out, pk, ug, zw


def _pool_bwd(db, xb, wugb, wdb, pk, ug, zw, C: int, n: int, k: int, dwug=None, dwd=None, w_t: bool = False,
              beta: float = 0.0):
    """Backward of _pool_fwd up to the combine: (dx_pairs bf16 [P, d] in pair order,
    dwug f32 [2F, d], dwd f32 [d, F], dw_slot f32 [P] = per-slot <z, dz>).  w_t: the weight
    gradients in the transposed layouts ([d, 2F], [F, d]); dwug / dwd given: written there
    (beta = 1: added to what they hold)."""
    T, d = xb.shape
    F = C * n
    P = T * k
    dev = xb.device
    dug = torch.empty((P, 2 * n), dtype=BF16, device=dev)
    dw_slot = torch.empty((P,), dtype=F32, device=dev)
    dxp = torch.empty((P, d), dtype=BF16, device=dev)
    if dwug is None:
        dwug = torch.empty((d, 2 * F) if w_t else (2 * F, d), dtype=F32, device=dev)
    if dwd is None:
        dwd = torch.empty((F, d) if w_t else (d, F), dtype=F32, device=dev)
    ws, nb = workspace(_lib.load().rte_grouped_swiglu_bwd_workspace_bytes(P, C, n, d), dev)
    call(_pool_entry("rte_grouped_swiglu_bwd", n, d), ptr(db), ptr(xb), T, d, ptr(pk.offsets), C, n, P,
         ptr(pk.tok_of_slot),
         ptr(pk.pair_of_slot), ptr(pk.w_of_slot), ptr(wugb), ptr(wdb), F, ptr(ug), ptr(zw), ptr(dug), ptr(dw_slot),
         ptr(dxp), ptr(dwug), ptr(dwd), int(w_t), float(beta), ws, nb, _s())
    return dxp, dwug, dwd, dw_slot


class RoutedClusterPoolFn(torch.autograd.Function):
    """Top-k routed cluster-pool SwiGLU FFN (cluster g owns neurons [g*n, (g+1)*n)).

    logits = x @ Wr^T (fp32), ids/weights = top-k + softmax over the selected logits,
    out[t] = resid[t] + sum_j w_tj * SwiGLU_{ids_tj}(x_t).  k = 1 with one cluster per token is the
    reference static cluster pool (rte/kernels/cluster_pool_ffn.py:143-162, :192-215).
    """

    @staticmethod
    def forward(ctx, x, wr, wug, wd, resid, k: int):
        _lib.require_device_tensors("routed_cluster_pool", x, wr, wug, wd, resid)
        shape = x.shape
        d = shape[-1]
        xb = x.reshape(-1, d).contiguous().to(BF16)
        C = wr.shape[0]
        F = wug.shape[0] // 2
        if F % C != 0:
            raise ValueError("d_ff must be divisible by the cluster count")
        n = F // C
        wrb = cast_bf16(wr)
        wugb = cast_bf16(wug)
        wdb = cast_bf16(wd)
        if route_pack_supported(C, k, d):
            ids, w, pk, _ = route_pack(xb, wrb, k)
        else:
            logits = gemm(xb, wrb, out_f32=True)
            ids, w = route_topk(logits, k)
            pk = None
        out, pk, ug, zw = _pool_fwd(xb, ids, w, wugb, wdb, C, n, resid, masked=False, pk=pk)
        ctx.save_for_backward(xb, wrb, wugb, wdb, ids, w, pk.offsets, pk.tok_of_slot, pk.pair_of_slot,
                              pk.slot_of_pair, pk.w_of_slot, ug, zw)
        ctx.meta = (shape, k, C, n, resid is not None, wr.dtype, wug.dtype, wd.dtype)
        ctx.mark_non_differentiable(ids, w)
        ctx.set_materialize_grads(False)  # no zero fills for the routing outputs
        return out.view(shape), ids, w

    @staticmethod
    def backward(ctx, dout, _dids, _dw):
        if dout is None:
            return (None,) * 6
        (xb, wrb, wugb, wdb, ids, w, offsets, tok, pos, sop, wos, ug, zw) = ctx.saved_tensors
        shape, k, C, n, has_resid, wr_dt, wug_dt, wd_dt = ctx.meta
        T, d = xb.shape
        dev = xb.device
        db = cast_bf16(dout.reshape(T, d))
        pk = PackIndex(offsets, tok, pos, sop, wos, C, k)
        dxp, dwug, dwd, dw_slot = _pool_bwd(db, xb, wugb, wdb, pk, ug, zw, C, n, k)
        dlog = torch.empty((T, C), dtype=BF16, device=dev)
        call("rte_route_bwd", ptr(ids), ptr(w), ptr(dw_slot), ptr(sop), T, C, k, ptr(dlog), None, _s())
        wr_k = wrb
        c8 = (C + 7) // 8 * 8  # the GEMM reads 8-element vectors along C
        if c8 != C:
            dlog = torch.nn.functional.pad(dlog, (0, c8 - C))
            wr_k = torch.nn.functional.pad(wrb, (0, 0, 0, c8 - C))
        dx_router = gemm(dlog, wr_k, b_t=True)                        # [T, d] = dlogits @ Wr
        dwr = gemm(dlog, xb, a_t=True, b_t=True, out_f32=True)[:C]    # [C, d] = dlogits^T @ x
        dx = combine_rows(dxp, T, k, extra=dx_router, out_f32=False)
        dres = dout if has_resid else None
        return dx.view(shape), dwr.to(wr_dt), dwug.to(wug_dt), dwd.to(wd_dt), dres, None


def routed_cluster_pool_swiglu(x, wr, wug, wd, k: int, resid=None):
    """Returns (out, ids, weights); ids/weights are the routing decisions (no gradient)."""
    if fp32_active():
        return _f32().routed_cluster_pool_swiglu(x, wr, wug, wd, k, resid)
    return RoutedClusterPoolFn.apply(x, wr, wug, wd, resid, k)


class GroupedPoolFn(torch.autograd.Function):
    """Grouped SwiGLU pool with routes given by the caller: out[t] = resid[t] +
    sum_j w[t, j] * SwiGLU_{ids[t, j]}(x_t); ids == -1 marks an absent pair (dropped by
    the pack, skipped by the combine).  ids / w carry no gradient.

    wug_t bf16 [2F, d] (rows [up F ; gate F]) and wd_t bf16 [d, F] are differentiable
    operands: their gradients come back in fp32."""

    @staticmethod
    def forward(ctx, x, ids, w, wug_t, wd_t, resid, n: int, pk=None, acc: "SharedGradAccum | None" = None):
        _lib.require_device_tensors("grouped_pool", x, ids, w, wug_t, wd_t, resid)
        shape = x.shape
        d = shape[-1]
        xb = x.reshape(-1, d).contiguous().to(BF16)
        T = xb.shape[0]
        F = wug_t.shape[0] // 2
        C = F // n
        if pk is None:
            idc = ids.reshape(T, -1).contiguous().to(torch.int32)
            wc = w.reshape(T, -1).contiguous().to(F32)
        else:
            idc = wc = None
        wugb, wdb = cast_bf16(wug_t), cast_bf16(wd_t)  # parameter views: once per step
        rs = None if resid is None else resid.reshape(T, d)
        out, pk, ug, zw = _pool_fwd(xb, idc, wc, wugb, wdb, C, n, rs, masked=True, pk=pk)
        ctx.save_for_backward(xb, wugb, wdb, pk.offsets, pk.tok_of_slot, pk.pair_of_slot, pk.slot_of_pair,
                              pk.w_of_slot, ug, zw)
        # weights that are transposed views get their gradients formed in their own layout
        ctx.w_t = _is_t_view(wug_t) and _is_t_view(wd_t)
        ctx.acc = acc if (acc is not None and ctx.needs_input_grad[3] and ctx.needs_input_grad[4]) else None
        if ctx.acc is not None:
            ctx.acc.register()
        ctx.meta = (shape, pk.k, C, n, resid is not None, x.dtype)
        return out.view(shape)

    @staticmethod
    def backward(ctx, dout):
        xb, wugb, wdb, offsets, tok, pos, sop, wos, ug, zw = ctx.saved_tensors
        shape, k, C, n, has_resid, x_dt = ctx.meta
        T, d = xb.shape
        F = C * n
        pk = PackIndex(offsets, tok, pos, sop, wos, C, k)
        w_t, dev = ctx.w_t, xb.device
        bufs, beta, last = (None, None), 0.0, True
        if ctx.acc is not None:
            shapes = ((d, 2 * F), (F, d)) if w_t else ((2 * F, d), (d, F))
            bufs, beta, last = ctx.acc.arrive(lambda: tuple(torch.empty(s_, dtype=F32, device=dev) for s_ in shapes))
        dxp, dwug, dwd, _ = _pool_bwd(cast_bf16(dout.reshape(T, d)), xb, wugb, wdb, pk, ug, zw, C, n, k,
                                      dwug=bufs[0], dwd=bufs[1], w_t=w_t, beta=beta)
        dx = combine_rows(dxp, T, k, out_f32=False, slot_of_pair=sop)
        if not last:
            dwug = dwd = None
        elif w_t:
            dwug, dwd = dwug.t(), dwd.t()
        return dx.view(shape).to(x_dt), None, None, dwug, dwd, (dout if has_resid else None), None, None, None


def grouped_pool_swiglu(x, ids, w, wug_t, wd_t, n: int, resid=None, pk: PackIndex | None = None,
                        acc: "SharedGradAccum | None" = None):
    """Grouped pool SwiGLU over the routes ids / w [T, k], or over a prebuilt pack pk (then ids
    and w are not read).  acc (optional): the calls of a forward that share these weights sum
    their weight gradients in one pair of buffers."""
    if fp32_active():
        return _f32().grouped_pool_swiglu(x, ids, w, wug_t, wd_t, n, resid, pk)
    return GroupedPoolFn.apply(x, ids, w, wug_t, wd_t, resid, n, pk, acc)


# ----------------------------------------------------------------------------- plain linear (LM head)

class LinearFn(torch.autograd.Function):
    """out = x @ W^T on the MFMA GEMM (bf16 operands, fp32 accumulate), fp32 or bf16 output."""

    @staticmethod
    def forward(ctx, x, w, out_f32: bool):
        _lib.require_device_tensors("linear", x, w)
        shape = x.shape
        xb = x.reshape(-1, shape[-1]).contiguous().to(BF16)
        wb = cast_bf16(w)
        out = gemm(xb, wb, out_f32=out_f32)
        ctx.save_for_backward(xb, wb)
        ctx.meta = (shape, x.dtype, w.dtype)
        return out.view(*shape[:-1], wb.shape[0])

    @staticmethod
    def backward(ctx, dout):
        xb, wb = ctx.saved_tensors
        shape, x_dt, w_dt = ctx.meta
        N = wb.shape[0]
        db = cast_bf16(dout.reshape(-1, N))
        n8 = (N + 7) // 8 * 8  # both backward GEMMs reduce over or read N in 8-element vectors
        if n8 != N:
            db = torch.nn.functional.pad(db, (0, n8 - N))
            wb = torch.nn.functional.pad(wb, (0, 0, 0, n8 - N))
        dx = gemm(db, wb, b_t=True)                              # [T, K]
        dw = gemm(db, xb, a_t=True, b_t=True, out_f32=True)[:N]  # [N, K]
        return dx.view(shape).to(x_dt), dw.to(w_dt), None


def linear(x, w, *, out_f32: bool = True):
    if fp32_active():
        return _f32().linear(x, w)
    return LinearFn.apply(x, w, out_f32)


class LinearBiasFn(torch.autograd.Function):
    """out = x @ W^T + b (nn.Linear with bias) on the MFMA GEMM: the bias is added in the GEMM
    epilogue as a broadcast residual row (fp32); the backward is two GEMMs and a column sum."""

    @staticmethod
    def forward(ctx, x, w, b, out_f32: bool):
        _lib.require_device_tensors("linear_bias", x, w, b)
        shape = x.shape
        xb = x.reshape(-1, shape[-1]).contiguous().to(BF16)
        wb = cast_bf16(w)
        M, N, K = xb.shape[0], wb.shape[0], xb.shape[1]
        bias = b.detach().reshape(N).contiguous().to(F32)
        out = torch.empty((M, N), dtype=F32 if out_f32 else BF16, device=x.device)
        wsp, wsn = _gemm_ws(M, N, K, x.device)
        call("rte_gemm_bf16", ptr(xb), K, 0, None, ptr(wb), K, 0, None, ptr(out), N, int(out_f32), M, N, K, 1.0, 0.0,
             ptr(bias), 0, wsp, wsn, _s())
        ctx.save_for_backward(xb, wb)
        ctx.meta = (shape, x.dtype, w.dtype, b.dtype)
        return out.view(*shape[:-1], N)

    @staticmethod
    def backward(ctx, dout):
        xb, wb = ctx.saved_tensors
        shape, x_dt, w_dt, b_dt = ctx.meta
        N = wb.shape[0]
        d2 = dout.reshape(-1, N)
        db = cast_bf16(d2)
        n8 = (N + 7) // 8 * 8  # both backward GEMMs reduce over or read N in 8-element vectors
        if n8 != N:
            db = torch.nn.functional.pad(db, (0, n8 - N))
            wb = torch.nn.functional.pad(wb, (0, 0, 0, n8 - N))
        dx = gemm(db, wb, b_t=True)                              # [M, K] = dout @ W
        dw = gemm(db, xb, a_t=True, b_t=True, out_f32=True)[:N]  # [N, K] = dout^T @ x
        dbias = d2.float().sum(0)
        return dx.view(shape).to(x_dt), dw.to(w_dt), dbias.to(b_dt), None


def linear_bias(x, w, b, *, out_f32: bool = True):
    if fp32_active():
        return _f32().linear(x, w, b)
    return LinearBiasFn.apply(x, w, b, out_f32)


# ----------------------------------------------------------------------------- recipe / depth router

ROUTER_FIELDS = ("recipe_logits", "recipe_probs", "recipe_id", "recipe_onehot_st", "depth_logits", "depth_probs",
                 "depth_id", "depth", "depth_onehot_st", "recipe_entropy", "depth_entropy", "router_entropy",
                 "expected_depth", "recipe_logits_by_pass", "recipe_probs_by_pass", "recipe_id_by_pass",
                 "recipe_onehot_st_by_pass")


def router_supported(hid: int, R: int, D: int, P: int, d: int) -> bool:
    return 1 <= hid <= 4096 and 1 <= R <= 64 and 1 <= D <= 64 and 0 <= P <= 16 and d % 8 == 0


class RouterFn(torch.autograd.Function):
    """Router.forward (rte/routing.py:80-188) for the recipe and depth heads: pooled mean of h0,
    the two Linear -> SiLU -> Linear MLPs (layer 1 on the MFMA GEMM with the bias in its epilogue,
    layer 2 and every head field in one launch with a wave per sample), per-pass recipe logits,
    softmax / argmax / straight-through one-hot / entropies / expected depth.  The backward is two
    small launches (heads, then layer 2 + SiLU + biases + pass bias) and the GEMMs of layer 1.
    Outputs are ROUTER_FIELDS in order; ids and depth are int64."""

    @staticmethod
    def forward(ctx, h0, w1r, b1r, w2r, b2r, w1d, b1d, w2d, b2d, pass_bias, depth_values, inv_t: float,
                fixed_recipe: int, fixed_depth: int):
        _lib.require_device_tensors("router", h0, w1r, b1r, w2r, b2r, w1d, b1d, w2d, b2d, pass_bias, depth_values)
        B, S, d = h0.shape
        hid, R, D, P = w1r.shape[0], w2r.shape[0], w2d.shape[0], pass_bias.shape[0]
        if not router_supported(hid, R, D, P, d) or w1d.shape[0] != hid:
            raise ValueError(f"router: unsupported sizes (hidden {hid}, recipes {R}, depths {D}, passes {P}, d {d})")
        dev = h0.device
        h0c = h0.detach().contiguous().to(F32)
        pooled = torch.empty((B, d), dtype=F32, device=dev)
        pooled_b = torch.empty((B, d), dtype=BF16, device=dev)
        call("rte_router_pool", ptr(h0c), B, S, d, ptr(pooled), ptr(pooled_b), _s())
        w1rb, w1db = cast_bf16(w1r), cast_bf16(w1d)
        z1 = torch.empty((2, B, hid), dtype=F32, device=dev)
        wsp, wsn = _gemm_ws(B, hid, d, dev)
        for i, (wb, bias) in enumerate(((w1rb, b1r), (w1db, b1d))):
            bias = bias.detach().reshape(hid).contiguous().to(F32)
            call("rte_gemm_bf16", ptr(pooled_b), d, 0, None, ptr(wb), d, 0, None, ptr(z1[i]), hid, 1, B, hid, d,
                 1.0, 0.0, ptr(bias), 0, wsp, wsn, _s())
        f32 = [w.detach().contiguous().to(F32) for w in (w2r, b2r, w2d, b2d, pass_bias)]
        dv = depth_values.detach().contiguous().to(torch.int64)

        def e(*shape, dt=F32):
            return torch.empty(shape, dtype=dt, device=dev)

        I64 = torch.int64
        out = (e(B, R), e(B, R), e(B, dt=I64), e(B, R), e(B, D), e(B, D), e(B, dt=I64), e(B, dt=I64), e(B, D),
               e(B), e(B), e(B), e(B), e(B, P, R), e(B, P, R), e(B, P, dt=I64), e(B, P, R))
        rlog, rprob, rid, roh, dlog, dprob, did, depth, doh, rent, dent, ent, edep, rlbp, rpbp, ridbp, rohbp = out
        call("rte_router_heads_fwd", ptr(z1[0]), ptr(z1[1]), B, hid, ptr(f32[0]), ptr(f32[1]), R, ptr(f32[2]),
             ptr(f32[3]), D, ptr(f32[4]), P, ptr(dv), float(inv_t), int(fixed_recipe), int(fixed_depth),
             *(ptr(t) for t in out), _s())
        ctx.save_for_backward(pooled_b, z1, w1rb, w1db, f32[0], f32[2], rprob, rpbp, dprob, dv)
        ctx.meta = (B, S, d, hid, R, D, P, float(inv_t), h0.dtype, [t.dtype for t in (w1r, b1r, w2r, b2r, w1d, b1d,
                                                                                      w2d, b2d, pass_bias)])
        ctx.mark_non_differentiable(rid, did, depth, ridbp)
        ctx.set_materialize_grads(False)
        return out

    @staticmethod
    def backward(ctx, *g):
        pooled_b, z1, w1rb, w1db, w2r, w2d, rprob, rpbp, dprob, dv = ctx.saved_tensors
        B, S, d, hid, R, D, P, inv_t, h0_dt, w_dts = ctx.meta
        dev = z1.device
        gi = {n: (None if t is None else t.detach().contiguous().to(F32)) for n, t in zip(ROUTER_FIELDS, g)}

        def gp(n):
            return ptr(gi[n])

        draw_r = torch.empty((B, R), dtype=F32, device=dev)
        draw_d = torch.empty((B, D), dtype=F32, device=dev)
        dlbp = torch.empty((B, P, R), dtype=F32, device=dev)
        call("rte_router_heads_bwd", ptr(rprob), ptr(rpbp), ptr(dprob), ptr(dv), B, R, D, P, inv_t,
             gp("recipe_logits"), gp("recipe_probs"), gp("recipe_onehot_st"), gp("depth_logits"), gp("depth_probs"),
             gp("depth_onehot_st"), gp("recipe_entropy"), gp("depth_entropy"), gp("router_entropy"),
             gp("expected_depth"), gp("recipe_logits_by_pass"), gp("recipe_probs_by_pass"),
             gp("recipe_onehot_st_by_pass"), ptr(draw_r), ptr(draw_d), ptr(dlbp), _s())
        dz1 = torch.empty((2, B, hid), dtype=BF16, device=dev)
        db1 = torch.empty((2, hid), dtype=F32, device=dev)
        dw2r = torch.empty((R, hid), dtype=F32, device=dev)
        dw2d = torch.empty((D, hid), dtype=F32, device=dev)
        db2r = torch.empty((R,), dtype=F32, device=dev)
        db2d = torch.empty((D,), dtype=F32, device=dev)
        dpass = torch.empty((P, R), dtype=F32, device=dev)
        call("rte_router_mlp_bwd", ptr(draw_r), ptr(draw_d), ptr(z1[0]), ptr(z1[1]), ptr(w2r), ptr(w2d), B, hid, R, D,
             ptr(dlbp), P, inv_t, ptr(dz1[0]), ptr(dz1[1]), ptr(db1[0]), ptr(db1[1]), ptr(dw2r), ptr(dw2d), ptr(db2r),
             ptr(db2d), ptr(dpass), _s())
        need = ctx.needs_input_grad
        dw1r = gemm(dz1[0], pooled_b, a_t=True, b_t=True, out_f32=True) if need[1] else None
        dw1d = gemm(dz1[1], pooled_b, a_t=True, b_t=True, out_f32=True) if need[5] else None
        dh0 = None
        if need[0]:
            # d pooled / S, broadcast over the sequence as a view
            dp = gemm(dz1[0], w1rb, b_t=True, out_f32=True, alpha=1.0 / S)
            dp = gemm(dz1[1], w1db, b_t=True, out_f32=True, alpha=1.0 / S, resid=dp)
            dh0 = dp.to(h0_dt).unsqueeze(1).expand(B, S, d)
        grads = [dw1r, db1[0], dw2r, db2r, dw1d, db1[1], dw2d, db2d, dpass]
        grads = [None if (t is None or not need[i + 1]) else t.to(dt) for i, (t, dt) in enumerate(zip(grads, w_dts))]
        return (dh0, *grads, None, None, None, None)


def router(h0, w1r, b1r, w2r, b2r, w1d, b1d, w2d, b2d, pass_bias, depth_values, *, inv_t: float = 1.0,
           fixed_recipe: int | None = None, fixed_depth: int | None = None) -> dict[str, torch.Tensor]:
    """The router's recipe / depth fields (ROUTER_FIELDS) from h0 [B, S, d]; fixed_depth is an
    index into depth_values."""
    if fp32_active():
        return _f32().router(h0, w1r, b1r, w2r, b2r, w1d, b1d, w2d, b2d, pass_bias, depth_values,
                             inv_t=inv_t, fixed_recipe=fixed_recipe, fixed_depth=fixed_depth)
    out = RouterFn.apply(h0, w1r, b1r, w2r, b2r, w1d, b1d, w2d, b2d, pass_bias, depth_values, float(inv_t),
                         -1 if fixed_recipe is None else int(fixed_recipe),
                         -1 if fixed_depth is None else int(fixed_depth))
    return dict(zip(ROUTER_FIELDS, out))


class RouterAuxFn(torch.autograd.Function):
    """router_aux_losses (rte/metrics.py:97-112) in one launch: load = lambda_load (R sum_r
    mean_b(p)^2 - 1), cover = lambda_cover sum_r relu(coverage_min - usage_ema)^2, depth =
    lambda_depth mean_b(expected_depth) as three scalar outputs; the backward is one launch (cover
    has no gradient)."""

    @staticmethod
    def forward(ctx, probs, expected_depth, usage_ema, coverage_min: float, l_load: float, l_cover: float,
                l_depth: float):
        usage_ema = usage_ema.to(probs.device)
        _lib.require_device_tensors("router_aux", probs, expected_depth, usage_ema)
        B, R = probs.shape
        if not (B >= 1 and 1 <= R <= 64):
            raise ValueError(f"router_aux: unsupported sizes ({B} rows, {R} recipes)")
        pc = probs.detach().contiguous().to(F32)
        ec = expected_depth.detach().contiguous().to(F32)
        ema = usage_ema.detach().contiguous().to(F32)
        mp = torch.empty((R,), dtype=F32, device=probs.device)
        out = torch.empty((3,), dtype=F32, device=probs.device)
        call("rte_router_aux_fwd", ptr(pc), ptr(ec), ptr(ema), B, R, float(coverage_min), float(l_load),
             float(l_cover), float(l_depth), ptr(mp), ptr(out), _s())
        ctx.save_for_backward(mp)
        ctx.meta = (B, R, float(l_load), float(l_depth), probs.dtype, expected_depth.dtype)
        ctx.set_materialize_grads(False)
        # three scalar outputs, so each loss term's gradient arrives without a select backward
        return out[0], out[1], out[2]

    @staticmethod
    def backward(ctx, g_load, g_cover, g_depth):
        (mp,) = ctx.saved_tensors
        B, R, l_load, l_depth, p_dt, e_dt = ctx.meta
        dev = mp.device
        gl = None if g_load is None else g_load.detach().reshape(1).contiguous().to(F32)
        gd = None if g_depth is None else g_depth.detach().reshape(1).contiguous().to(F32)
        dp = torch.empty((B, R), dtype=F32, device=dev)
        de = torch.empty((B,), dtype=F32, device=dev)
        call("rte_router_aux_bwd", ptr(mp), ptr(gl), ptr(gd), B, R, l_load, l_depth, ptr(dp), ptr(de), _s())
        return dp.to(p_dt), de.to(e_dt), None, None, None, None, None


def router_aux(probs, expected_depth, usage_ema, *, coverage_min: float, lambda_load: float, lambda_cover: float,
               lambda_depth: float) -> dict[str, torch.Tensor]:
    load, cover, depth = RouterAuxFn.apply(probs, expected_depth, usage_ema, coverage_min, lambda_load, lambda_cover,
                                           lambda_depth)
    return {"load": load, "cover": cover, "depth": depth}


# ----------------------------------------------------------------------------- LM head + cross-entropy

class LMHeadCEFn(torch.autograd.Function):
    """logits = hidden @ W^T (fp32) and per-token CE against targets in one operator.

    Returns (logits, token_loss).  Both are differentiable: the backward fuses the CE
    gradient, any gradient arriving on the logits themselves (e.g. a distillation KL term)
    and the cast to bf16 into one kernel, then runs the two head GEMMs."""

    @staticmethod
    def forward(ctx, hidden, w, targets):
        _lib.require_device_tensors("lm_head_ce", hidden, w, targets)
        shape = hidden.shape
        hb = hidden.reshape(-1, shape[-1]).contiguous().to(BF16)
        wb = cast_bf16(w)
        T, V = hb.shape[0], wb.shape[0]
        logits = gemm(hb, wb, out_f32=True)
        tg = targets.reshape(-1).contiguous().to(torch.int64)
        loss = torch.empty((T,), dtype=F32, device=hb.device)
        lse = torch.empty((T,), dtype=F32, device=hb.device)
        call("rte_ce_fwd", ptr(logits), V, T, V, ptr(tg), ptr(loss), ptr(lse), _s())
        ctx.save_for_backward(hb, wb, logits, tg, lse)
        ctx.meta = (shape, hidden.dtype, w.dtype)
        ctx.set_materialize_grads(False)  # no zero-filled [T, V] when only the loss has a gradient
        return logits.view(*shape[:-1], V), loss.view(shape[:-1])

    @staticmethod
    def backward(ctx, dlogits_ext, dloss):
        hb, wb, logits, tg, lse = ctx.saved_tensors
        shape, h_dt, w_dt = ctx.meta
        T, V = logits.shape
        ext = None if dlogits_ext is None else dlogits_ext.reshape(T, V).contiguous().to(F32)
        g = None if dloss is None else dloss.reshape(T).contiguous().to(F32)
        # gradients of whole-sample logit rows selected by select_logit_rows, in arrival order
        parts = [(sk.idx, gr) for sk in getattr(ctx, "row_sinks", ()) for gr in sk.take()]
        dl = torch.empty((T, V), dtype=BF16, device=hb.device)
        if parts and ext is None:
            S = shape[-2]
            if len(parts) == 1:
                ids, rows = parts[0][0], parts[0][1].reshape(-1, V)
            else:
                ids, rows = torch.cat([p[0] for p in parts]), torch.cat([p[1].reshape(-1, V) for p in parts])
            ids = ids.to(torch.int64).contiguous()
            rows = rows.contiguous().to(F32)
            call("rte_ce_bwd_rows", ptr(logits), V, T, V, ptr(tg), ptr(lse), ptr(g), ptr(rows), ptr(ids),
                 ids.numel(), S, ptr(dl), _s())
        else:
            if parts:  # a dense logit gradient as well: add the rows to it
                ext = ext.view(-1, shape[-2], V).clone()
                for ids, gr in parts:
                    ext.index_add_(0, ids, gr.to(F32))
                ext = ext.view(T, V)
            call("rte_ce_bwd", ptr(logits), V, T, V, ptr(tg), ptr(lse), ptr(g), ptr(ext), ptr(dl), _s())
        dh = gemm(dl, wb, b_t=True)                              # [T, d] = dlogits @ W
        dw = gemm(dl, hb, a_t=True, b_t=True, out_f32=True)      # [V, d] = dlogits^T @ hidden
        return dh.view(shape).to(h_dt), dw.to(w_dt), None


def lm_head_ce(hidden, w, targets):
    """(logits fp32, per-token cross-entropy) of hidden @ W^T against targets."""
    if fp32_active():
        return _f32().lm_head_ce(hidden, w, targets)
    return LMHeadCEFn.apply(hidden, w, targets)


def select_logit_rows(logits: torch.Tensor, idx: torch.Tensor) -> torch.Tensor:
    """Samples idx of [B, S, V] logits made by lm_head_ce (rte/audit.py:336, hot.meta.logits[mask]).
    Their gradient goes to the head's backward, whose CE kernel adds the rows of those samples
    only (rte_ce_bwd_rows): no zero-filled [B, S, V] gradient.  Other logits use index_select."""
    node = logits.grad_fn
    if not (torch.is_grad_enabled() and logits.requires_grad and logits.dim() == 3 and node is not None
            and type(node).__name__ == "LMHeadCEFnBackward"):
        return logits.index_select(0, idx)
    sink = _RowSink(idx)
    node.row_sinks = getattr(node, "row_sinks", []) + [sink]
    return SelectRowsFn.apply(logits, idx, sink)


# ----------------------------------------------------------------------------- audit distillation

DISTILL_LOSSES = ("delta_dir", "delta_rms", "endpoint_normed", "endpoint_raw", "rms_trust", "kl")
DISTILL_METRICS = ("hidden_cosine_exact_macro", "hidden_mse_exact_macro", "macro_norm", "exact_norm",
                   "macro_exact_norm_ratio", "delta_cosine_exact_macro", "delta_rms_exact", "delta_rms_pred",
                   "delta_rms_ratio", "logit_kl_exact_macro")


class DistillFn(torch.autograd.Function):
    """Hot-vs-exact distillation losses (rte/macro.py:394-471, with h0), each times its weight,
    and the alignment metrics (:499-546) of the audited samples in three launches; the backward
    is one launch for the hidden states and one for the logits.  The six weighted losses are six
    outputs (their gradients arrive separately, no selects).  exact, h0 and exact_logits carry
    no gradient."""

    @staticmethod
    def forward(ctx, hot, exact, h0, hot_logits, exact_logits, temperature, eps, weights):
        _lib.require_device_tensors("distill", hot, exact, h0, hot_logits, exact_logits)
        A, S, d = hot.shape
        dev = hot.device
        hv = hot.contiguous().to(F32)
        ev = exact.detach().contiguous().to(F32)
        zv = h0.detach().contiguous().to(F32)
        has_l = hot_logits is not None and exact_logits is not None and hot_logits.shape == exact_logits.shape
        V = hot_logits.shape[-1] if has_l else 0
        hl = hot_logits.reshape(A * S, V).contiguous().to(F32) if has_l else None
        el = exact_logits.detach().reshape(A * S, V).contiguous().to(F32) if has_l else None
        R = A * S if has_l else 0
        nbytes = _lib.load().rte_distill_workspace_bytes(A, R)
        ws = torch.empty(((nbytes + 3) // 4,), dtype=F32, device=dev)  # kept for the backward
        losses = torch.empty((6,), dtype=F32, device=dev)
        metrics = torch.empty((10,), dtype=F32, device=dev)
        w6 = (ctypes.c_float * 6)(*[float(x) for x in weights])
        call("rte_distill_fwd", ptr(hv), ptr(ev), ptr(zv), A, S, d, ptr(hl), ptr(el), V, float(temperature),
             float(eps), ctypes.addressof(w6), ptr(losses), ptr(metrics), ptr(ws), nbytes, _s())
        ctx.save_for_backward(hv, ev, zv, hl, el, ws)
        ctx.meta = (A, S, d, V, float(temperature), float(eps), nbytes, has_l,
                    None if not has_l else hot_logits.shape, tuple(float(x) for x in weights))
        ctx.mark_non_differentiable(metrics)
        ctx.set_materialize_grads(False)
        return (*losses.unbind(0), metrics)

    @staticmethod
    def backward(ctx, *grads):
        if all(g is None for g in grads[:6]):
            return (None,) * 8
        hv, ev, zv, hl, el, ws = ctx.saved_tensors
        A, S, d, V, t, eps, nbytes, has_l, lshape, weights = ctx.meta
        gs = [g if g is not None else torch.zeros((), dtype=F32, device=hv.device) for g in grads[:6]]
        gg = torch.stack([g.reshape(()).to(F32) for g in gs])
        dh = torch.empty_like(hv) if ctx.needs_input_grad[0] else None
        dl = torch.empty_like(hl) if (has_l and ctx.needs_input_grad[3]) else None
        w6 = (ctypes.c_float * 6)(*weights)
        call("rte_distill_bwd", ptr(hv), ptr(ev), ptr(zv), A, S, d, ptr(hl), ptr(el), V, t, eps,
             ctypes.addressof(w6), ptr(gg), ptr(ws), nbytes, ptr(dh), ptr(dl), _s())
        return dh, None, None, (dl.view(lshape) if dl is not None else None), None, None, None, None


def distill(hot, exact, h0, hot_logits=None, exact_logits=None, *, temperature: float = 1.0, eps: float = 1e-5,
            weights=(1.0, 1.0, 1.0, 1.0, 1.0, 1.0)):
    """(weighted losses: 6 scalars in the order DISTILL_LOSSES, metrics [10] in the order
    DISTILL_METRICS)."""
    *losses, metrics = DistillFn.apply(hot, exact, h0, hot_logits, exact_logits, temperature, eps, tuple(weights))
    return losses, metrics


# ----------------------------------------------------------------------------- audited-row selection

class _RowSink:
    """Gradients of one select_rows call, waiting for the hook on the source tensor.

    The selection's backward may run on another stream than the consumer of the gradient (the
    audit replay selects h0 rows on a side stream; h0's producer runs its backward on the main
    stream), and autograd inserts no stream wait for a gradient handed over outside its graph.
    Each gradient therefore travels with an event recorded on its producing stream; take()
    makes the consuming stream wait on it and marks the tensor as used there, so the caching
    allocator does not hand its memory to the producing stream's next allocation too early."""

    def __init__(self, idx: torch.Tensor):
        self.idx = idx
        self.grads: list[tuple[torch.Tensor, object]] = []
        self.pending = False

    def put(self, g: torch.Tensor) -> None:
        ev = None
        if g.is_cuda:
            ev = torch.cuda.Event()
            ev.record(torch.cuda.current_stream(g.device))
        self.grads.append((g, ev))

    def take(self) -> list[torch.Tensor]:
        """The stored gradients in arrival order, ordered before the current stream's next work."""
        out = []
        for g, ev in self.grads:
            if ev is not None:
                cur = torch.cuda.current_stream(g.device)
                cur.wait_event(ev)
                g.record_stream(cur)
            out.append(g)
        self.grads.clear()
        return out

    def check_drained(self) -> None:
        if self.grads:
            self.grads.clear()
            raise RuntimeError("select_rows: the selected rows received a gradient but the hook on the source "
                               "tensor that adds them never ran")
        self.pending = False


class SelectRowsFn(torch.autograd.Function):
    """x.index_select(0, idx) whose backward hands its gradient to a hook on x instead of returning a
    full-size gradient: the hook adds the rows into x's accumulated gradient (one index_add over
    the selected rows) in place of a zero fill, a scatter and a full-size add."""

    @staticmethod
    def forward(ctx, x, idx, sink):
        ctx.sink = sink
        ctx.set_materialize_grads(False)
        return x.index_select(0, idx)

    @staticmethod
    def backward(ctx, g):
        sink = ctx.sink
        if g is not None:
            sink.put(g)
            if not sink.pending:  # a backward in which x gets no other gradient must fail loudly
                sink.pending = True
                torch.autograd.Variable._execution_engine.queue_callback(sink.check_drained)
        return None, None, None


def select_rows(x: torch.Tensor, idx: torch.Tensor) -> torch.Tensor:
    """Rows idx of x (dim 0) with the gradient added into x's accumulated gradient by a hook on x.
    The hook returns a new tensor (gx with the rows added; the incoming gradient is never written,
    since a pending node may still hold it) on the stream x's backward runs on, after the
    selection's backward stream has produced the rows.  x must also receive a gradient from its
    other consumers (autograd lets no hook replace a missing gradient): otherwise the backward
    raises.  Leaves and no-grad inputs use index_select."""
    if not (torch.is_grad_enabled() and x.requires_grad and x.grad_fn is not None):
        return x.index_select(0, idx)
    sink = _RowSink(idx)

    def add_rows(gx):
        if not sink.grads:
            return gx
        if gx is None:
            sink.grads.clear()
            raise RuntimeError("select_rows: the source tensor received no gradient besides the selected rows'; "
                               "select with index_select there")
        for g in sink.take():  # in arrival order
            gx = gx.index_add(0, sink.idx, g.to(gx.dtype))
        return gx

    x.register_hook(add_rows)
    return SelectRowsFn.apply(x, idx, sink)


# ----------------------------------------------------------------------------- audit correction

class AuditCorrectFn(torch.autograd.Function):
    """Control-variate audit correction over token losses in one kernel (rte/audit.py:296-321):
    per-sample sums of the hot and exact token losses, residual, clip, corrected losses and the
    residual statistics; the backward broadcasts the per-sample gradient back to the tokens."""

    @staticmethod
    def forward(ctx, hot_tok, exact_tok, idx, p, clip, grad_corrected):
        _lib.require_device_tensors("audit_correct", hot_tok, exact_tok, idx, p)
        B, S = hot_tok.shape
        A = int(idx.numel())
        h = hot_tok.contiguous().to(F32)
        e = None if exact_tok is None or A == 0 else exact_tok.reshape(A, S).contiguous().to(F32)
        ix = idx.reshape(-1).contiguous().to(torch.int64)
        pp = p.reshape(-1).contiguous().to(F32)
        if pp.numel() != B:
            raise ValueError(f"audit_correct: {pp.numel()} probabilities for {B} samples")
        dev = h.device
        corrected = torch.empty((B,), dtype=F32, device=dev)
        exact_ps = torch.empty((A,), dtype=F32, device=dev)
        coef = torch.empty((B + A,), dtype=F32, device=dev)
        stats = torch.empty((4,), dtype=F32, device=dev)
        c = float("inf") if clip is None else float(clip)
        call("rte_audit_correct_fwd", ptr(h), ptr(e), B, S, ptr(ix), A, ptr(pp), c, int(bool(grad_corrected)),
             ptr(corrected), ptr(exact_ps), ptr(coef), ptr(stats), _s())
        ctx.save_for_backward(ix, coef)
        ctx.meta = (B, S, A, hot_tok.dtype, None if exact_tok is None else exact_tok.dtype)
        ctx.mark_non_differentiable(exact_ps, stats)
        ctx.set_materialize_grads(False)
        return corrected, exact_ps, stats

    @staticmethod
    def backward(ctx, g, _g_exact, _g_stats):
        if g is None:
            return (None,) * 6
        ix, coef = ctx.saved_tensors
        B, S, A, h_dt, e_dt = ctx.meta
        gg = g.contiguous().to(F32)
        dh = torch.empty((B, S), dtype=F32, device=gg.device)
        want_e = ctx.needs_input_grad[1] and A > 0
        de = torch.empty((A, S), dtype=F32, device=gg.device) if want_e else None
        call("rte_audit_correct_bwd", ptr(gg), B, S, ptr(ix), A, ptr(coef), ptr(dh), ptr(de), _s())
        return dh.to(h_dt), (de.to(e_dt) if want_e else None), None, None, None, None


def audit_sample_fixed(entropy, recipe_ids, coverage_ema, chosen, *, denom: float, p_min: float, p_max: float,
                       alpha: float, beta: float, gamma: float, residual: float, coverage_min: float):
    """The audit's requested probability (rte/audit.py:79-97) and the fixed-count sampler's mask
    and inclusion probability (rte/audit.py:99-132) in one launch.  Returns (req [B], incl [B],
    mask bool [B], stats [5] = mean incl, mean req, rate, count, mean incl)."""
    _lib.require_device_tensors("audit_sample_fixed", entropy, recipe_ids, coverage_ema, chosen)
    B = entropy.numel()
    k = 0 if chosen is None else chosen.numel()
    dev = entropy.device
    ent = entropy.detach().reshape(B).contiguous().to(F32)
    ids = recipe_ids.detach().reshape(B).contiguous().to(torch.int64)
    ema = coverage_ema.detach().contiguous().to(F32)
    ch = None if chosen is None else chosen.reshape(k).contiguous().to(torch.int64)
    req = torch.empty((B,), dtype=F32, device=dev)
    incl = torch.empty((B,), dtype=F32, device=dev)
    mask = torch.empty((B,), dtype=torch.bool, device=dev)
    stats = torch.empty((5,), dtype=F32, device=dev)
    call("rte_audit_sample_fixed", ptr(ent), ptr(ids), ptr(ema), ptr(ch), B, k, ema.numel(), float(denom),
         float(p_min), float(p_max), float(alpha), float(beta), float(gamma), float(residual), float(coverage_min),
         ptr(req), ptr(incl), ptr(mask), ptr(stats), _s())
    return req, incl, mask, stats


def count_ema(ids, mask, ema, beta: float) -> None:
    """In place: ema = beta ema + (1 - beta) counts / max(sum counts, 1), counts[r] the rows of
    ids equal to r (where mask, if given, is set); ema is a contiguous fp32 device tensor."""
    _lib.require_device_tensors("count_ema", ids, mask, ema)
    if ema.dtype != F32 or not ema.is_contiguous():
        raise TypeError("count_ema: ema must be a contiguous float32 tensor")
    i = ids.detach().reshape(-1).contiguous().to(torch.int64)
    m = None if mask is None else mask.detach().reshape(-1).contiguous().to(torch.bool)
    call("rte_count_ema", ptr(i), ptr(m), i.numel(), ptr(ema), ema.numel(), float(beta), _s())


def nonfinite_flags(x: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """(bad, ok) fp32 scalars: bad = 1 when the scalar x is inf or NaN, else 0; ok = 1 - bad."""
    _lib.require_device_tensors("nonfinite", x)
    xc = x.detach().reshape(1).contiguous().to(F32)
    out = torch.empty((2,), dtype=F32, device=x.device)
    call("rte_nonfinite", ptr(xc), ptr(out), ptr(out[1:]), _s())
    return out[0], out[1]


def step_metrics(hot_lps, corr_lps, depths, *, scale: float, seq: float) -> torch.Tensor:
    """fp32 [4] = mean(hot) / scale, mean(corr) / scale, mean(corr) / seq, mean(depth)."""
    _lib.require_device_tensors("step_metrics", hot_lps, corr_lps, depths)
    B = hot_lps.numel()
    h = hot_lps.detach().reshape(B).contiguous().to(F32)
    c = corr_lps.detach().reshape(B).contiguous().to(F32)
    d = depths.detach().reshape(B).contiguous().to(torch.int64)
    out = torch.empty((4,), dtype=F32, device=h.device)
    call("rte_step_metrics", ptr(h), ptr(c), ptr(d), B, float(scale), float(seq), ptr(out), _s())
    return out


class LossSumFn(torch.autograd.Function):
    """coef * sum(x) + sum of the scalar terms (the step's loss, rte/training.py:1381-1385) in
    one launch; the backward is one fill of dx = coef * g, and each term's gradient is g."""

    @staticmethod
    def forward(ctx, x, coef, *terms):
        xs = x.detach().reshape(-1).contiguous().to(F32)
        ts = [t.detach().reshape(()).to(F32).contiguous() for t in terms]
        out = torch.empty((), dtype=F32, device=xs.device)
        table = (ctypes.c_void_p * max(len(ts), 1))(*[t.data_ptr() for t in ts])
        call("rte_loss_sum", ptr(xs), xs.numel(), float(coef), ctypes.addressof(table), len(ts), ptr(out), _s())
        ctx.n, ctx.coef, ctx.xshape = xs.numel(), float(coef), x.shape
        ctx.tshapes = [t.shape for t in terms]
        return out

    @staticmethod
    def backward(ctx, g):
        g = g.detach().reshape(()).to(F32).contiguous()
        dx = None
        if ctx.needs_input_grad[0]:
            dx = torch.empty((ctx.n,), dtype=F32, device=g.device)
            call("rte_loss_sum_bwd", ptr(g), ctx.n, ctx.coef, ptr(dx), _s())
            dx = dx.view(ctx.xshape)
        return (dx, None, *[g.reshape(sh) if need else None
                            for sh, need in zip(ctx.tshapes, ctx.needs_input_grad[2:])])


def loss_sum(x: torch.Tensor, coef: float, terms) -> torch.Tensor:
    """coef * x.sum() + sum(terms): terms are scalar tensors (up to 32)."""
    _lib.require_device_tensors("loss_sum", x, *terms)
    if len(terms) > 32:
        raise ValueError("loss_sum: at most 32 terms")
    return LossSumFn.apply(x, float(coef), *terms)


def audit_correct(hot_tok, exact_tok, idx, p, *, clip=None, grad_corrected=True):
    """(corrected per-sample loss [B], exact per-sample loss [A], stats [4] = residual mean, std,
    var, corrected metric loss) from token losses hot_tok [B, S] and exact_tok [A, S]."""
    return AuditCorrectFn.apply(hot_tok, exact_tok, idx, p, clip, grad_corrected)


# ----------------------------------------------------------------------------- grouped linear

def group_rows(keys: torch.Tensor, n_groups: int) -> PackIndex:
    """Slot order of rows keyed to groups (ascending row inside a group; keys < 0 dropped)."""
    return pack_index(keys.reshape(-1, 1), n_groups)


class GroupedLinearFn(torch.autograd.Function):
    """y[t] = x[t] @ W[key(t)] with W [G, K, Nout] (one matrix per group), rows grouped by the
    pack of their keys: grouped MFMA GEMMs forward and backward, and the per-group weight
    gradient is the deterministic grouped-K reduction (no per-row weight copies)."""

    @staticmethod
    def forward(ctx, x, w, pk: PackIndex, out_f32: bool = True):
        _lib.require_device_tensors("grouped_linear", x, w)
        shape = x.shape
        K = shape[-1]
        G, K2, Nout = w.shape
        if K2 != K:
            raise ValueError(f"grouped_linear: x has {K} columns, W groups are [{K2}, {Nout}]")
        xb = x.reshape(-1, K).contiguous().to(BF16)
        N = xb.shape[0]
        wb = cast_bf16(w)
        y = torch.empty((N, Nout), dtype=F32 if out_f32 else BF16, device=x.device)
        P = pk.tok_of_slot.numel()
        call("rte_grouped_linear_fwd", ptr(xb), N, K, ptr(pk.offsets), G, P, ptr(pk.tok_of_slot),
             ptr(pk.pair_of_slot), ptr(wb), Nout, ptr(y), int(out_f32), _s())
        ctx.save_for_backward(xb, wb, pk.offsets, pk.tok_of_slot, pk.pair_of_slot)
        ctx.meta = (shape, x.dtype, w.dtype)
        return y.view(*shape[:-1], Nout)

    @staticmethod
    def backward(ctx, dy):
        xb, wb, offsets, tok, pos = ctx.saved_tensors
        shape, x_dt, w_dt = ctx.meta
        N, Nout = xb.shape[0], wb.shape[2]
        dx, dw = _grouped_linear_bwd(cast_bf16(dy.reshape(N, Nout)), xb, wb, offsets, tok, pos,
                                     ctx.needs_input_grad[0], ctx.needs_input_grad[1], x_dt != BF16)
        return (None if dx is None else dx.view(shape).to(x_dt), None if dw is None else dw.to(w_dt), None, None)


def _grouped_linear_fwd(xb, wb, pk: PackIndex, out_f32: bool, tok=None, n_out: int | None = None):
    """y[pair_of_slot] = x[tok] @ W[group] (tok defaults to pk.tok_of_slot; y has n_out rows,
    default the rows of x)."""
    N, K = xb.shape
    G, _, Nout = wb.shape
    tok = pk.tok_of_slot if tok is None else tok
    y = torch.empty((N if n_out is None else n_out, Nout), dtype=F32 if out_f32 else BF16, device=xb.device)
    call("rte_grouped_linear_fwd", ptr(xb), N, K, ptr(pk.offsets), G, tok.numel(), ptr(tok),
         ptr(pk.pair_of_slot), ptr(wb), Nout, ptr(y), int(out_f32), _s())
    return y


def _grouped_linear_bwd(dyb, xb, wb, offsets, tok, pos, need_x: bool, need_w: bool, dx_f32: bool,
                        n_x: int | None = None):
    """(dx [N, K] (fp32 or bf16) or None, dW fp32 [G, K, Nout] or None) of y = x @ W[key]; dx is
    scattered to the rows `tok` (n_x rows, default the rows of x)."""
    G, K, Nout = wb.shape
    N = xb.shape[0] if n_x is None else n_x
    dx = torch.empty((N, K), dtype=F32 if dx_f32 else BF16, device=xb.device) if need_x else None
    dw = torch.empty((G, K, Nout), dtype=F32, device=xb.device) if need_w else None
    P = tok.numel()
    ws, nb = workspace(_lib.load().rte_grouped_linear_bwd_workspace_bytes(P, G, K, Nout), xb.device)
    call("rte_grouped_linear_bwd", ptr(dyb), ptr(xb), N, K, ptr(offsets), G, P, ptr(tok), ptr(pos),
         ptr(wb), Nout, ptr(dx), int(dx_f32), ptr(dw), ws, nb, _s())
    return dx, dw


class MacroBoundedFn(torch.autograd.Function):
    """The bounded-residual macro operator Phi (rte/macro.py:201-236) with the default options
    (no gate, no second hidden layer, no extra input parts):

        z   = [rmsnorm(h) | mean_s rmsnorm(h) | h0]                 (prologue kernel, bf16)
        low = silu(z @ V[key]) @ U[key]                             (grouped MFMA GEMMs)
        out = h + c * scale[key] * tanh(gain[key] * h + low + bias[key])   (epilogue kernel)

    key = recipe * strides + stride per sample.  key may hold more samples than h and h0: sample
    b uses h[b % len(h)] and h0[b % len(h0)] (len(h0) | len(h) | len(key), at most 4 repeats of
    h), so one source batch runs under several keys without copies; z is formed once per source
    sample and the grouped GEMM gathers its rows.  The backward reduces the per-key table and
    matrix gradients in a fixed order and adds the repeats of a source sample in repeat order."""

    @staticmethod
    def forward(ctx, h, h0, key, pk, v, u, gain, bias, scale, c, eps):
        _lib.require_device_tensors("macro_bounded", h, h0, key, v, u, gain, bias, scale)
        Bh, S, d = h.shape
        Bh0 = h0.shape[0]
        kv = key.reshape(-1).contiguous().to(torch.int64)
        B = kv.numel()
        if Bh0 < 1 or Bh % Bh0 or B % Bh or B // Bh > 4 or h0.shape[1:] != h.shape[1:]:
            raise ValueError("macro_bounded: need len(h0) | len(h) | len(key) with at most 4 repeats of h")
        G = v.shape[0] * v.shape[1]
        hv = h.contiguous().to(F32)
        h0v = h0.contiguous().to(F32)
        dev = h.device
        z = torch.empty((Bh * S, 3 * d), dtype=BF16, device=dev)
        rstd = torch.empty((Bh * S,), dtype=F32, device=dev)
        wsb = _lib.load().rte_macro_workspace_bytes(Bh, S, d)
        ws = torch.empty((max(wsb // 4, 1),), dtype=F32, device=dev)
        call("rte_macro_prologue_fwd", ptr(hv), ptr(h0v), Bh, Bh0, S, d, float(eps), ptr(z), ptr(rstd), ptr(ws), wsb,
             _s())
        # rows of z for the slots: pk's rows are b * S + s over all B samples
        tok_z = pk.tok_of_slot if B == Bh else torch.remainder(pk.tok_of_slot, Bh * S)
        vb = cast_bf16(v.reshape(G, v.shape[-2], v.shape[-1]))
        ub = cast_bf16(u.reshape(G, u.shape[-2], u.shape[-1]))
        a = _grouped_linear_fwd(z, vb, pk, out_f32=False, tok=tok_z, n_out=B * S)
        sa = torch.nn.functional.silu(a)
        low = _grouped_linear_fwd(sa, ub, pk, out_f32=True)
        tabs = [t.reshape(G, d).contiguous().to(F32) for t in (gain, bias, scale)]
        out = torch.empty((B, S, d), dtype=F32, device=dev)
        call("rte_macro_epilogue_fwd", ptr(hv), ptr(low), ptr(kv), B, Bh, S, d, ptr(tabs[0]), ptr(tabs[1]),
             ptr(tabs[2]), float(c), ptr(out), _s())
        ctx.save_for_backward(hv, kv, pk.offsets, pk.tok_of_slot, pk.pair_of_slot, tok_z, vb, ub, z, rstd, a, sa,
                              low, *tabs)
        ctx.meta = (B, Bh, Bh0, S, d, G, float(c), v.shape, u.shape, gain.shape, h.dtype, h0.dtype)
        return out.to(h.dtype)

    @staticmethod
    def backward(ctx, dout):
        hv, kv, offsets, tok, pos, tok_z, vb, ub, z, rstd, a, sa, low, tg, tb, ts = ctx.saved_tensors
        B, Bh, Bh0, S, d, G, c, v_shape, u_shape, t_shape, h_dt, h0_dt = ctx.meta
        nia = ctx.needs_input_grad
        dev = hv.device
        do = dout.contiguous().to(F32)
        dh_epi = torch.empty((B, S, d), dtype=F32, device=dev)
        dlow = torch.empty((B * S, d), dtype=BF16, device=dev)
        wsb = _lib.load().rte_macro_workspace_bytes(B, S, d)
        ws = torch.empty((max(wsb // 4, 1),), dtype=F32, device=dev)
        call("rte_macro_epilogue_bwd", ptr(do), ptr(hv), ptr(low), ptr(kv), B, Bh, S, d, ptr(tg), ptr(tb), ptr(ts),
             c, ptr(dh_epi), ptr(dlow), ptr(ws), wsb, _s())
        tabs_out = [torch.empty((G, d), dtype=F32, device=dev) if nia[6 + i] else None for i in range(3)]
        call("rte_macro_table_grad", ptr(kv), B, S, G, d, ptr(ws), *(ptr(t) for t in tabs_out), _s())
        dsa, du = _grouped_linear_bwd(dlow, sa, ub, offsets, tok, pos, True, nia[5], False)
        da = torch.ops.aten.silu_backward(dsa, a)
        if B == Bh:
            dz, dv = _grouped_linear_bwd(da, z, vb, offsets, tok, pos, True, nia[4], False)
        else:
            # dz per sample (its own rows, added over the repeats by the prologue backward);
            # dV gathers the shared z rows
            dz, _ = _grouped_linear_bwd(da, z, vb, offsets, pos, pos, True, False, False, n_x=B * S)
            _, dv = _grouped_linear_bwd(da, z, vb, offsets, tok_z, pos, False, nia[4], False)
        dh = torch.empty((Bh, S, d), dtype=F32, device=dev)
        dh0 = torch.empty((Bh, S, d), dtype=F32, device=dev) if nia[1] else None
        call("rte_macro_prologue_bwd", ptr(dz), ptr(hv), ptr(rstd), ptr(dh_epi), B, Bh, S, d, ptr(dh), ptr(dh0),
             ptr(ws), wsb, _s())
        if dh0 is not None and Bh0 < Bh:
            dh0 = dh0.view(Bh // Bh0, Bh0, S, d).sum(0)

        def tab(i):
            return None if tabs_out[i] is None else tabs_out[i].view(t_shape)

        return (dh.to(h_dt), None if dh0 is None else dh0.to(h0_dt), None, None,
                None if dv is None else dv.view(v_shape), None if du is None else du.view(u_shape),
                tab(0), tab(1), tab(2), None, None)


def macro_bounded(h, h0, key, pk, v, u, gain, bias, scale, c: float, eps: float = 1e-5):
    return MacroBoundedFn.apply(h, h0, key, pk, v, u, gain, bias, scale, c, eps)


# ----------------------------------------------------------------------------- fused macro operator

MACRO_FUSED_RANK = 32


def _whole_param(t: torch.Tensor) -> bool:
    """t is a parameter, or a view covering exactly a parameter's memory (a per-step alias)."""
    if isinstance(t, torch.nn.Parameter):
        return True
    b = t._base
    return (isinstance(b, torch.nn.Parameter) and t.shape == b.shape and t.stride() == b.stride()
            and t.storage_offset() == b.storage_offset())


def macro_fused_supported(v: torch.Tensor, u: torch.Tensor, repeats: int = 1) -> bool:
    """Shapes the fused operator kernels take: hidden rank 32, d a multiple of 128 up to 1024,
    at most 8 repeats of a source sample."""
    if fp32_active():
        return False
    d = u.shape[-1]
    return (v.shape[-1] == MACRO_FUSED_RANK and u.shape[-2] == MACRO_FUSED_RANK and v.shape[-2] == 3 * d
            and d % 128 == 0 and 128 <= d <= 1024 and 1 <= repeats <= 8)


def macro_fused_weights(v: torch.Tensor, u: torch.Tensor):
    """bf16 (V, [V1; V3]^T, V2^T, U, U^T) of V [R, K, 3d, 32] and U [R, K, 32, d] in the layouts the fused
    kernels read, made in one launch; while a per-step cache is open (bf16_cache_begin) they are
    made once per step and stream."""
    _lib.require_device_tensors("macro_fused_weights", v, u)
    G = v.shape[0] * v.shape[1]
    d = u.shape[-1]
    key = None
    if _BF16_CACHE_ON[0] and _whole_param(v) and _whole_param(u):
        key = ("macro_fused", v.data_ptr(), v._version, u.data_ptr(), u._version, _lib.stream_ptr())
        hit = _BF16_CACHE.get(key)
        if hit is not None:
            return hit
    vf = v.detach().reshape(G, 3 * d, MACRO_FUSED_RANK).contiguous().to(F32)
    uf = u.detach().reshape(G, MACRO_FUSED_RANK, d).contiguous().to(F32)
    dev = v.device
    vb = torch.empty((G, 3 * d, MACRO_FUSED_RANK), dtype=BF16, device=dev)
    vct = torch.empty((G, MACRO_FUSED_RANK, 2 * d), dtype=BF16, device=dev)
    v2t = torch.empty((G, MACRO_FUSED_RANK, d), dtype=BF16, device=dev)
    ub = torch.empty((G, MACRO_FUSED_RANK, d), dtype=BF16, device=dev)
    ut = torch.empty((G, d, MACRO_FUSED_RANK), dtype=BF16, device=dev)
    call("rte_macro_fused_prep", ptr(vf), ptr(uf), G, d, ptr(vb), ptr(vct), ptr(v2t), ptr(ub), ptr(ut), _s())
    out = (vb, vct, v2t, ub, ut)
    if key is not None:
        _BF16_CACHE[key] = out
    return out


def macro_fused_weights_share(v, u, stream) -> None:
    """Make this step's fused-operator weight copies (macro_fused_weights) on the current stream
    and let `stream` read the same copies; `stream` must wait on the current stream before it
    uses them.  Outside a per-step cache it does nothing."""
    if not (_BF16_CACHE_ON[0] and _whole_param(v) and _whole_param(u)):
        return
    out = macro_fused_weights(v, u)
    _BF16_CACHE[("macro_fused", v.data_ptr(), v._version, u.data_ptr(), u._version, stream.cuda_stream)] = out
    for t in out:
        t.record_stream(stream)


class _MacroCall:
    """Buffers of one fused operator application (forward outputs saved for the backward).
    Per-sample buffers may be views into larger ones shared by two applications."""

    def __init__(self, h, h0, key, x2, pooled, a, sa, S, d):
        self.h, self.h0, self.key = h, h0, key
        self.Bh, self.Bh0, self.B = h.shape[0], h0.shape[0], key.numel()
        self.S, self.d = S, d
        self.x2, self.pooled, self.a, self.sa = x2, pooled, a, sa
        dev = h.device
        self.rstd = torch.empty((self.Bh * S,), dtype=F32, device=dev)
        self.P = torch.empty((self.B, MACRO_FUSED_RANK), dtype=F32, device=dev)
        self.out = torch.empty((self.B, S, d), dtype=F32, device=dev)

    def forward(self, G, eps, w, tabs, c, mse_ref=None, mse_part=None):
        vb, vct, v2t, ub, ut = w
        nb = _lib.load().rte_macro_fused_fwd_workspace_bytes(self.Bh, self.S, self.d)
        ws, nbytes = workspace(nb, self.h.device)
        call("rte_macro_fused_fwd", ptr(self.h), ptr(self.h0), self.Bh, self.Bh0, ptr(self.key), self.B, self.S,
             self.d, G, float(eps), ptr(vb), ptr(vct), ptr(ut), ptr(tabs[0]), ptr(tabs[1]), ptr(tabs[2]), float(c),
             ptr(self.x2), ptr(self.rstd), ptr(self.pooled), ptr(self.P), ptr(self.a), ptr(self.sa), ptr(self.out),
             ptr(mse_ref), ptr(mse_part), ws, nbytes, _s())

    def backward(self, G, w, tabs, c, du, da, part_tab, part_da, dsum, dh, *, dout=None, dout_lo=0, diff=None,
                 diff_lo=0, dh0=None, dh0_into_dh=False, extra=None, n_extra=0):
        """The upstream gradient of sample b: mul g (p - q)[b - diff_lo] for the len(p) samples from
        diff_lo on (diff = (p, q, g, mul)), plus dout[b - dout_lo] for the len(dout) samples from
        dout_lo on; the two ranges may overlap."""
        vb, vct, v2t, ub, ut = w
        p, q, g, mul = diff if diff is not None else (None, None, None, 0.0)
        n_diff = 0 if p is None else p.shape[0]
        n_dout = 0 if dout is None else dout.shape[0]
        nb = _lib.load().rte_macro_fused_bwd_workspace_bytes(self.B, self.S)
        ws, nbytes = workspace(nb, self.h.device)
        call("rte_macro_fused_bwd", ptr(p), ptr(q), ptr(g), float(mul), int(diff_lo), n_diff, ptr(dout),
             int(dout_lo), n_dout, ptr(self.h),
             ptr(self.rstd), ptr(self.x2), self.Bh, ptr(self.key), self.B, self.S, self.d, G, ptr(self.a),
             ptr(self.sa), ptr(vb), ptr(vct), ptr(v2t), ptr(ub), ptr(ut), ptr(tabs[0]), ptr(tabs[1]), ptr(tabs[2]),
             float(c), ptr(du), ptr(da), ptr(part_tab), ptr(part_da), ptr(dh), ptr(dh0), int(dh0_into_dh), ptr(extra),
             int(n_extra), ptr(dsum), ws, nbytes, _s())


def _macro_tabs(gain, bias, scale, G, d):
    return [t.detach().reshape(G, d).contiguous().to(F32) for t in (gain, bias, scale)]


def _macro_wgrad(keys, B0, Bh0, B1, Bh1, S, d, G, x2, sa, du, da, pooled, dsum, part_tab, need, v_shape, u_shape,
                 t_shape, dev):
    """(dV, dU, dgain, dbias, dscale) of one or two operator applications listed together."""
    dU = torch.empty((G, MACRO_FUSED_RANK, d), dtype=F32, device=dev) if need[1] else None
    dV = torch.empty((G, 3 * d, MACRO_FUSED_RANK), dtype=F32, device=dev) if need[0] else None
    tabs = [torch.empty((G, d), dtype=F32, device=dev) if need[2 + i] else None for i in range(3)]
    nb = _lib.load().rte_macro_fused_wgrad_workspace_bytes(B0 + B1, S, d, G)
    ws, nbytes = workspace(nb, dev)
    call("rte_macro_fused_wgrad", ptr(keys), B0, Bh0, B1, Bh1, S, d, G, ptr(x2), ptr(sa), ptr(du), ptr(da),
         ptr(pooled), ptr(dsum), ptr(part_tab), ptr(dU), ptr(dV), ptr(tabs[0]), ptr(tabs[1]), ptr(tabs[2]), ws,
         nbytes, _s())
    return (None if dV is None else dV.view(v_shape), None if dU is None else dU.view(u_shape),
            *(None if t is None else t.view(t_shape) for t in tabs))


class MacroFusedFn(torch.autograd.Function):
    """The bounded-residual macro operator Phi (rte/macro.py:201-236, default options) at hidden
    rank 32 on the fused kernels:

        a   = [rmsnorm(h) | h0] @ [V1; V3][key] + mean_s(rmsnorm(h)) @ V2[key]
        out = h + c * scale[key] * tanh(gain[key] * h + silu(a) @ U[key] + bias[key])

    (the reference's z = [rmsnorm(h) | mean | h0] @ V, split by rows of V).  Sample b reads
    h[b % len(h)] and h0[b % len(h0)] (len(h0) | len(h) | len(key), at most 8 repeats).  One
    workgroup owns 64 rows of one sample, so its products use a single key's matrices; weight
    gradients are grouped-K reductions over each key's rows in a fixed order."""

    @staticmethod
    def forward(ctx, h, h0, key, v, u, gain, bias, scale, c, eps):
        _lib.require_device_tensors("macro_fused", h, h0, key, v, u, gain, bias, scale)
        Bh, S, d = h.shape
        Bh0 = h0.shape[0]
        kv = key.reshape(-1).contiguous().to(torch.int64)
        B = kv.numel()
        if Bh0 < 1 or Bh % Bh0 or B % Bh or B // Bh > 8 or h0.shape[1:] != h.shape[1:]:
            raise ValueError("macro_fused: need len(h0) | len(h) | len(key) with at most 8 repeats of h")
        if not macro_fused_supported(v, u, B // Bh):
            raise ValueError("macro_fused: needs hidden rank 32 and d a multiple of 128 up to 1024")
        G = v.shape[0] * v.shape[1]
        same = h is h0
        hv = h.detach().contiguous().to(F32)
        h0v = hv if same else h0.detach().contiguous().to(F32)
        dev = h.device
        w = macro_fused_weights(v, u)
        tabs = _macro_tabs(gain, bias, scale, G, d)
        x2 = torch.empty((Bh * S, 2 * d), dtype=BF16, device=dev)
        pooled = torch.empty((Bh, d), dtype=BF16, device=dev)
        a = torch.empty((B * S, MACRO_FUSED_RANK), dtype=F32, device=dev)
        sa = torch.empty((B * S, MACRO_FUSED_RANK), dtype=BF16, device=dev)
        mc = _MacroCall(hv, h0v, kv, x2, pooled, a, sa, S, d)
        mc.forward(G, eps, w, tabs, c)
        out, mc.out = mc.out, None  # the output is not needed by the backward
        mc.h = mc.h0 = None         # saved below (version-checked)
        ctx.save_for_backward(hv)
        ctx.mc, ctx.w, ctx.tabs = mc, w, tabs
        ctx.meta = (G, float(c), same, v.shape, u.shape, gain.shape, h.dtype, h0.dtype)
        return out.to(h.dtype)

    @staticmethod
    def backward(ctx, dout):
        mc, w, tabs = ctx.mc, ctx.w, ctx.tabs
        (mc.h,) = ctx.saved_tensors
        G, c, same, v_shape, u_shape, t_shape, h_dt, h0_dt = ctx.meta
        nia = ctx.needs_input_grad
        B, Bh, Bh0, S, d = mc.B, mc.Bh, mc.Bh0, mc.S, mc.d
        dev = mc.h.device
        T = (S + 31) // 32
        do = dout.contiguous().to(F32)
        du = torch.empty((B * S, d), dtype=BF16, device=dev)
        da = torch.empty((B * S, MACRO_FUSED_RANK), dtype=BF16, device=dev)
        part_tab = torch.empty((B * T * 3 * d,), dtype=F32, device=dev)
        part_da = torch.empty((B * T * MACRO_FUSED_RANK,), dtype=F32, device=dev)
        dsum = torch.empty((B, MACRO_FUSED_RANK), dtype=BF16, device=dev)
        dh = torch.empty((Bh, S, d), dtype=F32, device=dev)
        want_h0 = nia[1] and not same
        dh0 = torch.empty((Bh, S, d), dtype=F32, device=dev) if want_h0 else None
        mc.backward(G, w, tabs, c, du, da, part_tab, part_da, dsum, dh, dout=do, dh0=dh0, dh0_into_dh=same)
        grads = _macro_wgrad(mc.key, B, Bh, 0, 0, S, d, G, mc.x2, mc.sa, du, da, mc.pooled, dsum, part_tab,
                             nia[3:8], v_shape, u_shape, t_shape, dev)
        if dh0 is not None and Bh0 < Bh:
            dh0 = dh0.view(Bh // Bh0, Bh0, S, d).sum(0)
        ctx.mc = ctx.w = ctx.tabs = None
        return (dh.to(h_dt), None if dh0 is None else dh0.to(h0_dt), None, *grads, None, None)


def macro_fused(h, h0, key, v, u, gain, bias, scale, c: float, eps: float = 1e-5):
    return MacroFusedFn.apply(h, h0, key, v, u, gain, bias, scale, c, eps)


class MacroConsistencyFn(torch.autograd.Function):
    """The macro consistency loss (rte/macro.py:342-359) on the fused operator:
    mse(Phi_{dst}(h), Phi_{src}(Phi_{src}(h))) over every (s, 2s) stride pair and sample.

    The first application runs nf key blocks of the b source samples of h (key_first, one h row
    block per source, nf <= 8): the pc src blocks from block src_lo on and the pc dst blocks from
    block dst_lo on.  When the stride pairs chain ((1, 2), (2, 4)) the src and dst ranges overlap
    and a shared key block is computed once.  The second application reads the src blocks of the
    first one's output with h0 = h.  The MSE is summed inside the second application's forward
    kernel (per-tile partial sums, fixed order).  The backward takes the MSE gradient inside the
    operator kernels (no difference tensors), feeds the second application's dh straight into
    the first one's src blocks (added to the MSE gradient of a block that is also a dst block),
    adds every path to h in the kernels, and reduces the weight gradients of both applications
    in one grouped pass."""

    @staticmethod
    def forward(ctx, h, key_first, key_src, src_lo, dst_lo, v, u, gain, bias, scale, c, eps):
        _lib.require_device_tensors("macro_consistency", h, key_first, key_src, v, u, gain, bias, scale)
        b, S, d = h.shape
        kf = key_first.reshape(-1).contiguous().to(torch.int64)
        ks = key_src.reshape(-1).contiguous().to(torch.int64)
        pcb, B0 = ks.numel(), kf.numel()
        if pcb == 0 or pcb % b or B0 % b or B0 // b > 8:
            raise ValueError("macro_consistency: need nf b first keys (nf <= 8) and pc b second keys")
        nf, pc = B0 // b, pcb // b
        if not (0 <= src_lo <= nf - pc and 0 <= dst_lo <= nf - pc):
            raise ValueError("macro_consistency: src / dst key blocks outside the first application")
        if not macro_fused_supported(v, u, nf):
            raise ValueError("macro_consistency: needs hidden rank 32 and d a multiple of 128 up to 1024")
        G = v.shape[0] * v.shape[1]
        dev = h.device
        hv = h.detach().contiguous().to(F32)
        w = macro_fused_weights(v, u)
        tabs = _macro_tabs(gain, bias, scale, G, d)
        R = MACRO_FUSED_RANK
        x2 = torch.empty(((b + pcb) * S, 2 * d), dtype=BF16, device=dev)
        pooled = torch.empty((b + pcb, d), dtype=BF16, device=dev)
        a = torch.empty(((B0 + pcb) * S, R), dtype=F32, device=dev)
        sa = torch.empty(((B0 + pcb) * S, R), dtype=BF16, device=dev)
        n0 = B0 * S
        first_call = _MacroCall(hv, hv, kf, x2[:b * S], pooled[:b], a[:n0], sa[:n0], S, d)
        first_call.forward(G, eps, w, tabs, c)
        s0, d0 = src_lo * b, dst_lo * b
        first, direct = first_call.out[s0:s0 + pcb], first_call.out[d0:d0 + pcb]
        T = (S + 31) // 32
        mse_part = torch.empty((pcb * T,), dtype=F32, device=dev)
        twice = _MacroCall(first, hv, ks, x2[b * S:], pooled[b:], a[n0:], sa[n0:], S, d)
        twice.forward(G, eps, w, tabs, c, mse_ref=direct, mse_part=mse_part)
        n = pcb * S * d
        loss = torch.empty((), dtype=F32, device=dev)
        call("rte_macro_fused_sum", ptr(mse_part), mse_part.numel(), float(1.0 / n), ptr(loss), _s())
        ctx.calls = (first_call, twice)
        ctx.bufs = (x2, pooled, a, sa, torch.cat([kf, ks]))
        ctx.w, ctx.tabs = w, tabs
        ctx.meta = (G, float(c), b, B0, pcb, s0, d0, S, d, n, v.shape, u.shape, gain.shape, h.dtype)
        return loss

    @staticmethod
    def backward(ctx, g):
        first_call, twice = ctx.calls
        x2, pooled, a, sa, keys = ctx.bufs
        w, tabs = ctx.w, ctx.tabs
        G, c, b, B0, pcb, s0, d0, S, d, n, v_shape, u_shape, t_shape, h_dt = ctx.meta
        nia = ctx.needs_input_grad
        dev = a.device
        R = MACRO_FUSED_RANK
        T = (S + 31) // 32
        gv = g.reshape(1).contiguous().to(F32)
        mul = 2.0 / n
        nb = B0 + pcb
        du = torch.empty((nb * S, d), dtype=BF16, device=dev)
        da = torch.empty((nb * S, R), dtype=BF16, device=dev)
        part_tab = torch.empty((nb * T * 3 * d,), dtype=F32, device=dev)
        part_da = torch.empty((nb * T * R,), dtype=F32, device=dev)
        dsum = torch.empty((nb, R), dtype=BF16, device=dev)
        n0 = B0 * S
        t0, r0 = B0 * T * 3 * d, B0 * T * R
        direct = first_call.out[d0:d0 + pcb]
        # second application: d loss / d twice = mul g (twice - direct); its dh is the upstream
        # gradient of the first application's src blocks, its dh0 goes to h
        d_first = torch.empty((pcb, S, d), dtype=F32, device=dev)
        dh0_tw = torch.empty((pcb, S, d), dtype=F32, device=dev)
        twice.backward(G, w, tabs, c, du[n0:], da[n0:], part_tab[t0:], part_da[r0:], dsum[B0:], d_first,
                       diff=(twice.out, direct, gv, mul), dh0=dh0_tw)
        # first application: dst blocks mul g (direct - twice), src blocks d_first (both where
        # they overlap), other blocks 0; h = h0 = h
        dh = torch.empty((b, S, d), dtype=F32, device=dev)
        first_call.backward(G, w, tabs, c, du[:n0], da[:n0], part_tab[:t0], part_da[:r0], dsum[:B0], dh,
                            dout=d_first, dout_lo=s0, diff=(direct, twice.out, gv, mul), diff_lo=d0,
                            dh0_into_dh=True, extra=dh0_tw, n_extra=pcb // b)
        grads = _macro_wgrad(keys, B0, b, pcb, pcb, S, d, G, x2, sa, du, da, pooled, dsum, part_tab,
                             nia[5:10], v_shape, u_shape, t_shape, dev)
        ctx.calls = ctx.bufs = ctx.w = ctx.tabs = None
        return (dh.to(h_dt) if nia[0] else None, None, None, None, None, *grads, None, None)


MACRO_CONS_MAX_KEYS = 4
# the one-pass consistency kernels (csrc/macro_cons.hip) where their shapes allow; off: the
# per-application fused operator calls of MacroConsistencyFn
MACRO_CONS_ONE_PASS = [True]


def macro_cons_supported(v: torch.Tensor, u: torch.Tensor, S: int, nf: int, pc: int) -> bool:
    """Shapes the one-pass consistency kernels take: hidden rank 32, d = 256 or 512, at most 64
    positions, 1 <= pc <= nf <= 4 key blocks."""
    if fp32_active():
        return False
    d = u.shape[-1]
    return (v.shape[-1] == MACRO_FUSED_RANK and u.shape[-2] == MACRO_FUSED_RANK and v.shape[-2] == 3 * d
            and d in (256, 512) and 1 <= S <= 64 and 1 <= pc <= nf <= MACRO_CONS_MAX_KEYS)


def macro_cons_weights(v: torch.Tensor, u: torch.Tensor):
    """bf16 [V1 | V3]^T [G, 32, 2d] and U [G, 32, d] with the middle two 4-column quads of every
    16 columns swapped (the operand order of the one-pass consistency kernels), once per step
    and stream while a per-step cache is open."""
    _lib.require_device_tensors("macro_cons_weights", v, u)
    G = v.shape[0] * v.shape[1]
    d = u.shape[-1]
    key = None
    if _BF16_CACHE_ON[0] and _whole_param(v) and _whole_param(u):
        key = ("macro_cons", v.data_ptr(), v._version, u.data_ptr(), u._version, _lib.stream_ptr())
        hit = _BF16_CACHE.get(key)
        if hit is not None:
            return hit
    vf = v.detach().reshape(G, 3 * d, MACRO_FUSED_RANK).contiguous().to(F32)
    uf = u.detach().reshape(G, MACRO_FUSED_RANK, d).contiguous().to(F32)
    vq = torch.empty((G, MACRO_FUSED_RANK, 2 * d), dtype=BF16, device=v.device)
    uq = torch.empty((G, MACRO_FUSED_RANK, d), dtype=BF16, device=v.device)
    call("rte_macro_cons_prep", ptr(vf), ptr(uf), G, d, ptr(vq), ptr(uq), _s())
    out = (vq, uq)
    if key is not None:
        _BF16_CACHE[key] = out
    return out


class MacroConsOnePassFn(torch.autograd.Function):
    """The macro consistency loss (rte/macro.py:342-359) for at most 64 positions and d = 256 or
    512 on the one-pass kernels: one workgroup per 32 rows of a sample runs the first
    application's codes, the second application and the squared differences (three launches),
    and the backward in three more; out and Phi(out) are recomputed from h and the rank-32
    codes instead of being stored.  Key layout and weight gradients as MacroConsistencyFn (the
    grouped reductions of the fused operator)."""

    @staticmethod
    def forward(ctx, h, key_first, key_src, src_lo, dst_lo, v, u, gain, bias, scale, c, eps):
        _lib.require_device_tensors("macro_cons", h, key_first, key_src, v, u, gain, bias, scale)
        b, S, d = h.shape
        kf = key_first.reshape(-1).contiguous().to(torch.int64)
        ks = key_src.reshape(-1).contiguous().to(torch.int64)
        if kf.numel() % b or ks.numel() % b:
            raise ValueError("macro_cons: need nf b first keys and pc b second keys")
        nf, pc = kf.numel() // b, ks.numel() // b
        if not macro_cons_supported(v, u, S, nf, pc):
            raise ValueError("macro_cons: needs rank 32, d = 256 or 512, S <= 64, 1 <= pc <= nf <= 4")
        if not (0 <= src_lo <= nf - pc and 0 <= dst_lo <= nf - pc):
            raise ValueError("macro_cons: src / dst key blocks outside the first application")
        G = v.shape[0] * v.shape[1]
        dev = h.device
        hv = h.detach().contiguous().to(F32)
        vb, _, _, _, ut = macro_fused_weights(v, u)
        vq, uq = macro_cons_weights(v, u)
        tabs = _macro_tabs(gain, bias, scale, G, d)
        R = MACRO_FUSED_RANK
        x2 = torch.empty(((b + pc * b) * S, 2 * d), dtype=BF16, device=dev)
        pooled = torch.empty((b + pc * b, d), dtype=BF16, device=dev)
        a = torch.empty(((nf + pc) * b * S, R), dtype=F32, device=dev)
        sa = torch.empty(((nf + pc) * b * S, R), dtype=BF16, device=dev)
        rstd = torch.empty(((1 + pc) * b * S,), dtype=F32, device=dev)
        loss = torch.empty((), dtype=F32, device=dev)
        ws, nbytes = workspace(_lib.load().rte_macro_cons_workspace_bytes(b, S, d, pc), dev)
        call("rte_macro_cons_fwd", ptr(hv), b, S, d, ptr(kf), nf, ptr(ks), pc, int(src_lo), int(dst_lo), G,
             float(eps), ptr(vb), ptr(vq), ptr(ut), ptr(uq), ptr(tabs[0]), ptr(tabs[1]), ptr(tabs[2]), float(c),
             ptr(x2), ptr(pooled), ptr(a), ptr(sa), ptr(rstd), ptr(loss), ws, nbytes, _s())
        ctx.save_for_backward(hv)
        ctx.bufs = (kf, ks, x2, pooled, a, sa, rstd, vb, ut, uq, tabs)
        ctx.meta = (G, float(c), b, S, d, nf, pc, int(src_lo), int(dst_lo), v.shape, u.shape, gain.shape, h.dtype)
        return loss

    @staticmethod
    def backward(ctx, g):
        (hv,) = ctx.saved_tensors
        kf, ks, x2, pooled, a, sa, rstd, vb, ut, uq, tabs = ctx.bufs
        G, c, b, S, d, nf, pc, src_lo, dst_lo, v_shape, u_shape, t_shape, h_dt = ctx.meta
        nia = ctx.needs_input_grad
        dev = hv.device
        R = MACRO_FUSED_RANK
        T = (S + 31) // 32
        nb = (nf + pc) * b
        gv = g.reshape(1).contiguous().to(F32)
        du = torch.empty((nb * S, d), dtype=BF16, device=dev)
        da = torch.empty((nb * S, R), dtype=BF16, device=dev)
        part_tab = torch.empty((nb * T * 3 * d,), dtype=F32, device=dev)
        part_da = torch.empty((nb * T * R,), dtype=F32, device=dev)
        dsum = torch.empty((nb, R), dtype=BF16, device=dev)
        dh = torch.empty((b, S, d), dtype=F32, device=dev)
        mul = 2.0 / (pc * b * S * d)
        call("rte_macro_cons_bwd", ptr(hv), b, S, d, ptr(kf), nf, ptr(ks), pc, src_lo, dst_lo, G, ptr(vb), ptr(ut),
             ptr(uq), ptr(tabs[0]), ptr(tabs[1]), ptr(tabs[2]), c, ptr(a), ptr(sa), ptr(rstd), ptr(gv), float(mul),
             ptr(du), ptr(da), ptr(part_tab), ptr(part_da), ptr(dsum), ptr(dh), _s())
        if ks.data_ptr() == kf.data_ptr() + kf.numel() * kf.element_size():
            keys = kf.as_strided((kf.numel() + ks.numel(),), (1,))  # ks follows kf in memory
        else:
            keys = torch.cat([kf, ks])
        grads = _macro_wgrad(keys, nf * b, b, pc * b, pc * b, S, d, G, x2, sa, du, da, pooled, dsum, part_tab,
                             nia[5:10], v_shape, u_shape, t_shape, dev)
        ctx.bufs = None
        return (dh.to(h_dt) if nia[0] else None, None, None, None, None, *grads, None, None)


def macro_consistency(h, key_first, key_src, v, u, gain, bias, scale, c: float, eps: float = 1e-5, *,
                      src_lo: int | None = None, dst_lo: int = 0):
    """key_first: the first application's nf key blocks of len(h) samples; key_src: the pc src
    blocks, which sit from block src_lo on in key_first (default nf - pc: the [dst; src] layout),
    the dst blocks from block dst_lo on."""
    b = h.shape[0]
    nf, pc = key_first.numel() // b, key_src.numel() // b
    lo = nf - pc if src_lo is None else int(src_lo)
    if MACRO_CONS_ONE_PASS[0] and macro_cons_supported(v, u, h.shape[1], nf, pc):
        return MacroConsOnePassFn.apply(h, key_first, key_src, lo, int(dst_lo), v, u, gain, bias, scale, c, eps)
    return MacroConsistencyFn.apply(h, key_first, key_src, lo, int(dst_lo), v, u, gain, bias, scale, c, eps)


class MseFn(torch.autograd.Function):
    """mean((a - b)^2) over all elements (F.mse_loss with mean reduction), fp32, in a fixed
    reduction order."""

    @staticmethod
    def forward(ctx, a, b):
        _lib.require_device_tensors("mse", a, b)
        if a.shape != b.shape or a.numel() == 0:
            raise ValueError("mse: a and b need the same non-empty shape")
        av, bv = a.contiguous().to(F32), b.contiguous().to(F32)
        n = av.numel()
        out = torch.empty((), dtype=F32, device=a.device)
        wsb = _lib.load().rte_mse_workspace_bytes(n)
        ws = torch.empty((max(wsb // 4, 1),), dtype=F32, device=a.device)
        call("rte_mse_fwd", ptr(av), ptr(bv), n, ptr(out), ptr(ws), wsb, _s())
        ctx.save_for_backward(av, bv)
        ctx.dtypes = (a.dtype, b.dtype)
        return out

    @staticmethod
    def backward(ctx, g):
        av, bv = ctx.saved_tensors
        nia = ctx.needs_input_grad
        gv = g.reshape(1).contiguous().to(F32)
        da = torch.empty_like(av) if nia[0] else None
        db = torch.empty_like(bv) if nia[1] else None
        call("rte_mse_bwd", ptr(av), ptr(bv), av.numel(), ptr(gv), ptr(da), ptr(db), _s())
        return (None if da is None else da.to(ctx.dtypes[0]), None if db is None else db.to(ctx.dtypes[1]))


def mse(a, b):
    return MseFn.apply(a, b)


def grouped_linear(x, w, pk: PackIndex, *, out_f32: bool = True):
    """Rows of x keyed by pk's groups times their group's matrix; every key must be valid."""
    if fp32_active():
        return _f32().grouped_linear(x, w, pk)
    return GroupedLinearFn.apply(x, w, pk, out_f32)


# ----------------------------------------------------------------------------- segmented row reduction

def segment_reduce_rows(keys, n_keys: int, rows, *, w=None, row_div: int = 1, out=None,
                        accumulate: bool = False) -> torch.Tensor:
    """out[v] (+)= sum over p with keys[p] = v of w[p] * rows[p // row_div] (fp32 [n_keys, d]),
    summed in a fixed order (deterministic, no atomics); keys outside [0, n_keys) are skipped."""
    _lib.require_device_tensors("segment_reduce_rows", keys, rows, w, out)
    k = keys.reshape(-1).contiguous().to(torch.int32)
    d = rows.shape[-1]
    r = rows.reshape(-1, d)
    if r.dtype not in (F32, BF16):
        r = r.to(F32)
    r = r.contiguous()
    if out is None:
        out = torch.empty((n_keys, d), dtype=F32, device=r.device)
        accumulate = False
    wc = None if w is None else w.reshape(-1).contiguous().to(F32)
    ws, nb = workspace(_lib.load().rte_segment_reduce_workspace_bytes(k.numel(), n_keys, d), r.device)
    call("rte_segment_reduce_rows", ptr(k), k.numel(), n_keys, int(row_div), ptr(wc), ptr(r), int(r.dtype == F32), d,
         ptr(out), int(accumulate), ws, nb, _s())
    return out


class EmbeddingFn(torch.autograd.Function):
    """weight[ids] with a deterministic backward: dW[v] = sum of the output gradients of the
    positions holding id v, reduced in a fixed order (replaces the embedding backward's
    sort + atomic scatter)."""

    @staticmethod
    def forward(ctx, weight, ids):
        _lib.require_device_tensors("embedding", weight, ids)
        out = weight.index_select(0, ids.reshape(-1)).view(*ids.shape, weight.shape[1])
        ctx.save_for_backward(ids)
        ctx.n = weight.shape[0]
        return out

    @staticmethod
    def backward(ctx, dout):
        (ids,) = ctx.saved_tensors
        dw = segment_reduce_rows(ids, ctx.n, dout.reshape(-1, dout.shape[-1]))
        return dw, None


def embedding(weight, ids):
    return EmbeddingFn.apply(weight, ids)


# ----------------------------------------------------------------------------- shortlist output head

def shortlist_build(targets, top_clusters, members, hard_negatives: int, random_negs, max_tokens: int,
                    vocab_size: int) -> tuple[torch.Tensor, torch.Tensor]:
    """First max_tokens distinct ids of [target | top-cluster members | hard | random | filler |
    target filler] per token (rte/output.py:46-110).  Returns (shortlist int32 [..., L],
    dup_per_token int32 [...]); the target sits at position 0."""
    _lib.require_device_tensors("shortlist_build", targets, top_clusters, members, random_negs)
    shape = targets.shape
    tg = targets.reshape(-1).contiguous().to(torch.int64)
    T = tg.shape[0]
    top = top_clusters.reshape(T, top_clusters.shape[-1]).contiguous().to(torch.int32)
    mem = members.contiguous().to(torch.int64)
    rnd = random_negs.reshape(T, random_negs.shape[-1]).contiguous().to(torch.int64)
    sl = torch.empty((T, max_tokens), dtype=torch.int32, device=tg.device)
    dup = torch.empty((T,), dtype=torch.int32, device=tg.device)
    call("rte_shortlist_build", ptr(tg), ptr(top), top.shape[1], ptr(mem), mem.shape[0], mem.shape[1], ptr(rnd),
         rnd.shape[1], int(hard_negatives), int(max_tokens), int(vocab_size), T, ptr(sl), ptr(dup), _s())
    return sl.view(*shape, max_tokens), dup.view(shape)


class ShortlistCEFn(torch.autograd.Function):
    """Shortlist logits hidden . W[shortlist] (fp32) and the per-token CE against position 0
    in one kernel; the backward fuses the CE gradient with any gradient on the logits and
    reduces the vocabulary-row gradient deterministically."""

    @staticmethod
    def forward(ctx, hidden, w, shortlist):
        _lib.require_device_tensors("shortlist_ce", hidden, w, shortlist)
        shape = hidden.shape
        d = shape[-1]
        hb = hidden.reshape(-1, d).contiguous().to(BF16)
        wb = cast_bf16(w)
        T, V = hb.shape[0], wb.shape[0]
        sl = shortlist.reshape(T, -1).contiguous().to(torch.int32)
        L = sl.shape[1]
        logits = torch.empty((T, L), dtype=F32, device=hb.device)
        lse = torch.empty((T,), dtype=F32, device=hb.device)
        loss = torch.empty((T,), dtype=F32, device=hb.device)
        call("rte_shortlist_fwd", ptr(hb), ptr(wb), d, V, ptr(sl), L, T, ptr(logits), ptr(lse), ptr(loss), _s())
        ctx.save_for_backward(hb, wb, sl, logits, lse)
        ctx.meta = (shape, hidden.dtype, w.dtype)
        return logits.view(*shape[:-1], L), loss.view(shape[:-1])

    @staticmethod
    def backward(ctx, dlogits_ext, dloss):
        hb, wb, sl, logits, lse = ctx.saved_tensors
        shape, h_dt, w_dt = ctx.meta
        T, L = logits.shape
        V, d = wb.shape
        ext = None if dlogits_ext is None else dlogits_ext.reshape(T, L).contiguous().to(F32)
        g = None if dloss is None else dloss.reshape(T).contiguous().to(F32)
        need_h, need_w = ctx.needs_input_grad[0], ctx.needs_input_grad[1]
        dh = torch.empty((T, d), dtype=BF16, device=hb.device) if need_h else None
        dw = torch.empty((V, d), dtype=F32, device=hb.device) if need_w else None
        ws, nb = workspace(_lib.load().rte_shortlist_bwd_workspace_bytes(T, L, V, d), hb.device)
        call("rte_shortlist_bwd", ptr(g), ptr(ext), ptr(hb), ptr(wb), d, V, ptr(sl), L, T, ptr(logits), ptr(lse),
             ptr(dh), ptr(dw), 0, ws, nb, _s())
        return (None if dh is None else dh.view(shape).to(h_dt),
                None if dw is None else dw.to(w_dt), None)


def shortlist_ce(hidden, w, shortlist):
    """(shortlist logits fp32 [..., L], per-token CE against position 0 [...])."""
    if fp32_active():
        return _f32().shortlist_ce(hidden, w, shortlist)
    return ShortlistCEFn.apply(hidden, w, shortlist)


# ----------------------------------------------------------------------------- SVD low-rank SwiGLU FFN

def svd_ffn_fused_supported(T: int, d: int, F: int, r: int) -> bool:
    """Shapes the on-chip SVD FFN path takes (rte_svd_ffn_fused_*); others use the four-GEMM path."""
    return r in (64, 128) and F % 128 == 0 and d % 8 == 0 and T % 8 == 0


class SVDFFNFn(torch.autograd.Function):
    """y = resid + SwiGLU FFN whose up / gate / down weights are rank-r factors.

    us_ug [d, 2r] = [U_up S_up | U_gate S_gate], v_ug [2F, r] = [V_up ; V_gate],
    v_dn [F, r], us_dn [d, r] = U_dn S_dn.  For rank 64 / 128 the [T, 2F] activations and the
    [T, F] SwiGLU output stay on chip (rte_svd_ffn_fused_*: the backward recomputes them);
    otherwise four MFMA GEMMs forward (the expand GEMM fuses SwiGLU and reads each half's
    low-rank code), eleven backward."""

    @staticmethod
    def forward(ctx, x, us_ug, v_ug, v_dn, us_dn, resid):
        _lib.require_device_tensors("svd_ffn", x, us_ug, v_ug, v_dn, us_dn, resid)
        shape = x.shape
        d = shape[-1]
        xb = x.reshape(-1, d).contiguous().to(BF16)
        T = xb.shape[0]
        r = us_dn.shape[1]
        F = v_dn.shape[0]
        w = [cast_bf16(t) for t in (us_ug, v_ug, v_dn, us_dn)]
        dev = x.device
        fused = svd_ffn_fused_supported(T, d, F, r)
        a_ug = torch.empty((T, 2 * r), dtype=BF16, device=dev)
        b = torch.empty((T, r), dtype=BF16, device=dev)
        y = torch.empty((T, d), dtype=F32, device=dev)
        rs = None if resid is None else resid.reshape(T, d).contiguous().to(F32)
        if fused:
            wsp, wsn = workspace(_lib.load().rte_svd_ffn_fused_workspace_bytes(T, d, F, r), dev)
            call("rte_svd_ffn_fused_fwd", ptr(xb), T, d, F, r, *[ptr(t) for t in w], ptr(rs), ptr(a_ug), ptr(b),
                 ptr(y), 1, wsp, wsn, _s())
            ctx.save_for_backward(xb, *w, a_ug, b)
        else:
            ug = torch.empty((T, 2 * F), dtype=BF16, device=dev)
            z = torch.empty((T, F), dtype=BF16, device=dev)
            call("rte_svd_ffn_fwd", ptr(xb), T, d, F, r, *[ptr(t) for t in w], ptr(rs), ptr(a_ug), ptr(ug),
                 ptr(z), ptr(b), ptr(y), 1, _s())
            ctx.save_for_backward(xb, *w, a_ug, b, ug, z)
        ctx.meta = (shape, r, F, fused, resid is not None, [t.dtype for t in (us_ug, v_ug, v_dn, us_dn)])
        return y.view(shape)

    @staticmethod
    def backward(ctx, dy):
        xb, us_ug, v_ug, v_dn, us_dn, a_ug, b, *wide = ctx.saved_tensors
        shape, r, F, fused, has_resid, dts = ctx.meta
        T, d = xb.shape
        dev = xb.device
        dyb = cast_bf16(dy.reshape(T, d))
        db = torch.empty((T, r), dtype=BF16, device=dev)
        da = torch.empty((T, 2 * r), dtype=BF16, device=dev)
        dx = torch.empty((T, d), dtype=BF16, device=dev)
        g = [torch.empty(t.shape, dtype=F32, device=dev) for t in (us_ug, v_ug, v_dn, us_dn)]
        if fused:
            wsp, wsn = workspace(_lib.load().rte_svd_ffn_fused_workspace_bytes(T, d, F, r), dev)
            call("rte_svd_ffn_fused_bwd", ptr(dyb), ptr(xb), T, d, F, r, ptr(us_ug), ptr(v_ug), ptr(v_dn),
                 ptr(us_dn), ptr(a_ug), ptr(b), ptr(db), ptr(da), ptr(dx), *[ptr(t) for t in g], wsp, wsn, _s())
        else:
            ug, z = wide
            dug = torch.empty((T, 2 * F), dtype=BF16, device=dev)
            wsp, wsn = _gemm_ws(max(d, F), 2 * r, T, dev)
            call("rte_svd_ffn_bwd", ptr(dyb), ptr(xb), T, d, F, r, ptr(us_ug), ptr(v_ug), ptr(v_dn), ptr(us_dn),
                 ptr(a_ug), ptr(ug), ptr(z), ptr(b), ptr(db), ptr(dug), ptr(da), ptr(dx), *[ptr(t) for t in g],
                 wsp, wsn, _s())
        return (dx.view(shape), *[t.to(dt) for t, dt in zip(g, dts)], dy if has_resid else None)


def svd_ffn(x, us_ug, v_ug, v_dn, us_dn, resid=None):
    return SVDFFNFn.apply(x, us_ug, v_ug, v_dn, us_dn, resid)


# ----------------------------------------------------------------------------- dispatch-symbol kernels

def _io_flag(t: torch.Tensor, op: str) -> int:
    if t.dtype == F32:
        return 1
    if t.dtype == BF16:
        return 0
    raise TypeError(f"{op}: float32 or bfloat16 tensors expected, got {t.dtype}")


class FusedRMSNormFn(torch.autograd.Function):
    """(y * rsqrt(mean(y^2) + eps) * w, y) with y = x + residual, in the dtype torch gives the
    reference's k_fused_rmsnorm (rte/kernels/reference.py:9-17): the output is
    promote(y.dtype, w.dtype), y keeps x's dtype."""

    @staticmethod
    def forward(ctx, x, w, residual, eps: float):
        _lib.require_device_tensors("k_fused_rmsnorm", x, w, residual)
        io = _io_flag(x, "k_fused_rmsnorm")
        if residual is not None and residual.dtype != x.dtype:
            raise TypeError("k_fused_rmsnorm: x and residual must share a dtype")
        shape = x.shape
        d = shape[-1]
        x2 = x.reshape(-1, d).contiguous()
        T = x2.shape[0]
        r2 = None if residual is None else residual.reshape(T, d).contiguous()
        w32 = w.detach().reshape(d).contiguous().to(F32)
        out_dt = torch.promote_types(x.dtype, w.dtype)
        if out_dt not in (F32, BF16):
            raise TypeError(f"k_fused_rmsnorm: output dtype {out_dt} unsupported")
        out = torch.empty((T, d), dtype=out_dt, device=x.device)
        y = torch.empty_like(x2) if r2 is not None else None
        rstd = torch.empty((T,), dtype=F32, device=x.device)
        call("rte_fused_rmsnorm_fwd", ptr(x2), ptr(r2), io, ptr(w32), T, d, float(eps), ptr(y), ptr(out),
             int(out_dt == F32), ptr(rstd), _s())
        ysave = y if y is not None else x2
        ctx.save_for_backward(ysave, w32, rstd)
        ctx.meta = (shape, io, residual is not None, w.dtype)
        ctx.set_materialize_grads(False)
        if y is None:
            return out.view(shape), None
        return out.view(shape), y.view(shape)

    @staticmethod
    def backward(ctx, g, gy):
        y, w32, rstd = ctx.saved_tensors
        shape, io, has_res, w_dt = ctx.meta
        T, d = y.shape
        if g is None:
            gx = None if gy is None else gy
            return gx, None, gx if has_res else None, None
        gc = g.reshape(T, d).contiguous()
        if gc.dtype not in (F32, BF16):
            gc = gc.to(F32)
        ey = None if gy is None else gy.reshape(T, d).contiguous().to(y.dtype)
        dy = torch.empty_like(y)
        dw = torch.empty((d,), dtype=F32, device=y.device)
        ws, nb = workspace(_lib.load().rte_fused_rmsnorm_bwd_workspace_bytes(T, d), y.device)
        call("rte_fused_rmsnorm_bwd", ptr(gc), int(gc.dtype == F32), ptr(ey), ptr(y), io, ptr(w32), ptr(rstd), T, d,
             ptr(dy), ptr(dw), ws, nb, _s())
        dyv = dy.view(shape)
        return dyv, dw.to(w_dt), (dyv if has_res else None), None


def fused_rmsnorm(x, w, residual=None, eps: float = 1e-5):
    return FusedRMSNormFn.apply(x, w, residual, eps)


class RopeApplyFn(torch.autograd.Function):
    """Interleaved RoPE of q and k (rte/kernels/reference.py:20-28) on the HIP kernel; q, k
    [..., S, hd] in float32 or bfloat16, cos / sin broadcastable [S, hd]; the output dtype is
    promote(q.dtype, cos.dtype) as in the reference.  cos / sin carry no gradient."""

    @staticmethod
    def forward(ctx, q, k, cos, sin):
        _lib.require_device_tensors("k_rope_apply", q, k, cos, sin)
        if q.shape != k.shape or q.dtype != k.dtype:
            raise ValueError("k_rope_apply: q and k must share shape and dtype")
        S, hd = q.shape[-2], q.shape[-1]
        c2 = cos.reshape(-1, cos.shape[-1])
        s2 = sin.reshape(-1, sin.shape[-1])
        if c2.shape != (S, hd) or s2.shape != (S, hd):
            raise ValueError(f"k_rope_apply: cos / sin must be [{S}, {hd}] (got {tuple(cos.shape)})")
        io = _io_flag(q, "k_rope_apply")
        out_dt = torch.promote_types(q.dtype, cos.dtype)
        if out_dt not in (F32, BF16):
            raise TypeError(f"k_rope_apply: output dtype {out_dt} unsupported")
        cf, sf = c2.contiguous().to(F32), s2.contiguous().to(F32)
        qc, kc = q.contiguous(), k.contiguous()
        qo = torch.empty(q.shape, dtype=out_dt, device=q.device)
        ko = torch.empty(k.shape, dtype=out_dt, device=k.device)
        rows = q.numel() // hd
        call("rte_rope_apply", ptr(qc), ptr(kc), io, rows, S, hd, ptr(cf), ptr(sf), ptr(qo), ptr(ko),
             int(out_dt == F32), 0, _s())
        ctx.save_for_backward(cf, sf)
        ctx.meta = (q.dtype, S, hd)
        ctx.set_materialize_grads(False)
        return qo, ko

    @staticmethod
    def backward(ctx, gq, gk):
        cf, sf = ctx.saved_tensors
        q_dt, S, hd = ctx.meta
        ref = gq if gq is not None else gk
        if ref is None:
            return None, None, None, None
        gq = torch.zeros_like(ref) if gq is None else gq
        gk = torch.zeros_like(ref) if gk is None else gk
        gin = torch.promote_types(gq.dtype, gk.dtype)
        if gin not in (F32, BF16):
            gin = F32
        gqc, gkc = gq.contiguous().to(gin), gk.contiguous().to(gin)
        dq = torch.empty(gq.shape, dtype=q_dt, device=gq.device)
        dk = torch.empty(gk.shape, dtype=q_dt, device=gk.device)
        call("rte_rope_apply", ptr(gqc), ptr(gkc), int(gin == F32), gq.numel() // hd, S, hd, ptr(cf), ptr(sf), ptr(dq),
             ptr(dk), int(q_dt == F32), 1, _s())
        return dq, dk, None, None


def rope_apply(q, k, cos, sin):
    return RopeApplyFn.apply(q, k, cos, sin)


class RowsLinearFn(torch.autograd.Function):
    """x @ W[rows, :] (the reference's k_out_proj_grouped, rte/kernels/reference.py:58-59): the GEMM
    reads W's rows through an index table (no gathered weight copy); dW's selected rows are
    reduced into W's rows in a fixed order (repeated indices add up)."""

    @staticmethod
    def forward(ctx, x, w, rows, out_dtype):
        _lib.require_device_tensors("k_out_proj_grouped", x, w, rows)
        shape = x.shape
        K = shape[-1]
        rid = rows.reshape(-1).contiguous().to(torch.int32)
        if rid.numel() != K:
            raise ValueError(f"k_out_proj_grouped: {rid.numel()} row indices for x of width {K}")
        xb = x.reshape(-1, K).contiguous().to(BF16)
        wb = cast_bf16(w)
        out = gemm(xb, wb, b_t=True, b_rows=rid, out_f32=out_dtype == F32)
        ctx.save_for_backward(xb, wb, rid)
        ctx.meta = (shape, x.dtype, w.dtype, w.shape[0])
        return out.view(*shape[:-1], wb.shape[1]).to(out_dtype)

    @staticmethod
    def backward(ctx, dout):
        xb, wb, rid = ctx.saved_tensors
        shape, x_dt, w_dt, n_rows = ctx.meta
        N = wb.shape[1]
        db = dout.reshape(-1, N).contiguous().to(BF16)
        dx = gemm(db, wb, b_rows=rid)                                  # [T, K] = dout @ W[rows]^T
        dsel = gemm(xb, db, a_t=True, b_t=True, out_f32=True)          # [K, N] = x^T dout
        dw = segment_reduce_rows(rid, n_rows, dsel)
        return dx.view(shape).to(x_dt), dw.to(w_dt), None, None


def rows_linear(x, w, rows, out_dtype=BF16):
    if fp32_active():  # x @ w[rows, :] on the fp32 GEMM
        return _f32().linear(x, w.index_select(0, rows.to(device=w.device, dtype=torch.long)).t())
    return RowsLinearFn.apply(x, w, rows, out_dtype)


def route_centers(q: torch.Tensor, centers: torch.Tensor) -> torch.Tensor:
    """argmax_c normalize(q[t]) . centers[c] (fp32, int32 ids) on the HIP kernel."""
    _lib.require_device_tensors("route_to_static_centers", q, centers)
    qf = q.reshape(-1, q.shape[-1]).contiguous().to(F32)
    cf = centers.contiguous().to(F32)
    if cf.ndim != 2 or cf.shape[1] != qf.shape[1]:
        raise ValueError(f"route_to_static_centers: centers {tuple(cf.shape)} do not match features {qf.shape[1]}")
    out = torch.empty((qf.shape[0],), dtype=torch.int32, device=qf.device)
    call("rte_route_centers", ptr(qf), qf.shape[0], qf.shape[1], ptr(cf), cf.shape[0], ptr(out), _s())
    return out.view(q.shape[:-1])


class CrossEntropyFn(torch.autograd.Function):
    """Per-token cross-entropy of fp32 logits [..., V] against int64 targets (negative targets,
    such as F.cross_entropy's ignore_index -100, give 0) on the fused CE kernel; the backward is
    (softmax - onehot) * dloss in fp32 from the saved log-sum-exp."""

    @staticmethod
    def forward(ctx, logits, targets):
        _lib.require_device_tensors("cross_entropy", logits, targets)
        V = logits.shape[-1]
        lg = logits.reshape(-1, V).contiguous().to(F32)
        T = lg.shape[0]
        tg = targets.reshape(-1).contiguous().to(torch.int64)
        if tg.numel() != T:
            raise ValueError(f"cross_entropy: {tg.numel()} targets for {T} rows")
        loss = torch.empty((T,), dtype=F32, device=lg.device)
        lse = torch.empty((T,), dtype=F32, device=lg.device)
        call("rte_ce_fwd", ptr(lg), V, T, V, ptr(tg), ptr(loss), ptr(lse), _s())
        ctx.save_for_backward(lg, tg, lse)
        ctx.meta = (logits.shape, logits.dtype)
        return loss.view(targets.shape)

    @staticmethod
    def backward(ctx, g):
        lg, tg, lse = ctx.saved_tensors
        shape, dt = ctx.meta
        valid = tg >= 0
        p = torch.exp(lg - lse[:, None])
        p[valid, tg[valid]] -= 1.0
        p *= (g.reshape(-1).to(F32) * valid.to(F32))[:, None]
        return p.view(shape).to(dt), None


def cross_entropy(logits, targets):
    return CrossEntropyFn.apply(logits, targets)


# ----------------------------------------------------------------------------- SVD-factor sparse FFN

class SVDSparseFn(torch.autograd.Function):
    """Per-token sparse SwiGLU with SVD-factor candidate retrieval and exact rerank
    (rte/layers.py:446-643): the selector GEMMs, one workgroup per token for the candidate union,
    activations, rerank and down-sum; the backward is one workgroup per token for dx and the
    selected activations' gradients, and three fixed-order segmented reductions keyed by the
    selected neuron ids for the weight rows."""

    @staticmethod
    def forward(ctx, x, w_up, w_gate, w_down, us_ug, v_ug, wd_norm, up_m: int, gate_m: int, product_m: int,
                top_k: int, exact: bool, product_only: bool, out_dtype):
        _lib.require_device_tensors("svd_sparse_ffn", x, w_up, w_gate, w_down, us_ug, v_ug, wd_norm)
        shape = x.shape
        d = shape[-1]
        xb = x.reshape(-1, d).contiguous().to(BF16)
        T = xb.shape[0]
        F = w_up.shape[0]
        r2 = us_ug.shape[1]
        wub, wgb, wdb = cast_bf16(w_up), cast_bf16(w_gate), cast_bf16(w_down)
        usb, vb = cast_bf16(us_ug), cast_bf16(v_ug)
        dev = x.device
        a_ug = torch.empty((T, r2), dtype=BF16, device=dev)
        ug = torch.empty((T, 2 * F), dtype=BF16, device=dev)
        zh = torch.empty((T, F), dtype=BF16, device=dev)
        out = torch.empty((T, d), dtype=out_dtype, device=dev)
        sel = torch.empty((T, top_k), dtype=torch.int32, device=dev)
        su = torch.empty((T, top_k), dtype=F32, device=dev)
        sg = torch.empty((T, top_k), dtype=F32, device=dev)
        nc = torch.empty((T,), dtype=torch.int32, device=dev)
        call("rte_svd_sparse_fwd", ptr(xb), T, d, F, r2 // 2, ptr(usb), ptr(vb), ptr(wub), ptr(wgb), ptr(wdb),
             ptr(wd_norm.contiguous().to(F32)), int(up_m), int(gate_m), int(product_m), int(top_k), int(exact),
             int(product_only), ptr(a_ug), ptr(ug), ptr(zh), ptr(out), int(out_dtype == F32), ptr(sel), ptr(su),
             ptr(sg), ptr(nc), _s())
        ctx.save_for_backward(xb, wub, wgb, wdb, sel, su, sg)
        ctx.meta = (shape, F, top_k, x.dtype, [t.dtype for t in (w_up, w_gate, w_down)])
        ctx.mark_non_differentiable(sel, nc)
        ctx.set_materialize_grads(False)
        return out.view(shape), sel.view(*shape[:-1], top_k), nc.view(shape[:-1])

    @staticmethod
    def backward(ctx, dout, _dsel, _dnc):
        if dout is None:
            return (None,) * 14
        xb, wub, wgb, wdb, sel, su, sg = ctx.saved_tensors
        shape, F, K, x_dt, w_dts = ctx.meta
        T, d = xb.shape
        dev = xb.device
        db = dout.reshape(T, d).contiguous().to(BF16)
        dx = torch.empty((T, d), dtype=BF16, device=dev)
        z = torch.empty((T, K), dtype=F32, device=dev)
        du = torch.empty((T, K), dtype=F32, device=dev)
        dg = torch.empty((T, K), dtype=F32, device=dev)
        call("rte_svd_sparse_bwd", ptr(db), T, d, K, ptr(wub), ptr(wgb), ptr(wdb), ptr(sel), ptr(su), ptr(sg),
             ptr(dx), ptr(z), ptr(du), ptr(dg), _s())
        keys = sel.reshape(-1)
        nia = ctx.needs_input_grad
        dwu = segment_reduce_rows(keys, F, xb, w=du, row_div=K) if nia[1] else None
        dwg = segment_reduce_rows(keys, F, xb, w=dg, row_div=K) if nia[2] else None
        dwd = segment_reduce_rows(keys, F, db, w=z, row_div=K) if nia[3] else None
        return (dx.view(shape).to(x_dt), None if dwu is None else dwu.to(w_dts[0]),
                None if dwg is None else dwg.to(w_dts[1]), None if dwd is None else dwd.to(w_dts[2]),
                None, None, None, None, None, None, None, None, None, None)


def svd_sparse_ffn(x, w_up, w_gate, w_down, up_a, up_b, gate_a, gate_b, *, up_m: int, gate_m: int, product_m: int,
                   top_k: int, exact: bool = True, product_only: bool = False, wd_norm=None, out_dtype=None):
    """(out, selected ids, candidate counts) of the SVD-factor sparse FFN.  up_a / gate_a [d, r],
    up_b / gate_b [r, F] (refresh_svd's factors); w_* [F, d].  The rank is zero-padded to a multiple
    of 8 (zero factor columns change no score)."""
    r = up_a.shape[1]
    pad = (-r) % 8
    us_ug = torch.cat([up_a, up_a.new_zeros(up_a.shape[0], pad), gate_a, gate_a.new_zeros(gate_a.shape[0], pad)], 1)
    v_ug = torch.cat([torch.cat([up_b.t(), up_b.new_zeros(up_b.shape[1], pad)], 1),
                      torch.cat([gate_b.t(), gate_b.new_zeros(gate_b.shape[1], pad)], 1)], 0)
    if wd_norm is None:
        wd_norm = w_down.detach().float().norm(dim=-1)
    out_dtype = out_dtype or (BF16 if x.dtype == BF16 else F32)
    return SVDSparseFn.apply(x, w_up, w_gate, w_down, us_ug.detach(), v_ug.detach(), wd_norm, up_m, gate_m,
                             product_m, top_k, exact, product_only, out_dtype)

