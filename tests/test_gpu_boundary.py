"""The reference's dispatch symbols and module backends on the HIP kernels, against the oracle
or an fp32/fp64 restatement of the reference formula (rte/kernels/reference.py,
rte/kernels/cluster_pool_ffn.py, rte/kernels/active_swiglu_triton.py, rte/layers.py:90-339).

Tolerances: fp32 paths 1e-5 relative; bf16 paths 2e-2 relative (Frobenius); indices bit-exact."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from helpers import BF16_RTOL, FP32_RTOL, assert_rel, bf16_round
from oracle import cluster_pool as CP
from oracle import routing as R
from oracle import swiglu as SW

pytestmark = pytest.mark.gpu

DEV = "cuda"


@pytest.fixture(scope="module", autouse=True)
def _hip():
    from rte_amd import _lib

    if not _lib.device_ready():
        pytest.fail("HIP backend not ready on this GPU box (library or gfx950 device missing)")
    yield


def _np(t):
    return t.detach().double().cpu().numpy()


def _K():
    from rte_amd.kernels import optimized

    return optimized


def _autocast():
    return torch.autocast("cuda", dtype=torch.bfloat16)


# ---------------------------------------------------------------- elementwise symbols, caller dtype

@pytest.mark.parametrize("with_res", [False, True])
def test_fused_rmsnorm_fp32_matches_reference_formula(with_res):
    """k_fused_rmsnorm in fp32 (rte/kernels/reference.py:9-17): output dtype and values within
    1e-5 of the fp64 formula, y returned only with a residual, gradients of x, residual, weight."""
    K = _K()
    g = torch.Generator().manual_seed(3)
    x0 = torch.randn(5, 37, 256, generator=g, dtype=torch.float64)
    r0 = torch.randn(5, 37, 256, generator=g, dtype=torch.float64)
    w0 = 1 + 0.1 * torch.randn(256, generator=g, dtype=torch.float64)
    gy = torch.randn(5, 37, 256, generator=g, dtype=torch.float64)
    gr = torch.randn(5, 37, 256, generator=g, dtype=torch.float64)
    x, w = x0.float().to(DEV).requires_grad_(), w0.float().to(DEV).requires_grad_()
    r = r0.float().to(DEV).requires_grad_() if with_res else None
    print(f"k_fused_rmsnorm fp32 residual={with_res}", flush=True)
    out, y = K.k_fused_rmsnorm(x, w, r, eps=1e-5)
    assert out.dtype == torch.float32 and (y is None) == (not with_res)
    loss = (out.double() * gy.to(DEV)).sum() + ((y.double() * gr.to(DEV)).sum() if with_res else 0)
    loss.backward()
    xr, wr = x0.clone().requires_grad_(), w0.clone().requires_grad_()
    rr = r0.clone().requires_grad_() if with_res else None
    yr = xr if rr is None else xr + rr
    ref = yr * torch.rsqrt(yr.pow(2).mean(-1, keepdim=True) + 1e-5) * wr
    (ref * gy).sum().add((yr * gr).sum() if with_res else 0).backward()
    assert_rel(_np(out), ref.detach().numpy(), FP32_RTOL, "rmsnorm out")
    assert_rel(_np(x.grad), xr.grad.numpy(), FP32_RTOL, "rmsnorm dx")
    assert_rel(_np(w.grad), wr.grad.numpy(), FP32_RTOL, "rmsnorm dw")
    if with_res:
        assert_rel(_np(y), yr.detach().numpy(), FP32_RTOL, "rmsnorm y")
        assert_rel(_np(r.grad), rr.grad.numpy(), FP32_RTOL, "rmsnorm dres")


def test_fused_rmsnorm_bf16_input():
    """bf16 x with an fp32 weight returns fp32 (promote), bf16 rounding points as torch's."""
    K = _K()
    g = torch.Generator().manual_seed(4)
    x = torch.randn(64, 512, generator=g).to(torch.bfloat16).to(DEV)
    w = (1 + 0.1 * torch.randn(512, generator=g)).to(DEV)
    out, y = K.k_fused_rmsnorm(x, w)
    ref = (x * torch.rsqrt(x.float().pow(2).mean(-1, keepdim=True) + 1e-5).to(x.dtype)) * w
    assert out.dtype == ref.dtype == torch.float32 and y is None
    assert_rel(_np(out), _np(ref), 1e-2, "rmsnorm bf16")


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_rope_apply_matches_reference_formula(dtype):
    """k_rope_apply (rte/kernels/reference.py:20-28) against the rotate_half formula, forward and
    backward (the transpose rotation)."""
    from oracle import attention as A

    K = _K()
    B, H, S, hd = 2, 4, 33, 64
    g = torch.Generator().manual_seed(5)
    q0 = torch.randn(B, H, S, hd, generator=g)
    k0 = torch.randn(B, H, S, hd, generator=g)
    inv = 1.0 / (10000.0 ** (torch.arange(0, hd, 2).float() / hd))
    ang = torch.repeat_interleave(torch.outer(torch.arange(S).float(), inv), 2, -1)
    cos, sin = ang.cos(), ang.sin()
    gq, gk = torch.randn(B, H, S, hd, generator=g), torch.randn(B, H, S, hd, generator=g)
    q = q0.to(dtype).to(DEV).requires_grad_()
    k = k0.to(dtype).to(DEV).requires_grad_()
    print(f"k_rope_apply {dtype}", flush=True)
    qo, ko = K.k_rope_apply(q, k, cos.to(DEV).to(dtype), sin.to(DEV).to(dtype))
    assert qo.dtype == dtype
    ((qo.float() * gq.to(DEV)).sum() + (ko.float() * gk.to(DEV)).sum()).backward()
    tol = FP32_RTOL if dtype == torch.float32 else BF16_RTOL
    qr = torch.tensor(np.asarray(q0.to(dtype).double()), requires_grad=True)
    kr = torch.tensor(np.asarray(k0.to(dtype).double()), requires_grad=True)

    def rot(x):
        return torch.stack((-x[..., 1::2], x[..., ::2]), dim=-1).flatten(-2)

    c, s = cos.to(dtype).double(), sin.to(dtype).double()
    qref, kref = qr * c + rot(qr) * s, kr * c + rot(kr) * s
    ((qref * gq.double()).sum() + (kref * gk.double()).sum()).backward()
    assert_rel(_np(qo), qref.detach().numpy(), tol, "rope q")
    assert_rel(_np(ko), kref.detach().numpy(), tol, "rope k")
    assert_rel(_np(q.grad), qr.grad.numpy(), tol, "rope dq")
    assert_rel(_np(k.grad), kr.grad.numpy(), tol, "rope dk")
    # the oracle's rotation agrees with the reference formula
    np.testing.assert_allclose(A.rope_apply(q0.numpy(), cos.numpy(), sin.numpy()),
                               (q0.double() * cos.double() + rot(q0.double()) * sin.double()).numpy(),
                               rtol=1e-6, atol=1e-6)


def test_cross_entropy_unreduced_matches_torch():
    K = _K()
    g = torch.Generator().manual_seed(6)
    logits = (torch.randn(4, 9, 300, generator=g) * 3).to(DEV).requires_grad_()
    tgt = torch.randint(0, 300, (4, 9), generator=g).to(DEV)
    tgt[0, 0] = -100  # ignore_index
    loss = K.k_cross_entropy_unreduced(logits, tgt)
    gl = torch.randn(4, 9, generator=g).to(DEV)
    (loss * gl).sum().backward()
    lr = logits.detach().double().cpu().requires_grad_()
    ref = torch.nn.functional.cross_entropy(lr.flatten(0, -2), tgt.cpu().flatten(), reduction="none").view(4, 9)
    (ref * gl.cpu().double()).sum().backward()
    assert_rel(_np(loss), ref.detach().numpy(), FP32_RTOL, "ce")
    assert_rel(_np(logits.grad), lr.grad.numpy(), FP32_RTOL, "ce grad")


# ---------------------------------------------------------------- matmul symbols (bf16 under autocast)

def _bfr(t):
    return torch.from_numpy(bf16_round(t.numpy().astype(np.float32))).double()


def test_out_proj_grouped_reads_weight_rows_through_indices():
    """k_out_proj_grouped(x, wo, rows) = x @ wo[rows, :] (rte/kernels/reference.py:58-59) with
    repeated rows; the weight gradient of repeated rows adds up."""
    K = _K()
    g = torch.Generator().manual_seed(7)
    T, d, n = 300, 256, 128
    x0 = torch.randn(T, n, generator=g)
    wo0 = torch.randn(d, d, generator=g) * 0.05
    rows = torch.randint(0, d, (n,), generator=g)
    rows[5] = rows[9]
    gy = torch.randn(T, d, generator=g)
    x = x0.to(DEV).requires_grad_()
    wo = wo0.to(DEV).requires_grad_()
    with _autocast():
        y = K.k_out_proj_grouped(x, wo, rows.to(DEV))
    assert y.dtype == torch.bfloat16
    (y.float() * gy.to(DEV)).sum().backward()
    xr, wr = _bfr(x0).requires_grad_(), _bfr(wo0).requires_grad_()
    yr = xr @ wr[rows]
    (yr * gy.double()).sum().backward()
    assert_rel(_np(y), yr.detach().numpy(), BF16_RTOL, "out_proj y")
    assert_rel(_np(x.grad), xr.grad.numpy(), BF16_RTOL, "out_proj dx")
    assert_rel(_np(wo.grad), wr.grad.numpy(), BF16_RTOL, "out_proj dwo")


def test_qkv_and_swiglu_symbols():
    """k_qkv_dense / k_qkv_grouped / k_swiglu_dense / k_swiglu_grouped against fp64 of the
    bf16-rounded operands (rte/kernels/reference.py:31-78), bf16 results under autocast; fp32
    operands outside autocast are refused."""
    K = _K()
    g = torch.Generator().manual_seed(8)
    T, d, m = 256, 128, 96
    x0 = torch.randn(T, d, generator=g)
    wq0, wk0, wv0 = (torch.randn(d, d, generator=g) * 0.05 for _ in range(3))
    wu0, wg0 = (torch.randn(d, 4 * m, generator=g) * 0.05 for _ in range(2))
    wd0 = torch.randn(4 * m, d, generator=g) * 0.05
    cols = torch.randperm(d, generator=g)[:64]
    slabs = torch.randperm(4 * m, generator=g)[:m]
    x = x0.to(DEV)
    with _autocast():
        q, k, v = K.k_qkv_dense(x, wq0.to(DEV), wk0.to(DEV), wv0.to(DEV))
        qg, kg, vg = K.k_qkv_grouped(x, wq0.to(DEV), wk0.to(DEV), wv0.to(DEV), cols.to(DEV))
        sd = K.k_swiglu_dense(x, wu0.to(DEV), wg0.to(DEV), wd0.to(DEV))
        sg = K.k_swiglu_grouped(x, wu0.to(DEV), wg0.to(DEV), wd0.to(DEV), slabs.to(DEV))
    xb = _bfr(x0)
    for got, w in ((q, wq0), (k, wk0), (v, wv0)):
        assert got.dtype == torch.bfloat16
        assert_rel(_np(got), (xb @ _bfr(w)).numpy(), BF16_RTOL, "qkv_dense")
    for got, w in ((qg, wq0), (kg, wk0), (vg, wv0)):
        assert_rel(_np(got), (xb @ _bfr(w)[:, cols]).numpy(), BF16_RTOL, "qkv_grouped")
    silu = torch.nn.functional.silu
    ref = (xb @ _bfr(wu0)) * silu(xb @ _bfr(wg0)) @ _bfr(wd0)
    assert_rel(_np(sd), ref.numpy(), BF16_RTOL, "swiglu_dense")
    refg = (xb @ _bfr(wu0)[:, slabs]) * silu(xb @ _bfr(wg0)[:, slabs]) @ _bfr(wd0)[slabs]
    assert_rel(_np(sg), refg.numpy(), BF16_RTOL, "swiglu_grouped")
    with pytest.raises(RuntimeError, match="bf16"):
        K.k_qkv_dense(x, wq0.to(DEV), wk0.to(DEV), wv0.to(DEV))


@pytest.mark.parametrize("per_sample", [False, True])
def test_macro_phi_symbol(per_sample):
    """k_macro_phi (rte/kernels/reference.py:111-124) with shared [3d, m] or per-sample [B, 3d, m]
    factors, against an fp64 restatement with bf16-rounded GEMM operands."""
    K = _K()
    g = torch.Generator().manual_seed(9)
    B, S, d, m = 3, 16, 64, 32
    h = torch.randn(B, S, d, generator=g)
    h0 = torch.randn(B, S, d, generator=g)
    vs = (B, 3 * d, m) if per_sample else (3 * d, m)
    us = (B, m, d) if per_sample else (m, d)
    v = torch.randn(*vs, generator=g) * 0.1
    u = torch.randn(*us, generator=g) * 0.1
    dg, bias = torch.randn(d, generator=g) * 0.1, torch.randn(d, generator=g) * 0.1
    with _autocast():
        out = K.k_macro_phi(h.to(DEV), h0.to(DEV), dg.to(DEV), v.to(DEV), u.to(DEV), bias.to(DEV))
    hd = h.double()
    normed = hd * torch.rsqrt(hd.pow(2).mean(-1, keepdim=True) + 1e-5)
    z = torch.cat([normed, normed.mean(1, keepdim=True).expand_as(normed), h0.double()], -1)
    z = _bfr(z.float())
    a = z @ _bfr(v)
    low = _bfr(torch.nn.functional.silu(_bfr(a.float()).float())) @ _bfr(u)
    ref = hd + dg.double() * hd + low + bias.double()
    assert_rel(_np(out) - h.double().numpy(), (ref - hd).numpy(), BF16_RTOL, "macro_phi")


# ---------------------------------------------------------------- module backends

def _pool_case(seed, T=512, d=128, F=256, C=6, M=64):
    rng = np.random.default_rng(seed)
    x = bf16_round(rng.standard_normal((T, d)).astype(np.float32))
    w_up = bf16_round((rng.standard_normal((F, d)) * 0.05).astype(np.float32))
    w_gate = bf16_round((rng.standard_normal((F, d)) * 0.05).astype(np.float32))
    w_down_rows = bf16_round((rng.standard_normal((F, d)) * 0.05).astype(np.float32))
    cand = np.stack([rng.choice(F, M, replace=False) for _ in range(C)])  # overlapping pools
    assign = rng.integers(0, C, T)
    return rng, x, w_up, w_gate, w_down_rows, cand, assign


def test_static_pack_gather_indices_bit_exact():
    from rte_amd.kernels import cluster_pool_ffn as CPF

    rng = np.random.default_rng(10)
    a = rng.integers(0, 7, 1000)
    a[a == 3] = 4  # an empty cluster
    pack, flat, counts, mc = CPF.build_static_pack_gather_indices(torch.from_numpy(a).to(DEV), cluster_count=7)
    rp, rf, rc, rmc = R.static_pack_gather(a, 7)
    assert mc == rmc
    np.testing.assert_array_equal(pack.cpu().numpy(), rp)
    np.testing.assert_array_equal(flat.cpu().numpy(), rf)
    np.testing.assert_array_equal(counts.cpu().numpy(), rc)


def test_preindexed_pool_ffn_and_grad_scatter():
    """prepare_cluster_pool_weights (overlapping candidate pools) + cluster_pool_ffn_forward_preindexed
    against the reference's per-cluster loop oracle; the pool gradients against fp64 autograd of
    that loop; scatter_cluster_pool_grads against np.add.at (fp32, 1e-5)."""
    from rte_amd.kernels import cluster_pool_ffn as CPF

    rng, x, w_up, w_gate, w_down_rows, cand, assign = _pool_case(11)
    F, d = w_up.shape
    dy = rng.standard_normal(x.shape)
    tw = [torch.from_numpy(a).to(DEV).requires_grad_() for a in (w_up, w_gate, w_down_rows)]
    pools = CPF.prepare_cluster_pool_weights(*tw, torch.from_numpy(cand).to(DEV))
    pk, fg, _, _ = CPF.build_static_pack_gather_indices(torch.from_numpy(assign).to(DEV), cluster_count=cand.shape[0])
    tx = torch.from_numpy(x).to(DEV).requires_grad_()
    with _autocast():
        out = CPF.cluster_pool_ffn_forward_preindexed(tx, pk, fg, *pools)
    assert out.dtype == torch.bfloat16
    out.float().backward(torch.from_numpy(dy).float().to(DEV))
    ref_pools = CP.prepare_pools(w_up, w_gate, w_down_rows, cand)
    assert_rel(_np(out), CP.cluster_pool_reference_loop(x, assign, *ref_pools), BF16_RTOL, "preindexed y")
    # fp64 autograd of the reference loop through the row gathers
    tr = [torch.tensor(a, dtype=torch.float64, requires_grad=True) for a in (w_up, w_gate, w_down_rows)]
    txr = torch.tensor(x, dtype=torch.float64, requires_grad=True)
    ids = torch.from_numpy(cand)
    outr = torch.zeros(x.shape, dtype=torch.float64)
    for c in range(cand.shape[0]):
        tok = torch.from_numpy(np.nonzero(assign == c)[0])
        up = txr[tok] @ tr[0][ids[c]].T
        gate = txr[tok] @ tr[1][ids[c]].T
        outr = outr.index_add(0, tok, (up * torch.nn.functional.silu(gate)) @ tr[2][ids[c]])
    (outr * torch.from_numpy(dy)).sum().backward()
    assert_rel(_np(tx.grad), txr.grad.numpy(), BF16_RTOL, "preindexed dx")
    for name, a, b in zip(("dup", "dgate", "ddown"), tw, tr):
        assert_rel(_np(a.grad), b.grad.numpy(), BF16_RTOL, f"preindexed {name}")
    # scatter of pool gradients into dense rows
    C, M = cand.shape
    gp = [rng.standard_normal(s).astype(np.float32) for s in ((C, d, M), (C, d, M), (C, M, d))]
    got = CPF.scatter_cluster_pool_grads(torch.from_numpy(cand).to(DEV), *(torch.from_numpy(a).to(DEV) for a in gp),
                                         d_ff=F)
    for i, (gg, arr) in enumerate(zip(got, (np.transpose(gp[0], (0, 2, 1)), np.transpose(gp[1], (0, 2, 1)), gp[2]))):
        want = np.zeros((F, d))
        np.add.at(want, cand.reshape(-1), arr.reshape(-1, d).astype(np.float64))
        assert_rel(_np(gg), want, FP32_RTOL, f"scatter {i}")


def test_forward_from_assignments_capacity_and_errors():
    """Inference path with a capacity: the tokens of a cluster beyond its first cap (ascending
    token order) give zero rows and set the overflow flag; grads are refused."""
    from rte_amd.kernels import cluster_pool_ffn as CPF

    rng, x, w_up, w_gate, w_down_rows, cand, assign = _pool_case(12)
    pools = [torch.from_numpy(p.copy()).to(DEV) for p in CP.prepare_pools(w_up, w_gate, w_down_rows, cand)]
    tx = torch.from_numpy(x).to(DEV)
    ta = torch.from_numpy(assign).to(DEV)
    cap = int(np.bincount(assign).min())
    with torch.no_grad():
        out, of = CPF.cluster_pool_ffn_forward_from_assignments(tx, ta, *pools, max_tokens_per_cluster=cap,
                                                                return_overflow=True)
    full = CP.cluster_pool_reference_loop(x, assign, *[p.cpu().numpy() for p in pools])
    keep = np.zeros(len(assign), bool)
    for c in range(cand.shape[0]):
        keep[np.nonzero(assign == c)[0][:cap]] = True
    assert int(of) == 1
    assert np.all(_np(out)[~keep] == 0)
    assert_rel(_np(out)[keep], full[keep], BF16_RTOL, "capacity y")
    with pytest.raises(RuntimeError, match="inference/eval only"):
        CPF.cluster_pool_ffn_forward_from_assignments(tx, ta, pools[0].requires_grad_(), pools[1], pools[2])


def test_route_to_static_centers_bit_exact():
    """route_to_static_centers on the kernel's selector features against the oracle's argmax."""
    from rte_amd.kernels import cluster_pool_ffn as CPF
    from rte_amd.kernels import hip_ops as H

    rng = np.random.default_rng(13)
    T, d, r, C = 4096, 256, 16, 64
    x = torch.from_numpy(rng.standard_normal((T, d)).astype(np.float32)).to(DEV)
    up_a = torch.from_numpy((rng.standard_normal((d, r)) * 0.1).astype(np.float32)).to(DEV)
    gate_a = torch.from_numpy((rng.standard_normal((d, r)) * 0.1).astype(np.float32)).to(DEV)
    centers = rng.standard_normal((C, 2 * r)).astype(np.float32)
    centers[9] = centers[4]
    got = CPF.route_to_static_centers(x, up_a, gate_a, torch.from_numpy(centers).to(DEV))
    assert got.dtype == torch.long
    q = H.gemm(x.to(torch.bfloat16), H.cast_bf16(torch.cat([up_a, gate_a], 1).t().contiguous()), out_f32=True)
    want, scores = R.static_centers(q.cpu().numpy(), centers)
    np.testing.assert_array_equal(got.cpu().numpy(), want)
    assert 9 not in got.cpu().numpy()


def test_triton_packed_swiglu_mirror_with_padding():
    """triton_packed_swiglu_ffn (rte/kernels/active_swiglu_triton.py:105-118) with a width that is not
    a multiple of 32 (zero-padded inside), forward and backward against the oracle."""
    from rte_amd.kernels import active_swiglu_triton as AS

    rng = np.random.default_rng(14)
    T, d, M = 384, 128, 72
    x = bf16_round(rng.standard_normal((T, d)).astype(np.float32))
    wug = bf16_round((rng.standard_normal((2 * M, d)) * 0.05).astype(np.float32))
    wdr = bf16_round((rng.standard_normal((M, d)) * 0.05).astype(np.float32))
    dy = bf16_round(rng.standard_normal((T, d)).astype(np.float32))
    tx, tw, td = (torch.from_numpy(a).to(DEV).requires_grad_() for a in (x, wug, wdr))
    with _autocast():
        y = AS.triton_packed_swiglu_ffn(tx, tw, td)
    y.float().backward(torch.from_numpy(dy).to(DEV))
    ref, cache = SW.dense_swiglu_fwd(x, wug, wdr, wd_rows=True)
    assert_rel(_np(y), ref, BF16_RTOL, "packed y")
    dx, dwug, dwd = SW.dense_swiglu_bwd(dy, x, wug, wdr, cache, wd_rows=True)
    assert_rel(_np(tx.grad), dx, BF16_RTOL, "packed dx")
    assert_rel(_np(tw.grad), dwug, BF16_RTOL, "packed dwug")
    assert_rel(_np(td.grad), dwd, BF16_RTOL, "packed dwd")


def test_static_cluster_pool_layer_overlapping_pools():
    """StaticClusterPoolSwiGLU (rte/layers.py:119-220) end to end with overlapping candidate pools:
    output against the loop oracle on the kernel's routing, dense-weight gradients against fp64
    autograd of the gathered-pool formulation (duplicated rows summed)."""
    from rte_amd.config import ModelConfig
    from rte_amd.kernels import cluster_pool_ffn as CPF
    from rte_amd.layers import DenseSwiGLU, StaticClusterPoolSwiGLU

    cfg = ModelConfig(topology="dense", vocab_size=64, d_model=128, n_heads=4, d_ff=256, n_dense_layers=1,
                      n_prelude=1, n_coda=1, t_max=1, depth_choices=[1], attn_banks=1, ffn_banks=1, head_groups=4,
                      ffn_groups=4, active_head_groups=1, active_ffn_groups=1, recipe_count=2)
    torch.manual_seed(15)
    dense = DenseSwiGLU(cfg)
    with torch.no_grad():
        dense.wug.weight.copy_(torch.from_numpy(bf16_round(dense.wug.weight.numpy())))
        dense.wd.weight.copy_(torch.from_numpy(bf16_round(dense.wd.weight.numpy())))
    rng = np.random.default_rng(15)
    C, M, r = 5, 64, 8
    cand = np.stack([rng.choice(256, M, replace=False) for _ in range(C)])
    factors = {"up_a": torch.randn(128, r) * 0.1, "gate_a": torch.randn(128, r) * 0.1}
    codebook = {"centers": torch.randn(C, 2 * r), "candidate_ids": torch.from_numpy(cand)}
    layer = StaticClusterPoolSwiGLU(dense, factors, codebook, rank=r).to(DEV)
    x = bf16_round(rng.standard_normal((2, 150, 128)).astype(np.float32))
    dy = rng.standard_normal((2, 150, 128))
    tx = torch.from_numpy(x).to(DEV)
    out = layer(tx)
    out.float().backward(torch.from_numpy(dy).float().to(DEV))
    assign = CPF.route_to_static_centers(tx.reshape(-1, 128), layer.up_a, layer.gate_a, layer.centers).cpu().numpy()
    wug = dense.wug.weight.detach().double()
    wd = dense.wd.weight.detach().double()
    tw = wug.clone().requires_grad_()
    td = wd.clone().requires_grad_()
    xf = torch.from_numpy(x.reshape(-1, 128)).double()
    outr = torch.zeros_like(xf)
    ids = torch.from_numpy(cand)
    for c in range(C):
        tok = torch.from_numpy(np.nonzero(assign == c)[0])
        up = xf[tok] @ tw[:256][ids[c]].T
        gate = xf[tok] @ tw[256:][ids[c]].T
        outr = outr.index_add(0, tok, (up * torch.nn.functional.silu(gate)) @ td.t()[ids[c]])
    (outr * torch.from_numpy(dy.reshape(-1, 128))).sum().backward()
    assert_rel(_np(out).reshape(-1, 128), outr.detach().numpy(), BF16_RTOL, "static pool y")
    assert_rel(_np(layer.wug.weight.grad), tw.grad.numpy(), BF16_RTOL, "static pool dwug")
    assert_rel(_np(layer.wd.weight.grad), td.grad.numpy(), BF16_RTOL, "static pool dwd")


# ---------------------------------------------------------------- router

def test_router_matches_oracle_and_factor_heads():
    """Router (rte/routing.py:80-188) on the bias-fused HIP GEMMs against the oracle with
    bf16-rounded GEMM operands: logits within 2e-2; ids, probabilities and entropies are exactly
    the softmax / argmax of the kernel's own logits; factor fields appear when read; the
    factorized top-k (rte/models.py:273-310) is bit-exact against the oracle on those logits."""
    from oracle import router as RO
    from rte_amd.config import ModelConfig
    from rte_amd.models import RecursiveModel

    cfg = ModelConfig(topology="recursive", vocab_size=64, d_model=128, n_heads=4, d_ff=256, n_dense_layers=1,
                      n_prelude=1, n_coda=1, t_max=4, depth_choices=[1, 2, 4], attn_banks=2, ffn_banks=3,
                      head_groups=4, ffn_groups=8, active_head_groups=2, active_ffn_groups=2, recipe_count=9)
    torch.manual_seed(16)
    model = RecursiveModel(cfg).to(DEV)
    with torch.no_grad():
        for prm in model.router.parameters():
            prm.add_(torch.randn_like(prm) * 0.05)
    h0 = torch.randn(6, 20, 128, device=DEV)
    route = model.router(h0, temperature=0.8)
    p = {k: v.detach().double().cpu().numpy() for k, v in model.router.state_dict().items()}
    for k in p:
        if k.endswith(".weight"):
            p[k] = bf16_round(p[k].astype(np.float32)).astype(np.float64)
    ref = RO.router(h0.cpu().numpy(), p, [1, 2, 4], temperature=0.8)
    assert_rel(_np(route.recipe_logits), ref["recipe_logits"], BF16_RTOL, "recipe logits")
    assert_rel(_np(route.depth_logits), ref["depth_logits"], BF16_RTOL, "depth logits")
    own = RO._softmax(_np(route.recipe_logits_by_pass))
    np.testing.assert_array_equal(route.recipe_id_by_pass.cpu().numpy(), own.argmax(-1))
    np.testing.assert_allclose(_np(route.recipe_probs_by_pass), own, rtol=1e-5, atol=1e-7)
    np.testing.assert_array_equal(route.depth_id.cpu().numpy(), _np(route.depth_logits).argmax(-1))
    assert route._factor is None  # nothing read the factor heads yet
    for name in ("attn_bank", "ffn_bank", "head_slot", "ffn_slot"):
        lg = getattr(route, name + "_logits_by_pass")
        assert_rel(_np(lg), ref[name + "_logits_by_pass"], BF16_RTOL, name)
        np.testing.assert_array_equal(getattr(route, name + "_id_by_pass").cpu().numpy(), _np(lg).argmax(-1))
    assert route.factor_entropy.shape == (6,)
    factors, w = model._factorized_topk_routes(route, pass_idx=2, top_k=7)
    rf, rw = RO.factorized_topk(*(_np(getattr(route, n + "_logits_by_pass"))[:, 2, :]
                                  for n in ("attn_bank", "ffn_bank", "head_slot", "ffn_slot")), 7)
    np.testing.assert_array_equal(factors.cpu().numpy(), rf)
    np.testing.assert_allclose(w.cpu().numpy(), rw, rtol=1e-5, atol=1e-7)


def _router_ref(h0, p, ids, inv_t):
    """fp64 torch restatement of Router.forward's recipe / depth heads (rte/routing.py:80-188)
    with the layer-1 GEMM operands (pooled state, W1) rounded to bf16 in the forward only; the
    one-hot rows come from the kernel's ids."""
    F_ = torch.nn.functional

    def rb(t):
        r = torch.from_numpy(bf16_round(t.detach().float().numpy())).double()
        return t + (r - t).detach()

    pooled = h0.mean(1)
    out = {}
    for head, (w1, b1, w2, b2) in (("recipe", p["r"]), ("depth", p["d"])):
        z1 = rb(pooled) @ rb(w1).T + b1
        out[head + "_logits"] = (F_.silu(z1) @ w2.T + b2) * inv_t

    def heads(lg, idv):
        pr = F_.softmax(lg, -1)
        hard = F_.one_hot(idv, pr.shape[-1]).double()
        return pr, hard + pr - pr.detach(), -(pr.clamp_min(1e-9).log() * pr).sum(-1)

    rl, dl = out["recipe_logits"], out["depth_logits"]
    out["recipe_probs"], out["recipe_onehot_st"], out["recipe_entropy"] = heads(rl, ids["recipe_id"])
    out["depth_probs"], out["depth_onehot_st"], out["depth_entropy"] = heads(dl, ids["depth_id"])
    out["router_entropy"] = out["recipe_entropy"] + out["depth_entropy"]
    out["expected_depth"] = (out["depth_probs"] * p["dv"]).sum(-1)
    lbp = rl.unsqueeze(1) + p["pass"].unsqueeze(0) * inv_t
    out["recipe_logits_by_pass"] = lbp
    out["recipe_probs_by_pass"], out["recipe_onehot_st_by_pass"], _ = heads(lbp, ids["recipe_id_by_pass"])
    return out


@pytest.mark.parametrize("fixed", [(None, None), (4, 1)])
def test_router_operator_fields_and_gradients(fixed):
    """hip_ops.router (pool + layer-1 GEMMs + one heads launch; backward in two launches + GEMMs)
    against the fp64 restatement: logits within 1e-4 (fp32 sums of bf16-exact layer-1 operands),
    ids the first argmax of the kernel's own probabilities (a tied pair of recipe rows picks the
    lower index), probabilities / entropies / expected depth within 1e-5 of the formulas on the
    kernel's logits, one-hot rows exactly (onehot + p) - p; gradients of h0 and every router
    parameter for upstream gradients on all differentiable fields within 2e-2."""
    from rte_amd.kernels import hip_ops

    g = torch.Generator().manual_seed(41)
    B, S, d, hid, R, D, P = 6, 20, 128, 128, 9, 3, 4
    inv_t = 1.0 / 0.7

    def rnd(*s, sc=1.0):
        return (torch.randn(*s, generator=g, dtype=torch.float64) * sc)

    w2r = rnd(R, hid, sc=0.2)
    b2r = rnd(R, sc=0.1)
    w2r[5] = w2r[2]
    b2r[5] = b2r[2] = 4.0  # recipes 2 and 5 tie for the maximum on every row
    cpu = {"r": [rnd(hid, d, sc=0.1), rnd(hid, sc=0.1), w2r, b2r],
           "d": [rnd(hid, d, sc=0.1), rnd(hid, sc=0.1), rnd(D, hid, sc=0.2), rnd(D, sc=0.1)],
           "pass": rnd(P, R, sc=0.5), "dv": torch.tensor([1.0, 2.0, 4.0], dtype=torch.float64)}
    h0c = rnd(B, S, d)
    dev = [t.float().to(DEV).requires_grad_() for t in (*cpu["r"], *cpu["d"], cpu["pass"])]
    h0 = h0c.float().to(DEV).requires_grad_()
    dvals = torch.tensor([1, 2, 4], dtype=torch.long, device=DEV)
    fr, fd = fixed
    f = hip_ops.router(h0, *dev[:8], dev[8], dvals, inv_t=inv_t, fixed_recipe=fr, fixed_depth=fd)
    rp = _np(f["recipe_probs"])
    if fr is None:
        assert (f["recipe_id"].cpu().numpy() == 2).all()
        np.testing.assert_array_equal(f["recipe_id"].cpu().numpy(), rp.argmax(-1))
        np.testing.assert_array_equal(f["recipe_id_by_pass"].cpu().numpy(), _np(f["recipe_probs_by_pass"]).argmax(-1))
        np.testing.assert_array_equal(f["depth_id"].cpu().numpy(), _np(f["depth_probs"]).argmax(-1))
    else:
        assert (f["recipe_id"].cpu().numpy() == fr).all() and (f["recipe_id_by_pass"].cpu().numpy() == fr).all()
        assert (f["depth_id"].cpu().numpy() == fd).all()
    np.testing.assert_array_equal(f["depth"].cpu().numpy(), np.array([1, 2, 4])[f["depth_id"].cpu().numpy()])
    for name in ("recipe", "depth"):
        lg = f[name + "_logits"].detach().cpu().numpy()
        own = RO_softmax(lg.astype(np.float64))
        np.testing.assert_allclose(_np(f[name + "_probs"]), own, rtol=1e-5, atol=1e-7)
        pf = f[name + "_probs"].detach().cpu().numpy()
        hard = np.eye(pf.shape[-1], dtype=np.float32)[f[name + "_id"].cpu().numpy()]
        np.testing.assert_array_equal(f[name + "_onehot_st"].detach().cpu().numpy(), (hard + pf) - pf)
        ent = -(np.log(np.maximum(own, 1e-9)) * own).sum(-1)
        np.testing.assert_allclose(_np(f[name + "_entropy"]), ent, rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(_np(f["router_entropy"]), _np(f["recipe_entropy"]) + _np(f["depth_entropy"]),
                               rtol=1e-6)
    np.testing.assert_allclose(_np(f["expected_depth"]), (_np(f["depth_probs"]) * [1.0, 2.0, 4.0]).sum(-1), rtol=1e-5)

    h0r = h0c.clone().requires_grad_()
    prm = {"r": [t.clone().requires_grad_() for t in cpu["r"]], "d": [t.clone().requires_grad_() for t in cpu["d"]],
           "pass": cpu["pass"].clone().requires_grad_(), "dv": cpu["dv"]}
    ids = {k: f[k].cpu() for k in ("recipe_id", "depth_id", "recipe_id_by_pass")}
    ref = _router_ref(h0r, prm, ids, inv_t)
    for k in ("recipe_logits", "depth_logits", "recipe_logits_by_pass"):
        assert_rel(_np(f[k]), ref[k].detach().numpy(), 1e-4, k)
    loss_k, loss_r = 0.0, 0.0
    for k, v in ref.items():
        gk = torch.randn(v.shape, generator=g, dtype=torch.float64)
        loss_r = loss_r + (v * gk).sum()
        loss_k = loss_k + (f[k] * gk.float().to(DEV)).sum()
    loss_k.backward()
    loss_r.backward()
    assert_rel(_np(h0.grad), h0r.grad.numpy(), BF16_RTOL, "d h0")
    refs = [*prm["r"], *prm["d"], prm["pass"]]
    names = ["w1r", "b1r", "w2r", "b2r", "w1d", "b1d", "w2d", "b2d", "pass_bias"]
    for n, a, b in zip(names, dev, refs):
        assert_rel(_np(a.grad), b.grad.numpy(), BF16_RTOL, n)


def RO_softmax(x):
    e = np.exp(x - x.max(-1, keepdims=True))
    return e / e.sum(-1, keepdims=True)


def test_router_aux_operator_matches_torch_formula():
    """hip_ops.router_aux (one launch forward, one backward) against router_aux_losses
    (rte/metrics.py:97-112 in torch ops) on the same device tensors: values and the gradients of
    the recipe probabilities and expected depth within 1e-5."""
    from types import SimpleNamespace

    from rte_amd.kernels import hip_ops
    from rte_amd.training import router_aux_losses

    tr = SimpleNamespace(lambda_load=0.3, lambda_cover=0.7, lambda_depth=0.05, coverage_min=0.2)
    g = torch.Generator().manual_seed(43)
    probs0 = torch.softmax(torch.randn(37, 16, generator=g), -1)
    ed0 = torch.rand(37, generator=g) * 4
    ema = torch.rand(16, generator=g) * 0.4
    outs, grads = [], []
    for fn in ("hip", "torch"):
        p = probs0.to(DEV).requires_grad_()
        e = ed0.to(DEV).requires_grad_()
        if fn == "hip":
            o = hip_ops.router_aux(p, e, ema.to(DEV), coverage_min=tr.coverage_min, lambda_load=tr.lambda_load,
                                   lambda_cover=tr.lambda_cover, lambda_depth=tr.lambda_depth)
        else:
            o = router_aux_losses(p, e, ema.to(DEV), tr)
        (2.0 * o["load"] + 3.0 * o["cover"] - 1.5 * o["depth"]).backward()
        outs.append([o[k].item() for k in ("load", "cover", "depth")])
        grads.append((_np(p.grad), _np(e.grad)))
    np.testing.assert_allclose(outs[0], outs[1], rtol=1e-5)
    np.testing.assert_allclose(grads[0][0], grads[1][0], rtol=1e-5, atol=1e-9)
    np.testing.assert_allclose(grads[0][1], grads[1][1], rtol=1e-5, atol=1e-9)


def test_audit_fixed_sampler_and_usage_ema_match_torch_formulas():
    """hip_ops.audit_sample_fixed against AuditEngine.compute_audit_prob + the fixed-count branch of
    sample_mask_with_prob (rte/audit.py:79-132, torch ops on the same device tensors): requested
    probability within 1e-6, mask and inclusion probability exact, the five means; hip_ops.count_ema
    against the bincount EMA (rte/recipes.py update_usage, the audit coverage update) with and
    without a mask, within 1e-6."""
    from types import SimpleNamespace

    from rte_amd.audit import AuditEngine
    from rte_amd.kernels import hip_ops

    cfg = SimpleNamespace(audit_fixed_count_per_batch=5, audit_p_min=0.02, audit_p_max=0.6, audit_alpha=0.7,
                          audit_beta=0.3, audit_gamma=0.9, coverage_min=0.15, coverage_beta=0.9)
    eng = AuditEngine(cfg)
    eng.recent_residual = 0.37
    g = torch.Generator().manual_seed(44)
    B, R, D = 300, 16, 3
    ids = torch.randint(0, R, (B,), generator=g).to(DEV)
    ent = (torch.rand(B, generator=g) * 3).to(DEV)
    eng.recipe_audit_ema = (torch.rand(R, generator=g) * 0.3).to(DEV)
    meta = SimpleNamespace(router=SimpleNamespace(router_entropy=ent, recipe_logits=torch.empty(1, R),
                                                  depth_logits=torch.empty(1, D)), recipe_ids=ids)
    chosen = torch.randperm(B, generator=g)[:5].to(DEV)
    req_t = eng.compute_audit_prob(meta)
    mask_t, incl_t, _, _ = eng.sample_mask_with_prob(req_t, seed=0, chosen=chosen)
    req, incl, mask, st = hip_ops.audit_sample_fixed(ent, ids, eng.recipe_audit_ema, chosen, denom=float(R + D),
                                                     p_min=0.02, p_max=0.6, alpha=0.7, beta=0.3, gamma=0.9,
                                                     residual=0.37, coverage_min=0.15)
    np.testing.assert_allclose(_np(req), _np(req_t), rtol=1e-6)
    np.testing.assert_array_equal(mask.cpu().numpy(), mask_t.cpu().numpy())
    np.testing.assert_array_equal(incl.cpu().numpy(), incl_t.cpu().numpy())
    ref = [incl_t.mean(), req_t.mean(), mask_t.float().mean(), mask_t.float().sum(), incl_t.mean()]
    np.testing.assert_allclose(_np(st), [float(v) for v in ref], rtol=1e-6)
    for m in (None, mask_t):
        ema0 = (torch.rand(R, generator=g) * 0.2).to(DEV)
        w = torch.ones(B, device=DEV) if m is None else m.float()
        counts = torch.zeros(R, device=DEV).index_add_(0, ids, w)
        ref_e = ema0 * 0.9 + (counts / counts.sum().clamp_min(1.0)) * 0.1
        e = ema0.clone()
        hip_ops.count_ema(ids, m, e, 0.9)
        np.testing.assert_allclose(_np(e), _np(ref_e), rtol=1e-6, atol=1e-8)


def test_step_flags_and_metrics_match_torch():
    """hip_ops.nonfinite_flags (the step's skip flag) on finite, inf, -inf and NaN losses, and
    hip_ops.step_metrics against the torch means of the metric keys (rte/training.py:1412-1472)."""
    from rte_amd.kernels import hip_ops

    for v, want in ((1.5, 0.0), (float("inf"), 1.0), (float("-inf"), 1.0), (float("nan"), 1.0), (0.0, 0.0)):
        bad, ok = hip_ops.nonfinite_flags(torch.tensor(v, device=DEV))
        assert (bad.item(), ok.item()) == (want, 1.0 - want), v
    g = torch.Generator().manual_seed(45)
    hot = (torch.rand(300, generator=g) * 50).to(DEV)
    corr = (torch.rand(300, generator=g) * 50).to(DEV)
    depth = torch.randint(1, 5, (300,), generator=g).to(DEV)
    m = hip_ops.step_metrics(hot, corr, depth, scale=64.0, seq=64.0)
    ref = [hot.mean() / 64.0, corr.mean() / 64.0, corr.mean() / 64.0, depth.float().mean()]
    np.testing.assert_allclose(_np(m), [float(r) for r in ref], rtol=1e-6)


def test_router_backward_small_heads():
    """Gradients through the router's Linear layers (the depth head has 3 outputs, not a multiple
    of the GEMM's 8-element vectors) against fp64 autograd of the same modules on the CPU."""
    from rte_amd.config import ModelConfig
    from rte_amd.routing import Router

    cfg = ModelConfig(topology="recursive", vocab_size=64, d_model=64, n_heads=4, d_ff=128, n_dense_layers=1,
                      n_prelude=1, n_coda=1, t_max=4, depth_choices=[1, 2, 4], attn_banks=1, ffn_banks=1,
                      head_groups=4, ffn_groups=4, active_head_groups=1, active_ffn_groups=1, recipe_count=5)
    torch.manual_seed(17)
    r = Router(cfg).to(DEV)
    with torch.no_grad():
        for prm in r.parameters():
            prm.copy_(torch.from_numpy(bf16_round(prm.detach().cpu().numpy())).to(DEV))
    h0 = torch.from_numpy(bf16_round(np.random.default_rng(17).standard_normal((4, 9, 64)).astype(np.float32)))
    out = r(h0.to(DEV))
    loss = (out.recipe_probs * torch.arange(5, device=DEV)).sum() + out.expected_depth.sum()
    loss.backward()
    ref = Router(cfg).double()
    ref.load_state_dict({k: v.detach().double().cpu() for k, v in r.state_dict().items()})
    F_ = torch.nn.functional
    pooled = h0.double().mean(1)
    rl = ref.recipe_mlp(pooled)
    dl = ref.depth_mlp(pooled)
    lref = (F_.softmax(rl, -1) * torch.arange(5)).sum() + (F_.softmax(dl, -1) * torch.tensor([1.0, 2.0, 4.0])).sum()
    lref.backward()
    for (n, a), (_, b) in zip(r.named_parameters(), ref.named_parameters()):
        if b.grad is not None:
            assert_rel(_np(a.grad), b.grad.numpy(), 5e-2, n)
