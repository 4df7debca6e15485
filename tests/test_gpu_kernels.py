"""GPU parity of the HIP kernels against the CPU oracle (same seeded inputs).

Indices bit-exact; fp32-output GEMMs of bf16-exact inputs within 1e-5 relative;
bf16 paths within 2e-2 relative (Frobenius norm), as the build contract states.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from helpers import BF16_RTOL, FP32_RTOL, assert_rel, bf16_round
from oracle import attention as A
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


def _ops():
    from rte_amd.kernels import hip_ops

    return hip_ops


def _bf(a: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a, np.float32)).to(DEV).to(torch.bfloat16)


def _np(t: torch.Tensor) -> np.ndarray:
    return t.detach().float().cpu().numpy()


# ---------------------------------------------------------------- GEMM core

@pytest.mark.parametrize("a_t", [False, True])
@pytest.mark.parametrize("b_t", [False, True])
@pytest.mark.parametrize("M,N,K", [(136, 72, 48), (512, 384, 512), (64, 2048, 96), (1000, 32, 64)])
def test_gemm_layouts_fp32_out(a_t, b_t, M, N, K):
    H = _ops()
    rng = np.random.default_rng(M * 7 + N + K)
    A_ = bf16_round(rng.standard_normal((M, K)).astype(np.float32))
    B_ = bf16_round(rng.standard_normal((N, K)).astype(np.float32))
    ref = A_.astype(np.float64) @ B_.astype(np.float64).T
    a = _bf(A_.T.copy() if a_t else A_)
    b = _bf(B_.T.copy() if b_t else B_)
    print(f"gemm a_t={a_t} b_t={b_t} M={M} N={N} K={K}", flush=True)
    c = H.gemm(a, b, a_t=a_t, b_t=b_t, out_f32=True)
    torch.cuda.synchronize()
    assert_rel(_np(c), ref, FP32_RTOL, "gemm fp32")


@pytest.mark.parametrize("M,N,K", [(129, 129, 64), (300, 200, 128), (1000, 520, 192), (2048, 1536, 512),
                                   (4100, 260, 1024), (700, 300, 2112)])
def test_gemm_layout_nn_k64_shapes(M, N, K):
    """Both operands k-contiguous with K a multiple of 64 (the direct-to-LDS main loop):
    ragged tile edges in M and N, one to sixteen k tiles, bf16 and fp32 outputs."""
    H = _ops()
    rng = np.random.default_rng(M + 3 * N + K)
    A_ = bf16_round(rng.standard_normal((M, K)).astype(np.float32))
    B_ = bf16_round(rng.standard_normal((N, K)).astype(np.float32))
    ref = A_.astype(np.float64) @ B_.astype(np.float64).T
    print(f"gemm nn M={M} N={N} K={K}", flush=True)
    c = H.gemm(_bf(A_), _bf(B_), out_f32=True)
    torch.cuda.synchronize()
    assert_rel(_np(c), ref, FP32_RTOL, "gemm nn fp32")
    cb = H.gemm(_bf(A_), _bf(B_))
    assert_rel(_np(cb), ref, 5e-3, "gemm nn bf16")


@pytest.mark.parametrize("a_t,b_t", [(False, True), (True, False), (True, True)])
@pytest.mark.parametrize("M,N,K", [(136, 200, 64), (512, 384, 512), (1000, 520, 192), (2048, 1536, 2112)])
def test_gemm_layout_t_k64_shapes(a_t, b_t, M, N, K):
    """Layout-T operands on the direct-to-LDS main loop (k-major LDS tiles read through the
    transposing LDS loads): ragged tile edges, one to 33 k stages, split-K on the small grids."""
    H = _ops()
    rng = np.random.default_rng(M + 5 * N + K + 2 * a_t + b_t)
    A_ = bf16_round(rng.standard_normal((M, K)).astype(np.float32))
    B_ = bf16_round(rng.standard_normal((N, K)).astype(np.float32))
    ref = A_.astype(np.float64) @ B_.astype(np.float64).T
    a = _bf(A_.T.copy() if a_t else A_)
    b = _bf(B_.T.copy() if b_t else B_)
    print(f"gemm T a_t={a_t} b_t={b_t} M={M} N={N} K={K}", flush=True)
    c = H.gemm(a, b, a_t=a_t, b_t=b_t, out_f32=True)
    torch.cuda.synchronize()
    assert_rel(_np(c), ref, FP32_RTOL, "gemm layout T fp32")


@pytest.mark.parametrize("a_t", [False, True])
@pytest.mark.parametrize("b_t", [False, True])
@pytest.mark.parametrize("M,N,K", [(24, 304, 128), (64, 520, 192), (712, 56, 256), (1000, 32, 64), (96, 32, 2048)])
def test_gemm_narrow_k64_shapes(a_t, b_t, M, N, K):
    """Narrow tiles (32- or 64-wide sides) on the direct-load loop for every layout pair."""
    H = _ops()
    rng = np.random.default_rng(7 * M + N + K + 2 * a_t + b_t)
    A_ = bf16_round(rng.standard_normal((M, K)).astype(np.float32))
    B_ = bf16_round(rng.standard_normal((N, K)).astype(np.float32))
    ref = A_.astype(np.float64) @ B_.astype(np.float64).T
    a = _bf(A_.T.copy() if a_t else A_)
    b = _bf(B_.T.copy() if b_t else B_)
    print(f"gemm narrow a_t={a_t} b_t={b_t} M={M} N={N} K={K}", flush=True)
    c = H.gemm(a, b, a_t=a_t, b_t=b_t, out_f32=True)
    torch.cuda.synchronize()
    assert_rel(_np(c), ref, FP32_RTOL, "gemm narrow fp32")


@pytest.mark.parametrize("M,N,K", [(1, 8, 8), (37, 40, 16), (1000, 520, 24), (4096, 512, 32), (70000, 64, 32)])
def test_gemm_short_k(M, N, K):
    """K <= 32 with k-contiguous operands (the barrier-free wave kernel): ragged 32-row and
    32-column edges, K not a multiple of 16, fp32 with alpha + residual and bf16 outputs."""
    H = _ops()
    rng = np.random.default_rng(M + 11 * N + K)
    A_ = bf16_round(rng.standard_normal((M, K)).astype(np.float32))
    B_ = bf16_round(rng.standard_normal((N, K)).astype(np.float32))
    r = rng.standard_normal((M, N)).astype(np.float32)
    ref = A_.astype(np.float64) @ B_.astype(np.float64).T
    print(f"gemm short-k M={M} N={N} K={K}", flush=True)
    c = H.gemm(_bf(A_), _bf(B_), alpha=0.5, resid=torch.from_numpy(r).to(DEV), out_f32=True)
    torch.cuda.synchronize()
    assert_rel(_np(c), 0.5 * ref + r, FP32_RTOL, "gemm short-k fp32")
    cb = H.gemm(_bf(A_), _bf(B_))
    assert_rel(_np(cb), ref, 5e-3, "gemm short-k bf16")


def test_gemm_bf16_out_resid_alpha():
    H = _ops()
    rng = np.random.default_rng(3)
    A_ = bf16_round(rng.standard_normal((300, 256)).astype(np.float32))
    B_ = bf16_round(rng.standard_normal((200, 256)).astype(np.float32))
    r = rng.standard_normal((300, 200)).astype(np.float32)
    c = H.gemm(_bf(A_), _bf(B_), alpha=0.5, resid=torch.from_numpy(r).to(DEV), out_f32=True)
    ref = 0.5 * (A_.astype(np.float64) @ B_.T) + r
    assert_rel(_np(c), ref, FP32_RTOL, "gemm alpha+resid")
    cb = H.gemm(_bf(A_), _bf(B_))
    assert cb.dtype == torch.bfloat16
    assert_rel(_np(cb), A_.astype(np.float64) @ B_.T, 5e-3, "gemm bf16 out")


# ---------------------------------------------------------------- attention core

def _attn_ref(q, k, v, hs):
    """fp64 CPU causal attention with scale 1/sqrt(hd) and a per-(b, h) output scale."""
    S, hd = q.shape[2], q.shape[3]
    s = (q @ k.transpose(-1, -2)) / np.sqrt(hd)
    mask = torch.ones(S, S, dtype=torch.bool).tril()
    p = torch.softmax(s.masked_fill(~mask, float("-inf")), dim=-1)
    out = p @ v
    return out if hs is None else out * hs[:, :, None, None]


@pytest.mark.parametrize("B,H,S,scaled,hd", [(2, 3, 64, False, 64), (1, 8, 64, True, 64), (2, 2, 100, True, 64),
                                             (1, 2, 512, False, 64), (3, 1, 33, True, 64), (2, 1, 1, False, 64),
                                             (2, 4, 16, True, 32), (2, 3, 70, False, 32), (1, 2, 130, True, 128)])
def test_attention_matches_reference(B, H, S, scaled, hd):
    """HIP causal attention against fp64 softmax attention: output and dq, dk, dv within the bf16
    tolerance, ragged 32-row blocks, zero head scales, head_dim 32 / 64 / 128, backward bitwise
    repeatable."""
    H_ = _ops()
    rng = np.random.default_rng(B * 1000 + H * 10 + S)
    qn, kn, vn = (bf16_round(rng.standard_normal((B, H, S, hd)).astype(np.float32)) for _ in range(3))
    hsn = None
    if scaled:
        hsn = rng.choice([0.0, 0.5, 1.0], size=(B, H)).astype(np.float32)
        hsn.flat[0] = 0.0
        hsn.flat[-1] = 1.0
    g = rng.standard_normal((B, H, S, hd)).astype(np.float32)
    tq, tk, tv = (_bf(a).requires_grad_() for a in (qn, kn, vn))
    ths = None if hsn is None else torch.from_numpy(hsn).to(DEV)
    print(f"attention B={B} H={H} S={S} hd={hd} scaled={scaled}", flush=True)
    out = H_.attention(tq, tk, tv, ths)
    out.backward(torch.from_numpy(g).to(DEV))
    torch.cuda.synchronize()
    rq, rk, rv = (torch.from_numpy(a).double().requires_grad_() for a in (qn, kn, vn))
    ref = _attn_ref(rq, rk, rv, None if hsn is None else torch.from_numpy(hsn).double())
    ref.backward(torch.from_numpy(g).double())
    assert_rel(_np(out), ref.detach().numpy(), BF16_RTOL, "attention out")
    for name, t, r in (("dq", tq, rq), ("dk", tk, rk), ("dv", tv, rv)):
        assert_rel(_np(t.grad), r.grad.numpy(), BF16_RTOL, f"attention {name}")
    first = [t.grad.clone() for t in (tq, tk, tv)]
    for t in (tq, tk, tv):
        t.grad = None
    H_.attention(tq, tk, tv, ths).backward(torch.from_numpy(g).to(DEV))
    assert all(torch.equal(a, t.grad) for a, t in zip(first, (tq, tk, tv))), "attention backward not repeatable"


# ---------------------------------------------------------------- routing / packing

@pytest.mark.parametrize("T,C,k", [(1, 4, 1), (513, 32, 4), (8192, 64, 8), (301, 100, 16), (64, 128, 16),
                                   (300, 256, 16), (77, 1000, 3), (20000, 64, 8), (17000, 100, 16),
                                   (16384, 128, 3), (16385, 7, 5)])
def test_route_topk_bit_exact(T, C, k):
    H = _ops()
    rng = np.random.default_rng(T + C)
    lg = rng.integers(-4, 5, size=(T, C)).astype(np.float32) + rng.standard_normal((T, C)).astype(np.float32) * (
        rng.random((T, C)) < 0.5
    )
    if T > 10:
        lg[7, 3] = np.nan
    ids, w = H.route_topk(torch.from_numpy(lg).to(DEV), k)
    rids, rw = R.route_topk(lg, k)
    np.testing.assert_array_equal(ids.cpu().numpy(), rids)
    ok = ~np.isnan(lg).any(-1)
    np.testing.assert_allclose(w.cpu().numpy()[ok], rw[ok], rtol=FP32_RTOL, atol=1e-7)


@pytest.mark.parametrize("C,k", [(64, 8), (100, 16), (7, 5)])
def test_route_topk_kernels_agree(C, k):
    """The one-lane-per-token kernel (T >= 16384) and the wave-per-token kernel give identical ids
    and weights on the same rows (same order, same softmax summation)."""
    H = _ops()
    rng = np.random.default_rng(C * 31 + k)
    lg = (rng.integers(-3, 4, size=(16400, C)) + rng.standard_normal((16400, C)) * (rng.random((16400, C)) < 0.7))
    lg = torch.from_numpy(lg.astype(np.float32)).to(DEV)
    ids_l, w_l = H.route_topk(lg, k)
    ids_w, w_w = H.route_topk(lg[:8000].contiguous(), k)
    assert torch.equal(ids_l[:8000], ids_w) and torch.equal(w_l[:8000], w_w)


@pytest.mark.parametrize("B,S,R,kmax,C", [(1, 64, 6, 8, 64), (128, 64, 16, 8, 64), (37, 5, 9, 4, 300),
                                          (1, 64, 16, 64, 64), (64, 8, 60, 8, 300)])
def test_pack_routes_matches_expanded_pack(B, S, R, kmax, C):
    """Route-list pack from recipe ids equals the counting-sort pack of the expanded per-token
    routes (every field bit-exact), with -1 padding, inactive samples and an unknown recipe id.
    The last case's recipe table is too large for the plan's LDS tables (the scanning plan)."""
    H = _ops()
    rng = np.random.default_rng(B + R + C)
    routes = np.full((R, kmax), -1, np.int32)
    for r in range(R):
        m = rng.integers(1, kmax + 1)
        routes[r, :m] = rng.choice(C, size=m, replace=False)
    rw = rng.random(R).astype(np.float32)
    rid = rng.integers(0, R, B).astype(np.int64)
    active = rng.random(B) < 0.8
    if B > 2:
        rid[2] = R + 3  # unknown recipe: no routes
    exp_ids = np.where((active[:, None] & (rid[:, None] < R)), routes[np.minimum(rid, R - 1)], -1)
    ids = np.repeat(exp_ids, S, axis=0)
    w = np.repeat(np.where(rid < R, rw[np.minimum(rid, R - 1)], 0.0), S)[:, None].repeat(kmax, 1).astype(np.float32)
    print(f"pack_routes B={B} S={S} R={R} kmax={kmax} C={C}", flush=True)
    got = H.pack_routes(torch.from_numpy(rid).to(DEV), torch.from_numpy(routes).to(DEV),
                        torch.from_numpy(rw).to(DEV), S, C, torch.from_numpy(active).to(DEV))
    want = H.pack_index(torch.from_numpy(ids).to(DEV), C, torch.from_numpy(w).to(DEV))
    n = int(want.offsets[-1].item())
    assert torch.equal(got.offsets, want.offsets)
    for name in ("tok_of_slot", "pair_of_slot", "w_of_slot"):
        assert torch.equal(getattr(got, name)[:n], getattr(want, name)[:n]), name
    assert torch.equal(got.slot_of_pair, want.slot_of_pair)


@pytest.mark.parametrize("T,k,C", [(1, 1, 1), (1000, 4, 32), (8192, 8, 64), (4096, 16, 256), (5000, 3, 77),
                                   (20000, 8, 64), (70001, 8, 64)])
def test_pack_index_bit_exact(T, k, C):
    H = _ops()
    rng = np.random.default_rng(T * k + C)
    # skewed (Zipf-like) cluster loads, distinct clusters per token
    p = 1.0 / np.arange(1, C + 1) ** 1.1
    p /= p.sum()
    cl = np.stack([rng.choice(C, size=k, replace=False, p=p) for _ in range(T)]).astype(np.int32)
    w = rng.random((T, k)).astype(np.float32)
    pk = H.pack_index(torch.from_numpy(cl).to(DEV), C, torch.from_numpy(w).to(DEV))
    ref = R.pack_index(cl, C, k)
    for name in ("offsets", "pair_of_slot", "tok_of_slot", "slot_of_pair"):
        np.testing.assert_array_equal(getattr(pk, name).cpu().numpy(), ref[name], err_msg=name)
    np.testing.assert_array_equal(pk.w_of_slot.cpu().numpy(), w.reshape(-1)[ref["pair_of_slot"]])


@pytest.mark.parametrize("T,d,C,k", [(8192, 512, 64, 8), (1000, 256, 32, 1), (777, 128, 128, 16),
                                     (4096, 1024, 128, 8), (31, 64, 64, 8)])
def test_route_pack_matches_gemm_topk_pack(T, d, C, k):
    """rte_route_pack (router GEMM + top-k + pack in two launches): its logits within fp32
    rounding of the oracle's x wr^T, its ids / weights bitwise route_topk of its own logits (and
    the oracle's top-k rule), its pack bitwise rte_pack_index of those ids; skewed router rows."""
    H = _ops()
    rng = np.random.default_rng(T + 7 * C + k)
    x = bf16_round(rng.standard_normal((T, d)).astype(np.float32))
    # Zipf-like load: cluster c's router row grows with its popularity
    wr = bf16_round((rng.standard_normal((C, d)) * 0.05 + 0.02 * (1.0 / np.arange(1, C + 1))[:, None]).astype(np.float32))
    print(f"route_pack T={T} d={d} C={C} k={k}", flush=True)
    ids, w, pk, logits = H.route_pack(_bf(x), _bf(wr), k, with_logits=True)
    ref_logits = x.astype(np.float64) @ wr.astype(np.float64).T
    assert_rel(_np(logits), ref_logits, FP32_RTOL, "route_pack logits")
    ids2, w2 = H.route_topk(logits, k)
    assert torch.equal(ids, ids2) and torch.equal(w, w2), "route_pack top-k differs from route_topk"
    ref_ids, _ = R.route_topk(_np(logits).astype(np.float32), k)
    np.testing.assert_array_equal(ids.cpu().numpy(), ref_ids)
    pk2 = H.pack_index(ids, C, w)
    for name in ("offsets", "tok_of_slot", "pair_of_slot", "slot_of_pair", "w_of_slot"):
        assert torch.equal(getattr(pk, name), getattr(pk2, name)), name


@pytest.mark.parametrize("T,C,k", [(8192, 64, 8), (333, 100, 5)])
def test_route_bwd_matches_oracle(T, C, k):
    """dlogits of the top-k softmax: bf16 and fp32 outputs; pairs whose slot is -1 carry no
    gradient (their dw counts as 0)."""
    from rte_amd import _lib

    H = _ops()
    rng = np.random.default_rng(T + k)
    lg = rng.standard_normal((T, C)).astype(np.float32)
    ids, w = H.route_topk(torch.from_numpy(lg).to(DEV), k)
    cl = ids.clone()
    cl[::7, 0] = -1  # dropped pairs
    pk = H.pack_index(cl, C, w)
    dw_slot = torch.from_numpy(rng.standard_normal(T * k).astype(np.float32)).to(DEV)
    d32 = torch.empty(T, C, device=DEV)
    d16 = torch.empty(T, C, device=DEV, dtype=torch.bfloat16)
    _lib.call("rte_route_bwd", ids.data_ptr(), w.data_ptr(), dw_slot.data_ptr(), pk.slot_of_pair.data_ptr(), T, C,
              k, d16.data_ptr(), d32.data_ptr(), _lib.stream_ptr())
    sop = pk.slot_of_pair.cpu().numpy().reshape(T, k)
    dw = np.where(sop >= 0, dw_slot.cpu().numpy()[np.maximum(sop, 0)], 0.0)
    ref = R.route_softmax_bwd(ids.cpu().numpy(), w.cpu().numpy(), dw, C)
    np.testing.assert_allclose(d32.cpu().numpy(), ref, rtol=1e-5, atol=1e-6)
    np.testing.assert_array_equal(d16.float().cpu().numpy(), d32.to(torch.bfloat16).float().cpu().numpy())


def test_pack_index_counts_invalid_ids():
    H = _ops()
    cl = torch.tensor([0, 5, 1, -1, 1], dtype=torch.int32, device=DEV)
    bad = torch.zeros(1, dtype=torch.int32, device=DEV)
    pk = H.pack_index(cl.view(-1, 1), 2, invalid=bad)
    assert int(bad.item()) == 2
    assert pk.offsets.tolist() == [0, 1, 3]
    assert pk.slot_of_pair.tolist() == [0, -1, 1, -1, 2]


def test_combine_rows_fixed_order():
    H = _ops()
    rng = np.random.default_rng(5)
    T, k, d = 257, 5, 64
    rows = bf16_round(rng.standard_normal((T * k, d)).astype(np.float32))
    extra = bf16_round(rng.standard_normal((T, d)).astype(np.float32))
    res = rng.standard_normal((T, d)).astype(np.float32)
    out = H.combine_rows(_bf(rows), T, k, extra=_bf(extra), resid=torch.from_numpy(res).to(DEV))
    ref = res.astype(np.float64) + rows.reshape(T, k, d).sum(1) + extra
    assert_rel(_np(out), ref, FP32_RTOL, "combine")


# ---------------------------------------------------------------- SwiGLU

@pytest.mark.parametrize("wd_rows", [False, True])
@pytest.mark.parametrize("T,d,F", [(256, 128, 256), (8192, 512, 2048)])
def test_dense_swiglu_fwd_bwd(T, d, F, wd_rows):
    H = _ops()
    rng = np.random.default_rng(T + d + F)
    x = bf16_round(rng.standard_normal((T, d)).astype(np.float32))
    wug = (rng.standard_normal((2 * F, d)) * 0.02).astype(np.float32)
    wd = (rng.standard_normal((F, d) if wd_rows else (d, F)) * 0.02).astype(np.float32)
    res = rng.standard_normal((T, d)).astype(np.float32)
    dy = rng.standard_normal((T, d)).astype(np.float32)
    tx = _bf(x).requires_grad_()
    tug = torch.from_numpy(wug).to(DEV).requires_grad_()
    twd = torch.from_numpy(wd).to(DEV).requires_grad_()
    tres = torch.from_numpy(res).to(DEV).requires_grad_()
    out = H.dense_swiglu(tx, tug, twd, tres, wd_rows=wd_rows)
    out.backward(torch.from_numpy(dy).to(DEV))
    y, cache = SW.dense_swiglu_fwd(x, bf16_round(wug), bf16_round(wd), wd_rows=wd_rows)
    assert_rel(_np(out) - res, y, BF16_RTOL, "swiglu y")
    dx, dwug, dwd = SW.dense_swiglu_bwd(bf16_round(dy), x, bf16_round(wug), bf16_round(wd), cache, wd_rows=wd_rows)
    assert_rel(_np(tx.grad), dx, BF16_RTOL, "swiglu dx")
    assert_rel(_np(tug.grad), dwug, BF16_RTOL, "swiglu dwug")
    assert_rel(_np(twd.grad), dwd, BF16_RTOL, "swiglu dwd")
    np.testing.assert_array_equal(_np(tres.grad), dy)


# ---------------------------------------------------------------- routed cluster pool

@pytest.mark.parametrize(
    "T,d,C,n,k,fused",
    [(64, 64, 4, 32, 1, True), (1024, 256, 32, 32, 4, True), (1024, 256, 32, 32, 4, False),
     (8192, 512, 64, 32, 8, True), (8192, 512, 64, 32, 8, False), (2048, 256, 16, 64, 2, True),
     (512, 128, 8, 32, 3, True)],
)
def test_routed_cluster_pool_fwd_bwd(T, d, C, n, k, fused, monkeypatch):
    """fused: the per-cluster fused kernels where the shape allows (n = 32, d 128 / 256 / 512),
    else the two-GEMM form."""
    H = _ops()
    monkeypatch.setattr(H, "POOL_FUSED", [fused])
    rng = np.random.default_rng(T + d + C + n + k)
    F = C * n
    x = bf16_round(rng.standard_normal((T, d)).astype(np.float32))
    wr = (rng.standard_normal((C, d)) * 0.02).astype(np.float32)
    wug = (rng.standard_normal((2 * F, d)) * 0.02).astype(np.float32)
    wd = (rng.standard_normal((d, F)) * 0.02).astype(np.float32)
    res = rng.standard_normal((T, d)).astype(np.float32)
    dy = rng.standard_normal((T, d)).astype(np.float32)
    tx = _bf(x).requires_grad_()
    twr, tug, twd = (torch.from_numpy(a).to(DEV).requires_grad_() for a in (wr, wug, wd))
    tres = torch.from_numpy(res).to(DEV)
    print(f"routed T={T} d={d} C={C} n={n} k={k} fused={fused}", flush=True)
    out, ids, w = H.routed_cluster_pool_swiglu(tx, twr, tug, twd, k, resid=tres)
    out.backward(torch.from_numpy(dy).to(DEV))
    torch.cuda.synchronize()
    # routing decisions: bit-exact against the oracle on the kernel's own logits
    logits = H.gemm(_bf(x), _bf(bf16_round(wr)), out_f32=True)
    rids, rw = R.route_topk(_np(logits), k)
    np.testing.assert_array_equal(ids.cpu().numpy(), rids)
    np.testing.assert_allclose(w.cpu().numpy(), rw, rtol=FP32_RTOL, atol=1e-7)
    wr_b, wug_b, wd_b = bf16_round(wr), bf16_round(wug), bf16_round(wd)
    ref = CP.routed_fwd(x, wug_b, wd_b, rids, rw, C, resid=res)
    assert_rel(_np(out) - res, ref - res, BF16_RTOL, "routed y")
    dx, dwr, dwug, dwd, _ = CP.routed_bwd(bf16_round(dy), x, wr_b, wug_b, wd_b, rids, rw, C)
    assert_rel(_np(tx.grad), dx, BF16_RTOL, "routed dx")
    assert_rel(_np(twr.grad), dwr, BF16_RTOL, "routed dwr")
    assert_rel(_np(tug.grad), dwug, BF16_RTOL, "routed dwug")
    assert_rel(_np(twd.grad), dwd, BF16_RTOL, "routed dwd")


def test_routed_cluster_pool_is_deterministic():
    H = _ops()
    rng = np.random.default_rng(42)
    T, d, C, n, k = 4096, 256, 64, 32, 8
    x = _bf(rng.standard_normal((T, d)))
    ws = [torch.from_numpy((rng.standard_normal(s) * 0.02).astype(np.float32)).to(DEV)
          for s in ((C, d), (2 * C * n, d), (d, C * n))]
    dy = torch.from_numpy(rng.standard_normal((T, d)).astype(np.float32)).to(DEV)
    grads = []
    for _ in range(2):
        tx = x.clone().requires_grad_()
        params = [w.clone().requires_grad_() for w in ws]
        out, _, _ = H.routed_cluster_pool_swiglu(tx, *params, k)
        out.backward(dy)
        grads.append([tx.grad.clone()] + [p.grad.clone() for p in params] + [out.detach().clone()])
    for a, b in zip(*grads):
        assert torch.equal(a, b)


@pytest.mark.parametrize("d", [128, 256, 512])
def test_grouped_swiglu_fused_matches_two_gemm(d):
    """rte_grouped_swiglu_fused_fwd / _bwd against rte_grouped_swiglu_fwd / _bwd on one pack with
    skewed routing: one cluster spread over several 128-slot tiles, clusters with ragged tails,
    empty clusters, absent pairs (id -1).  Every output of the fused kernels lies within bf16
    rounding of the two-GEMM form (their fp32 products add the reduction in another order; ug,
    zw, dug and the rows are bf16); dw_slot and the weight gradients within the same bound; two
    fused runs agree bit for bit; rows of absent pairs are left untouched."""
    from rte_amd import _lib

    H = _ops()
    lib = _lib.load()
    assert lib.rte_grouped_swiglu_fused_ok(32, d) == 1 and lib.rte_grouped_swiglu_fused_ok(64, d) == 0
    rng = np.random.default_rng(d)
    T, C, n, k = 1000, 24, 32, 4
    F = C * n
    ids = np.stack([rng.permutation(C - 4)[:k] for _ in range(T)]).astype(np.int32)  # clusters 20..23 empty
    ids[: 3 * T // 4, 0] = 0          # cluster 0: 750+ slots (six tiles, ragged tail)
    ids[::5, 2] = -1                  # absent pairs
    tid = torch.from_numpy(ids).to(DEV)
    w = torch.from_numpy(rng.random((T, k)).astype(np.float32)).to(DEV)
    pk = H.pack_index(tid, C, w)
    P = T * k
    bf = torch.bfloat16
    x = torch.from_numpy(rng.standard_normal((T, d)).astype(np.float32)).to(DEV).to(bf)
    wug = (torch.from_numpy(rng.standard_normal((2 * F, d)).astype(np.float32)) * 0.05).to(DEV).to(bf)
    wd = (torch.from_numpy(rng.standard_normal((d, F)).astype(np.float32)) * 0.05).to(DEV).to(bf)
    dout = torch.from_numpy(rng.standard_normal((T, d)).astype(np.float32)).to(DEV).to(bf)
    valid = pk.slot_of_pair.cpu().numpy() >= 0
    nslot = int(pk.offsets[-1])
    print(f"fused grouped SwiGLU vs two-GEMM d={d} T={T} C={C} k={k} slots={nslot}", flush=True)

    def run(fused):
        sfx = "fused_" if fused else ""
        ug = torch.zeros(P, 2 * n, device=DEV, dtype=bf)
        zw = torch.zeros(P, n, device=DEV, dtype=bf)
        yp = torch.full((P, d), 7.0, device=DEV, dtype=bf)
        _lib.call(f"rte_grouped_swiglu_{sfx}fwd", x.data_ptr(), T, d, pk.offsets.data_ptr(), C, n, P,
                  pk.tok_of_slot.data_ptr(), pk.pair_of_slot.data_ptr(), pk.w_of_slot.data_ptr(), wug.data_ptr(),
                  wd.data_ptr(), F, ug.data_ptr(), zw.data_ptr(), yp.data_ptr(), None)
        dug = torch.zeros(P, 2 * n, device=DEV, dtype=bf)
        dws = torch.zeros(P, device=DEV, dtype=torch.float32)
        dxp = torch.full((P, d), 7.0, device=DEV, dtype=bf)
        dwug = torch.empty(2 * F, d, device=DEV, dtype=torch.float32)
        dwd = torch.empty(d, F, device=DEV, dtype=torch.float32)
        nb = lib.rte_grouped_swiglu_bwd_workspace_bytes(P, C, n, d)
        ws = torch.empty(max(nb, 16), device=DEV, dtype=torch.uint8)
        _lib.call(f"rte_grouped_swiglu_{sfx}bwd", dout.data_ptr(), x.data_ptr(), T, d, pk.offsets.data_ptr(), C, n,
                  P, pk.tok_of_slot.data_ptr(), pk.pair_of_slot.data_ptr(), pk.w_of_slot.data_ptr(), wug.data_ptr(),
                  wd.data_ptr(), F, ug.data_ptr(), zw.data_ptr(), dug.data_ptr(), dws.data_ptr(), dxp.data_ptr(),
                  dwug.data_ptr(), dwd.data_ptr(), 0, 0.0, ws.data_ptr(), nb, None)
        torch.cuda.synchronize()
        return [t.float().cpu().numpy() for t in (ug, zw, yp, dug, dws, dxp, dwug, dwd)]

    ref = run(False)
    got = run(True)
    again = run(True)
    names = ("ug", "zw", "y_pairs", "dug", "dw_slot", "dx_pairs", "dwug", "dwd")
    for name, a, b, c in zip(names, got, ref, again):
        np.testing.assert_array_equal(a, c, err_msg=f"{name}: fused runs differ")
        if name in ("y_pairs", "dx_pairs"):
            assert np.all(a[~valid] == 7.0), f"{name}: rows of absent pairs written"
            a, b = a[valid], b[valid]
        elif name in ("ug", "zw", "dug", "dw_slot"):
            a, b = a[:nslot], b[:nslot]
        assert_rel(a, b, BF16_RTOL, f"fused {name}")
        # elementwise: within a few bf16 ulps of the two-GEMM value
        np.testing.assert_allclose(a, b, rtol=2e-2, atol=2e-2 * float(np.abs(b).max()), err_msg=name)


def test_rmsnorm_bwd_bf16_companion():
    """The norm backward also writes dx in bf16: cast_bf16 of dx (or of a whole view of it)
    returns those values, bit for bit the cast kernel's, without a cast; after an in-place change
    of dx, or for a partial view, it casts again."""
    H = _ops()
    rng = np.random.default_rng(21)
    T, d = 1000, 256
    x = torch.from_numpy(rng.standard_normal((T, d)).astype(np.float32)).to(DEV).requires_grad_()
    w = torch.from_numpy(rng.random(d).astype(np.float32) + 0.5).to(DEV)
    seen = {}

    def grab(g):
        seen["g"] = g
        return g

    x.register_hook(grab)
    y = H.rmsnorm(x, w)
    y.float().mul(torch.from_numpy(rng.standard_normal((T, d)).astype(np.float32)).to(DEV)).sum().backward()
    torch.cuda.synchronize()
    g = seen["g"]
    comp = H.cast_bf16(g)
    ref = torch.empty(T, d, dtype=torch.bfloat16, device=DEV)
    from rte_amd import _lib

    _lib.call("rte_cast_f32_bf16", g.contiguous().data_ptr(), g.numel(), ref.data_ptr(), None)
    torch.cuda.synchronize()
    base = g._base if g._base is not None else g
    assert getattr(base, "_rte_bf16", None) is not None
    assert comp.data_ptr() == base._rte_bf16[0].data_ptr()  # the companion, no new cast
    assert torch.equal(comp, ref)
    assert H.cast_bf16(g[: T // 2]).data_ptr() != comp.data_ptr()  # a partial view casts
    g.mul_(2.0)
    again = H.cast_bf16(g)
    torch.cuda.synchronize()
    assert again.data_ptr() != comp.data_ptr()
    assert torch.equal(again.float(), (ref.float() * 2.0).to(torch.bfloat16).float())


def test_loss_sum_matches_torch():
    """rte_loss_sum / _bwd: coef * sum(x) + sum of scalar terms, gradient coef for every row of x
    and 1 for every term, against torch in float64 (30 terms, one not requiring a gradient)."""
    H = _ops()
    rng = np.random.default_rng(3)
    x = torch.from_numpy(rng.standard_normal(131).astype(np.float32)).to(DEV).requires_grad_()
    terms = [torch.tensor(float(v), device=DEV, requires_grad=i != 7) for i, v in enumerate(rng.standard_normal(30))]
    coef = 1.0 / (131 * 64)
    print("loss_sum: 131 rows, 30 terms", flush=True)
    out = H.loss_sum(x, coef, terms)
    (out * 3.0).backward()
    torch.cuda.synchronize()
    ref = coef * x.detach().double().sum() + sum(t.detach().double() for t in terms)
    assert abs(float(out.detach()) - float(ref)) <= 1e-6 * max(1.0, abs(float(ref)))
    np.testing.assert_allclose(_np(x.grad), np.full(131, 3.0 * coef, np.float32), rtol=1e-6)
    for i, t in enumerate(terms):
        assert (t.grad is None) if i == 7 else float(t.grad) == 3.0


# ---------------------------------------------------------------- attention pieces

@pytest.mark.parametrize("T,d", [(5, 64), (8192, 512)])
def test_rmsnorm_fwd_bwd(T, d):
    H = _ops()
    rng = np.random.default_rng(T + d)
    x = rng.standard_normal((T, d)).astype(np.float32)
    w = (1 + 0.1 * rng.standard_normal(d)).astype(np.float32)
    dy = bf16_round(rng.standard_normal((T, d)).astype(np.float32))
    tx = torch.from_numpy(x).to(DEV).requires_grad_()
    tw = torch.from_numpy(w).to(DEV).requires_grad_()
    y = H.rmsnorm(tx, tw)
    y.backward(_bf(dy))
    assert_rel(_np(y), A.rmsnorm(x, w), 5e-3, "rmsnorm y")
    dx, dw = A.rmsnorm_bwd(dy, x, w)
    assert_rel(_np(tx.grad), dx, 1e-5, "rmsnorm dx")
    assert_rel(_np(tw.grad), dw, 1e-5, "rmsnorm dw")


@pytest.mark.parametrize("B,S,H_,hd", [(2, 16, 2, 64), (128, 64, 8, 64), (1, 64, 8, 64), (3, 40, 4, 64)])
def test_qkv_rope_fwd_bwd(B, S, H_, hd):
    """QKV + RoPE forward / backward against the oracle; (1, 64, 8, 64) and (3, 40, 4, 64) have
    few output tiles and run the split-K path whose reduce applies RoPE."""
    H = _ops()
    d = H_ * hd
    rng = np.random.default_rng(B + S)
    x = bf16_round(rng.standard_normal((B, S, d)).astype(np.float32))
    w = (rng.standard_normal((3 * d, d)) * 0.02).astype(np.float32)
    cos, sin = A.rope_tables(hd, S)
    tx = _bf(x).requires_grad_()
    tw = torch.from_numpy(w).to(DEV).requires_grad_()
    tc = torch.from_numpy(cos.astype(np.float32)).to(DEV)
    ts = torch.from_numpy(sin.astype(np.float32)).to(DEV)
    q, k, v = H.qkv_rope(tx, tw, tc, ts, H_)
    rq, rk, rv = A.qkv_rope(x, bf16_round(w), H_, cos, sin)
    for got, ref, nm in ((q, rq, "q"), (k, rk, "k"), (v, rv, "v")):
        assert_rel(_np(got), ref, BF16_RTOL, nm)
    g = [bf16_round(rng.standard_normal(q.shape).astype(np.float32)) for _ in range(3)]
    # non-contiguous gradient layouts like SDPA produces ([B,S,H,hd] memory)
    tg = [_bf(a.transpose(0, 2, 1, 3).copy()).transpose(1, 2) for a in g]
    torch.autograd.backward([q, k, v], tg)
    dx, dw = A.qkv_rope_bwd(*g, x, bf16_round(w), cos, sin)
    assert_rel(_np(tx.grad), dx, BF16_RTOL, "qkv dx")
    assert_rel(_np(tw.grad), dw, BF16_RTOL, "qkv dw")


def test_attn_out_proj_strided_input():
    H = _ops()
    B, S, H_, hd = 4, 32, 4, 64
    d = H_ * hd
    rng = np.random.default_rng(9)
    y = bf16_round(rng.standard_normal((B, S, H_, hd)).astype(np.float32))
    w = (rng.standard_normal((d, d)) * 0.05).astype(np.float32)
    r = rng.standard_normal((B, S, d)).astype(np.float32)
    dout = rng.standard_normal((B, S, d)).astype(np.float32)
    ty = _bf(y).transpose(1, 2).requires_grad_()  # [B,H,S,hd] view of [B,S,H,hd] memory
    ty.retain_grad()
    tw = torch.from_numpy(w).to(DEV).requires_grad_()
    out = H.attn_out_proj(ty, tw, torch.from_numpy(r).to(DEV))
    out.backward(torch.from_numpy(dout).to(DEV))
    y2 = y.reshape(B * S, d).astype(np.float64)
    ref = y2 @ bf16_round(w).T + r.reshape(B * S, d)
    assert_rel(_np(out).reshape(B * S, d), ref, 1e-5, "oproj")
    db = bf16_round(dout).reshape(B * S, d).astype(np.float64)
    assert_rel(_np(ty.grad.transpose(1, 2)).reshape(B * S, d), db @ bf16_round(w), BF16_RTOL, "oproj dy")
    assert_rel(_np(tw.grad), db.T @ y2, 1e-5, "oproj dw")


# ---------------------------------------------------------------- SVD low-rank FFN

@pytest.mark.parametrize("T,d,F,r", [(256, 128, 256, 32), (4096, 1024, 4096, 128), (1000, 256, 512, 64),
                                     (200, 128, 384, 128), (8, 64, 128, 64)])
def test_svd_ffn_fwd_bwd(T, d, F, r):
    """SVD FFN forward and backward against the oracle: rank 32 on the four-GEMM path, ranks 64 /
    128 on the on-chip path (token counts that fill no whole 128-token tile, one neuron tile)."""
    from oracle import svd_ffn as SV

    H = _ops()
    rng = np.random.default_rng(T + r)

    def orth(n, k):
        q, _ = np.linalg.qr(rng.standard_normal((n, k)))
        return q

    S = [10 ** rng.uniform(-2, 0, r) for _ in range(3)]
    m = dict(us_up=orth(d, r) * S[0], us_gate=orth(d, r) * S[1], v_up=orth(F, r), v_gate=orth(F, r),
             v_dn=orth(F, r), us_dn=orth(d, r) * S[2])
    m = {k: bf16_round(v.astype(np.float32)) for k, v in m.items()}
    x = bf16_round(rng.standard_normal((T, d)).astype(np.float32))
    dy = bf16_round(rng.standard_normal((T, d)).astype(np.float32))
    tw = {k: torch.from_numpy(v).to(DEV).requires_grad_() for k, v in m.items()}
    tx = _bf(x).requires_grad_()
    us_ug = torch.cat([tw["us_up"], tw["us_gate"]], 1)
    v_ug = torch.cat([tw["v_up"], tw["v_gate"]], 0)
    print(f"svd_ffn T={T} d={d} F={F} r={r}", flush=True)
    y = H.svd_ffn(tx, us_ug, v_ug, tw["v_dn"], tw["us_dn"])
    y.backward(torch.from_numpy(dy).to(DEV))
    ref, c = SV.svd_ffn_fwd(x, **m)
    assert_rel(_np(y), ref, BF16_RTOL, "svd y")
    g = SV.svd_ffn_bwd(dy, x, **m, c=c)
    assert_rel(_np(tx.grad), g["dx"], BF16_RTOL, "svd dx")
    for k in m:
        assert_rel(_np(tw[k].grad), g["d" + k], BF16_RTOL, f"svd d{k}")


@pytest.mark.parametrize("T,d,F,r", [(2048, 512, 1024, 128), (1016, 256, 512, 64)])
def test_svd_ffn_fused_matches_unfused_and_repeats(T, d, F, r):
    """rte_svd_ffn_fused_* against rte_svd_ffn_* through the C-ABI on the same inputs (bf16
    rounding apart: the unfused path rounds the activations to bf16 in HBM), and the fused call
    twice bitwise."""
    from rte_amd import _lib

    lib = _lib.load()
    g = torch.Generator(device=DEV)
    g.manual_seed(T + r)
    bf = torch.bfloat16

    def rnd(*shape, scale=1.0):
        return (torch.randn(*shape, device=DEV, generator=g) * scale).to(bf)

    x, dy = rnd(T, d), rnd(T, d)
    us_ug, v_ug = rnd(d, 2 * r, scale=d ** -0.5), rnd(2 * F, r, scale=r ** -0.5)
    v_dn, us_dn = rnd(F, r, scale=F ** -0.5), rnd(d, r, scale=r ** -0.5)
    st = _lib.stream_ptr()
    print(f"svd fused vs unfused T={T} d={d} F={F} r={r}", flush=True)

    def unfused():
        a, b = torch.empty(T, 2 * r, device=DEV, dtype=bf), torch.empty(T, r, device=DEV, dtype=bf)
        ug, z = torch.empty(T, 2 * F, device=DEV, dtype=bf), torch.empty(T, F, device=DEV, dtype=bf)
        y = torch.empty(T, d, device=DEV)
        _lib.call("rte_svd_ffn_fwd", x.data_ptr(), T, d, F, r, us_ug.data_ptr(), v_ug.data_ptr(), v_dn.data_ptr(),
                  us_dn.data_ptr(), None, a.data_ptr(), ug.data_ptr(), z.data_ptr(), b.data_ptr(), y.data_ptr(), 1, st)
        db, da = torch.empty(T, r, device=DEV, dtype=bf), torch.empty(T, 2 * r, device=DEV, dtype=bf)
        dug, dx = torch.empty(T, 2 * F, device=DEV, dtype=bf), torch.empty(T, d, device=DEV, dtype=bf)
        gr = [torch.empty(s, device=DEV) for s in ((d, 2 * r), (2 * F, r), (F, r), (d, r))]
        nb = lib.rte_gemm_workspace_bytes(max(d, F), 2 * r, T)
        ws = torch.empty(max(nb, 16), device=DEV, dtype=torch.uint8)
        _lib.call("rte_svd_ffn_bwd", dy.data_ptr(), x.data_ptr(), T, d, F, r, us_ug.data_ptr(), v_ug.data_ptr(),
                  v_dn.data_ptr(), us_dn.data_ptr(), a.data_ptr(), ug.data_ptr(), z.data_ptr(), b.data_ptr(),
                  db.data_ptr(), dug.data_ptr(), da.data_ptr(), dx.data_ptr(), *[t.data_ptr() for t in gr],
                  ws.data_ptr(), nb, st)
        return [y, dx, *gr]

    def fused():
        a, b = torch.empty(T, 2 * r, device=DEV, dtype=bf), torch.empty(T, r, device=DEV, dtype=bf)
        y = torch.empty(T, d, device=DEV)
        nb = lib.rte_svd_ffn_fused_workspace_bytes(T, d, F, r)
        ws = torch.empty(nb, device=DEV, dtype=torch.uint8)
        _lib.call("rte_svd_ffn_fused_fwd", x.data_ptr(), T, d, F, r, us_ug.data_ptr(), v_ug.data_ptr(),
                  v_dn.data_ptr(), us_dn.data_ptr(), None, a.data_ptr(), b.data_ptr(), y.data_ptr(), 1,
                  ws.data_ptr(), nb, st)
        db, da = torch.empty(T, r, device=DEV, dtype=bf), torch.empty(T, 2 * r, device=DEV, dtype=bf)
        dx = torch.empty(T, d, device=DEV, dtype=bf)
        gr = [torch.empty(s, device=DEV) for s in ((d, 2 * r), (2 * F, r), (F, r), (d, r))]
        _lib.call("rte_svd_ffn_fused_bwd", dy.data_ptr(), x.data_ptr(), T, d, F, r, us_ug.data_ptr(),
                  v_ug.data_ptr(), v_dn.data_ptr(), us_dn.data_ptr(), a.data_ptr(), b.data_ptr(), db.data_ptr(),
                  da.data_ptr(), dx.data_ptr(), *[t.data_ptr() for t in gr], ws.data_ptr(), nb, st)
        return [y, dx, *gr]

    ref, got, again = unfused(), fused(), fused()
    torch.cuda.synchronize()
    for name, a, b, c in zip(["y", "dx", "dus_ug", "dv_ug", "dv_dn", "dus_dn"], ref, got, again):
        assert_rel(_np(b), _np(a).astype(np.float64), BF16_RTOL, f"fused {name}")
        assert torch.equal(b, c), f"fused {name} not bitwise repeatable"


# ---------------------------------------------------------------- LM head + cross-entropy

@pytest.mark.parametrize("T,d,V", [(64, 64, 128), (8192, 512, 2048), (256, 64, 3000)])
def test_lm_head_ce_fwd_bwd(T, d, V):
    from oracle import losses as L

    H = _ops()
    rng = np.random.default_rng(T + V)
    h = bf16_round(rng.standard_normal((T, d)).astype(np.float32))
    w = (rng.standard_normal((V, d)) * 0.05).astype(np.float32)
    tg = rng.integers(0, V, T)
    gl = rng.standard_normal(T).astype(np.float32)
    ext = (rng.standard_normal((T, V)) * 1e-3).astype(np.float32)
    th = _bf(h).requires_grad_()
    tw = torch.from_numpy(w).to(DEV).requires_grad_()
    logits, loss = H.lm_head_ce(th, tw, torch.from_numpy(tg).to(DEV))
    torch.autograd.backward([loss, logits], [torch.from_numpy(gl).to(DEV), torch.from_numpy(ext).to(DEV)])
    wb = bf16_round(w).astype(np.float64)
    ref_logits = h.astype(np.float64) @ wb.T
    assert_rel(_np(logits), ref_logits, FP32_RTOL, "logits")
    rl, _, rg = L.cross_entropy(_np(logits), tg)
    assert_rel(_np(loss), rl, FP32_RTOL, "ce loss")
    dlog = gl[:, None] * rg + ext
    assert_rel(_np(th.grad), dlog @ wb, BF16_RTOL, "head dhidden")
    assert_rel(_np(tw.grad), dlog.T @ h, BF16_RTOL, "head dW")


@pytest.mark.parametrize("ids", [[3], [0, 6], [5, 2, 5]])
def test_ce_bwd_rows_matches_dense(ids):
    """rte_ce_bwd_rows (extra logit gradient for whole samples only) against rte_ce_bwd with the
    same rows scattered into a zero [T, V] gradient by index_add_ (a repeated sample adds its rows
    in list order): bitwise equal."""
    from rte_amd import _lib

    B, S, V = 8, 16, 256
    T = B * S
    print(f"ce_bwd_rows B={B} S={S} V={V} ids={ids}", flush=True)
    g = torch.Generator(device=DEV).manual_seed(7)
    logits = torch.randn(T, V, device=DEV, generator=g) * 3
    tg = torch.randint(0, V, (T,), device=DEV, generator=g)
    tg[5] = -1  # an ignored target
    lse = torch.logsumexp(logits, dim=1).contiguous()
    dloss = torch.randn(T, device=DEV, generator=g)
    ix = torch.tensor(ids, dtype=torch.int64, device=DEV)
    rows = torch.randn(len(ids), S, V, device=DEV, generator=g) * 1e-2
    dense = torch.zeros(B, S, V, device=DEV).index_add_(0, ix, rows).reshape(T, V).contiguous()
    p = _lib.ptr
    st = _lib.stream_ptr()
    want = torch.empty(T, V, dtype=torch.bfloat16, device=DEV)
    got = torch.empty_like(want)
    rows = rows.contiguous()
    _lib.call("rte_ce_bwd", p(logits), V, T, V, p(tg), p(lse), p(dloss), p(dense), p(want), st)
    _lib.call("rte_ce_bwd_rows", p(logits), V, T, V, p(tg), p(lse), p(dloss), p(rows), p(ix), len(ids), S, p(got), st)
    torch.cuda.synchronize()
    assert torch.equal(got, want)


def test_select_logit_rows_grads_match_index_select():
    """The audited-sample selection of lm_head_ce logits (gradient rows handed to the head's CE
    backward) against index_select of the same logits: same values, bitwise-equal gradients."""
    H = _ops()
    B, S, d, V = 4, 32, 64, 256
    print(f"select_logit_rows B={B} S={S} d={d} V={V}", flush=True)
    gen = torch.Generator(device=DEV).manual_seed(3)
    h0 = torch.randn(B, S, d, device=DEV, generator=gen).to(torch.bfloat16)
    w0 = torch.randn(V, d, device=DEV, generator=gen) * 0.05
    tg = torch.randint(0, V, (B, S), device=DEV, generator=gen)
    ix = torch.tensor([2, 0], dtype=torch.int64, device=DEV)
    c = torch.randn(2, S, V, device=DEV, generator=gen)
    res = []
    for select in (lambda x, i: x.index_select(0, i), H.select_logit_rows):
        h = h0.clone().requires_grad_()
        w = w0.clone().requires_grad_()
        logits, tok = H.lm_head_ce(h, w, tg)
        sel = select(logits, ix)
        (tok.sum() + (sel * c).sum()).backward()
        res.append((sel.detach(), h.grad, w.grad))
    for a, b in zip(res[0], res[1]):
        assert torch.equal(a, b)


# ---------------------------------------------------------------- shortlist head

def _sl_inputs(T, V, C, tc, H, R, L, seed, skew=False):
    from oracle import shortlist as SLO

    rng = np.random.default_rng(seed)
    members, _ = SLO.cluster_member_table(V, C)
    targets = rng.integers(0, V, T)
    top = np.stack([rng.permutation(C)[:tc] for _ in range(T)]).astype(np.int32)
    rnd = rng.integers(0, min(V, 8) if skew else V, (T, R))
    return SLO, members, targets, top, rnd


@pytest.mark.parametrize("T,V,C,tc,H,R,L", [
    (300, 97, 7, 2, 9, 11, 16),          # small, many duplicates across segments
    (257, 20, 3, 3, 40, 5, 15),          # V < 2L: the target filler wraps the vocabulary
    (4096, 8192, 64, 2, 32, 32, 128),    # the scaled shortlist configuration's widths
    (256, 65536, 64, 2, 32, 32, 128),    # largest vocabulary of the LDS bitmap
    (130, 512, 16, 0, 0, 0, 100),        # no members / negatives: fillers only
])
def test_shortlist_build_bit_exact(T, V, C, tc, H, R, L):
    H_ = _ops()
    SLO, members, targets, top, rnd = _sl_inputs(T, V, C, tc, H, R, L, seed=T + V, skew=(V == 97))
    print(f"shortlist_build T={T} V={V} C={C} tc={tc} H={H} R={R} L={L}", flush=True)
    sl, dup = H_.shortlist_build(torch.from_numpy(targets).to(DEV), torch.from_numpy(top).to(DEV),
                                 torch.from_numpy(members).to(DEV), H, torch.from_numpy(rnd).to(DEV), L, V)
    want, want_dup = SLO.build_shortlist(targets, top, members, H, rnd, L, V)
    np.testing.assert_array_equal(sl.cpu().numpy(), want)
    np.testing.assert_array_equal(dup.cpu().numpy(), want_dup)


@pytest.mark.parametrize("T,d,V,L", [(512, 256, 1000, 64), (333, 1024, 4096, 128), (200, 200, 300, 70),
                                     (64, 2048, 600, 40)])
def test_shortlist_ce_fwd_bwd(T, d, V, L):
    from oracle import shortlist as SLO

    H_ = _ops()
    rng = np.random.default_rng(T + d)
    h = bf16_round(rng.standard_normal((T, d)).astype(np.float32))
    w = bf16_round((rng.standard_normal((V, d)) * 0.05).astype(np.float32))
    sl = np.stack([rng.permutation(V)[:L] for _ in range(T)]).astype(np.int32)
    gl = rng.standard_normal(T).astype(np.float32)
    ext = (rng.standard_normal((T, L)) * 1e-2).astype(np.float32)
    print(f"shortlist_ce T={T} d={d} V={V} L={L}", flush=True)
    th = _bf(h).requires_grad_()
    tw = torch.from_numpy(w).to(DEV).requires_grad_()
    logits, loss = H_.shortlist_ce(th, tw, torch.from_numpy(sl).to(DEV))
    torch.autograd.backward([loss, logits], [torch.from_numpy(gl).to(DEV), torch.from_numpy(ext).to(DEV)])
    rl, rlse, rloss = SLO.shortlist_logits_ce(h, w, sl)
    assert_rel(_np(logits), rl, FP32_RTOL, "shortlist logits")
    assert_rel(_np(loss), rloss, FP32_RTOL, "shortlist loss")
    _, rdh, rdw = SLO.shortlist_logits_ce_bwd(h, w, sl, rl, rlse, gl, ext)
    assert_rel(_np(th.grad), rdh, BF16_RTOL, "shortlist dhidden")
    assert_rel(_np(tw.grad), rdw, FP32_RTOL, "shortlist dW")


def test_shortlist_bwd_skewed_rows_deterministic_and_accumulate():
    """Every token shares most shortlist ids (multi-chunk rows of the vocabulary reduction);
    dW is bitwise repeatable and dW_accumulate adds onto the existing gradient."""
    from oracle import shortlist as SLO
    from rte_amd import _lib

    H_ = _ops()
    rng = np.random.default_rng(77)
    T, d, V, L = 3000, 512, 700, 96
    h = bf16_round(rng.standard_normal((T, d)).astype(np.float32))
    w = bf16_round((rng.standard_normal((V, d)) * 0.05).astype(np.float32))
    base = rng.permutation(V)[:L]
    sl = np.stack([np.concatenate([base[:80], rng.permutation(np.setdiff1d(np.arange(V), base[:80]))[:16]])
                   for _ in range(T)]).astype(np.int32)
    gl = rng.standard_normal(T).astype(np.float32)
    hb, wb, slt = _bf(h), _bf(w), torch.from_numpy(sl).to(DEV)
    logits = torch.empty((T, L), dtype=torch.float32, device=DEV)
    lse = torch.empty((T,), dtype=torch.float32, device=DEV)
    loss = torch.empty((T,), dtype=torch.float32, device=DEV)
    _lib.call("rte_shortlist_fwd", _lib.ptr(hb), _lib.ptr(wb), d, V, _lib.ptr(slt), L, T, _lib.ptr(logits),
              _lib.ptr(lse), _lib.ptr(loss), _lib.stream_ptr())
    g = torch.from_numpy(gl).to(DEV)
    nb = _lib.load().rte_shortlist_bwd_workspace_bytes(T, L, V, d)
    ws = torch.empty((nb,), dtype=torch.uint8, device=DEV)
    outs = []
    for acc in (0, 0, 1):
        dw = torch.ones((V, d), dtype=torch.float32, device=DEV)
        dh = torch.empty((T, d), dtype=torch.bfloat16, device=DEV)
        _lib.call("rte_shortlist_bwd", _lib.ptr(g), None, _lib.ptr(hb), _lib.ptr(wb), d, V, _lib.ptr(slt), L, T,
                  _lib.ptr(logits), _lib.ptr(lse), _lib.ptr(dh), _lib.ptr(dw), acc, _lib.ptr(ws), nb,
                  _lib.stream_ptr())
        outs.append(dw.cpu().numpy())
    assert np.array_equal(outs[0], outs[1]), "dW not bitwise repeatable"
    _, _, rdw = SLO.shortlist_logits_ce_bwd(h, w, sl, _np(logits), _np(lse), gl)
    assert_rel(outs[0], rdw, FP32_RTOL, "skewed dW")
    assert_rel(outs[2], rdw + 1.0, FP32_RTOL, "accumulated dW")


def test_shortlist_head_matches_oracle():
    """ShortlistHead.loss end to end: router top-k, seeded random negatives, build, logits, CE."""
    from oracle import losses as LO
    from oracle import routing as RO
    from oracle import shortlist as SLO
    from rte_amd.config import OutputConfig
    from rte_amd.output import ShortlistHead

    torch.manual_seed(0)
    b, s, d, V = 4, 64, 256, 2048
    cfg = OutputConfig(mode="shortlist", num_clusters=64, shortlist_top_clusters=2, shortlist_max_tokens=128,
                       hard_negatives=32, random_negatives=32)
    head = ShortlistHead(d, V, cfg).to(DEV)
    hidden = torch.randn(b, s, d, device=DEV).to(torch.bfloat16)
    targets = torch.randint(0, V, (b, s), device=DEV)
    vw = (torch.randn(V, d, device=DEV) * 0.05).requires_grad_()
    res = head.loss(hidden, targets, vw, seed=11)
    cl = _np(res.cluster_logits).reshape(b * s, -1)
    top, _ = RO.route_topk(cl, 2)
    gen = torch.Generator(device=DEV)
    gen.manual_seed(11)
    rnd = torch.randint(0, V, (b, s, 32), device=DEV, generator=gen).cpu().numpy()
    tg = targets.cpu().numpy().reshape(-1)
    want, want_dup = SLO.build_shortlist(tg, top, head.cluster_members.cpu().numpy(), 32, rnd, 128, V)
    np.testing.assert_array_equal(res.shortlist.cpu().numpy().reshape(-1, 128), want)
    assert float(res.duplicate_count) == float(want_dup.sum())
    np.testing.assert_array_equal(res.target_positions.cpu().numpy(), 0)
    hb = _np(hidden).reshape(b * s, d)
    wb = bf16_round(_np(vw))
    rl, rlse, rloss = SLO.shortlist_logits_ce(hb, wb, want)
    assert_rel(_np(res.logits).reshape(b * s, -1), rl, FP32_RTOL, "head logits")
    assert_rel(_np(res.loss_per_sample), rloss.reshape(b, s).sum(-1), FP32_RTOL, "head loss per sample")
    res.loss_per_sample.sum().backward()
    _, _, rdw = SLO.shortlist_logits_ce_bwd(hb, wb, want, rl, rlse, np.ones(b * s))
    assert_rel(_np(vw.grad), rdw, FP32_RTOL, "head dW")
    _ = LO


# ---------------------------------------------------------------- segmented row reduction

@pytest.mark.parametrize("P,V,d,div,f32", [(5000, 300, 128, 1, True), (20000, 64, 512, 4, False),
                                         (70000, 2048, 64, 1, True), (3, 10, 8, 1, False), (0, 16, 32, 1, True),
                                         # one-launch path: few pairs over few keys
                                         (128, 16, 512, 1, True), (4096, 1024, 2048, 2, True),
                                         (4000, 7, 264, 1, False)])
def test_segment_reduce_rows(P, V, d, div, f32):
    H = _ops()
    rng = np.random.default_rng(P + V)
    keys = rng.integers(-3, V + 3, P)
    if P > 100:
        keys[: P // 3] = 7 % V                      # one key with many chunks
    rows = rng.standard_normal((max(P // div + 1, 1), d)).astype(np.float32)
    if not f32:
        rows = bf16_round(rows)
    w = rng.standard_normal(P).astype(np.float32)
    tk = torch.from_numpy(keys).to(DEV)
    tr = torch.from_numpy(rows).to(DEV)
    if not f32:
        tr = tr.to(torch.bfloat16)
    tw = torch.from_numpy(w).to(DEV)
    print(f"segment_reduce P={P} V={V} d={d} div={div} f32={f32}", flush=True)
    a = H.segment_reduce_rows(tk, V, tr, w=tw, row_div=div)
    b = H.segment_reduce_rows(tk, V, tr, w=tw, row_div=div)
    assert torch.equal(a, b), "segment reduce not bitwise repeatable"
    want = R.segment_reduce_rows(keys, V, rows, w, row_div=div)
    assert_rel(_np(a), want, FP32_RTOL, "segment reduce")
    acc = torch.ones_like(a)
    H.segment_reduce_rows(tk, V, tr, w=tw, row_div=div, out=acc, accumulate=True)
    assert_rel(_np(acc), want + 1.0, FP32_RTOL, "segment reduce accumulate")


def test_embedding_backward_deterministic():
    H = _ops()
    torch.manual_seed(0)
    W = torch.randn(300, 64, device=DEV, requires_grad=True)
    ids = torch.randint(0, 300, (8, 50), device=DEV)
    ids[:, :10] = 3
    g = torch.randn(8, 50, 64, device=DEV)
    out = H.embedding(W, ids)
    assert torch.equal(out, W.detach()[ids])
    out.backward(g)
    want = torch.zeros(300, 64, dtype=torch.float64).index_add_(0, ids.reshape(-1).cpu(), g.reshape(-1, 64).double().cpu())
    assert_rel(W.grad.double().cpu().numpy(), want.numpy(), FP32_RTOL, "embedding dW")


# ---------------------------------------------------------------- grouped linear

@pytest.mark.parametrize("N,K,Nout,G,skew", [(500, 96, 40, 7, False), (16384, 1536, 32, 48, False),
                                              (4096, 32, 512, 48, False), (16384, 1536, 32, 48, True),
                                              (8192, 32, 512, 48, True)])
def test_grouped_linear_fwd_bwd(N, K, Nout, G, skew):
    """Balanced and skewed groups (one group holding 90% of the rows: its weight-gradient
    reduction is cut into chunks that are added in a fixed order)."""
    from oracle import macro as MO

    H = _ops()
    rng = np.random.default_rng(N + K + skew)
    x = bf16_round(rng.standard_normal((N, K)).astype(np.float32))
    w = bf16_round((rng.standard_normal((G, K, Nout)) / np.sqrt(K)).astype(np.float32))
    keys = rng.integers(0, G, N)
    if skew:
        keys[rng.random(N) < 0.9] = 5
    keys[keys == 3] = 4                                   # group 3 empty
    dy = bf16_round(rng.standard_normal((N, Nout)).astype(np.float32))
    tx = _bf(x).float().requires_grad_()
    tw = torch.from_numpy(w).to(DEV).requires_grad_()
    pk = H.group_rows(torch.from_numpy(keys).to(DEV), G)
    print(f"grouped_linear N={N} K={K} Nout={Nout} G={G} skew={skew}", flush=True)
    y = H.grouped_linear(tx, tw, pk)
    y.backward(torch.from_numpy(dy).to(DEV))
    assert_rel(_np(y), MO.grouped_linear(x, w, keys), FP32_RTOL, "grouped linear y")
    rdx, rdw = MO.grouped_linear_bwd(dy, x, w, keys)
    assert_rel(_np(tx.grad), rdx, FP32_RTOL, "grouped linear dx")
    assert_rel(_np(tw.grad), rdw, FP32_RTOL, "grouped linear dW")
    assert not tw.grad[3].any(), "empty group must get a zero gradient"
    first = tw.grad.clone()
    tw.grad = None
    H.grouped_linear(tx, tw, pk).backward(torch.from_numpy(dy).to(DEV))
    assert torch.equal(first, tw.grad), "weight gradient not bitwise repeatable"


# ---------------------------------------------------------------- audit correction

@pytest.mark.parametrize("B,S,A,clip,grad_corrected", [
    (128, 64, 1, None, True),      # the cfg3 step: one audited sample, p = 1/128
    (32, 512, 4, 5.0, True),       # long rows, clipped and unclipped residuals
    (9, 7, 9, None, True),         # p = 1 on every sample
    (300, 33, 17, 1.0, False),     # not gradient-corrected: hot kept, no exact gradient
    (5, 3, 0, None, True),         # nothing audited
])
def test_audit_correct_matches_oracle(B, S, A, clip, grad_corrected):
    from oracle import audit as AU

    rng = np.random.default_rng(B * 7 + A)
    hot = rng.normal(size=(B, S)).astype(np.float32)
    idx = rng.permutation(B)[:A].astype(np.int64)
    exact = (hot[idx] + rng.normal(size=(A, S)) * 0.3).astype(np.float32)
    p = (np.ones(B) if A == B else rng.uniform(0.01, 1.0, B)).astype(np.float32)
    ops = _ops()
    th = torch.from_numpy(hot).to(DEV).requires_grad_(True)
    te = torch.from_numpy(exact).to(DEV).requires_grad_(grad_corrected)
    corr, ex, st = ops.audit_correct(th, te, torch.from_numpy(idx).to(DEV), torch.from_numpy(p).to(DEV), clip=clip,
                                     grad_corrected=grad_corrected)
    o_corr, o_ex, o_st = AU.correction(hot, exact, idx, p, clip, grad_corrected)
    np.testing.assert_allclose(corr.detach().cpu().numpy(), o_corr, rtol=1e-5, atol=1e-5 * np.abs(o_corr).max())
    if A:
        np.testing.assert_allclose(ex.cpu().numpy(), o_ex, rtol=1e-5, atol=1e-5 * np.abs(o_ex).max())
        scale = np.abs(o_st).max()
        np.testing.assert_allclose(st.cpu().numpy(), o_st, rtol=1e-5, atol=1e-5 * scale)
    g = rng.normal(size=B).astype(np.float32)
    corr.backward(torch.from_numpy(g).to(DEV))
    o_dh, o_de = AU.correction_bwd(g, hot, exact, idx, p, clip, grad_corrected)
    np.testing.assert_allclose(th.grad.cpu().numpy(), o_dh, rtol=1e-5, atol=1e-6 * np.abs(o_dh).max())
    if grad_corrected and A:
        np.testing.assert_allclose(te.grad.cpu().numpy(), o_de, rtol=1e-5, atol=1e-6 * np.abs(o_de).max())
    # repeated calls give identical bits (fixed reduction order)
    corr2, _, st2 = ops.audit_correct(th.detach(), te.detach(), torch.from_numpy(idx).to(DEV),
                                      torch.from_numpy(p).to(DEV), clip=clip, grad_corrected=grad_corrected)
    assert torch.equal(corr.detach(), corr2) and torch.equal(st, st2)


# ---------------------------------------------------------------- residual axpy + FiLM norm

def _torch_axpy_norm(a, b, c, keep, mask, w, gamma, beta, eps, S):
    """The recursive pass's glue in plain float64 torch (rte/layers.py:826-845)."""
    x = a if b is None else a + (1.0 if c is None else c) * b
    if mask is not None:
        act = mask.repeat_interleave(S)[:, None]
        x = torch.where(act, x, keep)
    if w is None:
        return x, None
    n = x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + eps) * w
    if gamma is not None:
        n = n * (1.0 + gamma)
    if beta is not None:
        n = n + beta
    return x, n


@pytest.mark.parametrize("B,S,d,norm,use_mask", [(2, 64, 512, True, False), (3, 17, 1024, True, True),
                                                 (4, 8, 64, False, True), (1, 64, 512, True, False)])
def test_axpy_norm_matches_float64(B, S, d, norm, use_mask):
    H = _ops()
    rng = np.random.default_rng(B * 100 + S + d)
    T = B * S
    f64 = torch.float64

    def t(x, grad=True):
        return torch.tensor(x, dtype=f64, requires_grad=grad)

    a_, b_, k_ = (rng.standard_normal((T, d)) for _ in range(3))
    c_ = np.array(rng.uniform(0.5, 1.5))
    w_, g_, be_ = rng.uniform(0.5, 1.5, d), rng.standard_normal(d) * 0.1, rng.standard_normal(d) * 0.1
    mask_ = rng.random(B) < 0.6 if use_mask else None
    # reference in float64
    ra, rb, rk, rc, rw, rg, rbe = t(a_), t(b_), t(k_), t(c_), t(w_), t(g_), t(be_)
    rm = None if mask_ is None else torch.tensor(mask_)
    rx, rn = _torch_axpy_norm(ra, rb, rc, rk if use_mask else None, rm, rw if norm else None, rg if norm else None,
                              rbe if norm else None, 1e-5, S)
    dx_ = rng.standard_normal((T, d))
    dn_ = bf16_round(rng.standard_normal((T, d)).astype(np.float32)).astype(np.float64)
    loss = (rx * t(dx_, False)).sum() + ((rn * t(dn_, False)).sum() if norm else 0.0)
    loss.backward()
    # device
    dev = lambda x: torch.tensor(x, dtype=torch.float32, device=DEV, requires_grad=True)  # noqa: E731
    da, db, dk, dc = dev(a_), dev(b_), dev(k_), dev(c_)
    dw, dg, dbe = dev(w_), dev(g_), dev(be_)
    dm = None if mask_ is None else torch.tensor(mask_, device=DEV)
    print(f"axpy_norm B={B} S={S} d={d} norm={norm} mask={use_mask}", flush=True)
    if norm:
        x, n = H.axpy_norm(da, db, dc, dw, dg, dbe, 1e-5, keep=dk if use_mask else None, mask=dm)
        assert_rel(_np(x), rx.detach().numpy(), FP32_RTOL, "x")
        assert_rel(_np(n), rn.detach().numpy(), 8e-3, "n (bf16)")
        ((x * torch.tensor(dx_, dtype=torch.float32, device=DEV)).sum()
         + (n.float() * torch.tensor(dn_, dtype=torch.float32, device=DEV)).sum()).backward()
        for got, ref, name in ((dw, rw, "dw"), (dg, rg, "dgamma"), (dbe, rbe, "dbeta")):
            assert_rel(_np(got.grad), ref.grad.numpy(), FP32_RTOL, name)
    else:
        x = H.axpy(da, db, dc, keep=dk if use_mask else None, mask=dm)
        assert_rel(_np(x), rx.detach().numpy(), FP32_RTOL, "x")
        (x * torch.tensor(dx_, dtype=torch.float32, device=DEV)).sum().backward()
    assert_rel(_np(da.grad), ra.grad.numpy(), FP32_RTOL, "da")
    assert_rel(_np(db.grad), rb.grad.numpy(), FP32_RTOL, "db")
    assert_rel(_np(dc.grad), rc.grad.numpy(), FP32_RTOL, "dc")
    if use_mask:
        assert_rel(_np(dk.grad), rk.grad.numpy(), FP32_RTOL, "dkeep")


# ---------------------------------------------------------------- audit distillation

@pytest.mark.parametrize("A,S,d,V", [(1, 64, 512, 2048), (3, 17, 96, 100), (2, 8, 64, 0), (1, 8, 64, 3000)])
def test_distill_matches_oracle(A, S, d, V):
    from oracle import distill as DI

    H = _ops()
    rng = np.random.default_rng(A * 1000 + S + d + V)
    h0 = rng.standard_normal((A, S, d))
    exact = h0 + rng.standard_normal((A, S, d)) * 0.7
    hot = exact + rng.standard_normal((A, S, d)) * 0.9
    hl = rng.standard_normal((A, S, V)) * 2 if V else None
    el = rng.standard_normal((A, S, V)) * 2 if V else None
    t = 2.0
    f = lambda x, g=False: None if x is None else torch.tensor(x, dtype=torch.float32, device=DEV,  # noqa: E731
                                                               requires_grad=g)
    hot32, exact32, h032 = (np.asarray(v, np.float32).astype(np.float64) for v in (hot, exact, h0))
    hl32 = None if hl is None else np.asarray(hl, np.float32).astype(np.float64)
    el32 = None if el is None else np.asarray(el, np.float32).astype(np.float64)
    th, tl = f(hot, True), f(hl, True)
    print(f"distill A={A} S={S} d={d} V={V}", flush=True)
    wts = [0.5, 2.0, 1.0, 0.05, 2.0, 1e-2]
    losses, mets = H.distill(th, f(exact), f(h0), tl, f(el), temperature=t, weights=wts)
    losses = torch.stack(losses)
    o_loss, o_met = DI.distill(hot32, exact32, h032, hl32, el32, t)
    np.testing.assert_allclose(_np(losses), [w * o_loss[k] for w, k in zip(wts, H.DISTILL_LOSSES)], rtol=1e-5,
                               atol=1e-7)
    want_m = [o_met.get(k, 0.0) for k in H.DISTILL_METRICS]
    np.testing.assert_allclose(_np(mets), want_m, rtol=1e-5, atol=1e-7)
    g = np.array([0.3, -1.1, 0.7, 1.9, 0.45, -0.8], np.float32)
    (losses * torch.from_numpy(g).to(DEV)).sum().backward()
    dh, dl = DI.distill_grad(hot32, exact32, h032, hl32, el32, t, g=g.astype(np.float64) * np.array(wts))
    assert_rel(_np(th.grad), dh, FP32_RTOL, "d hot")
    if V:
        assert_rel(_np(tl.grad), dl, FP32_RTOL, "d hot logits")


@pytest.mark.parametrize("shape,transposed", [((1536, 512), True), ((300, 77), True), ((64, 1), True),
                                              ((4096, 512), False), ((7, 13), False), ((1,), False)])
def test_cast_many_bit_exact(shape, transposed):
    """One-launch weight casts (contiguous and transposed views, ragged tile edges, an offset
    view) equal the per-tensor cast bit for bit, with NaN / inf / rounding-tie inputs."""
    H = _ops()
    from rte_amd import _lib

    lib = _lib.load()
    g = torch.Generator().manual_seed(sum(shape))
    n = int(np.prod(shape))
    x = torch.randn(n + 3, generator=g)
    x[:3] = torch.tensor([float("nan"), float("inf"), 1.0 + 2.0 ** -8])  # tie: rounds to even
    base = x.to(DEV)
    if transposed:
        src = base[3:].view(shape[1], shape[0]).t()  # element (r, c) at c * rows + r
    else:
        src = base[3:].view(shape)
    print(f"cast_many shape={shape} transposed={transposed}", flush=True)
    want = H.cast_bf16(src)
    rows, cols = (shape[0], shape[1]) if len(shape) == 2 else (1, shape[0])
    kind = 1 if transposed else 0
    out = torch.empty(shape, dtype=torch.bfloat16, device=DEV)
    other = torch.randn(5000, device=DEV)
    out2 = torch.empty(5000, dtype=torch.bfloat16, device=DEV)
    nb1 = lib.rte_cast_many_blocks(kind, rows, cols)
    nb2 = lib.rte_cast_many_blocks(0, 1, 5000)
    jobs = torch.tensor([[src.data_ptr(), out.data_ptr(), rows, cols, rows if transposed else 0, kind, 0, 0],
                         [other.data_ptr(), out2.data_ptr(), 1, 5000, 0, 0, nb1, 0]], dtype=torch.int64).to(DEV)
    blk = torch.tensor([0] * nb1 + [1] * nb2, dtype=torch.int32).to(DEV)
    H.call("rte_cast_many", jobs.data_ptr(), blk.data_ptr(), nb1 + nb2, torch.cuda.current_stream().cuda_stream)
    torch.cuda.synchronize()
    assert torch.equal(out.view(torch.int16), want.view(torch.int16))
    assert torch.equal(out2.view(torch.int16), H.cast_bf16(other).view(torch.int16))


@pytest.mark.parametrize("B,S,H,hd,scaled", [(2, 64, 8, 64, False), (3, 37, 4, 32, True), (1, 100, 2, 128, True)])
def test_qkv_rope_attention_fused_matches_two_nodes(B, S, H, hd, scaled):
    """QKV + RoPE + attention as one node (backward writes the packed, rotated-back dqkv in the
    attention kernels) equals qkv_rope followed by attention, outputs and gradients bit for bit."""
    H_ = _ops()
    d = H * hd
    g = torch.Generator().manual_seed(B * 100 + S)
    x0 = torch.randn(B, S, d, generator=g).to(DEV)
    w0 = (torch.randn(3 * d, d, generator=g) / d ** 0.5).to(DEV)
    pos = torch.arange(S, dtype=torch.float32)[:, None]
    inv = 10000.0 ** (-torch.arange(0, hd, 2, dtype=torch.float32) / hd)
    ang = (pos * inv).repeat_interleave(2, dim=1)
    cos, sin = ang.cos().to(DEV), ang.sin().to(DEV)
    hs = (torch.rand(B, H, generator=g) * (torch.rand(B, H, generator=g) < 0.7)).to(DEV) if scaled else None
    gy = torch.randn(B, H, S, hd, generator=g).to(DEV)
    print(f"qkv_rope_attention B={B} S={S} H={H} hd={hd} scaled={scaled}", flush=True)
    x1, w1 = x0.clone().requires_grad_(), w0.clone().requires_grad_()
    y1 = H_.qkv_rope_attention(x1, w1, cos, sin, H, hs)
    (y1.float() * gy).sum().backward()
    x2, w2 = x0.clone().requires_grad_(), w0.clone().requires_grad_()
    q, k, v = H_.qkv_rope(x2, w2, cos, sin, H)
    y2 = H_.attention(q, k, v, hs)
    (y2.float() * gy).sum().backward()
    assert torch.equal(y1, y2)
    assert torch.equal(x1.grad, x2.grad)
    assert torch.equal(w1.grad, w2.grad)


@pytest.mark.parametrize("transposed", [False, True])
def test_shared_weight_gradient_over_passes(transposed):
    """Three recursive passes through one attention weight pair: the shared weight gradient (one
    GEMM over every pass's rows, formed by the last backward call) equals the per-pass gradients
    summed by autograd (fp32 accumulation in another order: tolerance 1e-5 relative), inputs'
    gradients bit for bit, and a backward that reaches only some of the passes raises."""
    H_ = _ops()
    B, S, Hn, hd, T = 2, 64, 4, 32, 3  # the strided out-proj reads need power-of-two S
    d = Hn * hd
    g = torch.Generator().manual_seed(7 + transposed)
    x0 = torch.randn(B, S, d, generator=g).to(DEV)
    wq0 = (torch.randn(3 * d, d, generator=g) / d ** 0.5).to(DEV)
    wo0 = (torch.randn(d, d, generator=g) / d ** 0.5).to(DEV)
    pos = torch.arange(S, dtype=torch.float32)[:, None]
    inv = 10000.0 ** (-torch.arange(0, hd, 2, dtype=torch.float32) / hd)
    ang = (pos * inv).repeat_interleave(2, dim=1)
    cos, sin = ang.cos().to(DEV), ang.sin().to(DEV)
    gy = torch.randn(B, S, d, generator=g).to(DEV)
    print(f"shared weight gradient transposed={transposed}", flush=True)

    def run(shared, upto=T):
        x = x0.clone().requires_grad_()
        pq = (wq0.t().contiguous() if transposed else wq0.clone()).requires_grad_()
        po = (wo0.t().contiguous() if transposed else wo0.clone()).requires_grad_()
        wq, wo = (pq.t(), po.t()) if transposed else (pq, po)
        gq, go = (H_.SharedWGrad(), H_.SharedWGrad()) if shared else (None, None)
        h, hs = x, []
        for _ in range(T):
            y = H_.qkv_rope_attention(h, wq, cos, sin, Hn, None, wgrad=gq)
            h = H_.attn_out_proj(y, wo, h, wgrad=go)
            hs.append(h)
        (hs[upto - 1] * gy).sum().backward()
        return hs[-1], x.grad, pq.grad, po.grad

    h1, dx1, dq1, do1 = run(False)
    h2, dx2, dq2, do2 = run(True)
    assert torch.equal(h1, h2)
    assert torch.equal(dx1, dx2)
    assert dq2.is_contiguous() and do2.is_contiguous()
    assert_rel(_np(dq2), _np(dq1), FP32_RTOL, "dWqkv")
    assert_rel(_np(do2), _np(do1), FP32_RTOL, "dWo")
    h3, dx3, dq3, do3 = run(True)  # repeats bit for bit
    assert torch.equal(dq2, dq3) and torch.equal(do2, do3)
    with pytest.raises(RuntimeError, match="SharedWGrad"):
        run(True, upto=1)


def test_grouped_pool_transposed_and_accumulated_weight_grads():
    """Grouped pool SwiGLU used by three passes: weight gradients formed in the layout of
    transposed-view weights (rte_grouped_swiglu_bwd w_t = 1) and summed in place across the
    passes (beta = 1) equal the plain-layout per-pass gradients summed by autograd (fp32 sums in
    another order: 1e-5 relative); inputs' gradients bit for bit; repeat runs bit for bit; a
    backward that misses a pass raises."""
    H = _ops()
    rng = np.random.default_rng(5)
    T, d, C, n, k, P_ = 512, 256, 16, 32, 4, 3
    F = C * n
    xs0 = [torch.from_numpy(rng.standard_normal((T, d)).astype(np.float32)).to(DEV) for _ in range(P_)]
    ids = torch.from_numpy(np.stack([rng.permutation(C)[:k] for _ in range(T)]).astype(np.int32)).to(DEV)
    ids[::7, -1] = -1  # absent pairs
    w = torch.from_numpy(rng.random((T, k)).astype(np.float32)).to(DEV)
    wug0 = (torch.from_numpy(rng.standard_normal((d, 2 * F)).astype(np.float32)) * 0.05).to(DEV)  # [d, 2F]
    wd0 = (torch.from_numpy(rng.standard_normal((F, d)).astype(np.float32)) * 0.05).to(DEV)       # [F, d]
    dys = [torch.from_numpy(rng.standard_normal((T, d)).astype(np.float32)).to(DEV) for _ in range(P_)]
    print(f"grouped pool shared grads T={T} d={d} C={C} n={n} k={k}", flush=True)

    def run(view, acc_on, upto=P_):
        xs = [x.clone().requires_grad_() for x in xs0]
        pu, pd = wug0.clone().requires_grad_(), wd0.clone().requires_grad_()
        # view: transposed views of the parameters; else contiguous copies in the kernel layout
        wug_t, wd_t = (pu.t(), pd.t()) if view else (pu.t().contiguous(), pd.t().contiguous())
        acc = H.SharedGradAccum() if acc_on else None
        outs = [H.grouped_pool_swiglu(x, ids, w, wug_t, wd_t, n, acc=acc) for x in xs]
        sum((o * g).sum() for o, g in zip(outs[:upto], dys[:upto])).backward()
        return [x.grad for x in xs], pu.grad, pd.grad

    dx_ref, du_ref, dd_ref = run(False, False)
    for view, acc_on in ((True, False), (True, True), (False, True)):
        dx, du, dd = run(view, acc_on)
        for a, b in zip(dx, dx_ref):
            assert torch.equal(a, b)
        assert du.is_contiguous() and dd.is_contiguous()
        assert_rel(_np(du), _np(du_ref), FP32_RTOL, f"dwug view={view} acc={acc_on}")
        assert_rel(_np(dd), _np(dd_ref), FP32_RTOL, f"dwd view={view} acc={acc_on}")
    _, du1, dd1 = run(True, True)
    _, du2, dd2 = run(True, True)
    assert torch.equal(du1, du2) and torch.equal(dd1, dd2)
    with pytest.raises(RuntimeError, match="SharedGradAccum"):
        run(True, True, upto=2)
