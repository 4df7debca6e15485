"""Pins the CPU oracle before it is trusted as the checker of the HIP kernels.

The reference holds no literal golden vectors for this path (every reference
test is relational), so each oracle function is pinned by an independent route:
brute force, closed forms, finite differences, torch autograd on the CPU, and the
reference's own invariants (full pool == dense, rte/kernels test_kernels.py:82-148).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import attention as A
from oracle import cluster_pool as CP
from oracle import routing as R
from oracle import swiglu as SW


def _rng(seed=0):
    return np.random.default_rng(seed)


# ---------------------------------------------------------------- routing

def _brute_topk(row, k):
    keyed = sorted(range(len(row)), key=lambda i: (not np.isnan(row[i]), -row[i] if not np.isnan(row[i]) else 0, i))
    return keyed[:k]


@pytest.mark.parametrize("C,k", [(8, 1), (32, 4), (64, 8), (100, 16)])
def test_topk_matches_brute_force_with_ties(C, k):
    rng = _rng(C)
    lg = rng.integers(-3, 4, size=(50, C)).astype(np.float32)  # heavy ties
    lg[3, 5 % C] = np.nan
    ids, w = R.route_topk(lg, k)
    for t in range(lg.shape[0]):
        assert list(ids[t]) == _brute_topk(lg[t], k)
    finite = ~np.isnan(lg).any(-1)
    np.testing.assert_allclose(w[finite].sum(-1), 1.0, rtol=1e-6)


def test_topk_k1_is_argmax_routing():
    # route_to_static_centers uses argmax (rte/kernels/cluster_pool_ffn.py:140)
    lg = _rng(1).standard_normal((200, 32)).astype(np.float32)
    ids, w = R.route_topk(lg, 1)
    np.testing.assert_array_equal(ids[:, 0], lg.argmax(-1))
    np.testing.assert_array_equal(w, 1.0)


def test_topk_matches_torch_topk_on_distinct_values():
    lg = _rng(2).standard_normal((300, 64)).astype(np.float32)
    ids, w = R.route_topk(lg, 8)
    tv, ti = torch.topk(torch.from_numpy(lg), 8, dim=-1)
    np.testing.assert_array_equal(ids, ti.numpy())
    np.testing.assert_allclose(w, torch.softmax(tv, -1).numpy(), rtol=1e-6)


def test_pack_index_brute_force_and_roundtrip():
    rng = _rng(3)
    T, k, C = 97, 3, 11
    cl = np.stack([rng.permutation(C)[:k] for _ in range(T)]).astype(np.int32)
    pk = R.pack_index(cl, C, k)
    flat = cl.reshape(-1)
    for c in range(C):
        lo, hi = pk["offsets"][c], pk["offsets"][c + 1]
        expect = [p for p in range(T * k) if flat[p] == c]
        assert list(pk["pair_of_slot"][lo:hi]) == expect
        assert list(pk["tok_of_slot"][lo:hi]) == [p // k for p in expect]
    np.testing.assert_array_equal(pk["pair_of_slot"][pk["slot_of_pair"]], np.arange(T * k))
    assert pk["invalid"] == 0


def test_pack_index_invalid_ids_are_dropped():
    cl = np.array([0, 5, 1, -1, 1], dtype=np.int32)
    pk = R.pack_index(cl, 2, 1)
    assert pk["invalid"] == 2
    assert list(pk["offsets"]) == [0, 1, 3]
    assert list(pk["slot_of_pair"]) == [0, -1, 1, -1, 2]


def test_static_pack_gather_roundtrip():
    a = _rng(4).integers(0, 5, size=40)
    pack, flat, counts, mx = R.static_pack_gather(a, 5)
    assert counts.sum() == 40 and mx == counts.max()
    for t in range(40):
        c, r = divmod(int(flat[t]), mx)
        assert c == a[t] and pack[c, r] == t


def test_route_softmax_bwd_finite_difference():
    rng = _rng(5)
    T, C, k = 4, 7, 3
    lg = rng.standard_normal((T, C))
    ids, _ = R.route_topk(lg.astype(np.float32), k)
    dw = rng.standard_normal((T, k))

    def f(L):
        sel = np.take_along_axis(L, ids.astype(np.int64), -1)
        e = np.exp(sel - sel.max(-1, keepdims=True))
        return ((e / e.sum(-1, keepdims=True)) * dw).sum()

    _, w = R.route_topk(lg.astype(np.float32), k)
    g = R.route_softmax_bwd(ids, np.take_along_axis(
        np.exp(lg - lg.max(-1, keepdims=True)), ids.astype(np.int64), -1) / np.take_along_axis(
        np.exp(lg - lg.max(-1, keepdims=True)), ids.astype(np.int64), -1).sum(-1, keepdims=True), dw, C)
    eps = 1e-6
    num = np.zeros_like(lg)
    for i in range(T):
        for j in range(C):
            Lp = lg.copy(); Lp[i, j] += eps
            Lm = lg.copy(); Lm[i, j] -= eps
            num[i, j] = (f(Lp) - f(Lm)) / (2 * eps)
    np.testing.assert_allclose(g, num, atol=1e-7)
    assert w.shape == (T, k)


# ---------------------------------------------------------------- SwiGLU

@pytest.mark.parametrize("wd_rows", [False, True])
def test_dense_swiglu_matches_torch_autograd(wd_rows):
    rng = _rng(6)
    T, d, F = 9, 8, 12
    x = rng.standard_normal((T, d))
    wug = rng.standard_normal((2 * F, d)) * 0.3
    wd = rng.standard_normal((F, d) if wd_rows else (d, F)) * 0.3
    dy = rng.standard_normal((T, d))
    y, cache = SW.dense_swiglu_fwd(x, wug, wd, wd_rows=wd_rows)
    dx, dwug, dwd = SW.dense_swiglu_bwd(dy, x, wug, wd, cache, wd_rows=wd_rows)
    tx, tug, td = (torch.tensor(a, dtype=torch.float64, requires_grad=True) for a in (x, wug, wd))
    up, gate = (tx @ tug.t()).chunk(2, dim=-1)
    z = up * torch.nn.functional.silu(gate)
    ty = z @ (td if wd_rows else td.t())
    ty.backward(torch.tensor(dy))
    np.testing.assert_allclose(y, ty.detach().numpy(), rtol=1e-12)
    np.testing.assert_allclose(dx, tx.grad.numpy(), rtol=1e-10, atol=1e-12)
    np.testing.assert_allclose(dwug, tug.grad.numpy(), rtol=1e-10, atol=1e-12)
    np.testing.assert_allclose(dwd, td.grad.numpy(), rtol=1e-10, atol=1e-12)


def test_dense_swiglu_backward_finite_difference():
    rng = _rng(7)
    T, d, F = 3, 4, 5
    x = rng.standard_normal((T, d))
    wug = rng.standard_normal((2 * F, d))
    wd = rng.standard_normal((d, F))
    dy = rng.standard_normal((T, d))
    _, cache = SW.dense_swiglu_fwd(x, wug, wd)
    dx, _, _ = SW.dense_swiglu_bwd(dy, x, wug, wd, cache)
    eps = 1e-6
    for i in range(T):
        for j in range(d):
            xp = x.copy(); xp[i, j] += eps
            xm = x.copy(); xm[i, j] -= eps
            num = ((SW.dense_swiglu_fwd(xp, wug, wd)[0] - SW.dense_swiglu_fwd(xm, wug, wd)[0]) * dy).sum() / (2 * eps)
            assert abs(num - dx[i, j]) < 1e-6


# ---------------------------------------------------------------- cluster pool

def _pool_problem(seed, T=40, d=16, C=4, n=8, k=2):
    rng = _rng(seed)
    x = rng.standard_normal((T, d))
    wr = rng.standard_normal((C, d)) * 0.5
    wug = rng.standard_normal((2 * C * n, d)) * 0.2
    wd = rng.standard_normal((d, C * n)) * 0.2
    return x, wr, wug, wd


def test_all_clusters_uniform_weights_equal_dense_over_C():
    # the reference invariant "full pool == dense" (tests/test_kernels.py:82-107) in routed form
    x, wr, wug, wd = _pool_problem(8)
    C, k = 4, 4
    ids, w = R.route_topk(np.zeros((x.shape[0], C), np.float32), k)
    out = CP.routed_fwd(x, wug, wd, ids, w, C)
    dense, _ = SW.dense_swiglu_fwd(x, wug, wd)
    np.testing.assert_allclose(out * C, dense, rtol=1e-10, atol=1e-12)


def test_k1_matches_reference_loop_oracle():
    x, wr, wug, wd = _pool_problem(9, C=4, n=8)
    C, n, F = 4, 8, 32
    logits = (x @ wr.T).astype(np.float32)
    ids, w = R.route_topk(logits, 1)
    out = CP.routed_fwd(x, wug, wd, ids, w, C)
    cand = np.arange(F).reshape(C, n)
    wup_pool, wgate_pool, wdown_pool = CP.prepare_pools(wug[:F], wug[F:], wd.T, cand)
    ref = CP.cluster_pool_reference_loop(x, ids[:, 0], wup_pool, wgate_pool, wdown_pool)
    np.testing.assert_allclose(out, ref, rtol=1e-12, atol=1e-12)


def test_routed_backward_matches_torch_autograd():
    x, wr, wug, wd = _pool_problem(10, T=30, d=8, C=4, n=4, k=2)
    C, k = 4, 2
    T, d = x.shape
    F = wug.shape[0] // 2
    n = F // C
    dout = _rng(11).standard_normal((T, d))
    logits = x @ wr.T
    ids, _ = R.route_topk(logits.astype(np.float32), k)
    tx, twr, tug, twd = (torch.tensor(a, dtype=torch.float64, requires_grad=True) for a in (x, wr, wug, wd))
    tl = tx @ twr.t()
    tids = torch.from_numpy(ids.astype(np.int64))
    tw = torch.softmax(torch.gather(tl, 1, tids), -1)
    out = torch.zeros(T, d, dtype=torch.float64)
    for j in range(k):
        for t in range(T):
            c = int(ids[t, j])
            up = tug[c * n:(c + 1) * n] @ tx[t]
            gate = tug[F + c * n:F + (c + 1) * n] @ tx[t]
            out = out.index_add(0, torch.tensor([t]), (tw[t, j] * (up * torch.nn.functional.silu(gate)) @ twd[:, c * n:(c + 1) * n].t()).unsqueeze(0))
    out.backward(torch.tensor(dout))
    w = tw.detach().numpy()
    o = CP.routed_fwd(x, wug, wd, ids, w, C)
    np.testing.assert_allclose(o, out.detach().numpy(), rtol=1e-10, atol=1e-12)
    dx, dwr, dwug, dwd, _ = CP.routed_bwd(dout, x, wr, wug, wd, ids, w, C)
    np.testing.assert_allclose(dx, tx.grad.numpy(), rtol=1e-9, atol=1e-11)
    np.testing.assert_allclose(dwr, twr.grad.numpy(), rtol=1e-9, atol=1e-11)
    np.testing.assert_allclose(dwug, tug.grad.numpy(), rtol=1e-9, atol=1e-11)
    np.testing.assert_allclose(dwd, twd.grad.numpy(), rtol=1e-9, atol=1e-11)


# ---------------------------------------------------------------- attention pieces

def test_rmsnorm_matches_manual_and_backward():
    rng = _rng(12)
    x = rng.standard_normal((5, 16))
    w = rng.standard_normal(16)
    manual = x / np.sqrt((x**2).mean(-1, keepdims=True) + 1e-5) * w
    np.testing.assert_allclose(A.rmsnorm(x, w), manual, rtol=1e-12)
    tx = torch.tensor(x, requires_grad=True)
    tw = torch.tensor(w, requires_grad=True)
    y = tx * torch.rsqrt(tx.pow(2).mean(-1, keepdim=True) + 1e-5) * tw
    dy = rng.standard_normal((5, 16))
    y.backward(torch.tensor(dy))
    dx, dw = A.rmsnorm_bwd(dy, x, w)
    np.testing.assert_allclose(dx, tx.grad.numpy(), rtol=1e-10, atol=1e-12)
    np.testing.assert_allclose(dw, tw.grad.numpy(), rtol=1e-10, atol=1e-12)


def test_rope_is_complex_rotation():
    hd, S = 8, 7
    cos, sin = A.rope_tables(hd, S)
    x = _rng(13).standard_normal((2, 3, S, hd))
    y = A.rope_apply(x, cos, sin)
    inv = 1.0 / (10_000.0 ** (np.arange(0, hd, 2) / hd))
    theta = np.arange(S)[:, None] * inv[None, :]
    zc = (x[..., 0::2] + 1j * x[..., 1::2]) * np.exp(1j * theta)
    np.testing.assert_allclose(y[..., 0::2], zc.real, atol=1e-12)
    np.testing.assert_allclose(y[..., 1::2], zc.imag, atol=1e-12)
    np.testing.assert_allclose(y[:, :, 0], x[:, :, 0], atol=1e-15)  # position 0 is identity
    dy = _rng(14).standard_normal(y.shape)
    dx = A.rope_apply_bwd(dy, cos, sin)
    np.testing.assert_allclose((dy * y).sum(), (dx * x).sum(), rtol=1e-12)  # adjoint identity


def test_qkv_rope_backward_matches_torch():
    rng = _rng(15)
    B, S, H, hd = 2, 5, 2, 4
    d = H * hd
    cos, sin = A.rope_tables(hd, S)
    x = rng.standard_normal((B, S, d))
    w = rng.standard_normal((3 * d, d))
    q, k, v = A.qkv_rope(x, w, H, cos, sin)
    dq, dk, dv = (rng.standard_normal(q.shape) for _ in range(3))
    tx = torch.tensor(x, requires_grad=True)
    tw = torch.tensor(w, requires_grad=True)
    qkv = (tx @ tw.t()).view(B, S, 3, H, hd)
    tq, tk, tv = (t.transpose(1, 2) for t in qkv.unbind(2))
    tc, ts = torch.tensor(cos), torch.tensor(sin)

    def rot(t):
        return torch.stack((-t[..., 1::2], t[..., ::2]), -1).flatten(-2)

    tq = tq * tc + rot(tq) * ts
    tk = tk * tc + rot(tk) * ts
    np.testing.assert_allclose(q, tq.detach().numpy(), rtol=1e-12)
    (tq * torch.tensor(dq) + tk * torch.tensor(dk) + tv * torch.tensor(dv)).sum().backward()
    dx, dw = A.qkv_rope_bwd(dq, dk, dv, x, w, cos, sin)
    np.testing.assert_allclose(dx, tx.grad.numpy(), rtol=1e-10, atol=1e-12)
    np.testing.assert_allclose(dw, tw.grad.numpy(), rtol=1e-10, atol=1e-12)


# ---------------------------------------------------------------- SVD low-rank FFN

def _svd_problem(seed, T=6, d=8, F=12, r=3):
    rng = _rng(seed)
    x = rng.standard_normal((T, d))
    mats = dict(us_up=rng.standard_normal((d, r)), us_gate=rng.standard_normal((d, r)),
                v_up=rng.standard_normal((F, r)), v_gate=rng.standard_normal((F, r)),
                v_dn=rng.standard_normal((F, r)), us_dn=rng.standard_normal((d, r)))
    return x, {k: v * 0.3 for k, v in mats.items()}


def test_svd_ffn_equals_dense_on_reconstructed_weights():
    from oracle import svd_ffn as SV

    x, m = _svd_problem(20)
    y, _ = SV.svd_ffn_fwd(x, **m)
    w_up = (m["us_up"] @ m["v_up"].T).T       # nn.Linear layout [F, d]
    w_gate = (m["us_gate"] @ m["v_gate"].T).T
    wd_rows = m["v_dn"] @ m["us_dn"].T          # [F, d]
    dense, _ = SW.dense_swiglu_fwd(x, np.concatenate([w_up, w_gate]), wd_rows, wd_rows=True)
    np.testing.assert_allclose(y, dense, rtol=1e-10, atol=1e-12)


def test_svd_full_rank_factors_reproduce_dense_ffn():
    # reference invariant (tests/test_models_and_training.py:54-67): full rank == dense
    from oracle import svd_ffn as SV

    rng = _rng(21)
    d, F, T = 6, 10, 7
    w_up, w_gate = rng.standard_normal((F, d)), rng.standard_normal((F, d))
    wd = rng.standard_normal((d, F))
    x = rng.standard_normal((T, d))

    def factors(w_in_major):  # refresh_svd: A = U S, B = Vh (rte/layers.py:437-444)
        u, s, vh = np.linalg.svd(w_in_major, full_matrices=False)
        return u * s, vh.T

    us_up, v_up = factors(w_up.T)
    us_gate, v_gate = factors(w_gate.T)
    vd, usd = factors(wd.T)  # W_down = wd^T (F x d) = (U S) Vh: v_dn = U S, us_dn = Vh^T
    y, _ = SV.svd_ffn_fwd(x, us_up, us_gate, v_up, v_gate, vd, usd)
    dense, _ = SW.dense_swiglu_fwd(x, np.concatenate([w_up, w_gate]), wd)
    np.testing.assert_allclose(y, dense, rtol=1e-9, atol=1e-10)


def test_svd_ffn_backward_matches_torch():
    from oracle import svd_ffn as SV

    x, m = _svd_problem(22)
    dy = _rng(23).standard_normal((x.shape[0], x.shape[1]))
    y, c = SV.svd_ffn_fwd(x, **m)
    g = SV.svd_ffn_bwd(dy, x, **m, c=c)
    t = {k: torch.tensor(v, requires_grad=True) for k, v in m.items()}
    tx = torch.tensor(x, requires_grad=True)
    up = (tx @ t["us_up"]) @ t["v_up"].t()
    gate = (tx @ t["us_gate"]) @ t["v_gate"].t()
    ty = ((up * torch.nn.functional.silu(gate)) @ t["v_dn"]) @ t["us_dn"].t()
    ty.backward(torch.tensor(dy))
    np.testing.assert_allclose(g["dx"], tx.grad.numpy(), rtol=1e-9, atol=1e-11)
    for k in m:
        np.testing.assert_allclose(g["d" + k], t[k].grad.numpy(), rtol=1e-9, atol=1e-11, err_msg=k)


# ---------------------------------------------------------------- losses

def test_cross_entropy_matches_torch():
    from oracle import losses as L

    rng = _rng(24)
    lg = rng.standard_normal((9, 17)) * 3
    tg = rng.integers(0, 17, 9)
    loss, lse, grad = L.cross_entropy(lg, tg)
    tl = torch.tensor(lg, requires_grad=True)
    tt = torch.nn.functional.cross_entropy(tl, torch.tensor(tg), reduction="none")
    tt.sum().backward()
    np.testing.assert_allclose(loss, tt.detach().numpy(), rtol=1e-12)
    np.testing.assert_allclose(grad, tl.grad.numpy(), rtol=1e-10, atol=1e-12)
    np.testing.assert_allclose(lse, torch.logsumexp(tl, -1).detach().numpy(), rtol=1e-12)


def test_audit_correction_p1_is_exact():
    from oracle import losses as L

    hot, exact = np.array([1.0, 2.0]), np.array([1.5, 1.0])
    np.testing.assert_allclose(L.audit_corrected(hot, exact, np.ones(2)), exact)
    # unbiased: E[hot + mask (exact-hot)/p] = exact for inclusion probability p
    p = 0.25
    np.testing.assert_allclose(hot + p * (exact - hot) / p, exact)


def test_audit_oracle_p1_replaces_hot_with_exact():
    """tests/test_audit.py:12-37 of the reference: with p = 1 on every sample the corrected
    per-sample loss is the exact one."""
    from oracle import audit as AU

    rng = _rng(11)
    hot, exact = rng.normal(size=(4, 6)), rng.normal(size=(4, 6))
    corr, ex, st = AU.correction(hot, exact, np.arange(4), np.ones(4))
    np.testing.assert_allclose(corr, exact.sum(-1), rtol=1e-12)
    np.testing.assert_allclose(ex, exact.sum(-1), rtol=1e-12)
    np.testing.assert_allclose(st[3], exact.sum(-1).mean(), rtol=1e-12)
    # audit_mode other than gradient_corrected keeps the hot loss
    corr2, _, _ = AU.correction(hot, exact, np.arange(4), np.ones(4), grad_corrected=False)
    np.testing.assert_allclose(corr2, hot.sum(-1), rtol=1e-12)


def test_audit_oracle_fixed_count_is_unbiased_by_enumeration():
    """Every k-of-n subset drawn with equal probability (the fixed-count sampler,
    p = k / n): the mean of corrected over all subsets is the exact loss, row by row."""
    import itertools

    from oracle import audit as AU

    rng = _rng(12)
    n, k, S = 6, 2, 5
    hot, exact = rng.normal(size=(n, S)), rng.normal(size=(n, S))
    p = np.full(n, k / n)
    acc, cnt = np.zeros(n), 0
    for sub in itertools.combinations(range(n), k):
        corr, _, _ = AU.correction(hot, exact[list(sub)], np.array(sub), p)
        acc += corr
        cnt += 1
    np.testing.assert_allclose(acc / cnt, exact.sum(-1), rtol=1e-12)


def _torch_reference_correction(hot_tok, exact_tok, idx, p, clip, grad_corrected):
    """The reference's boolean-mask formulation (rte/audit.py:305-321) in float64 torch."""
    B = hot_tok.shape[0]
    mask = torch.zeros(B, dtype=torch.bool)
    mask[idx] = True
    order = torch.argsort(idx)  # the mask visits audited rows in ascending order
    hot = hot_tok.sum(-1)
    exact = exact_tok[order].sum(-1)
    corrected = hot.clone()
    hot_subset = hot[mask]
    residual = exact - hot_subset
    stats = [residual.mean(), residual.std(unbiased=False), residual.var(unbiased=False)]
    if clip is not None:
        residual = residual.clamp(-clip, clip)
    if not grad_corrected:
        residual = residual.detach()
    stats.append((hot_subset + residual.detach() / p[mask].clamp_min(1e-12)).mean())
    if grad_corrected:
        corrected[mask] = hot_subset + residual / p[mask].clamp_min(1e-12)
    return corrected, torch.stack(stats)


@pytest.mark.parametrize("clip,grad_corrected", [(None, True), (0.7, True), (0.7, False), (None, False)])
def test_audit_oracle_matches_reference_formulation_and_autograd(clip, grad_corrected):
    from oracle import audit as AU

    rng = _rng(13)
    B, S = 9, 7
    hot = rng.normal(size=(B, S))
    idx = np.array([7, 2, 4, 0])
    exact = hot[idx] + rng.normal(size=(4, S)) * 0.4
    p = rng.uniform(0.05, 1.0, B)
    corr, _, st = AU.correction(hot, exact, idx, p, clip, grad_corrected)
    th = torch.tensor(hot, requires_grad=True)
    te = torch.tensor(exact, requires_grad=True)
    tcorr, tst = _torch_reference_correction(th, te, torch.tensor(idx), torch.tensor(p), clip, grad_corrected)
    np.testing.assert_allclose(corr, tcorr.detach().numpy(), rtol=1e-12)
    np.testing.assert_allclose(st, tst.detach().numpy(), rtol=1e-12)
    g = rng.normal(size=B)
    tcorr.backward(torch.tensor(g))
    dh, de = AU.correction_bwd(g, hot, exact, idx, p, clip, grad_corrected)
    np.testing.assert_allclose(dh, th.grad.numpy(), rtol=1e-12)
    np.testing.assert_allclose(de, te.grad.numpy() if te.grad is not None else np.zeros_like(de), rtol=1e-12)
    if clip is not None:  # the case mixes clipped and unclipped rows
        r = exact.sum(-1) - hot.sum(-1)[idx]
        assert (np.abs(r) > clip).any() and (np.abs(r) <= clip).any()


def _distill_case(seed, A=2, S=5, d=12, V=9):
    rng = _rng(seed)
    h0 = rng.normal(size=(A, S, d))
    exact = h0 + rng.normal(size=(A, S, d)) * 0.7
    hot = exact + rng.normal(size=(A, S, d)) * 0.9       # mixes |z| < 1 and |z| > 1 smooth-L1 cases
    hl, el = rng.normal(size=(A, S, V)) * 2, rng.normal(size=(A, S, V)) * 2
    return hot, exact, h0, hl, el


def test_distill_oracle_matches_reference_formulation():
    """The oracle equals the reference's torch formulation (rte/macro.py:394-546, restated in
    rte_amd.macro) evaluated on float64 inputs on the CPU, losses and metrics.  The reference's
    _rms / _rmsnorm (rte/macro.py:12-18) reduce in float32 whatever the input dtype, hence
    the 1e-6 tolerance."""
    from oracle import distill as DI
    from rte_amd.macro import macro_alignment_metrics, macro_distill_loss

    hot, exact, h0, hl, el = _distill_case(21)
    t = 2.0
    o_loss, o_met = DI.distill(hot, exact, h0, hl, el, t)
    T = lambda x: torch.tensor(x, dtype=torch.float64)  # noqa: E731
    ref = macro_distill_loss(T(hot), T(exact), T(hl), T(el), h0=T(h0), lambda_kl=1.0, lambda_delta_dir=1.0,
                             lambda_delta_rms=1.0, lambda_endpoint_normed=1.0, lambda_endpoint_raw=1.0,
                             lambda_macro_rms_trust=1.0, temperature=t)
    for k in DI.LOSSES:
        np.testing.assert_allclose(o_loss[k], float(ref[k]), rtol=1e-6, err_msg=k)
    met = macro_alignment_metrics(T(hot), T(exact), h0=T(h0), hot_logits=T(hl), exact_logits=T(el))
    for k, v in o_met.items():
        np.testing.assert_allclose(v, float(met[k]), rtol=1e-6, err_msg=k)


def test_distill_oracle_gradient_matches_autograd():
    from oracle import distill as DI
    from rte_amd.macro import macro_distill_loss

    hot, exact, h0, hl, el = _distill_case(22)
    t = 2.0
    g = np.array([0.3, -1.1, 0.7, 1.9, 0.45, -0.8])
    th = torch.tensor(hot, requires_grad=True)
    tl = torch.tensor(hl, requires_grad=True)
    T = lambda x: torch.tensor(x, dtype=torch.float64)  # noqa: E731
    ref = macro_distill_loss(th, T(exact), tl, T(el), h0=T(h0), lambda_kl=g[5], lambda_delta_dir=g[0],
                             lambda_delta_rms=g[1], lambda_endpoint_normed=g[2], lambda_endpoint_raw=g[3],
                             lambda_macro_rms_trust=g[4], temperature=t)
    sum(ref.values()).backward()
    dh, dl = DI.distill_grad(hot, exact, h0, hl, el, t, g=g)
    # float32 reductions inside the reference's _rms / _rmsnorm: relative Frobenius 1e-6
    assert np.linalg.norm(dh - th.grad.numpy()) <= 1e-6 * np.linalg.norm(dh)
    assert np.linalg.norm(dl - tl.grad.numpy()) <= 1e-10 * np.linalg.norm(dl)


# ---------------------------------------------------------------- shortlist

def _brute_first_distinct(row, L):
    seen, out = set(), []
    for v in row:
        if v not in seen:
            seen.add(v)
            out.append(v)
    return out[:L], len(row) - len(seen)


def _shortlist_case(seed, T=24, V=97, C=7, tc=2, H=9, R=11, L=16):
    from oracle import shortlist as SL

    rng = _rng(seed)
    members, _ = SL.cluster_member_table(V, C)
    targets = rng.integers(0, V, T)
    top = np.stack([rng.permutation(C)[:tc] for _ in range(T)])
    rnd = rng.integers(0, V, (T, R))
    return SL, members, targets, top, rnd, H, L, V


def test_shortlist_member_table_partitions_vocab():
    from oracle import shortlist as SL

    members, counts = SL.cluster_member_table(23, 5)
    assert members.shape == (5, 5) and counts.tolist() == [5, 5, 5, 4, 4]
    got = sorted(int(members[c, i]) for c in range(5) for i in range(counts[c]))
    assert got == list(range(23))
    assert all(int(members[c, i]) % 5 == c for c in range(5) for i in range(counts[c]))
    assert members[3, 4] == 0 and members[4, 4] == 0          # padding id of short clusters


@pytest.mark.parametrize("seed", [0, 1, 2])
def test_shortlist_dedupe_matches_brute_force(seed):
    SL, members, targets, top, rnd, H, L, V = _shortlist_case(seed)
    cand = SL.build_candidates(targets, top, members, H, rnd, L, V)
    assert cand.shape[1] == 1 + top.shape[1] * members.shape[1] + H + rnd.shape[1] + 3 * L
    sl, dup = SL.dedupe_preserve_first(cand, L)
    for t in range(cand.shape[0]):
        want, want_dup = _brute_first_distinct(cand[t].tolist(), L)
        assert sl[t].tolist() == want
        assert dup[t] == want_dup


def test_shortlist_dedupe_matches_reference_formulation():
    """The reference keeps first occurrences with scatter_reduce(amin) over [T, V] first
    positions and topk(largest=False, sorted=True) (rte/output.py:52-69); run that
    formulation with torch on the CPU."""
    SL, members, targets, top, rnd, H, L, V = _shortlist_case(5, T=40, V=61, C=4, tc=3, H=70, R=30, L=20)
    cand = SL.build_candidates(targets, top, members, H, rnd, L, V)
    width = cand.shape[1]
    flat = torch.tensor(cand)
    pos = torch.arange(width, dtype=torch.float32).view(1, -1).expand_as(flat)
    first = torch.full((flat.shape[0], V), float(width + L))
    first.scatter_reduce_(1, flat, pos, reduce="amin", include_self=True)
    dup_ref = (width - (first < width).sum(-1)).numpy()
    _, ref = first.topk(k=L, dim=-1, largest=False, sorted=True)
    sl, dup = SL.dedupe_preserve_first(cand, L)
    np.testing.assert_array_equal(sl, ref.numpy())
    np.testing.assert_array_equal(dup, dup_ref)


def test_shortlist_reference_invariants():
    """Target at position 0 and L distinct ids per token (tests/test_models_and_training.py:465-477),
    also when V < 2L so that the target filler wraps around the vocabulary."""
    for V, L in ((97, 16), (20, 15), (15, 15)):
        SL, members, targets, top, rnd, H, _, _ = _shortlist_case(9, V=V, L=L, C=3)
        sl, dup = SL.build_shortlist(targets, top, members, H, rnd, L, V)
        np.testing.assert_array_equal(sl[:, 0], targets)
        assert all(len(set(row.tolist())) == L for row in sl)
        assert (dup >= 0).all()


def test_shortlist_logits_ce_and_backward_match_torch_autograd():
    from oracle import shortlist as SL

    rng = _rng(31)
    T, V, d, L = 12, 40, 8, 6
    h = rng.standard_normal((T, d))
    w = rng.standard_normal((V, d))
    sl = np.stack([rng.permutation(V)[:L] for _ in range(T)])
    sl[:3, 1] = sl[3:6, 2]                                   # shared rows across tokens
    dloss = rng.standard_normal(T)
    dlog = rng.standard_normal((T, L))
    logits, lse, loss = SL.shortlist_logits_ce(h, w, sl)
    g, dh, dw = SL.shortlist_logits_ce_bwd(h, w, sl, logits, lse, dloss, dlog)
    th = torch.tensor(h, requires_grad=True)
    tw = torch.tensor(w, requires_grad=True)
    tl = (th.unsqueeze(-2) * tw[torch.tensor(sl)]).sum(-1)  # rte/kernels/reference.py:142-143
    tloss = torch.nn.functional.cross_entropy(tl, torch.zeros(T, dtype=torch.long), reduction="none")
    (tloss * torch.tensor(dloss)).sum().add((tl * torch.tensor(dlog)).sum()).backward()
    np.testing.assert_allclose(logits, tl.detach().numpy(), rtol=1e-12)
    np.testing.assert_allclose(loss, tloss.detach().numpy(), rtol=1e-12)
    np.testing.assert_allclose(dh, th.grad.numpy(), rtol=1e-10, atol=1e-12)
    np.testing.assert_allclose(dw, tw.grad.numpy(), rtol=1e-10, atol=1e-12)


# ---------------------------------------------------------------- banked recursive core

def _banked_case(seed, A=1, FB=1, H=4, HG=4, AHG=2, G=8, AG=2, d=32, F=64, R=7, S=12):
    from oracle import banked as BK

    rng = _rng(seed)
    recipes = BK.recipe_templates(A, FB, HG, G, AHG, AG, R)
    wqkv = rng.standard_normal((A, d, 3 * d)) / np.sqrt(d)
    wo = rng.standard_normal((A, d, d)) / np.sqrt(d)
    wug = rng.standard_normal((FB, d, 2 * F)) / np.sqrt(d)
    wd = rng.standard_normal((FB, F, d)) / np.sqrt(F)
    x = rng.standard_normal((S, d))
    return BK, recipes, wqkv, wo, wug, wd, x


def test_banked_recipe_templates_match_recipe_bank():
    from oracle import banked as BK
    from rte_amd.config import ModelConfig
    from rte_amd.recipes import RecipeBank

    cfg = ModelConfig(topology="recursive", vocab_size=64, d_model=32, n_heads=4, d_ff=64, n_dense_layers=2,
                      n_prelude=1, n_coda=1, t_max=2, depth_choices=[1, 2], attn_banks=2, ffn_banks=3, head_groups=4,
                      ffn_groups=8, active_head_groups=2, active_ffn_groups=2, recipe_count=11)
    want = BK.recipe_templates(2, 3, 4, 8, 2, 2, 11)
    got = [dict(attention_banks=r.attention_banks, ffn_banks=r.ffn_banks, head_groups=r.head_groups,
                ffn_groups=r.ffn_groups) for r in RecipeBank(cfg).recipes]
    assert got == want


def test_banked_swiglu_dense_recipe_equals_dense_ffn():
    """Recipe 0 (every slab) of a single bank is the dense SwiGLU of that bank."""
    BK, recipes, _, _, wug, wd, x = _banked_case(40)
    got = BK.banked_swiglu(x, recipes[0], wug, wd, 8)
    want, _ = SW.dense_swiglu_fwd(x, wug[0].T, wd[0], wd_rows=True)
    np.testing.assert_allclose(got, want, rtol=1e-12, atol=1e-12)


def test_banked_swiglu_slab_partition_sums_to_dense():
    """The recipes of one bank whose slab groups partition the FFN add up to recipe 0."""
    BK, recipes, _, _, wug, wd, x = _banked_case(41)
    parts = [r for r in recipes[1:] if r["ffn_banks"] == (0,)][:4]
    assert sorted(g for r in parts for g in r["ffn_groups"]) == list(range(8))
    total = sum(BK.banked_swiglu(x, r, wug, wd, 8) for r in parts)
    np.testing.assert_allclose(total, BK.banked_swiglu(x, recipes[0], wug, wd, 8), rtol=1e-11, atol=1e-12)


def test_banked_swiglu_bank_mean():
    """A recipe over two banks is the mean of the single-bank outputs."""
    BK, _, _, _, wug, wd, x = _banked_case(42, FB=2)
    r2 = dict(attention_banks=(0,), ffn_banks=(0, 1), head_groups=(0,), ffn_groups=(1, 5))
    r0 = dict(r2, ffn_banks=(0,))
    r1 = dict(r2, ffn_banks=(1,))
    np.testing.assert_allclose(BK.banked_swiglu(x, r2, wug, wd, 8),
                               0.5 * (BK.banked_swiglu(x, r0, wug, wd, 8) + BK.banked_swiglu(x, r1, wug, wd, 8)),
                               rtol=1e-12, atol=1e-12)


def test_banked_attention_dense_recipe_matches_torch_sdpa():
    """Recipe 0 of one bank is dense causal attention: torch SDPA on the CPU as the check."""
    BK, recipes, wqkv, wo, _, _, x = _banked_case(43)
    S, d = x.shape
    H = 4
    hd = d // H
    cos, sin = A.rope_tables(hd, S)
    got = BK.banked_attention(x, recipes[0], wqkv, wo, H, 4, cos, sin)
    qkv = torch.tensor(x) @ torch.tensor(wqkv[0])
    q, k, v = (qkv[:, i * d:(i + 1) * d].view(S, H, hd).transpose(0, 1) for i in range(3))
    tc, ts = torch.tensor(cos), torch.tensor(sin)

    def rope(t):
        rot = torch.stack([-t[..., 1::2], t[..., 0::2]], dim=-1).flatten(-2)
        return t * tc + rot * ts

    y = torch.nn.functional.scaled_dot_product_attention(rope(q), rope(k), v, is_causal=True)
    want = y.transpose(0, 1).reshape(S, d) @ torch.tensor(wo[0])
    np.testing.assert_allclose(got, want.numpy(), rtol=1e-10, atol=1e-12)


def test_banked_attention_head_partition_sums_to_dense():
    BK, recipes, wqkv, wo, _, _, x = _banked_case(44)
    cos, sin = A.rope_tables(8, x.shape[0])
    parts = [r for r in recipes[1:] if r["attention_banks"] == (0,)][:2]
    assert sorted(g for r in parts for g in r["head_groups"]) == [0, 1, 2, 3]
    total = sum(BK.banked_attention(x, r, wqkv, wo, 4, 4, cos, sin) for r in parts)
    np.testing.assert_allclose(total, BK.banked_attention(x, recipes[0], wqkv, wo, 4, 4, cos, sin), rtol=1e-11,
                               atol=1e-12)


def test_banked_core_inactive_samples_keep_state():
    BK, recipes, wqkv, wo, wug, wd, _ = _banked_case(45)
    rng = _rng(45)
    d, t = 32, 2
    p = dict(norm1=np.ones(d), norm2=np.ones(d), wqkv=wqkv, wo=wo, wug=wug, wd=wd,
             pass_gamma1=rng.standard_normal((t, d)) * 0.1, pass_beta1=rng.standard_normal((t, d)) * 0.1,
             pass_gamma2=rng.standard_normal((t, d)) * 0.1, pass_beta2=rng.standard_normal((t, d)) * 0.1,
             pass_attn_scale=np.ones(t), pass_mlp_scale=np.ones(t), alpha_inj=None)
    h = rng.standard_normal((3, 12, d))
    cos, sin = A.rope_tables(8, 12)
    kw = dict(n_heads=4, head_groups=4, ffn_groups=8, cos=cos, sin=sin)
    out = BK.core_forward_step(h, h, [0, 3, 5], [True, False, True], recipes, p, 1, **kw)
    np.testing.assert_array_equal(out[1], h[1])
    np.testing.assert_allclose(out[2], BK.core_step(h[2], h[2], recipes[5], p, 1, **kw), rtol=1e-12)
    zero = dict(p, pass_attn_scale=np.zeros(t), pass_mlp_scale=np.zeros(t))
    np.testing.assert_allclose(BK.core_step(h[0], h[0], recipes[0], zero, 0, **kw), h[0], rtol=0, atol=0)


# ---------------------------------------------------------------- segmented row reduction

def test_segment_reduce_matches_index_add_and_loop():
    rng = _rng(60)
    P, V, d, div = 300, 17, 6, 3
    keys = rng.integers(-2, V + 2, P)
    rows = rng.standard_normal((P // div + 1, d))
    w = rng.standard_normal(P)
    got = R.segment_reduce_rows(keys, V, rows, w, row_div=div)
    want = np.zeros((V, d))
    for p in range(P):
        if 0 <= keys[p] < V:
            want[keys[p]] += w[p] * rows[p // div]
    np.testing.assert_allclose(got, want, rtol=1e-12, atol=1e-12)
    ok = (keys >= 0) & (keys < V)
    t = torch.zeros(V, d, dtype=torch.float64).index_add_(
        0, torch.tensor(keys[ok]), torch.tensor(w[ok, None] * rows[np.arange(P)[ok] // div]))
    np.testing.assert_allclose(got, t.numpy(), rtol=1e-12, atol=1e-12)


# ---------------------------------------------------------------- macro operators

def _macro_case(seed, B=6, S=5, d=8, m=3, R=4, K=3):
    rng = _rng(seed)
    p = dict(d_gain=rng.standard_normal((R, K, d)) * 0.1, bias=rng.standard_normal((R, K, d)) * 0.1,
             update_scale=rng.uniform(0.5, 1.5, (R, K, d)), v=rng.standard_normal((R, K, 3 * d, m)) / 5,
             u=rng.standard_normal((R, K, m, d)) / 3)
    h = rng.standard_normal((B, S, d))
    h0 = rng.standard_normal((B, S, d))
    return p, h, h0, rng.integers(0, R, B), rng.integers(0, K, B)


def test_macro_grouped_linear_matches_loop_and_backward():
    from oracle import macro as MO

    rng = _rng(70)
    x, w, keys = rng.standard_normal((30, 7)), rng.standard_normal((5, 7, 4)), rng.integers(0, 5, 30)
    y = MO.grouped_linear(x, w, keys)
    for t in range(30):
        np.testing.assert_allclose(y[t], x[t] @ w[keys[t]], rtol=1e-12)
    dy = rng.standard_normal((30, 4))
    dx, dw = MO.grouped_linear_bwd(dy, x, w, keys)
    tx, tw = torch.tensor(x, requires_grad=True), torch.tensor(w, requires_grad=True)
    (torch.bmm(tx.unsqueeze(1), tw[torch.tensor(keys)]).squeeze(1) * torch.tensor(dy)).sum().backward()
    np.testing.assert_allclose(dx, tx.grad.numpy(), rtol=1e-12)
    np.testing.assert_allclose(dw, tw.grad.numpy(), rtol=1e-12, atol=1e-14)


def test_macro_closed_form_without_low_rank_path():
    """u = 0 and gain = 0 leave Phi(h) = h + c * scale * tanh(bias)."""
    from oracle import macro as MO

    p, h, h0, r, k = _macro_case(71)
    p["u"][:] = 0.0
    p["d_gain"][:] = 0.0
    out = MO.bounded_apply(h, h0, r, k, p, 0.05)
    want = h + 0.05 * p["update_scale"][r, k][:, None, :] * np.tanh(p["bias"][r, k])[:, None, :]
    np.testing.assert_allclose(out, want, rtol=1e-12)


def test_macro_bounded_and_per_key():
    """|Phi(h) - h| <= c * |scale| (tanh bound); a sample's output depends only on its own
    (recipe, stride) parameters and on its own rows (equivariant under sample permutation)."""
    from oracle import macro as MO

    p, h, h0, r, k = _macro_case(72)
    out = MO.bounded_apply(h, h0, r, k, p, 0.05)
    assert (np.abs(out - h) <= 0.05 * p["update_scale"][r, k][:, None, :] + 1e-12).all()
    other = {kk: v.copy() for kk, v in p.items()}
    unused = [(a, b) for a in range(4) for b in range(3) if not ((r == a) & (k == b)).any()]
    for a, b in unused:
        for kk in other:
            other[kk][a, b] = 7.0
    np.testing.assert_allclose(MO.bounded_apply(h, h0, r, k, other, 0.05), out, rtol=1e-12)
    perm = _rng(73).permutation(h.shape[0])
    np.testing.assert_allclose(MO.bounded_apply(h[perm], h0[perm], r[perm], k[perm], p, 0.05), out[perm], rtol=1e-12)


# ---------------------------------------------------------------- pins by closed form / hand values

def _distill_rows(A=2, S=3, d=8, seed=90):
    rng = _rng(seed)
    return rng.normal(size=(A, S, d)), rng.normal(size=(A, S, d))


def test_distill_closed_form_identical_states():
    """hot == exact (and equal logits): every loss is 0, cosines 1, norm ratios 1, mse 0."""
    from oracle import distill as DI

    exact, h0 = _distill_rows()
    lg = _rng(91).normal(size=(2, 3, 5))
    loss, met = DI.distill(exact.copy(), exact, h0, lg.copy(), lg)
    for k in DI.LOSSES:
        assert abs(loss[k]) < 1e-12, k
    assert abs(met["hidden_cosine_exact_macro"] - 1.0) < 1e-12
    assert abs(met["delta_cosine_exact_macro"] - 1.0) < 1e-12
    assert met["hidden_mse_exact_macro"] == 0.0
    assert abs(met["macro_exact_norm_ratio"] - 1.0) < 1e-12
    assert abs(met["delta_rms_ratio"] - 1.0) < 1e-12
    assert abs(met["logit_kl_exact_macro"]) < 1e-12


def test_distill_closed_form_doubled_delta():
    """hot - h0 = 2 (exact - h0): delta_dir = 0, delta_rms = (ln 2)^2, delta_rms ratio 2."""
    from oracle import distill as DI

    exact, h0 = _distill_rows(seed=92)
    hot = h0 + 2.0 * (exact - h0)
    loss, met = DI.distill(hot, exact, h0)
    assert abs(loss["delta_dir"]) < 1e-12
    assert abs(loss["delta_rms"] - np.log(2.0) ** 2) < 1e-12
    assert abs(met["delta_rms_ratio"] - 2.0) < 1e-12
    assert abs(met["delta_cosine_exact_macro"] - 1.0) < 1e-12
    # hot - h0 = -(exact - h0): opposite direction, equal size
    loss, _ = DI.distill(h0 - (exact - h0), exact, h0)
    assert abs(loss["delta_dir"] - 2.0) < 1e-12 and abs(loss["delta_rms"]) < 1e-12


def test_distill_closed_form_scaled_endpoint():
    """hot = 3 exact: rms_trust = (ln 3)^2, norm ratio 3, hidden cosine 1, and the
    rms-normalised endpoint loss vanishes up to the norm's eps."""
    from oracle import distill as DI

    exact, h0 = _distill_rows(seed=93)
    loss, met = DI.distill(3.0 * exact, exact, h0)
    assert abs(loss["rms_trust"] - np.log(3.0) ** 2) < 1e-12
    assert abs(met["macro_exact_norm_ratio"] - 3.0) < 1e-12
    assert abs(met["hidden_cosine_exact_macro"] - 1.0) < 1e-12
    assert loss["endpoint_normed"] < 1e-9


@pytest.mark.parametrize("offset,want", [(0.5, 0.125), (-0.5, 0.125), (2.0, 1.5), (-2.0, 1.5), (1.0, 0.5)])
def test_distill_smooth_l1_constant_offset(offset, want):
    """smooth_l1 (beta 1) of a constant offset o: o^2 / 2 for |o| < 1, |o| - 1/2 otherwise."""
    from oracle import distill as DI

    exact, h0 = _distill_rows(seed=94)
    loss, met = DI.distill(exact + offset, exact, h0)
    assert abs(loss["endpoint_raw"] - want) < 1e-12
    assert abs(met["hidden_mse_exact_macro"] - offset * offset) < 1e-12


@pytest.mark.parametrize("t", [1.0, 2.0])
def test_distill_two_class_kl_closed_form(t):
    """Two classes with logits (0, a) exact and (0, b) hot: per row
    KL = p ln(p / q) + (1 - p) ln((1 - p) / (1 - q)), p = sigmoid(a / t), q = sigmoid(b / t);
    batchmean divides the sum over rows by the batch size A, times t^2."""
    from oracle import distill as DI

    A, S = 2, 3
    a = np.array([[0.3, -1.2, 2.0], [0.0, 1.5, -0.4]])
    b = np.array([[1.1, 0.2, -0.7], [0.9, -2.0, 0.4]])
    el = np.stack([np.zeros_like(a), a], -1)
    hl = np.stack([np.zeros_like(b), b], -1)
    exact, h0 = _distill_rows(A, S, 4, seed=95)
    loss, met = DI.distill(exact, exact, h0, hl, el, t)
    sig = lambda x: 1.0 / (1.0 + np.exp(-x))  # noqa: E731

    def kl_rows(tt):
        p, q = sig(a / tt), sig(b / tt)
        return p * np.log(p / q) + (1 - p) * np.log((1 - p) / (1 - q))

    assert abs(loss["kl"] - kl_rows(t).sum() / A * t * t) < 1e-12
    assert abs(met["logit_kl_exact_macro"] - kl_rows(1.0).mean()) < 1e-12


def test_macro_low_rank_path_hand_values():
    """One-hot v columns pick single coordinates of each block of
    z = [rmsnorm(h) | mean_s rmsnorm(h) | h0] and one-hot u rows route them to distinct output
    coordinates, so with gain = bias = 0 and scale = 1, atanh((Phi(h) - h) / c) exposes
    silu(rmsnorm(h)[s, 1]), silu(mean_s rmsnorm(h)[0]) and silu(h0[s, 2]).  The expected
    numbers are worked by hand (rows chosen with round rms values), so pooling h instead of
    rmsnorm(h), swapping blocks or transposing v / u fails (rte/macro.py:201-236)."""
    from oracle import macro as MO

    d, c = 4, 0.5
    h = np.array([[[3, 4, 0, 0], [1, 1, 1, 1], [2, 0, 0, 0]],           # rms 2.5, 1, 1
                  [[0, 0, 0, -2], [1, -1, 1, -1], [0, 6, 0, 8]]], float)  # rms 1, 1, 5
    h0 = np.array([[[0.1, 0.2, 0.7, 0.4], [0.5, 0.6, -0.3, 0.8], [0.9, 1.0, 1.1, 1.2]],
                   [[-0.1, -0.2, 0.25, -0.4], [0.3, 0.1, -1.5, 0.2], [0.0, 0.0, 2.0, 0.0]]])
    v = np.zeros((1, 1, 3 * d, 3))
    v[0, 0, 1, 0] = 1.0          # rmsnorm(h)[s, 1]
    v[0, 0, d + 0, 1] = 1.0      # mean_s rmsnorm(h)[0]
    v[0, 0, 2 * d + 2, 2] = 1.0  # h0[s, 2]
    u = np.zeros((1, 1, 3, d))
    u[0, 0, 0, 3] = u[0, 0, 1, 0] = u[0, 0, 2, 1] = 1.0
    p = dict(d_gain=np.zeros((1, 1, d)), bias=np.zeros((1, 1, d)), update_scale=np.ones((1, 1, d)), v=v, u=u)
    zero = np.zeros(2, int)
    out = MO.bounded_apply(h, h0, zero, zero, p, c)
    low = np.arctanh((out - h) / c)
    silu = lambda x: x / (1.0 + np.exp(-np.asarray(x, float)))  # noqa: E731
    normed_col1 = np.array([[1.6, 1.0, 0.0], [0.0, -1.0, 1.2]])        # h[b, s, 1] / rms
    pooled_col0 = np.array([(1.2 + 1.0 + 2.0) / 3, (0.0 + 1.0 + 0.0) / 3])
    np.testing.assert_allclose(low[..., 3], silu(normed_col1), rtol=1e-4, atol=1e-9)
    np.testing.assert_allclose(low[..., 0], silu(np.repeat(pooled_col0[:, None], 3, 1)), rtol=1e-4)
    np.testing.assert_allclose(low[..., 1], silu(h0[..., 2]), rtol=1e-9)
    np.testing.assert_allclose(low[..., 2], 0.0, atol=1e-12)
    # gain multiplies h itself, bias adds per coordinate, scale multiplies the tanh
    p2 = dict(p, d_gain=np.full((1, 1, d), 0.25), bias=np.array([[[0.1, -0.2, 0.3, 0.0]]]),
              update_scale=np.array([[[1.0, 0.5, 2.0, 1.0]]]))
    out2 = MO.bounded_apply(h, h0, zero, zero, p2, c)
    arg = np.arctanh((out2 - h) / (c * p2["update_scale"][0, 0]))
    np.testing.assert_allclose(arg - 0.25 * h - p2["bias"][0, 0], low, rtol=1e-9, atol=1e-9)


# Recipe tables enumerated by hand from the template rule of rte/recipes.py:65-100: recipe 0 is
# dense; sparse recipe idx + 1 takes head slot idx % head_slots, ffn slot idx % ffn_slots,
# attention bank (idx // head_slots) % attn_banks, ffn bank (idx // ffn_slots) % ffn_banks.
_RECIPE_TABLES = [
    (dict(attn_banks=2, ffn_banks=2, head_groups=4, ffn_groups=4, active_head_groups=2, active_ffn_groups=1,
          recipe_count=9),
     [((0,), (0,), (0, 1), (0,)), ((0,), (0,), (2, 3), (1,)), ((1,), (0,), (0, 1), (2,)),
      ((1,), (0,), (2, 3), (3,)), ((0,), (1,), (0, 1), (0,)), ((0,), (1,), (2, 3), (1,)),
      ((1,), (1,), (0, 1), (2,)), ((1,), (1,), (2, 3), (3,))]),
    (dict(attn_banks=3, ffn_banks=1, head_groups=4, ffn_groups=6, active_head_groups=1, active_ffn_groups=2,
          recipe_count=13),
     [((0,), (0,), (0,), (0, 1)), ((0,), (0,), (1,), (2, 3)), ((0,), (0,), (2,), (4, 5)),
      ((0,), (0,), (3,), (0, 1)), ((1,), (0,), (0,), (2, 3)), ((1,), (0,), (1,), (4, 5)),
      ((1,), (0,), (2,), (0, 1)), ((1,), (0,), (3,), (2, 3)), ((2,), (0,), (0,), (4, 5)),
      ((2,), (0,), (1,), (0, 1)), ((2,), (0,), (2,), (2, 3)), ((2,), (0,), (3,), (4, 5))]),
]


@pytest.mark.parametrize("case", range(len(_RECIPE_TABLES)))
def test_recipe_templates_enumerated_and_balanced(case):
    """The oracle's and the package's recipe tables equal the hand-enumerated ones, and every
    bank / group is used equally often (validate_balance spreads of rte/recipes.py:141-159 are 0)."""
    from oracle import banked as BK
    from rte_amd.config import ModelConfig
    from rte_amd.recipes import RecipeBank

    kw, sparse = _RECIPE_TABLES[case]
    want = [dict(attention_banks=tuple(range(kw["attn_banks"])), ffn_banks=tuple(range(kw["ffn_banks"])),
                 head_groups=tuple(range(kw["head_groups"])), ffn_groups=tuple(range(kw["ffn_groups"])))]
    want += [dict(attention_banks=a, ffn_banks=f, head_groups=h, ffn_groups=s) for a, f, h, s in sparse]
    got = BK.recipe_templates(kw["attn_banks"], kw["ffn_banks"], kw["head_groups"], kw["ffn_groups"],
                              kw["active_head_groups"], kw["active_ffn_groups"], kw["recipe_count"])
    assert got == want
    cfg = ModelConfig(topology="recursive", vocab_size=64, d_model=48, n_heads=12, d_ff=96, n_dense_layers=2,
                      n_prelude=1, n_coda=1, t_max=2, depth_choices=[1, 2], **kw)
    bank = RecipeBank(cfg)
    assert [dict(attention_banks=r.attention_banks, ffn_banks=r.ffn_banks, head_groups=r.head_groups,
                 ffn_groups=r.ffn_groups) for r in bank.recipes] == want
    counts = {key: np.zeros(n, int) for key, n in (("attention_banks", kw["attn_banks"]),
                                                    ("ffn_banks", kw["ffn_banks"]),
                                                    ("head_groups", kw["head_groups"]),
                                                    ("ffn_groups", kw["ffn_groups"]))}
    for r in want[1:]:
        for key, arr in counts.items():
            arr[list(r[key])] += 1
    assert all(a.max() - a.min() == 0 for a in counts.values())
    if hasattr(bank, "validate_balance"):
        assert all(v == 0 for v in bank.validate_balance().values())


def test_static_centers_brute_force_and_invariants():
    """route_to_static_centers (rte/kernels/cluster_pool_ffn.py:129-140) restated: a per-token
    loop with math.sqrt gives the same choice; scaling a token's features by a positive factor
    changes nothing (the features are normalised); equal centres go to the lower index; k = 1
    top-k of the scores agrees."""
    import math

    rng = _rng(80)
    q = rng.standard_normal((200, 12))
    centers = rng.standard_normal((9, 12))
    centers[7] = centers[2]  # a tie: index 2 wins
    ids, scores = R.static_centers(q, centers)
    for t in range(q.shape[0]):
        n = math.sqrt(sum(v * v for v in q[t]))
        best, bi = -math.inf, -1
        for c in range(centers.shape[0]):
            sc = sum(q[t, j] / n * centers[c, j] for j in range(12))
            if sc > best:
                best, bi = sc, c
        assert ids[t] == bi
    np.testing.assert_array_equal(R.static_centers(q * rng.uniform(0.1, 10.0, (200, 1)), centers)[0], ids)
    assert 7 not in ids
    np.testing.assert_array_equal(R.route_topk(scores.astype(np.float32), 1)[0][:, 0], ids)


def _router_params(rng, d=16, H=12, R=5, D=3, t=4, A=2, Fb=3, Hs=2, Fs=4):
    def lin(o, i):
        return rng.standard_normal((o, i)) * 0.3, rng.standard_normal(o) * 0.1

    p = {}
    for name, o, i in (("recipe_mlp.0", H, d), ("recipe_mlp.2", R, H), ("depth_mlp.0", H, d), ("depth_mlp.2", D, H),
                       ("factor_mlp.0", H, d), ("factor_mlp.2", H, H), ("attn_bank_head", A, H),
                       ("ffn_bank_head", Fb, H), ("head_slot_head", Hs, H), ("ffn_slot_head", Fs, H)):
        p[name + ".weight"], p[name + ".bias"] = lin(o, i)
    p["pass_recipe_bias"] = rng.standard_normal((t, R)) * 0.2
    p["pass_factor_bias"] = rng.standard_normal((t, H)) * 0.2
    return p


def test_router_oracle_matches_torch_modules():
    """The router oracle against the same computation by torch modules (nn.Linear, F.silu,
    F.softmax, argmax) on the CPU in float64, for every output field (rte/routing.py:80-188)."""
    from oracle import router as RO

    rng = _rng(81)
    p = _router_params(rng)
    h0 = rng.standard_normal((6, 7, 16))
    o = RO.router(h0, p, [1, 2, 4], temperature=0.7)
    T = lambda k: torch.tensor(p[k])  # noqa: E731
    F = torch.nn.functional
    lin = lambda x, n: F.linear(x, T(n + ".weight"), T(n + ".bias"))  # noqa: E731
    pooled = torch.tensor(h0).mean(1)
    mlp = lambda n: lin(F.silu(lin(pooled, n + ".0")), n + ".2")  # noqa: E731
    rl = mlp("recipe_mlp") / 0.7
    np.testing.assert_allclose(o["recipe_logits"], rl.numpy(), rtol=1e-12)
    np.testing.assert_allclose(o["recipe_logits_by_pass"], (rl[:, None] + T("pass_recipe_bias") / 0.7).numpy(),
                               rtol=1e-12)
    dp = F.softmax(mlp("depth_mlp") / 0.7, -1)
    np.testing.assert_allclose(o["depth_probs"], dp.numpy(), rtol=1e-12)
    np.testing.assert_array_equal(o["depth_id"], dp.argmax(-1).numpy())
    np.testing.assert_allclose(o["expected_depth"], (dp * torch.tensor([1.0, 2.0, 4.0])).sum(-1).numpy(), rtol=1e-12)
    fh = F.silu(mlp("factor_mlp")[:, None] + T("pass_factor_bias"))
    ent = 0
    for name in ("attn_bank", "ffn_bank", "head_slot", "ffn_slot"):
        pr = F.softmax(lin(fh, name + "_head") / 0.7, -1)
        np.testing.assert_array_equal(o[name + "_id_by_pass"], pr.argmax(-1).numpy())
        ent = ent - (pr.clamp_min(1e-9).log() * pr).sum(-1)
    np.testing.assert_allclose(o["factor_entropy"], ent.mean(-1).numpy(), rtol=1e-12)


def test_router_entropy_and_depth_closed_form():
    """Two equal logits give entropy ln 2 and expected depth the mean of the two choices."""
    from oracle import router as RO

    assert abs(RO._entropy(RO._softmax(np.array([[0.3, 0.3]])))[0] - np.log(2.0)) < 1e-12
    pr = RO._softmax(np.array([[1.0, 1.0]]))
    assert abs((pr * np.array([2.0, 4.0])).sum() - 3.0) < 1e-12


def test_factorized_topk_brute_force():
    """_factorized_topk_routes (rte/models.py:273-310): enumerate every (attn bank, ffn bank, head
    slot, ffn slot) tuple, sort by summed logit (value desc, flat index asc), softmax the top k."""
    import itertools

    from oracle import router as RO

    rng = _rng(82)
    A, Fb, Hs, Fs = 2, 3, 2, 4
    a, b, c, e = (rng.standard_normal((5, n)) for n in (A, Fb, Hs, Fs))
    factors, w = RO.factorized_topk(a, b, c, e, 6)
    for t in range(5):
        tuples = list(itertools.product(range(A), range(Fb), range(Hs), range(Fs)))
        sc = [np.float32(a[t, i] + b[t, j] + c[t, k] + e[t, m]) for i, j, k, m in tuples]
        order = sorted(range(len(tuples)), key=lambda q: (-sc[q], q))[:6]
        assert [tuple(x) for x in factors[t]] == [tuples[q] for q in order]
        sel = np.array([sc[q] for q in order], np.float64)
        np.testing.assert_allclose(w[t], np.exp(sel - sel.max()) / np.exp(sel - sel.max()).sum(), rtol=1e-6)


def _svd_sparse_case(seed, T=6, d=8, F=16):
    rng = _rng(seed)
    x = rng.standard_normal((T, d))
    wu, wg, wd = (rng.standard_normal((F, d)) * 0.5 for _ in range(3))
    uh = (x @ wu.T + rng.standard_normal((T, F)) * 0.3).astype(np.float32)
    gh = (x @ wg.T + rng.standard_normal((T, F)) * 0.3).astype(np.float32)
    return x, wu, wg, wd, uh, gh


def test_svd_sparse_all_neurons_is_dense_swiglu():
    """Every neuron a candidate and selected (top_k = d_ff): the sparse FFN is the dense SwiGLU
    (rte/layers.py:620-643 with the full candidate set)."""
    from oracle import svd_sparse as SS

    x, wu, wg, wd, uh, gh = _svd_sparse_case(83)
    out, sel, _, _ = SS.forward(x, wu, wg, wd, uh, gh, up_m=16, gate_m=0, product_m=0, top_k=16)
    dense, _ = SW.dense_swiglu_fwd(x, np.concatenate([wu, wg]), wd, wd_rows=True)
    np.testing.assert_allclose(out, dense, rtol=1e-12, atol=1e-12)
    assert (sel == np.arange(16)).all()


def test_svd_sparse_brute_force_selection():
    """Candidate union, fill and rerank against explicit sorts with (score desc, id asc) keys."""
    import math

    from oracle import svd_sparse as SS

    x, wu, wg, wd, uh, gh = _svd_sparse_case(84)
    w = np.sqrt((wd * wd).sum(-1)).astype(np.float32)
    for up_m, gate_m, product_m, top_k in ((3, 2, 2, 4), (1, 0, 0, 5), (4, 4, 4, 3)):
        _, sel, _, _ = SS.forward(x, wu, wg, wd, uh, gh, up_m=up_m, gate_m=gate_m, product_m=product_m, top_k=top_k)
        for t in range(x.shape[0]):
            def top(sc, m):
                return [j for _, j in sorted((-float(sc[j]), j) for j in range(16))[:m]]

            gs = [float(gh[t, j]) / (1 + math.exp(-float(gh[t, j]))) for j in range(16)]
            cand = set(top([abs(uh[t, j]) * w[j] for j in range(16)], up_m))
            cand |= set(top([abs(gs[j]) * w[j] for j in range(16)], gate_m))
            prod = [abs(uh[t, j] * np.float32(gs[j])) * w[j] for j in range(16)]
            cand |= set(top(prod, product_m))
            if len(cand) < top_k:
                cand |= set(top(prod, top_k))
            ex = {c: abs((x[t] @ wu[c]) * (x[t] @ wg[c]) / (1 + math.exp(-(x[t] @ wg[c])))) * w[c] for c in cand}
            want = sorted(c for _, c in sorted((-ex[c], c) for c in cand)[:top_k])
            assert sel[t].tolist() == want


def test_svd_sparse_backward_matches_autograd():
    from oracle import svd_sparse as SS

    x, wu, wg, wd, uh, gh = _svd_sparse_case(85)
    out, sel, u, g = SS.forward(x, wu, wg, wd, uh, gh, up_m=3, gate_m=3, product_m=2, top_k=4)
    dy = _rng(86).standard_normal(out.shape)
    dx, dwu, dwg, dwd = SS.backward(dy, x, wu, wg, wd, sel, u, g)
    tx, twu, twg, twd = (torch.tensor(a, requires_grad=True) for a in (x, wu, wg, wd))
    s = torch.from_numpy(sel)
    uu = (tx[:, None, :] * twu[s]).sum(-1)
    gg = (tx[:, None, :] * twg[s]).sum(-1)
    ((uu * torch.nn.functional.silu(gg))[:, :, None] * twd[s]).sum(1).mul(torch.tensor(dy)).sum().backward()
    for a, b in ((dx, tx), (dwu, twu), (dwg, twg), (dwd, twd)):
        np.testing.assert_allclose(a, b.grad.numpy(), rtol=1e-10, atol=1e-12)


def test_step_port_runs_and_updates():
    """The CPU step that bench.py times as its baseline: one AdamW step at a small cfg3-shaped
    model gives a finite loss and moves the parameters the step reaches (Phi, core, coda,
    embedding, prelude)."""
    import torch

    from oracle import step_port as SP
    from rte_amd.config import ExperimentConfig, ModelConfig, OutputConfig, TrainingConfig
    from rte_amd.models import RecursiveModel

    mc = ModelConfig(topology="recursive", vocab_size=64, d_model=64, n_heads=2, d_ff=256, n_dense_layers=2,
                     n_prelude=1, n_coda=1, t_max=4, depth_choices=[1, 2, 4], attn_banks=1, ffn_banks=1,
                     head_groups=2, ffn_groups=8, active_head_groups=1, active_ffn_groups=2, recipe_count=4,
                     macro_rank=8, ffn_kind="cluster_pool", ffn_clusters=8, ffn_top_k=2)
    tc = TrainingConfig(mode="recursive_macro", batch_size=2, seq_len=16, audit_sampler="fixed_count",
                        audit_fixed_count=1, fixed_depth=4)
    cfg = ExperimentConfig(model=mc, training=tc, output=OutputConfig())
    torch.manual_seed(0)
    m = RecursiveModel(mc, cfg.output)
    port = SP.StepPort(cfg, dict(m.named_parameters()), dict(m.named_buffers()))
    before = {k: v.detach().clone() for k, v in port.params(False).items()}
    opt = SP.make_optimizer(port)
    tok, tgt = SP.zipf_tokens(64, 2, 16, seed=1)
    loss = SP.train_step(port, opt, tok, tgt, chosen=torch.tensor([1]), usage_ema=torch.zeros(4))
    assert np.isfinite(loss)
    after = port.params(False)
    for k in ("macro.v", "core.attn.wqkv", "coda.0.mlp.wug.weight", "embed.weight", "prelude.0.attn.wqkv.weight"):
        assert not torch.equal(before[k], after[k]), k
