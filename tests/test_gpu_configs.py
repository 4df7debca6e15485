"""The BASELINE configurations at their own sizes on the GPU.

cfg1 (cluster-pool layer, T 8192, d 256, 32 x 32, top-4) against the oracle at full size;
cfg5's routed pool (d 1024, 256 pools x 64, top-16, Zipf-skewed routing) against the oracle at
T 4096 and at the full T 16384 through size-independent properties (per-token rows against
the oracle, additivity of the weight gradients over token halves, bitwise repeatability);
cfg4's SVD FFN at its full T 32768 through the same properties; the cfg3 train step (the
bench's engine) eager against captured; the cfg5 recursive_macro_shortlist step at its size.
Tolerances: routing ids bit-exact, bf16 paths 2e-2 relative (Frobenius)."""

from __future__ import annotations

import math
import warnings

import numpy as np
import pytest
import torch

from helpers import BF16_RTOL, assert_rel, bf16_round
from oracle import cluster_pool as CP
from oracle import routing as R

pytestmark = pytest.mark.gpu

DEV = "cuda"


@pytest.fixture(scope="module", autouse=True)
def _hip():
    from rte_amd import _lib

    if not _lib.device_ready():
        pytest.fail("HIP backend not ready on this GPU box (library or gfx950 device missing)")
    yield


def _np(t):
    return t.detach().float().cpu().numpy()


def _pool_case(T, d, C, n, seed, skew):
    """bf16-exact inputs; with skew, a shared input feature and a Zipf(1.1) bias on the router
    weights send most pairs to the low cluster ids."""
    rng = np.random.default_rng(seed)
    F = C * n
    x = rng.standard_normal((T, d)).astype(np.float32)
    wr = (rng.standard_normal((C, d)) * 0.02).astype(np.float32)
    if skew:
        x[:, 0] = 4.0
        zipf = -1.1 * np.log(np.arange(1, C + 1))
        wr[:, 0] = 0.25 * (zipf - zipf.mean())
    x = bf16_round(x)
    wug = (rng.standard_normal((2 * F, d)) * 0.02).astype(np.float32)
    wd = (rng.standard_normal((d, F)) * 0.02).astype(np.float32)
    dy = bf16_round(rng.standard_normal((T, d)).astype(np.float32))
    return x, wr, wug, wd, dy


def _run_pool(x, wr, wug, wd, dy, k, rows=None):
    from rte_amd.kernels import hip_ops as H

    sl = slice(None) if rows is None else rows
    tx = torch.from_numpy(x[sl]).to(DEV).to(torch.bfloat16).requires_grad_()
    twr, tug, twd = (torch.from_numpy(a).to(DEV).requires_grad_() for a in (wr, wug, wd))
    out, ids, w = H.routed_cluster_pool_swiglu(tx, twr, tug, twd, k)
    out.backward(torch.from_numpy(dy[sl]).to(DEV))
    torch.cuda.synchronize()
    return out, ids, w, tx.grad, twr.grad, tug.grad, twd.grad


def _oracle_check(x, wr, wug, wd, dy, k, C, got, what, routes=None):
    """Routing ids against the oracle's top-k of the kernel's own logits (bit-exact), then y and
    dx against the oracle under those routes.  routes = (ids, w) skips the routing check and uses
    the given decisions (for a row subset of a larger run)."""
    out, ids, w, dx, dwr, dwug, dwd = got
    from rte_amd.kernels import hip_ops as H

    if routes is None:
        logits = H.gemm(torch.from_numpy(x).to(DEV).to(torch.bfloat16),
                        torch.from_numpy(bf16_round(wr)).to(DEV).to(torch.bfloat16), out_f32=True)
        rids, rw = R.route_topk(_np(logits), k)
        np.testing.assert_array_equal(ids.cpu().numpy(), rids, err_msg=f"{what} ids")
    else:
        rids, rw = routes
    wr_b, wug_b, wd_b = bf16_round(wr), bf16_round(wug), bf16_round(wd)
    assert_rel(_np(out), CP.routed_fwd(x, wug_b, wd_b, rids, rw, C), BF16_RTOL, f"{what} y")
    gdx, gdwr, gdwug, gdwd, _ = CP.routed_bwd(dy, x, wr_b, wug_b, wd_b, rids, rw, C)
    assert_rel(_np(dx), gdx, BF16_RTOL, f"{what} dx")
    return gdwr, gdwug, gdwd, (dwr, dwug, dwd)


def test_cfg1_layer_full_size_vs_oracle():
    """BASELINE configs[0] shape (T 8192 = 128 x 64, d 256, 32 pools x 32, top-4), fwd + bwd."""
    T, d, C, n, k = 8192, 256, 32, 32, 4
    print(f"cfg1 layer T={T} d={d} C={C}x{n} k={k}", flush=True)
    x, wr, wug, wd, dy = _pool_case(T, d, C, n, seed=0, skew=False)
    got = _run_pool(x, wr, wug, wd, dy, k)
    gdwr, gdwug, gdwd, (dwr, dwug, dwd) = _oracle_check(x, wr, wug, wd, dy, k, C, got, "cfg1")
    assert_rel(_np(dwr), gdwr, BF16_RTOL, "cfg1 dwr")
    assert_rel(_np(dwug), gdwug, BF16_RTOL, "cfg1 dwug")
    assert_rel(_np(dwd), gdwd, BF16_RTOL, "cfg1 dwd")


def test_cfg5_pool_vs_oracle_skewed():
    """cfg5's routed pool (d 1024, 256 x 64, top-16) on Zipf-skewed routing against the oracle."""
    T, d, C, n, k = 4096, 1024, 256, 64, 16
    print(f"cfg5 pool T={T} d={d} C={C}x{n} k={k} skewed", flush=True)
    x, wr, wug, wd, dy = _pool_case(T, d, C, n, seed=5, skew=True)
    got = _run_pool(x, wr, wug, wd, dy, k)
    counts = np.bincount(got[1].cpu().numpy().reshape(-1), minlength=C)
    assert counts[:16].sum() > 4 * counts[-16:].sum(), "routing is not skewed"
    gdwr, gdwug, gdwd, (dwr, dwug, dwd) = _oracle_check(x, wr, wug, wd, dy, k, C, got, "cfg5")
    assert_rel(_np(dwr), gdwr, BF16_RTOL, "cfg5 dwr")
    assert_rel(_np(dwug), gdwug, BF16_RTOL, "cfg5 dwug")
    assert_rel(_np(dwd), gdwd, BF16_RTOL, "cfg5 dwd")


def test_cfg5_pool_full_size_properties():
    """T 16384 (= 32 x 512): rows are per-token functions (256 sampled rows of y and dx against
    the oracle), the weight gradients of the two token halves add up to the full one, and a
    repeat is bitwise identical."""
    T, d, C, n, k = 16384, 1024, 256, 64, 16
    print(f"cfg5 pool full T={T}", flush=True)
    x, wr, wug, wd, dy = _pool_case(T, d, C, n, seed=6, skew=True)
    full = _run_pool(x, wr, wug, wd, dy, k)
    again = _run_pool(x, wr, wug, wd, dy, k)
    for a, b in zip(full, again):
        assert torch.equal(a, b)
    rows = np.sort(np.random.default_rng(1).choice(T, 256, replace=False))
    out, ids, w, dx, *_ = full
    r = torch.from_numpy(rows).to(DEV)
    sub = (out[r], ids[r], w[r], dx[r], None, None, None)
    _oracle_check(x[rows], wr, wug, wd, dy[rows], k, C, sub, "cfg5 rows",
                  routes=(ids[r].cpu().numpy(), w[r].cpu().numpy()))
    h1 = _run_pool(x, wr, wug, wd, dy, k, rows=slice(0, T // 2))
    h2 = _run_pool(x, wr, wug, wd, dy, k, rows=slice(T // 2, T))
    for i, name in ((4, "dwr"), (5, "dwug"), (6, "dwd")):
        assert_rel(_np(h1[i]) + _np(h2[i]), _np(full[i]), 1e-4, f"cfg5 {name} halves")


def test_cfg4_svd_full_size_properties():
    """SVD FFN at BASELINE configs[3] (d 1024, F 4096, r 128, T 32768): 256 sampled rows of y
    and dx against the oracle, weight gradients additive over token halves, bitwise repeat."""
    from oracle import svd_ffn as SV
    from rte_amd.kernels import hip_ops as H

    T, d, F, r = 32768, 1024, 4096, 128
    rng = np.random.default_rng(44)

    def orth(a, b):
        return np.linalg.qr(rng.standard_normal((a, b)))[0]

    S = [10 ** rng.uniform(-2, 0, r) for _ in range(3)]
    m = dict(us_up=orth(d, r) * S[0], us_gate=orth(d, r) * S[1], v_up=orth(F, r), v_gate=orth(F, r),
             v_dn=orth(F, r), us_dn=orth(d, r) * S[2])
    m = {key: bf16_round(v.astype(np.float32)) for key, v in m.items()}
    x = bf16_round(rng.standard_normal((T, d)).astype(np.float32))
    dy = bf16_round(rng.standard_normal((T, d)).astype(np.float32))
    print(f"cfg4 svd full T={T}", flush=True)

    def run(sl):
        tw = {key: torch.from_numpy(v).to(DEV).requires_grad_() for key, v in m.items()}
        tx = torch.from_numpy(x[sl]).to(DEV).to(torch.bfloat16).requires_grad_()
        y = H.svd_ffn(tx, torch.cat([tw["us_up"], tw["us_gate"]], 1), torch.cat([tw["v_up"], tw["v_gate"]], 0),
                      tw["v_dn"], tw["us_dn"])
        y.backward(torch.from_numpy(dy[sl]).to(DEV))
        torch.cuda.synchronize()
        return y.detach(), tx.grad, {key: t.grad for key, t in tw.items()}

    y, dx, g = run(slice(None))
    y2, dx2, g2 = run(slice(None))
    assert torch.equal(y, y2) and torch.equal(dx, dx2) and all(torch.equal(g[key], g2[key]) for key in g)
    rows = np.sort(np.random.default_rng(2).choice(T, 256, replace=False))
    ref, c = SV.svd_ffn_fwd(x[rows], **m)
    assert_rel(_np(y)[rows], ref, BF16_RTOL, "cfg4 y rows")
    gref = SV.svd_ffn_bwd(dy[rows], x[rows], **m, c=c)
    assert_rel(_np(dx)[rows], gref["dx"], BF16_RTOL, "cfg4 dx rows")
    _, _, ga = run(slice(0, T // 2))
    _, _, gb = run(slice(T // 2, T))
    for key in m:
        assert_rel(_np(ga[key]) + _np(gb[key]), _np(g[key]), 1e-4, f"cfg4 d{key} halves")


def _engine_from(cfg):
    from rte_amd.training import TrainEngine

    return TrainEngine(cfg, device=torch.device("cuda"))


@pytest.mark.parametrize("side_streams", [True, False])
def test_cfg3_step_eager_vs_captured(side_streams):
    """The bench's cfg3 recursive_macro engine (d512, pool 64 x 32 top-8, depth 4, V2048,
    B128 x S64): the eager and captured engines from one seed agree step by step (4 steps: two
    eager warm-ups, the capture, a replay), parameters change, and every gradient of an extra
    eager forward / backward is finite.  The captured engine runs the replay's own coda on a side
    stream (side_streams) or appends the replay's rows to the hot coda call with everything on one
    stream; the eager engine does the same, so both sum in the same order."""
    import bench

    cfg = bench.cfg3_config()
    a, b = _engine_from(cfg), _engine_from(cfg)
    a.replay_coda_shared = not side_streams
    b.graph_side_streams = side_streams
    b.enable_graph_capture(True)
    gen = torch.Generator().manual_seed(cfg.training.seed)
    batches = [bench.zipf_batch(gen, cfg.model.vocab_size, 128, 64, DEV) for _ in range(4)]
    before = {n_: p.detach().clone() for n_, p in a.recursive_model.named_parameters()}
    for step, batch in enumerate(batches):
        print(f"cfg3 step {step} (captured side streams {side_streams})", flush=True)
        with warnings.catch_warnings(record=True) as caught:
            warnings.simplefilter("always")
            ra, rb = a.train_step(batch), b.train_step(batch)
            torch.cuda.synchronize()
        # the step results hold no autograd graph, so no gradient accumulator outlives its step
        assert not [w for w in caught if "AccumulateGrad" in str(w.message)], step
        la, lb = float(ra.loss.detach()), float(rb.loss)
        assert math.isfinite(la) and abs(la - lb) <= 1e-4 * max(abs(la), 1.0), (step, la, lb)
        assert bool(ra.metrics["stepped"]) and bool(rb.metrics["stepped"])
    changed = sum(int(not torch.equal(before[n_], p.detach())) for n_, p in a.recursive_model.named_parameters())
    assert changed > len(before) // 2
    for (na, pa), (_, pb) in zip(a.recursive_model.named_parameters(), b.recursive_model.named_parameters()):
        assert torch.allclose(pa, pb, rtol=1e-4, atol=1e-5), na
    # gradients of one more eager step, before the optimizer consumes them
    tok, tgt = batches[0]
    loss, *_ = a._macro_loss(tok, tgt, shortlist=False)
    loss.backward()
    a._flush_grad_sink()
    n_grads = 0
    for n_, p in a.recursive_model.named_parameters():
        if p.grad is not None:
            n_grads += 1
            assert torch.isfinite(p.grad).all(), n_
    assert n_grads > len(before) // 2
    a.optimizer.zero_grad(set_to_none=True)


def test_cfg3_side_launch_late_vs_early():
    """Issuing the audit replay and the consistency loss after the hot forward (side_launch_late,
    their streams waiting on an event from the routing point) against issuing them at routing:
    the same audited rows (the fixed-count sampler's seeded permutation, drawn on the main stream
    before that event) and the same losses, step by step, with the replay's own coda on side
    streams in eager steps."""
    import bench

    from rte_amd.audit import AuditEngine

    cfg = bench.cfg3_config()
    late, early = _engine_from(cfg), _engine_from(cfg)
    for e, flag in ((late, True), (early, False)):
        e.replay_coda_shared = False
        e.side_launch_late = flag
    gen = torch.Generator().manual_seed(cfg.training.seed)
    batches = [bench.zipf_batch(gen, cfg.model.vocab_size, 128, 64, DEV) for _ in range(3)]
    k = int(cfg.training.audit_fixed_count_per_batch)
    for step, batch in enumerate(batches):
        print(f"cfg3 late/early step {step}", flush=True)
        want = torch.zeros(128, dtype=torch.bool, device=DEV)
        want[AuditEngine.fixed_count_index(128, k, cfg.training.seed + 10_000 + late.global_step, DEV)] = True
        ra, rb = late.train_step(batch), early.train_step(batch)
        torch.cuda.synchronize()
        assert torch.equal(ra.audit.audit_mask.reshape(-1), want), step
        assert torch.equal(rb.audit.audit_mask.reshape(-1), want), step
        la, lb = float(ra.loss), float(rb.loss)
        assert math.isfinite(la) and abs(la - lb) <= 1e-6 * max(abs(la), 1.0), (step, la, lb)
    for (na, pa), (_, pb) in zip(late.recursive_model.named_parameters(), early.recursive_model.named_parameters()):
        assert torch.allclose(pa, pb, rtol=1e-5, atol=1e-6), na


def test_cfg3_consistency_backward_early_grad_accum():
    """The consistency term's backward issued right after its forward (on a detached h0 joined by
    a hook) against its backward inside the step's: with two accumulated micro-steps the same
    losses and, after the update, the same parameters (the early backward carries the step's
    1 / grad_accum_steps)."""
    import dataclasses

    import bench

    cfg = bench.cfg3_config(batch=16)
    cfg = dataclasses.replace(cfg, training=dataclasses.replace(cfg.training, grad_accum_steps=2))
    early, inside = _engine_from(cfg), _engine_from(cfg)
    for e, flag in ((early, True), (inside, False)):
        e.replay_coda_shared = False
        e.audit_engine.consistency_backward_early = flag
    gen = torch.Generator().manual_seed(cfg.training.seed)
    batches = [bench.zipf_batch(gen, cfg.model.vocab_size, 16, 64, DEV) for _ in range(4)]
    for step, batch in enumerate(batches):
        print(f"cfg3 consistency early / inside, micro-step {step}", flush=True)
        ra, rb = early.train_step(batch), inside.train_step(batch)
        torch.cuda.synchronize()
        la, lb = float(ra.loss), float(rb.loss)
        assert math.isfinite(la) and abs(la - lb) <= 1e-5 * max(abs(la), 1.0), (step, la, lb)
    assert early.global_step == inside.global_step == 2
    for (na, pa), (_, pb) in zip(early.recursive_model.named_parameters(), inside.recursive_model.named_parameters()):
        assert torch.allclose(pa, pb, rtol=1e-4, atol=1e-5), na


def test_cfg5_shortlist_step():
    """the scaled recursive_macro_shortlist step (d1024, 16 heads, depth 8,
    pool 256 x 64 top-16, V8192 shortlist, B32 x S512): finite losses, parameters change, the
    shortlist metrics are present, and the loss falls over repeated steps on one batch."""
    import bench
    from rte_amd.training import metrics_to_host

    cfg = bench.cfg5_config()
    eng = _engine_from(cfg)
    gen = torch.Generator().manual_seed(cfg.training.seed)
    batch = bench.zipf_batch(gen, cfg.model.vocab_size, 32, 512, DEV)
    before = {n_: p.detach().clone() for n_, p in eng.recursive_model.named_parameters()}
    losses = []
    for step in range(4):
        print(f"cfg5 step {step}", flush=True)
        res = eng.train_step(batch)
        m = metrics_to_host(res.metrics)
        losses.append(float(m["loss"]))
        assert math.isfinite(losses[-1]), m
        assert m["stepped"] if not isinstance(m["stepped"], torch.Tensor) else bool(m["stepped"])
    changed = sum(int(not torch.equal(before[n_], p.detach())) for n_, p in eng.recursive_model.named_parameters())
    assert changed > len(before) // 2
    assert losses[-1] < losses[0], losses
    sl = res.model_output.meta.shortlist
    assert sl is not None and sl.shortlist.shape[-1] == cfg.output.shortlist_max_tokens


def test_cfg3_side_stream_audit_gradients_match_main_stream():
    """gradient_corrected audit whose exact replay runs on a side stream (the replay selects h0 rows
    there, and their gradient is added into h0's on the main stream by a hook): every parameter
    gradient of one step equals, to fp32 summation order, the same step with the replay on the
    main stream.  Guards the cross-stream hand-over of the selected rows' gradient."""
    import bench

    cfg = bench.cfg3_config(batch=16)
    assert cfg.training.audit_mode == "gradient_corrected"
    eng = _engine_from(cfg)
    gen = torch.Generator().manual_seed(7)
    tok, tgt = bench.zipf_batch(gen, cfg.model.vocab_size, 16, 64, DEV)
    grads = []
    for streams in (True, False, True):
        print(f"side-stream audit step, audit_streams={streams}", flush=True)
        eng.audit_streams = streams
        eng._bf16.begin()
        loss, *_ = eng._macro_loss(tok, tgt, shortlist=False)
        loss.backward()
        eng._flush_grad_sink()
        eng._bf16.end()
        torch.cuda.synchronize()
        grads.append({n_: p.grad.detach().clone() for n_, p in eng.recursive_model.named_parameters()
                      if p.grad is not None})
        eng.optimizer.zero_grad(set_to_none=True)
    side, main, side2 = grads
    assert set(side) == set(main) and any(n_.startswith("embed") for n_ in side)
    for n_ in main:
        ref = main[n_]
        err = float((side[n_] - ref).norm() / ref.norm().clamp_min(1e-30))
        assert err <= 1e-5, (n_, err)
        assert torch.equal(side[n_], side2[n_]), n_


def test_captured_step_skips_nonfinite_and_reconciles_global_step(tmp_path):
    """A captured replay whose loss is non-finite (a weight set to NaN from the host) skips the
    update (parameters unchanged, stepped False); reconcile_global_step() and the checkpoint then
    count applied updates only, as the eager path (rte/training.py:445-468) does."""
    import bench

    cfg = bench.cfg3_config(batch=8)
    eng = _engine_from(cfg)
    eng.enable_graph_capture(True)
    m = eng.recursive_model
    gen = torch.Generator().manual_seed(3)
    batch = bench.zipf_batch(gen, cfg.model.vocab_size, 8, 64, DEV)
    for step in range(4):  # two eager warm-ups, the capture, a replay
        print(f"captured step {step}", flush=True)
        assert bool(eng.train_step(batch).metrics["stepped"])
    saved = m.final_norm.weight.detach().clone()
    with torch.no_grad():
        m.final_norm.weight.fill_(float("nan"))
    before = {n_: p.detach().clone() for n_, p in m.named_parameters() if n_ != "final_norm.weight"}
    res = eng.train_step(batch)
    torch.cuda.synchronize()
    assert not bool(res.metrics["stepped"])
    for n_, p in m.named_parameters():
        if n_ != "final_norm.weight":
            assert torch.equal(before[n_], p.detach()), n_
    with torch.no_grad():
        m.final_norm.weight.copy_(saved)
    assert bool(eng.train_step(batch).metrics["stepped"])
    assert eng.global_step == 6  # attempted replays, counted without a device read
    assert eng.reconcile_global_step() == 5
    eng.save_checkpoint(tmp_path / "ck.pt")
    assert torch.load(tmp_path / "ck.pt", weights_only=True)["global_step"] == 5
