"""The composed recursive_macro train step on the GPU against the CPU restatement of the
reference's step (oracle/step_port.py, pinned in tests/test_step_port.py).

One eager HIP step at the cfg3 layout (d512, 8 heads, prelude / coda routed pools of 64 x 32
top-8, banked core of 64 slabs x 32 with 8 active, depth 4, V2048, fixed-count audit of one
sample, consistency and distillation terms), batch 8 x 64, and the CPU port from the same
weights, batch, audited row and recipe-usage EMA.  Checked:
  * the routed pools' ids of every call (prelude, coda, the replay's coda) bit-exact against
    the oracle top-k of the kernel's own router logits;
  * every loss term and the total within 2e-2 relative at precision bf16 (bf16 GEMM operands on
    the GPU, fp32 on the CPU), within 1e-5 at precision fp32;
  * every parameter gradient within the same tolerance (Frobenius); parameters the step does not
    reach have no (or an all-zero) gradient on both sides.
The GPU's discrete decisions (pool ids, recipe ids) are handed to the port, so a tie broken
differently by bf16 rounding does not count as an arithmetic difference; the ids are checked
on their own above."""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import routing as OR
from oracle import step_port as SP

pytestmark = pytest.mark.gpu

DEV = "cuda"
RTOL = {"bf16": 2e-2, "fp32": 1e-5}


@pytest.fixture(scope="module", autouse=True)
def _hip():
    from rte_amd import _lib

    if not _lib.device_ready():
        pytest.fail("HIP backend not ready on this GPU box (library or gfx950 device missing)")
    yield


def _rel(a, b):
    return float((a.double() - b.double()).norm() / b.double().norm().clamp_min(1e-30))


def _run(cfg, B, S, seed, shared_coda=True):
    import bench
    from rte_amd.kernels import hip_ops
    from rte_amd.training import TrainEngine

    eng = TrainEngine(cfg, device=torch.device(DEV))
    eng.replay_coda_shared = shared_coda
    m = eng.recursive_model
    with torch.no_grad():
        # a macro update well above the rounding of h0: the distillation's delta terms divide by
        # rms(Phi(h0) - h0), which at the initial U (1e-3) is the difference of two nearly equal
        # fp32 values, so any two fp32 evaluations of it differ in the fourth digit
        m.macro.u.mul_(100.0)
    calls = []

    def hook(name):
        def rec(mod, args, out):
            calls.append((name, args[0].detach(), mod.last_ids.detach().clone(), mod))
        return rec

    handles = [m.prelude[0].mlp.register_forward_hook(hook("prelude")),
               m.coda[0].mlp.register_forward_hook(hook("coda"))]
    gen = torch.Generator().manual_seed(seed)
    tok, tgt = bench.zipf_batch(gen, cfg.model.vocab_size, B, S, DEV)
    usage = m.recipe_bank.usage_ema.detach().clone().cpu()
    params = {n: p.detach().clone().cpu() for n, p in m.named_parameters()}
    buffers = {n: b.detach().clone().cpu() for n, b in m.named_buffers()}
    eng._bf16.begin()
    loss, hot, audit, aux, scale = eng._macro_loss(tok, tgt, shortlist=False)
    loss.backward()
    eng._flush_grad_sink()  # the side work's parameter gradients (late launch) into .grad
    eng._bf16.end()
    torch.cuda.synchronize()
    for h in handles:
        h.remove()
    grads = {n: (p.grad.detach().float().cpu() if p.grad is not None else None) for n, p in m.named_parameters()}
    chosen = audit.audit_mask.nonzero().flatten().cpu()
    # the routed pools' decisions, by call: prelude and hot coda over B S rows, the replay's coda
    # over the audited rows (after the hot rows when the two share the coda call)
    pools = {"prelude": [], "coda": [], "replay_coda": []}
    k = cfg.model.ffn_top_k
    for name, x, ids, mod in calls:
        n = x.reshape(-1, x.shape[-1]).shape[0]
        if name == "coda" and n > B * S:
            pools["coda"].append(ids[:B * S].long().cpu())
            pools["replay_coda"].append(ids[B * S:].long().cpu())
        else:
            pools[name if n == B * S else "replay_coda"].append(ids.long().cpu())
        if cfg.training.precision == "fp32":  # the fp32 router product the pool used
            from rte_amd.kernels import f32_ops

            logits = f32_ops.linear(x.reshape(-1, x.shape[-1]), mod.router.weight.detach())
            rid, _ = OR.route_topk(logits.cpu().numpy(), k)
        else:
            xb = x.reshape(-1, x.shape[-1]).contiguous().to(torch.bfloat16)
            kid, _, _, logits = hip_ops.route_pack(xb, hip_ops.cast_bf16(mod.router.weight.detach()), k,
                                                   with_logits=True)
            rid, _ = OR.route_topk(logits.cpu().numpy(), k)
            assert np.array_equal(kid.cpu().numpy(), rid), name
        assert np.array_equal(ids.cpu().numpy(), rid), name
    assert [len(v) for v in pools.values()] == [1, 1, 1], {k_: len(v) for k_, v in pools.items()}
    route = hot.meta.router
    forced = {"recipe_id": route.recipe_id.cpu(), "recipe_id_by_pass": route.recipe_id_by_pass.cpu(),
              "pool_ids": pools}
    gpu_terms = {"loss": float(loss.detach()), "corrected_ce": float(audit.corrected_loss_per_sample.detach().mean() / scale),
                 **{f"macro_{k_}": float(v.detach()) for k_, v in audit.macro_aux.items()},
                 **{f"aux_{k_}": float(v.detach()) for k_, v in aux.items()}}
    return params, buffers, tok.cpu(), tgt.cpu(), chosen, usage, forced, gpu_terms, grads


@pytest.mark.parametrize("precision,B,shared_coda", [("bf16", 8, True), ("bf16", 8, False), ("fp32", 8, True)])
def test_cfg3_step_matches_cpu_port(precision, B, shared_coda):
    """shared_coda: the audit replay's rows go through the hot path's coda / head call, else the
    replay runs its own (the captured step with side streams)."""
    import dataclasses

    import bench

    cfg = bench.cfg3_config(batch=B)
    cfg = dataclasses.replace(cfg, training=dataclasses.replace(cfg.training, precision=precision))
    S = 64
    rtol = RTOL[precision]
    print(f"cfg3 layout step parity, precision {precision}, B={B} S={S}, shared coda {shared_coda}", flush=True)
    params, buffers, tok, tgt, chosen, usage, forced, gt, grads = _run(cfg, B, S, seed=11, shared_coda=shared_coda)
    assert chosen.numel() == 1
    # the fp32 step is checked against the restatement in float64 (its own rounding is then the
    # only difference), the bf16 step against fp32
    port = SP.StepPort(cfg, params, buffers, dtype=torch.float64 if precision == "fp32" else torch.float32)
    terms, pg = port.loss_and_grads(tok, tgt, chosen=chosen, usage_ema=usage, forced=forced)
    # the port's own recipe choice agrees with the GPU's on these samples (no near-tie forced)
    assert torch.equal(terms["route"]["recipe_id"], forced["recipe_id"])
    ct = {"loss": float(terms["loss"].detach()), "corrected_ce": float(terms["corrected_ce"].detach()),
          **{f"macro_{k}": float(torch.as_tensor(v).detach()) for k, v in terms["macro_aux"].items()},
          **{f"aux_{k}": float(torch.as_tensor(v).detach()) for k, v in terms["router_aux"].items()}}
    lines, bad = [], []
    # load = lambda (R sum mean_p^2 - 1) cancels to ~1e-3 of its terms: compare on their scale
    scale_of = {"aux_load": cfg.training.lambda_load}
    for k, v in ct.items():
        err = abs(gt[k] - v) / max(abs(v), 1e-6, scale_of.get(k, 0.0))
        lines.append(f"  term {k:24s} gpu {gt[k]: .6e} cpu {v: .6e} rel {err:.2e}")
        if err > rtol:
            bad.append(k)
    for name, g in pg.items():
        h = grads[name]
        if g is None or not bool(g.abs().max() > 0):
            ok = h is None or not bool(h.abs().max() > 0)
            lines.append(f"  grad {name:40s} none on the CPU, {'none' if h is None else 'zero' if ok else 'NONZERO'} on the GPU")
            if not ok:
                bad.append(name)
            continue
        if h is None:
            lines.append(f"  grad {name:40s} MISSING on the GPU")
            bad.append(name)
            continue
        err = _rel(h, g)
        lines.append(f"  grad {name:40s} rel {err:.2e}  |g| {float(g.norm()):.3e}")
        if err > rtol:
            bad.append(name)
    print("\n".join(lines), flush=True)
    assert not bad, bad
