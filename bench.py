"""Benchmark: recursive_macro bf16 train step on one MI355X.

Workload (cfg3): RecursiveModel d_model 512, 8 heads, prelude + coda blocks whose FFN is a
routed cluster pool of 64 clusters x 32 neurons (top-8 per token), banked recursive core
with 64 slabs x 32 (8 active), t_max = fixed depth 4, vocab 2048 tied head, batch 128 x
seq 64, token ids Zipf(1.1), fixed-count audit of 1 sample (p = 1/128), AdamW.  Synthetic
seeded data, random-init weights.  One step = forward_macro + audit correction + backward
+ AdamW, exactly TrainEngine.train_step.

Prints ONE JSON line.  Also reports the roofline of the operation that takes the most time per
step (every candidate timed live with HIP events on the launch stream, its HBM traffic from two
rocprofv3 --pmc runs of this script calibrated against a copy kernel) and a CPU baseline (the
reference's cfg3 step restated in float32 torch on this host's cores, on a bounded batch sample,
and the cfg1 cluster-pool layer in the reference's two CPU forms).
"""

from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
for p in (ROOT, ROOT / "speedup-thingy_amd"):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))

PEAK_BF16_TFLOPS = 2500.0  # MI355X dense bf16 MFMA
PEAK_HBM_GBS = 8000.0
METRIC = "train tokens/sec, recursive_macro bf16 1\u00d7MI355X; FFN MFMA% + route HBM GB/s"


def cfg3_config(batch: int = 128, seq: int = 64):
    from rte_amd.config import ExperimentConfig, ModelConfig, OutputConfig, TrainingConfig

    model = ModelConfig(
        topology="recursive", vocab_size=2048, d_model=512, n_heads=8, d_ff=2048, n_dense_layers=2,
        n_prelude=1, n_coda=1, t_max=4, depth_choices=[1, 2, 4], attn_banks=1, ffn_banks=1, head_groups=8,
        ffn_groups=64, active_head_groups=2, active_ffn_groups=8, recipe_count=16, macro_rank=32,
        ffn_kind="cluster_pool", ffn_clusters=64, ffn_top_k=8,
    )
    training = TrainingConfig(
        mode="recursive_macro", precision="bf16", lr=3e-4, weight_decay=0.1, batch_size=batch, seq_len=seq,
        audit_sampler="fixed_count", audit_fixed_count=1, fixed_depth=4, seed=1337,
    )
    return ExperimentConfig(model=model, training=training, output=OutputConfig(), run_name="bench_cfg3")


def cfg5_config(batch: int = 32, seq: int = 512):
    """scaled recursive_macro_shortlist step, d1024, 16 heads, depth 8,
    routed pool 256 clusters x 64 neurons (top-16) in the prelude / coda blocks and 256 slabs x 64
    (16 active) in the banked core, V8192 with the default shortlist head, B32 x S512."""
    from rte_amd.config import ExperimentConfig, ModelConfig, OutputConfig, TrainingConfig

    model = ModelConfig(
        topology="recursive", vocab_size=8192, d_model=1024, n_heads=16, d_ff=16384, n_dense_layers=2,
        n_prelude=1, n_coda=1, t_max=8, depth_choices=[1, 2, 4, 8], attn_banks=1, ffn_banks=1, head_groups=16,
        ffn_groups=256, active_head_groups=4, active_ffn_groups=16, recipe_count=16, macro_rank=32,
        ffn_kind="cluster_pool", ffn_clusters=256, ffn_top_k=16,
    )
    training = TrainingConfig(
        mode="recursive_macro_shortlist", precision="bf16", lr=3e-4, weight_decay=0.1, batch_size=batch,
        seq_len=seq, audit_sampler="fixed_count", audit_fixed_count=1, fixed_depth=8, seed=1337,
    )
    return ExperimentConfig(model=model, training=training, output=OutputConfig(mode="shortlist"),
                            run_name="bench_cfg5")


def zipf_batch(gen, vocab: int, batch: int, seq: int, device):
    import torch

    p = (torch.arange(vocab, dtype=torch.float64) + 1.0).pow(-1.1)
    p = (p / p.sum()).float()
    ids = torch.multinomial(p, batch * (seq + 1), replacement=True, generator=gen).view(batch, seq + 1)
    ids = ids.to(device)
    return ids[:, :-1].contiguous(), ids[:, 1:].contiguous()


def kernel_candidates(B: int, S: int):
    """Hot operations of the step at their cfg3 shapes, each one call of a C-ABI entry point (one
    or several kernels).  Entry: name, calls per step, kernels per call, algorithmic flop and HBM
    bytes per call (every input read once, every output written once), fn launching it on the
    current stream."""
    import torch

    from rte_amd import _lib
    from rte_amd.kernels import hip_ops

    dev = "cuda"
    T, d, V, C, n, k = B * S, 512, 2048, 64, 32, 8
    F = C * n
    g = torch.Generator(device=dev)
    g.manual_seed(7)
    bf = torch.bfloat16
    x = torch.randn(T, d, device=dev, generator=g).to(bf)
    w_head = (torch.randn(V, d, device=dev, generator=g) * 0.02).to(bf)
    wqkv = (torch.randn(3 * d, d, device=dev, generator=g) * 0.02).to(bf)
    wr = (torch.randn(C, d, device=dev, generator=g) * 0.02).to(bf)
    wug = (torch.randn(2 * F, d, device=dev, generator=g) * 0.02).to(bf)
    wd = (torch.randn(d, F, device=dev, generator=g) * 0.02).to(bf)
    cos = torch.randn(S, 64, device=dev)
    sin = torch.randn(S, 64, device=dev)
    q = torch.empty(B, 8, S, 64, device=dev, dtype=bf)
    kk, vv = torch.empty_like(q), torch.empty_like(q)
    logits = hip_ops.gemm(x, wr, out_f32=True)
    ids, w = hip_ops.route_topk(logits, k)
    pk = hip_ops.pack_index(ids, C, w)
    P = T * k
    ug = torch.empty(P, 2 * n, device=dev, dtype=bf)
    zw = torch.empty(P, n, device=dev, dtype=bf)
    yp = torch.empty(P, d, device=dev, dtype=bf)
    head_out = torch.empty(T, V, device=dev, dtype=torch.float32)
    st = _lib.stream_ptr
    lib = _lib.load()

    def gemm(a, lda, a_t, b, ldb, b_t, c, ldc, M, N, K, ws=None, wsb=0):
        _lib.call("rte_gemm_bf16", a.data_ptr(), lda, a_t, None, b.data_ptr(), ldb, b_t, None, c.data_ptr(), ldc, 1, M,
                  N, K, 1.0, 0.0, None, 0, None if ws is None else ws.data_ptr(), wsb, st())

    def head():
        gemm(x, d, 0, w_head, d, 0, head_out, V, T, V, d)

    def qkv():
        _lib.call("rte_qkv_rope_fwd", x.data_ptr(), wqkv.data_ptr(), cos.data_ptr(), sin.data_ptr(), B, S, 8, 64,
                  q.data_ptr(), kk.data_ptr(), vv.data_ptr(), None, 0, st())

    def split_ws(M, N, K):
        nb = lib.rte_gemm_workspace_bytes(M, N, K)
        return torch.empty(max(nb, 16), device=dev, dtype=torch.uint8), nb

    dqkv = torch.randn(T, 3 * d, device=dev, generator=g).to(bf)
    dw_qkv = torch.empty(3 * d, d, device=dev, dtype=torch.float32)
    ws_q, wsb_q = split_ws(3 * d, d, T)

    def wgrad_qkv():
        # dW_qkv[c, :] = sum_t dqkv[t, c] x[t, :]  (both operands token-major: layout T, split-K)
        gemm(dqkv, 3 * d, 1, x, d, 1, dw_qkv, d, 3 * d, d, T, ws_q, wsb_q)

    dlog = (torch.randn(T, V, device=dev, generator=g) * 0.01).to(bf)
    dx_head = torch.empty(T, d, device=dev, dtype=torch.float32)
    dw_head = torch.empty(V, d, device=dev, dtype=torch.float32)
    ws_h, wsb_h = split_ws(V, d, T)

    def head_dx():
        # dX = dlogits @ W  (W [V, d]: column index contiguous, layout T)
        gemm(dlog, V, 0, w_head, d, 1, dx_head, d, T, d, V)

    def head_wgrad():
        gemm(dlog, V, 1, x, d, 1, dw_head, d, V, d, T, ws_h, wsb_h)

    # the entry points the step's pools call: the fused per-cluster kernels where the shape allows
    fused = bool(lib.rte_grouped_swiglu_fused_ok(n, d))
    ffn_fwd_name = "rte_grouped_swiglu_fused_fwd" if fused else "rte_grouped_swiglu_fwd"
    ffn_bwd_name = "rte_grouped_swiglu_fused_bwd" if fused else "rte_grouped_swiglu_bwd"

    def ffn_fwd():
        _lib.call(ffn_fwd_name, x.data_ptr(), T, d, pk.offsets.data_ptr(), C, n, P,
                  pk.tok_of_slot.data_ptr(), pk.pair_of_slot.data_ptr(), pk.w_of_slot.data_ptr(), wug.data_ptr(),
                  wd.data_ptr(), F, ug.data_ptr(), zw.data_ptr(), yp.data_ptr(), st())

    ffn_fwd()
    dpool = (torch.randn(T, d, device=dev, generator=g) * 0.01).to(bf)
    dug = torch.empty(P, 2 * n, device=dev, dtype=bf)
    dw_slot = torch.empty(P, device=dev, dtype=torch.float32)
    dx_pairs = torch.empty(P, d, device=dev, dtype=bf)
    dwug = torch.empty(2 * F, d, device=dev, dtype=torch.float32)
    dwd = torch.empty(d, F, device=dev, dtype=torch.float32)
    gsb = lib.rte_grouped_swiglu_bwd_workspace_bytes(P, C, n, d)
    gs_ws = torch.empty(max(gsb, 16), device=dev, dtype=torch.uint8)

    def ffn_bwd():
        _lib.call(ffn_bwd_name, dpool.data_ptr(), x.data_ptr(), T, d, pk.offsets.data_ptr(), C, n, P,
                  pk.tok_of_slot.data_ptr(), pk.pair_of_slot.data_ptr(), pk.w_of_slot.data_ptr(), wug.data_ptr(),
                  wd.data_ptr(), F, ug.data_ptr(), zw.data_ptr(), dug.data_ptr(), dw_slot.data_ptr(),
                  dx_pairs.data_ptr(), dwug.data_ptr(), dwd.data_ptr(), 0, 0.0, gs_ws.data_ptr(), gsb, st())

    out_pool = torch.empty(T, d, device=dev, dtype=torch.float32)

    def combine():
        _lib.call("rte_combine_rows", yp.data_ptr(), T, k, d, None, None, None, out_pool.data_ptr(), 1, st())

    ids_out = torch.empty(T, k, device=dev, dtype=torch.int32)
    w_out = torch.empty(T, k, device=dev, dtype=torch.float32)

    def topk():
        _lib.call("rte_route_topk", logits.data_ptr(), T, C, k, ids_out.data_ptr(), w_out.data_ptr(), st())

    rp_ws_bytes = lib.rte_route_pack_workspace_bytes(T, C)
    rp_ws = torch.empty(max(rp_ws_bytes, 16), device=dev, dtype=torch.uint8)
    rp_ids = torch.empty(T, k, device=dev, dtype=torch.int32)
    rp_w = torch.empty(T, k, device=dev, dtype=torch.float32)
    rp_out = [torch.empty(P, device=dev, dtype=torch.int32) for _ in range(3)]
    rp_off = torch.empty(C + 1, device=dev, dtype=torch.int32)
    rp_wos = torch.empty(P, device=dev, dtype=torch.float32)

    def route_pack():
        _lib.call("rte_route_pack", x.data_ptr(), T, d, wr.data_ptr(), C, k, rp_ids.data_ptr(), rp_w.data_ptr(),
                  rp_off.data_ptr(), rp_out[0].data_ptr(), rp_out[1].data_ptr(), rp_out[2].data_ptr(),
                  rp_wos.data_ptr(), None, rp_ws.data_ptr(), rp_ws_bytes, st())

    pk_ws_bytes = lib.rte_pack_workspace_bytes(P, C)
    pk_ws = torch.empty(max(pk_ws_bytes, 16), device=dev, dtype=torch.uint8)
    pk_out = [torch.empty(P, device=dev, dtype=torch.int32) for _ in range(4)]
    pk_off = torch.empty(C + 1, device=dev, dtype=torch.int32)
    pk_w = torch.empty(P, device=dev, dtype=torch.float32)

    def pack():
        _lib.call("rte_pack_index", ids.data_ptr(), P, C, k, w.data_ptr(), pk_off.data_ptr(), pk_out[0].data_ptr(),
                  pk_out[1].data_ptr(), pk_out[2].data_ptr(), pk_w.data_ptr(), None, pk_ws.data_ptr(), pk_ws_bytes,
                  st())

    # macro consistency loss (both operator applications, MSE, backward, weight gradients): the
    # cfg3 operator tables (16 recipes x 3 strides, rank 32) over the whole batch's h0
    R3, K3, r = 16, 3, 32
    mv = (torch.randn(R3, K3, 3 * d, r, device=dev, generator=g) / (3 * d) ** 0.5).requires_grad_()
    mu = (torch.randn(R3, K3, r, d, device=dev, generator=g) * 0.05).requires_grad_()
    mg = (torch.randn(R3, K3, d, device=dev, generator=g) * 0.1).requires_grad_()
    mb = (torch.randn(R3, K3, d, device=dev, generator=g) * 0.1).requires_grad_()
    ms = torch.ones(R3, K3, d, device=dev)
    mh = torch.randn(B, S, d, device=dev, generator=g).requires_grad_()
    rid = torch.randint(0, R3, (B,), device=dev, generator=g)
    # the first application's keys: the union of the strides, src = blocks [0, 2), dst = [1, 3); the
    # second application's (the src blocks) right after them in one tensor, as the model makes them
    kall = (rid * K3).repeat(5) + torch.tensor([0, 1, 2, 0, 1], device=dev).repeat_interleave(B)
    kf, ks = kall[:3 * B], kall[3 * B:]

    def macro_cons():
        loss = hip_ops.macro_consistency(mh, kf, ks, mv, mu, mg, mb, ms, 0.1, src_lo=0, dst_lo=1)
        torch.autograd.grad(loss, [mh, mv, mu, mg, mb])

    # bytes of the consistency loss on the one-pass kernels (csrc/macro_cons.hip), nf = 3 first-
    # application key blocks and pc = 2 pairs over T rows: h read by each of the 6 kernels; x2
    # ([rmsnorm | h] bf16, 4d bytes per row) written for the 1 + pc inputs and read once by the
    # weight reductions; du (bf16) written per (key, row) and read once; dh written, read and
    # rewritten; the rank-32 codes a (fp32) / silu(a) / da (bf16) written and read; the fp32
    # weights read by the two bf16 weight preparations and their gradients written.
    rows_both, rows_tw = 3 * T, 2 * T
    f4, b2 = 4.0 * d, 2.0 * d
    nf, pc, G3 = 3, 2, R3 * K3
    wbytes = G3 * (3 * d * r + r * d) * 4.0
    macro_bytes = (6 * T * f4 + 2 * (1 + pc) * T * 2 * b2 + 2 * (nf + pc) * T * b2 + 3 * T * f4
                   + 2 * (nf + pc) * T * r * (4 + 2 + 2) + 3 * wbytes)
    # the operation's essential I/O: h in, dh out, the tables (V, U, gain, bias, scale) in and
    # their gradients out
    macro_essential = 2 * T * f4 + 2 * (wbytes + 3 * G3 * d * 4.0)
    macro_flop = (rows_both + rows_tw) * 2.0 * (2 * d * r + r * d) * 3

    return [
        dict(name="gemm_qkv_rope_fwd", per_step=2, kernels=1, flop=2.0 * T * 3 * d * d,
             bytes=2.0 * T * d + 2.0 * 3 * d * d + 3 * 2.0 * T * d, fn=qkv),
        dict(name="gemm_lm_head_fwd", per_step=1, kernels=1, flop=2.0 * T * V * d,
             bytes=2.0 * T * d + 2.0 * V * d + 4.0 * T * V, fn=head),
        dict(name="gemm_lm_head_dx", per_step=1, kernels=1, flop=2.0 * T * V * d,
             bytes=2.0 * T * V + 2.0 * V * d + 4.0 * T * d, fn=head_dx),
        dict(name="gemm_lm_head_wgrad", per_step=1, kernels=2, flop=2.0 * T * V * d,
             bytes=2.0 * T * V + 2.0 * T * d + 4.0 * V * d, fn=head_wgrad),
        dict(name="gemm_wgrad_qkv", per_step=2, kernels=2, flop=2.0 * T * 3 * d * d,
             bytes=2.0 * T * 3 * d + 2.0 * T * d + 4.0 * 3 * d * d, fn=wgrad_qkv),
        # x@[Wup|Wgate]^T, SwiGLU, zw@Wdown into pair-major rows (one fused launch at n = 32)
        dict(name="grouped_swiglu_fwd", per_step=2, kernels=1 if fused else 2, flop=2.0 * P * d * 2 * n + 2.0 * P * n * d,
             bytes=2.0 * T * d + 2.0 * 3 * F * d + 2.0 * P * 3 * n + 2.0 * P * d + 12.0 * P, fn=ffn_fwd),
        # backward: dZ / dW_down, SwiGLU derivative, dX-pairs / dW_up|gate; reads x, dout, weights,
        # ug, zw, slot tables; writes dug, dw_slot, dx_pairs and the fp32 weight gradients
        dict(name="grouped_swiglu_bwd", per_step=2, kernels=None, flop=2.0 * (2.0 * P * d * 2 * n + 2.0 * P * n * d),
             bytes=2.0 * T * d * 2 + 2.0 * 3 * F * d + 2.0 * P * 3 * n + 12.0 * P + 2.0 * P * 2 * n + 4.0 * P
             + 2.0 * P * d + 4.0 * 3 * F * d, fn=ffn_bwd),
        # combine unit: T*k*d*b + T*k*4 + T*d*b (bf16 rows in, fp32 rows out here)
        dict(name="combine_rows", per_step=2, kernels=1, flop=1.0 * P * d,
             bytes=2.0 * P * d + 4.0 * T * d, fn=combine),
        # router GEMM + top-k + pack (the step's routing): x and Wr in, ids + weights (8 B per pair)
        # and the slot tables (4 int32 + 1 fp32 per pair) out; the per-block cluster counts (T / 32 x C
        # int32) written and read once
        dict(name="route_pack", per_step=1, kernels=2, flop=2.0 * T * C * d,
             bytes=2.0 * T * d + 2.0 * C * d + 8.0 * P + 20.0 * P + 4.0 * (C + 1) + 8.0 * (T // 32) * C,
             fn=route_pack),
        # the standalone entry points (not in the cfg3 step, which routes through route_pack):
        # route unit: T*C*4 logits in, T*k*(4+4) ids + weights out
        dict(name="route_topk", per_step=0, kernels=1, flop=0.0, bytes=4.0 * T * C + 8.0 * T * k, fn=topk),
        # pack unit: P*(4+4) ids + weights in, 4*P*4 + P*4 slot tables out, (C+1)*4 offsets
        dict(name="pack_index", per_step=0, kernels=3, flop=0.0, bytes=8.0 * P + 20.0 * P + 4.0 * (C + 1),
             fn=pack),
        dict(name="macro_consistency_fwd_bwd", per_step=1, kernels=None, flop=macro_flop, bytes=macro_bytes,
             essential_bytes=macro_essential, fn=macro_cons),
    ]


def svd_cfg4_candidate(T: int = 32768):
    """the SVD low-rank FFN forward + backward (d 1024, F 4096, rank 128
    factors U diag(S) V^T for up / gate / down, S log-uniform in [1e-2, 1], U and V orthonormal from
    a seeded QR) over T tokens, as one autograd call of hip_ops.svd_ffn plus its backward."""
    import torch

    from rte_amd.kernels import hip_ops

    dev = "cuda"
    d, F, r = 1024, 4096, 128
    g = torch.Generator()
    g.manual_seed(3)

    def orth(a, b):
        return torch.linalg.qr(torch.randn(a, b, generator=g))[0]

    def svals():
        return 10.0 ** (torch.rand(r, generator=g) * 2.0 - 2.0)

    us_ug = torch.cat([orth(d, r) * svals(), orth(d, r) * svals()], 1).to(dev).requires_grad_()
    v_ug = torch.cat([orth(F, r), orth(F, r)], 0).to(dev).requires_grad_()
    v_dn = orth(F, r).to(dev).requires_grad_()
    us_dn = (orth(d, r) * svals()).to(dev).requires_grad_()
    x = torch.randn(T, d, generator=g).to(dev).to(torch.bfloat16).requires_grad_()
    dy = torch.randn(T, d, generator=g).to(dev)
    params = [x, us_ug, v_ug, v_dn, us_dn]

    def fn():
        y = hip_ops.svd_ffn(x, us_ug, v_ug, v_dn, us_dn)
        torch.autograd.grad(y, params, dy)

    # fwd 2T(d 2r + 2F r + F r + r d) FLOP, backward twice that; bytes: x, dy, dx (bf16), y (fp32),
    # the four factors read (fp32) and their gradients written (fp32)
    fwd = 2.0 * T * (d * 2 * r + 2 * F * r + F * r + r * d)
    wbytes = 4.0 * (d * 2 * r + 2 * F * r + F * r + d * r)
    return dict(name="svd_ffn_cfg4_fwd_bwd", per_step=0, kernels=None, flop=3.0 * fwd,
                bytes=2.0 * T * d * 3 + 4.0 * T * d + 2.0 * wbytes, fn=fn, T=T, d=d, F=F, r=r)


def svd_cfg4_row(iters: int = 5) -> dict:
    """Roofline line of the cfg4 SVD FFN forward + backward (not part of the cfg3 step)."""
    c = svd_cfg4_candidate()
    dt = time_launches(c["fn"], iters)
    tf = c["flop"] / dt / 1e12
    return {"workload": "SVD low-rank FFN fwd+bwd (BASELINE configs[3]): T 32768, d 1024, F 4096, rank 128",
            "avg_us": round(dt * 1e6, 1), "bound": "mfma", "achieved": round(tf, 1), "unit": "TFLOP/s",
            "peak": PEAK_BF16_TFLOPS, "frac": round(tf / PEAK_BF16_TFLOPS, 4), "flop": c["flop"],
            "algorithmic_bytes": c["bytes"], "tokens_per_s": round(c["T"] / dt, 1)}


def time_launches(fn, iters: int = 20) -> float:
    """Average duration (s) of one fn() call: `iters` calls captured in a HIP graph and
    replayed, timed with HIP events on the replaying stream (no host launch gaps)."""
    import torch

    fn()
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        fn()
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for _ in range(iters):
            fn()
    graph.replay()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    reps = 5
    start.record()
    for _ in range(reps):
        graph.replay()
    end.record()
    end.synchronize()
    return start.elapsed_time(end) / 1e3 / (iters * reps)


def roofline_rows(B: int, S: int) -> list[dict]:
    rows = []
    for c in kernel_candidates(B, S):
        dt = time_launches(c["fn"])
        t_mfma, t_hbm = c["flop"] / (PEAK_BF16_TFLOPS * 1e12), c["bytes"] / (PEAK_HBM_GBS * 1e9)
        bound = "mfma" if t_mfma >= t_hbm else "hbm"
        ach = c["flop"] / dt / 1e12 if bound == "mfma" else c["bytes"] / dt / 1e9
        peak = PEAK_BF16_TFLOPS if bound == "mfma" else PEAK_HBM_GBS
        rows.append({"kernel": c["name"], "launches_per_step": c["per_step"], "kernels_per_call": c["kernels"],
                     "avg_us": round(dt * 1e6, 2), "us_per_step": round(dt * 1e6 * c["per_step"], 1),
                     "bound": bound, "achieved": round(ach, 1),
                     "unit": "TFLOP/s" if bound == "mfma" else "GB/s", "peak": peak, "frac": round(ach / peak, 4),
                     "flop": c["flop"], "bytes": c["bytes"],
                     "tflops": round(c["flop"] / dt / 1e12, 1), "gbs": round(c["bytes"] / dt / 1e9, 1)})
        if c.get("essential_bytes"):
            rows[-1]["essential_bytes"] = c["essential_bytes"]
            rows[-1]["essential_frac"] = round(c["essential_bytes"] / dt / 1e9 / PEAK_HBM_GBS, 4)
    rows.sort(key=lambda r: -r["us_per_step"])
    return rows


def _pmc_per_call(csv_dir: Path, counter: str, calls: int, only=None):
    """Sum of `counter` over the profiled calls' dispatches / calls, in bytes (KiB counters), read
    from rocprofv3's counter_collection.csv; `only` filters kernel names, and kernels dispatched
    fewer than `calls` times (the candidates' set-up work) are left out.  `only` takes the CSV row."""
    import csv
    from collections import defaultdict

    files = sorted(csv_dir.rglob("*counter_collection.csv"))
    if not files:
        return None
    tot, n = defaultdict(float), defaultdict(int)
    with open(files[0]) as fh:
        for r in csv.DictReader(fh):
            if r.get("Counter_Name") != counter:
                continue
            k = r.get("Kernel_Name", "")
            if only is not None and not only(r):
                continue
            tot[k] += float(r["Counter_Value"])
            n[k] += 1
    return sum(v for k, v in tot.items() if n[k] >= calls) * 1024.0 / calls


COPY_ELEMS = 64 << 20  # calibration: rte_cast_f32_bf16 over 64 Mi elements (reads 256 MiB, writes 128 MiB)


def _is_copy(r: dict) -> bool:
    """A counter row of the calibration copy: the cast kernel at the calibration size (its launch
    runs one thread per 4 elements), told apart from casts the profiled operation makes itself."""
    return "cast_f32_bf16" in r.get("Kernel_Name", "") and int(r.get("Grid_Size", "0") or 0) == COPY_ELEMS // 4


def measure_traffic(name: str, B: int, S: int, iters: int = 20, timeout_s: int = 120) -> dict:
    """HBM bytes per call of candidate `name`, from two rocprofv3 --pmc runs of this script in
    --profile-kernel mode (FETCH_SIZE, then WRITE_SIZE), each scaled by what the same counter
    reads for the calibration copy kernel of known size.  Returns {"bytes": ..., ...} or
    {"bytes": None, "note": why}."""
    import shutil
    import subprocess
    import tempfile

    prof = shutil.which("rocprofv3") or "/opt/rocm/bin/rocprofv3"
    if not Path(prof).exists():
        return {"bytes": None, "note": "rocprofv3 not found"}
    out = {}
    tmp = Path(tempfile.mkdtemp(prefix="rte_pmc_"))
    try:
        for counter in ("FETCH_SIZE", "WRITE_SIZE"):
            d = tmp / counter
            cmd = [prof, "--pmc", counter, "-d", str(d), "-o", "p", "--output-format", "csv", "--",
                   sys.executable, str(ROOT / "bench.py"), "--profile-kernel", name, "--with-copy", "--iters",
                   str(iters), "--batch", str(B), "--seq", str(S)]
            r = subprocess.run(cmd, capture_output=True, text=True, timeout=timeout_s, cwd=str(ROOT))
            if r.returncode != 0:
                return {"bytes": None, "note": f"rocprofv3 --pmc {counter} exited {r.returncode}"}
            op = _pmc_per_call(d, counter, iters, lambda r: not _is_copy(r))
            cp = _pmc_per_call(d, counter, iters, _is_copy)
            known = COPY_ELEMS * (4.0 if counter == "FETCH_SIZE" else 2.0)
            if not op or not cp:
                return {"bytes": None, "note": f"no {counter} rows in the rocprofv3 output"}
            out[counter] = (op, known / cp)
    except subprocess.TimeoutExpired:
        return {"bytes": None, "note": "rocprofv3 --pmc run timed out"}
    finally:
        shutil.rmtree(tmp, ignore_errors=True)
    fetch = out["FETCH_SIZE"][0] * out["FETCH_SIZE"][1]
    write = out["WRITE_SIZE"][0] * out["WRITE_SIZE"][1]
    return {"bytes": round(fetch + write), "fetch": round(fetch), "write": round(write),
            "fetch_scale": round(out["FETCH_SIZE"][1], 4), "write_scale": round(out["WRITE_SIZE"][1], 4)}


def profile_kernel(name: str, iters: int, B: int, S: int, with_copy: bool = False) -> int:
    """Launch one candidate `iters` times (the program rocprofv3 --pmc profiles); with_copy (or
    name 'copy') also launches the calibration copy kernel `iters` times."""
    import torch

    from rte_amd import _lib

    if name != "copy":
        cands = {c["name"]: c for c in
                 ([svd_cfg4_candidate()] if name == "svd_ffn_cfg4_fwd_bwd" else kernel_candidates(B, S))}
        torch.cuda.synchronize()
        for _ in range(iters):
            cands[name]["fn"]()
    if with_copy or name == "copy":
        src = torch.randn(COPY_ELEMS, device="cuda")
        dst = torch.empty(COPY_ELEMS, device="cuda", dtype=torch.bfloat16)
        torch.cuda.synchronize()
        for _ in range(iters):
            _lib.call("rte_cast_f32_bf16", src.data_ptr(), COPY_ELEMS, dst.data_ptr(), _lib.stream_ptr())
    torch.cuda.synchronize()
    print(json.dumps({"profiled": name, "iters": iters}))
    return 0


def _kernel_family(name: str) -> str:
    base = name[5:] if name.startswith("void ") else name
    if base.startswith("rte::"):
        return "rte (HIP, this library)"
    if "Cijk_" in base:
        return "hipBLASLt / rocBLAS"
    if base.startswith("at::"):
        return "torch"
    return "other"


def _short_kernel(name: str, width: int = 110) -> str:
    base = name[5:] if name.startswith("void ") else name
    base = base.replace("(anonymous namespace)::", "")
    if base.startswith("rte::"):
        base = base.split("(", 1)[0]
    return base if len(base) <= width else base[: width - 3] + "..."


def trace_summary(csv_path: str, steps: int, top: int = 40) -> str:
    """Markdown report of a rocprofv3 --kernel-trace CSV of a bench.py run whose last dispatches
    are `steps` identical step replays: the dispatches of one step (found as the shortest period
    that repeats `steps` times at the end of the trace), their time by kernel family and the
    kernels that take the most time per step."""
    import csv
    from collections import defaultdict

    with open(csv_path) as fh:
        rows = [(int(r["Dispatch_Id"]), int(r["Start_Timestamp"]), int(r["End_Timestamp"]), r["Kernel_Name"])
                for r in csv.DictReader(fh)]
    rows.sort()  # dispatch order: fixed within a graph replay, whatever order parallel branches run in
    names = [r[3] for r in rows]
    n = len(names)
    period = None
    for p in range(1, n // max(steps, 1) + 1):
        tail = names[n - p * steps:]
        if all(tail[i] == tail[i % p] for i in range(len(tail))):
            period = p
            break
    if period is None:
        raise ValueError(f"no period repeating {steps} times at the end of {csv_path}")
    step_rows = rows[n - period * steps:]
    fam_us, fam_n, k_us, k_n = defaultdict(float), defaultdict(int), defaultdict(float), defaultdict(int)
    for _, s, e, k in step_rows:
        us = (e - s) / 1e3 / steps
        fam_us[_kernel_family(k)] += us
        fam_n[_kernel_family(k)] += 1
        k_us[k] += us
        k_n[k] += 1
    busy = sum(fam_us.values())
    wall = (max(r[2] for r in step_rows) - min(r[1] for r in step_rows)) / 1e3 / steps
    out = [f"Dispatches per step: {period}; kernel time per step {busy:.1f} us (sum of kernel durations, mean "
           f"over the last {steps} replays; first-start to last-end span under the tracer {wall:.1f} us per step).",
           "",
           "| family | dispatches / step | us / step | % of kernel time |", "|---|---:|---:|---:|"]
    for f in sorted(fam_us, key=lambda f: -fam_us[f]):
        out.append(f"| {f} | {fam_n[f] // steps} | {fam_us[f]:.1f} | {100 * fam_us[f] / busy:.1f} |")
    out += ["", f"Top {top} kernels by time per step:", "",
            "| us / step | dispatches / step | avg us | kernel |", "|---:|---:|---:|---|"]
    for k in sorted(k_us, key=lambda k: -k_us[k])[:top]:
        c = k_n[k] // steps
        out.append(f"| {k_us[k]:.1f} | {c} | {k_us[k] / max(c, 1):.1f} | `{_short_kernel(k)}` |")
    return "\n".join(out)


def pmc_summary(csv_dir: str, calls: int) -> str:
    """Markdown table of every counter in a rocprofv3 --pmc run's counter_collection.csv, summed
    per kernel over its dispatches and divided by `calls` (the --iters of a --profile-kernel run)."""
    import csv
    from collections import defaultdict

    files = sorted(Path(csv_dir).rglob("*counter_collection.csv"))
    if not files:
        raise FileNotFoundError(f"no counter_collection.csv under {csv_dir}")
    tot, disp = defaultdict(float), defaultdict(set)
    copy_name = "calibration copy (cast_f32_bf16, 64 Mi elements)"
    for f in files:
        with open(f) as fh:
            for r in csv.DictReader(fh):
                name = copy_name if _is_copy(r) else r["Kernel_Name"]
                tot[(name, r["Counter_Name"])] += float(r["Counter_Value"])
                disp[name].add((str(f), r.get("Dispatch_Id", r.get("Correlation_Id", ""))))
    out = [f"Per call (raw counters: sums over a kernel's dispatches / {calls} calls; derived ratios: mean per "
           "dispatch; kernels dispatched less than once per call, i.e. set-up work, are left out):", "",
           "| kernel | dispatches / call | counter | value / call |", "|---|---:|---|---:|"]
    for (k, c) in sorted(tot):
        if len(disp[k]) < calls:
            continue
        # raw counters (upper case) add up over a call's dispatches; derived ratios (MfmaUtil, ...)
        # are averaged over the dispatches
        v = tot[(k, c)] / calls if c.upper() == c else tot[(k, c)] / len(disp[k])
        out.append(f"| `{_short_kernel(k, 80)}` | {len(disp[k]) / calls:g} | {c} | {v:.6g} |")
    for c, per_elem in (("FETCH_SIZE", 4.0), ("WRITE_SIZE", 2.0)):
        keys = [k for (k, cc) in tot if cc == c and len(disp[k]) >= calls]
        if not keys:
            continue
        op = sum(tot[(k, c)] for k in keys if k != copy_name) * 1024.0 / calls
        cp = sum(tot[(k, c)] for k in keys if k == copy_name) * 1024.0 / calls
        line = f"{c}: operation kernels {op:.4g} B per call (counter KiB x 1024)"
        if cp:
            scale = COPY_ELEMS * per_elem / cp
            line += (f"; calibration copy counted {cp:.4g} B for a known {COPY_ELEMS * per_elem:.4g} B -> scale "
                     f"{scale:.4f}; operation {op * scale:.4g} B per call")
        out += ["", line]
    return "\n".join(out)


def _cpu_model() -> str:
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def _cpu_threads() -> tuple[int, int]:
    """(threads used, os.cpu_count()): the host cores this process may use -- its CPU affinity,
    capped by OMP_NUM_THREADS when the box sets it to this job's share of the host."""
    total = os.cpu_count() or 1
    try:
        avail = len(os.sched_getaffinity(0))
    except AttributeError:
        avail = total
    omp = int(os.environ.get("OMP_NUM_THREADS", "0") or 0)
    return (min(avail, omp) if omp > 0 else avail), total


def _median_time(fn, warmup: int, iters: int) -> float:
    for _ in range(warmup):
        fn()
    ts = []
    for _ in range(iters):
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
    return statistics.median(ts)


def cpu_baseline(step_budget_s: float = 16.0, warmup: int = 2, iters: int = 10) -> dict:
    """The reference's CPU path, timed on the host cores (median of `iters` timed runs after
    `warmup` untimed ones, rte/cli.py:7755-7760): the cfg3 recursive_macro train step restated in
    float32 torch (oracle/step_port.py: forward, exact replay of the audited sample with the
    control-variate correction, consistency and distillation terms, backward, AdamW) on a batch
    sample sized so the timed steps take about step_budget_s (rows are independent), and the
    cfg1 cluster-pool layer forward + backward in both of the reference's forms
    (oracle/pool_port.py: per-cluster loop and preindexed bmm) at its full size."""
    import torch

    import rte_amd.models as RM
    from oracle import pool_port as PP
    from oracle import step_port as SP

    threads, total = _cpu_threads()
    torch.set_num_threads(threads)
    S = 64

    def make(B):
        cfg = cfg3_config(batch=B, seq=S)
        torch.manual_seed(cfg.training.seed)
        m = RM.RecursiveModel(cfg.model, cfg.output)
        port = SP.StepPort(cfg, dict(m.named_parameters()), dict(m.named_buffers()))
        opt = SP.make_optimizer(port)
        tok, tgt = SP.zipf_tokens(cfg.model.vocab_size, B, S, seed=1)
        usage = torch.zeros(cfg.model.recipe_count)
        chosen = torch.zeros(1, dtype=torch.long)
        return lambda: SP.train_step(port, opt, tok, tgt, chosen=chosen, usage_ema=usage)

    probe = make(8)
    probe()
    t0 = time.perf_counter()
    probe()
    per_sample = (time.perf_counter() - t0) / 8
    B = int(max(8, min(128, step_budget_s / iters / max(per_sample, 1e-9))))
    step_s = _median_time(make(B), warmup, iters)
    x, wr, wup, wgate, wdown = PP.make_cfg1()
    dy = torch.randn(x.shape, generator=torch.Generator().manual_seed(1))
    layer = {}
    for name, form in (("loop", PP.layer_loop), ("preindexed", PP.layer_preindexed)):
        t = _median_time(lambda: PP.fwd_bwd(form, x, wr, wup, wgate, wdown, dy, 4, 32), warmup, iters)
        layer[name] = {"tokens_per_s": round(x.shape[0] / t, 1), "ms": round(t * 1e3, 2)}
    return {
        "value": round(B * S / step_s, 1),
        "unit": "tokens/s",
        "cores": threads,
        "kind": "port",
        "cpu": _cpu_model(),
        "host_cpu_count": total,
        "sample": (f"fp32 torch-CPU restatement of the cfg3 recursive_macro step (oracle/step_port.py), batch {B} of "
                   f"128 x seq {S} (rows independent), median of {iters} timed steps after {warmup} warm-ups; "
                   f"{threads} threads (this job's share of the host's {total})"),
        "cfg1_layer": {"workload": "BASELINE configs[0]: cluster-pool SwiGLU layer fwd+bwd, T 8192, d 256, "
                                  "32 x 32 neurons, top-4, fp32 (oracle/pool_port.py)",
                       "median_of": iters, **layer},
    }


def main(argv=None) -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--batch", type=int, default=128)
    ap.add_argument("--seq", type=int, default=64)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-roofline", action="store_true")
    ap.add_argument("--profile-kernel", default=None,
                    help="only launch this roofline candidate (or 'copy', the calibration kernel) --iters times")
    ap.add_argument("--iters", type=int, default=50)
    ap.add_argument("--with-copy", action="store_true", help="--profile-kernel: also launch the calibration copy")
    ap.add_argument("--no-traffic", action="store_true", help="skip the rocprofv3 --pmc traffic runs")
    ap.add_argument("--eager", action="store_true",
                    help="launch every kernel from Python instead of replaying the captured step graph")
    ap.add_argument("--trace-summary", default=None, metavar="CSV",
                    help="print the per-step breakdown of a rocprofv3 kernel-trace CSV of a bench.py run whose "
                         "last --steps dispatch groups are the timed steps, then exit (no GPU)")
    ap.add_argument("--pmc-summary", default=None, metavar="DIR",
                    help="print the counters of a rocprofv3 --pmc run of --profile-kernel per call (--iters "
                         "calls), then exit (no GPU)")
    args = ap.parse_args(argv)
    if args.trace_summary:
        print(trace_summary(args.trace_summary, args.steps))
        return 0
    if args.pmc_summary:
        print(pmc_summary(args.pmc_summary, args.iters))
        return 0
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print(json.dumps({"error": "this build measures one GPU only; run bench.py with --gpus 1"}))
        return 2

    import torch

    from rte_amd import _lib
    from rte_amd.training import TrainEngine

    if not _lib.device_ready():
        print(json.dumps({"error": "HIP backend unavailable (librte_hip.so not built or no gfx950 device)"}))
        return 1
    if args.profile_kernel:
        return profile_kernel(args.profile_kernel, args.iters, args.batch, args.seq, args.with_copy)
    cfg = cfg3_config(args.batch, args.seq)
    dev = torch.device("cuda:0")
    engine = TrainEngine(cfg, device=dev)
    if not args.eager:
        # the whole step (forward, audit replay, backward, AdamW) replays as one HIP graph; the
        # first two warm-up steps run eagerly and the third captures it
        engine.enable_graph_capture(True)
        args.warmup = max(args.warmup, 3)
    gen = torch.Generator()
    gen.manual_seed(cfg.training.seed)
    batches = [zipf_batch(gen, cfg.model.vocab_size, args.batch, args.seq, dev) for _ in range(4)]
    for i in range(args.warmup):
        engine.train_step(batches[i % len(batches)])
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(args.steps):
        engine.train_step(batches[i % len(batches)])
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    tokens = args.steps * args.batch * args.seq
    value = tokens / elapsed

    out = {
        "metric": METRIC,
        "value": round(value, 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(elapsed / args.steps * 1e3, 3),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded Zipf(1.1) token ids, random-init weights)",
        "config": {
            "workload": "recursive_macro train step (BASELINE configs[2]): d512 h8, prelude+coda FFN = routed "
                        "cluster pool 64x32 top-8, banked core 64 slabs x32 (8 active), depth 4, V2048, "
                        "fixed-count audit 1/128, AdamW",
            "global_batch": args.batch,
            "seq_len": args.seq,
            "parallelism": "single GPU",
            "launch": "eager" if args.eager else "captured step graph",
        },
    }
    if not args.no_roofline:
        rows = roofline_rows(args.batch, args.seq)  # sorted by time per step
        dom = rows[0]
        traffic = measure_traffic(dom["kernel"], args.batch, args.seq) if not args.no_traffic else {
            "bytes": None, "note": "--no-traffic"}
        out["roofline"] = {
            "kernel": dom["kernel"],
            "bound": dom["bound"],
            "achieved": dom["achieved"],
            "peak": dom["peak"],
            "unit": dom["unit"],
            "frac": dom["frac"],
            "traffic": traffic["bytes"],
            "traffic_detail": traffic,
            "avg_us": dom["avg_us"],
            "us_per_step": dom["us_per_step"],
            "flop_per_launch": dom["flop"],
            "algorithmic_bytes_per_launch": dom["bytes"],
        }
        if "essential_bytes" in dom:
            out["roofline"]["essential_bytes_per_launch"] = dom["essential_bytes"]
            out["roofline"]["essential_frac"] = dom["essential_frac"]
        out["kernels"] = rows
        out["svd_ffn_cfg4"] = svd_cfg4_row()
    if not args.no_cpu_baseline:
        out["cpu_baseline"] = cpu_baseline()
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
