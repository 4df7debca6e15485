"""Benchmark: recursive_macro bf16 train step on one MI355X.

Workload (cfg3): RecursiveModel d_model 512, 8 heads, prelude + coda blocks whose FFN is a
routed cluster pool of 64 clusters x 32 neurons (top-8 per token), banked recursive core
with 64 slabs x 32 (8 active), t_max = fixed depth 4, vocab 2048 tied head, batch 128 x
seq 64, token ids Zipf(1.1), fixed-count audit of 1 sample (p = 1/128), AdamW.  Synthetic
seeded data, random-init weights.  One step = forward_macro + audit correction + backward
+ AdamW, exactly TrainEngine.train_step.

Prints ONE JSON line.  Also reports the roofline of the dominant kernel (timed live with
HIP events on the launch stream) and a CPU baseline (the numpy oracle of the cluster-pool
SwiGLU layer, BASELINE.json configs[0], on a bounded token sample, this host's cores).
"""

from __future__ import annotations

import argparse
import json
import os
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
    """Hot kernels of the step at their cfg3 shapes.  Each entry: name, launches per step,
    kernels per call, algorithmic flop and HBM bytes per call (inputs read once, outputs
    written once), and fn launching it on the current stream."""
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

    def head():
        _lib.call("rte_gemm_bf16", x.data_ptr(), d, 0, None, w_head.data_ptr(), d, 0, None, head_out.data_ptr(), V,
                  1, T, V, d, 1.0, 0.0, None, 0, None, 0, st())

    def qkv():
        _lib.call("rte_qkv_rope_fwd", x.data_ptr(), wqkv.data_ptr(), cos.data_ptr(), sin.data_ptr(), B, S, 8, 64,
                  q.data_ptr(), kk.data_ptr(), vv.data_ptr(), st())

    dqkv = torch.randn(T, 3 * d, device=dev, generator=g).to(bf)
    dw_qkv = torch.empty(3 * d, d, device=dev, dtype=torch.float32)
    ws_bytes = _lib.load().rte_gemm_workspace_bytes(3 * d, d, T)
    ws = torch.empty(max(ws_bytes, 16), device=dev, dtype=torch.uint8)

    def wgrad():
        # dW_qkv[c, :] = sum_t dqkv[t, c] x[t, :]  (both operands token-major: layout T, split-K)
        _lib.call("rte_gemm_bf16", dqkv.data_ptr(), 3 * d, 1, None, x.data_ptr(), d, 1, None, dw_qkv.data_ptr(), d,
                  1, 3 * d, d, T, 1.0, 0.0, None, 0, ws.data_ptr(), ws_bytes, st())

    def ffn_fwd():
        _lib.call("rte_grouped_swiglu_fwd", x.data_ptr(), T, d, pk.offsets.data_ptr(), C, n, P,
                  pk.tok_of_slot.data_ptr(), pk.pair_of_slot.data_ptr(), pk.w_of_slot.data_ptr(), wug.data_ptr(),
                  wd.data_ptr(), F, ug.data_ptr(), zw.data_ptr(), yp.data_ptr(), st())

    out_pool = torch.empty(T, d, device=dev, dtype=torch.float32)

    def combine():
        _lib.call("rte_combine_rows", yp.data_ptr(), T, k, d, None, None, None, out_pool.data_ptr(), 1, st())

    ids_out = torch.empty(T, k, device=dev, dtype=torch.int32)
    w_out = torch.empty(T, k, device=dev, dtype=torch.float32)

    def topk():
        _lib.call("rte_route_topk", logits.data_ptr(), T, C, k, ids_out.data_ptr(), w_out.data_ptr(), st())

    pk_ws_bytes = _lib.load().rte_pack_workspace_bytes(P, C)
    pk_ws = torch.empty(max(pk_ws_bytes, 16), device=dev, dtype=torch.uint8)
    pk_out = [torch.empty(P, device=dev, dtype=torch.int32) for _ in range(4)]
    pk_off = torch.empty(C + 1, device=dev, dtype=torch.int32)
    pk_w = torch.empty(P, device=dev, dtype=torch.float32)

    def pack():
        _lib.call("rte_pack_index", ids.data_ptr(), P, C, k, w.data_ptr(), pk_off.data_ptr(), pk_out[0].data_ptr(),
                  pk_out[1].data_ptr(), pk_out[2].data_ptr(), pk_w.data_ptr(), None, pk_ws.data_ptr(), pk_ws_bytes,
                  st())

    return [
        dict(name="gemm_qkv_rope_fwd", per_step=2, kernels=1, flop=2.0 * T * 3 * d * d,
             bytes=2.0 * T * d + 2.0 * 3 * d * d + 3 * 2.0 * T * d, fn=qkv),
        dict(name="gemm_lm_head_fwd", per_step=1, kernels=1, flop=2.0 * T * V * d,
             bytes=2.0 * T * d + 2.0 * V * d + 4.0 * T * V, fn=head),
        # x@[Wup|Wgate]^T with the SwiGLU epilogue, then zw@Wdown into pair-major rows
        dict(name="grouped_swiglu_fwd", per_step=2, kernels=2, flop=2.0 * P * d * 2 * n + 2.0 * P * n * d,
             bytes=2.0 * T * d + 2.0 * 3 * F * d + 2.0 * P * 3 * n + 2.0 * P * d + 12.0 * P, fn=ffn_fwd),
        # combine unit: T*k*d*b + T*k*4 + T*d*b (bf16 rows in, fp32 rows out here)
        dict(name="combine_rows", per_step=2, kernels=1, flop=1.0 * P * d,
             bytes=2.0 * P * d + 4.0 * T * d, fn=combine),
        # route unit: T*C*4 logits in, T*k*(4+4) ids + weights out
        dict(name="route_topk", per_step=1, kernels=1, flop=0.0, bytes=4.0 * T * C + 8.0 * T * k, fn=topk),
        # pack unit: P*(4+4) ids + weights in, 4*P*4 + P*4 slot tables out, (C+1)*4 offsets
        dict(name="pack_index", per_step=1, kernels=3, flop=0.0, bytes=8.0 * P + 20.0 * P + 4.0 * (C + 1),
             fn=pack),
        dict(name="gemm_wgrad_qkv", per_step=2, kernels=2, flop=2.0 * T * 3 * d * d,
             bytes=2.0 * T * 3 * d + 2.0 * T * d + 4.0 * 3 * d * d, fn=wgrad),
    ]


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
                     "avg_us": round(dt * 1e6, 2), "bound": bound, "achieved": round(ach, 1),
                     "unit": "TFLOP/s" if bound == "mfma" else "GB/s", "peak": peak, "frac": round(ach / peak, 4),
                     "flop": c["flop"], "bytes": c["bytes"],
                     "tflops": round(c["flop"] / dt / 1e12, 1), "gbs": round(c["bytes"] / dt / 1e9, 1)})
    return rows


def measured_traffic(kernel: str):
    """HBM bytes per launch of `kernel` from the committed rocprofv3 --pmc summary
    (FETCH_SIZE + WRITE_SIZE, calibrated against a copy kernel), or None."""
    path = ROOT / "profiles" / "traffic.json"
    try:
        data = json.loads(path.read_text())
    except (OSError, ValueError):
        return None
    entry = data.get(kernel)
    return None if entry is None else entry.get("bytes_per_launch")


def profile_kernel(name: str, iters: int, B: int, S: int) -> int:
    """Launch one candidate kernel `iters` times (the program rocprofv3 --pmc profiles)."""
    import torch

    if name == "copy":
        # calibration: cast 64 Mi fp32 -> bf16 (reads 256 MiB, writes 128 MiB per launch)
        from rte_amd import _lib

        n = 64 << 20
        src = torch.randn(n, device="cuda")
        dst = torch.empty(n, device="cuda", dtype=torch.bfloat16)
        for _ in range(iters):
            _lib.call("rte_cast_f32_bf16", src.data_ptr(), n, dst.data_ptr(), _lib.stream_ptr())
    else:
        cands = {c["name"]: c for c in kernel_candidates(B, S)}
        for _ in range(iters):
            cands[name]["fn"]()
    torch.cuda.synchronize()
    print(json.dumps({"profiled": name, "iters": iters}))
    return 0


def cpu_baseline(budget_s: float = 15.0) -> dict:
    """numpy oracle of one cluster-pool SwiGLU layer fwd+bwd at BASELINE configs[0]
    (d 256, 32 clusters x 32, top-4, fp64 math), on a token sample sized to ~budget_s."""
    import numpy as np

    from oracle import cluster_pool as CP
    from oracle import routing as R

    rng = np.random.default_rng(0)
    d, C, n, k = 256, 32, 32, 4
    F = C * n
    wr = rng.standard_normal((C, d)) * 0.02
    wug = rng.standard_normal((2 * F, d)) * 0.02
    wd = rng.standard_normal((d, F)) * 0.02

    def run(T):
        x = rng.standard_normal((T, d))
        ids, w = R.route_topk((x @ wr.T).astype(np.float32), k)
        out = CP.routed_fwd(x, wug, wd, ids, w, C)
        CP.routed_bwd(np.ones_like(out) / out.size, x, wr, wug, wd, ids, w, C)

    t0 = time.perf_counter()
    run(256)
    per_tok = (time.perf_counter() - t0) / 256
    T = int(max(256, min(8192, budget_s / 3 / max(per_tok, 1e-9))))
    times = []
    for _ in range(3):
        t0 = time.perf_counter()
        run(T)
        times.append(time.perf_counter() - t0)
    med = sorted(times)[1]
    threads = int(os.environ.get("OMP_NUM_THREADS", "0") or 0) or os.cpu_count()
    return {
        "value": T / med,
        "unit": "tokens/s",
        "cores": threads,
        "kind": "port",
        "sample": f"numpy oracle, cluster-pool SwiGLU layer fwd+bwd (configs[0] shape: d256, 32x32, top-4), "
                  f"{T} of 8192 tokens x 3 runs, median; BLAS threads={threads}",
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
    ap.add_argument("--eager", action="store_true",
                    help="launch every kernel from Python instead of replaying the captured step graph")
    args = ap.parse_args(argv)
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
        return profile_kernel(args.profile_kernel, args.iters, args.batch, args.seq)
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
        rows = roofline_rows(args.batch, args.seq)
        single = [r for r in rows if r["kernels_per_call"] == 1]
        dom = max(single, key=lambda r: r["avg_us"] * r["launches_per_step"])
        out["roofline"] = {
            "kernel": dom["kernel"],
            "bound": dom["bound"],
            "achieved": dom["achieved"],
            "peak": dom["peak"],
            "unit": dom["unit"],
            "frac": dom["frac"],
            "traffic": measured_traffic(dom["kernel"]),
            "avg_us": dom["avg_us"],
            "flop_per_launch": dom["flop"],
            "algorithmic_bytes_per_launch": dom["bytes"],
        }
        out["kernels"] = rows
    if not args.no_cpu_baseline:
        out["cpu_baseline"] = cpu_baseline()
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
