"""training.precision = "fp32" on the GPU: the fp32 kernels (rte_gemm_f32 and its grouped form,
the causal softmax, SwiGLU, combine) and the model operators inside hip_ops.fp32_precision(),
against float64 references of the same math (torch on the device in float64 for the big shapes,
the numpy oracle for the routing).  Tolerance: fp32 within 1e-5 relative (Frobenius), ids
bit-exact.  Also: a model of the reference's configs/tiny.yaml preset (fp32, recursive_macro_
shortlist, Bernoulli audit) trains through TrainEngine."""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import routing as OR

pytestmark = pytest.mark.gpu

DEV = "cuda"
RTOL = 1e-5


@pytest.fixture(scope="module", autouse=True)
def _hip():
    from rte_amd import _lib

    if not _lib.device_ready():
        pytest.fail("HIP backend not ready on this GPU box (library or gfx950 device missing)")
    yield


def _rel(a, b):
    a, b = a.detach().double(), b.detach().double()
    return float((a - b).norm() / b.norm().clamp_min(1e-300))


def _g(seed):
    return torch.Generator(device=DEV).manual_seed(seed)


@pytest.mark.parametrize("M,N,K,a_t,b_t", [(64, 64, 16, 0, 0), (100, 37, 45, 0, 1), (77, 130, 260, 1, 0),
                                           (513, 255, 129, 1, 1), (8192, 512, 1536, 0, 1)])
def test_gemm_f32_dense(M, N, K, a_t, b_t):
    from rte_amd.kernels import f32_ops as F

    g = _g(M + N + K)
    A = torch.randn((K, M) if a_t else (M, K), device=DEV, generator=g)
    B = torch.randn((K, N) if b_t else (N, K), device=DEV, generator=g)
    C0 = torch.randn(M, N, device=DEV, generator=g)
    C = C0.clone()
    F.gemm(A, A.shape[1], a_t, B, B.shape[1], b_t, C, N, M, N, K, alpha=0.5, beta=2.0)
    Ad = A.double().t() if a_t else A.double()
    Bd = B.double() if b_t else B.double().t()
    ref = 0.5 * Ad @ Bd + 2.0 * C0.double()
    assert _rel(C, ref) < RTOL


def test_gemm_f32_batched_and_gathers():
    """Two-level batch strides (the attention's (sample, head) reads of packed rows), row gathers
    with per-row scales on A and B, scattered output rows."""
    from rte_amd.kernels import f32_ops as F

    g = _g(1)
    Z1, Z2, S, hd = 3, 4, 50, 32
    qkv = torch.randn(Z1, S, 3, Z2, hd, device=DEV, generator=g)
    out = torch.zeros(Z1, Z2, S, S, device=DEV)
    ld = 3 * Z2 * hd
    F.gemm(qkv, ld, 0, qkv[:, :, 1], ld, 0, out, S, S, S, hd, batch=(Z1, Z2), sA=(S * ld, hd), sB=(S * ld, hd),
           sC=(Z2 * S * S, S * S))
    q = qkv[:, :, 0].permute(0, 2, 1, 3).double()
    k = qkv[:, :, 1].permute(0, 2, 1, 3).double()
    assert _rel(out, q @ k.transpose(-1, -2)) < RTOL
    # gathers / scales / scatter
    A = torch.randn(40, 24, device=DEV, generator=g)
    B = torch.randn(30, 24, device=DEV, generator=g)
    ar = torch.randint(0, 40, (70,), device=DEV, generator=g, dtype=torch.int32)
    asc = torch.rand(70, device=DEV, generator=g)
    br = torch.randperm(30, device=DEV, generator=g)[:20].to(torch.int32)
    bsc = torch.rand(30, device=DEV, generator=g)
    cr = torch.randperm(90, device=DEV, generator=g)[:70].to(torch.int32)
    C = torch.zeros(90, 20, device=DEV)
    F.gemm(A, 24, 0, B, 24, 0, C, 20, 70, 20, 24, a_rows=ar, a_scale=asc, b_rows=br, b_scale=bsc, c_rows=cr)
    Ad = A.double()[ar.long()] * asc.double()[:, None]
    Bd = B.double()[br.long()] * bsc.double()[:20, None]
    ref = torch.zeros(90, 20, dtype=torch.float64, device=DEV)
    ref[cr.long()] = Ad @ Bd.t()
    assert _rel(C, ref) < RTOL


def test_gemm_f32_grouped_rows_and_reduction():
    """GROUP_M (per-group weight blocks, gathered rows) and GROUP_K (per-group reductions written
    to per-group blocks), with empty and ragged groups; GROUP_K repeats bitwise."""
    from rte_amd.kernels import f32_ops as F

    g = _g(2)
    G, Kin, Nout, T = 7, 48, 40, 300
    x = torch.randn(T, Kin, device=DEV, generator=g)
    W = torch.randn(G, Kin, Nout, device=DEV, generator=g)
    counts = torch.tensor([0, 90, 1, 64, 65, 0, 80])
    goff = torch.cat([torch.zeros(1, dtype=torch.long), counts.cumsum(0)]).to(torch.int32).to(DEV)
    P = int(counts.sum())
    tok = torch.randint(0, T, (P,), device=DEV, generator=g, dtype=torch.int32)
    y = torch.zeros(P, Nout, device=DEV)
    F.gemm_grouped(1, goff, G, x, Kin, 0, W, Nout, 1, y, Nout, P, Nout, Kin, a_rows=tok, b_gstride=Kin * Nout)
    grp = torch.repeat_interleave(torch.arange(G), counts).to(DEV)
    ref = torch.einsum("pk,pkn->pn", x.double()[tok.long()], W.double()[grp])
    assert _rel(y, ref) < RTOL
    dy = torch.randn(P, Nout, device=DEV, generator=g)
    dW = torch.full((G, Kin, Nout), 7.0, device=DEV)
    for rep in range(2):
        out = torch.full((G, Kin, Nout), 7.0, device=DEV)
        F.gemm_grouped(2, goff, G, x, Kin, 1, dy, Nout, 1, out, Nout, Kin, Nout, P, a_rows=tok,
                       c_gstride=Kin * Nout)
        if rep == 0:
            dW = out
        else:
            assert torch.equal(out, dW)
    refw = torch.zeros(G, Kin, Nout, dtype=torch.float64, device=DEV)
    refw.index_add_(0, grp, x.double()[tok.long()][:, :, None] * dy.double()[:, None, :])
    assert _rel(dW, refw) < RTOL
    assert torch.all(dW[0] == 0) and torch.all(dW[5] == 0)  # empty groups are written as zero


def _attn_ref(q, k, v, hs):
    S = q.shape[-2]
    s = q @ k.transpose(-1, -2) / math.sqrt(q.shape[-1])
    s = s.masked_fill(~torch.ones(S, S, dtype=torch.bool, device=q.device).tril(), float("-inf"))
    y = s.softmax(-1) @ v
    if hs is not None:
        y = y * hs[:, :, None, None]
    return y.transpose(1, 2).reshape(q.shape[0], S, -1)


@pytest.mark.parametrize("B,H,S,hd,masked", [(2, 4, 12, 4, False), (3, 8, 64, 64, True), (2, 2, 200, 40, True)])
def test_attention_f32(B, H, S, hd, masked):
    from rte_amd.kernels import f32_ops as F

    g = _g(S)
    q, k, v = (torch.randn(B, H, S, hd, device=DEV, generator=g, requires_grad=True) for _ in range(3))
    hs = (torch.rand(B, H, device=DEV, generator=g) > 0.4).float() * 0.5 if masked else None
    y = F.AttentionFn.apply(q, k, v, hs)
    dy = torch.randn(y.shape, device=DEV, generator=g)
    y.backward(dy)
    qd, kd, vd = (t.detach().double().requires_grad_() for t in (q, k, v))
    yr = _attn_ref(qd, kd, vd, None if hs is None else hs.double())
    yr.backward(dy.double())
    assert _rel(y, yr) < RTOL
    for a, b in ((q, qd), (k, kd), (v, vd)):
        assert _rel(a.grad, b.grad) < RTOL


def test_cfg1_layer_f32_full_size():
    """BASELINE configs[0] in fp32 at its full size (T 8192, d 256, 32 x 32 neurons, top-4): routing
    ids bit-exact against the oracle on the kernel's logits; output and every gradient within 1e-5
    of float64 autograd with the same routing."""
    from rte_amd.kernels import hip_ops
    from oracle import pool_port as PP

    x, wr, wup, wgate, wdown = (t.to(DEV) for t in PP.make_cfg1())
    k, C = 4, 32
    wr_l = wr.t().contiguous()                  # router Linear [C, d]
    wug = torch.cat([wup, wgate]).contiguous()  # [2F, d] rows [up ; gate]
    wd = wdown.t().contiguous()                 # Linear [d, F]
    ts = [t.clone().requires_grad_() for t in (x, wr_l, wug, wd)]
    with hip_ops.fp32_precision():
        out, ids, w = hip_ops.routed_cluster_pool_swiglu(ts[0], ts[1], ts[2], ts[3], k)
    dy = torch.randn(out.shape, device=DEV, generator=_g(3))
    out.backward(dy)
    from rte_amd.kernels import f32_ops as F

    logits = F.linear(x, wr_l)  # the routed pool's own router product (same kernel, same bits)
    rid, _ = OR.route_topk(logits.cpu().numpy(), k)
    assert np.array_equal(ids.cpu().numpy(), rid)
    # float64 autograd of the same layer with the GPU's routing decisions
    td = [t.detach().double().requires_grad_() for t in (x, wr_l, wug, wd)]
    lg = td[0] @ td[1].t()
    wsel = lg.gather(1, ids.long()).softmax(-1)
    F_ = wd.shape[1]
    n = F_ // C
    up = td[0] @ td[2][:F_].t()
    gate = td[0] @ td[2][F_:].t()
    z = up * torch.nn.functional.silu(gate)                         # [T, F]
    ref = torch.zeros_like(td[0])
    for j in range(k):
        c = ids[:, j].long()
        cols = (c[:, None] * n + torch.arange(n, device=DEV)[None, :])
        zc = z.gather(1, cols)                                     # [T, n]
        wdc = td[3].t()[cols]                                      # [T, n, d]
        ref = ref + wsel[:, j:j + 1] * torch.einsum("tn,tnd->td", zc, wdc)
    ref.backward(dy.double())
    assert _rel(out, ref) < RTOL
    for a, b, name in zip(ts, td, ("x", "wr", "wug", "wd")):
        assert _rel(a.grad, b.grad) < RTOL, name


def test_cfg2_block_f32_full_size():
    """BASELINE configs[1]'s block (fused QKV + RoPE + causal attention + O-proj, dense SwiGLU;
    T 8192 = 128 x 64, d 512, 8 heads, d_ff 2048) through the model's TransformerBlock under
    fp32 precision, against the reference block (rte/layers.py:53-87, 646-656) in float64."""
    from rte_amd.config import ModelConfig
    from rte_amd.kernels import hip_ops
    from rte_amd.layers import TransformerBlock
    from oracle import step_port as SP

    torch.manual_seed(0)
    cfg = ModelConfig(topology="dense", vocab_size=64, d_model=512, n_heads=8, d_ff=2048, n_dense_layers=1,
                      n_prelude=0, n_coda=0, t_max=1, depth_choices=[1], attn_banks=1, ffn_banks=1, head_groups=1,
                      ffn_groups=1, active_head_groups=1, active_ffn_groups=1, recipe_count=2)
    blk = TransformerBlock(cfg).to(DEV)
    with torch.no_grad():
        for name, p in blk.named_parameters():
            if "norm" in name:
                p.add_(0.1 * torch.randn(p.shape, device=DEV, generator=_g(5)))
            else:
                p.copy_(torch.randn(p.shape, device=DEV, generator=_g(6)) * 0.02)
    x = torch.randn(128, 64, 512, device=DEV, generator=_g(7), requires_grad=True)
    with hip_ops.fp32_precision():
        y = blk(x)
    dy = torch.randn(y.shape, device=DEV, generator=_g(8))
    y.backward(dy)
    P = {n_: p.detach().double().requires_grad_() for n_, p in blk.named_parameters()}
    xd = x.detach().double().requires_grad_()
    cos, sin = SP.rope_tables(64, 64, torch.float64)
    cos, sin = cos.to(DEV), sin.to(DEV)
    u = xd + SP.dense_attention(SP.rmsnorm(xd, P["norm1.weight"]), P["attn.wqkv.weight"], P["attn.wo.weight"], 8,
                                cos, sin)
    ref = u + SP.swiglu(SP.rmsnorm(u, P["norm2.weight"]), P["mlp.wug.weight"], P["mlp.wd.weight"])
    ref.backward(dy.double())
    assert _rel(y, ref) < RTOL
    assert _rel(x.grad, xd.grad) < RTOL
    for n_, p in blk.named_parameters():
        assert _rel(p.grad, P[n_].grad) < RTOL, n_


def _tiny_yaml_config():
    """The reference's configs/tiny.yaml (precision left at its default, fp32), written out."""
    from rte_amd.config import DataConfig, ExperimentConfig, ModelConfig, OutputConfig, TrainingConfig

    model = ModelConfig(topology="recursive", vocab_size=128, d_model=16, n_heads=4, d_ff=64, n_dense_layers=5,
                        n_prelude=1, n_coda=1, t_max=4, depth_choices=[1, 2, 4], attn_banks=1, ffn_banks=3,
                        head_groups=4, ffn_groups=4, active_head_groups=1, active_ffn_groups=1, recipe_count=4,
                        tie_embeddings=True, use_rope=True, use_recursive_input_skip=True, fairness_tolerance=0.01,
                        macro_rank=2, router_hidden=16)
    training = TrainingConfig(mode="recursive_macro_shortlist", optimizer="adamw", lr=0.0005, weight_decay=0.01,
                              batch_size=2, seq_len=12, grad_accum_steps=1, seed=1337, audit_p_min=0.25,
                              audit_p_max=1.0, lambda_depth=0.0001, lambda_load=0.01, lambda_cover=0.01,
                              lambda_hid=0.01, lambda_cos=0.01, lambda_kl=0.01, lambda_cons=0.001)
    output = OutputConfig(mode="shortlist", num_clusters=8, shortlist_top_clusters=2, shortlist_max_tokens=16,
                          hard_negatives=4, random_negatives=4)
    return ExperimentConfig(run_name="tiny", output_dir="runs", model=model, training=training, output=output,
                            data=DataConfig(dataset="synthetic", tokenizer="gpt2_bpe", synthetic_tokens=4096))


def test_tiny_yaml_preset_trains_fp32():
    """configs/tiny.yaml (fp32, d 16, 4 heads of 4, banked core 3 FFN banks, rank-2 macro, shortlist
    head, Bernoulli audit) trains through TrainEngine: finite losses, parameters move, the loss on a
    repeated batch falls."""
    from rte_amd.training import TrainEngine, metrics_to_host

    cfg = _tiny_yaml_config()
    assert cfg.training.precision == "fp32"
    eng = TrainEngine(cfg, device=torch.device(DEV))
    gen = torch.Generator().manual_seed(0)
    ids = torch.randint(0, 128, (2, 13), generator=gen)
    batch = (ids[:, :-1].to(DEV), ids[:, 1:].to(DEV))
    before = {n_: p.detach().clone() for n_, p in eng.recursive_model.named_parameters()}
    losses = []
    for step in range(12):
        m = metrics_to_host(eng.train_step(batch).metrics)
        losses.append(float(m["loss"]))
        assert math.isfinite(losses[-1]), (step, m)
    changed = sum(int(not torch.equal(before[n_], p.detach())) for n_, p in eng.recursive_model.named_parameters())
    assert changed > len(before) // 2
    assert min(losses[-3:]) < losses[0], losses
