"""GPU tests of the model-level path: a full dense block (fused QKV + RoPE + attention +
O-proj + dense SwiGLU) against a float32 torch reference of the same
block on the CPU, and one train step of every accelerated mode."""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F
from helpers import BF16_RTOL, FP32_RTOL, assert_rel
from helpers import BF16_RTOL, assert_rel

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def _hip():
    from rte_amd import _lib

    if not _lib.device_ready():
        pytest.fail("HIP backend not ready on this GPU box")


def _model_cfg(**over):
    from rte_amd.config import ModelConfig

    base = dict(topology="recursive", vocab_size=256, d_model=128, n_heads=4, d_ff=512, n_dense_layers=2, n_prelude=1,
                n_coda=1, t_max=4, depth_choices=[1, 2, 4], attn_banks=1, ffn_banks=2, head_groups=4, ffn_groups=16,
                active_head_groups=1, active_ffn_groups=4, recipe_count=6, macro_rank=8, router_hidden=64,
                ffn_kind="cluster_pool", ffn_clusters=16, ffn_top_k=2)
    base.update(over)
    return ModelConfig(**base)


def _ref_block(block, x):
    """float32 torch math of TransformerBlock (rte/layers.py:53-87, :646-656)."""
    def rms(v, w):
        return v * torch.rsqrt(v.pow(2).mean(-1, keepdim=True) + 1e-5) * w

    b, s, d = x.shape
    H = block.attn.n_heads
    hd = d // H
    n1 = rms(x, block.norm1.weight)
    qkv = (n1 @ block.attn.wqkv.weight.t()).view(b, s, 3, H, hd)
    q, k, v = (t.transpose(1, 2) for t in qkv.unbind(2))
    cos, sin = block.attn.rope.cos[:s], block.attn.rope.sin[:s]

    def rot(t):
        return torch.stack((-t[..., 1::2], t[..., ::2]), -1).flatten(-2)

    q = q * cos + rot(q) * sin
    k = k * cos + rot(k) * sin
    att = (q @ k.transpose(-1, -2)) / math.sqrt(hd)
    att = att.masked_fill(torch.triu(torch.ones(s, s, dtype=torch.bool), 1), float("-inf")).softmax(-1)
    y = (att @ v).transpose(1, 2).reshape(b, s, d)
    u = x + y @ block.attn.wo.weight.t()
    n2 = rms(u, block.norm2.weight)
    up, gate = (n2 @ block.mlp.wug.weight.t()).chunk(2, -1)
    return u + (up * F.silu(gate)) @ block.mlp.wd.weight.t()


@pytest.mark.parametrize("B,S,d,H,F_", [(4, 32, 128, 2, 256), (128, 64, 512, 8, 2048)])
def test_dense_block_matches_fp32_reference(B, S, d, H, F_):
    from rte_amd.config import ModelConfig
    from rte_amd.layers import TransformerBlock

    cfg = ModelConfig(topology="dense", vocab_size=64, d_model=d, n_heads=H, d_ff=F_, n_dense_layers=1, n_prelude=1,
                      n_coda=1, t_max=1, depth_choices=[1], attn_banks=1, ffn_banks=1, head_groups=1, ffn_groups=1,
                      active_head_groups=1, active_ffn_groups=1, recipe_count=2)
    torch.manual_seed(0)
    block = TransformerBlock(cfg)
    with torch.no_grad():
        for p in block.parameters():
            if p.ndim == 2:
                p.normal_(0.0, 0.02)
        # weights exactly representable in bf16 so both sides see the same operands
        for p in block.parameters():
            p.copy_(p.to(torch.bfloat16).float())
    x = torch.randn(B, S, d).to(torch.bfloat16).float()
    dy = torch.randn(B, S, d)
    xr = x.clone().requires_grad_()
    ref = _ref_block(block, xr)
    ref.backward(dy)
    ref_grads = {n: p.grad.clone() for n, p in block.named_parameters()}
    block.zero_grad()
    gb = block.cuda()
    xg = x.cuda().requires_grad_()
    out = gb(xg)
    out.backward(dy.cuda())
    assert_rel(out.detach().cpu().numpy(), ref.detach().numpy(), BF16_RTOL, "block out")
    assert_rel(xg.grad.cpu().numpy(), xr.grad.numpy(), BF16_RTOL, "block dx")
    for n, p in gb.named_parameters():
        assert_rel(p.grad.cpu().numpy(), ref_grads[n].numpy(), BF16_RTOL, f"block d{n}")


def _engine(mode="recursive_macro", **mover):
    from rte_amd.config import ExperimentConfig, OutputConfig, TrainingConfig
    from rte_amd.training import TrainEngine

    topo = "dense" if mode == "dense_exact" else "recursive"
    cfg = ExperimentConfig(
        model=_model_cfg(topology=topo, **mover),
        training=TrainingConfig(mode=mode, precision="bf16", batch_size=4, seq_len=16, audit_sampler="fixed_count",
                                audit_fixed_count=1, fixed_depth=4, seed=3),
        output=OutputConfig(num_clusters=8, shortlist_max_tokens=32, hard_negatives=4, random_negatives=4),
    )
    return TrainEngine(cfg, device=torch.device("cuda"))


@pytest.mark.parametrize("mode", ["recursive_macro", "recursive_macro_shortlist", "recursive_exact", "dense_exact"])
@pytest.mark.parametrize("ffn_kind", ["cluster_pool", "dense"])
def test_train_step_every_mode(mode, ffn_kind):
    from rte_amd.training import metrics_to_host

    eng = _engine(mode, ffn_kind=ffn_kind)
    model = eng.recursive_model if eng.recursive_model is not None else eng.dense_model
    before = {n: p.detach().clone() for n, p in model.named_parameters()}
    g = torch.Generator().manual_seed(0)
    tok = torch.randint(0, 256, (4, 17), generator=g)
    res = eng.train_step((tok[:, :-1], tok[:, 1:]))
    m = metrics_to_host(res.metrics)
    assert math.isfinite(float(res.loss)), m
    changed = sum(int(not torch.equal(before[n], p.detach())) for n, p in model.named_parameters())
    assert changed > 0


def test_audit_p1_corrected_equals_exact():
    """rte tests/test_audit.py:12-37: with every sample audited at p = 1 the corrected
    per-sample loss equals the exact replay's loss."""
    from rte_amd.config import ExperimentConfig, TrainingConfig
    from rte_amd.models import RecursiveModel

    cfg = ExperimentConfig(model=_model_cfg(), training=TrainingConfig(mode="recursive_macro", audit_fixed_count=4,
                                                                       batch_size=4, seed=5))
    torch.manual_seed(0)
    model = RecursiveModel(cfg.model, cfg.output).cuda()
    from rte_amd.audit import AuditEngine

    tok = torch.randint(0, 256, (4, 17), device="cuda")
    hot = model.forward_macro(tok[:, :-1], tok[:, 1:], return_states=True, return_loss_per_sample=True, fixed_depth=4)
    res = AuditEngine(cfg.training).correction(model, tok[:, :-1], tok[:, 1:], hot, seed=1)
    assert res.exact is not None
    # the fixed-count sampler draws randperm(n)[:k] from a generator seeded with `seed`;
    # exact losses come back in that order
    chosen = torch.randperm(4, device="cuda", generator=torch.Generator(device="cuda").manual_seed(1))[:4]
    ref = torch.empty_like(res.corrected_loss_per_sample)
    ref[chosen] = res.exact.loss_per_sample.detach()
    assert int(res.audit_mask.sum()) == 4
    np.testing.assert_allclose(res.corrected_loss_per_sample.detach().cpu().numpy(), ref.cpu().numpy(),
                               rtol=1e-5, atol=1e-5)


def test_backend_status_reports_hip():
    from rte_amd.kernels import optimized

    st = optimized.backend_status()
    assert st["mode"] == "rocm_hip_dispatch"
    assert st["uses_reference_fallback"] is False
    assert "gfx950" in st["device"]["arch"]


# ---------------------------------------------------------------- banked recursive core

def _banked_core(seed=0):
    from rte_amd.config import ModelConfig
    from rte_amd.layers import BankedRecursiveCore
    from rte_amd.recipes import RecipeBank

    cfg = ModelConfig(topology="recursive", vocab_size=64, d_model=128, n_heads=4, d_ff=256, n_dense_layers=2,
                      n_prelude=1, n_coda=1, t_max=2, depth_choices=[1, 2], attn_banks=2, ffn_banks=2, head_groups=4,
                      ffn_groups=8, active_head_groups=2, active_ffn_groups=2, recipe_count=7)
    torch.manual_seed(seed)
    core = BankedRecursiveCore(cfg, RecipeBank(cfg)).to("cuda")
    with torch.no_grad():
        for name in ("pass_gamma1", "pass_beta1", "pass_gamma2", "pass_beta2"):
            getattr(core, name).normal_(0.0, 0.1)
        core.pass_attn_scale.uniform_(0.5, 1.5)
        core.pass_mlp_scale.uniform_(0.5, 1.5)
        core.norm1.weight.uniform_(0.8, 1.2)
        core.norm2.weight.uniform_(0.8, 1.2)
    return cfg, core


def _core_params_np(core):
    p = {k: v.detach().double().cpu().numpy() for k, v in core.named_parameters()}
    return dict(norm1=p["norm1.weight"], norm2=p["norm2.weight"], wqkv=p["attn.wqkv"], wo=p["attn.wo"],
                wug=p["mlp.wug"], wd=p["mlp.wd"], pass_gamma1=p["pass_gamma1"], pass_beta1=p["pass_beta1"],
                pass_gamma2=p["pass_gamma2"], pass_beta2=p["pass_beta2"], pass_attn_scale=p["pass_attn_scale"],
                pass_mlp_scale=p["pass_mlp_scale"], alpha_inj=p.get("alpha_inj"))


def _oracle_recipes(core):
    return [dict(attention_banks=r.attention_banks, ffn_banks=r.ffn_banks, head_groups=r.head_groups,
                 ffn_groups=r.ffn_groups) for r in core.recipe_bank.recipes]


def test_banked_core_forward_step_matches_oracle():
    """Mixed recipes (including the dense fallback, two banks each) and an inactive sample in
    one device-side pass, against the per-sample reference restatement."""
    from oracle import attention as AO
    from oracle import banked as BK

    cfg, core = _banked_core(1)
    B, S, d = 5, 32, cfg.d_model
    h = torch.randn(B, S, d, device="cuda")
    h0 = torch.randn(B, S, d, device="cuda")
    rid = torch.tensor([0, 3, 6, 1, 3], device="cuda")
    active = torch.tensor([True, True, False, True, True], device="cuda")
    print("banked forward_step B=5 S=32 d=128", flush=True)
    out = core.forward_step(h, h0, rid, active, pass_idx=1)
    cos, sin = AO.rope_tables(d // cfg.n_heads, S)
    want = BK.core_forward_step(h.double().cpu().numpy(), h0.double().cpu().numpy(), rid.tolist(), active.tolist(),
                                _oracle_recipes(core), _core_params_np(core), 1, n_heads=cfg.n_heads,
                                head_groups=cfg.head_groups, ffn_groups=cfg.ffn_groups, cos=cos, sin=sin)
    got = out.detach().double().cpu().numpy()
    assert np.array_equal(got[2], h[2].double().cpu().numpy()), "inactive sample changed"
    assert_rel(got - h.double().cpu().numpy(), want - h.double().cpu().numpy(), BF16_RTOL, "banked step delta")


def _torch_core_step(h, h0, rid, active, recipes, p, pass_idx, cfg, cos, sin):
    """fp64 CPU torch restatement of BankedRecursiveCore.forward_step (rte/layers.py:659-870),
    per sample and per recipe; differentiable in every entry of p and in h, h0."""
    d, H = cfg.d_model, cfg.n_heads
    hd, hpg = d // H, H // cfg.head_groups
    slab = cfg.d_ff // cfg.ffn_groups

    def rms(v, w):
        return v * torch.rsqrt(v.pow(2).mean(-1, keepdim=True) + 1e-5) * w

    def rot(t):
        return torch.stack((-t[..., 1::2], t[..., ::2]), -1).flatten(-2)

    outs = []
    for i in range(h.shape[0]):
        if not active[i]:
            outs.append(h[i])
            continue
        r = recipes[rid[i]]
        S = h.shape[1]
        ht = h[i] + p["alpha_inj"] * h0[i] if "alpha_inj" in p else h[i]
        n1 = rms(ht, p["norm1"]) * (1 + p["pass_gamma1"][pass_idx]) + p["pass_beta1"][pass_idx]
        cols = torch.tensor([c for g in r["head_groups"] for hh in range(g * hpg, (g + 1) * hpg)
                             for c in range(hh * hd, (hh + 1) * hd)])
        a = cols.numel()
        att = torch.zeros(S, d, dtype=torch.float64)
        for b in r["attention_banks"]:
            qkv = n1 @ p["wqkv"][b][:, torch.cat([cols, cols + d, cols + 2 * d])]
            q, k, v = (qkv[:, j * a:(j + 1) * a].view(S, a // hd, hd).transpose(0, 1) for j in range(3))
            q, k = q * cos + rot(q) * sin, k * cos + rot(k) * sin
            y = torch.nn.functional.scaled_dot_product_attention(q, k, v, is_causal=True)
            att = att + y.transpose(0, 1).reshape(S, a) @ p["wo"][b][cols, :]
        u = ht + p["pass_attn_scale"][pass_idx] * att / len(r["attention_banks"])
        n2 = rms(u, p["norm2"]) * (1 + p["pass_gamma2"][pass_idx]) + p["pass_beta2"][pass_idx]
        slabs = torch.tensor([c for g in r["ffn_groups"] for c in range(g * slab, (g + 1) * slab)])
        mlp = torch.zeros(S, d, dtype=torch.float64)
        for b in r["ffn_banks"]:
            fused = n2 @ p["wug"][b][:, torch.cat([slabs, slabs + cfg.d_ff])]
            up, gate = fused.split(slabs.numel(), dim=-1)
            mlp = mlp + (up * torch.nn.functional.silu(gate)) @ p["wd"][b][slabs, :]
        outs.append(u + p["pass_mlp_scale"][pass_idx] * mlp / len(r["ffn_banks"]))
    return torch.stack(outs)


def test_banked_core_gradients_match_fp64_reference():
    """Gradients of every core parameter and of h, h0 against fp64 autograd of a CPU torch
    restatement whose forward is first checked against the numpy oracle."""
    from oracle import attention as AO
    from oracle import banked as BK
    from helpers import rel_err

    cfg, core = _banked_core(2)
    B, S, d = 4, 16, cfg.d_model
    gen = np.random.default_rng(2)
    hn = gen.standard_normal((B, S, d))
    h0n = gen.standard_normal((B, S, d))
    G = gen.standard_normal((B, S, d))
    rid, active = [0, 2, 5, 4], [True, True, True, False]
    h = torch.tensor(hn, dtype=torch.float32, device="cuda", requires_grad=True)
    h0 = torch.tensor(h0n, dtype=torch.float32, device="cuda", requires_grad=True)
    print("banked core gradients B=4 S=16 d=128", flush=True)
    out = core.forward_step(h, h0, torch.tensor(rid, device="cuda"), torch.tensor(active, device="cuda"),
                            pass_idx=0, weights=core.prepare())
    (out * torch.tensor(G, dtype=torch.float32, device="cuda")).sum().backward()
    cos, sin = AO.rope_tables(d // cfg.n_heads, S)
    recipes = _oracle_recipes(core)
    base = _core_params_np(core)
    tp = {k: torch.tensor(v, requires_grad=True) for k, v in base.items() if v is not None}
    th, th0 = torch.tensor(hn, requires_grad=True), torch.tensor(h0n, requires_grad=True)
    ref = _torch_core_step(th, th0, rid, active, recipes, tp, 0, cfg, torch.tensor(cos), torch.tensor(sin))
    want = BK.core_forward_step(hn, h0n, rid, active, recipes, base, 0, n_heads=cfg.n_heads,
                                head_groups=cfg.head_groups, ffn_groups=cfg.ffn_groups, cos=cos, sin=sin)
    assert rel_err(ref.detach().numpy(), want) < 1e-12, "torch restatement disagrees with the oracle"
    (ref * torch.tensor(G)).sum().backward()
    mods = {"norm1": core.norm1.weight, "norm2": core.norm2.weight, "wqkv": core.attn.wqkv, "wo": core.attn.wo,
            "wug": core.mlp.wug, "wd": core.mlp.wd, "pass_gamma1": core.pass_gamma1, "pass_beta1": core.pass_beta1,
            "pass_gamma2": core.pass_gamma2, "pass_beta2": core.pass_beta2, "pass_attn_scale": core.pass_attn_scale,
            "pass_mlp_scale": core.pass_mlp_scale}
    if core.alpha_inj is not None:
        mods["alpha_inj"] = core.alpha_inj
    for name, param in mods.items():
        assert_rel(param.grad.double().cpu().numpy(), tp[name].grad.numpy(), BF16_RTOL, f"d{name}")
    assert_rel(h.grad.double().cpu().numpy(), th.grad.numpy(), BF16_RTOL, "dh")
    if th0.grad is None:
        assert h0.grad is None or not h0.grad.any()
    else:
        assert_rel(h0.grad.double().cpu().numpy(), th0.grad.numpy(), BF16_RTOL, "dh0")


def test_banked_swiglu_weight_gradients_exact_layout():
    """Element-wise FFN weight gradients of the banked SwiGLU (bank/slab layout of the grouped
    kernel mapped back to [banks, d, 2F] / [banks, F, d]) against the dense-FFN oracle backward
    applied to each sample's slabs."""
    from oracle import swiglu as SWO

    cfg, core = _banked_core(3)
    B, S, d = 4, 16, cfg.d_model
    gen = np.random.default_rng(3)
    x = gen.standard_normal((B, S, d)).astype(np.float32)
    xb = torch.tensor(x, device="cuda").to(torch.bfloat16)
    rid = torch.tensor([0, 1, 4, 6], device="cuda")
    ids, w = core.mlp.routes_for(rid, S)
    out = core.mlp.forward_routes(xb, ids, w)
    G = gen.standard_normal((B, S, d))
    out.backward(torch.tensor(G, dtype=torch.float32, device="cuda"))
    wug = core.mlp.wug.detach().to(torch.bfloat16).double().cpu().numpy()
    wd = core.mlp.wd.detach().to(torch.bfloat16).double().cpu().numpy()
    F_ = cfg.d_ff
    slab = F_ // cfg.ffn_groups
    dwug, dwd = np.zeros_like(wug), np.zeros_like(wd)
    want = np.zeros((B, S, d))
    xs = xb.double().cpu().numpy()
    for i, r in enumerate(_oracle_recipes(core)[j] for j in rid.tolist()):
        slabs = np.array([c for g in r["ffn_groups"] for c in range(g * slab, (g + 1) * slab)])
        cols = np.concatenate([slabs, slabs + F_])
        for b in r["ffn_banks"]:
            sc = 1.0 / len(r["ffn_banks"])
            y, cache = SWO.dense_swiglu_fwd(xs[i], wug[b][:, cols].T, wd[b][slabs, :], wd_rows=True)
            want[i] += sc * y
            _, gw, gd = SWO.dense_swiglu_bwd(sc * G[i], xs[i], wug[b][:, cols].T, wd[b][slabs, :], cache, wd_rows=True)
            dwug[b][:, cols] += gw.T
            dwd[b][slabs, :] += gd
    assert_rel(out.detach().double().cpu().numpy(), want, BF16_RTOL, "banked ffn out")
    assert_rel(core.mlp.wug.grad.double().cpu().numpy(), dwug, BF16_RTOL, "banked dwug")
    assert_rel(core.mlp.wd.grad.double().cpu().numpy(), dwd, BF16_RTOL, "banked dwd")


def _graph_node_kinds(graph) -> dict[str, int]:
    """Node census of a captured graph through the HIP runtime API."""
    import collections
    import ctypes

    hip = ctypes.CDLL("libamdhip64.so")
    gp = ctypes.c_void_p(graph.raw_cuda_graph())
    n = ctypes.c_size_t(0)
    assert hip.hipGraphGetNodes(gp, None, ctypes.byref(n)) == 0
    nodes = (ctypes.c_void_p * max(n.value, 1))()
    assert hip.hipGraphGetNodes(gp, nodes, ctypes.byref(n)) == 0
    names = {0: "kernel", 1: "memcpy", 2: "memset", 3: "host", 4: "graph", 5: "empty", 6: "wait_event",
             7: "event_record"}
    kinds = collections.Counter()
    for i in range(n.value):
        t = ctypes.c_int(-1)
        hip.hipGraphNodeGetType(ctypes.c_void_p(nodes[i]), ctypes.byref(t))
        kinds[names.get(t.value, str(t.value))] += 1
    return dict(kinds)


@pytest.mark.parametrize("mode", ["recursive_macro", "recursive_macro_shortlist"])
def test_captured_step_matches_eager(mode):
    """Eager and captured engines from the same seed on the same batches: every replay (with
    eager work and synchronisation between replays) reproduces the eager step's loss and
    metrics, the parameters agree afterwards, and the graph holds no memset node."""
    a = _engine(mode)
    b = _engine(mode)
    b.enable_graph_capture(True, keep_graph=True)
    g = torch.Generator().manual_seed(11)
    batches = [torch.randint(0, 256, (4, 17), generator=g) for _ in range(3)]
    for step in range(6):
        tok = batches[step % 3]
        print(f"captured-vs-eager {mode} step {step}", flush=True)
        ra = a.train_step((tok[:, :-1], tok[:, 1:]))
        rb = b.train_step((tok[:, :-1], tok[:, 1:]))
        torch.cuda.synchronize()
        la, lb = float(ra.loss.detach()), float(rb.loss)
        assert abs(la - lb) <= 1e-5 * max(abs(la), 1.0), (step, la, lb)
        for k, v in ra.metrics.items():
            if isinstance(v, torch.Tensor) and v.numel() == 1 and v.dtype.is_floating_point:
                x, y = float(v), float(rb.metrics[k])
                assert abs(x - y) <= 1e-4 * max(abs(x), 1e-3) + 1e-6, (step, k, x, y)
        assert bool(rb.metrics["stepped"])
    for (na, pa), (nb, pb) in zip(a.recursive_model.named_parameters(), b.recursive_model.named_parameters()):
        assert torch.allclose(pa, pb, rtol=1e-5, atol=1e-6), na
    kinds = _graph_node_kinds(b._gstate["graph"])
    print("graph nodes", kinds, flush=True)
    assert kinds.get("memset", 0) == 0, kinds
    assert kinds.get("kernel", 0) > 100


def test_rmsnorm_resid_matches_separate_residual():
    """The norm that hands its input on as the residual branch gives the gradients of the plain
    norm plus a separate residual use (the residual gradient added inside the norm backward)."""
    from rte_amd.kernels import hip_ops

    g = torch.Generator().manual_seed(4)
    x0 = torch.randn(3, 37, 256, generator=g).to("cuda")
    w0 = (1.0 + 0.1 * torch.randn(256, generator=g)).to("cuda")
    g1 = torch.randn(3, 37, 256, generator=g).to("cuda")
    g2 = torch.randn(3, 37, 256, generator=g).to("cuda")
    print("rmsnorm_resid 3x37x256", flush=True)
    x, w = x0.clone().requires_grad_(), w0.clone().requires_grad_()
    n, xr = hip_ops.rmsnorm_resid(x, w)
    ((n.float() * g1).sum() + (xr * g2).sum()).backward()
    xa, wa = x0.clone().requires_grad_(), w0.clone().requires_grad_()
    na = hip_ops.rmsnorm(xa, wa)
    ((na.float() * g1).sum() + (xa * g2).sum()).backward()
    assert torch.equal(n, na) and torch.equal(xr, x0)
    assert_rel(x.grad.cpu().numpy(), xa.grad.cpu().numpy(), 1e-6, "dx")
    assert_rel(w.grad.cpu().numpy(), wa.grad.cpu().numpy(), 1e-6, "dw")
    # only the norm output used: the residual branch's gradient is absent
    x, w = x0.clone().requires_grad_(), w0.clone().requires_grad_()
    n, _ = hip_ops.rmsnorm_resid(x, w)
    (n.float() * g1).sum().backward()
    xa, wa = x0.clone().requires_grad_(), w0.clone().requires_grad_()
    (hip_ops.rmsnorm(xa, wa).float() * g1).sum().backward()
    assert torch.equal(x.grad, xa.grad) and torch.equal(w.grad, wa.grad)


def test_bf16_prefetch_matches_per_use_casts():
    """Engines with and without the one-launch weight cast (recorded on the first step, run
    from the second) take bit-identical steps: same losses, same parameters."""
    a = _engine("recursive_macro")
    b = _engine("recursive_macro")
    b._bf16.enabled = False
    g = torch.Generator().manual_seed(5)
    for step in range(4):
        tok = torch.randint(0, 256, (4, 17), generator=g)
        print(f"bf16 prefetch step {step}", flush=True)
        ra = a.train_step((tok[:, :-1], tok[:, 1:]))
        rb = b.train_step((tok[:, :-1], tok[:, 1:]))
        torch.cuda.synchronize()
        assert float(ra.loss.detach()) == float(rb.loss.detach()), step
    assert a._bf16.entries and a._bf16.tables is not None
    for (na, pa), (_, pb) in zip(a.recursive_model.named_parameters(), b.recursive_model.named_parameters()):
        assert torch.equal(pa, pb), na


# ---------------------------------------------------------------- macro operators

def _torch_bounded(h, h0, rid, sid, p, c):
    """fp64 CPU torch restatement of the bounded macro operator (rte/macro.py:201-236) with the
    reference's per-sample weight gather and bmm."""
    def rms(x):
        return x * torch.rsqrt(x.pow(2).mean(-1, keepdim=True) + 1e-5)

    g = lambda t: t[rid, sid]  # noqa: E731
    n = rms(h)
    z = torch.cat([n, n.mean(dim=1, keepdim=True).expand_as(n), h0], -1)
    low = torch.bmm(torch.nn.functional.silu(torch.bmm(z, g(p["v"]))), g(p["u"]))
    upd = g(p["d_gain"]).unsqueeze(1) * h + low + g(p["bias"]).unsqueeze(1)
    return h + c * g(p["update_scale"]).unsqueeze(1) * torch.tanh(upd)


@pytest.mark.parametrize("scale_init,B,S", [(1.0, 10, 16), (0.5, 10, 16), (1.0, 600, 37)])
def test_macro_operator_grouped_matches_reference(scale_init, B, S):
    """MacroOperators (bounded) on the grouped GEMMs: forward against the numpy oracle, gradients
    of every parameter and of h, h0 against fp64 autograd of the reference formula.  With
    macro_update_scale_init != 1 the per-key update scale is a parameter too.  B=600, S=37 splits
    each sample into uneven row slices (3 of 13, 13, 11 rows) and gives every key many samples."""
    from oracle import macro as MO
    from helpers import rel_err
    from rte_amd.macro import MacroOperators

    cfg = _model_cfg(d_model=128, macro_rank=32, recipe_count=6, depth_choices=[1, 2, 4], t_max=4,
                     macro_update_scale_init=scale_init)
    torch.manual_seed(4)
    mac = MacroOperators(cfg).cuda()
    with torch.no_grad():
        mac.d_gain.normal_(0, 0.1)
        mac.bias.normal_(0, 0.1)
        mac.u.normal_(0, 0.05)
    d = cfg.d_model
    gen = np.random.default_rng(4)
    hn, h0n = gen.standard_normal((B, S, d)), gen.standard_normal((B, S, d))
    rid = torch.tensor(gen.integers(0, 6, B), device="cuda")
    depths = torch.tensor(gen.choice([1, 2, 4], B), device="cuda")
    h = torch.tensor(hn, dtype=torch.float32, device="cuda", requires_grad=True)
    h0 = torch.tensor(h0n, dtype=torch.float32, device="cuda", requires_grad=True)
    G = gen.standard_normal((B, S, d))
    print(f"macro grouped B={B} S={S} d={d}", flush=True)
    out, _ = mac(h, h0, rid, depths)
    (out * torch.tensor(G, dtype=torch.float32, device="cuda")).sum().backward()
    sid = mac.stride_ids_for_depths(depths)
    p = {k: getattr(mac, k).detach().double().cpu() for k in ("d_gain", "bias", "update_scale", "v", "u")}
    want = MO.bounded_apply(hn, h0n, rid.cpu().numpy(), sid.cpu().numpy(), {k: v.numpy() for k, v in p.items()},
                            cfg.macro_update_scale)
    assert_rel(out.detach().double().cpu().numpy() - hn, want - hn, BF16_RTOL, "macro delta")
    scale_param = isinstance(mac.update_scale, torch.nn.Parameter)
    tp = {k: v.clone().requires_grad_(k != "update_scale" or scale_param) for k, v in p.items()}
    th, th0 = torch.tensor(hn, requires_grad=True), torch.tensor(h0n, requires_grad=True)
    ref = _torch_bounded(th, th0, rid.cpu(), sid.cpu(), tp, cfg.macro_update_scale)
    assert rel_err(ref.detach().numpy(), want) < 1e-12
    (ref * torch.tensor(G)).sum().backward()
    for k in ("d_gain", "bias", "v", "u") + (("update_scale",) if scale_param else ()):
        assert_rel(getattr(mac, k).grad.double().cpu().numpy(), tp[k].grad.numpy(), BF16_RTOL, f"macro d{k}")
    assert_rel(h.grad.double().cpu().numpy(), th.grad.numpy(), BF16_RTOL, "macro dh")
    assert_rel(h0.grad.double().cpu().numpy(), th0.grad.numpy(), BF16_RTOL, "macro dh0")


@pytest.mark.parametrize("Bh,Bh0,rep", [(6, 6, 4), (8, 4, 2), (5, 5, 1)])
def test_macro_repeated_sources_match_copies(Bh, Bh0, rep):
    """The bounded operator over Bt = rep * Bh samples reading h[b % Bh] and h0[b % Bh0] equals
    the operator on explicit copies: outputs bitwise, gradients of h, h0 and every parameter
    within the fp32 tolerance (repeats are added in the kernel instead of by autograd)."""
    from helpers import rel_err
    from rte_amd.kernels import hip_ops
    from rte_amd.macro import MacroOperators

    cfg = _model_cfg(d_model=128, macro_rank=32, recipe_count=6, depth_choices=[1, 2, 4], t_max=4,
                     macro_update_scale_init=0.5)
    torch.manual_seed(5)
    mac = MacroOperators(cfg).cuda()
    with torch.no_grad():
        mac.d_gain.normal_(0, 0.1)
        mac.bias.normal_(0, 0.1)
        mac.u.normal_(0, 0.05)
    S, d, Bt = 24, cfg.d_model, rep * Bh
    gen = torch.Generator(device="cuda").manual_seed(6)
    h = torch.randn(Bh, S, d, device="cuda", generator=gen, requires_grad=True)
    h0 = torch.randn(Bh0, S, d, device="cuda", generator=gen, requires_grad=True)
    rid = torch.randint(0, 6, (Bt,), device="cuda", generator=gen)
    sid = torch.randint(0, 3, (Bt,), device="cuda", generator=gen)
    g = torch.randn(Bt, S, d, device="cuda", generator=gen)
    print(f"macro repeated sources Bh={Bh} Bh0={Bh0} rep={rep}", flush=True)
    params = [mac.v, mac.u, mac.d_gain, mac.bias, mac.update_scale]

    def run(hh, hh0):
        for p in params + [h, h0]:
            p.grad = None
        out = mac._apply_bounded(hh, hh0, rid, sid)
        out.backward(g)
        return out.detach().clone(), [p.grad.clone() for p in params + [h, h0]]

    out_r, grads_r = run(h, h0)
    out_c, grads_c = run(h.repeat(rep, 1, 1), h0.repeat(Bt // Bh0, 1, 1))
    assert torch.equal(out_r, out_c), "outputs differ"
    for name, a, b in zip(["v", "u", "gain", "bias", "scale", "h", "h0"], grads_r, grads_c):
        assert rel_err(a.double().cpu().numpy(), b.double().cpu().numpy()) < FP32_RTOL, name


def test_consistency_loss_fused_matches_reference_formula():
    """The consistency loss on one merged operator call (rte/macro.py:342-359 restated with
    explicit copies of h and h0, three operator calls and torch's staged means) gives the same
    loss and gradients within the bf16 tolerance."""
    from helpers import rel_err
    from rte_amd.macro import MacroOperators

    cfg = _model_cfg(d_model=128, macro_rank=32, recipe_count=6, depth_choices=[1, 2, 4], t_max=4)
    torch.manual_seed(7)
    mac = MacroOperators(cfg).cuda()
    with torch.no_grad():
        mac.d_gain.normal_(0, 0.1)
        mac.bias.normal_(0, 0.1)
        mac.u.normal_(0, 0.05)
    B, S, d = 12, 20, cfg.d_model
    gen = torch.Generator(device="cuda").manual_seed(8)
    h = torch.randn(B, S, d, device="cuda", generator=gen, requires_grad=True)
    rid = torch.randint(0, 6, (B,), device="cuda", generator=gen)
    params = [mac.v, mac.u, mac.d_gain, mac.bias, h]
    print("consistency loss B=12 S=20 d=128", flush=True)
    loss = mac.consistency_loss(h, h, rid)
    loss.backward()
    got = [p.grad.clone() for p in params]
    for p in params:
        p.grad = None
    pc = mac.cons_src_idx.numel()
    h_rep = h.unsqueeze(0).expand(pc, *h.shape).reshape(pc * B, S, d)
    r_rep = rid.unsqueeze(0).expand(pc, B).reshape(-1)
    src = mac.cons_src_idx.unsqueeze(1).expand(pc, B).reshape(-1)
    dst = mac.cons_dst_idx.unsqueeze(1).expand(pc, B).reshape(-1)
    direct = mac.apply_vectorized(h_rep, h_rep, r_rep, dst)
    twice = mac.apply_vectorized(mac.apply_vectorized(h_rep, h_rep, r_rep, src), h_rep, r_rep, src)
    ref = (direct - twice).square().mean(dim=-1).mean(dim=-1).mean()
    ref.backward()
    assert abs(loss.item() - ref.item()) <= 1e-5 * max(abs(ref.item()), 1e-12) + 1e-9
    for name, a, p in zip(["v", "u", "gain", "bias", "h"], got, params):
        assert rel_err(a.double().cpu().numpy(), p.grad.double().cpu().numpy()) < BF16_RTOL, name


@pytest.mark.parametrize("d,B,S,depths", [(256, 7, 150, [1, 2, 4]), (1024, 3, 70, [1, 2, 4, 8]), (512, 40, 64, [1, 2, 4])])
def test_macro_fused_operator_matches_reference(d, B, S, depths):
    """The fused rank-32 operator (several 64-row tiles per sample with a ragged last one, d up to
    1024): forward and every gradient against fp64 autograd of the reference formula."""
    from helpers import rel_err
    from rte_amd.kernels import hip_ops
    from rte_amd.macro import MacroOperators

    cfg = _model_cfg(d_model=d, n_heads=d // 64, macro_rank=32, recipe_count=6, depth_choices=depths,
                     t_max=max(depths), macro_update_scale_init=0.5)
    torch.manual_seed(11)
    mac = MacroOperators(cfg).cuda()
    assert hip_ops.macro_fused_supported(mac.v, mac.u)
    with torch.no_grad():
        mac.d_gain.normal_(0, 0.1)
        mac.bias.normal_(0, 0.1)
        mac.u.normal_(0, 0.05)
    gen = torch.Generator(device="cuda").manual_seed(12)
    h = torch.randn(B, S, d, device="cuda", generator=gen, requires_grad=True)
    h0 = torch.randn(B, S, d, device="cuda", generator=gen, requires_grad=True)
    rid = torch.randint(0, 6, (B,), device="cuda", generator=gen)
    sid = torch.randint(0, len(depths), (B,), device="cuda", generator=gen)
    g = torch.randn(B, S, d, device="cuda", generator=gen)
    print(f"macro fused d={d} B={B} S={S}", flush=True)
    out = mac._apply_bounded(h, h0, rid, sid)
    out.backward(g)
    names = ("d_gain", "bias", "update_scale", "v", "u")
    tp = {k: getattr(mac, k).detach().double().cpu().requires_grad_(True) for k in names}
    th = h.detach().double().cpu().requires_grad_(True)
    th0 = h0.detach().double().cpu().requires_grad_(True)
    ref = _torch_bounded(th, th0, rid.cpu(), sid.cpu(), tp, cfg.macro_update_scale)
    (ref * g.double().cpu()).sum().backward()
    assert_rel(out.detach().double().cpu().numpy() - th.detach().numpy(), (ref - th).detach().numpy(), BF16_RTOL,
               "delta")
    for k in names:
        assert_rel(getattr(mac, k).grad.double().cpu().numpy(), tp[k].grad.numpy(), BF16_RTOL, f"d{k}")
    assert_rel(h.grad.double().cpu().numpy(), th.grad.numpy(), BF16_RTOL, "dh")
    assert_rel(h0.grad.double().cpu().numpy(), th0.grad.numpy(), BF16_RTOL, "dh0")
    # same tensor as h and h0 (the hot path's call): one gradient, equal to the sum of both paths
    for p in names:
        getattr(mac, p).grad = None
    hh = h.detach().clone().requires_grad_(True)
    mac._apply_bounded(hh, hh, rid, sid).backward(g)
    th2 = th.detach().clone().requires_grad_(True)
    _torch_bounded(th2, th2, rid.cpu(), sid.cpu(), {k: v.detach() for k, v in tp.items()},
                   cfg.macro_update_scale).mul(g.double().cpu()).sum().backward()
    assert_rel(hh.grad.double().cpu().numpy(), th2.grad.numpy(), BF16_RTOL, "dh (h is h0)")
    assert rel_err(out.detach().double().cpu().numpy(), ref.detach().numpy()) < 1e-3


@pytest.mark.parametrize("d,B,S,depths,one_pass", [(256, 5, 80, [1, 2, 4, 8], False), (512, 16, 64, [1, 2, 4], False),
                                                   (256, 6, 40, [1, 2, 3, 6], False), (512, 16, 64, [1, 2, 4], True),
                                                   (256, 6, 40, [1, 2, 3, 6], True), (256, 5, 64, [1, 2, 4, 8], True),
                                                   (512, 3, 24, [1, 2, 4], True)])
def test_macro_fused_consistency_matches_reference(d, B, S, depths, one_pass):
    """The fused consistency loss (both operator applications, the MSE and the backward in the
    fused kernels) against fp64 autograd of rte/macro.py:342-359 restated with explicit copies:
    chained stride pairs sharing first-application key blocks (strides 1, 2, 4 (, 8): src and dst
    blocks overlap), and unchained pairs in the [dst; src] layout (strides 1, 2, 3, 6).  one_pass:
    the one-pass kernels (csrc/macro_cons.hip: a ragged second half at S = 40, one half at S = 24,
    four first-application blocks with three pairs at strides 1, 2, 4, 8); otherwise the
    per-application fused operator calls."""
    from rte_amd.kernels import hip_ops
    from rte_amd.macro import MacroOperators

    cfg = _model_cfg(d_model=d, n_heads=d // 64, macro_rank=32, recipe_count=6, depth_choices=depths,
                     t_max=max(depths))
    torch.manual_seed(13)
    mac = MacroOperators(cfg).cuda()
    with torch.no_grad():
        mac.d_gain.normal_(0, 0.1)
        mac.bias.normal_(0, 0.1)
        mac.u.normal_(0, 0.05)
    gen = torch.Generator(device="cuda").manual_seed(14)
    h = torch.randn(B, S, d, device="cuda", generator=gen, requires_grad=True)
    rid = torch.randint(0, 6, (B,), device="cuda", generator=gen)
    nf, pc = mac.cons_key_idx.numel(), mac.cons_src_idx.numel()
    if one_pass:
        assert hip_ops.macro_cons_supported(mac.v, mac.u, S, nf, pc)
    print(f"fused consistency d={d} B={B} S={S} pairs={pc} one_pass={one_pass}", flush=True)
    hip_ops.MACRO_CONS_ONE_PASS[0] = one_pass
    try:
        loss = mac.consistency_loss(h, h, rid)
        loss.backward()
    finally:
        hip_ops.MACRO_CONS_ONE_PASS[0] = True
    names = ("d_gain", "bias", "v", "u")
    tp = {k: getattr(mac, k).detach().double().cpu().requires_grad_(k != "update_scale")
          for k in names + ("update_scale",)}
    th = h.detach().double().cpu().requires_grad_(True)
    pc = mac.cons_src_idx.numel()
    r_rep = rid.cpu().repeat(pc)
    src = mac.cons_src_idx.cpu().repeat_interleave(B)
    dst = mac.cons_dst_idx.cpu().repeat_interleave(B)
    h_rep = th.repeat(pc, 1, 1)
    c = cfg.macro_update_scale
    direct = _torch_bounded(h_rep, h_rep, r_rep, dst, tp, c)
    twice = _torch_bounded(_torch_bounded(h_rep, h_rep, r_rep, src, tp, c), h_rep, r_rep, src, tp, c)
    ref = (direct - twice).square().mean()
    ref.backward()
    assert abs(loss.item() - ref.item()) <= 2e-2 * abs(ref.item()) + 1e-9
    for k in names:
        assert_rel(getattr(mac, k).grad.double().cpu().numpy(), tp[k].grad.numpy(), BF16_RTOL, f"d{k}")
    assert_rel(h.grad.double().cpu().numpy(), th.grad.numpy(), BF16_RTOL, "dh")


@pytest.mark.parametrize("n", [1, 7, 4096, 100003, 256 * 64 * 512])
def test_mse_matches_torch(n):
    """Fused mean squared difference and its gradients against float64 torch; bitwise repeatable."""
    from rte_amd.kernels import hip_ops

    gen = torch.Generator(device="cuda").manual_seed(n % 1000)
    a = torch.randn(n, device="cuda", generator=gen, requires_grad=True)
    b = torch.randn(n, device="cuda", generator=gen, requires_grad=True)
    print(f"mse n={n}", flush=True)
    out = hip_ops.mse(a, b)
    (out * 3.0).backward()
    ad, bd = a.detach().double(), b.detach().double()
    want = ((ad - bd) ** 2).mean()
    assert abs(out.item() - want.item()) <= 1e-5 * want.item()
    gw = 3.0 * 2.0 * (ad - bd) / n
    assert_rel(a.grad.double().cpu().numpy(), gw.cpu().numpy(), FP32_RTOL, "mse da")
    assert_rel(b.grad.double().cpu().numpy(), (-gw).cpu().numpy(), FP32_RTOL, "mse db")
    assert torch.equal(hip_ops.mse(a, b), out), "mse not repeatable"


# ---------------------------------------------------------------- fused AdamW

@pytest.mark.parametrize("clip", [None, 0.5])
def test_fused_adamw_matches_torch_adamw(clip):
    """FusedAdamW against torch.optim.AdamW (float64 on the CPU, after the same
    clip_grad_norm_) over three steps: two groups with their own lr / weight decay, a
    parameter without a gradient, the per-group metrics of rte/training.py:385-443 and the
    found_inf skip (no update, no step count)."""
    from rte_amd.optim import FusedAdamW

    torch.manual_seed(0)
    shapes = [(300, 17), (4097,), (64, 64), (5,)]
    init = [torch.randn(s) for s in shapes]
    dev = [torch.nn.Parameter(t.clone().cuda()) for t in init]
    ref = [torch.nn.Parameter(t.clone().double()) for t in init]
    mk = lambda ps: [{"params": ps[:2], "lr": 1e-2, "name": "a"},  # noqa: E731
                     {"params": ps[2:], "lr": 3e-3, "weight_decay": 0.0, "name": "b"}]
    opt = FusedAdamW(mk(dev), weight_decay=0.1, extra_metrics=[("first_two", dev[:2], "b")], clip_grad_norm=clip)
    ropt = torch.optim.AdamW(mk(ref), weight_decay=0.1, foreach=False)
    for step in range(4):
        grads = [torch.randn(s) * (1 + step) for s in shapes]
        for i, (p, q) in enumerate(zip(dev, ref)):
            if i == 3 and step == 1:  # no gradient for this parameter this step
                p.grad = q.grad = None
                continue
            p.grad = grads[i].cuda()
            q.grad = grads[i].double()
        if step == 2:  # non-finite step: nothing changes
            opt.found_inf = torch.ones((), device="cuda")
            before = [p.detach().clone() for p in dev]
            opt.step()
            opt.found_inf = None
            for a, b in zip(before, dev):
                assert torch.equal(a, b.detach())
            continue
        if clip is not None:
            torch.nn.utils.clip_grad_norm_([q for q in ref if q.grad is not None], clip)
        gsq = {n: sum(float(q.grad.pow(2).sum()) for q in qs if q.grad is not None)
               for n, qs in (("a", ref[:2]), ("b", ref[2:]), ("first_two", ref[:2]))}
        psq = {n: sum(float(q.detach().pow(2).sum()) for q in qs)
               for n, qs in (("a", ref[:2]), ("b", ref[2:]), ("first_two", ref[:2]))}
        lrs = {"a": 1e-2, "b": 3e-3, "first_two": 3e-3}
        opt.step()
        ropt.step()
        m = opt.metrics_dict()
        for n in ("a", "b", "first_two"):
            gn = gsq[n] ** 0.5
            np.testing.assert_allclose(float(m[f"grad_norm_{n}"]), gn, rtol=1e-5)
            np.testing.assert_allclose(float(m[f"update_ratio_{n}"]), lrs[n] * gn / max(psq[n] ** 0.5, 1e-12),
                                       rtol=1e-5)
        for p, q in zip(dev, ref):
            assert_rel(p.detach().double().cpu().numpy(), q.detach().numpy(), 1e-5, "param")
            st, rst = opt.state[p], ropt.state[q]
            if rst:
                assert float(st["step"]) == float(rst["step"])
                assert_rel(st["exp_avg"].double().cpu().numpy(), rst["exp_avg"].numpy(), 1e-5, "exp_avg")
                assert_rel(st["exp_avg_sq"].double().cpu().numpy(), rst["exp_avg_sq"].numpy(), 1e-5, "exp_avg_sq")
