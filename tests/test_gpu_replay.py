"""The fused exact replay of the banked core (rte_amd/kernels/replay_core.py, csrc/replay.hip):
every pass of forward_exact (rte/models.py:416-512 over BankedRecursiveCore.forward_step,
rte/layers.py:806-870) as one node, against fp64 autograd of the per-pass torch restatement
_torch_core_step (itself checked against oracle/banked.py in test_gpu_model.py), composed over
the passes: outputs, a kept intermediate state, the gradient of h0 and of every core parameter
within the bf16 tolerance.  Cases: the bench's cfg3 layout (d512, 8 heads of which 2 active, 64
slabs x 32 of which 8 active, depth 4, one audited sample), and mixed recipes including the dense
fallback with ragged S, inactive samples, slabs of two 32-neuron blocks and the input skip."""

from __future__ import annotations

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

BF16_RTOL = 2e-2


@pytest.fixture(scope="module", autouse=True)
def _hip():
    from rte_amd import _lib

    if not _lib.device_ready():
        pytest.fail("HIP backend not ready on this GPU box (library or gfx950 device missing)")
    yield


def _rel(a, b):
    a, b = torch.as_tensor(a).double(), torch.as_tensor(b).double()
    return float((a - b).norm() / b.norm().clamp_min(1e-300))


CASES = {
    "cfg3": dict(d_model=512, n_heads=8, d_ff=2048, head_groups=8, ffn_groups=64, active_head_groups=2,
                 active_ffn_groups=8, recipe_count=16, t_max=4, depth_choices=[1, 2, 4], skip=False, B=1, S=64,
                 rids=None, active=None),
    "mixed": dict(d_model=256, n_heads=4, d_ff=512, head_groups=4, ffn_groups=8, active_head_groups=1,
                  active_ffn_groups=2, recipe_count=5, t_max=3, depth_choices=[1, 2, 3], skip=True, B=3, S=40,
                  rids=[[0, 2, 4], [1, 0, 3], [2, 4, 0]],
                  active=[[True, True, True], [True, False, True], [False, False, True]]),
}


def _core(case, seed):
    from rte_amd.config import ModelConfig
    from rte_amd.layers import BankedRecursiveCore
    from rte_amd.recipes import RecipeBank

    c = CASES[case]
    cfg = ModelConfig(topology="recursive", vocab_size=64, d_model=c["d_model"], n_heads=c["n_heads"], d_ff=c["d_ff"],
                      n_dense_layers=2, n_prelude=1, n_coda=1, t_max=c["t_max"], depth_choices=c["depth_choices"],
                      attn_banks=1, ffn_banks=1, head_groups=c["head_groups"], ffn_groups=c["ffn_groups"],
                      active_head_groups=c["active_head_groups"], active_ffn_groups=c["active_ffn_groups"],
                      recipe_count=c["recipe_count"], use_recursive_input_skip=c["skip"])
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


def _params(core):
    mods = {"norm1": core.norm1.weight, "norm2": core.norm2.weight, "wqkv": core.attn.wqkv, "wo": core.attn.wo,
            "wug": core.mlp.wug, "wd": core.mlp.wd, "pass_gamma1": core.pass_gamma1, "pass_beta1": core.pass_beta1,
            "pass_gamma2": core.pass_gamma2, "pass_beta2": core.pass_beta2, "pass_attn_scale": core.pass_attn_scale,
            "pass_mlp_scale": core.pass_mlp_scale}
    if core.alpha_inj is not None:
        mods["alpha_inj"] = core.alpha_inj
    return mods


def _inputs(case, cfg, seed, S=None):
    c = CASES[case]
    B, S, T = c["B"], S or c["S"], cfg.t_max
    g = torch.Generator().manual_seed(seed)
    h0 = torch.randn(B, S, cfg.d_model, generator=g, dtype=torch.float64)
    rids = (torch.tensor(c["rids"]) if c["rids"] is not None
            else torch.randint(1, cfg.recipe_count, (T, B), generator=g))
    active = None if c["active"] is None else torch.tensor(c["active"])
    G = torch.randn(B, S, cfg.d_model, generator=g, dtype=torch.float64)
    Gs = torch.randn(B, S, cfg.d_model, generator=g, dtype=torch.float64)
    return h0, rids, active, G, Gs


@pytest.mark.parametrize("case", ["cfg3", "mixed"])
def test_replay_core_matches_fp64_reference(case):
    from oracle import attention as AO
    from test_gpu_model import _core_params_np, _oracle_recipes, _torch_core_step

    cfg, core = _core(case, 3)
    assert core.replay_fused_ok(torch.empty(1, 1, cfg.d_model, device="cuda"))
    h0n, rids, active, G, Gs = _inputs(case, cfg, 4)
    B, S, d, T = h0n.shape[0], h0n.shape[1], cfg.d_model, cfg.t_max
    h0 = h0n.float().cuda().requires_grad_(True)
    print(f"fused replay {case}: B={B} S={S} d={d} T={T}", flush=True)
    out, state = core.forward_replay(h0, rids.cuda(), None if active is None else active.cuda(), keep=[0])
    ((out * G.float().cuda()).sum() + (state * Gs.float().cuda()).sum()).backward()

    recipes = _oracle_recipes(core)
    base = _core_params_np(core)
    tp = {k: torch.tensor(v, requires_grad=True) for k, v in base.items() if v is not None}
    cos, sin = (torch.tensor(t) for t in AO.rope_tables(d // cfg.n_heads, S))
    th0 = h0n.clone().requires_grad_(True)
    h = th0
    states = []
    for t in range(T):
        act = [True] * B if active is None else active[t].tolist()
        h = _torch_core_step(h, th0, rids[t].tolist(), act, recipes, tp, t, cfg, cos, sin)
        states.append(h)
    ((h * G).sum() + (states[0] * Gs).sum()).backward()

    assert _rel(out.detach().cpu() - h0n, h.detach() - h0n) < BF16_RTOL, "h_T"
    assert _rel(state.detach().cpu() - h0n, states[0].detach() - h0n) < BF16_RTOL, "state after pass 1"
    if active is not None:  # sample 1 sits out passes 2 and 3: it leaves with its pass-1 rows exactly
        assert torch.equal(out[1].detach(), state[1].detach())
    errs = {"h0": _rel(h0.grad.cpu(), th0.grad)}
    for name, param in _params(core).items():
        assert param.grad is not None, name
        errs[name] = _rel(param.grad.cpu(), tp[name].grad)
    bad = {k: v for k, v in errs.items() if not v < BF16_RTOL}
    assert not bad, bad


def test_replay_core_repeats_bitwise_and_matches_unfused_path():
    """Two runs give identical outputs and gradients; the unfused per-operator passes
    (fused_replay off, here at S = 40: the O-projection reads the token-major attention rows
    without the power-of-two split) agree within the bf16 tolerance."""
    from rte_amd.layers import BankedRecursiveCore

    cfg, core = _core("mixed", 5)
    h0n, rids, active, G, _ = _inputs("mixed", cfg, 6)
    rc, ac, Gc = rids.cuda(), active.cuda(), G.float().cuda()

    def run(fused):
        BankedRecursiveCore.fused_replay = fused
        try:
            core.zero_grad(set_to_none=True)
            h0 = h0n.float().cuda().requires_grad_(True)
            if fused:
                out, = core.forward_replay(h0, rc, ac)
            else:
                h, weights = h0, core.prepare()
                for t in range(cfg.t_max):
                    hs = core.attn.recipe_head_scale[rc[t]]
                    h = core.forward_step(h, h0, rc[t], ac[t], pass_idx=t, weights=weights, head_scale=hs)
                out = h
            (out * Gc).sum().backward()
            return out.detach().clone(), h0.grad.clone(), {n: p.grad.clone() for n, p in _params(core).items()}
        finally:
            BankedRecursiveCore.fused_replay = True

    print("fused replay repeat + unfused comparison (mixed)", flush=True)
    o1, g1, p1 = run(True)
    o2, g2, p2 = run(True)
    assert torch.equal(o1, o2) and torch.equal(g1, g2)
    for n in p1:
        assert torch.equal(p1[n], p2[n]), n
    o3, g3, p3 = run(False)
    h0c = h0n.float().cuda()
    assert _rel(o1 - h0c, o3 - h0c) < BF16_RTOL
    assert _rel(g1, g3) < BF16_RTOL
    for n in p1:
        assert _rel(p1[n], p3[n]) < BF16_RTOL, n
