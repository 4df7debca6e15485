"""CPU tests of host-side logic that needs no device: configuration schema, recipe tables,
router auxiliary losses, the audit samplers and the strict / fallback contract."""

from __future__ import annotations

import pytest
import torch

from rte_amd.config import ExperimentConfig, ModelConfig, TrainingConfig, config_from_dict, load_config


def _model(**over):
    base = dict(topology="recursive", vocab_size=128, d_model=16, n_heads=4, d_ff=64, n_dense_layers=5, n_prelude=1,
                n_coda=1, t_max=4, depth_choices=[1, 2, 4], attn_banks=1, ffn_banks=3, head_groups=4, ffn_groups=4,
                active_head_groups=1, active_ffn_groups=1, recipe_count=4)
    base.update(over)
    return base


def test_unknown_config_keys_rejected():
    with pytest.raises(ValueError, match="unknown"):
        config_from_dict({"model": {**_model(), "bogus": 1}, "training": {"mode": "recursive_macro"}})
    with pytest.raises(ValueError, match="unknown"):
        config_from_dict({"model": _model(), "training": {"mode": "recursive_macro", "nope": 2}})


def test_reference_tiny_yaml_schema_loads(tmp_path):
    # the keys of the reference's configs/tiny.yaml fixture
    import yaml

    raw = {"run_name": "tiny", "output_dir": "runs", "model": {**_model(), "tie_embeddings": True, "use_rope": True,
           "use_recursive_input_skip": True, "fairness_tolerance": 0.01, "macro_rank": 2, "router_hidden": 16},
           "training": {"mode": "recursive_macro_shortlist", "optimizer": "adamw", "lr": 0.0005, "weight_decay": 0.01,
                        "batch_size": 2, "seq_len": 12, "grad_accum_steps": 1, "seed": 1337, "audit_p_min": 0.25,
                        "audit_p_max": 1.0, "lambda_cons": 0.001},
           "output": {"mode": "shortlist", "num_clusters": 8, "shortlist_top_clusters": 2, "shortlist_max_tokens": 16,
                      "hard_negatives": 4, "random_negatives": 4},
           "data": {"dataset": "synthetic", "tokenizer": "gpt2_bpe", "synthetic_tokens": 4096}}
    p = tmp_path / "tiny.yaml"
    p.write_text(yaml.safe_dump(raw))
    cfg = load_config(p)
    assert cfg.training.mode == "recursive_macro_shortlist" and cfg.output.shortlist_max_tokens == 16


def test_model_config_validation():
    with pytest.raises(ValueError):
        ModelConfig(**_model(d_model=18))
    with pytest.raises(ValueError, match="multiple of 32"):
        ModelConfig(**_model(d_ff=64, ffn_kind="cluster_pool", ffn_clusters=4))
    ModelConfig(**_model(d_ff=256, ffn_groups=4, ffn_kind="cluster_pool", ffn_clusters=4, ffn_top_k=2))


def test_fixed_count_implies_sampler_and_bounds():
    tr = TrainingConfig(mode="recursive_macro", audit_fixed_count=2, batch_size=4)
    assert tr.audit_sampler == "fixed_count" and tr.audit_fixed_count_per_batch == 2
    with pytest.raises(ValueError):
        TrainingConfig(mode="recursive_macro", audit_fixed_count=5, batch_size=4)


def test_recipe_bank_templates():
    from rte_amd.recipes import RecipeBank

    bank = RecipeBank(ModelConfig(**_model()))
    assert bank.recipes[0].dense_fallback and bank.recipes[0].ffn_groups == (0, 1, 2, 3)
    # sparse recipes walk (bank, slot) round robin (rte/recipes.py:77-99)
    assert [r.ffn_groups for r in bank.recipes[1:]] == [(0,), (1,), (2,)]
    assert [r.ffn_banks for r in bank.recipes[1:]] == [(0,), (0,), (0,)]
    assert bank.active_touch_table[0] > bank.active_touch_table[1]


def test_router_aux_losses_closed_form():
    from rte_amd.training import router_aux_losses

    tr = TrainingConfig(mode="recursive_macro", lambda_load=1.0, lambda_cover=1.0, lambda_depth=1.0, coverage_min=0.5)
    probs = torch.full((3, 4), 0.25)
    out = router_aux_losses(probs, torch.tensor([1.0, 2.0, 3.0]), torch.tensor([0.0, 0.5, 1.0, 0.25]), tr)
    assert abs(float(out["load"])) < 1e-6  # uniform usage: r * sum(p^2) - 1 = 0
    assert abs(float(out["cover"]) - (0.25 + 0.0625)) < 1e-6
    assert abs(float(out["depth"]) - 2.0) < 1e-6


def test_fixed_count_sampler_inclusion_probability():
    # rte tests/test_audit_fixes.py:62-79: one audit per batch of 8 gives p = 1/8
    from rte_amd.audit import AuditEngine

    eng = AuditEngine(TrainingConfig(mode="recursive_macro", audit_fixed_count=1, batch_size=8))
    mask, p, chosen, k = eng.sample_mask_with_prob(torch.full((8,), 0.3), seed=4)
    assert int(mask.sum()) == 1 and k == 1 and chosen.numel() == 1
    assert torch.allclose(p, torch.full((8,), 1 / 8))


def test_bernoulli_cap_inclusion_probability():
    # rte tests/test_audit_fixes.py:52-59: cap halves an all-audited batch -> two-stage p
    from rte_amd.audit import AuditEngine

    eng = AuditEngine(TrainingConfig(mode="recursive_macro", audit_cap=2, batch_size=4, audit_p_max=1.0))
    mask, p, _, _ = eng.sample_mask_with_prob(torch.full((4,), 0.5), seed=0)
    assert int(mask.sum()) <= 2
    if eng.last_candidate_count > 2:
        assert torch.allclose(p, torch.full((4,), 0.5 * 2 / eng.last_candidate_count))


def test_strict_cuda_refuses_cpu_tensors():
    # rte tests/test_kernels.py:57-63
    from rte_amd.kernels import optimized

    optimized.set_strict_cuda(True)
    try:
        with pytest.raises(RuntimeError, match="strict_cuda"):
            optimized.k_fused_rmsnorm(torch.randn(2, 3, 4), torch.ones(4))
    finally:
        optimized.set_strict_cuda(False)


def test_hot_symbols_never_fall_back_on_cpu():
    from rte_amd.kernels import optimized

    if optimized.hip_available():
        pytest.skip("ROCm device present")
    with pytest.raises(RuntimeError, match="HIP backend is required"):
        optimized.k_fused_rmsnorm(torch.randn(2, 3, 8), torch.ones(8))
    with pytest.raises(RuntimeError):
        optimized.cuda_required()
    st = optimized.backend_status()
    assert st["mode"] == "hip_unavailable" and st["uses_reference_fallback"] is False
    assert st["symbols"]["k_swiglu_dense"] == "hip"


def test_glue_symbols_match_reference_math():
    from rte_amd.kernels import optimized

    hidden = torch.randn(4, 2, 3)
    packed = optimized.k_pack_by_recipe(hidden, torch.tensor([2, 1, 2, 1]), torch.tensor([0, 0, 1, 1]))
    assert torch.allclose(optimized.k_unpack_from_recipe(packed.packed, packed.inverse_permutation), hidden)
    # the shortlist logits run on the HIP kernel: without a device they fail loudly
    with pytest.raises(RuntimeError, match="HIP backend is required"):
        optimized.k_logits_shortlist(torch.randn(2, 3, 4), torch.randn(10, 4), torch.randint(0, 10, (2, 3, 5)))


def test_accelerated_modes_only():
    from rte_amd.training import TrainEngine

    cfg = ExperimentConfig(model=ModelConfig(**_model()), training=TrainingConfig(mode="recursive_exact_route_em"))
    with pytest.raises(NotImplementedError):
        TrainEngine(cfg, device=torch.device("cpu"))


def test_deterministic_gathers_match_indexing_gradients():
    from rte_amd.gather import gather_cols, gather_rk, gather_rows

    torch.manual_seed(0)
    table = torch.randn(4, 3, 5, 2, dtype=torch.float64, requires_grad=True)
    r = torch.tensor([1, 3, 1, 0, 1])
    s = torch.tensor([2, 0, 2, 1, 0])
    g = torch.randn(5, 5, 2, dtype=torch.float64)
    (gather_rk(table, r, s) * g).sum().backward()
    ref = torch.zeros_like(table).index_put_((r, s), g, accumulate=True)
    assert torch.allclose(table.grad, ref)
    mat = torch.randn(6, 7, requires_grad=True)
    cols = torch.tensor([6, 1, 1, 3])
    out = gather_cols(mat, cols)
    assert torch.equal(out, mat[:, cols])
    out.sum().backward()
    assert torch.allclose(mat.grad, torch.zeros(6, 7).index_add_(1, cols, torch.ones(6, 4)))
    w = torch.randn(5, 3, requires_grad=True)
    gather_rows(w, torch.tensor([4, 4, 0])).sum().backward()
    assert torch.allclose(w.grad[4], torch.full((3,), 2.0)) and torch.allclose(w.grad[1], torch.zeros(3))


def test_staged_reductions_equal_torch_losses():
    """The per-row forms used for the distillation KL and the consistency MSE equal
    F.kl_div(batchmean) and F.mse_loss."""
    from rte_amd.macro import macro_distill_loss

    torch.manual_seed(3)
    hot, exact = torch.randn(2, 5, 11, dtype=torch.float64), torch.randn(2, 5, 11, dtype=torch.float64)
    hh, eh = torch.randn(2, 5, 4, dtype=torch.float64), torch.randn(2, 5, 4, dtype=torch.float64)
    t = 1.7
    got = macro_distill_loss(hh, eh, hot, exact, lambda_kl=1.0, temperature=t)["kl"]
    want = torch.nn.functional.kl_div(torch.log_softmax(hot / t, -1), torch.softmax(exact / t, -1),
                                      reduction="batchmean") * t * t
    assert torch.allclose(got, want, rtol=1e-12, atol=1e-12)
    a, b = torch.randn(6, 7, 9, dtype=torch.float64), torch.randn(6, 7, 9, dtype=torch.float64)
    assert torch.allclose((a - b).square().mean(dim=-1).mean(dim=-1).mean(), torch.nn.functional.mse_loss(a, b))


def test_router_subset_indexes_each_field_on_first_read():
    """The audited rows' routing decisions equal direct indexing of every field, and a field
    that is never read is never indexed (nested subsets compose)."""
    from rte_amd.config import ModelConfig
    from rte_amd.routing import Router

    cfg = ModelConfig(**_model(d_model=32, n_heads=4, d_ff=64))
    torch.manual_seed(0)
    route = Router(cfg)(torch.randn(6, 5, 32))
    idx = torch.tensor([4, 1, 3])
    sub = route.subset(idx)
    assert "recipe_probs" not in vars(sub)
    for name in route.__dataclass_fields__:
        v = getattr(route, name)
        got = getattr(sub, name)
        if isinstance(v, torch.Tensor):
            assert torch.equal(got, v[idx]), name
        else:
            assert got == v, name
    assert "recipe_probs" in vars(sub)
    mask = torch.tensor([True, False, True])
    assert torch.equal(sub.subset(mask).depth, route.depth[idx][mask])


def test_bench_refuses_more_than_one_gpu():
    """bench.py --gpus N with N > 1 prints a message and exits nonzero (one GPU per box)."""
    import subprocess
    import sys
    from pathlib import Path

    root = Path(__file__).resolve().parents[1]
    r = subprocess.run([sys.executable, str(root / "bench.py"), "--gpus", "2"], capture_output=True, text=True,
                       cwd=root, timeout=300)
    assert r.returncode != 0
    assert "one GPU" in r.stdout


def test_bf16_prefetch_tables():
    """The one-launch weight-cast plan: contiguous views cast flat, 2-D transposed views by
    tiles, other strides left to the per-use cast; repeated views share one job and buffer."""
    from rte_amd import _lib
    from rte_amd.kernels import hip_ops

    lib = _lib.load()
    w = torch.nn.Parameter(torch.randn(2, 48, 80))
    v = torch.nn.Parameter(torch.randn(1000))
    t = w[1].t()                 # [80, 48], stride (1, 80): transposed view
    odd = v[::2]                 # stride 2: not planned
    rec = [(w, tuple(w.shape), tuple(w.stride()), 0, None),
           (w, tuple(t.shape), tuple(t.stride()), t.storage_offset(), None),
           (v, tuple(odd.shape), tuple(odd.stride()), 0, None),
           (w, tuple(t.shape), tuple(t.stride()), t.storage_offset(), "side")]
    plan = hip_ops.Bf16Prefetch(enabled=False)
    plan._build(rec)
    jobs, blk, nblk, outs, _ = plan.tables
    jobs = jobs.tolist()
    assert len(jobs) == 2 and len(outs) == 2 and len(plan.entries) == 3
    assert jobs[0][2:7] == [1, w.numel(), 0, 0, 0]
    assert jobs[1][2:7] == [80, 48, 80, 1, lib.rte_cast_many_blocks(0, 1, w.numel())]
    assert jobs[1][0] == t.data_ptr() and tuple(outs[1].shape) == (80, 48)
    assert nblk == lib.rte_cast_many_blocks(0, 1, w.numel()) + lib.rte_cast_many_blocks(1, 80, 48)
    assert blk.tolist() == [0] * jobs[1][6] + [1] * (nblk - jobs[1][6])
    assert plan.entries[1][5] == plan.entries[2][5] == 1  # same view on two streams: one buffer
