"""CPU oracle for the recursive_macro hot path — TEST INFRASTRUCTURE ONLY.

A from-scratch numpy restatement of the reference's PyTorch math for each
operator the HIP library replaces.  Every function cites the reference file:line
(paths relative to the reference repository, rte/ = src/recursive_training_engine/)
it follows.  Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg
may import this package, and only as the checker or the CPU baseline; the
product path (speedup-thingy_amd/) never does.

How each function is pinned (tests/test_oracle.py):
  routing.route_topk         brute-force sort with the (value desc, index asc) rule;
                             k = 1 equals the reference argmax routing
  routing.pack_index         brute-force per-cluster ascending lists; permutation round trip
  routing.static_pack_gather the padded pack_index / flat_gather of the reference builder
  routing.static_centers     brute-force per-token loop over the centres; invariance of the
                             choice under positive scaling of a token's features; k = 1 of
                             route_topk on the centre scores
  swiglu.*                   finite differences (fp64) + torch autograd on CPU
  cluster_pool.*             all clusters with uniform weights == dense SwiGLU / C;
                             k = 1 equals the reference per-cluster loop; finite differences
  attention.rope / rmsnorm   complex-rotation closed form, norm preservation, manual formula
  losses.*                   closed forms; p = 1 correction == exact loss
  distill.distill            closed forms: hot == exact (all losses 0, cosines / ratios 1);
                             hot - h0 = 2 (exact - h0) (delta_dir 0, delta_rms (ln 2)^2);
                             hot = 3 exact (rms_trust (ln 3)^2); smooth-L1 of constant offsets
                             0.5 / 1 / 2; the two-class KL in closed form at t = 1 and 2
  distill.distill_grad       torch autograd (fp64) of the reference formulation
  macro.bounded_apply        hand-worked values: one-hot v / u expose rmsnorm(h)[s, j],
                             mean_s rmsnorm(h)[j] and h0[s, j] separately on a 2x3x4 input with
                             round rms values; u = gain = 0 closed form; tanh bound; per-key
                             locality and permutation equivariance
  macro.grouped_linear*      explicit loop + torch autograd
  router.router              torch autograd-free restatement checked against nn.Linear / softmax /
                             argmax run with torch on the CPU (same weights), entropies and
                             expected depth by hand on a 2-class case
  router.factorized_topk     brute-force enumeration of the (bank, bank, slot, slot) tuples
  banked.recipe_templates    two hand-enumerated recipe tables (every recipe's banks and
                             groups) with zero balance spread; recipe 0 == dense bank

  step_port.StepPort         the whole recursive_macro step (tests/test_step_port.py): its loss,
                             term by term (corrected CE, every distillation term, consistency,
                             router load / cover / depth), equals a composition of the functions
                             above (attention, routed pool, router, bounded_apply, banked core,
                             cross_entropy, audit.correction, distill.distill) on a small model
                             with per-sample depths, to 1e-6; its gradients equal central
                             finite differences of its own loss (float64) on 40 entries of 20
                             parameters of every kind, with the step's decisions and the
                             distillation's detached operands held fixed.  It is the checker of
                             the GPU step (tests/test_gpu_step_parity.py) and the cfg3 CPU
                             baseline bench.py times.
  pool_port.layer_*          the cfg1 layer's two CPU forms (per-cluster loop, preindexed bmm):
                             outputs equal cluster_pool.routed_fwd on the same routing; the two
                             forms' gradients agree and match finite differences
                             (tests/test_pool_port.py).  Timed as the cfg1 CPU baseline.
"""
