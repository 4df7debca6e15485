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
  swiglu.*                   finite differences (fp64) + torch autograd on CPU
  cluster_pool.*             all clusters with uniform weights == dense SwiGLU / C;
                             k = 1 equals the reference per-cluster loop; finite differences
  attention.rope / rmsnorm   complex-rotation closed form, norm preservation, manual formula
  losses.*                   closed forms; p = 1 correction == exact loss
"""
