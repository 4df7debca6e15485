"""Kernel boundary: `optimized` (k_* dispatch symbols + backend_status), `hip_ops`
(autograd operators over librte_hip), `cluster_pool_ffn` (reference cluster-pool API)."""
