/*
 * librte_hip — C ABI of the MI355X (gfx950) kernels behind the recursive_macro
 * hot path.  Plain pointers and sizes only: device pointers to caller-owned
 * buffers, `stream` is a hipStream_t passed as void*.  Nothing here allocates
 * device memory; workspaces are sized by the *_workspace_bytes helpers and
 * passed in.  Every int-returning entry point returns 0 on success, otherwise a
 * nonzero code with a message in rte_last_error() (per host thread).
 *
 * Element types: "bf16" buffers hold raw bfloat16 words (uint16), "f32" IEEE
 * float, index buffers int32.  Matrices are row-major unless stated.
 *
 * Reference interfaces replaced (paths relative to the reference repository,
 * src/recursive_training_engine = rte/):
 *   rte/kernels/optimized.py:58-154 k_* dispatch symbols, backend_status :27-43
 *   rte/kernels/cluster_pool_ffn.py:32-87 Triton slot/pack/gather kernels,
 *       :129-241 routing, pack-index build, preindexed pooled FFN, grad scatter
 *   rte/kernels/active_swiglu_triton.py:20-102 fused SwiGLU fwd/bwd
 *   rte/layers.py:53-87 fused QKV attention projection + dense SwiGLU
 */
#ifndef RTE_HIP_H
#define RTE_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ---- status (replaces backend_status(), rte/kernels/optimized.py:27-43) ---- */
int rte_abi_version(void);
const char* rte_last_error(void);
/* Writes "arch=gfx950;cus=256;lds_per_block=...;..." for the current device. */
int rte_device_info(char* buf, int buf_len);

/* ---- generic bf16 MFMA GEMM:  C[m,n] = alpha * sum_k A(m,k) B(n,k) (+beta C) (+resid) ----
 * a_t == 0: A(m,k) = a[m*lda + k]   a_t == 1: A(m,k) = a[k*lda + m]  (same for B with n)
 * a_rows / b_rows (optional, int32): memory-row indirection, applied to m (a_t=0) or k (a_t=1).
 * c_f32 selects fp32 or bf16 output; resid (fp32, optional) is added element-wise.
 * Replaces the torch matmuls behind nn.Linear in rte/layers.py:53-87. */
int rte_gemm_bf16(const void* a, int64_t lda, int a_t, const int32_t* a_rows,
                  const void* b, int64_t ldb, int b_t, const int32_t* b_rows,
                  void* c, int64_t ldc, int c_f32, int M, int N, int K,
                  float alpha, float beta, const float* resid, int64_t ld_resid,
                  void* workspace, size_t workspace_bytes, void* stream);
/* Workspace that lets a dense problem of this shape split its reduction along K
 * (fp32 partials summed in a fixed order: deterministic).  A smaller or NULL
 * workspace only disables the split. */
size_t rte_gemm_workspace_bytes(int M, int N, int K);

/* Same, with attention-layout operands: row r -> (r / rdiv)*rs_hi + (r % rdiv)*ld and
 * contiguous index c -> (c / cdiv)*cs_hi + c % cdiv  (rdiv/cdiv = 0: plain).
 * layout[] = {ld, rdiv, rs_hi, cdiv, cs_hi}.  Used for [B,H,S,hd] attention outputs
 * feeding the output projection (rte/layers.py:73-75). */
int rte_gemm_bf16_split(const void* a, const int64_t* a_layout, int a_t,
                        const void* b, const int64_t* b_layout, int b_t,
                        void* c, int64_t ldc, int c_f32, int M, int N, int K,
                        float alpha, float beta, const float* resid, int64_t ld_resid,
                        void* workspace, size_t workspace_bytes, void* stream);

/* ---- routing (rte/kernels/cluster_pool_ffn.py:129-140 generalised to per-token top-k;
 *      rte/models.py:300-309 softmax-over-selected combine rule) ----
 * ids[t*k + j]: j-th best cluster (value descending, ties -> lower index, NaN first).
 * weights: softmax over the k selected logits.  C <= 1024, k <= 16. */
int rte_route_topk(const float* logits, int T, int C, int k, int32_t* ids, float* weights, void* stream);

/* ---- router GEMM, top-k and pack in two launches (replaces the router linear + top-k routing of
 *      rte/kernels/cluster_pool_ffn.py:129-140 / rte/models.py:300-309 and the pack index build
 *      :165-189 for the routed cluster pool) ----
 * x bf16 [T, d], wr bf16 [C, d]: logits = x wr^T (fp32 accumulation; written to logits [T, C] fp32
 * when it is not NULL), ids int32 [T, k] / weights fp32 [T, k] = route_topk of those logits (the
 * same selection order and softmax, bitwise), and the pack outputs of rte_pack_index for cl = ids
 * (offsets [C+1], tok_of_slot, pair_of_slot, slot_of_pair, w_of_slot [T*k], all written).
 * C in {32, 64, 128}, 1 <= k <= min(16, C), d % 64 == 0; workspace
 * rte_route_pack_workspace_bytes(T, C) bytes (per-block cluster counts). */
size_t rte_route_pack_workspace_bytes(int T, int C);
int rte_route_pack(const void* x, int T, int d, const void* wr, int C, int k, int32_t* ids, float* weights,
                   int32_t* offsets, int32_t* tok_of_slot, int32_t* pair_of_slot, int32_t* slot_of_pair,
                   float* w_of_slot, float* logits, void* workspace, size_t workspace_bytes, void* stream);

/* ---- deterministic pack index (replaces build_static_pack_gather_indices
 *      rte/kernels/cluster_pool_ffn.py:165-189 and _assign_slots_kernel :32-45) ----
 * cl[p] = cluster of pair p (p = t*k + j).  Stable counting sort by cluster:
 *   offsets[C+1], tok_of_slot[P] = p / k, pair_of_slot[P], slot_of_pair[P] (-1 if cl invalid),
 *   w_of_slot[P] = w[p] (1 if w is NULL).  invalid (optional, int32, caller-zeroed) counts
 *   pairs whose cluster id is outside [0, C).  Any output pointer may be NULL. */
size_t rte_pack_workspace_bytes(int P, int C);
int rte_pack_index(const int32_t* cl, int P, int C, int k, const float* w, int32_t* offsets,
                   int32_t* tok_of_slot, int32_t* pair_of_slot, int32_t* slot_of_pair,
                   float* w_of_slot, int32_t* invalid, void* workspace, size_t workspace_bytes,
                   void* stream);

/* rte_pack_index without a workspace argument: no counterpart in the reference.  For callers
 * that cannot allocate device memory (code under HIP graph capture, tight serving loops, harnesses
 * that forbid hipMalloc).  Same outputs as rte_pack_index (bit-identical); its histogram lives in a
 * static device array of rte_pack_index_noalloc_max_bytes() bytes (1 MiB) per device, so sizes whose
 * rte_pack_workspace_bytes(P, C) exceeds that are rejected with an error.  The library allocates
 * nothing in this call.  Every call on one device shares that device's array: calls that overlap
 * on one device (other streams or host threads) race. */
size_t rte_pack_index_noalloc_max_bytes(void);
int rte_pack_index_noalloc(const int32_t* cl, int P, int C, int k, const float* w, int32_t* offsets,
                           int32_t* tok_of_slot, int32_t* pair_of_slot, int32_t* slot_of_pair, float* w_of_slot,
                           int32_t* invalid, void* stream);

/* out[t] = resid[t] + extra[t] + sum_{j<k} rows[t*k + j]  (j ascending; fp32 accumulation)
 * rows, extra: bf16; resid: f32 (optional); out: f32 (out_f32=1) or bf16.
 * slot_of_pair (optional, from rte_pack_index): pairs whose slot is -1 (invalid cluster id,
 * dropped by the pack) are skipped, so their rows are never read.
 * Replaces _gather_y_kernel (rte/kernels/cluster_pool_ffn.py:69-87) plus the top-k sum. */
int rte_combine_rows(const void* rows, int T, int k, int d, const int32_t* slot_of_pair, const void* extra,
                     const float* resid, void* out, int out_f32, void* stream);

/* Routing-weight backward: dlogits[t, ids[t,j]] = w_j (dw_j - sum_i w_i dw_i), zero elsewhere.
 * dw_slot is indexed by slot (slot_of_pair maps pairs).  Either output may be NULL. */
int rte_route_bwd(const int32_t* ids, const float* w, const float* dw_slot, const int32_t* slot_of_pair,
                  int T, int C, int k, void* dlogits_bf16, float* dlogits_f32, void* stream);

/* ---- pack of per-sample route lists (the banked FFN's recipe routing, rte/layers.py:744-779):
 *      every token of sample b visits clusters routes[recipe_ids[b], j] (int32 [n_recipes, kmax],
 *      -1 = none; recipe ids outside [0, n_recipes) route nowhere) with weight route_w[recipe_ids[b]] (f32 [R], NULL = 1); samples with active[b] == 0
 *      (uint8 [B], optional) visit none.  Outputs as rte_pack_index for the B*seq*kmax expanded
 *      (token, j) pairs (a route list must not repeat a cluster); two launches.
 *      Workspace: rte_pack_routes_workspace_bytes(B, kmax). ---- */
size_t rte_pack_routes_workspace_bytes(int B, int kmax);
int rte_pack_routes(const int64_t* recipe_ids, const uint8_t* active, int B, int seq, const int32_t* routes,
                    int n_recipes, int kmax,
                    const float* route_w, int C, int32_t* offsets, int32_t* tok_of_slot, int32_t* pair_of_slot,
                    int32_t* slot_of_pair, float* w_of_slot, void* workspace, size_t workspace_bytes, void* stream);

/* ---- routed cluster-pool SwiGLU (rte/kernels/cluster_pool_ffn.py:192-241,
 *      rte/layers.py:119-220 StaticClusterPoolSwiGLU, rte/layers.py:731-779 BankedSwiGLU) ----
 * Cluster g owns neurons [g*n, (g+1)*n) of a d_ff = G*n SwiGLU:
 *   wug: bf16 [2*d_ff, d] rows [W_up ; W_gate] (nn.Linear(d, 2*d_ff).weight layout)
 *   wd : bf16 [d, ld_wd] with column g*n + j = W_down row of neuron j of cluster g
 *        (nn.Linear(d_ff, d).weight layout when ld_wd = d_ff)
 * Slots come from rte_pack_index.  Forward writes
 *   ug [P, 2n] bf16 pre-activations (per 64 columns: 32 up | 32 gate),
 *   zw [P, n]  bf16 w_of_slot * up * silu(gate),
 *   y_pairs [T*k, d] bf16 in pair order, y = zw @ W_down_g   (combine with rte_combine_rows).
 * max_tiles bound: P/128 + G + 1 is always enough. */
int rte_grouped_swiglu_fwd(const void* x, int T, int d, const int32_t* offsets, int G, int n, int P,
                           const int32_t* tok_of_slot, const int32_t* pair_of_slot, const float* w_of_slot,
                           const void* wug, const void* wd, int64_t ld_wd,
                           void* ug, void* zw, void* y_pairs, void* stream);

/* Backward.  dout [T, d] bf16 is dL/d(out) of the combined output.  Writes
 *   dug     [P, 2n] bf16 (workspace-like output),
 *   dw_slot [P] f32    = <dout[t], y_unweighted>  (routing-weight gradient per slot),
 *   dx_pairs[T*k, d] bf16 in pair order (combine them for dx),
 *   dwug    [2*d_ff, d] f32 and dwd [d, ld_wd] f32 (every neuron row is owned by exactly one
 *           cluster, so no reduction across clusters is needed); with w_t = 1 their transposes
 *           instead: dwug [d, 2*d_ff] (columns [up | gate]) and dwd [d_ff, d], the layouts of
 *           weights whose transposes the kernel reads.  beta = 0 overwrites dwug / dwd, beta = 1
 *           adds the gradients to what they hold (several uses of one weight summed in the
 *           order of the calls, no separate adds). */
int rte_grouped_swiglu_bwd(const void* dout, const void* x, int T, int d, const int32_t* offsets, int G,
                           int n, int P, const int32_t* tok_of_slot, const int32_t* pair_of_slot,
                           const float* w_of_slot, const void* wug, const void* wd, int64_t ld_wd,
                           const void* ug, const void* zw, void* dug, float* dw_slot, void* dx_pairs,
                           float* dwug, float* dwd, int w_t, float beta, void* workspace, size_t workspace_bytes,
                           void* stream);
/* Workspace with which the per-cluster weight gradients of rte_grouped_swiglu_bwd are
 * reduced by several workgroups per cluster when routing is skewed (fixed chunk order, so
 * still deterministic).  NULL / too small: one workgroup column per cluster. */
size_t rte_grouped_swiglu_bwd_workspace_bytes(int P, int G, int n, int d);

/* The same two operations as rte_grouped_swiglu_fwd / rte_grouped_swiglu_bwd (same arguments,
 * same outputs) with the per-cluster products fused: one launch computes ug, zw and y_pairs, one
 * launch computes dug, dw_slot and dx_pairs (the weight gradients are the same grouped-K
 * reductions).  Each workgroup stages its cluster's weights in LDS and keeps the [128 x 2n]
 * up/gate and [128 x n] z blocks of its 128 slots on chip (rte/kernels/cluster_pool_ffn.py:192-241).
 * Shapes: n = 32 and d in {128, 256, 512} (rte_grouped_swiglu_fused_ok(n, d) returns 1); other
 * shapes return -1.  ld_wd must be a multiple of 8. */
int rte_grouped_swiglu_fused_ok(int n, int d);
int rte_grouped_swiglu_fused_fwd(const void* x, int T, int d, const int32_t* offsets, int G, int n, int P,
                                 const int32_t* tok_of_slot, const int32_t* pair_of_slot, const float* w_of_slot,
                                 const void* wug, const void* wd, int64_t ld_wd,
                                 void* ug, void* zw, void* y_pairs, void* stream);
int rte_grouped_swiglu_fused_bwd(const void* dout, const void* x, int T, int d, const int32_t* offsets, int G,
                                 int n, int P, const int32_t* tok_of_slot, const int32_t* pair_of_slot,
                                 const float* w_of_slot, const void* wug, const void* wd, int64_t ld_wd,
                                 const void* ug, const void* zw, void* dug, float* dw_slot, void* dx_pairs,
                                 float* dwug, float* dwd, int w_t, float beta, void* workspace,
                                 size_t workspace_bytes, void* stream);

/* ---- dense SwiGLU (rte/layers.py:78-116 DenseSwiGLU / PackedDenseSwiGLU;
 *      rte/kernels/active_swiglu_triton.py:62-102 fused activation fwd/bwd) ----
 * wug bf16 [2F, d] rows [up ; gate].  wd_rows = 0: wd is [d, F] (nn.Linear(F, d).weight),
 * wd_rows = 1: wd is [F, d] (the packed "wdown_rows" layout).
 * out [T,d] = resid + (up * silu(gate)) @ W_down, f32 (out_f32=1) or bf16; resid f32 optional.
 * ug [T, 2F] bf16 (interleaved per 64: 32 up | 32 gate), z [T, F] bf16. */
int rte_dense_swiglu_fwd(const void* x, int T, int d, int F, const void* wug, const void* wd, int wd_rows,
                         const float* resid, void* ug, void* z, void* out, int out_f32, void* stream);
/* dout bf16 [T, d]; writes dug [T, 2F] bf16, dx [T, d] bf16, dwug [2F, d] f32,
 * dwd f32 in the layout of wd (overwritten).  workspace: split-K partials of the dx and weight
 * gradients, max of rte_gemm_workspace_bytes(T, d, 2F), (2F, d, T) and (d, F, T) bytes (fewer
 * bytes: fewer splits). */
int rte_dense_swiglu_bwd(const void* dout, const void* x, int T, int d, int F, const void* wug,
                         const void* wd, int wd_rows, const void* ug, const void* z, void* dug, void* dx,
                         float* dwug, float* dwd, void* workspace, size_t workspace_bytes, void* stream);

/* ---- fused QKV projection + interleaved RoPE (rte/layers.py:53-75, rte/kernels/reference.py:20-37) ----
 * x [B*S, d] bf16, wqkv [3d, d] bf16 (nn.Linear(d, 3d).weight), cos/sin [S, hd] f32.
 * q, k, v written as contiguous [B, H, S, hd] bf16.  workspace (optional, see
 * rte_gemm_workspace_bytes(B*S, 3d, d)): with few output tiles (short batches) the reduction is
 * split, the partials added in split order and rotated by the split-K reduce. */
int rte_qkv_rope_fwd(const void* x, const void* wqkv, const float* cos_t, const float* sin_t, int B, int S,
                     int H, int hd, void* q, void* k, void* v, void* workspace, size_t workspace_bytes,
                     void* stream);
/* dq/dk/dv: [B,H,S,hd] bf16 with element strides s*[4] (innermost must be 1).
 * dqkv: [B*S, 3d] bf16 workspace (dq = NULL: dqkv is the input, already packed and rotated back
 * by rte_attention_bwd_qkv); dx [B*S, d] bf16; dw [3d, d] f32 (overwritten; NULL: no weight
 * gradient, for callers that form it in another layout).
 * workspace: split-K partials of dx and dw, max of rte_gemm_workspace_bytes(B*S, d, 3d) and
 * (3d, d, B*S) bytes (fewer bytes: fewer splits). */
int rte_qkv_rope_bwd(const void* dq, const int64_t* sq, const void* dk, const int64_t* sk, const void* dv,
                     const int64_t* sv, const void* x, const void* wqkv, const float* cos_t,
                     const float* sin_t, int B, int S, int H, int hd, void* dqkv, void* dx, float* dw,
                     void* workspace, size_t workspace_bytes, void* stream);

/* ---- causal attention core, head_dim 32, 64 or 128 (the SDPA call of k_flash_causal_dense / _grouped,
 *      rte/kernels/optimized.py:75-91, in rte/layers.py:53-75 and the banked attention :659-730) ----
 * q, k, v bf16 [B, H, seq, hd] contiguous; out bf16 [B, seq, H, hd] (token-major rows of the
 * O-projection input); lse f32 [B, H, seq] (log2 units: max + log2(sum 2^(s - max)) of
 * s = q.k * scale * log2(e)), written by fwd and read by bwd.  head_scale f32 [B * H] (optional):
 * out = head_scale[b, h] * softmax(q k^T * scale, causal) v.
 * bwd: dout bf16 [B, seq, H, hd] (token-major); dq, dk, dv bf16 [B, H, seq, hd] (overwritten).
 * Deterministic (fixed reduction order); 16-byte aligned buffers. */
int rte_attention_fwd(const void* q, const void* k, const void* v, int B, int H, int seq, int head_dim, float scale,
                      const float* head_scale, void* out, float* lse, void* stream);
int rte_attention_bwd(const void* q, const void* k, const void* v, const void* out, const void* dout,
                      const float* lse, int B, int H, int seq, int head_dim, float scale, const float* head_scale,
                      void* dq, void* dk, void* dv, void* stream);
/* The same backward writing the fused QKV projection's input gradient directly: dqkv bf16
 * [B*seq, 3 H hd] rows [dq | dk | dv] with dq and dk rotated back by the RoPE angle of their
 * position (cos / sin f32 [seq, hd] as in rte_qkv_rope_fwd), bit-identical to rte_attention_bwd
 * followed by the packing step of rte_qkv_rope_bwd; pass dqkv to rte_qkv_rope_bwd with dq,
 * dk, dv = NULL. */
int rte_attention_bwd_qkv(const void* q, const void* k, const void* v, const void* out, const void* dout,
                          const float* lse, int B, int H, int seq, int head_dim, float scale,
                          const float* head_scale, const float* cos_t, const float* sin_t, void* dqkv, void* stream);

/* ---- SVD low-rank SwiGLU FFN (rte/layers.py:342-643 SVDFactorSparseFFN factors
 *      up_a = U S, up_b = V^T from refresh_svd :437-444) ----
 * us_ug bf16 [d, 2r] = [U_up S_up | U_gate S_gate], v_ug bf16 [2F, r] = [V_up ; V_gate],
 * v_dn bf16 [F, r], us_dn bf16 [d, r] = U_dn S_dn (W_down^T = U_dn S_dn V_dn^T).
 * fwd: a_ug [T, 2r], ug [T, 2F] (interleaved per 64), z [T, F], b [T, r] (all bf16),
 *      y [T, d] = resid + ((z V_dn) us_dn^T), f32 (y_f32=1) or bf16.  r % 8, F % 64, d % 8 == 0. */
int rte_svd_ffn_fwd(const void* x, int T, int d, int F, int r, const void* us_ug, const void* v_ug,
                    const void* v_dn, const void* us_dn, const float* resid, void* a_ug, void* ug, void* z,
                    void* b, void* y, int y_f32, void* stream);
/* bwd from dy bf16 [T, d]: scratch db [T, r], dug [T, 2F], da_ug [T, 2r] (bf16); dx [T, d] bf16;
 * weight grads f32 (overwritten) dus_ug [d, 2r], dv_ug [2F, r], dv_dn [F, r], dus_dn [d, r]. */
int rte_svd_ffn_bwd(const void* dy, const void* x, int T, int d, int F, int r, const void* us_ug,
                    const void* v_ug, const void* v_dn, const void* us_dn, const void* a_ug, const void* ug,
                    const void* z, const void* b, void* db, void* dug, void* da_ug, void* dx, float* dus_ug,
                    float* dv_ug, float* dv_dn, float* dus_dn, void* workspace, size_t workspace_bytes,
                    void* stream);
/* The same FFN with the wide activations kept on chip (the fused "x A -> B -> SwiGLU -> V_d ->
 * U_d^T" path; same factor layouts, results within bf16 rounding of rte_svd_ffn_fwd / _bwd):
 * the [T, 2F] up / gate pre-activations and the [T, F] SwiGLU output are never written; the
 * backward recomputes them per (token, neuron) block.  fwd writes a_ug [T, 2r], b [T, r] (bf16)
 * and y; bwd writes db [T, r], da_ug [T, 2r] (bf16 scratch), dx and the four fp32 weight
 * gradients (overwritten).  r in {64, 128}, F % 128 == 0, d % 8 == 0, T % 8 == 0; both calls take
 * rte_svd_ffn_fused_workspace_bytes(T, d, F, r) bytes of workspace.  Sums over neuron / token
 * ranges are fp32 partials added in a fixed order: bitwise repeatable. */
size_t rte_svd_ffn_fused_workspace_bytes(int T, int d, int F, int r);
int rte_svd_ffn_fused_fwd(const void* x, int T, int d, int F, int r, const void* us_ug, const void* v_ug,
                          const void* v_dn, const void* us_dn, const float* resid, void* a_ug, void* b, void* y,
                          int y_f32, void* workspace, size_t workspace_bytes, void* stream);
int rte_svd_ffn_fused_bwd(const void* dy, const void* x, int T, int d, int F, int r, const void* us_ug,
                          const void* v_ug, const void* v_dn, const void* us_dn, const void* a_ug, const void* b,
                          void* db, void* da_ug, void* dx, float* dus_ug, float* dv_ug, float* dv_dn,
                          float* dus_dn, void* workspace, size_t workspace_bytes, void* stream);

/* ---- SVD-factor sparse SwiGLU FFN, per-token candidates (SVDFactorSparseFFN, rte/layers.py:342-643,
 *      modes mask / slots; the device driver rte/kernels/svd_sparse_ffn_triton.py:480-714) ----
 * Selector: a_ug [T, 2r] = x @ us_ug (us_ug bf16 [d, 2r] = [A_up | A_gate], the rank-r factors
 * U S of refresh_svd), ug [T, 2F] = [a_up B_up | a_gate B_gate] (v_ug bf16 [2F, r] = [B_up^T ;
 * B_gate^T], interleaved per 64 as rte_svd_ffn_fwd), z_hat [T, F] (workspaces, bf16).
 * Per token: the top up_m of |up_hat| w, top gate_m of |silu(gate_hat)| w and top product_m of
 * |up_hat silu(gate_hat)| w (w = wd_norm f32 [F] = ||W_down row||) united; fewer than top_k
 * candidates: the top top_k of the product scores are added; activations u = <x, W_up[c]>,
 * g = <x, W_gate[c]> (exact = 1) or the selector's (exact = 0); the top top_k of |u silu(g)| w
 * are selected; out [T, d] (f32 if out_f32 else bf16) = sum of u silu(g) W_down[c] over them.
 * product_only = 1: the selected are the top top_k of the product scores (approximate activations).
 * Every top-m takes the larger scores first, then ties by lower neuron id (NaN ranks first).
 * sel_ids int32 / sel_u / sel_g f32 [T, top_k] (ascending id; -1 / 0 pads), n_cand int32 [T]
 * (optional).  w_up, w_gate, w_down bf16 [F, d] (rows = neurons).  F % 64, d % 8, r % 8 == 0.
 * bwd: dout bf16 [T, d] -> dx bf16 [T, d], z = u silu(g), du = dz silu(g), dg = dz u silu'(g)
 * (f32 [T, top_k], dz = <dout, W_down[c]>); the weight gradients are rte_segment_reduce_rows
 * keyed by sel_ids: dW_down rows (w = z, rows = dout), dW_up (w = du, rows = x), dW_gate (w = dg). */
int rte_svd_sparse_fwd(const void* x, int T, int d, int F, int r, const void* us_ug, const void* v_ug,
                       const void* w_up, const void* w_gate, const void* w_down, const float* wd_norm, int up_m,
                       int gate_m, int product_m, int top_k, int exact, int product_only, void* a_ug, void* ug,
                       void* z_hat, void* out, int out_f32, int32_t* sel_ids, float* sel_u, float* sel_g,
                       int32_t* n_cand, void* stream);
int rte_svd_sparse_bwd(const void* dout, int T, int d, int top_k, const void* w_up, const void* w_gate,
                       const void* w_down, const int32_t* sel_ids, const float* sel_u, const float* sel_g, void* dx,
                       float* z, float* du, float* dg, void* stream);

/* ---- RMSNorm (rte/kernels/reference.py:9-17, rte/layers.py:26-33) ----
 * out bf16 = bf16(x * rsqrt(mean(x^2) + eps) * w), rstd [T] f32 saved for backward. */
int rte_rmsnorm_fwd(const float* x, const float* w, int T, int d, float eps, void* out, float* rstd,
                    void* stream);
size_t rte_rmsnorm_bwd_workspace_bytes(int T, int d);
/* dy bf16; dx f32 (= dres + norm backward, dres optional); dx_bf16 (optional) the same values in
 * bf16; dw f32 [d] (accumulated if dw_accumulate). */
int rte_rmsnorm_bwd(const void* dy, const float* x, const float* w, const float* rstd, const float* dres,
                    int T, int d, float* dx, void* dx_bf16, float* dw, int dw_accumulate, void* workspace,
                    size_t workspace_bytes, void* stream);

/* ---- elementwise dispatch symbols in the caller's dtype ----
 * Fused RMSNorm (replaces k_fused_rmsnorm, rte/kernels/reference.py:9-17): y = x + residual
 * (residual optional; y written when both y and residual are given), rstd f32 [T] =
 * rsqrt(mean(y^2) + eps), out = (y * rstd) * w.  x, residual, y: f32 (io_f32 = 1) or bf16 [T, d];
 * w f32 [d]; out f32 (out_f32 = 1) or bf16.  bf16 inputs are rounded where torch's bf16 ops round
 * (the sum, the rsqrt factor, the normalised row).  d % 8 == 0, d <= 4096.
 * bwd: g (f32 if g_f32 else bf16) = dL/d(out); dy (io dtype) = dL/dy = rstd w g - y rstd^3
 * mean(w g y) (+ dy_extra, io dtype, optional: the gradient of the returned y); dw f32 [d] = sum
 * over rows of g y rstd, in a fixed order.  d <= 2048; workspace
 * rte_fused_rmsnorm_bwd_workspace_bytes(T, d). */
int rte_fused_rmsnorm_fwd(const void* x, const void* residual, int io_f32, const float* w, int T, int d, float eps,
                          void* y, void* out, int out_f32, float* rstd, void* stream);
size_t rte_fused_rmsnorm_bwd_workspace_bytes(int T, int d);
int rte_fused_rmsnorm_bwd(const void* g, int g_f32, const void* dy_extra, const void* y, int io_f32, const float* w,
                          const float* rstd, int T, int d, void* dy, float* dw, void* workspace, size_t workspace_bytes,
                          void* stream);
/* Interleaved RoPE (replaces k_rope_apply, rte/kernels/reference.py:20-28): q, k contiguous
 * [rows, S, hd] (f32 if in_f32 else bf16), cos / sin f32 [S, hd];
 *   out[2i] = x[2i] cos[2i] - x[2i+1] sin[2i], out[2i+1] = x[2i+1] cos[2i+1] + x[2i] sin[2i+1];
 * inverse = 1 applies the transpose (the backward).  Outputs f32 (out_f32 = 1) or bf16; hd % 8 == 0. */
int rte_rope_apply(const void* q, const void* k, int in_f32, int64_t rows, int S, int hd, const float* cos_t,
                   const float* sin_t, void* q_out, void* k_out, int out_f32, int inverse, void* stream);
/* Static-centre routing (replaces route_to_static_centers, rte/kernels/cluster_pool_ffn.py:129-140):
 * q f32 [T, R2] = [x A_up | x A_gate]; out int32 [T] = argmax_c normalize(q[t]) . centers[c]
 * (centers f32 [C, R2]; F.normalize's 1e-12 clamp; first index of the maximum, NaN counts as
 * the maximum).  R2 <= 8192. */
int rte_route_centers(const float* q, int T, int R2, const float* centers, int C, int32_t* out, void* stream);

/* ---- token cross-entropy on full logits (rte/models.py:73-75, rte/kernels/reference.py:146-147) ----
 * logits f32 [T, ld] (first V columns used), targets int64 [T] (negative = ignored row).
 * fwd: loss[t] = logsumexp(logits[t]) - logits[t, target], lse[t] saved.
 * bwd: dlogits bf16 [T, V] = dloss[t] * (softmax - onehot(target)) + extra (f32 [T, V], optional). */
int rte_ce_fwd(const float* logits, int64_t ld, int T, int V, const int64_t* targets, float* loss, float* lse,
               void* stream);
int rte_ce_bwd(const float* logits, int64_t ld, int T, int V, const int64_t* targets, const float* lse,
               const float* dloss, const float* extra, void* dlogits, void* stream);
/* rte_ce_bwd with the extra logit gradient given only for whole samples: extra_rows f32
 * [n_samples * seq, V] holds the rows of samples sample_ids[0, n_samples) (seq tokens each; token t
 * belongs to sample t / seq), every other token has none.  Replaces the zero-filled [T, V] gradient
 * of the audited-sample selection of the hot logits (hot.meta.logits[mask], rte/audit.py:336, fed to
 * macro_distill_loss, rte/macro.py:394); a sample listed twice adds its rows in list order. */
int rte_ce_bwd_rows(const float* logits, int64_t ld, int T, int V, const int64_t* targets, const float* lse,
                    const float* dloss, const float* extra_rows, const int64_t* sample_ids, int n_samples, int seq,
                    void* dlogits, void* stream);

/* ---- residual axpy + FiLM RMSNorm of a recursive pass (replaces the elementwise glue of
 *      BankedRecursiveCore._step, rte/layers.py:826-845: h~ = h + alpha h0, rmsnorm * (1 + gamma)
 *      + beta, u = h~ + s_attn attn, h' = u + s_mlp mlp, inactive samples keep h) ----
 * fwd: x = a + c b (c: device fp32 scalar, NULL = 1; b optional); samples with mask[row / seq] == 0
 *      (mask uint8 [T / seq], optional, needs keep) take keep's row; x_out f32 [T, d] optional;
 *      n_out bf16 = x * rstd * w * (1 + gamma) + beta (gamma, beta optional), rstd f32 [T].
 * bwd: g = dn (1 + gamma); dx = dx_ext + rstd w g - x rstd^3 mean(w g x) (dn, dx_ext optional);
 *      da = active ? dx : 0; db = c da; dkeep = active ? 0 : dx (each output optional);
 *      dparams f32 [3 d + 1] = (dw | dgamma | dbeta | dc), reduced in a fixed order.
 * All arrays f32 [T, d] row-major, 16-byte aligned; d % 8 == 0, d <= 1024. */
int rte_axpy_norm_fwd(const float* a, const float* b, const float* c, const float* keep, const uint8_t* mask,
                      int seq, int T, int d, const float* w, const float* gamma, const float* beta, float eps,
                      float* x_out, void* n_out, float* rstd_out, void* stream);
size_t rte_axpy_norm_bwd_workspace_bytes(int T, int d);
int rte_axpy_norm_bwd(const void* dn, const float* dx_ext, const float* x, const float* rstd, const float* w,
                      const float* gamma, const float* b, const float* c, const uint8_t* mask, int seq, int T, int d,
                      float* da, float* db, float* dkeep, float* dparams, void* workspace, size_t workspace_bytes,
                      void* stream);

/* ---- bounded-residual macro operator Phi, elementwise ends (rte/macro.py:201-236; the
 *      (recipe, stride) low-rank matrices in between run as rte_grouped_linear_*) ----
 * Samples b < B (key int64 [B]) read h rows of sample b % B_h and h0 rows of sample b % B_h0
 * (B_h0 | B_h | B: one source batch evaluated under several keys, as the consistency loss does).
 * prologue fwd (B = B_h samples): z bf16 [B_h*seq, 3d] = [h * rstd | mean over the sample's rows
 *               of h * rstd | h0], rstd f32 [B_h*seq] = rsqrt(mean(h^2) + eps) per row
 *               (h f32 [B_h, seq, d], h0 f32 [B_h0, seq, d]).
 * prologue bwd: for each source sample b < B_h, over its repeats b + t B_h (B / B_h <= 4, in t
 *               order): dh[b] = sum_t dh_extra[b + t B_h] (optional) + rmsnorm backward of
 *               dz[b + t B_h, :d] + dz[b + t B_h, d:2d] / seq broadcast over the rows;
 *               dh0[b] = sum_t dz[b + t B_h, 2d:] (optional; dh, dh0 f32 [B_h, seq, d], dz bf16
 *               [B*seq, 3d]).
 * epilogue fwd: out = h + c * scale[k] * tanh(gain[k] * h + low + bias[k]), k = key[b],
 *               tables gain / bias / scale f32 [keys, d], low f32 [B*seq, d].
 * epilogue bwd: dh = dout + dupd * gain[k] (f32 [B, seq, d]), dlow bf16 = dupd,
 *               dupd = dout c scale[k] (1 - t^2); part (rte_macro_workspace_bytes(B, ...)) =
 *               per-sample, per-row-slice sums (dupd h | dupd | dout c t) for the tables.
 * table grad: dgain / dbias / dscale f32 [n_keys, d] (each optional) = sums of part's three column
 *               blocks over the samples with that key, in sample order (zero rows for unused keys);
 *               part as written by rte_macro_epilogue_bwd with the same B, seq, d.
 * The prologues take a workspace of rte_macro_workspace_bytes(B, seq, d) for their per-slice sums
 * (B: the prologue's own batch, B_h for fwd and B for bwd).
 * d % 8 == 0, d <= 1024, B <= 65535 (table grad: B <= 16384), 16-byte aligned buffers. */
size_t rte_macro_workspace_bytes(int B, int seq, int d);
int rte_macro_prologue_fwd(const float* h, const float* h0, int B, int B_h0, int seq, int d, float eps, void* z,
                           float* rstd, void* workspace, size_t workspace_bytes, void* stream);
int rte_macro_prologue_bwd(const void* dz, const float* h, const float* rstd, const float* dh_extra, int B, int B_h,
                           int seq, int d, float* dh, float* dh0, void* workspace, size_t workspace_bytes,
                           void* stream);
int rte_macro_epilogue_fwd(const float* h, const float* low, const int64_t* key, int B, int B_h, int seq, int d,
                           const float* gain, const float* bias, const float* scale, float c, float* out,
                           void* stream);
int rte_macro_epilogue_bwd(const float* dout, const float* h, const float* low, const int64_t* key, int B, int B_h,
                           int seq, int d, const float* gain, const float* bias, const float* scale, float c,
                           float* dh, void* dlow, void* part, size_t part_bytes, void* stream);
int rte_macro_table_grad(const int64_t* key, int B, int seq, int n_keys, int d, const void* part, float* dgain,
                         float* dbias, float* dscale, void* stream);

/* Fused bounded macro operator Phi at hidden rank 32 (rte/macro.py:201-236, the path of
 * MacroOperators._apply_vectorized_bounded and consistency_loss at rte/macro.py:342-359 with
 * the default options).  z = [rmsnorm(h) | mean_s rmsnorm(h) | h0] of the reference is split by
 * the rows of V = [V1; V2; V3]: a = x2 @ [V1; V3][k] + pooled @ V2[k] with x2 = [bf16(h rstd) |
 * bf16(h0)] per source row and pooled = bf16(mean_s h rstd) per source sample; low = silu(a) @
 * U[k]; out = h + c scale[k] tanh(gain[k] h + low + bias[k]).  Sample b of B reads h row block
 * b % B_h and h0 row block b % B_h0 (B_h0 | B_h | B, B / B_h <= 8); k = key[b] in [0, n_keys).
 * prep  : bf16 weight layouts from v f32 [n_keys, 3d, 32] and u f32 [n_keys, 32, d]: v_b (same
 *         layout), vc_t [n_keys, 32, 2d] (V1 | V3 transposed), v2_t [n_keys, 32, d], u_b (same),
 *         u_t [n_keys, d, 32].
 * fwd   : x2 bf16 [B_h*seq, 2d], rstd f32 [B_h*seq], pooled bf16 [B_h, d], p f32 [B, 32], a f32
 *         [B*seq, 32], sa = bf16(silu(a)) [B*seq, 32], out f32 [B, seq, d]; with mse_ref (f32
 *         [B, seq, d]) also mse_part f32 [B * tiles] = per-tile sums of (out - mse_ref)^2, tiles =
 *         rte_macro_fused_tiles(seq); workspace rte_macro_fused_fwd_workspace_bytes(B_h, seq, d).
 * sum   : out[0] = inv_n * sum of part[0, n) in a fixed order.
 * bwd   : upstream gradient of sample b: mul * g[0] * (dout_p - dout_q)[b - diff_lo] for b in
 *         [diff_lo, diff_lo + n_diff), plus dout[b - dout_lo] for b in [dout_lo, dout_lo + n_dout)
 *         (the ranges may overlap; a sample in neither has gradient 0).  Writes du bf16 [B*seq, d], da bf16 [B*seq, 32], part_tab f32
 *         [B, tiles, 3, d] (du h | du | dout c tanh column sums), part_da f32 [B, tiles, 32], da_sum bf16
 *         [B, 32] (sum over the sample's rows of da), dh f32
 *         [B_h, seq, d] (all repeats added in repeat order; with dh0_into_dh the h0 gradient too;
 *         plus n_extra blocks of extra f32 [n_extra * B_h, seq, d]) and dh0 f32 [B_h, seq, d]
 *         (optional, per h source sample).  Workspace rte_macro_fused_bwd_workspace_bytes(B, seq).
 * wgrad : weight gradients of one call (B1 = 0) or of two calls listed together (call 1's
 *         samples follow call 0's in key / du / da / part buffers, its x2 and pooled rows follow
 *         call 0's B_h0 source blocks): du_w f32 [n_keys, 32, d], dv_w f32 [n_keys, 3d, 32],
 *         dgain / dbias / dscale f32 [n_keys, d] (each optional), every sum in a fixed order.
 *         Workspace rte_macro_fused_wgrad_workspace_bytes(B0 + B1, seq, d, n_keys).
 * d % 128 == 0, d <= 1024, seq <= 65536, B <= 65535 (wgrad: B0 + B1 <= 16384). */
int rte_macro_fused_tiles(int seq);
size_t rte_macro_fused_fwd_workspace_bytes(int B_h, int seq, int d);
size_t rte_macro_fused_bwd_workspace_bytes(int B, int seq);
size_t rte_macro_fused_wgrad_workspace_bytes(int B_total, int seq, int d, int n_keys);
int rte_macro_fused_prep(const float* v, const float* u, int n_keys, int d, void* v_b, void* vc_t, void* v2_t,
                         void* u_b, void* u_t, void* stream);
int rte_macro_fused_fwd(const float* h, const float* h0, int B_h, int B_h0, const int64_t* key, int B, int seq, int d,
                        int n_keys, float eps, const void* v_b, const void* vc_t, const void* u_t, const float* gain,
                        const float* bias, const float* scale, float c, void* x2, float* rstd, void* pooled, float* p,
                        float* a, void* sa, float* out, const float* mse_ref, float* mse_part, void* workspace,
                        size_t workspace_bytes, void* stream);
int rte_macro_fused_sum(const float* part, int n, float inv_n, float* out, void* stream);
int rte_macro_fused_bwd(const float* dout_p, const float* dout_q, const float* g, float mul, int diff_lo,
                        int n_diff, const float* dout, int dout_lo, int n_dout, const float* h, const float* rstd, const void* x2, int B_h,
                        const int64_t* key, int B, int seq, int d, int n_keys, const float* a, const void* sa,
                        const void* v_b, const void* vc_t, const void* v2_t, const void* u_b, const void* u_t,
                        const float* gain, const float* bias, const float* scale, float c, void* du, void* da,
                        float* part_tab, float* part_da, float* dh, float* dh0, int dh0_into_dh, const float* extra,
                        int n_extra, void* da_sum, void* workspace, size_t workspace_bytes, void* stream);
int rte_macro_fused_wgrad(const int64_t* key, int B0, int B_h0, int B1, int B_h1, int seq, int d, int n_keys,
                          const void* x2, const void* sa, const void* du, const void* da, const void* pooled,
                          const void* da_sum, const float* part_tab, float* du_w, float* dv_w, float* dgain,
                          float* dbias, float* dscale, void* workspace, size_t workspace_bytes, void* stream);

/* Macro consistency loss in one pass per application for seq <= 64 and d = 256 or 512
 * (rte/macro.py:342-359 with the operator of rte/macro.py:201-236 at hidden rank 32, h0 = h):
 * loss = mean over j < pc, samples, rows, columns of (Phi_{j}(out_{src_lo + j}) -
 * out_{dst_lo + j})^2, out_k = Phi_k(h) for the nf first-application key blocks (key_first
 * [nf * b], block k of sample i at k * b + i), key_src [pc * b] the second application's keys.
 * One workgroup per 32 rows of a sample; out and the second application's output are never
 * stored (recomputed from h and the rank-32 codes).  Buffers, in the layouts of
 * rte_macro_fused_wgrad with call 0 = the nf * b first-application samples over B_h0 = b source
 * blocks and call 1 = the pc * b second-application samples over their own pc * b blocks:
 * x2 bf16 [(b + pc b) seq, 2d], pooled bf16 [b + pc b, d], a f32 / sa bf16 [(nf b + pc b) seq, 32],
 * rstd f32 [(b + pc b) seq] (h, then the second application's inputs), loss f32 [1];
 * backward: du bf16 [(nf b + pc b) seq, d], da bf16 [., 32], part_tab f32 [nf b + pc b, tiles, 3, d],
 * part_da f32 [., tiles, 32], da_sum bf16 [nf b + pc b, 32], dh f32 [b, seq, d] (the whole
 * gradient of h), tiles = ceil(seq / 32); g f32 [1] the loss gradient, mul = 2 / (pc b seq d).
 * prep: vq_t bf16 [n_keys, 32, 2d] (V1 | V3 transposed) and u_q bf16 [n_keys, 32, d] with the
 * middle two 4-column quads of every 16 columns swapped (the kernels' operand order).
 * Requires 1 <= pc <= nf <= 4 and the src / dst blocks inside the first application. */
size_t rte_macro_cons_workspace_bytes(int b, int seq, int d, int pc);
int rte_macro_cons_prep(const float* v, const float* u, int n_keys, int d, void* vq_t, void* u_q, void* stream);
int rte_macro_cons_fwd(const float* h, int b, int seq, int d, const int64_t* key_first, int nf, const int64_t* key_src,
                       int pc, int src_lo, int dst_lo, int n_keys, float eps, const void* v_b, const void* vq_t,
                       const void* u_t, const void* u_q, const float* gain, const float* bias, const float* scale,
                       float c, void* x2, void* pooled, float* a, void* sa, float* rstd, float* loss,
                       void* workspace, size_t workspace_bytes, void* stream);
int rte_macro_cons_bwd(const float* h, int b, int seq, int d, const int64_t* key_first, int nf, const int64_t* key_src,
                       int pc, int src_lo, int dst_lo, int n_keys, const void* v_b, const void* u_t, const void* u_q,
                       const float* gain, const float* bias, const float* scale, float c, const float* a,
                       const void* sa, const float* rstd, const float* g, float mul, void* du, void* da,
                       float* part_tab, float* part_da, void* da_sum, float* dh, void* stream);

/* ---- mean squared difference (F.mse_loss of the macro consistency loss, rte/macro.py:342-359) ----
 * fwd: out f32 [1] = mean((a - b)^2) over n f32 elements (fixed-order block sums, then one
 * workgroup adds them in order); workspace rte_mse_workspace_bytes(n).
 * bwd: da = dout[0] 2 (a - b) / n, db = -da (each optional).  16-byte aligned buffers. */
size_t rte_mse_workspace_bytes(int64_t n);
int rte_mse_fwd(const float* a, const float* b, int64_t n, float* out, void* workspace, size_t workspace_bytes,
                void* stream);
int rte_mse_bwd(const float* a, const float* b, int64_t n, const float* dout, float* da, float* db, void* stream);

/* ---- per-sample recipe / depth router (replaces Router.forward's recipe and depth heads,
 *      rte/routing.py:80-188, and router_aux_losses, rte/metrics.py:97-112) ----
 * pool: pooled f32 / bf16 [B, d] = mean over S of h0 f32 [B, S, d].
 * Layer 1 of both MLPs (z1 = pooled W1^T + b1, f32 [B, hid]) runs on rte_gemm_bf16.
 * heads_fwd (one wave per row): raw = silu(z1) W2^T + b2 (w2 f32 [N, hid]); logits = raw inv_t;
 *   probs = softmax; id = first argmax of probs (NaN counts as maximal) or fixed_* when >= 0
 *   (fixed_depth indexes depth_values); onehot_st = (onehot(id) + p) - p; entropy =
 *   -sum log(max(p, 1e-9)) p; per pass t < P: logits + pass_bias[t] inv_t -> softmax / argmax /
 *   one-hot; expected_depth = sum p_j depth_values[j]; depth = depth_values[depth id];
 *   router entropy = recipe + depth entropy.  Outputs in this order: recipe logits, probs, id (i64),
 *   onehot [B, R]; depth logits, probs, id (i64), depth (i64), onehot [B, D]; recipe / depth /
 *   router entropy, expected depth [B]; per-pass logits, probs [B, P, R], ids (i64) [B, P],
 *   onehot [B, P, R].  hid <= 4096, R and D <= 64, P <= 16.
 * heads_bwd: gradients of those outputs (each optional, null = zero; same order without the ids
 *   and depth) -> d raw logits draw_r [B, R], draw_d [B, D] and per-pass logit gradients dlbp
 *   [B, P, R].
 * mlp_bwd: dW2 [N, hid], db2 [N], dz1 bf16 [B, hid] (= (draw W2) silu'(z1)), db1 [hid] for both
 *   MLPs and d pass_bias [P, R] = inv_t sum_rows dlbp; dW1 and d pooled then run on rte_gemm_bf16.
 * aux_fwd: out f32 [3] = lambda_load (R sum_r mean_b(p)^2 - 1), lambda_cover sum_r
 *   relu(coverage_min - ema_r)^2, lambda_depth mean_b(expected_depth); mean_prob [R] for the
 *   backward.  aux_bwd: gradients of the load and depth terms (scalars, null = zero) -> dprobs
 *   [B, R], d expected_depth [B].
 * Every sum runs in a fixed order. */
int rte_router_pool(const float* h0, int B, int S, int d, float* pooled, void* pooled_bf16, void* stream);
int rte_router_heads_fwd(const float* z1r, const float* z1d, int B, int hid, const float* w2r, const float* b2r,
                         int R, const float* w2d, const float* b2d, int D, const float* pass_bias, int P,
                         const int64_t* depth_values, float inv_t, int fixed_recipe, int fixed_depth, float* rlog,
                         float* rprob, int64_t* rid, float* ronehot, float* dlog, float* dprob, int64_t* did,
                         int64_t* depth, float* donehot, float* rent, float* dent, float* ent, float* edepth,
                         float* rlog_bp, float* rprob_bp, int64_t* rid_bp, float* ronehot_bp, void* stream);
int rte_router_heads_bwd(const float* rprob, const float* rprob_bp, const float* dprob, const int64_t* depth_values,
                         int B, int R, int D, int P, float inv_t, const float* g_rlog, const float* g_rprob,
                         const float* g_ronehot, const float* g_dlog, const float* g_dprob, const float* g_donehot,
                         const float* g_rent, const float* g_dent, const float* g_ent, const float* g_edepth,
                         const float* g_rlog_bp, const float* g_rprob_bp, const float* g_ronehot_bp, float* draw_r,
                         float* draw_d, float* dlbp, void* stream);
int rte_router_mlp_bwd(const float* draw_r, const float* draw_d, const float* z1r, const float* z1d,
                       const float* w2r, const float* w2d, int B, int hid, int R, int D, const float* dlbp, int P,
                       float inv_t, void* dz1r, void* dz1d, float* db1r, float* db1d, float* dw2r, float* dw2d,
                       float* db2r, float* db2d, float* dpass, void* stream);
int rte_router_aux_fwd(const float* probs, const float* edepth, const float* ema, int B, int R, float coverage_min,
                       float lambda_load, float lambda_cover, float lambda_depth, float* mean_prob, float* out,
                       void* stream);
int rte_router_aux_bwd(const float* mean_prob, const float* g_load, const float* g_depth, int B, int R,
                       float lambda_load, float lambda_depth, float* dprobs, float* dedepth, void* stream);

/* ---- audit sampler and usage statistics (replaces AuditEngine.compute_audit_prob and the
 *      fixed-count branch of sample_mask_with_prob, rte/audit.py:79-132, and the bincount EMAs of
 *      RecipeBank.update_usage / the audit coverage update) ----
 * audit_sample_fixed (one workgroup): req[b] = clamp(p_min + alpha entropy[b] / denom + beta
 *   residual + gamma max(coverage_min - coverage_ema[recipe_ids[b]], 0) / max(coverage_min,
 *   1e-12), p_min, p_max); incl[b] = k / B; mask (bool bytes) [b] = b in chosen[0..k); stats f32
 *   [5] = mean incl, mean req, count / B, count, mean incl.
 * count_ema (one workgroup, bins R <= 4096): counts[r] = #{i < n : ids[i] == r and (mask null or
 *   mask[i])}; ema[r] = ema[r] beta + (1 - beta) counts[r] / max(sum counts, 1), in place. */
int rte_audit_sample_fixed(const float* entropy, const int64_t* recipe_ids, const float* coverage_ema,
                           const int64_t* chosen, int B, int k, int R, float denom, float p_min, float p_max,
                           float alpha, float beta, float gamma, float residual, float coverage_min, float* req,
                           float* incl, void* mask, float* stats, void* stream);
int rte_count_ema(const int64_t* ids, const void* mask, int n, float* ema, int R, float beta, void* stream);
/* nonfinite: bad[0] = 1 when x[0] is inf or NaN, else 0; ok[0] = 1 - bad[0] (the optimizer's
 * skip flag and the "stepped" metric of rte/training.py:445-468 without a host read).
 * step_metrics (one workgroup): out f32 [4] = mean(hot) / scale, mean(corr) / scale,
 * mean(corr) / seq, mean(depth) over B samples (the metric keys hot_lm_loss, corrected_lm_loss,
 * nll_per_token, avg_depth of rte/training.py:1412-1472). */
int rte_nonfinite(const float* x, float* bad, float* ok, void* stream);
int rte_step_metrics(const float* hot, const float* corr, const int64_t* depth, int B, float scale, float seq,
                     float* out, void* stream);

/* The step's loss (rte/training.py:1381-1385): out[0] = coef * sum_b x[b] + sum_i *terms[i] (x f32
 * [n], e.g. the corrected per-sample cross-entropy with coef = 1 / (n * seq); terms: up to 32
 * device f32 scalars given as a host array of pointers, added in order after the row sum, which
 * is in a fixed order).  bwd: dx[b] = coef * g[0] (the terms' gradients are g itself). */
int rte_loss_sum(const float* x, int n, float coef, const float* const* terms, int n_terms, float* out,
                 void* stream);
int rte_loss_sum_bwd(const float* g, int n, float coef, float* dx, void* stream);

/* ---- fused AdamW step with the trainer's per-group norms (replaces torch.optim.AdamW.step,
 *      clip_grad_norm_ and _optimizer_grad_metrics of rte/training.py:385-468) ----
 * rows: device array of n_tensors records {p, g, exp_avg, exp_avg_sq, step (f32 scalar) pointers,
 *       numel, optimizer group, metric-group bit mask} (8 int64 each); g == 0 leaves the tensor
 *       (and its step) untouched.  blocks: int32 pairs (tensor, chunk of rte_adamw_chunk()
 *       elements), tensors' chunks consecutive; first_block[n_tensors + 1] their starts.
 * hyper f64 [n_groups][5] = lr, beta1, beta2, eps, weight_decay.  metric_lr_group int32
 *       [n_metrics]: the group whose lr scales metric j's update ratio.  clip_max <= 0: no clip.
 * found_inf (optional device f32): > 0 skips the update and the step counters.
 * metrics f32 [n_metrics][2] = grad norm (after clipping), lr * grad norm / max(param norm, 1e-12),
 *       both from the values before the update.  Three launches, fixed reduction order. */
int rte_adamw_chunk(void);
size_t rte_adamw_workspace_bytes(int n_tensors, int n_blocks, int n_groups);
int rte_adamw_step(const void* rows, int n_tensors, const int32_t* blocks, const int32_t* first_block, int n_blocks,
                   const double* hyper, int n_groups, const int32_t* metric_lr_group, int n_metrics, float clip_max,
                   const float* found_inf, float* metrics, void* workspace, size_t workspace_bytes, void* stream);

/* ---- hot-vs-exact distillation losses + alignment metrics of the audit (replaces
 *      macro_distill_loss rte/macro.py:394-471 and macro_alignment_metrics :499-546 on the
 *      path with the residual origin h0; rte/audit.py:326-352 calls both) ----
 * hot, exact, h0 f32 [A, seq, d]; hot_logits / exact_logits f32 [A, seq, V] (both optional).
 * fwd: losses f32 [6] = weights[i] (host array of 6 floats, NULL = all 1) times delta_dir, delta_rms,
 *      endpoint_normed, endpoint_raw, rms_trust, kl (temperature t, batchmean over A, times t^2;
 *      0 without logits);
 *      metrics f32 [10] = hidden_cosine, hidden_mse, macro_norm, exact_norm, macro_exact_norm_ratio,
 *      delta_cosine, delta_rms_exact, delta_rms_pred, delta_rms_ratio, logit_kl (t = 1).
 *      The workspace (rte_distill_workspace_bytes(A, rows = A * seq or 0)) keeps the per-sample
 *      sums and logit lse's for the backward: keep it untouched until then.
 * bwd: dhot f32 [A, seq, d] and dhot_logits f32 [A, seq, V] (each optional) for dlosses [6] (device)
 *      of the weighted losses (same weights). */
size_t rte_distill_workspace_bytes(int A, int rows);
int rte_distill_fwd(const float* hot, const float* exact, const float* h0, int A, int seq, int d,
                    const float* hot_logits, const float* exact_logits, int V, float temperature, float eps,
                    const float* weights, float* losses, float* metrics, void* workspace, size_t workspace_bytes,
                    void* stream);
int rte_distill_bwd(const float* hot, const float* exact, const float* h0, int A, int seq, int d,
                    const float* hot_logits, const float* exact_logits, int V, float temperature, float eps,
                    const float* weights, const float* dlosses, const void* workspace, size_t workspace_bytes,
                    float* dhot, float* dhot_logits, void* stream);

/* ---- control-variate audit correction (replaces AuditEngine.correction's loss arithmetic,
 *      rte/audit.py:296-321, over lm_loss_per_sample rte/models.py:73-75) ----
 * hot_tok f32 [B, seq] token losses of the hot (macro) pass; exact_tok f32 [A, seq] token losses
 * of the exact replay of the audited rows idx int64 [A] (distinct, in [0, B)); p f32 [B]
 * inclusion probabilities (clamped below at 1e-12); clip >= 0 (INFINITY for no clip).
 * fwd, one workgroup, fixed reduction order:
 *   hot[m] = sum_s hot_tok[m, s], exact_ps[a] = sum_s exact_tok[a, s], r_a = exact_ps[a] - hot[idx[a]]
 *   corrected[m] = hot[m]; if grad_corrected: corrected[idx[a]] = hot[idx[a]] + clamp(r_a, +-clip) / p
 *   coef f32 [B + A]: per-row and per-audited-row gradient coefficient (1/p inside the clip when
 *   grad_corrected, else 0), kept for the backward
 *   stats f32 [4] = mean r, std r, var r (population, unclipped), mean(hot + clamp(r)/p);
 *   NaN if some idx lies outside [0, B).  B <= 8192.
 * bwd: dhot_tok[m, s] = g[m] (1 - coef[m]), dexact_tok[a, s] = g[idx[a]] coef[B + a] (optional). */
int rte_audit_correct_fwd(const float* hot_tok, const float* exact_tok, int B, int seq, const int64_t* idx, int A,
                          const float* p, float clip, int grad_corrected, float* corrected, float* exact_ps,
                          float* coef, float* stats, void* stream);
int rte_audit_correct_bwd(const float* g, int B, int seq, const int64_t* idx, int A, const float* coef,
                          float* dhot_tok, float* dexact_tok, void* stream);

/* ---- grouped linear: rows keyed to a group, one weight matrix per group ----
 * Replaces the per-sample weight gather + bmm of the macro operators (rte/macro.py:201-236,
 * gather of v / u by (recipe, stride) at :208-212) without materialising per-sample weights.
 * Slots come from rte_pack_index over the rows' group keys (k = 1): offsets [G+1],
 * row_of_slot (tok_of_slot) and out_row_of_slot (pair_of_slot).  w bf16 [G, K, Nout] row-major.
 *   fwd: y[out_row(s)] = x[row(s)] @ W_g            x bf16 [N, K], y f32 (y_f32=1) or bf16 [N, Nout]
 *   bwd: dx[row(s)] = dy[out_row(s)] @ W_g^T        (dx optional, f32 or bf16)
 *        dW_g = sum_s x[row(s)]^T dy[out_row(s)]   (dw f32 [G, K, Nout], optional; fixed order)
 * Rows of invalid keys are not written.  K % 8 == 0, Nout % 8 == 0. */
int rte_grouped_linear_fwd(const void* x, int N, int K, const int32_t* offsets, int G, int P,
                           const int32_t* row_of_slot, const int32_t* out_row_of_slot, const void* w, int Nout,
                           void* y, int y_f32, void* stream);
int rte_grouped_linear_bwd(const void* dy, const void* x, int N, int K, const int32_t* offsets, int G, int P,
                           const int32_t* row_of_slot, const int32_t* out_row_of_slot, const void* w, int Nout,
                           void* dx, int dx_f32, float* dw, void* workspace, size_t workspace_bytes,
                           void* stream);
/* Workspace that splits large groups of the dW reduction over several workgroups (same
 * contract as rte_grouped_swiglu_bwd_workspace_bytes). */
size_t rte_grouped_linear_bwd_workspace_bytes(int P, int G, int K, int Nout);

/* ---- deterministic segmented row reduction (rte/kernels/cluster_pool_ffn.py:218-241 index_add_
 * of pool gradients; the backward of every row gather / embedding lookup) ----
 *   out[v] (+)= sum over p < P with keys[p] = v of w[p] * rows[p / row_div]
 * keys int32 [P] (values outside [0, V) are skipped), w f32 [P] (NULL = 1), rows f32 (rows_f32=1)
 * or bf16 [*, d]; out f32 [V, d], overwritten unless accumulate.  V <= 32768, d % 8 == 0, d <= 2048.
 * Summation order is fixed (ascending p per key, 256-pair chunks added in order): bitwise
 * repeatable, no atomics. */
size_t rte_segment_reduce_workspace_bytes(int64_t P, int V, int d);
int rte_segment_reduce_rows(const int32_t* keys, int64_t P, int V, int row_div, const float* w, const void* rows,
                            int rows_f32, int d, float* out, int accumulate, void* workspace, size_t workspace_bytes,
                            void* stream);

/* ---- shortlist output head (rte/output.py:46-136, rte/kernels/reference.py:141-147) ----
 * build: replaces ShortlistHead.build_shortlist / _dedupe_preserve_first (rte/output.py:46-110).
 *   Candidates per token t, in order: targets[t]; members[top_clusters[t, c], :] for c < tc
 *   (members int64 [n_clusters, per_cluster], the padded table of rte/output.py:30-40);
 *   arange(H) % V; random_negs[t, :R]; arange(L) % V; (targets[t] + arange(2L)) % V.
 *   shortlist int32 [T, L] = the first L distinct ids in that order (target at 0);
 *   dup_per_token int32 [T] = candidates - distinct candidates (sum = duplicate_count).
 *   Requires 1 <= L <= V <= 65536. */
int rte_shortlist_build(const int64_t* targets, const int32_t* top_clusters, int tc, const int64_t* members,
                        int n_clusters, int per_cluster, const int64_t* random_negs, int R, int H, int L, int V,
                        int T, int32_t* shortlist, int32_t* dup_per_token, void* stream);
/* fwd: replaces k_logits_shortlist (rte/kernels/reference.py:141-143) + the CE at target position 0
 * (rte/output.py:125-129).  hidden bf16 [T, d], W bf16 [V, d], d % 8 == 0, d <= 2048, L <= 4096.
 * logits f32 [T, L] = hidden . W[shortlist]; lse f32 [T]; loss f32 [T] = lse - logits[:, 0]. */
int rte_shortlist_fwd(const void* hidden, const void* W, int d, int V, const int32_t* shortlist, int L, int T,
                      float* logits, float* lse, float* loss, void* stream);
size_t rte_shortlist_bwd_workspace_bytes(int T, int L, int V, int d);
/* bwd: g = dloss[t] (softmax - e_0) + dlogits (both optional); dhidden bf16 [T, d] (optional) =
 * g . W[shortlist]; dW f32 [V, d] (optional, V <= 32768; overwritten unless dW_accumulate) gets
 * the per-row sums of g * hidden in ascending (t, j) order (deterministic, no atomics). */
int rte_shortlist_bwd(const float* dloss, const float* dlogits, const void* hidden, const void* W, int d, int V,
                      const int32_t* shortlist, int L, int T, const float* logits, const float* lse,
                      void* dhidden, float* dW, int dW_accumulate, void* workspace, size_t workspace_bytes,
                      void* stream);

/* fp32 -> bf16 (round to nearest even) */
int rte_cast_f32_bf16(const float* x, int64_t n, void* y, void* stream);

/* Several fp32 -> bf16 casts in one launch: a training step's bf16 weight copies (the
 * per-step cast of every nn.Linear / bank weight behind the autocast matmuls of
 * rte/layers.py:53-87, 659-779).  jobs (device, int64 [njobs, 8]): {src, dst, rows, cols, ld,
 * kind, first_blk, 0}; dst contiguous bf16 [rows, cols]; kind 0: src the same matrix
 * contiguous; kind 1: src column by column, (r, c) at src[c * ld + r] (a transposed view).
 * Job j owns workgroups first_blk .. first_blk + rte_cast_many_blocks(kind, rows, cols) - 1;
 * blk (device, int32 [nblk]) holds each workgroup's job.  Bit-identical to rte_cast_f32_bf16. */
int rte_cast_many_blocks(int kind, int64_t rows, int64_t cols);
int rte_cast_many(const int64_t* jobs, const int32_t* blk, int nblk, void* stream);

/* ---- fp32 arithmetic: training.precision = "fp32", the reference default (rte/config.py:118),
 * where every matmul of rte/layers.py, rte/macro.py and rte/models.py runs in float32 outside
 * autocast (rte/training.py:356-363).  All buffers f32, fp32 accumulation. ---- */
/* C(m,n) = alpha sum_k A(m,k) B(n,k) + beta C(m,n) on v_mfma_f32_32x32x2_f32.
 * a_t == 0: A(m,k) = A[row(m)*lda + k]   a_t == 1: A(m,k) = A[row(k)*lda + m]   (same for B with n)
 * row(i) = a_rows ? a_rows[i] : i; a_scale (optional) multiplies A's memory row i by a_scale[i]
 * (same for B); c_rows (optional) scatters output row m to c_rows[m].
 * Batch z in [0, Z1*Z2): operand X starts at X + (z / Z2) sX1 + (z % Z2) sX2 (at most 65535).
 * Replaces torch's fp32 matmuls: nn.Linear (rte/layers.py:53-87), the SDPA products
 * (rte/kernels/optimized.py:75-91), k_qkv_dense / k_swiglu_dense / k_logits_* (rte/kernels/reference.py). */
int rte_gemm_f32(const float* A, int64_t lda, int a_t, const int32_t* a_rows, const float* a_scale, const float* B,
                 int64_t ldb, int b_t, const int32_t* b_rows, const float* b_scale, float* C, int64_t ldc,
                 const int32_t* c_rows, int M, int N, int K, float alpha, float beta, int Z1, int Z2, int64_t sA1,
                 int64_t sA2, int64_t sB1, int64_t sB2, int64_t sC1, int64_t sC2, void* stream);
/* Grouped form over device offsets goff[G+1] (int32).  mode 1 (rows): group g computes output rows
 * [goff[g], goff[g+1]) of the M total with B at b_goff[g] (int64, optional) or g*b_gstride and
 * b_rows shifted by g*b_rows_gstride: the routed / banked pools' per-cluster products and the macro
 * operator's per-(recipe, stride) products (replacing the bmm over gathered per-sample weights of
 * rte/macro.py:208-221 and the pooled bmm of rte/kernels/cluster_pool_ffn.py:192-215).  mode 2
 * (reduction): group g sums k over [goff[g], goff[g+1]) into C at c_goff[g] or g*c_gstride, rows
 * through c_rows shifted by g*c_rows_gstride: their weight gradients, one workgroup per output tile
 * summing its group's rows in order (replacing index_add_ scatter, :218-241; deterministic). */
int rte_gemm_f32_grouped(int mode, const int32_t* goff, int G, const float* A, int64_t lda, int a_t,
                         const int32_t* a_rows, const float* a_scale, const float* B, int64_t ldb, int b_t,
                         const int32_t* b_rows, const float* b_scale, const int64_t* b_goff, int64_t b_gstride,
                         int64_t b_rows_gstride, float* C, int64_t ldc, const int32_t* c_rows, const int64_t* c_goff,
                         int64_t c_gstride, int64_t c_rows_gstride, int M, int N, int K, float alpha, float beta,
                         void* stream);
/* Causal softmax of score rows s [Z, S, S] (F.scaled_dot_product_attention(is_causal=True)'s
 * softmax, rte/kernels/optimized.py:75-91): p = softmax(scale s) over keys <= query, y = oscale[z] p
 * (oscale optional: the banked recipe's head mask, rte/layers.py:702-728).  rows = Z*S. */
int rte_softmax_causal_f32_fwd(const float* s, int64_t rows, int S, float scale, const float* oscale, float* p,
                               float* y, void* stream);
/* ds = scale p (g - sum p g) with g = oscale[z] dy */
int rte_softmax_causal_f32_bwd(const float* p, const float* dy, int64_t rows, int S, float scale,
                               const float* oscale, float* ds, void* stream);
/* z = up silu(gate) over rows [up (n) | gate (n)] of width ld (rte/layers.py:78-87), and its
 * backward (rte/kernels/active_swiglu_triton.py:87-102) into dug with the same layout. */
int rte_swiglu_f32_fwd(const float* ug, int64_t rows, int n, int64_t ld, float* z, void* stream);
int rte_swiglu_f32_bwd(const float* ug, const float* dz, int64_t rows, int n, int64_t ld, float* dug, void* stream);
/* out[t] = resid[t] + sum_j w[t,j] rows[slot[t k + j]] in j order (slot < 0: no pair; w, resid
 * optional): the pooled FFN's gather back to tokens (rte/kernels/cluster_pool_ffn.py:215). */
int rte_combine_f32(const float* rows, const int32_t* slot, const float* w, int T, int k, int d, const float* resid,
                    float* out, void* stream);
/* dw[p] = dout[p / k] . rows[slot[p]] (0 for slot < 0): the routing weights' gradient. */
int rte_pair_dot_f32(const float* dout, const float* rows, const int32_t* slot, int64_t pairs, int k, int d, float* dw,
                     void* stream);

/* ---------------------------------------------------------------- exact replay of the banked core
 * One exact recursive pass of BankedRecursiveCore.forward_step (rte/layers.py:806-870, one bank of
 * heads and of FFN slabs) for the few samples of the audit's exact replay, which forward_exact runs
 * pass by pass (rte/models.py:416-512, called from rte/audit.py:245-387 on the audited rows):
 *   h~ = h + alpha h0; n1 = rmsnorm(h~) w1 (1 + g1) + b1; attention over the recipe's heads (RoPE,
 *   causal, scale 1/8); u = h~ + s_attn attn; n2 = rmsnorm(u) w2 (1 + g2) + b2; SwiGLU over the
 *   recipe's slabs (route weight route_w); h' = act ? u + s_mlp mlp : h.
 * Shapes: B samples x S positions (M = B S rows), d <= 512 (d % 128 == 0), H heads of width 64
 * (H 64 = d), F = n_blk 32 FFN neurons.  info int32 [B, W] (W = 4 + 2 H + 2 n_blk), one record per
 * sample for this pass: act | nh | nb | 0 | heads[H] (the recipe's heads, ascending) | ihead[H]
 * (slot of each head or -1) | blks[n_blk] (its 32-neuron slab blocks, ascending) | iblk[n_blk];
 * h_max / nb_max = the largest nh / nb.  Weights bf16: wqkv_t [3d, d], wo_t [d, d], wug_t [2F, d]
 * (rows up F then gate F), wd_t [d, F] for the forward; wqkv [d, 3d], wo [d, d], wug [d, 2F], wd
 * [F, d] for the backward.  cos / sin f32 [S, 64].  Scalars s_attn, s_mlp, alpha: device f32.
 * fwd outputs: ht, attn, u, mlp, h_out f32 [M, d]; n1, n2 bf16 [M, d]; rstd1, rstd2 f32 [M]; q, k, v
 * bf16 [B, h_max, S, 64] (compact heads); y bf16 [M, h_max 64]; lse f32 [B, h_max, S]; ug bf16
 * [M, nb_max 64] ([up 32 | gate 32] per slot); z bf16 [M, nb_max 32]; y_full bf16 [M, d], z_full
 * bf16 [M, F] (zeros outside the recipe's heads / blocks).
 * bwd_prep (once, for the first pass the backward visits): a_mlp = bf16(s_mlp dh) bf16 [M, d] and
 * p_sm f32 [nt] (per row-workgroup sums of dh mlp), nt = rte_replay_row_tiles(B, S) = ceil(M / 4).
 * bwd (dh f32 [M, d] = gradient of h_out, a_mlp from bwd_prep or the previous bwd call):
 * dh_in f32 [M, d], dh0 f32 [M, d] (alpha dh~, added to its contents when accumulate), the
 * weight-gradient operands d_attn bf16 [M, d], dug_full bf16 [M, 2F], dqkv_full bf16 [M, 3d]
 * (dW = operand^T pair summed over passes: dWqkv = n1^T dqkv_full, dWo = y_full^T d_attn,
 * dWug = n2^T dug_full, dWd = z_full^T a_mlp), and per-row-workgroup partials: p_film1, p_film2
 * f32 [nt, 3d] (dw | dg | db), p_sa, p_alpha f32 [nt].  With a_next (the pass before this one):
 * its down operand a_next = bf16(s_mlp_next dh_in) [M, d] and p_sm_next f32 [nt] from mlp_next.
 * Scratch: dug bf16 [M, nb_max 64], dn2, dn1, du f32 [M, d], dy bf16 [M, h_max 64], dqkv bf16
 * [M, 3 h_max 64].
 * param_reduce: out f32 [T, 6d] (per pass dw1 | dg1 | db1 | dw2 | dg2 | db2), then dw1 [d], dw2 [d]
 * over the T passes, ds_attn [T], ds_mlp [T], dalpha [1]; partials stacked pass-major. */
int rte_replay_row_tiles(int B, int S);
int rte_replay_fwd_pass(int B, int S, int d, int H, int F, int n_blk, int h_max, int nb_max, const int32_t* info,
                        const float* h, const float* h0, const float* alpha, const float* w1, const float* g1,
                        const float* b1, float eps1, const float* w2, const float* g2, const float* b2, float eps2,
                        const float* s_attn, const float* s_mlp, float route_w, const void* wqkv_t, const void* wo_t,
                        const void* wug_t, const void* wd_t, const float* cos_t, const float* sin_t, float* ht,
                        void* n1, float* rstd1, void* q, void* k, void* v, void* y, float* lse, float* attn, float* u,
                        void* y_full, void* n2, float* rstd2, void* ug, void* z, float* mlp, float* h_out,
                        void* z_full, void* stream);
int rte_replay_bwd_prep(int B, int S, int d, const float* dh, const float* mlp, const float* s_mlp, void* a_mlp,
                        float* p_sm, void* stream);
int rte_replay_bwd_pass(int B, int S, int d, int H, int F, int n_blk, int h_max, int nb_max, const int32_t* info,
                        const float* dh, const void* a_mlp, const void* wd, const void* ug, float route_w, void* dug,
                        const void* wug, float* dn2, void* dug_full, const float* u, const float* rstd2,
                        const float* w2, const float* g2, const float* attn, const float* s_attn, float* du,
                        void* d_attn, float* p_film2, float* p_sa, const void* wo, void* dy, const void* q,
                        const void* k, const void* v, const void* y, const float* lse, const float* cos_t,
                        const float* sin_t, void* dqkv, const void* wqkv, float* dn1, void* dqkv_full,
                        const float* ht, const float* rstd1, const float* w1, const float* g1, const float* h0,
                        const float* alpha, int accumulate, float* dh_in, float* dh0, float* p_film1, float* p_alpha,
                        const float* mlp_next, const float* s_mlp_next, void* a_next, float* p_sm_next, void* stream);
int rte_replay_param_reduce(int T, int B, int S, int d, const float* p_film1, const float* p_film2,
                            const float* p_sa, const float* p_sm, const float* p_alpha, float* out, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* RTE_HIP_H */
