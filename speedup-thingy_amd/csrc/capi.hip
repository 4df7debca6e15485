// extern "C" entry points of librte_hip (declared in include/rte_hip.h).
// Composite operators are sequences of GEMM launches from gemm.hip plus the
// routing / norm helpers; nothing here allocates device memory.
#include "../../include/rte_hip.h"
#include "gemm.hpp"

#include <stdio.h>
#include <string.h>

namespace rte {
const char* last_error();
int svd_sparse_select(const bf16* x, const bf16* ug, const bf16* w_up, const bf16* w_gate, const bf16* w_down,
                      const float* wdn, int T, int d, int F, int up_m, int gate_m, int product_m, int top_k,
                      int exact, int product_only, void* out, int out_f32, int32_t* sel_ids, float* sel_u,
                      float* sel_g, int32_t* n_cand, hipStream_t s);
int svd_sparse_bwd(const bf16* dout, const bf16* w_up, const bf16* w_gate, const bf16* w_down, const int32_t* sel_ids,
                   const float* sel_u, const float* sel_g, int T, int d, int top_k, bf16* dx, float* z, float* du,
                   float* dg, hipStream_t s);
int route_topk(const float* logits, int T, int C, int k, int32_t* ids, float* weights, hipStream_t s);
size_t route_pack_workspace_bytes(int T, int C);
int route_pack(const bf16* x, int T, int d, const bf16* wr, int C, int k, int32_t* ids, float* weights,
               int32_t* offsets, int32_t* tok_of_slot, int32_t* pair_of_slot, int32_t* slot_of_pair,
               float* w_of_slot, float* logits, void* ws, size_t ws_bytes, hipStream_t s);
size_t pack_workspace_bytes(int P, int C);
int pack_pairs(const int32_t* cl, int P, int C, int k, const float* w, int32_t* offsets,
               int32_t* tok_of_slot, int32_t* pair_of_slot, int32_t* slot_of_pair, float* w_of_slot,
               int32_t* invalid, void* ws, size_t ws_bytes, hipStream_t s);
int combine_rows(const bf16* rows, int T, int k, int d, const int32_t* slot_of_pair, const bf16* extra,
                 const float* resid, void* out,
                 int out_f32, hipStream_t s);
int route_bwd(const int32_t* ids, const float* w, const float* dw_slot, const int32_t* slot_of_pair, int T,
              int C, int k, bf16* dlogits, float* dlogits_f32, hipStream_t s);
int rmsnorm_fwd(const float* x, const float* w, int T, int d, float eps, bf16* out, float* rstd,
                hipStream_t s);
size_t rmsnorm_bwd_workspace_bytes(int T, int d);
int rmsnorm_bwd(const bf16* dy, const float* x, const float* w, const float* rstd, const float* dres, int T,
                int d, float* dx, bf16* dx_bf16, float* dw, int dw_accumulate, void* ws, size_t ws_bytes, hipStream_t s);
int rope_bwd_pack(const bf16* dq, const int64_t* sq, const bf16* dk, const int64_t* sk, const bf16* dv,
                  const int64_t* sv, const float* cos_t, const float* sin_t, int B, int H, int S, int hd,
                  bf16* dqkv, hipStream_t s);
int cast_f32_bf16(const float* x, int64_t n, bf16* y, hipStream_t s);
int cast_many_blocks(int kind, int64_t rows, int64_t cols);
int cast_many(const int64_t* jobs, const int32_t* blk, int nblk, hipStream_t s);
int ce_fwd(const float* logits, int64_t ld, int T, int V, const int64_t* targets, float* loss, float* lse,
           hipStream_t s);
int ce_bwd(const float* logits, int64_t ld, int T, int V, const int64_t* targets, const float* lse, const float* g,
           const float* extra, const int64_t* ext_ids, int ext_k, int ext_S, bf16* dlogits, hipStream_t s);
int axpy_norm_fwd(const float* a, const float* b, const float* c, const float* keep, const uint8_t* mask, int S,
                  int T, int d, const float* w, const float* gamma, const float* beta, float eps, float* x_out,
                  bf16* n_out, float* rstd_out, hipStream_t s);
size_t axpy_norm_bwd_workspace_bytes(int T, int d);
int axpy_norm_bwd(const bf16* dn, const float* dx_ext, const float* x, const float* rstd, const float* w,
                  const float* gamma, const float* b, const float* c, const uint8_t* mask, int S, int T, int d,
                  float* da, float* db, float* dkeep, float* dparams, void* ws, size_t ws_bytes, hipStream_t s);
int macro_parts(int B, int S);
size_t macro_workspace_bytes(int B, int S, int d);
int macro_prologue_fwd(const float* h, const float* h0, int B, int Bh0, int S, int d, float eps, bf16* z, float* rstd,
                       void* ws, size_t ws_bytes, hipStream_t s);
int macro_prologue_bwd(const bf16* dz, const float* h, const float* rstd, const float* dh_extra, int Bt, int Bh, int S,
                       int d, float* dh, float* dh0, void* ws, size_t ws_bytes, hipStream_t s);
int macro_epilogue_fwd(const float* h, const float* low, const int64_t* key, int B, int Bh, int S, int d,
                       const float* gain, const float* bias, const float* scale, float c, float* out, hipStream_t s);
int macro_epilogue_bwd(const float* dout, const float* h, const float* low, const int64_t* key, int B, int Bh, int S,
                       int d, const float* gain, const float* bias, const float* scale, float c, float* dh, bf16* dlow,
                       void* part, size_t part_bytes, hipStream_t s);
int macro_table_grad(const int64_t* key, int B, int S, int G, int d, const void* part, float* dgain, float* dbias,
                     float* dscale, hipStream_t s);
int macro_fused_tiles(int S);
size_t macro_fused_fwd_workspace_bytes(int Bh, int S, int d);
size_t macro_fused_wgrad_workspace_bytes(int Bt, int S, int d, int G);
int macro_fused_prep(const float* V, const float* U, int G, int d, bf16* Vb, bf16* VcT, bf16* V2T, bf16* Ub, bf16* UT,
                     hipStream_t s);
size_t macro_fused_bwd_workspace_bytes(int B, int S);
int macro_fused_fwd(const float* h, const float* h0, int Bh, int Bh0, const int64_t* key, int B, int S, int d, int G,
                    float eps, const bf16* Vb, const bf16* VcT, const bf16* UT, const float* gain, const float* bias,
                    const float* scale, float c, bf16* x2, float* rstd, bf16* pooled, float* P, float* a, bf16* sa,
                    float* out, const float* mse_ref, float* mse_part, void* ws, size_t ws_bytes, hipStream_t s);
int macro_fused_sum(const float* part, int n, float inv_n, float* out, hipStream_t s);
int macro_fused_bwd(const float* dp, const float* dq, const float* g, float mul, int diff_lo, int n_diff,
                    const float* dbuf, int buf_lo, int n_buf,
                    const float* h, const float* rstd, const bf16* x2, int Bh, const int64_t* key, int B, int S, int d,
                    int G, const float* a, const bf16* sa, const bf16* Vb, const bf16* VcT, const bf16* V2T,
                    const bf16* Ub, const bf16* UT, const float* gain, const float* bias, const float* scale, float c,
                    bf16* du, bf16* da, float* part_tab, float* part_da, float* dh, float* dh0, int dh0_into_dh,
                    const float* extra, int n_extra, bf16* dsum, void* ws, size_t ws_bytes, hipStream_t s);
int macro_fused_wgrad(const int64_t* key, int B0, int Bh0, int B1, int Bh1, int S, int d, int G, const bf16* x2,
                      const bf16* sa, const bf16* du, const bf16* da, const bf16* pooled, const bf16* dsum,
                      const float* part_tab, float* dU, float* dV, float* dgain, float* dbias, float* dscale,
                      void* ws, size_t ws_bytes, hipStream_t s);
size_t mse_workspace_bytes(int64_t n);
int mse_fwd(const float* a, const float* b, int64_t n, float* out, void* ws, size_t ws_bytes, hipStream_t s);
int mse_bwd(const float* a, const float* b, int64_t n, const float* g, float* da, float* db, hipStream_t s);
size_t pack_routes_workspace_bytes(int B, int kmax);
int pack_routes(const int64_t* rid, const uint8_t* active, int B, int S, const int32_t* routes, int R, int kmax,
                const float* route_w, int C, int32_t* offsets, int32_t* tok_of_slot, int32_t* pair_of_slot,
                int32_t* slot_of_pair, float* w_of_slot, void* ws, size_t ws_bytes, hipStream_t s);
int adamw_chunk();
size_t adamw_workspace_bytes(int nt, int nblk, int G);
int adamw_step(const void* rows, int nt, const int32_t* blk, const int32_t* first_blk, int nblk, const double* hyper,
               int G, const int32_t* metric_lr_group, int M, float clip_max, const float* found_inf, float* metrics,
               void* ws, size_t ws_bytes, hipStream_t s);
int attention_fwd(const bf16* q, const bf16* k, const bf16* v, int B, int H, int S, int head_dim, float scale,
                  const float* hscale, bf16* out, float* lse, hipStream_t s);
int attention_bwd(const bf16* q, const bf16* k, const bf16* v, const bf16* out, const bf16* dout, const float* lse,
                  int B, int H, int S, int head_dim, float scale, const float* hscale, bf16* dq, bf16* dk, bf16* dv,
                  hipStream_t s);
int attention_bwd_qkv(const bf16* q, const bf16* k, const bf16* v, const bf16* out, const bf16* dout,
                      const float* lse, int B, int H, int S, int head_dim, float scale, const float* hscale,
                      const float* cos_t, const float* sin_t, bf16* dqkv, hipStream_t s);
size_t distill_workspace_bytes(int A, int R);
int distill_fwd(const float* hot, const float* exact, const float* h0, int A, int S, int d, const float* hot_logits,
                const float* exact_logits, int V, float t, float eps, const float* weights, float* losses,
                float* metrics, void* ws, size_t ws_bytes, hipStream_t s);
int distill_bwd(const float* hot, const float* exact, const float* h0, int A, int S, int d, const float* hot_logits,
                const float* exact_logits, int V, float t, float eps, const float* weights, const float* g,
                const void* ws, size_t ws_bytes, float* dhot, float* dhot_logits, hipStream_t s);
int audit_fwd(const float* hot_tok, const float* exact_tok, int B, int S, const int64_t* idx, int A, const float* p,
              float clip, int grad_corrected, float* corrected, float* exact_ps, float* coef, float* stats,
              hipStream_t s);
int audit_bwd(const float* g, int B, int S, const int64_t* idx, int A, const float* coef, float* dhot_tok,
              float* dexact_tok, hipStream_t s);
int shortlist_build(const int64_t* targets, const int32_t* top_clusters, int tc, const int64_t* members,
                    int n_clusters, int per_cluster, const int64_t* random_negs, int R, int H, int L, int V, int T,
                    int32_t* shortlist, int32_t* dup_per_token, hipStream_t s);
int shortlist_fwd(const bf16* hidden, const bf16* W, int d, int V, const int32_t* sl, int L, int T, float* logits,
                  float* lse, float* loss, hipStream_t s);
size_t shortlist_bwd_workspace_bytes(int T, int L, int V, int d);
int shortlist_bwd(const float* dloss, const float* dlext, const bf16* hidden, const bf16* W, int d, int V,
                  const int32_t* sl, int L, int T, const float* logits, const float* lse, bf16* dhidden, float* dW,
                  int dW_accumulate, void* ws, size_t ws_bytes, hipStream_t s);
size_t segreduce_workspace_bytes(int64_t P, int V, int d);
int segreduce_rows(const int32_t* keys, int64_t P, int V, int row_div, const float* w, const void* rows, int rows_f32,
                   int d, float* out, int accumulate, void* ws, size_t ws_bytes, hipStream_t s);
bool pool_fused_supported(int n, int d);
int pool_fused_fwd(const bf16* x, int d, const int32_t* offsets, int G, int n, int P, const int32_t* tok_of_slot,
                   const int32_t* pair_of_slot, const float* w_of_slot, const bf16* wug, const bf16* wd,
                   int64_t ld_wd, bf16* ug, bf16* zw, bf16* y_pairs, hipStream_t s);
int pool_fused_bwd(const bf16* dout, int d, const int32_t* offsets, int G, int n, int P, const int32_t* tok_of_slot,
                   const int32_t* pair_of_slot, const float* w_of_slot, const bf16* wug, const bf16* wd,
                   int64_t ld_wd, const bf16* ug, bf16* dug, float* dw_slot, bf16* dx_pairs, hipStream_t s);
}  // namespace rte

using namespace rte;

namespace {

inline hipStream_t S(void* s) { return reinterpret_cast<hipStream_t>(s); }
inline const bf16* B16(const void* p) { return static_cast<const bf16*>(p); }
inline bf16* B16(void* p) { return static_cast<bf16*>(p); }

Operand plain(const void* p, int64_t ld) {
  Operand o;
  o.ptr = B16(p);
  o.ld = ld;
  return o;
}

Operand from_layout(const void* p, const int64_t* L) {
  Operand o;
  o.ptr = B16(p);
  o.ld = L[0];
  o.rdiv = (int32_t)L[1];
  o.rs_hi = L[2];
  o.cdiv = (int32_t)L[3];
  o.cs_hi = L[4];
  return o;
}

// Weight gradients of the grouped SwiGLU (grouped-K reductions over each cluster's slots): dWug from
// x[tok] and dUG, dWd from zw and dout[tok], in the parameters' layout (w_t = 0) or transposed.
int pool_wgrad(const void* dout, const void* x, int d, const int32_t* offsets, int G, int n, int P,
               const int32_t* tok_of_slot, int64_t ld_wd, const void* zw, const void* dug, float* dwug, float* dwd,
               int w_t, float beta, void* workspace, size_t workspace_bytes, hipStream_t stream) {
  const int dff = G * n;
  if (w_t) {
    // dWug^T[:, ilv(g*2n + c)] = sum_slot x[tok(slot), :] dUG[slot, c]   ([d, 2F]: columns [up F | gate F])
    GemmArgs p;
    p.mode = MODE_GROUP_K;
    p.goff = offsets;
    p.G = G;
    p.M = d;
    p.N = 2 * n;
    p.K = P;
    p.a = plain(x, d);
    p.a.rows = tok_of_slot;
    p.a_t = 1;
    p.b = plain(dug, 2 * n);
    p.b_t = 1;
    p.epi.c = dwug;
    p.epi.ldc = 2 * (int64_t)dff;
    p.epi.c_f32 = 1;
    p.epi.c_gstride = 2 * n;
    p.epi.c_col_ilv = dff;
    p.epi.beta = beta;
    RTE_TRY(gemm_launch(p, EPI_STORE, stream, workspace, workspace_bytes));
  } else {
    // dWug_g[c, :] = sum_slot dUG[slot, c] x[tok(slot), :]
    GemmArgs p;
    p.mode = MODE_GROUP_K;
    p.goff = offsets;
    p.G = G;
    p.M = 2 * n;
    p.N = d;
    p.K = P;
    p.a = plain(dug, 2 * n);
    p.a_t = 1;
    p.b = plain(x, d);
    p.b.rows = tok_of_slot;
    p.b_t = 1;
    p.epi.c = dwug;
    p.epi.ldc = d;
    p.epi.c_f32 = 1;
    p.epi.c_growstride = 2 * n;
    p.epi.c_ilv = dff;
    p.epi.beta = beta;
    RTE_TRY(gemm_launch(p, EPI_STORE, stream, workspace, workspace_bytes));
  }
  if (w_t) {
    // dWd^T[g*n + j, :] = sum_slot zw[slot, j] dout[tok(slot), :]   ([F, d])
    GemmArgs p;
    p.mode = MODE_GROUP_K;
    p.goff = offsets;
    p.G = G;
    p.M = n;
    p.N = d;
    p.K = P;
    p.a = plain(zw, n);
    p.a_t = 1;
    p.b = plain(dout, d);
    p.b.rows = tok_of_slot;
    p.b_t = 1;
    p.epi.c = dwd;
    p.epi.ldc = d;
    p.epi.c_f32 = 1;
    p.epi.c_growstride = n;
    p.epi.beta = beta;
    RTE_TRY(gemm_launch(p, EPI_STORE, stream, workspace, workspace_bytes));
  } else {
    // dWd[:, g*n + j] = sum_slot dout[tok(slot), :] zw[slot, j]
    GemmArgs p;
    p.mode = MODE_GROUP_K;
    p.goff = offsets;
    p.G = G;
    p.M = d;
    p.N = n;
    p.K = P;
    p.a = plain(dout, d);
    p.a.rows = tok_of_slot;
    p.a_t = 1;
    p.b = plain(zw, n);
    p.b_t = 1;
    p.epi.c = dwd;
    p.epi.ldc = ld_wd;
    p.epi.c_f32 = 1;
    p.epi.c_gstride = n;
    p.epi.beta = beta;
    RTE_TRY(gemm_launch(p, EPI_STORE, stream, workspace, workspace_bytes));
  }
  return 0;
}

}  // namespace

extern "C" {

int rte_abi_version(void) { return 1; }

const char* rte_last_error(void) { return last_error(); }

int rte_device_info(char* buf, int buf_len) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) {
    set_error("hipGetDevice: %s", hipGetErrorString(e));
    return (int)e;
  }
  hipDeviceProp_t prop;
  e = hipGetDeviceProperties(&prop, dev);
  if (e != hipSuccess) {
    set_error("hipGetDeviceProperties: %s", hipGetErrorString(e));
    return (int)e;
  }
  int lds_optin = 0;
  hipDeviceGetAttribute(&lds_optin, hipDeviceAttributeSharedMemPerBlockOptin, dev);
  snprintf(buf, buf_len, "arch=%s;name=%s;cus=%d;lds_per_block=%zu;lds_optin=%d;clock_khz=%d;hbm_bytes=%zu",
           prop.gcnArchName, prop.name, prop.multiProcessorCount, (size_t)prop.sharedMemPerBlock, lds_optin,
           prop.clockRate, (size_t)prop.totalGlobalMem);
  return 0;
}

size_t rte_gemm_workspace_bytes(int M, int N, int K) { return gemm_splitk_bytes(M, N, K); }

int rte_gemm_bf16(const void* a, int64_t lda, int a_t, const int32_t* a_rows, const void* b, int64_t ldb,
                  int b_t, const int32_t* b_rows, void* c, int64_t ldc, int c_f32, int M, int N, int K,
                  float alpha, float beta, const float* resid, int64_t ld_resid, void* workspace,
                  size_t workspace_bytes, void* stream) {
  GemmArgs p;
  p.a = plain(a, lda);
  p.a.rows = a_rows;
  p.b = plain(b, ldb);
  p.b.rows = b_rows;
  p.a_t = a_t;
  p.b_t = b_t;
  p.M = M;
  p.N = N;
  p.K = K;
  p.epi.c = c;
  p.epi.ldc = ldc;
  p.epi.c_f32 = c_f32;
  p.epi.alpha = alpha;
  p.epi.beta = beta;
  p.epi.resid = resid;
  p.epi.ld_resid = ld_resid;
  return gemm_launch(p, EPI_STORE, S(stream), workspace, workspace_bytes);
}

int rte_gemm_bf16_split(const void* a, const int64_t* a_layout, int a_t, const void* b, const int64_t* b_layout,
                        int b_t, void* c, int64_t ldc, int c_f32, int M, int N, int K, float alpha, float beta,
                        const float* resid, int64_t ld_resid, void* workspace, size_t workspace_bytes,
                        void* stream) {
  GemmArgs p;
  p.a = from_layout(a, a_layout);
  p.b = from_layout(b, b_layout);
  p.a_t = a_t;
  p.b_t = b_t;
  p.M = M;
  p.N = N;
  p.K = K;
  p.epi.c = c;
  p.epi.ldc = ldc;
  p.epi.c_f32 = c_f32;
  p.epi.alpha = alpha;
  p.epi.beta = beta;
  p.epi.resid = resid;
  p.epi.ld_resid = ld_resid;
  // split columns must keep 8-element vectors inside one segment
  if (p.a.cdiv) RTE_REQUIRE(p.a.cdiv % 8 == 0, "gemm_split: A cdiv must be a multiple of 8");
  if (p.b.cdiv) RTE_REQUIRE(p.b.cdiv % 8 == 0, "gemm_split: B cdiv must be a multiple of 8");
  return gemm_launch(p, EPI_STORE, S(stream), workspace, workspace_bytes);
}

int rte_route_topk(const float* logits, int T, int C, int k, int32_t* ids, float* weights, void* stream) {
  return route_topk(logits, T, C, k, ids, weights, S(stream));
}

size_t rte_pack_workspace_bytes(int P, int C) { return pack_workspace_bytes(P, C); }

size_t rte_route_pack_workspace_bytes(int T, int C) { return route_pack_workspace_bytes(T, C); }

int rte_route_pack(const void* x, int T, int d, const void* wr, int C, int k, int32_t* ids, float* weights,
                   int32_t* offsets, int32_t* tok_of_slot, int32_t* pair_of_slot, int32_t* slot_of_pair,
                   float* w_of_slot, float* logits, void* workspace, size_t workspace_bytes, void* stream) {
  return route_pack(B16(x), T, d, B16(wr), C, k, ids, weights, offsets, tok_of_slot, pair_of_slot, slot_of_pair,
                    w_of_slot, logits, workspace, workspace_bytes, S(stream));
}

int rte_pack_index(const int32_t* cl, int P, int C, int k, const float* w, int32_t* offsets,
                   int32_t* tok_of_slot, int32_t* pair_of_slot, int32_t* slot_of_pair, float* w_of_slot,
                   int32_t* invalid, void* workspace, size_t workspace_bytes, void* stream) {
  return pack_pairs(cl, P, C, k, w, offsets, tok_of_slot, pair_of_slot, slot_of_pair, w_of_slot, invalid,
                    workspace, workspace_bytes, S(stream));
}

int rte_combine_rows(const void* rows, int T, int k, int d, const int32_t* slot_of_pair, const void* extra,
                     const float* resid, void* out, int out_f32, void* stream) {
  return combine_rows(B16(rows), T, k, d, slot_of_pair, B16(extra), resid, out, out_f32, S(stream));
}

int rte_route_bwd(const int32_t* ids, const float* w, const float* dw_slot, const int32_t* slot_of_pair, int T,
                  int C, int k, void* dlogits_bf16, float* dlogits_f32, void* stream) {
  return route_bwd(ids, w, dw_slot, slot_of_pair, T, C, k, B16(dlogits_bf16), dlogits_f32, S(stream));
}

int rte_grouped_swiglu_fwd(const void* x, int T, int d, const int32_t* offsets, int G, int n, int P,
                           const int32_t* tok_of_slot, const int32_t* pair_of_slot, const float* w_of_slot,
                           const void* wug, const void* wd, int64_t ld_wd, void* ug, void* zw, void* y_pairs,
                           void* stream) {
  RTE_REQUIRE(n % 32 == 0, "grouped_swiglu: neurons per cluster must be a multiple of 32");
  RTE_REQUIRE(d % 8 == 0, "grouped_swiglu: d_model must be a multiple of 8");
  RTE_REQUIRE(T >= 0 && P >= 0 && G >= 1, "grouped_swiglu: bad sizes");
  if (P == 0) return 0;
  const int dff = G * n;
  const int tiles = P / kGroupTileM + G + 1;
  // stage 1: UG = x[tok] @ [W_up_g ; W_gate_g]^T  (interleaved per 32), SwiGLU -> zw
  {
    GemmArgs p;
    p.mode = MODE_GROUP_M;
    p.goff = offsets;
    p.G = G;
    p.max_tiles_m = tiles;
    p.M = P;
    p.N = 2 * n;
    p.K = d;
    p.a = plain(x, d);
    p.a.rows = tok_of_slot;
    p.b = plain(wug, d);
    p.b.growstride = 2 * n;
    p.b.ilv = dff;
    p.epi.ug = B16(ug);
    p.epi.ld_ug = 2 * n;
    p.epi.z = B16(zw);
    p.epi.ld_z = n;
    p.epi.row_scale = w_of_slot;
    RTE_TRY(gemm_launch(p, EPI_SWIGLU_FWD, S(stream)));
  }
  // stage 2: y_pairs[pair] = zw @ W_down_g    (B(n=dcol, k=j) = wd[dcol*ld_wd + g*n + j])
  {
    GemmArgs p;
    p.mode = MODE_GROUP_M;
    p.goff = offsets;
    p.G = G;
    p.max_tiles_m = tiles;
    p.M = P;
    p.N = d;
    p.K = n;
    p.a = plain(zw, n);
    p.b = plain(wd, ld_wd);
    p.b.gstride = n;
    p.epi.c = y_pairs;
    p.epi.ldc = d;
    p.epi.c_rows = pair_of_slot;
    RTE_TRY(gemm_launch(p, EPI_STORE, S(stream)));
  }
  (void)T;
  return 0;
}

int rte_grouped_swiglu_bwd(const void* dout, const void* x, int T, int d, const int32_t* offsets, int G, int n,
                           int P, const int32_t* tok_of_slot, const int32_t* pair_of_slot,
                           const float* w_of_slot, const void* wug, const void* wd, int64_t ld_wd, const void* ug,
                           const void* zw, void* dug, float* dw_slot, void* dx_pairs, float* dwug, float* dwd,
                           int w_t, float beta, void* workspace, size_t workspace_bytes, void* stream) {
  RTE_REQUIRE(n % 32 == 0 && n <= 128, "grouped_swiglu_bwd: n must be a multiple of 32 and <= 128");
  RTE_REQUIRE(w_t == 0 || w_t == 1, "grouped_swiglu_bwd: w_t must be 0 or 1");
  RTE_REQUIRE(d % 8 == 0, "grouped_swiglu_bwd: d_model must be a multiple of 8");
  const int dff = G * n;
  const int tiles = P / kGroupTileM + G + 1;
  if (P > 0) {
    // dZw = dout[tok] @ W_down_g^T  -> SwiGLU backward epilogue (dz = w * dZw), dw_slot = <z, dZw>
    GemmArgs p;
    p.mode = MODE_GROUP_M;
    p.goff = offsets;
    p.G = G;
    p.max_tiles_m = tiles;
    p.M = P;
    p.N = n;
    p.K = d;
    p.a = plain(dout, d);
    p.a.rows = tok_of_slot;
    p.b = plain(wd, ld_wd);  // B(n=j, k=dcol) = wd[dcol*ld_wd + g*n + j]  -> layout T
    p.b.gstride = n;
    p.b_t = 1;
    p.epi.ug_in = B16(ug);
    p.epi.ug = B16(dug);
    p.epi.ld_ug = 2 * n;
    p.epi.row_scale = w_of_slot;
    p.epi.dw_row = dw_slot;
    RTE_TRY(gemm_launch(p, EPI_SWIGLU_BWD, S(stream)));
  }
  if (P > 0) {
    // dx_pairs[pair] = dUG @ [W_up_g ; W_gate_g]   (B(n=dcol, k=c) = wug[ilv(g*2n + c)][dcol] -> layout T)
    GemmArgs p;
    p.mode = MODE_GROUP_M;
    p.goff = offsets;
    p.G = G;
    p.max_tiles_m = tiles;
    p.M = P;
    p.N = d;
    p.K = 2 * n;
    p.a = plain(dug, 2 * n);
    p.b = plain(wug, d);
    p.b.growstride = 2 * n;
    p.b.ilv = dff;
    p.b_t = 1;
    p.epi.c = dx_pairs;
    p.epi.ldc = d;
    p.epi.c_rows = pair_of_slot;
    RTE_TRY(gemm_launch(p, EPI_STORE, S(stream)));
  }
  RTE_TRY(pool_wgrad(dout, x, d, offsets, G, n, P, tok_of_slot, ld_wd, zw, dug, dwug, dwd, w_t, beta, workspace,
                     workspace_bytes, S(stream)));
  (void)T;
  (void)pair_of_slot;
  return 0;
}

size_t rte_grouped_swiglu_bwd_workspace_bytes(int P, int G, int n, int d) {
  const size_t a = gemm_groupk_bytes(2 * n, d, P, G), b = gemm_groupk_bytes(d, n, P, G);
  return a > b ? a : b;
}

int rte_grouped_swiglu_fused_ok(int n, int d) { return pool_fused_supported(n, d) ? 1 : 0; }

int rte_grouped_swiglu_fused_fwd(const void* x, int T, int d, const int32_t* offsets, int G, int n, int P,
                                 const int32_t* tok_of_slot, const int32_t* pair_of_slot, const float* w_of_slot,
                                 const void* wug, const void* wd, int64_t ld_wd, void* ug, void* zw, void* y_pairs,
                                 void* stream) {
  (void)T;
  return pool_fused_fwd(B16(x), d, offsets, G, n, P, tok_of_slot, pair_of_slot, w_of_slot, B16(wug), B16(wd), ld_wd,
                        B16(ug), B16(zw), B16(y_pairs), S(stream));
}

int rte_grouped_swiglu_fused_bwd(const void* dout, const void* x, int T, int d, const int32_t* offsets, int G, int n,
                                 int P, const int32_t* tok_of_slot, const int32_t* pair_of_slot,
                                 const float* w_of_slot, const void* wug, const void* wd, int64_t ld_wd,
                                 const void* ug, const void* zw, void* dug, float* dw_slot, void* dx_pairs,
                                 float* dwug, float* dwd, int w_t, float beta, void* workspace, size_t workspace_bytes,
                                 void* stream) {
  RTE_REQUIRE(w_t == 0 || w_t == 1, "grouped_swiglu_bwd: w_t must be 0 or 1");
  (void)T;
  RTE_TRY(pool_fused_bwd(B16(dout), d, offsets, G, n, P, tok_of_slot, pair_of_slot, w_of_slot, B16(wug), B16(wd),
                         ld_wd, B16(ug), B16(dug), dw_slot, B16(dx_pairs), S(stream)));
  return pool_wgrad(dout, x, d, offsets, G, n, P, tok_of_slot, ld_wd, zw, dug, dwug, dwd, w_t, beta, workspace,
                    workspace_bytes, S(stream));
}

int rte_dense_swiglu_fwd(const void* x, int T, int d, int F, const void* wug, const void* wd, int wd_rows,
                         const float* resid, void* ug, void* z, void* out, int out_f32, void* stream) {
  RTE_REQUIRE(F % 32 == 0 && d % 8 == 0, "dense_swiglu: F %% 32 and d %% 8 must be 0");
  {
    GemmArgs p;
    p.M = T;
    p.N = 2 * F;
    p.K = d;
    p.a = plain(x, d);
    p.b = plain(wug, d);
    p.b.ilv = F;
    p.epi.ug = B16(ug);
    p.epi.ld_ug = 2 * F;
    p.epi.z = B16(z);
    p.epi.ld_z = F;
    RTE_TRY(gemm_launch(p, EPI_SWIGLU_FWD, S(stream)));
  }
  {
    // out = z @ W_down:  B(n=dcol, k=f) = wd[dcol][f] (layout N) or wd[f][dcol] (layout T)
    GemmArgs p;
    p.M = T;
    p.N = d;
    p.K = F;
    p.a = plain(z, F);
    p.b = plain(wd, wd_rows ? d : F);
    p.b_t = wd_rows ? 1 : 0;
    p.epi.c = out;
    p.epi.ldc = d;
    p.epi.c_f32 = out_f32;
    p.epi.resid = resid;
    p.epi.ld_resid = d;
    RTE_TRY(gemm_launch(p, EPI_STORE, S(stream)));
  }
  return 0;
}

int rte_dense_swiglu_bwd(const void* dout, const void* x, int T, int d, int F, const void* wug, const void* wd,
                         int wd_rows, const void* ug, const void* z, void* dug, void* dx, float* dwug,
                         float* dwd, void* workspace, size_t workspace_bytes, void* stream) {
  RTE_REQUIRE(F % 32 == 0 && d % 8 == 0, "dense_swiglu: F %% 32 and d %% 8 must be 0");
  {
    // dZ = dout @ W_down^T: B(n=f, k=dcol) = wd[dcol][f] (layout T) or wd[f][dcol] (layout N)
    GemmArgs p;
    p.M = T;
    p.N = F;
    p.K = d;
    p.a = plain(dout, d);
    p.b = plain(wd, wd_rows ? d : F);
    p.b_t = wd_rows ? 0 : 1;
    p.epi.ug_in = B16(ug);
    p.epi.ug = B16(dug);
    p.epi.ld_ug = 2 * F;
    RTE_TRY(gemm_launch(p, EPI_SWIGLU_BWD, S(stream)));
  }
  {
    // dx = dUG @ W_ug   (B(n=dcol, k=c) = wug[ilv(c)][dcol] -> layout T)
    GemmArgs p;
    p.M = T;
    p.N = d;
    p.K = 2 * F;
    p.a = plain(dug, 2 * F);
    p.b = plain(wug, d);
    p.b.ilv = F;
    p.b_t = 1;
    p.epi.c = dx;
    p.epi.ldc = d;
    // few row tiles (short T): split the reduction in the workspace, as the weight gradients do
    RTE_TRY(gemm_launch(p, EPI_STORE, S(stream), workspace, workspace_bytes));
  }
  {
    // dW_ug[ilv(c), :] = sum_t dUG[t, c] x[t, :]
    GemmArgs p;
    p.M = 2 * F;
    p.N = d;
    p.K = T;
    p.a = plain(dug, 2 * F);
    p.a_t = 1;
    p.b = plain(x, d);
    p.b_t = 1;
    p.epi.c = dwug;
    p.epi.ldc = d;
    p.epi.c_f32 = 1;
    p.epi.c_ilv = F;
    RTE_TRY(gemm_launch(p, EPI_STORE, S(stream), workspace, workspace_bytes));
  }
  {
    GemmArgs p;
    p.K = T;
    p.a_t = 1;
    p.b_t = 1;
    p.epi.c = dwd;
    p.epi.c_f32 = 1;
    if (wd_rows) {
      // dW_rows[f, dcol] = sum_t z[t, f] dout[t, dcol]
      p.M = F;
      p.N = d;
      p.a = plain(z, F);
      p.b = plain(dout, d);
      p.epi.ldc = d;
    } else {
      // dW_d[dcol, f] = sum_t dout[t, dcol] z[t, f]
      p.M = d;
      p.N = F;
      p.a = plain(dout, d);
      p.b = plain(z, F);
      p.epi.ldc = F;
    }
    RTE_TRY(gemm_launch(p, EPI_STORE, S(stream), workspace, workspace_bytes));
  }
  return 0;
}

int rte_qkv_rope_fwd(const void* x, const void* wqkv, const float* cos_t, const float* sin_t, int B, int S_,
                     int H, int hd, void* q, void* k, void* v, void* workspace, size_t workspace_bytes,
                     void* stream) {
  const int d = H * hd;
  RTE_REQUIRE(d % 8 == 0 && hd % 8 == 0, "qkv_rope: head_dim must be a multiple of 8");
  RTE_REQUIRE(((uintptr_t)cos_t & 15) == 0 && ((uintptr_t)sin_t & 15) == 0,
              "qkv_rope: cos / sin tables must be 16-byte aligned");
  GemmArgs p;
  p.M = B * S_;
  p.N = 3 * d;
  p.K = d;
  p.a = plain(x, d);
  p.b = plain(wqkv, d);
  p.epi.q = B16(q);
  p.epi.k = B16(k);
  p.epi.v = B16(v);
  p.epi.cos_t = cos_t;
  p.epi.sin_t = sin_t;
  p.epi.S = S_;
  p.epi.H = H;
  p.epi.hd = hd;
  p.epi.dmodel = d;
  return gemm_launch(p, EPI_ROPE_QKV, S(stream), workspace, workspace_bytes);
}

int rte_qkv_rope_bwd(const void* dq, const int64_t* sq, const void* dk, const int64_t* sk, const void* dv,
                     const int64_t* sv, const void* x, const void* wqkv, const float* cos_t, const float* sin_t,
                     int B, int S_, int H, int hd, void* dqkv, void* dx, float* dw, void* workspace,
                     size_t workspace_bytes, void* stream) {
  const int d = H * hd;
  const int T = B * S_;
  if (dq)  // else dqkv already holds the packed, rotated-back gradient (rte_attention_bwd_qkv)
    RTE_TRY(rope_bwd_pack(B16(dq), sq, B16(dk), sk, B16(dv), sv, cos_t, sin_t, B, H, S_, hd, B16(dqkv),
                          S(stream)));
  {
    // dx = dqkv @ Wqkv   (B(n=dcol, k=c) = wqkv[c][dcol] -> layout T)
    GemmArgs p;
    p.M = T;
    p.N = d;
    p.K = 3 * d;
    p.a = plain(dqkv, 3 * d);
    p.b = plain(wqkv, d);
    p.b_t = 1;
    p.epi.c = dx;
    p.epi.ldc = d;
    // few row tiles (short T): split the reduction in the workspace, as dW does after it
    RTE_TRY(gemm_launch(p, EPI_STORE, S(stream), workspace, workspace_bytes));
  }
  if (dw) {
    // dW[c, :] = sum_t dqkv[t, c] x[t, :]
    GemmArgs p;
    p.M = 3 * d;
    p.N = d;
    p.K = T;
    p.a = plain(dqkv, 3 * d);
    p.a_t = 1;
    p.b = plain(x, d);
    p.b_t = 1;
    p.epi.c = dw;
    p.epi.ldc = d;
    p.epi.c_f32 = 1;
    RTE_TRY(gemm_launch(p, EPI_STORE, S(stream), workspace, workspace_bytes));
  }
  return 0;
}

// ------------------------------------------------------------------ SVD low-rank SwiGLU FFN
// Low-rank factors per projection: W_up = U_up diag(S_up) V_up^T (d x F), same for gate;
// W_down^T = U_dn diag(S_dn) V_dn^T.  With us_* = U * S folded by the caller:
//   a_ug = x @ [us_up | us_gate]            [T, 2r]
//   ug   = [a_up V_up^T | a_gate V_gate^T]  [T, 2F] (interleaved per 64), z = up * silu(gate)
//   b    = z @ V_dn                         [T, r]
//   y    = resid + b @ us_dn^T              [T, d]

int rte_svd_sparse_fwd(const void* x, int T, int d, int F, int r, const void* us_ug, const void* v_ug,
                       const void* w_up, const void* w_gate, const void* w_down, const float* wd_norm, int up_m,
                       int gate_m, int product_m, int top_k, int exact, int product_only, void* a_ug, void* ug,
                       void* z_hat, void* out, int out_f32, int32_t* sel_ids, float* sel_u, float* sel_g,
                       int32_t* n_cand, void* stream) {
  RTE_REQUIRE(r % 8 == 0 && F % 64 == 0 && d % 8 == 0, "svd_sparse: need r %% 8, F %% 64, d %% 8 == 0");
  if (T == 0) return 0;
  {
    GemmArgs p;  // selector codes a_ug = x @ [A_up | A_gate]
    p.M = T;
    p.N = 2 * r;
    p.K = d;
    p.a = plain(x, d);
    p.b = plain(us_ug, 2 * r);
    p.b_t = 1;
    p.epi.c = a_ug;
    p.epi.ldc = 2 * r;
    RTE_TRY(gemm_launch(p, EPI_STORE, S(stream)));
  }
  {
    GemmArgs p;  // approximate activations up_hat | gate_hat (interleaved) and z_hat
    p.M = T;
    p.N = 2 * F;
    p.K = r;
    p.a = plain(a_ug, 2 * r);
    p.a_koff2 = r;
    p.b = plain(v_ug, r);
    p.b.ilv = F;
    p.epi.ug = B16(ug);
    p.epi.ld_ug = 2 * F;
    p.epi.z = B16(z_hat);
    p.epi.ld_z = F;
    RTE_TRY(gemm_launch(p, EPI_SWIGLU_FWD, S(stream)));
  }
  return svd_sparse_select(B16(x), B16(ug), B16(w_up), B16(w_gate), B16(w_down), wd_norm, T, d, F, up_m, gate_m,
                           product_m, top_k, exact, product_only, out, out_f32, sel_ids, sel_u, sel_g, n_cand,
                           S(stream));
}

int rte_svd_sparse_bwd(const void* dout, int T, int d, int top_k, const void* w_up, const void* w_gate,
                       const void* w_down, const int32_t* sel_ids, const float* sel_u, const float* sel_g, void* dx,
                       float* z, float* du, float* dg, void* stream) {
  return svd_sparse_bwd(B16(dout), B16(w_up), B16(w_gate), B16(w_down), sel_ids, sel_u, sel_g, T, d, top_k, B16(dx),
                        z, du, dg, S(stream));
}

int rte_svd_ffn_fwd(const void* x, int T, int d, int F, int r, const void* us_ug, const void* v_ug,
                    const void* v_dn, const void* us_dn, const float* resid, void* a_ug, void* ug, void* z,
                    void* b, void* y, int y_f32, void* stream) {
  RTE_REQUIRE(r % 8 == 0 && F % 64 == 0 && d % 8 == 0, "svd_ffn: need r %% 8, F %% 64, d %% 8 == 0");
  {
    GemmArgs p;  // a_ug = x @ us_ug : B(n=j, k=dcol) = us_ug[dcol][j]
    p.M = T;
    p.N = 2 * r;
    p.K = d;
    p.a = plain(x, d);
    p.b = plain(us_ug, 2 * r);
    p.b_t = 1;
    p.epi.c = a_ug;
    p.epi.ldc = 2 * r;
    RTE_TRY(gemm_launch(p, EPI_STORE, S(stream)));
  }
  {
    GemmArgs p;  // expand + SwiGLU: up blocks read a_ug[:, 0:r], gate blocks a_ug[:, r:2r]
    p.M = T;
    p.N = 2 * F;
    p.K = r;
    p.a = plain(a_ug, 2 * r);
    p.a_koff2 = r;
    p.b = plain(v_ug, r);
    p.b.ilv = F;
    p.epi.ug = B16(ug);
    p.epi.ld_ug = 2 * F;
    p.epi.z = B16(z);
    p.epi.ld_z = F;
    RTE_TRY(gemm_launch(p, EPI_SWIGLU_FWD, S(stream)));
  }
  {
    GemmArgs p;  // b = z @ v_dn : B(n=j, k=f) = v_dn[f][j]
    p.M = T;
    p.N = r;
    p.K = F;
    p.a = plain(z, F);
    p.b = plain(v_dn, r);
    p.b_t = 1;
    p.epi.c = b;
    p.epi.ldc = r;
    RTE_TRY(gemm_launch(p, EPI_STORE, S(stream)));
  }
  {
    GemmArgs p;  // y = resid + b @ us_dn^T : B(n=dcol, k=j) = us_dn[dcol][j]
    p.M = T;
    p.N = d;
    p.K = r;
    p.a = plain(b, r);
    p.b = plain(us_dn, r);
    p.epi.c = y;
    p.epi.ldc = d;
    p.epi.c_f32 = y_f32;
    p.epi.resid = resid;
    p.epi.ld_resid = d;
    RTE_TRY(gemm_launch(p, EPI_STORE, S(stream)));
  }
  return 0;
}

int rte_svd_ffn_bwd(const void* dy, const void* x, int T, int d, int F, int r, const void* us_ug, const void* v_ug,
                    const void* v_dn, const void* us_dn, const void* a_ug, const void* ug, const void* z,
                    const void* b, void* db, void* dug, void* da_ug, void* dx, float* dus_ug, float* dv_ug,
                    float* dv_dn, float* dus_dn, void* workspace, size_t workspace_bytes, void* stream) {
  RTE_REQUIRE(r % 8 == 0 && F % 64 == 0 && d % 8 == 0, "svd_ffn: need r %% 8, F %% 64, d %% 8 == 0");
  hipStream_t st = S(stream);
  {
    GemmArgs p;  // db = dy @ us_dn : B(n=j, k=dcol) = us_dn[dcol][j]
    p.M = T;
    p.N = r;
    p.K = d;
    p.a = plain(dy, d);
    p.b = plain(us_dn, r);
    p.b_t = 1;
    p.epi.c = db;
    p.epi.ldc = r;
    RTE_TRY(gemm_launch(p, EPI_STORE, st));
  }
  {
    GemmArgs p;  // dus_dn[dcol, j] = sum_t dy[t, dcol] b[t, j]
    p.M = d;
    p.N = r;
    p.K = T;
    p.a = plain(dy, d);
    p.a_t = 1;
    p.b = plain(b, r);
    p.b_t = 1;
    p.epi.c = dus_dn;
    p.epi.ldc = r;
    p.epi.c_f32 = 1;
    RTE_TRY(gemm_launch(p, EPI_STORE, st, workspace, workspace_bytes));
  }
  {
    GemmArgs p;  // dZ = db @ v_dn^T with the SwiGLU backward epilogue -> dUG
    p.M = T;
    p.N = F;
    p.K = r;
    p.a = plain(db, r);
    p.b = plain(v_dn, r);
    p.epi.ug_in = B16(ug);
    p.epi.ug = B16(dug);
    p.epi.ld_ug = 2 * F;
    RTE_TRY(gemm_launch(p, EPI_SWIGLU_BWD, st));
  }
  {
    GemmArgs p;  // dv_dn[f, j] = sum_t z[t, f] db[t, j]
    p.M = F;
    p.N = r;
    p.K = T;
    p.a = plain(z, F);
    p.a_t = 1;
    p.b = plain(db, r);
    p.b_t = 1;
    p.epi.c = dv_dn;
    p.epi.ldc = r;
    p.epi.c_f32 = 1;
    RTE_TRY(gemm_launch(p, EPI_STORE, st, workspace, workspace_bytes));
  }
  for (int half = 0; half < 2; ++half) {
    // dUP / dGATE read from the interleaved dUG: column f -> (f/32)*64 + f%32 (+32 for gate)
    Operand dsel = plain(static_cast<const bf16*>(dug) + 32 * half, 2 * F);
    dsel.cdiv = 32;
    dsel.cs_hi = 64;
    {
      GemmArgs p;  // da_half = dHALF @ V_half : B(n=j, k=f) = v_ug[half*F + f][j]
      p.M = T;
      p.N = r;
      p.K = F;
      p.a = dsel;
      p.b = plain(static_cast<const bf16*>(v_ug) + (int64_t)half * F * r, r);
      p.b_t = 1;
      p.epi.c = static_cast<bf16*>(da_ug) + half * r;
      p.epi.ldc = 2 * r;
      RTE_TRY(gemm_launch(p, EPI_STORE, st));
    }
    {
      GemmArgs p;  // dv_half[f, j] = sum_t dHALF[t, f] a_half[t, j]
      p.M = F;
      p.N = r;
      p.K = T;
      p.a = dsel;
      p.a_t = 1;
      p.b = plain(static_cast<const bf16*>(a_ug) + half * r, 2 * r);
      p.b_t = 1;
      p.epi.c = dv_ug + (int64_t)half * F * r;
      p.epi.ldc = r;
      p.epi.c_f32 = 1;
      RTE_TRY(gemm_launch(p, EPI_STORE, st, workspace, workspace_bytes));
    }
  }
  {
    GemmArgs p;  // dx = da_ug @ us_ug^T : B(n=dcol, k=j) = us_ug[dcol][j]
    p.M = T;
    p.N = d;
    p.K = 2 * r;
    p.a = plain(da_ug, 2 * r);
    p.b = plain(us_ug, 2 * r);
    p.epi.c = dx;
    p.epi.ldc = d;
    RTE_TRY(gemm_launch(p, EPI_STORE, st));
  }
  {
    GemmArgs p;  // dus_ug[dcol, j] = sum_t x[t, dcol] da_ug[t, j]
    p.M = d;
    p.N = 2 * r;
    p.K = T;
    p.a = plain(x, d);
    p.a_t = 1;
    p.b = plain(da_ug, 2 * r);
    p.b_t = 1;
    p.epi.c = dus_ug;
    p.epi.ldc = 2 * r;
    p.epi.c_f32 = 1;
    RTE_TRY(gemm_launch(p, EPI_STORE, st, workspace, workspace_bytes));
  }
  return 0;
}

int rte_rmsnorm_fwd(const float* x, const float* w, int T, int d, float eps, void* out, float* rstd,
                    void* stream) {
  return rmsnorm_fwd(x, w, T, d, eps, B16(out), rstd, S(stream));
}

size_t rte_rmsnorm_bwd_workspace_bytes(int T, int d) { return rmsnorm_bwd_workspace_bytes(T, d); }

int rte_rmsnorm_bwd(const void* dy, const float* x, const float* w, const float* rstd, const float* dres, int T,
                    int d, float* dx, void* dx_bf16, float* dw, int dw_accumulate, void* workspace,
                    size_t workspace_bytes, void* stream) {
  return rmsnorm_bwd(B16(dy), x, w, rstd, dres, T, d, dx, B16(dx_bf16), dw, dw_accumulate, workspace,
                     workspace_bytes, S(stream));
}

int rte_ce_fwd(const float* logits, int64_t ld, int T, int V, const int64_t* targets, float* loss, float* lse,
               void* stream) {
  return ce_fwd(logits, ld, T, V, targets, loss, lse, S(stream));
}

int rte_ce_bwd(const float* logits, int64_t ld, int T, int V, const int64_t* targets, const float* lse,
               const float* dloss, const float* extra, void* dlogits, void* stream) {
  return ce_bwd(logits, ld, T, V, targets, lse, dloss, extra, nullptr, 0, 1, B16(dlogits), S(stream));
}

int rte_ce_bwd_rows(const float* logits, int64_t ld, int T, int V, const int64_t* targets, const float* lse,
                    const float* dloss, const float* extra_rows, const int64_t* sample_ids, int n_samples, int seq,
                    void* dlogits, void* stream) {
  RTE_REQUIRE(extra_rows && sample_ids && n_samples >= 1 && seq >= 1 && T % seq == 0,
              "ce_bwd_rows: need the rows, their sample ids, and T a multiple of the tokens per sample");
  return ce_bwd(logits, ld, T, V, targets, lse, dloss, extra_rows, sample_ids, n_samples, seq, B16(dlogits),
                S(stream));
}

int rte_axpy_norm_fwd(const float* a, const float* b, const float* c, const float* keep, const uint8_t* mask,
                      int seq, int T, int d, const float* w, const float* gamma, const float* beta, float eps,
                      float* x_out, void* n_out, float* rstd_out, void* stream) {
  return axpy_norm_fwd(a, b, c, keep, mask, seq, T, d, w, gamma, beta, eps, x_out, B16(n_out), rstd_out, S(stream));
}

size_t rte_axpy_norm_bwd_workspace_bytes(int T, int d) { return axpy_norm_bwd_workspace_bytes(T, d); }

int rte_axpy_norm_bwd(const void* dn, const float* dx_ext, const float* x, const float* rstd, const float* w,
                      const float* gamma, const float* b, const float* c, const uint8_t* mask, int seq, int T, int d,
                      float* da, float* db, float* dkeep, float* dparams, void* workspace, size_t workspace_bytes,
                      void* stream) {
  return axpy_norm_bwd(reinterpret_cast<const bf16*>(dn), dx_ext, x, rstd, w, gamma, b, c, mask, seq, T, d, da, db,
                       dkeep, dparams, workspace, workspace_bytes, S(stream));
}

size_t rte_macro_workspace_bytes(int B, int seq, int d) { return macro_workspace_bytes(B, seq, d); }

int rte_macro_prologue_fwd(const float* h, const float* h0, int B, int B_h0, int seq, int d, float eps, void* z,
                           float* rstd, void* workspace, size_t workspace_bytes, void* stream) {
  return macro_prologue_fwd(h, h0, B, B_h0, seq, d, eps, B16(z), rstd, workspace, workspace_bytes, S(stream));
}

int rte_macro_prologue_bwd(const void* dz, const float* h, const float* rstd, const float* dh_extra, int B, int B_h,
                           int seq, int d, float* dh, float* dh0, void* workspace, size_t workspace_bytes,
                           void* stream) {
  return macro_prologue_bwd(reinterpret_cast<const bf16*>(dz), h, rstd, dh_extra, B, B_h, seq, d, dh, dh0, workspace,
                            workspace_bytes, S(stream));
}

int rte_macro_epilogue_fwd(const float* h, const float* low, const int64_t* key, int B, int B_h, int seq, int d,
                           const float* gain, const float* bias, const float* scale, float c, float* out,
                           void* stream) {
  return macro_epilogue_fwd(h, low, key, B, B_h, seq, d, gain, bias, scale, c, out, S(stream));
}

int rte_macro_epilogue_bwd(const float* dout, const float* h, const float* low, const int64_t* key, int B, int B_h,
                           int seq, int d, const float* gain, const float* bias, const float* scale, float c,
                           float* dh, void* dlow, void* part, size_t part_bytes, void* stream) {
  return macro_epilogue_bwd(dout, h, low, key, B, B_h, seq, d, gain, bias, scale, c, dh, B16(dlow), part, part_bytes,
                            S(stream));
}

int rte_macro_table_grad(const int64_t* key, int B, int seq, int n_keys, int d, const void* part, float* dgain,
                         float* dbias, float* dscale, void* stream) {
  return macro_table_grad(key, B, seq, n_keys, d, part, dgain, dbias, dscale, S(stream));
}

int rte_macro_fused_tiles(int seq) { return seq >= 1 ? macro_fused_tiles(seq) : 0; }

size_t rte_macro_fused_fwd_workspace_bytes(int B_h, int seq, int d) {
  return macro_fused_fwd_workspace_bytes(B_h, seq, d);
}

size_t rte_macro_fused_wgrad_workspace_bytes(int B_total, int seq, int d, int n_keys) {
  return macro_fused_wgrad_workspace_bytes(B_total, seq, d, n_keys);
}

int rte_macro_fused_prep(const float* v, const float* u, int n_keys, int d, void* v_b, void* vc_t, void* v2_t,
                         void* u_b, void* u_t, void* stream) {
  return macro_fused_prep(v, u, n_keys, d, B16(v_b), B16(vc_t), B16(v2_t), B16(u_b), B16(u_t), S(stream));
}

size_t rte_macro_fused_bwd_workspace_bytes(int B, int seq) { return macro_fused_bwd_workspace_bytes(B, seq); }

int rte_macro_fused_fwd(const float* h, const float* h0, int B_h, int B_h0, const int64_t* key, int B, int seq, int d,
                        int n_keys, float eps, const void* v_b, const void* vc_t, const void* u_t, const float* gain,
                        const float* bias, const float* scale, float c, void* x2, float* rstd, void* pooled, float* p,
                        float* a, void* sa, float* out, const float* mse_ref, float* mse_part, void* workspace,
                        size_t workspace_bytes, void* stream) {
  return macro_fused_fwd(h, h0, B_h, B_h0, key, B, seq, d, n_keys, eps, reinterpret_cast<const bf16*>(v_b),
                         reinterpret_cast<const bf16*>(vc_t), reinterpret_cast<const bf16*>(u_t), gain, bias, scale, c,
                         B16(x2), rstd, B16(pooled), p, a, B16(sa), out, mse_ref, mse_part, workspace, workspace_bytes,
                         S(stream));
}

int rte_macro_fused_sum(const float* part, int n, float inv_n, float* out, void* stream) {
  return macro_fused_sum(part, n, inv_n, out, S(stream));
}

int rte_macro_fused_bwd(const float* dout_p, const float* dout_q, const float* g, float mul, int diff_lo,
                        int n_diff, const float* dout, int dout_lo, int n_dout, const float* h, const float* rstd, const void* x2, int B_h,
                        const int64_t* key, int B, int seq, int d, int n_keys, const float* a, const void* sa,
                        const void* v_b, const void* vc_t, const void* v2_t, const void* u_b, const void* u_t,
                        const float* gain, const float* bias, const float* scale, float c, void* du, void* da,
                        float* part_tab, float* part_da, float* dh, float* dh0, int dh0_into_dh, const float* extra,
                        int n_extra, void* da_sum, void* workspace, size_t workspace_bytes, void* stream) {
  auto cb = [](const void* p) { return reinterpret_cast<const bf16*>(p); };
  return macro_fused_bwd(dout_p, dout_q, g, mul, diff_lo, n_diff, dout, dout_lo, n_dout, h, rstd, cb(x2), B_h, key, B, seq, d, n_keys, a, cb(sa),
                         cb(v_b), cb(vc_t), cb(v2_t), cb(u_b), cb(u_t), gain, bias, scale, c, B16(du), B16(da), part_tab,
                         part_da, dh, dh0, dh0_into_dh, extra, n_extra, B16(da_sum), workspace, workspace_bytes,
                         S(stream));
}

int rte_macro_fused_wgrad(const int64_t* key, int B0, int B_h0, int B1, int B_h1, int seq, int d, int n_keys,
                          const void* x2, const void* sa, const void* du, const void* da, const void* pooled,
                          const void* da_sum, const float* part_tab, float* du_w, float* dv_w, float* dgain,
                          float* dbias, float* dscale, void* workspace, size_t workspace_bytes, void* stream) {
  auto cb = [](const void* p) { return reinterpret_cast<const bf16*>(p); };
  return macro_fused_wgrad(key, B0, B_h0, B1, B_h1, seq, d, n_keys, cb(x2), cb(sa), cb(du), cb(da), cb(pooled),
                           cb(da_sum), part_tab, du_w, dv_w, dgain, dbias, dscale, workspace, workspace_bytes,
                           S(stream));
}

int rte_attention_fwd(const void* q, const void* k, const void* v, int B, int H, int seq, int head_dim, float scale,
                      const float* head_scale, void* out, float* lse, void* stream) {
  return attention_fwd(reinterpret_cast<const bf16*>(q), reinterpret_cast<const bf16*>(k),
                       reinterpret_cast<const bf16*>(v), B, H, seq, head_dim, scale, head_scale, B16(out), lse,
                       S(stream));
}

int rte_attention_bwd(const void* q, const void* k, const void* v, const void* out, const void* dout,
                      const float* lse, int B, int H, int seq, int head_dim, float scale, const float* head_scale,
                      void* dq, void* dk, void* dv, void* stream) {
  return attention_bwd(reinterpret_cast<const bf16*>(q), reinterpret_cast<const bf16*>(k),
                       reinterpret_cast<const bf16*>(v), reinterpret_cast<const bf16*>(out),
                       reinterpret_cast<const bf16*>(dout), lse, B, H, seq, head_dim, scale, head_scale, B16(dq),
                       B16(dk), B16(dv), S(stream));
}

int rte_attention_bwd_qkv(const void* q, const void* k, const void* v, const void* out, const void* dout,
                          const float* lse, int B, int H, int seq, int head_dim, float scale, const float* head_scale,
                          const float* cos_t, const float* sin_t, void* dqkv, void* stream) {
  RTE_REQUIRE(cos_t && sin_t && dqkv, "attention_bwd_qkv: cos, sin and dqkv are required");
  return attention_bwd_qkv(reinterpret_cast<const bf16*>(q), reinterpret_cast<const bf16*>(k),
                           reinterpret_cast<const bf16*>(v), reinterpret_cast<const bf16*>(out),
                           reinterpret_cast<const bf16*>(dout), lse, B, H, seq, head_dim, scale, head_scale, cos_t,
                           sin_t, B16(dqkv), S(stream));
}

size_t rte_mse_workspace_bytes(int64_t n) { return mse_workspace_bytes(n); }

int rte_mse_fwd(const float* a, const float* b, int64_t n, float* out, void* workspace, size_t workspace_bytes,
                void* stream) {
  return mse_fwd(a, b, n, out, workspace, workspace_bytes, S(stream));
}

int rte_mse_bwd(const float* a, const float* b, int64_t n, const float* dout, float* da, float* db, void* stream) {
  return mse_bwd(a, b, n, dout, da, db, S(stream));
}

size_t rte_pack_routes_workspace_bytes(int B, int kmax) { return pack_routes_workspace_bytes(B, kmax); }

int rte_pack_routes(const int64_t* recipe_ids, const uint8_t* active, int B, int seq, const int32_t* routes,
                    int n_recipes, int kmax,
                    const float* route_w, int C, int32_t* offsets, int32_t* tok_of_slot, int32_t* pair_of_slot,
                    int32_t* slot_of_pair, float* w_of_slot, void* workspace, size_t workspace_bytes, void* stream) {
  return pack_routes(recipe_ids, active, B, seq, routes, n_recipes, kmax, route_w, C, offsets, tok_of_slot, pair_of_slot,
                     slot_of_pair, w_of_slot, workspace, workspace_bytes, S(stream));
}

int rte_adamw_chunk(void) { return adamw_chunk(); }

size_t rte_adamw_workspace_bytes(int n_tensors, int n_blocks, int n_groups) {
  return adamw_workspace_bytes(n_tensors, n_blocks, n_groups);
}

int rte_adamw_step(const void* rows, int n_tensors, const int32_t* blocks, const int32_t* first_block, int n_blocks,
                   const double* hyper, int n_groups, const int32_t* metric_lr_group, int n_metrics, float clip_max,
                   const float* found_inf, float* metrics, void* workspace, size_t workspace_bytes, void* stream) {
  return adamw_step(rows, n_tensors, blocks, first_block, n_blocks, hyper, n_groups, metric_lr_group, n_metrics,
                    clip_max, found_inf, metrics, workspace, workspace_bytes, S(stream));
}

size_t rte_distill_workspace_bytes(int A, int rows) { return distill_workspace_bytes(A, rows); }

int rte_distill_fwd(const float* hot, const float* exact, const float* h0, int A, int seq, int d,
                    const float* hot_logits, const float* exact_logits, int V, float temperature, float eps,
                    const float* weights, float* losses, float* metrics, void* workspace, size_t workspace_bytes,
                    void* stream) {
  return distill_fwd(hot, exact, h0, A, seq, d, hot_logits, exact_logits, V, temperature, eps, weights, losses,
                     metrics, workspace, workspace_bytes, S(stream));
}

int rte_distill_bwd(const float* hot, const float* exact, const float* h0, int A, int seq, int d,
                    const float* hot_logits, const float* exact_logits, int V, float temperature, float eps,
                    const float* weights, const float* dlosses, const void* workspace, size_t workspace_bytes,
                    float* dhot, float* dhot_logits, void* stream) {
  return distill_bwd(hot, exact, h0, A, seq, d, hot_logits, exact_logits, V, temperature, eps, weights, dlosses,
                     workspace, workspace_bytes, dhot, dhot_logits, S(stream));
}

int rte_audit_correct_fwd(const float* hot_tok, const float* exact_tok, int B, int seq, const int64_t* idx, int A,
                          const float* p, float clip, int grad_corrected, float* corrected, float* exact_ps,
                          float* coef, float* stats, void* stream) {
  return audit_fwd(hot_tok, exact_tok, B, seq, idx, A, p, clip, grad_corrected, corrected, exact_ps, coef, stats,
                   S(stream));
}

int rte_audit_correct_bwd(const float* g, int B, int seq, const int64_t* idx, int A, const float* coef,
                          float* dhot_tok, float* dexact_tok, void* stream) {
  return audit_bwd(g, B, seq, idx, A, coef, dhot_tok, dexact_tok, S(stream));
}

int rte_cast_f32_bf16(const float* x, int64_t n, void* y, void* stream) {
  return cast_f32_bf16(x, n, B16(y), S(stream));
}

int rte_cast_many_blocks(int kind, int64_t rows, int64_t cols) {
  if (kind != 0 && kind != 1) return -1;
  return cast_many_blocks(kind, rows, cols);
}

int rte_cast_many(const int64_t* jobs, const int32_t* blk, int nblk, void* stream) {
  RTE_REQUIRE(nblk >= 0 && (nblk == 0 || (jobs && blk)), "cast_many: bad tables");
  return cast_many(jobs, blk, nblk, S(stream));
}

int rte_shortlist_build(const int64_t* targets, const int32_t* top_clusters, int tc, const int64_t* members,
                        int n_clusters, int per_cluster, const int64_t* random_negs, int R, int H, int L, int V,
                        int T, int32_t* shortlist, int32_t* dup_per_token, void* stream) {
  return shortlist_build(targets, top_clusters, tc, members, n_clusters, per_cluster, random_negs, R, H, L, V, T,
                         shortlist, dup_per_token, S(stream));
}

int rte_shortlist_fwd(const void* hidden, const void* W, int d, int V, const int32_t* shortlist, int L, int T,
                      float* logits, float* lse, float* loss, void* stream) {
  return shortlist_fwd(B16(hidden), B16(W), d, V, shortlist, L, T, logits, lse, loss, S(stream));
}

size_t rte_shortlist_bwd_workspace_bytes(int T, int L, int V, int d) {
  return shortlist_bwd_workspace_bytes(T, L, V, d);
}

int rte_shortlist_bwd(const float* dloss, const float* dlogits, const void* hidden, const void* W, int d, int V,
                      const int32_t* shortlist, int L, int T, const float* logits, const float* lse,
                      void* dhidden, float* dW, int dW_accumulate, void* workspace, size_t workspace_bytes,
                      void* stream) {
  return shortlist_bwd(dloss, dlogits, B16(hidden), B16(W), d, V, shortlist, L, T, logits, lse,
                       static_cast<bf16*>(dhidden), dW, dW_accumulate, workspace, workspace_bytes, S(stream));
}

size_t rte_segment_reduce_workspace_bytes(int64_t P, int V, int d) { return segreduce_workspace_bytes(P, V, d); }

int rte_segment_reduce_rows(const int32_t* keys, int64_t P, int V, int row_div, const float* w, const void* rows,
                            int rows_f32, int d, float* out, int accumulate, void* workspace, size_t workspace_bytes,
                            void* stream) {
  return segreduce_rows(keys, P, V, row_div, w, rows, rows_f32, d, out, accumulate, workspace, workspace_bytes,
                        S(stream));
}

int rte_grouped_linear_fwd(const void* x, int N, int K, const int32_t* offsets, int G, int P,
                           const int32_t* row_of_slot, const int32_t* out_row_of_slot, const void* w, int Nout,
                           void* y, int y_f32, void* stream) {
  RTE_REQUIRE(K % 8 == 0 && Nout % 8 == 0, "grouped_linear: K and Nout must be multiples of 8");
  RTE_REQUIRE(N >= 0 && P >= 0 && G >= 1, "grouped_linear: bad sizes");
  if (P == 0) return 0;
  // y[out_row(slot)] = x[row(slot)] @ W_g   with W_g [K, Nout] row-major (layout T for B)
  GemmArgs p;
  p.mode = MODE_GROUP_M;
  p.goff = offsets;
  p.G = G;
  p.max_tiles_m = P / kGroupTileM + G + 1;
  p.M = P;
  p.N = Nout;
  p.K = K;
  p.a = plain(x, K);
  p.a.rows = row_of_slot;
  p.b = plain(w, Nout);
  p.b.gstride = (int64_t)K * Nout;
  p.b_t = 1;
  p.epi.c = y;
  p.epi.ldc = Nout;
  p.epi.c_rows = out_row_of_slot;
  p.epi.c_f32 = y_f32;
  (void)N;
  return gemm_launch(p, EPI_STORE, S(stream));
}

int rte_grouped_linear_bwd(const void* dy, const void* x, int N, int K, const int32_t* offsets, int G, int P,
                           const int32_t* row_of_slot, const int32_t* out_row_of_slot, const void* w, int Nout,
                           void* dx, int dx_f32, float* dw, void* workspace, size_t workspace_bytes,
                           void* stream) {
  RTE_REQUIRE(K % 8 == 0 && Nout % 8 == 0, "grouped_linear: K and Nout must be multiples of 8");
  RTE_REQUIRE(N >= 0 && P >= 0 && G >= 1, "grouped_linear: bad sizes");
  if (dx && P > 0) {
    // dx[row(slot)] = dy[out_row(slot)] @ W_g^T   (B(n=kk, k=j) = W_g[kk, j]: layout N)
    GemmArgs p;
    p.mode = MODE_GROUP_M;
    p.goff = offsets;
    p.G = G;
    p.max_tiles_m = P / kGroupTileM + G + 1;
    p.M = P;
    p.N = K;
    p.K = Nout;
    p.a = plain(dy, Nout);
    p.a.rows = out_row_of_slot;
    p.b = plain(w, Nout);
    p.b.gstride = (int64_t)K * Nout;
    p.epi.c = dx;
    p.epi.ldc = K;
    p.epi.c_rows = row_of_slot;
    p.epi.c_f32 = dx_f32;
    RTE_TRY(gemm_launch(p, EPI_STORE, S(stream)));
  }
  if (dw) {
    // dW_g[kk, j] = sum over the group's slots of x[row(slot), kk] dy[out_row(slot), j]
    GemmArgs p;
    p.mode = MODE_GROUP_K;
    p.goff = offsets;
    p.G = G;
    p.M = K;
    p.N = Nout;
    p.K = P;
    p.a = plain(x, K);
    p.a.rows = row_of_slot;
    p.a_t = 1;
    p.b = plain(dy, Nout);
    p.b.rows = out_row_of_slot;
    p.b_t = 1;
    p.epi.c = dw;
    p.epi.ldc = Nout;
    p.epi.c_f32 = 1;
    p.epi.c_gstride = (int64_t)K * Nout;
    RTE_TRY(gemm_launch(p, EPI_STORE, S(stream), workspace, workspace_bytes));
  }
  (void)N;
  return 0;
}

size_t rte_grouped_linear_bwd_workspace_bytes(int P, int G, int K, int Nout) {
  return gemm_groupk_bytes(K, Nout, P, G);
}

}  // extern "C"
