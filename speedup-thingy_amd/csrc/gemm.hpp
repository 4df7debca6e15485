// Generic bf16 MFMA GEMM for gfx950:  C[m, n] = sum_k A(m, k) * B(n, k)
//
// Each operand is described by how it sits in memory, so one kernel covers the
// forward (x W^T), input-gradient (dY W) and weight-gradient (dY^T X) products
// with no explicit transposes:
//   layout N : the reduction index k is contiguous     elem(i, k) = row(i) + col(k)
//   layout T : the output index i (m or n) is contiguous elem(i, k) = row(k) + col(i)
// "row(r)" applies, in order: a per-group row shift, the optional SwiGLU
// interleave (see Operand::ilv), an optional int32 row indirection (gather), and
// an optional two-level split (r / rdiv, r % rdiv) so [B,H,S,hd]-strided
// attention tensors can be read as [B*S, H*hd] matrices.  "col(c)" optionally
// splits c the same way with a second stride.  Split sizes are powers of two.
//
// Grouping (cluster pools): mode GROUP_M gives each group its own contiguous
// range of m (slots of one cluster) with an in-kernel tile map; mode GROUP_K
// gives each group its own range of k (the per-cluster weight-gradient reduction).
// Dense problems with few output tiles and a long reduction are split along k
// into fp32 partials that a second kernel sums in a fixed order (deterministic).
#pragma once

#include "common.hpp"

namespace rte {

struct Operand {
  const bf16* ptr = nullptr;
  const int32_t* rows = nullptr;  // optional indirection of memory rows
  int64_t ld = 0;                 // elements between memory rows
  int64_t gstride = 0;            // element offset per group
  int64_t growstride = 0;         // row-index offset per group (before indirection)
  int32_t ilv = 0;                // >0: SwiGLU interleave, row r -> (r%64<32 ? 0 : ilv) + (r/64)*32 + r%32
  int32_t rdiv = 0;               // 0: plain rows, else (power of 2) row r -> (r/rdiv)*rs_hi + (r%rdiv)*ld
  int64_t rs_hi = 0;
  int32_t cdiv = 0;               // 0: plain cols, else (power of 2) col c -> (c/cdiv)*cs_hi + c%cdiv
  int64_t cs_hi = 0;
};

enum EpiKind : int {
  EPI_STORE = 0,        // C = alpha*acc*row_scale + beta*C + resid   (bf16 or fp32)
  EPI_SWIGLU_FWD = 1,   // columns interleaved per 64: [32 up | 32 gate]; writes UG and Z
  EPI_SWIGLU_BWD = 2,   // acc = dZ; reads UG; writes dUG (+ optional per-row <z, acc>)
  EPI_ROPE_QKV = 3,     // columns [q | k | v]; interleaved RoPE on q,k; writes [B,H,S,hd]
};

enum GemmMode : int { MODE_DENSE = 0, MODE_GROUP_M = 1, MODE_GROUP_K = 2 };

struct Epilogue {
  void* c = nullptr;
  int64_t ldc = 0;
  int64_t c_gstride = 0;
  int64_t c_growstride = 0;
  const int32_t* c_rows = nullptr;
  int32_t c_ilv = 0;                 // SwiGLU interleave of output rows (see Operand::ilv)
  int32_t c_col_ilv = 0;             // SwiGLU interleave of output columns g * c_gstride + n (then
                                     // c_gstride is a column offset per group, a multiple of 32)
  int c_f32 = 0;
  float alpha = 1.0f;
  float beta = 0.0f;
  const float* row_scale = nullptr;  // indexed by m (slot space)
  const float* resid = nullptr;      // fp32, indexed like C
  int64_t ld_resid = 0;
  // SwiGLU
  bf16* ug = nullptr;                // fwd output (UG) / bwd output (dUG); same interleaved layout
  const bf16* ug_in = nullptr;       // bwd input (UG)
  int64_t ld_ug = 0;
  bf16* z = nullptr;                 // fwd: Z[m, neuron]
  int64_t ld_z = 0;
  float* dw_row = nullptr;           // bwd: per-row <z, dZ>
  // RoPE + head split
  bf16* q = nullptr;
  bf16* k = nullptr;
  bf16* v = nullptr;
  const float* cos_t = nullptr;      // [S, hd]
  const float* sin_t = nullptr;
  int S = 0, H = 0, hd = 0, dmodel = 0;
};

struct GemmArgs {
  Operand a, b;
  int a_t = 0, b_t = 0;   // layout T flags
  int M = 0, N = 0, K = 0;
  int mode = MODE_DENSE;
  const int32_t* goff = nullptr;   // [G+1] group offsets along m (GROUP_M) or k (GROUP_K)
  int G = 1;
  int max_tiles_m = 0;             // GROUP_M: grid bound on m-tiles, >= sum_g ceil(cnt_g / 128)
  // split-K (dense EPI_STORE only): fp32 partials [splits, M, N] in `splitk_ws`
  int splits = 1;
  int k_chunk = 0;
  float* splitk_ws = nullptr;
  int splits_forced = 0;           // set: the launch must split (the reduce stores the output)
  // EPI_SWIGLU_FWD only: gate columns read A at k + a_koff2 (two low-rank codes side by
  // side in one A row, e.g. [x U_up | x U_gate]); 0 = both halves read the same A columns.
  int a_koff2 = 0;
  // GROUP_K with chunked groups (set by gemm_launch when a workspace is given): group g's k
  // range is cut into chunks of gk_chunk; work item i (grid z) is chunk i - gk_first[g] of the
  // group g with gk_first[g] <= i < gk_first[g + 1] (an empty group has one, with an empty
  // k range).  A group of one chunk stores directly; larger groups store fp32 partials
  // [item, M, N] that a second kernel adds in chunk order.
  int gk_chunk = 0;
  const int32_t* gk_first = nullptr;  // [G + 1]
  float* gk_part = nullptr;
  Epilogue epi;
};

// Picks a tile configuration for the problem and launches it on `stream`.
// `ws`/`ws_bytes` (optional) enable split-K for dense problems with few tiles.
// Returns 0 or -1 with rte_last_error() set.
int gemm_launch(const GemmArgs& args, int epi_kind, hipStream_t stream, void* ws = nullptr,
                size_t ws_bytes = 0);

// Workspace that lets gemm_launch split a dense problem of this shape along k.
size_t gemm_splitk_bytes(int M, int N, int K);

// Workspace that lets gemm_launch cut the groups of a GROUP_K problem (K = total rows of all
// groups) into chunks, so one large group is reduced by many workgroups (deterministic).
size_t gemm_groupk_bytes(int M, int N, int K, int G);

// Every GROUP_M configuration uses this tile height.
constexpr int kGroupTileM = 128;

}  // namespace rte
