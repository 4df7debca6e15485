// Exact recursive passes of the banked core for the few samples of the audit replay
// (BankedRecursiveCore.forward_step, rte/layers.py:806-870, driven pass by pass by
// forward_exact, rte/models.py:416-512; the audit replays the chosen rows, rte/audit.py:245-387),
// forward and backward, one bank of attention heads and one bank of FFN slabs:
//
//   h~ = h + alpha h0                      n1 = rmsnorm(h~) w1 (1 + g1) + b1
//   q, k, v = rope(n1 Wqkv) on the recipe's heads      y = causal attention (q, k, v)
//   attn = y Wo (recipe heads' rows)        u = h~ + s_attn attn
//   n2 = rmsnorm(u) w2 (1 + g2) + b2        z = up silu(gate), [up | gate] = n2 Wug (recipe slabs)
//   mlp = z Wd (recipe slabs' rows)         h' = active ? u + s_mlp mlp : h
//
// The replay runs a handful of samples (64 rows each at the bench shape).  There every launch is
// bound by memory latency, not work: a dependent global access costs about as much as the whole
// tile's arithmetic.  So every kernel owns a 64-row tile of one sample and a 64-column output
// tile, issues all the loads that do not depend on the recipe together with the sample's recipe
// record (one round trip), then the recipe-dependent weight panel (a second round trip, overlapped
// with the row arithmetic), and runs its MFMAs from LDS.  Only the recipe's heads (64 columns
// each) and 32-neuron slab blocks take part.  The record of each (pass, sample), gathered once per
// replay, is int32 [W], W = 4 + 2 H + 2 NB:
//   act | nh | nb | 0 | heads[H] (ascending) | ihead[H] (slot or -1) | blks[NB] | iblk[NB]
//
//   forward per pass : qkv (norm1 + QKV + RoPE, compact heads) -> attention (attention.hip) ->
//                      oproj (O-projection + residual) -> upgate (norm2 + up/gate + SwiGLU) ->
//                      down (down-projection + residual)
//   backward per pass: down_bwd (dz + SwiGLU backward) -> upgate_bwd (dn2) -> oproj_bwd (norm2
//                      backward, residual, dy) -> attention backward (dqkv, RoPE undone) ->
//                      qkv_bwd (dn1) -> norm_bwd (norm1 backward, residual, dh, dh0 and every
//                      FiLM / scale / skip partial)
//
// Weight gradients are not formed here: the kernels write each pass's product operands at full
// width (zeros outside the recipe's heads / slabs), so one plain GEMM per weight over all passes'
// rows forms them afterwards.  FiLM, scale and skip gradients leave as per-(tile, column)
// partials, summed by param_reduce in a fixed order.  No atomics: results repeat bitwise.
//
// MFMA lane layout (32x32x16 bf16): lane l supplies A row l % 32 and B column l % 32 with k values
// 8 (l / 32) .. +7 of each 16-step; output register r of lane l holds row 8 (r / 4) + 4 (l / 32)
// + r % 4, column l % 32.  Eight waves (512 threads) per workgroup: waves w and w + 4 take the two
// halves of K on quadrant w % 4 of the 64 x 64 tile.  Row work maps thread t to row t / 8 and the
// 64-column segment t % 8 of that row.
#include "common.hpp"

namespace rte {

namespace {

constexpr int kThreads = 512;             // 8 waves: 8 threads per row of a 64-row tile
constexpr int kRows = 64;                 // rows (tokens of one sample) per workgroup
constexpr int kCols = 64;                 // output columns per workgroup
constexpr int kKC = 512;                  // K per staged panel
constexpr int kLda = kKC + 8;             // panel pitch in bf16 (16 bytes of padding per row)
constexpr int kPanel = kRows * kLda;      // bf16 elements per panel
constexpr int kCp = kCols + 4;            // epilogue staging pitch (fp32)
constexpr int kMaxD = 512;
constexpr int kSeg = 64;                  // columns of a row per thread (d <= 8 kSeg)
constexpr int kHd = 64;                   // head width
constexpr int kBlk = 32;                  // neurons per slab block
constexpr int kInfoMax = 1024;            // record words
constexpr int kUnits = kRows * (kKC / 8) / kThreads;  // 16-byte panel units per thread
constexpr size_t kPanelBytes = (size_t)kPanel * sizeof(bf16);
constexpr size_t kVecOff = 2 * kPanelBytes;                       // 4 d floats of norm vectors
constexpr size_t kRedOff = kVecOff + 4 * kMaxD * sizeof(float);   // 64 floats
constexpr size_t kInfoOff = kRedOff + 64 * sizeof(float);         // the record
constexpr size_t kLds = kInfoOff + kInfoMax * sizeof(int);

struct Meta {
  int B, S, d, F, rts;  // rts: 64-row tiles per sample
  int H, NB, Hmax, NBmax, W;
};

struct Info {
  const int* p;
  int H, NB;
  __device__ int act() const { return p[0]; }
  __device__ int nh() const { return p[1]; }
  __device__ int nb() const { return p[2]; }
  __device__ int head(int i) const { return p[4 + i]; }
  __device__ int ihead(int h) const { return p[4 + H + h]; }
  __device__ int blk(int i) const { return p[4 + 2 * H + i]; }
  __device__ int iblk(int k) const { return p[4 + 2 * H + NB + k]; }
};

struct Tile {
  int b, s0, nrows;  // sample, first position, valid rows (<= 64)
  int64_t row0;      // global row of tile row 0 (b * S + s0)
};

__device__ __forceinline__ Tile tile_of(const Meta& M) {
  Tile t;
  const int y = blockIdx.y;
  t.b = y / M.rts;
  t.s0 = (y - t.b * M.rts) * kRows;
  t.nrows = M.S - t.s0 < kRows ? M.S - t.s0 : kRows;
  t.row0 = (int64_t)t.b * M.S + t.s0;
  return t;
}

// Row work: thread -> (row, segment of kSeg columns)
struct RowPos {
  int row, seg, cb;
  bool ok;        // row inside the sample and segment inside d
  int64_t base;   // offset of the segment in a [M, d] matrix
};

__device__ __forceinline__ RowPos row_pos(const Tile& T, int d) {
  RowPos p;
  p.row = threadIdx.x >> 3;
  p.seg = threadIdx.x & 7;
  p.cb = p.seg * kSeg;
  p.ok = p.row < T.nrows && p.cb < d;
  p.base = (T.row0 + p.row) * d + p.cb;
  return p;
}

struct Smem {
  bf16* A;
  bf16* B;
  float* vec;
  float* red;
  int* inf;
};

__device__ __forceinline__ Smem smem_of(char* s) {
  return Smem{reinterpret_cast<bf16*>(s), reinterpret_cast<bf16*>(s + kPanelBytes),
              reinterpret_cast<float*>(s + kVecOff), reinterpret_cast<float*>(s + kRedOff),
              reinterpret_cast<int*>(s + kInfoOff)};
}

// The sample's record: loaded with the other independent loads, stored to LDS afterwards (the
// caller synchronises before reading it).
struct InfoLoad {
  int v[kInfoMax / kThreads];
  __device__ __forceinline__ void issue(const int32_t* info, const Meta& M, int b) {
#pragma unroll
    for (int k = 0; k < kInfoMax / kThreads; ++k) {
      const int i = threadIdx.x + kThreads * k;
      v[k] = i < M.W ? info[(int64_t)b * M.W + i] : 0;
    }
  }
  __device__ __forceinline__ void commit(int* dst, const Meta& M) const {
#pragma unroll
    for (int k = 0; k < kInfoMax / kThreads; ++k) {
      const int i = threadIdx.x + kThreads * k;
      if (i < M.W) dst[i] = v[k];
    }
  }
};

// Norm vectors into LDS: vec[j d + c] = p_j[c] for up to four vectors (null: zeros)
struct VecLoad {
  float v[4];
  int n;
  __device__ __forceinline__ void issue(const float* p0, const float* p1, const float* p2, const float* p3, int nv,
                                        int d) {
    n = nv * d;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int i = threadIdx.x + kThreads * k;
      const int j = i / d, c = i - j * d;
      const float* p = j == 0 ? p0 : (j == 1 ? p1 : (j == 2 ? p2 : p3));
      v[k] = (i < n && p) ? p[c] : 0.0f;
    }
  }
  __device__ __forceinline__ void commit(float* dst) const {
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int i = threadIdx.x + kThreads * k;
      if (i < n) dst[i] = v[k];
    }
  }
};

__device__ __forceinline__ f32x16_v zero16() {
  f32x16_v z;
#pragma unroll
  for (int i = 0; i < 16; ++i) z[i] = 0.0f;
  return z;
}

__device__ __forceinline__ float wsum(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

// Sum of v over the row's 8 segment threads (adjacent lanes)
__device__ __forceinline__ float row_sum(float v) {
  v += __shfl_xor(v, 1, 64);
  v += __shfl_xor(v, 2, 64);
  v += __shfl_xor(v, 4, 64);
  return v;
}

// Sum of v over the workgroup (red: 8 floats of LDS); every thread gets it, in a fixed order.
__device__ __forceinline__ float block_sum(float v, float* red) {
  v = wsum(v);
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  return ((red[0] + red[1]) + (red[2] + red[3])) + ((red[4] + red[5]) + (red[6] + red[7]));
}

__device__ __forceinline__ void to_f8(uint4 u, float* v) {
  const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    v[2 * i] = __uint_as_float(w[i] << 16);
    v[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
  }
}

__device__ __forceinline__ uint4 from_f8(const float* v) {
  uint4 o;
  o.x = pack_bf2(v[0], v[1]);
  o.y = pack_bf2(v[2], v[3]);
  o.z = pack_bf2(v[4], v[5]);
  o.w = pack_bf2(v[6], v[7]);
  return o;
}

__device__ __forceinline__ void ld4f(const float* p, float* v) {
  const float4 a = *reinterpret_cast<const float4*>(p);
  v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
}

__device__ __forceinline__ void st4f(float* p, const float* v) {
  *reinterpret_cast<float4*>(p) = make_float4(v[0], v[1], v[2], v[3]);
}

// N consecutive floats (N % 4 == 0) of p into v, zeros when !ok
template <int N>
__device__ __forceinline__ void ldn(const float* p, bool ok, float* v) {
#pragma unroll
  for (int j = 0; j < N; j += 4) {
    if (ok) {
      ld4f(p + j, v + j);
    } else {
      v[j] = v[j + 1] = v[j + 2] = v[j + 3] = 0.0f;
    }
  }
}

// N consecutive floats of an LDS vector (16-byte aligned)
template <int N>
__device__ __forceinline__ void lds_n(const float* p, float* v) {
#pragma unroll
  for (int j = 0; j < N; j += 4) {
    const float4 a = *reinterpret_cast<const float4*>(p + j);
    v[j] = a.x; v[j + 1] = a.y; v[j + 2] = a.z; v[j + 3] = a.w;
  }
}

// A [64 x kn] bf16 panel of K columns [k0, k0 + kn) (kn <= kKC, kn % 8 == 0): element (r, k) from
// src(r, k) (a pointer to 8 consecutive bf16, nullptr for zeros).  issue() puts every load in
// flight, commit() writes the panel.
struct PanelLoad {
  uint4 v[kUnits];
  int off[kUnits];
  template <class Src>
  __device__ __forceinline__ void issue(int k0, int kn, const Src& src) {
    const int tid = threadIdx.x;
    const int cpr = kn >> 3;
    // unit u = tid + kThreads i sits at row u / cpr, chunk u % cpr: step by kThreads = dq cpr + dr
    const int dq = kThreads / cpr, dr = kThreads - dq * cpr;
    int r = tid / cpr, c = tid - (tid / cpr) * cpr;
#pragma unroll
    for (int i = 0; i < kUnits; ++i) {
      v[i] = make_uint4(0u, 0u, 0u, 0u);
      off[i] = -1;
      if (r < kRows) {
        const bf16* p = src(r, k0 + c * 8);
        if (p) v[i] = *reinterpret_cast<const uint4*>(p);
        off[i] = r * kLda + c * 8;
      }
      r += dq;
      c += dr;
      if (c >= cpr) {
        c -= cpr;
        ++r;
      }
    }
  }
  __device__ __forceinline__ void commit(bf16* P) const {
#pragma unroll
    for (int i = 0; i < kUnits; ++i)
      if (off[i] >= 0) *reinterpret_cast<uint4*>(P + off[i]) = v[i];
  }
};

// acc += A[:, k range] B[:, k range]^T of the staged panels: waves 0-3 take the first half of the
// 16-steps of [0, kn), waves 4-7 the rest, each on the quadrant (wave % 4) of the 64 x 64 tile.
__device__ __forceinline__ void mma(f32x16_v& acc, const bf16* A, const bf16* Bp, int kn) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, quad = wave & 3;
  const int half = (kn >> 5) << 4;  // 16-steps of the first half
  const int k0 = wave < 4 ? 0 : half, k1 = wave < 4 ? half : kn;
  const bf16* ap = A + (32 * (quad >> 1) + (lane & 31)) * kLda + 8 * (lane >> 5);
  const bf16* bp = Bp + (32 * (quad & 1) + (lane & 31)) * kLda + 8 * (lane >> 5);
  for (int k = k0; k < k1; k += 16)
    acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(*reinterpret_cast<const bf16x8_v*>(ap + k),
                                                  *reinterpret_cast<const bf16x8_v*>(bp + k), acc, 0, 0, 0);
}

// Panels [k0, K) in chunks of kKC, A and B loaded together per chunk.
template <class SA, class SB>
__device__ __forceinline__ void mma_chunks(f32x16_v& acc, bf16* Ap, bf16* Bp, int k0, int K, const SA& srcA,
                                           const SB& srcB) {
  for (; k0 < K; k0 += kKC) {
    const int kn = K - k0 < kKC ? K - k0 : kKC;
    PanelLoad la, lb;
    la.issue(k0, kn, srcA);
    lb.issue(k0, kn, srcB);
    __syncthreads();  // the previous panels have been read
    la.commit(Ap);
    lb.commit(Bp);
    __syncthreads();
    mma(acc, Ap, Bp, kn);
  }
}

// The accumulator tile into C [64][kCp] fp32, the two K halves added in wave order (C may alias
// the B panel: called after the MFMAs, it synchronises first and last).
__device__ __forceinline__ void stage_acc(float* C, const f32x16_v& acc) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, quad = wave & 3;
  const int r0 = 32 * (quad >> 1) + 4 * (lane >> 5), c = 32 * (quad & 1) + (lane & 31);
  __syncthreads();
  if (wave < 4) {
#pragma unroll
    for (int r = 0; r < 16; ++r) C[(r0 + 8 * (r >> 2) + (r & 3)) * kCp + c] = acc[r];
  }
  __syncthreads();
  if (wave >= 4) {
#pragma unroll
    for (int r = 0; r < 16; ++r) C[(r0 + 8 * (r >> 2) + (r & 3)) * kCp + c] += acc[r];
  }
  __syncthreads();
}

// rstd of the row from the thread's kSeg columns
__device__ __forceinline__ float norm_rstd(const float* x, int d, float eps) {
  float ss = 0.0f;
#pragma unroll
  for (int i = 0; i < kSeg; ++i) ss += x[i] * x[i];
  return rsqrtf(row_sum(ss) / (float)d + eps);
}

// n = bf16(x rstd w (1 + g) + beta) of the thread's segment into the A panel, vec = w | g | beta
// (length d each, LDS); the writer stores x and n.
__device__ __forceinline__ void norm_to_panel(bf16* Ap, const float* vec, const float* x, float rstd, int d,
                                              const RowPos& P, bool writer, float* x_out, bf16* n_out) {
  if (P.cb >= d) return;
  if (writer && P.ok && x_out) {
#pragma unroll
    for (int j = 0; j < kSeg; j += 4) st4f(x_out + P.base + j, x + j);
  }
#pragma unroll
  for (int g = 0; g < kSeg / 8; ++g) {
    float w8[8], g8[8], b8[8], o[8];
    lds_n<8>(vec + P.cb + 8 * g, w8);
    lds_n<8>(vec + d + P.cb + 8 * g, g8);
    lds_n<8>(vec + 2 * d + P.cb + 8 * g, b8);
#pragma unroll
    for (int j = 0; j < 8; ++j) o[j] = P.ok ? x[8 * g + j] * rstd * w8[j] * (1.0f + g8[j]) + b8[j] : 0.0f;
    const uint4 u = from_f8(o);
    *reinterpret_cast<uint4*>(Ap + P.row * kLda + P.cb + 8 * g) = u;
    if (writer && P.ok && n_out) *reinterpret_cast<uint4*>(n_out + P.base + 8 * g) = u;
  }
}

// Zero rows [row0, row0 + nrows) x columns [c0, c0 + nc) of a bf16 matrix (nc % 8 == 0)
__device__ __forceinline__ void zero_bf16(bf16* p, int64_t ld, int64_t row0, int nrows, int c0, int nc) {
  const int upr = nc >> 3;
  for (int u = threadIdx.x; u < nrows * upr; u += kThreads) {
    const int r = u / upr;
    *reinterpret_cast<uint4*>(p + (row0 + r) * ld + c0 + (u - r * upr) * 8) = make_uint4(0u, 0u, 0u, 0u);
  }
}

// Columns [f0, f0 + fn) of a full-width bf16 operand from a compact one: col_of(f) is column f's
// position in the compact row (-1: not the recipe's, zero), read from the staged A panel when it
// holds the whole compact row, else from global memory.  Thread -> 8-column units.
template <class ColOf>
__device__ __forceinline__ void scatter_full(bf16* full, int64_t ldf, const Tile& T, int f0, int fn, const bf16* Ap,
                                             bool from_lds, const bf16* compact, int64_t ldc, const ColOf& col_of) {
  const int upr = fn >> 3;
  for (int uu = threadIdx.x; uu < T.nrows * upr; uu += kThreads) {
    const int r = uu / upr, f = f0 + (uu - r * upr) * 8;
    const int col = col_of(f);
    uint4 val = make_uint4(0u, 0u, 0u, 0u);
    if (col >= 0)
      val = from_lds ? *reinterpret_cast<const uint4*>(Ap + r * kLda + col)
                     : *reinterpret_cast<const uint4*>(compact + (T.row0 + r) * ldc + col);
    *reinterpret_cast<uint4*>(full + (T.row0 + r) * ldf + f) = val;
  }
}

// This tile's share [f0, f0 + fn) of F columns split over gridDim.x tiles (multiples of 8)
__device__ __forceinline__ void share_of(int F, int* f0, int* fn) {
  const int nct = gridDim.x;
  const int fw = ((F + nct - 1) / nct + 7) / 8 * 8;
  *f0 = blockIdx.x * fw;
  *fn = F - *f0 < fw ? (F - *f0 > 0 ? F - *f0 : 0) : fw;
}

// Epilogue position: thread -> (row, 8 consecutive columns) of the 64 x 64 tile
__device__ __forceinline__ int epi_row() { return threadIdx.x >> 3; }
__device__ __forceinline__ int epi_col() { return (threadIdx.x & 7) * 8; }

// ============================================================================ forward

// grid (3 Hmax, B rts): column tile c = (part, slot) of the compact q | k | v heads.
__global__ void __launch_bounds__(kThreads) rp_qkv_fwd_kernel(Meta M, const int32_t* __restrict__ info,
                                                               const float* __restrict__ h,
                                                               const float* __restrict__ h0,
                                                               const float* __restrict__ alpha, const float* w1,
                                                               const float* g1, const float* b1, float eps,
                                                               const bf16* __restrict__ wqkv_t,
                                                               const float* __restrict__ cs,
                                                               const float* __restrict__ sn, float* __restrict__ ht,
                                                               bf16* __restrict__ n1, float* __restrict__ rstd1,
                                                               bf16* __restrict__ q, bf16* __restrict__ k,
                                                               bf16* __restrict__ v) {
  extern __shared__ __align__(16) char smem[];
  const Smem L = smem_of(smem);
  const Tile T = tile_of(M);
  const int d = M.d;
  const RowPos P = row_pos(T, d);
  const int c = blockIdx.x, part = c / M.Hmax, slot = c - part * M.Hmax;
  const bool writer = c == 0;
  // round trip 1: the record, the rows, the norm vectors, this thread's RoPE factors
  InfoLoad il;
  il.issue(info, M, T.b);
  float x[kSeg], y[kSeg];
  ldn<kSeg>(h + P.base, P.ok, x);
  if (alpha) ldn<kSeg>(h0 + P.base, P.ok, y);
  const float al = alpha ? *alpha : 0.0f;
  VecLoad vl;
  vl.issue(w1, g1, b1, nullptr, 3, d);
  const int er = epi_row(), ec = epi_col(), s = T.s0 + er;
  float cv[8], sv[8];
  ldn<8>(cs + (int64_t)s * kHd + ec, part < 2 && er < T.nrows, cv);
  ldn<8>(sn + (int64_t)s * kHd + ec, part < 2 && er < T.nrows, sv);
  il.commit(L.inf, M);
  vl.commit(L.vec);
  __syncthreads();
  const Info I{L.inf, M.H, M.NB};
  bf16* dst = part == 0 ? q : (part == 1 ? k : v);
  const int64_t head_base = ((int64_t)T.b * M.Hmax + slot) * M.S;  // row (b, slot, s) = head_base + s
  if (!I.act() || slot >= I.nh()) {
    // an inactive sample or an unused head slot: zeros (the attention reads every slot)
    zero_bf16(dst, kHd, head_base + T.s0, T.nrows, 0, kHd);
    if (!I.act() && writer) zero_bf16(n1, d, T.row0, T.nrows, 0, d);
    return;
  }
  // round trip 2: the head's weight rows, overlapped with the norm
  const bf16* wrow = wqkv_t + ((int64_t)part * d + (int64_t)I.head(slot) * kHd) * d;
  PanelLoad lb;
  lb.issue(0, d, [&](int r, int kk) -> const bf16* { return wrow + (int64_t)r * d + kk; });
  if (alpha) {
#pragma unroll
    for (int i = 0; i < kSeg; ++i) x[i] += al * y[i];
  }
  const float rstd = norm_rstd(x, d, eps);
  if (writer && P.ok && P.seg == 0) rstd1[T.row0 + P.row] = rstd;
  norm_to_panel(L.A, L.vec, x, rstd, d, P, writer, ht, n1);
  lb.commit(L.B);
  __syncthreads();
  f32x16_v acc = zero16();
  mma(acc, L.A, L.B, d);
  float* C = reinterpret_cast<float*>(L.B);
  stage_acc(C, acc);
  if (er >= T.nrows) return;
  float o[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) o[j] = C[er * kCp + ec + j];
  if (part < 2) {
#pragma unroll
    for (int j = 0; j < 8; j += 2) {
      const float x0 = o[j], x1 = o[j + 1];
      o[j] = x0 * cv[j] - x1 * sv[j];
      o[j + 1] = x1 * cv[j + 1] + x0 * sv[j + 1];
    }
  }
  *reinterpret_cast<uint4*>(dst + (head_base + s) * kHd + ec) = from_f8(o);
}

// grid (d / 64, B rts): attn = y Wo over the recipe's heads, u = h~ + s_attn attn; y_full (the
// O-projection weight gradient's operand) gets head c's 64 columns or zeros.
__global__ void __launch_bounds__(kThreads) rp_oproj_fwd_kernel(Meta M, const int32_t* __restrict__ info,
                                                                 const bf16* __restrict__ y,
                                                                 const bf16* __restrict__ wo_t,
                                                                 const float* __restrict__ ht,
                                                                 const float* __restrict__ s_attn,
                                                                 float* __restrict__ attn, float* __restrict__ u,
                                                                 bf16* __restrict__ y_full) {
  extern __shared__ __align__(16) char smem[];
  const Smem L = smem_of(smem);
  const Tile T = tile_of(M);
  const int c = blockIdx.x, d = M.d, er = epi_row(), ec = epi_col();
  const int ldy = M.Hmax * kHd;  // <= 512: the whole compact row is one panel
  const bool rok = er < T.nrows;
  const int64_t off = (T.row0 + er) * d + c * kCols + ec;
  InfoLoad il;
  il.issue(info, M, T.b);
  PanelLoad la;
  la.issue(0, ldy, [&](int r, int kk) -> const bf16* {
    return r < T.nrows ? y + (T.row0 + r) * ldy + kk : nullptr;
  });
  float hv[8];
  ldn<8>(ht + off, rok, hv);
  const float sa = *s_attn;
  il.commit(L.inf, M);
  la.commit(L.A);
  __syncthreads();
  const Info I{L.inf, M.H, M.NB};
  if (!I.act()) {
    zero_bf16(y_full, d, T.row0, T.nrows, c * kHd, kHd);
    return;
  }
  const int K = I.nh() * kHd;
  PanelLoad lb;
  lb.issue(0, K, [&](int r, int kk) -> const bf16* {
    return wo_t + (int64_t)(c * kCols + r) * d + I.head(kk / kHd) * kHd + (kk % kHd);
  });
  lb.commit(L.B);
  __syncthreads();
  f32x16_v acc = zero16();
  mma(acc, L.A, L.B, K);
  float* C = reinterpret_cast<float*>(L.B);
  stage_acc(C, acc);
  if (!rok) return;
  float a8[8], u8[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    a8[j] = C[er * kCp + ec + j];
    u8[j] = hv[j] + sa * a8[j];
  }
  st4f(attn + off, a8);
  st4f(attn + off + 4, a8 + 4);
  st4f(u + off, u8);
  st4f(u + off + 4, u8 + 4);
  const int sl = I.ihead(c);  // head c's slot in the compact row (still in the A panel)
  uint4 v0 = make_uint4(0u, 0u, 0u, 0u);
  if (sl >= 0) v0 = *reinterpret_cast<const uint4*>(L.A + er * kLda + sl * kHd + ec);
  *reinterpret_cast<uint4*>(y_full + off) = v0;
}

// grid (NBmax, B rts): slot c's 32 neurons: [up | gate] = n2 [Wup | Wgate] rows, SwiGLU; ug keeps the
// bf16 pre-activations ([up 32 | gate 32] per slot), z = w up silu(gate).
__global__ void __launch_bounds__(kThreads) rp_upgate_fwd_kernel(Meta M, const int32_t* __restrict__ info,
                                                                  const float* __restrict__ u, const float* w2,
                                                                  const float* g2, const float* b2, float eps,
                                                                  const bf16* __restrict__ wug_t, float route_w,
                                                                  bf16* __restrict__ n2, float* __restrict__ rstd2,
                                                                  bf16* __restrict__ ug, bf16* __restrict__ z) {
  extern __shared__ __align__(16) char smem[];
  const Smem L = smem_of(smem);
  const Tile T = tile_of(M);
  const int c = blockIdx.x, d = M.d;
  const RowPos P = row_pos(T, d);
  const bool writer = c == 0;
  InfoLoad il;
  il.issue(info, M, T.b);
  float x[kSeg];
  ldn<kSeg>(u + P.base, P.ok, x);
  VecLoad vl;
  vl.issue(w2, g2, b2, nullptr, 3, d);
  il.commit(L.inf, M);
  vl.commit(L.vec);
  __syncthreads();
  const Info I{L.inf, M.H, M.NB};
  if (!I.act()) {
    if (writer) zero_bf16(n2, d, T.row0, T.nrows, 0, d);
    return;
  }
  if (c >= I.nb()) return;
  const int blk = I.blk(c);
  const int64_t F = M.F;
  PanelLoad lb;
  lb.issue(0, d, [&](int r, int kk) -> const bf16* {
    const int64_t nrow = r < kBlk ? (int64_t)blk * kBlk + r : F + (int64_t)blk * kBlk + (r - kBlk);
    return wug_t + nrow * d + kk;
  });
  const float rstd = norm_rstd(x, d, eps);
  if (writer && P.ok && P.seg == 0) rstd2[T.row0 + P.row] = rstd;
  norm_to_panel(L.A, L.vec, x, rstd, d, P, writer, nullptr, n2);
  lb.commit(L.B);
  __syncthreads();
  f32x16_v acc = zero16();
  mma(acc, L.A, L.B, d);
  float* C = reinterpret_cast<float*>(L.B);
  stage_acc(C, acc);
  // thread -> (row, 4 neurons)
  const int row = threadIdx.x >> 3, n0 = (threadIdx.x & 7) * 4;
  if (row >= T.nrows) return;
  float up[4], gt[4], zz[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    up[j] = round_bf(C[row * kCp + n0 + j]);
    gt[j] = round_bf(C[row * kCp + kBlk + n0 + j]);
    zz[j] = up[j] * gt[j] * sigmoidf_(gt[j]) * route_w;
  }
  const int64_t m = T.row0 + row;
  const int64_t ldu = (int64_t)M.NBmax * 2 * kBlk, ldz = (int64_t)M.NBmax * kBlk;
  *reinterpret_cast<uint2*>(ug + m * ldu + c * 2 * kBlk + n0) = make_uint2(pack_bf2(up[0], up[1]), pack_bf2(up[2], up[3]));
  *reinterpret_cast<uint2*>(ug + m * ldu + c * 2 * kBlk + kBlk + n0) =
      make_uint2(pack_bf2(gt[0], gt[1]), pack_bf2(gt[2], gt[3]));
  *reinterpret_cast<uint2*>(z + m * ldz + c * kBlk + n0) = make_uint2(pack_bf2(zz[0], zz[1]), pack_bf2(zz[2], zz[3]));
}

// grid (d / 64, B rts): mlp = z Wd over the recipe's slabs, h' = u + s_mlp mlp (inactive: h' = h);
// z_full (the down weight gradient's operand) spread over the column tiles.
__global__ void __launch_bounds__(kThreads) rp_down_fwd_kernel(Meta M, const int32_t* __restrict__ info,
                                                                const bf16* __restrict__ z,
                                                                const bf16* __restrict__ wd_t,
                                                                const float* __restrict__ u,
                                                                const float* __restrict__ h_in,
                                                                const float* __restrict__ s_mlp,
                                                                float* __restrict__ mlp, float* __restrict__ h_out,
                                                                bf16* __restrict__ z_full) {
  extern __shared__ __align__(16) char smem[];
  const Smem L = smem_of(smem);
  const Tile T = tile_of(M);
  const int c = blockIdx.x, d = M.d, F = M.F, er = epi_row(), ec = epi_col();
  const int ldz = M.NBmax * kBlk;
  const int kn0 = ldz < kKC ? ldz : kKC;
  const bool rok = er < T.nrows;
  const int64_t off = (T.row0 + er) * d + c * kCols + ec;
  auto srcA = [&](int r, int kk) -> const bf16* { return r < T.nrows ? z + (T.row0 + r) * ldz + kk : nullptr; };
  InfoLoad il;
  il.issue(info, M, T.b);
  PanelLoad la;
  la.issue(0, kn0, srcA);
  float uv[8], hv[8];
  ldn<8>(u + off, rok, uv);
  ldn<8>(h_in + off, rok, hv);
  const float sm = *s_mlp;
  il.commit(L.inf, M);
  la.commit(L.A);
  __syncthreads();
  const Info I{L.inf, M.H, M.NB};
  int f0, fn;
  share_of(F, &f0, &fn);
  if (!I.act()) {
    if (rok) {
      const float zf[4] = {0.f, 0.f, 0.f, 0.f};
      st4f(h_out + off, hv);
      st4f(h_out + off + 4, hv + 4);
      st4f(mlp + off, zf);
      st4f(mlp + off + 4, zf);
    }
    if (fn > 0) zero_bf16(z_full, F, T.row0, T.nrows, f0, fn);
    return;
  }
  const int K = I.nb() * kBlk;
  auto srcB = [&](int r, int kk) -> const bf16* {
    return wd_t + (int64_t)(c * kCols + r) * F + I.blk(kk / kBlk) * kBlk + (kk % kBlk);
  };
  const int kn = K < kKC ? K : kKC;
  PanelLoad lb;
  lb.issue(0, kn, srcB);
  lb.commit(L.B);
  __syncthreads();
  f32x16_v acc = zero16();
  mma(acc, L.A, L.B, kn);
  mma_chunks(acc, L.A, L.B, kKC, K, srcA, srcB);
  float* C = reinterpret_cast<float*>(L.B);
  stage_acc(C, acc);
  if (rok) {
    float m8[8], o8[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      m8[j] = C[er * kCp + ec + j];
      o8[j] = uv[j] + sm * m8[j];
    }
    st4f(mlp + off, m8);
    st4f(mlp + off + 4, m8 + 4);
    st4f(h_out + off, o8);
    st4f(h_out + off + 4, o8 + 4);
  }
  scatter_full(z_full, F, T, f0, fn, L.A, K <= kKC, z, ldz, [&](int f) {
    const int sl = I.iblk(f / kBlk);
    return sl >= 0 ? sl * kBlk + (f % kBlk) : -1;
  });
}

// ============================================================================ backward

// grid (ceil(NBmax / 2), B rts): dz = s_mlp dh Wd^T over two slots (64 neurons), SwiGLU backward
// into dug ([d up 32 | d gate 32] per slot).  The writer (c = 0) stores d_mlp = bf16(s_mlp dh) (the
// down weight gradient's operand) and the tile's sum of dh mlp (the s_mlp gradient).
__global__ void __launch_bounds__(kThreads) rp_down_bwd_kernel(Meta M, const int32_t* __restrict__ info,
                                                                const float* __restrict__ dh,
                                                                const float* __restrict__ mlp,
                                                                const float* __restrict__ s_mlp,
                                                                const bf16* __restrict__ wd,
                                                                const bf16* __restrict__ ug, float route_w,
                                                                bf16* __restrict__ dug, bf16* __restrict__ d_mlp,
                                                                float* __restrict__ p_sm) {
  extern __shared__ __align__(16) char smem[];
  const Smem L = smem_of(smem);
  const Tile T = tile_of(M);
  const int c = blockIdx.x, d = M.d, tid = threadIdx.x;
  const RowPos P = row_pos(T, d);
  const bool writer = c == 0;
  const int64_t ldu = (int64_t)M.NBmax * 2 * kBlk;
  const int er = epi_row(), e = tid & 7;
  const int sl = 2 * c + (e >> 2), n0 = (e & 3) * 8;  // epilogue: 8 neurons of one slot
  const bool eok = er < T.nrows && sl < M.NBmax;
  InfoLoad il;
  il.issue(info, M, T.b);
  float x[kSeg], mv[kSeg];
  ldn<kSeg>(dh + P.base, P.ok, x);
  if (writer) ldn<kSeg>(mlp + P.base, P.ok, mv);
  const float sm = *s_mlp;
  uint4 uq[2] = {};
  if (eok) {
    const bf16* ugr = ug + (T.row0 + er) * ldu + sl * 2 * kBlk;
    uq[0] = *reinterpret_cast<const uint4*>(ugr + n0);
    uq[1] = *reinterpret_cast<const uint4*>(ugr + kBlk + n0);
  }
  il.commit(L.inf, M);
  __syncthreads();
  const Info I{L.inf, M.H, M.NB};
  if (!I.act()) {
    if (writer) {
      zero_bf16(d_mlp, d, T.row0, T.nrows, 0, d);
      if (tid == 0) p_sm[blockIdx.y] = 0.0f;
    }
    return;
  }
  const int nbv = I.nb();
  if (2 * c >= nbv) return;
  PanelLoad lb;
  lb.issue(0, d, [&](int r, int kk) -> const bf16* {
    const int s_ = 2 * c + r / kBlk;
    return s_ < nbv ? wd + ((int64_t)I.blk(s_) * kBlk + (r % kBlk)) * d + kk : nullptr;
  });
  float dsum = 0.0f;
  if (P.cb < d) {
#pragma unroll
    for (int g = 0; g < kSeg / 8; ++g) {
      float o[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        o[j] = x[8 * g + j] * sm;
        if (writer) dsum += x[8 * g + j] * mv[8 * g + j];
      }
      const uint4 uv = from_f8(o);
      *reinterpret_cast<uint4*>(L.A + P.row * kLda + P.cb + 8 * g) = uv;
      if (writer && P.ok) *reinterpret_cast<uint4*>(d_mlp + P.base + 8 * g) = uv;
    }
  }
  if (writer) {
    const float tot = block_sum(dsum, L.red);
    if (tid == 0) p_sm[blockIdx.y] = tot;
  }
  lb.commit(L.B);
  __syncthreads();
  f32x16_v acc = zero16();
  mma(acc, L.A, L.B, d);
  float* C = reinterpret_cast<float*>(L.B);
  stage_acc(C, acc);
  if (!eok || sl >= nbv) return;
  float up[8], gt[8], du_[8], dg_[8];
  to_f8(uq[0], up);
  to_f8(uq[1], gt);
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const float dz = C[er * kCp + (e >> 2) * kBlk + n0 + j] * route_w;
    const float sg = sigmoidf_(gt[j]);
    du_[j] = dz * gt[j] * sg;
    dg_[j] = dz * up[j] * sg * (1.0f + gt[j] * (1.0f - sg));
  }
  bf16* dgr = dug + (T.row0 + er) * ldu + sl * 2 * kBlk;
  *reinterpret_cast<uint4*>(dgr + n0) = from_f8(du_);
  *reinterpret_cast<uint4*>(dgr + kBlk + n0) = from_f8(dg_);
}

// grid (d / 64, B rts): dn2 = dug [Wup | Wgate]^T over the recipe's slabs; dug_full (the up / gate
// weight gradient's operand, [M, 2F] columns [up F | gate F]) spread over the column tiles.
__global__ void __launch_bounds__(kThreads) rp_upgate_bwd_kernel(Meta M, const int32_t* __restrict__ info,
                                                                  const bf16* __restrict__ dug,
                                                                  const bf16* __restrict__ wug,
                                                                  float* __restrict__ dn2,
                                                                  bf16* __restrict__ dug_full) {
  extern __shared__ __align__(16) char smem[];
  const Smem L = smem_of(smem);
  const Tile T = tile_of(M);
  const int c = blockIdx.x, d = M.d, F = M.F, F2 = 2 * M.F;
  const int ldu = M.NBmax * 2 * kBlk;
  const int kn0 = ldu < kKC ? ldu : kKC;
  auto srcA = [&](int r, int kk) -> const bf16* { return r < T.nrows ? dug + (T.row0 + r) * ldu + kk : nullptr; };
  InfoLoad il;
  il.issue(info, M, T.b);
  PanelLoad la;
  la.issue(0, kn0, srcA);
  il.commit(L.inf, M);
  la.commit(L.A);
  __syncthreads();
  const Info I{L.inf, M.H, M.NB};
  int f0, fn;
  share_of(F2, &f0, &fn);
  if (!I.act()) {
    if (fn > 0) zero_bf16(dug_full, F2, T.row0, T.nrows, f0, fn);
    return;
  }
  const int K = I.nb() * 2 * kBlk;
  auto srcB = [&](int r, int kk) -> const bf16* {
    const int s_ = kk / (2 * kBlk), w = kk % (2 * kBlk);
    const int64_t col = (w < kBlk ? 0 : (int64_t)F) + (int64_t)I.blk(s_) * kBlk + (w % kBlk);
    return wug + (int64_t)(c * kCols + r) * F2 + col;
  };
  const int kn = K < kKC ? K : kKC;
  PanelLoad lb;
  lb.issue(0, kn, srcB);
  lb.commit(L.B);
  __syncthreads();
  f32x16_v acc = zero16();
  mma(acc, L.A, L.B, kn);
  mma_chunks(acc, L.A, L.B, kKC, K, srcA, srcB);
  float* C = reinterpret_cast<float*>(L.B);
  stage_acc(C, acc);
  const int er = epi_row(), ec = epi_col();
  if (er < T.nrows) {
    const int64_t off = (T.row0 + er) * d + c * kCols + ec;
    st4f(dn2 + off, C + er * kCp + ec);
    st4f(dn2 + off + 4, C + er * kCp + ec + 4);
  }
  scatter_full(dug_full, F2, T, f0, fn, L.A, K <= kKC, dug, ldu, [&](int f2) {
    const int part = f2 >= F ? 1 : 0, f = f2 - part * F;
    const int sl = I.iblk(f / kBlk);
    return sl >= 0 ? sl * 2 * kBlk + part * kBlk + (f % kBlk) : -1;
  });
}

// grid (d / 64, B rts).  Every tile: du = dh + the rmsnorm-FiLM backward of dn2 (the row dot over the
// whole row), A = bf16(s_attn du).  Tile c stores du and d_attn = A (the O weight gradient's operand)
// on its 64 columns, and for c < Hmax forms head slot c of dy = A Wo^T (zeros for an unused slot).
__global__ void __launch_bounds__(kThreads) rp_oproj_bwd_kernel(Meta M, const int32_t* __restrict__ info,
                                                                 const float* __restrict__ dh,
                                                                 const float* __restrict__ dn2,
                                                                 const float* __restrict__ u,
                                                                 const float* __restrict__ rstd2, const float* w2,
                                                                 const float* g2, const float* __restrict__ s_attn,
                                                                 const bf16* __restrict__ wo, float* __restrict__ du,
                                                                 bf16* __restrict__ d_attn, bf16* __restrict__ dy) {
  extern __shared__ __align__(16) char smem[];
  const Smem L = smem_of(smem);
  const Tile T = tile_of(M);
  const int c = blockIdx.x, d = M.d, tid = threadIdx.x;
  const RowPos P = row_pos(T, d);
  const int64_t ldy = (int64_t)M.Hmax * kHd;
  InfoLoad il;
  il.issue(info, M, T.b);
  float a[kSeg], x[kSeg], g[kSeg];
  ldn<kSeg>(dn2 + P.base, P.ok, a);
  ldn<kSeg>(u + P.base, P.ok, x);
  ldn<kSeg>(dh + P.base, P.ok, g);
  const float rs = P.row < T.nrows ? rstd2[T.row0 + P.row] : 0.0f;
  const float sa = *s_attn;
  VecLoad vl;
  vl.issue(w2, g2, nullptr, nullptr, 2, d);
  il.commit(L.inf, M);
  vl.commit(L.vec);
  __syncthreads();
  const Info I{L.inf, M.H, M.NB};
  auto zero_dy = [&]() {
    const int upr = kHd / 8;
    for (int uu = tid; uu < T.nrows * upr; uu += kThreads) {
      const int r = uu / upr;
      *reinterpret_cast<uint4*>(dy + (T.row0 + r) * ldy + c * kHd + (uu - r * upr) * 8) = make_uint4(0u, 0u, 0u, 0u);
    }
  };
  if (!I.act()) {
    if (c < M.Hmax) zero_dy();
    zero_bf16(d_attn, d, T.row0, T.nrows, c * kCols, kCols);
    return;
  }
  float dot = 0.0f;
  if (P.cb < d) {
#pragma unroll
    for (int gg = 0; gg < kSeg / 8; ++gg) {
      float w8[8], g8[8];
      lds_n<8>(L.vec + P.cb + 8 * gg, w8);
      lds_n<8>(L.vec + d + P.cb + 8 * gg, g8);
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        a[8 * gg + j] *= w8[j] * (1.0f + g8[j]);  // dn^
        dot += a[8 * gg + j] * x[8 * gg + j];
      }
    }
  }
  const float mean = row_sum(dot) * rs / (float)d;
#pragma unroll
  for (int i = 0; i < kSeg; ++i) a[i] = rs * (a[i] - x[i] * rs * mean);  // the norm term; x is done
  // round trip 2: the head's weight rows, overlapped with du and the A panel
  const bool mm = c < M.Hmax && c < I.nh();
  PanelLoad lb;
  if (mm) {
    const int head = I.head(c);
    lb.issue(0, d, [&](int r, int kk) -> const bf16* { return wo + ((int64_t)head * kHd + r) * d + kk; });
  }
  // du = dh + norm term; A panel and (from segment c of the row) tile c's du / d_attn columns
  if (P.cb < d) {
#pragma unroll
    for (int gg = 0; gg < kSeg / 8; ++gg) {
      float o[8], dv[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int i = 8 * gg + j;
        dv[j] = P.ok ? g[i] + a[i] : 0.0f;
        o[j] = sa * dv[j];
      }
      const uint4 av = from_f8(o);
      *reinterpret_cast<uint4*>(L.A + P.row * kLda + P.cb + 8 * gg) = av;
      if (P.ok && P.seg == c) {
        st4f(du + P.base + 8 * gg, dv);
        st4f(du + P.base + 8 * gg + 4, dv + 4);
        *reinterpret_cast<uint4*>(d_attn + P.base + 8 * gg) = av;
      }
    }
  }
  if (c >= M.Hmax) return;
  if (!mm) {
    zero_dy();
    return;
  }
  lb.commit(L.B);
  __syncthreads();
  f32x16_v acc = zero16();
  mma(acc, L.A, L.B, d);
  float* C = reinterpret_cast<float*>(L.B);
  stage_acc(C, acc);
  const int er = epi_row(), ec = epi_col();
  if (er >= T.nrows) return;
  float o[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) o[j] = C[er * kCp + ec + j];
  *reinterpret_cast<uint4*>(dy + (T.row0 + er) * ldy + c * kHd + ec) = from_f8(o);
}

// grid (d / 64, B rts): dn1 = dqkv [Wq | Wk | Wv]^T over the recipe's heads; dqkv_full (the QKV
// weight gradient's operand, [M, 3d]) spread over the column tiles.  dqkv is the attention
// backward's compact [M, 3 Hmax 64] (dq slots | dk slots | dv slots).
__global__ void __launch_bounds__(kThreads) rp_qkv_bwd_kernel(Meta M, const int32_t* __restrict__ info,
                                                               const bf16* __restrict__ dqkv,
                                                               const bf16* __restrict__ wqkv,
                                                               float* __restrict__ dn1,
                                                               bf16* __restrict__ dqkv_full) {
  extern __shared__ __align__(16) char smem[];
  const Smem L = smem_of(smem);
  const Tile T = tile_of(M);
  const int c = blockIdx.x, d = M.d, d3 = 3 * M.d;
  const int64_t ldq = (int64_t)3 * M.Hmax * kHd, ps = (int64_t)M.Hmax * kHd;
  InfoLoad il;
  il.issue(info, M, T.b);
  il.commit(L.inf, M);
  __syncthreads();
  const Info I{L.inf, M.H, M.NB};
  int f0, fn;
  share_of(d3, &f0, &fn);
  if (!I.act()) {
    if (fn > 0) zero_bf16(dqkv_full, d3, T.row0, T.nrows, f0, fn);
    return;
  }
  const int kp = I.nh() * kHd, K = 3 * kp;
  auto srcA = [&](int r, int kk) -> const bf16* {
    const int part = kk / kp;
    return r < T.nrows ? dqkv + (T.row0 + r) * ldq + part * ps + (kk - part * kp) : nullptr;
  };
  auto srcB = [&](int r, int kk) -> const bf16* {
    const int part = kk / kp, w = kk - part * kp;
    return wqkv + (int64_t)(c * kCols + r) * d3 + (int64_t)part * d + I.head(w / kHd) * kHd + (w % kHd);
  };
  f32x16_v acc = zero16();
  mma_chunks(acc, L.A, L.B, 0, K, srcA, srcB);
  float* C = reinterpret_cast<float*>(L.B);
  stage_acc(C, acc);
  const int er = epi_row(), ec = epi_col();
  if (er < T.nrows) {
    const int64_t off = (T.row0 + er) * d + c * kCols + ec;
    st4f(dn1 + off, C + er * kCp + ec);
    st4f(dn1 + off + 4, C + er * kCp + ec + 4);
  }
  // the panel holds [dq live | dk live | dv live] when K fits one panel
  scatter_full(dqkv_full, d3, T, f0, fn, L.A, K <= kKC, dqkv, ldq, [&](int f) {
    const int part = f / d, hc = f - part * d;
    const int sl = I.ihead(hc / kHd);
    if (sl < 0) return -1;
    return K <= kKC ? part * kp + sl * kHd + (hc % kHd) : (int)(part * ps) + sl * kHd + (hc % kHd);
  });
}

// grid (d / 64, B rts): dh~ = du + the rmsnorm-FiLM backward of dn1 (the row dot over the whole row,
// every tile), then tile c's columns: dh_in = dh~ (inactive samples: dh_in = dh), dh0 (+)= alpha dh~,
// and the tile's partials: dw1 | dg1 | db1 and dw2 | dg2 | db2 per column, sum du attn (s_attn)
// and sum dh~ h0 (alpha).
__global__ void __launch_bounds__(kThreads) rp_norm_bwd_kernel(Meta M, const int32_t* __restrict__ info,
                                                                const float* __restrict__ dn1,
                                                                const float* __restrict__ du,
                                                                const float* __restrict__ dh,
                                                                const float* __restrict__ ht,
                                                                const float* __restrict__ rstd1, const float* w1,
                                                                const float* g1, const float* __restrict__ h0,
                                                                const float* __restrict__ alpha,
                                                                const float* __restrict__ dn2,
                                                                const float* __restrict__ u,
                                                                const float* __restrict__ rstd2, const float* w2,
                                                                const float* g2, const float* __restrict__ attn,
                                                                int accumulate, float* __restrict__ dh_in,
                                                                float* __restrict__ dh0, float* __restrict__ p_film1,
                                                                float* __restrict__ p_film2, float* __restrict__ p_sa,
                                                                float* __restrict__ p_alpha) {
  extern __shared__ __align__(16) char smem[];
  const Smem L = smem_of(smem);
  float* Pw = reinterpret_cast<float*>(smem);  // 6 x [64][kCols] partial terms (panel area)
  const Tile T = tile_of(M);
  const int c = blockIdx.x, d = M.d, tid = threadIdx.x;
  const RowPos P = row_pos(T, d);
  const int nct = gridDim.x;
  const int er = epi_row(), ec = epi_col();
  const bool rok = er < T.nrows;
  const int own0 = c * kCols;
  const int64_t off = (T.row0 + er) * d + own0 + ec;
  InfoLoad il;
  il.issue(info, M, T.b);
  float a[kSeg], x[kSeg];
  ldn<kSeg>(dn1 + P.base, P.ok, a);
  ldn<kSeg>(ht + P.base, P.ok, x);
  const float rs1r = P.row < T.nrows ? rstd1[T.row0 + P.row] : 0.0f;
  const float rs1 = rok ? rstd1[T.row0 + er] : 0.0f;
  const float rs2 = rok ? rstd2[T.row0 + er] : 0.0f;
  const float al = alpha ? *alpha : 0.0f;
  VecLoad vl;
  vl.issue(w1, g1, w2, g2, 4, d);
  // this thread's 8 columns of tile c
  float a1[8], x1[8], uu[8], zz[8], dd[8], a2[8], x2[8], at[8];
  ldn<8>(dn1 + off, rok, a1);
  ldn<8>(ht + off, rok, x1);
  ldn<8>(du + off, rok, uu);
  ldn<8>(h0 + off, rok && h0, zz);
  ldn<8>(dh + off, rok, dd);
  ldn<8>(dn2 + off, rok, a2);
  ldn<8>(u + off, rok, x2);
  ldn<8>(attn + off, rok, at);
  il.commit(L.inf, M);
  vl.commit(L.vec);
  __syncthreads();
  const Info I{L.inf, M.H, M.NB};
  float* pf1 = p_film1 + (int64_t)blockIdx.y * 3 * d;
  float* pf2 = p_film2 + (int64_t)blockIdx.y * 3 * d;
  if (!I.act()) {
    if (rok) {
      st4f(dh_in + off, dd);
      st4f(dh_in + off + 4, dd + 4);
      if (dh0 && !accumulate) {
        const float zf[4] = {0.f, 0.f, 0.f, 0.f};
        st4f(dh0 + off, zf);
        st4f(dh0 + off + 4, zf);
      }
    }
    for (int i = tid; i < 3 * kCols; i += kThreads) {
      pf1[(i / kCols) * d + own0 + (i % kCols)] = 0.0f;
      pf2[(i / kCols) * d + own0 + (i % kCols)] = 0.0f;
    }
    if (tid == 0) {
      p_sa[(int64_t)blockIdx.y * nct + c] = 0.0f;
      p_alpha[(int64_t)blockIdx.y * nct + c] = 0.0f;
    }
    return;
  }
  const float* v1 = L.vec;           // w1 | g1
  const float* v2 = L.vec + 2 * d;   // w2 | g2
  float dot = 0.0f;
  if (P.cb < d) {
#pragma unroll
    for (int gg = 0; gg < kSeg / 8; ++gg) {
      float w8[8], g8[8];
      lds_n<8>(v1 + P.cb + 8 * gg, w8);
      lds_n<8>(v1 + d + P.cb + 8 * gg, g8);
#pragma unroll
      for (int j = 0; j < 8; ++j) dot += a[8 * gg + j] * w8[j] * (1.0f + g8[j]) * x[8 * gg + j];
    }
  }
  // the row mapping and the tile-column mapping both put thread t on row t / 8
  const float mean = row_sum(dot) * rs1r / (float)d;
  float w1v[8], g1v[8], w2v[8], g2v[8];
  lds_n<8>(v1 + own0 + ec, w1v);
  lds_n<8>(v1 + d + own0 + ec, g1v);
  lds_n<8>(v2 + own0 + ec, w2v);
  lds_n<8>(v2 + d + own0 + ec, g2v);
  __syncthreads();  // the vectors are read; the panel area becomes the partial terms
  float osa = 0.0f, oal = 0.0f;
  float o[8], s0[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const float xh1 = x1[j] * rs1, xh2 = x2[j] * rs2;
    const float dnh = a1[j] * w1v[j] * (1.0f + g1v[j]);
    o[j] = uu[j] + rs1 * (dnh - xh1 * mean);
    osa += uu[j] * at[j];
    oal += o[j] * zz[j];
    Pw[(0 * kRows + er) * kCols + ec + j] = rok ? a1[j] * (1.0f + g1v[j]) * xh1 : 0.0f;  // dw1
    Pw[(1 * kRows + er) * kCols + ec + j] = rok ? a1[j] * w1v[j] * xh1 : 0.0f;            // dg1
    Pw[(2 * kRows + er) * kCols + ec + j] = rok ? a1[j] : 0.0f;                           // db1
    Pw[(3 * kRows + er) * kCols + ec + j] = rok ? a2[j] * (1.0f + g2v[j]) * xh2 : 0.0f;  // dw2
    Pw[(4 * kRows + er) * kCols + ec + j] = rok ? a2[j] * w2v[j] * xh2 : 0.0f;            // dg2
    Pw[(5 * kRows + er) * kCols + ec + j] = rok ? a2[j] : 0.0f;                           // db2
  }
  if (rok) {
    st4f(dh_in + off, o);
    st4f(dh_in + off + 4, o + 4);
    if (dh0) {
      float p8[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
      if (accumulate) {
        ld4f(dh0 + off, p8);
        ld4f(dh0 + off + 4, p8 + 4);
      }
#pragma unroll
      for (int j = 0; j < 8; ++j) s0[j] = p8[j] + al * o[j];
      st4f(dh0 + off, s0);
      st4f(dh0 + off + 4, s0 + 4);
    }
  } else {
    osa = oal = 0.0f;
  }
  __syncthreads();
  for (int i = tid; i < 6 * kCols; i += kThreads) {
    const int term = i / kCols, col = i - term * kCols;
    float s = 0.0f;
    for (int r = 0; r < kRows; ++r) s += Pw[(term * kRows + r) * kCols + col];
    float* pf = term < 3 ? pf1 : pf2;
    pf[(term % 3) * d + own0 + col] = s;
  }
  const float tsa = block_sum(osa, L.red);
  const float tal = block_sum(oal, L.red);
  if (tid == 0) {
    p_sa[(int64_t)blockIdx.y * nct + c] = tsa;
    p_alpha[(int64_t)blockIdx.y * nct + c] = tal;
  }
}

// Fixed-order sums of the per-tile partials of T passes: out [T, 6d] = (dw1 | dg1 | db1 | dw2 | dg2 |
// db2) of each pass, then dw1 [d] and dw2 [d] over all passes, ds_attn [T], ds_mlp [T], dalpha.
__global__ void __launch_bounds__(256) rp_param_reduce_kernel(int T, int nt, int nct, int d, const float* __restrict__ p1,
                                                               const float* __restrict__ p2, const float* __restrict__ psa,
                                                               const float* __restrict__ psm, const float* __restrict__ pal,
                                                               float* __restrict__ out) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int W = 6 * d;
  const int64_t n_pass = (int64_t)T * W;
  if (i < n_pass) {
    const int t = (int)(i / W), col = (int)(i - (int64_t)t * W);
    const float* p = col < 3 * d ? p1 + (int64_t)t * nt * 3 * d + col : p2 + (int64_t)t * nt * 3 * d + (col - 3 * d);
    float s = 0.0f;
    for (int r = 0; r < nt; ++r) s += p[(int64_t)r * 3 * d];
    out[i] = s;
    return;
  }
  const int64_t j = i - n_pass;
  if (j < 2 * d) {
    const int which = (int)(j / d), col = (int)(j - which * d);
    const float* p = which == 0 ? p1 : p2;
    float s = 0.0f;
    for (int t = 0; t < T; ++t)
      for (int r = 0; r < nt; ++r) s += p[((int64_t)t * nt + r) * 3 * d + col];
    out[n_pass + j] = s;
    return;
  }
  const int64_t k = j - 2 * d;
  if (k < T) {
    float s = 0.0f;
    for (int r = 0; r < nt * nct; ++r) s += psa[(int64_t)k * nt * nct + r];
    out[n_pass + 2 * d + k] = s;
  } else if (k < 2 * T) {
    float s = 0.0f;
    for (int r = 0; r < nt; ++r) s += psm[(k - T) * nt + r];
    out[n_pass + 2 * d + k] = s;
  } else if (k == 2 * T) {
    float s = 0.0f;
    for (int r = 0; r < T * nt * nct; ++r) s += pal[r];
    out[n_pass + 2 * d + k] = s;
  }
}

bool set_lds(const void* fn, size_t bytes) {
  return hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes) == hipSuccess;
}

bool g_lds_set = false;

int replay_prepare() {
  if (g_lds_set) return 0;
  const void* fns[] = {(const void*)rp_qkv_fwd_kernel,   (const void*)rp_oproj_fwd_kernel,
                       (const void*)rp_upgate_fwd_kernel, (const void*)rp_down_fwd_kernel,
                       (const void*)rp_down_bwd_kernel,   (const void*)rp_upgate_bwd_kernel,
                       (const void*)rp_oproj_bwd_kernel,  (const void*)rp_qkv_bwd_kernel,
                       (const void*)rp_norm_bwd_kernel};
  for (const void* f : fns) RTE_REQUIRE(set_lds(f, kLds), "replay: cannot raise the LDS limit to %zu bytes", kLds);
  g_lds_set = true;
  return 0;
}

int make_meta(int B, int S, int d, int H, int F, int NB, int h_max, int nb_max, Meta* M) {
  RTE_REQUIRE(B >= 1 && S >= 1, "replay: need B >= 1 and S >= 1");
  RTE_REQUIRE(d % 128 == 0 && d <= kMaxD, "replay: d must be a multiple of 128 up to %d", kMaxD);
  RTE_REQUIRE(H * kHd == d, "replay: head width must be %d", kHd);
  RTE_REQUIRE(F % kBlk == 0 && NB * kBlk == F, "replay: d_ff must be a whole number of 32-neuron blocks");
  RTE_REQUIRE(h_max >= 1 && h_max <= H && nb_max >= 1 && nb_max <= NB, "replay: bad recipe widths");
  const int W = 4 + 2 * H + 2 * NB;
  RTE_REQUIRE(W <= kInfoMax, "replay: recipe record of %d words exceeds %d", W, kInfoMax);
  const int rts = (S + kRows - 1) / kRows;
  RTE_REQUIRE((int64_t)B * rts <= 65535, "replay: too many row tiles");
  *M = Meta{B, S, d, F, rts, H, NB, h_max, nb_max, W};
  return replay_prepare();
}

}  // namespace

int attention_fwd(const bf16* q, const bf16* k, const bf16* v, int B, int H, int S, int head_dim, float scale,
                  const float* hscale, bf16* out, float* lse, hipStream_t s);
int attention_bwd_qkv(const bf16* q, const bf16* k, const bf16* v, const bf16* out, const bf16* dout,
                      const float* lse, int B, int H, int S, int head_dim, float scale, const float* hscale,
                      const float* cos_t, const float* sin_t, bf16* dqkv, hipStream_t s);

int replay_fwd_pass(int B, int S, int d, int H, int F, int NB, int h_max, int nb_max, const int32_t* info,
                    const float* h, const float* h0, const float* alpha, const float* w1, const float* g1,
                    const float* b1, float eps1, const float* w2, const float* g2, const float* b2, float eps2,
                    const float* s_attn, const float* s_mlp, float route_w, const bf16* wqkv_t, const bf16* wo_t,
                    const bf16* wug_t, const bf16* wd_t, const float* cs, const float* sn, float* ht, bf16* n1,
                    float* rstd1, bf16* q, bf16* k, bf16* v, bf16* y, float* lse, float* attn, float* u,
                    bf16* y_full, bf16* n2, float* rstd2, bf16* ug, bf16* z, float* mlp, float* h_out, bf16* z_full,
                    hipStream_t s) {
  Meta M;
  RTE_TRY(make_meta(B, S, d, H, F, NB, h_max, nb_max, &M));
  RTE_REQUIRE(info && h && h0 && w1 && w2 && s_attn && s_mlp && wqkv_t && wo_t && wug_t && wd_t && cs && sn,
              "replay_fwd: missing input");
  const unsigned rt = (unsigned)(B * M.rts);
  hipLaunchKernelGGL(rp_qkv_fwd_kernel, dim3(3 * h_max, rt), dim3(kThreads), kLds, s, M, info, h, h0, alpha, w1, g1, b1,
                     eps1, wqkv_t, cs, sn, ht, n1, rstd1, q, k, v);
  RTE_TRY(check_launch("replay_qkv_fwd"));
  RTE_TRY(attention_fwd(q, k, v, B, h_max, S, kHd, 0.125f, nullptr, y, lse, s));
  hipLaunchKernelGGL(rp_oproj_fwd_kernel, dim3(d / kCols, rt), dim3(kThreads), kLds, s, M, info, y, wo_t, ht, s_attn, attn,
                     u, y_full);
  RTE_TRY(check_launch("replay_oproj_fwd"));
  hipLaunchKernelGGL(rp_upgate_fwd_kernel, dim3(nb_max, rt), dim3(kThreads), kLds, s, M, info, u, w2, g2, b2, eps2, wug_t,
                     route_w, n2, rstd2, ug, z);
  RTE_TRY(check_launch("replay_upgate_fwd"));
  hipLaunchKernelGGL(rp_down_fwd_kernel, dim3(d / kCols, rt), dim3(kThreads), kLds, s, M, info, z, wd_t, u, h, s_mlp, mlp,
                     h_out, z_full);
  return check_launch("replay_down_fwd");
}

int replay_bwd_pass(int B, int S, int d, int H, int F, int NB, int h_max, int nb_max, const int32_t* info,
                    const float* dh, const float* mlp, const float* s_mlp, const bf16* wd, const bf16* ug,
                    float route_w, bf16* dug, bf16* d_mlp, float* p_sm, const bf16* wug, float* dn2, bf16* dug_full,
                    const float* u, const float* rstd2, const float* w2, const float* g2, const float* attn,
                    const float* s_attn, const bf16* wo, float* du, bf16* d_attn, bf16* dy, float* p_film2,
                    float* p_sa, const bf16* q, const bf16* k, const bf16* v, const bf16* y, const float* lse,
                    const float* cs, const float* sn, bf16* dqkv, const bf16* wqkv, float* dn1, bf16* dqkv_full,
                    const float* ht, const float* rstd1, const float* w1, const float* g1, const float* h0,
                    const float* alpha, int accumulate, float* dh_in, float* dh0, float* p_film1, float* p_alpha,
                    hipStream_t s) {
  Meta M;
  RTE_TRY(make_meta(B, S, d, H, F, NB, h_max, nb_max, &M));
  RTE_REQUIRE(info && dh && mlp && s_mlp && wd && ug && dug && d_mlp && p_sm && wug && dn2 && dug_full && u &&
                  rstd2 && w2 && attn && s_attn && wo && du && d_attn && dy && p_film2 && p_sa && q && k && v && y &&
                  lse && cs && sn && dqkv && wqkv && dn1 && dqkv_full && ht && rstd1 && w1 && dh_in && p_film1 &&
                  p_alpha,
              "replay_bwd: missing buffer");
  RTE_REQUIRE(!alpha || (h0 && dh0), "replay_bwd: the input skip needs h0 and dh0");
  const unsigned rt = (unsigned)(B * M.rts);
  hipLaunchKernelGGL(rp_down_bwd_kernel, dim3((nb_max + 1) / 2, rt), dim3(kThreads), kLds, s, M, info, dh, mlp, s_mlp, wd,
                     ug, route_w, dug, d_mlp, p_sm);
  RTE_TRY(check_launch("replay_down_bwd"));
  hipLaunchKernelGGL(rp_upgate_bwd_kernel, dim3(d / kCols, rt), dim3(kThreads), kLds, s, M, info, dug, wug, dn2, dug_full);
  RTE_TRY(check_launch("replay_upgate_bwd"));
  hipLaunchKernelGGL(rp_oproj_bwd_kernel, dim3(d / kCols, rt), dim3(kThreads), kLds, s, M, info, dh, dn2, u, rstd2, w2, g2,
                     s_attn, wo, du, d_attn, dy);
  RTE_TRY(check_launch("replay_oproj_bwd"));
  RTE_TRY(attention_bwd_qkv(q, k, v, y, dy, lse, B, h_max, S, kHd, 0.125f, nullptr, cs, sn, dqkv, s));
  hipLaunchKernelGGL(rp_qkv_bwd_kernel, dim3(d / kCols, rt), dim3(kThreads), kLds, s, M, info, dqkv, wqkv, dn1, dqkv_full);
  RTE_TRY(check_launch("replay_qkv_bwd"));
  hipLaunchKernelGGL(rp_norm_bwd_kernel, dim3(d / kCols, rt), dim3(kThreads), kLds, s, M, info, dn1, du, dh, ht, rstd1, w1,
                     g1, h0, alpha, dn2, u, rstd2, w2, g2, attn, accumulate, dh_in, dh0, p_film1, p_film2, p_sa,
                     p_alpha);
  return check_launch("replay_norm_bwd");
}

int replay_param_reduce(int T, int B, int S, int d, const float* p1, const float* p2, const float* psa,
                        const float* psm, const float* pal, float* out, hipStream_t s) {
  RTE_REQUIRE(T >= 1 && B >= 1 && S >= 1 && d % 128 == 0 && d <= kMaxD, "replay_param_reduce: bad shape");
  const int nt = B * ((S + kRows - 1) / kRows), nct = d / kCols;
  const int64_t n = (int64_t)T * 6 * d + 2 * d + 2 * T + 1;
  hipLaunchKernelGGL(rp_param_reduce_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, T, nt, nct, d, p1,
                     p2, psa, psm, pal, out);
  return check_launch("replay_param_reduce");
}

}  // namespace rte

using namespace rte;

extern "C" {

int rte_replay_fwd_pass(int B, int S, int d, int H, int F, int n_blk, int h_max, int nb_max, const int32_t* info,
                        const float* h, const float* h0, const float* alpha, const float* w1, const float* g1,
                        const float* b1, float eps1, const float* w2, const float* g2, const float* b2, float eps2,
                        const float* s_attn, const float* s_mlp, float route_w, const void* wqkv_t, const void* wo_t,
                        const void* wug_t, const void* wd_t, const float* cos_t, const float* sin_t, float* ht,
                        void* n1, float* rstd1, void* q, void* k, void* v, void* y, float* lse, float* attn, float* u,
                        void* y_full, void* n2, float* rstd2, void* ug, void* z, float* mlp, float* h_out,
                        void* z_full, void* stream) {
  auto cb = [](const void* p) { return static_cast<const bf16*>(p); };
  auto b16 = [](void* p) { return static_cast<bf16*>(p); };
  return replay_fwd_pass(B, S, d, H, F, n_blk, h_max, nb_max, info, h, h0, alpha, w1, g1, b1, eps1, w2, g2, b2, eps2,
                         s_attn, s_mlp, route_w, cb(wqkv_t), cb(wo_t), cb(wug_t), cb(wd_t), cos_t, sin_t, ht, b16(n1),
                         rstd1, b16(q), b16(k), b16(v), b16(y), lse, attn, u, b16(y_full), b16(n2), rstd2, b16(ug),
                         b16(z), mlp, h_out, b16(z_full), static_cast<hipStream_t>(stream));
}

int rte_replay_bwd_pass(int B, int S, int d, int H, int F, int n_blk, int h_max, int nb_max, const int32_t* info,
                        const float* dh, const float* mlp, const float* s_mlp, const void* wd, const void* ug,
                        float route_w, void* dug, void* d_mlp, float* p_sm, const void* wug, float* dn2,
                        void* dug_full, const float* u, const float* rstd2, const float* w2, const float* g2,
                        const float* attn, const float* s_attn, const void* wo, float* du, void* d_attn, void* dy,
                        float* p_film2, float* p_sa, const void* q, const void* k, const void* v, const void* y,
                        const float* lse, const float* cos_t, const float* sin_t, void* dqkv, const void* wqkv,
                        float* dn1, void* dqkv_full, const float* ht, const float* rstd1, const float* w1,
                        const float* g1, const float* h0, const float* alpha, int accumulate, float* dh_in,
                        float* dh0, float* p_film1, float* p_alpha, void* stream) {
  auto cb = [](const void* p) { return static_cast<const bf16*>(p); };
  auto b16 = [](void* p) { return static_cast<bf16*>(p); };
  return replay_bwd_pass(B, S, d, H, F, n_blk, h_max, nb_max, info, dh, mlp, s_mlp, cb(wd), cb(ug), route_w, b16(dug),
                         b16(d_mlp), p_sm, cb(wug), dn2, b16(dug_full), u, rstd2, w2, g2, attn, s_attn, cb(wo), du,
                         b16(d_attn), b16(dy), p_film2, p_sa, cb(q), cb(k), cb(v), cb(y), lse, cos_t, sin_t,
                         b16(dqkv), cb(wqkv), dn1, b16(dqkv_full), ht, rstd1, w1, g1, h0, alpha, accumulate, dh_in,
                         dh0, p_film1, p_alpha, static_cast<hipStream_t>(stream));
}

int rte_replay_param_reduce(int T, int B, int S, int d, const float* p_film1, const float* p_film2,
                            const float* p_sa, const float* p_sm, const float* p_alpha, float* out, void* stream) {
  return replay_param_reduce(T, B, S, d, p_film1, p_film2, p_sa, p_sm, p_alpha, out,
                             static_cast<hipStream_t>(stream));
}

}  // extern "C"
