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
// bound by memory latency and by how much one CU can pull, not by arithmetic.  So the products run
// as tile kernels that read only bf16 panels: each owns a 64-row tile of one sample and a 64-column
// output tile, loads its A panel together with the sample's recipe record (one round trip), then
// the recipe's weight rows (a second), and runs its MFMAs from LDS.  The RMSNorm forward and
// backward, whose row statistics need whole rows, run as row kernels spread over many workgroups
// (one wave per row).  Only the recipe's heads (64 columns each) and 32-neuron slab blocks take
// part.  The record of each (pass, sample), gathered once per replay, is int32 [W],
// W = 4 + 2 H + 2 NB:
//   act | nh | nb | 0 | heads[H] (ascending) | ihead[H] (slot or -1) | blks[NB] | iblk[NB]
//
//   forward per pass : axpy_norm (h~, n1) -> qkv (QKV + RoPE, compact heads) -> attention
//                      (attention.hip) -> oproj (O-projection) -> axpy_norm (u, n2) -> upgate
//                      (up/gate + SwiGLU) -> down (down-projection + residual)
//   backward per pass: down_bwd (dz + SwiGLU backward) -> upgate_bwd (dn2) -> norm2_bwd (du,
//                      d_attn, FiLM2 / s_attn partials) -> dy (O-projection backward) ->
//                      attention backward (dqkv, RoPE undone) -> qkv_bwd (dn1) -> norm1_bwd (dh,
//                      dh0, FiLM1 / alpha partials, and the next pass's down operand)
//
// Weight gradients are not formed here: the kernels write each pass's product operands at full
// width (zeros outside the recipe's heads / slabs), so one plain GEMM per weight over all passes'
// rows forms them afterwards.  FiLM, scale and skip gradients leave as per-workgroup partials,
// summed by param_reduce in a fixed order.  No atomics: results repeat bitwise.
//
// MFMA lane layout (32x32x16 bf16): lane l supplies A row l % 32 and B column l % 32 with k values
// 8 (l / 32) .. +7 of each 16-step; output register r of lane l holds row 8 (r / 4) + 4 (l / 32)
// + r % 4, column l % 32.  Eight waves (512 threads) per tile workgroup: waves w and w + 4 take the
// two halves of K on quadrant w % 4 of the 64 x 64 tile.
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

// grid (3 Hmax, B rts): column tile c = (part, slot) of the compact q | k | v heads from the bf16
// norm rows n1 (A panel), RoPE on q and k.
__global__ void __launch_bounds__(kThreads) rp_qkv_fwd_kernel(Meta M, const int32_t* __restrict__ info,
                                                               const bf16* __restrict__ n1,
                                                               const bf16* __restrict__ wqkv_t,
                                                               const float* __restrict__ cs,
                                                               const float* __restrict__ sn, bf16* __restrict__ q,
                                                               bf16* __restrict__ k, bf16* __restrict__ v) {
  extern __shared__ __align__(16) char smem[];
  const Smem L = smem_of(smem);
  const Tile T = tile_of(M);
  const int d = M.d;
  const int c = blockIdx.x, part = c / M.Hmax, slot = c - part * M.Hmax;
  // round trip 1: the record, the A panel, this thread's RoPE factors
  InfoLoad il;
  il.issue(info, M, T.b);
  PanelLoad la;
  la.issue(0, d, [&](int r, int kk) -> const bf16* { return r < T.nrows ? n1 + (T.row0 + r) * d + kk : nullptr; });
  const int er = epi_row(), ec = epi_col(), s = T.s0 + er;
  float cv[8], sv[8];
  ldn<8>(cs + (int64_t)s * kHd + ec, part < 2 && er < T.nrows, cv);
  ldn<8>(sn + (int64_t)s * kHd + ec, part < 2 && er < T.nrows, sv);
  il.commit(L.inf, M);
  la.commit(L.A);
  __syncthreads();
  const Info I{L.inf, M.H, M.NB};
  bf16* dst = part == 0 ? q : (part == 1 ? k : v);
  const int64_t head_base = ((int64_t)T.b * M.Hmax + slot) * M.S;  // row (b, slot, s) = head_base + s
  if (!I.act() || slot >= I.nh()) {
    // an inactive sample or an unused head slot: zeros (the attention reads every slot)
    zero_bf16(dst, kHd, head_base + T.s0, T.nrows, 0, kHd);
    return;
  }
  // round trip 2: the head's weight rows
  const bf16* wrow = wqkv_t + ((int64_t)part * d + (int64_t)I.head(slot) * kHd) * d;
  PanelLoad lb;
  lb.issue(0, d, [&](int r, int kk) -> const bf16* { return wrow + (int64_t)r * d + kk; });
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

// grid (d / 64, B rts): attn = y Wo over the recipe's heads; y_full (the O-projection weight
// gradient's operand) gets head c's 64 columns or zeros.
__global__ void __launch_bounds__(kThreads) rp_oproj_fwd_kernel(Meta M, const int32_t* __restrict__ info,
                                                                 const bf16* __restrict__ y,
                                                                 const bf16* __restrict__ wo_t,
                                                                 float* __restrict__ attn,
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
  st4f(attn + off, C + er * kCp + ec);
  st4f(attn + off + 4, C + er * kCp + ec + 4);
  const int sl = I.ihead(c);  // head c's slot in the compact row (still in the A panel)
  uint4 v0 = make_uint4(0u, 0u, 0u, 0u);
  if (sl >= 0) v0 = *reinterpret_cast<const uint4*>(L.A + er * kLda + sl * kHd + ec);
  *reinterpret_cast<uint4*>(y_full + off) = v0;
}

// grid (NBmax, B rts): slot c's 32 neurons: [up | gate] = n2 [Wup | Wgate] rows from the bf16 norm
// rows n2, SwiGLU; ug keeps the bf16 pre-activations ([up 32 | gate 32] per slot), z = w up silu(gate).
__global__ void __launch_bounds__(kThreads) rp_upgate_fwd_kernel(Meta M, const int32_t* __restrict__ info,
                                                                  const bf16* __restrict__ n2,
                                                                  const bf16* __restrict__ wug_t, float route_w,
                                                                  bf16* __restrict__ ug, bf16* __restrict__ z) {
  extern __shared__ __align__(16) char smem[];
  const Smem L = smem_of(smem);
  const Tile T = tile_of(M);
  const int c = blockIdx.x, d = M.d;
  InfoLoad il;
  il.issue(info, M, T.b);
  PanelLoad la;
  la.issue(0, d, [&](int r, int kk) -> const bf16* { return r < T.nrows ? n2 + (T.row0 + r) * d + kk : nullptr; });
  il.commit(L.inf, M);
  la.commit(L.A);
  __syncthreads();
  const Info I{L.inf, M.H, M.NB};
  if (!I.act() || c >= I.nb()) return;
  const int blk = I.blk(c);
  const int64_t F = M.F;
  PanelLoad lb;
  lb.issue(0, d, [&](int r, int kk) -> const bf16* {
    const int64_t nrow = r < kBlk ? (int64_t)blk * kBlk + r : F + (int64_t)blk * kBlk + (r - kBlk);
    return wug_t + nrow * d + kk;
  });
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

// grid (ceil(NBmax / 2), B rts): dz = a_mlp Wd^T over two slots (64 neurons) with a_mlp =
// bf16(s_mlp dh) (row kernels make it), SwiGLU backward into dug ([d up 32 | d gate 32] per slot).
__global__ void __launch_bounds__(kThreads) rp_down_bwd_kernel(Meta M, const int32_t* __restrict__ info,
                                                                const bf16* __restrict__ a_mlp,
                                                                const bf16* __restrict__ wd,
                                                                const bf16* __restrict__ ug, float route_w,
                                                                bf16* __restrict__ dug) {
  extern __shared__ __align__(16) char smem[];
  const Smem L = smem_of(smem);
  const Tile T = tile_of(M);
  const int c = blockIdx.x, d = M.d;
  const int64_t ldu = (int64_t)M.NBmax * 2 * kBlk;
  const int er = epi_row(), e = threadIdx.x & 7;
  const int sl = 2 * c + (e >> 2), n0 = (e & 3) * 8;  // epilogue: 8 neurons of one slot
  const bool eok = er < T.nrows && sl < M.NBmax;
  InfoLoad il;
  il.issue(info, M, T.b);
  PanelLoad la;
  la.issue(0, d, [&](int r, int kk) -> const bf16* { return r < T.nrows ? a_mlp + (T.row0 + r) * d + kk : nullptr; });
  uint4 uq[2] = {};
  if (eok) {
    const bf16* ugr = ug + (T.row0 + er) * ldu + sl * 2 * kBlk;
    uq[0] = *reinterpret_cast<const uint4*>(ugr + n0);
    uq[1] = *reinterpret_cast<const uint4*>(ugr + kBlk + n0);
  }
  il.commit(L.inf, M);
  la.commit(L.A);
  __syncthreads();
  const Info I{L.inf, M.H, M.NB};
  const int nbv = I.nb();
  if (!I.act() || 2 * c >= nbv) return;
  PanelLoad lb;
  lb.issue(0, d, [&](int r, int kk) -> const bf16* {
    const int s_ = 2 * c + r / kBlk;
    return s_ < nbv ? wd + ((int64_t)I.blk(s_) * kBlk + (r % kBlk)) * d + kk : nullptr;
  });
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

// grid (Hmax, B rts): head slot c of dy = d_attn Wo^T (d_attn = bf16(s_attn du), the row kernel's
// output), zeros for an unused slot or an inactive sample (the attention backward reads every slot).
__global__ void __launch_bounds__(kThreads) rp_dy_kernel(Meta M, const int32_t* __restrict__ info,
                                                          const bf16* __restrict__ d_attn,
                                                          const bf16* __restrict__ wo, bf16* __restrict__ dy) {
  extern __shared__ __align__(16) char smem[];
  const Smem L = smem_of(smem);
  const Tile T = tile_of(M);
  const int c = blockIdx.x, d = M.d;
  const int64_t ldy = (int64_t)M.Hmax * kHd;
  InfoLoad il;
  il.issue(info, M, T.b);
  PanelLoad la;
  la.issue(0, d, [&](int r, int kk) -> const bf16* { return r < T.nrows ? d_attn + (T.row0 + r) * d + kk : nullptr; });
  il.commit(L.inf, M);
  la.commit(L.A);
  __syncthreads();
  const Info I{L.inf, M.H, M.NB};
  if (!I.act() || c >= I.nh()) {
    const int upr = kHd / 8;
    for (int uu = threadIdx.x; uu < T.nrows * upr; uu += kThreads) {
      const int r = uu / upr;
      *reinterpret_cast<uint4*>(dy + (T.row0 + r) * ldy + c * kHd + (uu - r * upr) * 8) = make_uint4(0u, 0u, 0u, 0u);
    }
    return;
  }
  const int head = I.head(c);
  PanelLoad lb;
  lb.issue(0, d, [&](int r, int kk) -> const bf16* { return wo + ((int64_t)head * kHd + r) * d + kk; });
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

// ---------------------------------------------------------------------------- row kernels
// One wave per row (four rows per workgroup), lane l on columns [8 l, 8 l + 8) (d <= 512): the
// norm backwards, whose row dots need whole rows.  Per-workgroup partials of the parameter
// gradients (sums over the workgroup's rows, fixed order) go to param_reduce.

constexpr int kRowWG = 4;

struct RowCtx {
  int64_t m;      // global row
  int c0;         // first column of the lane
  bool ok, act;   // row exists, lane inside d; sample takes this pass
};

__device__ __forceinline__ RowCtx row_ctx(const Meta& M, const int32_t* info) {
  RowCtx r;
  r.m = (int64_t)blockIdx.x * kRowWG + (threadIdx.x >> 6);
  r.c0 = (threadIdx.x & 63) * 8;
  const bool row_ok = r.m < (int64_t)M.B * M.S;
  r.ok = row_ok && r.c0 < M.d;
  r.act = row_ok && info[(r.m / M.S) * M.W] != 0;
  return r;
}

__device__ __forceinline__ void ld8(const float* p, bool ok, float* v) { ldn<8>(p, ok, v); }

__device__ __forceinline__ void st8(float* p, const float* v) {
  st4f(p, v);
  st4f(p + 4, v + 4);
}

// Column partials of NT terms [kRowWG waves][NT][d] in LDS summed over the waves into out[t d + c]
template <int NT>
__device__ __forceinline__ void wave_col_partials(float* lds, const float (&terms)[NT][8], int d, int c0,
                                                  float* out) {
  const int wave = threadIdx.x >> 6;
  if (c0 < d) {
#pragma unroll
    for (int t = 0; t < NT; ++t)
#pragma unroll
      for (int j = 0; j < 8; ++j) lds[(wave * NT + t) * kMaxD + c0 + j] = terms[t][j];
  }
  __syncthreads();
  for (int i = threadIdx.x; i < NT * d; i += 256) {
    const int t = i / d, c = i - t * d;
    float s = 0.0f;
    for (int w = 0; w < kRowWG; ++w) s += lds[(w * NT + t) * kMaxD + c];
    out[t * d + c] = s;
  }
}

__device__ __forceinline__ float wg_sum(float v, float* red) {
  v = wsum(v);
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  return (red[0] + red[1]) + (red[2] + red[3]);
}

// a_mlp = bf16(s_mlp dh) and the workgroup's sum of dh mlp (the s_mlp gradient): the down
// backward's operand for the first pass the backward visits (later passes get it from norm1_bwd).
__global__ void __launch_bounds__(256) rp_dh_prep_kernel(Meta M, const float* __restrict__ dh,
                                                          const float* __restrict__ mlp,
                                                          const float* __restrict__ s_mlp, bf16* __restrict__ a_mlp,
                                                          float* __restrict__ p_sm) {
  __shared__ float red[4];
  const int64_t m = (int64_t)blockIdx.x * kRowWG + (threadIdx.x >> 6);
  const int c0 = (threadIdx.x & 63) * 8, d = M.d;
  const bool ok = m < (int64_t)M.B * M.S && c0 < d;
  float x[8], mv[8];
  ld8(dh + m * d + c0, ok, x);
  ld8(mlp + m * d + c0, ok, mv);
  const float sm = *s_mlp;
  float s = 0.0f, o[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    s += x[j] * mv[j];
    o[j] = sm * x[j];
  }
  if (ok) *reinterpret_cast<uint4*>(a_mlp + m * d + c0) = from_f8(o);
  const float tot = wg_sum(s, red);
  if (threadIdx.x == 0) p_sm[blockIdx.x] = tot;
}

// du = dh + rmsnorm-FiLM backward of dn2 (w2, g2, rstd2, u), d_attn = bf16(s_attn du) (zeros for an
// inactive sample), partials dw2 | dg2 | db2 [nt, 3d] and sum du attn (the s_attn gradient) [nt].
__global__ void __launch_bounds__(256) rp_norm2_bwd_kernel(Meta M, const int32_t* __restrict__ info,
                                                            const float* __restrict__ dh, const float* __restrict__ dn2,
                                                            const float* __restrict__ u, const float* __restrict__ rstd2,
                                                            const float* __restrict__ w2, const float* __restrict__ g2,
                                                            const float* __restrict__ attn,
                                                            const float* __restrict__ s_attn, float* __restrict__ du,
                                                            bf16* __restrict__ d_attn, float* __restrict__ p_film2,
                                                            float* __restrict__ p_sa) {
  __shared__ float lds[kRowWG * 3 * kMaxD];
  __shared__ float red[4];
  const RowCtx R = row_ctx(M, info);
  const int d = M.d;
  const int64_t off = R.m * d + R.c0;
  float a[8], x[8], g[8], at[8], w8[8], g8[8];
  ld8(dn2 + off, R.ok, a);
  ld8(u + off, R.ok, x);
  ld8(dh + off, R.ok, g);
  ld8(attn + off, R.ok, at);
  ld8(w2 + R.c0, R.c0 < d, w8);
  ld8(g2 + R.c0, R.c0 < d, g8);
  const float rs = R.ok ? rstd2[R.m] : 0.0f;
  const float sa = *s_attn;
  float dot = 0.0f;
#pragma unroll
  for (int j = 0; j < 8; ++j) dot += a[j] * w8[j] * (1.0f + g8[j]) * x[j];
  const float mean = wsum(dot) * rs / (float)d;
  float terms[3][8], dv[8], o[8], sat = 0.0f;
  const bool act = R.act && R.ok;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const float xh = x[j] * rs, dnh = a[j] * w8[j] * (1.0f + g8[j]);
    dv[j] = g[j] + rs * (dnh - xh * mean);
    o[j] = act ? sa * dv[j] : 0.0f;
    terms[0][j] = act ? a[j] * (1.0f + g8[j]) * xh : 0.0f;
    terms[1][j] = act ? a[j] * w8[j] * xh : 0.0f;
    terms[2][j] = act ? a[j] : 0.0f;
    sat += act ? dv[j] * at[j] : 0.0f;
  }
  if (R.ok) {
    if (R.act) st8(du + off, dv);
    *reinterpret_cast<uint4*>(d_attn + off) = from_f8(o);
  }
  wave_col_partials<3>(lds, terms, d, R.c0, p_film2 + (int64_t)blockIdx.x * 3 * d);
  const float tot = wg_sum(sat, red);
  if (threadIdx.x == 0) p_sa[blockIdx.x] = tot;
}

// dh~ = du + rmsnorm-FiLM backward of dn1 (w1, g1, rstd1, h~); dh_in = dh~ (inactive: dh_in = dh),
// dh0 (+)= alpha dh~; partials dw1 | dg1 | db1 [nt, 3d] and sum dh~ h0 (the alpha gradient) [nt].
// With a_next: the next pass's down operand bf16(s_mlp_next dh_in) and its sum dh_in mlp_next.
__global__ void __launch_bounds__(256) rp_norm1_bwd_kernel(Meta M, const int32_t* __restrict__ info,
                                                            const float* __restrict__ dn1, const float* __restrict__ du,
                                                            const float* __restrict__ dh, const float* __restrict__ ht,
                                                            const float* __restrict__ rstd1,
                                                            const float* __restrict__ w1, const float* __restrict__ g1,
                                                            const float* __restrict__ h0,
                                                            const float* __restrict__ alpha, int accumulate,
                                                            float* __restrict__ dh_in, float* __restrict__ dh0,
                                                            float* __restrict__ p_film1, float* __restrict__ p_alpha,
                                                            const float* __restrict__ mlp_next,
                                                            const float* __restrict__ s_mlp_next,
                                                            bf16* __restrict__ a_next, float* __restrict__ p_sm_next) {
  __shared__ float lds[kRowWG * 3 * kMaxD];
  __shared__ float red[4];
  const RowCtx R = row_ctx(M, info);
  const int d = M.d;
  const int64_t off = R.m * d + R.c0;
  const bool act = R.act && R.ok;
  float a[8], x[8], uu[8], g[8], z8[8], w8[8], g8[8], mv[8];
  ld8(dn1 + off, R.ok, a);
  ld8(ht + off, R.ok, x);
  ld8(du + off, act, uu);
  ld8(dh + off, R.ok, g);
  ld8(h0 + off, R.ok && h0, z8);
  ld8(w1 + R.c0, R.c0 < d, w8);
  ld8(g1 + R.c0, R.c0 < d, g8);
  ld8(mlp_next + off, R.ok && a_next, mv);
  const float rs = R.ok ? rstd1[R.m] : 0.0f;
  const float al = alpha ? *alpha : 0.0f;
  const float smn = a_next ? *s_mlp_next : 0.0f;
  float dot = 0.0f;
#pragma unroll
  for (int j = 0; j < 8; ++j) dot += a[j] * w8[j] * (1.0f + g8[j]) * x[j];
  const float mean = wsum(dot) * rs / (float)d;
  float terms[3][8], o[8], s0[8], nx[8], sal = 0.0f, ssm = 0.0f;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const float xh = x[j] * rs, dnh = a[j] * w8[j] * (1.0f + g8[j]);
    const float dht = uu[j] + rs * (dnh - xh * mean);
    o[j] = act ? dht : g[j];
    terms[0][j] = act ? a[j] * (1.0f + g8[j]) * xh : 0.0f;
    terms[1][j] = act ? a[j] * w8[j] * xh : 0.0f;
    terms[2][j] = act ? a[j] : 0.0f;
    sal += act ? dht * z8[j] : 0.0f;
    nx[j] = smn * o[j];
    ssm += o[j] * mv[j];
  }
  if (R.ok) {
    st8(dh_in + off, o);
    if (dh0) {
      float p8[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
      if (accumulate) ld8(dh0 + off, true, p8);
#pragma unroll
      for (int j = 0; j < 8; ++j) s0[j] = p8[j] + (act ? al * o[j] : 0.0f);
      st8(dh0 + off, s0);
    }
    if (a_next) *reinterpret_cast<uint4*>(a_next + off) = from_f8(nx);
  }
  wave_col_partials<3>(lds, terms, d, R.c0, p_film1 + (int64_t)blockIdx.x * 3 * d);
  const float tal = wg_sum(sal, red);
  if (threadIdx.x == 0) p_alpha[blockIdx.x] = tal;
  if (a_next) {
    const float tsm = wg_sum(ssm, red);
    if (threadIdx.x == 0) p_sm_next[blockIdx.x] = tsm;
  }
}

// Fixed-order sums of the per-workgroup partials of T passes (nt row workgroups each): out [T, 6d] =
// (dw1 | dg1 | db1 | dw2 | dg2 | db2) of each pass, then dw1 [d] and dw2 [d] over all passes,
// ds_attn [T], ds_mlp [T], dalpha.
__global__ void __launch_bounds__(256) rp_param_reduce_kernel(int T, int nt, int d, const float* __restrict__ p1,
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
    for (int r = 0; r < nt; ++r) s += psa[(int64_t)k * nt + r];
    out[n_pass + 2 * d + k] = s;
  } else if (k < 2 * T) {
    float s = 0.0f;
    for (int r = 0; r < nt; ++r) s += psm[(k - T) * nt + r];
    out[n_pass + 2 * d + k] = s;
  } else if (k == 2 * T) {
    float s = 0.0f;
    for (int r = 0; r < T * nt; ++r) s += pal[r];
    out[n_pass + 2 * d + k] = s;
  }
}

bool set_lds(const void* fn, size_t bytes) {
  return hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes) == hipSuccess;
}

bool g_lds_set = false;

int replay_prepare() {
  if (g_lds_set) return 0;
  const void* fns[] = {(const void*)rp_qkv_fwd_kernel,  (const void*)rp_oproj_fwd_kernel,
                       (const void*)rp_upgate_fwd_kernel, (const void*)rp_down_fwd_kernel,
                       (const void*)rp_down_bwd_kernel,  (const void*)rp_upgate_bwd_kernel,
                       (const void*)rp_dy_kernel,         (const void*)rp_qkv_bwd_kernel};
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
int axpy_norm_fwd(const float* a, const float* b, const float* c, const float* keep, const uint8_t* mask, int S,
                  int T, int d, const float* w, const float* gamma, const float* beta, float eps, float* x_out,
                  bf16* n_out, float* rstd_out, hipStream_t s);

int replay_row_tiles(int B, int S) { return (B * S + kRowWG - 1) / kRowWG; }

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
  const int Mrows = B * S;
  // h~ = h + alpha h0 and its FiLM norm (the axpy / norm row kernel of the per-operator pass)
  RTE_TRY(axpy_norm_fwd(h, alpha ? h0 : nullptr, alpha, nullptr, nullptr, S, Mrows, d, w1, g1, b1, eps1, ht, n1,
                        rstd1, s));
  hipLaunchKernelGGL(rp_qkv_fwd_kernel, dim3(3 * h_max, rt), dim3(kThreads), kLds, s, M, info, n1, wqkv_t, cs, sn, q,
                     k, v);
  RTE_TRY(check_launch("replay_qkv_fwd"));
  RTE_TRY(attention_fwd(q, k, v, B, h_max, S, kHd, 0.125f, nullptr, y, lse, s));
  hipLaunchKernelGGL(rp_oproj_fwd_kernel, dim3(d / kCols, rt), dim3(kThreads), kLds, s, M, info, y, wo_t, attn,
                     y_full);
  RTE_TRY(check_launch("replay_oproj_fwd"));
  // u = h~ + s_attn attn and its FiLM norm
  RTE_TRY(axpy_norm_fwd(ht, attn, s_attn, nullptr, nullptr, S, Mrows, d, w2, g2, b2, eps2, u, n2, rstd2, s));
  hipLaunchKernelGGL(rp_upgate_fwd_kernel, dim3(nb_max, rt), dim3(kThreads), kLds, s, M, info, n2, wug_t, route_w, ug,
                     z);
  RTE_TRY(check_launch("replay_upgate_fwd"));
  hipLaunchKernelGGL(rp_down_fwd_kernel, dim3(d / kCols, rt), dim3(kThreads), kLds, s, M, info, z, wd_t, u, h, s_mlp,
                     mlp, h_out, z_full);
  return check_launch("replay_down_fwd");
}

int replay_bwd_prep(int B, int S, int d, const float* dh, const float* mlp, const float* s_mlp, bf16* a_mlp,
                    float* p_sm, hipStream_t s) {
  RTE_REQUIRE(B >= 1 && S >= 1 && d % 128 == 0 && d <= kMaxD && dh && mlp && s_mlp && a_mlp && p_sm,
              "replay_bwd_prep: bad arguments");
  Meta M{B, S, d, 0, 0, 0, 0, 0, 0, 0};
  hipLaunchKernelGGL(rp_dh_prep_kernel, dim3(replay_row_tiles(B, S)), dim3(256), 0, s, M, dh, mlp, s_mlp, a_mlp, p_sm);
  return check_launch("replay_bwd_prep");
}

int replay_bwd_pass(int B, int S, int d, int H, int F, int NB, int h_max, int nb_max, const int32_t* info,
                    const float* dh, const bf16* a_mlp, const bf16* wd, const bf16* ug, float route_w, bf16* dug,
                    const bf16* wug, float* dn2, bf16* dug_full, const float* u, const float* rstd2,
                    const float* w2, const float* g2, const float* attn, const float* s_attn, float* du,
                    bf16* d_attn, float* p_film2, float* p_sa, const bf16* wo, bf16* dy, const bf16* q, const bf16* k,
                    const bf16* v, const bf16* y, const float* lse, const float* cs, const float* sn, bf16* dqkv,
                    const bf16* wqkv, float* dn1, bf16* dqkv_full, const float* ht, const float* rstd1,
                    const float* w1, const float* g1, const float* h0, const float* alpha, int accumulate,
                    float* dh_in, float* dh0, float* p_film1, float* p_alpha, const float* mlp_next,
                    const float* s_mlp_next, bf16* a_next, float* p_sm_next, hipStream_t s) {
  Meta M;
  RTE_TRY(make_meta(B, S, d, H, F, NB, h_max, nb_max, &M));
  RTE_REQUIRE(info && dh && a_mlp && wd && ug && dug && wug && dn2 && dug_full && u && rstd2 && w2 && attn && s_attn &&
                  du && d_attn && p_film2 && p_sa && wo && dy && q && k && v && y && lse && cs && sn && dqkv &&
                  wqkv && dn1 && dqkv_full && ht && rstd1 && w1 && dh_in && p_film1 && p_alpha,
              "replay_bwd: missing buffer");
  RTE_REQUIRE(!alpha || (h0 && dh0), "replay_bwd: the input skip needs h0 and dh0");
  RTE_REQUIRE(!a_next || (mlp_next && s_mlp_next && p_sm_next), "replay_bwd: the next pass's operand needs mlp");
  const unsigned rt = (unsigned)(B * M.rts), nrow = (unsigned)replay_row_tiles(B, S);
  hipLaunchKernelGGL(rp_down_bwd_kernel, dim3((nb_max + 1) / 2, rt), dim3(kThreads), kLds, s, M, info, a_mlp, wd, ug,
                     route_w, dug);
  RTE_TRY(check_launch("replay_down_bwd"));
  hipLaunchKernelGGL(rp_upgate_bwd_kernel, dim3(d / kCols, rt), dim3(kThreads), kLds, s, M, info, dug, wug, dn2,
                     dug_full);
  RTE_TRY(check_launch("replay_upgate_bwd"));
  hipLaunchKernelGGL(rp_norm2_bwd_kernel, dim3(nrow), dim3(256), 0, s, M, info, dh, dn2, u, rstd2, w2, g2, attn, s_attn,
                     du, d_attn, p_film2, p_sa);
  RTE_TRY(check_launch("replay_norm2_bwd"));
  hipLaunchKernelGGL(rp_dy_kernel, dim3(h_max, rt), dim3(kThreads), kLds, s, M, info, d_attn, wo, dy);
  RTE_TRY(check_launch("replay_dy"));
  RTE_TRY(attention_bwd_qkv(q, k, v, y, dy, lse, B, h_max, S, kHd, 0.125f, nullptr, cs, sn, dqkv, s));
  hipLaunchKernelGGL(rp_qkv_bwd_kernel, dim3(d / kCols, rt), dim3(kThreads), kLds, s, M, info, dqkv, wqkv, dn1,
                     dqkv_full);
  RTE_TRY(check_launch("replay_qkv_bwd"));
  hipLaunchKernelGGL(rp_norm1_bwd_kernel, dim3(nrow), dim3(256), 0, s, M, info, dn1, du, dh, ht, rstd1, w1, g1, h0,
                     alpha, accumulate, dh_in, dh0, p_film1, p_alpha, mlp_next, s_mlp_next, a_next, p_sm_next);
  return check_launch("replay_norm1_bwd");
}

int replay_param_reduce(int T, int B, int S, int d, const float* p1, const float* p2, const float* psa,
                        const float* psm, const float* pal, float* out, hipStream_t s) {
  RTE_REQUIRE(T >= 1 && B >= 1 && S >= 1 && d % 128 == 0 && d <= kMaxD, "replay_param_reduce: bad shape");
  const int nt = replay_row_tiles(B, S);
  const int64_t n = (int64_t)T * 6 * d + 2 * d + 2 * T + 1;
  hipLaunchKernelGGL(rp_param_reduce_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, T, nt, d, p1, p2,
                     psa, psm, pal, out);
  return check_launch("replay_param_reduce");
}

}  // namespace rte

using namespace rte;

extern "C" {

int rte_replay_row_tiles(int B, int S) { return replay_row_tiles(B, S); }

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

int rte_replay_bwd_prep(int B, int S, int d, const float* dh, const float* mlp, const float* s_mlp, void* a_mlp,
                        float* p_sm, void* stream) {
  return replay_bwd_prep(B, S, d, dh, mlp, s_mlp, static_cast<bf16*>(a_mlp), p_sm, static_cast<hipStream_t>(stream));
}

int rte_replay_bwd_pass(int B, int S, int d, int H, int F, int n_blk, int h_max, int nb_max, const int32_t* info,
                        const float* dh, const void* a_mlp, const void* wd, const void* ug, float route_w, void* dug,
                        const void* wug, float* dn2, void* dug_full, const float* u, const float* rstd2,
                        const float* w2, const float* g2, const float* attn, const float* s_attn, float* du,
                        void* d_attn, float* p_film2, float* p_sa, const void* wo, void* dy, const void* q,
                        const void* k, const void* v, const void* y, const float* lse, const float* cos_t,
                        const float* sin_t, void* dqkv, const void* wqkv, float* dn1, void* dqkv_full,
                        const float* ht, const float* rstd1, const float* w1, const float* g1, const float* h0,
                        const float* alpha, int accumulate, float* dh_in, float* dh0, float* p_film1, float* p_alpha,
                        const float* mlp_next, const float* s_mlp_next, void* a_next, float* p_sm_next, void* stream) {
  auto cb = [](const void* p) { return static_cast<const bf16*>(p); };
  auto b16 = [](void* p) { return static_cast<bf16*>(p); };
  return replay_bwd_pass(B, S, d, H, F, n_blk, h_max, nb_max, info, dh, cb(a_mlp), cb(wd), cb(ug), route_w, b16(dug),
                         cb(wug), dn2, b16(dug_full), u, rstd2, w2, g2, attn, s_attn, du, b16(d_attn), p_film2, p_sa,
                         cb(wo), b16(dy), cb(q), cb(k), cb(v), cb(y), lse, cos_t, sin_t, b16(dqkv), cb(wqkv), dn1,
                         b16(dqkv_full), ht, rstd1, w1, g1, h0, alpha, accumulate, dh_in, dh0, p_film1, p_alpha,
                         mlp_next, s_mlp_next, b16(a_next), p_sm_next, static_cast<hipStream_t>(stream));
}

int rte_replay_param_reduce(int T, int B, int S, int d, const float* p_film1, const float* p_film2,
                            const float* p_sa, const float* p_sm, const float* p_alpha, float* out, void* stream) {
  return replay_param_reduce(T, B, S, d, p_film1, p_film2, p_sa, p_sm, p_alpha, out,
                             static_cast<hipStream_t>(stream));
}

}  // extern "C"
