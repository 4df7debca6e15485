// Consistency loss of the bounded-residual macro operator (rte/macro.py:342-359 over the operator
// of rte/macro.py:201-236, default options, hidden rank 32), fused for sequences of at most 64
// positions and d = 256 or 512:
//
//   loss = mean over pairs j, samples, rows, columns of (direct_j - twice_j)^2
//   out_k   = Phi_k(h, h0 = h)            the first application, nf key blocks per sample
//   twice_j = Phi_j(out_{src_lo + j}, h)   the second application, pc key blocks
//   direct_j = out_{dst_lo + j}
//   Phi(x): a = [rmsnorm(x) | h0] @ [V1; V3] + mean_s(rmsnorm(x)) @ V2,
//           out = x + c scale tanh(gain x + silu(a) @ U + bias)
//
// One workgroup (8 waves) owns 32 rows of one sample (half of a 64-position sample): the only
// couplings between its rows and the other half's are the pooled means over the sample (forward)
// and the sums over the sample of da (backward), which cross the kernel boundaries below as small
// per-half partials.  Every [rows x d] quantity of the workgroup lives in registers in the
// transposed MFMA layout (lane l of wave w: row l % 32, the 16 CPW columns of
// 32 (w CPW + cb) + 8 (r / 4) + 4 (l / 32) + r % 4, register r of column block cb), so that
//   * row x rank products (silu(a) @ U, da @ V) are v_mfma_f32_32x32x16_bf16 with the weight
//     rows as the first operand and a [32 x 32] rank tile from LDS as the second, their
//     accumulators landing in that same layout, and
//   * column reductions (x @ V, dz @ U^T) take the register tile itself as the second operand
//     (a lane's 8 k values of a 16-column step are columns 4 h .. +3 and 8 + 4 h .. +3) against
//     weight rows stored with the middle two quads of every 16 columns swapped (VqT, Uq), the
//     eight waves' partial sums added in wave order through LDS.
// Nothing of width d is re-read between the products of one kernel; out, Phi_s(out) and their
// gradients are recomputed from h and the rank-32 codes instead of being stored.
//
//   forward : stats (rmsnorm(h) and its per-half column sums), fwd1 (first application codes a,
//             the second application's inputs and their column sums), fwd2 (second application
//             codes, the MSE per workgroup), then the fixed-order loss sum
//   backward: bwd1 (second application: du, table partials, da), bwd2 (its input gradient, the
//             first application's du / da / table partials, dh without the first application's
//             pooled term), bwd3 (that term: dh += rstd (m - n <m, n> / d), m = sum_s da @ V2^T / S)
//
// The weight gradients are left to the grouped reductions of the fused operator
// (macro_fused_wgrad): this file writes their operands in that pass's layouts (x2, pooled, silu(a),
// du, da, sum_s da, per-tile table sums).  No atomics: every sum has a fixed order.
#include "common.hpp"

#include <type_traits>

namespace rte {

int macro_fused_sum(const float* part, int n, float inv_n, float* out, hipStream_t s);

namespace {

constexpr int kR = 32;         // hidden rank
constexpr int kThr = 512;      // 8 waves
constexpr int kRows = 32;      // rows per workgroup
constexpr int kP = 40;         // LDS pitch (bf16) of a [32][32] rank tile
constexpr int kMaxKeys = 4;    // key blocks per application
constexpr int kMaxD = 512;

__device__ __forceinline__ f32x16_v mfma(bf16x8_v a, bf16x8_v b, f32x16_v c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ bf16x8_v ld8b(const bf16* p) { return *reinterpret_cast<const bf16x8_v*>(p); }

__device__ __forceinline__ f32x16_v zero16() {
  f32x16_v z;
#pragma unroll
  for (int i = 0; i < 16; ++i) z[i] = 0.0f;
  return z;
}

__device__ __forceinline__ bf16x8_v pack8(const float* v) {
  uint4 u;
  u.x = pack_bf2(v[0], v[1]);
  u.y = pack_bf2(v[2], v[3]);
  u.z = pack_bf2(v[4], v[5]);
  u.w = pack_bf2(v[6], v[7]);
  return __builtin_bit_cast(bf16x8_v, u);
}

// tanh in fp32 (the fused operator's form): odd Taylor polynomial below 0.25, else
// 1 - 2 / (e^(2|x|) + 1) with the sign of x; about 2e-7 relative error.
__device__ __forceinline__ float tanh_fast(float x) {
  const float a = fabsf(x), x2 = x * x;
  const float small = x + x * x2 * (-0.333333333f + x2 * (0.133333333f + x2 * (-0.0539682540f + x2 * 0.0218694885f)));
  const float big = copysignf(1.0f - 2.0f * __builtin_amdgcn_rcpf(__expf(2.0f * a) + 1.0f), x);
  return a < 0.25f ? small : big;  // both evaluated: no divergent branch per element
}

__device__ __forceinline__ float sigmoid_fast(float x) { return 1.0f / (1.0f + __expf(-x)); }

__device__ __forceinline__ int64_t clamp_key(int64_t k, int G) { return k < 0 ? 0 : (k >= G ? G - 1 : k); }

// base + a 32-bit byte offset: the (workgroup-uniform) base stays in scalar registers and each
// lane adds one 32-bit offset
template <typename T>
__device__ __forceinline__ T* at(T* base, uint32_t byte_off) {
  using C = typename std::conditional<std::is_const<T>::value, const char, char>::type;
  return reinterpret_cast<T*>(reinterpret_cast<C*>(base) + byte_off);
}

struct McArgs {
  const float* h;
  int b, S, d, nh, G, nf, pc, src_lo, dst_lo;
  float eps, c, mul;
  const int64_t* kf;   // [nf b] keys of the first application (block k, sample i at k b + i)
  const int64_t* ks;   // [pc b] keys of the second application
  const bf16* Vb;      // [G][3d][32]
  const bf16* VqT;     // [G][32][2d]  [V1 | V3]^T, middle quads of every 16 columns swapped
  const bf16* UT;      // [G][d][32]
  const bf16* Uq;      // [G][32][d]   U, middle quads swapped
  const float* gain;
  const float* bias;
  const float* scale;  // [G][d] each
  bf16* x2;            // [(b + pc b) S][2d]
  bf16* pooled;        // [b + pc b][d]
  float* a;            // [(nf b + pc b) S][32]
  bf16* sa;            // same rows, silu(a)
  float* rstd;         // [b S] of h, then [pc b S] of the second application's inputs
  float* ppool;        // [b][nh][d]     column sums of rmsnorm(h) per half
  float* ppool2;       // [pc b][nh][d]  of rmsnorm(out_src)
  float* mse_part;     // [b nh]
  float* loss_out;     // [1] mean of the squared differences
  const float* g;      // upstream gradient of the loss (1 element)
  bf16* du;            // [(nf b + pc b) S][d]
  bf16* da;            // [(nf b + pc b) S][32]
  float* part_tab;     // [nf b + pc b][nh][3][d]
  float* part_da;      // [nf b + pc b][nh][32]
  bf16* dsum;          // [nf b + pc b][32]
  float* dh;           // [b S][d]
};

// Lane context: sample i, half hf (rows s0 .. s0 + nrow), lane row l (clamped copy `row` for loads).
struct Ctx {
  int lane, wave, h, l, hf, s0, nrow, row;
  int64_t i;
  bool ok;
};

__device__ __forceinline__ Ctx make_ctx(int S) {
  Ctx c;
  c.lane = threadIdx.x & 63;
  c.wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  c.h = c.lane >> 5;
  c.l = c.lane & 31;
  c.i = blockIdx.x;
  c.hf = blockIdx.y;
  c.s0 = c.hf * kRows;
  c.nrow = min(kRows, S - c.s0);
  c.ok = c.l < c.nrow;
  c.row = c.ok ? c.l : c.nrow - 1;
  return c;
}

// first column of the lane's 4-column group q of column block cb
template <int CPW>
__device__ __forceinline__ int gcol(const Ctx& c, int cb, int q) {
  return (c.wave * CPW + cb) * 32 + 8 * q + 4 * c.h;
}

// register tile of rows [s0, s0 + 32) of an fp32 matrix with row pitch d
template <int CPW>
__device__ __forceinline__ void load_tile(const float* base, int d, const Ctx& c, float (&x)[CPW][16]) {
  const uint32_t off = (uint32_t)(c.row * d + 4 * c.h) * 4u;
#pragma unroll
  for (int cb = 0; cb < CPW; ++cb)
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const float4 v = *at(reinterpret_cast<const float4*>(base + (c.wave * CPW + cb) * 32 + 8 * q), off);
      x[cb][4 * q] = v.x;
      x[cb][4 * q + 1] = v.y;
      x[cb][4 * q + 2] = v.z;
      x[cb][4 * q + 3] = v.w;
    }
}

// the lane's 16 CPW values of a [d] vector in LDS
template <int CPW>
__device__ __forceinline__ void lds_vec(const float* v, const Ctx& c, float (&x)[CPW][16]) {
#pragma unroll
  for (int cb = 0; cb < CPW; ++cb)
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const float4 t = *reinterpret_cast<const float4*>(v + gcol<CPW>(c, cb, q));
      x[cb][4 * q] = t.x;
      x[cb][4 * q + 1] = t.y;
      x[cb][4 * q + 2] = t.z;
      x[cb][4 * q + 3] = t.w;
    }
}

// bf16 row [lo | hi] of x2 (row pitch 2d): lo = a, hi = b
// rows [s0, s0 + 32) of x2 from `blk` (row s0) on, row pitch 2d; lanes past the half do not store
template <int CPW>
__device__ __forceinline__ void store_x2(bf16* blk, int d, const Ctx& c, const float (&a)[CPW][16],
                                         const float (&b)[CPW][16]) {
  if (!c.ok) return;
  const uint32_t off = (uint32_t)(c.l * 2 * d + 4 * c.h) * 2u;
#pragma unroll
  for (int cb = 0; cb < CPW; ++cb)
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      bf16* row = at(blk + (c.wave * CPW + cb) * 32 + 8 * q, off);
      uint2 u, v;
      u.x = pack_bf2(a[cb][4 * q], a[cb][4 * q + 1]);
      u.y = pack_bf2(a[cb][4 * q + 2], a[cb][4 * q + 3]);
      v.x = pack_bf2(b[cb][4 * q], b[cb][4 * q + 1]);
      v.y = pack_bf2(b[cb][4 * q + 2], b[cb][4 * q + 3]);
      *reinterpret_cast<uint2*>(row) = u;
      *reinterpret_cast<uint2*>(row + d) = v;
    }
}

// rows [s0, s0 + 32) of a bf16 [., d] matrix from `blk` (row s0) on
template <int CPW>
__device__ __forceinline__ void store_bf16_rows(bf16* blk, int d, const Ctx& c, const float (&a)[CPW][16]) {
  if (!c.ok) return;
  const uint32_t off = (uint32_t)(c.l * d + 4 * c.h) * 2u;
#pragma unroll
  for (int cb = 0; cb < CPW; ++cb)
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      uint2 u;
      u.x = pack_bf2(a[cb][4 * q], a[cb][4 * q + 1]);
      u.y = pack_bf2(a[cb][4 * q + 2], a[cb][4 * q + 3]);
      *at(reinterpret_cast<uint2*>(blk + (c.wave * CPW + cb) * 32 + 8 * q), off) = u;
    }
}

// rows [s0, s0 + 32) of an fp32 [., d] matrix from `blk` (row s0) on
template <int CPW>
__device__ __forceinline__ void store_f32_rows(float* blk, int d, const Ctx& c, const float (&a)[CPW][16]) {
  if (!c.ok) return;
  const uint32_t off = (uint32_t)(c.l * d + 4 * c.h) * 4u;
#pragma unroll
  for (int cb = 0; cb < CPW; ++cb)
#pragma unroll
    for (int q = 0; q < 4; ++q)
      *at(reinterpret_cast<float4*>(blk + (c.wave * CPW + cb) * 32 + 8 * q), off) =
          make_float4(a[cb][4 * q], a[cb][4 * q + 1], a[cb][4 * q + 2], a[cb][4 * q + 3]);
}

// Sum over the row's d columns: the lane pair (l, l + 32), then the 8 waves in order.  buf
// [8][32]: two consecutive calls must use different buffers (the barrier inside one call orders
// the other buffer's reads before its next writes).
__device__ __forceinline__ float row_total(float v, float* buf, const Ctx& c) {
  v += __shfl_xor(v, 32, 64);
  if (c.h == 0) buf[c.wave * 32 + c.l] = v;
  __syncthreads();
  float s = 0.0f;
#pragma unroll
  for (int w = 0; w < 8; ++w) s += buf[w * 32 + c.l];
  return s;
}

typedef float v32f __attribute__((ext_vector_type(32)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef float v8f __attribute__((ext_vector_type(8)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef float v2f __attribute__((ext_vector_type(2)));

// Lanes whose bit `bit` (1, 2, ..., 32) of the lane index is set
__device__ __forceinline__ constexpr uint64_t lane_mask(int bit) {
  return bit == 1 ? 0xAAAAAAAAAAAAAAAAull
                  : (bit == 2 ? 0xCCCCCCCCCCCCCCCCull
                              : (bit == 4 ? 0xF0F0F0F0F0F0F0F0ull
                                          : (bit == 8 ? 0xFF00FF00FF00FF00ull
                                                      : (bit == 16 ? 0xFFFF0000FFFF0000ull : 0xFFFFFFFF00000000ull))));
}

// m[lane] ? t : f as one v_cndmask_b32: an opaque select, so the compiler cannot turn a select
// between two elements of one register array into a lane-dependent index (a chain of compares)
__device__ __forceinline__ float vsel(uint64_t m, float t, float f) {
  float r;
  asm("v_cndmask_b32_e64 %0, %1, %2, %3" : "=v"(r) : "v"(f), "v"(t), "s"(m));
  return r;
}

// One butterfly step over lane bit BIT: a lane keeps the half of its values its bit selects and
// adds the partner's copy of that half
template <typename VO, int H, int BIT, typename VI>
__device__ __forceinline__ VO bstep(const VI& v) {
  VO o;
  constexpr uint64_t m = lane_mask(BIT);
#pragma unroll
  for (int k = 0; k < H; ++k) {
    const float keep = vsel(m, v[k + H], v[k]);
    const float give = vsel(m, v[k], v[k + H]);
    o[k] = keep + __shfl_xor(give, BIT, 64);
  }
  return o;
}

// Sum over the 32 lanes of each lane half: lane l gets the sum over its half of v[l % 16], lanes
// l and l ^ 16 holding the same sum
__device__ __forceinline__ float butterfly16(const v16f& v) {
  const v8f a = bstep<v8f, 8, 8>(v);
  const v4f b = bstep<v4f, 4, 4>(a);
  const v2f c = bstep<v2f, 2, 2>(b);
  const float r = vsel(lane_mask(1), c[1], c[0]) + __shfl_xor(vsel(lane_mask(1), c[0], c[1]), 1, 64);
  return r + __shfl_xor(r, 16, 64);
}

// ... of v[l % 32] (lane bits 4..0)
__device__ __forceinline__ float butterfly32(const v32f& v) {
  const v16f a = bstep<v16f, 16, 16>(v);
  const v8f b = bstep<v8f, 8, 8>(a);
  const v4f c = bstep<v4f, 4, 4>(b);
  const v2f e = bstep<v2f, 2, 2>(c);
  return vsel(lane_mask(1), e[1], e[0]) + __shfl_xor(vsel(lane_mask(1), e[0], e[1]), 1, 64);
}

// Column sums over the 32 rows of each lane half of a register tile
template <int CPW>
__device__ __forceinline__ float col_sum(const float (&x)[CPW][16], int lane) {
  if constexpr (CPW == 2) {
    v32f v;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      v[r] = x[0][r];
      v[16 + r] = x[1][r];
    }
    return butterfly32(v);
  } else {
    v16f v;
#pragma unroll
    for (int r = 0; r < 16; ++r) v[r] = x[0][r];
    return butterfly16(v);
  }
}

// column of the lane's col_sum result, and whether this lane writes it
template <int CPW>
__device__ __forceinline__ int col_sum_col(const Ctx& c) {
  const int f = c.l & (16 * CPW - 1);
  const int cb = f >> 4, r = f & 15;
  return (c.wave * CPW + cb) * 32 + 8 * (r >> 2) + 4 * c.h + (r & 3);
}

template <int CPW>
__device__ __forceinline__ bool col_sum_writer(const Ctx& c) {
  return CPW == 2 || (c.l & 16) == 0;
}

// Column sums over the half's rows of one column block (16 values, consumed) into pt[column]
// (column 32 cbg + 8 (r / 4) + 4 h + r % 4 of register r = l % 16, written by lanes l % 32 < 16)
__device__ __forceinline__ void put_block_sum(const v16f& v, const Ctx& c, int cbg, float* pt) {
  const float s = butterfly16(v);
  const int r = c.l & 15;
  if ((c.l & 16) == 0) pt[cbg * 32 + 8 * (r >> 2) + 4 * c.h + (r & 3)] = s;
}

// column block cbg of (rank tile @ W^T), W [d][32] rows of a weight (UT for silu(a) @ U, a V
// part of Vb for da @ V^T), the rank tile [32][kP] in LDS
__device__ __forceinline__ f32x16_v expand_blk(const bf16* W, const bf16* tile, int cbg, const Ctx& c) {
  const bf16x8_v s0 = ld8b(tile + c.l * kP + 8 * c.h), s1 = ld8b(tile + c.l * kP + 16 + 8 * c.h);
  const bf16* ap = at(W + cbg * 32 * kR, (uint32_t)(c.l * kR + 8 * c.h) * 2u);
  f32x16_v acc = zero16();
  acc = mfma(ld8b(ap), s0, acc);
  return mfma(ld8b(ap + 16), s1, acc);
}

// acc += this wave's column block cbg of z @ Wq^T, z given as 16 register values (the block's
// 16-column steps are registers 0..7 and 8..15), Wq quad-swapped rows [rank][ld]
__device__ __forceinline__ void reduce_blk(f32x16_v& acc, const bf16* Wq, int ld, const v16f& z, int cbg,
                                           const Ctx& c) {
  const uint32_t off = (uint32_t)(c.l * ld + 8 * c.h) * 2u;
  uint4 u0, u1;
  u0.x = pack_bf2(z[0], z[1]);
  u0.y = pack_bf2(z[2], z[3]);
  u0.z = pack_bf2(z[4], z[5]);
  u0.w = pack_bf2(z[6], z[7]);
  u1.x = pack_bf2(z[8], z[9]);
  u1.y = pack_bf2(z[10], z[11]);
  u1.z = pack_bf2(z[12], z[13]);
  u1.w = pack_bf2(z[14], z[15]);
  acc = mfma(ld8b(at(Wq + cbg * 32, off)), __builtin_bit_cast(bf16x8_v, u0), acc);
  acc = mfma(ld8b(at(Wq + cbg * 32 + 16, off)), __builtin_bit_cast(bf16x8_v, u1), acc);
}

// 16 bf16 of one column block to rows [s0, s0 + 32) of a [., d] matrix from blk (row s0) on
__device__ __forceinline__ void store_blk_bf16(bf16* blk, int d, const Ctx& c, int cbg, const v16f& v) {
  if (!c.ok) return;
  const uint32_t off = (uint32_t)(c.l * d + 4 * c.h) * 2u;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    uint2 u;
    u.x = pack_bf2(v[4 * q], v[4 * q + 1]);
    u.y = pack_bf2(v[4 * q + 2], v[4 * q + 3]);
    *at(reinterpret_cast<uint2*>(blk + cbg * 32 + 8 * q), off) = u;
  }
}

__device__ __forceinline__ float4 ld4(const float* p) { return *reinterpret_cast<const float4*>(p); }
__device__ __forceinline__ float f4(const float4& v, int j) { return j == 0 ? v.x : (j == 1 ? v.y : (j == 2 ? v.z : v.w)); }

// [rows x d] tile = rank tile (LDS [32][kP], row l, ranks) @ W^T with W [d][32] rows of the
// weight (UT for silu(a) @ U, a V part of Vb for da @ V^T)
template <int CPW>
__device__ __forceinline__ void rank_expand(float (&o)[CPW][16], const bf16* W, const bf16* tile, const Ctx& c) {
  const bf16x8_v s0 = ld8b(tile + c.l * kP + 8 * c.h), s1 = ld8b(tile + c.l * kP + 16 + 8 * c.h);
  const uint32_t off = (uint32_t)(c.l * kR + 8 * c.h) * 2u;
#pragma unroll
  for (int cb = 0; cb < CPW; ++cb) {
    const bf16* ap = at(W + (c.wave * CPW + cb) * 32 * kR, off);
    f32x16_v acc = zero16();
    acc = mfma(ld8b(ap), s0, acc);
    acc = mfma(ld8b(ap + 16), s1, acc);
#pragma unroll
    for (int r = 0; r < 16; ++r) o[cb][r] = acc[r];
  }
}

// this wave's partial of x @ W over its columns, W given as quad-swapped rows Wq[rank][d]
// (pitch ld): acc[r] = sum over the wave's columns of Wq[rank][.] x[l][.], rank = 8 (r / 4) + 4 h + r % 4
template <int CPW>
__device__ __forceinline__ void col_reduce(f32x16_v& acc, const bf16* Wq, int ld, const bf16x8_v (&xb)[CPW][2],
                                           const Ctx& c) {
  const uint32_t off = (uint32_t)(c.l * ld + 8 * c.h) * 2u;
#pragma unroll
  for (int cb = 0; cb < CPW; ++cb)
#pragma unroll
    for (int t = 0; t < 2; ++t) acc = mfma(ld8b(at(Wq + (c.wave * CPW + cb) * 32 + 16 * t, off)), xb[cb][t], acc);
}

template <int CPW>
__device__ __forceinline__ void frags(const float (&x)[CPW][16], bf16x8_v (&xb)[CPW][2]) {
#pragma unroll
  for (int cb = 0; cb < CPW; ++cb) {
    xb[cb][0] = pack8(&x[cb][0]);
    xb[cb][1] = pack8(&x[cb][8]);
  }
}

// the waves' partials [8][32 rows][33] of a column reduction
__device__ __forceinline__ void stash_partial(float* part, const f32x16_v& acc, const Ctx& c) {
#pragma unroll
  for (int r = 0; r < 16; ++r) part[(c.wave * 32 + c.l) * 33 + 8 * (r >> 2) + 4 * c.h + (r & 3)] = acc[r];
}

__device__ __forceinline__ float sum_partial(const float* part, int row, int n) {
  float s = 0.0f;
#pragma unroll
  for (int w = 0; w < 8; ++w) s += part[(w * 32 + row) * 33 + n];
  return s;
}

// For each of the lane's cells: th = tanh(gain x + low + bias), out = x + c scale th with
// low = (rank tile @ W^T) (W: UT of the key, [d][32]) and the key's tables in LDS [3][d] (gain | bias
// | scale), computed one column block at a time; sink(cb, r, out, th, gain, scale) consumes them.
template <int CPW, typename F>
__device__ __forceinline__ void phi_apply(const bf16* W, const bf16* tile, const float* tab, int d, float cc,
                                          const Ctx& c, const float (&x)[CPW][16], F&& sink) {
  const bf16x8_v s0 = ld8b(tile + c.l * kP + 8 * c.h), s1 = ld8b(tile + c.l * kP + 16 + 8 * c.h);
  const uint32_t off = (uint32_t)(c.l * kR + 8 * c.h) * 2u;
#pragma unroll
  for (int cb = 0; cb < CPW; ++cb) {
    const bf16* ap = at(W + (c.wave * CPW + cb) * 32 * kR, off);
    f32x16_v acc = zero16();
    acc = mfma(ld8b(ap), s0, acc);
    acc = mfma(ld8b(ap + 16), s1, acc);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int col = gcol<CPW>(c, cb, q);
      const float4 gn = *reinterpret_cast<const float4*>(tab + col);
      const float4 bs = *reinterpret_cast<const float4*>(tab + d + col);
      const float4 sc = *reinterpret_cast<const float4*>(tab + 2 * d + col);
      const float g4[4] = {gn.x, gn.y, gn.z, gn.w}, b4[4] = {bs.x, bs.y, bs.z, bs.w}, s4[4] = {sc.x, sc.y, sc.z, sc.w};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int r = 4 * q + j;
        const float th = tanh_fast(g4[j] * x[cb][r] + acc[r] + b4[j]);
        sink(cb, r, x[cb][r] + cc * s4[j] * th, th, g4[j], s4[j]);
      }
    }
  }
}

template <int CPW>
__device__ __forceinline__ void phi_out(float (&o)[CPW][16], const bf16* W, const bf16* tile, const float* tab, int d,
                                        float cc, const Ctx& c, const float (&x)[CPW][16]) {
  phi_apply<CPW>(W, tile, tab, d, cc, c, x, [&](int cb, int r, float out, float, float, float) { o[cb][r] = out; });
}

// tables of key g into LDS [3][d]
__device__ __forceinline__ void load_tab(float* dst, const McArgs& p, int64_t g) {
  for (int e = threadIdx.x; e < p.d; e += kThr) {
    dst[e] = p.gain[g * p.d + e];
    dst[p.d + e] = p.bias[g * p.d + e];
    dst[2 * p.d + e] = p.scale[g * p.d + e];
  }
}

// a bf16 [32][32] rank tile (rows s0 .. of sample row block) into LDS (rows past nrow: zeros)
__device__ __forceinline__ void load_rank_tile(bf16* dst, const bf16* src, int64_t row0, int nrow) {
  for (int e = threadIdx.x; e < kRows * 4; e += kThr) {
    const int row = e >> 2, q = e & 3;
    uint4 v = make_uint4(0u, 0u, 0u, 0u);
    if (row < nrow) v = *reinterpret_cast<const uint4*>(src + (row0 + row) * kR + 8 * q);
    *reinterpret_cast<uint4*>(dst + row * kP + 8 * q) = v;
  }
}

// P[n] = pooled @ V2_g for pooled in LDS pm[d]: thread t takes ranks 8 (t % 4) .. +7 of the
// columns t / 4 + 128 m (16-byte weight loads), each wave adds its 16 column groups (butterfly
// over lane bits 5..2), pv [8][32] gets the wave sums; pooled_v2_total adds the waves in order
// (after a barrier).
__device__ __forceinline__ void pooled_v2_part(float* pv, const float* pm, const McArgs& p, int64_t g) {
  const int t = threadIdx.x, lane = t & 63, o = t & 3;
  const bf16* w = p.Vb + (g * 3 * p.d + p.d) * kR + 8 * o;
  v8f v = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll 4
  for (int col = t >> 2; col < p.d; col += kThr / 4) {
    const uint4 u = *reinterpret_cast<const uint4*>(w + (int64_t)col * kR);
    const float pmv = pm[col];
    const uint32_t wd[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v[2 * i] += pmv * __uint_as_float(wd[i] << 16);
      v[2 * i + 1] += pmv * __uint_as_float(wd[i] & 0xffff0000u);
    }
  }
  const v4f v4 = bstep<v4f, 4, 32>(v);
  const v2f v2 = bstep<v2f, 2, 16>(v4);
  const float v1 = vsel(lane_mask(8), v2[1], v2[0]) + __shfl_xor(vsel(lane_mask(8), v2[0], v2[1]), 8, 64);
  const float r = v1 + __shfl_xor(v1, 4, 64);
  const int i = ((lane >> 5) & 1) * 4 + ((lane >> 4) & 1) * 2 + ((lane >> 3) & 1);
  if ((lane & 4) == 0) pv[(t >> 6) * 32 + 8 * o + i] = r;
}

__device__ __forceinline__ float pooled_v2_total(const float* pv, int n) {
  float s = 0.0f;
#pragma unroll
  for (int w = 0; w < 8; ++w) s += pv[w * 32 + n];
  return s;
}

// ------------------------------------------------------------------ forward

// rstd of h, x2 = [bf16(rmsnorm(h)) | bf16(h)], per-half column sums of rmsnorm(h)
template <int CPW>
__global__ void __launch_bounds__(kThr) mc_stats_kernel(McArgs p) {
  __shared__ float rsum[8 * 32];
  const Ctx c = make_ctx(p.S);
  const int d = p.d;
  const int64_t rb = c.i * p.S + c.s0;
  float x[CPW][16];
  load_tile<CPW>(p.h + rb * d, d, c, x);
  float ss = 0.0f;
#pragma unroll
  for (int cb = 0; cb < CPW; ++cb)
#pragma unroll
    for (int r = 0; r < 16; ++r) ss += x[cb][r] * x[cb][r];
  const float rs = rsqrtf(row_total(ss, rsum, c) / (float)d + p.eps);
  if (c.h == 0 && c.ok) p.rstd[rb + c.l] = rs;
  float n[CPW][16];
#pragma unroll
  for (int cb = 0; cb < CPW; ++cb)
#pragma unroll
    for (int r = 0; r < 16; ++r) n[cb][r] = x[cb][r] * rs;
  store_x2<CPW>(p.x2 + rb * 2 * d, d, c, n, x);
#pragma unroll
  for (int cb = 0; cb < CPW; ++cb)
#pragma unroll
    for (int r = 0; r < 16; ++r) n[cb][r] = c.ok ? n[cb][r] : 0.0f;
  const float cs = col_sum<CPW>(n, c.lane);
  if (col_sum_writer<CPW>(c)) p.ppool[(c.i * p.nh + c.hf) * d + col_sum_col<CPW>(c)] = cs;
}

struct F1Smem {
  float* part;  // [8][32][33]
  float* rsum;  // [2][8][32]
  float* pm;    // [d]
  float* pv;    // [16][32]
  float* tab;   // [pc][3][d]
  bf16* sat;    // [nf][32][kP]
};

__device__ __forceinline__ F1Smem f1_smem(char* s, int d, int pc) {
  F1Smem m;
  m.part = reinterpret_cast<float*>(s);
  m.rsum = m.part + 8 * 32 * 33;
  m.pm = m.rsum + 2 * 8 * 32;
  m.pv = m.pm + kMaxD;
  m.tab = m.pv + 16 * 32;
  m.sat = reinterpret_cast<bf16*>(m.tab + kMaxKeys * 3 * kMaxD);
  return m;
}

constexpr size_t kF1Lds = (8 * 32 * 33 + 2 * 8 * 32 + kMaxD + 16 * 32 + kMaxKeys * 3 * kMaxD) * 4 +
                          (size_t)kMaxKeys * 32 * kP * 2;

// First application (codes a, silu(a) of every first key), then the second application's inputs
// out_{src_lo + j} = Phi(h): their rstd, x2 rows [bf16(rmsnorm) | bf16(h)] and per-half column sums.
template <int CPW>
__global__ void __launch_bounds__(kThr) mc_fwd1_kernel(McArgs p) {
  extern __shared__ __align__(16) char smem[];
  const F1Smem L = f1_smem(smem, p.d, p.pc);
  const Ctx c = make_ctx(p.S);
  const int d = p.d, tid = threadIdx.x;
  const int64_t rb = c.i * p.S + c.s0;
  float x[CPW][16];
  load_tile<CPW>(p.h + rb * d, d, c, x);
  const float rs = p.rstd[rb + c.row];
  bf16x8_v xn[CPW][2], xh[CPW][2];
  {
    float n[CPW][16];
#pragma unroll
    for (int cb = 0; cb < CPW; ++cb)
#pragma unroll
      for (int r = 0; r < 16; ++r) n[cb][r] = x[cb][r] * rs;
    frags<CPW>(n, xn);
    frags<CPW>(x, xh);
  }
  const float invS = 1.0f / (float)p.S;
  for (int col = tid; col < d; col += kThr) {
    float s = 0.0f;
    for (int q = 0; q < p.nh; ++q) s += p.ppool[(c.i * p.nh + q) * d + col];
    const bf16 pb = f2bf(s * invS);
    L.pm[col] = bf2f(pb);
    if (c.hf == 0) p.pooled[c.i * d + col] = pb;
  }
  for (int j = 0; j < p.pc; ++j) load_tab(L.tab + j * 3 * d, p, clamp_key(p.kf[(p.src_lo + j) * p.b + c.i], p.G));
  __syncthreads();
  for (int k = 0; k < p.nf; ++k) {
    const int64_t smp = k * p.b + c.i;
    const int64_t g = clamp_key(p.kf[smp], p.G);
    pooled_v2_part(L.pv, L.pm, p, g);
    f32x16_v acc = zero16();
    const bf16* wq = p.VqT + g * kR * 2 * d;
    col_reduce<CPW>(acc, wq, 2 * d, xn, c);
    col_reduce<CPW>(acc, wq + d, 2 * d, xh, c);
    stash_partial(L.part, acc, c);
    __syncthreads();
    for (int e = tid; e < kRows * kR; e += kThr) {
      const int row = e >> 5, n = e & 31;
      const float av = sum_partial(L.part, row, n) + pooled_v2_total(L.pv, n);
      const bf16 sb = f2bf(av * sigmoid_fast(av));
      if (row < c.nrow) {
        const int64_t gr = smp * p.S + c.s0 + row;
        p.a[gr * kR + n] = av;
        p.sa[gr * kR + n] = sb;
      }
      L.sat[(k * 32 + row) * kP + n] = sb;
    }
    __syncthreads();
  }
  for (int j = 0; j < p.pc; ++j) {
    const int k = p.src_lo + j;
    const int64_t g = clamp_key(p.kf[k * p.b + c.i], p.G);
    float y[CPW][16];
    phi_out<CPW>(y, p.UT + g * d * kR, L.sat + k * 32 * kP, L.tab + j * 3 * d, d, p.c, c, x);
    float ss = 0.0f;
#pragma unroll
    for (int cb = 0; cb < CPW; ++cb)
#pragma unroll
      for (int r = 0; r < 16; ++r) ss += y[cb][r] * y[cb][r];
    const float ry = rsqrtf(row_total(ss, L.rsum + (j & 1) * 256, c) / (float)d + p.eps);
    const int64_t s2 = (int64_t)j * p.b + c.i;  // second-application sample
    if (c.h == 0 && c.ok) p.rstd[(int64_t)p.b * p.S + s2 * p.S + c.s0 + c.l] = ry;
#pragma unroll
    for (int cb = 0; cb < CPW; ++cb)
#pragma unroll
      for (int r = 0; r < 16; ++r) y[cb][r] *= ry;
    store_x2<CPW>(p.x2 + ((int64_t)p.b * p.S + s2 * p.S + c.s0) * 2 * d, d, c, y, x);
#pragma unroll
    for (int cb = 0; cb < CPW; ++cb)
#pragma unroll
      for (int r = 0; r < 16; ++r) y[cb][r] = c.ok ? y[cb][r] : 0.0f;
    const float cs = col_sum<CPW>(y, c.lane);
    if (col_sum_writer<CPW>(c)) p.ppool2[(s2 * p.nh + c.hf) * d + col_sum_col<CPW>(c)] = cs;
  }
}

struct F2Smem {
  float* part;  // [8][32][33]
  float* rsum;  // [8][32]
  float* pm;    // [d]
  float* pv;    // [16][32]
  float* tab;   // [3 slots: src, second, dst][3][d]
  bf16* st;     // [3 tiles: src, second, dst][32][kP]
  float* red;   // [8]
};

__device__ __forceinline__ F2Smem f2_smem(char* s) {
  F2Smem m;
  m.part = reinterpret_cast<float*>(s);
  m.rsum = m.part + 8 * 32 * 33;
  m.pm = m.rsum + 8 * 32;
  m.pv = m.pm + kMaxD;
  m.tab = m.pv + 16 * 32;
  m.red = m.tab + 3 * 3 * kMaxD;
  m.st = reinterpret_cast<bf16*>(m.red + 8);
  return m;
}

constexpr size_t kF2Lds = (8 * 32 * 33 + 8 * 32 + kMaxD + 16 * 32 + 3 * 3 * kMaxD + 8) * 4 + (size_t)3 * 32 * kP * 2;

// out_src (recomputed as in fwd1), the second application's codes, twice, direct = out_dst and
// the workgroup's sum of (twice - direct)^2 over every pair (waves in order)
template <int CPW>
__global__ void __launch_bounds__(kThr) mc_fwd2_kernel(McArgs p) {
  extern __shared__ __align__(16) char smem[];
  const F2Smem L = f2_smem(smem);
  const Ctx c = make_ctx(p.S);
  const int d = p.d, tid = threadIdx.x;
  const int64_t rb = c.i * p.S + c.s0;
  float x[CPW][16];
  load_tile<CPW>(p.h + rb * d, d, c, x);
  bf16x8_v xh[CPW][2];
  frags<CPW>(x, xh);
  const float invS = 1.0f / (float)p.S;
  float mse = 0.0f;
  for (int j = 0; j < p.pc; ++j) {
    const int64_t sm_s = (int64_t)(p.src_lo + j) * p.b + c.i, sm_d = (int64_t)(p.dst_lo + j) * p.b + c.i;
    const int64_t s2 = (int64_t)j * p.b + c.i, sm2 = (int64_t)p.nf * p.b + s2;
    const int64_t gs = clamp_key(p.kf[sm_s], p.G), gd = clamp_key(p.kf[sm_d], p.G), g2 = clamp_key(p.ks[s2], p.G);
    if (j > 0) __syncthreads();  // the previous pair's LDS reads are done
    load_tab(L.tab, p, gs);
    load_tab(L.tab + 3 * d, p, g2);
    load_tab(L.tab + 6 * d, p, gd);
    load_rank_tile(L.st, p.sa, sm_s * p.S + c.s0, c.nrow);
    load_rank_tile(L.st + 2 * 32 * kP, p.sa, sm_d * p.S + c.s0, c.nrow);
    for (int col = tid; col < d; col += kThr) {
      float s = 0.0f;
      for (int q = 0; q < p.nh; ++q) s += p.ppool2[(s2 * p.nh + q) * d + col];
      const bf16 pb = f2bf(s * invS);
      L.pm[col] = bf2f(pb);
      if (c.hf == 0) p.pooled[((int64_t)p.b + s2) * d + col] = pb;
    }
    __syncthreads();
    pooled_v2_part(L.pv, L.pm, p, g2);
    float y[CPW][16];
    phi_out<CPW>(y, p.UT + gs * d * kR, L.st, L.tab, d, p.c, c, x);
    const float ry = p.rstd[(int64_t)p.b * p.S + s2 * p.S + c.s0 + c.row];
    {
      float n[CPW][16];
#pragma unroll
      for (int cb = 0; cb < CPW; ++cb)
#pragma unroll
        for (int r = 0; r < 16; ++r) n[cb][r] = y[cb][r] * ry;
      bf16x8_v xn[CPW][2];
      frags<CPW>(n, xn);
      f32x16_v acc = zero16();
      const bf16* wq = p.VqT + g2 * kR * 2 * d;
      col_reduce<CPW>(acc, wq, 2 * d, xn, c);
      col_reduce<CPW>(acc, wq + d, 2 * d, xh, c);
      stash_partial(L.part, acc, c);
    }
    __syncthreads();
    for (int e = tid; e < kRows * kR; e += kThr) {
      const int row = e >> 5, n = e & 31;
      const float av = sum_partial(L.part, row, n) + pooled_v2_total(L.pv, n);
      const bf16 sb = f2bf(av * sigmoid_fast(av));
      if (row < c.nrow) {
        const int64_t gr = sm2 * p.S + c.s0 + row;
        p.a[gr * kR + n] = av;
        p.sa[gr * kR + n] = sb;
      }
      L.st[(32 + row) * kP + n] = sb;
    }
    __syncthreads();
#pragma unroll
    for (int cb = 0; cb < CPW; ++cb) {  // twice = Phi_2(y), direct = Phi_dst(h), one column block at a time
      const int cbg = c.wave * CPW + cb;
      const f32x16_v lt = expand_blk(p.UT + g2 * d * kR, L.st + 32 * kP, cbg, c);
      const f32x16_v lr = expand_blk(p.UT + gd * d * kR, L.st + 2 * 32 * kP, cbg, c);
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int col = gcol<CPW>(c, cb, q);
        const float4 g2v = ld4(L.tab + 3 * d + col), b2v = ld4(L.tab + 4 * d + col), s2v = ld4(L.tab + 5 * d + col);
        const float4 gdv = ld4(L.tab + 6 * d + col), bdv = ld4(L.tab + 7 * d + col), sdv = ld4(L.tab + 8 * d + col);
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) {
          const int r = 4 * q + jj;
          const float xv = x[cb][r], yv = y[cb][r];
          const float dr = xv + p.c * f4(sdv, jj) * tanh_fast(f4(gdv, jj) * xv + lr[r] + f4(bdv, jj));
          const float tw = yv + p.c * f4(s2v, jj) * tanh_fast(f4(g2v, jj) * yv + lt[r] + f4(b2v, jj));
          const float df = tw - dr;
          mse += c.ok ? df * df : 0.0f;
        }
      }
    }
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) mse += __shfl_xor(mse, off, 64);
  if (c.lane == 0) L.red[c.wave] = mse;
  __syncthreads();
  if (tid == 0) {
    float s = 0.0f;
#pragma unroll
    for (int w = 0; w < 8; ++w) s += L.red[w];
    p.mse_part[c.i * p.nh + c.hf] = s;
  }
}

// ------------------------------------------------------------------ backward

struct BSmem {
  float* part;   // [8][32][33]
  float* rsum;   // [2][8][32]
  float* tab;    // [nf + pc][3][d]: first keys, then second keys
  bf16* sat;     // [nf][32][kP]  silu(a) of the first keys
  bf16* sat2;    // [pc][32][kP]  of the second keys
  bf16* dat;     // [nf][32][kP]  da of the first keys
  bf16* dat2;    // [pc][32][kP]  of the second keys
  float* al;     // [32][33]      a of the key being differentiated, then its da
  float* mv;     // [pc][d]       sum_s da @ V2^T / S of the second keys
  float* sv;     // [kMaxKeys][32] sum_s da / S
};

__device__ __forceinline__ BSmem b_smem(char* s) {
  BSmem m;
  m.part = reinterpret_cast<float*>(s);
  m.rsum = m.part + 8 * 32 * 33;
  m.tab = m.rsum + 2 * 8 * 32;
  m.al = m.tab + 2 * kMaxKeys * 3 * kMaxD;
  m.mv = m.al + 32 * 33;
  m.sv = m.mv + kMaxKeys * kMaxD;
  m.sat = reinterpret_cast<bf16*>(m.sv + kMaxKeys * 32);
  m.sat2 = m.sat + kMaxKeys * 32 * kP;
  m.dat = m.sat2 + kMaxKeys * 32 * kP;
  m.dat2 = m.dat + kMaxKeys * 32 * kP;
  return m;
}

constexpr size_t kBLds = (8 * 32 * 33 + 2 * 8 * 32 + 2 * kMaxKeys * 3 * kMaxD + 32 * 33 + kMaxKeys * kMaxD +
                          kMaxKeys * 32) * 4 + (size_t)4 * kMaxKeys * 32 * kP * 2;

// tables and silu(a) tiles of both applications' keys into LDS (first keys, then second keys)
__device__ __forceinline__ void b_stage(const BSmem& L, const McArgs& p, const Ctx& c) {
  for (int k = 0; k < p.nf; ++k) {
    const int64_t smp = k * p.b + c.i;
    load_tab(L.tab + k * 3 * p.d, p, clamp_key(p.kf[smp], p.G));
    load_rank_tile(L.sat + k * 32 * kP, p.sa, smp * p.S + c.s0, c.nrow);
  }
  for (int j = 0; j < p.pc; ++j) {
    const int64_t s2 = (int64_t)j * p.b + c.i, sm2 = (int64_t)p.nf * p.b + s2;
    load_tab(L.tab + (p.nf + j) * 3 * p.d, p, clamp_key(p.ks[s2], p.G));
    load_rank_tile(L.sat2 + j * 32 * kP, p.sa, sm2 * p.S + c.s0, c.nrow);
  }
}

// Keys and LDS operands of the second application's pair j
struct Pair {
  int64_t gs, g2, gd;          // keys: first application src block, second application, dst block
  const float *ts, *t2, *td;   // their tables
  const bf16 *ss, *s2, *sd;    // their silu(a) tiles
};

__device__ __forceinline__ Pair pair_of(const McArgs& p, const BSmem& L, const Ctx& c, int j) {
  const int ks_ = p.src_lo + j, kd_ = p.dst_lo + j;
  Pair q;
  q.gs = clamp_key(p.kf[ks_ * p.b + c.i], p.G);
  q.gd = clamp_key(p.kf[kd_ * p.b + c.i], p.G);
  q.g2 = clamp_key(p.ks[(int64_t)j * p.b + c.i], p.G);
  q.ts = L.tab + ks_ * 3 * p.d;
  q.td = L.tab + kd_ * 3 * p.d;
  q.t2 = L.tab + (p.nf + j) * 3 * p.d;
  q.ss = L.sat + ks_ * 32 * kP;
  q.sd = L.sat + kd_ * 32 * kP;
  q.s2 = L.sat2 + j * 32 * kP;
  return q;
}

// Pair j at the 16 cells of column block cbg: y = out_src, gv = coef (twice - direct) (0 on rows
// past the half), th = the second application's tanh; sink(r, y, gv, th, gain2, scale2)
template <typename F>
__device__ __forceinline__ void pair_blk(const McArgs& p, const Pair& q, const Ctx& c, int cbg, const float* x,
                                         float coef, F&& sink) {
  const int d = p.d;
  const f32x16_v ls = expand_blk(p.UT + q.gs * d * kR, q.ss, cbg, c);
  const f32x16_v lr = expand_blk(p.UT + q.gd * d * kR, q.sd, cbg, c);
  const f32x16_v l2 = expand_blk(p.UT + q.g2 * d * kR, q.s2, cbg, c);
#pragma unroll
  for (int qq = 0; qq < 4; ++qq) {
    __builtin_amdgcn_sched_barrier(0);
    const int col = cbg * 32 + 8 * qq + 4 * c.h;
    const float4 gs = ld4(q.ts + col), bs = ld4(q.ts + d + col), ss = ld4(q.ts + 2 * d + col);
    const float4 gd = ld4(q.td + col), bd = ld4(q.td + d + col), sd = ld4(q.td + 2 * d + col);
    const float4 g2 = ld4(q.t2 + col), b2 = ld4(q.t2 + d + col), s2 = ld4(q.t2 + 2 * d + col);
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) {
      const int r = 4 * qq + jj;
      const float xv = x[r];
      const float y = xv + p.c * f4(ss, jj) * tanh_fast(f4(gs, jj) * xv + ls[r] + f4(bs, jj));
      const float dr = xv + p.c * f4(sd, jj) * tanh_fast(f4(gd, jj) * xv + lr[r] + f4(bd, jj));
      const float th = tanh_fast(f4(g2, jj) * y + l2[r] + f4(b2, jj));
      const float tw = y + p.c * f4(s2, jj) * th;
      sink(r, y, c.ok ? coef * (tw - dr) : 0.0f, th, f4(g2, jj), f4(s2, jj));
    }
  }
}

// The key's da from its P3 accumulator (this wave's partial of dz @ U^T): the waves' partials
// added in order, da = (dz @ U^T) silu'(a) to LDS tile `dat`, the global da rows and the half's
// column sums of da
__device__ __forceinline__ void key_finish(const McArgs& p, const BSmem& L, const Ctx& c, int64_t smp,
                                           const f32x16_v& acc, bf16* dat) {
  const int tid = threadIdx.x;
  const int64_t rb = smp * p.S + c.s0;
  for (int e = tid; e < kRows * kR; e += kThr) {  // a of this key (the caller's barrier precedes)
    const int row = e >> 5, n = e & 31;
    L.al[row * 33 + n] = row < c.nrow ? p.a[(rb + row) * kR + n] : 0.0f;
  }
  stash_partial(L.part, acc, c);
  __syncthreads();
  for (int e = tid; e < kRows * kR; e += kThr) {
    const int row = e >> 5, n = e & 31;
    const float av = L.al[row * 33 + n];
    const float sg = sigmoid_fast(av);
    const float dav = row < c.nrow ? sum_partial(L.part, row, n) * sg * (1.0f + av * (1.0f - sg)) : 0.0f;
    const bf16 db = f2bf(dav);
    if (row < c.nrow) p.da[(rb + row) * kR + n] = db;
    dat[row * kP + n] = db;
    L.al[row * 33 + n] = dav;
  }
  __syncthreads();
  if (tid < kR) {  // column sums of da over the half's rows, in row order
    float s = 0.0f;
    for (int row = 0; row < kRows; ++row) s += L.al[row * 33 + tid];
    p.part_da[(smp * p.nh + c.hf) * kR + tid] = s;
  }
  __syncthreads();  // al / part are reused by the next key
}

// One column block of a key's backward given its dz and ps = dout c t (16 values each, rows past
// the half 0; x the application's input): du rows, the table column sums (dz x | dz | ps) into
// pt [3][d], and acc += dz @ U^T (this wave's part).  dz / ps are consumed.
__device__ __forceinline__ void key_blk(const McArgs& p, const Ctx& c, int64_t smp, int64_t g, int cbg,
                                        const float* x, const v16f& dz, const v16f& ps, f32x16_v& acc) {
  const int d = p.d;
  store_blk_bf16(p.du + (smp * p.S + c.s0) * d, d, c, cbg, dz);
  reduce_blk(acc, p.Uq + g * kR * d, d, dz, cbg, c);
  float* pt = p.part_tab + ((smp * p.nh + c.hf) * 3) * d;
  v16f pg;
#pragma unroll
  for (int r = 0; r < 16; ++r) pg[r] = dz[r] * x[r];
  put_block_sum(pg, c, cbg, pt);
  put_block_sum(dz, c, cbg, pt + d);
  put_block_sum(ps, c, cbg, pt + 2 * d);
}

// second application, first part: du, table partials and da of every pair
template <int CPW>
__global__ void __launch_bounds__(kThr) mc_bwd1_kernel(McArgs p) {
  extern __shared__ __align__(16) char smem[];
  const BSmem L = b_smem(smem);
  const Ctx c = make_ctx(p.S);
  const int64_t rb = c.i * p.S + c.s0;
  float x[CPW][16];
  load_tile<CPW>(p.h + rb * p.d, p.d, c, x);
  b_stage(L, p, c);
  const float coef = p.mul * p.g[0];
  __syncthreads();
  for (int j = 0; j < p.pc; ++j) {
    const Pair q = pair_of(p, L, c, j);
    const int64_t sm2 = (int64_t)p.nf * p.b + (int64_t)j * p.b + c.i;
    f32x16_v acc = zero16();
#pragma unroll
    for (int cb = 0; cb < CPW; ++cb) {
      const int cbg = c.wave * CPW + cb;
      float y[16];
      v16f dz, ps;
      pair_blk(p, q, c, cbg, x[cb], coef, [&](int r, float yv, float gv, float th, float, float s2) {
        y[r] = yv;
        dz[r] = gv * p.c * s2 * (1.0f - th * th);
        ps[r] = gv * p.c * th;
      });
      key_blk(p, c, sm2, q.g2, cbg, y, dz, ps, acc);
    }
    key_finish(p, L, c, sm2, acc, L.dat2 + j * 32 * kP);
  }
}

// Second application, second part (its input gradients dy_j = dout of the first application's
// src blocks; -g_j that of its dst blocks), the first application's du, table partials and da,
// and dh without the first application's pooled term.
template <int CPW>
__global__ void __launch_bounds__(kThr) mc_bwd2_kernel(McArgs p) {
  extern __shared__ __align__(16) char smem[];
  const BSmem L = b_smem(smem);
  const Ctx c = make_ctx(p.S);
  const int d = p.d, tid = threadIdx.x;
  const int64_t rb = c.i * p.S + c.s0;
  float x[CPW][16];
  load_tile<CPW>(p.h + rb * d, d, c, x);
  b_stage(L, p, c);
  for (int j = 0; j < p.pc; ++j) {
    const int64_t sm2 = (int64_t)p.nf * p.b + (int64_t)j * p.b + c.i;
    load_rank_tile(L.dat2 + j * 32 * kP, p.da, sm2 * p.S + c.s0, c.nrow);
  }
  const float invS = 1.0f / (float)p.S;
  for (int e = tid; e < p.pc * kR; e += kThr) {  // sum_s da of the second keys
    const int j = e >> 5, n = e & 31;
    const int64_t sm2 = (int64_t)p.nf * p.b + (int64_t)j * p.b + c.i;
    float s = 0.0f;
    for (int q = 0; q < p.nh; ++q) s += p.part_da[(sm2 * p.nh + q) * kR + n];
    L.sv[e] = s * invS;
    if (c.hf == 0) p.dsum[sm2 * kR + n] = f2bf(s);
  }
  __syncthreads();
  for (int e = tid; e < p.pc * d; e += kThr) {  // mv_j = (sum_s da / S) @ V2^T
    const int j = e / d, col = e - j * d;
    const int64_t g2 = clamp_key(p.ks[(int64_t)j * p.b + c.i], p.G);
    const uint4* w = reinterpret_cast<const uint4*>(p.Vb + (g2 * 3 * d + d + col) * kR);
    float s = 0.0f;
#pragma unroll
    for (int q4 = 0; q4 < 4; ++q4) {
      const uint4 u = w[q4];
      const uint32_t wd[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        s += L.sv[j * kR + 8 * q4 + 2 * i] * __uint_as_float(wd[i] << 16);
        s += L.sv[j * kR + 8 * q4 + 2 * i + 1] * __uint_as_float(wd[i] & 0xffff0000u);
      }
    }
    L.mv[j * d + col] = s;
  }
  const float coef = p.mul * p.g[0];
  const float rs = p.rstd[rb + c.row];
  float dh[CPW][16];
#pragma unroll
  for (int cb = 0; cb < CPW; ++cb)
#pragma unroll
    for (int r = 0; r < 16; ++r) dh[cb][r] = 0.0f;
  __syncthreads();
  int rbuf = 0;
  for (int k = 0; k < p.nf; ++k) {
    const int j1 = k - p.src_lo, j2 = k - p.dst_lo;
    const bool has1 = j1 >= 0 && j1 < p.pc, has2 = j2 >= 0 && j2 < p.pc;
    // pass 1: the row dot <dn, n> of the second application's input (pair j1)
    float ry = 0.0f, mdot = 0.0f;
    const Pair q1 = pair_of(p, L, c, has1 ? j1 : 0);
    if (has1) {
      const int64_t s2 = (int64_t)j1 * p.b + c.i;
      ry = p.rstd[(int64_t)p.b * p.S + s2 * p.S + c.s0 + c.row];
      float dot = 0.0f;
#pragma unroll
      for (int cb = 0; cb < CPW; ++cb) {
        const int cbg = c.wave * CPW + cb;
        const f32x16_v ls = expand_blk(p.UT + q1.gs * d * kR, q1.ss, cbg, c);
        const f32x16_v dn = expand_blk(p.Vb + q1.g2 * 3 * d * kR, L.dat2 + j1 * 32 * kP, cbg, c);
#pragma unroll
        for (int qq = 0; qq < 4; ++qq) {
          const int col = cbg * 32 + 8 * qq + 4 * c.h;
          const float4 gs = ld4(q1.ts + col), bs = ld4(q1.ts + d + col), ss = ld4(q1.ts + 2 * d + col);
          const float4 mv = ld4(L.mv + j1 * d + col);
#pragma unroll
          for (int jj = 0; jj < 4; ++jj) {
            const int r = 4 * qq + jj;
            const float xv = x[cb][r];
            const float y = xv + p.c * f4(ss, jj) * tanh_fast(f4(gs, jj) * xv + ls[r] + f4(bs, jj));
            dot += (dn[r] + f4(mv, jj)) * y * ry;
          }
        }
      }
      mdot = row_total(dot, L.rsum + rbuf * 256, c) / (float)d;
      rbuf ^= 1;
    }
    // pass 2: dout of key k, then its dz / ps, du, table sums, dz @ U^T and dh
    const int64_t smp = k * p.b + c.i;
    const int64_t g = clamp_key(p.kf[smp], p.G);
    const float* tk = L.tab + k * 3 * d;
    const Pair q2 = pair_of(p, L, c, has2 ? j2 : 0);
    f32x16_v acc = zero16();
#pragma unroll
    for (int cb = 0; cb < CPW; ++cb) {
      __builtin_amdgcn_sched_barrier(0);
      const int cbg = c.wave * CPW + cb;
      float dout[16];
#pragma unroll
      for (int r = 0; r < 16; ++r) dout[r] = 0.0f;
      if (has1) {
        // dy = g + dz gain2 + rstd_y (dn - n <dn, n> / d), dn = da @ V1^T + mv
        float y[16];
        pair_blk(p, q1, c, cbg, x[cb], coef, [&](int r, float yv, float gv, float th, float g2, float s2) {
          y[r] = yv;
          dout[r] += gv + gv * p.c * s2 * (1.0f - th * th) * g2;
        });
        __builtin_amdgcn_sched_barrier(0);
        const f32x16_v dn = expand_blk(p.Vb + q1.g2 * 3 * d * kR, L.dat2 + j1 * 32 * kP, cbg, c);
#pragma unroll
        for (int qq = 0; qq < 4; ++qq) {
          const float4 mv = ld4(L.mv + j1 * d + cbg * 32 + 8 * qq + 4 * c.h);
#pragma unroll
          for (int jj = 0; jj < 4; ++jj) {
            const int r = 4 * qq + jj;
            dout[r] += c.ok ? ry * (dn[r] + f4(mv, jj) - y[r] * ry * mdot) : 0.0f;
          }
        }
      }
      __builtin_amdgcn_sched_barrier(0);
      if (has2)
        pair_blk(p, q2, c, cbg, x[cb], coef, [&](int r, float, float gv, float, float, float) { dout[r] -= gv; });
      __builtin_amdgcn_sched_barrier(0);
      const f32x16_v lk = expand_blk(p.UT + g * d * kR, L.sat + k * 32 * kP, cbg, c);
      v16f dz, ps;
#pragma unroll
      for (int qq = 0; qq < 4; ++qq) {
        __builtin_amdgcn_sched_barrier(0);
        const int col = cbg * 32 + 8 * qq + 4 * c.h;
        const float4 gk = ld4(tk + col), bk = ld4(tk + d + col), sk = ld4(tk + 2 * d + col);
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) {
          const int r = 4 * qq + jj;
          const float xv = x[cb][r];
          const float th = tanh_fast(f4(gk, jj) * xv + lk[r] + f4(bk, jj));
          const float go = c.ok ? dout[r] : 0.0f;
          const float z = go * p.c * f4(sk, jj) * (1.0f - th * th);
          dz[r] = z;
          ps[r] = go * p.c * th;
          dh[cb][r] += go + z * f4(gk, jj);
        }
      }
      key_blk(p, c, smp, g, cbg, x[cb], dz, ps, acc);
    }
    key_finish(p, L, c, smp, acc, L.dat + k * 32 * kP);
  }
  // the first application's rmsnorm backward without its pooled term (dn = sum_k da_k @ V1_k^T),
  // and every key's h0 path (da @ V3^T)
  {
    float dot = 0.0f;
#pragma unroll
    for (int cb = 0; cb < CPW; ++cb) {
      const int cbg = c.wave * CPW + cb;
      f32x16_v dn = zero16();
      for (int k = 0; k < p.nf; ++k) {
        const int64_t g = clamp_key(p.kf[k * p.b + c.i], p.G);
        const f32x16_v t = expand_blk(p.Vb + g * 3 * d * kR, L.dat + k * 32 * kP, cbg, c);
#pragma unroll
        for (int r = 0; r < 16; ++r) dn[r] += t[r];
      }
#pragma unroll
      for (int r = 0; r < 16; ++r) dot += dn[r] * x[cb][r] * rs;
    }
    const float mdot = row_total(dot, L.rsum + rbuf * 256, c) / (float)d;
#pragma unroll
    for (int cb = 0; cb < CPW; ++cb) {
      const int cbg = c.wave * CPW + cb;
      f32x16_v dn = zero16(), v3 = zero16();
      for (int k = 0; k < p.nf; ++k) {
        __builtin_amdgcn_sched_barrier(0);
        const int64_t g = clamp_key(p.kf[k * p.b + c.i], p.G);
        const f32x16_v t = expand_blk(p.Vb + g * 3 * d * kR, L.dat + k * 32 * kP, cbg, c);
        const f32x16_v u = expand_blk(p.Vb + (g * 3 * d + 2 * d) * kR, L.dat + k * 32 * kP, cbg, c);
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          dn[r] += t[r];
          v3[r] += u[r];
        }
      }
      for (int j = 0; j < p.pc; ++j) {
        const int64_t g2 = clamp_key(p.ks[(int64_t)j * p.b + c.i], p.G);
        const f32x16_v u = expand_blk(p.Vb + (g2 * 3 * d + 2 * d) * kR, L.dat2 + j * 32 * kP, cbg, c);
#pragma unroll
        for (int r = 0; r < 16; ++r) v3[r] += u[r];
      }
#pragma unroll
      for (int r = 0; r < 16; ++r) dh[cb][r] += rs * (dn[r] - x[cb][r] * rs * mdot) + v3[r];
    }
  }
  store_f32_rows<CPW>(p.dh + rb * d, d, c, dh);
}

// dh += rstd (m - n <m, n> / d), m = sum_k (sum_s da_k / S) @ V2_k^T: the first application's pooled
// term; sum_s da of its keys to dsum
template <int CPW>
__global__ void __launch_bounds__(kThr) mc_bwd3_kernel(McArgs p) {
  __shared__ float sv[kMaxKeys * kR];
  __shared__ __align__(16) float mv[kMaxD];
  __shared__ float rsum[8 * 32];
  const Ctx c = make_ctx(p.S);
  const int d = p.d, tid = threadIdx.x;
  const int64_t rb = c.i * p.S + c.s0;
  float x[CPW][16], o[CPW][16];
  load_tile<CPW>(p.h + rb * d, d, c, x);
  load_tile<CPW>(p.dh + rb * d, d, c, o);
  const float invS = 1.0f / (float)p.S;
  for (int e = tid; e < p.nf * kR; e += kThr) {
    const int k = e >> 5, n = e & 31;
    const int64_t smp = k * p.b + c.i;
    float s = 0.0f;
    for (int q = 0; q < p.nh; ++q) s += p.part_da[(smp * p.nh + q) * kR + n];
    sv[e] = s * invS;
    if (c.hf == 0) p.dsum[smp * kR + n] = f2bf(s);
  }
  __syncthreads();
  for (int col = tid; col < d; col += kThr) {
    float s = 0.0f;
    for (int k = 0; k < p.nf; ++k) {
      const int64_t g = clamp_key(p.kf[k * p.b + c.i], p.G);
      const bf16* v2 = p.Vb + (g * 3 * d + d + col) * kR;
#pragma unroll
      for (int n = 0; n < kR; ++n) s += sv[k * kR + n] * bf2f(v2[n]);
    }
    mv[col] = s;
  }
  __syncthreads();
  const float rs = p.rstd[rb + c.row];
  float m[CPW][16];
  lds_vec<CPW>(mv, c, m);
  float dot = 0.0f;
#pragma unroll
  for (int cb = 0; cb < CPW; ++cb)
#pragma unroll
    for (int r = 0; r < 16; ++r) dot += m[cb][r] * x[cb][r] * rs;
  const float mdot = row_total(dot, rsum, c) / (float)d;
#pragma unroll
  for (int cb = 0; cb < CPW; ++cb)
#pragma unroll
    for (int r = 0; r < 16; ++r) o[cb][r] += rs * (m[cb][r] - x[cb][r] * rs * mdot);
  store_f32_rows<CPW>(p.dh + rb * d, d, c, o);
}

// VqT [G][32][2d] ([V1 | V3]^T) and Uq [G][32][d] with the middle two quads of every 16 columns
// swapped.  Block i < G * 2d / 32: 32 rows of V1 or V3; else 32 columns of U.
__device__ __forceinline__ int quad_swap(int p) {
  const int q = (p >> 2) & 3;
  const int sq = q == 1 ? 2 : (q == 2 ? 1 : q);
  return (p & ~12) | (sq << 2);
}

__global__ void __launch_bounds__(256) mc_prep_kernel(const float* __restrict__ V, const float* __restrict__ U, int G,
                                                      int d, bf16* __restrict__ VqT, bf16* __restrict__ Uq) {
  __shared__ float t[32][33];
  const int nv = 2 * d / 32, nu = d / 32, tid = threadIdx.x;
  int blk = blockIdx.x;
  if (blk < G * nv) {
    const int g = blk / nv, pos0 = (blk % nv) * 32;        // position in [V1 | V3]
    const int k0 = pos0 < d ? pos0 : pos0 + d;              // row of V
    for (int e = tid; e < 1024; e += 256) t[e >> 5][e & 31] = V[((int64_t)g * 3 * d + k0 + (e >> 5)) * kR + (e & 31)];
    __syncthreads();
    for (int e = tid; e < 1024; e += 256) {
      const int n = e >> 5, pp = e & 31;
      VqT[((int64_t)g * kR + n) * 2 * d + pos0 + pp] = f2bf(t[quad_swap(pp)][n]);
    }
  } else {
    blk -= G * nv;
    const int g = blk / nu, c0 = (blk % nu) * 32;
    for (int e = tid; e < 1024; e += 256) t[e >> 5][e & 31] = U[((int64_t)g * kR + (e >> 5)) * d + c0 + (e & 31)];
    __syncthreads();
    for (int e = tid; e < 1024; e += 256) {
      const int n = e >> 5, pp = e & 31;
      Uq[((int64_t)g * kR + n) * d + c0 + pp] = f2bf(t[n][quad_swap(pp)]);
    }
  }
}

bool g_cons_lds = false;

int cons_prepare() {
  if (g_cons_lds) return 0;
  const void* fns[] = {(const void*)mc_fwd1_kernel<1>, (const void*)mc_fwd1_kernel<2>,
                       (const void*)mc_fwd2_kernel<1>, (const void*)mc_fwd2_kernel<2>,
                       (const void*)mc_bwd1_kernel<1>, (const void*)mc_bwd1_kernel<2>,
                       (const void*)mc_bwd2_kernel<1>, (const void*)mc_bwd2_kernel<2>};
  const size_t need[] = {kF1Lds, kF1Lds, kF2Lds, kF2Lds, kBLds, kBLds, kBLds, kBLds};
  for (int i = 0; i < 8; ++i)
    RTE_REQUIRE(hipFuncSetAttribute(fns[i], hipFuncAttributeMaxDynamicSharedMemorySize, (int)need[i]) == hipSuccess,
                "macro_cons: cannot raise the LDS limit to %zu bytes", need[i]);
  g_cons_lds = true;
  return 0;
}

int check_args(const McArgs& p) {
  RTE_REQUIRE(p.b >= 1 && p.S >= 1 && p.S <= 2 * kRows, "macro_cons: need 1 <= S <= 64");
  RTE_REQUIRE(p.d == 256 || p.d == 512, "macro_cons: d must be 256 or 512");
  RTE_REQUIRE(p.nf >= 1 && p.nf <= kMaxKeys && p.pc >= 1 && p.pc <= p.nf, "macro_cons: need 1 <= pc <= nf <= %d",
              kMaxKeys);
  RTE_REQUIRE(p.src_lo >= 0 && p.src_lo + p.pc <= p.nf && p.dst_lo >= 0 && p.dst_lo + p.pc <= p.nf,
              "macro_cons: src / dst key blocks outside the first application");
  RTE_REQUIRE(p.G >= 1 && p.h && p.kf && p.ks && p.Vb && p.UT && p.Uq && p.gain && p.bias && p.scale,
              "macro_cons: missing input");
  return cons_prepare();
}

template <typename K>
void launch(K kernel, const McArgs& p, size_t lds, hipStream_t s) {
  hipLaunchKernelGGL(kernel, dim3((unsigned)p.b, (unsigned)p.nh), dim3(kThr), lds, s, p);
}

}  // namespace

int macro_cons_prep(const float* V, const float* U, int G, int d, bf16* VqT, bf16* Uq, hipStream_t s) {
  RTE_REQUIRE(G >= 1 && (d == 256 || d == 512) && V && U && VqT && Uq, "macro_cons_prep: bad arguments");
  hipLaunchKernelGGL(mc_prep_kernel, dim3((unsigned)(G * 3 * d / 32)), dim3(256), 0, s, V, U, G, d, VqT, Uq);
  return check_launch("macro_cons_prep");
}

size_t macro_cons_workspace_bytes(int b, int S, int d, int pc) {
  const size_t nh = (size_t)(S + kRows - 1) / kRows;
  return ((size_t)b * nh * d + (size_t)pc * b * nh * d + (size_t)b * nh) * sizeof(float) + 256;
}

int macro_cons_fwd(McArgs p, void* ws, size_t ws_bytes, hipStream_t s) {
  p.nh = (p.S + kRows - 1) / kRows;
  RTE_TRY(check_args(p));
  RTE_REQUIRE(p.VqT && p.x2 && p.pooled && p.a && p.sa && p.rstd && p.loss_out, "macro_cons_fwd: missing output");
  RTE_REQUIRE(ws && ws_bytes >= macro_cons_workspace_bytes(p.b, p.S, p.d, p.pc), "macro_cons_fwd: workspace too small");
  float* w = static_cast<float*>(ws);
  p.ppool = w;
  p.ppool2 = p.ppool + (size_t)p.b * p.nh * p.d;
  p.mse_part = p.ppool2 + (size_t)p.pc * p.b * p.nh * p.d;
  if (p.d == 512) {
    launch(mc_stats_kernel<2>, p, 0, s);
    RTE_TRY(check_launch("macro_cons_stats"));
    launch(mc_fwd1_kernel<2>, p, kF1Lds, s);
    RTE_TRY(check_launch("macro_cons_fwd1"));
    launch(mc_fwd2_kernel<2>, p, kF2Lds, s);
  } else {
    launch(mc_stats_kernel<1>, p, 0, s);
    RTE_TRY(check_launch("macro_cons_stats"));
    launch(mc_fwd1_kernel<1>, p, kF1Lds, s);
    RTE_TRY(check_launch("macro_cons_fwd1"));
    launch(mc_fwd2_kernel<1>, p, kF2Lds, s);
  }
  RTE_TRY(check_launch("macro_cons_fwd2"));
  const double n = (double)p.pc * p.b * p.S * p.d;
  return macro_fused_sum(p.mse_part, p.b * p.nh, (float)(1.0 / n), p.loss_out, s);
}

int macro_cons_bwd(McArgs p, hipStream_t s) {
  p.nh = (p.S + kRows - 1) / kRows;
  RTE_TRY(check_args(p));
  RTE_REQUIRE(p.a && p.sa && p.rstd && p.g && p.du && p.da && p.part_tab && p.part_da && p.dsum && p.dh,
              "macro_cons_bwd: missing buffer");
  if (p.d == 512) {
    launch(mc_bwd1_kernel<2>, p, kBLds, s);
    RTE_TRY(check_launch("macro_cons_bwd1"));
    launch(mc_bwd2_kernel<2>, p, kBLds, s);
    RTE_TRY(check_launch("macro_cons_bwd2"));
    launch(mc_bwd3_kernel<2>, p, 0, s);
  } else {
    launch(mc_bwd1_kernel<1>, p, kBLds, s);
    RTE_TRY(check_launch("macro_cons_bwd1"));
    launch(mc_bwd2_kernel<1>, p, kBLds, s);
    RTE_TRY(check_launch("macro_cons_bwd2"));
    launch(mc_bwd3_kernel<1>, p, 0, s);
  }
  return check_launch("macro_cons_bwd3");
}

}  // namespace rte

using namespace rte;

extern "C" {

int rte_macro_cons_prep(const float* V, const float* U, int G, int d, void* VqT, void* Uq, void* stream) {
  return macro_cons_prep(V, U, G, d, static_cast<bf16*>(VqT), static_cast<bf16*>(Uq),
                         static_cast<hipStream_t>(stream));
}

size_t rte_macro_cons_workspace_bytes(int b, int S, int d, int pc) { return macro_cons_workspace_bytes(b, S, d, pc); }

int rte_macro_cons_fwd(const float* h, int b, int S, int d, const int64_t* key_first, int nf, const int64_t* key_src,
                       int pc, int src_lo, int dst_lo, int G, float eps, const void* Vb, const void* VqT,
                       const void* UT, const void* Uq, const float* gain, const float* bias, const float* scale,
                       float c, void* x2, void* pooled, float* a, void* sa, float* rstd, float* loss, void* ws,
                       size_t ws_bytes, void* stream) {
  McArgs p{};
  p.h = h;
  p.b = b;
  p.S = S;
  p.d = d;
  p.G = G;
  p.nf = nf;
  p.pc = pc;
  p.src_lo = src_lo;
  p.dst_lo = dst_lo;
  p.eps = eps;
  p.c = c;
  p.kf = key_first;
  p.ks = key_src;
  p.Vb = static_cast<const bf16*>(Vb);
  p.VqT = static_cast<const bf16*>(VqT);
  p.UT = static_cast<const bf16*>(UT);
  p.Uq = static_cast<const bf16*>(Uq);
  p.gain = gain;
  p.bias = bias;
  p.scale = scale;
  p.x2 = static_cast<bf16*>(x2);
  p.pooled = static_cast<bf16*>(pooled);
  p.a = a;
  p.sa = static_cast<bf16*>(sa);
  p.rstd = rstd;
  p.loss_out = loss;
  return macro_cons_fwd(p, ws, ws_bytes, static_cast<hipStream_t>(stream));
}

int rte_macro_cons_bwd(const float* h, int b, int S, int d, const int64_t* key_first, int nf, const int64_t* key_src,
                       int pc, int src_lo, int dst_lo, int G, const void* Vb, const void* UT, const void* Uq,
                       const float* gain, const float* bias, const float* scale, float c, const float* a,
                       const void* sa, const float* rstd, const float* g, float mul, void* du, void* da,
                       float* part_tab, float* part_da, void* dsum, float* dh, void* stream) {
  McArgs p{};
  p.h = h;
  p.b = b;
  p.S = S;
  p.d = d;
  p.G = G;
  p.nf = nf;
  p.pc = pc;
  p.src_lo = src_lo;
  p.dst_lo = dst_lo;
  p.c = c;
  p.mul = mul;
  p.kf = key_first;
  p.ks = key_src;
  p.Vb = static_cast<const bf16*>(Vb);
  p.UT = static_cast<const bf16*>(UT);
  p.Uq = static_cast<const bf16*>(Uq);
  p.gain = gain;
  p.bias = bias;
  p.scale = scale;
  p.a = const_cast<float*>(a);
  p.sa = static_cast<bf16*>(const_cast<void*>(sa));
  p.rstd = const_cast<float*>(rstd);
  p.g = g;
  p.du = static_cast<bf16*>(du);
  p.da = static_cast<bf16*>(da);
  p.part_tab = part_tab;
  p.part_da = part_da;
  p.dsum = static_cast<bf16*>(dsum);
  p.dh = dh;
  return macro_cons_bwd(p, static_cast<hipStream_t>(stream));
}

}  // extern "C"
