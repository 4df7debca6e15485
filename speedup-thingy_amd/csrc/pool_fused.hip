// Routed cluster-pool SwiGLU of 32-neuron clusters in one launch per direction
// (rte/kernels/cluster_pool_ffn.py:192-241: per cluster, x rows of the tokens routed to it,
// z = up silu(gate) scaled by the routing weight, then the down projection), for d = 128, 256
// or 512:
//
//   forward : ug = x[tok] [W_up; W_gate]^T (bf16), zw = w up silu(gate) (bf16),
//             y_pairs[pair] = zw W_down^T                      (rte_grouped_swiglu_fwd's outputs)
//   backward: dZw = dout[tok] W_down, dug = SwiGLU backward of dZw (bf16), dw_slot = <z, dZw>,
//             dx_pairs[pair] = dug [W_up; W_gate]              (rte_grouped_swiglu_bwd's input
//                                                               gradients; its weight gradients
//                                                               stay grouped-K GEMMs)
//
// One workgroup (8 waves) owns 128 slots of one cluster (the slot ranges of rte_pack_index; the
// workgroup -> (cluster, tile) map is the prefix sum of the clusters' 128-slot tile counts).  The
// cluster's weights (96 KB of bf16 at d = 512) are staged in LDS once, each lane loads its slot's
// gathered row straight into MFMA operand registers (16 bytes per k step), and the [128 x 64]
// up/gate block and the [128 x 32] z block never leave the chip.  Both products run transposed
// (v_mfma_f32_32x32x16_bf16 with the weight rows as the first operand, the slots as the second):
// the accumulator of lane l then holds one slot (l % 32) and 16 output columns, and staging the
// weight rows with bits 2 and 3 of the row index swapped makes those 16 columns
// 8 h .. 8 h + 7 and 16 + 8 h .. 16 + 8 h + 7 (h = l / 32), so every output row is written with
// 16-byte stores.  Waves 0-3 and 4-7 reduce the two halves of d; their partial products are added
// in that order through LDS.  The backward stages both weights transposed (d-major) with 2-byte
// LDS writes.  No atomics: every sum has a fixed order.

#include "common.hpp"

namespace rte {

namespace {

constexpr int kThr = 512;    // 8 waves
constexpr int kRows = 128;   // slots per workgroup
constexpr int kN = 32;       // neurons per cluster

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

// Row m of a 32-row operand block holds logical row perm32(m) (bits 2 and 3 swapped; the map is
// its own inverse): accumulator register r of lane l is then logical row 16 (r / 8) + 8 (l / 32) + r % 8.
__device__ __forceinline__ int perm32(int m) { return (m & ~12) | ((m & 4) << 1) | ((m & 8) >> 1); }

// 8 bf16 of v[o .. o + 7]
__device__ __forceinline__ uint4 pack8u(const float* v) {
  uint4 u;
  u.x = pack_bf2(v[0], v[1]);
  u.y = pack_bf2(v[2], v[3]);
  u.z = pack_bf2(v[4], v[5]);
  u.w = pack_bf2(v[6], v[7]);
  return u;
}

// the lane's 16 columns (8 h .. +7, 16 + 8 h .. +7) of a bf16 row
__device__ __forceinline__ void store_row16(bf16* row, int h, const float* v) {
  *reinterpret_cast<uint4*>(row + 8 * h) = pack8u(v);
  *reinterpret_cast<uint4*>(row + 16 + 8 * h) = pack8u(v + 8);
}

// workgroup -> (cluster, 128-slot tile) by prefix sums of the clusters' tile counts, 64 clusters
// per step (wave 0): st = {cluster, first slot, end of the cluster's slots}, st[0] = -1 when the
// workgroup has no tile.  Workgroup b runs on XCD b % 8:
// tile (b % 8) (grid / 8) + b / 8 puts consecutive tiles, the tiles of one cluster, on one XCD, so
// its L2 serves the cluster's weights to all of them (grid a multiple of 8).
__device__ __forceinline__ void tile_map(const int32_t* goff, int G, int* st) {
  const int tid = threadIdx.x;
  if (tid < 64) {
    if (tid == 0) st[0] = -1;
    const int x = (int)(blockIdx.x & 7) * (int)(gridDim.x >> 3) + (int)(blockIdx.x >> 3);
    int base = 0;
    for (int c0 = 0; c0 < G; c0 += 64) {
      const int gg = c0 + tid;
      const int lo = gg < G ? goff[gg] : 0, hi = gg < G ? goff[gg + 1] : 0;
      const int cnt = (hi - lo + kRows - 1) / kRows;
      int incl = cnt;
#pragma unroll
      for (int off = 1; off < 64; off <<= 1) {
        const int y = __shfl_up(incl, off, 64);
        if (tid >= off) incl += y;
      }
      const int excl = incl - cnt;
      if (cnt > 0 && x >= base + excl && x < base + incl) {
        st[0] = gg;
        st[1] = lo + (x - base - excl) * kRows;
        st[2] = hi;
      }
      base += __shfl(incl, 63, 64);
    }
  }
  __syncthreads();
}

constexpr size_t max_sz(size_t a, size_t b) { return a > b ? a : b; }

// Forward: the first region holds the up/gate rows for the first product, then the second half's
// partial products (fp32 [4 slot blocks][8][64 lanes][4], 32 KB) and the down rows ([D][32], 64-byte
// rows whose 16-byte chunks q sit at q ^ ((row / 4) % 4): 16 lanes reading 16 consecutive rows
// touch every bank once).  About 75 KB in all: two workgroups per CU.
template <int D>
struct FwdLds {
  static constexpr int WP = D + 8;    // up/gate rows [64][WP]: 16 B row padding
  static constexpr int DP = kN + 8;   // z rows [128][DP]
  static constexpr size_t red_bytes = (size_t)4 * 32 * 64 * 4;
  static constexpr size_t r0 = max_sz((size_t)64 * WP * 2, red_bytes + (size_t)D * kN * 2);
  static constexpr size_t bytes = r0 + (size_t)kRows * DP * 2;
};

// element offset of 16-byte chunk q of row `row` in the swizzled [rows][32] down rows
__device__ __forceinline__ int wd_at(int row, int q) { return row * kN + 8 * (q ^ ((row >> 2) & 3)); }

// Backward: the first region holds W_down^T for the first product, then the second half's partial
// products (16 KB), then each wave's 4 KB output staging (32 KB).
template <int D>
struct BwdLds {
  static constexpr int TP = D + 8;    // transposed down rows [32][TP]
  static constexpr int UP = 64 + 8;   // transposed up/gate rows [D][UP], dug rows [128][UP]
  static constexpr size_t r0 = max_sz((size_t)kN * TP * 2, (size_t)8 * 32 * 64 * 2);
  static constexpr size_t bytes = r0 + (size_t)(D * UP + kRows * UP) * 2;
};

// ------------------------------------------------------------------ forward

template <int D>
__global__ void __launch_bounds__(kThr) __attribute__((amdgpu_waves_per_eu(4, 4))) pf_fwd_kernel(const bf16* __restrict__ x, const int32_t* __restrict__ goff,
                                                      int G, const int32_t* __restrict__ tok_of_slot,
                                                      const int32_t* __restrict__ pair_of_slot,
                                                      const float* __restrict__ w_of_slot,
                                                      const bf16* __restrict__ wug, int F,
                                                      const bf16* __restrict__ wd, int64_t ld_wd,
                                                      bf16* __restrict__ ug, bf16* __restrict__ zw,
                                                      bf16* __restrict__ yp) {
  using L = FwdLds<D>;
  constexpr int WP = L::WP, DP = L::DP, KH = D / 2, KS = KH / 16, CB = D / 64;
  constexpr int UC = 64 * D / 8 / kThr, DC = D * kN / 8 / kThr;
  static_assert(UC >= 1 && DC >= 1 && 64 * D / 8 == UC * kThr && D * kN / 8 == DC * kThr, "staging split");
  extern __shared__ __align__(16) char smem[];
  bf16* wug_s = reinterpret_cast<bf16*>(smem);  // [64][WP]: rows 0..31 up, 32..63 gate (perm32 order)
  float* red = reinterpret_cast<float*>(smem);   // after the first product: [4][8][64][4] partials
  bf16* wd_s = reinterpret_cast<bf16*>(smem + L::red_bytes);  // ... and [D][32] down rows (perm32, swizzled)
  bf16* z_s = reinterpret_cast<bf16*>(smem + L::r0);          // [128][DP]: z of the tile's slots
  __shared__ int st[3];

  tile_map(goff, G, st);
  const int g = st[0];
  if (g < 0) return;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, h = lane >> 5, l32 = lane & 31;
  const int m0 = st[1], mlim = st[2];

  // the cluster's up/gate rows, the lane's slot and the down rows in one round trip; the up/gate
  // rows go to LDS before the x rows are loaded (registers), the down rows after the first product
  uint4 wu[UC], wv[DC];
#pragma unroll
  for (int i = 0; i < UC; ++i) {
    const int e = tid + i * kThr, row = e / (D / 8), c = e % (D / 8);
    const int grow = (row < kN ? 0 : F) + g * kN + perm32(row & 31);
    wu[i] = *reinterpret_cast<const uint4*>(wug + (int64_t)grow * D + 8 * c);
  }
  const int sb = wave & 3, kh = wave >> 2;
  const int slot = m0 + sb * 32 + l32;
  const bool ok = slot < mlim;
  const int tok = tok_of_slot[ok ? slot : m0];
#pragma unroll
  for (int i = 0; i < DC; ++i) {
    const int e = tid + i * kThr, row = e >> 2, q = e & 3;
    const int dcol = (row & ~31) | perm32(row & 31);
    wv[i] = *reinterpret_cast<const uint4*>(wd + (int64_t)dcol * ld_wd + (int64_t)g * kN + 8 * q);
  }
#pragma unroll
  for (int i = 0; i < UC; ++i) {
    const int e = tid + i * kThr, row = e / (D / 8), c = e % (D / 8);
    *reinterpret_cast<uint4*>(wug_s + row * WP + 8 * c) = wu[i];
  }
  // this lane's x row, half kh of d
  const bf16* xr = x + (int64_t)tok * D + kh * KH + 8 * h;
  bf16x8_v xv[KS];
#pragma unroll
  for (int t = 0; t < KS; ++t) xv[t] = ld8b(xr + 16 * t);
  __syncthreads();

  // [up; gate]^T of the wave's 32 slots over its half of d: rows = neurons, columns = slots
  f32x16_v cu = zero16(), cg = zero16();
  {
    const bf16* au = wug_s + l32 * WP + kh * KH + 8 * h;
    const bf16* ag = au + 32 * WP;
#pragma unroll
    for (int t = 0; t < KS; ++t) {
      cu = mfma(ld8b(au + 16 * t), xv[t], cu);
      cg = mfma(ld8b(ag + 16 * t), xv[t], cg);
    }
  }
  __syncthreads();  // the up/gate rows are no longer read: their space takes the partials and the down rows
#pragma unroll
  for (int i = 0; i < DC; ++i) {
    const int e = tid + i * kThr;
    *reinterpret_cast<uint4*>(wd_s + wd_at(e >> 2, e & 3)) = wv[i];
  }
  if (kh == 1) {
#pragma unroll
    for (int v = 0; v < 8; ++v) {
      float4 o;
      const f32x16_v& s = v < 4 ? cu : cg;
      const int r = 4 * (v & 3);
      o.x = s[r];
      o.y = s[r + 1];
      o.z = s[r + 2];
      o.w = s[r + 3];
      *reinterpret_cast<float4*>(red + ((sb * 8 + v) * 64 + lane) * 4) = o;
    }
  }
  __syncthreads();
  if (kh == 0) {
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const float4 o = *reinterpret_cast<const float4*>(red + ((sb * 8 + v) * 64 + lane) * 4);
      const float4 p = *reinterpret_cast<const float4*>(red + ((sb * 8 + 4 + v) * 64 + lane) * 4);
      cu[4 * v] += o.x;
      cu[4 * v + 1] += o.y;
      cu[4 * v + 2] += o.z;
      cu[4 * v + 3] += o.w;
      cg[4 * v] += p.x;
      cg[4 * v + 1] += p.y;
      cg[4 * v + 2] += p.z;
      cg[4 * v + 3] += p.w;
    }
    const float rs = (ok && w_of_slot) ? w_of_slot[slot] : 1.0f;
    // columns 8 h .. +7 (registers 0..7), then 16 + 8 h .. +7 (registers 8..15)
#pragma unroll
    for (int half = 0; half < 2; ++half) {
      float ub[8], gb[8], zz[8];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        ub[j] = round_bf(cu[8 * half + j]);
        gb[j] = round_bf(cg[8 * half + j]);
        zz[j] = ok ? ub[j] * gb[j] * sigmoidf_(gb[j]) * rs : 0.0f;
      }
      const int col = 16 * half + 8 * h;
      const uint4 zq = pack8u(zz);
      if (ok) {
        *reinterpret_cast<uint4*>(ug + (int64_t)slot * 64 + col) = pack8u(ub);
        *reinterpret_cast<uint4*>(ug + (int64_t)slot * 64 + 32 + col) = pack8u(gb);
        *reinterpret_cast<uint4*>(zw + (int64_t)slot * kN + col) = zq;
      }
      *reinterpret_cast<uint4*>(z_s + (sb * 32 + l32) * DP + col) = zq;
    }
  }
  const int64_t prow = ok ? pair_of_slot[slot] : 0;
  __syncthreads();

  // y^T = W_down z^T: rows = output columns, columns = slots, k = the 32 neurons.  Each wave
  // turns 64 columns of its 32 slots at a time around through its own 4 KB of LDS (the partials'
  // space: [32 slots][64 columns], 16-byte chunk c of slot r at c ^ (r % 8)), so each store
  // instruction writes 8 slots' rows with 128 contiguous bytes each.
  {
    const int ch = wave >> 2;
    const bf16* zr = z_s + (sb * 32 + l32) * DP + 8 * h;
    const bf16x8_v b0 = ld8b(zr), b1 = ld8b(zr + 16);
    bf16* stg = reinterpret_cast<bf16*>(smem) + wave * 32 * 64;
    const int c8 = lane & 7, r8 = lane >> 3;
    int64_t orow[4];
    bool rok[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = r8 + 8 * i;
      orow[i] = __shfl(prow, r, 64) * D;
      rok[i] = m0 + sb * 32 + r < mlim;
    }
#pragma unroll
    for (int i = 0; i < CB; i += 2) {
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int row = (ch * CB + i + j) * 32 + l32;
        f32x16_v acc = mfma(ld8b(wd_s + wd_at(row, h)), b0, zero16());
        acc = mfma(ld8b(wd_s + wd_at(row, 2 + h)), b1, acc);
        float v[16];
#pragma unroll
        for (int r = 0; r < 16; ++r) v[r] = acc[r];
        const int c0 = 4 * j + h;  // 16-byte chunks c0 and c0 + 2 of the 64 columns
        *reinterpret_cast<uint4*>(stg + l32 * 64 + 8 * (c0 ^ (l32 & 7))) = pack8u(v);
        *reinterpret_cast<uint4*>(stg + l32 * 64 + 8 * ((c0 + 2) ^ (l32 & 7))) = pack8u(v + 8);
      }
      const int col = (ch * CB + i) * 32 + 8 * c8;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int r = r8 + 8 * q;
        const uint4 val = *reinterpret_cast<const uint4*>(stg + r * 64 + 8 * (c8 ^ (r & 7)));
        if (rok[q]) *reinterpret_cast<uint4*>(yp + orow[q] + col) = val;
      }
    }
  }
}

// ------------------------------------------------------------------ backward (input side)

template <int D>
__global__ void __launch_bounds__(kThr) pf_bwd_kernel(const bf16* __restrict__ dout, const int32_t* __restrict__ goff,
                                                      int G, const int32_t* __restrict__ tok_of_slot,
                                                      const int32_t* __restrict__ pair_of_slot,
                                                      const float* __restrict__ w_of_slot,
                                                      const bf16* __restrict__ wug, int F,
                                                      const bf16* __restrict__ wd, int64_t ld_wd,
                                                      const bf16* __restrict__ ug, bf16* __restrict__ dug,
                                                      float* __restrict__ dw_slot, bf16* __restrict__ dxp) {
  using L = BwdLds<D>;
  constexpr int TP = L::TP, UP = L::UP, KH = D / 2, KS = KH / 16, CB = D / 64;
  constexpr int UC = 64 * D / 8 / kThr, DC = D * kN / 8 / kThr;
  static_assert(UC >= 1 && DC >= 1 && 64 * D / 8 == UC * kThr && D * kN / 8 == DC * kThr, "staging split");
  extern __shared__ __align__(16) char smem[];
  bf16* wdT_s = reinterpret_cast<bf16*>(smem);  // [32][TP]: W_down^T, rows = neurons (perm32 order)
  bf16* wugT_s = reinterpret_cast<bf16*>(smem + L::r0);  // [D][UP]: [W_up; W_gate]^T, rows = columns of d
  bf16* dug_s = wugT_s + D * UP;                 // [128][UP]: dug of the tile's slots
  float* red = reinterpret_cast<float*>(smem);   // [4][4][64][4]: second-half partials (over wdT_s)
  __shared__ int st[3];

  tile_map(goff, G, st);
  const int g = st[0];
  if (g < 0) return;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, h = lane >> 5, l32 = lane & 31;
  const int m0 = st[1], mlim = st[2];

  // weights, d-major for the transposed LDS copies: consecutive threads take consecutive columns
  // of d (down) or consecutive up/gate rows (up/gate), so the 2-byte LDS writes of a wave are
  // consecutive
  uint4 wv[DC], wu[UC];
#pragma unroll
  for (int i = 0; i < DC; ++i) {
    const int e = tid + i * kThr, dcol = e % D, q = e / D;
    wv[i] = *reinterpret_cast<const uint4*>(wd + (int64_t)dcol * ld_wd + (int64_t)g * kN + 8 * q);
  }
#pragma unroll
  for (int i = 0; i < UC; ++i) {
    const int e = tid + i * kThr, uu = e & 63, c = e >> 6;
    const int grow = (uu < kN ? 0 : F) + g * kN + (uu & 31);
    wu[i] = *reinterpret_cast<const uint4*>(wug + (int64_t)grow * D + 8 * c);
  }
  const int sb = wave & 3, kh = wave >> 2;
  const int slot = m0 + sb * 32 + l32;
  const bool ok = slot < mlim;
  const int srow = ok ? slot : m0;
  const int tok = tok_of_slot[srow];
  const bf16* dr = dout + (int64_t)tok * D + kh * KH + 8 * h;
  bf16x8_v dv[KS];
#pragma unroll
  for (int t = 0; t < KS; ++t) dv[t] = ld8b(dr + 16 * t);
  uint4 ugv[4];
  if (kh == 0) {
    const bf16* ur = ug + (int64_t)srow * 64 + 8 * h;
    ugv[0] = *reinterpret_cast<const uint4*>(ur);
    ugv[1] = *reinterpret_cast<const uint4*>(ur + 16);
    ugv[2] = *reinterpret_cast<const uint4*>(ur + 32);
    ugv[3] = *reinterpret_cast<const uint4*>(ur + 48);
  }
#pragma unroll
  for (int i = 0; i < DC; ++i) {
    const int e = tid + i * kThr, dcol = e % D, q = e / D;
    const bf16* s = reinterpret_cast<const bf16*>(&wv[i]);
#pragma unroll
    for (int j = 0; j < 8; ++j) wdT_s[perm32(8 * q + j) * TP + dcol] = s[j];
  }
#pragma unroll
  for (int i = 0; i < UC; ++i) {
    const int e = tid + i * kThr, uu = e & 63, c = e >> 6;
    const bf16* s = reinterpret_cast<const bf16*>(&wu[i]);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      const int dcol = 8 * c + j;
      wugT_s[((dcol & ~31) | perm32(dcol & 31)) * UP + uu] = s[j];
    }
  }
  __syncthreads();

  // dZw^T = W_down^T dout[tok]^T over the wave's half of d: rows = neurons, columns = slots
  f32x16_v acc = zero16();
  {
    const bf16* ar = wdT_s + l32 * TP + kh * KH + 8 * h;
#pragma unroll
    for (int t = 0; t < KS; ++t) acc = mfma(ld8b(ar + 16 * t), dv[t], acc);
  }
  __syncthreads();  // W_down^T is no longer read: its space takes the partials
  if (kh == 1) {
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      float4 o;
      o.x = acc[4 * v];
      o.y = acc[4 * v + 1];
      o.z = acc[4 * v + 2];
      o.w = acc[4 * v + 3];
      *reinterpret_cast<float4*>(red + ((sb * 4 + v) * 64 + lane) * 4) = o;
    }
  }
  __syncthreads();
  if (kh == 0) {
    const float rs = (ok && w_of_slot) ? w_of_slot[slot] : 1.0f;
    const bf16* uv = reinterpret_cast<const bf16*>(ugv);  // up: 0..7, 8..15; gate: 16..23, 24..31
    float du[16], dg[16], part = 0.0f;
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const float4 o = *reinterpret_cast<const float4*>(red + ((sb * 4 + v) * 64 + lane) * 4);
      const float add[4] = {o.x, o.y, o.z, o.w};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int r = 4 * v + j;
        const float draw = acc[r] + add[j];
        const float up = bf2f(uv[r]), gt = bf2f(uv[16 + r]);
        const float s = sigmoidf_(gt);
        const float silu = gt * s;
        const float dz = draw * rs;
        du[r] = ok ? dz * silu : 0.0f;
        dg[r] = ok ? dz * up * s * (1.0f + gt * (1.0f - s)) : 0.0f;
        part += up * silu * draw;
      }
    }
    part += __shfl_xor(part, 32, 64);
    if (ok) {
      store_row16(dug + (int64_t)slot * 64, h, du);
      store_row16(dug + (int64_t)slot * 64 + 32, h, dg);
      if (dw_slot && h == 0) dw_slot[slot] = part;
    }
    store_row16(dug_s + (sb * 32 + l32) * UP, h, du);
    store_row16(dug_s + (sb * 32 + l32) * UP + 32, h, dg);
  }
  const int64_t prow = ok ? pair_of_slot[slot] : 0;
  __syncthreads();

  // dx^T = [W_up; W_gate]^T dug^T: rows = columns of d, columns = slots, k = the 64 up/gate values;
  // 64 columns of the wave's 32 slots at a time turned around through its 4 KB of LDS (as in the
  // forward), so each store instruction writes 8 rows with 128 contiguous bytes each
  {
    const int ch = wave >> 2;
    const bf16* br = dug_s + (sb * 32 + l32) * UP + 8 * h;
    const bf16x8_v b0 = ld8b(br), b1 = ld8b(br + 16), b2 = ld8b(br + 32), b3 = ld8b(br + 48);
    bf16* stg = reinterpret_cast<bf16*>(smem) + wave * 32 * 64;
    const int c8 = lane & 7, r8 = lane >> 3;
    int64_t orow[4];
    bool rok[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int r = r8 + 8 * i;
      orow[i] = __shfl(prow, r, 64) * D;
      rok[i] = m0 + sb * 32 + r < mlim;
    }
#pragma unroll
    for (int i = 0; i < CB; i += 2) {
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const bf16* ar = wugT_s + ((ch * CB + i + j) * 32 + l32) * UP + 8 * h;
        f32x16_v a = mfma(ld8b(ar), b0, zero16());
        a = mfma(ld8b(ar + 16), b1, a);
        a = mfma(ld8b(ar + 32), b2, a);
        a = mfma(ld8b(ar + 48), b3, a);
        float v[16];
#pragma unroll
        for (int r = 0; r < 16; ++r) v[r] = a[r];
        const int c0 = 4 * j + h;
        *reinterpret_cast<uint4*>(stg + l32 * 64 + 8 * (c0 ^ (l32 & 7))) = pack8u(v);
        *reinterpret_cast<uint4*>(stg + l32 * 64 + 8 * ((c0 + 2) ^ (l32 & 7))) = pack8u(v + 8);
      }
      const int col = (ch * CB + i) * 32 + 8 * c8;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int r = r8 + 8 * q;
        const uint4 val = *reinterpret_cast<const uint4*>(stg + r * 64 + 8 * (c8 ^ (r & 7)));
        if (rok[q]) *reinterpret_cast<uint4*>(dxp + orow[q] + col) = val;
      }
    }
  }
}

bool g_lds_set = false;

template <int D>
bool raise_lds() {
  return hipFuncSetAttribute((const void*)pf_fwd_kernel<D>, hipFuncAttributeMaxDynamicSharedMemorySize,
                             (int)FwdLds<D>::bytes) == hipSuccess &&
         hipFuncSetAttribute((const void*)pf_bwd_kernel<D>, hipFuncAttributeMaxDynamicSharedMemorySize,
                             (int)BwdLds<D>::bytes) == hipSuccess;
}

int prepare() {
  if (g_lds_set) return 0;
  RTE_REQUIRE(raise_lds<128>() && raise_lds<256>() && raise_lds<512>(),
              "pool_fused: cannot raise the LDS limit to %zu bytes", BwdLds<512>::bytes);
  g_lds_set = true;
  return 0;
}

}  // namespace

bool pool_fused_supported(int n, int d) { return n == kN && (d == 128 || d == 256 || d == 512); }

int pool_fused_fwd(const bf16* x, int d, const int32_t* offsets, int G, int n, int P, const int32_t* tok_of_slot,
                   const int32_t* pair_of_slot, const float* w_of_slot, const bf16* wug, const bf16* wd,
                   int64_t ld_wd, bf16* ug, bf16* zw, bf16* y_pairs, hipStream_t s) {
  RTE_REQUIRE(pool_fused_supported(n, d), "pool_fused: needs 32-neuron clusters and d in {128, 256, 512}");
  RTE_REQUIRE(G >= 1 && P >= 0 && ld_wd >= (int64_t)G * n, "pool_fused: bad sizes");
  RTE_REQUIRE(x && offsets && tok_of_slot && pair_of_slot && wug && wd && ug && zw && y_pairs,
              "pool_fused: null pointer");
  RTE_REQUIRE(ld_wd % 8 == 0, "pool_fused: the down weight's row pitch must be a multiple of 8");
  if (P == 0) return 0;
  RTE_TRY(prepare());
  const int F = G * n;
  const dim3 grid((unsigned)((P / kRows + G + 1 + 7) & ~7));
  switch (d) {
    case 128:
      hipLaunchKernelGGL(pf_fwd_kernel<128>, grid, dim3(kThr), FwdLds<128>::bytes, s, x, offsets, G, tok_of_slot,
                         pair_of_slot, w_of_slot, wug, F, wd, ld_wd, ug, zw, y_pairs);
      break;
    case 256:
      hipLaunchKernelGGL(pf_fwd_kernel<256>, grid, dim3(kThr), FwdLds<256>::bytes, s, x, offsets, G, tok_of_slot,
                         pair_of_slot, w_of_slot, wug, F, wd, ld_wd, ug, zw, y_pairs);
      break;
    default:
      hipLaunchKernelGGL(pf_fwd_kernel<512>, grid, dim3(kThr), FwdLds<512>::bytes, s, x, offsets, G, tok_of_slot,
                         pair_of_slot, w_of_slot, wug, F, wd, ld_wd, ug, zw, y_pairs);
      break;
  }
  return check_launch("pool_fused_fwd");
}

int pool_fused_bwd(const bf16* dout, int d, const int32_t* offsets, int G, int n, int P, const int32_t* tok_of_slot,
                   const int32_t* pair_of_slot, const float* w_of_slot, const bf16* wug, const bf16* wd,
                   int64_t ld_wd, const bf16* ug, bf16* dug, float* dw_slot, bf16* dx_pairs, hipStream_t s) {
  RTE_REQUIRE(pool_fused_supported(n, d), "pool_fused: needs 32-neuron clusters and d in {128, 256, 512}");
  RTE_REQUIRE(G >= 1 && P >= 0 && ld_wd >= (int64_t)G * n, "pool_fused: bad sizes");
  RTE_REQUIRE(dout && offsets && tok_of_slot && pair_of_slot && wug && wd && ug && dug && dx_pairs,
              "pool_fused: null pointer");
  RTE_REQUIRE(ld_wd % 8 == 0, "pool_fused: the down weight's row pitch must be a multiple of 8");
  if (P == 0) return 0;
  RTE_TRY(prepare());
  const int F = G * n;
  const dim3 grid((unsigned)((P / kRows + G + 1 + 7) & ~7));
  switch (d) {
    case 128:
      hipLaunchKernelGGL(pf_bwd_kernel<128>, grid, dim3(kThr), BwdLds<128>::bytes, s, dout, offsets, G, tok_of_slot,
                         pair_of_slot, w_of_slot, wug, F, wd, ld_wd, ug, dug, dw_slot, dx_pairs);
      break;
    case 256:
      hipLaunchKernelGGL(pf_bwd_kernel<256>, grid, dim3(kThr), BwdLds<256>::bytes, s, dout, offsets, G, tok_of_slot,
                         pair_of_slot, w_of_slot, wug, F, wd, ld_wd, ug, dug, dw_slot, dx_pairs);
      break;
    default:
      hipLaunchKernelGGL(pf_bwd_kernel<512>, grid, dim3(kThr), BwdLds<512>::bytes, s, dout, offsets, G, tok_of_slot,
                         pair_of_slot, w_of_slot, wug, F, wd, ld_wd, ug, dug, dw_slot, dx_pairs);
      break;
  }
  return check_launch("pool_fused_bwd");
}

}  // namespace rte
