// bf16 MFMA GEMM core for gfx950 (v_mfma_f32_32x32x16_bf16), fp32 accumulation.
//
// Tiling: a workgroup of 256 threads (4 wave64) owns a BM x BN output tile and
// walks k in steps of BK through double-buffered LDS.  Global tiles are fetched
// into registers one step ahead (16-byte loads), then written to LDS in a
// k-contiguous layout [row][BK+8] so every MFMA operand fetch is one 16-byte LDS
// read per lane (rows 36 dwords apart: 8 consecutive rows hit disjoint banks).
// Operands whose output index is contiguous in memory (layout T) are loaded as
// 4(k) x 8(i) blocks and transposed in registers before the LDS write; threads
// walk k fastest there so each 8-byte LDS write wave touches every bank twice.
// Row addresses of layout-N operands are resolved once per tile; the loop only
// advances k.  Results leave through LDS so every global store is 16 bytes.
//
// MFMA lane layout used below (32x32x16): lane l supplies A row (l % 32) and
// B column (l % 32) with 8 consecutive k values starting at 8*(l / 32); output
// register r of lane l holds row 8*(r/4) + 4*(l/32) + (r%4), column l % 32.
// Any consistent k permutation gives the same dot products, so only the output
// mapping has to match the hardware; the GPU parity tests pin it.
#include "gemm.hpp"

#include <stdio.h>
#include <stdlib.h>

#include <type_traits>

namespace rte {

namespace {

constexpr int kThreads = 256;
constexpr int kMaxSplits = 32;                      // split-K partials per output tile
constexpr size_t kMaxSplitBytes = (size_t)64 << 20;  // split-K workspace ceiling

__device__ __forceinline__ int64_t ilv_row(int64_t r, int32_t half) {
  return ((r & 63) < 32 ? 0 : half) + (r >> 6) * 32 + (r & 31);
}

__device__ __forceinline__ int log2i(int v) { return 31 - __clz(v); }

__device__ __forceinline__ int64_t row_off(const Operand& o, int64_t r) {
  if (o.ilv) r = ilv_row(r, o.ilv);
  if (o.rows) r = o.rows[r];
  if (o.rdiv) return (r >> log2i(o.rdiv)) * o.rs_hi + (r & (o.rdiv - 1)) * o.ld;
  return r * o.ld;
}

__device__ __forceinline__ int64_t col_off(const Operand& o, int c) {
  if (o.cdiv) return (int64_t)(c >> log2i(o.cdiv)) * o.cs_hi + (c & (o.cdiv - 1));
  return c;
}

// ------------------------------------------------------------------ loaders

template <int R, int BK>
struct LoaderN {
  static constexpr int LDP = BK + 8;
  static constexpr int CPR = BK / 8;
  static constexpr int UNITS = R * CPR;
  static constexpr int PER = (UNITS + kThreads - 1) / kThreads;
  const bf16* rowp[PER];
  bool ok[PER];
  uint4 r[2][PER];  // two staged k tiles in flight

  __device__ __forceinline__ void init(const Operand& o, const bf16* base, int64_t rowshift, int i0, int ilim,
                                       int tid) {
#pragma unroll
    for (int u = 0; u < PER; ++u) {
      const int q = tid + u * kThreads;
      const int i = i0 + q / CPR;
      ok[u] = q < UNITS && i < ilim;
      rowp[u] = ok[u] ? base + row_off(o, i + rowshift) : base;
    }
  }
  // Every lane issues its load (masked lanes read a valid address and keep zeros), so the
  // number of loads in flight per stage is fixed and the wait for a stage is exact.
  template <int S>
  __device__ __forceinline__ void load(const Operand& o, int k0, int klim, int tid) {
#pragma unroll
    for (int u = 0; u < PER; ++u) {
      const int q = tid + u * kThreads;
      const int k = k0 + (q % CPR) * 8;
      const bool valid = ok[u] && k < klim;
      const uint4 v = *reinterpret_cast<const uint4*>(rowp[u] + (valid ? col_off(o, k) : 0));
      r[S][u] = valid ? v : make_uint4(0u, 0u, 0u, 0u);
    }
  }
  template <int S>
  __device__ __forceinline__ void store(bf16* lds, int tid) const {
#pragma unroll
    for (int u = 0; u < PER; ++u) {
      const int q = tid + u * kThreads;
      if (q >= UNITS) continue;
      *reinterpret_cast<uint4*>(lds + (q / CPR) * LDP + (q % CPR) * 8) = r[S][u];
    }
  }
};

template <int R, int BK>
struct LoaderT {
  static constexpr int LDP = BK + 8;
  static constexpr int KB = BK / 4;
  static constexpr int UNITS = (R / 8) * KB;
  static constexpr int PER = (UNITS + kThreads - 1) / kThreads;
  int64_t coff[PER];
  bool ok[PER];
  uint4 r[2][PER * 4];  // two staged k tiles in flight

  __device__ __forceinline__ void init(const Operand& o, const bf16*, int64_t, int i0, int ilim, int tid) {
#pragma unroll
    for (int u = 0; u < PER; ++u) {
      const int q = tid + u * kThreads;
      const int i = i0 + (q / KB) * 8;
      ok[u] = q < UNITS && i < ilim;
      coff[u] = ok[u] ? col_off(o, i) : 0;
    }
  }
  // Masked lanes read row min(k, klim - 1) (valid: the first tile starts below klim) and keep
  // zeros, so every stage issues the same loads.
  template <int S>
  __device__ __forceinline__ void load(const Operand& o, const bf16* base, int64_t rowshift, int k0, int klim,
                                       int tid) {
#pragma unroll
    for (int u = 0; u < PER; ++u) {
      const int q = tid + u * kThreads;
      const int kb = q % KB;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int k = k0 + kb * 4 + j;
        const bool valid = ok[u] && k < klim;
        const int kk = k < klim ? k : klim - 1;
        const uint4 v = *reinterpret_cast<const uint4*>(base + row_off(o, kk + rowshift) + coff[u]);
        r[S][u * 4 + j] = valid ? v : make_uint4(0u, 0u, 0u, 0u);
      }
    }
  }
  __device__ __forceinline__ static uint32_t lo2(uint32_t a, uint32_t b) { return (a & 0xffffu) | (b << 16); }
  __device__ __forceinline__ static uint32_t hi2(uint32_t a, uint32_t b) { return (a >> 16) | (b & 0xffff0000u); }
  template <int S>
  __device__ __forceinline__ void store(bf16* lds, int tid) const {
#pragma unroll
    for (int u = 0; u < PER; ++u) {
      const int q = tid + u * kThreads;
      if (q >= UNITS) continue;
      const int kb = q % KB, mb = q / KB;
      const uint4 a = r[S][u * 4 + 0], b = r[S][u * 4 + 1], c = r[S][u * 4 + 2], d = r[S][u * 4 + 3];
      const uint32_t aw[4] = {a.x, a.y, a.z, a.w};
      const uint32_t bw[4] = {b.x, b.y, b.z, b.w};
      const uint32_t cw[4] = {c.x, c.y, c.z, c.w};
      const uint32_t dw[4] = {d.x, d.y, d.z, d.w};
#pragma unroll
      for (int w = 0; w < 4; ++w) {
        uint2 e, f;
        e.x = lo2(aw[w], bw[w]);
        e.y = lo2(cw[w], dw[w]);
        f.x = hi2(aw[w], bw[w]);
        f.y = hi2(cw[w], dw[w]);
        *reinterpret_cast<uint2*>(lds + (mb * 8 + 2 * w) * LDP + kb * 4) = e;
        *reinterpret_cast<uint2*>(lds + (mb * 8 + 2 * w + 1) * LDP + kb * 4) = f;
      }
    }
  }
};

// Uniform interface over the two loaders.
template <int R, int BK, bool T>
struct Loader;
template <int R, int BK>
struct Loader<R, BK, false> {
  LoaderN<R, BK> l;
  __device__ __forceinline__ void init(const Operand& o, const bf16* base, int64_t sh, int i0, int ilim, int tid) {
    l.init(o, base, sh, i0, ilim, tid);
  }
  template <int S>
  __device__ __forceinline__ void load(const Operand& o, const bf16*, int64_t, int k0, int klim, int tid) {
    l.template load<S>(o, k0, klim, tid);
  }
  template <int S>
  __device__ __forceinline__ void store(bf16* lds, int tid) const { l.template store<S>(lds, tid); }
};
template <int R, int BK>
struct Loader<R, BK, true> {
  LoaderT<R, BK> l;
  __device__ __forceinline__ void init(const Operand& o, const bf16* base, int64_t sh, int i0, int ilim, int tid) {
    l.init(o, base, sh, i0, ilim, tid);
  }
  template <int S>
  __device__ __forceinline__ void load(const Operand& o, const bf16* base, int64_t sh, int k0, int klim, int tid) {
    l.template load<S>(o, base, sh, k0, klim, tid);
  }
  template <int S>
  __device__ __forceinline__ void store(bf16* lds, int tid) const { l.template store<S>(lds, tid); }
};

// ------------------------------------------------------------------ output chunks

// Writes W consecutive outputs (row m of the tile space, columns n..n+W-1) applying
// alpha, row_scale, output-row mapping, residual and beta.  vec: 16-byte path allowed.
template <int W>
__device__ __forceinline__ void store_chunk(const Epilogue& e, int g, int m, int n, int N, float* v, bool vec) {
  const float rs = e.row_scale ? e.row_scale[m] : 1.0f;
  int64_t orow = m + (int64_t)g * e.c_growstride;
  if (e.c_ilv) orow = ilv_row(orow, e.c_ilv);
  if (e.c_rows) orow = e.c_rows[orow];
  const int nv = N - n < W ? N - n : W;
#pragma unroll
  for (int t = 0; t < W; ++t) v[t] *= e.alpha * rs;
  if (e.resid) {
    const float* rp = e.resid + orow * e.ld_resid + n;
    if (vec && nv == W) {
#pragma unroll
      for (int t = 0; t < W; t += 4) {
        const float4 x = *reinterpret_cast<const float4*>(rp + t);
        v[t] += x.x; v[t + 1] += x.y; v[t + 2] += x.z; v[t + 3] += x.w;
      }
    } else {
      for (int t = 0; t < nv; ++t) v[t] += rp[t];
    }
  }
  // W-column chunks start at multiples of W and never cross a 32-column run of the interleave
  const int64_t ocol = e.c_col_ilv ? ilv_row((int64_t)g * e.c_gstride + n, e.c_col_ilv) : (int64_t)g * e.c_gstride + n;
  if (e.c_f32) {
    float* cp = reinterpret_cast<float*>(e.c) + orow * e.ldc + ocol;
    if (vec && nv == W) {
#pragma unroll
      for (int t = 0; t < W; t += 4) {
        if (e.beta != 0.0f) {
          const float4 o = *reinterpret_cast<const float4*>(cp + t);
          v[t] += e.beta * o.x; v[t + 1] += e.beta * o.y; v[t + 2] += e.beta * o.z; v[t + 3] += e.beta * o.w;
        }
        *reinterpret_cast<float4*>(cp + t) = make_float4(v[t], v[t + 1], v[t + 2], v[t + 3]);
      }
    } else {
      for (int t = 0; t < nv; ++t) cp[t] = v[t] + (e.beta != 0.0f ? e.beta * cp[t] : 0.0f);
    }
  } else {
    bf16* cp = reinterpret_cast<bf16*>(e.c) + orow * e.ldc + ocol;
    if (vec && nv == W && W == 8) {
      if (e.beta != 0.0f) {
        const uint4 o = *reinterpret_cast<const uint4*>(cp);
        const uint32_t ow[4] = {o.x, o.y, o.z, o.w};
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          v[2 * t] += e.beta * __uint_as_float(ow[t] << 16);
          v[2 * t + 1] += e.beta * __uint_as_float(ow[t] & 0xffff0000u);
        }
      }
      uint4 o;
      o.x = pack_bf2(v[0], v[1]);
      o.y = pack_bf2(v[2], v[3]);
      o.z = pack_bf2(v[4], v[5]);
      o.w = pack_bf2(v[6], v[7]);
      *reinterpret_cast<uint4*>(cp) = o;
    } else {
      for (int t = 0; t < nv; ++t) cp[t] = f2bf(v[t] + (e.beta != 0.0f ? e.beta * bf2f(cp[t]) : 0.0f));
    }
  }
}

struct EpiFlags {
  int vec;  // 16-byte stores / residual loads are aligned
};

// ------------------------------------------------------------------ kernel

// Tiles larger than 128x128 keep one workgroup per CU (their LDS and accumulators fill it).
// Row slices of the direct-load kernels' staged epilogue: two when each wave's rows fit one half.
template <int BM, int WM, int DLS>
constexpr int dl_slices() {
  return (DLS > 0 && BM >= 64 && ((BM / 2) % (BM / WM)) == 0) ? 2 : 1;
}

template <int BM, int BN, int BK = 64, int DLS = 0, int WM = 2>
constexpr int wg_per_cu() {
  if constexpr (DLS > 0) {
    // direct-load kernels: as many workgroups as their LDS allows, at most 4
    constexpr int rows = BM / dl_slices<BM, WM, DLS>();
    constexpr int lds = DLS * (BM + BN) * BK * 2 > rows * (BN + 8) * 4 ? DLS * (BM + BN) * BK * 2
                                                                      : rows * (BN + 8) * 4;
    constexpr int n = 163840 / lds;
    return n < 1 ? 1 : (n > 4 ? 4 : n);
  }
  return BM * BN > 128 * 128 ? 1 : 2;
}

// Direct-to-LDS stage layout: a tile row holds BK k values = CPR chunks of 16 bytes, chunk c
// stored at position c ^ swz(row), so that 32 lanes reading the same logical chunk of 32
// consecutive rows (the MFMA operand reads) spread over all LDS banks.  Both swizzles were
// chosen by measurement (SQ_LDS_BANK_CONFLICT of ds_read_b128 patterns on gfx950: zero
// conflicts for these two, conflicts for the unswizzled rows and for (row & 7), (row >> 1) & 3).
template <int CPR>
__device__ __forceinline__ int dl_swz(int row) {
  if constexpr (CPR == 8) return (row ^ (row >> 3)) & 7;  // 128-byte rows
  else return (row >> 2) & 3;                             // 64-byte rows
}

// 16 bytes per lane from global memory straight into LDS at (LDS base + 16 * lane); the LDS
// base must be wave-uniform.  The host pass of the compiler has no such builtin and never
// runs kernel bodies, so it only sees the declaration.
__device__ __forceinline__ void lds_dma16(const void* src, void* lds_base) {
#if defined(__HIP_DEVICE_COMPILE__)
  __builtin_amdgcn_global_load_lds(src, lds_base, 16, 0, 0);
#else
  (void)src;
  (void)lds_base;
#endif
}

// Four bf16 of a k-major LDS tile, transposed across the 16 lanes of each lane group
// (ds_read_b64_tr_b16, gfx950).  Measured lane layout: within a group of 16 lanes, lane i
// receives element (i % 4) of the 8-byte rows that lanes 4j + i / 4 (j = 0..3) point at, in j
// order.  So if lane s of the group points at k-row (kb + s / 4) and columns (cb + 4 (s % 4))..+3,
// lane i gets column cb + i at k-rows kb..kb + 3: an MFMA operand fragment.
typedef short short4_v __attribute__((ext_vector_type(4)));

// 16 zero bytes in global memory: the source of direct loads past the end of a k range (a
// layout-T tile's rows beyond the group of a grouped-K problem), so LDS gets exact zeros.
__device__ __align__(16) unsigned int kDlZero[4] = {0u, 0u, 0u, 0u};  // never written
__device__ __forceinline__ short4_v lds_read_tr4(const unsigned char* lds_byte_ptr) {
#if defined(__HIP_DEVICE_COMPILE__)
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) short4_v*)lds_byte_ptr);
#else
  (void)lds_byte_ptr;
  return short4_v{0, 0, 0, 0};
#endif
}

// One operand of the direct-to-LDS main loop: R tile rows (the output index i) by BK k per
// stage.  Layout N (k contiguous in memory): LDS rows are i, BK * 2 bytes each, chunk c (8 k)
// at c ^ dl_swz(i).  Layout T (i contiguous): LDS rows are k, R * 2 bytes each, chunk c (8 i)
// at c ^ tr_swz(k); the MFMA fragments then come out of ds_read_b64_tr_b16 pairs.
template <int R, int BK, bool T>
struct DlOperand {
  static constexpr int ROWB = T ? R * 2 : BK * 2;  // bytes per LDS row
  static constexpr int CPR = ROWB / 16;            // 16-byte chunks per LDS row
  static constexpr int BYTES = R * BK * 2;
  static constexpr int INS = BYTES / 16 / kThreads;  // loads per thread per stage
  static_assert(INS >= 1, "tile too small for one load per thread");
  static_assert(!T || CPR >= 4, "layout-T tiles need at least 32 columns");

  // k-rows r, r+1, r+2, r+3 of a layout-T tile land in four distinct 64-byte windows of the
  // row (XOR of the window index), so the 8 rows read by one ds_read_b64_tr_b16 spread over
  // the banks.
  __device__ __forceinline__ static int tr_swz(int krow) { return (krow % (CPR / 4)) * 4; }

  const bf16* ptr[INS];
  int off[INS];  // N: k offset of the chunk; T: k-row of the load within the stage

  __device__ __forceinline__ void init(const Operand& o, const bf16* base, int64_t shift, int i0, int ilim,
                                       int tid) {
#pragma unroll
    for (int u = 0; u < INS; ++u) {
      const int q = u * kThreads + tid, row = q / CPR, pc = q % CPR;
      if constexpr (!T) {
        int i = i0 + row;
        if (i >= ilim) i = ilim - 1;
        ptr[u] = base + row_off(o, i + shift);
        off[u] = (pc ^ dl_swz<CPR>(row)) * 8;
      } else {
        int i = i0 + (pc ^ tr_swz(row)) * 8;
        if (i + 8 > ilim) i = ilim - 8;  // layout-T extents are multiples of 8
        ptr[u] = base + col_off(o, i);
        off[u] = row;
      }
    }
  }
  // global source of load u for the stage starting at k0 (k rows from klim on read zeros;
  // layout-N k ranges are whole stages)
  __device__ __forceinline__ const void* src(const Operand& o, int64_t shift, int k0, int klim, int u,
                                             bool plain) const {
    if constexpr (!T) {
      return ptr[u] + (plain ? (int64_t)(k0 + off[u]) : col_off(o, k0 + off[u]));
    } else {
      const int k = k0 + off[u];
      if (k >= klim) return kDlZero;
      return ptr[u] + row_off(o, (int64_t)k + shift);
    }
  }
  // per-lane fragment addresses of the 32-row blocks of this wave (rows rb + 32 b)
  template <int NB>
  __device__ __forceinline__ static void frag_offsets(int rb, int lane, int (&fo)[NB], int (&fs)[NB]) {
#pragma unroll
    for (int b = 0; b < NB; ++b) {
      if constexpr (!T) {
        const int r = rb + 32 * b + (lane & 31);
        fo[b] = r * ROWB;
        fs[b] = dl_swz<CPR>(r);
      } else {
        const int g = lane >> 4, s = lane & 15;
        const int kr = 8 * (g >> 1) + (s >> 2);           // k-row of this lane's 8-byte read
        const int col = rb + 32 * b + 16 * (g & 1) + 4 * (s & 3);
        fo[b] = kr * ROWB + (((col >> 3) ^ tr_swz(kr)) << 4) + (col & 7) * 2;
        fs[b] = 0;
      }
    }
  }
  // MFMA operand of block b at k-step ks (16 k)
  __device__ __forceinline__ static bf16x8_v frag(const unsigned char* st, int fo, int fs, int ks, int lane) {
    if constexpr (!T) {
      const int c = ks * 2 + (lane >> 5);
      return *reinterpret_cast<const bf16x8_v*>(st + fo + ((c ^ fs) << 4));
    } else {
      const short4_v lo = lds_read_tr4(st + fo + (ks * 16) * ROWB);
      const short4_v hi = lds_read_tr4(st + fo + (ks * 16 + 4) * ROWB);
      typedef short short8_v __attribute__((ext_vector_type(8)));
      const short8_v v = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
      return __builtin_bit_cast(bf16x8_v, v);
    }
  }
};

// s_waitcnt with vmcnt <= n and the other counters unconstrained (gfx9 encoding).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

template <int BM, int BN, int BK, int WM, int WN, bool AT, bool BT, int EPI, bool DUALA = false, int DLS = 0>
__global__ void __launch_bounds__(256, (wg_per_cu<BM, BN, BK, DLS, WM>())) gemm_kernel(GemmArgs p, EpiFlags fl) {
  static_assert(!DUALA || (EPI == EPI_SWIGLU_FWD && !AT), "dual-A is a SwiGLU-forward layout-N mode");
  static_assert(DLS == 0 || (!DUALA && (BK == 64 || BK == 32) && DLS >= 2 && DLS <= 4),
                "direct-to-LDS loads: BK 32 or 64, 2 to 4 stages");
  constexpr int LDP = BK + 8;
  constexpr int WTM = BM / WM, WTN = BN / WN;
  constexpr int TM = WTM / 32, TN = WTN / 32;
  static_assert(WM * WN == 4, "4 waves per workgroup");
  static_assert(TM >= 1 && TN >= 1, "wave tile must hold a 32x32 block");

  extern __shared__ __align__(16) unsigned char smem_raw[];
  // LDS buffers are addressed as offsets from the shared base (a runtime-selected
  // pointer would lose the LDS address space and turn every access into a flat op)
  bf16* smem = reinterpret_cast<bf16*>(smem_raw);
  constexpr int A_TILE = BM * LDP;
  constexpr int A_STAGE = (DUALA ? 2 : 1) * A_TILE, B_STAGE = BN * LDP, B_BASE = 2 * A_STAGE;
  __shared__ int s_tile[3];

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int wm = wave / WN, wn = wave % WN;

  int g = 0, m0 = 0, n0 = 0, mlim = p.M, kbeg = 0, kend = p.K;
  float* partial_dst = nullptr;  // fp32 [M, N] partial of this work item (split-K / chunked group)
  if (p.mode == MODE_GROUP_M) {
    if (tid < 64) {
      if (tid == 0) s_tile[0] = -1;
      const int x = blockIdx.x;
      int base = 0;
      for (int c0 = 0; c0 < p.G; c0 += 64) {
        const int gg = c0 + tid;
        int cnt = 0;
        if (gg < p.G) cnt = (p.goff[gg + 1] - p.goff[gg] + BM - 1) / BM;
        int incl = cnt;
#pragma unroll
        for (int off = 1; off < 64; off <<= 1) {
          const int y = __shfl_up(incl, off, 64);
          if (tid >= off) incl += y;
        }
        const int excl = incl - cnt;
        if (cnt > 0 && x >= base + excl && x < base + incl) {
          s_tile[0] = gg;
          s_tile[1] = x - base - excl;
        }
        base += __shfl(incl, 63, 64);
      }
    }
    __syncthreads();
    g = s_tile[0];
    if (g < 0) return;
    mlim = p.goff[g + 1];
    m0 = p.goff[g] + s_tile[1] * BM;
    n0 = blockIdx.y * BN;
  } else if (p.mode == MODE_GROUP_K) {
    if (p.gk_chunk > 0) {
      // work item blockIdx.z -> (group, chunk): prefix sums of the groups' chunk counts, 64 groups
      // per step; workgroup (0, 0, 0) also writes the chunk starts gk_first[0..G] for the
      // partial-sum kernel that runs after this one
      const int item = blockIdx.z;
      const bool writer = blockIdx.x == 0 && blockIdx.y == 0 && blockIdx.z == 0;
      if (tid < 64) {
        if (tid == 0) s_tile[0] = -1;
        int base = 0;
        for (int c0 = 0; c0 < p.G; c0 += 64) {
          const int gg = c0 + tid;
          // an empty group still takes one work item: its empty k range stores the epilogue of
          // a zero sum, so every group's output is written by this kernel
          int cnt = 0;
          if (gg < p.G) {
            cnt = (p.goff[gg + 1] - p.goff[gg] + p.gk_chunk - 1) / p.gk_chunk;
            if (cnt < 1) cnt = 1;
          }
          int incl = cnt;
#pragma unroll
          for (int off = 1; off < 64; off <<= 1) {
            const int y = __shfl_up(incl, off, 64);
            if (tid >= off) incl += y;
          }
          const int excl = incl - cnt;
          if (writer && gg < p.G) const_cast<int32_t*>(p.gk_first)[gg] = base + excl;
          if (cnt > 0 && item >= base + excl && item < base + incl) {
            s_tile[0] = gg;
            s_tile[1] = item - base - excl;
            s_tile[2] = cnt;
          }
          base += __shfl(incl, 63, 64);
        }
        if (writer && tid == 0) const_cast<int32_t*>(p.gk_first)[p.G] = base;
      }
      __syncthreads();
      g = s_tile[0];
      if (g < 0) return;  // uniform per workgroup
      const int c = s_tile[1];
      kbeg = p.goff[g] + c * p.gk_chunk;
      kend = kbeg + p.gk_chunk < p.goff[g + 1] ? kbeg + p.gk_chunk : p.goff[g + 1];
      if (s_tile[2] > 1) partial_dst = p.gk_part + (int64_t)item * p.M * p.N;
    } else {
      g = blockIdx.z;
      kbeg = p.goff[g];
      kend = p.goff[g + 1];
    }
    m0 = blockIdx.x * BM;
    n0 = blockIdx.y * BN;
  } else {
    // XCD-aware order: dispatch id d runs on XCD d % 8; give each XCD a contiguous
    // band of tiles in m-major order so its L2 keeps the A panel resident.
    const int gx = gridDim.x, gy = gridDim.y, total = gx * gy;
    int lin = blockIdx.y * gx + blockIdx.x;
    if ((total & 7) == 0) lin = (lin & 7) * (total >> 3) + (lin >> 3);
    m0 = (lin / gy) * BM;
    n0 = (lin % gy) * BN;
    if (p.splits > 1) {
      const int split = blockIdx.z;
      kbeg = split * p.k_chunk;
      kend = kbeg + p.k_chunk < p.K ? kbeg + p.k_chunk : p.K;
      partial_dst = p.splitk_ws + (int64_t)split * p.M * p.N;
    }
  }

  const bf16* abase = p.a.ptr + (int64_t)g * p.a.gstride;
  const bf16* bbase = p.b.ptr + (int64_t)g * p.b.gstride;
  const int64_t ashift = (int64_t)g * p.a.growstride;
  const int64_t bshift = (int64_t)g * p.b.growstride;

  f32x16_v acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

  if constexpr (DLS > 0) {
    // Global -> LDS without registers (global_load_lds_dwordx4): load u of thread tid fills
    // 16-byte unit q = u * 256 + tid of the operand's stage tile (see DlOperand for the row /
    // chunk layouts).  Tile rows or columns past the operand's extent re-read the last valid
    // ones; their results are never stored.  The k range is a multiple of BK.
    using OpA = DlOperand<BM, BK, AT>;
    using OpB = DlOperand<BN, BK, BT>;
    constexpr int A_INS = OpA::INS, B_INS = OpB::INS;
    constexpr int A_BYTES = OpA::BYTES, STAGE = OpA::BYTES + OpB::BYTES;
    const int wv = __builtin_amdgcn_readfirstlane(wave);
    OpA la;
    OpB lb;
    la.init(p.a, abase, ashift, m0, mlim, tid);
    lb.init(p.b, bbase, bshift, n0, p.N, tid);
    const bool plain_cols = p.a.cdiv == 0 && p.b.cdiv == 0;  // uniform: layout-N k offsets are affine
    auto issue = [&](int stage, int t) {
      const int k0 = kbeg + t * BK;
      unsigned char* dst = smem_raw + stage * STAGE + wv * 1024;
#pragma unroll
      for (int u = 0; u < A_INS; ++u) lds_dma16(la.src(p.a, ashift, k0, kend, u, plain_cols), dst + u * 4096);
#pragma unroll
      for (int u = 0; u < B_INS; ++u)
        lds_dma16(lb.src(p.b, bshift, k0, kend, u, plain_cols), dst + A_BYTES + u * 4096);
    };
    // fragment addresses of this lane
    int aoff[TM], asw[TM], boff[TN], bsw[TN];
    OpA::frag_offsets(wm * WTM, lane, aoff, asw);
    OpB::frag_offsets(wn * WTN, lane, boff, bsw);
    auto compute = [&](int stage) {
      const unsigned char* st = smem_raw + stage * STAGE;
#pragma unroll
      for (int ks = 0; ks < BK / 16; ++ks) {
        bf16x8_v af[TM], bfr[TN];
#pragma unroll
        for (int i = 0; i < TM; ++i) af[i] = OpA::frag(st, aoff[i], asw[i], ks, lane);
#pragma unroll
        for (int j = 0; j < TN; ++j) bfr[j] = OpB::frag(st + A_BYTES, boff[j], bsw[j], ks, lane);
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
          for (int j = 0; j < TN; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[i], bfr[j], acc[i][j], 0, 0, 0);
      }
    };
    // whole stages; a grouped-K tail (both operands layout T) reads zero rows past kend
    const int nk = kend > kbeg ? (kend - kbeg + BK - 1) / BK : 0;
#pragma unroll
    for (int t = 0; t < DLS - 1; ++t)
      if (t < nk) issue(t, t);
    int stage = 0;
    for (int kt = 0; kt < nk; ++kt) {
      // tile kt has landed once at most the (DLS - 2) younger tiles' loads are in flight
      if constexpr (DLS == 4) {
        if (kt + 2 < nk) wait_vmcnt<2 * (A_INS + B_INS)>();
        else if (kt + 1 < nk) wait_vmcnt<A_INS + B_INS>();
        else wait_vmcnt<0>();
      } else if constexpr (DLS == 3) {
        if (kt + 1 < nk) wait_vmcnt<A_INS + B_INS>(); else wait_vmcnt<0>();
      } else {
        wait_vmcnt<0>();
      }
      __syncthreads();  // tile kt visible to all waves; every wave is done with tile kt - 1
      if (kt + DLS - 1 < nk) {
        int ns = stage + DLS - 1;
        if (ns >= DLS) ns -= DLS;
        issue(ns, kt + DLS - 1);
      }
      compute(stage);
      stage = stage + 1 == DLS ? 0 : stage + 1;
    }
    __syncthreads();  // the epilogue reuses the stage buffers
  } else {
    Loader<BM, BK, AT> la;
    Loader<BM, BK, AT> la2;  // DUALA: gate half of A
    Loader<BN, BK, BT> lb;
    la.init(p.a, abase, ashift, m0, mlim, tid);
    if constexpr (DUALA) la2.init(p.a, abase, ashift, m0, mlim, tid);
    lb.init(p.b, bbase, bshift, n0, p.N, tid);
    const int nk = kend > kbeg ? (kend - kbeg + BK - 1) / BK : 0;
    const int ko2 = p.a_koff2;

    // Pipeline: tile t's payload sits in register set t % 2 and LDS buffer t % 2.  While tile t
    // is multiplied out of LDS, tile t + 2 is being fetched into the set tile t came through
    // and tile t + 1 (fetched one step earlier) is written to the other LDS buffer, so global
    // latency is covered by two compute steps.
    auto load_tile = [&](auto stage, int t) {
      constexpr int S = decltype(stage)::value;
      const int k0 = kbeg + t * BK;
      la.template load<S>(p.a, abase, ashift, k0, kend, tid);
      if constexpr (DUALA) la2.template load<S>(p.a, abase, ashift, k0 + ko2, kend + ko2, tid);
      lb.template load<S>(p.b, bbase, bshift, k0, kend, tid);
    };
    auto store_tile = [&](auto stage) {
      constexpr int S = decltype(stage)::value;
      la.template store<S>(smem + S * A_STAGE, tid);
      if constexpr (DUALA) la2.template store<S>(smem + S * A_STAGE + A_TILE, tid);
      lb.template store<S>(smem + B_BASE + S * B_STAGE, tid);
    };
    auto compute = [&](auto stage) {
      constexpr int S = decltype(stage)::value;
      const bf16* a_s = smem + S * A_STAGE;
      const bf16* b_s = smem + B_BASE + S * B_STAGE;
#pragma unroll
      for (int ks = 0; ks < BK / 16; ++ks) {
        bf16x8_v af[TM], ag[DUALA ? TM : 1], bfr[TN];
        const int kof = ks * 16 + (lane >> 5) * 8;
#pragma unroll
        for (int i = 0; i < TM; ++i) {
          af[i] = *reinterpret_cast<const bf16x8_v*>(a_s + (wm * WTM + i * 32 + (lane & 31)) * LDP + kof);
          if constexpr (DUALA)
            ag[i] = *reinterpret_cast<const bf16x8_v*>(a_s + A_TILE + (wm * WTM + i * 32 + (lane & 31)) * LDP + kof);
        }
#pragma unroll
        for (int j = 0; j < TN; ++j)
          bfr[j] = *reinterpret_cast<const bf16x8_v*>(b_s + (wn * WTN + j * 32 + (lane & 31)) * LDP + kof);
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
          for (int j = 0; j < TN; ++j) {
            // DUALA: odd column blocks are gate blocks and take the second A code
            const bf16x8_v& a_op = (DUALA && (j & 1)) ? ag[DUALA ? i : 0] : af[i];
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a_op, bfr[j], acc[i][j], 0, 0, 0);
          }
      }
    };
    using S0 = std::integral_constant<int, 0>;
    using S1 = std::integral_constant<int, 1>;
    if (nk > 0) {
      load_tile(S0{}, 0);
      load_tile(S1{}, 1);
      store_tile(S0{});
    }
    __syncthreads();
    for (int kt = 0; kt < nk; kt += 2) {
      load_tile(S0{}, kt + 2);
      compute(S0{});
      if (kt + 1 < nk) store_tile(S1{});
      __syncthreads();
      if (kt + 1 >= nk) break;
      load_tile(S1{}, kt + 3);
      compute(S1{});
      if (kt + 2 < nk) store_tile(S0{});
      __syncthreads();
    }

  }

  // ---------------------------------------------------------------- epilogues (LDS staged)
  const Epilogue& e = p.epi;
  const int rbase = wm * WTM + (lane >> 5) * 4;  // + i*32 + (r>>2)*8 + (r&3)
  const int cbase = wn * WTN + (lane & 31);      // + j*32

  if constexpr (EPI == EPI_STORE) {
    // the direct-load kernels stage the tile in NH row slices so their LDS stays small
    constexpr int CP = BN + 8, NH = dl_slices<BM, WM, DLS>(), HR = BM / NH;
    static_assert(HR % WTM == 0, "a wave's rows lie in one slice");
    float* Cs = reinterpret_cast<float*>(smem_raw);
    for (int h = 0; h < NH; ++h) {
      if (h > 0) __syncthreads();  // the previous slice has been written out
      if ((wm * WTM) / HR == h) {
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
          for (int j = 0; j < TN; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r)
              Cs[(rbase - h * HR + i * 32 + (r >> 2) * 8 + (r & 3)) * CP + cbase + j * 32] = acc[i][j][r];
      }
      __syncthreads();
      const int mh = m0 + h * HR;
      if (partial_dst) {
        // fp32 partial of this k range, plain [M, N]
        float* ws = partial_dst;
        constexpr int CH = BN / 4;
        for (int c = tid; c < HR * CH; c += kThreads) {
          const int row = c / CH, cc = (c % CH) * 4;
          const int m = mh + row, n = n0 + cc;
          if (m >= mlim || n >= p.N) continue;
          const float* src = Cs + row * CP + cc;
          float* dst = ws + (int64_t)m * p.N + n;
          if (fl.vec && n + 4 <= p.N) {
            *reinterpret_cast<float4*>(dst) = *reinterpret_cast<const float4*>(src);
          } else {
            for (int t = 0; t < 4 && n + t < p.N; ++t) dst[t] = src[t];
          }
        }
      } else if (e.c_f32) {
        constexpr int CH = BN / 4;
        for (int c = tid; c < HR * CH; c += kThreads) {
          const int row = c / CH, cc = (c % CH) * 4;
          const int m = mh + row, n = n0 + cc;
          if (m >= mlim || n >= p.N) continue;
          float v[4];
          const float4 x = *reinterpret_cast<const float4*>(Cs + row * CP + cc);
          v[0] = x.x; v[1] = x.y; v[2] = x.z; v[3] = x.w;
          store_chunk<4>(e, g, m, n, p.N, v, fl.vec);
        }
      } else {
        constexpr int CH = BN / 8;
        for (int c = tid; c < HR * CH; c += kThreads) {
          const int row = c / CH, cc = (c % CH) * 8;
          const int m = mh + row, n = n0 + cc;
          if (m >= mlim || n >= p.N) continue;
          float v[8];
          const float4 x = *reinterpret_cast<const float4*>(Cs + row * CP + cc);
          const float4 y = *reinterpret_cast<const float4*>(Cs + row * CP + cc + 4);
          v[0] = x.x; v[1] = x.y; v[2] = x.z; v[3] = x.w;
          v[4] = y.x; v[5] = y.y; v[6] = y.z; v[7] = y.w;
          store_chunk<8>(e, g, m, n, p.N, v, fl.vec);
        }
      }
    }
  } else if constexpr (EPI == EPI_SWIGLU_FWD) {
    // Column blocks of 32 alternate up / gate for the same 32 neurons, so the
    // up value and its gate sit in the same register of neighbouring blocks.
    static_assert(TN % 2 == 0, "SwiGLU epilogue pairs column blocks");
    constexpr int HP = BN + 8, ZP = BN / 2 + 8;
    bf16* Us = smem;
    bf16* Zs = smem + BM * HP;
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int rl = rbase + i * 32 + (r >> 2) * 8 + (r & 3);
        const int m = m0 + rl;
        const float rs = (e.row_scale && m < mlim) ? e.row_scale[m] : 1.0f;
#pragma unroll
        for (int jp = 0; jp < TN / 2; ++jp) {
          const int cl = cbase + jp * 64;  // up column (tile-local)
          const bf16 ub = f2bf(acc[i][2 * jp][r]);
          const bf16 gb = f2bf(acc[i][2 * jp + 1][r]);
          const float up = bf2f(ub), gt = bf2f(gb);
          Us[rl * HP + cl] = ub;
          Us[rl * HP + cl + 32] = gb;
          Zs[rl * ZP + (cl >> 6) * 32 + (cl & 31)] = f2bf(up * gt * sigmoidf_(gt) * rs);
        }
      }
    __syncthreads();
    {
      constexpr int CH = BN / 8;
      for (int c = tid; c < BM * CH; c += kThreads) {
        const int row = c / CH, cc = (c % CH) * 8;
        const int m = m0 + row, n = n0 + cc;
        if (m >= mlim || n >= p.N) continue;
        *reinterpret_cast<uint4*>(e.ug + (int64_t)m * e.ld_ug + n) = *reinterpret_cast<const uint4*>(Us + row * HP + cc);
      }
    }
    {
      constexpr int CH = BN / 16;
      for (int c = tid; c < BM * CH; c += kThreads) {
        const int row = c / CH, cc = (c % CH) * 8;
        const int m = m0 + row, nz = n0 / 2 + cc;
        if (m >= mlim || nz >= p.N / 2) continue;
        *reinterpret_cast<uint4*>(e.z + (int64_t)m * e.ld_z + nz) = *reinterpret_cast<const uint4*>(Zs + row * ZP + cc);
      }
    }
  } else if constexpr (EPI == EPI_SWIGLU_BWD) {
    static_assert(WN == 1, "row reduction needs the whole N range in one wave");
    // UG tile of this block: rows m0.., columns [(n0/32)*64, +2*BN) of the interleaved layout
    constexpr int HP = 2 * BN + 8;
    bf16* Us = smem;
    const int64_t ucol0 = (int64_t)(n0 >> 5) * 64;
    const int ucols = 2 * (p.N - n0 < BN ? p.N - n0 : BN);
    {
      constexpr int CH = 2 * BN / 8;
      for (int c = tid; c < BM * CH; c += kThreads) {
        const int row = c / CH, cc = (c % CH) * 8;
        const int m = m0 + row;
        uint4 v = make_uint4(0u, 0u, 0u, 0u);
        if (m < mlim && cc < ucols) v = *reinterpret_cast<const uint4*>(e.ug_in + (int64_t)m * e.ld_ug + ucol0 + cc);
        *reinterpret_cast<uint4*>(Us + row * HP + cc) = v;
      }
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int rl = rbase + i * 32 + (r >> 2) * 8 + (r & 3);
        const int m = m0 + rl;
        const bool mok = m < mlim;
        const float rs = (mok && e.row_scale) ? e.row_scale[m] : 1.0f;
        float part = 0.0f;
#pragma unroll
        for (int j = 0; j < TN; ++j) {
          const int nl = cbase + j * 32;  // tile-local neuron
          const int cl = (nl >> 5) * 64 + (nl & 31);
          const float up = bf2f(Us[rl * HP + cl]);
          const float gt = bf2f(Us[rl * HP + cl + 32]);
          const float s = sigmoidf_(gt);
          const float silu = gt * s;
          const float draw = acc[i][j][r];
          const float dz = draw * rs;
          Us[rl * HP + cl] = f2bf(dz * silu);
          Us[rl * HP + cl + 32] = f2bf(dz * up * s * (1.0f + gt * (1.0f - s)));
          part += up * silu * draw;
        }
        if (e.dw_row) {
#pragma unroll
          for (int off = 16; off >= 1; off >>= 1) part += __shfl_xor(part, off, 64);
          if ((lane & 31) == 0 && mok) e.dw_row[m] = part;
        }
      }
    __syncthreads();
    {
      constexpr int CH = 2 * BN / 8;
      for (int c = tid; c < BM * CH; c += kThreads) {
        const int row = c / CH, cc = (c % CH) * 8;
        const int m = m0 + row;
        if (m >= mlim || cc >= ucols) continue;
        *reinterpret_cast<uint4*>(e.ug + (int64_t)m * e.ld_ug + ucol0 + cc) =
            *reinterpret_cast<const uint4*>(Us + row * HP + cc);
      }
    }
  } else if constexpr (EPI == EPI_ROPE_QKV) {
    // Stage the fp32 tile, then each thread rotates and writes 8 consecutive columns of one
    // row: the RoPE pairs (2i, 2i+1) sit inside the chunk, and the chunk's cos / sin values
    // are two 16-byte loads each.
    constexpr int CP = BN + 4, NH = dl_slices<BM, WM, DLS>(), HR = BM / NH;
    static_assert(HR % WTM == 0, "a wave's rows lie in one slice");
    float* Cs = reinterpret_cast<float*>(smem_raw);
    for (int h = 0; h < NH; ++h) {
      if (h > 0) __syncthreads();  // the previous slice has been written out
      if ((wm * WTM) / HR == h) {
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
          for (int j = 0; j < TN; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r)
              Cs[(rbase - h * HR + i * 32 + (r >> 2) * 8 + (r & 3)) * CP + cbase + j * 32] = acc[i][j][r];
      }
      __syncthreads();
      // a thread keeps one 8-column chunk for the whole slice (kThreads % CH == 0), so the
      // column's (part, head, dim) are divided out once and the row's (b, s) advance by steps
      constexpr int CH = BN / 8, RSTEP = kThreads / CH;
      static_assert(kThreads % CH == 0, "fixed column chunk per thread");
      const int cc = (tid % CH) * 8, n = n0 + cc;
      const int part = n / e.dmodel;
      const int within = n - part * e.dmodel;
      const int hh = within / e.hd, dim = within - hh * e.hd;
      int row = tid / CH;
      int m = m0 + h * HR + row;
      int b = m / e.S, s = m - b * e.S;
      for (; row < HR; row += RSTEP, m += RSTEP) {
        if (row > tid / CH) {
          s += RSTEP;
          while (s >= e.S) {
            s -= e.S;
            ++b;
          }
        }
        if (m >= mlim || n >= p.N) continue;
        const float4 x0 = *reinterpret_cast<const float4*>(Cs + row * CP + cc);
        const float4 x1 = *reinterpret_cast<const float4*>(Cs + row * CP + cc + 4);
        float v[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
        if (part < 2) {
          const float* cp = e.cos_t + (int64_t)s * e.hd + dim;
          const float* sp = e.sin_t + (int64_t)s * e.hd + dim;
          const float4 c0 = *reinterpret_cast<const float4*>(cp), c1 = *reinterpret_cast<const float4*>(cp + 4);
          const float4 s0 = *reinterpret_cast<const float4*>(sp), s1 = *reinterpret_cast<const float4*>(sp + 4);
          const float cv[8] = {c0.x, c0.y, c0.z, c0.w, c1.x, c1.y, c1.z, c1.w};
          const float sv[8] = {s0.x, s0.y, s0.z, s0.w, s1.x, s1.y, s1.z, s1.w};
#pragma unroll
          for (int t = 0; t < 4; ++t) {
            const float xe = v[2 * t], xo = v[2 * t + 1];
            v[2 * t] = xe * cv[2 * t] - xo * sv[2 * t];
            v[2 * t + 1] = xo * cv[2 * t + 1] + xe * sv[2 * t + 1];
          }
        }
        uint4 o;
        o.x = pack_bf2(v[0], v[1]);
        o.y = pack_bf2(v[2], v[3]);
        o.z = pack_bf2(v[4], v[5]);
        o.w = pack_bf2(v[6], v[7]);
        bf16* dst = part == 0 ? e.q : (part == 1 ? e.k : e.v);
        *reinterpret_cast<uint4*>(dst + (((int64_t)b * e.H + hh) * e.S + s) * e.hd + dim) = o;
      }
    }
  }
}

// Groups cut into several chunks (or none): add the chunk partials in chunk order and apply
// the EPI_STORE epilogue.  One-chunk groups were stored by the GEMM itself.
// Grid (chunks of 256 column groups of 4 over M x N / 4, G): 32-bit index math only.
__global__ void __launch_bounds__(256) groupk_reduce_kernel(GemmArgs p, EpiFlags fl) {
  const int chunks = (p.N + 3) / 4;
  const int per_g = p.M * chunks;  // < 2^31, checked at launch
  const int r = blockIdx.x * blockDim.x + threadIdx.x;
  if (r >= per_g) return;
  const int g = blockIdx.y;
  const int m = r / chunks, n = (r - m * chunks) * 4;
  const int q0 = p.gk_first[g], q1 = p.gk_first[g + 1];
  if (q1 - q0 == 1) return;
  float v[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  const int64_t plane = (int64_t)p.M * p.N;
  const float* base = p.gk_part + (int64_t)m * p.N + n;
  int q = q0;
  if ((p.N & 3) == 0 && n + 4 <= p.N) {  // rows of the partial planes are 16-byte aligned
    for (; q + 8 <= q1; q += 8) {  // eight partials in flight, added in chunk order
      float4 x[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) x[u] = *reinterpret_cast<const float4*>(base + (q + u) * plane);
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        v[0] += x[u].x;
        v[1] += x[u].y;
        v[2] += x[u].z;
        v[3] += x[u].w;
      }
    }
  }
  for (; q < q1; ++q) {
    const float* src = base + q * plane;
    for (int t = 0; t < 4 && n + t < p.N; ++t) v[t] += src[t];
  }
  store_chunk<4>(p.epi, g, m, n, p.N, v, fl.vec);
}

// Columns n .. n + 3 of row m of the fused QKV product: RoPE on the q / k parts (pairs (2i, 2i+1)
// inside the 4 columns, cos / sin of the row's position), bf16 into q / k / v [B, H, S, hd].
__device__ __forceinline__ void rope_store4(const Epilogue& e, int m, int n, const float* v) {
  const int part = n / e.dmodel;
  const int within = n - part * e.dmodel;
  const int hh = within / e.hd, dim = within - hh * e.hd;
  const int b = m / e.S, s = m - b * e.S;
  float o[4] = {v[0], v[1], v[2], v[3]};
  if (part < 2) {
    const float4 c = *reinterpret_cast<const float4*>(e.cos_t + (int64_t)s * e.hd + dim);
    const float4 sn = *reinterpret_cast<const float4*>(e.sin_t + (int64_t)s * e.hd + dim);
    o[0] = v[0] * c.x - v[1] * sn.x;
    o[1] = v[1] * c.y + v[0] * sn.y;
    o[2] = v[2] * c.z - v[3] * sn.z;
    o[3] = v[3] * c.w + v[2] * sn.w;
  }
  bf16* dst = part == 0 ? e.q : (part == 1 ? e.k : e.v);
  uint2 w;
  w.x = pack_bf2(o[0], o[1]);
  w.y = pack_bf2(o[2], o[3]);
  *reinterpret_cast<uint2*>(dst + (((int64_t)b * e.H + hh) * e.S + s) * e.hd + dim) = w;
}

// Sums split-K partials in split order and applies the EPI_STORE epilogue (or the QKV RoPE store).
__global__ void __launch_bounds__(256) splitk_reduce_kernel(GemmArgs p, EpiFlags fl) {
  const int chunks = (p.N + 3) / 4;
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= (int64_t)p.M * chunks) return;
  const int m = (int)(idx / chunks), n = (int)(idx % chunks) * 4;
  float v[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  const int64_t plane = (int64_t)p.M * p.N;
  const float* base = p.splitk_ws + (int64_t)m * p.N + n;
  if (fl.vec && n + 4 <= p.N) {
    int s = 0;
    for (; s + 4 <= p.splits; s += 4) {  // four partials in flight, added in split order
      float4 x[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) x[u] = *reinterpret_cast<const float4*>(base + (s + u) * plane);
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        v[0] += x[u].x; v[1] += x[u].y; v[2] += x[u].z; v[3] += x[u].w;
      }
    }
    for (; s < p.splits; ++s) {
      const float4 x = *reinterpret_cast<const float4*>(base + s * plane);
      v[0] += x.x; v[1] += x.y; v[2] += x.z; v[3] += x.w;
    }
  } else {
    for (int s = 0; s < p.splits; ++s)
      for (int t = 0; t < 4 && n + t < p.N; ++t) v[t] += base[s * plane + t];
  }
  if (p.epi.q) {  // QKV with RoPE: the split-K path of small-M projections
    rope_store4(p.epi, m, n, v);
    return;
  }
  store_chunk<4>(p.epi, 0, m, n, p.N, v, fl.vec);
}

// Chunk of a GROUP_K group: about half the mean group size, at least 256 rows, so a long
// reduction is shared by a few workgroups (the fp32 partials cost less than the serial k
// steps: measured on the cfg3 cluster-pool weight gradients) and a dominant group by many.
int groupk_chunk(int K, int G) {
  static const int env = [] {  // RTE_GK_CHUNK: fixed chunk for diagnostics
    const char* v = getenv("RTE_GK_CHUNK");
    return v && *v ? atoi(v) : 0;
  }();
  if (env >= 64) return (env + 63) / 64 * 64;
  int64_t c = ((int64_t)K + G - 1) / (G > 0 ? G : 1) / 2;
  if (c < 256) c = 256;
  return (int)((c + 63) / 64 * 64);
}

size_t groupk_first_bytes(int G) { return (((size_t)(G + 1) * 4 + 255) / 256) * 256; }

template <int BM, int BN, int BK, int EPI, bool DUALA = false, int DLS = 0, int WM = 2>
constexpr size_t lds_bytes() {
  constexpr size_t main_loop = DLS > 0 ? (size_t)DLS * (BM + BN) * BK * 2
                                       : (size_t)2 * ((DUALA ? 2 : 1) * BM + BN) * (BK + 8) * 2;
  constexpr size_t rows = BM / dl_slices<BM, WM, DLS>();  // direct-load kernels stage it in slices
  constexpr size_t epi = EPI == EPI_STORE        ? rows * (BN + 8) * 4
                         : EPI == EPI_SWIGLU_FWD ? (size_t)BM * (BN + 8) * 2 + (size_t)BM * (BN / 2 + 8) * 2
                         : EPI == EPI_SWIGLU_BWD ? (size_t)BM * (2 * BN + 8) * 2
                                                 : rows * (BN + 4) * 4;  // EPI_ROPE_QKV: fp32 tile
  return main_loop > epi ? main_loop : epi;
}

template <int BM, int BN, int BK, int WM, int WN, bool AT, bool BT, int EPI, bool DUALA = false, int DLS = 0>
int launch_cfg(const GemmArgs& p0, hipStream_t stream, void* ws, size_t ws_bytes, int vec) {
  constexpr size_t lds = lds_bytes<BM, BN, BK, EPI, DUALA, DLS, WM>();
  auto fn = gemm_kernel<BM, BN, BK, WM, WN, AT, BT, EPI, DUALA, DLS>;
  static bool attr_done = false;
  if (!attr_done) {
    if (lds > 65536) {
      hipError_t err = hipFuncSetAttribute(reinterpret_cast<const void*>(fn),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
      if (err != hipSuccess) {
        set_error("gemm: cannot reserve %zu bytes of LDS: %s", lds, hipGetErrorString(err));
        return -1;
      }
    }
    attr_done = true;
  }
  GemmArgs p = p0;
  EpiFlags fl{vec};
  dim3 grid;
  if (p.mode == MODE_GROUP_M) {
    grid = dim3(p.max_tiles_m, (p.N + BN - 1) / BN, 1);
  } else if (p.mode == MODE_GROUP_K) {
    grid = dim3((p.M + BM - 1) / BM, (p.N + BN - 1) / BN, p.G);
    p.gk_chunk = 0;
    if (EPI == EPI_STORE && ws && p.N % 4 == 0 && p.G >= 1) {
      const size_t need = gemm_groupk_bytes(p.M, p.N, p.K, p.G);
      if (need > 0 && ws_bytes >= need) {
        const int chunk = groupk_chunk(p.K, p.G);
        p.gk_chunk = chunk;
        p.gk_first = static_cast<int32_t*>(ws);
        p.gk_part = reinterpret_cast<float*>(static_cast<char*>(ws) + groupk_first_bytes(p.G));
        grid.z = (unsigned)((p.K + chunk - 1) / chunk + p.G);
      }
    }
  } else {
    grid = dim3((p.M + BM - 1) / BM, (p.N + BN - 1) / BN, 1);
    // split the reduction when the tile grid cannot fill the GPU: about 512 workgroups,
    // at least 128 k per split
    const int tiles = (int)(grid.x * grid.y);
    p.splits = 1;
    static const int target = [] {  // RTE_SPLIT_WG: workgroup target of the split, for diagnostics
      const char* v = getenv("RTE_SPLIT_WG");
      return v && *v && atoi(v) >= 64 ? atoi(v) : 512;
    }();
    if (EPI == EPI_STORE && ws && tiles < 256 && p.K >= 256) {
      int splits = (target + tiles - 1) / tiles;
      const int max_by_k = p.K / 128;
      if (splits > max_by_k) splits = max_by_k;
      if (splits > kMaxSplits) splits = kMaxSplits;
      if (p.splits_forced && splits < 2) splits = 2;
      while (splits > 1 && (size_t)splits * p.M * p.N * sizeof(float) > ws_bytes) --splits;
      if (splits > 1) {
        int kc = (p.K + splits - 1) / splits;
        kc = (kc + BK - 1) / BK * BK;
        p.k_chunk = kc;
        p.splits = (p.K + kc - 1) / kc;
        p.splitk_ws = static_cast<float*>(ws);
        grid.z = p.splits;
      }
    }
  }
  if (grid.x == 0 || grid.y == 0 || grid.z == 0) return 0;
  RTE_REQUIRE(EPI != EPI_STORE || p.epi.c || p.splits > 1, "gemm: the QKV split-K path needs at least two splits");
  hipLaunchKernelGGL(fn, grid, dim3(kThreads), lds, stream, p, fl);
  RTE_TRY(check_launch("gemm"));
  if (p.splits > 1) {
    const int64_t n = (int64_t)p.M * ((p.N + 3) / 4);
    hipLaunchKernelGGL(splitk_reduce_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream, p, fl);
    RTE_TRY(check_launch("gemm_splitk_reduce"));
  }
  if (p.mode == MODE_GROUP_K && p.gk_chunk > 0) {
    const int64_t n = (int64_t)p.M * ((p.N + 3) / 4);
    RTE_REQUIRE(n < ((int64_t)1 << 31) && p.G <= 65535, "gemm: grouped-K output too large");
    hipLaunchKernelGGL(groupk_reduce_kernel, dim3((unsigned)((n + 255) / 256), (unsigned)p.G), dim3(256), 0, stream, p,
                       fl);
    RTE_TRY(check_launch("gemm_groupk_reduce"));
  }
  return 0;
}

template <int BM, int BN, int BK, int WM, int WN, int EPI>
int launch_layouts(const GemmArgs& p, hipStream_t stream, void* ws, size_t ws_bytes, int vec) {
  if (!p.a_t && !p.b_t) return launch_cfg<BM, BN, BK, WM, WN, false, false, EPI>(p, stream, ws, ws_bytes, vec);
  if (!p.a_t && p.b_t) return launch_cfg<BM, BN, BK, WM, WN, false, true, EPI>(p, stream, ws, ws_bytes, vec);
  if (p.a_t && !p.b_t) return launch_cfg<BM, BN, BK, WM, WN, true, false, EPI>(p, stream, ws, ws_bytes, vec);
  return launch_cfg<BM, BN, BK, WM, WN, true, true, EPI>(p, stream, ws, ws_bytes, vec);
}

// ------------------------------------------------------------------ short reductions

// K <= 64 with both operands k-contiguous and the plain store epilogue (low-rank and cluster
// down-projections: K = rank or neurons per cluster).  Such products are bound by their output
// writes, so the kernel drops the shared tile: one wave owns 32 output rows and a run of
// 32-column blocks, loads its MFMA operands straight from global memory (16 bytes per lane per
// 16 k; k past K reads zeros), and sends each 32x32 result block through a wave-private LDS
// patch so every global store is 16 bytes of one row.  Waves never wait for each other; the
// next block's B fragments are loaded before the current block is stored.
constexpr int kSkPitch = 36;  // floats per patch row (144 bytes: 16-byte aligned rows)

__device__ __forceinline__ bf16x8_v ld_frag16(const bf16* p) {
  return __builtin_bit_cast(bf16x8_v, *reinterpret_cast<const uint4*>(p));
}

__device__ __forceinline__ void wave_lds_fence() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

template <int KS>
__global__ void __launch_bounds__(256) gemm_sk_kernel(GemmArgs p, EpiFlags fl, int nch, int cpt) {
  __shared__ __align__(16) float patch[4][32 * kSkPitch];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int half = lane >> 5, l32 = lane & 31;
  const int task = blockIdx.x * 4 + wave;
  const int rb = task / nch, ch = task - rb * nch;
  int g = 0, m0 = 0, mlim = p.M;
  if (p.mode == MODE_GROUP_M) {
    // row block rb -> (group, block within the group): prefix sums of the groups' 32-row
    // block counts, 64 groups per step
    g = -1;
    int local = 0, base = 0;
    for (int c0 = 0; c0 < p.G; c0 += 64) {
      const int gg = c0 + lane;
      const int cnt = gg < p.G ? (p.goff[gg + 1] - p.goff[gg] + 31) / 32 : 0;
      int incl = cnt;
#pragma unroll
      for (int off = 1; off < 64; off <<= 1) {
        const int y = __shfl_up(incl, off, 64);
        if (lane >= off) incl += y;
      }
      const int excl = incl - cnt;
      const unsigned long long hit = __ballot(cnt > 0 && rb >= base + excl && rb < base + incl);
      if (hit) {
        const int l = __ffsll((long long)hit) - 1;
        g = c0 + l;
        local = rb - base - __shfl(excl, l, 64);
        break;
      }
      base += __shfl(incl, 63, 64);
    }
    if (g < 0) return;
    mlim = p.goff[g + 1];
    m0 = p.goff[g] + local * 32;
  } else {
    m0 = rb * 32;
    if (m0 >= p.M) return;
  }
  const bf16* abase = p.a.ptr + (int64_t)g * p.a.gstride;
  const bf16* bbase = p.b.ptr + (int64_t)g * p.b.gstride;
  const int64_t ashift = (int64_t)g * p.a.growstride, bshift = (int64_t)g * p.b.growstride;
  const bf16x8_v zero = __builtin_bit_cast(bf16x8_v, make_uint4(0u, 0u, 0u, 0u));

  bf16x8_v af[KS];
  {
    int m = m0 + l32;
    if (m >= mlim) m = mlim - 1;  // rows past the end re-read the last one; never stored
    const bf16* ap = abase + row_off(p.a, m + ashift);
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      const int k = ks * 16 + half * 8;
      af[ks] = k < p.K ? ld_frag16(ap + col_off(p.a, k)) : zero;
    }
  }
  const int CB = (p.N + 31) / 32;
  const int cb0 = ch * cpt;
  const int cb1 = cb0 + cpt < CB ? cb0 + cpt : CB;
  auto load_b = [&](int cb, bf16x8_v(&bf)[KS]) {
    int n = cb * 32 + l32;
    if (n >= p.N) n = p.N - 1;
    const bf16* bp = bbase + row_off(p.b, n + bshift);
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      const int k = ks * 16 + half * 8;
      bf[ks] = k < p.K ? ld_frag16(bp + col_off(p.b, k)) : zero;
    }
  };
  float* pt = patch[wave];
  bf16x8_v bcur[KS], bnext[KS];
  if (cb0 < cb1) load_b(cb0, bcur);
  for (int cb = cb0; cb < cb1; ++cb) {
    if (cb + 1 < cb1) load_b(cb + 1, bnext);
    f32x16_v acc;
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[r] = 0.0f;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[ks], bcur[ks], acc, 0, 0, 0);
    wave_lds_fence();  // the previous block's patch reads are done
#pragma unroll
    for (int r = 0; r < 16; ++r) pt[(8 * (r >> 2) + 4 * half + (r & 3)) * kSkPitch + l32] = acc[r];
    wave_lds_fence();
#pragma unroll
    for (int q = lane; q < 128; q += 64) {
      const int row = q >> 2, cc = (q & 3) * 8;
      const int m = m0 + row, n = cb * 32 + cc;
      if (m >= mlim || n >= p.N) continue;
      float v[8];
      const float4 x = *reinterpret_cast<const float4*>(pt + row * kSkPitch + cc);
      const float4 y = *reinterpret_cast<const float4*>(pt + row * kSkPitch + cc + 4);
      v[0] = x.x; v[1] = x.y; v[2] = x.z; v[3] = x.w;
      v[4] = y.x; v[5] = y.y; v[6] = y.z; v[7] = y.w;
      store_chunk<8>(p.epi, g, m, n, p.N, v, fl.vec);
    }
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) bcur[ks] = bnext[ks];
  }
}

// Wave tasks: (32-row block, run of cpt column blocks), about 8192 of them (32 waves per CU)
// when the problem has that many blocks.
int launch_sk(const GemmArgs& p, hipStream_t stream, int vec) {
  if (p.M == 0 || p.N == 0) return 0;
  const int CB = (p.N + 31) / 32;
  const int64_t rbound = p.mode == MODE_GROUP_M ? (int64_t)p.M / 32 + p.G + 1 : ((int64_t)p.M + 31) / 32;
  int64_t c = rbound * CB / 8192;
  if (c < 1) c = 1;
  if (c > CB) c = CB;
  const int cpt = (int)c, nch = (CB + cpt - 1) / cpt;
  const int64_t tasks = rbound * nch;
  RTE_REQUIRE(tasks / 4 < (int64_t)1 << 31, "gemm: problem too large for the short-K kernel");
  const dim3 grid((unsigned)((tasks + 3) / 4));
  EpiFlags fl{vec};
  switch ((p.K + 15) / 16) {
    case 1: hipLaunchKernelGGL(gemm_sk_kernel<1>, grid, dim3(256), 0, stream, p, fl, nch, cpt); break;
    case 2: hipLaunchKernelGGL(gemm_sk_kernel<2>, grid, dim3(256), 0, stream, p, fl, nch, cpt); break;
    case 3: hipLaunchKernelGGL(gemm_sk_kernel<3>, grid, dim3(256), 0, stream, p, fl, nch, cpt); break;
    default: hipLaunchKernelGGL(gemm_sk_kernel<4>, grid, dim3(256), 0, stream, p, fl, nch, cpt); break;
  }
  return check_launch("gemm_short_k");
}

// Direct-to-LDS mainloop selection.  Default: K <= 1024 -> BK 32, 2 stages (four workgroups
// per CU: short reductions are latency-bound, occupancy hides it best); longer K -> BK 64,
// 2 stages (fewer barriers per MFMA).  RTE_GEMM_DL overrides it for diagnostics: 0 keeps the
// register-staged loop everywhere; otherwise 128x128 tiles with (BK, stages) = 2: (64, 2),
// 3: (64, 3), 5: (32, 4), 6: (32, 3), 7: (32, 2); 4 = 256x128 tiles, (64, 2).
int dl_env() {
  static int mode = [] {
    const char* v = getenv("RTE_GEMM_DL");
    if (!v || !*v) return -1;
    const int m = atoi(v);
    return (m == 0 || (m >= 2 && m <= 7)) ? m : -1;
  }();
  return mode;
}

int dl_mode(const GemmArgs& p) {
  const int env = dl_env();
  if (env >= 0) return env;
  const int klen = p.splits > 1 ? p.k_chunk : p.K;
  return klen <= 1024 ? 7 : 2;
}

bool dl_ok(const GemmArgs& p) {
  const int mode = dl_mode(p);
  if (mode == 0 || p.a_koff2 || p.K <= 0) return false;
  const int bk = mode >= 5 ? 32 : 64;
  // dense / grouped-M: whole stages over K; grouped-K (both operands layout T): any group sizes
  if (p.mode == MODE_GROUP_K) return p.a_t && p.b_t;
  return p.K % bk == 0;
}

template <int BM, int BK, int DLS, int EPI>
int launch_dl_layouts(const GemmArgs& p, hipStream_t stream, void* ws, size_t ws_bytes, int vec) {
  if (!p.a_t && !p.b_t) return launch_cfg<BM, 128, BK, 2, 2, false, false, EPI, false, DLS>(p, stream, ws, ws_bytes, vec);
  if constexpr (EPI == EPI_STORE) {
    if (!p.a_t) return launch_cfg<BM, 128, BK, 2, 2, false, true, EPI, false, DLS>(p, stream, ws, ws_bytes, vec);
    if (!p.b_t) return launch_cfg<BM, 128, BK, 2, 2, true, false, EPI, false, DLS>(p, stream, ws, ws_bytes, vec);
    return launch_cfg<BM, 128, BK, 2, 2, true, true, EPI, false, DLS>(p, stream, ws, ws_bytes, vec);
  }
  set_error("gemm: direct-load layout-T operands need the plain store epilogue");
  return -1;
}

// Tile height: 128 rows when that already gives two workgroups per CU or when the reduction
// is long enough to split instead (K > 2048), else 64 (dense only: grouped modes keep their
// 128-row tiles).
template <int BK, int DLS, int EPI>
int launch_dl_shape(const GemmArgs& p, hipStream_t stream, void* ws, size_t ws_bytes, int vec) {
  const int64_t tiles128 = (int64_t)((p.M + 127) / 128) * ((p.N + 127) / 128);
  if (p.mode == MODE_DENSE && tiles128 < 512 && p.M > 64 && p.K <= 2048)
    return launch_dl_layouts<64, BK, DLS, EPI>(p, stream, ws, ws_bytes, vec);
  return launch_dl_layouts<128, BK, DLS, EPI>(p, stream, ws, ws_bytes, vec);
}

// Narrow tiles (a 32- or 64-wide side) on the direct-load loop, any operand layouts; BK 64
// (a 32-row tile holds one 16-byte load per thread only at BK 64).
template <int BM, int BN, int WM, int WN>
int launch_dl_narrow(const GemmArgs& p, hipStream_t stream, void* ws, size_t ws_bytes, int vec) {
  if (!p.a_t && !p.b_t) return launch_cfg<BM, BN, 64, WM, WN, false, false, EPI_STORE, false, 2>(p, stream, ws, ws_bytes, vec);
  if (!p.a_t) return launch_cfg<BM, BN, 64, WM, WN, false, true, EPI_STORE, false, 2>(p, stream, ws, ws_bytes, vec);
  if (!p.b_t) return launch_cfg<BM, BN, 64, WM, WN, true, false, EPI_STORE, false, 2>(p, stream, ws, ws_bytes, vec);
  return launch_cfg<BM, BN, 64, WM, WN, true, true, EPI_STORE, false, 2>(p, stream, ws, ws_bytes, vec);
}

template <int EPI>
int launch_dl(const GemmArgs& p, hipStream_t stream, void* ws, size_t ws_bytes, int vec) {
  const bool nn = !p.a_t && !p.b_t;
  switch (nn ? dl_mode(p) : (dl_mode(p) >= 5 ? 7 : 2)) {  // layout T: the two default shapes
    case 3: return launch_cfg<128, 128, 64, 2, 2, false, false, EPI, false, 3>(p, stream, ws, ws_bytes, vec);
    case 4: return launch_cfg<256, 128, 64, 2, 2, false, false, EPI, false, 2>(p, stream, ws, ws_bytes, vec);
    case 5: return launch_cfg<128, 128, 32, 2, 2, false, false, EPI, false, 4>(p, stream, ws, ws_bytes, vec);
    case 6: return launch_cfg<128, 128, 32, 2, 2, false, false, EPI, false, 3>(p, stream, ws, ws_bytes, vec);
    case 7: return launch_dl_shape<32, 2, EPI>(p, stream, ws, ws_bytes, vec);
    default: return launch_dl_shape<64, 2, EPI>(p, stream, ws, ws_bytes, vec);
  }
}

// The SwiGLU epilogue kernels' direct-load loop: whole 64-k stages of layout-N A.
bool dl_whole64(const GemmArgs& p) {
  return dl_mode(p) != 0 && !p.a_koff2 && !p.a_t && p.mode != MODE_GROUP_K && p.K > 0 && p.K % 64 == 0;
}

bool pow2_or_zero(int v) { return v == 0 || (v > 0 && (v & (v - 1)) == 0); }

bool aligned16(const void* ptr) { return ((uintptr_t)ptr & 15) == 0; }

}  // namespace

size_t gemm_groupk_bytes(int M, int N, int K, int G) {
  if (M <= 0 || N <= 0 || K <= 0 || G <= 0) return 0;
  const int chunk = groupk_chunk(K, G);
  const size_t items = (size_t)((K + chunk - 1) / chunk) + (size_t)G;
  return groupk_first_bytes(G) + items * (size_t)M * N * sizeof(float);
}

size_t gemm_splitk_bytes(int M, int N, int K) {
  int splits = K / 128;
  if (splits > kMaxSplits) splits = kMaxSplits;
  if (splits < 2) return 0;
  const size_t b = (size_t)splits * M * N * sizeof(float);
  return b < kMaxSplitBytes ? b : kMaxSplitBytes;  // the launch uses fewer splits to fit
}

int gemm_launch(const GemmArgs& p, int epi_kind, hipStream_t stream, void* ws, size_t ws_bytes) {
  RTE_REQUIRE(p.M >= 0 && p.N >= 0 && p.K >= 0, "gemm: negative size");
  RTE_REQUIRE(p.a.ptr && p.b.ptr, "gemm: null operand");
  // 16-byte vector loads: every contiguous run the kernel reads must hold whole
  // groups of 8 elements.
  if (!p.a_t) RTE_REQUIRE(p.K % 8 == 0 || p.mode == MODE_GROUP_K, "gemm: K %% 8 != 0 for layout-N A");
  if (!p.b_t) RTE_REQUIRE(p.K % 8 == 0 || p.mode == MODE_GROUP_K, "gemm: K %% 8 != 0 for layout-N B");
  if (p.a_t) RTE_REQUIRE(p.M % 8 == 0, "gemm: M %% 8 != 0 for layout-T A");
  if (p.b_t) RTE_REQUIRE(p.N % 8 == 0, "gemm: N %% 8 != 0 for layout-T B");
  if (p.mode == MODE_GROUP_K) RTE_REQUIRE(p.a_t && p.b_t, "gemm: GROUP_K needs both operands in layout T");
  if (p.mode == MODE_GROUP_M) RTE_REQUIRE(!p.a_t, "gemm: GROUP_M needs layout-N A");
  if (p.mode != MODE_DENSE) RTE_REQUIRE(p.goff && p.G >= 1, "gemm: grouped mode needs offsets");
  for (const Operand* o : {&p.a, &p.b}) {
    RTE_REQUIRE(aligned16(o->ptr), "gemm: operand pointer must be 16-byte aligned");
    RTE_REQUIRE(o->ld % 8 == 0 && o->gstride % 8 == 0 && o->rs_hi % 8 == 0 && o->cs_hi % 8 == 0,
                "gemm: operand strides must be multiples of 8 elements");
    RTE_REQUIRE(o->cdiv % 8 == 0, "gemm: split column segments must be multiples of 8");
    RTE_REQUIRE(pow2_or_zero(o->rdiv) && pow2_or_zero(o->cdiv), "gemm: split sizes must be powers of two");
  }
  const Epilogue& e = p.epi;
  int vec = 1;
  if (epi_kind == EPI_STORE) {
    // no C with the RoPE outputs set: the split-K partials are stored as QKV by the reduce
    RTE_REQUIRE(e.c || (e.q && p.splits_forced), "gemm: null output");
    const int esz = e.c_f32 ? 4 : 2;
    vec = aligned16(e.c) && (e.ldc * esz) % 16 == 0 && (e.c_gstride * esz) % 16 == 0 &&
          ((int64_t)e.c_col_ilv * esz) % 16 == 0;
    RTE_REQUIRE(!e.c_col_ilv || (e.c_gstride % 32 == 0 && !e.c_ilv), "gemm: column interleave needs 32-column groups");
    if (e.resid) vec = vec && aligned16(e.resid) && e.ld_resid % 4 == 0;
  } else if (epi_kind == EPI_SWIGLU_FWD) {
    RTE_REQUIRE(aligned16(e.ug) && aligned16(e.z) && e.ld_ug % 8 == 0 && e.ld_z % 8 == 0,
                "gemm: SwiGLU outputs must be 16-byte aligned with ld %% 8 == 0");
  } else if (epi_kind == EPI_SWIGLU_BWD) {
    RTE_REQUIRE(aligned16(e.ug) && aligned16(e.ug_in) && e.ld_ug % 8 == 0,
                "gemm: SwiGLU buffers must be 16-byte aligned with ld %% 8 == 0");
  } else if (epi_kind == EPI_ROPE_QKV) {
    RTE_REQUIRE(aligned16(e.q) && aligned16(e.k) && aligned16(e.v) && e.hd % 8 == 0,
                "gemm: QKV outputs must be 16-byte aligned with head_dim %% 8 == 0");
  }

  switch (epi_kind) {
    case EPI_STORE: {
      // short reductions over k-contiguous operands: output-bound, the barrier-free wave kernel
      if (p.K <= 32 && !p.a_t && !p.b_t && p.mode != MODE_GROUP_K)
        return launch_sk(p, stream, vec);
      // narrow problems: the direct-load loop when the reduction is whole 64-k stages (or
      // grouped-K over layout-T operands), else the register-staged loop
      const bool dl64 = dl_ok(p) && (p.mode == MODE_GROUP_K || p.K % 64 == 0);
      if (p.M <= 32)
        return dl64 ? launch_dl_narrow<32, 128, 1, 4>(p, stream, ws, ws_bytes, vec)
                    : launch_layouts<32, 128, 64, 1, 4, EPI_STORE>(p, stream, ws, ws_bytes, vec);
      if (p.M <= 64 && p.mode != MODE_GROUP_M)
        return dl64 ? launch_dl_narrow<64, 128, 2, 2>(p, stream, ws, ws_bytes, vec)
                    : launch_layouts<64, 128, 64, 2, 2, EPI_STORE>(p, stream, ws, ws_bytes, vec);
      if (p.N <= 32 && dl64) return launch_dl_narrow<128, 32, 4, 1>(p, stream, ws, ws_bytes, vec);
      if (p.N <= 64)
        return dl64 ? launch_dl_narrow<128, 64, 4, 1>(p, stream, ws, ws_bytes, vec)
                    : launch_layouts<128, 64, 64, 4, 1, EPI_STORE>(p, stream, ws, ws_bytes, vec);
      if (p.K <= 32 && p.mode != MODE_GROUP_K)
        return launch_layouts<128, 128, 32, 2, 2, EPI_STORE>(p, stream, ws, ws_bytes, vec);
      if (dl_ok(p)) return launch_dl<EPI_STORE>(p, stream, ws, ws_bytes, vec);
      return launch_layouts<128, 128, 64, 2, 2, EPI_STORE>(p, stream, ws, ws_bytes, vec);
    }
    case EPI_SWIGLU_FWD:
      RTE_REQUIRE(!p.a_t && !p.b_t, "gemm: SwiGLU forward expects layout-N operands");
      RTE_REQUIRE(p.N % 64 == 0, "gemm: SwiGLU forward needs N %% 64 == 0");
      RTE_REQUIRE(p.epi.ug && p.epi.z, "gemm: SwiGLU forward needs UG and Z outputs");
      if (p.a_koff2) {
        RTE_REQUIRE(p.mode == MODE_DENSE && p.N % 128 == 0, "gemm: dual-A SwiGLU needs dense mode and N %% 128 == 0");
        return launch_cfg<128, 128, 32, 2, 2, false, false, EPI_SWIGLU_FWD, true>(p, stream, ws, ws_bytes, 1);
      }
      if (dl_whole64(p)) {
        if (p.N == 64)
          return launch_cfg<128, 64, 64, 4, 1, false, false, EPI_SWIGLU_FWD, false, 2>(p, stream, ws, ws_bytes, 1);
        return launch_cfg<128, 128, 64, 2, 2, false, false, EPI_SWIGLU_FWD, false, 2>(p, stream, ws, ws_bytes, 1);
      }
      if (p.N == 64) return launch_cfg<128, 64, 64, 4, 1, false, false, EPI_SWIGLU_FWD>(p, stream, ws, ws_bytes, 1);
      return launch_cfg<128, 128, 64, 2, 2, false, false, EPI_SWIGLU_FWD>(p, stream, ws, ws_bytes, 1);
    case EPI_SWIGLU_BWD:
      RTE_REQUIRE(!p.a_t, "gemm: SwiGLU backward expects layout-N dY");
      RTE_REQUIRE(p.epi.ug && p.epi.ug_in, "gemm: SwiGLU backward needs UG input and dUG output");
      RTE_REQUIRE(p.N % 32 == 0, "gemm: SwiGLU backward needs N %% 32 == 0");
      if (p.epi.dw_row) RTE_REQUIRE(p.N <= 128, "gemm: per-row reduction supports N <= 128");
      if (dl_whole64(p)) {
        if (p.N <= 32)
          return p.b_t ? launch_cfg<128, 32, 64, 4, 1, false, true, EPI_SWIGLU_BWD, false, 2>(p, stream, ws, ws_bytes, 1)
                       : launch_cfg<128, 32, 64, 4, 1, false, false, EPI_SWIGLU_BWD, false, 2>(p, stream, ws, ws_bytes, 1);
        if (p.N <= 64)
          return p.b_t ? launch_cfg<128, 64, 64, 4, 1, false, true, EPI_SWIGLU_BWD, false, 2>(p, stream, ws, ws_bytes, 1)
                       : launch_cfg<128, 64, 64, 4, 1, false, false, EPI_SWIGLU_BWD, false, 2>(p, stream, ws, ws_bytes, 1);
      }
      if (p.N <= 32) {
        return p.b_t ? launch_cfg<128, 32, 64, 4, 1, false, true, EPI_SWIGLU_BWD>(p, stream, ws, ws_bytes, 1)
                     : launch_cfg<128, 32, 64, 4, 1, false, false, EPI_SWIGLU_BWD>(p, stream, ws, ws_bytes, 1);
      }
      if (p.N <= 64) {
        return p.b_t ? launch_cfg<128, 64, 64, 4, 1, false, true, EPI_SWIGLU_BWD>(p, stream, ws, ws_bytes, 1)
                     : launch_cfg<128, 64, 64, 4, 1, false, false, EPI_SWIGLU_BWD>(p, stream, ws, ws_bytes, 1);
      }
      return p.b_t ? launch_cfg<128, 128, 64, 4, 1, false, true, EPI_SWIGLU_BWD>(p, stream, ws, ws_bytes, 1)
                   : launch_cfg<128, 128, 64, 4, 1, false, false, EPI_SWIGLU_BWD>(p, stream, ws, ws_bytes, 1);
    case EPI_ROPE_QKV:
      RTE_REQUIRE(!p.a_t && !p.b_t, "gemm: QKV epilogue expects layout-N operands");
      RTE_REQUIRE(p.epi.q && p.epi.k && p.epi.v && p.epi.cos_t && p.epi.sin_t, "gemm: QKV outputs");
      RTE_REQUIRE(p.epi.hd % 2 == 0 && p.epi.dmodel * 3 == p.N, "gemm: QKV shape");
      if (ws && p.mode == MODE_DENSE && p.K >= 256 && p.N % 4 == 0 &&
          (int64_t)((p.M + 31) / 32) * ((p.N + 127) / 128) < 256 &&
          ws_bytes >= (size_t)2 * p.M * p.N * sizeof(float)) {
        // few output tiles (a short sequence batch): split the reduction, the split-K reduce
        // applies RoPE and the head split (tiles < 256, K >= 256 and room for two partial
        // planes always give at least two splits)
        GemmArgs ps = p;
        ps.epi.c = nullptr;
        ps.splits_forced = 1;
        return gemm_launch(ps, EPI_STORE, stream, ws, ws_bytes);
      }
      if (dl_ok(p)) return launch_dl<EPI_ROPE_QKV>(p, stream, ws, ws_bytes, 1);
      return launch_cfg<128, 128, 64, 2, 2, false, false, EPI_ROPE_QKV>(p, stream, ws, ws_bytes, 1);
    default:
      set_error("gemm: unknown epilogue %d", epi_kind);
      return -1;
  }
}

}  // namespace rte
