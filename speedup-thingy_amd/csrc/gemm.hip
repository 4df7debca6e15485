// bf16 MFMA GEMM core for gfx950 (v_mfma_f32_32x32x16_bf16), fp32 accumulation.
//
// Tiling: a workgroup of 256 threads (4 wave64) owns a BM x BN output tile and
// walks k in steps of BK through double-buffered LDS.  Global tiles are fetched
// into registers one step ahead (16-byte loads), then written to LDS in a
// k-contiguous layout [row][BK+8] so every MFMA operand fetch is one 16-byte LDS
// read per lane.  Operands whose output index is contiguous in memory (layout T)
// are loaded as 4(k) x 8(i) blocks and transposed in registers before the LDS
// write, so weight gradients (reduction over tokens) need no transposed copies.
//
// MFMA lane layout used below (32x32x16): lane l supplies A row (l % 32) and
// B column (l % 32) with 8 consecutive k values starting at 8*(l / 32); output
// register r of lane l holds row 8*(r/4) + 4*(l/32) + (r%4), column l % 32.
// Any consistent k permutation gives the same dot products, so only the output
// mapping has to match the hardware; the GPU parity tests pin it.
#include "gemm.hpp"

#include <stdarg.h>
#include <stdio.h>

namespace rte {

namespace {

__device__ __forceinline__ int64_t ilv_row(int64_t r, int32_t half) {
  return ((r & 63) < 32 ? 0 : half) + (r >> 6) * 32 + (r & 31);
}

__device__ __forceinline__ int64_t row_off(const Operand& o, int64_t r) {
  if (o.ilv) r = ilv_row(r, o.ilv);
  if (o.rows) r = o.rows[r];
  if (o.rdiv) return (r / o.rdiv) * o.rs_hi + (r % o.rdiv) * o.ld;
  return r * o.ld;
}

__device__ __forceinline__ int64_t col_off(const Operand& o, int c) {
  if (o.cdiv) return (int64_t)(c / o.cdiv) * o.cs_hi + (c % o.cdiv);
  return c;
}

template <int R, int BK, bool T>
struct TileLoader {
  static constexpr int LDP = BK + 8;
  static constexpr int UNITS = T ? (R / 8) * (BK / 4) : R * (BK / 8);
  static constexpr int PER = (UNITS + 255) / 256;
  static constexpr int NREG = T ? PER * 4 : PER;
  uint4 r[NREG];

  // i: output-index tile origin (m or n), ilim: its bound; k0/klim: reduction range.
  __device__ __forceinline__ void load(const Operand& o, const bf16* base, int64_t rowshift, int i0,
                                       int ilim, int k0, int klim, int tid) {
#pragma unroll
    for (int u = 0; u < PER; ++u) {
      const int q = tid + u * 256;
      if (T) {
        const int mb = q % (R / 8), kb = q / (R / 8);
        const int i = i0 + mb * 8;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int k = k0 + kb * 4 + j;
          uint4 v = make_uint4(0u, 0u, 0u, 0u);
          if (q < UNITS && i < ilim && k < klim)
            v = *reinterpret_cast<const uint4*>(base + row_off(o, k + rowshift) + col_off(o, i));
          r[u * 4 + j] = v;
        }
      } else {
        const int rr = q / (BK / 8), kc = q % (BK / 8);
        const int i = i0 + rr, k = k0 + kc * 8;
        uint4 v = make_uint4(0u, 0u, 0u, 0u);
        if (q < UNITS && i < ilim && k < klim)
          v = *reinterpret_cast<const uint4*>(base + row_off(o, i + rowshift) + col_off(o, k));
        r[u] = v;
      }
    }
  }

  __device__ __forceinline__ static uint32_t lo2(uint32_t a, uint32_t b) {
    return (a & 0xffffu) | (b << 16);
  }
  __device__ __forceinline__ static uint32_t hi2(uint32_t a, uint32_t b) {
    return (a >> 16) | (b & 0xffff0000u);
  }

  __device__ __forceinline__ void store(bf16* lds, int tid) const {
#pragma unroll
    for (int u = 0; u < PER; ++u) {
      const int q = tid + u * 256;
      if (q >= UNITS) continue;
      if (T) {
        const int mb = q % (R / 8), kb = q / (R / 8);
        const uint4 a = r[u * 4 + 0], b = r[u * 4 + 1], c = r[u * 4 + 2], d = r[u * 4 + 3];
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
      } else {
        const int rr = q / (BK / 8), kc = q % (BK / 8);
        *reinterpret_cast<uint4*>(lds + rr * LDP + kc * 8) = r[u];
      }
    }
  }
};

template <int BM, int BN, int BK, int WM, int WN, bool AT, bool BT, int EPI>
__global__ void __launch_bounds__(256) gemm_kernel(GemmArgs p) {
  constexpr int LDP = BK + 8;
  constexpr int WTM = BM / WM, WTN = BN / WN;
  constexpr int TM = WTM / 32, TN = WTN / 32;
  static_assert(WM * WN == 4, "4 waves per workgroup");
  static_assert(TM >= 1 && TN >= 1, "wave tile must hold a 32x32 block");

  extern __shared__ __align__(16) unsigned char smem_raw[];
  bf16* smem = reinterpret_cast<bf16*>(smem_raw);
  bf16* As[2] = {smem, smem + BM * LDP};
  bf16* Bs[2] = {smem + 2 * BM * LDP, smem + 2 * BM * LDP + BN * LDP};
  __shared__ int s_tile[2];

  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int wm = wave / WN, wn = wave % WN;

  int g = 0, m0 = 0, n0 = 0, mlim = p.M, kbeg = 0, kend = p.K;
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
    const int gb = p.goff[g];
    mlim = p.goff[g + 1];
    m0 = gb + s_tile[1] * BM;
    n0 = blockIdx.y * BN;
  } else if (p.mode == MODE_GROUP_K) {
    g = blockIdx.z;
    kbeg = p.goff[g];
    kend = p.goff[g + 1];
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

  TileLoader<BM, BK, AT> la;
  TileLoader<BN, BK, BT> lb;
  const int nk = kend > kbeg ? (kend - kbeg + BK - 1) / BK : 0;
  if (nk > 0) {
    la.load(p.a, abase, ashift, m0, mlim, kbeg, kend, tid);
    lb.load(p.b, bbase, bshift, n0, p.N, kbeg, kend, tid);
    la.store(As[0], tid);
    lb.store(Bs[0], tid);
  }
  __syncthreads();

  for (int kt = 0; kt < nk; ++kt) {
    const int cur = kt & 1;
    const bool more = kt + 1 < nk;
    if (more) {
      const int k0 = kbeg + (kt + 1) * BK;
      la.load(p.a, abase, ashift, m0, mlim, k0, kend, tid);
      lb.load(p.b, bbase, bshift, n0, p.N, k0, kend, tid);
    }
    const bf16* a_s = As[cur];
    const bf16* b_s = Bs[cur];
#pragma unroll
    for (int ks = 0; ks < BK / 16; ++ks) {
      bf16x8_v af[TM], bfr[TN];
      const int kof = ks * 16 + (lane >> 5) * 8;
#pragma unroll
      for (int i = 0; i < TM; ++i)
        af[i] = *reinterpret_cast<const bf16x8_v*>(a_s + (wm * WTM + i * 32 + (lane & 31)) * LDP + kof);
#pragma unroll
      for (int j = 0; j < TN; ++j)
        bfr[j] = *reinterpret_cast<const bf16x8_v*>(b_s + (wn * WTN + j * 32 + (lane & 31)) * LDP + kof);
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[i], bfr[j], acc[i][j], 0, 0, 0);
    }
    if (more) {
      la.store(As[cur ^ 1], tid);
      lb.store(Bs[cur ^ 1], tid);
    }
    __syncthreads();
  }

  // ---------------------------------------------------------------- epilogues
  const Epilogue& e = p.epi;
  const int mw = m0 + wm * WTM + (lane >> 5) * 4;
  const int nw = n0 + wn * WTN + (lane & 31);

  if constexpr (EPI == EPI_STORE) {
    char* cbase = reinterpret_cast<char*>(e.c) +
                  (int64_t)g * e.c_gstride * (e.c_f32 ? 4 : 2);
    const int64_t crow_shift = (int64_t)g * e.c_growstride;
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int m = mw + i * 32 + (r >> 2) * 8 + (r & 3);
        if (m >= mlim) continue;
        const float rs = e.row_scale ? e.row_scale[m] : 1.0f;
        int64_t orow = m + crow_shift;
        if (e.c_ilv) orow = ilv_row(orow, e.c_ilv);
        if (e.c_rows) orow = e.c_rows[orow];
#pragma unroll
        for (int j = 0; j < TN; ++j) {
          const int n = nw + j * 32;
          if (n >= p.N) continue;
          float v = acc[i][j][r] * e.alpha * rs;
          if (e.resid) v += e.resid[orow * e.ld_resid + n];
          if (e.c_f32) {
            float* cp = reinterpret_cast<float*>(cbase) + orow * e.ldc + n;
            if (e.beta != 0.0f) v += e.beta * *cp;
            *cp = v;
          } else {
            bf16* cp = reinterpret_cast<bf16*>(cbase) + orow * e.ldc + n;
            if (e.beta != 0.0f) v += e.beta * bf2f(*cp);
            *cp = f2bf(v);
          }
        }
      }
  } else if constexpr (EPI == EPI_SWIGLU_FWD) {
    // Column blocks of 32 alternate up / gate for the same 32 neurons, so the
    // up value and its gate sit in the same register of neighbouring blocks.
    static_assert(TN % 2 == 0, "SwiGLU epilogue pairs column blocks");
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int m = mw + i * 32 + (r >> 2) * 8 + (r & 3);
        if (m >= mlim) continue;
        const float rs = e.row_scale ? e.row_scale[m] : 1.0f;
#pragma unroll
        for (int jp = 0; jp < TN / 2; ++jp) {
          const int ncol = nw + jp * 64;  // up column in the interleaved layout
          if (ncol >= p.N) continue;
          const bf16 ub = f2bf(acc[i][2 * jp][r]);
          const bf16 gb = f2bf(acc[i][2 * jp + 1][r]);
          const float up = bf2f(ub), gt = bf2f(gb);
          const float zval = up * gt * sigmoidf_(gt) * rs;
          e.ug[(int64_t)m * e.ld_ug + ncol] = ub;
          e.ug[(int64_t)m * e.ld_ug + ncol + 32] = gb;
          const int neuron = (ncol >> 6) * 32 + (ncol & 31);
          e.z[(int64_t)m * e.ld_z + neuron] = f2bf(zval);
        }
      }
  } else if constexpr (EPI == EPI_SWIGLU_BWD) {
    static_assert(WN == 1, "row reduction needs the whole N range in one wave");
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int m = mw + i * 32 + (r >> 2) * 8 + (r & 3);
        const bool mok = m < mlim;
        const float rs = (mok && e.row_scale) ? e.row_scale[m] : 1.0f;
        float part = 0.0f;
#pragma unroll
        for (int j = 0; j < TN; ++j) {
          const int n = nw + j * 32;  // neuron index
          if (!mok || n >= p.N) continue;
          const int col = (n >> 5) * 64 + (n & 31);
          const float up = bf2f(e.ug_in[(int64_t)m * e.ld_ug + col]);
          const float gt = bf2f(e.ug_in[(int64_t)m * e.ld_ug + col + 32]);
          const float s = sigmoidf_(gt);
          const float silu = gt * s;
          const float draw = acc[i][j][r];
          const float dz = draw * rs;
          const float dup = dz * silu;
          const float dgt = dz * up * s * (1.0f + gt * (1.0f - s));
          e.ug[(int64_t)m * e.ld_ug + col] = f2bf(dup);
          e.ug[(int64_t)m * e.ld_ug + col + 32] = f2bf(dgt);
          part += up * silu * draw;
        }
        if (e.dw_row) {
#pragma unroll
          for (int off = 16; off >= 1; off >>= 1) part += __shfl_xor(part, off, 64);
          if ((lane & 31) == 0 && mok) e.dw_row[m] = part;
        }
      }
  } else if constexpr (EPI == EPI_ROPE_QKV) {
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int m = mw + i * 32 + (r >> 2) * 8 + (r & 3);
#pragma unroll
        for (int j = 0; j < TN; ++j) {
          const int n = nw + j * 32;
          const float x = acc[i][j][r];
          const float partner = __shfl_xor(x, 1, 64);
          if (m >= mlim || n >= p.N) continue;
          const int part = n / e.dmodel;
          const int within = n - part * e.dmodel;
          const int h = within / e.hd;
          const int dim = within - h * e.hd;
          const int b = m / e.S;
          const int s = m - b * e.S;
          float y = x;
          if (part < 2) {
            const float c = e.cos_t[(int64_t)s * e.hd + dim];
            const float sn = e.sin_t[(int64_t)s * e.hd + dim];
            y = (dim & 1) ? (x * c + partner * sn) : (x * c - partner * sn);
          }
          bf16* dst = part == 0 ? e.q : (part == 1 ? e.k : e.v);
          dst[(((int64_t)b * e.H + h) * e.S + s) * e.hd + dim] = f2bf(y);
        }
      }
  }
}

template <int BM, int BN, int BK, int WM, int WN, bool AT, bool BT, int EPI>
int launch_cfg(const GemmArgs& p, hipStream_t stream) {
  constexpr int LDP = BK + 8;
  constexpr size_t lds = (size_t)2 * (BM + BN) * LDP * sizeof(bf16);
  auto fn = gemm_kernel<BM, BN, BK, WM, WN, AT, BT, EPI>;
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
  dim3 grid;
  if (p.mode == MODE_GROUP_M) {
    grid = dim3(p.max_tiles_m, (p.N + BN - 1) / BN, 1);
  } else if (p.mode == MODE_GROUP_K) {
    grid = dim3((p.M + BM - 1) / BM, (p.N + BN - 1) / BN, p.G);
  } else {
    grid = dim3((p.M + BM - 1) / BM, (p.N + BN - 1) / BN, 1);
  }
  if (grid.x == 0 || grid.y == 0 || grid.z == 0) return 0;
  hipLaunchKernelGGL(fn, grid, dim3(256), lds, stream, p);
  return check_launch("gemm");
}

template <int BM, int BN, int BK, int WM, int WN, int EPI>
int launch_layouts(const GemmArgs& p, hipStream_t stream) {
  if (!p.a_t && !p.b_t) return launch_cfg<BM, BN, BK, WM, WN, false, false, EPI>(p, stream);
  if (!p.a_t && p.b_t) return launch_cfg<BM, BN, BK, WM, WN, false, true, EPI>(p, stream);
  if (p.a_t && !p.b_t) return launch_cfg<BM, BN, BK, WM, WN, true, false, EPI>(p, stream);
  return launch_cfg<BM, BN, BK, WM, WN, true, true, EPI>(p, stream);
}

}  // namespace

int gemm_launch(const GemmArgs& p, int epi_kind, hipStream_t stream) {
  RTE_REQUIRE(p.M >= 0 && p.N >= 0 && p.K >= 0, "gemm: negative size");
  RTE_REQUIRE(p.a.ptr && p.b.ptr, "gemm: null operand");
  // 16-byte vector loads: every contiguous run the kernel reads must hold whole
  // groups of 8 elements.
  if (!p.a_t) RTE_REQUIRE(p.K % 8 == 0 || p.mode == MODE_GROUP_K, "gemm: K %% 8 != 0 for layout-N A");
  if (!p.b_t) RTE_REQUIRE(p.K % 8 == 0 || p.mode == MODE_GROUP_K, "gemm: K %% 8 != 0 for layout-N B");
  if (p.a_t) RTE_REQUIRE(p.M % 8 == 0, "gemm: M %% 8 != 0 for layout-T A");
  if (p.b_t) RTE_REQUIRE(p.N % 8 == 0, "gemm: N %% 8 != 0 for layout-T B");
  if (p.mode == MODE_GROUP_K)
    RTE_REQUIRE(p.a_t && p.b_t, "gemm: GROUP_K needs both operands in layout T");
  if (p.mode == MODE_GROUP_M) RTE_REQUIRE(!p.a_t, "gemm: GROUP_M needs layout-N A");
  if (p.mode != MODE_DENSE) RTE_REQUIRE(p.goff && p.G >= 1, "gemm: grouped mode needs offsets");
  for (const Operand* o : {&p.a, &p.b}) {
    RTE_REQUIRE(((uintptr_t)o->ptr & 15) == 0, "gemm: operand pointer must be 16-byte aligned");
    RTE_REQUIRE(o->ld % 8 == 0 && o->gstride % 8 == 0 && o->rs_hi % 8 == 0 && o->cs_hi % 8 == 0,
                "gemm: operand strides must be multiples of 8 elements");
    RTE_REQUIRE(o->cdiv % 8 == 0, "gemm: split column segments must be multiples of 8");
  }

  switch (epi_kind) {
    case EPI_STORE:
      if (p.M <= 32) return launch_layouts<32, 128, 64, 1, 4, EPI_STORE>(p, stream);
      if (p.M <= 64 && p.mode != MODE_GROUP_M) return launch_layouts<64, 128, 64, 2, 2, EPI_STORE>(p, stream);
      if (p.N <= 64) return launch_layouts<128, 64, 64, 4, 1, EPI_STORE>(p, stream);
      if (p.K <= 32 && p.mode != MODE_GROUP_K) return launch_layouts<128, 128, 32, 2, 2, EPI_STORE>(p, stream);
      return launch_layouts<128, 128, 64, 2, 2, EPI_STORE>(p, stream);
    case EPI_SWIGLU_FWD:
      RTE_REQUIRE(!p.a_t && !p.b_t, "gemm: SwiGLU forward expects layout-N operands");
      RTE_REQUIRE(p.N % 64 == 0, "gemm: SwiGLU forward needs N %% 64 == 0");
      RTE_REQUIRE(p.epi.ug && p.epi.z, "gemm: SwiGLU forward needs UG and Z outputs");
      if (p.N == 64) return launch_cfg<128, 64, 64, 4, 1, false, false, EPI_SWIGLU_FWD>(p, stream);
      return launch_cfg<128, 128, 64, 2, 2, false, false, EPI_SWIGLU_FWD>(p, stream);
    case EPI_SWIGLU_BWD:
      RTE_REQUIRE(!p.a_t, "gemm: SwiGLU backward expects layout-N dY");
      RTE_REQUIRE(p.epi.ug && p.epi.ug_in, "gemm: SwiGLU backward needs UG input and dUG output");
      RTE_REQUIRE(p.N % 32 == 0, "gemm: SwiGLU backward needs N %% 32 == 0");
      if (p.epi.dw_row) RTE_REQUIRE(p.N <= 128, "gemm: per-row reduction supports N <= 128");
      if (p.N <= 32) {
        return p.b_t ? launch_cfg<128, 32, 64, 4, 1, false, true, EPI_SWIGLU_BWD>(p, stream)
                     : launch_cfg<128, 32, 64, 4, 1, false, false, EPI_SWIGLU_BWD>(p, stream);
      }
      if (p.N <= 64) {
        return p.b_t ? launch_cfg<128, 64, 64, 4, 1, false, true, EPI_SWIGLU_BWD>(p, stream)
                     : launch_cfg<128, 64, 64, 4, 1, false, false, EPI_SWIGLU_BWD>(p, stream);
      }
      return p.b_t ? launch_cfg<128, 128, 64, 4, 1, false, true, EPI_SWIGLU_BWD>(p, stream)
                   : launch_cfg<128, 128, 64, 4, 1, false, false, EPI_SWIGLU_BWD>(p, stream);
    case EPI_ROPE_QKV:
      RTE_REQUIRE(!p.a_t && !p.b_t, "gemm: QKV epilogue expects layout-N operands");
      RTE_REQUIRE(p.epi.q && p.epi.k && p.epi.v && p.epi.cos_t && p.epi.sin_t, "gemm: QKV outputs");
      RTE_REQUIRE(p.epi.hd % 2 == 0 && p.epi.dmodel * 3 == p.N, "gemm: QKV shape");
      return launch_cfg<128, 128, 64, 2, 2, false, false, EPI_ROPE_QKV>(p, stream);
    default:
      set_error("gemm: unknown epilogue %d", epi_kind);
      return -1;
  }
}

}  // namespace rte
