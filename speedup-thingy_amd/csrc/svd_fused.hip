// SVD low-rank SwiGLU FFN with the wide activations kept on chip (rte/layers.py:342-643, the
// low-rank factor products of SVDFactorSparseFFN; BASELINE cfg4 uses U diag(S) V^T as the up,
// gate and down weights):
//
//   a    = x @ [A_up | A_gate]                  [T, 2r]   (A = U diag(S), GEMM)
//   u, g = a_up V_up^T, a_gate V_gate^T         [T, F]    never written
//   z    = u * silu(g)                          [T, F]    never written
//   b    = z @ V_dn                             [T, r]
//   y    = resid + b @ A_dn^T                   [T, d]    (GEMM)
//
// The middle part runs per 32 x 32 (token, neuron) block on v_mfma_f32_32x32x16_bf16 with the
// neuron index as the MFMA row dimension: the u / g / dz blocks then sit in the accumulators
// with the token index across lanes and the neuron index across registers, which is exactly the
// B-operand layout of the next product that sums over neurons (b, da) or, computed the other
// way round (token index as the row dimension), over tokens (the weight gradients).  The order
// in which the 32 neurons of a block enter that reduction is the accumulator's register order;
// the A operand is read from LDS in the same order.  Nothing of width F reaches HBM.
//
// Backward:
//   db = dy @ A_dn, dA_dn = dy^T b                                       (GEMMs)
//   bwdx (per token tile):  recompute u, g; dz = db V_dn^T; du = dz silu(g);
//                           dg = dz u silu'(g); da = [du V_up | dg V_gate]
//   bwdw (per neuron tile, split over tokens): recompute u, g, dz, z, du, dg and
//                           dV_up = du^T a_up, dV_gate = dg^T a_gate, dV_dn = z^T db
//   dx = da @ [A_up | A_gate]^T, d[A_up | A_gate] = x^T da                (GEMMs)
// Split partial sums (over neuron ranges in fwd / bwdx, over token ranges in bwdw) are fp32 and
// added in split order by a separate kernel: results are bitwise repeatable.
//
// MFMA lane layout (32x32x16): lane l supplies A row l % 32 and B column l % 32 with k values
// 8 (l / 32) .. +7 of each 16-step; output register r of lane l holds row 8 (r / 4) + 4 (l / 32)
// + r % 4, column l % 32.
#include "common.hpp"
#include "gemm.hpp"

namespace rte {
namespace {

// LDS pitch (bf16) of a transposed [R][32] tile: 72-byte rows.  Its reads (sv_ld_perm: 8 bytes per
// lane from 32 consecutive rows) then start at 32 distinct even banks, so a wave's read covers the
// 64 banks once (an 80-byte pitch maps rows r and r + 16 to the same banks).  Rows are 8-byte
// aligned only: the tiles are written with 8-byte stores (sv_st16).
constexpr int kTP = 36;

// 16 bytes at an 8-byte aligned LDS address
__device__ __forceinline__ void sv_st16(bf16* dst, uint4 v) {
  *reinterpret_cast<uint2*>(dst) = make_uint2(v.x, v.y);
  *reinterpret_cast<uint2*>(dst + 4) = make_uint2(v.z, v.w);
}

__device__ __forceinline__ f32x16_v sv_mfma(bf16x8_v a, bf16x8_v b, f32x16_v c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ bf16x8_v sv_ld8(const bf16* p) {
  return __builtin_bit_cast(bf16x8_v, *reinterpret_cast<const uint4*>(p));
}

// the 8 k-slots of a reduction over the 32 entries of an accumulator block, for step s and lane
// half h: entries 16 s + 4 h + (0..3) and 16 s + 8 + 4 h + (0..3), read from a row of a
// transposed [.][kTP] LDS tile
__device__ __forceinline__ bf16x8_v sv_ld_perm(const bf16* row, int s, int h) {
  const uint2 a = *reinterpret_cast<const uint2*>(row + 16 * s + 4 * h);
  const uint2 b = *reinterpret_cast<const uint2*>(row + 16 * s + 8 + 4 * h);
  return __builtin_bit_cast(bf16x8_v, make_uint4(a.x, a.y, b.x, b.y));
}

// accumulator registers 8 s .. 8 s + 7 as a B operand (the matching k-slots of sv_ld_perm)
__device__ __forceinline__ bf16x8_v sv_pack(const float* v) {
  return __builtin_bit_cast(bf16x8_v, make_uint4(pack_bf2(v[0], v[1]), pack_bf2(v[2], v[3]),
                                                 pack_bf2(v[4], v[5]), pack_bf2(v[6], v[7])));
}

__device__ __forceinline__ f32x16_v sv_zero() {
  f32x16_v z;
#pragma unroll
  for (int i = 0; i < 16; ++i) z[i] = 0.0f;
  return z;
}

// logistic function through the hardware exp and reciprocal (about 1 ulp each; the results
// feed bf16 MFMA operands)
__device__ __forceinline__ float sv_sigmoid(float x) { return __builtin_amdgcn_rcpf(1.0f + __expf(-x)); }

// v where m is all ones, zeros where m is 0 (loads stay unconditional at a clamped address)
__device__ __forceinline__ uint4 sv_mask(uint4 v, uint32_t m) { return make_uint4(v.x & m, v.y & m, v.z & m, v.w & m); }

// Forward middle: b (or fp32 partials over neuron splits) from a = [a_up | a_gate].
// grid (ceil(T / 128), splits), 256 threads; wave w owns tokens blockIdx.x * 128 + 32 w + (0..31);
// split y covers neuron chunks [y cps, (y + 1) cps) of 32 neurons.
template <int R>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 2))) void svd_mid_fwd_kernel(const bf16* __restrict__ a_ug,
                                                          const bf16* __restrict__ v_ug,
                                                          const bf16* __restrict__ v_dnT, int T, int F, int cps,
                                                          bf16* __restrict__ b_out, float* __restrict__ part) {
  constexpr int KS = R / 16, JB = R / 32, P = R + 8, NV = R / 64;
  __shared__ __align__(16) bf16 s_vu[32 * P];
  __shared__ __align__(16) bf16 s_vg[32 * P];
  __shared__ __align__(16) bf16 s_vdT[R * kTP];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, h = lane >> 5, l32 = lane & 31;
  const int t = blockIdx.x * 128 + w * 32 + l32;
  const int tl = t < T ? t : T - 1;
  const int nc = F / 32;
  const int c0 = blockIdx.y * cps;
  const int c1 = c0 + cps < nc ? c0 + cps : nc;

  bf16x8_v bu[KS], bg[KS];
  {
    const bf16* arow = a_ug + (int64_t)tl * 2 * R + 8 * h;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      bu[ks] = sv_ld8(arow + 16 * ks);
      bg[ks] = sv_ld8(arow + R + 16 * ks);
    }
  }
  f32x16_v acc[JB];
#pragma unroll
  for (int jb = 0; jb < JB; ++jb) acc[jb] = sv_zero();

  // staging: chunk c's three tiles go global -> registers (issued one chunk ahead) -> LDS
  uint4 rv0_0, rv1_0, rv2_0, rv0_1, rv1_1, rv2_1;  // [matrix]_[vector]
#define SVD_FWD_GLOAD1(c, q) \
  { \
    const int f0 = (c) * 32; \
    const int i = tid + 256 * (q); \
    const int row = i / (R / 8), col = (i % (R / 8)) * 8; \
    rv0_##q = *reinterpret_cast<const uint4*>(v_ug + (int64_t)(f0 + row) * R + col); \
    rv1_##q = *reinterpret_cast<const uint4*>(v_ug + (int64_t)(F + f0 + row) * R + col); \
    const int j = i >> 2, cj = (i & 3) * 8; \
    rv2_##q = *reinterpret_cast<const uint4*>(v_dnT + (int64_t)j * F + f0 + cj); \
  }
#define SVD_FWD_GLOAD(c) \
  { \
    SVD_FWD_GLOAD1(c, 0) \
    if constexpr (NV > 1) SVD_FWD_GLOAD1(c, 1) \
  }
  if (c0 < c1) SVD_FWD_GLOAD(c0)
  for (int c = c0; c < c1; ++c) {
    __syncthreads();  // every wave is done reading the previous chunk
    {
      const int i = tid + 256 * 0;
      const int row = i / (R / 8), col = (i % (R / 8)) * 8;
      *reinterpret_cast<uint4*>(s_vu + row * P + col) = rv0_0;
      *reinterpret_cast<uint4*>(s_vg + row * P + col) = rv1_0;
      const int j = i >> 2, cj = (i & 3) * 8;
      sv_st16(s_vdT + j * kTP + cj, rv2_0);
    }
    if constexpr (NV > 1) {
      const int i = tid + 256 * 1;
      const int row = i / (R / 8), col = (i % (R / 8)) * 8;
      *reinterpret_cast<uint4*>(s_vu + row * P + col) = rv0_1;
      *reinterpret_cast<uint4*>(s_vg + row * P + col) = rv1_1;
      const int j = i >> 2, cj = (i & 3) * 8;
      sv_st16(s_vdT + j * kTP + cj, rv2_1);
    }
    __syncthreads();
    if (c + 1 < c1) SVD_FWD_GLOAD(c + 1)  // in flight during this chunk's products
    f32x16_v u = sv_zero(), g = sv_zero();
    const bf16* vu = s_vu + l32 * P + 8 * h;
    const bf16* vg = s_vg + l32 * P + 8 * h;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      u = sv_mfma(sv_ld8(vu + 16 * ks), bu[ks], u);
      g = sv_mfma(sv_ld8(vg + 16 * ks), bg[ks], g);
    }
    bf16x8_v zb[2];
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      float zz[8];
#pragma unroll
      for (int m = 0; m < 8; ++m) {
        const float gv = g[8 * s + m];
        zz[m] = u[8 * s + m] * gv * sv_sigmoid(gv);
      }
      zb[s] = sv_pack(zz);
    }
#pragma unroll
    for (int jb = 0; jb < JB; ++jb) {
      const bf16* row = s_vdT + (jb * 32 + l32) * kTP;
#pragma unroll
      for (int s = 0; s < 2; ++s) acc[jb] = sv_mfma(sv_ld_perm(row, s, h), zb[s], acc[jb]);
    }
  }
  if (t >= T) return;
#pragma unroll
  for (int jb = 0; jb < JB; ++jb) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int j = jb * 32 + 8 * q + 4 * h;
      if (part != nullptr) {
        *reinterpret_cast<float4*>(part + ((int64_t)blockIdx.y * T + t) * R + j) =
            make_float4(acc[jb][4 * q], acc[jb][4 * q + 1], acc[jb][4 * q + 2], acc[jb][4 * q + 3]);
      } else {
        *reinterpret_cast<uint2*>(b_out + (int64_t)t * R + j) =
            make_uint2(pack_bf2(acc[jb][4 * q], acc[jb][4 * q + 1]), pack_bf2(acc[jb][4 * q + 2], acc[jb][4 * q + 3]));
      }
    }
  }
}

// Backward to the low-rank codes: da = [du V_up | dg V_gate] per token tile (fp32 partials over
// neuron splits when splits > 1).  Layout and grid as svd_mid_fwd_kernel; v_ugT = [V_up; V_gate]^T
// ([R][2F]).
template <int R>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1))) void svd_mid_bwdx_kernel(const bf16* __restrict__ a_ug, const bf16* __restrict__ db,
                                                           const bf16* __restrict__ v_ug,
                                                           const bf16* __restrict__ v_dn,
                                                           const bf16* __restrict__ v_ugT, int T, int F, int cps,
                                                           bf16* __restrict__ da_out, float* __restrict__ part) {
  constexpr int KS = R / 16, JB = R / 32, P = R + 8, NV = R / 64;
  __shared__ __align__(16) bf16 s_vu[32 * P];
  __shared__ __align__(16) bf16 s_vg[32 * P];
  __shared__ __align__(16) bf16 s_vd[32 * P];
  __shared__ __align__(16) bf16 s_vuT[R * kTP];
  __shared__ __align__(16) bf16 s_vgT[R * kTP];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, h = lane >> 5, l32 = lane & 31;
  const int t = blockIdx.x * 128 + w * 32 + l32;
  const int tl = t < T ? t : T - 1;
  const int nc = F / 32;
  const int c0 = blockIdx.y * cps;
  const int c1 = c0 + cps < nc ? c0 + cps : nc;

  bf16x8_v bu[KS], bg[KS], bd[KS];
  {
    const bf16* arow = a_ug + (int64_t)tl * 2 * R + 8 * h;
    const bf16* drow = db + (int64_t)tl * R + 8 * h;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      bu[ks] = sv_ld8(arow + 16 * ks);
      bg[ks] = sv_ld8(arow + R + 16 * ks);
      bd[ks] = sv_ld8(drow + 16 * ks);
    }
  }
  f32x16_v acc_u[JB], acc_g[JB];
#pragma unroll
  for (int kb = 0; kb < JB; ++kb) {
    acc_u[kb] = sv_zero();
    acc_g[kb] = sv_zero();
  }

  uint4 rv0_0, rv1_0, rv2_0, rv3_0, rv4_0, rv0_1, rv1_1, rv2_1, rv3_1, rv4_1;
#define SVD_BWDX_GLOAD1(c, q) \
  { \
    const int f0 = (c) * 32; \
    const int i = tid + 256 * (q); \
    const int row = i / (R / 8), col = (i % (R / 8)) * 8; \
    rv0_##q = *reinterpret_cast<const uint4*>(v_ug + (int64_t)(f0 + row) * R + col); \
    rv1_##q = *reinterpret_cast<const uint4*>(v_ug + (int64_t)(F + f0 + row) * R + col); \
    rv2_##q = *reinterpret_cast<const uint4*>(v_dn + (int64_t)(f0 + row) * R + col); \
    const int k = i >> 2, ck = (i & 3) * 8; \
    rv3_##q = *reinterpret_cast<const uint4*>(v_ugT + (int64_t)k * 2 * F + f0 + ck); \
    rv4_##q = *reinterpret_cast<const uint4*>(v_ugT + (int64_t)k * 2 * F + F + f0 + ck); \
  }
#define SVD_BWDX_GLOAD(c) \
  { \
    SVD_BWDX_GLOAD1(c, 0) \
    if constexpr (NV > 1) SVD_BWDX_GLOAD1(c, 1) \
  }
  if (c0 < c1) SVD_BWDX_GLOAD(c0)
  for (int c = c0; c < c1; ++c) {
    __syncthreads();
    {
      const int i = tid + 256 * 0;
      const int row = i / (R / 8), col = (i % (R / 8)) * 8;
      *reinterpret_cast<uint4*>(s_vu + row * P + col) = rv0_0;
      *reinterpret_cast<uint4*>(s_vg + row * P + col) = rv1_0;
      *reinterpret_cast<uint4*>(s_vd + row * P + col) = rv2_0;
      const int k = i >> 2, ck = (i & 3) * 8;
      sv_st16(s_vuT + k * kTP + ck, rv3_0);
      sv_st16(s_vgT + k * kTP + ck, rv4_0);
    }
    if constexpr (NV > 1) {
      const int i = tid + 256 * 1;
      const int row = i / (R / 8), col = (i % (R / 8)) * 8;
      *reinterpret_cast<uint4*>(s_vu + row * P + col) = rv0_1;
      *reinterpret_cast<uint4*>(s_vg + row * P + col) = rv1_1;
      *reinterpret_cast<uint4*>(s_vd + row * P + col) = rv2_1;
      const int k = i >> 2, ck = (i & 3) * 8;
      sv_st16(s_vuT + k * kTP + ck, rv3_1);
      sv_st16(s_vgT + k * kTP + ck, rv4_1);
    }
    __syncthreads();
    if (c + 1 < c1) SVD_BWDX_GLOAD(c + 1)
    f32x16_v u = sv_zero(), g = sv_zero(), dz = sv_zero();
    const int off = l32 * P + 8 * h;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      u = sv_mfma(sv_ld8(s_vu + off + 16 * ks), bu[ks], u);
      g = sv_mfma(sv_ld8(s_vg + off + 16 * ks), bg[ks], g);
      dz = sv_mfma(sv_ld8(s_vd + off + 16 * ks), bd[ks], dz);
    }
    bf16x8_v dub[2], dgb[2];
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      float du[8], dg[8];
#pragma unroll
      for (int m = 0; m < 8; ++m) {
        const int r = 8 * s + m;
        const float sg = sv_sigmoid(g[r]);
        du[m] = dz[r] * g[r] * sg;
        dg[m] = dz[r] * u[r] * sg * (1.0f + g[r] * (1.0f - sg));
      }
      dub[s] = sv_pack(du);
      dgb[s] = sv_pack(dg);
    }
#pragma unroll
    for (int kb = 0; kb < JB; ++kb) {
      const bf16* ru = s_vuT + (kb * 32 + l32) * kTP;
      const bf16* rg = s_vgT + (kb * 32 + l32) * kTP;
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        acc_u[kb] = sv_mfma(sv_ld_perm(ru, s, h), dub[s], acc_u[kb]);
        acc_g[kb] = sv_mfma(sv_ld_perm(rg, s, h), dgb[s], acc_g[kb]);
      }
    }
  }
  if (t >= T) return;
#pragma unroll
  for (int half = 0; half < 2; ++half) {
#pragma unroll
    for (int kb = 0; kb < JB; ++kb) {
      const f32x16_v& a = half ? acc_g[kb] : acc_u[kb];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int k = half * R + kb * 32 + 8 * q + 4 * h;
        if (part != nullptr) {
          *reinterpret_cast<float4*>(part + ((int64_t)blockIdx.y * T + t) * 2 * R + k) =
              make_float4(a[4 * q], a[4 * q + 1], a[4 * q + 2], a[4 * q + 3]);
        } else {
          *reinterpret_cast<uint2*>(da_out + (int64_t)t * 2 * R + k) =
              make_uint2(pack_bf2(a[4 * q], a[4 * q + 1]), pack_bf2(a[4 * q + 2], a[4 * q + 3]));
        }
      }
    }
  }
}

// Backward to the factors V_up, V_gate, V_dn: grid (F / 128, splits), 256 threads; wave w owns
// neurons blockIdx.x * 128 + 32 w + (0..31) (the lane index); split y reduces token tiles
// [y tps, (y + 1) tps) of 32 tokens.  Writes [dV_up; dV_gate] ([2F][R]) and dV_dn ([F][R]) in
// fp32, or fp32 partials [split][3F][R] when splits > 1.  a_ugT ([2R][T]) and dbT ([R][T]) are
// the transposes of a_ug and db.  T % 8 == 0.
template <int R>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(1, 1))) void svd_mid_bwdw_kernel(const bf16* __restrict__ a_ug, const bf16* __restrict__ db,
                                                           const bf16* __restrict__ a_ugT,
                                                           const bf16* __restrict__ dbT,
                                                           const bf16* __restrict__ v_ug,
                                                           const bf16* __restrict__ v_dn, int T, int F, int tps,
                                                           float* __restrict__ dv_ug, float* __restrict__ dv_dn,
                                                           float* __restrict__ part) {
  constexpr int KS = R / 16, JB = R / 32, P = R + 8, NV = R / 64;
  // dynamic LDS (svd_bwdw_lds_bytes): the token tile's rows and transposes, then the workgroup's
  // 128 rows of V_up and V_gate (the B operands of the recomputed products; V_dn's rows stay in
  // registers)
  extern __shared__ __align__(16) unsigned char sm_raw[];
  bf16* s_au = reinterpret_cast<bf16*>(sm_raw);
  bf16* s_ag = s_au + 32 * P;
  bf16* s_db = s_ag + 32 * P;
  bf16* s_auT = s_db + 32 * P;
  bf16* s_agT = s_auT + R * kTP;
  bf16* s_dbT = s_agT + R * kTP;
  bf16* s_wu = s_dbT + R * kTP;
  bf16* s_wg = s_wu + 128 * P;
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6, h = lane >> 5, l32 = lane & 31;
  const int f = blockIdx.x * 128 + w * 32 + l32;
  const int nt = (T + 31) / 32;
  const int t0 = blockIdx.y * tps;
  const int t1 = t0 + tps < nt ? t0 + tps : nt;

  // the workgroup's 128 V_up / V_gate rows -> LDS (made visible by the loop's first barrier)
  for (int i = tid; i < 128 * R / 8; i += 256) {
    const int row = i / (R / 8), col = (i % (R / 8)) * 8;
    const int64_t fr = (int64_t)blockIdx.x * 128 + row;
    *reinterpret_cast<uint4*>(s_wu + row * P + col) = *reinterpret_cast<const uint4*>(v_ug + fr * R + col);
    *reinterpret_cast<uint4*>(s_wg + row * P + col) = *reinterpret_cast<const uint4*>(v_ug + (F + fr) * R + col);
  }
  bf16x8_v wd[KS];
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) wd[ks] = sv_ld8(v_dn + (int64_t)f * R + 16 * ks + 8 * h);
  f32x16_v acc_u[JB], acc_g[JB], acc_d[JB];
#pragma unroll
  for (int kb = 0; kb < JB; ++kb) {
    acc_u[kb] = sv_zero();
    acc_g[kb] = sv_zero();
    acc_d[kb] = sv_zero();
  }

  uint4 rv0_0, rv1_0, rv2_0, rv3_0, rv4_0, rv5_0, rv0_1, rv1_1, rv2_1, rv3_1, rv4_1, rv5_1;
  // rows of tokens at or past T load as zeros (T % 8 == 0: a vector of 8 tokens is all in or
  // all out), so they add nothing to the reductions
#define SVD_BWDW_GLOAD1(tt, q) \
  { \
    const int tb = (tt) * 32; \
    const int i = tid + 256 * (q); \
    const int row = i / (R / 8), col = (i % (R / 8)) * 8; \
    const uint32_t rm = tb + row < T ? 0xffffffffu : 0u; \
    const int64_t tr = rm ? tb + row : 0; \
    rv0_##q = sv_mask(*reinterpret_cast<const uint4*>(a_ug + tr * 2 * R + col), rm); \
    rv1_##q = sv_mask(*reinterpret_cast<const uint4*>(a_ug + tr * 2 * R + R + col), rm); \
    rv2_##q = sv_mask(*reinterpret_cast<const uint4*>(db + tr * R + col), rm); \
    const int k = i >> 2, ct = (i & 3) * 8; \
    const uint32_t cm = tb + ct < T ? 0xffffffffu : 0u; \
    const int64_t tc = cm ? tb + ct : 0; \
    rv3_##q = sv_mask(*reinterpret_cast<const uint4*>(a_ugT + (int64_t)k * T + tc), cm); \
    rv4_##q = sv_mask(*reinterpret_cast<const uint4*>(a_ugT + (int64_t)(R + k) * T + tc), cm); \
    rv5_##q = sv_mask(*reinterpret_cast<const uint4*>(dbT + (int64_t)k * T + tc), cm); \
  }
#define SVD_BWDW_GLOAD(tt) \
  { \
    SVD_BWDW_GLOAD1(tt, 0) \
    if constexpr (NV > 1) SVD_BWDW_GLOAD1(tt, 1) \
  }
  if (t0 < t1) SVD_BWDW_GLOAD(t0)
  for (int tt = t0; tt < t1; ++tt) {
    __syncthreads();
    {
      const int i = tid + 256 * 0;
      const int row = i / (R / 8), col = (i % (R / 8)) * 8;
      *reinterpret_cast<uint4*>(s_au + row * P + col) = rv0_0;
      *reinterpret_cast<uint4*>(s_ag + row * P + col) = rv1_0;
      *reinterpret_cast<uint4*>(s_db + row * P + col) = rv2_0;
      const int k = i >> 2, ct = (i & 3) * 8;
      sv_st16(s_auT + k * kTP + ct, rv3_0);
      sv_st16(s_agT + k * kTP + ct, rv4_0);
      sv_st16(s_dbT + k * kTP + ct, rv5_0);
    }
    if constexpr (NV > 1) {
      const int i = tid + 256 * 1;
      const int row = i / (R / 8), col = (i % (R / 8)) * 8;
      *reinterpret_cast<uint4*>(s_au + row * P + col) = rv0_1;
      *reinterpret_cast<uint4*>(s_ag + row * P + col) = rv1_1;
      *reinterpret_cast<uint4*>(s_db + row * P + col) = rv2_1;
      const int k = i >> 2, ct = (i & 3) * 8;
      sv_st16(s_auT + k * kTP + ct, rv3_1);
      sv_st16(s_agT + k * kTP + ct, rv4_1);
      sv_st16(s_dbT + k * kTP + ct, rv5_1);
    }
    __syncthreads();
    if (tt + 1 < t1) SVD_BWDW_GLOAD(tt + 1)
    // token index as the MFMA row dimension: u[t][f] etc. with the neuron across lanes
    f32x16_v u = sv_zero(), g = sv_zero(), dz = sv_zero();
    const int off = l32 * P + 8 * h;
    const int woff = (w * 32 + l32) * P + 8 * h;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      u = sv_mfma(sv_ld8(s_au + off + 16 * ks), sv_ld8(s_wu + woff + 16 * ks), u);
      g = sv_mfma(sv_ld8(s_ag + off + 16 * ks), sv_ld8(s_wg + woff + 16 * ks), g);
      dz = sv_mfma(sv_ld8(s_db + off + 16 * ks), wd[ks], dz);
    }
    bf16x8_v zb[2], dub[2], dgb[2];
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      float zz[8], du[8], dg[8];
#pragma unroll
      for (int m = 0; m < 8; ++m) {
        const int r = 8 * s + m;
        const float sg = sv_sigmoid(g[r]);
        zz[m] = u[r] * g[r] * sg;
        du[m] = dz[r] * g[r] * sg;
        dg[m] = dz[r] * u[r] * sg * (1.0f + g[r] * (1.0f - sg));
      }
      zb[s] = sv_pack(zz);
      dub[s] = sv_pack(du);
      dgb[s] = sv_pack(dg);
    }
#pragma unroll
    for (int kb = 0; kb < JB; ++kb) {
      const bf16* ru = s_auT + (kb * 32 + l32) * kTP;
      const bf16* rg = s_agT + (kb * 32 + l32) * kTP;
      const bf16* rd = s_dbT + (kb * 32 + l32) * kTP;
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        acc_u[kb] = sv_mfma(sv_ld_perm(ru, s, h), dub[s], acc_u[kb]);
        acc_g[kb] = sv_mfma(sv_ld_perm(rg, s, h), dgb[s], acc_g[kb]);
        acc_d[kb] = sv_mfma(sv_ld_perm(rd, s, h), zb[s], acc_d[kb]);
      }
    }
  }
#pragma unroll
  for (int m3 = 0; m3 < 3; ++m3) {
#pragma unroll
    for (int kb = 0; kb < JB; ++kb) {
      const f32x16_v& a = m3 == 0 ? acc_u[kb] : (m3 == 1 ? acc_g[kb] : acc_d[kb]);
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int k = kb * 32 + 8 * q + 4 * h;
        const float4 v = make_float4(a[4 * q], a[4 * q + 1], a[4 * q + 2], a[4 * q + 3]);
        float* dst;
        if (part != nullptr) {
          dst = part + ((int64_t)blockIdx.y * 3 * F + (int64_t)m3 * F + f) * R + k;
        } else {
          dst = m3 < 2 ? dv_ug + ((int64_t)m3 * F + f) * R + k : dv_dn + (int64_t)f * R + k;
        }
        *reinterpret_cast<float4*>(dst) = v;
      }
    }
  }
}

// out = sum over splits y (in order) of part[y][e]; elements e < n0 go to out0 (fp32 or bf16),
// the rest to out1 (same type) at e - n0.  n0 and n are multiples of 4.
__global__ __launch_bounds__(256) void svd_split_sum_kernel(const float* __restrict__ part, int splits, int64_t n,
                                                            int64_t n0, void* out0, void* out1, int out_bf16) {
  const int64_t e = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 4;
  if (e >= n) return;
  float4 s = *reinterpret_cast<const float4*>(part + e);
  for (int y = 1; y < splits; ++y) {
    const float4 v = *reinterpret_cast<const float4*>(part + (int64_t)y * n + e);
    s.x += v.x;
    s.y += v.y;
    s.z += v.z;
    s.w += v.w;
  }
  const bool first = e < n0;
  const int64_t o = first ? e : e - n0;
  void* base = first ? out0 : out1;
  if (out_bf16) {
    *reinterpret_cast<uint2*>(static_cast<bf16*>(base) + o) = make_uint2(pack_bf2(s.x, s.y), pack_bf2(s.z, s.w));
  } else {
    *reinterpret_cast<float4*>(static_cast<float*>(base) + o) = s;
  }
}

// out[c][r] = in[r][c] (bf16), 64 x 64 tiles through LDS; rows % 4 == 0, cols % 4 == 0.
__global__ __launch_bounds__(256) void svd_transpose_kernel(const bf16* __restrict__ in, int rows, int cols,
                                                            int64_t ld_in, bf16* __restrict__ out, int64_t ld_out) {
  __shared__ bf16 tile[64][66];
  const int r0 = blockIdx.y * 64, c0 = blockIdx.x * 64;
  const int tx = threadIdx.x & 15, ty = threadIdx.x >> 4;  // 16 x 16 threads, 4 elements each way
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const int r = r0 + ty + 16 * k, c = c0 + 4 * tx;
    if (r < rows && c < cols) {
      const uint2 v = *reinterpret_cast<const uint2*>(in + (int64_t)r * ld_in + c);
      tile[ty + 16 * k][4 * tx] = (bf16)(v.x & 0xffffu);
      tile[ty + 16 * k][4 * tx + 1] = (bf16)(v.x >> 16);
      tile[ty + 16 * k][4 * tx + 2] = (bf16)(v.y & 0xffffu);
      tile[ty + 16 * k][4 * tx + 3] = (bf16)(v.y >> 16);
    }
  }
  __syncthreads();
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const int c = c0 + ty + 16 * k, r = r0 + 4 * tx;
    if (c < cols && r < rows) {
      const int lc = ty + 16 * k, lr = 4 * tx;
      const uint32_t lo = (uint32_t)tile[lr][lc] | ((uint32_t)tile[lr + 1][lc] << 16);
      const uint32_t hi = (uint32_t)tile[lr + 2][lc] | ((uint32_t)tile[lr + 3][lc] << 16);
      *reinterpret_cast<uint2*>(out + (int64_t)c * ld_out + r) = make_uint2(lo, hi);
    }
  }
}

int transpose_bf16(const bf16* in, int rows, int cols, int64_t ld_in, bf16* out, int64_t ld_out, hipStream_t s) {
  dim3 grid((cols + 63) / 64, (rows + 63) / 64);
  hipLaunchKernelGGL(svd_transpose_kernel, grid, dim3(256), 0, s, in, rows, cols, ld_in, out, ld_out);
  return check_launch("svd_transpose");
}

int split_sum(const float* part, int splits, int64_t n, int64_t n0, void* out0, void* out1, int out_bf16,
              hipStream_t s) {
  const int64_t blocks = (n / 4 + 255) / 256;
  hipLaunchKernelGGL(svd_split_sum_kernel, dim3((unsigned)blocks), dim3(256), 0, s, part, splits, n, n0, out0, out1,
                     out_bf16);
  return check_launch("svd_split_sum");
}

Operand op_plain(const void* p, int64_t ld) {
  Operand o;
  o.ptr = static_cast<const bf16*>(p);
  o.ld = ld;
  return o;
}

size_t align256(size_t n) { return (n + 255) & ~(size_t)255; }

constexpr size_t svd_bwdw_lds_bytes(int R) {
  return ((size_t)3 * 32 * (R + 8) + (size_t)3 * R * kTP + (size_t)2 * 128 * (R + 8)) * 2;
}

template <int R>
int launch_bwdw(dim3 grid, hipStream_t st, const bf16* a_ug, const bf16* db, const bf16* a_ugT, const bf16* dbT,
                const bf16* v_ug, const bf16* v_dn, int T, int F, int tps, float* dv_ug, float* dv_dn, float* part) {
  constexpr size_t lds = svd_bwdw_lds_bytes(R);
  static bool attr_done = false;
  if (!attr_done) {
    hipError_t err = hipFuncSetAttribute(reinterpret_cast<const void*>(svd_mid_bwdw_kernel<R>),
                                         hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (err != hipSuccess) {
      set_error("svd_ffn_fused: cannot reserve %zu bytes of LDS: %s", lds, hipGetErrorString(err));
      return -1;
    }
    attr_done = true;
  }
  hipLaunchKernelGGL(svd_mid_bwdw_kernel<R>, grid, dim3(256), lds, st, a_ug, db, a_ugT, dbT, v_ug, v_dn, T, F, tps,
                     dv_ug, dv_dn, part);
  return check_launch("svd_mid_bwdw");
}

// neuron-range splits of the per-token-tile kernels: enough workgroups for `target` (two per CU
// for the forward, one for bwdx), at least 2 chunks of 32 neurons per split
int mid_splits(int T, int F, int target) {
  const int gx = (T + 127) / 128;
  int fs = (target + gx - 1) / gx;
  const int cap = F / 64 > 1 ? F / 64 : 1;
  if (fs > cap) fs = cap;
  return fs < 1 ? 1 : fs;
}

int w_splits(int T, int F) {
  const int gx = F / 128;
  const int nt = (T + 31) / 32;
  int ts = (256 + gx - 1) / gx;
  if (ts > nt) ts = nt;
  return ts < 1 ? 1 : ts;
}

struct FusedWs {
  size_t gemm = 0, v_t = 0, a_t = 0, db_t = 0, part = 0, total = 0;
};

FusedWs fused_layout(int T, int d, int F, int r) {
  FusedWs L;
  size_t g = gemm_splitk_bytes(d, 2 * r, T);
  const size_t g2 = gemm_splitk_bytes(d, r, T);
  L.gemm = align256(g > g2 ? g : g2);
  L.v_t = align256((size_t)r * 2 * F * 2);  // v_dnT [r][F] (fwd) / v_ugT [r][2F] (bwd)
  L.a_t = align256((size_t)2 * r * T * 2);
  L.db_t = align256((size_t)r * T * 2);
  const size_t p_fwd = (size_t)mid_splits(T, F, 512) * T * r * 4;
  const size_t p_bx = (size_t)mid_splits(T, F, 256) * T * 2 * r * 4;
  const size_t p_bw = (size_t)w_splits(T, F) * 3 * F * r * 4;
  size_t p = p_fwd > p_bx ? p_fwd : p_bx;
  p = p > p_bw ? p : p_bw;
  L.part = align256(p);
  L.total = L.gemm + L.v_t + L.a_t + L.db_t + L.part;
  return L;
}

}  // namespace
}  // namespace rte

using namespace rte;

extern "C" {

size_t rte_svd_ffn_fused_workspace_bytes(int T, int d, int F, int r) {
  if (T <= 0 || d <= 0 || F <= 0 || r <= 0) return 256;
  return fused_layout(T, d, F, r).total;
}

int rte_svd_ffn_fused_fwd(const void* x, int T, int d, int F, int r, const void* us_ug, const void* v_ug,
                          const void* v_dn, const void* us_dn, const float* resid, void* a_ug, void* b, void* y,
                          int y_f32, void* workspace, size_t workspace_bytes, void* stream) {
  RTE_REQUIRE(r == 64 || r == 128, "svd_ffn_fused: rank must be 64 or 128 (got %d)", r);
  RTE_REQUIRE(F % 128 == 0 && d % 8 == 0 && T % 8 == 0 && T >= 0,
              "svd_ffn_fused: need F %% 128, d %% 8, T %% 8 == 0 (F=%d d=%d T=%d)", F, d, T);
  if (T == 0) return 0;
  const FusedWs L = fused_layout(T, d, F, r);
  RTE_REQUIRE(workspace != nullptr && workspace_bytes >= L.total,
              "svd_ffn_fused: workspace of %zu bytes needed", L.total);
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  char* ws = static_cast<char*>(workspace);
  bf16* v_dnT = reinterpret_cast<bf16*>(ws + L.gemm);
  float* part = reinterpret_cast<float*>(ws + L.gemm + L.v_t + L.a_t + L.db_t);
  {
    GemmArgs p;  // a_ug = x @ us_ug : B(n=j, k=dcol) = us_ug[dcol][j]
    p.M = T;
    p.N = 2 * r;
    p.K = d;
    p.a = op_plain(x, d);
    p.b = op_plain(us_ug, 2 * r);
    p.b_t = 1;
    p.epi.c = a_ug;
    p.epi.ldc = 2 * r;
    RTE_TRY(gemm_launch(p, EPI_STORE, st));
  }
  RTE_TRY(transpose_bf16(static_cast<const bf16*>(v_dn), F, r, r, v_dnT, F, st));
  const int fs = mid_splits(T, F, 512);
  const int nc = F / 32;
  const int cps = (nc + fs - 1) / fs;
  dim3 grid((T + 127) / 128, fs);
  float* pp = fs > 1 ? part : nullptr;
  if (r == 128)
    hipLaunchKernelGGL(svd_mid_fwd_kernel<128>, grid, dim3(256), 0, st, static_cast<const bf16*>(a_ug),
                       static_cast<const bf16*>(v_ug), v_dnT, T, F, cps, static_cast<bf16*>(b), pp);
  else
    hipLaunchKernelGGL(svd_mid_fwd_kernel<64>, grid, dim3(256), 0, st, static_cast<const bf16*>(a_ug),
                       static_cast<const bf16*>(v_ug), v_dnT, T, F, cps, static_cast<bf16*>(b), pp);
  RTE_TRY(check_launch("svd_mid_fwd"));
  if (fs > 1) RTE_TRY(split_sum(part, fs, (int64_t)T * r, (int64_t)T * r, b, b, 1, st));
  {
    GemmArgs p;  // y = resid + b @ us_dn^T : B(n=dcol, k=j) = us_dn[dcol][j]
    p.M = T;
    p.N = d;
    p.K = r;
    p.a = op_plain(b, r);
    p.b = op_plain(us_dn, r);
    p.epi.c = y;
    p.epi.ldc = d;
    p.epi.c_f32 = y_f32;
    p.epi.resid = resid;
    p.epi.ld_resid = d;
    RTE_TRY(gemm_launch(p, EPI_STORE, st));
  }
  return 0;
}

int rte_svd_ffn_fused_bwd(const void* dy, const void* x, int T, int d, int F, int r, const void* us_ug,
                          const void* v_ug, const void* v_dn, const void* us_dn, const void* a_ug, const void* b,
                          void* db, void* da_ug, void* dx, float* dus_ug, float* dv_ug, float* dv_dn, float* dus_dn,
                          void* workspace, size_t workspace_bytes, void* stream) {
  RTE_REQUIRE(r == 64 || r == 128, "svd_ffn_fused: rank must be 64 or 128 (got %d)", r);
  RTE_REQUIRE(F % 128 == 0 && d % 8 == 0 && T % 8 == 0 && T >= 0,
              "svd_ffn_fused: need F %% 128, d %% 8, T %% 8 == 0 (F=%d d=%d T=%d)", F, d, T);
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  if (T == 0) {
    RTE_TRY(fill_f32(dus_ug, 0.0f, (int64_t)d * 2 * r, st));
    RTE_TRY(fill_f32(dv_ug, 0.0f, (int64_t)2 * F * r, st));
    RTE_TRY(fill_f32(dv_dn, 0.0f, (int64_t)F * r, st));
    return fill_f32(dus_dn, 0.0f, (int64_t)d * r, st);
  }
  const FusedWs L = fused_layout(T, d, F, r);
  RTE_REQUIRE(workspace != nullptr && workspace_bytes >= L.total,
              "svd_ffn_fused: workspace of %zu bytes needed", L.total);
  char* ws = static_cast<char*>(workspace);
  void* gws = ws;
  bf16* v_ugT = reinterpret_cast<bf16*>(ws + L.gemm);
  bf16* a_ugT = reinterpret_cast<bf16*>(ws + L.gemm + L.v_t);
  bf16* dbT = reinterpret_cast<bf16*>(ws + L.gemm + L.v_t + L.a_t);
  float* part = reinterpret_cast<float*>(ws + L.gemm + L.v_t + L.a_t + L.db_t);
  {
    GemmArgs p;  // db = dy @ us_dn : B(n=j, k=dcol) = us_dn[dcol][j]
    p.M = T;
    p.N = r;
    p.K = d;
    p.a = op_plain(dy, d);
    p.b = op_plain(us_dn, r);
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
    p.a = op_plain(dy, d);
    p.a_t = 1;
    p.b = op_plain(b, r);
    p.b_t = 1;
    p.epi.c = dus_dn;
    p.epi.ldc = r;
    p.epi.c_f32 = 1;
    RTE_TRY(gemm_launch(p, EPI_STORE, st, gws, L.gemm));
  }
  RTE_TRY(transpose_bf16(static_cast<const bf16*>(v_ug), 2 * F, r, r, v_ugT, 2 * F, st));
  {
    const int fs = mid_splits(T, F, 256);
    const int nc = F / 32;
    const int cps = (nc + fs - 1) / fs;
    dim3 grid((T + 127) / 128, fs);
    float* pp = fs > 1 ? part : nullptr;
    if (r == 128)
      hipLaunchKernelGGL(svd_mid_bwdx_kernel<128>, grid, dim3(256), 0, st, static_cast<const bf16*>(a_ug),
                         static_cast<const bf16*>(db), static_cast<const bf16*>(v_ug),
                         static_cast<const bf16*>(v_dn), v_ugT, T, F, cps, static_cast<bf16*>(da_ug), pp);
    else
      hipLaunchKernelGGL(svd_mid_bwdx_kernel<64>, grid, dim3(256), 0, st, static_cast<const bf16*>(a_ug),
                         static_cast<const bf16*>(db), static_cast<const bf16*>(v_ug),
                         static_cast<const bf16*>(v_dn), v_ugT, T, F, cps, static_cast<bf16*>(da_ug), pp);
    RTE_TRY(check_launch("svd_mid_bwdx"));
    if (fs > 1) RTE_TRY(split_sum(part, fs, (int64_t)T * 2 * r, (int64_t)T * 2 * r, da_ug, da_ug, 1, st));
  }
  RTE_TRY(transpose_bf16(static_cast<const bf16*>(a_ug), T, 2 * r, 2 * r, a_ugT, T, st));
  RTE_TRY(transpose_bf16(static_cast<const bf16*>(db), T, r, r, dbT, T, st));
  {
    const int ts = w_splits(T, F);
    const int nt = (T + 31) / 32;
    const int tps = (nt + ts - 1) / ts;
    dim3 grid(F / 128, ts);
    float* pp = ts > 1 ? part : nullptr;
    if (r == 128)
      RTE_TRY(launch_bwdw<128>(grid, st, static_cast<const bf16*>(a_ug), static_cast<const bf16*>(db), a_ugT, dbT,
                               static_cast<const bf16*>(v_ug), static_cast<const bf16*>(v_dn), T, F, tps, dv_ug,
                               dv_dn, pp));
    else
      RTE_TRY(launch_bwdw<64>(grid, st, static_cast<const bf16*>(a_ug), static_cast<const bf16*>(db), a_ugT, dbT,
                              static_cast<const bf16*>(v_ug), static_cast<const bf16*>(v_dn), T, F, tps, dv_ug, dv_dn,
                              pp));
    if (ts > 1) RTE_TRY(split_sum(part, ts, (int64_t)3 * F * r, (int64_t)2 * F * r, dv_ug, dv_dn, 0, st));
  }
  {
    GemmArgs p;  // dx = da_ug @ us_ug^T : B(n=dcol, k=j) = us_ug[dcol][j]
    p.M = T;
    p.N = d;
    p.K = 2 * r;
    p.a = op_plain(da_ug, 2 * r);
    p.b = op_plain(us_ug, 2 * r);
    p.epi.c = dx;
    p.epi.ldc = d;
    RTE_TRY(gemm_launch(p, EPI_STORE, st));
  }
  {
    GemmArgs p;  // dus_ug[dcol, j] = sum_t x[t, dcol] da_ug[t, j]
    p.M = d;
    p.N = 2 * r;
    p.K = T;
    p.a = op_plain(x, d);
    p.a_t = 1;
    p.b = op_plain(da_ug, 2 * r);
    p.b_t = 1;
    p.epi.c = dus_ug;
    p.epi.ldc = 2 * r;
    p.epi.c_f32 = 1;
    RTE_TRY(gemm_launch(p, EPI_STORE, st, gws, L.gemm));
  }
  return 0;
}

}  // extern "C"
