// Kernels behind the reference's elementwise dispatch symbols, in the caller's dtype:
//   fused RMSNorm with optional residual (k_fused_rmsnorm, rte/kernels/reference.py:9-17),
//   interleaved RoPE on q and k (k_rope_apply, rte/kernels/reference.py:20-28),
//   static-centre routing (route_to_static_centers, rte/kernels/cluster_pool_ffn.py:129-140).
// fp32 inputs are computed in fp32 throughout; bf16 inputs follow torch's bf16 rounding points
// (the sum x + residual, the rsqrt factor and the normalised row are rounded to bf16 as the
// reference's bf16 tensor ops round them).
#include "../../include/rte_hip.h"
#include "common.hpp"

namespace rte {
namespace {

__device__ __forceinline__ float wsum(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

template <bool F32>
__device__ __forceinline__ void ld8(const void* base, int64_t i, float* v) {
  if constexpr (F32) {
    const float4 a = *reinterpret_cast<const float4*>(static_cast<const float*>(base) + i);
    const float4 b = *reinterpret_cast<const float4*>(static_cast<const float*>(base) + i + 4);
    v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w; v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
  } else {
    const uint4 u = *reinterpret_cast<const uint4*>(static_cast<const bf16*>(base) + i);
    const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      v[2 * q] = __uint_as_float(w[q] << 16);
      v[2 * q + 1] = __uint_as_float(w[q] & 0xffff0000u);
    }
  }
}

template <bool F32>
__device__ __forceinline__ void st8(void* base, int64_t i, const float* v) {
  if constexpr (F32) {
    float* p = static_cast<float*>(base) + i;
    *reinterpret_cast<float4*>(p) = make_float4(v[0], v[1], v[2], v[3]);
    *reinterpret_cast<float4*>(p + 4) = make_float4(v[4], v[5], v[6], v[7]);
  } else {
    uint4 o;
    o.x = pack_bf2(v[0], v[1]);
    o.y = pack_bf2(v[2], v[3]);
    o.z = pack_bf2(v[4], v[5]);
    o.w = pack_bf2(v[6], v[7]);
    *reinterpret_cast<uint4*>(static_cast<bf16*>(base) + i) = o;
  }
}

constexpr int kMaxChunks = 8;  // d <= 64 lanes * 8 * 8 = 4096
constexpr int kBwdChunks = 4;  // backward: d <= 2048

// One wave per row: y = x (+ residual), rstd = rsqrt(mean(y^2) + eps), out = (y * rstd) * w.
template <bool IOF32, bool OUTF32>
__global__ void __launch_bounds__(256) fused_rmsnorm_fwd_kernel(const void* __restrict__ x, const void* __restrict__ res,
                                                                const float* __restrict__ w, int T, int d, float eps,
                                                                void* __restrict__ y_out, void* __restrict__ out,
                                                                float* __restrict__ rstd_out) {
  const int lane = threadIdx.x & 63;
  const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= T) return;
  const int nch = d / 8;
  float y[kMaxChunks][8];
  float ss = 0.0f;
#pragma unroll
  for (int c = 0; c < kMaxChunks; ++c) {
    const int ch = lane + 64 * c;
    if (ch >= nch) continue;
    const int64_t i = (int64_t)t * d + ch * 8;
    ld8<IOF32>(x, i, y[c]);
    if (res) {
      float r[8];
      ld8<IOF32>(res, i, r);
#pragma unroll
      for (int q = 0; q < 8; ++q) y[c][q] = IOF32 ? y[c][q] + r[q] : round_bf(y[c][q] + r[q]);
      if (y_out) st8<IOF32>(y_out, i, y[c]);
    }
#pragma unroll
    for (int q = 0; q < 8; ++q) ss += y[c][q] * y[c][q];
  }
  ss = wsum(ss);
  const float rs = rsqrtf(ss / (float)d + eps);
  if (lane == 0 && rstd_out) rstd_out[t] = rs;
  const float rsy = IOF32 ? rs : round_bf(rs);  // .to(y.dtype) of the rsqrt factor
#pragma unroll
  for (int c = 0; c < kMaxChunks; ++c) {
    const int ch = lane + 64 * c;
    if (ch >= nch) continue;
    float wv[8], o[8];
    ld8<true>(w, ch * 8, wv);
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      const float nrm = IOF32 ? y[c][q] * rsy : round_bf(y[c][q] * rsy);
      o[q] = nrm * wv[q];
    }
    st8<OUTF32>(out, (int64_t)t * d + ch * 8, o);
  }
}

// Backward of out = y * rstd * w with y = x (+ residual):
//   dy = rstd (w g) - y rstd^3 mean(w g y) (+ dy_extra),  dw partial = sum_rows g y rstd.
// One wave per row, rows [blockIdx.x * rpb, +rpb) per workgroup; per-workgroup dw partials
// summed in block order afterwards (fixed order, no atomics).
template <bool IOF32, bool GF32>
__global__ void __launch_bounds__(256) fused_rmsnorm_bwd_kernel(const void* __restrict__ g_in, const void* __restrict__ dyx,
                                                                const void* __restrict__ yv, const float* __restrict__ w,
                                                                const float* __restrict__ rstd, int T, int d,
                                                                void* __restrict__ dy_out, float* __restrict__ dw_part,
                                                                int rpb) {
  extern __shared__ float sdw[];  // [4][d]
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int nch = d / 8;
  float acc[kBwdChunks][8];
#pragma unroll
  for (int c = 0; c < kBwdChunks; ++c)
#pragma unroll
    for (int q = 0; q < 8; ++q) acc[c][q] = 0.0f;
  const int r0 = blockIdx.x * rpb;
  for (int rr = wave; rr < rpb; rr += 4) {
    const int t = r0 + rr;
    if (t >= T) break;
    const float rs = rstd[t];
    float g[kBwdChunks][8], y[kBwdChunks][8], wv[kBwdChunks][8];
    float dot = 0.0f;
#pragma unroll
    for (int c = 0; c < kBwdChunks; ++c) {
      const int ch = lane + 64 * c;
      if (ch >= nch) continue;
      const int64_t i = (int64_t)t * d + ch * 8;
      ld8<GF32>(g_in, i, g[c]);
      ld8<IOF32>(yv, i, y[c]);
      ld8<true>(w, ch * 8, wv[c]);
#pragma unroll
      for (int q = 0; q < 8; ++q) dot += wv[c][q] * g[c][q] * y[c][q];
    }
    dot = wsum(dot);
    const float coef = rs * rs * rs * dot / (float)d;
#pragma unroll
    for (int c = 0; c < kBwdChunks; ++c) {
      const int ch = lane + 64 * c;
      if (ch >= nch) continue;
      const int64_t i = (int64_t)t * d + ch * 8;
      float o[8], e[8];
      if (dyx) ld8<IOF32>(dyx, i, e);
#pragma unroll
      for (int q = 0; q < 8; ++q) {
        o[q] = rs * wv[c][q] * g[c][q] - y[c][q] * coef + (dyx ? e[q] : 0.0f);
        acc[c][q] += g[c][q] * y[c][q] * rs;
      }
      st8<IOF32>(dy_out, i, o);
    }
  }
#pragma unroll
  for (int c = 0; c < kBwdChunks; ++c) {
    const int ch = lane + 64 * c;
    if (ch < nch) st8<true>(sdw, (int64_t)wave * d + ch * 8, acc[c]);
  }
  __syncthreads();
  for (int c = threadIdx.x; c < d; c += 256)
    dw_part[(int64_t)blockIdx.x * d + c] = ((sdw[c] + sdw[d + c]) + sdw[2 * d + c]) + sdw[3 * d + c];
}

// out[c] = sum_r part[r, c] in row order per phase, phases added in order (fixed order).
__global__ void __launch_bounds__(256) dw_colsum_kernel(const float* __restrict__ part, int nrows, int d,
                                                        float* __restrict__ out) {
  __shared__ float sh[32][8];
  const int l = threadIdx.x & 7, phase = threadIdx.x >> 3;
  const int col = blockIdx.x * 8 + l;
  float s = 0.0f;
  if (col < d)
    for (int r = phase; r < nrows; r += 32) s += part[(int64_t)r * d + col];
  sh[phase][l] = s;
  __syncthreads();
  if (threadIdx.x < 8 && col < d) {
    float tot = 0.0f;
#pragma unroll
    for (int q = 0; q < 32; ++q) tot += sh[q][l];
    out[col] = tot;
  }
}

int rows_per_block(int T) {
  int r = ((T + 255) / 256 + 3) / 4 * 4;
  return r < 4 ? 4 : (r > 32 ? 32 : r);
}

// Interleaved rotation of 8 consecutive dims (4 pairs) of one row.  forward:
//   o[2i] = x[2i] c[2i] - x[2i+1] s[2i],  o[2i+1] = x[2i+1] c[2i+1] + x[2i] s[2i+1]
// inverse (the transpose, for the backward):
//   o[2i] = x[2i] c[2i] + x[2i+1] s[2i+1],  o[2i+1] = x[2i+1] c[2i+1] - x[2i] s[2i]
template <bool INV>
__device__ __forceinline__ void rot8(const float* x, const float* c, const float* s, float* o) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float xe = x[2 * i], xo = x[2 * i + 1];
    if constexpr (!INV) {
      o[2 * i] = xe * c[2 * i] - xo * s[2 * i];
      o[2 * i + 1] = xo * c[2 * i + 1] + xe * s[2 * i + 1];
    } else {
      o[2 * i] = xe * c[2 * i] + xo * s[2 * i + 1];
      o[2 * i + 1] = xo * c[2 * i + 1] - xe * s[2 * i];
    }
  }
}

// One thread per 8 consecutive dims of one row of q (blockIdx.y = 0) or k (blockIdx.y = 1);
// row r of a [rows, S, hd] tensor sits at position r % S.
template <bool INF32, bool OUTF32, bool INV>
__global__ void __launch_bounds__(256) rope_apply_kernel(const void* __restrict__ q, const void* __restrict__ k,
                                                         int64_t rows, int S, int hd, const float* __restrict__ cos_t,
                                                         const float* __restrict__ sin_t, void* __restrict__ qo,
                                                         void* __restrict__ ko) {
  const int per = hd / 8;
  const int64_t u = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (u >= rows * per) return;
  const void* src = blockIdx.y == 0 ? q : k;
  void* dst = blockIdx.y == 0 ? qo : ko;
  const int64_t row = u / per;
  const int dim = (int)(u - row * per) * 8;
  const int s = (int)(row % S);
  float x[8], c[8], sn[8], o[8];
  ld8<INF32>(src, row * hd + dim, x);
  ld8<true>(cos_t, (int64_t)s * hd + dim, c);
  ld8<true>(sin_t, (int64_t)s * hd + dim, sn);
  rot8<INV>(x, c, sn, o);
  st8<OUTF32>(dst, row * hd + dim, o);
}

// One wave per token: features f = normalize([x A_up | x A_gate]) (fp32, norm clamped below at
// 1e-12 as F.normalize), scores f . centers[c], out = first index of the maximum (NaN counts as
// the maximum, as torch.argmax).  The normalised row sits in the wave's LDS slice; lanes stride
// over the centers.
__global__ void __launch_bounds__(256) route_centers_kernel(const float* __restrict__ q, int T, int R2,
                                                            const float* __restrict__ centers, int C,
                                                            int32_t* __restrict__ out) {
  extern __shared__ float srow[];  // [4][R2]
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int t = blockIdx.x * 4 + wave;
  float* f = srow + wave * R2;
  if (t < T) {
    float ss = 0.0f;
    for (int j = lane; j < R2; j += 64) {
      const float v = q[(int64_t)t * R2 + j];
      f[j] = v;
      ss += v * v;
    }
    ss = wsum(ss);
    const float inv = 1.0f / fmaxf(sqrtf(ss), 1e-12f);
    for (int j = lane; j < R2; j += 64) f[j] *= inv;
  }
  __syncthreads();
  if (t >= T) return;
  float best = -INFINITY;
  int bi = -1;
  bool bnan = false;
  for (int c = lane; c < C; c += 64) {
    const float* cr = centers + (int64_t)c * R2;
    float acc = 0.0f;
    for (int j = 0; j < R2; ++j) acc = fmaf(f[j], cr[j], acc);
    const bool isn = acc != acc;
    // (NaN first, then larger value, then lower index): the lane keeps its best in stride order
    if (bi < 0 || (isn && !bnan) || (!bnan && !isn && acc > best)) {
      best = acc;
      bi = c;
      bnan = isn;
    }
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    const float ov = __shfl_xor(best, off, 64);
    const int oi = __shfl_xor(bi, off, 64);
    const bool on = __shfl_xor((int)bnan, off, 64) != 0;
    bool take;
    if (oi < 0) take = false;
    else if (bi < 0) take = true;
    else if (on != bnan) take = on;
    else if (!on && ov != best) take = ov > best;
    else take = oi < bi;
    if (take) {
      best = ov;
      bi = oi;
      bnan = on;
    }
  }
  if (lane == 0) out[t] = bi;
}

}  // namespace
}  // namespace rte

using namespace rte;

extern "C" {

int rte_fused_rmsnorm_fwd(const void* x, const void* residual, int io_f32, const float* w, int T, int d, float eps,
                          void* y, void* out, int out_f32, float* rstd, void* stream) {
  RTE_REQUIRE(T >= 0 && d > 0 && d % 8 == 0 && d <= 64 * 8 * kMaxChunks,
              "fused_rmsnorm: d must be a multiple of 8 and at most 4096");
  RTE_REQUIRE(x && w && out, "fused_rmsnorm: null input or output");
  if (T == 0) return 0;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const dim3 grid((T + 3) / 4);
  if (io_f32) {
    if (out_f32)
      hipLaunchKernelGGL((fused_rmsnorm_fwd_kernel<true, true>), grid, dim3(256), 0, s, x, residual, w, T, d, eps, y, out, rstd);
    else
      hipLaunchKernelGGL((fused_rmsnorm_fwd_kernel<true, false>), grid, dim3(256), 0, s, x, residual, w, T, d, eps, y, out, rstd);
  } else {
    if (out_f32)
      hipLaunchKernelGGL((fused_rmsnorm_fwd_kernel<false, true>), grid, dim3(256), 0, s, x, residual, w, T, d, eps, y, out, rstd);
    else
      hipLaunchKernelGGL((fused_rmsnorm_fwd_kernel<false, false>), grid, dim3(256), 0, s, x, residual, w, T, d, eps, y, out, rstd);
  }
  return check_launch("fused_rmsnorm_fwd");
}

size_t rte_fused_rmsnorm_bwd_workspace_bytes(int T, int d) {
  if (T <= 0 || d <= 0) return 0;
  const int rpb = rows_per_block(T);
  return (size_t)((T + rpb - 1) / rpb) * (size_t)d * sizeof(float);
}

int rte_fused_rmsnorm_bwd(const void* g, int g_f32, const void* dy_extra, const void* y, int io_f32, const float* w,
                          const float* rstd, int T, int d, void* dy, float* dw, void* workspace, size_t workspace_bytes,
                          void* stream) {
  // the per-wave dw rows of a workgroup live in LDS: 4 d floats
  RTE_REQUIRE(T >= 0 && d > 0 && d % 8 == 0 && d <= 2048,
              "fused_rmsnorm_bwd: d must be a multiple of 8 and at most 2048");
  RTE_REQUIRE(g && y && w && rstd && dy && dw, "fused_rmsnorm_bwd: null argument");
  if (T == 0) return fill_f32(dw, 0.0f, d, static_cast<hipStream_t>(stream));
  RTE_REQUIRE(workspace && workspace_bytes >= rte_fused_rmsnorm_bwd_workspace_bytes(T, d),
              "fused_rmsnorm_bwd: workspace too small");
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int rpb = rows_per_block(T), nblk = (T + rpb - 1) / rpb;
  float* part = static_cast<float*>(workspace);
  const size_t lds = (size_t)4 * d * sizeof(float);
#define RTE_RMS_BWD(IO, GF)                                                                                       \
  hipLaunchKernelGGL((fused_rmsnorm_bwd_kernel<IO, GF>), dim3(nblk), dim3(256), lds, s, g, dy_extra, y, w, rstd, T, d, \
                     dy, part, rpb)
  if (io_f32) {
    if (g_f32) RTE_RMS_BWD(true, true); else RTE_RMS_BWD(true, false);
  } else {
    if (g_f32) RTE_RMS_BWD(false, true); else RTE_RMS_BWD(false, false);
  }
#undef RTE_RMS_BWD
  RTE_TRY(check_launch("fused_rmsnorm_bwd"));
  hipLaunchKernelGGL(dw_colsum_kernel, dim3((d + 7) / 8), dim3(256), 0, s, part, nblk, d, dw);
  return check_launch("fused_rmsnorm_bwd_colsum");
}

int rte_rope_apply(const void* q, const void* k, int in_f32, int64_t rows, int S, int hd, const float* cos_t,
                   const float* sin_t, void* q_out, void* k_out, int out_f32, int inverse, void* stream) {
  RTE_REQUIRE(rows >= 0 && S > 0 && hd > 0 && hd % 8 == 0, "rope_apply: head_dim must be a multiple of 8");
  RTE_REQUIRE(q && k && cos_t && sin_t && q_out && k_out, "rope_apply: null argument");
  const int64_t n = rows * (hd / 8);
  if (n == 0) return 0;
  RTE_REQUIRE((n + 255) / 256 < ((int64_t)1 << 31), "rope_apply: too many rows");
  hipStream_t s = static_cast<hipStream_t>(stream);
  const dim3 grid((unsigned)((n + 255) / 256), 2);
#define RTE_ROPE(I, O, V) \
  hipLaunchKernelGGL((rope_apply_kernel<I, O, V>), grid, dim3(256), 0, s, q, k, rows, S, hd, cos_t, sin_t, q_out, k_out)
  if (in_f32) {
    if (out_f32) { if (inverse) RTE_ROPE(true, true, true); else RTE_ROPE(true, true, false); }
    else { if (inverse) RTE_ROPE(true, false, true); else RTE_ROPE(true, false, false); }
  } else {
    if (out_f32) { if (inverse) RTE_ROPE(false, true, true); else RTE_ROPE(false, true, false); }
    else { if (inverse) RTE_ROPE(false, false, true); else RTE_ROPE(false, false, false); }
  }
#undef RTE_ROPE
  return check_launch("rope_apply");
}

int rte_route_centers(const float* q, int T, int R2, const float* centers, int C, int32_t* out, void* stream) {
  RTE_REQUIRE(T >= 0 && R2 >= 1 && R2 <= 8192 && C >= 1, "route_centers: bad sizes");
  RTE_REQUIRE(q && centers && out, "route_centers: null argument");
  if (T == 0) return 0;
  hipLaunchKernelGGL(route_centers_kernel, dim3((T + 3) / 4), dim3(256), (size_t)4 * R2 * sizeof(float),
                     static_cast<hipStream_t>(stream), q, T, R2, centers, C, out);
  return check_launch("route_centers");
}

}  // extern "C"
