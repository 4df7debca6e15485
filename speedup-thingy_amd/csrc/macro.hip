// Elementwise ends of the bounded-residual macro operator Phi (rte/macro.py:201-236):
//
//   prologue : z = [rmsnorm(h) | mean_s rmsnorm(h) | h0] in bf16 (the grouped GEMMs' input),
//              rmsnorm without weight, eps as given (rte/macro.py:16-18)
//   epilogue : out = h + c * scale[key] * tanh(gain[key] * h + low + bias[key])
//
// with the per-(recipe, stride) rows gain / bias / scale read straight from their tables by
// the sample's key.  Backward: the epilogue gives dh, dlow (bf16, for the GEMM backward) and
// per-sample column sums of the table gradients; the prologue adds the rmsnorm / mean
// backward to dh and gives dh0.
//
// Layout: one wave per row, each lane owning NCH chunks of 8 consecutive columns (16- and
// 32-byte accesses; d % 8 == 0, d <= 512 * NCH).  Reductions over a sample's rows run in one
// workgroup of 8 waves: per-lane partials, then the 8 wave partials in wave order, so every
// sum has a fixed order.  Each input element is read once.
#include "common.hpp"

namespace rte {

namespace {

constexpr int kMacroWaves = 8;  // waves per workgroup of the per-sample kernels

__device__ __forceinline__ float wsum_m(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

__device__ __forceinline__ void ld8m(const float* p, float* v) {
  const float4 a = *reinterpret_cast<const float4*>(p);
  const float4 b = *reinterpret_cast<const float4*>(p + 4);
  v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
  v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
}

__device__ __forceinline__ void ld8m(const bf16* p, float* v) {
  const uint4 u = *reinterpret_cast<const uint4*>(p);
  const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    v[2 * i] = __uint_as_float(w[i] << 16);
    v[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
  }
}

__device__ __forceinline__ void st8m(float* p, const float* v) {
  *reinterpret_cast<float4*>(p) = make_float4(v[0], v[1], v[2], v[3]);
  *reinterpret_cast<float4*>(p + 4) = make_float4(v[4], v[5], v[6], v[7]);
}

__device__ __forceinline__ void st8m(bf16* p, const float* v) {
  uint4 o;
  o.x = (uint32_t)f2bf(v[0]) | ((uint32_t)f2bf(v[1]) << 16);
  o.y = (uint32_t)f2bf(v[2]) | ((uint32_t)f2bf(v[3]) << 16);
  o.z = (uint32_t)f2bf(v[4]) | ((uint32_t)f2bf(v[5]) << 16);
  o.w = (uint32_t)f2bf(v[6]) | ((uint32_t)f2bf(v[7]) << 16);
  *reinterpret_cast<uint4*>(p) = o;
}

// Sum of the 8 wave partials (red [8][d]) for this thread's columns into red row 0.
__device__ __forceinline__ void combine_waves(float* red, int d) {
  __syncthreads();
  for (int c = threadIdx.x; c < d; c += kMacroWaves * 64) {
    float s = 0.0f;
#pragma unroll
    for (int w = 0; w < kMacroWaves; ++w) s += red[w * d + c];
    red[c] = s;
  }
  __syncthreads();
}

template <int NCH>
__global__ void __launch_bounds__(512) macro_prologue_fwd_kernel(const float* __restrict__ h,
                                                                 const float* __restrict__ h0, int S, int d,
                                                                 float eps, bf16* __restrict__ z,
                                                                 float* __restrict__ rstd) {
  extern __shared__ float red[];  // [8][d]
  const int b = blockIdx.x;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int nch = d / 8, D3 = 3 * d;
  const int64_t base = (int64_t)b * S;
  float pool[NCH][8];
#pragma unroll
  for (int j = 0; j < NCH; ++j)
#pragma unroll
    for (int i = 0; i < 8; ++i) pool[j][i] = 0.0f;
  for (int s = wave; s < S; s += kMacroWaves) {
    const int64_t r = base + s;
    float x[NCH][8];
    float ss = 0.0f;
#pragma unroll
    for (int j = 0; j < NCH; ++j) {
      const int ch = lane + 64 * j;
      if (ch >= nch) continue;
      ld8m(h + r * d + ch * 8, x[j]);
#pragma unroll
      for (int i = 0; i < 8; ++i) ss += x[j][i] * x[j][i];
    }
    ss = wsum_m(ss);
    const float rr = rsqrtf(ss / (float)d + eps);
    if (lane == 0) rstd[r] = rr;
#pragma unroll
    for (int j = 0; j < NCH; ++j) {
      const int ch = lane + 64 * j;
      if (ch >= nch) continue;
      float y[8], o[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        y[i] = x[j][i] * rr;
        pool[j][i] += y[i];
      }
      st8m(z + r * D3 + ch * 8, y);
      ld8m(h0 + r * d + ch * 8, o);
      st8m(z + r * D3 + 2 * d + ch * 8, o);
    }
  }
#pragma unroll
  for (int j = 0; j < NCH; ++j) {
    const int ch = lane + 64 * j;
    if (ch < nch) st8m(red + wave * d + ch * 8, pool[j]);
  }
  combine_waves(red, d);
  const float invS = 1.0f / (float)S;
  for (int s = wave; s < S; s += kMacroWaves) {
    const int64_t r = base + s;
#pragma unroll
    for (int j = 0; j < NCH; ++j) {
      const int ch = lane + 64 * j;
      if (ch >= nch) continue;
      float p[8];
      ld8m(red + ch * 8, p);
#pragma unroll
      for (int i = 0; i < 8; ++i) p[i] *= invS;
      st8m(z + r * D3 + d + ch * 8, p);
    }
  }
}

// dh = dh_extra + rmsnorm backward of (dz[:, :d] + mean-broadcast of dz[:, d:2d]); dh0 = dz[:, 2d:]
template <int NCH>
__global__ void __launch_bounds__(512) macro_prologue_bwd_kernel(const bf16* __restrict__ dz,
                                                                 const float* __restrict__ h,
                                                                 const float* __restrict__ rstd,
                                                                 const float* __restrict__ dh_extra, int S, int d,
                                                                 float* __restrict__ dh, float* __restrict__ dh0) {
  extern __shared__ float red[];  // [8][d]
  const int b = blockIdx.x;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int nch = d / 8, D3 = 3 * d;
  const int64_t base = (int64_t)b * S;
  float gp[NCH][8];
#pragma unroll
  for (int j = 0; j < NCH; ++j)
#pragma unroll
    for (int i = 0; i < 8; ++i) gp[j][i] = 0.0f;
  for (int s = wave; s < S; s += kMacroWaves) {
    const int64_t r = base + s;
#pragma unroll
    for (int j = 0; j < NCH; ++j) {
      const int ch = lane + 64 * j;
      if (ch >= nch) continue;
      float g[8];
      ld8m(dz + r * D3 + d + ch * 8, g);
#pragma unroll
      for (int i = 0; i < 8; ++i) gp[j][i] += g[i];
    }
  }
#pragma unroll
  for (int j = 0; j < NCH; ++j) {
    const int ch = lane + 64 * j;
    if (ch < nch) st8m(red + wave * d + ch * 8, gp[j]);
  }
  combine_waves(red, d);
  const float invS = 1.0f / (float)S;
#pragma unroll
  for (int j = 0; j < NCH; ++j) {
    const int ch = lane + 64 * j;
    if (ch >= nch) continue;
    ld8m(red + ch * 8, gp[j]);
#pragma unroll
    for (int i = 0; i < 8; ++i) gp[j][i] *= invS;
  }
  for (int s = wave; s < S; s += kMacroWaves) {
    const int64_t r = base + s;
    const float rr = rstd[r];
    float g[NCH][8], x[NCH][8];
    float dot = 0.0f;
#pragma unroll
    for (int j = 0; j < NCH; ++j) {
      const int ch = lane + 64 * j;
      if (ch >= nch) continue;
      ld8m(dz + r * D3 + ch * 8, g[j]);
      ld8m(h + r * d + ch * 8, x[j]);
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        g[j][i] += gp[j][i];
        dot += g[j][i] * x[j][i];
      }
    }
    dot = wsum_m(dot);
    const float coef = rr * rr * rr * dot / (float)d;
#pragma unroll
    for (int j = 0; j < NCH; ++j) {
      const int ch = lane + 64 * j;
      if (ch >= nch) continue;
      float o[8], e[8] = {0, 0, 0, 0, 0, 0, 0, 0};
      if (dh_extra) ld8m(dh_extra + r * d + ch * 8, e);
#pragma unroll
      for (int i = 0; i < 8; ++i) o[i] = rr * g[j][i] - x[j][i] * coef + e[i];
      st8m(dh + r * d + ch * 8, o);
      if (dh0) {
        float q[8];
        ld8m(dz + r * D3 + 2 * d + ch * 8, q);
        st8m(dh0 + r * d + ch * 8, q);
      }
    }
  }
}

// One wave per row, 4 rows per workgroup of 256.
template <int NCH>
__global__ void __launch_bounds__(256) macro_epilogue_fwd_kernel(const float* __restrict__ h,
                                                                 const float* __restrict__ low,
                                                                 const int64_t* __restrict__ key, int S, int64_t R,
                                                                 int d, const float* __restrict__ gain,
                                                                 const float* __restrict__ bias,
                                                                 const float* __restrict__ scale, float c,
                                                                 float* __restrict__ out) {
  const int lane = threadIdx.x & 63;
  const int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (r >= R) return;
  const int nch = d / 8;
  const int64_t kb = key[r / S] * d;
#pragma unroll
  for (int j = 0; j < NCH; ++j) {
    const int ch = lane + 64 * j;
    if (ch >= nch) continue;
    const int col = ch * 8;
    float x[8], l[8], gn[8], bs[8], sc[8], o[8];
    ld8m(h + r * d + col, x);
    ld8m(low + r * d + col, l);
    ld8m(gain + kb + col, gn);
    ld8m(bias + kb + col, bs);
    ld8m(scale + kb + col, sc);
#pragma unroll
    for (int i = 0; i < 8; ++i) o[i] = x[i] + c * sc[i] * tanhf(gn[i] * x[i] + l[i] + bs[i]);
    st8m(out + r * d + col, o);
  }
}

// Per sample: dh (= dout + dupd * gain), dlow (bf16) and the column sums of the table
// gradients part[b] = (sum dupd * h | sum dupd | sum dout * c * tanh), dupd = dout c scale (1 - t^2).
template <int NCH>
__global__ void __launch_bounds__(512) macro_epilogue_bwd_kernel(const float* __restrict__ dout,
                                                                 const float* __restrict__ h,
                                                                 const float* __restrict__ low,
                                                                 const int64_t* __restrict__ key, int S, int d,
                                                                 const float* __restrict__ gain,
                                                                 const float* __restrict__ bias,
                                                                 const float* __restrict__ scale, float c,
                                                                 float* __restrict__ dh, bf16* __restrict__ dlow,
                                                                 float* __restrict__ part) {
  extern __shared__ float red[];  // [8][d], reused for the three sums
  const int b = blockIdx.x;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int nch = d / 8;
  const int64_t base = (int64_t)b * S;
  const int64_t kb = key[b] * d;
  float gn[NCH][8], bs[NCH][8], sc[NCH][8], pg[NCH][8], pb[NCH][8], ps[NCH][8];
#pragma unroll
  for (int j = 0; j < NCH; ++j) {
    const int ch = lane + 64 * j;
#pragma unroll
    for (int i = 0; i < 8; ++i) pg[j][i] = pb[j][i] = ps[j][i] = 0.0f;
    if (ch >= nch) continue;
    ld8m(gain + kb + ch * 8, gn[j]);
    ld8m(bias + kb + ch * 8, bs[j]);
    ld8m(scale + kb + ch * 8, sc[j]);
  }
  for (int s = wave; s < S; s += kMacroWaves) {
    const int64_t r = base + s;
#pragma unroll
    for (int j = 0; j < NCH; ++j) {
      const int ch = lane + 64 * j;
      if (ch >= nch) continue;
      const int64_t off = r * d + ch * 8;
      float x[8], l[8], go[8], oh[8], ol[8];
      ld8m(h + off, x);
      ld8m(low + off, l);
      ld8m(dout + off, go);
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const float t = tanhf(gn[j][i] * x[i] + l[i] + bs[j][i]);
        const float du = go[i] * c * sc[j][i] * (1.0f - t * t);
        oh[i] = go[i] + du * gn[j][i];
        ol[i] = du;
        pg[j][i] += du * x[i];
        pb[j][i] += du;
        ps[j][i] += go[i] * c * t;
      }
      st8m(dh + off, oh);
      st8m(dlow + off, ol);
    }
  }
  float* pr = part + (int64_t)b * 3 * d;
  for (int q = 0; q < 3; ++q) {
    if (q > 0) __syncthreads();  // the previous sum has been read out of red
#pragma unroll
    for (int j = 0; j < NCH; ++j) {
      const int ch = lane + 64 * j;
      if (ch < nch) st8m(red + wave * d + ch * 8, q == 0 ? pg[j] : (q == 1 ? pb[j] : ps[j]));
    }
    combine_waves(red, d);
    for (int col = threadIdx.x; col < d; col += kMacroWaves * 64) pr[q * d + col] = red[col];
  }
}

// Table gradients: for key v (one workgroup each), the per-sample sums part[b] of the samples
// with key[b] == v, added in sample order, written to the three tables (rows of keys no sample
// uses come out zero).
__global__ void __launch_bounds__(256) macro_table_grad_kernel(const int64_t* __restrict__ key, int B, int d,
                                                               const float* __restrict__ part,
                                                               float* __restrict__ dgain, float* __restrict__ dbias,
                                                               float* __restrict__ dscale) {
  const int v = blockIdx.x;
  for (int col = threadIdx.x; col < d; col += 256) {
    float g = 0.0f, bb = 0.0f, sc = 0.0f;
    for (int b = 0; b < B; ++b) {
      if (key[b] != v) continue;
      const float* pr = part + (int64_t)b * 3 * d;
      g += pr[col];
      bb += pr[d + col];
      sc += pr[2 * d + col];
    }
    if (dgain) dgain[(int64_t)v * d + col] = g;
    if (dbias) dbias[(int64_t)v * d + col] = bb;
    if (dscale) dscale[(int64_t)v * d + col] = sc;
  }
}

bool al16m(const void* p) { return ((uintptr_t)p & 15) == 0; }

}  // namespace

#define MACRO_SIZES(what)                                                                                  \
  RTE_REQUIRE(B >= 0 && S >= 1 && d >= 8 && d % 8 == 0 && d <= 1024, what ": need d % 8 == 0, d <= 1024")

int macro_prologue_fwd(const float* h, const float* h0, int B, int S, int d, float eps, bf16* z, float* rstd,
                       hipStream_t s) {
  MACRO_SIZES("macro_prologue");
  RTE_REQUIRE(al16m(h) && al16m(h0) && al16m(z), "macro_prologue: 16-byte aligned buffers");
  if (B == 0) return 0;
  const size_t lds = (size_t)kMacroWaves * d * sizeof(float);
  if (d <= 512)
    hipLaunchKernelGGL(macro_prologue_fwd_kernel<1>, dim3(B), dim3(512), lds, s, h, h0, S, d, eps, z, rstd);
  else
    hipLaunchKernelGGL(macro_prologue_fwd_kernel<2>, dim3(B), dim3(512), lds, s, h, h0, S, d, eps, z, rstd);
  return check_launch("macro_prologue_fwd");
}

int macro_prologue_bwd(const bf16* dz, const float* h, const float* rstd, const float* dh_extra, int B, int S, int d,
                       float* dh, float* dh0, hipStream_t s) {
  MACRO_SIZES("macro_prologue_bwd");
  RTE_REQUIRE(al16m(dz) && al16m(h) && al16m(dh_extra) && al16m(dh) && al16m(dh0),
              "macro_prologue_bwd: 16-byte aligned buffers");
  if (B == 0) return 0;
  const size_t lds = (size_t)kMacroWaves * d * sizeof(float);
  if (d <= 512)
    hipLaunchKernelGGL(macro_prologue_bwd_kernel<1>, dim3(B), dim3(512), lds, s, dz, h, rstd, dh_extra, S, d, dh, dh0);
  else
    hipLaunchKernelGGL(macro_prologue_bwd_kernel<2>, dim3(B), dim3(512), lds, s, dz, h, rstd, dh_extra, S, d, dh, dh0);
  return check_launch("macro_prologue_bwd");
}

int macro_epilogue_fwd(const float* h, const float* low, const int64_t* key, int B, int S, int d, const float* gain,
                       const float* bias, const float* scale, float c, float* out, hipStream_t s) {
  MACRO_SIZES("macro_epilogue");
  RTE_REQUIRE(al16m(h) && al16m(low) && al16m(gain) && al16m(bias) && al16m(scale) && al16m(out),
              "macro_epilogue: 16-byte aligned buffers");
  const int64_t R = (int64_t)B * S;
  if (R == 0) return 0;
  const dim3 grid((unsigned)((R + 3) / 4));
  if (d <= 512)
    hipLaunchKernelGGL(macro_epilogue_fwd_kernel<1>, grid, dim3(256), 0, s, h, low, key, S, R, d, gain, bias, scale, c,
                       out);
  else
    hipLaunchKernelGGL(macro_epilogue_fwd_kernel<2>, grid, dim3(256), 0, s, h, low, key, S, R, d, gain, bias, scale, c,
                       out);
  return check_launch("macro_epilogue_fwd");
}

int macro_table_grad(const int64_t* key, int B, int G, int d, const float* part, float* dgain, float* dbias,
                     float* dscale, hipStream_t s) {
  RTE_REQUIRE(B >= 0 && G >= 1 && d >= 1, "macro_table_grad: bad sizes");
  if (!dgain && !dbias && !dscale) return 0;
  hipLaunchKernelGGL(macro_table_grad_kernel, dim3(G), dim3(256), 0, s, key, B, d, part, dgain, dbias, dscale);
  return check_launch("macro_table_grad");
}

int macro_epilogue_bwd(const float* dout, const float* h, const float* low, const int64_t* key, int B, int S, int d,
                       const float* gain, const float* bias, const float* scale, float c, float* dh, bf16* dlow,
                       float* part, hipStream_t s) {
  MACRO_SIZES("macro_epilogue_bwd");
  RTE_REQUIRE(al16m(dout) && al16m(h) && al16m(low) && al16m(gain) && al16m(bias) && al16m(scale) && al16m(dh) &&
                  al16m(dlow),
              "macro_epilogue_bwd: 16-byte aligned buffers");
  if (B == 0) return 0;
  const size_t lds = (size_t)kMacroWaves * d * sizeof(float);
  if (d <= 512)
    hipLaunchKernelGGL(macro_epilogue_bwd_kernel<1>, dim3(B), dim3(512), lds, s, dout, h, low, key, S, d, gain, bias,
                       scale, c, dh, dlow, part);
  else
    hipLaunchKernelGGL(macro_epilogue_bwd_kernel<2>, dim3(B), dim3(512), lds, s, dout, h, low, key, S, d, gain, bias,
                       scale, c, dh, dlow, part);
  return check_launch("macro_epilogue_bwd");
}

}  // namespace rte
