// Elementwise ends of the bounded-residual macro operator Phi (rte/macro.py:201-236):
//
//   prologue : z = [rmsnorm(h) | mean_s rmsnorm(h) | h0] in bf16 (the grouped GEMMs' input),
//              rmsnorm without weight, eps as given (rte/macro.py:16-18)
//   epilogue : out = h + c * scale[key] * tanh(gain[key] * h + low + bias[key])
//
// with the per-(recipe, stride) rows gain / bias / scale read straight from their tables by
// the sample's key.  Backward: the epilogue gives dh, dlow (bf16, for the GEMM backward) and
// per-sample column sums of the table gradients; the prologue adds the rmsnorm / mean
// backward to dh and gives dh0.  One workgroup per sample wherever rows are reduced, so every
// sum runs in a fixed order.
#include "common.hpp"

namespace rte {

namespace {

constexpr int kMacroMaxS = 4096;  // rows per sample held in LDS (rstd)

__device__ __forceinline__ float wsum_m(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

__global__ void __launch_bounds__(256) macro_prologue_fwd_kernel(const float* __restrict__ h,
                                                                 const float* __restrict__ h0, int S, int d,
                                                                 float eps, bf16* __restrict__ z,
                                                                 float* __restrict__ rstd) {
  __shared__ float rs[kMacroMaxS];
  extern __shared__ float pooled[];  // [d]
  const int b = blockIdx.x;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t base = (int64_t)b * S;
  for (int s = wave; s < S; s += 4) {
    const float* row = h + (base + s) * d;
    float ss = 0.0f;
    for (int c = lane; c < d; c += 64) ss += row[c] * row[c];
    ss = wsum_m(ss);
    const float r = rsqrtf(ss / (float)d + eps);
    if (lane == 0) {
      rs[s] = r;
      rstd[base + s] = r;
    }
  }
  __syncthreads();
  for (int c = threadIdx.x; c < d; c += 256) {
    float acc = 0.0f;
    for (int s = 0; s < S; ++s) acc += h[(base + s) * d + c] * rs[s];
    pooled[c] = acc / (float)S;
  }
  __syncthreads();
  const int D3 = 3 * d;
  for (int s = wave; s < S; s += 4) {
    const float r = rs[s];
    const float* row = h + (base + s) * d;
    const float* row0 = h0 + (base + s) * d;
    bf16* zr = z + (base + s) * D3;
    for (int c = lane; c < d; c += 64) {
      zr[c] = f2bf(row[c] * r);
      zr[d + c] = f2bf(pooled[c]);
      zr[2 * d + c] = f2bf(row0[c]);
    }
  }
}

// dh = dh_extra + rmsnorm backward of (dz[:, :d] + mean-broadcast of dz[:, d:2d]); dh0 = dz[:, 2d:]
__global__ void __launch_bounds__(256) macro_prologue_bwd_kernel(const bf16* __restrict__ dz,
                                                                 const float* __restrict__ h,
                                                                 const float* __restrict__ rstd,
                                                                 const float* __restrict__ dh_extra, int S, int d,
                                                                 float* __restrict__ dh, float* __restrict__ dh0) {
  extern __shared__ float gp[];  // [d]
  const int b = blockIdx.x;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t base = (int64_t)b * S;
  const int D3 = 3 * d;
  for (int c = threadIdx.x; c < d; c += 256) {
    float acc = 0.0f;
    for (int s = 0; s < S; ++s) acc += bf2f(dz[(base + s) * D3 + d + c]);
    gp[c] = acc / (float)S;
  }
  __syncthreads();
  for (int s = wave; s < S; s += 4) {
    const int64_t r = base + s;
    const float rr = rstd[r];
    const float* hr = h + r * d;
    const bf16* zr = dz + r * D3;
    float dot = 0.0f;
    for (int c = lane; c < d; c += 64) dot += (bf2f(zr[c]) + gp[c]) * hr[c];
    dot = wsum_m(dot);
    const float coef = rr * rr * rr * dot / (float)d;
    for (int c = lane; c < d; c += 64) {
      const float g = bf2f(zr[c]) + gp[c];
      float v = rr * g - hr[c] * coef;
      if (dh_extra) v += dh_extra[r * d + c];
      dh[r * d + c] = v;
      if (dh0) dh0[r * d + c] = bf2f(zr[2 * d + c]);
    }
  }
}

__global__ void __launch_bounds__(256) macro_epilogue_fwd_kernel(const float* __restrict__ h,
                                                                 const float* __restrict__ low,
                                                                 const int64_t* __restrict__ key, int S, int64_t n,
                                                                 int d, const float* __restrict__ gain,
                                                                 const float* __restrict__ bias,
                                                                 const float* __restrict__ scale, float c,
                                                                 float* __restrict__ out) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n) return;
  const int64_t row = i / d;
  const int col = (int)(i - row * d);
  const int64_t kr = key[row / S] * d + col;
  const float x = h[i];
  out[i] = x + c * scale[kr] * tanhf(gain[kr] * x + low[i] + bias[kr]);
}

// Per sample: dh (= dout + dupd * gain), dlow (bf16) and the column sums of the table
// gradients part[b] = (sum dupd * h | sum dupd | sum dout * c * tanh), dupd = dout c scale (1 - t^2).
__global__ void __launch_bounds__(256) macro_epilogue_bwd_kernel(const float* __restrict__ dout,
                                                                 const float* __restrict__ h,
                                                                 const float* __restrict__ low,
                                                                 const int64_t* __restrict__ key, int S, int d,
                                                                 const float* __restrict__ gain,
                                                                 const float* __restrict__ bias,
                                                                 const float* __restrict__ scale, float c,
                                                                 float* __restrict__ dh, bf16* __restrict__ dlow,
                                                                 float* __restrict__ part) {
  const int b = blockIdx.x;
  const int64_t base = (int64_t)b * S;
  const int64_t kb = key[b] * d;
  for (int col = threadIdx.x; col < d; col += 256) {
    const float gn = gain[kb + col], bs = bias[kb + col], sc = scale[kb + col];
    float pg = 0.0f, pb = 0.0f, ps = 0.0f;
    for (int s = 0; s < S; ++s) {
      const int64_t i = (base + s) * d + col;
      const float x = h[i], go = dout[i];
      const float t = tanhf(gn * x + low[i] + bs);
      const float du = go * c * sc * (1.0f - t * t);
      dh[i] = go + du * gn;
      dlow[i] = f2bf(du);
      pg += du * x;
      pb += du;
      ps += go * c * t;
    }
    float* pr = part + (int64_t)b * 3 * d;
    pr[col] = pg;
    pr[d + col] = pb;
    pr[2 * d + col] = ps;
  }
}

}  // namespace

int macro_prologue_fwd(const float* h, const float* h0, int B, int S, int d, float eps, bf16* z, float* rstd,
                       hipStream_t s) {
  RTE_REQUIRE(B >= 0 && S >= 1 && S <= kMacroMaxS && d >= 1 && d <= 4096, "macro_prologue: bad sizes");
  if (B == 0) return 0;
  hipLaunchKernelGGL(macro_prologue_fwd_kernel, dim3(B), dim3(256), (size_t)d * sizeof(float), s, h, h0, S, d, eps,
                     z, rstd);
  return check_launch("macro_prologue_fwd");
}

int macro_prologue_bwd(const bf16* dz, const float* h, const float* rstd, const float* dh_extra, int B, int S, int d,
                       float* dh, float* dh0, hipStream_t s) {
  RTE_REQUIRE(B >= 0 && S >= 1 && d >= 1 && d <= 4096, "macro_prologue_bwd: bad sizes");
  if (B == 0) return 0;
  hipLaunchKernelGGL(macro_prologue_bwd_kernel, dim3(B), dim3(256), (size_t)d * sizeof(float), s, dz, h, rstd,
                     dh_extra, S, d, dh, dh0);
  return check_launch("macro_prologue_bwd");
}

int macro_epilogue_fwd(const float* h, const float* low, const int64_t* key, int B, int S, int d, const float* gain,
                       const float* bias, const float* scale, float c, float* out, hipStream_t s) {
  RTE_REQUIRE(B >= 0 && S >= 1 && d >= 1, "macro_epilogue: bad sizes");
  const int64_t n = (int64_t)B * S * d;
  if (n == 0) return 0;
  hipLaunchKernelGGL(macro_epilogue_fwd_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, h, low, key, S, n,
                     d, gain, bias, scale, c, out);
  return check_launch("macro_epilogue_fwd");
}

int macro_epilogue_bwd(const float* dout, const float* h, const float* low, const int64_t* key, int B, int S, int d,
                       const float* gain, const float* bias, const float* scale, float c, float* dh, bf16* dlow,
                       float* part, hipStream_t s) {
  RTE_REQUIRE(B >= 0 && S >= 1 && d >= 1, "macro_epilogue_bwd: bad sizes");
  if (B == 0) return 0;
  hipLaunchKernelGGL(macro_epilogue_bwd_kernel, dim3(B), dim3(256), 0, s, dout, h, low, key, S, d, gain, bias, scale,
                     c, dh, dlow, part);
  return check_launch("macro_epilogue_bwd");
}

}  // namespace rte
