// Elementwise / row-reduction kernels around the GEMMs: RMSNorm forward and
// backward (deterministic two-stage weight-gradient reduction), the inverse
// RoPE + [B,H,S,hd] -> [T, 3d] repack for the fused-QKV backward, dtype casts,
// fills, and the library's error state.
#include "common.hpp"

#include <stdarg.h>
#include <stdio.h>
#include <string.h>

namespace rte {

static thread_local char g_err[1024] = "";

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
}

const char* last_error() { return g_err; }

int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error("%s: launch failed: %s", what, hipGetErrorString(e));
    return (int)e;
  }
  return 0;
}

namespace {

template <typename T>
__global__ void fill_kernel(T* p, T v, int64_t n) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = v;
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

// One wave per row.  x fp32 [T, d]; out bf16 = bf16(x * rstd * w); rstd [T].
__global__ void __launch_bounds__(256) rmsnorm_fwd_kernel(const float* __restrict__ x,
                                                          const float* __restrict__ w, int T, int d,
                                                          float eps, bf16* __restrict__ out,
                                                          float* __restrict__ rstd_out) {
  const int lane = threadIdx.x & 63;
  const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= T) return;
  const float* xr = x + (int64_t)t * d;
  float ss = 0.0f;
  for (int c = lane * 4; c < d; c += 256) {
    const float4 v = *reinterpret_cast<const float4*>(xr + c);
    ss += v.x * v.x + v.y * v.y + v.z * v.z + v.w * v.w;
  }
  ss = wave_sum(ss);
  const float rstd = rsqrtf(ss / (float)d + eps);
  if (lane == 0 && rstd_out) rstd_out[t] = rstd;
  bf16* orow = out + (int64_t)t * d;
  for (int c = lane * 4; c < d; c += 256) {
    const float4 v = *reinterpret_cast<const float4*>(xr + c);
    const float4 g = *reinterpret_cast<const float4*>(w + c);
    uint2 o;
    o.x = pack_bf2(v.x * rstd * g.x, v.y * rstd * g.y);
    o.y = pack_bf2(v.z * rstd * g.z, v.w * rstd * g.w);
    *reinterpret_cast<uint2*>(orow + c) = o;
  }
}

// dx = rstd * (w*dy) - x * rstd^3 * mean(w*dy*x)  (+ dres);   partial dw per row block;
// optionally also dx in bf16 (the operand of the GEMMs that consume it).
// One wave per row, 8 columns per lane per step (16-byte dy loads, 32-byte x loads);
// each lane keeps its columns' dw partial in registers across the block's rows, so
// dw needs no atomics: per-block partials are summed in block order by colsum_kernel.
constexpr int kNormRowsPerBlock = 32;  // upper bound; small T uses fewer rows per block

constexpr int kNormMaxChunks = 4;  // d <= 64 lanes * 8 * 4 = 2048

// 8-column chunks per lane of the backward kernel instantiated for d
inline int norm_chunks(int d) { return (d / 8 + 63) / 64; }

// Rows per backward workgroup: 4 (one per wave) for small T, up to 32 once the grid is full.
// With one chunk per lane (d <= 512) the kernel is small enough for 8 waves per SIMD, so the
// grid aims at 1024 workgroups (two rows per wave at T = 8192) instead of 256.
inline int norm_rows_per_block(int T, int d) {
  const int target = norm_chunks(d) == 1 ? 1024 : 256;
  int r = ((T + target - 1) / target + 3) / 4 * 4;
  return r < 4 ? 4 : (r > kNormRowsPerBlock ? kNormRowsPerBlock : r);
}

__device__ __forceinline__ void load8_bf16(const bf16* p, float* v) {
  const uint4 u = *reinterpret_cast<const uint4*>(p);
  const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    v[2 * i] = __uint_as_float(w[i] << 16);
    v[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
  }
}

__device__ __forceinline__ void load8_f32(const float* p, float* v) {
  const float4 a = *reinterpret_cast<const float4*>(p);
  const float4 b = *reinterpret_cast<const float4*>(p + 4);
  v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
  v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
}

__device__ __forceinline__ void store8_f32(float* p, const float* v) {
  *reinterpret_cast<float4*>(p) = make_float4(v[0], v[1], v[2], v[3]);
  *reinterpret_cast<float4*>(p + 4) = make_float4(v[4], v[5], v[6], v[7]);
}

template <int NCH>
__global__ void __launch_bounds__(256) rmsnorm_bwd_kernel(
    const bf16* __restrict__ dy, const float* __restrict__ x, const float* __restrict__ w,
    const float* __restrict__ rstd, const float* __restrict__ dres, int T, int d,
    float* __restrict__ dx, bf16* __restrict__ dx_bf16, float* __restrict__ dw_part, int rpb) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  extern __shared__ float sdw[];  // [4][d]
  const int nchunk = d / 8;
  float wv[NCH][8];
  float acc[NCH][8];
#pragma unroll
  for (int c = 0; c < NCH; ++c) {
#pragma unroll
    for (int t = 0; t < 8; ++t) {
      acc[c][t] = 0.0f;
      wv[c][t] = 0.0f;
    }
    if (lane + 64 * c < nchunk) load8_f32(w + (lane + 64 * c) * 8, wv[c]);
  }
  const int r0 = blockIdx.x * rpb;
  for (int rr = wave; rr < rpb; rr += 4) {
    const int t = r0 + rr;
    if (t >= T) break;
    const float rs = rstd[t];
    float g[NCH][8], xv[NCH][8];
    float dot = 0.0f;
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
      if (lane + 64 * c >= nchunk) continue;
      const int col = (lane + 64 * c) * 8;
      load8_bf16(dy + (int64_t)t * d + col, g[c]);
      load8_f32(x + (int64_t)t * d + col, xv[c]);
#pragma unroll
      for (int i = 0; i < 8; ++i) dot += wv[c][i] * g[c][i] * xv[c][i];
    }
    dot = wave_sum(dot);
    const float coef = rs * rs * rs * dot / (float)d;
#pragma unroll
    for (int c = 0; c < NCH; ++c) {
      if (lane + 64 * c >= nchunk) continue;
      const int col = (lane + 64 * c) * 8;
      float o[8];
      if (dres) load8_f32(dres + (int64_t)t * d + col, o);
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const float v = rs * wv[c][i] * g[c][i] - xv[c][i] * coef;
        o[i] = dres ? o[i] + v : v;
        acc[c][i] += g[c][i] * xv[c][i] * rs;
      }
      store8_f32(dx + (int64_t)t * d + col, o);
      if (dx_bf16) {
        uint4 ob;
        ob.x = pack_bf2(o[0], o[1]);
        ob.y = pack_bf2(o[2], o[3]);
        ob.z = pack_bf2(o[4], o[5]);
        ob.w = pack_bf2(o[6], o[7]);
        *reinterpret_cast<uint4*>(dx_bf16 + (int64_t)t * d + col) = ob;
      }
    }
  }
#pragma unroll
  for (int c = 0; c < NCH; ++c)
    if (lane + 64 * c < nchunk) store8_f32(sdw + wave * d + (lane + 64 * c) * 8, acc[c]);
  __syncthreads();
  for (int c = threadIdx.x; c < d; c += 256)
    dw_part[(int64_t)blockIdx.x * d + c] = ((sdw[c] + sdw[d + c]) + sdw[2 * d + c]) + sdw[3 * d + c];
}

// out[c] (+)= sum_r part[r, c]: 8 columns per workgroup, 32 row phases per column, the phase
// sums combined in phase order (fixed order; 8x more workgroups than one column per lane).
__global__ void __launch_bounds__(256) colsum_kernel(const float* __restrict__ part, int nrows, int d,
                                                     float* __restrict__ out, int accumulate) {
  __shared__ float sh[32][8];
  const int l = threadIdx.x & 7, phase = threadIdx.x >> 3;
  const int col = blockIdx.x * 8 + l;
  float s = 0.0f;
  if (col < d) {
    // eight rows' loads in flight at a time, added in row order
    int r = phase;
    for (; r + 7 * 32 < nrows; r += 8 * 32) {
      float v[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) v[u] = part[(int64_t)(r + 32 * u) * d + col];
#pragma unroll
      for (int u = 0; u < 8; ++u) s += v[u];
    }
    for (; r < nrows; r += 32) s += part[(int64_t)r * d + col];
  }
  sh[phase][l] = s;
  __syncthreads();
  if (threadIdx.x < 8 && col < d) {
    float tot = 0.0f;
#pragma unroll
    for (int q = 0; q < 32; ++q) tot += sh[q][l];
    out[col] = accumulate ? out[col] + tot : tot;
  }
}

// One workgroup per token row of dqkv [T, 3d]: each thread writes 8 consecutive columns (a
// 16-byte store) from 8 consecutive dims of one head of dq / dk / dv (16-byte loads), with the
// inverse interleaved rotation on the q and k parts.  Row (b, s) is divided out once per
// workgroup, the column's (part, head, dim) once per chunk.
__global__ void __launch_bounds__(256) rope_bwd_pack_kernel(
    const bf16* __restrict__ dq, const bf16* __restrict__ dk, const bf16* __restrict__ dv,
    int64_t sb, int64_t sh, int64_t ss, int64_t sbk, int64_t shk, int64_t ssk, int64_t sbv, int64_t shv,
    int64_t ssv, const float* __restrict__ cos_t, const float* __restrict__ sin_t, int B, int H, int S,
    int hd, bf16* __restrict__ dqkv) {
  const int d = H * hd, nch = 3 * d / 8;
  const int t = blockIdx.x;
  const int b = t / S, sq = t - b * S;
  bf16* orow = dqkv + (int64_t)t * 3 * d;
  for (int c = threadIdx.x; c < nch; c += 256) {
    const int col = c * 8;
    const int part = col / d, within = col - part * d;
    const int h = within / hd, dim = within - h * hd;
    const bf16* src;
    if (part == 0) src = dq + b * sb + h * sh + sq * ss + dim;
    else if (part == 1) src = dk + b * sbk + h * shk + sq * ssk + dim;
    else src = dv + b * sbv + h * shv + sq * ssv + dim;
    const uint4 u = *reinterpret_cast<const uint4*>(src);
    const uint32_t w[4] = {u.x, u.y, u.z, u.w};
    float y[8];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      y[2 * i] = __uint_as_float(w[i] << 16);
      y[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
    }
    if (part < 2) {
      const float* cp = cos_t + (int64_t)sq * hd + dim;
      const float* sp = sin_t + (int64_t)sq * hd + dim;
      const float4 c0 = *reinterpret_cast<const float4*>(cp), c1 = *reinterpret_cast<const float4*>(cp + 4);
      const float4 s0 = *reinterpret_cast<const float4*>(sp), s1 = *reinterpret_cast<const float4*>(sp + 4);
      const float cv[8] = {c0.x, c0.y, c0.z, c0.w, c1.x, c1.y, c1.z, c1.w};
      const float sv[8] = {s0.x, s0.y, s0.z, s0.w, s1.x, s1.y, s1.z, s1.w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float ye = y[2 * i], yo = y[2 * i + 1];  // fma order shared with the attention backward
        y[2 * i] = fmaf(ye, cv[2 * i], yo * sv[2 * i + 1]);
        y[2 * i + 1] = fmaf(yo, cv[2 * i + 1], -(ye * sv[2 * i]));
      }
    }
    uint4 o;
    o.x = pack_bf2(y[0], y[1]);
    o.y = pack_bf2(y[2], y[3]);
    o.z = pack_bf2(y[4], y[5]);
    o.w = pack_bf2(y[6], y[7]);
    *reinterpret_cast<uint4*>(orow + col) = o;
  }
}

__global__ void __launch_bounds__(256) cast_f32_bf16_kernel(const float* __restrict__ x, int64_t n,
                                                            bf16* __restrict__ y) {
  const int64_t i = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * 4;
  if (i + 3 < n) {
    const float4 v = *reinterpret_cast<const float4*>(x + i);
    uint2 o;
    o.x = pack_bf2(v.x, v.y);
    o.y = pack_bf2(v.z, v.w);
    *reinterpret_cast<uint2*>(y + i) = o;
  } else {
    for (int64_t j = i; j < n; ++j) y[j] = f2bf(x[j]);
  }
}

// Several fp32 -> bf16 casts in one launch.  Job row (int64 x 8): {src, dst, rows, cols, ld,
// kind, first_blk, 0}; dst is a contiguous [rows, cols] bf16 matrix.  kind 0: src is the same
// matrix contiguous, cast in runs of kCastRun elements per workgroup; kind 1: src holds the
// matrix column by column (element (r, c) at src[c * ld + r], a transposed view), cast in
// 64 x 64 tiles staged through LDS so reads and writes both run along memory.  blk[b] is the
// job of workgroup b.  Rounding as cast_f32_bf16_kernel (nearest even, the same conversion).
constexpr int kCastRun = 4096;

__global__ void __launch_bounds__(256) cast_many_kernel(const int64_t* __restrict__ jobs,
                                                        const int32_t* __restrict__ blk) {
  __shared__ float tile[64][65];
  const int b = blockIdx.x, tid = threadIdx.x;
  const int64_t* jr = jobs + 8 * blk[b];
  const float* src = reinterpret_cast<const float*>(jr[0]);
  bf16* dst = reinterpret_cast<bf16*>(jr[1]);
  const int64_t rows = jr[2], cols = jr[3], ld = jr[4];
  const int64_t t = b - jr[6];
  if (jr[5] == 0) {
    const int64_t n = rows * cols;
    const int64_t i0 = t * kCastRun, i1 = i0 + kCastRun < n ? i0 + kCastRun : n;
    const bool vec = ((reinterpret_cast<uintptr_t>(src) | reinterpret_cast<uintptr_t>(dst)) & 15) == 0;
    for (int64_t i = i0 + 4 * tid; i < i1; i += 4 * 256) {
      if (vec && i + 4 <= i1) {
        const float4 v = *reinterpret_cast<const float4*>(src + i);
        uint2 o;
        o.x = pack_bf2(v.x, v.y);
        o.y = pack_bf2(v.z, v.w);
        *reinterpret_cast<uint2*>(dst + i) = o;
      } else {
        for (int64_t j = i; j < i + 4 && j < i1; ++j) dst[j] = f2bf(src[j]);
      }
    }
  } else {
    const int64_t tiles_c = (cols + 63) / 64;
    const int64_t r0 = (t / tiles_c) * 64, c0 = (t % tiles_c) * 64;
    for (int e = tid; e < 64 * 64; e += 256) {  // read along r (contiguous in src)
      const int r = e & 63, c = e >> 6;
      if (r0 + r < rows && c0 + c < cols) tile[c][r] = src[(c0 + c) * ld + r0 + r];
    }
    __syncthreads();
    for (int e = tid; e < 64 * 64; e += 256) {  // write along c (contiguous in dst)
      const int c = e & 63, r = e >> 6;
      if (r0 + r < rows && c0 + c < cols) dst[(r0 + r) * cols + c0 + c] = f2bf(tile[c][r]);
    }
  }
}

}  // namespace

int cast_many_blocks(int kind, int64_t rows, int64_t cols) {
  if (rows <= 0 || cols <= 0) return 0;
  if (kind == 0) return (int)((rows * cols + kCastRun - 1) / kCastRun);
  return (int)(((rows + 63) / 64) * ((cols + 63) / 64));
}

int cast_many(const int64_t* jobs, const int32_t* blk, int nblk, hipStream_t s) {
  if (nblk <= 0) return 0;
  hipLaunchKernelGGL(cast_many_kernel, dim3((unsigned)nblk), dim3(256), 0, s, jobs, blk);
  return check_launch("cast_many");
}

int fill_i32(int32_t* p, int32_t value, int64_t n, hipStream_t s) {
  if (n <= 0) return 0;
  hipLaunchKernelGGL(fill_kernel<int32_t>, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, p, value, n);
  return check_launch("fill_i32");
}

int fill_f32(float* p, float value, int64_t n, hipStream_t s) {
  if (n <= 0) return 0;
  hipLaunchKernelGGL(fill_kernel<float>, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, p, value, n);
  return check_launch("fill_f32");
}

int rmsnorm_fwd(const float* x, const float* w, int T, int d, float eps, bf16* out, float* rstd,
                hipStream_t s) {
  RTE_REQUIRE(d % 4 == 0, "rmsnorm: d must be a multiple of 4");
  if (T == 0) return 0;
  hipLaunchKernelGGL(rmsnorm_fwd_kernel, dim3((T + 3) / 4), dim3(256), 0, s, x, w, T, d, eps, out, rstd);
  return check_launch("rmsnorm_fwd");
}

size_t rmsnorm_bwd_workspace_bytes(int T, int d) {
  const int rpb = norm_rows_per_block(T, d);
  const int nblk = (T + rpb - 1) / rpb;
  return (size_t)(nblk > 0 ? nblk : 1) * d * sizeof(float);
}

int rmsnorm_bwd(const bf16* dy, const float* x, const float* w, const float* rstd, const float* dres, int T,
                int d, float* dx, bf16* dx_bf16, float* dw, int dw_accumulate, void* ws, size_t ws_bytes,
                hipStream_t s) {
  RTE_REQUIRE(ws_bytes >= rmsnorm_bwd_workspace_bytes(T, d), "rmsnorm_bwd: workspace too small");
  RTE_REQUIRE(d % 8 == 0 && d <= 64 * 8 * kNormMaxChunks, "rmsnorm_bwd: d must be a multiple of 8 and <= 2048");
  const int rpb = norm_rows_per_block(T, d);
  const int nblk = (T + rpb - 1) / rpb;
  float* part = static_cast<float*>(ws);
  if (nblk > 0) {
    const size_t lds = 4 * d * sizeof(float);
    switch (norm_chunks(d)) {
      case 1:
        hipLaunchKernelGGL(rmsnorm_bwd_kernel<1>, dim3(nblk), dim3(256), lds, s, dy, x, w, rstd, dres, T, d, dx,
                           dx_bf16, part, rpb);
        break;
      case 2:
        hipLaunchKernelGGL(rmsnorm_bwd_kernel<2>, dim3(nblk), dim3(256), lds, s, dy, x, w, rstd, dres, T, d, dx,
                           dx_bf16, part, rpb);
        break;
      default:
        hipLaunchKernelGGL(rmsnorm_bwd_kernel<kNormMaxChunks>, dim3(nblk), dim3(256), lds, s, dy, x, w, rstd, dres,
                           T, d, dx, dx_bf16, part, rpb);
    }
    RTE_TRY(check_launch("rmsnorm_bwd"));
  }
  if (dw) {
    if (nblk == 0) return dw_accumulate ? 0 : fill_f32(dw, 0.0f, d, s);
    hipLaunchKernelGGL(colsum_kernel, dim3((d + 7) / 8), dim3(256), 0, s, part, nblk, d, dw, dw_accumulate);
    RTE_TRY(check_launch("rmsnorm_dw"));
  }
  return 0;
}

int rope_bwd_pack(const bf16* dq, const int64_t* sq, const bf16* dk, const int64_t* sk, const bf16* dv,
                  const int64_t* sv, const float* cos_t, const float* sin_t, int B, int H, int S, int hd,
                  bf16* dqkv, hipStream_t s) {
  RTE_REQUIRE(hd % 8 == 0, "rope_bwd: head_dim must be a multiple of 8");
  for (int i = 0; i < 3; ++i) {
    const int64_t* st = i == 0 ? sq : (i == 1 ? sk : sv);
    const bf16* base = i == 0 ? dq : (i == 1 ? dk : dv);
    RTE_REQUIRE(st[3] == 1, "rope_bwd: innermost stride must be 1");
    RTE_REQUIRE(st[0] % 8 == 0 && st[1] % 8 == 0 && st[2] % 8 == 0 && ((uintptr_t)base & 15) == 0,
                "rope_bwd: gradients need 16-byte aligned rows (strides multiples of 8)");
  }
  RTE_REQUIRE(((uintptr_t)dqkv & 15) == 0 && ((uintptr_t)cos_t & 15) == 0 && ((uintptr_t)sin_t & 15) == 0,
              "rope_bwd: 16-byte aligned buffers");
  const int64_t T = (int64_t)B * S;
  if (T == 0 || H * hd == 0) return 0;
  RTE_REQUIRE(T < ((int64_t)1 << 31), "rope_bwd: too many tokens");
  hipLaunchKernelGGL(rope_bwd_pack_kernel, dim3((unsigned)T), dim3(256), 0, s, dq, dk, dv, sq[0], sq[1], sq[2],
                     sk[0], sk[1], sk[2], sv[0], sv[1], sv[2], cos_t, sin_t, B, H, S, hd, dqkv);
  return check_launch("rope_bwd_pack");
}

int cast_f32_bf16(const float* x, int64_t n, bf16* y, hipStream_t s) {
  if (n <= 0) return 0;
  const int64_t threads = (n + 3) / 4;
  hipLaunchKernelGGL(cast_f32_bf16_kernel, dim3((unsigned)((threads + 255) / 256)), dim3(256), 0, s, x, n, y);
  return check_launch("cast_f32_bf16");
}

}  // namespace rte
