// Residual axpy + FiLM RMSNorm of the recursive core's pass (rte/layers.py:826-845):
//
//   h~ = h + alpha * h0;  n1 = rmsnorm(h~) * (1 + gamma1) + beta1
//   u  = h~ + s_attn * attn(n1);  n2 = rmsnorm(u) * (1 + gamma2) + beta2
//   h' = active ? u + s_mlp * mlp(n2) : h
//
// each line is one launch forward (axpy_norm_fwd) and two backward (axpy_norm_bwd, then the
// fixed-order column sum of the per-block parameter-gradient partials):
//
//   fwd : x = a + c * b  (c a device scalar, 1 when absent; b optional); rows of inactive
//         samples (mask[row / S] == 0) take keep instead; optional norm output
//         n = bf16(x * rstd * w * (1 + gamma) + beta), rstd = rsqrt(mean(x^2) + eps)
//   bwd : g = dn * (1 + gamma);  dx = dx_ext + rstd * w * g - x * rstd^3 * mean(w * g * x)
//         da = active ? dx : 0,  db = c * da,  dkeep = active ? 0 : dx
//         partials per block of rows: dw += g * x * rstd, dgamma += dn * x * rstd * w,
//         dbeta += dn, dc += sum(b * da)
#include "common.hpp"

namespace rte {

namespace {

constexpr int kGlueRows = 32;  // most rows per backward workgroup

// Rows per backward workgroup: one per wave for small T, up to 32 once the grid is full.
inline int glue_rows_per_block(int T) {
  int r = ((T + 255) / 256 + 3) / 4 * 4;
  return r < 4 ? 4 : (r > kGlueRows ? kGlueRows : r);
}

__device__ __forceinline__ float wave_sum_g(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

__device__ __forceinline__ void ld8(const float* p, float* v) {
  const float4 a = *reinterpret_cast<const float4*>(p);
  const float4 b = *reinterpret_cast<const float4*>(p + 4);
  v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
  v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
}

__device__ __forceinline__ void ld8(const bf16* p, float* v) {
  const uint4 u = *reinterpret_cast<const uint4*>(p);
  const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    v[2 * i] = __uint_as_float(w[i] << 16);
    v[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
  }
}

__device__ __forceinline__ void st8(float* p, const float* v) {
  *reinterpret_cast<float4*>(p) = make_float4(v[0], v[1], v[2], v[3]);
  *reinterpret_cast<float4*>(p + 4) = make_float4(v[4], v[5], v[6], v[7]);
}

__device__ __forceinline__ void st8(bf16* p, const float* v) {
  uint4 o;
  o.x = pack_bf2(v[0], v[1]);
  o.y = pack_bf2(v[2], v[3]);
  o.z = pack_bf2(v[4], v[5]);
  o.w = pack_bf2(v[6], v[7]);
  *reinterpret_cast<uint4*>(p) = o;
}

// One wave per row, NCH chunks of 8 columns per lane (d <= 512 * NCH, d <= 1024).
template <int NCH>
__global__ void __launch_bounds__(256) axpy_norm_fwd_kernel(
    const float* __restrict__ a, const float* __restrict__ b, const float* __restrict__ c,
    const float* __restrict__ keep, const uint8_t* __restrict__ mask, int S, int T, int d,
    const float* __restrict__ w, const float* __restrict__ gamma, const float* __restrict__ beta, float eps,
    float* __restrict__ x_out, bf16* __restrict__ n_out, float* __restrict__ rstd_out) {
  const int lane = threadIdx.x & 63;
  const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= T) return;
  const int nchunk = d / 8;
  const float cs = c ? *c : 1.0f;
  const bool active = mask ? mask[t / S] != 0 : true;
  const int64_t rb = (int64_t)t * d;
  float x[NCH][8];
  float ss = 0.0f;
#pragma unroll
  for (int j = 0; j < NCH; ++j) {
    const int ch = lane + 64 * j;
    if (ch >= nchunk) continue;
    const int col = ch * 8;
    if (active) {
      ld8(a + rb + col, x[j]);
      if (b) {
        float bv[8];
        ld8(b + rb + col, bv);
#pragma unroll
        for (int i = 0; i < 8; ++i) x[j][i] += cs * bv[i];
      }
    } else {
      ld8(keep + rb + col, x[j]);
    }
    if (x_out) st8(x_out + rb + col, x[j]);
#pragma unroll
    for (int i = 0; i < 8; ++i) ss += x[j][i] * x[j][i];
  }
  if (!n_out) return;
  ss = wave_sum_g(ss);
  const float rstd = rsqrtf(ss / (float)d + eps);
  if (lane == 0) rstd_out[t] = rstd;
#pragma unroll
  for (int j = 0; j < NCH; ++j) {
    const int ch = lane + 64 * j;
    if (ch >= nchunk) continue;
    const int col = ch * 8;
    float wv[8], o[8];
    ld8(w + col, wv);
    float gv[8] = {0, 0, 0, 0, 0, 0, 0, 0}, bt[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    if (gamma) ld8(gamma + col, gv);
    if (beta) ld8(beta + col, bt);
#pragma unroll
    for (int i = 0; i < 8; ++i) o[i] = x[j][i] * rstd * wv[i] * (1.0f + gv[i]) + bt[i];
    st8(n_out + rb + col, o);
  }
}

// Row-parallel backward; each workgroup keeps per-lane column partials across its rows and
// writes one row of part [nblk, 3 d + 1] (dw | dgamma | dbeta | dc), summed later in order.
template <int NCH>
__global__ void __launch_bounds__(256) axpy_norm_bwd_kernel(
    const bf16* __restrict__ dn, const float* __restrict__ dx_ext, const float* __restrict__ x,
    const float* __restrict__ rstd, const float* __restrict__ w, const float* __restrict__ gamma,
    const float* __restrict__ b, const float* __restrict__ c, const uint8_t* __restrict__ mask, int S, int T,
    int d, float* __restrict__ da, float* __restrict__ db, float* __restrict__ dkeep, float* __restrict__ part,
    int rpb) {
  extern __shared__ float sh[];  // [4][3 d + 1]
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int nchunk = d / 8, W = 3 * d + 1;
  const float cs = c ? *c : 1.0f;
  float wv[NCH][8], gm[NCH][8], pw[NCH][8], pg[NCH][8], pb[NCH][8];
#pragma unroll
  for (int j = 0; j < NCH; ++j)
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      wv[j][i] = 0.0f;
      gm[j][i] = 0.0f;
      pw[j][i] = 0.0f;
      pg[j][i] = 0.0f;
      pb[j][i] = 0.0f;
    }
  if (dn) {
#pragma unroll
    for (int j = 0; j < NCH; ++j) {
      const int ch = lane + 64 * j;
      if (ch >= nchunk) continue;
      ld8(w + ch * 8, wv[j]);
      if (gamma) ld8(gamma + ch * 8, gm[j]);
    }
  }
  float pc = 0.0f;
  const int r0 = blockIdx.x * rpb;
  for (int rr = wave; rr < rpb; rr += 4) {
    const int t = r0 + rr;
    if (t >= T) break;
    const int64_t rb = (int64_t)t * d;
    const bool active = mask ? mask[t / S] != 0 : true;
    float g[NCH][8], dnv[NCH][8], xv[NCH][8], dx[NCH][8];
    float rs = 0.0f, dot = 0.0f;
    if (dn) rs = rstd[t];
#pragma unroll
    for (int j = 0; j < NCH; ++j) {
      const int ch = lane + 64 * j;
      if (ch >= nchunk) continue;
      const int col = ch * 8;
      if (dx_ext) ld8(dx_ext + rb + col, dx[j]);
      else
#pragma unroll
        for (int i = 0; i < 8; ++i) dx[j][i] = 0.0f;
      if (dn) {
        ld8(dn + rb + col, dnv[j]);
        ld8(x + rb + col, xv[j]);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          g[j][i] = dnv[j][i] * (1.0f + gm[j][i]);
          dot += wv[j][i] * g[j][i] * xv[j][i];
        }
      }
    }
    if (dn) {
      dot = wave_sum_g(dot);
      const float coef = rs * rs * rs * dot / (float)d;
#pragma unroll
      for (int j = 0; j < NCH; ++j) {
        const int ch = lane + 64 * j;
        if (ch >= nchunk) continue;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          dx[j][i] += rs * wv[j][i] * g[j][i] - xv[j][i] * coef;
          pw[j][i] += g[j][i] * xv[j][i] * rs;
          pg[j][i] += dnv[j][i] * xv[j][i] * rs * wv[j][i];
          pb[j][i] += dnv[j][i];
        }
      }
    }
#pragma unroll
    for (int j = 0; j < NCH; ++j) {
      const int ch = lane + 64 * j;
      if (ch >= nchunk) continue;
      const int col = ch * 8;
      float zero[8] = {0, 0, 0, 0, 0, 0, 0, 0};
      if (da) st8(da + rb + col, active ? dx[j] : zero);
      if (dkeep) st8(dkeep + rb + col, active ? zero : dx[j]);
      if (b && active) {
        float bv[8], o[8];
        ld8(b + rb + col, bv);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          o[i] = cs * dx[j][i];
          pc += bv[i] * dx[j][i];
        }
        if (db) st8(db + rb + col, o);
      } else if (db) {
        st8(db + rb + col, zero);
      }
    }
  }
  pc = wave_sum_g(pc);
  float* mine = sh + wave * W;
#pragma unroll
  for (int j = 0; j < NCH; ++j) {
    const int ch = lane + 64 * j;
    if (ch >= nchunk) continue;
    st8(mine + ch * 8, pw[j]);
    st8(mine + d + ch * 8, pg[j]);
    st8(mine + 2 * d + ch * 8, pb[j]);
  }
  if (lane == 0) mine[3 * d] = pc;
  __syncthreads();
  for (int q = threadIdx.x; q < W; q += 256)
    part[(int64_t)blockIdx.x * W + q] = ((sh[q] + sh[W + q]) + sh[2 * W + q]) + sh[3 * W + q];
}

// out[q] = sum_r part[r, q]: 8 columns per workgroup, 32 row phases combined in phase order.
__global__ void __launch_bounds__(256) glue_colsum_kernel(const float* __restrict__ part, int nrows, int W,
                                                          float* __restrict__ out) {
  __shared__ float s32[32][8];
  const int l = threadIdx.x & 7, phase = threadIdx.x >> 3;
  const int q = blockIdx.x * 8 + l;
  float s = 0.0f;
  if (q < W)
    for (int r = phase; r < nrows; r += 32) s += part[(int64_t)r * W + q];
  s32[phase][l] = s;
  __syncthreads();
  if (threadIdx.x < 8 && q < W) {
    float tot = 0.0f;
#pragma unroll
    for (int p = 0; p < 32; ++p) tot += s32[p][l];
    out[q] = tot;
  }
}

bool al16(const void* p) { return ((uintptr_t)p & 15) == 0; }

// ---- mean squared difference (the macro consistency loss, rte/macro.py:342-359) ----
// fwd: per-block sums of (a - b)^2 over fixed contiguous ranges (block-local tree in a fixed
// order), then one workgroup adds the block sums in block order and scales by 1/n.
constexpr int kMseThreads = 256, kMseMaxBlocks = 1024;

__device__ __forceinline__ float block_sum_g(float v, float* red) {
  v = wave_sum_g(v);
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  __syncthreads();
  if (lane == 0) red[w] = v;
  __syncthreads();
  float t = 0.0f;
  for (int i = 0; i < (int)(blockDim.x >> 6); ++i) t += red[i];
  return t;
}

__global__ void __launch_bounds__(kMseThreads) mse_partial_kernel(const float* __restrict__ a, const float* __restrict__ b,
                                                                  int64_t n, int64_t chunk, float* __restrict__ part) {
  __shared__ float red[kMseThreads / 64];
  const int64_t lo = (int64_t)blockIdx.x * chunk;
  const int64_t hi = lo + chunk < n ? lo + chunk : n;
  float s = 0.0f;
  for (int64_t i = lo + 4 * threadIdx.x; i < hi; i += 4 * kMseThreads) {  // chunk is a multiple of 4
    if (i + 4 <= hi) {
      const float4 x = *reinterpret_cast<const float4*>(a + i), y = *reinterpret_cast<const float4*>(b + i);
      const float d0 = x.x - y.x, d1 = x.y - y.y, d2 = x.z - y.z, d3 = x.w - y.w;
      s += d0 * d0 + d1 * d1 + d2 * d2 + d3 * d3;
    } else {
      for (int64_t j = i; j < hi; ++j) {
        const float dd = a[j] - b[j];
        s += dd * dd;
      }
    }
  }
  s = block_sum_g(s, red);
  if (threadIdx.x == 0) part[blockIdx.x] = s;
}

__global__ void __launch_bounds__(kMseMaxBlocks) mse_final_kernel(const float* __restrict__ part, int nb, float inv_n,
                                                                  float* __restrict__ out) {
  __shared__ float red[kMseMaxBlocks / 64];
  const float v = (int)threadIdx.x < nb ? part[threadIdx.x] : 0.0f;
  const float t = block_sum_g(v, red);
  if (threadIdx.x == 0) out[0] = t * inv_n;
}

// da = g 2 (a - b) / n, db = -da (each optional)
__global__ void __launch_bounds__(256) mse_bwd_kernel(const float* __restrict__ a, const float* __restrict__ b, int64_t n,
                                                      const float* __restrict__ g, float two_over_n,
                                                      float* __restrict__ da, float* __restrict__ db) {
  const float f = g[0] * two_over_n;
  for (int64_t i = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 4; i < n; i += (int64_t)gridDim.x * 256 * 4) {
    if (i + 4 <= n) {
      const float4 x = *reinterpret_cast<const float4*>(a + i), y = *reinterpret_cast<const float4*>(b + i);
      const float4 o = make_float4(f * (x.x - y.x), f * (x.y - y.y), f * (x.z - y.z), f * (x.w - y.w));
      if (da) *reinterpret_cast<float4*>(da + i) = o;
      if (db) *reinterpret_cast<float4*>(db + i) = make_float4(-o.x, -o.y, -o.z, -o.w);
    } else {
      for (int64_t j = i; j < n; ++j) {
        const float o = f * (a[j] - b[j]);
        if (da) da[j] = o;
        if (db) db[j] = -o;
      }
    }
  }
}

int mse_blocks(int64_t n, int64_t* chunk) {
  int64_t nb = (n + 16383) / 16384;  // about 16 Ki elements per block
  if (nb < 1) nb = 1;
  if (nb > kMseMaxBlocks) nb = kMseMaxBlocks;
  int64_t c = (n + nb - 1) / nb;
  c = (c + 3) / 4 * 4;
  *chunk = c;
  return (int)((n + c - 1) / c > 0 ? (n + c - 1) / c : 1);
}

}  // namespace

int axpy_norm_fwd(const float* a, const float* b, const float* c, const float* keep, const uint8_t* mask, int S,
                  int T, int d, const float* w, const float* gamma, const float* beta, float eps, float* x_out,
                  bf16* n_out, float* rstd_out, hipStream_t s) {
  RTE_REQUIRE(d % 8 == 0 && d >= 8 && d <= 1024, "axpy_norm: d must be a multiple of 8 in [8, 1024]");
  RTE_REQUIRE(a && (x_out || n_out), "axpy_norm: need the input and an output");
  RTE_REQUIRE(!mask || (keep && S >= 1), "axpy_norm: a sample mask needs keep rows and S >= 1");
  RTE_REQUIRE(!n_out || (w && rstd_out), "axpy_norm: the norm output needs w and rstd");
  for (const void* p : {(const void*)a, (const void*)b, (const void*)keep, (const void*)w, (const void*)gamma,
                        (const void*)beta, (const void*)x_out, (const void*)n_out})
    RTE_REQUIRE(!p || al16(p), "axpy_norm: buffers must be 16-byte aligned");
  if (T == 0) return 0;
  const dim3 grid((T + 3) / 4);
  if (d <= 512)
    hipLaunchKernelGGL(axpy_norm_fwd_kernel<1>, grid, dim3(256), 0, s, a, b, c, keep, mask, S, T, d, w, gamma, beta,
                       eps, x_out, n_out, rstd_out);
  else
    hipLaunchKernelGGL(axpy_norm_fwd_kernel<2>, grid, dim3(256), 0, s, a, b, c, keep, mask, S, T, d, w, gamma, beta,
                       eps, x_out, n_out, rstd_out);
  return check_launch("axpy_norm_fwd");
}

size_t axpy_norm_bwd_workspace_bytes(int T, int d) {
  const int rpb = glue_rows_per_block(T);
  const int nblk = (T + rpb - 1) / rpb;
  return (size_t)(nblk > 0 ? nblk : 1) * (size_t)(3 * d + 1) * sizeof(float);
}

int axpy_norm_bwd(const bf16* dn, const float* dx_ext, const float* x, const float* rstd, const float* w,
                  const float* gamma, const float* b, const float* c, const uint8_t* mask, int S, int T, int d,
                  float* da, float* db, float* dkeep, float* dparams, void* ws, size_t ws_bytes, hipStream_t s) {
  RTE_REQUIRE(d % 8 == 0 && d >= 8 && d <= 1024, "axpy_norm_bwd: d must be a multiple of 8 in [8, 1024]");
  RTE_REQUIRE(!dn || (x && rstd && w), "axpy_norm_bwd: the norm gradient needs x, rstd and w");
  RTE_REQUIRE(!mask || S >= 1, "axpy_norm_bwd: a sample mask needs S >= 1");
  RTE_REQUIRE(dparams, "axpy_norm_bwd: need the parameter-gradient output (3 d + 1 floats)");
  RTE_REQUIRE(ws_bytes >= axpy_norm_bwd_workspace_bytes(T, d), "axpy_norm_bwd: workspace too small");
  for (const void* p : {(const void*)dn, (const void*)dx_ext, (const void*)x, (const void*)w, (const void*)gamma,
                        (const void*)b, (const void*)da, (const void*)db, (const void*)dkeep})
    RTE_REQUIRE(!p || al16(p), "axpy_norm_bwd: buffers must be 16-byte aligned");
  const int W = 3 * d + 1;
  if (T == 0) return fill_f32(dparams, 0.0f, W, s);
  const int rpb = glue_rows_per_block(T);
  const int nblk = (T + rpb - 1) / rpb;
  float* part = static_cast<float*>(ws);
  const size_t lds = (size_t)4 * W * sizeof(float);
  if (d <= 512)
    hipLaunchKernelGGL(axpy_norm_bwd_kernel<1>, dim3(nblk), dim3(256), lds, s, dn, dx_ext, x, rstd, w, gamma, b, c,
                       mask, S, T, d, da, db, dkeep, part, rpb);
  else
    hipLaunchKernelGGL(axpy_norm_bwd_kernel<2>, dim3(nblk), dim3(256), lds, s, dn, dx_ext, x, rstd, w, gamma, b, c,
                       mask, S, T, d, da, db, dkeep, part, rpb);
  RTE_TRY(check_launch("axpy_norm_bwd"));
  hipLaunchKernelGGL(glue_colsum_kernel, dim3((W + 7) / 8), dim3(256), 0, s, part, nblk, W, dparams);
  return check_launch("axpy_norm_colsum");
}

size_t mse_workspace_bytes(int64_t n) {
  int64_t chunk;
  return (size_t)mse_blocks(n, &chunk) * sizeof(float);
}

int mse_fwd(const float* a, const float* b, int64_t n, float* out, void* ws, size_t ws_bytes, hipStream_t s) {
  RTE_REQUIRE(n >= 1, "mse: need at least one element");
  RTE_REQUIRE(((uintptr_t)a & 15) == 0 && ((uintptr_t)b & 15) == 0, "mse: 16-byte aligned inputs");
  int64_t chunk;
  const int nb = mse_blocks(n, &chunk);
  RTE_REQUIRE(ws && ws_bytes >= (size_t)nb * sizeof(float), "mse: workspace too small");
  float* part = static_cast<float*>(ws);
  hipLaunchKernelGGL(mse_partial_kernel, dim3(nb), dim3(kMseThreads), 0, s, a, b, n, chunk, part);
  RTE_TRY(check_launch("mse_partial"));
  hipLaunchKernelGGL(mse_final_kernel, dim3(1), dim3(kMseMaxBlocks), 0, s, part, nb, (float)(1.0 / (double)n), out);
  return check_launch("mse_final");
}

int mse_bwd(const float* a, const float* b, int64_t n, const float* g, float* da, float* db, hipStream_t s) {
  RTE_REQUIRE(n >= 1, "mse: need at least one element");
  RTE_REQUIRE(((uintptr_t)a & 15) == 0 && ((uintptr_t)b & 15) == 0 && ((uintptr_t)da & 15) == 0 &&
                  ((uintptr_t)db & 15) == 0,
              "mse: 16-byte aligned buffers");
  if (!da && !db) return 0;
  int64_t blocks = (n + 1023) / 1024;
  if (blocks > 4096) blocks = 4096;
  hipLaunchKernelGGL(mse_bwd_kernel, dim3((unsigned)blocks), dim3(256), 0, s, a, b, n, g, (float)(2.0 / (double)n), da,
                     db);
  return check_launch("mse_bwd");
}

}  // namespace rte
