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
// Repeated sources: the operator may run on Bt samples whose h rows are those of sample b % Bh
// and whose h0 rows are those of sample b % Bh0 (Bh0 | Bh | Bt), e.g. one source batch under
// several (recipe, stride) keys.  z depends on (h, h0) only, so the prologue runs on the Bh
// distinct samples and the grouped GEMMs gather its rows; the prologue backward adds the Bt / Bh
// repeats of a sample in repeat order.
//
// Layout: one wave per row, each lane owning NCH chunks of 8 consecutive columns (16- and
// 32-byte accesses; d % 8 == 0, d <= 512 * NCH).  Reductions over a sample's rows run in one
// workgroup of 8 waves: per-lane partials, then the 8 wave partials in wave order, so every
// sum has a fixed order.  Each input element is read once.
#include "common.hpp"

namespace rte {

namespace {

constexpr int kMacroWaves = 8;  // waves per workgroup of the per-sample kernels

// tanh in fp32 at a fraction of the library routine's cost: odd Taylor polynomial below 0.25
// (truncation < 4e-9), else 1 - 2 / (e^(2|x|) + 1) with the sign of x (no cancellation there:
// the result is at least 0.24).  About 2e-7 relative error.
__device__ __forceinline__ float tanh_f(float x) {
  const float a = fabsf(x);
  if (a < 0.25f) {
    const float x2 = x * x;
    return x + x * x2 * (-0.333333333f + x2 * (0.133333333f + x2 * (-0.0539682540f + x2 * 0.0218694885f)));
  }
  const float e = __expf(2.0f * a);
  return copysignf(1.0f - 2.0f * __builtin_amdgcn_rcpf(e + 1.0f), x);
}

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
  o.x = pack_bf2(v[0], v[1]);
  o.y = pack_bf2(v[2], v[3]);
  o.z = pack_bf2(v[4], v[5]);
  o.w = pack_bf2(v[6], v[7]);
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

// Rows [s0, s1) of sample blockIdx.y: part blockIdx.x of the P equal slices of its seq rows.
// Per-sample sums are formed per part (8 wave partials in wave order) and the P part sums are
// added in part order by the consumer, so every sum keeps a fixed order.
struct RowPart {
  int64_t base;
  int s0, s1;
};

__device__ __forceinline__ RowPart row_part(int S, int P) {
  const int rb = (S + P - 1) / P;
  RowPart rp;
  rp.base = (int64_t)blockIdx.y * S;
  rp.s0 = min(S, (int)blockIdx.x * rb);
  rp.s1 = min(S, rp.s0 + rb);
  return rp;
}

// Column sums of this block's 8 wave partials (vals per lane chunk) into dst[0, d).
template <int NCH>
__device__ __forceinline__ void store_part_sum(float* red, const float (&vals)[NCH][8], int d, float* dst) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
  for (int j = 0; j < NCH; ++j) {
    const int ch = lane + 64 * j;
    if (ch < d / 8) st8m(red + wave * d + ch * 8, vals[j]);
  }
  combine_waves(red, d);
  for (int col = threadIdx.x; col < d; col += kMacroWaves * 64) dst[col] = red[col];
}

// mean[0, d) = (sum over the sample's P part sums, in part order) / S, in LDS.
__device__ __forceinline__ void part_mean(const float* __restrict__ part, int S, int P, int d, float* mean,
                                          int64_t sample) {
  const float* pb = part + sample * P * d;
  const float invS = 1.0f / (float)S;
  for (int col = threadIdx.x; col < d; col += kMacroWaves * 64) {
    float s = 0.0f;
    for (int q0 = 0; q0 < P; q0 += 8) {  // 8 independent loads in flight, added in part order
      float v[8];
#pragma unroll
      for (int k = 0; k < 8; ++k) v[k] = q0 + k < P ? pb[(int64_t)(q0 + k) * d + col] : 0.0f;
#pragma unroll
      for (int k = 0; k < 8; ++k) s += v[k];
    }
    mean[col] = s * invS;
  }
  __syncthreads();
}

// z[:, :d] = h * rstd, z[:, 2d:] = h0, rstd per row; part[b, p] = column sums of h * rstd.
template <int NCH>
__global__ void __launch_bounds__(512) macro_prologue_fwd_kernel(const float* __restrict__ h,
                                                                 const float* __restrict__ h0, int Bh0, int S, int P,
                                                                 int d, float eps, bf16* __restrict__ z,
                                                                 float* __restrict__ rstd, float* __restrict__ part) {
  extern __shared__ float red[];  // [8][d]
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int nch = d / 8, D3 = 3 * d;
  const RowPart rp = row_part(S, P);
  const int64_t base0 = (int64_t)(blockIdx.y % Bh0) * S;  // h0 rows of this sample
  float pool[NCH][8];
#pragma unroll
  for (int j = 0; j < NCH; ++j)
#pragma unroll
    for (int i = 0; i < 8; ++i) pool[j][i] = 0.0f;
  for (int s = rp.s0 + wave; s < rp.s1; s += kMacroWaves) {
    const int64_t r = rp.base + s;
    float x[NCH][8], o[NCH][8];
    float ss = 0.0f;
#pragma unroll
    for (int j = 0; j < NCH; ++j) {  // both rows' loads issued before the reduction
      const int ch = lane + 64 * j;
      if (ch >= nch) continue;
      ld8m(h + r * d + ch * 8, x[j]);
      ld8m(h0 + (base0 + s) * d + ch * 8, o[j]);
    }
#pragma unroll
    for (int j = 0; j < NCH; ++j) {
      const int ch = lane + 64 * j;
      if (ch >= nch) continue;
      st8m(z + r * D3 + 2 * d + ch * 8, o[j]);
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
      float y[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        y[i] = x[j][i] * rr;
        pool[j][i] += y[i];
      }
      st8m(z + r * D3 + ch * 8, y);
    }
  }
  store_part_sum<NCH>(red, pool, d, part + ((int64_t)blockIdx.y * P + blockIdx.x) * d);
}

// z[:, d:2d] of this part's rows = the sample's mean of h * rstd.
template <int NCH>
__global__ void __launch_bounds__(512) macro_prologue_mean_kernel(const float* __restrict__ part, int S, int P, int d,
                                                                  bf16* __restrict__ z) {
  __shared__ float mean[1024];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int nch = d / 8, D3 = 3 * d;
  const RowPart rp = row_part(S, P);
  part_mean(part, S, P, d, mean, blockIdx.y);
  for (int s = rp.s0 + wave; s < rp.s1; s += kMacroWaves) {
    const int64_t r = rp.base + s;
#pragma unroll
    for (int j = 0; j < NCH; ++j) {
      const int ch = lane + 64 * j;
      if (ch >= nch) continue;
      float m[8];
      ld8m(mean + ch * 8, m);
      st8m(z + r * D3 + d + ch * 8, m);
    }
  }
}

// part[b, p] = column sums of dz[:, d:2d] over this part's rows.
template <int NCH>
__global__ void __launch_bounds__(512) macro_prologue_bwd_sum_kernel(const bf16* __restrict__ dz, int S, int P,
                                                                     int d, float* __restrict__ part) {
  extern __shared__ float red[];  // [8][d]
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int nch = d / 8, D3 = 3 * d;
  const RowPart rp = row_part(S, P);
  float gp[NCH][8];
#pragma unroll
  for (int j = 0; j < NCH; ++j)
#pragma unroll
    for (int i = 0; i < 8; ++i) gp[j][i] = 0.0f;
  for (int s = rp.s0 + wave; s < rp.s1; s += kMacroWaves) {
    const int64_t r = rp.base + s;
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
  store_part_sum<NCH>(red, gp, d, part + ((int64_t)blockIdx.y * P + blockIdx.x) * d);
}

constexpr int kMaxRep = 4;  // repeats of a source sample the prologue backward adds

// Per source sample b (grid y over Bh) and its repeats b + t Bh (t < rep):
//   dh[b]  = sum_t dh_extra[b + t Bh] + rmsnorm backward of (dz[b + t Bh, :d] + mean-broadcast of
//            dz[b + t Bh, d:2d])        (x and rstd are the source sample's)
//   dh0[b] = sum_t dz[b + t Bh, 2d:]
template <int NCH>
__global__ void __launch_bounds__(512) macro_prologue_bwd_kernel(const bf16* __restrict__ dz,
                                                                 const float* __restrict__ h,
                                                                 const float* __restrict__ rstd,
                                                                 const float* __restrict__ dh_extra,
                                                                 const float* __restrict__ part, int Bh, int rep,
                                                                 int S, int P, int d, float* __restrict__ dh,
                                                                 float* __restrict__ dh0) {
  __shared__ float mean[kMaxRep][1024];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int nch = d / 8, D3 = 3 * d;
  const RowPart rp = row_part(S, P);
  for (int t = 0; t < rep; ++t) part_mean(part, S, P, d, mean[t], (int64_t)blockIdx.y + (int64_t)t * Bh);
  for (int s = rp.s0 + wave; s < rp.s1; s += kMacroWaves) {
    const int64_t r = rp.base + s;  // source row
    const float rr = rstd[r];
    float x[NCH][8], acc[NCH][8], acc0[NCH][8];
#pragma unroll
    for (int j = 0; j < NCH; ++j) {
      const int ch = lane + 64 * j;
#pragma unroll
      for (int i = 0; i < 8; ++i) acc[j][i] = acc0[j][i] = 0.0f;
      if (ch < nch) ld8m(h + r * d + ch * 8, x[j]);
    }
    for (int t = 0; t < rep; ++t) {
      const int64_t rt = r + (int64_t)t * Bh * S;  // row of repeat t
      float g[NCH][8], e[NCH][8];
      float dot = 0.0f;
#pragma unroll
      for (int j = 0; j < NCH; ++j) {  // every load of the row issued before the reduction
        const int ch = lane + 64 * j;
        if (ch >= nch) continue;
        ld8m(dz + rt * D3 + ch * 8, g[j]);
        if (dh_extra) {
          ld8m(dh_extra + rt * d + ch * 8, e[j]);
        } else {
#pragma unroll
          for (int i = 0; i < 8; ++i) e[j][i] = 0.0f;
        }
        if (dh0) {
          float q[8];
          ld8m(dz + rt * D3 + 2 * d + ch * 8, q);
#pragma unroll
          for (int i = 0; i < 8; ++i) acc0[j][i] += q[i];
        }
      }
#pragma unroll
      for (int j = 0; j < NCH; ++j) {
        const int ch = lane + 64 * j;
        if (ch >= nch) continue;
        float m[8];
        ld8m(mean[t] + ch * 8, m);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          g[j][i] += m[i];
          dot += g[j][i] * x[j][i];
        }
      }
      dot = wsum_m(dot);
      const float coef = rr * rr * rr * dot / (float)d;
#pragma unroll
      for (int j = 0; j < NCH; ++j) {
        const int ch = lane + 64 * j;
        if (ch >= nch) continue;
#pragma unroll
        for (int i = 0; i < 8; ++i) acc[j][i] += rr * g[j][i] - x[j][i] * coef + e[j][i];
      }
    }
#pragma unroll
    for (int j = 0; j < NCH; ++j) {
      const int ch = lane + 64 * j;
      if (ch >= nch) continue;
      st8m(dh + r * d + ch * 8, acc[j]);
      if (dh0) st8m(dh0 + r * d + ch * 8, acc0[j]);
    }
  }
}

// One wave per row, 4 rows per workgroup of 256.
template <int NCH>
__global__ void __launch_bounds__(256) macro_epilogue_fwd_kernel(const float* __restrict__ h,
                                                                 const float* __restrict__ low,
                                                                 const int64_t* __restrict__ key, int Bh, int S,
                                                                 int64_t R, int d, const float* __restrict__ gain,
                                                                 const float* __restrict__ bias,
                                                                 const float* __restrict__ scale, float c,
                                                                 float* __restrict__ out) {
  const int lane = threadIdx.x & 63;
  const int64_t r = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (r >= R) return;
  const int nch = d / 8;
  const int64_t kb = key[r / S] * d;
  const int64_t hr = ((r / S) % Bh) * S + r % S;  // source row of h
#pragma unroll
  for (int j = 0; j < NCH; ++j) {
    const int ch = lane + 64 * j;
    if (ch >= nch) continue;
    const int col = ch * 8;
    float x[8], l[8], gn[8], bs[8], sc[8], o[8];
    ld8m(h + hr * d + col, x);
    ld8m(low + r * d + col, l);
    ld8m(gain + kb + col, gn);
    ld8m(bias + kb + col, bs);
    ld8m(scale + kb + col, sc);
#pragma unroll
    for (int i = 0; i < 8; ++i) o[i] = x[i] + c * sc[i] * tanh_f(gn[i] * x[i] + l[i] + bs[i]);
    st8m(out + r * d + col, o);
  }
}

// Per part of a sample: dh (= dout + dupd * gain), dlow (bf16) and the column sums of the
// table gradients part[b, p] = (sum dupd * h | sum dupd | sum dout * c * tanh),
// dupd = dout c scale (1 - t^2).
template <int NCH>
__global__ void __launch_bounds__(512) macro_epilogue_bwd_kernel(const float* __restrict__ dout,
                                                                 const float* __restrict__ h,
                                                                 const float* __restrict__ low,
                                                                 const int64_t* __restrict__ key, int Bh, int S,
                                                                 int P, int d, const float* __restrict__ gain,
                                                                 const float* __restrict__ bias,
                                                                 const float* __restrict__ scale, float c,
                                                                 float* __restrict__ dh, bf16* __restrict__ dlow,
                                                                 float* __restrict__ part) {
  extern __shared__ float red[];  // [8][d], reused for the three sums
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int nch = d / 8;
  const RowPart rp = row_part(S, P);
  const int64_t kb = key[blockIdx.y] * d;
  const int64_t hoff = (int64_t)(blockIdx.y % Bh) * S * d;  // source rows of h
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
  for (int s = rp.s0 + wave; s < rp.s1; s += kMacroWaves) {
    const int64_t r = rp.base + s;
#pragma unroll
    for (int j = 0; j < NCH; ++j) {
      const int ch = lane + 64 * j;
      if (ch >= nch) continue;
      const int64_t off = r * d + ch * 8;
      float x[8], l[8], go[8], oh[8], ol[8];
      ld8m(h + hoff + s * d + ch * 8, x);
      ld8m(low + off, l);
      ld8m(dout + off, go);
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const float t = tanh_f(gn[j][i] * x[i] + l[i] + bs[j][i]);
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
  float* pr = part + ((int64_t)blockIdx.y * P + blockIdx.x) * 3 * d;
  store_part_sum<NCH>(red, pg, d, pr);
  __syncthreads();  // red has been read out
  store_part_sum<NCH>(red, pb, d, pr + d);
  __syncthreads();
  store_part_sum<NCH>(red, ps, d, pr + 2 * d);
}

// Table gradients of key v = blockIdx.x for columns blockIdx.y * 64 + [0, 64) of the 3d part
// columns: the part sums of the samples with key[b] == v, in (sample, part) order, written to
// the three tables (rows of keys no sample uses come out zero).  The samples of v are first
// listed in order in LDS (one ballot per 64 samples); the contributions j = (list index) * P +
// part are then split over 4 thread groups by j mod 4, each summing its share in order with
// 16 loads in flight, and the 4 group sums are added in group order.
__global__ void __launch_bounds__(256) macro_table_grad_kernel(const int64_t* __restrict__ key, int B, int P, int d,
                                                               const float* __restrict__ part,
                                                               float* __restrict__ dgain, float* __restrict__ dbias,
                                                               float* __restrict__ dscale) {
  extern __shared__ int list[];  // [B]
  __shared__ int cnt;
  __shared__ float gsum[4][64];
  const int v = blockIdx.x;
  const int lane = threadIdx.x & 63, grp = threadIdx.x >> 6;
  if (threadIdx.x < 64) {
    int n = 0;
    for (int b0 = 0; b0 < B; b0 += 64) {
      const int b = b0 + lane;
      const bool m = b < B && key[b] == v;
      const unsigned long long bal = __ballot(m);
      if (m) list[n + __popcll(bal & ((1ull << lane) - 1ull))] = b;
      n += __popcll(bal);
    }
    if (lane == 0) cnt = n;
  }
  __syncthreads();
  const int m = cnt * P, D3 = 3 * d;
  const int col = blockIdx.y * 64 + lane;
  float acc = 0.0f;
  if (col < D3) {
    for (int j0 = grp; j0 < m; j0 += 64) {  // 16 loads in flight per thread
      float x[16];
#pragma unroll
      for (int k = 0; k < 16; ++k) {
        const int j = j0 + 4 * k;
        const int jj = j < m ? j : grp;  // past the end: re-read a valid entry, weight 0
        const int i = jj / P, q = jj - i * P;
        x[k] = part[((int64_t)list[i] * P + q) * D3 + col];
      }
#pragma unroll
      for (int k = 0; k < 16; ++k) acc += j0 + 4 * k < m ? x[k] : 0.0f;
    }
  }
  gsum[grp][lane] = acc;
  __syncthreads();
  if (grp != 0 || col >= D3) return;
  const float tot = ((gsum[0][lane] + gsum[1][lane]) + gsum[2][lane]) + gsum[3][lane];
  const int t = col / d, c = col - t * d;
  float* dst = t == 0 ? dgain : (t == 1 ? dbias : dscale);
  if (dst) dst[(int64_t)v * d + c] = tot;
}

bool al16m(const void* p) { return ((uintptr_t)p & 15) == 0; }

}  // namespace

#define MACRO_SIZES(what)                                                                                   \
  RTE_REQUIRE(B >= 0 && B <= 65535 && S >= 1 && d >= 8 && d % 8 == 0 && d <= 1024,                          \
              what ": need B <= 65535, d % 8 == 0, d <= 1024")

// Row parts per sample: slices of about 8 rows (one per wave), halved while the grid would
// exceed 2048 workgroups.
int macro_parts(int B, int S) {
  // at most 512 (sample, part) items: measured at cfg3 (B 128 / 256, S 64, d 512) the forward
  // and backward kernels together take 10% less than with 2048 (fewer partial rows to write
  // and sum, still two workgroups per CU); RTE_MACRO_ITEMS overrides the cap for diagnostics
  static const int max_items = [] {
    const char* v = getenv("RTE_MACRO_ITEMS");
    return v && *v && atoi(v) >= 1 ? atoi(v) : 512;
  }();
  int P = (S + kMacroWaves - 1) / kMacroWaves;
  while (P > 1 && (int64_t)B * P > max_items) P = (P + 1) / 2;
  return P;
}

size_t macro_workspace_bytes(int B, int S, int d) {
  if (B <= 0 || S <= 0 || d <= 0) return 0;
  return (size_t)B * macro_parts(B, S) * 3 * d * sizeof(float);
}

#define MACRO_LAUNCH(kern, lds, ...)                                                           \
  do {                                                                                        \
    if (d <= 512)                                                                             \
      hipLaunchKernelGGL(kern<1>, dim3(P, B), dim3(kMacroWaves * 64), lds, s, __VA_ARGS__);   \
    else                                                                                      \
      hipLaunchKernelGGL(kern<2>, dim3(P, B), dim3(kMacroWaves * 64), lds, s, __VA_ARGS__);   \
  } while (0)

int macro_prologue_fwd(const float* h, const float* h0, int B, int Bh0, int S, int d, float eps, bf16* z, float* rstd,
                       void* ws, size_t ws_bytes, hipStream_t s) {
  MACRO_SIZES("macro_prologue");
  RTE_REQUIRE(Bh0 >= 1 && B % Bh0 == 0, "macro_prologue: the h0 batch must divide the h batch");
  RTE_REQUIRE(al16m(h) && al16m(h0) && al16m(z), "macro_prologue: 16-byte aligned buffers");
  if (B == 0) return 0;
  RTE_REQUIRE(ws && ws_bytes >= macro_workspace_bytes(B, S, d), "macro_prologue: workspace too small");
  const int P = macro_parts(B, S);
  float* part = static_cast<float*>(ws);
  const size_t lds = (size_t)kMacroWaves * d * sizeof(float);
  MACRO_LAUNCH(macro_prologue_fwd_kernel, lds, h, h0, Bh0, S, P, d, eps, z, rstd, part);
  RTE_TRY(check_launch("macro_prologue_fwd"));
  MACRO_LAUNCH(macro_prologue_mean_kernel, 0, part, S, P, d, z);
  return check_launch("macro_prologue_mean");
}

int macro_prologue_bwd(const bf16* dz, const float* h, const float* rstd, const float* dh_extra, int Bt, int Bh, int S,
                       int d, float* dh, float* dh0, void* ws, size_t ws_bytes, hipStream_t s) {
  const int B = Bt;
  MACRO_SIZES("macro_prologue_bwd");
  RTE_REQUIRE(Bh >= 1 && Bt % Bh == 0 && Bt / Bh <= kMaxRep, "macro_prologue_bwd: Bt must be 1 to 4 times Bh");
  RTE_REQUIRE(al16m(dz) && al16m(h) && al16m(dh_extra) && al16m(dh) && al16m(dh0),
              "macro_prologue_bwd: 16-byte aligned buffers");
  if (Bt == 0) return 0;
  RTE_REQUIRE(ws && ws_bytes >= macro_workspace_bytes(Bt, S, d), "macro_prologue_bwd: workspace too small");
  const int P = macro_parts(Bt, S);
  float* part = static_cast<float*>(ws);
  const size_t lds = (size_t)kMacroWaves * d * sizeof(float);
  MACRO_LAUNCH(macro_prologue_bwd_sum_kernel, lds, dz, S, P, d, part);
  RTE_TRY(check_launch("macro_prologue_bwd_sum"));
  {
    const int B = Bh;  // one workgroup per source sample and row slice
    MACRO_LAUNCH(macro_prologue_bwd_kernel, 0, dz, h, rstd, dh_extra, part, Bh, Bt / Bh, S, P, d, dh, dh0);
  }
  return check_launch("macro_prologue_bwd");
}

int macro_epilogue_fwd(const float* h, const float* low, const int64_t* key, int B, int Bh, int S, int d,
                       const float* gain, const float* bias, const float* scale, float c, float* out, hipStream_t s) {
  MACRO_SIZES("macro_epilogue");
  RTE_REQUIRE(Bh >= 1 && B % Bh == 0, "macro_epilogue: the h batch must divide the batch");
  RTE_REQUIRE(al16m(h) && al16m(low) && al16m(gain) && al16m(bias) && al16m(scale) && al16m(out),
              "macro_epilogue: 16-byte aligned buffers");
  const int64_t R = (int64_t)B * S;
  if (R == 0) return 0;
  const dim3 grid((unsigned)((R + 3) / 4));
  if (d <= 512)
    hipLaunchKernelGGL(macro_epilogue_fwd_kernel<1>, grid, dim3(256), 0, s, h, low, key, Bh, S, R, d, gain, bias, scale,
                       c, out);
  else
    hipLaunchKernelGGL(macro_epilogue_fwd_kernel<2>, grid, dim3(256), 0, s, h, low, key, Bh, S, R, d, gain, bias, scale,
                       c, out);
  return check_launch("macro_epilogue_fwd");
}

int macro_epilogue_bwd(const float* dout, const float* h, const float* low, const int64_t* key, int B, int Bh, int S,
                       int d, const float* gain, const float* bias, const float* scale, float c, float* dh, bf16* dlow,
                       void* part, size_t part_bytes, hipStream_t s) {
  MACRO_SIZES("macro_epilogue_bwd");
  RTE_REQUIRE(Bh >= 1 && B % Bh == 0, "macro_epilogue_bwd: the h batch must divide the batch");
  RTE_REQUIRE(al16m(dout) && al16m(h) && al16m(low) && al16m(gain) && al16m(bias) && al16m(scale) && al16m(dh) &&
                  al16m(dlow),
              "macro_epilogue_bwd: 16-byte aligned buffers");
  if (B == 0) return 0;
  RTE_REQUIRE(part && part_bytes >= macro_workspace_bytes(B, S, d), "macro_epilogue_bwd: part buffer too small");
  const int P = macro_parts(B, S);
  const size_t lds = (size_t)kMacroWaves * d * sizeof(float);
  MACRO_LAUNCH(macro_epilogue_bwd_kernel, lds, dout, h, low, key, Bh, S, P, d, gain, bias, scale, c, dh, dlow,
               static_cast<float*>(part));
  return check_launch("macro_epilogue_bwd");
}

int macro_table_grad(const int64_t* key, int B, int S, int G, int d, const void* part, float* dgain, float* dbias,
                     float* dscale, hipStream_t s) {
  RTE_REQUIRE(B >= 0 && B <= 16384 && S >= 1 && G >= 1 && G <= 65535 && d >= 1 && d <= 1024,
              "macro_table_grad: need B <= 16384, n_keys <= 65535, d <= 1024");
  if (!dgain && !dbias && !dscale) return 0;
  const int P = B > 0 ? macro_parts(B, S) : 1;
  const dim3 grid((unsigned)G, (unsigned)((3 * d + 63) / 64));
  hipLaunchKernelGGL(macro_table_grad_kernel, grid, dim3(256), (size_t)(B > 0 ? B : 1) * sizeof(int), s, key, B, P, d,
                     static_cast<const float*>(part), dgain, dbias, dscale);
  return check_launch("macro_table_grad");
}

// As macro_table_grad with the number of part rows per sample given (part [B][P][3d]).
int macro_table_grad_parts(const int64_t* key, int B, int P, int G, int d, const void* part, float* dgain,
                           float* dbias, float* dscale, hipStream_t s) {
  RTE_REQUIRE(B >= 0 && B <= 16384 && P >= 1 && G >= 1 && G <= 65535 && d >= 1 && d <= 1024,
              "macro_table_grad: need B <= 16384, n_keys <= 65535, d <= 1024");
  if (!dgain && !dbias && !dscale) return 0;
  const dim3 grid((unsigned)G, (unsigned)((3 * d + 63) / 64));
  hipLaunchKernelGGL(macro_table_grad_kernel, grid, dim3(256), (size_t)(B > 0 ? B : 1) * sizeof(int), s, key, B, P, d,
                     static_cast<const float*>(part), dgain, dbias, dscale);
  return check_launch("macro_table_grad");
}

}  // namespace rte
