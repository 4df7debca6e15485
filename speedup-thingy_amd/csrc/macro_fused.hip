// Fused bounded-residual macro operator Phi (rte/macro.py:201-236, default options: no gate,
// no second hidden layer, no extra input parts) for hidden rank 32, forward and backward:
//
//   x2   = [rmsnorm(h) | h0]                       bf16, once per source row (stats kernel)
//   a    = x2 @ [V1; V3][key] + mean_s(rmsnorm(h)) @ V2[key]      V = [V1; V2; V3] by rows
//   low  = silu(a) @ U[key]
//   out  = h + c * scale[key] * tanh(gain[key] * h + low + bias[key])
//
// z = [rmsnorm(h) | mean_s rmsnorm(h) | h0] of the reference is never formed: its middle block
// is the same vector for every row of a sample, so z @ V splits into the row part x2 @ [V1; V3]
// and one [rank] vector per sample (pooled @ V2).  One workgroup owns 64 rows of one sample, so
// every matrix it multiplies by belongs to a single (recipe, stride) key: the rank-32 products
// run as v_mfma_f32_32x32x16_bf16 straight from global memory (x2 rows, the key's weights) and
// from LDS (silu(a), du), and nothing of width 3d or d is written besides the outputs.
//
// Backward, per call:
//   bwd_a   (one workgroup per 64 rows of one sample): recomputes low, du = dout c scale (1-t^2)
//           (bf16 to HBM for the dU reduction), the table-gradient column sums of the tile, and
//           dsa = du @ U^T -> da = dsa silu'(a) (bf16) with its per-tile column sums.
//   bwd_b   (one workgroup per 64 rows of one source sample, all its repeats): dnormed =
//           da @ V1^T + (sum_s da) @ V2^T / S, the rmsnorm backward, dh0 = da @ V3^T, plus the
//           epilogue term dout + du gain recomputed from low; the repeats are added in repeat
//           order in registers.
//   wgrad   dU and [dV1; dV3] as grouped-K MFMA GEMMs over the rows of each key (chunked,
//           summed in a fixed order), dV2 and the table gradients as fixed-order sums over the
//           key's samples.  Two calls (the consistency loss's two operator applications) can
//           share one wgrad pass: their rows are listed together.
//
// Repeated sources as in the unfused operator: sample b reads h row block b % Bh and h0 row
// block b % Bh0 (Bh0 | Bh | B, B / Bh <= 8).  No float atomics: every sum has a fixed order.
//
// MFMA lane layout (32x32x16): lane l supplies A row l % 32 and B column l % 32 with k values
// 8 (l / 32) .. +7 of each 16-step; output register r of lane l holds row 8 (r / 4) + 4 (l / 32)
// + r % 4, column l % 32.
#include "common.hpp"
#include "gemm.hpp"

extern "C" int rte_grouped_linear_bwd(const void* dy, const void* x, int N, int K, const int32_t* offsets, int G,
                                      int P, const int32_t* row_of_slot, const int32_t* out_row_of_slot,
                                      const void* w, int Nout, void* dx, int dx_f32, float* dw, void* workspace,
                                      size_t workspace_bytes, void* stream);
extern "C" size_t rte_grouped_linear_bwd_workspace_bytes(int P, int G, int K, int Nout);

namespace rte {

int macro_table_grad_parts(const int64_t* key, int B, int P, int G, int d, const void* part, float* dgain,
                           float* dbias, float* dscale, hipStream_t s);

namespace {

constexpr int kRank = 32;          // hidden width of the operator
constexpr int kTile = 32;          // rows per workgroup of the operator kernels
constexpr int kStatRows = 16;      // rows per workgroup of the statistics kernel
constexpr int kPitch = kRank + 8;  // LDS row pitch (bf16) of a [64][32] operand tile: 80 bytes
constexpr int kMaxRepeats = 8;

__device__ __forceinline__ f32x16_v mfma16(bf16x8_v a, bf16x8_v b, f32x16_v c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ bf16x8_v ld8b(const bf16* p) { return *reinterpret_cast<const bf16x8_v*>(p); }

__device__ __forceinline__ int acc_row(int r, int lane) { return 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3); }

// row of accumulator register r clamped into the tile's valid rows: loads stay in bounds and
// are issued unconditionally (all 16 in flight at once); results of rows past the tile are
// dropped at the stores
__device__ __forceinline__ int acc_row_ld(int r, int lane, int rb, int nrow) {
  const int row = rb * 32 + acc_row(r, lane);
  return row < nrow ? row : nrow - 1;
}

__device__ __forceinline__ f32x16_v zero16() {
  f32x16_v z;
#pragma unroll
  for (int i = 0; i < 16; ++i) z[i] = 0.0f;
  return z;
}

// tanh in fp32: odd Taylor polynomial below 0.25 (truncation < 4e-9), else
// 1 - 2 / (e^(2|x|) + 1) with the sign of x; about 2e-7 relative error.
__device__ __forceinline__ float tanh_fast(float x) {
  const float a = fabsf(x);
  if (a < 0.25f) {
    const float x2 = x * x;
    return x + x * x2 * (-0.333333333f + x2 * (0.133333333f + x2 * (-0.0539682540f + x2 * 0.0218694885f)));
  }
  const float e = __expf(2.0f * a);
  return copysignf(1.0f - 2.0f * __builtin_amdgcn_rcpf(e + 1.0f), x);
}

__device__ __forceinline__ float sigmoid_fast(float x) { return 1.0f / (1.0f + __expf(-x)); }

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

// sum over the 32 lanes that share lane / 32
__device__ __forceinline__ float half_sum(float v) {
#pragma unroll
  for (int off = 16; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

__device__ __forceinline__ void ld8f(const float* p, float* v) {
  const float4 a = *reinterpret_cast<const float4*>(p);
  const float4 b = *reinterpret_cast<const float4*>(p + 4);
  v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
  v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
}

__device__ __forceinline__ void st8f(float* p, const float* v) {
  *reinterpret_cast<float4*>(p) = make_float4(v[0], v[1], v[2], v[3]);
  *reinterpret_cast<float4*>(p + 4) = make_float4(v[4], v[5], v[6], v[7]);
}

__device__ __forceinline__ void st8b(bf16* p, const float* v) {
  uint4 o;
  o.x = pack_bf2(v[0], v[1]);
  o.y = pack_bf2(v[2], v[3]);
  o.z = pack_bf2(v[4], v[5]);
  o.w = pack_bf2(v[6], v[7]);
  *reinterpret_cast<uint4*>(p) = o;
}

__device__ __forceinline__ int64_t clamp_key(int64_t k, int G) { return k < 0 ? 0 : (k >= G ? G - 1 : k); }

// Upstream gradient of the operator's output, per sample b: coef (p - q) row block b - diff_lo
// of two saved tensors when b lies in [diff_lo, diff_lo + n_diff) (the MSE of the consistency
// loss, coef = mul * g[0] read on the device), plus buf row block b - buf_lo when b lies in
// [buf_lo, buf_lo + n_buf); 0 for a sample in neither range.  The ranges may overlap (an
// operator application shared by both roles of the consistency loss).
struct DoutDesc {
  const float* p;
  const float* q;
  const float* g;
  float mul;
  int diff_lo, n_diff;
  const float* buf;
  int buf_lo, n_buf;
};

// The upstream gradient rows of sample b from row s0 on
struct DoutRows {
  const float* p;
  const float* q;
  const float* buf;
  bool diff, has_buf;
};

__device__ __forceinline__ DoutRows dout_rows(const DoutDesc& dd, int64_t b, int64_t sd, int64_t start) {
  DoutRows r;
  r.diff = b >= dd.diff_lo && b < dd.diff_lo + dd.n_diff;
  r.has_buf = b >= dd.buf_lo && b < dd.buf_lo + dd.n_buf;
  r.p = r.diff ? dd.p + (b - dd.diff_lo) * sd + start : nullptr;
  r.q = r.diff ? dd.q + (b - dd.diff_lo) * sd + start : nullptr;
  r.buf = r.has_buf ? dd.buf + (b - dd.buf_lo) * sd + start : nullptr;
  return r;
}

// base[off] with a 32-bit byte offset (offsets inside one sample's row block), so the load can
// take the uniform base in scalar registers
__device__ __forceinline__ float ldf(const float* base, uint32_t off) {
  return *reinterpret_cast<const float*>(reinterpret_cast<const char*>(base) + (off << 2));
}

// The upstream gradient at the 16 offsets: every load of the branch is issued before any is
// used (one memory round trip; a select over a conditional load would wait per row).
__device__ __forceinline__ void dout16(const DoutRows& gr, float coef, const uint32_t* off, float* gv) {
  if (gr.diff && gr.has_buf) {
    float a[16], b[16], e[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      a[r] = ldf(gr.p, off[r]);
      b[r] = ldf(gr.q, off[r]);
      e[r] = ldf(gr.buf, off[r]);
    }
#pragma unroll
    for (int r = 0; r < 16; ++r) gv[r] = coef * (a[r] - b[r]) + e[r];
  } else if (gr.diff) {
    float a[16], b[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      a[r] = ldf(gr.p, off[r]);
      b[r] = ldf(gr.q, off[r]);
    }
#pragma unroll
    for (int r = 0; r < 16; ++r) gv[r] = coef * (a[r] - b[r]);
  } else if (gr.has_buf) {
#pragma unroll
    for (int r = 0; r < 16; ++r) gv[r] = ldf(gr.buf, off[r]);
  } else {
#pragma unroll
    for (int r = 0; r < 16; ++r) gv[r] = 0.0f;
  }
}

__device__ __forceinline__ float dout_coef(const DoutDesc& dd) { return dd.n_diff > 0 ? dd.mul * (dd.g ? dd.g[0] : 1.0f) : 0.0f; }

// ------------------------------------------------------------------ weights

// bf16 copies of V [G][3d][32] and U [G][32][d] in the layouts the kernels read: Vb (same
// layout), VcT [G][32][2d] (V1 and V3 transposed), V2T [G][32][d], Ub (same), UT [G][d][32].
// Block i < G * 3d / 32: a 32-row slice of V; else a 32-column slice of U.
__global__ void __launch_bounds__(256) mf_prep_kernel(const float* __restrict__ V, const float* __restrict__ U, int G,
                                                      int d, bf16* __restrict__ Vb, bf16* __restrict__ VcT,
                                                      bf16* __restrict__ V2T, bf16* __restrict__ Ub,
                                                      bf16* __restrict__ UT) {
  __shared__ float t[32][33];
  const int nv = 3 * d / 32, nu = d / 32;
  const int tid = threadIdx.x;
  int blk = blockIdx.x;
  if (blk < G * nv) {
    const int g = blk / nv, k0 = (blk % nv) * 32;
    const int64_t base = ((int64_t)g * 3 * d + k0) * kRank;
    for (int e = tid; e < 1024; e += 256) {
      const float v = V[base + e];
      Vb[base + e] = f2bf(v);
      t[e >> 5][e & 31] = v;
    }
    __syncthreads();
    const bool mid = k0 >= d && k0 < 2 * d;
    bf16* dst = mid ? V2T + (int64_t)g * kRank * d + (k0 - d) : VcT + (int64_t)g * kRank * 2 * d + (k0 < d ? k0 : k0 - d);
    const int ld = mid ? d : 2 * d;
    for (int e = tid; e < 1024; e += 256) {
      const int n = e >> 5, kk = e & 31;
      dst[(int64_t)n * ld + kk] = f2bf(t[kk][n]);
    }
  } else {
    blk -= G * nv;
    const int g = blk / nu, c0 = (blk % nu) * 32;
    for (int e = tid; e < 1024; e += 256) {
      const int n = e >> 5, cc = e & 31;
      const int64_t i = ((int64_t)g * kRank + n) * d + c0 + cc;
      const float v = U[i];
      Ub[i] = f2bf(v);
      t[n][cc] = v;
    }
    __syncthreads();
    for (int e = tid; e < 1024; e += 256) {
      const int cc = e >> 5, n = e & 31;
      UT[((int64_t)g * d + c0 + cc) * kRank + n] = f2bf(t[n][cc]);
    }
  }
}

// ------------------------------------------------------------------ forward

// Rows [16 blockIdx.x, +16) of source sample blockIdx.y (wave w: 4 consecutive rows, loads of
// all four issued first): rstd, x2 = [bf16(h rstd) | bf16(h0)] and the chunk's column sums of
// h rstd (waves in order) into ppart[src][chunk].
template <int NCH>
__global__ void __launch_bounds__(256) mf_stats_kernel(const float* __restrict__ h, const float* __restrict__ h0,
                                                       int Bh0, int S, int d, float eps, bf16* __restrict__ x2,
                                                       float* __restrict__ rstd, float* __restrict__ ppart) {
  __shared__ float red[4][1024];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int src = blockIdx.y, chunk = blockIdx.x, nchunk = gridDim.x;
  const int nch = d / 8;
  const int64_t hb = (int64_t)src * S, h0b = (int64_t)(src % Bh0) * S;
  float x[4][NCH][8], o[4][NCH][8];
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    int s = chunk * kStatRows + wave * 4 + q;
    s = s < S ? s : S - 1;
#pragma unroll
    for (int j = 0; j < NCH; ++j) {
      const int ch = lane + 64 * j;
      if (ch >= nch) continue;
      ld8f(h + (hb + s) * d + ch * 8, x[q][j]);
      ld8f(h0 + (h0b + s) * d + ch * 8, o[q][j]);
    }
  }
  float pool[NCH][8];
#pragma unroll
  for (int j = 0; j < NCH; ++j)
#pragma unroll
    for (int i = 0; i < 8; ++i) pool[j][i] = 0.0f;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int s = chunk * kStatRows + wave * 4 + q;
    float ss = 0.0f;
#pragma unroll
    for (int j = 0; j < NCH; ++j) {
      if (lane + 64 * j >= nch) continue;
#pragma unroll
      for (int i = 0; i < 8; ++i) ss += x[q][j][i] * x[q][j][i];
    }
    ss = wave_sum(ss);
    if (s >= S) continue;
    const float rr = rsqrtf(ss / (float)d + eps);
    if (lane == 0) rstd[hb + s] = rr;
    bf16* xr = x2 + (hb + s) * 2 * d;
#pragma unroll
    for (int j = 0; j < NCH; ++j) {
      const int ch = lane + 64 * j;
      if (ch >= nch) continue;
      float y[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        y[i] = x[q][j][i] * rr;
        pool[j][i] += y[i];
      }
      st8b(xr + ch * 8, y);
      st8b(xr + d + ch * 8, o[q][j]);
    }
  }
#pragma unroll
  for (int j = 0; j < NCH; ++j) {
    const int ch = lane + 64 * j;
    if (ch < nch) st8f(&red[wave][ch * 8], pool[j]);
  }
  __syncthreads();
  for (int col = threadIdx.x; col < d; col += 256)
    ppart[((int64_t)src * nchunk + chunk) * d + col] = ((red[0][col] + red[1][col]) + red[2][col]) + red[3][col];
}

// Per source sample: pooled = bf16(sum of the chunk sums in chunk order / S), and for each
// repeat b = src + t Bh the rank vector P[b] = pooled @ V2[key[b]] (thread: 8 columns, rows
// grp, grp + 64, ...; the 64 row-group partials added in group order).
__global__ void __launch_bounds__(256) mf_pool_kernel(const float* __restrict__ ppart, int nchunk, int S, int d,
                                                      const int64_t* __restrict__ key, int G, int Bh, int rep,
                                                      const bf16* __restrict__ Vb, bf16* __restrict__ pooled,
                                                      float* __restrict__ P) {
  __shared__ float pm[1024];
  __shared__ float red[64][kRank];
  const int src = blockIdx.x, tid = threadIdx.x;
  const float invS = 1.0f / (float)S;
  for (int col = tid; col < d; col += 256) {
    float s = 0.0f;
    for (int q = 0; q < nchunk; ++q) s += ppart[((int64_t)src * nchunk + q) * d + col];
    const bf16 pb = f2bf(s * invS);
    pooled[(int64_t)src * d + col] = pb;
    pm[col] = bf2f(pb);
  }
  __syncthreads();
  const int n8 = tid & 3, grp = tid >> 2;
  for (int t = 0; t < rep; ++t) {
    const int64_t b = src + (int64_t)t * Bh;
    const int64_t k = clamp_key(key[b], G);
    const bf16* v2 = Vb + (k * 3 * d + d) * kRank + n8 * 8;
    float acc[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) acc[i] = 0.0f;
    for (int j0 = grp; j0 < d; j0 += 256) {
      uint4 u[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) {  // rows past d re-read row d - 1 with weight 0
        const int j = j0 + 64 * q < d ? j0 + 64 * q : d - 1;
        u[q] = *reinterpret_cast<const uint4*>(v2 + (int64_t)j * kRank);
      }
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const float pj = j0 + 64 * q < d ? pm[j0 + 64 * q] : 0.0f;
        const uint32_t w[4] = {u[q].x, u[q].y, u[q].z, u[q].w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          acc[2 * i] += pj * __uint_as_float(w[i] << 16);
          acc[2 * i + 1] += pj * __uint_as_float(w[i] & 0xffff0000u);
        }
      }
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) red[grp][n8 * 8 + i] = acc[i];
    __syncthreads();
    if (tid < kRank) {
      float s = 0.0f;
      for (int q = 0; q < 64; ++q) s += red[q][tid];
      P[b * kRank + tid] = s;
    }
    __syncthreads();
  }
}

// Tile blockIdx.x (32 rows) of sample blockIdx.y: a (fp32, saved), silu(a) (bf16, saved), out;
// with a reference tensor, the tile's sum of (out - ref)^2 (waves in order).  Wave w computes the
// quarter w of the 2d-long products, the four partials are added in wave order.
template <bool MSE>
__global__ void __launch_bounds__(256) mf_fwd_kernel(const bf16* __restrict__ x2, const float* __restrict__ h, int Bh,
                                                     int S, int d, const int64_t* __restrict__ key, int G,
                                                     const bf16* __restrict__ VcT, const float* __restrict__ P,
                                                     const bf16* __restrict__ UT, const float* __restrict__ gain,
                                                     const float* __restrict__ bias, const float* __restrict__ scale,
                                                     float c, float* __restrict__ a_out, bf16* __restrict__ sa_out,
                                                     float* __restrict__ out, const float* __restrict__ mse_ref,
                                                     float* __restrict__ mse_part) {
  __shared__ float apart[4][kTile][kRank + 1];
  __shared__ __align__(16) bf16 sal[kTile][kPitch];
  __shared__ float mred[4];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, tid = threadIdx.x;
  const int tile = blockIdx.x, T = gridDim.x;
  const int64_t b = blockIdx.y;
  const int64_t src = b % Bh;
  const int64_t k = clamp_key(key[b], G);
  const int s0 = tile * kTile, nrow = min(kTile, S - s0);
  {
    int rl = lane & 31;
    if (rl >= nrow) rl = nrow - 1;  // rows past the sample re-read its last row; never stored
    const int kq = wave * (d / 2);
    const bf16* ap = x2 + (src * S + s0 + rl) * 2 * d + kq + 8 * (lane >> 5);
    const bf16* bp = VcT + (k * kRank + (lane & 31)) * 2 * d + kq + 8 * (lane >> 5);
    f32x16_v acc = zero16();
    for (int kk = 0; kk < d / 2; kk += 64) {
      bf16x8_v af[4], bfr[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        af[u] = ld8b(ap + kk + 16 * u);
        bfr[u] = ld8b(bp + kk + 16 * u);
      }
#pragma unroll
      for (int u = 0; u < 4; ++u) acc = mfma16(af[u], bfr[u], acc);
    }
#pragma unroll
    for (int r = 0; r < 16; ++r) apart[wave][acc_row(r, lane)][lane & 31] = acc[r];
  }
  __syncthreads();
  for (int e = tid; e < kTile * kRank; e += 256) {
    const int row = e >> 5, n = e & 31;
    const float av = (((apart[0][row][n] + apart[1][row][n]) + apart[2][row][n]) + apart[3][row][n]) + P[b * kRank + n];
    const bf16 sb = f2bf(av * sigmoid_fast(av));
    sal[row][n] = sb;
    if (row < nrow) {
      const int64_t gr = b * S + s0 + row;
      a_out[gr * kRank + n] = av;
      sa_out[gr * kRank + n] = sb;
    }
  }
  __syncthreads();
  float msum = 0.0f;
  const float* hs = h + (src * S + s0) * (int64_t)d;
  float* ob = out + (b * S + s0) * (int64_t)d;
  const float* rf = MSE ? mse_ref + (b * S + s0) * (int64_t)d : nullptr;
  const float* gk = gain + k * d;
  const float* bk = bias + k * d;
  const float* sk = scale + k * d;
  const bf16* lp = &sal[lane & 31][8 * (lane >> 5)];
  const bf16x8_v s0v = ld8b(lp), s1v = ld8b(lp + 16);
  for (int cb = wave; cb < d / 32; cb += 4) {
    const int col = cb * 32 + (lane & 31);
    const bf16* up = UT + (k * d + col) * kRank + 8 * (lane >> 5);
    const float gn = gk[col], bs = bk[col], sc = sk[col];
    float xv[16], rv[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int oi = acc_row_ld(r, lane, 0, nrow) * d + col;
      xv[r] = hs[oi];
      if (MSE) rv[r] = rf[oi];
    }
    f32x16_v acc = zero16();
    acc = mfma16(s0v, ld8b(up), acc);
    acc = mfma16(s1v, ld8b(up + 16), acc);
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int row = acc_row(r, lane);
      if (row < nrow) {
        const float o = xv[r] + c * sc * tanh_fast(gn * xv[r] + acc[r] + bs);
        ob[row * d + col] = o;
        if (MSE) {
          const float df = o - rv[r];
          msum += df * df;
        }
      }
    }
  }
  if (MSE) {
    msum = wave_sum(msum);
    if (lane == 0) mred[wave] = msum;
    __syncthreads();
    if (tid == 0) mse_part[b * T + tile] = ((mred[0] + mred[1]) + mred[2]) + mred[3];
  }
}

// out[0] = (sum of part[0, n) in a fixed order) * inv_n
__global__ void __launch_bounds__(256) mf_sum_kernel(const float* __restrict__ part, int n, float inv_n,
                                                     float* __restrict__ out) {
  __shared__ float red[4];
  float s = 0.0f;
  for (int i = threadIdx.x; i < n; i += 256) s += part[i];
  s = wave_sum(s);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = s;
  __syncthreads();
  if (threadIdx.x == 0) out[0] = (((red[0] + red[1]) + red[2]) + red[3]) * inv_n;
}

// ------------------------------------------------------------------ backward

// Tile blockIdx.x (32 rows) of sample blockIdx.y:
//   du (bf16), table column sums part_tab[b][tile][3][d] = (du h | du | dout c tanh),
//   da = (du @ U^T) silu'(a) (bf16) and its column sums part_da[b][tile],
//   rd[row]  = <da @ V1^T, h_row> = da_row . (x2[:, :d] @ V1) / rstd   (the row-local part of the
//              rmsnorm dot, from the bf16 normalised rows as the pooled part below)
//   xv2[row] = h_row @ V2 = (x2[:, :d] @ V2) / rstd   (the pooled part's per-row factor)
__global__ void __launch_bounds__(256) mf_bwd_a_kernel(DoutDesc dd, const float* __restrict__ h,
                                                       const float* __restrict__ rstd, const bf16* __restrict__ x2,
                                                       int Bh, int S, int d, const int64_t* __restrict__ key, int G,
                                                       const float* __restrict__ a_buf, const bf16* __restrict__ VcT,
                                                       const bf16* __restrict__ V2T, const bf16* __restrict__ UT,
                                                       const bf16* __restrict__ Ub, const float* __restrict__ gain,
                                                       const float* __restrict__ bias, const float* __restrict__ scale,
                                                       float c, bf16* __restrict__ du_buf, bf16* __restrict__ da_buf,
                                                       float* __restrict__ part_tab, float* __restrict__ part_da,
                                                       float* __restrict__ rd_out, float* __restrict__ xv2_out) {
  __shared__ float al[kTile][kRank + 1];
  __shared__ __align__(16) bf16 sal[kTile][kPitch];
  __shared__ __align__(16) bf16 dul[4][kTile][kPitch];
  __shared__ float red[4][kTile][kRank + 1];
  __shared__ float rdw[4][kTile];
  __shared__ float rs[kTile];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, tid = threadIdx.x;
  const int tile = blockIdx.x, T = gridDim.x;
  const int64_t b = blockIdx.y;
  const int64_t src = b % Bh;
  const int64_t k = clamp_key(key[b], G);
  const int s0 = tile * kTile, nrow = min(kTile, S - s0);
  const int64_t sd = (int64_t)S * d;
  const float coef = dout_coef(dd);
  const DoutRows gr = dout_rows(dd, b, sd, (int64_t)s0 * d);
  const float* hs = h + src * sd + (int64_t)s0 * d;
  bf16* dub = du_buf + b * sd + (int64_t)s0 * d;
  for (int e = tid; e < kTile * kRank; e += 256) {
    const int row = e >> 5, n = e & 31;
    const float av = row < nrow ? a_buf[(b * S + s0 + row) * kRank + n] : 0.0f;
    al[row][n] = av;
    sal[row][n] = f2bf(av * sigmoid_fast(av));
  }
  if (tid < kTile) rs[tid] = tid < nrow ? rstd[src * S + s0 + tid] : 0.0f;
  __syncthreads();
  f32x16_v dsa = zero16();
  const float* gk = gain + k * d;
  const float* bk = bias + k * d;
  const float* sk = scale + k * d;
  {
    const bf16* lp = &sal[lane & 31][8 * (lane >> 5)];
    const bf16x8_v s0v = ld8b(lp), s1v = ld8b(lp + 16);
    for (int cb = wave; cb < d / 32; cb += 4) {
      const int col = cb * 32 + (lane & 31);
      const bf16* up = UT + (k * d + col) * kRank + 8 * (lane >> 5);
      const bf16* ubp = Ub + (k * kRank + (lane & 31)) * d + cb * 32 + 8 * (lane >> 5);
      const float gn = gk[col], bs = bk[col], sc = sk[col];
      float xv[16], gv[16];
      uint32_t off[16];
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        off[r] = (uint32_t)(acc_row_ld(r, lane, 0, nrow) * d + col);
        xv[r] = ldf(hs, off[r]);
      }
      dout16(gr, coef, off, gv);
      f32x16_v acc = zero16();
      acc = mfma16(s0v, ld8b(up), acc);
      acc = mfma16(s1v, ld8b(up + 16), acc);
      float pg = 0.0f, pb = 0.0f, ps = 0.0f;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int row = acc_row(r, lane);
        float du = 0.0f;
        if (row < nrow) {
          const float tt = tanh_fast(gn * xv[r] + acc[r] + bs);
          du = gv[r] * c * sc * (1.0f - tt * tt);
          dub[row * d + col] = f2bf(du);
          pg += du * xv[r];
          pb += du;
          ps += gv[r] * c * tt;
        }
        dul[wave][row][lane & 31] = f2bf(du);
      }
      pg += __shfl_xor(pg, 32, 64);
      pb += __shfl_xor(pb, 32, 64);
      ps += __shfl_xor(ps, 32, 64);
      if (lane < 32) {
        float* pt = part_tab + ((b * T + tile) * 3) * d + col;
        pt[0] = pg;
        pt[d] = pb;
        pt[2 * d] = ps;
      }
      wave_lds_sync();
      const bf16* dp = &dul[wave][lane & 31][8 * (lane >> 5)];
      dsa = mfma16(ld8b(dp), ld8b(ubp), dsa);
      dsa = mfma16(ld8b(dp + 16), ld8b(ubp + 16), dsa);
      wave_lds_sync();  // the next column block overwrites this wave's du block
    }
  }
#pragma unroll
  for (int r = 0; r < 16; ++r) red[wave][acc_row(r, lane)][lane & 31] = dsa[r];
  __syncthreads();
  for (int e = tid; e < kTile * kRank; e += 256) {
    const int row = e >> 5, n = e & 31;
    const float v = ((red[0][row][n] + red[1][row][n]) + red[2][row][n]) + red[3][row][n];
    const float av = al[row][n];
    const float sg = sigmoid_fast(av);
    const float dav = row < nrow ? v * sg * (1.0f + av * (1.0f - sg)) : 0.0f;
    const bf16 db = f2bf(dav);
    if (row < nrow) da_buf[(b * S + s0 + row) * kRank + n] = db;
    al[row][n] = dav;  // only this thread reads or writes element (row, n) here
  }
  __syncthreads();
  if (tid < kRank) {  // column sums of da over the tile's rows, in row order
    float s = 0.0f;
    for (int row = 0; row < kTile; ++row) s += al[row][tid];
    part_da[(b * T + tile) * kRank + tid] = s;
  }
  // xv2 = x2[:, :d] @ V2 and xv1 = x2[:, :d] @ V1 (wave w: quarter w of the d-long products);
  // the wave's rd part is da_row . xv1 over its quarter (the 4 quarters are added in order)
  {
    int rl = lane & 31;
    if (rl >= nrow) rl = nrow - 1;
    const int kq = wave * (d / 4);
    const bf16* ap = x2 + (src * S + s0 + rl) * 2 * d + kq + 8 * (lane >> 5);
    const bf16* bp = V2T + (k * kRank + (lane & 31)) * d + kq + 8 * (lane >> 5);
    const bf16* cp = VcT + (k * kRank + (lane & 31)) * 2 * d + kq + 8 * (lane >> 5);
    {  // one accumulator at a time (register budget)
      f32x16_v acc1 = zero16();
      for (int kk = 0; kk < d / 4; kk += 32) {
        acc1 = mfma16(ld8b(ap + kk), ld8b(cp + kk), acc1);
        acc1 = mfma16(ld8b(ap + kk + 16), ld8b(cp + kk + 16), acc1);
      }
#pragma unroll
      for (int r = 0; r < 16; ++r) {  // rows past the tile have da = 0
        const float v = half_sum(acc1[r] * al[acc_row(r, lane)][lane & 31]);
        if ((lane & 31) == 0) rdw[wave][acc_row(r, lane)] = v;
      }
    }
    f32x16_v acc = zero16();
    for (int kk = 0; kk < d / 4; kk += 32) {
      const bf16x8_v a0 = ld8b(ap + kk), a1 = ld8b(ap + kk + 16);
      const bf16x8_v b0 = ld8b(bp + kk), b1 = ld8b(bp + kk + 16);
      acc = mfma16(a0, b0, acc);
      acc = mfma16(a1, b1, acc);
    }
    __syncthreads();  // every wave is done with red
#pragma unroll
    for (int r = 0; r < 16; ++r) red[wave][acc_row(r, lane)][lane & 31] = acc[r];
  }
  __syncthreads();
  for (int e = tid; e < kTile * kRank; e += 256) {
    const int row = e >> 5, n = e & 31;
    if (row >= nrow) continue;
    const float v = ((red[0][row][n] + red[1][row][n]) + red[2][row][n]) + red[3][row][n];
    xv2_out[(b * S + s0 + row) * kRank + n] = v / rs[row];
  }
  if (tid < nrow) rd_out[b * S + s0 + tid] = (((rdw[0][tid] + rdw[1][tid]) + rdw[2][tid]) + rdw[3][tid]) / rs[tid];
}

// LDS of mf_bwd_b_kernel for rep repeats
__host__ __device__ constexpr size_t bwd_b_lds(int rep) {
  return (size_t)rep * 2 * kTile * kPitch * sizeof(bf16)   // da, silu(a) tiles
         + (size_t)rep * 128 * sizeof(float)               // (sum_s da) @ V2^T / S, this block's columns
         + (size_t)rep * kTile * sizeof(float)             // rmsnorm coefficients
         + (size_t)rep * kRank * sizeof(float)             // sum_s da / S
         + (size_t)kTile * sizeof(float);                  // rstd
}

// Rows [32 blockIdx.x, +32) of source sample blockIdx.y, columns [128 blockIdx.z, +128) (one 32-
// column block per wave), all repeats b = src + t Bh (t < rep), added in repeat order:
//   dh  = sum_t [dout + du gain + rstd dn - h rstd^3 <dn, h> / d],
//         dn = da @ V1^T + (sum_s da) @ V2^T / S,  <dn, h> = rd + (sum_s da / S) . xv2
//   dh0 = sum_t da @ V3^T
// With dh0_into_dh (h and h0 are one tensor) dh0 is added to dh; `extra` adds n_extra further
// [Bh, S, d] blocks to dh (in block order).
template <bool INTO>
__global__ void __launch_bounds__(256, INTO ? 3 : 2) mf_bwd_b_kernel(DoutDesc dd, const float* __restrict__ h,
                                                       const float* __restrict__ rstd, int Bh, int rep, int S, int d,
                                                       const int64_t* __restrict__ key, int G,
                                                       const bf16* __restrict__ da_buf, const bf16* __restrict__ sa_buf,
                                                       const float* __restrict__ part_da, int T,
                                                       const float* __restrict__ rd, const float* __restrict__ xv2,
                                                       const bf16* __restrict__ Vb, const bf16* __restrict__ UT,
                                                       const float* __restrict__ gain, const float* __restrict__ bias,
                                                       const float* __restrict__ scale, float c, float* __restrict__ dh,
                                                       float* __restrict__ dh0,
                                                       const float* __restrict__ extra, int n_extra,
                                                       bf16* __restrict__ dsum_out) {
  extern __shared__ __align__(16) unsigned char smem[];
  bf16* dal = reinterpret_cast<bf16*>(smem);                                   // [rep][32][kPitch]
  bf16* sal = dal + (size_t)rep * kTile * kPitch;                              // [rep][32][kPitch]
  float* cs = reinterpret_cast<float*>(sal + (size_t)rep * kTile * kPitch);    // [rep][128]
  float* cf = cs + rep * 128;                                                  // [rep][32]
  float* dsum = cf + rep * kTile;                                              // [rep][32]
  float* rs = dsum + rep * kRank;                                              // [32]
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, tid = threadIdx.x;
  const int tile = blockIdx.x, c0 = blockIdx.z * 128;
  const int64_t src = blockIdx.y;
  const int s0 = tile * kTile, nrow = min(kTile, S - s0);
  const int64_t sd = (int64_t)S * d;
  const float coef = dout_coef(dd);
  const float invS = 1.0f / (float)S;
  const float* hs = h + src * sd + (int64_t)s0 * d;
  // da / silu(a) tiles of every repeat: 16-byte pieces (8 of the 32 rank values; rows past the
  // tile read the last valid row and store zeros)
  for (int e = tid; e < rep * kTile * 4; e += 256) {
    const int t = e / (kTile * 4), row = (e >> 2) & (kTile - 1), q = e & 3;
    const int64_t b = src + (int64_t)t * Bh;
    const int64_t g = (b * S + s0 + (row < nrow ? row : nrow - 1)) * kRank + 8 * q;
    uint4 dv = *reinterpret_cast<const uint4*>(da_buf + g);
    uint4 sv = *reinterpret_cast<const uint4*>(sa_buf + g);
    if (row >= nrow) dv = sv = make_uint4(0u, 0u, 0u, 0u);
    const size_t l = ((size_t)t * kTile + row) * kPitch + 8 * q;
    *reinterpret_cast<uint4*>(dal + l) = dv;
    *reinterpret_cast<uint4*>(sal + l) = sv;
  }
  for (int e = tid; e < rep * kRank; e += 256) {
    const int t = e >> 5, n = e & 31;
    const int64_t b = src + (int64_t)t * Bh;
    float s = 0.0f;
    for (int q = 0; q < T; ++q) s += part_da[(b * T + q) * kRank + n];
    dsum[e] = s * invS;
    if (blockIdx.x == 0 && blockIdx.z == 0) dsum_out[b * kRank + n] = f2bf(s);  // sum_s da for dV2
  }
  if (tid < kTile) rs[tid] = tid < nrow ? rstd[src * S + s0 + tid] : 0.0f;
  __syncthreads();
  for (int e = tid; e < rep * kTile; e += 256) {
    const int t = e / kTile, row = e - t * kTile;
    float v = 0.0f;
    if (row < nrow) {
      const int64_t gr = (src + (int64_t)t * Bh) * S + s0 + row;
      const float4* xp = reinterpret_cast<const float4*>(xv2 + gr * kRank);
      float s = 0.0f;
#pragma unroll
      for (int q = 0; q < kRank / 4; ++q) {
        const float4 w = xp[q];
        s += dsum[t * kRank + 4 * q] * w.x + dsum[t * kRank + 4 * q + 1] * w.y + dsum[t * kRank + 4 * q + 2] * w.z +
             dsum[t * kRank + 4 * q + 3] * w.w;
      }
      const float r = rs[row];
      v = r * r * r * (rd[gr] + s) / (float)d;
    }
    cf[e] = v;
  }
  for (int e = tid; e < rep * 128; e += 256) {
    const int t = e >> 7, cc = e & 127;
    float s = 0.0f;
    if (c0 + cc < d) {
      const int64_t k = clamp_key(key[src + (int64_t)t * Bh], G);
      const uint4* v2 = reinterpret_cast<const uint4*>(Vb + (k * 3 * d + d + c0 + cc) * kRank);
      uint4 u[4];
#pragma unroll
      for (int q = 0; q < 4; ++q) u[q] = v2[q];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const uint32_t w[4] = {u[q].x, u[q].y, u[q].z, u[q].w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          s += dsum[t * kRank + 8 * q + 2 * i] * __uint_as_float(w[i] << 16);
          s += dsum[t * kRank + 8 * q + 2 * i + 1] * __uint_as_float(w[i] & 0xffff0000u);
        }
      }
    }
    cs[e] = s;
  }
  __syncthreads();
  const int cl = wave * 32 + (lane & 31), col = c0 + cl;
  if (c0 + wave * 32 >= d) return;  // no barrier follows
  float x[16], ah[16], ah0[INTO ? 1 : 16];  // INTO: the h0 gradient goes straight into ah
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    x[r] = hs[acc_row_ld(r, lane, 0, nrow) * d + col];
    ah[r] = 0.0f;
    if constexpr (!INTO) ah0[r] = 0.0f;
  }
  for (int t = 0; t < rep; ++t) {
    const int64_t b = src + (int64_t)t * Bh;
    const int64_t k = clamp_key(key[b], G);
    const DoutRows gr = dout_rows(dd, b, sd, (int64_t)s0 * d);
    float gv[16];
    uint32_t off[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) off[r] = (uint32_t)(acc_row_ld(r, lane, 0, nrow) * d + col);
    dout16(gr, coef, off, gv);
    const bf16* vp = Vb + (k * 3 * d + col) * kRank + 8 * (lane >> 5);
    const bf16* wp = Vb + (k * 3 * d + 2 * d + col) * kRank + 8 * (lane >> 5);
    const bf16* up = UT + (k * d + col) * kRank + 8 * (lane >> 5);
    const bf16* lp = dal + ((size_t)t * kTile + (lane & 31)) * kPitch + 8 * (lane >> 5);
    const bf16* sp = sal + ((size_t)t * kTile + (lane & 31)) * kPitch + 8 * (lane >> 5);
    const bf16x8_v a0 = ld8b(lp), a1 = ld8b(lp + 16);
    const float gn = gain[k * d + col], bs = bias[k * d + col], sc = scale[k * d + col];
    const float cv = cs[t * 128 + cl];
    {
      f32x16_v lo = zero16();
      lo = mfma16(ld8b(sp), ld8b(up), lo);
      lo = mfma16(ld8b(sp + 16), ld8b(up + 16), lo);
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int row = acc_row(r, lane);
        const float tt = tanh_fast(gn * x[r] + lo[r] + bs);
        const float du = gv[r] * c * sc * (1.0f - tt * tt);
        ah[r] += gv[r] + du * gn - x[r] * cf[t * kTile + row];
      }
    }
    {
      f32x16_v dn = zero16();
      dn = mfma16(a0, ld8b(vp), dn);
      dn = mfma16(a1, ld8b(vp + 16), dn);
#pragma unroll
      for (int r = 0; r < 16; ++r) ah[r] += rs[acc_row(r, lane)] * (dn[r] + cv);
    }
    {
      f32x16_v dq = zero16();
      dq = mfma16(a0, ld8b(wp), dq);
      dq = mfma16(a1, ld8b(wp + 16), dq);
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        if constexpr (INTO) {
          ah[r] += dq[r];
        } else {
          ah0[r] += dq[r];
        }
      }
    }
  }
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int row = acc_row(r, lane);
    if (row >= nrow) continue;
    const int64_t off = src * sd + (int64_t)(s0 + row) * d + col;
    float v = ah[r];
    for (int e = 0; e < n_extra; ++e) v += extra[(int64_t)e * Bh * sd + off];
    dh[off] = v;
    if constexpr (!INTO) {
      if (dh0) dh0[off] = ah0[r];
    }
  }
}

// ------------------------------------------------------------------ weight gradients

// Rows of every key for the grouped reductions, over the samples of up to two calls (call 0:
// samples [0, B0) with x2 row blocks j % Bh0; call 1: samples [B0, B0 + B1) with x2 row blocks
// Bh0 + (j - B0) % Bh1; pooled rows likewise).  A key's samples keep increasing order (one
// wave per key: ballots over the samples in order).  Outputs: offsets / tok / pos in rows
// (tok: x2 row, pos: row of the per-sample buffers), soff / slist / psrc in samples (psrc: pooled
// row of the listed sample).
__global__ void __launch_bounds__(1024) mf_pack_kernel(const int64_t* __restrict__ key, int B0, int Bh0, int B1,
                                                       int Bh1, int S, int G, int32_t* __restrict__ offsets,
                                                       int32_t* __restrict__ tok, int32_t* __restrict__ pos,
                                                       int32_t* __restrict__ soff, int32_t* __restrict__ slist,
                                                       int32_t* __restrict__ psrc) {
  extern __shared__ int sm[];
  int* cnt = sm;                // [G]
  int* kl = sm + G;             // [B0 + B1]
  int* sl = kl + B0 + B1;       // [B0 + B1] slist
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, Bt = B0 + B1;
  for (int j = tid; j < Bt; j += 1024) kl[j] = (int)clamp_key(key[j], G);
  __syncthreads();
  for (int g = wave; g < G; g += 16) {
    int n = 0;
    for (int j0 = 0; j0 < Bt; j0 += 64) n += __popcll(__ballot(j0 + lane < Bt && kl[j0 + lane] == g));
    if (lane == 0) cnt[g] = n;
  }
  __syncthreads();
  if (tid == 0) {
    int s = 0;
    for (int g = 0; g < G; ++g) {
      const int n = cnt[g];
      soff[g] = s;
      offsets[g] = s * S;
      cnt[g] = s;
      s += n;
    }
    soff[G] = s;
    offsets[G] = s * S;
  }
  __syncthreads();
  for (int g = wave; g < G; g += 16) {
    int base = cnt[g];
    for (int j0 = 0; j0 < Bt; j0 += 64) {
      const int j = j0 + lane;
      const bool m = j < Bt && kl[j] == g;
      const unsigned long long bal = __ballot(m);
      if (m) {
        const int slot = base + __popcll(bal & ((1ull << lane) - 1ull));
        slist[slot] = j;
        sl[slot] = j;
        psrc[slot] = j < B0 ? j % Bh0 : Bh0 + (j - B0) % Bh1;
      }
      base += __popcll(bal);
    }
  }
  __syncthreads();
  for (int slot = wave; slot < Bt; slot += 16) {  // one wave per listed sample: S rows
    const int j = sl[slot];
    const int xr = (j < B0 ? j % Bh0 : Bh0 + (j - B0) % Bh1) * S;
    for (int s = lane; s < S; s += 64) {
      tok[slot * S + s] = xr + s;
      pos[slot * S + s] = j * S + s;
    }
  }
}

// The same lists for up to 256 keys and 4096 samples without per-key scans over all samples:
// each thread holds one sample's key, each wave ranks its 64 samples per key with one ballot per
// key, and a per-key prefix over the waves (in wave order) places them, so a key's samples keep
// ascending sample order (the lists are identical to mf_pack_kernel's).  Every workgroup builds
// the sample lists in its LDS (a few microseconds); workgroup 0 writes them, and the row lists
// (S rows per listed sample) are written by all workgroups, a slice of the slots each.
constexpr int kPackFastKeys = 256, kPackFastSamples = 4096;

__global__ void __launch_bounds__(1024) mf_pack_fast_kernel(const int64_t* __restrict__ key, int B0, int Bh0, int B1,
                                                            int Bh1, int S, int G, int32_t* __restrict__ offsets,
                                                            int32_t* __restrict__ tok, int32_t* __restrict__ pos,
                                                            int32_t* __restrict__ soff, int32_t* __restrict__ slist,
                                                            int32_t* __restrict__ psrc) {
  __shared__ int cw[16][kPackFastKeys];  // per wave, per key: counts, then slot bases
  __shared__ int run[kPackFastKeys];     // per key: totals, then the running slot base
  __shared__ int sl[kPackFastSamples];   // listed sample of each slot
  __shared__ int sp[kPackFastSamples];   // its source row block
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, Bt = B0 + B1;
  const unsigned long long lt = (1ull << lane) - 1ull;
  for (int g = tid; g < G; g += 1024) run[g] = 0;
  __syncthreads();
  for (int j0 = 0; j0 < Bt; j0 += 1024) {
    const int j = j0 + tid;
    const int k = j < Bt ? (int)clamp_key(key[j], G) : -1;
    for (int g = 0; g < G; ++g) {
      const unsigned long long m = __ballot(k == g);
      if (lane == 0 && m != 0ull) atomicAdd(&run[g], __popcll(m));  // integer totals: order-free
    }
  }
  __syncthreads();
  if (wave == 0) {  // exclusive scan of the per-key totals: lane l owns keys [4 l, 4 l + 4)
    int v[4], sum = 0;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int g = 4 * lane + q;
      v[q] = g < G ? run[g] : 0;
      sum += v[q];
    }
    int inc = sum;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const int y = __shfl_up(inc, off, 64);
      if (lane >= off) inc += y;
    }
    int s = inc - sum;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int g = 4 * lane + q;
      if (g < G) {
        if (blockIdx.x == 0) {
          soff[g] = s;
          offsets[g] = s * S;
        }
        run[g] = s;
      }
      s += v[q];
    }
    if (lane == 63 && blockIdx.x == 0) {
      soff[G] = s;
      offsets[G] = s * S;
    }
  }
  __syncthreads();
  for (int j0 = 0; j0 < Bt; j0 += 1024) {
    const int j = j0 + tid;
    const int k = j < Bt ? (int)clamp_key(key[j], G) : -1;
    int rank = 0;
    for (int g = 0; g < G; ++g) {
      const unsigned long long m = __ballot(k == g);
      if (k == g) rank = __popcll(m & lt);
      if (lane == 0) cw[wave][g] = __popcll(m);
    }
    __syncthreads();
    for (int g = tid; g < G; g += 1024) {
      int s = run[g];
      for (int w = 0; w < 16; ++w) {
        const int c = cw[w][g];
        cw[w][g] = s;
        s += c;
      }
      run[g] = s;
    }
    __syncthreads();
    if (k >= 0) {
      const int slot = cw[wave][k] + rank;
      const int src = j < B0 ? j % Bh0 : Bh0 + (j - B0) % Bh1;
      if (blockIdx.x == 0) {
        slist[slot] = j;
        psrc[slot] = src;
      }
      sl[slot] = j;
      sp[slot] = src;
    }
    __syncthreads();
  }
  // one wave per listed sample (S rows), four samples in flight per wave, the waves of all
  // workgroups striding over the slots
  const int gw = blockIdx.x * 16 + wave, nw = gridDim.x * 16;
  for (int slot0 = gw; slot0 < Bt; slot0 += 4 * nw) {
    int js[4], xs[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int slot = slot0 + nw * u;
      js[u] = slot < Bt ? sl[slot] : 0;
      xs[u] = slot < Bt ? sp[slot] * S : 0;
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int slot = slot0 + nw * u;
      if (slot < Bt) {
        for (int s = lane; s < S; s += 64) {
          tok[slot * S + s] = xs[u] + s;
          pos[slot * S + s] = js[u] * S + s;
        }
      }
    }
  }
}

// dV [G][3d][32] = [dVc[:, :d]; dV2; dVc[:, d:]]
__global__ void __launch_bounds__(256) mf_vassemble_kernel(const float4* __restrict__ dVc, const float4* __restrict__ dV2,
                                                           int G, int d, float4* __restrict__ dV) {
  const int64_t q = (int64_t)d * kRank / 4;  // float4s per d x 32 block
  const int64_t n = (int64_t)G * 3 * q;
  for (int64_t e = (int64_t)blockIdx.x * 256 + threadIdx.x; e < n; e += (int64_t)gridDim.x * 256) {
    const int64_t g = e / (3 * q), r = e - g * 3 * q;
    dV[e] = r < q ? dVc[g * 2 * q + r] : (r < 2 * q ? dV2[g * q + r - q] : dVc[g * 2 * q + r - q]);
  }
}

bool al16(const void* p) { return ((uintptr_t)p & 15) == 0; }

}  // namespace

// ------------------------------------------------------------------ host side

#define MF_SHAPES(what)                                                                                 \
  RTE_REQUIRE(d >= 128 && d % 128 == 0 && d <= 1024 && S >= 1 && S <= 65536 && G >= 1 && G <= 65535, \
              what ": need d % 128 == 0, d <= 1024, 1 <= S <= 65536, 1 <= n_keys <= 65535")

int macro_fused_tiles(int S) { return (S + kTile - 1) / kTile; }

static int stat_chunks(int S) { return (S + kStatRows - 1) / kStatRows; }

size_t macro_fused_fwd_workspace_bytes(int Bh, int S, int d) {
  return (size_t)(Bh > 0 ? Bh : 1) * stat_chunks(S > 0 ? S : 1) * (d > 0 ? d : 1) * sizeof(float);
}

int macro_fused_prep(const float* V, const float* U, int G, int d, bf16* Vb, bf16* VcT, bf16* V2T, bf16* Ub, bf16* UT,
                     hipStream_t s) {
  const int S = 1;
  MF_SHAPES("macro_fused_prep");
  RTE_REQUIRE(V && U && Vb && VcT && V2T && Ub && UT, "macro_fused_prep: null buffer");
  const int blocks = G * (3 * d / 32 + d / 32);
  hipLaunchKernelGGL(mf_prep_kernel, dim3(blocks), dim3(256), 0, s, V, U, G, d, Vb, VcT, V2T, Ub, UT);
  return check_launch("macro_fused_prep");
}

int macro_fused_fwd(const float* h, const float* h0, int Bh, int Bh0, const int64_t* key, int B, int S, int d, int G,
                    float eps, const bf16* Vb, const bf16* VcT, const bf16* UT, const float* gain, const float* bias,
                    const float* scale, float c, bf16* x2, float* rstd, bf16* pooled, float* P, float* a, bf16* sa,
                    float* out, const float* mse_ref, float* mse_part, void* ws, size_t ws_bytes, hipStream_t s) {
  MF_SHAPES("macro_fused_fwd");
  RTE_REQUIRE(Bh >= 1 && Bh0 >= 1 && Bh % Bh0 == 0 && B % Bh == 0 && B / Bh <= kMaxRepeats && B <= 65535,
              "macro_fused_fwd: need len(h0) | len(h) | len(key), at most 8 repeats, <= 65535 samples");
  RTE_REQUIRE(al16(h) && al16(h0) && al16(x2) && al16(Vb) && al16(VcT) && al16(UT) && al16(out),
              "macro_fused_fwd: 16-byte aligned buffers");
  RTE_REQUIRE(ws && ws_bytes >= macro_fused_fwd_workspace_bytes(Bh, S, d), "macro_fused_fwd: workspace too small");
  RTE_REQUIRE(!mse_ref || mse_part, "macro_fused_fwd: an MSE reference needs a partial-sum buffer");
  const int T = macro_fused_tiles(S), nchunk = stat_chunks(S);
  float* ppart = static_cast<float*>(ws);
  if (d <= 512)
    hipLaunchKernelGGL(mf_stats_kernel<1>, dim3(nchunk, Bh), dim3(256), 0, s, h, h0, Bh0, S, d, eps, x2, rstd, ppart);
  else
    hipLaunchKernelGGL(mf_stats_kernel<2>, dim3(nchunk, Bh), dim3(256), 0, s, h, h0, Bh0, S, d, eps, x2, rstd, ppart);
  RTE_TRY(check_launch("macro_fused_stats"));
  hipLaunchKernelGGL(mf_pool_kernel, dim3(Bh), dim3(256), 0, s, ppart, nchunk, S, d, key, G, Bh, B / Bh, Vb, pooled,
                     P);
  RTE_TRY(check_launch("macro_fused_pool"));
  if (mse_ref)
    hipLaunchKernelGGL(mf_fwd_kernel<true>, dim3(T, B), dim3(256), 0, s, x2, h, Bh, S, d, key, G, VcT, P, UT, gain,
                       bias, scale, c, a, sa, out, mse_ref, mse_part);
  else
    hipLaunchKernelGGL(mf_fwd_kernel<false>, dim3(T, B), dim3(256), 0, s, x2, h, Bh, S, d, key, G, VcT, P, UT, gain,
                       bias, scale, c, a, sa, out, nullptr, nullptr);
  return check_launch("macro_fused_fwd");
}

int macro_fused_sum(const float* part, int n, float inv_n, float* out, hipStream_t s) {
  RTE_REQUIRE(n >= 1 && part && out, "macro_fused_sum: need at least one partial sum");
  hipLaunchKernelGGL(mf_sum_kernel, dim3(1), dim3(256), 0, s, part, n, inv_n, out);
  return check_launch("macro_fused_sum");
}

size_t macro_fused_bwd_workspace_bytes(int B, int S) {
  return (size_t)(B > 0 ? B : 1) * (S > 0 ? S : 1) * (kRank + 1) * sizeof(float) + 256;
}

int macro_fused_bwd(const float* dp, const float* dq, const float* g, float mul, int diff_lo, int n_diff,
                    const float* dbuf, int buf_lo, int n_buf,
                    const float* h, const float* rstd, const bf16* x2, int Bh, const int64_t* key, int B, int S, int d,
                    int G, const float* a, const bf16* sa, const bf16* Vb, const bf16* VcT, const bf16* V2T,
                    const bf16* Ub, const bf16* UT, const float* gain, const float* bias, const float* scale, float c,
                    bf16* du,
                    bf16* da, float* part_tab, float* part_da, float* dh, float* dh0, int dh0_into_dh,
                    const float* extra, int n_extra, bf16* dsum, void* ws, size_t ws_bytes, hipStream_t s) {
  MF_SHAPES("macro_fused_bwd");
  RTE_REQUIRE(Bh >= 1 && B % Bh == 0 && B / Bh <= kMaxRepeats && B <= 65535,
              "macro_fused_bwd: need len(h) | len(key), at most 8 repeats");
  RTE_REQUIRE(diff_lo >= 0 && n_diff >= 0 && diff_lo + n_diff <= B && (n_diff == 0 || (dp && dq)) && buf_lo >= 0 &&
                  n_buf >= 0 && buf_lo + n_buf <= B && (n_buf == 0 || dbuf),
              "macro_fused_bwd: bad upstream-gradient description");
  RTE_REQUIRE(n_extra >= 0 && (n_extra == 0 || extra), "macro_fused_bwd: missing extra gradient blocks");
  RTE_REQUIRE(dh && dsum, "macro_fused_bwd: dh and dsum are required");
  RTE_REQUIRE(al16(da) && al16(sa), "macro_fused_bwd: da and silu(a) must be 16-byte aligned");
  RTE_REQUIRE(ws && ws_bytes >= macro_fused_bwd_workspace_bytes(B, S), "macro_fused_bwd: workspace too small");
  const int T = macro_fused_tiles(S), rep = B / Bh;
  float* xv2 = static_cast<float*>(ws);
  float* rd = xv2 + (size_t)B * S * kRank;
  DoutDesc dd{dp, dq, g, mul, diff_lo, n_diff, dbuf, buf_lo, n_buf};
  hipLaunchKernelGGL(mf_bwd_a_kernel, dim3(T, B), dim3(256), 0, s, dd, h, rstd, x2, Bh, S, d, key, G, a, VcT, V2T, UT,
                     Ub, gain, bias, scale, c, du, da, part_tab, part_da, rd, xv2);
  RTE_TRY(check_launch("macro_fused_bwd_a"));
  const size_t lds = bwd_b_lds(rep);
  if (dh0_into_dh)
    hipLaunchKernelGGL(mf_bwd_b_kernel<true>, dim3(T, Bh, d / 128), dim3(256), lds, s, dd, h, rstd, Bh, rep, S, d, key,
                       G, da, sa, part_da, T, rd, xv2, Vb, UT, gain, bias, scale, c, dh, dh0, extra, n_extra, dsum);
  else
    hipLaunchKernelGGL(mf_bwd_b_kernel<false>, dim3(T, Bh, d / 128), dim3(256), lds, s, dd, h, rstd, Bh, rep, S, d,
                       key, G, da, sa, part_da, T, rd, xv2, Vb, UT, gain, bias, scale, c, dh, dh0, extra, n_extra,
                       dsum);
  return check_launch("macro_fused_bwd_b");
}

// workspace of macro_fused_wgrad: pack arrays, dVc, dV2, then the grouped-K partials
static size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }

static size_t wgrad_fixed_bytes(int Bt, int S, int d, int G) {
  const size_t P = (size_t)Bt * S;
  return align256((size_t)(G + 1) * 4) * 2 + align256(P * 4) * 2 + align256((size_t)Bt * 4) * 2 +
         align256((size_t)G * 2 * d * kRank * 4) +
         align256((size_t)G * d * kRank * 4);
}

size_t macro_fused_wgrad_workspace_bytes(int Bt, int S, int d, int G) {
  if (Bt <= 0 || S <= 0 || d <= 0 || G <= 0) return 256;
  const int P = Bt * S;
  size_t gk = rte_grouped_linear_bwd_workspace_bytes(P, G, kRank, d);
  const size_t gv = rte_grouped_linear_bwd_workspace_bytes(P, G, 2 * d, kRank);
  const size_t g2 = rte_grouped_linear_bwd_workspace_bytes(Bt, G, d, kRank);
  gk = gk > gv ? gk : gv;
  gk = gk > g2 ? gk : g2;
  return wgrad_fixed_bytes(Bt, S, d, G) + align256(gk);
}

int macro_fused_wgrad(const int64_t* key, int B0, int Bh0, int B1, int Bh1, int S, int d, int G, const bf16* x2,
                      const bf16* sa, const bf16* du, const bf16* da, const bf16* pooled, const bf16* dsum,
                      const float* part_tab, float* dU, float* dV, float* dgain, float* dbias, float* dscale,
                      void* ws, size_t ws_bytes, hipStream_t s) {
  MF_SHAPES("macro_fused_wgrad");
  const int Bt = B0 + B1;
  RTE_REQUIRE(B0 >= 1 && B1 >= 0 && Bh0 >= 1 && (B1 == 0 || Bh1 >= 1) && Bt <= 16384 &&
                  (int64_t)Bt * S < ((int64_t)1 << 31),
              "macro_fused_wgrad: need 1 <= samples <= 16384 and rows < 2^31");
  RTE_REQUIRE(ws && ws_bytes >= macro_fused_wgrad_workspace_bytes(Bt, S, d, G),
              "macro_fused_wgrad: workspace too small");
  const int T = macro_fused_tiles(S);
  const int P = Bt * S;
  char* w = static_cast<char*>(ws);
  auto take = [&w](size_t n) {
    char* p = w;
    w += align256(n);
    return p;
  };
  int32_t* offsets = reinterpret_cast<int32_t*>(take((size_t)(G + 1) * 4));
  int32_t* soff = reinterpret_cast<int32_t*>(take((size_t)(G + 1) * 4));
  int32_t* tok = reinterpret_cast<int32_t*>(take((size_t)P * 4));
  int32_t* pos = reinterpret_cast<int32_t*>(take((size_t)P * 4));
  int32_t* slist = reinterpret_cast<int32_t*>(take((size_t)Bt * 4));
  int32_t* psrc = reinterpret_cast<int32_t*>(take((size_t)Bt * 4));
  float* dVc = reinterpret_cast<float*>(take((size_t)G * 2 * d * kRank * 4));
  float* dV2 = reinterpret_cast<float*>(take((size_t)G * d * kRank * 4));
  const size_t gk_bytes = ws_bytes - (size_t)(w - static_cast<char*>(ws));
  if (G <= kPackFastKeys && Bt <= kPackFastSamples) {
    const int nwg = std::max(1, std::min(32, (Bt + 63) / 64));  // about 64 listed samples per workgroup
    hipLaunchKernelGGL(mf_pack_fast_kernel, dim3(nwg), dim3(1024), 0, s, key, B0, Bh0, B1, Bh1 > 0 ? Bh1 : 1, S, G,
                       offsets, tok, pos, soff, slist, psrc);
  } else {
    const size_t lds = (size_t)(G + 2 * Bt) * sizeof(int);
    RTE_REQUIRE(lds <= 64 * 1024, "macro_fused_wgrad: too many keys and samples for one pack workgroup");
    hipLaunchKernelGGL(mf_pack_kernel, dim3(1), dim3(1024), lds, s, key, B0, Bh0, B1, Bh1 > 0 ? Bh1 : 1, S, G,
                       offsets, tok, pos, soff, slist, psrc);
  }
  RTE_TRY(check_launch("macro_fused_pack"));
  if (dU)
    RTE_TRY(rte_grouped_linear_bwd(du, sa, P, kRank, offsets, G, P, pos, pos, nullptr, d, nullptr, 0, dU, w,
                                   gk_bytes, s));
  if (dV) {
    RTE_TRY(rte_grouped_linear_bwd(da, x2, P, 2 * d, offsets, G, P, tok, pos, nullptr, kRank, nullptr, 0, dVc, w,
                                   gk_bytes, s));
    RTE_TRY(rte_grouped_linear_bwd(dsum, pooled, Bt, d, soff, G, Bt, psrc, slist, nullptr, kRank, nullptr, 0, dV2,
                                   w, gk_bytes, s));
    const int64_t n4 = (int64_t)G * 3 * d * kRank / 4;
    const int blocks = (int)((n4 + 255) / 256 < 4096 ? (n4 + 255) / 256 : 4096);
    hipLaunchKernelGGL(mf_vassemble_kernel, dim3(blocks), dim3(256), 0, s, reinterpret_cast<const float4*>(dVc),
                       reinterpret_cast<const float4*>(dV2), G, d, reinterpret_cast<float4*>(dV));
    RTE_TRY(check_launch("macro_fused_vassemble"));
  }
  return macro_table_grad_parts(key, Bt, T, G, d, part_tab, dgain, dbias, dscale, s);
}

}  // namespace rte
