// fp32 arithmetic for training.precision = "fp32" (the reference's default precision, where every
// matmul runs in float32 and nothing is cast to bf16).
//
//  * rte_gemm_f32: C = alpha op(A) op(B)^T + beta C on v_mfma_f32_32x32x2_f32 with fp32 operands and
//    accumulation.  One kernel covers the dense products, batched products (two-level batch
//    strides: the attention's (sample, head) pairs read straight out of the packed QKV rows), and
//    grouped products over device-side group offsets: GROUP_M (each group a row range with its own
//    weight block: routed / banked pools, per-key macro products) and GROUP_K (each group a
//    reduction range writing its own output block: their weight gradients, one workgroup per
//    output tile summing its group's rows in order, so results repeat bitwise).  Rows of A and B
//    may be gathered through index arrays and scaled per row; rows of C may be scattered.
//  * causal softmax over score rows (scaled, optional per-(batch) output scale), forward and backward
//  * SwiGLU over [up | gate] rows, forward and backward
//  * pair combine (out[t] = resid[t] + sum_j w[t, j] rows[slot(t, j)]) and the pair row dots of its
//    weight gradient
//
// Tile: 64 x 64 outputs per 256-thread workgroup (four waves of 32 x 32), k steps of 16 staged
// through LDS k-major (each MFMA operand a contiguous 32-float LDS row segment), the next k tile's
// global loads issued before the current tile's MFMAs.
#include "common.hpp"

namespace rte {
namespace {

typedef __attribute__((__vector_size__(16 * sizeof(float)))) float f32x16;

constexpr int kBM = 64, kBN = 64, kBK = 16, kThreads = 256;
constexpr int kPad = 4;

struct GemmF32 {
  const float* A;
  int64_t lda;
  int a_t;
  const int32_t* a_rows;
  const float* a_scale;
  const float* B;
  int64_t ldb;
  int b_t;
  const int32_t* b_rows;
  const float* b_scale;
  float* C;
  int64_t ldc;
  const int32_t* c_rows;
  int M, N, K;
  float alpha, beta;
  // batch z = z1 * Z2 + z2: operand offsets z1 * s1 + z2 * s2
  int Z2;
  int64_t sA1, sA2, sB1, sB2, sC1, sC2;
  // groups: mode 1 = GROUP_M (rows), 2 = GROUP_K (reduction); goff[G + 1] device offsets
  int mode;
  const int32_t* goff;
  int G;
  const int64_t* b_goff;  // GROUP_M: B element offset of group g (else g * b_gstride)
  int64_t b_gstride, b_rows_gstride;
  const int64_t* c_goff;  // GROUP_K: C element offset of group g (else g * c_gstride)
  int64_t c_gstride, c_rows_gstride;
};

// One 64 x 16 operand tile into registers: element e of thread t.  Non-transposed operands are
// contiguous along k (thread: one row, four k), transposed ones along the row index (thread: one
// k, four rows).  Rows outside [r0, r_end) and k outside [k0, k_end) read as 0.
__device__ __forceinline__ void load_tile(const float* X, int64_t ld, int x_t, const int32_t* rows,
                                          const float* scale, int r0, int r_end, int k0, int k_end, float v[4]) {
  const int t = threadIdx.x;
  if (!x_t) {
    const int r = r0 + (t >> 2);
    const int kq = k0 + (t & 3) * 4;
    if (r < r_end) {
      const int64_t row = rows ? (int64_t)rows[r] : (int64_t)r;
      const float sc = scale ? scale[r] : 1.0f;
      const float* p = X + row * ld;
#pragma unroll
      for (int i = 0; i < 4; ++i) v[i] = (kq + i < k_end) ? p[kq + i] * sc : 0.0f;
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) v[i] = 0.0f;
    }
  } else {
    const int k = k0 + (t >> 4);
    const int rq = r0 + (t & 15) * 4;
    if (k < k_end) {
      const int64_t row = rows ? (int64_t)rows[k] : (int64_t)k;
      const float sc = scale ? scale[k] : 1.0f;
      const float* p = X + row * ld;
#pragma unroll
      for (int i = 0; i < 4; ++i) v[i] = (rq + i < r_end) ? p[rq + i] * sc : 0.0f;
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i) v[i] = 0.0f;
    }
  }
}

__device__ __forceinline__ void store_tile(float (*S)[kBM + kPad], int x_t, const float v[4]) {
  const int t = threadIdx.x;
  if (!x_t) {
    const int r = t >> 2, kq = (t & 3) * 4;
#pragma unroll
    for (int i = 0; i < 4; ++i) S[kq + i][r] = v[i];
  } else {
    const int k = t >> 4, rq = (t & 15) * 4;
#pragma unroll
    for (int i = 0; i < 4; ++i) S[k][rq + i] = v[i];
  }
}

__global__ void __launch_bounds__(kThreads) gemm_f32_kernel(GemmF32 p) {
  __shared__ float As[kBK][kBM + kPad];
  __shared__ float Bs[kBK][kBN + kPad];
  __shared__ int s_info[3];
  const float* A = p.A;
  const float* B = p.B;
  float* C = p.C;
  const int32_t* b_rows = p.b_rows;
  const int32_t* c_rows = p.c_rows;
  int m0, m_end = p.M, k_lo = 0, k_hi = p.K;
  const int n0 = blockIdx.y * kBN;
  if (p.mode == 1) {
    // GROUP_M: the x index enumerates each group's row tiles in group order (one thread walks the
    // offsets; tile counts are ceil(rows / 64) per group)
    if (threadIdx.x == 0) {
      int tile = blockIdx.x, g = 0, found = -1, start = 0;
      for (; g < p.G; ++g) {
        const int lo = p.goff[g], hi = p.goff[g + 1];
        const int nt = (hi - lo + kBM - 1) / kBM;
        if (tile < nt) {
          found = g;
          start = lo + tile * kBM;
          break;
        }
        tile -= nt;
      }
      s_info[0] = found;
      s_info[1] = start;
      s_info[2] = found >= 0 ? p.goff[found + 1] : 0;
    }
    __syncthreads();
    const int g = s_info[0];
    if (g < 0) return;
    m0 = s_info[1];
    m_end = s_info[2];
    B += p.b_goff ? p.b_goff[g] : (int64_t)g * p.b_gstride;
    if (b_rows) b_rows += (int64_t)g * p.b_rows_gstride;
  } else if (p.mode == 2) {
    const int g = blockIdx.z;
    m0 = blockIdx.x * kBM;
    k_lo = p.goff[g];
    k_hi = p.goff[g + 1];
    C += p.c_goff ? p.c_goff[g] : (int64_t)g * p.c_gstride;
    if (c_rows) c_rows += (int64_t)g * p.c_rows_gstride;
  } else {
    m0 = blockIdx.x * kBM;
    const int z = blockIdx.z, z1 = z / p.Z2, z2 = z - z1 * p.Z2;
    A += z1 * p.sA1 + z2 * p.sA2;
    B += z1 * p.sB1 + z2 * p.sB2;
    C += z1 * p.sC1 + z2 * p.sC2;
  }
  if (m0 >= m_end || n0 >= p.N) return;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  f32x16 acc;
#pragma unroll
  for (int r = 0; r < 16; ++r) acc[r] = 0.0f;
  float va[4], vb[4];
  // a_t: A's memory rows run over k; else over m (rows gathered / scaled by the logical index)
  load_tile(A, p.lda, p.a_t, p.a_rows, p.a_scale, m0, m_end, k_lo, k_hi, va);
  load_tile(B, p.ldb, p.b_t, b_rows, p.b_scale, n0, p.N, k_lo, k_hi, vb);
  for (int k0 = k_lo; k0 < k_hi; k0 += kBK) {
    store_tile(As, p.a_t, va);
    store_tile(Bs, p.b_t, vb);
    __syncthreads();
    if (k0 + kBK < k_hi) {
      load_tile(A, p.lda, p.a_t, p.a_rows, p.a_scale, m0, m_end, k0 + kBK, k_hi, va);
      load_tile(B, p.ldb, p.b_t, b_rows, p.b_scale, n0, p.N, k0 + kBK, k_hi, vb);
    }
#pragma unroll
    for (int kk = 0; kk < kBK; kk += 2) {
      const float a = As[kk + (lane >> 5)][wm * 32 + (lane & 31)];
      const float b = Bs[kk + (lane >> 5)][wn * 32 + (lane & 31)];
      acc = __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, acc, 0, 0, 0);
    }
    __syncthreads();
  }
  const int col = n0 + wn * 32 + (lane & 31);
  if (col >= p.N) return;
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int m = m0 + wm * 32 + (lane >> 5) * 4 + (r >> 2) * 8 + (r & 3);
    if (m < m_end) {
      const int64_t row = c_rows ? (int64_t)c_rows[m] : (int64_t)m;
      float* c = C + row * p.ldc + col;
      const float v = p.alpha * acc[r];
      *c = p.beta != 0.0f ? v + p.beta * *c : v;
    }
  }
}

// ---------------------------------------------------------------------------------------------
// causal softmax over rows of [Z, S, S] scores: P = softmax(scale * s, keys <= query); the output
// is oscale[z] * P (oscale optional).  One wave per row, the row read in 64-column chunks.

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
  return v;
}
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
  return v;
}

__global__ void softmax_causal_fwd_kernel(const float* s, int64_t rows, int S, float scale, const float* oscale,
                                          float* p_out, float* y_out) {
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const int lane = threadIdx.x & 63;
  const int q = (int)(row % S);
  const int64_t z = row / S;
  const float* x = s + row * S;
  float mx = -INFINITY;
  for (int c = lane; c <= q; c += 64) mx = fmaxf(mx, x[c] * scale);
  mx = wave_max(mx);
  float sum = 0.0f;
  for (int c = lane; c <= q; c += 64) sum += __expf(x[c] * scale - mx);
  sum = wave_sum(sum);
  const float inv = 1.0f / sum;
  const float os = oscale ? oscale[z] : 1.0f;
  float* pr = p_out + row * S;
  float* yr = y_out + row * S;
  for (int c = lane; c < S; c += 64) {
    const float v = c <= q ? __expf(x[c] * scale - mx) * inv : 0.0f;
    pr[c] = v;
    yr[c] = v * os;
  }
}

// ds = scale * P (g - sum_c P g) with g = oscale * dy
__global__ void softmax_causal_bwd_kernel(const float* P, const float* dy, int64_t rows, int S, float scale,
                                          const float* oscale, float* ds) {
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const int lane = threadIdx.x & 63;
  const int64_t z = row / S;
  const float os = oscale ? oscale[z] : 1.0f;
  const float* pr = P + row * S;
  const float* gr = dy + row * S;
  float dot = 0.0f;
  for (int c = lane; c < S; c += 64) dot += pr[c] * gr[c];
  dot = wave_sum(dot) * os;
  float* o = ds + row * S;
  for (int c = lane; c < S; c += 64) o[c] = scale * pr[c] * (os * gr[c] - dot);
}

// ---------------------------------------------------------------------------------------------
// SwiGLU over rows [up (n) | gate (n)] of width ld: z = up silu(gate)

__global__ void swiglu_f32_fwd_kernel(const float* ug, int64_t rows, int n, int64_t ld, float* z) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= rows * n) return;
  const int64_t r = i / n;
  const int j = (int)(i - r * n);
  const float u = ug[r * ld + j], g = ug[r * ld + n + j];
  z[i] = u * g * sigmoidf_(g);
}

__global__ void swiglu_f32_bwd_kernel(const float* ug, const float* dz, int64_t rows, int n, int64_t ld, float* dug) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= rows * n) return;
  const int64_t r = i / n;
  const int j = (int)(i - r * n);
  const float u = ug[r * ld + j], g = ug[r * ld + n + j], d = dz[i];
  const float sg = sigmoidf_(g);
  dug[r * ld + j] = d * g * sg;
  dug[r * ld + n + j] = d * u * sg * (1.0f + g * (1.0f - sg));
}

// ---------------------------------------------------------------------------------------------
// pair combine: out[t] = resid[t] + sum_j w[t, j] rows[slot[t k + j]] (slot < 0: no pair; w
// optional = 1), the pairs summed in j order.  One workgroup of 64 lanes per token row, lanes
// over the columns.
__global__ void combine_f32_kernel(const float* rows, const int32_t* slot, const float* w, int T, int k, int d,
                                   const float* resid, float* out) {
  const int t = blockIdx.x;
  for (int c = threadIdx.x; c < d; c += blockDim.x) {
    float acc = resid ? resid[(int64_t)t * d + c] : 0.0f;
    for (int j = 0; j < k; ++j) {
      const int s = slot[(int64_t)t * k + j];
      if (s >= 0) acc += (w ? w[(int64_t)t * k + j] : 1.0f) * rows[(int64_t)s * d + c];
    }
    out[(int64_t)t * d + c] = acc;
  }
}

// dw[t, j] = sum_c dout[t, c] rows[slot[t k + j], c]  (0 for an absent pair): one wave per pair
__global__ void pair_dot_f32_kernel(const float* dout, const float* rows, const int32_t* slot, int64_t pairs, int k,
                                    int d, float* dw) {
  const int64_t pr = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (pr >= pairs) return;
  const int lane = threadIdx.x & 63;
  const int s = slot[pr];
  float acc = 0.0f;
  if (s >= 0) {
    const float* a = dout + (pr / k) * d;
    const float* b = rows + (int64_t)s * d;
    for (int c = lane; c < d; c += 64) acc += a[c] * b[c];
  }
  acc = wave_sum(acc);
  if (lane == 0) dw[pr] = acc;
}

}  // namespace
}  // namespace rte

using namespace rte;

extern "C" {

int rte_gemm_f32(const float* A, int64_t lda, int a_t, const int32_t* a_rows, const float* a_scale, const float* B,
                 int64_t ldb, int b_t, const int32_t* b_rows, const float* b_scale, float* C, int64_t ldc,
                 const int32_t* c_rows, int M, int N, int K, float alpha, float beta, int Z1, int Z2, int64_t sA1,
                 int64_t sA2, int64_t sB1, int64_t sB2, int64_t sC1, int64_t sC2, void* stream) {
  RTE_REQUIRE(M >= 0 && N >= 0 && K >= 0 && Z1 >= 1 && Z2 >= 1, "gemm_f32: bad sizes");
  RTE_REQUIRE(A && B && C, "gemm_f32: null operand");
  RTE_REQUIRE((int64_t)Z1 * Z2 <= 65535, "gemm_f32: at most 65535 batches");
  if (M == 0 || N == 0) return 0;
  GemmF32 p{A, lda, a_t, a_rows, a_scale, B, ldb, b_t, b_rows, b_scale, C, ldc, c_rows, M, N, K, alpha, beta,
            Z2, sA1, sA2, sB1, sB2, sC1, sC2, 0, nullptr, 0, nullptr, 0, 0, nullptr, 0, 0};
  dim3 grid((M + kBM - 1) / kBM, (N + kBN - 1) / kBN, Z1 * Z2);
  RTE_REQUIRE(grid.y <= 65535, "gemm_f32: N too large");
  hipLaunchKernelGGL(gemm_f32_kernel, grid, dim3(kThreads), 0, static_cast<hipStream_t>(stream), p);
  return check_launch("gemm_f32");
}

// Grouped products.  mode 1 (GROUP_M): group g owns rows [goff[g], goff[g+1]) of the M total and
// reads B at b_goff[g] (or g * b_gstride) with b_rows shifted by g * b_rows_gstride.  mode 2
// (GROUP_K): group g reduces over k in [goff[g], goff[g+1]) and writes C at c_goff[g] (or
// g * c_gstride) with c_rows shifted by g * c_rows_gstride.
int rte_gemm_f32_grouped(int mode, const int32_t* goff, int G, const float* A, int64_t lda, int a_t,
                         const int32_t* a_rows, const float* a_scale, const float* B, int64_t ldb, int b_t,
                         const int32_t* b_rows, const float* b_scale, const int64_t* b_goff, int64_t b_gstride,
                         int64_t b_rows_gstride, float* C, int64_t ldc, const int32_t* c_rows, const int64_t* c_goff,
                         int64_t c_gstride, int64_t c_rows_gstride, int M, int N, int K, float alpha, float beta,
                         void* stream) {
  RTE_REQUIRE(mode == 1 || mode == 2, "gemm_f32_grouped: mode must be 1 (rows) or 2 (reduction)");
  RTE_REQUIRE(G >= 0 && M >= 0 && N >= 0 && K >= 0, "gemm_f32_grouped: bad sizes");
  RTE_REQUIRE(goff && A && B && C, "gemm_f32_grouped: null argument");
  if (G == 0 || N == 0 || (mode == 1 && M == 0) || (mode == 2 && M == 0)) return 0;
  GemmF32 p{A, lda, a_t, a_rows, a_scale, B, ldb, b_t, b_rows, b_scale, C, ldc, c_rows, M, N, K, alpha, beta,
            1, 0, 0, 0, 0, 0, 0, mode, goff, G, b_goff, b_gstride, b_rows_gstride, c_goff, c_gstride,
            c_rows_gstride};
  dim3 grid;
  if (mode == 1) {
    grid = dim3((M + kBM - 1) / kBM + G, (N + kBN - 1) / kBN, 1);  // a bound on the groups' row tiles
  } else {
    RTE_REQUIRE(G <= 65535, "gemm_f32_grouped: at most 65535 reduction groups");
    grid = dim3((M + kBM - 1) / kBM, (N + kBN - 1) / kBN, G);
  }
  hipLaunchKernelGGL(gemm_f32_kernel, grid, dim3(kThreads), 0, static_cast<hipStream_t>(stream), p);
  return check_launch("gemm_f32_grouped");
}

int rte_softmax_causal_f32_fwd(const float* s, int64_t rows, int S, float scale, const float* oscale, float* p,
                               float* y, void* stream) {
  RTE_REQUIRE(rows >= 0 && S >= 1 && s && p && y, "softmax_causal_f32_fwd: bad arguments");
  if (rows == 0) return 0;
  hipLaunchKernelGGL(softmax_causal_fwd_kernel, dim3((unsigned)((rows + 3) / 4)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), s, rows, S, scale, oscale, p, y);
  return check_launch("softmax_causal_f32_fwd");
}

int rte_softmax_causal_f32_bwd(const float* p, const float* dy, int64_t rows, int S, float scale,
                               const float* oscale, float* ds, void* stream) {
  RTE_REQUIRE(rows >= 0 && S >= 1 && p && dy && ds, "softmax_causal_f32_bwd: bad arguments");
  if (rows == 0) return 0;
  hipLaunchKernelGGL(softmax_causal_bwd_kernel, dim3((unsigned)((rows + 3) / 4)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), p, dy, rows, S, scale, oscale, ds);
  return check_launch("softmax_causal_f32_bwd");
}

int rte_swiglu_f32_fwd(const float* ug, int64_t rows, int n, int64_t ld, float* z, void* stream) {
  RTE_REQUIRE(rows >= 0 && n >= 1 && ld >= 2 * (int64_t)n && ug && z, "swiglu_f32_fwd: bad arguments");
  const int64_t total = rows * n;
  if (total == 0) return 0;
  hipLaunchKernelGGL(swiglu_f32_fwd_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), ug, rows, n, ld, z);
  return check_launch("swiglu_f32_fwd");
}

int rte_swiglu_f32_bwd(const float* ug, const float* dz, int64_t rows, int n, int64_t ld, float* dug, void* stream) {
  RTE_REQUIRE(rows >= 0 && n >= 1 && ld >= 2 * (int64_t)n && ug && dz && dug, "swiglu_f32_bwd: bad arguments");
  const int64_t total = rows * n;
  if (total == 0) return 0;
  hipLaunchKernelGGL(swiglu_f32_bwd_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), ug, dz, rows, n, ld, dug);
  return check_launch("swiglu_f32_bwd");
}

int rte_combine_f32(const float* rows, const int32_t* slot, const float* w, int T, int k, int d, const float* resid,
                    float* out, void* stream) {
  RTE_REQUIRE(T >= 0 && k >= 1 && d >= 1 && rows && slot && out, "combine_f32: bad arguments");
  if (T == 0) return 0;
  hipLaunchKernelGGL(combine_f32_kernel, dim3(T), dim3(d >= 256 ? 256 : 64), 0, static_cast<hipStream_t>(stream),
                     rows, slot, w, T, k, d, resid, out);
  return check_launch("combine_f32");
}

int rte_pair_dot_f32(const float* dout, const float* rows, const int32_t* slot, int64_t pairs, int k, int d, float* dw,
                     void* stream) {
  RTE_REQUIRE(pairs >= 0 && k >= 1 && d >= 1 && dout && rows && slot && dw, "pair_dot_f32: bad arguments");
  if (pairs == 0) return 0;
  hipLaunchKernelGGL(pair_dot_f32_kernel, dim3((unsigned)((pairs + 3) / 4)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), dout, rows, slot, pairs, k, d, dw);
  return check_launch("pair_dot_f32");
}

}  // extern "C"
