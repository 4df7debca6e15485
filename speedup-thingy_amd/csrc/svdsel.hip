// Per-token kernels of the SVD-factor sparse SwiGLU FFN (SVDFactorSparseFFN, rte/layers.py:342-643;
// device driver rte/kernels/svd_sparse_ffn_triton.py:480-714).
//
// Forward, one workgroup per token, from the selector's approximate activations (the expand GEMM
// of the low-rank factors: up_hat, gate_hat in the interleaved [T, 2F] layout, z_hat = up_hat *
// silu(gate_hat)):
//   1. candidate views: top up_m of |up_hat| w, top gate_m of |silu(gate_hat)| w, top product_m of
//      |z_hat| w (w = ||W_down row||), united in a bitmap; fewer than top_k candidates: the top
//      top_k of the product view are added (the reference's fill rule);
//   2. the candidates' activations: exact (<x, W_up[c]>, <x, W_gate[c]>) or the approximate ones;
//   3. rerank: top top_k of |u silu(g)| w among the candidates;
//   4. out = sum over the selected (ascending neuron id) of u silu(g) W_down[c].
// "product" strategy: the top top_k of the product view, approximate activations, no union.
// Every top-m is exact and deterministic: the m-th largest score is found by a 32-step binary
// search over the scores' bit patterns (scores are >= 0 or NaN, so the bit order is the value
// order and NaN ranks first), then all larger scores and the lowest-index ties are taken.
//
// Backward, one workgroup per token: dz = <dout, W_down[c]>, du = dz silu(g), dg = dz u silu'(g),
// dx = sum du W_up[c] + dg W_gate[c]; the weight gradients are segmented reductions keyed by the
// selected ids (run by the caller).
#include "common.hpp"

namespace rte {
namespace {

constexpr int kSelThreads = 256;

__device__ __forceinline__ int wave_isum(int v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

__device__ __forceinline__ float wave_fsum(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

// Block sum of one int per thread (every thread gets the total).
__device__ __forceinline__ int block_isum(int v, int* red) {
  v = wave_isum(v);
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  return red[0] + red[1] + red[2] + red[3];
}

// Exclusive block scan of one int per thread; returns the prefix, *total gets the sum.
__device__ __forceinline__ int block_iscan(int v, int* red, int* total) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  int inc = v;
#pragma unroll
  for (int off = 1; off < 64; off <<= 1) {
    const int y = __shfl_up(inc, off, 64);
    if (lane >= off) inc += y;
  }
  __syncthreads();
  if (lane == 63) red[wave] = inc;
  __syncthreads();
  int before = 0;
  for (int w = 0; w < wave; ++w) before += red[w];
  *total = red[0] + red[1] + red[2] + red[3];
  return before + inc - v;
}

// Sets the bits (in bitmap) of the m largest keys of key[0..n); of keys equal to the m-th
// largest, the lowest indices.  Keys are float bit patterns of non-negative scores or NaN (so the
// bit order is the value order, NaN first).  1 <= m <= n.
__device__ void select_top(const uint32_t* key, int n, int m, uint32_t* bitmap, int* red) {
  uint32_t thr = 0;
  for (int bit = 31; bit >= 0; --bit) {
    const uint32_t cand = thr | (1u << bit);
    int c = 0;
    for (int j = threadIdx.x; j < n; j += kSelThreads) c += key[j] >= cand;
    if (block_isum(c, red) >= m) thr = cand;
  }
  const int per = (n + kSelThreads - 1) / kSelThreads;
  const int j0 = threadIdx.x * per, j1 = j0 + per < n ? j0 + per : n;
  int gt = 0, eq = 0;
  for (int j = j0; j < j1; ++j) {
    gt += key[j] > thr;
    eq += key[j] == thr;
  }
  int gtot, etot;
  block_iscan(gt, red, &gtot);
  int epos = block_iscan(eq, red, &etot);
  const int need = m - gtot;  // ties taken, lowest index first
  for (int j = j0; j < j1; ++j) {
    bool take = key[j] > thr;
    if (!take && key[j] == thr && epos < need) {
      take = true;
      ++epos;
    }
    if (take) atomicOr(&bitmap[j >> 5], 1u << (j & 31));
  }
  __syncthreads();
}

// The same selection, listed in ascending index order (larger scores and ties interleaved).
__device__ int select_top_list(const uint32_t* key, int n, int m, int* out_ids, uint32_t* scratch_bm, int* red) {
  for (int w = threadIdx.x; w < (n + 31) / 32; w += kSelThreads) scratch_bm[w] = 0u;
  __syncthreads();
  select_top(key, n, m, scratch_bm, red);
  // enumerate set bits in ascending order
  const int nw = (n + 31) / 32;
  const int per = (nw + kSelThreads - 1) / kSelThreads;
  const int w0 = threadIdx.x * per, w1 = w0 + per < nw ? w0 + per : nw;
  int cnt = 0;
  for (int w = w0; w < w1; ++w) cnt += __popc(scratch_bm[w]);
  int tot;
  int pos = block_iscan(cnt, red, &tot);
  for (int w = w0; w < w1; ++w) {
    uint32_t b = scratch_bm[w];
    while (b) {
      const int l = __ffs(b) - 1;
      b &= b - 1;
      out_ids[pos++] = w * 32 + l;
    }
  }
  __syncthreads();
  return tot;
}

__device__ __forceinline__ float siluf(float g) { return g / (1.0f + __expf(-g)); }

__device__ __forceinline__ uint32_t score_key(float s) { return __float_as_uint(fabsf(s)); }

// interleaved [2F] row: neuron j's up at (j / 32) * 64 + j % 32, its gate 32 further
__device__ __forceinline__ int ilv_up(int j) { return (j >> 5) * 64 + (j & 31); }

struct SelArgs {
  const bf16* x;      // [T, d]
  const bf16* ug;     // [T, 2F] interleaved
  const bf16* w_up;   // [F, d]
  const bf16* w_gate;
  const bf16* w_down;
  const float* wdn;   // [F]
  int T, d, F, up_m, gate_m, product_m, top_k, max_cand, exact, product_only;
  void* out;          // [T, d]
  int out_f32;
  int32_t* sel_ids;   // [T, top_k]
  float* sel_u;
  float* sel_g;
  int32_t* n_cand;    // [T] (optional)
};

__global__ void __launch_bounds__(kSelThreads) svd_sparse_fwd_kernel(SelArgs a) {
  extern __shared__ __align__(16) unsigned char smem[];
  const int F = a.F, d = a.d, t = blockIdx.x;
  uint32_t* key = reinterpret_cast<uint32_t*>(smem);                   // [max(F, max_cand)]
  const int keyn = F > a.max_cand ? F : a.max_cand;
  uint32_t* bm = key + keyn;                                           // [F / 32]
  uint32_t* bm2 = bm + (F + 31) / 32;                                  // [max(F, max_cand) / 32 + 1]
  int* cid = reinterpret_cast<int*>(bm2 + (keyn + 31) / 32 + 1);       // [max_cand]
  float* cu = reinterpret_cast<float*>(cid + a.max_cand);              // [max_cand]
  float* cg = cu + a.max_cand;                                         // [max_cand]
  int* sel = reinterpret_cast<int*>(cg + a.max_cand);                  // [top_k]
  float* xs = reinterpret_cast<float*>(sel + a.top_k);                 // [d]
  __shared__ int red[4];
  const bf16* ugr = a.ug + (int64_t)t * 2 * F;
  const int tid = threadIdx.x;

  for (int w = tid; w < (F + 31) / 32; w += kSelThreads) bm[w] = 0u;
  // 1. candidate views
  const int views[3] = {a.up_m, a.gate_m, a.product_m};
  int nc = 0;
  if (!a.product_only) {
    for (int v = 0; v < 3; ++v) {
      const int m = views[v] < F ? views[v] : F;
      if (m <= 0) continue;
      __syncthreads();
      for (int j = tid; j < F; j += kSelThreads) {
        const float u = bf2f(ugr[ilv_up(j)]), g = bf2f(ugr[ilv_up(j) + 32]);
        const float s = v == 0 ? u : (v == 1 ? siluf(g) : u * siluf(g));
        key[j] = score_key(s * a.wdn[j]);
      }
      __syncthreads();
      select_top(key, F, m, bm, red);
    }
    // count the union; fill from the product view when it is smaller than top_k
    int c = 0;
    for (int w = tid; w < (F + 31) / 32; w += kSelThreads) c += __popc(bm[w]);
    nc = block_isum(c, red);
  }
  if (nc < a.top_k) {
    __syncthreads();
    for (int j = tid; j < F; j += kSelThreads) {
      const float u = bf2f(ugr[ilv_up(j)]), g = bf2f(ugr[ilv_up(j) + 32]);
      key[j] = score_key(u * siluf(g) * a.wdn[j]);
    }
    __syncthreads();
    select_top(key, F, a.top_k < F ? a.top_k : F, bm, red);
  }
  // enumerate the candidates (ascending id), at most max_cand (the lowest ids beyond that are dropped)
  {
    const int nw = (F + 31) / 32;
    const int per = (nw + kSelThreads - 1) / kSelThreads;
    const int w0 = tid * per, w1 = w0 + per < nw ? w0 + per : nw;
    int cnt = 0;
    for (int w = w0; w < w1; ++w) cnt += __popc(bm[w]);
    int pos = block_iscan(cnt, red, &nc);
    for (int w = w0; w < w1; ++w) {
      uint32_t b = bm[w];
      while (b) {
        const int l = __ffs(b) - 1;
        b &= b - 1;
        if (pos < a.max_cand) cid[pos] = w * 32 + l;
        ++pos;
      }
    }
    if (nc > a.max_cand) nc = a.max_cand;
    __syncthreads();
  }
  if (tid == 0 && a.n_cand) a.n_cand[t] = nc;
  // 2. candidate activations
  if (a.exact) {
    for (int j = tid; j < d; j += kSelThreads) xs[j] = bf2f(a.x[(int64_t)t * d + j]);
    __syncthreads();
    const int lane = tid & 63, wave = tid >> 6;
    for (int c = wave; c < nc; c += 4) {
      const bf16* ru = a.w_up + (int64_t)cid[c] * d;
      const bf16* rg = a.w_gate + (int64_t)cid[c] * d;
      float su = 0.0f, sg = 0.0f;
      for (int j = lane * 8; j < d; j += 512) {
        const uint4 pu = *reinterpret_cast<const uint4*>(ru + j);
        const uint4 pg = *reinterpret_cast<const uint4*>(rg + j);
        const uint32_t wu[4] = {pu.x, pu.y, pu.z, pu.w}, wg[4] = {pg.x, pg.y, pg.z, pg.w};
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          su = fmaf(xs[j + 2 * q], __uint_as_float(wu[q] << 16), su);
          su = fmaf(xs[j + 2 * q + 1], __uint_as_float(wu[q] & 0xffff0000u), su);
          sg = fmaf(xs[j + 2 * q], __uint_as_float(wg[q] << 16), sg);
          sg = fmaf(xs[j + 2 * q + 1], __uint_as_float(wg[q] & 0xffff0000u), sg);
        }
      }
      su = wave_fsum(su);
      sg = wave_fsum(sg);
      if (lane == 0) {
        cu[c] = su;
        cg[c] = sg;
      }
    }
  } else {
    for (int c = tid; c < nc; c += kSelThreads) {
      cu[c] = bf2f(ugr[ilv_up(cid[c])]);
      cg[c] = bf2f(ugr[ilv_up(cid[c]) + 32]);
    }
  }
  __syncthreads();
  // 3. rerank
  for (int c = tid; c < nc; c += kSelThreads) key[c] = score_key(cu[c] * siluf(cg[c]) * a.wdn[cid[c]]);
  __syncthreads();
  const int k = a.top_k < nc ? a.top_k : nc;
  const int ns = select_top_list(key, nc, k, sel, bm2, red);
  // 4. outputs
  for (int i = tid; i < a.top_k; i += kSelThreads) {
    const int64_t o = (int64_t)t * a.top_k + i;
    if (i < ns) {
      const int c = sel[i];
      a.sel_ids[o] = cid[c];
      a.sel_u[o] = cu[c];
      a.sel_g[o] = cg[c];
    } else {
      a.sel_ids[o] = -1;
      a.sel_u[o] = 0.0f;
      a.sel_g[o] = 0.0f;
    }
  }
  for (int col = tid * 4; col < d; col += kSelThreads * 4) {
    float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int i = 0; i < ns; ++i) {
      const int c = sel[i];
      const float z = cu[c] * siluf(cg[c]);
      const uint2 w = *reinterpret_cast<const uint2*>(a.w_down + (int64_t)cid[c] * d + col);
      acc[0] = fmaf(z, __uint_as_float(w.x << 16), acc[0]);
      acc[1] = fmaf(z, __uint_as_float(w.x & 0xffff0000u), acc[1]);
      acc[2] = fmaf(z, __uint_as_float(w.y << 16), acc[2]);
      acc[3] = fmaf(z, __uint_as_float(w.y & 0xffff0000u), acc[3]);
    }
    if (a.out_f32) {
      *reinterpret_cast<float4*>(static_cast<float*>(a.out) + (int64_t)t * d + col) =
          make_float4(acc[0], acc[1], acc[2], acc[3]);
    } else {
      uint2 o;
      o.x = pack_bf2(acc[0], acc[1]);
      o.y = pack_bf2(acc[2], acc[3]);
      *reinterpret_cast<uint2*>(static_cast<bf16*>(a.out) + (int64_t)t * d + col) = o;
    }
  }
}

struct SelBwdArgs {
  const bf16* dout;   // [T, d]
  const bf16* w_up;
  const bf16* w_gate;
  const bf16* w_down;
  const int32_t* sel_ids;
  const float* sel_u;
  const float* sel_g;
  int T, d, top_k;
  bf16* dx;           // [T, d]
  float* z;           // [T, top_k] (u silu(g), the weights of dW_down)
  float* du;          // [T, top_k]
  float* dg;
};

__global__ void __launch_bounds__(kSelThreads) svd_sparse_bwd_kernel(SelBwdArgs a) {
  extern __shared__ __align__(16) unsigned char smem[];
  const int d = a.d, K = a.top_k, t = blockIdx.x, tid = threadIdx.x;
  float* go = reinterpret_cast<float*>(smem);  // [d]
  float* sdu = go + d;                         // [K]
  float* sdg = sdu + K;                        // [K]
  for (int j = tid; j < d; j += kSelThreads) go[j] = bf2f(a.dout[(int64_t)t * d + j]);
  __syncthreads();
  const int lane = tid & 63, wave = tid >> 6;
  for (int i = wave; i < K; i += 4) {
    const int64_t o = (int64_t)t * K + i;
    const int c = a.sel_ids[o];
    float dz = 0.0f;
    if (c >= 0) {
      const bf16* rd = a.w_down + (int64_t)c * d;
      for (int j = lane * 8; j < d; j += 512) {
        const uint4 p = *reinterpret_cast<const uint4*>(rd + j);
        const uint32_t w[4] = {p.x, p.y, p.z, p.w};
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          dz = fmaf(go[j + 2 * q], __uint_as_float(w[q] << 16), dz);
          dz = fmaf(go[j + 2 * q + 1], __uint_as_float(w[q] & 0xffff0000u), dz);
        }
      }
    }
    dz = wave_fsum(dz);
    if (lane == 0) {
      const float u = a.sel_u[o], g = a.sel_g[o];
      const float s = 1.0f / (1.0f + __expf(-g));
      const float sl = g * s;
      const float vu = c >= 0 ? dz * sl : 0.0f;
      const float vg = c >= 0 ? dz * u * s * (1.0f + g * (1.0f - s)) : 0.0f;
      sdu[i] = vu;
      sdg[i] = vg;
      a.du[o] = vu;
      a.dg[o] = vg;
      a.z[o] = c >= 0 ? u * sl : 0.0f;
    }
  }
  __syncthreads();
  for (int col = tid * 4; col < d; col += kSelThreads * 4) {
    float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int i = 0; i < K; ++i) {
      const int c = a.sel_ids[(int64_t)t * K + i];
      if (c < 0) continue;
      const uint2 wu = *reinterpret_cast<const uint2*>(a.w_up + (int64_t)c * d + col);
      const uint2 wg = *reinterpret_cast<const uint2*>(a.w_gate + (int64_t)c * d + col);
      const float u = sdu[i], g = sdg[i];
      acc[0] = fmaf(g, __uint_as_float(wg.x << 16), fmaf(u, __uint_as_float(wu.x << 16), acc[0]));
      acc[1] = fmaf(g, __uint_as_float(wg.x & 0xffff0000u), fmaf(u, __uint_as_float(wu.x & 0xffff0000u), acc[1]));
      acc[2] = fmaf(g, __uint_as_float(wg.y << 16), fmaf(u, __uint_as_float(wu.y << 16), acc[2]));
      acc[3] = fmaf(g, __uint_as_float(wg.y & 0xffff0000u), fmaf(u, __uint_as_float(wu.y & 0xffff0000u), acc[3]));
    }
    uint2 o;
    o.x = pack_bf2(acc[0], acc[1]);
    o.y = pack_bf2(acc[2], acc[3]);
    *reinterpret_cast<uint2*>(a.dx + (int64_t)t * d + col) = o;
  }
}

size_t sel_lds_bytes(int F, int max_cand, int top_k, int d) {
  const int keyn = F > max_cand ? F : max_cand;
  return (size_t)keyn * 4 + (size_t)((F + 31) / 32) * 4 + (size_t)((keyn + 31) / 32 + 1) * 4 +
         (size_t)max_cand * 12 + (size_t)top_k * 4 + (size_t)d * 4;
}

}  // namespace

int svd_sparse_select(const bf16* x, const bf16* ug, const bf16* w_up, const bf16* w_gate, const bf16* w_down,
                      const float* wdn, int T, int d, int F, int up_m, int gate_m, int product_m, int top_k,
                      int exact, int product_only, void* out, int out_f32, int32_t* sel_ids, float* sel_u,
                      float* sel_g, int32_t* n_cand, hipStream_t s) {
  RTE_REQUIRE(T >= 0 && d > 0 && d % 8 == 0 && F > 0 && top_k >= 1 && top_k <= F,
              "svd_sparse: bad sizes (d %% 8 == 0, 1 <= top_k <= d_ff)");
  const int m = (up_m > 0 ? up_m : 0) + (gate_m > 0 ? gate_m : 0) + (product_m > 0 ? product_m : 0);
  int max_cand = product_only ? top_k : (m > top_k ? m : top_k) + top_k;
  if (max_cand > F) max_cand = F;
  const size_t lds = sel_lds_bytes(F, max_cand, top_k, d);
  RTE_REQUIRE(lds <= 150 * 1024, "svd_sparse: d_ff %d / %d candidates / d_model %d need %zu bytes of LDS", F,
              max_cand, d, lds);
  if (T == 0) return 0;
  SelArgs a{x, ug, w_up, w_gate, w_down, wdn, T, d, F, up_m, gate_m, product_m, top_k, max_cand, exact,
            product_only, out, out_f32, sel_ids, sel_u, sel_g, n_cand};
  hipLaunchKernelGGL(svd_sparse_fwd_kernel, dim3(T), dim3(kSelThreads), lds, s, a);
  return check_launch("svd_sparse_fwd");
}

int svd_sparse_bwd(const bf16* dout, const bf16* w_up, const bf16* w_gate, const bf16* w_down, const int32_t* sel_ids,
                   const float* sel_u, const float* sel_g, int T, int d, int top_k, bf16* dx, float* z, float* du,
                   float* dg, hipStream_t s) {
  RTE_REQUIRE(T >= 0 && d > 0 && d % 8 == 0 && top_k >= 1, "svd_sparse_bwd: bad sizes");
  const size_t lds = (size_t)d * 4 + (size_t)top_k * 8;
  RTE_REQUIRE(lds <= 150 * 1024, "svd_sparse_bwd: sizes need too much LDS");
  if (T == 0) return 0;
  SelBwdArgs a{dout, w_up, w_gate, w_down, sel_ids, sel_u, sel_g, T, d, top_k, dx, z, du, dg};
  hipLaunchKernelGGL(svd_sparse_bwd_kernel, dim3(T), dim3(kSelThreads), lds, s, a);
  return check_launch("svd_sparse_bwd");
}

}  // namespace rte
