// Shortlist output head (rte/output.py:46-136, rte/kernels/reference.py:141-147):
// candidate build with first-occurrence dedupe, shortlist logits fused with the
// cross-entropy at target position 0, and the backward with a deterministic
// vocabulary-row gradient reduction.
//
// build   : one wave64 per token walks the candidate sequence
//             [target | members of its top vocab clusters | hard negatives arange(H) % V |
//              random negatives | filler arange(L) % V | (target + arange(2L)) % V]
//           64 candidates at a time.  A candidate is new when its bit is clear in the
//           wave's LDS bitmap of the vocabulary and no earlier lane of the chunk holds
//           it; new candidates take the next shortlist positions (ballot prefix count),
//           so the shortlist holds the first L distinct ids in candidate order -- the
//           order the reference obtains from scatter_reduce(amin) over [T, V] first
//           positions followed by topk(largest=False, sorted=True).
// fwd     : logits[t, j] = hidden[t] . W[shortlist[t, j]]; 8 lanes per vocab row, 8 rows
//           per wave pass; lse[t] = logsumexp_j logits[t, j]; loss[t] = lse[t] - logits[t, 0].
// bwd     : g[t, j] = dloss[t] (softmax_j - [j == 0]) + dlogits_ext[t, j]
//           dhidden[t] = sum_j g[t, j] W[shortlist[t, j]]             (ascending j)
//           dW[v]      = sum over pairs (t, j) with shortlist[t, j] = v of g[t, j] hidden[t]
//           The pairs are counting-sorted by vocab row (stable: ascending pair index),
//           each row's run is summed in 256-pair chunks by one wave, and chunk partials
//           are added in chunk order: no floating-point atomics, bitwise repeatable.
#include "common.hpp"

namespace rte {

size_t segreduce_workspace_bytes(int64_t P, int V, int d);
int segreduce_rows(const int32_t* keys, int64_t P, int V, int row_div, const float* w, const void* rows, int rows_f32,
                   int d, float* out, int accumulate, void* ws, size_t ws_bytes, hipStream_t s);

namespace {

constexpr int kMaxBuildVocab = 65536;  // 4 waves x 8 KB bitmap per block
constexpr int kMaxSortVocab = 32768;   // key range of the segmented reduction

// ----------------------------------------------------------------------------- build

__global__ void __launch_bounds__(256) shortlist_build_kernel(
    const int64_t* __restrict__ targets, const int32_t* __restrict__ top_clusters, int tc,
    const int64_t* __restrict__ members, int n_clusters, int per_cluster, const int64_t* __restrict__ random_negs,
    int R, int H, int L, int V, int T, int32_t* __restrict__ shortlist, int32_t* __restrict__ dup_per_token) {
  extern __shared__ uint32_t bitmap_all[];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int t = blockIdx.x * 4 + wave;
  const int words = (V + 31) / 32;
  uint32_t* bm = bitmap_all + wave * words;
  for (int w = lane; w < words; w += 64) bm[w] = 0u;
  __syncthreads();
  if (t >= T) return;  // no block-wide barrier below
  const int64_t tgt = targets[t];
  const int n_members = tc * per_cluster;
  const int width = 1 + n_members + H + R + L + 2 * L;
  int count = 0;
  for (int c0 = 0; c0 < width; c0 += 64) {
    const int i = c0 + lane;
    int64_t cand = -1;
    if (i < width) {
      int rem = i;
      if (rem == 0) {
        cand = tgt;
      } else if ((rem -= 1) < n_members) {
        const int32_t cl = top_clusters[(int64_t)t * tc + rem / per_cluster];
        cand = (cl >= 0 && cl < n_clusters) ? members[(int64_t)cl * per_cluster + rem % per_cluster] : -1;
      } else if ((rem -= n_members) < H) {
        cand = rem % V;
      } else if ((rem -= H) < R) {
        cand = random_negs[(int64_t)t * R + rem];
      } else if ((rem -= R) < L) {
        cand = rem % V;
      } else {
        rem -= L;
        cand = ((tgt + rem) % V + V) % V;
      }
    }
    const int cv = (cand >= 0 && cand < V) ? (int)cand : -1;
    bool dup_in_chunk = false;
    for (int j = 0; j < 64; ++j) {
      const int other = __shfl(cv, j, 64);
      dup_in_chunk |= (j < lane) && (other == cv);
    }
    const bool fresh = cv >= 0 && !dup_in_chunk && !((bm[cv >> 5] >> (cv & 31)) & 1u);
    const unsigned long long mask = __ballot(fresh);
    const int rank = __popcll(mask & ((1ull << lane) - 1ull));
    if (fresh) {
      const int pos = count + rank;
      if (pos < L) shortlist[(int64_t)t * L + pos] = cv;
      atomicOr(&bm[cv >> 5], 1u << (cv & 31));
    }
    count += __popcll(mask);
  }
  if (lane == 0) dup_per_token[t] = width - count;
}

// ----------------------------------------------------------------------------- logits + CE

__device__ __forceinline__ float dot8(uint4 a, uint4 b) {
  const uint32_t aw[4] = {a.x, a.y, a.z, a.w};
  const uint32_t bw[4] = {b.x, b.y, b.z, b.w};
  float s = 0.0f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    s += __uint_as_float(aw[i] << 16) * __uint_as_float(bw[i] << 16);
    s += __uint_as_float(aw[i] & 0xffff0000u) * __uint_as_float(bw[i] & 0xffff0000u);
  }
  return s;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
  return v;
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

// One wave per token.  Lane = G * grp + sub: group grp handles vocab row j0 + grp of the
// current pass (64 / G rows per pass), lane sub holds the 16-byte chunks sub, sub + G, ...
// of the row, so each load instruction reads whole 128-byte segments.  A lane holds at most
// NCMAX chunks: G grows with d so that the row chunks stay in registers.
template <int G, int NCMAX>
__global__ void __launch_bounds__(256) shortlist_fwd_kernel(const bf16* __restrict__ hidden,
                                                            const bf16* __restrict__ W, int d, int V,
                                                            const int32_t* __restrict__ sl, int L, int T,
                                                            float* __restrict__ logits, float* __restrict__ lse_out,
                                                            float* __restrict__ loss_out) {
  extern __shared__ float lg_all[];
  constexpr int RP = 64 / G;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int t = blockIdx.x * 4 + wave;
  const bool active = t < T;
  float* lg = lg_all + wave * L;
  const int grp = lane / G, sub = lane % G;
  const int nch = d >> 3;
  if (active) {
    uint4 h[NCMAX];
    const bf16* hrow = hidden + (int64_t)t * d;
#pragma unroll
    for (int i = 0; i < NCMAX; ++i)
      h[i] = sub + G * i < nch ? *reinterpret_cast<const uint4*>(hrow + (sub + G * i) * 8) : make_uint4(0u, 0u, 0u, 0u);
    for (int j0 = 0; j0 < L; j0 += RP) {
      const int j = j0 + grp;
      float s = 0.0f;
      if (j < L) {
        const int v = sl[(int64_t)t * L + j];
        if (v >= 0 && v < V) {
          const bf16* row = W + (int64_t)v * d;
          uint4 w[NCMAX];
#pragma unroll
          for (int i = 0; i < NCMAX; ++i)
            if (sub + G * i < nch) w[i] = *reinterpret_cast<const uint4*>(row + (sub + G * i) * 8);
#pragma unroll
          for (int i = 0; i < NCMAX; ++i)
            if (sub + G * i < nch) s += dot8(h[i], w[i]);
        } else {
          s = __builtin_nanf("");
        }
      }
#pragma unroll
      for (int off = 1; off < G; off <<= 1) s += __shfl_xor(s, off, 64);
      if (sub == 0 && j < L) {
        lg[j] = s;
        logits[(int64_t)t * L + j] = s;
      }
    }
  }
  __syncthreads();
  if (!active) return;
  float mx = -__builtin_inff();
  for (int j = lane; j < L; j += 64) mx = fmaxf(mx, lg[j]);
  mx = wave_max(mx);
  float se = 0.0f;
  for (int j = lane; j < L; j += 64) se += __expf(lg[j] - mx);
  se = wave_sum(se);
  if (lane == 0) {
    const float lse = mx + logf(se);
    lse_out[t] = lse;
    loss_out[t] = lse - lg[0];
  }
}

// g[t, :] and dhidden[t] = sum_j g[t, j] W[sl[t, j]].  One wave per token, lanes across
// d (lane owns 16-byte chunks lane, lane + 64, ...); rows are taken four at a time.
template <int NC2>
__global__ void __launch_bounds__(256) shortlist_bwd_dh_kernel(
    const float* __restrict__ dloss, const float* __restrict__ dlext, const bf16* __restrict__ W, int d, int V,
    const int32_t* __restrict__ sl, int L, int T, const float* __restrict__ logits, const float* __restrict__ lse,
    float* __restrict__ g_out, bf16* __restrict__ dh) {
  extern __shared__ float gl_all[];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int t = blockIdx.x * 4 + wave;
  const bool active = t < T;
  float* gl = gl_all + wave * L;
  if (active) {
    const float gt = dloss ? dloss[t] : 0.0f;
    const float l = lse[t];
    for (int j = lane; j < L; j += 64) {
      const int64_t o = (int64_t)t * L + j;
      float gj = dloss ? gt * (__expf(logits[o] - l) - (j == 0 ? 1.0f : 0.0f)) : 0.0f;
      if (dlext) gj += dlext[o];
      gl[j] = gj;
      g_out[o] = gj;
    }
  }
  __syncthreads();
  if (!active || dh == nullptr) return;
  const int nch = d >> 3;
  float acc[NC2][8];
#pragma unroll
  for (int c = 0; c < NC2; ++c)
#pragma unroll
    for (int i = 0; i < 8; ++i) acc[c][i] = 0.0f;
  const int32_t* srow = sl + (int64_t)t * L;
  auto load_row = [&](int j, uint4* u) {
    const int v = srow[j];
    const bool ok = v >= 0 && v < V;
    const bf16* row = W + (int64_t)(ok ? v : 0) * d;
#pragma unroll
    for (int c = 0; c < NC2; ++c)
      u[c] = (ok && lane + 64 * c < nch) ? *reinterpret_cast<const uint4*>(row + (lane + 64 * c) * 8)
                                         : make_uint4(0u, 0u, 0u, 0u);
  };
  auto fma_row = [&](float gj, const uint4* u) {
#pragma unroll
    for (int c = 0; c < NC2; ++c) {
      const uint32_t w[4] = {u[c].x, u[c].y, u[c].z, u[c].w};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        acc[c][2 * i] += gj * __uint_as_float(w[i] << 16);
        acc[c][2 * i + 1] += gj * __uint_as_float(w[i] & 0xffff0000u);
      }
    }
  };
  int j = 0;
  for (; j + 4 <= L; j += 4) {
    uint4 u0[NC2], u1[NC2], u2[NC2], u3[NC2];
    load_row(j, u0);
    load_row(j + 1, u1);
    load_row(j + 2, u2);
    load_row(j + 3, u3);
    fma_row(gl[j], u0);
    fma_row(gl[j + 1], u1);
    fma_row(gl[j + 2], u2);
    fma_row(gl[j + 3], u3);
  }
  for (; j < L; ++j) {
    uint4 u0[NC2];
    load_row(j, u0);
    fma_row(gl[j], u0);
  }
#pragma unroll
  for (int c = 0; c < NC2; ++c) {
    if (lane + 64 * c >= nch) continue;
    uint4 o;
    o.x = pack_bf2(acc[c][0], acc[c][1]);
    o.y = pack_bf2(acc[c][2], acc[c][3]);
    o.z = pack_bf2(acc[c][4], acc[c][5]);
    o.w = pack_bf2(acc[c][6], acc[c][7]);
    *reinterpret_cast<uint4*>(dh + (int64_t)t * d + (lane + 64 * c) * 8) = o;
  }
}

}  // namespace

int shortlist_build(const int64_t* targets, const int32_t* top_clusters, int tc, const int64_t* members,
                    int n_clusters, int per_cluster, const int64_t* random_negs, int R, int H, int L, int V, int T,
                    int32_t* shortlist, int32_t* dup_per_token, hipStream_t s) {
  RTE_REQUIRE(V >= 1 && V <= kMaxBuildVocab, "shortlist_build: vocab size must be in [1, %d]", kMaxBuildVocab);
  RTE_REQUIRE(L >= 1 && L <= V, "shortlist_build: need 1 <= L <= V (got L=%d, V=%d)", L, V);
  RTE_REQUIRE(tc >= 0 && per_cluster >= 0 && R >= 0 && H >= 0 && T >= 0, "shortlist_build: negative size");
  RTE_REQUIRE(tc == 0 || (n_clusters >= 1 && per_cluster >= 1), "shortlist_build: empty member table");
  RTE_REQUIRE((int64_t)tc * per_cluster + H + R + 3LL * L + 1 < (1LL << 30), "shortlist_build: too many candidates");
  if (T == 0) return 0;
  const size_t lds = (size_t)4 * ((V + 31) / 32) * sizeof(uint32_t);
  hipLaunchKernelGGL(shortlist_build_kernel, dim3((T + 3) / 4), dim3(256), lds, s, targets, top_clusters, tc,
                     members, n_clusters, per_cluster, random_negs, R, H, L, V, T, shortlist, dup_per_token);
  return check_launch("shortlist_build");
}

int shortlist_fwd(const bf16* hidden, const bf16* W, int d, int V, const int32_t* sl, int L, int T, float* logits,
                  float* lse, float* loss, hipStream_t s) {
  RTE_REQUIRE(d >= 8 && d % 8 == 0 && d <= 2048, "shortlist_fwd: d must be a multiple of 8 in [8, 2048]");
  RTE_REQUIRE(L >= 1 && L <= 4096 && V >= 1, "shortlist_fwd: need 1 <= L <= 4096");
  RTE_REQUIRE(((uintptr_t)hidden & 15) == 0 && ((uintptr_t)W & 15) == 0, "shortlist_fwd: 16-byte alignment");
  if (T == 0) return 0;
  const size_t lds = (size_t)4 * L * sizeof(float);
  const dim3 grid((T + 3) / 4), block(256);
#define RTE_SL_FWD(G, NC) \
  hipLaunchKernelGGL((shortlist_fwd_kernel<G, NC>), grid, block, lds, s, hidden, W, d, V, sl, L, T, logits, lse, loss)
  if (d <= 256)
    RTE_SL_FWD(8, 4);
  else if (d <= 512)
    RTE_SL_FWD(8, 8);
  else if (d <= 1024)
    RTE_SL_FWD(16, 8);
  else
    RTE_SL_FWD(32, 8);
#undef RTE_SL_FWD
  return check_launch("shortlist_fwd");
}

size_t shortlist_bwd_workspace_bytes(int T, int L, int V, int d) {
  if (T < 0 || L < 1 || V < 1 || d < 1) return 0;
  const size_t g_bytes = (((size_t)T * L * 4 + 255) / 256) * 256;
  return g_bytes + segreduce_workspace_bytes((int64_t)T * L, V, d);
}

int shortlist_bwd(const float* dloss, const float* dlext, const bf16* hidden, const bf16* W, int d, int V,
                  const int32_t* sl, int L, int T, const float* logits, const float* lse, bf16* dhidden, float* dW,
                  int dW_accumulate, void* ws, size_t ws_bytes, hipStream_t s) {
  RTE_REQUIRE(d >= 8 && d % 8 == 0 && d <= 2048, "shortlist_bwd: d must be a multiple of 8 in [8, 2048]");
  RTE_REQUIRE(L >= 1 && L <= 4096 && V >= 1, "shortlist_bwd: need 1 <= L <= 4096");
  RTE_REQUIRE(dW == nullptr || V <= kMaxSortVocab, "shortlist_bwd: dW needs vocab size <= %d", kMaxSortVocab);
  RTE_REQUIRE((int64_t)T * L < (1LL << 31), "shortlist_bwd: T * L must fit in int32");
  RTE_REQUIRE(((uintptr_t)hidden & 15) == 0 && ((uintptr_t)W & 15) == 0 && ((uintptr_t)ws & 255) == 0,
              "shortlist_bwd: hidden / W need 16-byte and workspace 256-byte alignment");
  const size_t need = shortlist_bwd_workspace_bytes(T, L, V, d);
  RTE_REQUIRE(ws_bytes >= need, "shortlist_bwd: workspace too small (%zu < %zu)", ws_bytes, need);
  if (T == 0) {
    if (dW && !dW_accumulate) return fill_f32(dW, 0.0f, (int64_t)V * d, s);
    return 0;
  }
  float* g = static_cast<float*>(ws);
  const size_t g_bytes = (((size_t)T * L * 4 + 255) / 256) * 256;
  const size_t lds_g = (size_t)4 * L * sizeof(float);
  const dim3 grid_t((T + 3) / 4), block(256);
  const int nc2 = (d / 8 + 63) / 64;
  if (nc2 <= 1)
    hipLaunchKernelGGL(shortlist_bwd_dh_kernel<1>, grid_t, block, lds_g, s, dloss, dlext, W, d, V, sl, L, T, logits,
                       lse, g, dhidden);
  else if (nc2 <= 2)
    hipLaunchKernelGGL(shortlist_bwd_dh_kernel<2>, grid_t, block, lds_g, s, dloss, dlext, W, d, V, sl, L, T, logits,
                       lse, g, dhidden);
  else
    hipLaunchKernelGGL(shortlist_bwd_dh_kernel<4>, grid_t, block, lds_g, s, dloss, dlext, W, d, V, sl, L, T, logits,
                       lse, g, dhidden);
  RTE_TRY(check_launch("shortlist_bwd_dhidden"));
  if (!dW) return 0;
  // dW[v] = sum over pairs (t, j) with sl[t, j] = v of g[t, j] hidden[t]: key = sl, row = p / L
  return segreduce_rows(sl, (int64_t)T * L, V, L, g, hidden, 0, d, dW, dW_accumulate,
                        static_cast<char*>(ws) + g_bytes, ws_bytes - g_bytes, s);
}

}  // namespace rte
