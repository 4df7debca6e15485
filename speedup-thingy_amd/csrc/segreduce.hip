// Deterministic segmented row reduction (the weight-gradient scatter of
// rte/kernels/cluster_pool_ffn.py:218-241 and of every index/gather backward):
//   out[v] (+)= sum over pairs p with keys[p] = v of w[p] * rows[p / row_div]
// The pairs are counting-sorted by key (stable: ascending p), each key's run is summed in
// 256-pair chunks by one wave, and chunk partials are added in chunk order; up to 4096 pairs
// over up to 1024 keys take a one-launch path (per-key pair lists, summed in ascending p).  No
// floating-point atomics: the result is bitwise repeatable for a given input.
#include "common.hpp"

namespace rte {

namespace {

constexpr int kSortChunk = 1024;      // pairs per counting-sort block
constexpr int kSortSub = 256;         // pairs ranked together inside a sort block
constexpr int kMaxSortKeys = 32768;   // LDS histogram of the sort: 128 KB
constexpr int kSegChunk = 64;         // pairs per partial sum (a long run is cut into many)

// hist[v * nblk + b] = pairs of sort block b whose key is v.

__global__ void __launch_bounds__(256) sort_count_kernel(const int32_t* __restrict__ keys, int P, int V,
                                                         int32_t* __restrict__ hist, int nblk) {
  extern __shared__ int32_t hcount[];
  for (int c = threadIdx.x; c < V; c += 256) hcount[c] = 0;
  __syncthreads();
  const int64_t p0 = (int64_t)blockIdx.x * kSortChunk;
  for (int i = threadIdx.x; i < kSortChunk; i += 256) {
    const int64_t p = p0 + i;
    if (p < P) {
      const int k = keys[p];
      if (k >= 0 && k < V) atomicAdd(&hcount[k], 1);
    }
  }
  __syncthreads();
  for (int c = threadIdx.x; c < V; c += 256) hist[(int64_t)c * nblk + blockIdx.x] = hcount[c];
}

// Exclusive scan of each key's row of hist (one wave per key), totals[v] = row sum.
__global__ void __launch_bounds__(256) sort_rowscan_kernel(int32_t* __restrict__ hist, int V, int nblk,
                                                           int32_t* __restrict__ totals) {
  const int lane = threadIdx.x & 63;
  const int v = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (v >= V) return;
  int32_t* row = hist + (int64_t)v * nblk;
  int32_t run = 0;
  for (int b0 = 0; b0 < nblk; b0 += 64) {
    const int b = b0 + lane;
    const int32_t x = b < nblk ? row[b] : 0;
    int32_t inc = x;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const int32_t y = __shfl_up(inc, off, 64);
      if (lane >= off) inc += y;
    }
    if (b < nblk) row[b] = run + inc - x;
    run += __shfl(inc, 63, 64);
  }
  if (lane == 0) totals[v] = run;
}

// offsets = exclusive scan of totals, chunk_off = exclusive scan of ceil(totals / 256).
__global__ void __launch_bounds__(1024) sort_keyscan_kernel(const int32_t* __restrict__ totals, int V,
                                                            int32_t* __restrict__ offsets,
                                                            int32_t* __restrict__ chunk_off) {
  __shared__ int32_t ps[1024], pc[1024];
  const int tid = threadIdx.x;
  const int seg = (V + 1023) / 1024;
  const int b0 = tid * seg, b1 = min(V, b0 + seg);
  int32_t s = 0, sc = 0;
  for (int v = b0; v < b1; ++v) {
    s += totals[v];
    sc += (totals[v] + kSegChunk - 1) / kSegChunk;
  }
  ps[tid] = s;
  pc[tid] = sc;
  __syncthreads();
  for (int o = 1; o < 1024; o <<= 1) {
    const int32_t y = tid >= o ? ps[tid - o] : 0;
    const int32_t yc = tid >= o ? pc[tid - o] : 0;
    __syncthreads();
    ps[tid] += y;
    pc[tid] += yc;
    __syncthreads();
  }
  int32_t run = ps[tid] - s, runc = pc[tid] - sc;
  for (int v = b0; v < b1; ++v) {
    offsets[v] = run;
    chunk_off[v] = runc;
    run += totals[v];
    runc += (totals[v] + kSegChunk - 1) / kSegChunk;
  }
  if (tid == 1023) {
    offsets[V] = ps[1023];
    chunk_off[V] = pc[1023];
  }
}

// Stable scatter: pair p of block b with key v goes to slot offsets[v] + hist[v, b] +
// (pairs of block b before p with key v).  Writes the pair's row (p / row_div) and weight.
__global__ void __launch_bounds__(256) sort_scatter_kernel(const int32_t* __restrict__ keys, int P, int V,
                                                           int row_div, const int32_t* __restrict__ hist, int nblk,
                                                           const int32_t* __restrict__ offsets,
                                                           const float* __restrict__ g,
                                                           int32_t* __restrict__ tok_of_slot,
                                                           float* __restrict__ w_of_slot) {
  extern __shared__ int32_t cursor[];
  __shared__ __align__(16) int32_t sk[kSortSub];
  const int tid = threadIdx.x;
  for (int c = tid; c < V; c += 256) cursor[c] = offsets[c] + hist[(int64_t)c * nblk + blockIdx.x];
  const int64_t p0 = (int64_t)blockIdx.x * kSortChunk;
  constexpr int NQ = kSortChunk / kSortSub;
  int kq[NQ];  // every key of the block loaded up front (one memory latency, not one per sub-chunk)
#pragma unroll
  for (int q = 0; q < NQ; ++q) {
    const int64_t p = p0 + q * kSortSub + tid;
    kq[q] = p < P ? keys[p] : -1;
  }
#pragma unroll
  for (int q = 0; q < NQ; ++q) {
    const int64_t p = p0 + q * kSortSub + tid;
    const int k = kq[q];
    const bool valid = k >= 0 && k < V;
    __syncthreads();  // cursor ready / previous sub-chunk done with sk
    sk[tid] = valid ? k : -1;
    __syncthreads();
    int rank = 0;  // pairs of this sub-chunk before tid with the same key (16-byte LDS reads)
    if (valid) {
      const int4* s4 = reinterpret_cast<const int4*>(sk);
#pragma unroll 4
      for (int i4 = 0; 4 * i4 < tid; ++i4) {
        const int4 v = s4[i4];
        const int b = 4 * i4;
        rank += (b < tid && v.x == k) + (b + 1 < tid && v.y == k) + (b + 2 < tid && v.z == k) +
                (b + 3 < tid && v.w == k);
      }
    }
    const int slot = valid ? cursor[k] + rank : 0;
    __syncthreads();
    if (valid) {
      atomicAdd(&cursor[k], 1);
      tok_of_slot[slot] = (int32_t)(p / row_div);
      w_of_slot[slot] = g ? g[p] : 1.0f;
    }
  }
}

__device__ __forceinline__ void load8(const bf16* p, float* v) {
  const uint4 u = *reinterpret_cast<const uint4*>(p);
  const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    v[2 * i] = __uint_as_float(w[i] << 16);
    v[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
  }
}

__device__ __forceinline__ void load8(const float* p, float* v) {
  const float4 a = reinterpret_cast<const float4*>(p)[0], b = reinterpret_cast<const float4*>(p)[1];
  v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
  v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
}

// One wave per 64-pair chunk of one key's run: sum_s w[s] * rows[tok[s]].  A key with a
// single chunk writes out directly; otherwise the chunk's partial goes to part[item].
template <int NC2, typename RowT>
__global__ void __launch_bounds__(256) sort_segsum_kernel(const int32_t* __restrict__ offsets,
                                                          const int32_t* __restrict__ chunk_off, int V,
                                                          const int32_t* __restrict__ tok,
                                                          const float* __restrict__ w,
                                                          const RowT* __restrict__ hidden, int d,
                                                          float* __restrict__ part, float* __restrict__ dW,
                                                          int accumulate) {
  const int lane = threadIdx.x & 63;
  const int item = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (item >= chunk_off[V]) return;
  int lo = 0, hi = V;  // largest v with chunk_off[v] <= item
  while (hi - lo > 1) {
    const int mid = (lo + hi) >> 1;
    if (chunk_off[mid] <= item) lo = mid; else hi = mid;
  }
  const int v = lo;
  const int nq = chunk_off[v + 1] - chunk_off[v];
  const int s0 = offsets[v] + (item - chunk_off[v]) * kSegChunk;
  const int s1 = min(offsets[v + 1], s0 + kSegChunk);
  const int nch = d >> 3;
  float acc[NC2][8];
#pragma unroll
  for (int c = 0; c < NC2; ++c)
#pragma unroll
    for (int i = 0; i < 8; ++i) acc[c][i] = 0.0f;
  auto fma_row = [&](int s) {
    const RowT* row = hidden + (int64_t)tok[s] * d;
    const float gs = w[s];
#pragma unroll
    for (int c = 0; c < NC2; ++c) {
      if (lane + 64 * c >= nch) continue;
      float v[8];
      load8(row + (lane + 64 * c) * 8, v);
#pragma unroll
      for (int i = 0; i < 8; ++i) acc[c][i] += gs * v[i];
    }
  };
  int s = s0;
  for (; s + 8 <= s1; s += 8) {  // 8 rows in flight: indices and weights first, then the rows
    int t8[8];
    float g8[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      t8[j] = tok[s + j];
      g8[j] = w[s + j];
    }
#pragma unroll
    for (int c = 0; c < NC2; ++c) {
      if (lane + 64 * c >= nch) continue;
      float v[8][8];
#pragma unroll
      for (int j = 0; j < 8; ++j) load8(hidden + (int64_t)t8[j] * d + (lane + 64 * c) * 8, v[j]);
#pragma unroll
      for (int j = 0; j < 8; ++j)
#pragma unroll
        for (int i = 0; i < 8; ++i) acc[c][i] += g8[j] * v[j][i];
    }
  }
  for (; s < s1; ++s) fma_row(s);
  float* dst = nq == 1 ? dW + (int64_t)v * d : part + (int64_t)item * d;
  const bool add = nq == 1 && accumulate;
#pragma unroll
  for (int c = 0; c < NC2; ++c) {
    if (lane + 64 * c >= nch) continue;
    float4* o = reinterpret_cast<float4*>(dst + (lane + 64 * c) * 8);
    float4 a = make_float4(acc[c][0], acc[c][1], acc[c][2], acc[c][3]);
    float4 b = make_float4(acc[c][4], acc[c][5], acc[c][6], acc[c][7]);
    if (add) {
      const float4 a0 = o[0], b0 = o[1];
      a.x += a0.x; a.y += a0.y; a.z += a0.z; a.w += a0.w;
      b.x += b0.x; b.y += b0.y; b.z += b0.z; b.w += b0.w;
    }
    o[0] = a;
    o[1] = b;
  }
}

// Keys with zero or several chunks: dW[v] (+)= sum of the key's partials in chunk order.
__global__ void __launch_bounds__(256) sort_final_kernel(const int32_t* __restrict__ chunk_off, int V, int d,
                                                         const float* __restrict__ part, float* __restrict__ dW,
                                                         int accumulate) {
  const int64_t idx4 = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int d4 = d >> 2;
  if (idx4 >= (int64_t)V * d4) return;
  const int v = (int)(idx4 / d4), c = (int)(idx4 % d4) * 4;
  const int q0 = chunk_off[v], q1 = chunk_off[v + 1];
  if (q1 - q0 == 1) return;
  if (q1 == q0 && accumulate) return;
  float4 s = make_float4(0.f, 0.f, 0.f, 0.f);
  for (int q = q0; q < q1; ++q) {
    const float4 x = *reinterpret_cast<const float4*>(part + (int64_t)q * d + c);
    s.x += x.x; s.y += x.y; s.z += x.z; s.w += x.w;
  }
  float4* o = reinterpret_cast<float4*>(dW + (int64_t)v * d + c);
  if (accumulate) {
    const float4 a = *o;
    s.x += a.x; s.y += a.y; s.z += a.z; s.w += a.w;
  }
  *o = s;
}

template <typename K>
int set_lds_limit(K kernel, size_t bytes, const char* what) {
  if (bytes <= 65536) return 0;
  const hipError_t err = hipFuncSetAttribute(reinterpret_cast<const void*>(kernel),
                                             hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes);
  if (err != hipSuccess) {
    set_error("%s: cannot reserve %zu bytes of LDS: %s", what, bytes, hipGetErrorString(err));
    return -1;
  }
  return 0;
}

struct SegCarve {
  int32_t* hist;
  int32_t* totals;
  int32_t* offsets;
  int32_t* chunk_off;
  int32_t* tok;
  float* wslot;
  float* part;
  size_t bytes;
};

SegCarve carve(void* base, int64_t P, int V, int d) {
  const size_t nblk = ((size_t)P + kSortChunk - 1) / kSortChunk;
  const size_t max_items = ((size_t)P + kSegChunk - 1) / kSegChunk + (size_t)V;
  SegCarve c{};
  size_t off = 0;
  auto take = [&](size_t bytes) {
    char* p = base ? static_cast<char*>(base) + off : nullptr;
    off += ((bytes + 255) / 256) * 256;
    return static_cast<void*>(p);
  };
  c.hist = static_cast<int32_t*>(take((size_t)V * (nblk ? nblk : 1) * 4));
  c.totals = static_cast<int32_t*>(take((size_t)V * 4));
  c.offsets = static_cast<int32_t*>(take((size_t)(V + 1) * 4));
  c.chunk_off = static_cast<int32_t*>(take((size_t)(V + 1) * 4));
  c.tok = static_cast<int32_t*>(take((size_t)P * 4));
  c.wslot = static_cast<float*>(take((size_t)P * 4));
  c.part = static_cast<float*>(take(max_items * (size_t)d * 4));
  c.bytes = off;
  return c;
}

// Few pairs (P <= kSmallPairs) and few keys: one workgroup per key lists its pairs in
// ascending order (ballot compaction into LDS), then each thread sums 8 columns over the list
// in that order.  One launch instead of the sort pipeline; still deterministic.
constexpr int kSmallPairs = 4096;
constexpr int kSmallKeys = 1024;

template <typename RowT>
__global__ void __launch_bounds__(256) segsum_small_kernel(const int32_t* __restrict__ keys, int P, int row_div,
                                                           const float* __restrict__ w,
                                                           const RowT* __restrict__ rows, int d,
                                                           float* __restrict__ out, int accumulate) {
  __shared__ int32_t list[kSmallPairs];
  __shared__ int32_t wcnt[4];
  const int v = blockIdx.x;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  int n = 0;
  for (int base = 0; base < P; base += 256) {
    const int p = base + tid;
    const bool hit = p < P && keys[p] == v;
    const unsigned long long m = __ballot(hit);
    if (lane == 0) wcnt[wave] = __popcll(m);
    __syncthreads();
    int off = n;
    for (int q = 0; q < wave; ++q) off += wcnt[q];
    if (hit) list[off + __popcll(m & ((1ull << lane) - 1ull))] = p;
    n += ((wcnt[0] + wcnt[1]) + wcnt[2]) + wcnt[3];
    __syncthreads();
  }
  for (int col = tid * 8; col < d; col += 256 * 8) {
    float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
    for (int i = 0; i < n; ++i) {
      const int p = list[i];
      const float wp = w ? w[p] : 1.0f;
      float r[8];
      load8(rows + (int64_t)(p / row_div) * d + col, r);
#pragma unroll
      for (int t = 0; t < 8; ++t) acc[t] += wp * r[t];
    }
    float* o = out + (int64_t)v * d + col;
    if (accumulate) {
      float prev[8];
      load8(o, prev);
#pragma unroll
      for (int t = 0; t < 8; ++t) acc[t] += prev[t];
    }
    *reinterpret_cast<float4*>(o) = make_float4(acc[0], acc[1], acc[2], acc[3]);
    *reinterpret_cast<float4*>(o + 4) = make_float4(acc[4], acc[5], acc[6], acc[7]);
  }
}

template <typename RowT>
int launch_segsum(int nc2, dim3 grid, hipStream_t s, const SegCarve& c, int V, const RowT* rows, int d, float* out,
                  int accumulate) {
  if (nc2 <= 1)
    hipLaunchKernelGGL((sort_segsum_kernel<1, RowT>), grid, dim3(256), 0, s, c.offsets, c.chunk_off, V, c.tok,
                       c.wslot, rows, d, c.part, out, accumulate);
  else if (nc2 <= 2)
    hipLaunchKernelGGL((sort_segsum_kernel<2, RowT>), grid, dim3(256), 0, s, c.offsets, c.chunk_off, V, c.tok,
                       c.wslot, rows, d, c.part, out, accumulate);
  else
    hipLaunchKernelGGL((sort_segsum_kernel<4, RowT>), grid, dim3(256), 0, s, c.offsets, c.chunk_off, V, c.tok,
                       c.wslot, rows, d, c.part, out, accumulate);
  return check_launch("segment_reduce_sum");
}

}  // namespace

size_t segreduce_workspace_bytes(int64_t P, int V, int d) {
  if (P < 0 || V < 1 || d < 1) return 0;
  return carve(nullptr, P, V, d).bytes;
}

int segreduce_rows(const int32_t* keys, int64_t P, int V, int row_div, const float* w, const void* rows, int rows_f32,
                   int d, float* out, int accumulate, void* ws, size_t ws_bytes, hipStream_t s) {
  RTE_REQUIRE(V >= 1 && V <= kMaxSortKeys, "segment_reduce: key count must be in [1, %d]", kMaxSortKeys);
  RTE_REQUIRE(d >= 8 && d % 8 == 0 && d <= 2048, "segment_reduce: d must be a multiple of 8 in [8, 2048]");
  RTE_REQUIRE(P >= 0 && P < (1LL << 31) && row_div >= 1, "segment_reduce: bad pair count / row divisor");
  RTE_REQUIRE(((uintptr_t)rows & 15) == 0 && ((uintptr_t)out & 15) == 0 && ((uintptr_t)ws & 255) == 0,
              "segment_reduce: rows / out need 16-byte and workspace 256-byte alignment");
  const SegCarve c = carve(ws, P, V, d);
  RTE_REQUIRE(ws_bytes >= c.bytes, "segment_reduce: workspace too small (%zu < %zu)", ws_bytes, c.bytes);
  if (P == 0) {
    if (!accumulate) return fill_f32(out, 0.0f, (int64_t)V * d, s);
    return 0;
  }
  const int Pi = (int)P;
  if (Pi <= kSmallPairs && V <= kSmallKeys) {
    if (rows_f32)
      hipLaunchKernelGGL(segsum_small_kernel<float>, dim3(V), dim3(256), 0, s, keys, Pi, row_div, w,
                         static_cast<const float*>(rows), d, out, accumulate);
    else
      hipLaunchKernelGGL(segsum_small_kernel<bf16>, dim3(V), dim3(256), 0, s, keys, Pi, row_div, w,
                         static_cast<const bf16*>(rows), d, out, accumulate);
    return check_launch("segment_reduce_small");
  }
  const int nblk = (Pi + kSortChunk - 1) / kSortChunk;
  const dim3 block(256);
  const size_t lds_hist = (size_t)V * sizeof(int32_t);
  RTE_TRY(set_lds_limit(sort_count_kernel, lds_hist, "segment_reduce"));
  RTE_TRY(set_lds_limit(sort_scatter_kernel, lds_hist + kSortSub * sizeof(int32_t), "segment_reduce"));
  hipLaunchKernelGGL(sort_count_kernel, dim3(nblk), block, lds_hist, s, keys, Pi, V, c.hist, nblk);
  RTE_TRY(check_launch("segment_reduce_count"));
  hipLaunchKernelGGL(sort_rowscan_kernel, dim3((V + 3) / 4), block, 0, s, c.hist, V, nblk, c.totals);
  RTE_TRY(check_launch("segment_reduce_rowscan"));
  hipLaunchKernelGGL(sort_keyscan_kernel, dim3(1), dim3(1024), 0, s, c.totals, V, c.offsets, c.chunk_off);
  RTE_TRY(check_launch("segment_reduce_keyscan"));
  hipLaunchKernelGGL(sort_scatter_kernel, dim3(nblk), block, lds_hist, s, keys, Pi, V, row_div, c.hist, nblk,
                     c.offsets, w, c.tok, c.wslot);
  RTE_TRY(check_launch("segment_reduce_scatter"));
  // the chunk count lives on the device: launch its upper bound, extra waves exit at once
  const int64_t max_items = ((int64_t)Pi + kSegChunk - 1) / kSegChunk + V;
  const dim3 grid_i((unsigned)((max_items + 3) / 4));
  const int nc2 = (d / 8 + 63) / 64;
  if (rows_f32)
    RTE_TRY(launch_segsum(nc2, grid_i, s, c, V, static_cast<const float*>(rows), d, out, accumulate));
  else
    RTE_TRY(launch_segsum(nc2, grid_i, s, c, V, static_cast<const bf16*>(rows), d, out, accumulate));
  const int64_t n4 = (int64_t)V * (d / 4);
  hipLaunchKernelGGL(sort_final_kernel, dim3((unsigned)((n4 + 255) / 256)), block, 0, s, c.chunk_off, V, d, c.part,
                     out, accumulate);
  return check_launch("segment_reduce_final");
}

}  // namespace rte
