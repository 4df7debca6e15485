// Token -> cluster routing, deterministic packing and fixed-order combine.
//
//  route_topk  : one wave64 per token; C <= 128: each logit ranked against the row
//                (readlane broadcast), else k rounds of a wave arg-max over the C
//                router logits (value descending, index ascending on ties,
//                NaN above everything as torch.topk does), then softmax over
//                the k selected logits.  Many tokens (T >= 16384, C <= 128): one lane
//                per token instead, rows staged through LDS and a sorted top-k kept in
//                registers by insertion (same order, same softmax summation tree).
//  pack        : stable counting sort of the T*k (token, cluster) pairs by
//                cluster.  Slots inside a cluster follow ascending pair index,
//                i.e. ascending token, like the nonzero()-based index build of
//                the reference.  Three launches, integer-only, no atomics whose
//                order could leak into the result.
//  combine     : out[t] = extra[t] + resid[t] + sum_j rows[t*k + j], j in order.
#include "common.hpp"

namespace rte {

namespace {

__device__ __forceinline__ bool better(float a, int ia, float b, int ib) {
  const bool na = a != a, nb = b != b;
  if (na != nb) return na;
  if (!na && a != b) return a > b;
  return ia < ib;
}

constexpr int kMaxPerLane = 16;  // C <= 1024

__global__ void __launch_bounds__(256) route_topk_kernel(const float* __restrict__ logits, int T, int C,
                                                         int k, int32_t* __restrict__ ids,
                                                         float* __restrict__ weights) {
  const int lane = threadIdx.x & 63;
  const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= T) return;
  const float* row = logits + (int64_t)t * C;
  float v[kMaxPerLane];
  bool used[kMaxPerLane];
  const int per = (C + 63) / 64;
#pragma unroll
  for (int i = 0; i < kMaxPerLane; ++i) {
    const int c = lane + 64 * i;
    used[i] = !(i < per && c < C);
    v[i] = used[i] ? 0.0f : row[c];
  }
  float my_v = 0.0f;
  int my_i = 0;
  for (int r = 0; r < k; ++r) {
    // lane-local best among unused
    float bv = 0.0f;
    int bi = 0x7fffffff;
#pragma unroll
    for (int i = 0; i < kMaxPerLane; ++i) {
      if (used[i]) continue;
      const int c = lane + 64 * i;
      if (bi == 0x7fffffff || better(v[i], c, bv, bi)) {
        bv = v[i];
        bi = c;
      }
    }
    // wave arg-max (butterfly: every lane ends with the winner); empty lanes carry INT_MAX
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
      const float ov = __shfl_xor(bv, off, 64);
      const int oi = __shfl_xor(bi, off, 64);
      if (oi != 0x7fffffff && (bi == 0x7fffffff || better(ov, oi, bv, bi))) {
        bv = ov;
        bi = oi;
      }
    }
    if (bi != 0x7fffffff && (bi & 63) == lane) {
#pragma unroll
      for (int i = 0; i < kMaxPerLane; ++i)
        if (i == (bi >> 6)) used[i] = true;
    }
    if (lane == r) {
      my_v = bv;
      my_i = bi;
    }
  }
  // lane j < k holds the j-th selection; softmax over the selected logits
  const float mx = __shfl(my_v, 0, 64);
  const float ex = lane < k ? expf(my_v - mx) : 0.0f;
  float denom = ex;
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) denom += __shfl_xor(denom, off, 64);
  if (lane < k) {
    ids[(int64_t)t * k + lane] = my_i;
    weights[(int64_t)t * k + lane] = ex / denom;
  }
}

// Small pools (C <= 64 * PER): the rank of element c is the number of elements better
// than it, counted against every logit of the row broadcast with readlane (no LDS round
// trips on the critical path); the k best land in LDS at their rank, then lanes j < k
// finish exactly like route_topk_kernel (same selection values, same softmax order).
template <int PER, bool kNaN>
__device__ __forceinline__ void rank_row(const float (&v)[PER], int lane, int C, int (&rank)[PER]) {
#pragma unroll
  for (int q = 0; q < PER; ++q) {
    const int nq = C - 64 * q < 64 ? C - 64 * q : 64;
    for (int l = 0; l < nq; ++l) {
      const float vj = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v[q]), l));
      const int j = 64 * q + l;
#pragma unroll
      for (int i = 0; i < PER; ++i) {
        const int c = lane + 64 * i;
        if (kNaN)
          rank[i] += better(vj, j, v[i], c) ? 1 : 0;
        else
          rank[i] += (vj > v[i] || (vj == v[i] && j < c)) ? 1 : 0;
      }
    }
  }
}

template <int PER>
__global__ void __launch_bounds__(256) route_topk_rank_kernel(const float* __restrict__ logits, int T, int C, int k,
                                                              int32_t* __restrict__ ids,
                                                              float* __restrict__ weights) {
  __shared__ float sel_v[4][16];
  __shared__ int sel_i[4][16];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int t = blockIdx.x * 4 + wave;
  const bool live = t < T;  // no early exit: every wave reaches the barrier below
  const float* row = logits + (int64_t)(live ? t : 0) * C;
  float v[PER];
  int rank[PER];
  bool nan_here = false;
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int c = lane + 64 * i;
    v[i] = (live && c < C) ? row[c] : 0.0f;
    rank[i] = 0;
    nan_here |= v[i] != v[i];
  }
  if (__ballot(nan_here) != 0)
    rank_row<PER, true>(v, lane, C, rank);
  else
    rank_row<PER, false>(v, lane, C, rank);
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int c = lane + 64 * i;
    if (c < C && rank[i] < k) {
      sel_v[wave][rank[i]] = v[i];
      sel_i[wave][rank[i]] = c;
    }
  }
  __syncthreads();
  if (!live) return;
  const float my_v = lane < k ? sel_v[wave][lane] : 0.0f;
  const int my_i = lane < k ? sel_i[wave][lane] : 0;
  const float mx = __shfl(my_v, 0, 64);
  const float ex = lane < k ? expf(my_v - mx) : 0.0f;
  float denom = ex;
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) denom += __shfl_xor(denom, off, 64);
  if (lane < k) {
    ids[(int64_t)t * k + lane] = my_i;
    weights[(int64_t)t * k + lane] = ex / denom;
  }
}

constexpr int kPackChunk = 256;

// hist layout: hist[c * nblk + b] = pairs of block b routed to cluster c.
// A block covers nsub consecutive 256-pair sub-chunks (more for large P, so the histogram the
// single-workgroup scan walks stays short).
__global__ void __launch_bounds__(256) pack_count_kernel(const int32_t* __restrict__ cl, int P, int C, int nsub,
                                                         int32_t* __restrict__ hist, int nblk,
                                                         int32_t* __restrict__ invalid) {
  extern __shared__ int32_t sh[];
  for (int c = threadIdx.x; c < C; c += blockDim.x) sh[c] = 0;
  __syncthreads();
  const int64_t pb = (int64_t)blockIdx.x * nsub * kPackChunk;
  for (int q = 0; q < nsub; ++q) {
    const int64_t p = pb + (int64_t)q * kPackChunk + threadIdx.x;
    if (p < P) {
      const int c = cl[p];
      if (c >= 0 && c < C) {
        atomicAdd(&sh[c], 1);
      } else if (invalid) {
        atomicAdd(invalid, 1);
      }
    }
  }
  __syncthreads();
  for (int c = threadIdx.x; c < C; c += blockDim.x) hist[(int64_t)c * nblk + blockIdx.x] = sh[c];
}

// Exclusive scan of hist (length L = C * nblk) in place, single workgroup of 1024, in tiles of
// 8192 entries: coalesced loads into LDS, each thread scans 8 consecutive entries, a wave scan
// of the thread totals (shuffles), the 16 wave totals in LDS, and a carry across tiles.
constexpr int kScanThreads = 1024, kScanPer = 8, kScanTile = kScanThreads * kScanPer;

__global__ void __launch_bounds__(kScanThreads) pack_scan_kernel(int32_t* __restrict__ hist, int C, int nblk,
                                                                 int32_t* __restrict__ offsets, int P) {
  __shared__ int32_t tile[kScanTile + kScanTile / 32];  // one pad word per 32 entries
  __shared__ int32_t wsum[kScanThreads / 64];
  __shared__ int32_t carry_sh;
  const int64_t L = (int64_t)C * nblk;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  auto at = [](int i) { return i + (i >> 5); };
  int32_t carry = 0;
  for (int64_t base = 0; base < L; base += kScanTile) {
    const int n = L - base < kScanTile ? (int)(L - base) : kScanTile;
#pragma unroll
    for (int r = 0; r < kScanPer; ++r) {
      const int i = r * kScanThreads + tid;
      tile[at(i)] = i < n ? hist[base + i] : 0;
    }
    __syncthreads();
    int32_t v[kScanPer], sum = 0;
#pragma unroll
    for (int r = 0; r < kScanPer; ++r) {
      v[r] = tile[at(tid * kScanPer + r)];
      sum += v[r];
    }
    // inclusive wave scan of the thread totals
    int32_t inc = sum;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const int32_t y = __shfl_up(inc, off, 64);
      if (lane >= off) inc += y;
    }
    if (lane == 63) wsum[wave] = inc;
    __syncthreads();
    int32_t before = carry;
    for (int w2 = 0; w2 < wave; ++w2) before += wsum[w2];
    int32_t run = before + inc - sum;
#pragma unroll
    for (int r = 0; r < kScanPer; ++r) {
      tile[at(tid * kScanPer + r)] = run;
      run += v[r];
    }
    if (tid == kScanThreads - 1) carry_sh = run;
    __syncthreads();
#pragma unroll
    for (int r = 0; r < kScanPer; ++r) {
      const int i = r * kScanThreads + tid;
      if (i < n) hist[base + i] = tile[at(i)];
    }
    carry = carry_sh;
    __syncthreads();
  }
  // every thread's last global write precedes this barrier; offsets read the scanned hist
  for (int c = tid; c < C; c += kScanThreads) offsets[c] = hist[(int64_t)c * nblk];
  if (tid == 0) offsets[C] = carry;
  (void)P;
}

// One thread per pair of each sub-chunk: its slot is the block's running base for its cluster
// (the block's scanned histogram entry plus the cluster's pairs in earlier sub-chunks) plus the
// number of earlier pairs of the sub-chunk with the same cluster (stable: ascending pair order
// inside a cluster).
__global__ void __launch_bounds__(256) pack_scatter_kernel(const int32_t* __restrict__ cl, int P, int C, int nsub,
                                                           int k, const int32_t* __restrict__ hist,
                                                           int nblk, const float* __restrict__ w,
                                                           int32_t* __restrict__ tok_of_slot,
                                                           int32_t* __restrict__ pair_of_slot,
                                                           int32_t* __restrict__ slot_of_pair,
                                                           float* __restrict__ w_of_slot) {
  extern __shared__ int32_t cursor[];  // [C]
  __shared__ __align__(16) int32_t sc[kPackChunk];
  const int tid = threadIdx.x;
  for (int c = tid; c < C; c += kPackChunk) cursor[c] = hist[(int64_t)c * nblk + blockIdx.x];
  const int64_t pb = (int64_t)blockIdx.x * nsub * kPackChunk;
  for (int q = 0; q < nsub; ++q) {
    const int64_t p = pb + (int64_t)q * kPackChunk + tid;
    __syncthreads();  // cursor ready / the previous sub-chunk is done with sc and cursor
    sc[tid] = p < P ? cl[p] : -1;
    __syncthreads();
    const int c = sc[tid];
    const bool valid = p < P && c >= 0 && c < C;
    int slot = -1;
    if (valid) {
      int rank = 0;
      const int4* s4 = reinterpret_cast<const int4*>(sc);
      const int full = tid >> 2;
      for (int j = 0; j < full; ++j) {
        const int4 v = s4[j];
        rank += (v.x == c) + (v.y == c) + (v.z == c) + (v.w == c);
      }
      for (int j = full * 4; j < tid; ++j) rank += sc[j] == c;
      slot = cursor[c] + rank;
    }
    __syncthreads();  // every slot read its cursor before the cursors advance
    if (valid) {
      atomicAdd(&cursor[c], 1);
      if (tok_of_slot) tok_of_slot[slot] = (int32_t)(p / k);
      if (pair_of_slot) pair_of_slot[slot] = (int32_t)p;
      if (w_of_slot) w_of_slot[slot] = w ? w[p] : 1.0f;
    }
    if (p < P && slot_of_pair) slot_of_pair[p] = slot;
  }
}

// One lane per token: the wave's 64 rows are staged in LDS (row pitch C + 1: lanes reading
// the same column hit distinct banks), each lane inserts its row's logits in index order into
// a sorted top-K list (the element carried down by an insertion is compared with the full order,
// index ascending on equal values), then the softmax over the k selected logits is summed with the xor tree the
// wave-per-token kernel's butterfly forms, so both kernels give identical results.
template <int K, bool kNaN>
__device__ __forceinline__ void insert_row(const float* rowl, int C, float (&tv)[K], int (&ti)[K]) {
  for (int c = 0; c < C; ++c) {
    float v = rowl[c];
    int i = c;
#pragma unroll
    for (int j = 0; j < K; ++j) {
      bool take;
      if (kNaN)
        take = ti[j] < 0 || better(v, i, tv[j], ti[j]);
      else  // a carried (displaced) element meets later equal values: index ascending
        take = ti[j] < 0 || v > tv[j] || (v == tv[j] && i < ti[j]);
      const float ov = tv[j];
      const int oi = ti[j];
      tv[j] = take ? v : ov;
      ti[j] = take ? i : oi;
      v = take ? ov : v;
      i = take ? oi : i;
    }
  }
}

// softmax over the k selected logits (sorted, tv[0] the largest) summed with the xor tree the
// wave-per-token kernel's butterfly forms, then the k ids and weights stored
template <int K>
__device__ __forceinline__ void topk_softmax_store(const float (&tv)[K], const int (&ti)[K], int k, int32_t* ids,
                                                   float* weights) {
  float ex[K], sm[K];
#pragma unroll
  for (int j = 0; j < K; ++j) {
    ex[j] = j < k ? expf(tv[j] - tv[0]) : 0.0f;
    sm[j] = ex[j];
  }
#pragma unroll
  for (int off = K / 2; off >= 1; off >>= 1) {
    float nx[K];
#pragma unroll
    for (int j = 0; j < K; ++j) nx[j] = sm[j] + sm[j ^ off];
#pragma unroll
    for (int j = 0; j < K; ++j) sm[j] = nx[j];
  }
#pragma unroll
  for (int j = 0; j < K; ++j)
    if (j < k) {
      ids[j] = ti[j];
      weights[j] = ex[j] / sm[0];
    }
}

template <int K>
__global__ void __launch_bounds__(64) route_topk_lanes_kernel(const float* __restrict__ logits, int T, int C, int k,
                                                              int32_t* __restrict__ ids,
                                                              float* __restrict__ weights) {
  extern __shared__ float rows[];  // [64][C + 1]
  const int lane = threadIdx.x;
  const int t0 = blockIdx.x * 64;
  const int nt = T - t0 < 64 ? T - t0 : 64;
  const int P = C + 1;
  const float* src = logits + (int64_t)t0 * C;
  bool nan_here = false;
  if ((C & 3) == 0) {  // 16-byte loads: consecutive lanes, consecutive logits
    for (int e = 4 * lane; e < nt * C; e += 256) {
      const float4 x = *reinterpret_cast<const float4*>(src + e);
      nan_here |= x.x != x.x || x.y != x.y || x.z != x.z || x.w != x.w;
      const int r = e / C, c = e - r * C;  // C % 4 == 0: the four stay in one row
      float* d = rows + r * P + c;
      d[0] = x.x;
      d[1] = x.y;
      d[2] = x.z;
      d[3] = x.w;
    }
  } else {
    for (int e = lane; e < nt * C; e += 64) {
      const float x = src[e];
      nan_here |= x != x;
      const int r = e / C, c = e - r * C;
      rows[r * P + c] = x;
    }
  }
  __syncthreads();
  if (lane >= nt) return;
  float tv[K];
  int ti[K];
#pragma unroll
  for (int j = 0; j < K; ++j) {
    tv[j] = 0.0f;
    ti[j] = -1;  // empty: below every logit
  }
  if (__ballot(nan_here) != 0)
    insert_row<K, true>(rows + lane * P, C, tv, ti);
  else
    insert_row<K, false>(rows + lane * P, C, tv, ti);
  topk_softmax_store<K>(tv, ti, k, ids + (int64_t)(t0 + lane) * k, weights + (int64_t)(t0 + lane) * k);
}

// ---- pack of per-sample route lists (the banked FFN: every token of sample b visits the
// clusters routes[rid[b], j], j < kmax, -1 = none, with weight route_w[rid[b]]; samples with
// active[b] == 0 visit none).  Produces the slots pack_pairs gives for the expanded (token, j)
// pairs: clusters in order, inside a cluster ascending token (sample, then position).
// Plan (one workgroup): per-cluster sample counts, offsets, and for each (b, j) the number of
// earlier samples routed to the same cluster; then one thread per pair writes its slot.
// With `fast` (the host checked that the tables fit in LDS) the plan keeps each sample's
// recipe (-1: routes nowhere) and an inverse table inv[r][c] = the j with routes[r][j] == c in
// LDS, so the counts run over all (b, j) at once and each cluster's ranks over the samples
// alone; a recipe that lists a cluster twice drops back to the (b, j) scan of the general
// plan.
// With `fused` (few pairs: the host checked that offsets and ranks fit in LDS beside the tables)
// the same workgroup then writes every pair's slot, as pack_routes_write_kernel does.
__global__ void __launch_bounds__(256) pack_routes_plan_kernel(const int64_t* __restrict__ rid,
                                                               const uint8_t* __restrict__ active, int B, int S,
                                                               const int32_t* __restrict__ routes, int R, int kmax,
                                                               int C, int32_t* __restrict__ offsets,
                                                               int32_t* __restrict__ base, int fast, int fused,
                                                               const float* __restrict__ route_w,
                                                               int32_t* __restrict__ tok_of_slot,
                                                               int32_t* __restrict__ pair_of_slot,
                                                               int32_t* __restrict__ slot_of_pair,
                                                               float* __restrict__ w_of_slot) {
  // cnt [C]; fast: inv [R * C], recipe [B]; fused: offsets [C + 1], ranks [B * kmax]
  extern __shared__ int32_t sh[];
  __shared__ int dup;
  int32_t* cnt = sh;
  int32_t* inv = sh + C;
  int32_t* rec = inv + (fast ? R * C : 0);
  int32_t* offs = rec + (fast ? B : 0);
  int32_t* ranks = offs + (C + 1);
  const int tid = threadIdx.x, lane = tid & 63;
  auto recipe_of = [&](int b) -> int {  // recipe of sample b, -1 when it routes nowhere
    const int64_t r = rid[b];
    return ((active && !active[b]) || r < 0 || r >= R) ? -1 : (int)r;
  };
  for (int c = tid; c < C; c += 256) cnt[c] = 0;
  if (fast) {
    for (int i = tid; i < R * C; i += 256) inv[i] = -1;
    for (int b = tid; b < B; b += 256) rec[b] = recipe_of(b);
    if (tid == 0) dup = 0;
  }
  __syncthreads();
  if (fast) {
    for (int i = tid; i < R * kmax; i += 256) {
      const int r = i / kmax, c = routes[i];
      if (c >= 0 && c < C && atomicExch(&inv[r * C + c], i - r * kmax) != -1) dup = 1;
    }
    for (int i = tid; i < B * kmax; i += 256) {
      const int b = i / kmax, r = rec[b];
      if (r < 0) continue;
      const int c = routes[r * kmax + (i - b * kmax)];
      if (c >= 0 && c < C) atomicAdd(&cnt[c], 1);  // integer counts: order-independent
    }
  } else {
    for (int b = tid; b < B; b += 256) {
      const int r = recipe_of(b);
      if (r < 0) continue;
      const int32_t* rr = routes + (int64_t)r * kmax;
      for (int j = 0; j < kmax; ++j) {
        const int c = rr[j];
        if (c >= 0 && c < C) atomicAdd(&cnt[c], 1);
      }
    }
  }
  __syncthreads();
  if (tid < 64) {  // exclusive prefix over the clusters, 64 at a time
    int carry = 0;
    for (int c0 = 0; c0 < C; c0 += 64) {
      const int c = c0 + lane;
      const int v = c < C ? cnt[c] : 0;
      int incl = v;
#pragma unroll
      for (int off = 1; off < 64; off <<= 1) {
        const int y = __shfl_up(incl, off, 64);
        if (lane >= off) incl += y;
      }
      if (c < C) {
        offsets[c] = (carry + incl - v) * S;
        if (fused) offs[c] = (carry + incl - v) * S;
      }
      carry += __shfl(incl, 63, 64);
    }
    if (lane == 0) {
      offsets[C] = carry * S;
      if (fused) offs[C] = carry * S;
    }
  }
  if (fast && !dup) {  // dup was settled before the barrier above
    for (int c = tid; c < C; c += 256) {  // samples in order: rank among the cluster's samples
      int r = 0;
      for (int b = 0; b < B; ++b) {
        const int rc = rec[b];
        if (rc < 0) continue;
        const int j = inv[rc * C + c];
        if (j >= 0) {
          if (fused) ranks[b * kmax + j] = r;
          base[b * kmax + j] = r++;
        }
      }
    }
  } else {
    for (int c = tid; c < C; c += 256) {
      int r = 0;
      for (int b = 0; b < B; ++b) {
        const int rc = recipe_of(b);
        if (rc < 0) continue;
        const int32_t* rr = routes + (int64_t)rc * kmax;
        for (int j = 0; j < kmax; ++j)
          if (rr[j] == c) {
            if (fused) ranks[b * kmax + j] = r;
            base[b * kmax + j] = r++;
          }
      }
    }
  }
  if (!fused) return;
  __syncthreads();
  const int P = B * S * kmax;
  for (int p = tid; p < P; p += 256) {
    const int t = p / kmax, j = p - t * kmax;
    const int b = t / S, s = t - b * S;
    const int rc = recipe_of(b);
    const int c = rc >= 0 ? routes[rc * kmax + j] : -1;
    if (c < 0 || c >= C) {
      if (slot_of_pair) slot_of_pair[p] = -1;
      continue;
    }
    const int slot = offs[c] + ranks[b * kmax + j] * S + s;
    if (tok_of_slot) tok_of_slot[slot] = t;
    if (pair_of_slot) pair_of_slot[slot] = p;
    if (slot_of_pair) slot_of_pair[p] = slot;
    if (w_of_slot) w_of_slot[slot] = route_w ? route_w[rc] : 1.0f;
  }
}

__global__ void __launch_bounds__(256) pack_routes_write_kernel(const int64_t* __restrict__ rid,
                                                                const uint8_t* __restrict__ active, int B, int S,
                                                                const int32_t* __restrict__ routes, int R, int kmax,
                                                                const float* __restrict__ route_w, int C,
                                                                const int32_t* __restrict__ offsets,
                                                                const int32_t* __restrict__ base,
                                                                int32_t* __restrict__ tok_of_slot,
                                                                int32_t* __restrict__ pair_of_slot,
                                                                int32_t* __restrict__ slot_of_pair,
                                                                float* __restrict__ w_of_slot) {
  const int P = B * S * kmax;
  const int p = blockIdx.x * 256 + threadIdx.x;
  if (p >= P) return;
  const int t = p / kmax, j = p - t * kmax;
  const int b = t / S, s = t - b * S;
  const bool on = !(active && !active[b]) && rid[b] >= 0 && rid[b] < R;  // unknown recipes route nowhere
  const int c = on ? routes[rid[b] * kmax + j] : -1;
  if (c < 0 || c >= C) {
    if (slot_of_pair) slot_of_pair[p] = -1;
    return;
  }
  const int slot = offsets[c] + base[b * kmax + j] * S + s;
  if (tok_of_slot) tok_of_slot[slot] = t;
  if (pair_of_slot) pair_of_slot[slot] = p;
  if (slot_of_pair) slot_of_pair[p] = slot;
  if (w_of_slot) w_of_slot[slot] = route_w ? route_w[rid[b]] : 1.0f;
}

template <typename OutT>
__device__ __forceinline__ void store8(OutT* dst, const float* v);

template <>
__device__ __forceinline__ void store8<float>(float* dst, const float* v) {
  reinterpret_cast<float4*>(dst)[0] = make_float4(v[0], v[1], v[2], v[3]);
  reinterpret_cast<float4*>(dst)[1] = make_float4(v[4], v[5], v[6], v[7]);
}

template <>
__device__ __forceinline__ void store8<bf16>(bf16* dst, const float* v) {
  uint4 o;
  o.x = pack_bf2(v[0], v[1]);
  o.y = pack_bf2(v[2], v[3]);
  o.z = pack_bf2(v[4], v[5]);
  o.w = pack_bf2(v[6], v[7]);
  *reinterpret_cast<uint4*>(dst) = o;
}

__device__ __forceinline__ void add8_bf16(float* acc, uint4 u) {
  const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    acc[2 * i] += __uint_as_float(w[i] << 16);
    acc[2 * i + 1] += __uint_as_float(w[i] & 0xffff0000u);
  }
}

// rows: [T*k, d] bf16 in pair order; extra: [T, d] bf16 or null; resid: [T, d] fp32 or null.
template <typename OutT>
__global__ void __launch_bounds__(256) combine_kernel(const bf16* __restrict__ rows, int T, int k, int d,
                                                      const int32_t* __restrict__ slot_of_pair,
                                                      const bf16* __restrict__ extra,
                                                      const float* __restrict__ resid,
                                                      OutT* __restrict__ out) {
  const int per_row = d / 8;
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= (int64_t)T * per_row) return;
  const int t = (int)(idx / per_row);
  const int c = (int)(idx % per_row) * 8;
  float acc[8];
  if (resid) {
    const float4 a = *reinterpret_cast<const float4*>(resid + (int64_t)t * d + c);
    const float4 b = *reinterpret_cast<const float4*>(resid + (int64_t)t * d + c + 4);
    acc[0] = a.x; acc[1] = a.y; acc[2] = a.z; acc[3] = a.w;
    acc[4] = b.x; acc[5] = b.y; acc[6] = b.z; acc[7] = b.w;
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i) acc[i] = 0.0f;
  }
  float sum[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) sum[i] = 0.0f;
  if (k <= 16) {
    // every pair's slot flag and row loaded before the (ascending j) sum: one memory latency
    uint4 v[16];
    bool use[16];
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      use[j] = j < k && (!slot_of_pair || slot_of_pair[(int64_t)t * k + j] >= 0);  // dropped pairs skip
      v[j] = j < k ? *reinterpret_cast<const uint4*>(rows + ((int64_t)t * k + j) * d + c) : make_uint4(0, 0, 0, 0);
    }
#pragma unroll
    for (int j = 0; j < 16; ++j)
      if (use[j]) add8_bf16(sum, v[j]);
  } else {
    for (int j = 0; j < k; ++j) {
      if (slot_of_pair && slot_of_pair[(int64_t)t * k + j] < 0) continue;  // dropped (invalid) pair
      add8_bf16(sum, *reinterpret_cast<const uint4*>(rows + ((int64_t)t * k + j) * d + c));
    }
  }
  if (extra) add8_bf16(sum, *reinterpret_cast<const uint4*>(extra + (int64_t)t * d + c));
#pragma unroll
  for (int i = 0; i < 8; ++i) acc[i] += sum[i];
  store8<OutT>(out + (int64_t)t * d + c, acc);
}

// Routing-weight gradient: weights are softmax over the k selected logits, so
// dlogit_j = w_j * (dw_j - sum_i w_i dw_i); everything else in the row is 0.
// One thread per logit (t, c): the per-token sum s = sum_j w_j dw_j in j order, then the
// gradient of the j that selected c (the last one, if an id repeats), zero elsewhere.  Rows
// are written whole and coalesced.
__global__ void __launch_bounds__(256) route_bwd_kernel(const int32_t* __restrict__ ids,
                                                        const float* __restrict__ w,
                                                        const float* __restrict__ dw_slot,
                                                        const int32_t* __restrict__ slot_of_pair, int T,
                                                        int C, int k, bf16* __restrict__ dlogits,
                                                        float* __restrict__ dlogits_f32) {
  const int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= (int64_t)T * C) return;
  const int64_t t = e / C;
  const int c = (int)(e - t * C);
  const int32_t* it = ids + t * k;
  const float* wt = w + t * k;
  const int32_t* st = slot_of_pair + t * k;
  float s = 0.0f, wsel = 0.0f, dsel = 0.0f;
  bool hit = false;
  if (k <= 16) {
    // the row's slots, weights and ids first, then the slot gradients: two memory latencies
    int sl[16], id[16];
    float wv[16], dv[16];
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      sl[j] = j < k ? st[j] : -1;
      wv[j] = j < k ? wt[j] : 0.0f;
      id[j] = j < k ? it[j] : -1;
    }
#pragma unroll
    for (int j = 0; j < 16; ++j) dv[j] = sl[j] >= 0 ? dw_slot[sl[j]] : 0.0f;
#pragma unroll
    for (int j = 0; j < 16; ++j)
      if (j < k) {
        s += wv[j] * dv[j];
        if (id[j] == c) {
          hit = true;
          wsel = wv[j];
          dsel = dv[j];
        }
      }
  } else {
    for (int j = 0; j < k; ++j) {
      const int slot = st[j];
      const float dw = slot >= 0 ? dw_slot[slot] : 0.0f;
      const float wj = wt[j];
      s += wj * dw;
      if (it[j] == c) {
        hit = true;
        wsel = wj;
        dsel = dw;
      }
    }
  }
  const float g = hit ? wsel * (dsel - s) : 0.0f;
  if (dlogits) dlogits[e] = f2bf(g);
  if (dlogits_f32) dlogits_f32[e] = g;
}

// ---- router GEMM + top-k + pack in two launches (C % 32 == 0, C <= 128, d % 64 == 0) ----
//
// route_gemm_topk: one workgroup per 32 tokens: router logits on MFMA, the top-k and softmax of
// route_topk (same selections and weights on the same logits), and the block's cluster counts
// to hist[block][C].
// pack_place: one workgroup per 32 tokens (one route block): cluster offsets and the block's
// base per cluster from the histograms (integer sums), then per 256-pair chunk one ballot per
// cluster and wave ranks the pairs; slots follow cluster, then ascending pair index, as
// rte_pack_index.
constexpr int kRouteTok = 32;     // tokens per route_gemm_topk block
constexpr int kPlaceTok = 32;     // tokens per pack_place block (one route block)

__device__ __forceinline__ f32x16_v rt_mfma(bf16x8_v a, bf16x8_v b, f32x16_v c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

// 64-bit selection keys whose unsigned order is better(): high word the float's order-preserving
// bit pattern (every NaN maximal, -0 as +0), low word ~index (ties: lower index first); an empty
// entry is key 0, below every logit.
__device__ __forceinline__ uint64_t rt_key(float v, int i) {
  const uint32_t u = __float_as_uint(v == 0.0f ? 0.0f : v);
  const uint32_t hi = v != v ? 0xffffffffu : ((u & 0x80000000u) ? ~u : (u | 0x80000000u));
  return ((uint64_t)hi << 32) | (uint64_t)(~(uint32_t)i);
}

__device__ __forceinline__ float rt_key_val(uint64_t key) {
  const uint32_t hi = (uint32_t)(key >> 32);
  if (hi == 0xffffffffu) return __uint_as_float(0x7fc00000u);
  return __uint_as_float((hi & 0x80000000u) ? (hi & 0x7fffffffu) : ~hi);
}

__device__ __forceinline__ int rt_key_idx(uint64_t key) { return (int)~(uint32_t)key; }

__device__ __forceinline__ uint64_t rt_shfl_xor(uint64_t v, int off) {
  const uint32_t lo = __shfl_xor((uint32_t)v, off, 64), hi = __shfl_xor((uint32_t)(v >> 32), off, 64);
  return ((uint64_t)hi << 32) | lo;
}

// keys sorted descending by a bitonic network (N a power of two)
template <int N>
__device__ __forceinline__ void rt_sort(uint64_t (&key)[N]) {
#pragma unroll
  for (int size = 2; size <= N; size <<= 1)
#pragma unroll
    for (int stride = size / 2; stride > 0; stride >>= 1)
#pragma unroll
      for (int i = 0; i < N; ++i) {
        const int j = i ^ stride;
        if (j > i) {
          const uint64_t x = key[i], y = key[j];
          const bool sw = ((i & size) == 0) ? (y > x) : (x > y);
          key[i] = sw ? y : x;
          key[j] = sw ? x : y;
        }
      }
}

template <int CB, int K>
__global__ void __launch_bounds__(256) route_gemm_topk_kernel(const bf16* __restrict__ x, int T, int d,
                                                              const bf16* __restrict__ wr, int k,
                                                              int32_t* __restrict__ ids, float* __restrict__ weights,
                                                              int32_t* __restrict__ hist, float* __restrict__ logits) {
  constexpr int C = 32 * CB;
  constexpr int PER = C / 8;  // logits per lane in the top-k
  // row pitch 40 floats: the two half-waves' stores (rows 4 apart) and the top-k phase's reads
  // (8 clusters x 8 tokens per wave) each cover 64 distinct banks
  __shared__ float part[4][C][kRouteTok + 8];
  __shared__ int hs[C];
  const int tid = threadIdx.x, w = tid >> 6, lane = tid & 63, h = lane >> 5, l32 = lane & 31;
  const int t0 = blockIdx.x * kRouteTok;
  for (int c = tid; c < C; c += 256) hs[c] = 0;
  {
    f32x16_v acc[CB];
#pragma unroll
    for (int cb = 0; cb < CB; ++cb)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[cb][r] = 0.0f;
    const int tl = t0 + l32 < T ? t0 + l32 : T - 1;
    const int kq = d / 4;  // a multiple of 16
    const bf16* xr = x + (int64_t)tl * d + w * kq + 8 * h;
    const bf16* wrow = wr + (int64_t)l32 * d + w * kq + 8 * h;
    for (int k0 = 0; k0 < kq; k0 += 128) {
      bf16x8_v b[8], a[8][CB];
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int kk = k0 + 16 * j < kq ? k0 + 16 * j : 0;  // a step past the quarter re-reads step 0, skipped
        b[j] = __builtin_bit_cast(bf16x8_v, *reinterpret_cast<const uint4*>(xr + kk));
#pragma unroll
        for (int cb = 0; cb < CB; ++cb)
          a[j][cb] = __builtin_bit_cast(bf16x8_v, *reinterpret_cast<const uint4*>(wrow + (int64_t)cb * 32 * d + kk));
      }
#pragma unroll
      for (int j = 0; j < 8; ++j)
        if (k0 + 16 * j < kq) {
#pragma unroll
          for (int cb = 0; cb < CB; ++cb) acc[cb] = rt_mfma(a[j][cb], b[j], acc[cb]);
        }
    }
    // register r of lane: cluster 32 cb + 8 (r / 4) + 4 h + r % 4, token l32
#pragma unroll
    for (int cb = 0; cb < CB; ++cb)
#pragma unroll
      for (int r = 0; r < 16; ++r) part[w][cb * 32 + 8 * (r >> 2) + 4 * h + (r & 3)][l32] = acc[cb][r];
  }
  __syncthreads();
  const int tt = tid >> 3, s = tid & 7, t = t0 + tt;
  float v[PER];
#pragma unroll
  for (int i = 0; i < PER; ++i) {
    const int c = s + 8 * i;
    v[i] = ((part[0][c][tt] + part[1][c][tt]) + part[2][c][tt]) + part[3][c][tt];
  }
  if (logits != nullptr && t < T) {
#pragma unroll
    for (int i = 0; i < PER; ++i) logits[(int64_t)t * C + s + 8 * i] = v[i];
  }
  // the lane's PER logits sorted, its best K kept (empty keys past PER), then the eight lanes'
  // lists merged pairwise
  uint64_t key[PER];
#pragma unroll
  for (int i = 0; i < PER; ++i) key[i] = rt_key(v[i], s + 8 * i);
  rt_sort<PER>(key);
  uint64_t top[K];
#pragma unroll
  for (int j = 0; j < K; ++j) top[j] = j < PER ? key[j < PER ? j : 0] : 0ull;
#pragma unroll
  for (int off = 1; off < 8; off <<= 1) {
    uint64_t m[K];
#pragma unroll
    for (int j = 0; j < K; ++j) {
      const uint64_t o = rt_shfl_xor(top[K - 1 - j], off);
      m[j] = top[j] > o ? top[j] : o;
    }
#pragma unroll
    for (int o2 = K / 2; o2 >= 1; o2 >>= 1)
#pragma unroll
      for (int j = 0; j < K; ++j)
        if ((j & o2) == 0) {
          const uint64_t x = m[j], y = m[j + o2];
          m[j] = x > y ? x : y;
          m[j + o2] = x > y ? y : x;
        }
#pragma unroll
    for (int j = 0; j < K; ++j) top[j] = m[j];
  }
  float tv[K];
  int ti[K];
#pragma unroll
  for (int j = 0; j < K; ++j) {
    tv[j] = rt_key_val(top[j]);
    ti[j] = rt_key_idx(top[j]);
  }
  if (s == 0 && t < T) {
    topk_softmax_store<K>(tv, ti, k, ids + (int64_t)t * k, weights + (int64_t)t * k);
#pragma unroll
    for (int j = 0; j < K; ++j)
      if (j < k) atomicAdd(&hs[ti[j]], 1);  // integer counts: order-free
  }
  __syncthreads();
  for (int c = tid; c < C; c += 256) hist[(int64_t)blockIdx.x * C + c] = hs[c];
}

template <int C, int K>
__global__ void __launch_bounds__(256) pack_place_kernel(const int32_t* __restrict__ ids, const float* __restrict__ w,
                                                         int T, int k, const int32_t* __restrict__ hist, int nblk,
                                                         int32_t* __restrict__ offsets,
                                                         int32_t* __restrict__ tok_of_slot,
                                                         int32_t* __restrict__ pair_of_slot,
                                                         int32_t* __restrict__ slot_of_pair,
                                                         float* __restrict__ w_of_slot) {
  constexpr int VPR = C / 4;          // 16-byte vectors per histogram row
  constexpr int RPP = 256 / VPR;      // histogram rows per pass of the 256 threads
  constexpr int MW = C / 64 > 0 ? C / 64 : 1;  // 64-bit route-mask words per token
  constexpr int SEG = kPlaceTok / 4;  // tokens per segment mask (one per wave, at most 32)
  __shared__ int sb[RPP][C], st[RPP][C];
  __shared__ int base[C];
  __shared__ unsigned long long mask[kPlaceTok][MW];
  __shared__ uint32_t segbits[4][C];  // per cluster, which tokens of each 32-token segment route to it
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int t0 = blockIdx.x * kPlaceTok;
  const int first = blockIdx.x * (kPlaceTok / kRouteTok);  // this block's first route block
  // every global load first: the token's ids and weights (threads < kPlaceTok), the histograms
  const int tok = t0 + tid;
  const bool own = tid < kPlaceTok && tok < T;
  int cs[K];
  float ws[K];
#pragma unroll
  for (int j = 0; j < K; ++j) {
    cs[j] = (own && j < k) ? ids[(int64_t)tok * k + j] : -1;
    ws[j] = (own && j < k) ? w[(int64_t)tok * k + j] : 0.0f;
  }
  {
    // thread: clusters 4 (tid % VPR) .. +3 of rows tid / VPR + RPP i
    const int c0 = 4 * (tid % VPR), r0 = tid / VPR;
    int4 bef = make_int4(0, 0, 0, 0), tot = make_int4(0, 0, 0, 0);
#pragma unroll 16
    for (int b = r0; b < nblk; b += RPP) {
      const int4 v = *reinterpret_cast<const int4*>(hist + (int64_t)b * C + c0);
      tot.x += v.x;
      tot.y += v.y;
      tot.z += v.z;
      tot.w += v.w;
      if (b < first) {
        bef.x += v.x;
        bef.y += v.y;
        bef.z += v.z;
        bef.w += v.w;
      }
    }
    *reinterpret_cast<int4*>(&sb[r0][c0]) = bef;
    *reinterpret_cast<int4*>(&st[r0][c0]) = tot;
  }
  // the route mask of each of the block's tokens (its k clusters are distinct: a top-k)
  if (tid < kPlaceTok) {
    unsigned long long m[MW];
#pragma unroll
    for (int q = 0; q < MW; ++q) m[q] = 0ull;
#pragma unroll
    for (int j = 0; j < K; ++j)
      if (cs[j] >= 0) {
#pragma unroll
        for (int q = 0; q < MW; ++q)
          if ((cs[j] >> 6) == q) m[q] |= 1ull << (cs[j] & 63);
      }
#pragma unroll
    for (int q = 0; q < MW; ++q) mask[tid][q] = m[q];
  }
  __syncthreads();
  if (wave == 0) {  // exclusive scan of the cluster totals: lane l owns clusters [2 l, 2 l + 2)
    int v[2], b[2], sum = 0;
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int c = 2 * lane + u;
      v[u] = 0;
      b[u] = 0;
      if (c < C) {
#pragma unroll
        for (int q = 0; q < RPP; ++q) {
          v[u] += st[q][c];
          b[u] += sb[q][c];
        }
      }
      sum += v[u];
    }
    int inc = sum;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const int y = __shfl_up(inc, off, 64);
      if (lane >= off) inc += y;
    }
    int s = inc - sum;
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int c = 2 * lane + u;
      if (c < C) {
        base[c] = s + b[u];
        if (blockIdx.x == 0) offsets[c] = s;
      }
      s += v[u];
    }
    if (blockIdx.x == 0 && lane == 63) offsets[C] = s;
  }
  // wave w: per cluster, the bit mask of the tokens of segment w routed to it (independent
  // broadcast reads of the route masks)
  for (int c = lane; c < C; c += 64) {
    uint32_t bits = 0u;
#pragma unroll
    for (int r = 0; r < SEG; ++r) bits |= (uint32_t)((mask[wave * SEG + r][c >> 6] >> (c & 63)) & 1ull) << r;
    segbits[wave][c] = bits;
  }
  __syncthreads();
  // one thread per token writes its k slots: cluster base + earlier segments + earlier tokens
  if (own) {
    const int sg = tid / SEG, r = tid % SEG;
    const uint32_t below = (1u << r) - 1u;
#pragma unroll
    for (int j = 0; j < K; ++j)
      if (j < k) {
        const int64_t p = (int64_t)tok * k + j;
        const int c = cs[j];
        int slot = base[c] + __popc(segbits[sg][c] & below);
        for (int q = 0; q < sg; ++q) slot += __popc(segbits[q][c]);
        tok_of_slot[slot] = tok;
        pair_of_slot[slot] = (int32_t)p;
        slot_of_pair[p] = slot;
        w_of_slot[slot] = ws[j];
      }
  }
}


}  // namespace

int route_topk(const float* logits, int T, int C, int k, int32_t* ids, float* weights, hipStream_t s) {
  RTE_REQUIRE(T >= 0 && C >= 1 && C <= 64 * kMaxPerLane, "route_topk: C must be in [1, 1024]");
  RTE_REQUIRE(k >= 1 && k <= 16 && k <= C, "route_topk: k must be in [1, min(16, C)]");
  if (T == 0) return 0;
  if (T >= 16384 && C <= 128) {
    const size_t lds = (size_t)64 * (C + 1) * sizeof(float);
    if (k <= 8)
      hipLaunchKernelGGL(route_topk_lanes_kernel<8>, dim3((T + 63) / 64), dim3(64), lds, s, logits, T, C, k, ids,
                         weights);
    else
      hipLaunchKernelGGL(route_topk_lanes_kernel<16>, dim3((T + 63) / 64), dim3(64), lds, s, logits, T, C, k, ids,
                         weights);
    return check_launch("route_topk");
  }
  const dim3 grid((T + 3) / 4);
  if (C <= 64)
    hipLaunchKernelGGL(route_topk_rank_kernel<1>, grid, dim3(256), 0, s, logits, T, C, k, ids, weights);
  else if (C <= 128)
    hipLaunchKernelGGL(route_topk_rank_kernel<2>, grid, dim3(256), 0, s, logits, T, C, k, ids, weights);
  else
    hipLaunchKernelGGL(route_topk_kernel, grid, dim3(256), 0, s, logits, T, C, k, ids, weights);
  return check_launch("route_topk");
}

// 256-pair sub-chunks per pack block: one up to 64 Ki pairs, growing to 16 for large P
int pack_nsub(int P) {
  int64_t n = (int64_t)P / (kPackChunk * 256);
  if (n < 1) n = 1;
  if (n > 16) n = 16;
  return (int)n;
}

int pack_blocks(int P) {
  const int64_t per = (int64_t)pack_nsub(P) * kPackChunk;
  return (int)(((int64_t)P + per - 1) / per);
}

size_t pack_workspace_bytes(int P, int C) {
  const int nblk = pack_blocks(P);
  return (size_t)C * (size_t)(nblk > 0 ? nblk : 1) * sizeof(int32_t);
}

int pack_pairs(const int32_t* cl, int P, int C, int k, const float* w, int32_t* offsets,
               int32_t* tok_of_slot, int32_t* pair_of_slot, int32_t* slot_of_pair, float* w_of_slot,
               int32_t* invalid, void* ws, size_t ws_bytes, hipStream_t s) {
  RTE_REQUIRE(P >= 0 && C >= 1 && k >= 1, "pack: bad sizes");
  RTE_REQUIRE(ws_bytes >= pack_workspace_bytes(P, C), "pack: workspace too small (%zu < %zu)", ws_bytes,
              pack_workspace_bytes(P, C));
  const int nsub = pack_nsub(P), nblk = pack_blocks(P);
  int32_t* hist = static_cast<int32_t*>(ws);
  if (nblk == 0) return fill_i32(offsets, 0, C + 1, s);
  {
    hipLaunchKernelGGL(pack_count_kernel, dim3(nblk), dim3(kPackChunk), C * sizeof(int32_t), s, cl, P, C, nsub,
                       hist, nblk, invalid);
    RTE_TRY(check_launch("pack_count"));
  }
  hipLaunchKernelGGL(pack_scan_kernel, dim3(1), dim3(1024), 0, s, hist, C, nblk, offsets, P);
  RTE_TRY(check_launch("pack_scan"));
  {
    hipLaunchKernelGGL(pack_scatter_kernel, dim3(nblk), dim3(kPackChunk), C * sizeof(int32_t), s, cl, P, C, nsub,
                       k, hist, nblk, w, tok_of_slot, pair_of_slot, slot_of_pair, w_of_slot);
    RTE_TRY(check_launch("pack_scatter"));
  }
  return 0;
}

size_t route_pack_workspace_bytes(int T, int C) {
  const int nblk = (T + kRouteTok - 1) / kRouteTok;
  return (size_t)(nblk > 0 ? nblk : 1) * (size_t)(C > 0 ? C : 1) * sizeof(int32_t);
}

int route_pack(const bf16* x, int T, int d, const bf16* wr, int C, int k, int32_t* ids, float* weights,
               int32_t* offsets, int32_t* tok_of_slot, int32_t* pair_of_slot, int32_t* slot_of_pair,
               float* w_of_slot, float* logits, void* ws, size_t ws_bytes, hipStream_t s) {
  RTE_REQUIRE(C == 32 || C == 64 || C == 128, "route_pack: C must be 32, 64 or 128 (got %d)", C);
  RTE_REQUIRE(k >= 1 && k <= 16 && k <= C, "route_pack: k must be in [1, min(16, C)]");
  RTE_REQUIRE(d >= 64 && d % 64 == 0, "route_pack: d must be a positive multiple of 64");
  RTE_REQUIRE(T >= 0 && (int64_t)T * k < ((int64_t)1 << 31), "route_pack: too many pairs");
  if (T == 0) return fill_i32(offsets, 0, C + 1, s);
  RTE_REQUIRE(ws != nullptr && ws_bytes >= route_pack_workspace_bytes(T, C), "route_pack: workspace too small");
  const int nblk = (T + kRouteTok - 1) / kRouteTok;
  int32_t* hist = static_cast<int32_t*>(ws);
#define RTE_ROUTE_GEMM(CB, K)                                                                                 \
  hipLaunchKernelGGL((route_gemm_topk_kernel<CB, K>), dim3(nblk), dim3(256), 0, s, x, T, d, wr, k, ids, weights, \
                     hist, logits)
#define RTE_PACK_PLACE(C, K)                                                                                     \
  hipLaunchKernelGGL((pack_place_kernel<C, K>), grid, dim3(256), 0, s, ids, weights, T, k, hist, nblk, offsets, \
                     tok_of_slot, pair_of_slot, slot_of_pair, w_of_slot)
  const dim3 grid((T + kPlaceTok - 1) / kPlaceTok);
  if (k <= 8) {
    if (C == 32) RTE_ROUTE_GEMM(1, 8);
    else if (C == 64) RTE_ROUTE_GEMM(2, 8);
    else RTE_ROUTE_GEMM(4, 8);
    RTE_TRY(check_launch("route_gemm_topk"));
    if (C == 32) RTE_PACK_PLACE(32, 8);
    else if (C == 64) RTE_PACK_PLACE(64, 8);
    else RTE_PACK_PLACE(128, 8);
  } else {
    if (C == 32) RTE_ROUTE_GEMM(1, 16);
    else if (C == 64) RTE_ROUTE_GEMM(2, 16);
    else RTE_ROUTE_GEMM(4, 16);
    RTE_TRY(check_launch("route_gemm_topk"));
    if (C == 32) RTE_PACK_PLACE(32, 16);
    else if (C == 64) RTE_PACK_PLACE(64, 16);
    else RTE_PACK_PLACE(128, 16);
  }
#undef RTE_ROUTE_GEMM
#undef RTE_PACK_PLACE
  return check_launch("pack_place");
}

int combine_rows(const bf16* rows, int T, int k, int d, const int32_t* slot_of_pair, const bf16* extra,
                 const float* resid, void* out,
                 int out_f32, hipStream_t s) {
  RTE_REQUIRE(d % 8 == 0, "combine: d must be a multiple of 8");
  RTE_REQUIRE(k >= 0, "combine: k must be >= 0");
  const int64_t n = (int64_t)T * (d / 8);
  if (n == 0) return 0;
  const dim3 grid((unsigned)((n + 255) / 256));
  if (out_f32)
    hipLaunchKernelGGL(combine_kernel<float>, grid, dim3(256), 0, s, rows, T, k, d, slot_of_pair, extra, resid,
                       static_cast<float*>(out));
  else
    hipLaunchKernelGGL(combine_kernel<bf16>, grid, dim3(256), 0, s, rows, T, k, d, slot_of_pair, extra, resid,
                       static_cast<bf16*>(out));
  return check_launch("combine");
}

int route_bwd(const int32_t* ids, const float* w, const float* dw_slot, const int32_t* slot_of_pair, int T,
              int C, int k, bf16* dlogits, float* dlogits_f32, hipStream_t s) {
  RTE_REQUIRE(k >= 1 && k <= 16, "route_bwd: k must be in [1, 16]");
  if (T == 0) return 0;
  const int64_t n = (int64_t)T * C;
  hipLaunchKernelGGL(route_bwd_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, ids, w, dw_slot,
                     slot_of_pair, T, C, k, dlogits, dlogits_f32);
  return check_launch("route_bwd");
}

size_t pack_routes_workspace_bytes(int B, int kmax) {
  return (size_t)(B > 0 ? B : 1) * (kmax > 0 ? kmax : 1) * sizeof(int32_t);
}

int pack_routes(const int64_t* rid, const uint8_t* active, int B, int S, const int32_t* routes, int R, int kmax,
                const float* route_w, int C, int32_t* offsets, int32_t* tok_of_slot, int32_t* pair_of_slot,
                int32_t* slot_of_pair, float* w_of_slot, void* ws, size_t ws_bytes, hipStream_t s) {
  RTE_REQUIRE(B >= 0 && S >= 1 && R >= 1 && kmax >= 1 && C >= 1 && C <= 16384, "pack_routes: bad sizes");
  RTE_REQUIRE((int64_t)B * S * kmax < ((int64_t)1 << 31), "pack_routes: too many pairs");
  RTE_REQUIRE(ws && ws_bytes >= pack_routes_workspace_bytes(B, kmax), "pack_routes: workspace too small");
  if (B == 0) return fill_i32(offsets, 0, C + 1, s);
  int32_t* base = static_cast<int32_t*>(ws);
  const size_t fast_lds = ((size_t)C + (size_t)R * C + (size_t)B) * sizeof(int32_t);
  const int fast = fast_lds <= 65536 ? 1 : 0;
  const size_t plan_lds = fast ? fast_lds : (size_t)C * sizeof(int32_t);
  const int P = B * S * kmax;
  // few pairs: the plan's workgroup writes the slots too (one launch)
  const size_t fused_lds = plan_lds + ((size_t)C + 1 + (size_t)B * kmax) * sizeof(int32_t);
  const int fused = (P <= 16384 && fused_lds <= 65536) ? 1 : 0;
  hipLaunchKernelGGL(pack_routes_plan_kernel, dim3(1), dim3(256), fused ? fused_lds : plan_lds, s, rid, active, B, S,
                     routes, R, kmax, C, offsets, base, fast, fused, route_w, tok_of_slot, pair_of_slot, slot_of_pair,
                     w_of_slot);
  RTE_TRY(check_launch("pack_routes_plan"));
  if (fused) return 0;
  hipLaunchKernelGGL(pack_routes_write_kernel, dim3((P + 255) / 256), dim3(256), 0, s, rid, active, B, S, routes, R,
                     kmax, route_w, C, offsets, base, tok_of_slot, pair_of_slot, slot_of_pair, w_of_slot);
  return check_launch("pack_routes_write");
}

}  // namespace rte
