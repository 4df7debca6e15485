// Token cross-entropy over full-vocabulary logits (rte/models.py:73-75,
// rte/kernels/reference.py:146-147), forward and backward, one wave64 per row.
//
//  ce_fwd : lse[t] = logsumexp(logits[t, :]), loss[t] = lse[t] - logits[t, target[t]]
//           (target < 0: ignored row, loss 0)
//  ce_bwd : dlogits[t, v] = g[t] * (softmax[t, v] - [v == target]) + extra[t, v]
//           written as bf16 for the LM-head backward GEMMs (the fp32->bf16 cast fused)
#include "common.hpp"

namespace rte {

namespace {

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

__global__ void __launch_bounds__(256) ce_fwd_kernel(const float* __restrict__ logits, int64_t ld, int T, int V,
                                                     const int64_t* __restrict__ targets, float* __restrict__ loss,
                                                     float* __restrict__ lse_out) {
  const int lane = threadIdx.x & 63;
  const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= T) return;
  const float* row = logits + (int64_t)t * ld;
  float mx = -INFINITY;
  for (int c = lane * 4; c < V; c += 256) {
    if (c + 4 <= V) {
      const float4 v = *reinterpret_cast<const float4*>(row + c);
      mx = fmaxf(mx, fmaxf(fmaxf(v.x, v.y), fmaxf(v.z, v.w)));
    } else {
      for (int i = c; i < V; ++i) mx = fmaxf(mx, row[i]);
    }
  }
  mx = wave_max(mx);
  float s = 0.0f;
  for (int c = lane * 4; c < V; c += 256) {
    if (c + 4 <= V) {
      const float4 v = *reinterpret_cast<const float4*>(row + c);
      s += __expf(v.x - mx) + __expf(v.y - mx) + __expf(v.z - mx) + __expf(v.w - mx);
    } else {
      for (int i = c; i < V; ++i) s += __expf(row[i] - mx);
    }
  }
  s = wave_sum(s);
  if (lane == 0) {
    const float lse = mx + logf(s);
    const int64_t tg = targets[t];
    lse_out[t] = lse;
    loss[t] = (tg >= 0 && tg < V) ? lse - row[tg] : 0.0f;
  }
}

__global__ void __launch_bounds__(256) ce_bwd_kernel(const float* __restrict__ logits, int64_t ld, int T, int V,
                                                     const int64_t* __restrict__ targets,
                                                     const float* __restrict__ lse, const float* __restrict__ g,
                                                     const float* __restrict__ extra, bf16* __restrict__ dlogits) {
  const int lane = threadIdx.x & 63;
  const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= T) return;
  const float* row = logits + (int64_t)t * ld;
  const float* ex = extra ? extra + (int64_t)t * V : nullptr;
  bf16* out = dlogits + (int64_t)t * V;
  const int64_t tg = targets[t];
  const bool valid = tg >= 0 && tg < V;
  const float gt = (g && valid) ? g[t] : 0.0f;
  const float l = lse[t];
  for (int c = lane * 4; c < V; c += 256) {
    const int n = c + 4 <= V ? 4 : V - c;
    float d[4];
    if (n == 4) {
      const float4 x = *reinterpret_cast<const float4*>(row + c);
      const float xs[4] = {x.x, x.y, x.z, x.w};
      float4 e4 = make_float4(0.f, 0.f, 0.f, 0.f);
      if (ex) e4 = *reinterpret_cast<const float4*>(ex + c);
      const float es[4] = {e4.x, e4.y, e4.z, e4.w};
#pragma unroll
      for (int i = 0; i < 4; ++i) d[i] = gt * (__expf(xs[i] - l) - (c + i == tg ? 1.0f : 0.0f)) + es[i];
    } else {
      for (int i = 0; i < n; ++i) {
        const int v = c + i;
        d[i] = gt * (__expf(row[v] - l) - (v == tg ? 1.0f : 0.0f)) + (ex ? ex[v] : 0.0f);
      }
    }
    if (n == 4) {
      uint2 o;
      o.x = (uint32_t)f2bf(d[0]) | ((uint32_t)f2bf(d[1]) << 16);
      o.y = (uint32_t)f2bf(d[2]) | ((uint32_t)f2bf(d[3]) << 16);
      *reinterpret_cast<uint2*>(out + c) = o;
    } else {
      for (int i = 0; i < n; ++i) out[c + i] = f2bf(d[i]);
    }
  }
}

}  // namespace

int ce_fwd(const float* logits, int64_t ld, int T, int V, const int64_t* targets, float* loss, float* lse,
           hipStream_t s) {
  RTE_REQUIRE(V >= 1 && ld >= V && ld % 4 == 0, "ce_fwd: logits row stride must be >= V and a multiple of 4");
  RTE_REQUIRE(((uintptr_t)logits & 15) == 0, "ce_fwd: logits must be 16-byte aligned");
  if (T == 0) return 0;
  hipLaunchKernelGGL(ce_fwd_kernel, dim3((T + 3) / 4), dim3(256), 0, s, logits, ld, T, V, targets, loss, lse);
  return check_launch("ce_fwd");
}

int ce_bwd(const float* logits, int64_t ld, int T, int V, const int64_t* targets, const float* lse, const float* g,
           const float* extra, bf16* dlogits, hipStream_t s) {
  RTE_REQUIRE(V % 4 == 0 && ld % 4 == 0, "ce_bwd: V and the row stride must be multiples of 4");
  RTE_REQUIRE(((uintptr_t)logits & 15) == 0 && ((uintptr_t)extra & 15) == 0 && ((uintptr_t)dlogits & 7) == 0,
              "ce_bwd: misaligned buffers");
  if (T == 0) return 0;
  hipLaunchKernelGGL(ce_bwd_kernel, dim3((T + 3) / 4), dim3(256), 0, s, logits, ld, T, V, targets, lse, g, extra,
                     dlogits);
  return check_launch("ce_bwd");
}

}  // namespace rte
