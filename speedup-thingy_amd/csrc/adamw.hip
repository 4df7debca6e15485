// Fused AdamW step over every parameter of a model, with the per-group gradient / parameter
// norms the trainer reports (rte/training.py:385-443) and optional gradient clipping
// (torch.nn.utils.clip_grad_norm_, rte/training.py:456-462), in three launches:
//
//   norms    : one workgroup per chunk of a tensor: partial sum(g^2), sum(p^2)
//   finalize : one workgroup: per-tensor sums (chunks in order), per-metric-group sums (tensors
//              in order), clip coefficient, metrics, step counters and bias corrections
//   update   : one workgroup per chunk: torch AdamW (decoupled decay p -= lr wd p, moments
//              m = b1 m + (1 - b1) g, v = b2 v + (1 - b2) g^2, p -= lr / (1 - b1^t) m /
//              (sqrt(v) / sqrt(1 - b2^t) + eps)), skipped entirely when found_inf is set
//
// Without clipping the update does not depend on the norms, so the update kernel also forms
// the per-chunk partial norms (of the gradient and of the parameter before it changes) and the
// finish runs last: two launches and one pass over p and g.
//
// Tensors are described by a device table (one row per parameter, pointers and sizes) and a
// block table (tensor, chunk) built once per layout, so the same three launches serve any
// parameter set and can be captured in a graph.
#include "common.hpp"

namespace rte {

namespace {

constexpr int kChunk = 4096;  // elements per workgroup chunk (256 threads x 16)

struct AdamRow {
  int64_t p, g, m, v, step;  // pointers (g == 0: no gradient this step -> untouched)
  int64_t numel;
  int64_t group;             // optimizer group
  int64_t metric_mask;       // bit j: tensor belongs to metric group j
};

__device__ __forceinline__ float bsum(float v, float* red) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  __syncthreads();
  if (lane == 0) red[w] = v;
  __syncthreads();
  float t = 0.0f;
  for (int i = 0; i < (int)(blockDim.x >> 6); ++i) t += red[i];
  return t;
}

__global__ void __launch_bounds__(256) adamw_norms_kernel(const AdamRow* __restrict__ rows,
                                                          const int32_t* __restrict__ blk, float* __restrict__ part) {
  __shared__ float red[4];
  const int b = blockIdx.x;
  const AdamRow r = rows[blk[2 * b]];
  const int64_t off = (int64_t)blk[2 * b + 1] * kChunk;
  const float* p = reinterpret_cast<const float*>(r.p);
  const float* g = reinterpret_cast<const float*>(r.g);
  float sg = 0.0f, sp = 0.0f;
  for (int64_t i = off + threadIdx.x; i < off + kChunk && i < r.numel; i += 256) {
    const float x = p[i];
    sp += x * x;
    if (g) {
      const float y = g[i];
      sg += y * y;
    }
  }
  sg = bsum(sg, red);
  sp = bsum(sp, red);
  if (threadIdx.x == 0) {
    part[2 * b] = sg;
    part[2 * b + 1] = sp;
  }
}

// hyper per optimizer group (float64): lr, beta1, beta2, eps, weight_decay.
// scal (out): scal[4 * G] = clip coefficient, scal[4 * G + 1] = 1 when the update runs.
// metrics (out): per metric group j: grad_norm (after clipping), update_ratio = lr_j gn / max(pn, 1e-12).
__global__ void __launch_bounds__(1024) adamw_finalize_kernel(const AdamRow* __restrict__ rows, int nt,
                                                              const int32_t* __restrict__ first_blk,
                                                              const float* __restrict__ part,
                                                              const double* __restrict__ hyper, int G,
                                                              const int32_t* __restrict__ metric_lr_group, int M,
                                                              float clip_max, const float* __restrict__ found_inf,
                                                              float* __restrict__ tsum, float* __restrict__ scal,
                                                              float* __restrict__ metrics) {
  __shared__ double acc[64][2];
  __shared__ double gtot;
  extern __shared__ double ts[];  // [nt][2] per-tensor sums, then [nt] metric masks
  int64_t* tmask = reinterpret_cast<int64_t*>(ts + 2 * nt);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
  // per-tensor sums: one wave per tensor, lanes stride its chunks, then a fixed xor tree
  for (int i = wave; i < nt; i += nw) {
    double sg = 0.0, sp = 0.0;
    for (int b = first_blk[i] + lane; b < first_blk[i + 1]; b += 64) {
      sg += part[2 * b];
      sp += part[2 * b + 1];
    }
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
      sg += __shfl_xor(sg, off, 64);
      sp += __shfl_xor(sp, off, 64);
    }
    if (lane == 0) {
      ts[2 * i] = sg;
      ts[2 * i + 1] = sp;
      tmask[i] = rows[i].metric_mask;
      tsum[2 * i] = (float)sg;
      tsum[2 * i + 1] = (float)sp;
    }
  }
  __syncthreads();
  // metric group j (thread j) and the global total (thread 64) sum the tensors in order
  if (threadIdx.x < M) {
    const int j = threadIdx.x;
    double sg = 0.0, sp = 0.0;
    for (int i = 0; i < nt; ++i)
      if ((tmask[i] >> j) & 1) {
        sg += ts[2 * i];
        sp += ts[2 * i + 1];
      }
    acc[j][0] = sg;
    acc[j][1] = sp;
  } else if (threadIdx.x == 64) {
    double tot = 0.0;
    for (int i = 0; i < nt; ++i) tot += ts[2 * i];
    gtot = tot;
  }
  __syncthreads();
  const bool skip_all = found_inf && *found_inf > 0.0f;
  // step counters advance once per tensor with a gradient (in parallel)
  if (!skip_all)
    for (int i = threadIdx.x; i < nt; i += blockDim.x)
      if (rows[i].g) *reinterpret_cast<float*>(rows[i].step) += 1.0f;
  if (threadIdx.x != 0) return;
  const bool skip = found_inf && *found_inf > 0.0f;
  // torch.nn.utils.clip_grad_norm_: coef = max_norm / (total_norm + 1e-6), clamped to 1
  float coef = 1.0f;
  if (clip_max > 0.0f) {
    const float tn = (float)sqrt(gtot);
    coef = fminf(clip_max / (tn + 1e-6f), 1.0f);
  }
  for (int j = 0; j < M; ++j) {
    const float gn = (float)sqrt(acc[j][0]) * coef;
    const float pn = (float)sqrt(acc[j][1]);
    const float lr = (float)hyper[5 * metric_lr_group[j]];
    metrics[2 * j] = gn;
    metrics[2 * j + 1] = lr * gn / fmaxf(pn, 1e-12f);
  }
  scal[4 * G] = coef;
  scal[4 * G + 1] = skip ? 0.0f : 1.0f;
}

// NORMS: also write the chunk's partial sums of g^2 and p^2 (p before the update) to part, and
// run whatever found_inf says (the finish kernel then skips the counters and the metrics use
// the same values as without the update).  Otherwise the finish kernel ran first: scal holds the
// clip coefficient and the skip flag, and the step counters are already advanced.
//
// One pass over the chunk: each thread loads its 16 elements of p, g, m, v into registers (four
// 16-byte loads per tensor when the chunk is whole and aligned: elements 4 t + 1024 j + 0..3),
// forms the norm partials from the loaded p and g, updates and stores them; p and g are read once.
template <bool NORMS>
__global__ void __launch_bounds__(256) adamw_update_kernel(const AdamRow* __restrict__ rows,
                                                           const int32_t* __restrict__ blk,
                                                           const double* __restrict__ hyper, int G,
                                                           const float* __restrict__ scal,
                                                           const float* __restrict__ found_inf,
                                                           float* __restrict__ part) {
  __shared__ float red[4];
  constexpr int kPer = kChunk / 256;  // 16 elements per thread
  const int b = blockIdx.x, tid = threadIdx.x;
  const AdamRow r = rows[blk[2 * b]];
  const int64_t off = (int64_t)blk[2 * b + 1] * kChunk;
  float* p = reinterpret_cast<float*>(r.p);
  const float* g = reinterpret_cast<const float*>(r.g);
  float* m = reinterpret_cast<float*>(r.m);
  float* v = reinterpret_cast<float*>(r.v);
  const bool vec = off + kChunk <= r.numel &&
                   ((r.p | r.g | r.m | r.v) & 15) == 0;  // whole chunk, 16-byte aligned tensors
  // element e of this thread: vec ? off + 4 (t + 256 (e / 4)) + e % 4 : off + t + 256 e
  auto idx = [&](int e) -> int64_t {
    return vec ? off + 4 * (tid + 256 * (e >> 2)) + (e & 3) : off + tid + 256 * e;
  };
  bool skip;
  if constexpr (NORMS) {
    skip = found_inf && *found_inf > 0.0f;
  } else {
    skip = scal[4 * G + 1] == 0.0f;  // found_inf: no update
  }
  const bool upd = !skip && g != nullptr;
  float pv[kPer], gv[kPer], mv[kPer], vv[kPer];
  if (vec) {
#pragma unroll
    for (int j = 0; j < kPer / 4; ++j) {
      const int64_t i = off + 4 * (tid + 256 * j);
      const float4 a = *reinterpret_cast<const float4*>(p + i);
      pv[4 * j] = a.x; pv[4 * j + 1] = a.y; pv[4 * j + 2] = a.z; pv[4 * j + 3] = a.w;
      if (g) {
        const float4 c = *reinterpret_cast<const float4*>(g + i);
        gv[4 * j] = c.x; gv[4 * j + 1] = c.y; gv[4 * j + 2] = c.z; gv[4 * j + 3] = c.w;
      }
      if (upd) {
        const float4 e = *reinterpret_cast<const float4*>(m + i);
        const float4 f = *reinterpret_cast<const float4*>(v + i);
        mv[4 * j] = e.x; mv[4 * j + 1] = e.y; mv[4 * j + 2] = e.z; mv[4 * j + 3] = e.w;
        vv[4 * j] = f.x; vv[4 * j + 1] = f.y; vv[4 * j + 2] = f.z; vv[4 * j + 3] = f.w;
      }
    }
  } else {
#pragma unroll
    for (int e = 0; e < kPer; ++e) {
      const int64_t i = idx(e);
      const bool in = i < r.numel;
      pv[e] = in ? p[i] : 0.0f;
      gv[e] = (in && g) ? g[i] : 0.0f;
      mv[e] = (in && upd) ? m[i] : 0.0f;
      vv[e] = (in && upd) ? v[i] : 0.0f;
    }
  }
  if constexpr (NORMS) {
    float sg = 0.0f, sp = 0.0f;
#pragma unroll
    for (int e = 0; e < kPer; ++e) {
      sp += pv[e] * pv[e];
      if (g) sg += gv[e] * gv[e];
    }
    sg = bsum(sg, red);
    sp = bsum(sp, red);
    if (tid == 0) {
      part[2 * b] = sg;
      part[2 * b + 1] = sp;
    }
  }
  if (!upd) return;
  const int gi = (int)r.group;
  // scalar coefficients in double (the betas' complements and bias corrections lose about
  // 1e-5 relative when formed from float betas), applied in float
  const double lr_d = hyper[5 * gi], b1_d = hyper[5 * gi + 1], b2_d = hyper[5 * gi + 2];
  // the step this update is (the finish kernel advances the counter after it when NORMS)
  const double step_d = (double)*reinterpret_cast<const float*>(r.step) + (NORMS ? 1.0 : 0.0);
  const float b1 = (float)b1_d, b2 = (float)b2_d, omb1 = (float)(1.0 - b1_d), omb2 = (float)(1.0 - b2_d);
  const float eps = (float)hyper[5 * gi + 3];
  const float lr_wd = (float)(lr_d * hyper[5 * gi + 4]);
  const float step_size = (float)(lr_d / (1.0 - pow(b1_d, step_d)));
  const float bc2_sqrt = (float)sqrt(1.0 - pow(b2_d, step_d));
  const float inv_bc2 = 1.0f / bc2_sqrt;  // once per workgroup; torch divides by bc2_sqrt
  const float coef = NORMS ? 1.0f : scal[4 * G];
#pragma unroll
  for (int e = 0; e < kPer; ++e) {
    const float gr = gv[e] * coef;
    float x = pv[e];
    x -= lr_wd * x;
    const float mi = b1 * mv[e] + omb1 * gr;
    const float vi = b2 * vv[e] + omb2 * gr * gr;
    const float denom = sqrtf(vi) * inv_bc2 + eps;
    x -= step_size * (mi * __builtin_amdgcn_rcpf(denom));  // hardware reciprocal (1 ulp)
    pv[e] = x;
    mv[e] = mi;
    vv[e] = vi;
  }
  if (vec) {
#pragma unroll
    for (int j = 0; j < kPer / 4; ++j) {
      const int64_t i = off + 4 * (tid + 256 * j);
      *reinterpret_cast<float4*>(p + i) = make_float4(pv[4 * j], pv[4 * j + 1], pv[4 * j + 2], pv[4 * j + 3]);
      *reinterpret_cast<float4*>(m + i) = make_float4(mv[4 * j], mv[4 * j + 1], mv[4 * j + 2], mv[4 * j + 3]);
      *reinterpret_cast<float4*>(v + i) = make_float4(vv[4 * j], vv[4 * j + 1], vv[4 * j + 2], vv[4 * j + 3]);
    }
  } else {
#pragma unroll
    for (int e = 0; e < kPer; ++e) {
      const int64_t i = idx(e);
      if (i < r.numel) {
        p[i] = pv[e];
        m[i] = mv[e];
        v[i] = vv[e];
      }
    }
  }
}

}  // namespace

int adamw_chunk() { return kChunk; }

size_t adamw_workspace_bytes(int nt, int nblk, int G) {
  return ((size_t)2 * nblk + 2 * (size_t)nt + 4 * (size_t)G + 8) * sizeof(float);
}

int adamw_step(const void* rows, int nt, const int32_t* blk, const int32_t* first_blk, int nblk, const double* hyper,
               int G, const int32_t* metric_lr_group, int M, float clip_max, const float* found_inf, float* metrics,
               void* ws, size_t ws_bytes, hipStream_t s) {
  RTE_REQUIRE(nt >= 0 && nblk >= 0 && G >= 1 && M >= 0 && M <= 64, "adamw: bad table sizes (at most 64 metric groups)");
  RTE_REQUIRE(ws_bytes >= adamw_workspace_bytes(nt, nblk, G), "adamw: workspace too small");
  if (nt == 0) return 0;
  float* part = static_cast<float*>(ws);
  float* tsum = part + 2 * (size_t)nblk;
  float* scal = tsum + 2 * (size_t)nt;
  const AdamRow* r = static_cast<const AdamRow*>(rows);
  const size_t lds = (size_t)3 * nt * sizeof(double);
  RTE_REQUIRE(lds <= 60 * 1024, "adamw: at most 2560 tensors");
  if (clip_max <= 0.0f) {
    // no clipping: update with the partial norms, then the finish (metrics, step counters)
    if (nblk > 0) {
      hipLaunchKernelGGL(adamw_update_kernel<true>, dim3(nblk), dim3(256), 0, s, r, blk, hyper, G, scal, found_inf,
                         part);
      RTE_TRY(check_launch("adamw_update"));
    }
    hipLaunchKernelGGL(adamw_finalize_kernel, dim3(1), dim3(1024), lds, s, r, nt, first_blk, part, hyper, G,
                       metric_lr_group, M, clip_max, found_inf, tsum, scal, metrics);
    return check_launch("adamw_finalize");
  }
  if (nblk > 0) {
    hipLaunchKernelGGL(adamw_norms_kernel, dim3(nblk), dim3(256), 0, s, r, blk, part);
    RTE_TRY(check_launch("adamw_norms"));
  }
  hipLaunchKernelGGL(adamw_finalize_kernel, dim3(1), dim3(1024), lds, s, r, nt, first_blk, part, hyper, G,
                     metric_lr_group, M, clip_max, found_inf, tsum, scal, metrics);
  RTE_TRY(check_launch("adamw_finalize"));
  if (nblk > 0) {
    hipLaunchKernelGGL(adamw_update_kernel<false>, dim3(nblk), dim3(256), 0, s, r, blk, hyper, G, scal, found_inf,
                       part);
    RTE_TRY(check_launch("adamw_update"));
  }
  return 0;
}

}  // namespace rte
