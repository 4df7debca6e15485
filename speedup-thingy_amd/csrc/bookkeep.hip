// Per-step bookkeeping of the audit sampler and the recipe usage statistics, one workgroup each
// (a batch's B samples are a few hundred rows, so one launch replaces a chain of small torch ops):
//
//   audit_sample_fixed (rte/audit.py:79-132 with the fixed-count sampler):
//     req[b]  = clamp(p_min + alpha ent[b] / denom + beta residual
//                     + gamma max(cmin - ema[id[b]], 0) / max(cmin, 1e-12), p_min, p_max)
//     incl[b] = k / B;  mask[b] = b in chosen
//     stats   = mean(incl), mean(req), count / B, count, mean(incl)
//   count_ema (rte/recipes.py update_usage, rte/audit.py coverage update):
//     counts[r] = #{i : ids[i] == r and mask[i]};  ema = ema beta + (1 - beta) counts / max(sum counts, 1)
//   nonfinite (the step's skip test on the loss, rte/training.py:445-468) and step_metrics (the
//     per-sample means of rte/training.py:1412-1472: hot / corrected loss, nll per token, depth)
//   loss_sum (the step's loss, rte/training.py:1381-1385): loss = coef sum_b x[b] + sum_i term_i
//     (term_i device scalars, added in order after the row sum); its backward fills
//     dx[b] = coef g[0]
//
// Row sums run in a fixed order (per-thread row strides, then an LDS tree); the counts are
// integer LDS atomics, exact in any order.
#include "common.hpp"

namespace rte {

namespace {

constexpr int kBkThreads = 256;
constexpr int kBkMaxBins = 4096;

__device__ __forceinline__ float bk_block_sum(float v, float* red) {
  const int t = threadIdx.x;
  red[t] = v;
  __syncthreads();
  for (int s = kBkThreads / 2; s > 0; s >>= 1) {
    if (t < s) red[t] += red[t + s];
    __syncthreads();
  }
  const float r = red[0];
  __syncthreads();
  return r;
}

__global__ void __launch_bounds__(kBkThreads)
    audit_sample_fixed_kernel(const float* ent, const int64_t* ids, const float* ema, const int64_t* chosen, int B,
                              int k, int R, float denom, float p_min, float p_max, float alpha, float beta,
                              float gamma, float residual, float cmin, float cdiv, float* req, float* incl,
                              uint8_t* mask, float* stats) {
  __shared__ float red[kBkThreads];
  const int t = threadIdx.x;
  const float inc = (float)k / (float)B;
  const float bres = beta * residual;
  float s_req = 0.0f, s_inc = 0.0f;
  for (int b = t; b < B; b += kBkThreads) {
    const int64_t id = ids[b];
    const float e = (id >= 0 && id < R) ? ema[id] : 0.0f;
    float dft = cmin - e;
    dft = (dft < 0.0f ? 0.0f : dft) / cdiv;
    float p = p_min + alpha * (ent[b] / denom);
    p = p + bres;
    p = p + gamma * dft;
    p = p < p_min ? p_min : (p > p_max ? p_max : p);  // NaN stays NaN, as torch.clamp
    req[b] = p;
    incl[b] = inc;
    mask[b] = 0;
    s_req += p;
    s_inc += inc;
  }
  __syncthreads();
  for (int j = t; j < k; j += kBkThreads) {
    const int64_t c = chosen[j];
    if (c >= 0 && c < B) mask[c] = 1;
  }
  __syncthreads();
  float s_cnt = 0.0f;
  for (int b = t; b < B; b += kBkThreads) s_cnt += mask[b] ? 1.0f : 0.0f;
  const float tr = bk_block_sum(s_req, red);
  const float ti = bk_block_sum(s_inc, red);
  const float tc = bk_block_sum(s_cnt, red);
  if (t == 0) {
    stats[0] = ti / (float)B;
    stats[1] = tr / (float)B;
    stats[2] = tc / (float)B;
    stats[3] = tc;
    stats[4] = ti / (float)B;
  }
}

__global__ void __launch_bounds__(kBkThreads)
    count_ema_kernel(const int64_t* ids, const uint8_t* mask, int n, float* ema, int R, float beta) {
  __shared__ int cnt[kBkMaxBins];
  __shared__ float red[kBkThreads];
  const int t = threadIdx.x;
  for (int r = t; r < R; r += kBkThreads) cnt[r] = 0;
  __syncthreads();
  for (int i = t; i < n; i += kBkThreads) {
    const int64_t id = ids[i];
    if ((mask == nullptr || mask[i]) && id >= 0 && id < R) atomicAdd(&cnt[id], 1);
  }
  __syncthreads();
  float s = 0.0f;
  for (int r = t; r < R; r += kBkThreads) s += (float)cnt[r];
  const float tot = bk_block_sum(s, red);
  const float den = tot < 1.0f ? 1.0f : tot;
  for (int r = t; r < R; r += kBkThreads) ema[r] = ema[r] * beta + (1.0f - beta) * ((float)cnt[r] / den);
}

// bad = 1 when x[0] is not finite (inf or NaN), else 0; ok = 1 - bad
__global__ void nonfinite_kernel(const float* x, float* bad, float* ok) {
  if (threadIdx.x == 0) {
    const float v = x[0];
    const float b = (v - v) != 0.0f || v != v ? 1.0f : 0.0f;  // inf - inf and NaN are NaN
    bad[0] = b;
    ok[0] = 1.0f - b;
  }
}

// out = mean(hot) / scale, mean(corr) / scale, mean(corr) / seq, mean(depth)
__global__ void __launch_bounds__(kBkThreads)
    step_metrics_kernel(const float* hot, const float* corr, const int64_t* depth, int B, float scale, float seq,
                        float* out) {
  __shared__ float red[kBkThreads];
  const int t = threadIdx.x;
  float sh = 0.0f, sc = 0.0f, sd = 0.0f;
  for (int b = t; b < B; b += kBkThreads) {
    sh += hot[b];
    sc += corr[b];
    sd += (float)depth[b];
  }
  const float th = bk_block_sum(sh, red), tc = bk_block_sum(sc, red), td = bk_block_sum(sd, red);
  if (t == 0) {
    const float mh = th / (float)B, mc = tc / (float)B;
    out[0] = mh / scale;
    out[1] = mc / scale;
    out[2] = mc / seq;
    out[3] = td / (float)B;
  }
}

constexpr int kLossTerms = 32;

struct LossTerms {
  const float* t[kLossTerms];
};

__global__ void __launch_bounds__(kBkThreads)
    loss_sum_kernel(const float* x, int n, float coef, LossTerms terms, int nt, float* out) {
  __shared__ float red[kBkThreads];
  float s = 0.0f;
  for (int b = threadIdx.x; b < n; b += kBkThreads) s += x[b];
  const float tot = bk_block_sum(s, red);
  if (threadIdx.x == 0) {
    float r = coef * tot;
    for (int i = 0; i < nt; ++i) r += *terms.t[i];
    out[0] = r;
  }
}

__global__ void __launch_bounds__(kBkThreads) loss_sum_bwd_kernel(const float* g, int n, float coef, float* dx) {
  const float v = coef * g[0];
  for (int b = blockIdx.x * kBkThreads + threadIdx.x; b < n; b += gridDim.x * kBkThreads) dx[b] = v;
}

}  // namespace

}  // namespace rte

using namespace rte;

extern "C" {

int rte_audit_sample_fixed(const float* entropy, const int64_t* recipe_ids, const float* coverage_ema,
                           const int64_t* chosen, int B, int k, int R, float denom, float p_min, float p_max,
                           float alpha, float beta, float gamma, float residual, float coverage_min, float* req,
                           float* incl, void* mask, float* stats, void* stream) {
  RTE_REQUIRE(B >= 1 && k >= 0 && k <= B && R >= 1, "audit_sample_fixed: bad sizes");
  RTE_REQUIRE(entropy && recipe_ids && coverage_ema && req && incl && mask && stats && (k == 0 || chosen),
              "audit_sample_fixed: null argument");
  const float cdiv = coverage_min > 1e-12f ? coverage_min : 1e-12f;
  hipLaunchKernelGGL(audit_sample_fixed_kernel, dim3(1), dim3(kBkThreads), 0, static_cast<hipStream_t>(stream),
                     entropy, recipe_ids, coverage_ema, chosen, B, k, R, denom, p_min, p_max, alpha, beta, gamma,
                     residual, coverage_min, cdiv, req, incl, static_cast<uint8_t*>(mask), stats);
  return check_launch("audit_sample_fixed");
}

int rte_count_ema(const int64_t* ids, const void* mask, int n, float* ema, int R, float beta, void* stream) {
  RTE_REQUIRE(n >= 0 && R >= 1 && R <= kBkMaxBins, "count_ema: bad sizes (1 <= bins <= 4096)");
  RTE_REQUIRE(ema && (n == 0 || ids), "count_ema: null argument");
  hipLaunchKernelGGL(count_ema_kernel, dim3(1), dim3(kBkThreads), 0, static_cast<hipStream_t>(stream), ids,
                     static_cast<const uint8_t*>(mask), n, ema, R, beta);
  return check_launch("count_ema");
}

int rte_nonfinite(const float* x, float* bad, float* ok, void* stream) {
  RTE_REQUIRE(x && bad && ok, "nonfinite: null argument");
  hipLaunchKernelGGL(nonfinite_kernel, dim3(1), dim3(64), 0, static_cast<hipStream_t>(stream), x, bad, ok);
  return check_launch("nonfinite");
}

int rte_step_metrics(const float* hot, const float* corr, const int64_t* depth, int B, float scale, float seq,
                     float* out, void* stream) {
  RTE_REQUIRE(B >= 1 && hot && corr && depth && out, "step_metrics: bad arguments");
  hipLaunchKernelGGL(step_metrics_kernel, dim3(1), dim3(kBkThreads), 0, static_cast<hipStream_t>(stream), hot, corr,
                     depth, B, scale, seq, out);
  return check_launch("step_metrics");
}

int rte_loss_sum(const float* x, int n, float coef, const float* const* terms, int n_terms, float* out,
                 void* stream) {
  RTE_REQUIRE(n >= 0 && n_terms >= 0 && n_terms <= kLossTerms, "loss_sum: 0 <= n, 0 <= terms <= 32");
  RTE_REQUIRE(out && (n == 0 || x) && (n_terms == 0 || terms), "loss_sum: null argument");
  LossTerms lt{};
  for (int i = 0; i < n_terms; ++i) {
    RTE_REQUIRE(terms[i], "loss_sum: null term");
    lt.t[i] = terms[i];
  }
  hipLaunchKernelGGL(loss_sum_kernel, dim3(1), dim3(kBkThreads), 0, static_cast<hipStream_t>(stream), x, n, coef, lt,
                     n_terms, out);
  return check_launch("loss_sum");
}

int rte_loss_sum_bwd(const float* g, int n, float coef, float* dx, void* stream) {
  RTE_REQUIRE(n >= 0 && g && (n == 0 || dx), "loss_sum_bwd: bad arguments");
  if (n == 0) return 0;
  const int blocks = (n + kBkThreads - 1) / kBkThreads;
  hipLaunchKernelGGL(loss_sum_bwd_kernel, dim3(blocks < 64 ? blocks : 64), dim3(kBkThreads), 0,
                     static_cast<hipStream_t>(stream), g, n, coef, dx);
  return check_launch("loss_sum_bwd");
}

}  // extern "C"
