// Hot-vs-exact distillation losses and alignment metrics of the audit (rte/macro.py:394-471,
// 499-546) for A audited samples of S rows x d, with the residual origin h0 given:
//
//   dp = hot - h0, de = exact - h0 (exact and h0 carry no gradient), N = S * d
//   delta_dir       = 1 - mean_a cos(dp_a, de_a)
//   delta_rms       = mean_a (log max(rms(dp_a), 1e-8) - log max(rms(de_a), 1e-8))^2
//   endpoint_normed = mean smooth_l1(rmsnorm_row(hot) - rmsnorm_row(exact))   (beta 1)
//   endpoint_raw    = mean smooth_l1(hot - exact)
//   rms_trust       = mean_a log(max(rms(hot_a), 1e-8) / max(rms(exact_a), 1e-8))^2
//   kl              = sum_rows KL(softmax(exact / t) || softmax(hot / t)) / A * t^2
// plus the alignment metrics (cosines, mse, rms norms and ratios, KL at t = 1).
//
// Forward: 16 workgroups per sample reduce partial sums, one wave per logit row reduces the KL
// rows, one workgroup adds the partials in order and one lane finishes in double precision
// (3 launches, fixed order).
// Backward: one wave per hidden row and one per logit row.
#include "common.hpp"

namespace rte {

namespace {

constexpr int kStats = 10;  // per-sample sums
constexpr int kSplit = 16;  // workgroups per sample in the forward reduction
// w12 = dp.de, w1 = |dp|^2, w2 = |de|^2, hh = |hot|^2, ee = |exact|^2, he = hot.exact,
// sl1n = sum smooth_l1 of the row-normalised difference, sl1r = sum smooth_l1(hot - exact),
// mse = sum (hot - exact)^2, (unused)
enum { W12, W1, W2, HH, EE, HE, SL1N, SL1R, MSE };

__device__ __forceinline__ float wsum(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

__device__ __forceinline__ float wmax(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, 64));
  return v;
}

__device__ __forceinline__ float sl1(float z) {
  const float a = fabsf(z);
  return a < 1.0f ? 0.5f * z * z : a - 0.5f;
}

__device__ __forceinline__ float sl1_grad(float z) { return fminf(fmaxf(z, -1.0f), 1.0f); }

__global__ void __launch_bounds__(256) distill_sample_kernel(const float* __restrict__ hot,
                                                             const float* __restrict__ ex,
                                                             const float* __restrict__ h0, int S, int d, float eps,
                                                             float* __restrict__ stats) {
  __shared__ float red[4][kStats];
  const int a = blockIdx.x, y = blockIdx.y;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  float acc[kStats];
#pragma unroll
  for (int k = 0; k < kStats; ++k) acc[k] = 0.0f;
  // rows 4 * (y + kSplit * i) + wave of sample a
  for (int s = 4 * y + wave; s < S; s += 4 * kSplit) {
    const int64_t rb = ((int64_t)a * S + s) * d;
    float rh = 0.0f, re = 0.0f;
    for (int c = lane; c < d; c += 64) {
      const float x = hot[rb + c], y = ex[rb + c], o = h0[rb + c];
      const float dp = x - o, de = y - o, df = x - y;
      acc[W12] += dp * de;
      acc[W1] += dp * dp;
      acc[W2] += de * de;
      acc[HE] += x * y;
      acc[SL1R] += sl1(df);
      acc[MSE] += df * df;
      rh += x * x;
      re += y * y;
    }
    rh = wsum(rh);
    re = wsum(re);
    if (lane == 0) {
      acc[HH] += rh;
      acc[EE] += re;
    }
    const float rsh = rsqrtf(rh / (float)d + eps), rse = rsqrtf(re / (float)d + eps);
    for (int c = lane; c < d; c += 64) acc[SL1N] += sl1(hot[rb + c] * rsh - ex[rb + c] * rse);
  }
#pragma unroll
  for (int k = 0; k < kStats; ++k) {
    const float v = wsum(acc[k]);
    if (lane == 0) red[wave][k] = v;
  }
  __syncthreads();
  if (threadIdx.x < kStats) {
    const int k = threadIdx.x;
    stats[((int64_t)a * kSplit + y) * kStats + k] = ((red[0][k] + red[1][k]) + red[2][k]) + red[3][k];
  }
}

// One wave per logit row: KL at temperature t (and its lse's for the backward) and the
// t = 1 metric KL(softmax(exact) || softmax(hot)).

__global__ void __launch_bounds__(256) kl_rows_kernel(const float* __restrict__ hot, const float* __restrict__ ex,
                                                      int R, int V, float inv_t, float* __restrict__ kl_row,
                                                      float* __restrict__ klm_row, float* __restrict__ lse) {
  const int lane = threadIdx.x & 63;
  const int r = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (r >= R) return;
  const float* hr = hot + (int64_t)r * V;
  const float* er = ex + (int64_t)r * V;
  // maxima of hot, exact (the t-scaled maxima are these times inv_t, inv_t > 0)
  float mh = -INFINITY, me = -INFINITY;
  for (int c = lane; c < V; c += 64) {
    mh = fmaxf(mh, hr[c]);
    me = fmaxf(me, er[c]);
  }
  mh = wmax(mh);
  me = wmax(me);
  float sh_t = 0.0f, se_t = 0.0f, sh_1 = 0.0f, se_1 = 0.0f;
  for (int c = lane; c < V; c += 64) {
    const float x = hr[c], y = er[c];
    sh_t += __expf((x - mh) * inv_t);
    se_t += __expf((y - me) * inv_t);
    sh_1 += __expf(x - mh);
    se_1 += __expf(y - me);
  }
  sh_t = wsum(sh_t);
  se_t = wsum(se_t);
  sh_1 = wsum(sh_1);
  se_1 = wsum(se_1);
  const float lq_t = mh * inv_t + logf(sh_t), lp_t = me * inv_t + logf(se_t);  // lse of hot/t, exact/t
  const float lq_1 = mh + logf(sh_1), lp_1 = me + logf(se_1);
  float kt = 0.0f, k1 = 0.0f;
  for (int c = lane; c < V; c += 64) {
    const float x = hr[c], y = er[c];
    const float logp = y * inv_t - lp_t, logq = x * inv_t - lq_t;
    const float p = __expf(logp);
    kt += p > 0.0f ? p * (logp - logq) : 0.0f;
    const float te = y - lp_1, th = x - lq_1;
    k1 += __expf(te) * (te - th);
  }
  kt = wsum(kt);
  k1 = wsum(k1);
  if (lane == 0) {
    kl_row[r] = kt;
    klm_row[r] = k1;
    lse[2 * r] = lq_t;
    lse[2 * r + 1] = lp_t;
  }
}

// The same for V <= 64 NV: both rows are read once into registers and the three passes run over
// them in the order of kl_rows_kernel (bitwise the same results).
template <int NV>
__global__ void __launch_bounds__(256) kl_rows_reg_kernel(const float* __restrict__ hot, const float* __restrict__ ex,
                                                          int R, int V, float inv_t, float* __restrict__ kl_row,
                                                          float* __restrict__ klm_row, float* __restrict__ lse) {
  const int lane = threadIdx.x & 63;
  const int r = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (r >= R) return;
  const float* hr = hot + (int64_t)r * V;
  const float* er = ex + (int64_t)r * V;
  float xs[NV], ys[NV];
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int c = lane + 64 * i;
    xs[i] = c < V ? hr[c] : 0.0f;
    ys[i] = c < V ? er[c] : 0.0f;
  }
  float mh = -INFINITY, me = -INFINITY;
#pragma unroll
  for (int i = 0; i < NV; ++i)
    if (lane + 64 * i < V) {
      mh = fmaxf(mh, xs[i]);
      me = fmaxf(me, ys[i]);
    }
  mh = wmax(mh);
  me = wmax(me);
  float sh_t = 0.0f, se_t = 0.0f, sh_1 = 0.0f, se_1 = 0.0f;
#pragma unroll
  for (int i = 0; i < NV; ++i)
    if (lane + 64 * i < V) {
      const float x = xs[i], y = ys[i];
      sh_t += __expf((x - mh) * inv_t);
      se_t += __expf((y - me) * inv_t);
      sh_1 += __expf(x - mh);
      se_1 += __expf(y - me);
    }
  sh_t = wsum(sh_t);
  se_t = wsum(se_t);
  sh_1 = wsum(sh_1);
  se_1 = wsum(se_1);
  const float lq_t = mh * inv_t + logf(sh_t), lp_t = me * inv_t + logf(se_t);
  const float lq_1 = mh + logf(sh_1), lp_1 = me + logf(se_1);
  float kt = 0.0f, k1 = 0.0f;
#pragma unroll
  for (int i = 0; i < NV; ++i)
    if (lane + 64 * i < V) {
      const float x = xs[i], y = ys[i];
      const float logp = y * inv_t - lp_t, logq = x * inv_t - lq_t;
      const float p = __expf(logp);
      kt += p > 0.0f ? p * (logp - logq) : 0.0f;
      const float te = y - lp_1, th = x - lq_1;
      k1 += __expf(te) * (te - th);
    }
  kt = wsum(kt);
  k1 = wsum(k1);
  if (lane == 0) {
    kl_row[r] = kt;
    klm_row[r] = k1;
    lse[2 * r] = lq_t;
    lse[2 * r + 1] = lp_t;
  }
}

// losses: [0..4] delta_dir, delta_rms, endpoint_normed, endpoint_raw, rms_trust, [5] kl;
// metrics: [0] hidden_cosine, [1] hidden_mse, [2] macro_norm, [3] exact_norm,
// [4] macro_exact_norm_ratio, [5] delta_cosine, [6] delta_rms_exact, [7] delta_rms_pred,
// [8] delta_rms_ratio, [9] logit_kl_exact_macro
struct LossWeights {
  float w[6];
};

__global__ void distill_final_kernel(const float* __restrict__ parts, float* __restrict__ stats, int A, int S,
                                     int d, const float* __restrict__ kl_row, const float* __restrict__ klm_row,
                                     int R, float t, LossWeights lw, float* __restrict__ out,
                                     float* __restrict__ met) {
  // per-sample sums of the kSplit partials, in order (kept for the backward)
  for (int q = threadIdx.x; q < A * kStats; q += blockDim.x) {
    const int a = q / kStats, k = q - a * kStats;
    float v = 0.0f;
    for (int y = 0; y < kSplit; ++y) v += parts[((int64_t)a * kSplit + y) * kStats + k];
    stats[q] = v;
  }
  __syncthreads();
  if (threadIdx.x != 0) return;
  const double N = (double)S * d;
  double cos_d = 0, cos_h = 0, lrms = 0, trust = 0, sl1n = 0, sl1r = 0, mse = 0, mn = 0, en = 0, pr = 0, er = 0;
  for (int a = 0; a < A; ++a) {
    const float* st = stats + (int64_t)a * kStats;
    const double w12 = st[W12], w1 = st[W1], w2 = st[W2], hh = st[HH], ee = st[EE], he = st[HE];
    cos_d += w12 / fmax(sqrt(w1 * w2), 1e-8);
    cos_h += he / fmax(sqrt(hh * ee), 1e-8);
    const double rp = sqrt(w1 / N), re_ = sqrt(w2 / N), rh = sqrt(hh / N), rx = sqrt(ee / N);
    const double l = log(fmax(rp, 1e-8)) - log(fmax(re_, 1e-8));
    lrms += l * l;
    const double lt = log(fmax(rh, 1e-8) / fmax(rx, 1e-8));
    trust += lt * lt;
    sl1n += st[SL1N];
    sl1r += st[SL1R];
    mse += st[MSE];
    mn += rh;
    en += rx;
    pr += rp;
    er += re_;
  }
  const double iA = A > 0 ? 1.0 / A : 0.0;
  out[0] = lw.w[0] * (float)(1.0 - cos_d * iA);
  out[1] = lw.w[1] * (float)(lrms * iA);
  out[2] = lw.w[2] * (float)(sl1n * iA / N);
  out[3] = lw.w[3] * (float)(sl1r * iA / N);
  out[4] = lw.w[4] * (float)(trust * iA);
  double kl = 0, klm = 0;
  for (int r = 0; r < R; ++r) {
    kl += kl_row[r];
    klm += klm_row[r];
  }
  out[5] = R > 0 ? lw.w[5] * (float)(kl * iA * (double)t * t) : 0.0f;
  met[0] = (float)(cos_h * iA);
  met[1] = (float)(mse * iA / N);
  met[2] = (float)(mn * iA);
  met[3] = (float)(en * iA);
  met[4] = (float)(mn * iA / fmax(en * iA, 1e-8));
  met[5] = (float)(cos_d * iA);
  met[6] = (float)(er * iA);
  met[7] = (float)(pr * iA);
  met[8] = (float)(pr * iA / fmax(er * iA, 1e-8));
  met[9] = R > 0 ? (float)(klm / R) : 0.0f;
}

// d hot for upstream gradients g[0..4] of out[0..4]; one wave per hidden row.
__global__ void __launch_bounds__(256) distill_bwd_kernel(const float* __restrict__ hot, const float* __restrict__ ex,
                                                          const float* __restrict__ h0,
                                                          const float* __restrict__ stats, int A, int S, int d,
                                                          float eps, const float* __restrict__ gin, LossWeights lw,
                                                          float* __restrict__ dhot) {
  const int lane = threadIdx.x & 63;
  const int row = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= A * S) return;
  float g[5];
#pragma unroll
  for (int q = 0; q < 5; ++q) g[q] = gin[q] * lw.w[q];
  const int a = row / S;
  const float* st = stats + (int64_t)a * kStats;
  const float N = (float)S * d, iA = 1.0f / (float)A;
  const float w12 = st[W12], w1 = st[W1], w2 = st[W2], hh = st[HH], ee = st[EE];
  // delta_dir: d(1 - cos)/d dp = -(de / D - cos dp / w1) with D = max(|dp||de|, 1e-8)
  const float D = sqrtf(w1 * w2);
  const float cosd = w12 / fmaxf(D, 1e-8f);
  const float al = -g[0] * iA / fmaxf(D, 1e-8f);
  const float be = D > 1e-8f ? g[0] * iA * cosd / w1 : 0.0f;
  // delta_rms: 2 (log rp - log re) / rp * drp/ddp, drp/ddp = dp / (N rp)
  const float rp = sqrtf(w1 / N), rre = sqrtf(w2 / N);
  const float ga = rp > 1e-8f ? g[1] * iA * 2.0f * (logf(rp) - logf(fmaxf(rre, 1e-8f))) / (rp * rp * N) : 0.0f;
  // rms_trust: 2 log(rh / rx) / rh * hot / (N rh)
  const float rh = sqrtf(hh / N), rx = sqrtf(ee / N);
  const float de_ = rh > 1e-8f ? g[4] * iA * 2.0f * logf(rh / fmaxf(rx, 1e-8f)) / (rh * rh * N) : 0.0f;
  const float cr = g[3] * iA / N, cn = g[2] * iA / N;
  const int64_t rb = (int64_t)row * d;
  float sx = 0.0f, sy = 0.0f;
  for (int c = lane; c < d; c += 64) {
    const float x = hot[rb + c], y = ex[rb + c];
    sx += x * x;
    sy += y * y;
  }
  sx = wsum(sx);
  sy = wsum(sy);
  const float rsh = rsqrtf(sx / (float)d + eps), rse = rsqrtf(sy / (float)d + eps);
  float dot = 0.0f;  // sum_j u_j x_j of the endpoint_normed upstream u
  for (int c = lane; c < d; c += 64) dot += cn * sl1_grad(hot[rb + c] * rsh - ex[rb + c] * rse) * hot[rb + c];
  dot = wsum(dot);
  const float coef = rsh * rsh * rsh * dot / (float)d;
  for (int c = lane; c < d; c += 64) {
    const float x = hot[rb + c], y = ex[rb + c], o = h0[rb + c];
    const float dp = x - o, dv = y - o;
    const float u = cn * sl1_grad(x * rsh - y * rse);
    dhot[rb + c] = al * dv + (be + ga) * dp + de_ * x + cr * sl1_grad(x - y) + (rsh * u - x * coef);
  }
}

// d hot_logits = g * t / A * (softmax(hot / t) - softmax(exact / t)); one wave per row.
__global__ void __launch_bounds__(256) kl_bwd_kernel(const float* __restrict__ hot, const float* __restrict__ ex,
                                                     const float* __restrict__ lse, int R, int V, float inv_t,
                                                     float scale, const float* __restrict__ g,
                                                     float* __restrict__ dhot) {
  const int lane = threadIdx.x & 63;
  const int r = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (r >= R) return;
  const float k = g[0] * scale;  // scale includes the KL weight
  const float lq = lse[2 * r], lp = lse[2 * r + 1];
  const int64_t rb = (int64_t)r * V;
  for (int c = lane; c < V; c += 64)
    dhot[rb + c] = k * (__expf(hot[rb + c] * inv_t - lq) - __expf(ex[rb + c] * inv_t - lp));
}

}  // namespace

// workspace: per-sample sums [A][kStats] | KL rows [R] | metric KL rows [R] | lse [2R] |
// forward partials [A][kSplit][kStats]
size_t distill_workspace_bytes(int A, int R) {
  return ((size_t)A * kStats * (1 + kSplit) + (size_t)R * 4 + 64) * sizeof(float);
}

int distill_fwd(const float* hot, const float* exact, const float* h0, int A, int S, int d, const float* hot_logits,
                const float* exact_logits, int V, float t, float eps, const float* weights, float* losses,
                float* metrics, void* ws, size_t ws_bytes, hipStream_t s) {
  RTE_REQUIRE(A >= 1 && S >= 1 && d >= 1, "distill: need at least one audited sample");
  RTE_REQUIRE(hot && exact && h0 && losses && metrics, "distill: hot, exact, h0 and the outputs are required");
  RTE_REQUIRE(t > 0.0f, "distill: temperature must be positive");
  const int R = (hot_logits && exact_logits) ? A * S : 0;
  RTE_REQUIRE(R == 0 || V >= 1, "distill: logits need V >= 1");
  RTE_REQUIRE(ws_bytes >= distill_workspace_bytes(A, R), "distill: workspace too small");
  float* stats = static_cast<float*>(ws);
  float* kl_row = stats + (size_t)A * kStats;
  float* klm_row = kl_row + R;
  float* lse = klm_row + R;
  float* parts = lse + 2 * (size_t)R;
  hipLaunchKernelGGL(distill_sample_kernel, dim3(A, kSplit), dim3(256), 0, s, hot, exact, h0, S, d, eps, parts);
  RTE_TRY(check_launch("distill_sample"));
  if (R > 0) {
    if (V <= 64 * 32)
      hipLaunchKernelGGL(kl_rows_reg_kernel<32>, dim3((R + 3) / 4), dim3(256), 0, s, hot_logits, exact_logits, R, V,
                         1.0f / t, kl_row, klm_row, lse);
    else
      hipLaunchKernelGGL(kl_rows_kernel, dim3((R + 3) / 4), dim3(256), 0, s, hot_logits, exact_logits, R, V,
                         1.0f / t, kl_row, klm_row, lse);
    RTE_TRY(check_launch("distill_kl_rows"));
  }
  LossWeights lw;
  for (int q = 0; q < 6; ++q) lw.w[q] = weights ? weights[q] : 1.0f;
  hipLaunchKernelGGL(distill_final_kernel, dim3(1), dim3(256), 0, s, parts, stats, A, S, d, kl_row, klm_row, R, t, lw,
                     losses, metrics);
  return check_launch("distill_final");
}

int distill_bwd(const float* hot, const float* exact, const float* h0, int A, int S, int d, const float* hot_logits,
                const float* exact_logits, int V, float t, float eps, const float* weights, const float* g,
                const void* ws, size_t ws_bytes, float* dhot, float* dhot_logits, hipStream_t s) {
  RTE_REQUIRE(A >= 1 && S >= 1 && d >= 1 && g, "distill_bwd: bad arguments");
  RTE_REQUIRE(ws_bytes >= distill_workspace_bytes(A, (hot_logits && exact_logits) ? A * S : 0),
              "distill_bwd: workspace too small");
  const int R = (hot_logits && exact_logits) ? A * S : 0;
  const float* stats = static_cast<const float*>(ws);
  const float* lse = stats + (size_t)A * kStats + 2 * (size_t)R;
  if (dhot) {
    LossWeights lw;
    for (int q = 0; q < 6; ++q) lw.w[q] = weights ? weights[q] : 1.0f;
    hipLaunchKernelGGL(distill_bwd_kernel, dim3((A * S + 3) / 4), dim3(256), 0, s, hot, exact, h0, stats, A, S, d,
                       eps, g, lw, dhot);
    RTE_TRY(check_launch("distill_bwd"));
  }
  if (dhot_logits && R > 0) {
    const float wkl = weights ? weights[5] : 1.0f;
    hipLaunchKernelGGL(kl_bwd_kernel, dim3((R + 3) / 4), dim3(256), 0, s, hot_logits, exact_logits, lse, R, V,
                       1.0f / t, wkl * t / (float)A, g + 5, dhot_logits);
    RTE_TRY(check_launch("distill_kl_bwd"));
  }
  return 0;
}

}  // namespace rte
