// Per-sample recipe / depth router (rte/routing.py:80-188) and its auxiliary losses
// (rte/metrics.py:97-112) as a handful of launches instead of one torch kernel per elementwise op.
//
//   pooled  = mean_s h0[b, s, :]                                   (rtr_pool: fp32 + bf16 copy)
//   z1      = pooled W1^T + b1        (recipe and depth MLPs)      (the MFMA GEMM, bias epilogue)
//   raw     = silu(z1) W2^T + b2                                   \
//   logits  = raw * inv_t; probs = softmax; id = argmax(probs)      |  rtr_heads_fwd: one wave per
//   by pass: logits + pass_bias[t] * inv_t -> softmax, argmax       |  sample row
//   onehot_st = (onehot(id) + p) - p; entropy = -sum log(max(p, 1e-9)) p
//   expected_depth = sum_j p_j depth_values[j]                     /
//
// backward: rtr_heads_bwd (one wave per row: entropy, straight-through, expected-depth and
// softmax backward, d raw logits = inv_t d logits), rtr_mlp_bwd (per 64 hidden columns: dW2, db2,
// dz1 = (d raw W2) silu'(z1), db1, and the pass-bias gradient), then the MFMA GEMMs for dW1 and
// d pooled.  Every sum runs in a fixed order (wave xor trees, rows in order), so results repeat
// bitwise.  argmax follows torch: the first maximal index, NaN counting as the maximum.
#include "common.hpp"

namespace rte {

namespace {

constexpr float kEntEps = 1e-9f;
constexpr int kRtrMaxOut = 64;    // recipes or depth choices per head
constexpr int kRtrMaxPass = 16;   // recursive passes with their own recipe bias
constexpr int kRtrMaxHid = 4096;  // hidden width of the router MLPs
constexpr int kRtrRowChunk = 64;  // rows of d raw logits staged per LDS pass in rtr_mlp_bwd

__device__ __forceinline__ float rtr_wsum(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
  return v;
}

// NaN-propagating maximum (softmax of a row holding NaN is NaN everywhere, as in torch)
__device__ __forceinline__ float rtr_wmax(float v) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    const float o = __shfl_xor(v, off, 64);
    v = (v != v || o != o) ? __int_as_float(0x7fc00000) : (o > v ? o : v);
  }
  return v;
}

// index of the first maximal value over the wave (lanes >= n hold -inf / index n); NaN wins
__device__ __forceinline__ int rtr_wargmax(float v, int i) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    const float ov = __shfl_xor(v, off, 64);
    const int oi = __shfl_xor(i, off, 64);
    const bool vn = v != v, on = ov != ov;
    bool take;
    if (vn || on) take = on && (!vn || oi < i);
    else take = ov > v || (ov == v && oi < i);
    if (take) { v = ov; i = oi; }
  }
  return i;
}

__device__ __forceinline__ float rtr_silu(float z) { return z / (1.0f + expf(-z)); }

// softmax, argmax, straight-through one-hot and entropy of one head row held one value per lane
// (lanes >= n idle).  Returns the lane's probability; writes the row's outputs.
__device__ __forceinline__ float rtr_head_row(float logit, int lane, int n, int fixed_id, float* probs,
                                              int64_t* id_out, float* onehot, float* ent_out) {
  const bool on = lane < n;
  const float mx = rtr_wmax(on ? logit : -INFINITY);
  const float e = on ? expf(logit - mx) : 0.0f;
  const float s = rtr_wsum(e);
  const float p = e / s;
  int id = rtr_wargmax(on ? p : -INFINITY, on ? lane : n);
  if (fixed_id >= 0) id = fixed_id;
  const float c = p < kEntEps ? kEntEps : p;  // clamp_min keeps NaN
  const float ent = -rtr_wsum(on ? logf(c) * p : 0.0f);
  if (on) {
    if (probs) probs[lane] = p;
    if (onehot) onehot[lane] = ((lane == id ? 1.0f : 0.0f) + p) - p;
  }
  if (lane == 0) {
    if (id_out) *id_out = id;
    if (ent_out) *ent_out = ent;
  }
  return p;
}

struct RtrFwd {
  const float* z1r;  // [B, hid] recipe MLP layer-1 output (bias added)
  const float* z1d;  // [B, hid] depth MLP layer-1 output
  const float* w2r;  // [R, hid]
  const float* b2r;  // [R]
  const float* w2d;  // [D, hid]
  const float* b2d;  // [D]
  const float* pass_bias;        // [P, R]
  const int64_t* depth_values;   // [D]
  int B, hid, R, D, P;
  float inv_t;
  int fixed_recipe, fixed_depth;  // -1: argmax
  float* rlog;  float* rprob;  int64_t* rid;  float* ronehot;       // [B, R] / [B]
  float* dlog;  float* dprob;  int64_t* did;  int64_t* depth;  float* donehot;
  float* rent;  float* dent;  float* ent;  float* edepth;           // [B]
  float* rlog_bp;  float* rprob_bp;  int64_t* rid_bp;  float* ronehot_bp;  // [B, P, R] / [B, P]
};

__global__ void __launch_bounds__(64) rtr_heads_fwd_kernel(RtrFwd a) {
  __shared__ float act[2][kRtrMaxHid];
  __shared__ float raw[2 * kRtrMaxOut];
  const int b = blockIdx.x, lane = threadIdx.x;
  for (int j = lane; j < a.hid; j += 64) {
    act[0][j] = rtr_silu(a.z1r[(int64_t)b * a.hid + j]);
    act[1][j] = rtr_silu(a.z1d[(int64_t)b * a.hid + j]);
  }
  __syncthreads();
  // layer 2: each output a wave-wide dot product over the hidden units (fixed xor tree)
  for (int o = 0; o < a.R + a.D; ++o) {
    const bool isr = o < a.R;
    const float* w = isr ? a.w2r + (int64_t)o * a.hid : a.w2d + (int64_t)(o - a.R) * a.hid;
    const float* x = act[isr ? 0 : 1];
    float acc = 0.0f;
    for (int j = lane; j < a.hid; j += 64) acc += x[j] * w[j];
    acc = rtr_wsum(acc);
    if (lane == 0) raw[o] = acc + (isr ? a.b2r[o] : a.b2d[o - a.R]);
  }
  __syncthreads();
  const int R = a.R, D = a.D;
  const int64_t rb = (int64_t)b * R, db = (int64_t)b * D;
  // recipe head
  const float lg = lane < R ? raw[lane] * a.inv_t : 0.0f;
  if (lane < R) a.rlog[rb + lane] = lg;
  float re = 0.0f;
  rtr_head_row(lg, lane, R, a.fixed_recipe, a.rprob + rb, a.rid + b, a.ronehot + rb, &re);
  // per-pass recipe heads
  for (int t = 0; t < a.P; ++t) {
    const int64_t o = ((int64_t)b * a.P + t) * R;
    const float l2 = lane < R ? lg + a.pass_bias[t * R + lane] * a.inv_t : 0.0f;
    if (lane < R) a.rlog_bp[o + lane] = l2;
    rtr_head_row(l2, lane, R, a.fixed_recipe, a.rprob_bp + o, a.rid_bp + (int64_t)b * a.P + t, a.ronehot_bp + o,
                 nullptr);
  }
  // depth head
  const float dl = lane < D ? raw[R + lane] * a.inv_t : 0.0f;
  if (lane < D) a.dlog[db + lane] = dl;
  float de = 0.0f;
  int64_t did_l = 0;
  const float pd = rtr_head_row(dl, lane, D, a.fixed_depth, a.dprob + db, &did_l, a.donehot + db, &de);
  const float ed = rtr_wsum(lane < D ? pd * (float)a.depth_values[lane] : 0.0f);
  if (lane == 0) {
    // rtr_head_row wrote the entropies and the depth id through lane 0
    a.rent[b] = re;
    a.dent[b] = de;
    a.ent[b] = re + de;
    a.did[b] = did_l;
    a.depth[b] = a.depth_values[did_l];
    a.edepth[b] = ed;
  }
}

struct RtrBwd {
  const float* rprob;  const float* rprob_bp;  const float* dprob;  // saved probabilities
  const int64_t* depth_values;
  int B, R, D, P;
  float inv_t;
  // incoming gradients, each optional (null = zero)
  const float* g_rlog;  const float* g_rprob;  const float* g_ronehot;
  const float* g_dlog;  const float* g_dprob;  const float* g_donehot;
  const float* g_rent;  const float* g_dent;  const float* g_ent;  const float* g_edepth;
  const float* g_rlog_bp;  const float* g_rprob_bp;  const float* g_ronehot_bp;
  float* draw_r;  // [B, R]  d (raw recipe logits) = inv_t d logits
  float* draw_d;  // [B, D]
  float* dlbp;    // [B, P, R] d per-pass logits (reduced over rows into the pass-bias gradient)
};

__device__ __forceinline__ float rtr_ld(const float* p, int64_t i) { return p ? p[i] : 0.0f; }

// d entropy / d p for H = -sum log(max(p, eps)) p  (torch's clamp_min passes the gradient where p >= eps)
__device__ __forceinline__ float rtr_dent(float p, float g) {
  const float c = p < kEntEps ? kEntEps : p;
  return -g * (logf(c) + (p >= kEntEps ? p / c : 0.0f));
}

__device__ __forceinline__ float rtr_softmax_bwd(float p, float dp, bool on) {
  const float s = rtr_wsum(on ? p * dp : 0.0f);
  return (dp - s) * p;
}

__global__ void __launch_bounds__(64) rtr_heads_bwd_kernel(RtrBwd a) {
  const int b = blockIdx.x, lane = threadIdx.x;
  const int R = a.R, D = a.D;
  const bool onr = lane < R, ond = lane < D;
  const int64_t ir = (int64_t)b * R + lane, id = (int64_t)b * D + lane;
  const float gre = rtr_ld(a.g_rent, b) + rtr_ld(a.g_ent, b);
  const float gde = rtr_ld(a.g_dent, b) + rtr_ld(a.g_ent, b);
  // recipe head
  const float pr = onr ? a.rprob[ir] : 0.0f;
  float dp = onr ? rtr_ld(a.g_rprob, ir) + rtr_ld(a.g_ronehot, ir) + rtr_dent(pr, gre) : 0.0f;
  float dl = rtr_softmax_bwd(pr, dp, onr) + (onr ? rtr_ld(a.g_rlog, ir) : 0.0f);
  for (int t = 0; t < a.P; ++t) {
    const int64_t o = ((int64_t)b * a.P + t) * R + lane;
    const float pt = onr ? a.rprob_bp[o] : 0.0f;
    const float dpt = onr ? rtr_ld(a.g_rprob_bp, o) + rtr_ld(a.g_ronehot_bp, o) : 0.0f;
    const float dlt = rtr_softmax_bwd(pt, dpt, onr) + (onr ? rtr_ld(a.g_rlog_bp, o) : 0.0f);
    if (onr) a.dlbp[o] = dlt;
    dl += dlt;
  }
  if (onr) a.draw_r[ir] = dl * a.inv_t;
  // depth head
  const float pd = ond ? a.dprob[id] : 0.0f;
  const float dpd = ond ? rtr_ld(a.g_dprob, id) + rtr_ld(a.g_donehot, id) + rtr_dent(pd, gde) +
                              rtr_ld(a.g_edepth, b) * (float)a.depth_values[lane]
                        : 0.0f;
  const float dld = rtr_softmax_bwd(pd, dpd, ond) + (ond ? rtr_ld(a.g_dlog, id) : 0.0f);
  if (ond) a.draw_d[id] = dld * a.inv_t;
}

struct RtrMlpBwd {
  const float* draw[2];  // [B, N_m] d raw logits of the recipe / depth head
  const float* z1[2];    // [B, hid]
  const float* w2[2];    // [N_m, hid]
  int N[2];
  int B, hid, P, R;
  const float* dlbp;  // [B, P, R]
  float inv_t;
  bf16* dz1[2];   // [B, hid]
  float* db1[2];  // [hid]
  float* dw2[2];  // [N_m, hid]
  float* db2[2];  // [N_m]
  float* dpass;   // [P, R]
};

// grid (hid / 64, 2 MLPs), 256 threads: thread column j = 64 blockIdx.x + lane; the four waves
// take interleaved row chunks of 16 and their partial sums meet in LDS in wave order.
__global__ void __launch_bounds__(256) rtr_mlp_bwd_kernel(RtrMlpBwd a) {
  __shared__ float sd[kRtrRowChunk * kRtrMaxOut];
  __shared__ float part[4][kRtrMaxOut + 1][64];
  const int m = blockIdx.y, lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int N = a.N[m], hid = a.hid, B = a.B;
  const int j = blockIdx.x * 64 + lane;
  const bool onj = j < hid;
  float w2c[kRtrMaxOut];
  float dw2[kRtrMaxOut];
#pragma unroll
  for (int n = 0; n < kRtrMaxOut; ++n) {
    w2c[n] = (n < N && onj) ? a.w2[m][(int64_t)n * hid + j] : 0.0f;
    dw2[n] = 0.0f;
  }
  float db1 = 0.0f;
  for (int r0 = 0; r0 < B; r0 += kRtrRowChunk) {
    const int rows = B - r0 < kRtrRowChunk ? B - r0 : kRtrRowChunk;
    __syncthreads();
    for (int i = threadIdx.x; i < rows * N; i += 256) sd[i] = a.draw[m][(int64_t)r0 * N + i];
    __syncthreads();
    // wave w takes rows 16w .. 16w + 15 of the chunk
    for (int rr = 16 * w; rr < rows && rr < 16 * w + 16; ++rr) {
      const int64_t row = r0 + rr;
      const float z = onj ? a.z1[m][row * hid + j] : 0.0f;
      const float sg = 1.0f / (1.0f + expf(-z));
      const float act = rtr_silu(z);
      float da = 0.0f;
#pragma unroll
      for (int n = 0; n < kRtrMaxOut; ++n)
        if (n < N) {
          const float g = sd[rr * N + n];
          da += g * w2c[n];
          dw2[n] += g * act;
        }
      const float dz = da * (sg * (1.0f + z * (1.0f - sg)));
      if (onj) a.dz1[m][row * hid + j] = f2bf(dz);
      db1 += dz;
    }
  }
  // the waves' partials in wave order
#pragma unroll
  for (int n = 0; n < kRtrMaxOut; ++n)
    if (n < N) part[w][n][lane] = dw2[n];
  part[w][kRtrMaxOut][lane] = db1;
  __syncthreads();
  for (int i = threadIdx.x; i < (N + 1) * 64; i += 256) {
    const int n = i / 64 < N ? i / 64 : kRtrMaxOut, l = i % 64;
    const int jj = blockIdx.x * 64 + l;
    const float s = ((part[0][n][l] + part[1][n][l]) + part[2][n][l]) + part[3][n][l];
    if (jj < hid) {
      if (n < kRtrMaxOut) a.dw2[m][(int64_t)n * hid + jj] = s;
      else a.db1[m][jj] = s;
    }
  }
  if (blockIdx.x == 0) {
    // bias of layer 2: rows in order
    for (int n = threadIdx.x; n < N; n += 256) {
      float s = 0.0f;
      for (int r = 0; r < B; ++r) s += a.draw[m][(int64_t)r * N + n];
      a.db2[m][n] = s;
    }
    if (m == 0 && a.dpass) {
      for (int i = threadIdx.x; i < a.P * a.R; i += 256) {
        float s = 0.0f;
        for (int r = 0; r < B; ++r) s += a.dlbp[(int64_t)r * a.P * a.R + i];
        a.dpass[i] = s * a.inv_t;
      }
    }
  }
}

// pooled[b, c] = (sum_s h0[b, s, c]) / S, fp32 and bf16
__global__ void __launch_bounds__(256) rtr_pool_kernel(const float* h0, int S, int d, float* pooled, bf16* pooled_b) {
  const int c = blockIdx.x * 256 + threadIdx.x, b = blockIdx.y;
  if (c >= d) return;
  const float* p = h0 + (int64_t)b * S * d + c;
  float s = 0.0f;
  for (int i = 0; i < S; ++i) s += p[(int64_t)i * d];
  const float v = s / (float)S;
  pooled[(int64_t)b * d + c] = v;
  pooled_b[(int64_t)b * d + c] = f2bf(v);
}

// load = lambda_load (R sum_r mean_b(p)^2 - 1), cover = lambda_cover sum_r relu(cmin - ema_r)^2,
// depth = lambda_depth mean_b(expected_depth); mean_prob kept for the backward
__global__ void __launch_bounds__(256) rtr_aux_fwd_kernel(const float* probs, const float* edepth, const float* ema,
                                                          int B, int R, float cmin, float l_load, float l_cover,
                                                          float l_depth, float* mean_prob, float* out) {
  __shared__ float mp[kRtrMaxOut];
  const int t = threadIdx.x;
  if (t < R) {
    float s = 0.0f;
    for (int b = 0; b < B; ++b) s += probs[(int64_t)b * R + t];
    mp[t] = s / (float)B;
    mean_prob[t] = mp[t];
  }
  __syncthreads();
  if (t == 0) {
    float sq = 0.0f, cv = 0.0f;
    for (int r = 0; r < R; ++r) {
      sq += mp[r] * mp[r];
      const float g = cmin - ema[r];
      const float rl = g > 0.0f ? g : 0.0f;
      cv += rl * rl;
    }
    float e = 0.0f;
    for (int b = 0; b < B; ++b) e += edepth[b];
    out[0] = l_load * ((float)R * sq - 1.0f);
    out[1] = l_cover * cv;
    out[2] = l_depth * (e / (float)B);
  }
}

// d probs[b, r] = g_load lambda_load R 2 mean_prob[r] / B;  d expected_depth[b] = g_depth lambda_depth / B
__global__ void __launch_bounds__(256) rtr_aux_bwd_kernel(const float* mean_prob, const float* g, int B, int R,
                                                          float l_load, float l_depth, float* dprobs,
                                                          float* dedepth) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const float gl = g[0], gd = g[2];
  if (i < (int64_t)B * R) dprobs[i] = gl * l_load * (float)R * (2.0f * mean_prob[i % R]) / (float)B;
  if (i < B) dedepth[i] = gd * l_depth / (float)B;
}

}  // namespace

}  // namespace rte

using namespace rte;

extern "C" {

int rte_router_pool(const float* h0, int B, int S, int d, float* pooled, void* pooled_bf16, void* stream) {
  RTE_REQUIRE(B >= 0 && S >= 1 && d >= 1, "router_pool: bad sizes");
  RTE_REQUIRE(h0 && pooled && pooled_bf16, "router_pool: null argument");
  if (B == 0) return 0;
  hipLaunchKernelGGL(rtr_pool_kernel, dim3((d + 255) / 256, B), dim3(256), 0, static_cast<hipStream_t>(stream), h0,
                     S, d, pooled, static_cast<bf16*>(pooled_bf16));
  return check_launch("router_pool");
}

int rte_router_heads_fwd(const float* z1r, const float* z1d, int B, int hid, const float* w2r, const float* b2r,
                         int R, const float* w2d, const float* b2d, int D, const float* pass_bias, int P,
                         const int64_t* depth_values, float inv_t, int fixed_recipe, int fixed_depth, float* rlog,
                         float* rprob, int64_t* rid, float* ronehot, float* dlog, float* dprob, int64_t* did,
                         int64_t* depth, float* donehot, float* rent, float* dent, float* ent, float* edepth,
                         float* rlog_bp, float* rprob_bp, int64_t* rid_bp, float* ronehot_bp, void* stream) {
  RTE_REQUIRE(B >= 0 && hid >= 1 && hid <= kRtrMaxHid && R >= 1 && R <= kRtrMaxOut && D >= 1 && D <= kRtrMaxOut &&
                  P >= 0 && P <= kRtrMaxPass,
              "router_heads_fwd: sizes out of range (hid <= 4096, R, D <= 64, passes <= 16)");
  RTE_REQUIRE(fixed_recipe < R && fixed_depth < D, "router_heads_fwd: fixed id out of range");
  RTE_REQUIRE(z1r && z1d && w2r && b2r && w2d && b2d && depth_values && rlog && rprob && rid && ronehot && dlog &&
                  dprob && did && depth && donehot && rent && dent && ent && edepth,
              "router_heads_fwd: null argument");
  RTE_REQUIRE(P == 0 || (pass_bias && rlog_bp && rprob_bp && rid_bp && ronehot_bp), "router_heads_fwd: null pass output");
  if (B == 0) return 0;
  RtrFwd a{z1r, z1d, w2r, b2r, w2d, b2d, pass_bias, depth_values, B, hid, R, D, P, inv_t, fixed_recipe, fixed_depth,
           rlog, rprob, rid, ronehot, dlog, dprob, did, depth, donehot, rent, dent, ent, edepth, rlog_bp, rprob_bp,
           rid_bp, ronehot_bp};
  hipLaunchKernelGGL(rtr_heads_fwd_kernel, dim3(B), dim3(64), 0, static_cast<hipStream_t>(stream), a);
  return check_launch("router_heads_fwd");
}

int rte_router_heads_bwd(const float* rprob, const float* rprob_bp, const float* dprob, const int64_t* depth_values,
                         int B, int R, int D, int P, float inv_t, const float* g_rlog, const float* g_rprob,
                         const float* g_ronehot, const float* g_dlog, const float* g_dprob, const float* g_donehot,
                         const float* g_rent, const float* g_dent, const float* g_ent, const float* g_edepth,
                         const float* g_rlog_bp, const float* g_rprob_bp, const float* g_ronehot_bp, float* draw_r,
                         float* draw_d, float* dlbp, void* stream) {
  RTE_REQUIRE(B >= 0 && R >= 1 && R <= kRtrMaxOut && D >= 1 && D <= kRtrMaxOut && P >= 0 && P <= kRtrMaxPass,
              "router_heads_bwd: sizes out of range");
  RTE_REQUIRE(rprob && dprob && depth_values && draw_r && draw_d, "router_heads_bwd: null argument");
  RTE_REQUIRE(P == 0 || (rprob_bp && dlbp), "router_heads_bwd: null pass argument");
  if (B == 0) return 0;
  RtrBwd a{rprob, rprob_bp, dprob, depth_values, B, R, D, P, inv_t, g_rlog, g_rprob, g_ronehot, g_dlog, g_dprob,
           g_donehot, g_rent, g_dent, g_ent, g_edepth, g_rlog_bp, g_rprob_bp, g_ronehot_bp, draw_r, draw_d, dlbp};
  hipLaunchKernelGGL(rtr_heads_bwd_kernel, dim3(B), dim3(64), 0, static_cast<hipStream_t>(stream), a);
  return check_launch("router_heads_bwd");
}

int rte_router_mlp_bwd(const float* draw_r, const float* draw_d, const float* z1r, const float* z1d,
                       const float* w2r, const float* w2d, int B, int hid, int R, int D, const float* dlbp, int P,
                       float inv_t, void* dz1r, void* dz1d, float* db1r, float* db1d, float* dw2r, float* dw2d,
                       float* db2r, float* db2d, float* dpass, void* stream) {
  RTE_REQUIRE(B >= 0 && hid >= 1 && R >= 1 && R <= kRtrMaxOut && D >= 1 && D <= kRtrMaxOut && P >= 0 &&
                  P <= kRtrMaxPass,
              "router_mlp_bwd: sizes out of range");
  RTE_REQUIRE(draw_r && draw_d && z1r && z1d && w2r && w2d && dz1r && dz1d && db1r && db1d && dw2r && dw2d && db2r &&
                  db2d,
              "router_mlp_bwd: null argument");
  RTE_REQUIRE(P == 0 || !dpass || dlbp, "router_mlp_bwd: pass-bias gradient needs the per-pass logit gradients");
  if (B == 0) return 0;
  RtrMlpBwd a{{draw_r, draw_d}, {z1r, z1d}, {w2r, w2d}, {R, D}, B, hid, P, R, dlbp, inv_t,
              {static_cast<bf16*>(dz1r), static_cast<bf16*>(dz1d)}, {db1r, db1d}, {dw2r, dw2d}, {db2r, db2d},
              P > 0 ? dpass : nullptr};
  hipLaunchKernelGGL(rtr_mlp_bwd_kernel, dim3((hid + 63) / 64, 2), dim3(256), 0, static_cast<hipStream_t>(stream),
                     a);
  return check_launch("router_mlp_bwd");
}

int rte_router_aux_fwd(const float* probs, const float* edepth, const float* ema, int B, int R, float coverage_min,
                       float lambda_load, float lambda_cover, float lambda_depth, float* mean_prob, float* out,
                       void* stream) {
  RTE_REQUIRE(B >= 1 && R >= 1 && R <= kRtrMaxOut, "router_aux_fwd: sizes out of range (1 <= R <= 64)");
  RTE_REQUIRE(probs && edepth && ema && mean_prob && out, "router_aux_fwd: null argument");
  hipLaunchKernelGGL(rtr_aux_fwd_kernel, dim3(1), dim3(256), 0, static_cast<hipStream_t>(stream), probs, edepth, ema,
                     B, R, coverage_min, lambda_load, lambda_cover, lambda_depth, mean_prob, out);
  return check_launch("router_aux_fwd");
}

int rte_router_aux_bwd(const float* mean_prob, const float* grad_out, int B, int R, float lambda_load,
                       float lambda_depth, float* dprobs, float* dedepth, void* stream) {
  RTE_REQUIRE(B >= 1 && R >= 1 && R <= kRtrMaxOut, "router_aux_bwd: sizes out of range");
  RTE_REQUIRE(mean_prob && grad_out && dprobs && dedepth, "router_aux_bwd: null argument");
  const int64_t n = (int64_t)B * R > B ? (int64_t)B * R : B;
  hipLaunchKernelGGL(rtr_aux_bwd_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), mean_prob, grad_out, B, R, lambda_load, lambda_depth, dprobs,
                     dedepth);
  return check_launch("router_aux_bwd");
}

}  // extern "C"
