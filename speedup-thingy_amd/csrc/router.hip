// Per-sample recipe / depth router (rte/routing.py:80-188) and its auxiliary losses
// (rte/metrics.py:97-112) as a handful of launches instead of one torch kernel per elementwise op.
//
//   pooled  = mean_s h0[b, s, :]                                   (rtr_pool: fp32 + bf16 copy)
//   z1      = pooled W1^T + b1        (recipe and depth MLPs)      (the MFMA GEMM, bias epilogue)
//   raw     = silu(z1) W2^T + b2                                   \
//   logits  = raw * inv_t; probs = softmax; id = argmax(probs)      |  rtr_heads_fwd: one wave per
//   by pass: logits + pass_bias[t] * inv_t -> softmax, argmax       |  sample row, W2 through LDS
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
constexpr int kRtrMaxHid = 4096;  // hidden width of the router MLPs (a launch-size bound only)

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

constexpr int kRtrRows = 4;           // sample rows per workgroup (one wave each)
constexpr int kRtrWsFloats = 12288;   // LDS for W2 columns (both heads)
constexpr int kRtrMaxChunk = 512;     // hidden columns per staging pass

// Loads n float4 (n <= 256 * U) from src rows into registers in one batch, then hands each to
// put(i, value): every load of the batch is in flight before the first use.
template <int U, typename Src, typename Put>
__device__ __forceinline__ void rtr_stage4(int n, Src src, Put put) {
  float4 v[U];
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int i = threadIdx.x + 256 * u;
    if (i < n) v[u] = src(i);
  }
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int i = threadIdx.x + 256 * u;
    if (i < n) put(i, v[u]);
  }
}

// raw[w][o] for the workgroup's rows: W2 of both heads ([R + D] rows, column-major in LDS) and the
// rows' silu(z1) are staged in one batch of 16-byte loads per pass (every pass when hid fits:
// ch = min(hid, 512, 12288 / (R + D)) columns); lane o of wave w sums output o over the columns in
// order (lanes o and o + 64 when R + D > 64).
__global__ void __launch_bounds__(256) rtr_heads_fwd_kernel(RtrFwd a) {
  __shared__ float ws[kRtrWsFloats];
  __shared__ float act[kRtrRows][2][kRtrMaxChunk];
  __shared__ float raws[kRtrRows][2 * kRtrMaxOut];
  const int t = threadIdx.x, w = t >> 6, lane = t & 63;
  const int b0 = blockIdx.x * kRtrRows, NO = a.R + a.D, hid = a.hid;
  int ch = kRtrWsFloats / NO;
  ch = (ch < kRtrMaxChunk ? ch : kRtrMaxChunk) & ~3;
  float acc0 = 0.0f, acc1 = 0.0f;
  for (int j0 = 0; j0 < hid; j0 += ch) {
    const int nc = hid - j0 < ch ? hid - j0 : ch;  // a multiple of 4
    const int q4 = nc / 4;
    __syncthreads();
    rtr_stage4<12>(
        NO * q4,
        [&](int i) {
          const int o = i / q4, c = 4 * (i % q4);
          const float* src = o < a.R ? a.w2r + (int64_t)o * hid : a.w2d + (int64_t)(o - a.R) * hid;
          return *reinterpret_cast<const float4*>(src + j0 + c);
        },
        [&](int i, float4 v) {
          const int o = i / q4, c = 4 * (i % q4);
          ws[(c + 0) * NO + o] = v.x;
          ws[(c + 1) * NO + o] = v.y;
          ws[(c + 2) * NO + o] = v.z;
          ws[(c + 3) * NO + o] = v.w;
        });
    rtr_stage4<4>(
        kRtrRows * 2 * q4,
        [&](int i) {
          const int r = i / (2 * q4), m = (i / q4) & 1, c = 4 * (i % q4);
          const int row = b0 + r < a.B ? b0 + r : a.B - 1;
          return *reinterpret_cast<const float4*>((m ? a.z1d : a.z1r) + (int64_t)row * hid + j0 + c);
        },
        [&](int i, float4 v) {
          const int r = i / (2 * q4), m = (i / q4) & 1, c = 4 * (i % q4);
          act[r][m][c + 0] = rtr_silu(v.x);
          act[r][m][c + 1] = rtr_silu(v.y);
          act[r][m][c + 2] = rtr_silu(v.z);
          act[r][m][c + 3] = rtr_silu(v.w);
        });
    __syncthreads();
    if (lane < NO) {
      const float* x = act[w][lane < a.R ? 0 : 1];
#pragma unroll 16
      for (int c = 0; c < nc; ++c) acc0 += x[c] * ws[c * NO + lane];
    }
    if (lane + 64 < NO) {
      const float* x = act[w][lane + 64 < a.R ? 0 : 1];
#pragma unroll 16
      for (int c = 0; c < nc; ++c) acc1 += x[c] * ws[c * NO + lane + 64];
    }
  }
  if (lane < NO) raws[w][lane] = acc0 + (lane < a.R ? a.b2r[lane] : a.b2d[lane - a.R]);
  if (lane + 64 < NO) raws[w][lane + 64] = acc1 + (lane + 64 < a.R ? a.b2r[lane + 64] : a.b2d[lane + 64 - a.R]);
  __syncthreads();
  const int b = b0 + w;
  if (b >= a.B) return;  // whole wave: the heads below use only wave-level reductions
  const float* raw = raws[w];
  const int R = a.R, D = a.D;
  const int64_t rb = (int64_t)b * R, db = (int64_t)b * D;
  // recipe head
  const float lg = lane < R ? raw[lane] * a.inv_t : 0.0f;
  if (lane < R) a.rlog[rb + lane] = lg;
  float re = 0.0f;
  rtr_head_row(lg, lane, R, a.fixed_recipe, a.rprob + rb, a.rid + b, a.ronehot + rb, &re);
  // per-pass recipe heads
  for (int tp = 0; tp < a.P; ++tp) {
    const int64_t o = ((int64_t)b * a.P + tp) * R;
    const float l2 = lane < R ? lg + a.pass_bias[tp * R + lane] * a.inv_t : 0.0f;
    if (lane < R) a.rlog_bp[o + lane] = l2;
    rtr_head_row(l2, lane, R, a.fixed_recipe, a.rprob_bp + o, a.rid_bp + (int64_t)b * a.P + tp, a.ronehot_bp + o,
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

constexpr int kRtrStage = 8192;  // fp32 values per LDS staging pass of a column sum

// out[c] = (mul sum_{r < rows} src[r cols + c]) / div for c < cols <= 1024, by one workgroup of
// 256 threads: rows are staged through LDS (16-byte loads when cols % 4 == 0), each column summed
// in row order.
__device__ void rtr_colsum_block(const float* src, int rows, int cols, float mul, float div, float* out,
                                 float* stage) {
  const int t = threadIdx.x;
  float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  const int chunk = kRtrStage / cols;
  for (int r0 = 0; r0 < rows; r0 += chunk) {
    const int nr = rows - r0 < chunk ? rows - r0 : chunk;
    const int n = nr * cols;
    const float* s0 = src + (int64_t)r0 * cols;
    __syncthreads();
    if (cols % 4 == 0) {
      rtr_stage4<8>(
          n / 4, [&](int i) { return *reinterpret_cast<const float4*>(s0 + 4 * i); },
          [&](int i, float4 v) { *reinterpret_cast<float4*>(stage + 4 * i) = v; });
    } else {
#pragma unroll 8
      for (int i = t; i < n; i += 256) stage[i] = s0[i];
    }
    __syncthreads();
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int c = t + 256 * q;
      if (c < cols) {
        float s = acc[q];
#pragma unroll 8
        for (int r = 0; r < nr; ++r) s += stage[r * cols + c];
        acc[q] = s;
      }
    }
  }
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const int c = t + 256 * q;
    if (c < cols) out[c] = (acc[q] * mul) / div;
  }
}

// grid (max(hid / 64, 3), 3), 256 threads.  y = 0, 1 (recipe, depth MLP): thread column
// j = 64 blockIdx.x + lane; each RC-row chunk of d raw logits and z1[:, block columns] is staged
// in LDS in one batch of loads, wave w takes rows w RC/4 .. (w + 1) RC/4 - 1 and the waves'
// partial sums meet in LDS in wave order.  y = 2: x = 0, 1 the layer-2 bias gradients, x = 2 the
// pass-bias gradient (column sums).
template <int NB, int RC>
__global__ void __launch_bounds__(256) rtr_mlp_bwd_kernel(RtrMlpBwd a) {
  constexpr int kMain = RC * NB + RC * 64 + 4 * (NB + 1) * 64;
  __shared__ __align__(16) float lds[kMain > kRtrStage ? kMain : kRtrStage];
  float* sd = lds;                                              // [RC][N]
  float (*zs)[64] = reinterpret_cast<float (*)[64]>(lds + RC * NB);  // [RC][64]
  float (*part)[NB + 1][64] = reinterpret_cast<float (*)[NB + 1][64]>(lds + RC * NB + RC * 64);
  const int t = threadIdx.x, lane = t & 63, w = t >> 6;
  const int B = a.B, hid = a.hid;
  if (blockIdx.y == 2) {
    if (blockIdx.x < 2) rtr_colsum_block(a.draw[blockIdx.x], B, a.N[blockIdx.x], 1.0f, 1.0f, a.db2[blockIdx.x], lds);
    else if (blockIdx.x == 2 && a.dpass) rtr_colsum_block(a.dlbp, B, a.P * a.R, a.inv_t, 1.0f, a.dpass, lds);
    return;
  }
  if (blockIdx.x * 64 >= hid) return;
  const int m = blockIdx.y, N = a.N[m];
  const int j = blockIdx.x * 64 + lane;
  const bool onj = j < hid;
  float w2c[NB];
  float dw2[NB];
#pragma unroll
  for (int n = 0; n < NB; ++n) {
    w2c[n] = (n < N && onj) ? a.w2[m][(int64_t)n * hid + j] : 0.0f;
    dw2[n] = 0.0f;
  }
  float db1 = 0.0f;
  const int c0 = blockIdx.x * 64;
  const int ncol = hid - c0 < 64 ? hid - c0 : 64;  // a multiple of 4
  for (int r0 = 0; r0 < B; r0 += RC) {
    const int rows = B - r0 < RC ? B - r0 : RC;
    const float* dr = a.draw[m] + (int64_t)r0 * N;
    const float* zr = a.z1[m] + (int64_t)r0 * hid + c0;
    __syncthreads();
    rtr_stage4<RC / 16>(
        rows * 16, [&](int i) {
          const int rr = i >> 4, c = 4 * (i & 15);
          return c < ncol ? *reinterpret_cast<const float4*>(zr + (int64_t)rr * hid + c) : make_float4(0, 0, 0, 0);
        },
        [&](int i, float4 v) { *reinterpret_cast<float4*>(&zs[i >> 4][4 * (i & 15)]) = v; });
#pragma unroll 8
    for (int i = t; i < rows * N; i += 256) sd[i] = dr[i];
    __syncthreads();
    const int rlo = w * (RC / 4), rhi = rlo + RC / 4 < rows ? rlo + RC / 4 : rows;
#pragma unroll 4
    for (int rr = rlo; rr < rhi; ++rr) {
      const float z = zs[rr][lane];
      const float sg = 1.0f / (1.0f + expf(-z));
      const float act = rtr_silu(z);
      float da = 0.0f;
#pragma unroll
      for (int n = 0; n < NB; ++n)
        if (n < N) {
          const float g = sd[rr * N + n];
          da += g * w2c[n];
          dw2[n] += g * act;
        }
      const float dz = da * (sg * (1.0f + z * (1.0f - sg)));
      if (onj) a.dz1[m][(int64_t)(r0 + rr) * hid + j] = f2bf(dz);
      db1 += dz;
    }
  }
  __syncthreads();
#pragma unroll
  for (int n = 0; n < NB; ++n)
    if (n < N) part[w][n][lane] = dw2[n];
  part[w][NB][lane] = db1;
  __syncthreads();
  for (int i = t; i < (N + 1) * 64; i += 256) {
    const int n = i / 64 < N ? i / 64 : NB, l = i % 64;
    const int jj = c0 + l;
    const float s = ((part[0][n][l] + part[1][n][l]) + part[2][n][l]) + part[3][n][l];
    if (jj < hid) {
      if (n < NB) a.dw2[m][(int64_t)n * hid + jj] = s;
      else a.db1[m][jj] = s;
    }
  }
}

// pooled[b, c] = (sum_s h0[b, s, c]) / S, fp32 and bf16.  Block: 64 columns x 4 sequence
// quarters (16 loads in flight per thread), quarters added in order.
__global__ void __launch_bounds__(256) rtr_pool_kernel(const float* h0, int S, int d, float* pooled, bf16* pooled_b) {
  __shared__ float part[4][64];
  const int lane = threadIdx.x & 63, q = threadIdx.x >> 6;
  const int c = blockIdx.x * 64 + lane, b = blockIdx.y;
  const int per = (S + 3) / 4, s0 = q * per < S ? q * per : S, s1 = s0 + per < S ? s0 + per : S;
  float s = 0.0f;
  if (c < d) {
    const float* p = h0 + (int64_t)b * S * d + c;
    int i = s0;
    for (; i + 16 <= s1; i += 16) {
      float v[16];
#pragma unroll
      for (int u = 0; u < 16; ++u) v[u] = p[(int64_t)(i + u) * d];
#pragma unroll
      for (int u = 0; u < 16; ++u) s += v[u];
    }
    for (; i < s1; ++i) s += p[(int64_t)i * d];
  }
  part[q][lane] = s;
  __syncthreads();
  if (q == 0 && c < d) {
    const float v = (((part[0][lane] + part[1][lane]) + part[2][lane]) + part[3][lane]) / (float)S;
    pooled[(int64_t)b * d + c] = v;
    pooled_b[(int64_t)b * d + c] = f2bf(v);
  }
}

// load = lambda_load (R sum_r mean_b(p)^2 - 1), cover = lambda_cover sum_r relu(cmin - ema_r)^2,
// depth = lambda_depth mean_b(expected_depth); mean_prob kept for the backward
__global__ void __launch_bounds__(256) rtr_aux_fwd_kernel(const float* probs, const float* edepth, const float* ema,
                                                          int B, int R, float cmin, float l_load, float l_cover,
                                                          float l_depth, float* mean_prob, float* out) {
  __shared__ __align__(16) float stage[kRtrStage];
  __shared__ float mp[kRtrMaxOut];
  __shared__ float em[1];
  rtr_colsum_block(probs, B, R, 1.0f, (float)B, mp, stage);
  rtr_colsum_block(edepth, B, 1, 1.0f, (float)B, em, stage);
  __syncthreads();
  const int t = threadIdx.x;
  if (t < R) mean_prob[t] = mp[t];
  if (t == 0) {
    float sq = 0.0f, cv = 0.0f;
    for (int r = 0; r < R; ++r) {
      sq += mp[r] * mp[r];
      const float g = cmin - ema[r];
      const float rl = g > 0.0f ? g : 0.0f;
      cv += rl * rl;
    }
    out[0] = l_load * ((float)R * sq - 1.0f);
    out[1] = l_cover * cv;
    out[2] = l_depth * em[0];
  }
}

// d probs[b, r] = g_load lambda_load R 2 mean_prob[r] / B;  d expected_depth[b] = g_depth lambda_depth / B
// (a null gradient is zero)
__global__ void __launch_bounds__(256) rtr_aux_bwd_kernel(const float* mean_prob, const float* g_load,
                                                          const float* g_depth, int B, int R, float l_load,
                                                          float l_depth, float* dprobs, float* dedepth) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const float gl = g_load ? g_load[0] : 0.0f, gd = g_depth ? g_depth[0] : 0.0f;
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
  hipLaunchKernelGGL(rtr_pool_kernel, dim3((d + 63) / 64, B), dim3(256), 0, static_cast<hipStream_t>(stream), h0,
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
  RTE_REQUIRE(hid % 4 == 0, "router_heads_fwd: hidden width must be a multiple of 4");
  RTE_REQUIRE(fixed_recipe < R && fixed_depth < D, "router_heads_fwd: fixed id out of range");
  RTE_REQUIRE(z1r && z1d && w2r && b2r && w2d && b2d && depth_values && rlog && rprob && rid && ronehot && dlog &&
                  dprob && did && depth && donehot && rent && dent && ent && edepth,
              "router_heads_fwd: null argument");
  RTE_REQUIRE(P == 0 || (pass_bias && rlog_bp && rprob_bp && rid_bp && ronehot_bp), "router_heads_fwd: null pass output");
  if (B == 0) return 0;
  RtrFwd a{z1r, z1d, w2r, b2r, w2d, b2d, pass_bias, depth_values, B, hid, R, D, P, inv_t, fixed_recipe, fixed_depth,
           rlog, rprob, rid, ronehot, dlog, dprob, did, depth, donehot, rent, dent, ent, edepth, rlog_bp, rprob_bp,
           rid_bp, ronehot_bp};
  hipLaunchKernelGGL(rtr_heads_fwd_kernel, dim3((B + kRtrRows - 1) / kRtrRows), dim3(256), 0,
                     static_cast<hipStream_t>(stream), a);
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
  RTE_REQUIRE(hid % 4 == 0, "router_mlp_bwd: hidden width must be a multiple of 4");
  RTE_REQUIRE(draw_r && draw_d && z1r && z1d && w2r && w2d && dz1r && dz1d && db1r && db1d && dw2r && dw2d && db2r &&
                  db2d,
              "router_mlp_bwd: null argument");
  RTE_REQUIRE(P == 0 || !dpass || dlbp, "router_mlp_bwd: pass-bias gradient needs the per-pass logit gradients");
  if (B == 0) return 0;
  RtrMlpBwd a{{draw_r, draw_d}, {z1r, z1d}, {w2r, w2d}, {R, D}, B, hid, P, R, dlbp, inv_t,
              {static_cast<bf16*>(dz1r), static_cast<bf16*>(dz1d)}, {db1r, db1d}, {dw2r, dw2d}, {db2r, db2d},
              P > 0 ? dpass : nullptr};
  const int nbx = (hid + 63) / 64 > 3 ? (hid + 63) / 64 : 3;
  const int nmax = R > D ? R : D;
  const dim3 grid(nbx, 3);
  hipStream_t st = static_cast<hipStream_t>(stream);
  if (nmax <= 16) hipLaunchKernelGGL((rtr_mlp_bwd_kernel<16, 128>), grid, dim3(256), 0, st, a);
  else if (nmax <= 32) hipLaunchKernelGGL((rtr_mlp_bwd_kernel<32, 128>), grid, dim3(256), 0, st, a);
  else hipLaunchKernelGGL((rtr_mlp_bwd_kernel<64, 64>), grid, dim3(256), 0, st, a);
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

int rte_router_aux_bwd(const float* mean_prob, const float* g_load, const float* g_depth, int B, int R,
                       float lambda_load, float lambda_depth, float* dprobs, float* dedepth, void* stream) {
  RTE_REQUIRE(B >= 1 && R >= 1 && R <= kRtrMaxOut, "router_aux_bwd: sizes out of range");
  RTE_REQUIRE(mean_prob && dprobs && dedepth, "router_aux_bwd: null argument");
  const int64_t n = (int64_t)B * R > B ? (int64_t)B * R : B;
  hipLaunchKernelGGL(rtr_aux_bwd_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), mean_prob, g_load, g_depth, B, R, lambda_load, lambda_depth,
                     dprobs, dedepth);
  return check_launch("router_aux_bwd");
}

}  // extern "C"
