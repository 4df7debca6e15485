// Token cross-entropy over full-vocabulary logits (rte/models.py:73-75,
// rte/kernels/reference.py:146-147), forward and backward, one wave64 per row.
//
//  ce_fwd : lse[t] = logsumexp(logits[t, :]), loss[t] = lse[t] - logits[t, target[t]]
//           (target < 0: ignored row, loss 0)
//  ce_bwd : dlogits[t, v] = g[t] * (softmax[t, v] - [v == target]) + extra[t, v]
//           written as bf16 for the LM-head backward GEMMs (the fp32->bf16 cast fused)
//
// Control-variate audit correction (rte/audit.py:245-387), fused into one workgroup:
//  audit_fwd : per-sample sums of the hot and exact token losses, residual r = exact - hot,
//              clamp to the clip, corrected[m] = hot[m] + r/p[m] on audited rows, and the
//              residual statistics, all in a fixed reduction order
//  audit_bwd : dhot_tok = g (1 - c), dexact_tok = g c broadcast over the sequence, with
//              c = 1/p on audited rows whose residual is inside the clip, else 0
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

// The same for V <= 4 * 64 * NV with V % 4 == 0: the row is read once into registers and both
// passes run over them in the order of ce_fwd_kernel (bitwise the same results).
template <int NV>
__global__ void __launch_bounds__(256) ce_fwd_reg_kernel(const float* __restrict__ logits, int64_t ld, int T, int V,
                                                         const int64_t* __restrict__ targets,
                                                         float* __restrict__ loss, float* __restrict__ lse_out) {
  const int lane = threadIdx.x & 63;
  const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= T) return;
  const float* row = logits + (int64_t)t * ld;
  float4 v[NV];
#pragma unroll
  for (int i = 0; i < NV; ++i) {
    const int c = lane * 4 + 256 * i;
    v[i] = c < V ? *reinterpret_cast<const float4*>(row + c) : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
  }
  float mx = -INFINITY;
#pragma unroll
  for (int i = 0; i < NV; ++i)
    if (lane * 4 + 256 * i < V) mx = fmaxf(mx, fmaxf(fmaxf(v[i].x, v[i].y), fmaxf(v[i].z, v[i].w)));
  mx = wave_max(mx);
  float s = 0.0f;
#pragma unroll
  for (int i = 0; i < NV; ++i)
    if (lane * 4 + 256 * i < V)
      s += __expf(v[i].x - mx) + __expf(v[i].y - mx) + __expf(v[i].z - mx) + __expf(v[i].w - mx);
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
                                                     const float* __restrict__ extra,
                                                     const int64_t* __restrict__ ext_ids, int ext_k, int ext_S,
                                                     bf16* __restrict__ dlogits) {
  const int lane = threadIdx.x & 63;
  const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= T) return;
  const float* row = logits + (int64_t)t * ld;
  const float* ex = nullptr;
  int j0 = 0;
  if (extra && !ext_ids) {
    ex = extra + (int64_t)t * V;
  } else if (extra) {  // rows of the samples ext_ids (ext_S tokens each): the first match, more below
    const int64_t smp = t / ext_S;
    for (; j0 < ext_k && ext_ids[j0] != smp; ++j0) {
    }
    if (j0 < ext_k) ex = extra + ((int64_t)j0 * ext_S + t % ext_S) * V;
  }
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
      if (ex) {
        e4 = *reinterpret_cast<const float4*>(ex + c);
        if (ext_ids) {  // a sample listed again adds its rows in list order (index_add_ order)
          const float4 z = make_float4(0.f, 0.f, 0.f, 0.f);
          e4 = make_float4(z.x + e4.x, z.y + e4.y, z.z + e4.z, z.w + e4.w);
          for (int j = j0 + 1; j < ext_k; ++j) {
            if (ext_ids[j] != t / ext_S) continue;
            const float4 f = *reinterpret_cast<const float4*>(extra + ((int64_t)j * ext_S + t % ext_S) * V + c);
            e4.x += f.x; e4.y += f.y; e4.z += f.z; e4.w += f.w;
          }
        }
      }
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
      o.x = pack_bf2(d[0], d[1]);
      o.y = pack_bf2(d[2], d[3]);
      *reinterpret_cast<uint2*>(out + c) = o;
    } else {
      for (int i = 0; i < n; ++i) out[c + i] = f2bf(d[i]);
    }
  }
}

constexpr int kAuditThreads = 1024;
constexpr int kAuditMaxRows = 8192;

// Sum of row r of a [rows, S] matrix by one wave, fixed lane order and a fixed xor tree.
__device__ __forceinline__ float wave_row_sum(const float* __restrict__ x, int64_t r, int S, int lane) {
  const float* row = x + r * (int64_t)S;
  float acc = 0.0f;
  for (int s = lane; s < S; s += 64) acc += row[s];
  return wave_sum(acc);
}

// Block-wide double sum in fixed order: per-wave xor tree, then wave partials in index order.
__device__ double block_sum(double v, double* red) {
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  __syncthreads();
  if (lane == 0) red[w] = v;
  __syncthreads();
  double t = 0.0;
  for (int i = 0; i < kAuditThreads / 64; ++i) t += red[i];
  return t;
}

__global__ void __launch_bounds__(kAuditThreads) audit_fwd_kernel(
    const float* __restrict__ hot_tok, const float* __restrict__ exact_tok, int B, int S,
    const int64_t* __restrict__ idx, int A, const float* __restrict__ p, float clip, int grad_corrected,
    float* __restrict__ corrected, float* __restrict__ exact_ps, float* __restrict__ coef,
    float* __restrict__ stats) {
  __shared__ float hot_ps[kAuditMaxRows];
  __shared__ double red[kAuditThreads / 64];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = kAuditThreads / 64;
  for (int m = wave; m < B; m += nw) {
    const float v = wave_row_sum(hot_tok, m, S, lane);
    if (lane == 0) hot_ps[m] = v;
  }
  for (int a = wave; a < A; a += nw) {
    const float v = wave_row_sum(exact_tok, a, S, lane);
    if (lane == 0) exact_ps[a] = v;
  }
  __syncthreads();  // makes exact_ps (global) visible to the whole workgroup
  // residuals: sum r, sum (hot + clip(r)/p) and, in a second pass, sum (r - mean)^2
  double sr = 0.0, sm = 0.0;
  bool bad = false;
  for (int a = threadIdx.x; a < A; a += kAuditThreads) {
    const int64_t m = idx[a];
    if (m < 0 || m >= B) { bad = true; continue; }
    const float h = hot_ps[m];
    const float r = exact_ps[a] - h;
    const float rc = fminf(fmaxf(r, -clip), clip);
    const float ps = fmaxf(p[m], 1e-12f);
    sr += (double)r;
    sm += (double)h + (double)rc / (double)ps;
  }
  const double bad_any = block_sum(bad ? 1.0 : 0.0, red);
  sr = block_sum(sr, red);
  sm = block_sum(sm, red);
  const double mean = A > 0 ? sr / A : 0.0;
  double sq = 0.0;
  for (int a = threadIdx.x; a < A; a += kAuditThreads) {
    const int64_t m = idx[a];
    if (m < 0 || m >= B) continue;
    const double dv = (double)(exact_ps[a] - hot_ps[m]) - mean;
    sq += dv * dv;
  }
  sq = block_sum(sq, red);
  // corrected rows: every row keeps its hot sum except the audited ones (distinct rows, so
  // the thread of row a is the only reader and writer of hot_ps[idx[a]] from here on)
  for (int m = threadIdx.x; m < B; m += kAuditThreads) coef[m] = 0.0f;
  __syncthreads();
  for (int a = threadIdx.x; a < A; a += kAuditThreads) {
    const int64_t m = idx[a];
    float c = 0.0f;
    if (m >= 0 && m < B) {
      const float h = hot_ps[m];
      const float r = exact_ps[a] - h;
      const float ps = fmaxf(p[m], 1e-12f);
      const bool inside = r >= -clip && r <= clip;
      c = (grad_corrected && inside) ? 1.0f / ps : 0.0f;
      if (grad_corrected) hot_ps[m] = h + fminf(fmaxf(r, -clip), clip) / ps;
      coef[m] = c;
    }
    coef[B + a] = c;
  }
  __syncthreads();
  for (int m = threadIdx.x; m < B; m += kAuditThreads) corrected[m] = hot_ps[m];
  if (threadIdx.x == 0) {
    const float nan = __builtin_nanf("");
    const bool poison = bad_any > 0.0;
    const double var = A > 0 ? sq / A : 0.0;
    stats[0] = poison ? nan : (float)mean;
    stats[1] = poison ? nan : (float)sqrt(var);
    stats[2] = poison ? nan : (float)var;
    stats[3] = poison ? nan : (A > 0 ? (float)(sm / A) : 0.0f);
  }
}

__global__ void __launch_bounds__(256) audit_bwd_kernel(const float* __restrict__ g, int B, int S,
                                                        const int64_t* __restrict__ idx, int A,
                                                        const float* __restrict__ coef, float* __restrict__ dhot_tok,
                                                        float* __restrict__ dexact_tok) {
  // one thread per token of the hot rows, then one per token of the audited rows
  const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t nh = (int64_t)B * S;
  if (t < nh) {
    const int m = (int)(t / S);
    dhot_tok[t] = g[m] * (1.0f - coef[m]);
  } else if (dexact_tok && t < nh + (int64_t)A * S) {
    const int64_t u = t - nh;
    const int a = (int)(u / S);
    const int64_t m = idx[a];
    dexact_tok[u] = (m >= 0 && m < B) ? g[m] * coef[B + a] : 0.0f;
  }
}

}  // namespace

int audit_fwd(const float* hot_tok, const float* exact_tok, int B, int S, const int64_t* idx, int A, const float* p,
              float clip, int grad_corrected, float* corrected, float* exact_ps, float* coef, float* stats,
              hipStream_t s) {
  RTE_REQUIRE(B >= 1 && B <= kAuditMaxRows, "audit_fwd: sample count must be in [1, %d]", kAuditMaxRows);
  RTE_REQUIRE(A >= 0 && A <= B && S >= 1, "audit_fwd: need 0 <= audited rows <= samples and S >= 1");
  RTE_REQUIRE(!(clip < 0.0f), "audit_fwd: clip must be >= 0 (inf for none)");
  hipLaunchKernelGGL(audit_fwd_kernel, dim3(1), dim3(kAuditThreads), 0, s, hot_tok, exact_tok, B, S, idx, A, p,
                     clip, grad_corrected, corrected, exact_ps, coef, stats);
  return check_launch("audit_fwd");
}

int audit_bwd(const float* g, int B, int S, const int64_t* idx, int A, const float* coef, float* dhot_tok,
              float* dexact_tok, hipStream_t s) {
  RTE_REQUIRE(B >= 1 && A >= 0 && A <= B && S >= 1, "audit_bwd: bad sizes");
  const int64_t n = (int64_t)B * S + (dexact_tok ? (int64_t)A * S : 0);
  hipLaunchKernelGGL(audit_bwd_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, g, B, S, idx, A, coef,
                     dhot_tok, dexact_tok);
  return check_launch("audit_bwd");
}

int ce_fwd(const float* logits, int64_t ld, int T, int V, const int64_t* targets, float* loss, float* lse,
           hipStream_t s) {
  RTE_REQUIRE(V >= 1 && ld >= V && ld % 4 == 0, "ce_fwd: logits row stride must be >= V and a multiple of 4");
  RTE_REQUIRE(((uintptr_t)logits & 15) == 0, "ce_fwd: logits must be 16-byte aligned");
  if (T == 0) return 0;
  if (V % 4 == 0 && V <= 4 * 64 * 8)
    hipLaunchKernelGGL(ce_fwd_reg_kernel<8>, dim3((T + 3) / 4), dim3(256), 0, s, logits, ld, T, V, targets, loss,
                       lse);
  else
    hipLaunchKernelGGL(ce_fwd_kernel, dim3((T + 3) / 4), dim3(256), 0, s, logits, ld, T, V, targets, loss, lse);
  return check_launch("ce_fwd");
}

int ce_bwd(const float* logits, int64_t ld, int T, int V, const int64_t* targets, const float* lse, const float* g,
           const float* extra, const int64_t* ext_ids, int ext_k, int ext_S, bf16* dlogits, hipStream_t s) {
  RTE_REQUIRE(V % 4 == 0 && ld % 4 == 0, "ce_bwd: V and the row stride must be multiples of 4");
  RTE_REQUIRE(!ext_ids || (extra && ext_k >= 1 && ext_S >= 1),
              "ce_bwd: extra rows by sample need the rows, a sample count and tokens per sample");
  RTE_REQUIRE(((uintptr_t)logits & 15) == 0 && ((uintptr_t)extra & 15) == 0 && ((uintptr_t)dlogits & 7) == 0,
              "ce_bwd: misaligned buffers");
  if (T == 0) return 0;
  hipLaunchKernelGGL(ce_bwd_kernel, dim3((T + 3) / 4), dim3(256), 0, s, logits, ld, T, V, targets, lse, g, extra,
                     ext_ids, ext_ids ? ext_k : 0, ext_ids ? ext_S : 1, dlogits);
  return check_launch("ce_bwd");
}

}  // namespace rte
