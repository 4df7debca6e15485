// Causal self-attention core for head_dim 32, 64 or 128 on gfx950 (the SDPA call behind k_flash_causal_dense /
// k_flash_causal_grouped, rte/kernels/optimized.py:75-91; attention of rte/layers.py:53-75 and
// the banked attention of rte/layers.py:659-730), forward and backward, softmax scale given.
//
// Layouts: q, k, v bf16 [B, H, S, hd] contiguous (what the QKV+RoPE GEMM epilogue writes);
// out and dout bf16 [B, S, H, hd] (token-major: the O-projection's input rows); dq, dk, dv bf16
// [B, H, S, hd]; lse f32 [B, H, S] in log2 units of the scaled scores (lse2 = max + log2(sum
// 2^(s - max)), s = q.k * scale * log2(e)).  Optional per-(b, h) output scale hs f32 [B * H]:
// out = hs * softmax(q k^T scale) v, the recipe head mask of the banked attention applied to v.
//
// Work split: one wave per 32-row block of one (b, h); no workgroup barriers.  Products use
// v_mfma_f32_32x32x16_bf16 with the operands arranged so that each lane owns one query (or key)
// row of the score block:
//   forward  S^T = K Q^T, O^T += V^T P^T      (lane = query: row max / sum are one xor-32 step)
//   dQ       S^T = K Q^T, dP^T = V dO^T, dQ^T += K^T dS^T            (lane = query)
//   dK, dV   S = Q K^T, dP = dO V^T, dV^T += dO^T P, dK^T += Q^T dS   (lane = key)
// The backward is one launch: each wave forms dK, dV of its key block, then dQ of its query block.
// The score registers of a lane are fed back as the MFMA operand of the second product
// directly: a 32x32 MFMA output register r of lane l holds row 8(r/4) + 4(l/32) + r%4, so the
// 8 registers 8t..8t+7 of half h hold rows 16t + 4h + {0..3, 8..11}; the other operand reads
// its k rows in that same order from a wave-private LDS block with ds_read_b64_tr_b16 (rows
// kb..kb+3 and kb+8..kb+11 of a column), so no score ever goes through memory.
// Reductions (softmax sums, dQ / dK / dV over blocks) run in a fixed order: results are
// bitwise repeatable.
#include "common.hpp"

namespace rte {

namespace {

// LDS row pitch (bf16) of a wave's 32 x HD block: 16 bytes of padding per row
template <int HD>
constexpr int pitch() { return HD + 8; }
constexpr float kLog2e = 1.4426950408889634f;

typedef short short4_v __attribute__((ext_vector_type(4)));
typedef short short8_v __attribute__((ext_vector_type(8)));
typedef unsigned int u32x4_v __attribute__((ext_vector_type(4)));

__device__ __forceinline__ bf16x8_v ld16(const bf16* p) {
  return *reinterpret_cast<const bf16x8_v*>(p);
}

// bf16 of v[O .. O+7] (compile-time offset keeps v in registers)
template <int O>
__device__ __forceinline__ bf16x8_v pack8(const float (&v)[16]) {
  uint4 u;
  u.x = pack_bf2(v[O], v[O + 1]);
  u.y = pack_bf2(v[O + 2], v[O + 3]);
  u.z = pack_bf2(v[O + 4], v[O + 5]);
  u.w = pack_bf2(v[O + 6], v[O + 7]);
  return __builtin_bit_cast(bf16x8_v, u);
}

__device__ __forceinline__ float dot8(u32x4_v a, u32x4_v b) {
  float s = 0.0f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    s += __uint_as_float(a[i] << 16) * __uint_as_float(b[i] << 16);
    s += __uint_as_float(a[i] & 0xffff0000u) * __uint_as_float(b[i] & 0xffff0000u);
  }
  return s;
}

__device__ __forceinline__ void wave_lds_fence() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

__device__ __forceinline__ short4_v tr_read(const bf16* lds) {
#if defined(__HIP_DEVICE_COMPILE__)
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) short4_v*)lds);
#else
  (void)lds;
  return short4_v{0, 0, 0, 0};
#endif
}

// MFMA operand holding column (cb + lane % 16) of rows kb..kb+3, kb+8..kb+11 of a wave's
// [32][pitch] LDS block.  ds_read_b64_tr_b16 (lane layout measured on gfx950): within a group
// of 16 lanes, lane s points at row kb + s / 4, columns cb + 4 (s % 4) .. +3, and lane i receives
// column cb + i of rows kb..kb+3.  kb and cb must be uniform over each 16-lane group.
template <int HD>
__device__ __forceinline__ bf16x8_v tr_frag(const bf16* blk, int kb, int cb, int lane) {
  constexpr int P = pitch<HD>();
  const int s = lane & 15;
  const bf16* p0 = blk + (kb + (s >> 2)) * P + cb + 4 * (s & 3);
  const short4_v lo = tr_read(p0);
  const short4_v hi = tr_read(p0 + 8 * P);
  const short8_v v = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
  return __builtin_bit_cast(bf16x8_v, v);
}

// Rows r0..r0+31 (clamped to S - 1) of a [rows][HD] bf16 matrix with row stride `ld` into a
// wave's LDS block (HD / 16 loads of 16 bytes per lane).
template <int HD>
__device__ __forceinline__ void load_block(const bf16* src, int64_t ld, int r0, int S, int lane,
                                           u32x4_v (&v)[HD / 16]) {
  constexpr int CPR = HD / 8;
#pragma unroll
  for (int u = 0; u < HD / 16; ++u) {
    const int c = lane + 64 * u, row = c / CPR, ch = c % CPR;
    const int r = r0 + row < S ? r0 + row : S - 1;
    v[u] = *reinterpret_cast<const u32x4_v*>(src + (int64_t)r * ld + ch * 8);
  }
}

template <int HD>
__device__ __forceinline__ void store_block(bf16* blk, int lane, const u32x4_v (&v)[HD / 16]) {
  constexpr int CPR = HD / 8;
#pragma unroll
  for (int u = 0; u < HD / 16; ++u) {
    const int c = lane + 64 * u, row = c / CPR, ch = c % CPR;
    *reinterpret_cast<u32x4_v*>(blk + row * pitch<HD>() + ch * 8) = v[u];
  }
}

// Lane l holds row (its query or key) l % 32 and, in block db, columns 32 db + 8 j + 4 (l / 32)
// + {0..3} of acc[db][4 j .. 4 j + 3]: written as 8-byte runs, times f.
// Backward outputs: row (b, h, s) of dq / dk / dv starts at p + b sb + h sh + s ss (the same
// strides for the three).  cs / sn (cos, sin [S, HD], optional): dq and dk rows leave rotated
// back by their position's RoPE angle, exactly as rope_bwd_pack does it (bf16 value first,
// then the rotation in fp32 with the same fma order), so the QKV backward reads them directly.
struct BwdOut {
  bf16 *dq, *dk, *dv;
  int64_t sb, sh, ss;
  const float *cs, *sn;
};

template <int NB>
__device__ __forceinline__ void store_rows_rot(bf16* row, const f32x16_v (&acc)[NB], float f, int hf,
                                               const float* cs, const float* sn) {
#pragma unroll
  for (int db = 0; db < NB; ++db)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int col = 32 * db + 8 * j + 4 * hf;
      float y[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) y[i] = bf2f(f2bf(acc[db][4 * j + i] * f));
      const float4 c = *reinterpret_cast<const float4*>(cs + col);
      const float4 sv = *reinterpret_cast<const float4*>(sn + col);
      const float r0 = fmaf(y[0], c.x, y[1] * sv.y), r1 = fmaf(y[1], c.y, -(y[0] * sv.x));
      const float r2 = fmaf(y[2], c.z, y[3] * sv.w), r3 = fmaf(y[3], c.w, -(y[2] * sv.z));
      uint2 w;
      w.x = pack_bf2(r0, r1);
      w.y = pack_bf2(r2, r3);
      *reinterpret_cast<uint2*>(row + col) = w;
    }
}

template <int NB>
__device__ __forceinline__ void store_rows(bf16* row, const f32x16_v (&acc)[NB], float f, int hf) {
#pragma unroll
  for (int db = 0; db < NB; ++db)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      uint2 w;
      w.x = pack_bf2(acc[db][4 * j] * f, acc[db][4 * j + 1] * f);
      w.y = pack_bf2(acc[db][4 * j + 2] * f, acc[db][4 * j + 3] * f);
      *reinterpret_cast<uint2*>(row + 32 * db + 8 * j + 4 * hf) = w;
    }
}

template <int HD>
__global__ void __launch_bounds__(256) attn_fwd_kernel(const bf16* __restrict__ q, const bf16* __restrict__ k,
                                                       const bf16* __restrict__ v, int BH, int H, int S, float c2,
                                                       const float* __restrict__ hscale, bf16* __restrict__ out,
                                                       float* __restrict__ lse) {
  constexpr int KS = HD / 16, NB = HD / 32, P = pitch<HD>();
  __shared__ __align__(16) bf16 vs[4][32 * P];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, l32 = lane & 31, hf = lane >> 5;
  const int nqb = (S + 31) / 32;
  const int task = blockIdx.x * 4 + wave;
  const int bh = task / nqb, qb = task - bh * nqb;
  if (bh >= BH) return;
  const int q0 = qb * 32, qi = q0 + l32;
  const int64_t base = (int64_t)bh * S * HD;
  bf16x8_v qf[KS];
  {
    const bf16* qp = q + base + (int64_t)(qi < S ? qi : S - 1) * HD + 8 * hf;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) qf[ks] = ld16(qp + 16 * ks);
  }
  f32x16_v o[NB];
#pragma unroll
  for (int r = 0; r < 16; ++r)
#pragma unroll
    for (int db = 0; db < NB; ++db) o[db][r] = 0.0f;
  float m = -INFINITY, lsum = 0.0f;
  bf16* blk = vs[wave];
  const int g1 = (lane >> 4) & 1;
  const int kend = S < q0 + 32 ? S : q0 + 32;  // causal: keys up to the block's last query
  for (int kb0 = 0; kb0 < kend; kb0 += 32) {
    bf16x8_v kf[KS];
    {
      const int kr = kb0 + l32 < S ? kb0 + l32 : S - 1;
      const bf16* kp = k + base + (int64_t)kr * HD + 8 * hf;
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) kf[ks] = ld16(kp + 16 * ks);
    }
    u32x4_v vr[KS];
    load_block<HD>(v + base, HD, kb0, S, lane, vr);
    f32x16_v st;
#pragma unroll
    for (int r = 0; r < 16; ++r) st[r] = 0.0f;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) st = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf[ks], qf[ks], st, 0, 0, 0);
    float p[16], mx = -INFINITY;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int key = kb0 + 8 * (r >> 2) + 4 * hf + (r & 3);
      p[r] = (key <= qi && key < S) ? st[r] * c2 : -INFINITY;
      mx = fmaxf(mx, p[r]);
    }
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
    const float mnew = fmaxf(m, mx);  // finite: key 0 is visible to every query
    const float alpha = exp2f(m - mnew);
    float rs = 0.0f;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      p[r] = exp2f(p[r] - mnew);
      rs += p[r];
    }
    rs += __shfl_xor(rs, 32, 64);
    lsum = lsum * alpha + rs;
    m = mnew;
#pragma unroll
    for (int r = 0; r < 16; ++r)
#pragma unroll
      for (int db = 0; db < NB; ++db) o[db][r] *= alpha;
    wave_lds_fence();  // the previous block's reads are done
    store_block<HD>(blk, lane, vr);
    wave_lds_fence();
    const bf16x8_v pb[2] = {pack8<0>(p), pack8<8>(p)};
#pragma unroll
    for (int db = 0; db < NB; ++db)
#pragma unroll
      for (int t = 0; t < 2; ++t)
        o[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(tr_frag<HD>(blk, 16 * t + 4 * hf, 32 * db + 16 * g1, lane), pb[t],
                                                        o[db], 0, 0, 0);
  }
  if (qi < S) {
    const int b = bh / H, h = bh - b * H;
    const float f = (hscale ? hscale[bh] : 1.0f) / lsum;
    store_rows(out + (((int64_t)b * S + qi) * H + h) * HD, o, f, hf);
    if (hf == 0) lse[(int64_t)bh * S + qi] = m + log2f(lsum);
  }
}

// dQ of one 32-query block (wave task `task`): loop over the key blocks up to the diagonal.
// blk: the wave's [32][pitch] LDS block.
template <int HD>
__device__ __forceinline__ void attn_bwd_dq_task(const bf16* __restrict__ q, const bf16* __restrict__ k,
                                                 const bf16* __restrict__ v, const bf16* __restrict__ out,
                                                 const bf16* __restrict__ dout, const float* __restrict__ lse,
                                                 int BH, int H, int S, float c2, float scale,
                                                 const float* __restrict__ hscale, const BwdOut& o, int task,
                                                 bf16* blk) {
  constexpr int KS = HD / 16, NB = HD / 32;
  const int lane = threadIdx.x & 63, l32 = lane & 31, hf = lane >> 5;
  const int nqb = (S + 31) / 32;
  const int bh = task / nqb, qb = task - bh * nqb;
  if (bh >= BH) return;
  const int b = bh / H, h = bh - b * H;
  const int q0 = qb * 32, qi = q0 + l32, qc = qi < S ? qi : S - 1;
  const int64_t base = (int64_t)bh * S * HD;
  const int64_t trow = (((int64_t)b * S + qc) * H + h) * HD;  // token-major row of out / dout
  bf16x8_v qf[KS], dof[KS];
  float dsum = 0.0f;
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) {
    const int d0 = 16 * ks + 8 * hf;
    qf[ks] = ld16(q + base + (int64_t)qc * HD + d0);
    const u32x4_v du = *reinterpret_cast<const u32x4_v*>(dout + trow + d0);
    dof[ks] = __builtin_bit_cast(bf16x8_v, du);
    dsum += dot8(du, *reinterpret_cast<const u32x4_v*>(out + trow + d0));
  }
  const float D = dsum + __shfl_xor(dsum, 32, 64);  // rowsum(dO * O)
  const float l2 = lse[(int64_t)bh * S + qc];
  const float hs = hscale ? hscale[bh] : 1.0f;
  f32x16_v acc[NB];
#pragma unroll
  for (int r = 0; r < 16; ++r)
#pragma unroll
    for (int db = 0; db < NB; ++db) acc[db][r] = 0.0f;
  const int g1 = (lane >> 4) & 1;
  const int kend = S < q0 + 32 ? S : q0 + 32;
  for (int kb0 = 0; kb0 < kend; kb0 += 32) {
    bf16x8_v kf[KS], vf[KS];
    {
      const int kr = kb0 + l32 < S ? kb0 + l32 : S - 1;
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        kf[ks] = ld16(k + base + (int64_t)kr * HD + 16 * ks + 8 * hf);
        vf[ks] = ld16(v + base + (int64_t)kr * HD + 16 * ks + 8 * hf);
      }
    }
    u32x4_v kr4[KS];
    load_block<HD>(k + base, HD, kb0, S, lane, kr4);
    f32x16_v st, dp;
#pragma unroll
    for (int r = 0; r < 16; ++r) st[r] = dp[r] = 0.0f;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      st = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf[ks], qf[ks], st, 0, 0, 0);
      dp = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vf[ks], dof[ks], dp, 0, 0, 0);
    }
    float ds[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int key = kb0 + 8 * (r >> 2) + 4 * hf + (r & 3);
      const float p = (key <= qi && key < S) ? exp2f(st[r] * c2 - l2) : 0.0f;
      ds[r] = p * (dp[r] * hs - D);
    }
    wave_lds_fence();
    store_block<HD>(blk, lane, kr4);
    wave_lds_fence();
    const bf16x8_v db8[2] = {pack8<0>(ds), pack8<8>(ds)};
#pragma unroll
    for (int db = 0; db < NB; ++db)
#pragma unroll
      for (int t = 0; t < 2; ++t)
        acc[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(tr_frag<HD>(blk, 16 * t + 4 * hf, 32 * db + 16 * g1, lane),
                                                          db8[t], acc[db], 0, 0, 0);
  }
  if (qi < S) {
    bf16* row = o.dq + b * o.sb + h * o.sh + qi * o.ss;
    if (o.cs) store_rows_rot(row, acc, scale, hf, o.cs + (int64_t)qi * HD, o.sn + (int64_t)qi * HD);
    else store_rows(row, acc, scale, hf);
  }
}

// dK, dV of one 32-key block (wave task `task`): loop over the query blocks from the diagonal on.
// qblk, dblk: the wave's two [32][pitch] LDS blocks.
template <int HD>
__device__ __forceinline__ void attn_bwd_dkdv_task(const bf16* __restrict__ q, const bf16* __restrict__ k,
                                                   const bf16* __restrict__ v, const bf16* __restrict__ out,
                                                   const bf16* __restrict__ dout, const float* __restrict__ lse,
                                                   int BH, int H, int S, float c2, float scale,
                                                   const float* __restrict__ hscale, const BwdOut& o, int task,
                                                   bf16* qblk, bf16* dblk) {
  constexpr int KS = HD / 16, NB = HD / 32, P = pitch<HD>();
  const int lane = threadIdx.x & 63, l32 = lane & 31, hf = lane >> 5;
  const int nkb = (S + 31) / 32;
  const int bh = task / nkb, kb = task - bh * nkb;
  if (bh >= BH) return;
  const int b = bh / H, h = bh - b * H;
  const int k0 = kb * 32, ki = k0 + l32, kc = ki < S ? ki : S - 1;
  const int64_t base = (int64_t)bh * S * HD;
  const int64_t tstride = (int64_t)H * HD;                     // token-major row stride
  const bf16* dob = dout + ((int64_t)b * S * H + h) * HD;      // row s of this head: dob + s * tstride
  const bf16* ob = out + ((int64_t)b * S * H + h) * HD;
  bf16x8_v kf[KS], vf[KS];
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) {
    kf[ks] = ld16(k + base + (int64_t)kc * HD + 16 * ks + 8 * hf);
    vf[ks] = ld16(v + base + (int64_t)kc * HD + 16 * ks + 8 * hf);
  }
  const float hs = hscale ? hscale[bh] : 1.0f;
  f32x16_v dva[NB], dka[NB];
#pragma unroll
  for (int r = 0; r < 16; ++r)
#pragma unroll
    for (int db = 0; db < NB; ++db) dva[db][r] = dka[db][r] = 0.0f;
  const int g1 = (lane >> 4) & 1;
  for (int qb = kb; qb < nkb; ++qb) {
    const int q0 = qb * 32;
    u32x4_v qr4[KS], dr4[KS];
    load_block<HD>(q + base, HD, q0, S, lane, qr4);
    load_block<HD>(dob, tstride, q0, S, lane, dr4);
    // per-query softmax statistics of row q0 + l32 (both halves hold them)
    const int qo = q0 + l32 < S ? q0 + l32 : S - 1;
    float dsum = 0.0f;
#pragma unroll
    for (int t = 0; t < KS; ++t) {
      const int d0 = (HD / 2) * hf + 8 * t;
      dsum += dot8(*reinterpret_cast<const u32x4_v*>(dob + (int64_t)qo * tstride + d0),
                   *reinterpret_cast<const u32x4_v*>(ob + (int64_t)qo * tstride + d0));
    }
    const float Dl = dsum + __shfl_xor(dsum, 32, 64);
    const float l2l = lse[(int64_t)bh * S + qo];
    wave_lds_fence();
    store_block<HD>(qblk, lane, qr4);
    store_block<HD>(dblk, lane, dr4);
    wave_lds_fence();
    f32x16_v sc, dp;
#pragma unroll
    for (int r = 0; r < 16; ++r) sc[r] = dp[r] = 0.0f;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      const int d0 = 16 * ks + 8 * hf;
      const bf16x8_v qa = *reinterpret_cast<const bf16x8_v*>(qblk + l32 * P + d0);
      const bf16x8_v da = *reinterpret_cast<const bf16x8_v*>(dblk + l32 * P + d0);
      sc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(qa, kf[ks], sc, 0, 0, 0);
      dp = __builtin_amdgcn_mfma_f32_32x32x16_bf16(da, vf[ks], dp, 0, 0, 0);
    }
    float p[16], ds[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int ql = 8 * (r >> 2) + 4 * hf + (r & 3);
      const float l2 = __shfl(l2l, ql, 64), D = __shfl(Dl, ql, 64);
      const int qr = q0 + ql;
      p[r] = (ki <= qr && qr < S) ? exp2f(sc[r] * c2 - l2) : 0.0f;
      ds[r] = p[r] * (dp[r] * hs - D);
    }
    const bf16x8_v pb[2] = {pack8<0>(p), pack8<8>(p)};
    const bf16x8_v sb[2] = {pack8<0>(ds), pack8<8>(ds)};
#pragma unroll
    for (int db = 0; db < NB; ++db)
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        const int kr = 16 * t + 4 * hf, cb = 32 * db + 16 * g1;
        dva[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(tr_frag<HD>(dblk, kr, cb, lane), pb[t], dva[db], 0, 0, 0);
        dka[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(tr_frag<HD>(qblk, kr, cb, lane), sb[t], dka[db], 0, 0, 0);
      }
  }
  if (ki < S) {
    const int64_t off = b * o.sb + h * o.sh + ki * o.ss;
    store_rows(o.dv + off, dva, hs, hf);
    if (o.cs) store_rows_rot(o.dk + off, dka, scale, hf, o.cs + (int64_t)ki * HD, o.sn + (int64_t)ki * HD);
    else store_rows(o.dk + off, dka, scale, hf);
  }
}

// The whole backward in one launch: wave task t (a (b, h) and a 32-row block) first forms dK, dV
// of key block t, then dQ of query block t (the dQ pass reuses the first LDS block).  A wave's
// two loops together visit nb + 1 score blocks for every block index, so long sequences balance.
template <int HD>
__global__ void __launch_bounds__(256) attn_bwd_kernel(const bf16* __restrict__ q, const bf16* __restrict__ k,
                                                       const bf16* __restrict__ v, const bf16* __restrict__ out,
                                                       const bf16* __restrict__ dout, const float* __restrict__ lse,
                                                       int BH, int H, int S, float c2, float scale,
                                                       const float* __restrict__ hscale, BwdOut o) {
  constexpr int P = pitch<HD>();
  __shared__ __align__(16) bf16 qsm[4][32 * P];
  __shared__ __align__(16) bf16 dsm[4][32 * P];
  const int wave = threadIdx.x >> 6;
  const int task = blockIdx.x * 4 + wave;
  attn_bwd_dkdv_task<HD>(q, k, v, out, dout, lse, BH, H, S, c2, scale, hscale, o, task, qsm[wave], dsm[wave]);
  wave_lds_fence();  // the dQ pass overwrites the wave's first block
  attn_bwd_dq_task<HD>(q, k, v, out, dout, lse, BH, H, S, c2, scale, hscale, o, task, qsm[wave]);
}

bool al16a(const void* p) { return ((uintptr_t)p & 15) == 0; }

}  // namespace

#define ATTN_CHECK(what)                                                                                    \
  RTE_REQUIRE(head_dim == 32 || head_dim == 64 || head_dim == 128, what ": head_dim must be 32, 64 or 128"); \
  RTE_REQUIRE(B >= 0 && H >= 1 && S >= 1 && (int64_t)B * H * ((S + 31) / 32) < ((int64_t)1 << 31) - 4,  \
              what ": bad sizes")

namespace {

template <int HD>
void launch_attn_fwd(const bf16* q, const bf16* k, const bf16* v, int BH, int H, int S, float scale,
                     const float* hscale, bf16* out, float* lse, hipStream_t s) {
  const int64_t tasks = (int64_t)BH * ((S + 31) / 32);
  hipLaunchKernelGGL(attn_fwd_kernel<HD>, dim3((unsigned)((tasks + 3) / 4)), dim3(256), 0, s, q, k, v, BH, H, S,
                     scale * kLog2e, hscale, out, lse);
}

template <int HD>
int launch_attn_bwd(const bf16* q, const bf16* k, const bf16* v, const bf16* out, const bf16* dout,
                    const float* lse, int BH, int H, int S, float scale, const float* hscale, const BwdOut& o,
                    hipStream_t s) {
  const int64_t tasks = (int64_t)BH * ((S + 31) / 32);
  const dim3 grid((unsigned)((tasks + 3) / 4));
  hipLaunchKernelGGL(attn_bwd_kernel<HD>, grid, dim3(256), 0, s, q, k, v, out, dout, lse, BH, H, S, scale * kLog2e,
                     scale, hscale, o);
  return check_launch("attention_bwd");
}

int attn_bwd_dispatch(const bf16* q, const bf16* k, const bf16* v, const bf16* out, const bf16* dout,
                      const float* lse, int B, int H, int S, int head_dim, float scale, const float* hscale,
                      const BwdOut& o, hipStream_t s) {
  if (B == 0) return 0;
  if (head_dim == 32) return launch_attn_bwd<32>(q, k, v, out, dout, lse, B * H, H, S, scale, hscale, o, s);
  if (head_dim == 64) return launch_attn_bwd<64>(q, k, v, out, dout, lse, B * H, H, S, scale, hscale, o, s);
  return launch_attn_bwd<128>(q, k, v, out, dout, lse, B * H, H, S, scale, hscale, o, s);
}

}  // namespace

int attention_fwd(const bf16* q, const bf16* k, const bf16* v, int B, int H, int S, int head_dim, float scale,
                  const float* hscale, bf16* out, float* lse, hipStream_t s) {
  ATTN_CHECK("attention_fwd");
  RTE_REQUIRE(al16a(q) && al16a(k) && al16a(v) && al16a(out), "attention_fwd: 16-byte aligned buffers");
  if (B == 0) return 0;
  if (head_dim == 32) launch_attn_fwd<32>(q, k, v, B * H, H, S, scale, hscale, out, lse, s);
  else if (head_dim == 64) launch_attn_fwd<64>(q, k, v, B * H, H, S, scale, hscale, out, lse, s);
  else launch_attn_fwd<128>(q, k, v, B * H, H, S, scale, hscale, out, lse, s);
  return check_launch("attention_fwd");
}

int attention_bwd(const bf16* q, const bf16* k, const bf16* v, const bf16* out, const bf16* dout, const float* lse,
                  int B, int H, int S, int head_dim, float scale, const float* hscale, bf16* dq, bf16* dk, bf16* dv,
                  hipStream_t s) {
  ATTN_CHECK("attention_bwd");
  RTE_REQUIRE(al16a(q) && al16a(k) && al16a(v) && al16a(out) && al16a(dout) && al16a(dq) && al16a(dk) && al16a(dv),
              "attention_bwd: 16-byte aligned buffers");
  const BwdOut o{dq, dk, dv, (int64_t)H * S * head_dim, (int64_t)S * head_dim, head_dim, nullptr, nullptr};
  return attn_bwd_dispatch(q, k, v, out, dout, lse, B, H, S, head_dim, scale, hscale, o, s);
}

int attention_bwd_qkv(const bf16* q, const bf16* k, const bf16* v, const bf16* out, const bf16* dout,
                      const float* lse, int B, int H, int S, int head_dim, float scale, const float* hscale,
                      const float* cos_t, const float* sin_t, bf16* dqkv, hipStream_t s) {
  ATTN_CHECK("attention_bwd_qkv");
  RTE_REQUIRE(al16a(q) && al16a(k) && al16a(v) && al16a(out) && al16a(dout) && al16a(dqkv) && al16a(cos_t) &&
                  al16a(sin_t),
              "attention_bwd_qkv: 16-byte aligned buffers");
  const int64_t d = (int64_t)H * head_dim;
  const BwdOut o{dqkv, dqkv + d, dqkv + 2 * d, (int64_t)S * 3 * d, head_dim, 3 * d, cos_t, sin_t};
  return attn_bwd_dispatch(q, k, v, out, dout, lse, B, H, S, head_dim, scale, hscale, o, s);
}

}  // namespace rte
