// Per-token pieces of K2, the mHC-lite coefficient chain (block.py:161-170 of
// alint77/flash-mHC), used by the K2 kernels.
// Every value the reference holds in a bf16 tensor is rounded with rb(); the
// fp32 operations run in the reference's order, with contraction off.
#pragma once

#include "fmhc_common.h"

namespace fmhc {

constexpr int kN = 4;
constexpr int kNF = 24;             // n! for n = 4
constexpr int kDk = 2 * kN + kNF;   // 32 projection columns
constexpr int kNPar = 3 + kDk;      // alpha_pre, alpha_post, alpha_res, bias[32]
// K2's backward runs 32 lanes per token, kK2BwdTok tokens per workgroup, up to
// kK2BwdSmallT tokens (k2_bwd_small, and the pre-map's k3_reduce_k2_bwd), four
// lanes per token above (k2_bwd_quad); k2.hip gives the measurements.
constexpr int64_t kK2BwdSmallT = 6144;
constexpr int kK2BwdTok = 8;
__device__ __forceinline__ float rb(float v) { return bf16_to_f32(f32_to_bf16(v)); }

// The block parameters K2 reads, in their storage dtype: all fp32 or all bf16
// (bf16 = true).  Every value is rounded to bf16 on use, so the two give the
// same results.
struct K2Params {
  const void* alpha_pre;
  const void* alpha_post;
  const void* alpha_res;
  const void* bias;
  const void* perm;
  bool bf16;
};

// Up to two 16-bit words a forward launch also sets to zero (the pre-map
// ops' zero-stride gradient placeholders, whose one stored element would
// otherwise need a fill kernel of its own); null pointers are skipped.
struct ZeroWords {
  uint16_t* a = nullptr;
  uint16_t* b = nullptr;
};

__device__ __forceinline__ void zero_words(const ZeroWords& z) {
  if (blockIdx.x == 0 && threadIdx.x == 0) {
    if (z.a) *z.a = 0;
    if (z.b) *z.b = 0;
  }
}

__device__ __forceinline__ float ld_param(const void* p, int i, bool bf16) {
  return bf16 ? bf16_to_f32(static_cast<const uint16_t*>(p)[i]) : static_cast<const float*>(p)[i];
}

// All K2 parameters rounded to bf16 (the values the reference's ops see after
// .to(bf16)), staged in LDS once per block; every lane then reads the same
// addresses (broadcast).  perm (24 x 16) as 96 f32x4, then alpha_pre,
// alpha_post, alpha_res and bias[32].
struct K2Smem {
  f32x4 perm[kNF * 4];
  float sc[3 + kDk];
};

template <int THREADS>
__device__ __forceinline__ void stage_params(const K2Params& P, K2Smem& sm) {
  float* pf = reinterpret_cast<float*>(sm.perm);
  for (int i = threadIdx.x; i < kNF * kN * kN; i += THREADS) pf[i] = rb(ld_param(P.perm, i, P.bf16));
  for (int i = threadIdx.x; i < 3 + kDk; i += THREADS) {
    const void* src = i == 0 ? P.alpha_pre : (i == 1 ? P.alpha_post : (i == 2 ? P.alpha_res : P.bias));
    sm.sc[i] = rb(ld_param(src, i < 3 ? 0 : i - 3, P.bf16));
  }
  __syncthreads();
}

// stage_params in two halves, so that a kernel can issue the parameter loads
// early and store them to LDS later, before a barrier of its own: the same
// values in the same places.  The loads keep the raw parameter words and the
// conversion waits for store(), so issuing them does not wait for them.
__device__ __forceinline__ uint32_t ld_param_raw(const void* p, int i, bool bf16) {
  return bf16 ? static_cast<uint32_t>(static_cast<const uint16_t*>(p)[i]) : static_cast<const uint32_t*>(p)[i];
}

__device__ __forceinline__ float param_value(uint32_t raw, bool bf16) {
  return rb(__uint_as_float(bf16 ? raw << 16 : raw));  // ld_param's value, rounded as stage_params does
}

template <int THREADS>
struct K2ParamRegs {
  static constexpr int kPerm = (kNF * kN * kN + THREADS - 1) / THREADS;
  uint32_t perm[kPerm];
  uint32_t sc = 0;
  bool bf16 = false;

  __device__ __forceinline__ void load(const K2Params& P) {
    bf16 = P.bf16;
#pragma unroll
    for (int r = 0; r < kPerm; ++r) {
      const int i = static_cast<int>(threadIdx.x) + r * THREADS;
      perm[r] = i < kNF * kN * kN ? ld_param_raw(P.perm, i, P.bf16) : 0u;
    }
    const int i = static_cast<int>(threadIdx.x);
    if (i < 3 + kDk) {
      const void* src = i == 0 ? P.alpha_pre : (i == 1 ? P.alpha_post : (i == 2 ? P.alpha_res : P.bias));
      sc = ld_param_raw(src, i < 3 ? 0 : i - 3, P.bf16);
    }
  }
  __device__ __forceinline__ void store(K2Smem& sm) const {
    float* pf = reinterpret_cast<float*>(sm.perm);
#pragma unroll
    for (int r = 0; r < kPerm; ++r) {
      const int i = static_cast<int>(threadIdx.x) + r * THREADS;
      if (i < kNF * kN * kN) pf[i] = param_value(perm[r], bf16);
    }
    if (threadIdx.x < 3 + kDk) sm.sc[threadIdx.x] = param_value(sc, bf16);
  }
};

__device__ __forceinline__ void load_params(const K2Smem& sm, float& ap, float& apo, float& ar, float b[kDk]) {
  ap = sm.sc[0];
  apo = sm.sc[1];
  ar = sm.sc[2];
#pragma unroll
  for (int k = 0; k < kDk; ++k) b[k] = sm.sc[3 + k];
}

__device__ __forceinline__ float sigmoid_f32(float z) {
#pragma clang fp contract(off)
  const float d = 1.f + expf(-z);
  return 1.f / d;
}

template <bool VEC>
__device__ __forceinline__ void load_proj(const uint16_t* __restrict__ row, float p[kDk]) {
  if constexpr (VEC) {
#pragma unroll
    for (int i = 0; i < 4; ++i) unpack8(reinterpret_cast<const u32x4*>(row)[i], p + 8 * i);
  } else {
#pragma unroll
    for (int i = 0; i < kDk; ++i) p[i] = bf16_to_f32(row[i]);
  }
}

// K2 backward's parameter gradients from its partials (partial[b * kNPar + k]
// for partial b): parameter k (0-2: the alphas, 3 + j: bias j) as one
// 256-thread workgroup's sum, thread t adding partials t, t + 256, ... in
// order, then wave_sum in each wave and the four waves' sums in wave order;
// rounded to bf16 (the reference sums a bf16 tensor) and stored in the
// parameters' dtype.  nblocks = 0 writes zeros.
struct K2ParamSums {
  const float* partial = nullptr;
  int64_t nblocks = 0;
  void* g_ap = nullptr;
  void* g_apo = nullptr;
  void* g_ar = nullptr;
  void* g_bias = nullptr;
  bool bf16 = false;
};

constexpr int kK2SumThreads = 256;

// Every thread of the workgroup must call it.
__device__ __forceinline__ void k2_param_sum(const K2ParamSums& r, int k) {
  __shared__ float wsum[kK2SumThreads / kWave];
  const int t = static_cast<int>(threadIdx.x);
  float v = 0.f;
  for (int64_t b = t; b < r.nblocks; b += kK2SumThreads) v += r.partial[b * kNPar + k];
  v = wave_sum(v);
  if ((t & (kWave - 1)) == 0) wsum[t / kWave] = v;
  __syncthreads();
  if (t == 0) {
    float tot = wsum[0];
#pragma unroll
    for (int w = 1; w < kK2SumThreads / kWave; ++w) tot += wsum[w];
    void* dst = k == 0 ? r.g_ap : (k == 1 ? r.g_apo : (k == 2 ? r.g_ar : r.g_bias));
    const int i = k < 3 ? 0 : k - 3;
    if (r.bf16)
      static_cast<uint16_t*>(dst)[i] = f32_to_bf16(tot);
    else
      static_cast<float*>(dst)[i] = rb(tot);
  }
}

// Forward chain of one token.  Fills the values the backward reuses.
struct K2Fwd {
  float hp[kN], hq[kN], sq[kN];  // h_pre, h_post, sigmoid of the post logits
  float a[kNF];                  // softmax weights
};

__device__ __forceinline__ void k2_chain(const float p[kDk], float ap, float apo, float ar,
                                         const float b[kDk], K2Fwd& f) {
#pragma clang fp contract(off)
#pragma unroll
  for (int j = 0; j < kN; ++j) {
    const float z = rb(rb(ap * p[j]) + b[j]);
    f.hp[j] = rb(sigmoid_f32(z));
  }
#pragma unroll
  for (int j = 0; j < kN; ++j) {
    const float z = rb(rb(apo * p[kN + j]) + b[kN + j]);
    f.sq[j] = rb(sigmoid_f32(z));
    f.hq[j] = rb(2.f * f.sq[j]);
  }
  float z[kNF];
  float mx = -INFINITY;
#pragma unroll
  for (int m = 0; m < kNF; ++m) {
    z[m] = rb(rb(ar * p[2 * kN + m]) + b[2 * kN + m]);
    mx = fmaxf(mx, z[m]);
  }
  float sum = 0.f;
#pragma unroll
  for (int m = 0; m < kNF; ++m) {
    z[m] = expf(z[m] - mx);
    sum = sum + z[m];
  }
#pragma unroll
  for (int m = 0; m < kNF; ++m) f.a[m] = rb(z[m] / sum);
}

// H_merged row i of one token: rb(rb(sum_m a[m] perm[m, 4i + j]) - rb(h_post[i] h_pre[j])),
// the sum over m in order.
__device__ __forceinline__ void k2_h_merged(const K2Fwd& f, const f32x4 sperm[kNF * 4], f32x4 H[kN]) {
#pragma clang fp contract(off)
  float acc[kN * kN];
#pragma unroll
  for (int ij = 0; ij < kN * kN; ++ij) acc[ij] = 0.f;
#pragma unroll
  for (int m = 0; m < kNF; ++m)
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const f32x4 pm = sperm[m * 4 + q];
#pragma unroll
      for (int e = 0; e < 4; ++e) acc[4 * q + e] = acc[4 * q + e] + f.a[m] * pm[e];
    }
#pragma unroll
  for (int i = 0; i < kN; ++i)
#pragma unroll
    for (int j = 0; j < kN; ++j) H[i][j] = rb(rb(acc[i * kN + j]) - rb(f.hq[i] * f.hp[j]));
}

// Lane K of the calling lane's quad (DPP quad_perm [K, K, K, K]).
template <int K>
__device__ __forceinline__ float quad_lane(float v) {
  return __uint_as_float(__builtin_amdgcn_update_dpp(0u, __float_as_uint(v), K * 0x55, 0xf, 0xf, false));
}

// K2's backward of one token on a quad (the per-token body of k2_bwd_quad,
// k2.hip; the pre-map backward's split kernel runs it too): lane qd holds
// projections 8 qd .. 8 qd + 7 in p, and every lane the token's 16
// grad_H_merged values (rounded in place), grad_h_post and grad_h_pre.  Gives
// the lane's grad_proj values gp, its logit gradients gz (the bias terms) and
// the alpha terms s0 (h_pre's), s1 (h_post's), s2 (the softmax's), valid on
// lane qd = 0.  sm holds the staged parameters; the quad's four lanes must be
// active.
__device__ __forceinline__ void k2_bwd_quad_token(const K2Smem& sm, int qd, const float (&p)[8], float (&gH)[kN * kN],
                                                  const float (&gpost)[kN], const float (&gpre)[kN], float (&gp)[8],
                                                  float (&gz)[8], float& s0, float& s1, float& s2) {
#pragma clang fp contract(off)
  // Forward.  Lane 0: y[u] = h_pre[u] (u < 4), the sigmoid of post logit u - 4
  // (u >= 4); lanes 1-3: y[u] = the softmax weight of their term u.
  float alpha[8], z[8];
  float mx = -INFINITY;
#pragma unroll
  for (int u = 0; u < 8; ++u) {
    alpha[u] = qd == 0 ? (u < kN ? sm.sc[0] : sm.sc[1]) : sm.sc[2];
    z[u] = rb(rb(alpha[u] * p[u]) + sm.sc[3 + 8 * qd + u]);
    if (qd != 0) mx = fmaxf(mx, z[u]);
  }
  // The quad's maximum (quad_perm [1, 0, 3, 2], then [2, 3, 0, 1]); exact in any order.
  mx = fmaxf(mx, __uint_as_float(__builtin_amdgcn_update_dpp(0u, __float_as_uint(mx), 0xb1, 0xf, 0xf, false)));
  mx = fmaxf(mx, __uint_as_float(__builtin_amdgcn_update_dpp(0u, __float_as_uint(mx), 0x4e, 0xf, 0xf, false)));
  float ex[8];
#pragma unroll
  for (int u = 0; u < 8; ++u) ex[u] = expf(qd == 0 ? -z[u] : z[u] - mx);
  float sum = 0.f;
#pragma unroll
  for (int u = 0; u < 8; ++u) sum = sum + quad_lane<1>(ex[u]);
#pragma unroll
  for (int u = 0; u < 8; ++u) sum = sum + quad_lane<2>(ex[u]);
#pragma unroll
  for (int u = 0; u < 8; ++u) sum = sum + quad_lane<3>(ex[u]);
  float y[8];
#pragma unroll
  for (int u = 0; u < 8; ++u) y[u] = qd == 0 ? rb(1.f / (1.f + ex[u])) : rb(ex[u] / sum);
  float hp[kN], sq[kN], hq[kN];
  hp[0] = quad_lane<0>(y[0]);
  hp[1] = quad_lane<0>(y[1]);
  hp[2] = quad_lane<0>(y[2]);
  hp[3] = quad_lane<0>(y[3]);
  sq[0] = quad_lane<0>(y[4]);
  sq[1] = quad_lane<0>(y[5]);
  sq[2] = quad_lane<0>(y[6]);
  sq[3] = quad_lane<0>(y[7]);
#pragma unroll
  for (int i = 0; i < kN; ++i) hq[i] = rb(2.f * sq[i]);

  // Incoming gradients, rounded to bf16 (the .float() casts' backward).
#pragma unroll
  for (int ij = 0; ij < kN * kN; ++ij) gH[ij] = rb(gH[ij]);
  if (qd == 0) {
    // H_merged = H_res - outer(h_post, h_pre), then the sigmoid backward.
#pragma unroll
    for (int i = 0; i < kN; ++i) {
      float s = 0.f;
#pragma unroll
      for (int j = 0; j < kN; ++j) s = s + rb(-gH[i * kN + j] * hp[j]);
      const float ghq = rb(rb(gpost[i]) + rb(s));
      const float gs = rb(ghq * 2.f);
      gz[kN + i] = rb(rb(gs * rb(1.f - sq[i])) * sq[i]);
    }
#pragma unroll
    for (int j = 0; j < kN; ++j) {
      float s = 0.f;
#pragma unroll
      for (int i = 0; i < kN; ++i) s = s + rb(-gH[i * kN + j] * hq[i]);
      const float ghp = rb(rb(gpre[j]) + rb(s));
      gz[j] = rb(rb(ghp * rb(1.f - hp[j])) * hp[j]);
    }
  } else {
    // H_res = a @ perm: gy = rb(rb(gH . perm_m) a).
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int m = 8 * (qd - 1) + u;
      float acc = 0.f;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const f32x4 pm = sm.perm[m * 4 + q];
#pragma unroll
        for (int e = 0; e < 4; ++e) acc = acc + gH[4 * q + e] * pm[e];
      }
      gz[u] = rb(rb(acc) * y[u]);  // gy for now
    }
  }
  // Softmax backward: gz = rb(gy - a sum(gy)), the sum over m in order.
  float sgy = 0.f;
#pragma unroll
  for (int u = 0; u < 8; ++u) sgy = sgy + quad_lane<1>(gz[u]);
#pragma unroll
  for (int u = 0; u < 8; ++u) sgy = sgy + quad_lane<2>(gz[u]);
#pragma unroll
  for (int u = 0; u < 8; ++u) sgy = sgy + quad_lane<3>(gz[u]);
  if (qd != 0) {
#pragma unroll
    for (int u = 0; u < 8; ++u) gz[u] = rb(gz[u] - y[u] * sgy);
  }
  float pc[8];
#pragma unroll
  for (int u = 0; u < 8; ++u) {
    gp[u] = rb(gz[u] * alpha[u]);
    pc[u] = rb(gz[u] * p[u]);
  }
  // This token's parameter terms: the alphas' sums over their logits in
  // order, the bias gradients gz.
  s0 = 0.f;
  s1 = 0.f;
  s2 = 0.f;
#pragma unroll
  for (int u = 0; u < kN; ++u) s0 += pc[u];
#pragma unroll
  for (int u = kN; u < 8; ++u) s1 += pc[u];
#pragma unroll
  for (int u = 0; u < 8; ++u) s2 += quad_lane<1>(pc[u]);
#pragma unroll
  for (int u = 0; u < 8; ++u) s2 += quad_lane<2>(pc[u]);
#pragma unroll
  for (int u = 0; u < 8; ++u) s2 += quad_lane<3>(pc[u]);
}

// K2 forward of one token on the four lanes of a quad (qd = lane & 3; p: the
// token's 32 projections as bf16 values).  Lane qd computes logit qd (h_pre),
// 4 + qd (h_post) and the softmax terms m = qd, qd + 4, ..., 20 + qd, gathers
// the quad's exponentials and weights to add them in k2_chain's order (m = 0,
// 1, ..., 23), and computes H_merged row qd in k2_h_merged's order: the values
// of k2_chain + k2_h_merged, bit for bit, at a quarter of the arithmetic per
// lane.  hp_all receives h_pre[0..3].  Every lane of the quad must be active.
__device__ __forceinline__ void k2_token4(const float* p, const K2Smem& sm, int qd, float& hp, float& hq,
                                          f32x4& hrow, float hp_all[kN]) {
#pragma clang fp contract(off)
  hp = rb(sigmoid_f32(rb(rb(sm.sc[0] * p[qd]) + sm.sc[3 + qd])));
  hq = rb(2.f * rb(sigmoid_f32(rb(rb(sm.sc[1] * p[kN + qd]) + sm.sc[3 + kN + qd]))));
  constexpr int kS = kNF / 4;  // softmax terms per lane
  float z[kS];
  float mx = -INFINITY;
#pragma unroll
  for (int s = 0; s < kS; ++s) {
    const int m = 4 * s + qd;
    z[s] = rb(rb(sm.sc[2] * p[2 * kN + m]) + sm.sc[3 + 2 * kN + m]);
    mx = fmaxf(mx, z[s]);
  }
  // The quad's maximum (quad_perm [1, 0, 3, 2], then [2, 3, 0, 1]); a maximum
  // is exact in any order.
  mx = fmaxf(mx, __uint_as_float(__builtin_amdgcn_update_dpp(0u, __float_as_uint(mx), 0xb1, 0xf, 0xf, false)));
  mx = fmaxf(mx, __uint_as_float(__builtin_amdgcn_update_dpp(0u, __float_as_uint(mx), 0x4e, 0xf, 0xf, false)));
  float sum = 0.f;
#pragma unroll
  for (int s = 0; s < kS; ++s) {
    z[s] = expf(z[s] - mx);
    const float e0 = quad_lane<0>(z[s]), e1 = quad_lane<1>(z[s]), e2 = quad_lane<2>(z[s]), e3 = quad_lane<3>(z[s]);
    sum = sum + e0;
    sum = sum + e1;
    sum = sum + e2;
    sum = sum + e3;
  }
  float acc[kN] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int s = 0; s < kS; ++s) {
    const float a = rb(z[s] / sum);
    const float am[4] = {quad_lane<0>(a), quad_lane<1>(a), quad_lane<2>(a), quad_lane<3>(a)};
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const f32x4 pm = sm.perm[(4 * s + k) * 4 + qd];
#pragma unroll
      for (int j = 0; j < kN; ++j) acc[j] = acc[j] + am[k] * pm[j];
    }
  }
  hp_all[0] = quad_lane<0>(hp);
  hp_all[1] = quad_lane<1>(hp);
  hp_all[2] = quad_lane<2>(hp);
  hp_all[3] = quad_lane<3>(hp);
#pragma unroll
  for (int j = 0; j < kN; ++j) hrow[j] = rb(rb(acc[j]) - rb(hq * hp_all[j]));
}

// K2 forward of token t with 32 lanes (lane q of a 32-lane group, p = the
// token's projection q as a bf16 value): lane q computes logit q (q < 4:
// h_pre, q < 8: h_post, else a softmax term), then lanes 0-15 one H_merged
// entry each.  Every sum keeps k2_chain's / k2_h_merged's order (the softmax
// denominator and each H_res entry are added sequentially over m), so the
// results are bit-identical to the one-thread chain's.
// Returns lane q's sigmoid value: h_pre[t, q] for q < 4.
__device__ __forceinline__ float k2_token32(const K2Smem& sm, float p, int q, int64_t t, float* __restrict__ h_pre,
                                            float* __restrict__ h_post, float* __restrict__ H) {
#pragma clang fp contract(off)
  const float alpha = q < kN ? sm.sc[0] : (q < 2 * kN ? sm.sc[1] : sm.sc[2]);
  const float z = rb(rb(alpha * p) + sm.sc[3 + q]);
  const float y = q < 2 * kN ? rb(sigmoid_f32(z)) : 0.f;  // h_pre (q < 4), sigmoid of the post logit
  const float hq = rb(2.f * y);                             // h_post for 4 <= q < 8
  float mx = q >= 2 * kN ? z : -INFINITY;
#pragma unroll
  for (int o = 16; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, 32));
  const float e = q >= 2 * kN ? expf(z - mx) : 0.f;
  float sum = 0.f;
#pragma unroll
  for (int m = 0; m < kNF; ++m) sum = sum + __shfl(e, 2 * kN + m, 32);
  const float a = rb(e / sum);
  const float* pf = reinterpret_cast<const float*>(sm.perm);
  float acc = 0.f;
#pragma unroll
  for (int m = 0; m < kNF; ++m) acc = acc + __shfl(a, 2 * kN + m, 32) * pf[m * kN * kN + (q & 15)];
  const float hp_j = __shfl(y, q & 3, 32);
  const float hq_i = __shfl(hq, kN + ((q & 15) >> 2), 32);
  if (q < kN * kN) H[t * kN * kN + q] = rb(rb(acc) - rb(hq_i * hp_j));
  if (q < kN)
    h_pre[t * kN + q] = y;
  else if (q < 2 * kN)
    h_post[t * kN + (q - kN)] = hq;
  return y;
}

// K2 backward of token t on a 32-lane group (lane q: logit q; the group's
// lanes must all be active, width-32 shuffles).  p: the token's projection
// q; gh_in: grad_H_merged[t, q] for q < 16; gpost / gpre: grad_h_post[t, (q -
// 4) & 3] and grad_h_pre[t, q & 3], fp32 as they come in.  Writes
// grad_proj[t, q] when valid and, when write, the token's 35 parameter terms
// to red_row (zeros for an invalid token): the alphas' sums over their
// logits in order, then the 32 bias terms gz.  The forward is k2_token32's
// (bit-identical to the chain) and each sum over the token's terms runs
// through shuffles in the chain's order.
__device__ __forceinline__ void k2_bwd_token32(const K2Smem& sm, int q, int64_t t, bool valid, bool write, float p,
                                               float gh_in, float gpost, float gpre, uint16_t* __restrict__ grad_proj,
                                               float* red_row) {
#pragma clang fp contract(off)
  const int i4 = (q - kN) & 3, j4 = q & 3;
  // Forward, as k2_token32: y = h_pre (q < 4) or the post sigmoid (q < 8),
  // hq = h_post, a = the softmax weight of permutation q - 8.
  const float alpha = q < kN ? sm.sc[0] : (q < 2 * kN ? sm.sc[1] : sm.sc[2]);
  const float z = rb(rb(alpha * p) + sm.sc[3 + q]);
  const float y = q < 2 * kN ? rb(sigmoid_f32(z)) : 0.f;
  const float hq = rb(2.f * y);
  float mx = q >= 2 * kN ? z : -INFINITY;
#pragma unroll
  for (int o = 16; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, 32));
  const float e = q >= 2 * kN ? expf(z - mx) : 0.f;
  float sum = 0.f;
#pragma unroll
  for (int m = 0; m < kNF; ++m) sum = sum + __shfl(e, 2 * kN + m, 32);
  const float a = rb(e / sum);

  // Incoming gradients, rounded to bf16 (the .float() casts' backward).
  const float gh = rb(gh_in);
  // grad of h_post[i] (lanes 4 + i) and of h_pre[j] (lanes j) through
  // H_merged = H_res - outer(h_post, h_pre), each sum in the chain's order.
  float sq = 0.f, sp = 0.f;
#pragma unroll
  for (int k = 0; k < kN; ++k) {
    sq = sq + rb(-__shfl(gh, i4 * kN + k, 32) * __shfl(y, k, 32));
    sp = sp + rb(-__shfl(gh, k * kN + j4, 32) * __shfl(hq, kN + k, 32));
  }
  const float ghq = rb(rb(gpost) + rb(sq));
  const float ghp = rb(rb(gpre) + rb(sp));
  // Softmax backward (lanes 8 + m): gy = rb(rb(gH . perm_m) a), gz = rb(gy - a sum(gy)).
  const int m8 = q >= 2 * kN ? q - 2 * kN : 0;
  const float* pf = reinterpret_cast<const float*>(sm.perm);
  float acc = 0.f;
#pragma unroll
  for (int k = 0; k < kN * kN; ++k) acc = acc + __shfl(gh, k, 32) * pf[m8 * kN * kN + k];
  const float gy = q >= 2 * kN ? rb(rb(acc) * a) : 0.f;
  float sgy = 0.f;
#pragma unroll
  for (int m = 0; m < kNF; ++m) sgy = sgy + __shfl(gy, 2 * kN + m, 32);
  float gz;
  if (q < kN) {
    gz = rb(rb(ghp * rb(1.f - y)) * y);
  } else if (q < 2 * kN) {
    const float gs = rb(ghq * 2.f);
    gz = rb(rb(gs * rb(1.f - y)) * y);
  } else {
    gz = rb(gy - a * sgy);
  }
  if (valid) grad_proj[t * kDk + q] = f32_to_bf16(rb(gz * alpha));

  // This token's parameter terms: the alphas' sums over their logits in
  // order, the bias gradients gz.
  const float pc = rb(gz * p);
  float s0 = 0.f, s1 = 0.f, s2 = 0.f;
#pragma unroll
  for (int k = 0; k < kDk; ++k) {
    const float v = __shfl(pc, k, 32);
    if (k < kN)
      s0 += v;
    else if (k < 2 * kN)
      s1 += v;
    else
      s2 += v;
  }
  if (write) {
    red_row[3 + q] = valid ? gz : 0.f;
    if (q == 0) {
      red_row[0] = valid ? s0 : 0.f;
      red_row[1] = valid ? s1 : 0.f;
      red_row[2] = valid ? s2 : 0.f;
    }
  }
}

// K2 forward for T tokens (k2.hip), also zeroing z: fmhc_k2_fwd's launch
// after its checks.  k2_params validates and packs the parameters.
bool k2_params(const void* ap, const void* apo, const void* ar, const void* bias, const void* perm, int dtype,
               K2Params& P);
int k2_fwd_launch(const uint16_t* proj, const K2Params& P, float* h_pre, float* h_post, float* H_merged, int64_t T,
                  ZeroWords z, hipStream_t s);

}  // namespace fmhc
