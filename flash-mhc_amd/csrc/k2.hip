// K2: the mHC-lite coefficient math of the fused path (block.py:161-170 of
// alint77/flash-mHC), forward and backward, one thread per token.
//
// The reference evaluates K2 as a chain of PyTorch ops on bf16 tensors: every
// op computes in fp32 from bf16 inputs and rounds its output to bf16 (RNE), and
// autograd does the same for each backward op.  These kernels run the same
// chain with the same rounding points (rb() below wherever the reference
// produces a bf16 tensor) and the same fp32 operation order, with
// floating-point contraction off so that no two roundings merge into an FMA.
// Per token (p = proj row (32,), a_* = bf16(alpha_*), b = bf16(bias)):
//   h_pre  = rb(sigmoid(rb(rb(a_pre  * p[0:4])  + b[0:4])))
//   h_post = rb(2 * rb(sigmoid(rb(rb(a_post * p[4:8])  + b[4:8]))))
//   a      = rb(softmax(rb(rb(a_res  * p[8:32]) + b[8:32])))
//   H_res  = rb(a @ perm),  H_merged = rb(H_res - rb(h_post (x) h_pre))
// The outputs are the fp32 casts the fused path hands to K3 / K4
// (block.py:176-177).  The backward follows PyTorch's GPU kernels, whose bf16
// sigmoid and softmax backward round intermediate products as well.  The
// backward also produces per-workgroup partial sums of the alpha and bias
// gradients (sums over tokens), which k2_param_sum adds in a fixed order
// (k2_param_reduce, or the pre-map backward's grad_W reduce).

#include <hip/hip_runtime.h>

#include "flash_mhc_hip.h"
#include "fmhc_common.h"
#include "k2_chain.h"

namespace fmhc {
namespace {

constexpr int kK2Threads = 256;
// 32 lanes per token (k2_fwd_small, k2_bwd_small) up to this many tokens, one
// thread per token above.  The one-thread kernels take T / 256 workgroups,
// too few to hide their chain's latency until about 12000 tokens: at
// T = 4097 / 8192 / 12000 / 16384 the backward takes 13.2 / 13.4 / 13.2 /
// 13.3 us against 6.9 / 9.7 / 12.7 / 15.3 us with 32 lanes, the forward
// 7.7 / 7.9 / 8.0 / 8.1 against 4.7 / 6.3 / 7.6 / 9.0 us.
constexpr int64_t kK2SmallT = 8192;

template <bool VEC>
__global__ __launch_bounds__(kK2Threads) void k2_fwd_kernel(
    const uint16_t* __restrict__ proj, const K2Params P, float* __restrict__ h_pre,
    float* __restrict__ h_post, float* __restrict__ H, int64_t T, const ZeroWords z) {
#pragma clang fp contract(off)
  __shared__ K2Smem sm;
  zero_words(z);
  stage_params<kK2Threads>(P, sm);
  const int64_t t = static_cast<int64_t>(blockIdx.x) * kK2Threads + threadIdx.x;
  if (t >= T) return;
  float p[kDk];
  load_proj<VEC>(proj + t * kDk, p);
  float ap, apo, ar, b[kDk];
  load_params(sm, ap, apo, ar, b);
  K2Fwd f;
  k2_chain(p, ap, apo, ar, b, f);
  f32x4 hp = {f.hp[0], f.hp[1], f.hp[2], f.hp[3]};
  f32x4 hq = {f.hq[0], f.hq[1], f.hq[2], f.hq[3]};
  reinterpret_cast<f32x4*>(h_pre)[t] = hp;
  reinterpret_cast<f32x4*>(h_post)[t] = hq;
  f32x4 Hm[kN];
  k2_h_merged(f, sm.perm, Hm);
#pragma unroll
  for (int i = 0; i < kN; ++i) reinterpret_cast<f32x4*>(H)[t * kN + i] = Hm[i];
}

// Few tokens: 32 lanes per token.  Lane q computes logit q (q < 4: h_pre,
// q < 8: h_post, else a softmax term), then lanes 0-15 one H_merged entry
// each.  Every sum keeps k2_chain's / k2_h_merged's order (the softmax
// denominator and each H_res entry are added sequentially over m), so the
// results are bit-identical to k2_fwd_kernel's.
__global__ __launch_bounds__(kK2Threads) void k2_fwd_small(const uint16_t* __restrict__ proj, const K2Params P,
                                                          float* __restrict__ h_pre, float* __restrict__ h_post,
                                                          float* __restrict__ H, int64_t T, const ZeroWords z) {
#pragma clang fp contract(off)
  __shared__ K2Smem sm;
  zero_words(z);
  stage_params<kK2Threads>(P, sm);
  const int q = threadIdx.x & 31;
  const int64_t t = static_cast<int64_t>(blockIdx.x) * (kK2Threads / 32) + (threadIdx.x >> 5);
  if (t >= T) return;  // a whole 32-lane group leaves together
  k2_token32(sm, bf16_to_f32(proj[t * kDk + q]), q, t, h_pre, h_post, H);
}

// Backward of one token (autograd's rounding points on the GPU; gradients of
// the fp32 outputs are first rounded to bf16, as the .float() casts' backward
// does).
// Writes grad_proj and accumulates this token's terms of the 35 parameter
// gradients into par[]: sum_j rb(gz_pre p_pre), sum_j rb(gz_post p_post),
// sum_m rb(gz_res p_res), and the 32 logit gradients (the bias terms).
template <bool VEC>
__global__ __launch_bounds__(kK2Threads) void k2_bwd_kernel(
    const uint16_t* __restrict__ proj, const K2Params P,
    const float* __restrict__ g_hpre, const float* __restrict__ g_hpost,
    const float* __restrict__ g_H, uint16_t* __restrict__ grad_proj,
    float* __restrict__ partial, int64_t T) {
#pragma clang fp contract(off)
  __shared__ K2Smem sm;
  stage_params<kK2Threads>(P, sm);
  const int64_t t = static_cast<int64_t>(blockIdx.x) * kK2Threads + threadIdx.x;
  float par[kNPar];
#pragma unroll
  for (int k = 0; k < kNPar; ++k) par[k] = 0.f;

  if (t < T) {
    float p[kDk];
    load_proj<VEC>(proj + t * kDk, p);
    float ap, apo, ar, b[kDk];
    load_params(sm, ap, apo, ar, b);
    K2Fwd f;
    k2_chain(p, ap, apo, ar, b, f);

    float gH[kN * kN], ghp[kN], ghq[kN];
#pragma unroll
    for (int ij = 0; ij < kN * kN; ++ij) gH[ij] = g_H ? rb(g_H[t * kN * kN + ij]) : 0.f;
    // H_merged = H_res - outer(h_post, h_pre): the outer product's gradient
    // is -gH; its two factors get the sums over the other index.
#pragma unroll
    for (int i = 0; i < kN; ++i) {
      float s = 0.f;
#pragma unroll
      for (int j = 0; j < kN; ++j) s = s + rb(-gH[i * kN + j] * f.hp[j]);
      ghq[i] = rb((g_hpost ? rb(g_hpost[t * kN + i]) : 0.f) + rb(s));
    }
#pragma unroll
    for (int j = 0; j < kN; ++j) {
      float s = 0.f;
#pragma unroll
      for (int i = 0; i < kN; ++i) s = s + rb(-gH[i * kN + j] * f.hq[i]);
      ghp[j] = rb((g_hpre ? rb(g_hpre[t * kN + j]) : 0.f) + rb(s));
    }
    // H_res = a @ perm, then the softmax backward as PyTorch's GPU kernel
    // rounds it for bf16: gy = rb(g a), gz = rb(gy - a sum(gy)).
    float gy[kNF];
    float s = 0.f;
#pragma unroll
    for (int m = 0; m < kNF; ++m) {
      float acc = 0.f;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const f32x4 pm = sm.perm[m * 4 + q];
#pragma unroll
        for (int e = 0; e < 4; ++e) acc = acc + gH[4 * q + e] * pm[e];
      }
      gy[m] = rb(rb(acc) * f.a[m]);
      s = s + gy[m];
    }
    float gz[kDk];
#pragma unroll
    for (int m = 0; m < kNF; ++m) gz[2 * kN + m] = rb(gy[m] - f.a[m] * s);
    // Sigmoid backward, grad (1 - y) y with every step rounded to bf16 as
    // PyTorch's GPU kernel does for bf16; h_post = 2 sigmoid gives the factor 2 first.
#pragma unroll
    for (int j = 0; j < kN; ++j) {
      gz[j] = rb(rb(ghp[j] * rb(1.f - f.hp[j])) * f.hp[j]);
      const float gs = rb(ghq[j] * 2.f);
      gz[kN + j] = rb(rb(gs * rb(1.f - f.sq[j])) * f.sq[j]);
    }
    float gp[kDk];
#pragma unroll
    for (int k = 0; k < kDk; ++k) {
      const float a = k < kN ? ap : (k < 2 * kN ? apo : ar);
      gp[k] = rb(gz[k] * a);
      par[k < kN ? 0 : (k < 2 * kN ? 1 : 2)] += rb(gz[k] * p[k]);
      par[3 + k] = gz[k];
    }
    uint16_t* row = grad_proj + t * kDk;
    if constexpr (VEC) {
#pragma unroll
      for (int i = 0; i < 4; ++i) reinterpret_cast<u32x4*>(row)[i] = pack8(gp + 8 * i);
    } else {
#pragma unroll
      for (int k = 0; k < kDk; ++k) row[k] = f32_to_bf16(gp[k]);
    }
  }

  // Block partial sums: in-wave butterfly (every lane is here), then the
  // four waves in order.
  __shared__ float red[kK2Threads / kWave][kNPar];
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = threadIdx.x / kWave;
#pragma unroll
  for (int k = 0; k < kNPar; ++k) {
    const float v = wave_sum(par[k]);
    if (lane == 0) red[wave][k] = v;
  }
  __syncthreads();
  if (threadIdx.x < kNPar) {
    float v = 0.f;
#pragma unroll
    for (int w = 0; w < kK2Threads / kWave; ++w) v += red[w][threadIdx.x];
    partial[static_cast<int64_t>(blockIdx.x) * kNPar + threadIdx.x] = v;
  }
}

// Backward for few tokens, 32 lanes per token (lane q: logit q) and 8 tokens
// per workgroup.  Every per-token value is k2_bwd_kernel's: the forward is
// k2_token32's (bit-identical to the chain), and each sum over a token's
// terms runs through shuffles in the chain's order.  The workgroup's
// parameter partials add its 8 tokens in order (a different order over tokens
// than k2_bwd_kernel's, still fixed).
constexpr int kK2BwdTok = kK2Threads / 32;

__global__ __launch_bounds__(kK2Threads) void k2_bwd_small(
    const uint16_t* __restrict__ proj, const K2Params P, const float* __restrict__ g_hpre,
    const float* __restrict__ g_hpost, const float* __restrict__ g_H, uint16_t* __restrict__ grad_proj,
    float* __restrict__ partial, int64_t T) {
#pragma clang fp contract(off)
  __shared__ K2Smem sm;
  __shared__ float red[kK2BwdTok][kNPar];
  stage_params<kK2Threads>(P, sm);
  const int q = threadIdx.x & 31;
  const int slot = static_cast<int>(threadIdx.x) >> 5;
  const int64_t tq = static_cast<int64_t>(blockIdx.x) * kK2BwdTok + slot;
  const bool valid = tq < T;
  const int64_t t = valid ? tq : T - 1;  // idle slots recompute the last token, store nothing

  // Forward, as k2_token32: y = h_pre (q < 4) or the post sigmoid (q < 8),
  // hq = h_post, a = the softmax weight of permutation q - 8.
  const float p = bf16_to_f32(proj[t * kDk + q]);
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
  const float gh = (q < kN * kN && g_H) ? rb(g_H[t * kN * kN + q]) : 0.f;
  // grad of h_post[i] (lanes 4 + i) and of h_pre[j] (lanes j) through
  // H_merged = H_res - outer(h_post, h_pre), each sum in the chain's order.
  const int i4 = (q - kN) & 3, j4 = q & 3;
  float sq = 0.f, sp = 0.f;
#pragma unroll
  for (int k = 0; k < kN; ++k) {
    sq = sq + rb(-__shfl(gh, i4 * kN + k, 32) * __shfl(y, k, 32));
    sp = sp + rb(-__shfl(gh, k * kN + j4, 32) * __shfl(hq, kN + k, 32));
  }
  const float ghq = rb((g_hpost ? rb(g_hpost[t * kN + i4]) : 0.f) + rb(sq));
  const float ghp = rb((g_hpre ? rb(g_hpre[t * kN + j4]) : 0.f) + rb(sp));
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
  red[slot][3 + q] = valid ? gz : 0.f;
  if (q == 0) {
    red[slot][0] = valid ? s0 : 0.f;
    red[slot][1] = valid ? s1 : 0.f;
    red[slot][2] = valid ? s2 : 0.f;
  }
  __syncthreads();
  if (threadIdx.x < kNPar) {
    float v = 0.f;
#pragma unroll
    for (int w = 0; w < kK2BwdTok; ++w) v += red[w][threadIdx.x];
    partial[static_cast<int64_t>(blockIdx.x) * kNPar + threadIdx.x] = v;
  }
}

// One wave per parameter gradient (k2_param_sum).
__global__ __launch_bounds__(kWave) void k2_param_reduce(const K2ParamSums r) {
  k2_param_sum(r, static_cast<int>(blockIdx.x), static_cast<int>(threadIdx.x));
}

bool k2_bad(int64_t T, int64_t n) { return T < 0 || n != kN; }

int64_t k2_blocks(int64_t T) { return (T + kK2Threads - 1) / kK2Threads; }
// Workgroups (and parameter partials) of the backward: k2_bwd_small up to
// kK2SmallT tokens, k2_bwd_kernel above.
int64_t k2_bwd_blocks(int64_t T) { return T <= kK2SmallT ? (T + kK2BwdTok - 1) / kK2BwdTok : k2_blocks(T); }

}  // namespace

bool k2_params(const void* ap, const void* apo, const void* ar, const void* bias, const void* perm, int dtype,
               K2Params& P) {
  if (!ap || !apo || !ar || !bias || !perm || (dtype != FMHC_PARAM_F32 && dtype != FMHC_PARAM_BF16)) return false;
  P = K2Params{ap, apo, ar, bias, perm, dtype == FMHC_PARAM_BF16};
  return true;
}

int k2_fwd_launch(const uint16_t* proj, const K2Params& P, float* h_pre, float* h_post, float* H_merged, int64_t T,
                  ZeroWords z, hipStream_t s) {
  if (T <= kK2SmallT) {
    k2_fwd_small<<<dim3(static_cast<unsigned>((T + 7) / 8)), kK2Threads, 0, s>>>(proj, P, h_pre, h_post,
                                                                                H_merged, T, z);
    return launch_status();
  }
  const dim3 grid(static_cast<unsigned>(k2_blocks(T)));
  if (aligned16(proj))
    k2_fwd_kernel<true><<<grid, kK2Threads, 0, s>>>(proj, P, h_pre, h_post, H_merged, T, z);
  else
    k2_fwd_kernel<false><<<grid, kK2Threads, 0, s>>>(proj, P, h_pre, h_post, H_merged, T, z);
  return launch_status();
}

}  // namespace fmhc

extern "C" int fmhc_k2_fwd(const uint16_t* proj, const void* alpha_pre, const void* alpha_post,
                           const void* alpha_res, const void* bias, const void* perm, int param_dtype,
                           float* h_pre, float* h_post, float* H_merged, int64_t T, int64_t n,
                           void* stream) {
  using namespace fmhc;
  if (k2_bad(T, n)) return FMHC_ERR_INVALID_ARGUMENT;
  K2Params P;
  if (!k2_params(alpha_pre, alpha_post, alpha_res, bias, perm, param_dtype, P)) return FMHC_ERR_INVALID_ARGUMENT;
  if (T == 0) return FMHC_OK;
  if (!proj || !h_pre || !h_post || !H_merged) return FMHC_ERR_INVALID_ARGUMENT;
  if (!aligned16(h_pre) || !aligned16(h_post) || !aligned16(H_merged)) return FMHC_ERR_INVALID_ARGUMENT;
  return k2_fwd_launch(proj, P, h_pre, h_post, H_merged, T, ZeroWords{}, static_cast<hipStream_t>(stream));
}

extern "C" int64_t fmhc_k2_bwd_workspace_bytes(int64_t T) {
  using namespace fmhc;
  if (T <= 0) return 0;
  return k2_bwd_blocks(T) * kNPar * static_cast<int64_t>(sizeof(float));
}

namespace fmhc {

int k2_bwd_partials(const uint16_t* proj, const K2Params& P, const float* grad_h_pre, const float* grad_h_post,
                    const float* grad_H_merged, uint16_t* grad_proj, void* grad_alpha_pre, void* grad_alpha_post,
                    void* grad_alpha_res, void* grad_bias, void* workspace, int64_t workspace_bytes, int64_t T,
                    hipStream_t s, K2ParamSums* sums) {
  if (!grad_alpha_pre || !grad_alpha_post || !grad_alpha_res || !grad_bias) return FMHC_ERR_INVALID_ARGUMENT;
  const int64_t nblocks = k2_bwd_blocks(T);
  float* partial = static_cast<float*>(workspace);
  if (T > 0) {
    if (!proj || !grad_proj) return FMHC_ERR_INVALID_ARGUMENT;
    if (!workspace || workspace_bytes < fmhc_k2_bwd_workspace_bytes(T)) return FMHC_ERR_INVALID_ARGUMENT;
    const dim3 grid(static_cast<unsigned>(nblocks));
    if (T <= kK2SmallT)
      k2_bwd_small<<<grid, kK2Threads, 0, s>>>(proj, P, grad_h_pre, grad_h_post, grad_H_merged, grad_proj,
                                               partial, T);
    else if (aligned16(proj) && aligned16(grad_proj))
      k2_bwd_kernel<true><<<grid, kK2Threads, 0, s>>>(proj, P, grad_h_pre, grad_h_post, grad_H_merged,
                                                      grad_proj, partial, T);
    else
      k2_bwd_kernel<false><<<grid, kK2Threads, 0, s>>>(proj, P, grad_h_pre, grad_h_post, grad_H_merged,
                                                       grad_proj, partial, T);
    const int st = launch_status();
    if (st != FMHC_OK) return st;
  }
  // T == 0: the sums write zero gradients (nblocks = 0 partials).
  *sums = K2ParamSums{partial, T > 0 ? nblocks : 0, grad_alpha_pre, grad_alpha_post, grad_alpha_res, grad_bias,
                      P.bf16};
  return FMHC_OK;
}

void launch_k2_param_reduce(const K2ParamSums& sums, hipStream_t s) {
  k2_param_reduce<<<dim3(kNPar), kWave, 0, s>>>(sums);
}

}  // namespace fmhc

extern "C" int fmhc_k2_bwd(const uint16_t* proj, const void* alpha_pre, const void* alpha_post,
                           const void* alpha_res, const void* bias, const void* perm, int param_dtype,
                           const float* grad_h_pre, const float* grad_h_post,
                           const float* grad_H_merged, uint16_t* grad_proj, void* grad_alpha_pre,
                           void* grad_alpha_post, void* grad_alpha_res, void* grad_bias,
                           void* workspace, int64_t workspace_bytes, int64_t T, int64_t n,
                           void* stream) {
  using namespace fmhc;
  if (k2_bad(T, n)) return FMHC_ERR_INVALID_ARGUMENT;
  K2Params P;
  if (!k2_params(alpha_pre, alpha_post, alpha_res, bias, perm, param_dtype, P)) return FMHC_ERR_INVALID_ARGUMENT;
  hipStream_t s = static_cast<hipStream_t>(stream);
  K2ParamSums sums;
  const int st = k2_bwd_partials(proj, P, grad_h_pre, grad_h_post, grad_H_merged, grad_proj, grad_alpha_pre,
                                 grad_alpha_post, grad_alpha_res, grad_bias, workspace, workspace_bytes, T, s, &sums);
  if (st != FMHC_OK) return st;
  launch_k2_param_reduce(sums, s);
  return launch_status();
}
