// K2: the mHC-lite coefficient math of the fused path (block.py:161-170 of
// alint77/flash-mHC), forward and backward, one to 32 lanes per token.
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
// 32 lanes per token (k2_fwd_small, k2_bwd_small) up to these many tokens,
// four lanes per token (k2_fwd_quad, k2_bwd_quad) above.  Four lanes carry
// eight logits each, so a token's chain takes longer (backward about 8 us at
// any T up to 48000 against 5.6 us with 32 lanes at T <= 2048) but the lanes
// do 8 times less redundant work per token: alone, T = 2048 / 4096 / 6000 /
// 8192, forward 4.2 / 4.9 / 5.6 / 6.4 us with 32 lanes against 4.4 / 4.5 /
// 4.5 / 4.4 us with four, backward 5.6 / 6.9 / 8.5 / 10.3 against 8.1 /
// 8.1 / 8.2 / 8.0 us.  One thread per token, the earlier form above 8192
// tokens, took T / 256 workgroups, too few to hide the chain's latency: at
// T = 12000 / 16384 / 65536 / 262144 the forward took 8.2 / 8.2 / 9.8 /
// 20.2 us (four lanes: 4.7 / 4.8 / 8.8 / 24.5), the backward 13.8 / 13.6 /
// 14.7 / 38.8 us (8.8 / 8.8 / 15.4 / 41.1); from T = 65536 on both forms are
// bound by their arithmetic.
constexpr int64_t kK2FwdSmallT = 2048;  // kK2BwdSmallT: k2_chain.h
constexpr int kK2QuadTok = kK2Threads / 4;  // tokens per workgroup of the four-lane kernels
// The four-lane backward's parameter partials sum 16 consecutive tokens
// each (four per workgroup of 64 tokens): the unit in which the pre-map
// backward's split kernel (premap_split.hip) runs K2, whose partials must be
// the same sums.  (One 16-token workgroup per partial took 21.9 against
// 17.5 us at T = 65536: the parameters staged four times as often.)
constexpr int kK2BwdQuadThreads = kK2Threads;
constexpr int kK2PartTok = 16;

// Forward with four lanes per token (k2_token4: lane qd writes h_pre[qd],
// h_post[qd] and H_merged row qd), kK2QuadTok tokens per workgroup; the
// values of k2_chain + k2_h_merged, bit for bit.
template <bool VEC>
__global__ __launch_bounds__(kK2Threads) void k2_fwd_quad(const uint16_t* __restrict__ proj, const K2Params P,
                                                         float* __restrict__ h_pre, float* __restrict__ h_post,
                                                         float* __restrict__ H, int64_t T, const ZeroWords z) {
  __shared__ K2Smem sm;
  __shared__ float prow[kK2QuadTok][kDk];
  zero_words(z);
  const int qd = threadIdx.x & 3;
  const int slot = static_cast<int>(threadIdx.x) >> 2;
  const int64_t tq = static_cast<int64_t>(blockIdx.x) * kK2QuadTok + slot;
  const bool valid = tq < T;
  const int64_t t = valid ? tq : T - 1;  // idle slots recompute the last token, store nothing
  float p[8];
  if constexpr (VEC) {
    unpack8(*reinterpret_cast<const u32x4*>(proj + t * kDk + 8 * qd), p);
  } else {
#pragma unroll
    for (int u = 0; u < 8; ++u) p[u] = bf16_to_f32(proj[t * kDk + 8 * qd + u]);
  }
#pragma unroll
  for (int u = 0; u < 8; ++u) prow[slot][8 * qd + u] = p[u];
  stage_params<kK2Threads>(P, sm);  // ends with the barrier that also covers prow
  float hp, hq, hp_all[kN];
  f32x4 hrow;
  k2_token4(prow[slot], sm, qd, hp, hq, hrow, hp_all);
  if (valid) {
    h_pre[t * kN + qd] = hp;
    h_post[t * kN + qd] = hq;
    reinterpret_cast<f32x4*>(H)[t * kN + qd] = hrow;
  }
}

// Few tokens: 32 lanes per token.  Lane q computes logit q (q < 4: h_pre,
// q < 8: h_post, else a softmax term), then lanes 0-15 one H_merged entry
// each.  Every sum keeps k2_chain's / k2_h_merged's order (the softmax
// denominator and each H_res entry are added sequentially over m), so the
// results are bit-identical to k2_chain + k2_h_merged.
__global__ __launch_bounds__(kK2Threads) void k2_fwd_small(const uint16_t* __restrict__ proj, const K2Params P,
                                                          float* __restrict__ h_pre, float* __restrict__ h_post,
                                                          float* __restrict__ H, int64_t T, const ZeroWords z) {
#pragma clang fp contract(off)
  __shared__ K2Smem sm;
  zero_words(z);
  const int q = threadIdx.x & 31;
  const int64_t t = static_cast<int64_t>(blockIdx.x) * (kK2Threads / 32) + (threadIdx.x >> 5);
  const float p = t < T ? bf16_to_f32(proj[t * kDk + q]) : 0.f;  // loaded before the barrier
  stage_params<kK2Threads>(P, sm);
  if (t >= T) return;  // a whole 32-lane group leaves together
  k2_token32(sm, p, q, t, h_pre, h_post, H);
}

// Backward of one token (autograd's rounding points on the GPU; gradients of
// the fp32 outputs are first rounded to bf16, as the .float() casts' backward
// does), in the chain's order:
//   gH = rb(grad_H), ghq[i] = rb(rb(grad_h_post[i]) + rb(sum_j rb(-gH[i, j] h_pre[j]))),
//   ghp[j] = rb(rb(grad_h_pre[j]) + rb(sum_i rb(-gH[i, j] h_post[i]))),
//   gy[m] = rb(rb(sum_ij gH[ij] perm[m, ij]) a[m]), gz_res[m] = rb(gy[m] - a[m] sum_m gy[m])
//   (PyTorch's bf16 softmax backward), gz_pre[j] = rb(rb(ghp[j] rb(1 - h_pre[j])) h_pre[j]),
//   gz_post[j] = rb(rb(rb(2 ghq[j]) rb(1 - s[j])) s[j]) (s: the post sigmoid),
//   grad_proj[k] = rb(gz[k] alpha_k);
// each sum in index order.  The 35 parameter terms of a token are
// sum_j rb(gz_pre p_pre), sum_j rb(gz_post p_post), sum_m rb(gz_res p_res)
// and the 32 logit gradients gz (the bias terms); a workgroup writes their
// sums over its tokens, in token order, to its partial.
//
// Few tokens: 32 lanes per token (lane q: logit q) and 8 tokens per
// workgroup.  The forward is k2_token32's (bit-identical to the chain), and
// each sum over a token's terms runs through shuffles in the chain's order.
static_assert(kK2BwdTok == kK2Threads / 32, "32 lanes per token");

__global__ __launch_bounds__(kK2Threads) void k2_bwd_small(
    const uint16_t* __restrict__ proj, const K2Params P, const float* __restrict__ g_hpre,
    const float* __restrict__ g_hpost, const float* __restrict__ g_H, uint16_t* __restrict__ grad_proj,
    float* __restrict__ partial, int64_t T) {
#pragma clang fp contract(off)
  __shared__ K2Smem sm;
  __shared__ float red[kK2BwdTok][kNPar];
  const int q = threadIdx.x & 31;
  const int slot = static_cast<int>(threadIdx.x) >> 5;
  const int64_t tq = static_cast<int64_t>(blockIdx.x) * kK2BwdTok + slot;
  const bool valid = tq < T;
  const int64_t t = valid ? tq : T - 1;  // idle slots recompute the last token, store nothing
  const int i4 = (q - kN) & 3, j4 = q & 3;
  // The token's operands are loaded before the parameters' barrier, so that
  // the two loads' latencies overlap.
  const float p = bf16_to_f32(proj[t * kDk + q]);
  const float gh_in = (q < kN * kN && g_H) ? g_H[t * kN * kN + q] : 0.f;
  const float gpost = g_hpost ? g_hpost[t * kN + i4] : 0.f;
  const float gpre = g_hpre ? g_hpre[t * kN + j4] : 0.f;
  stage_params<kK2Threads>(P, sm);

  k2_bwd_token32(sm, q, t, valid, true, p, gh_in, gpost, gpre, grad_proj, red[slot]);
  __syncthreads();
  if (threadIdx.x < kNPar) {
    float v = 0.f;
#pragma unroll
    for (int w = 0; w < kK2BwdTok; ++w) v += red[w][threadIdx.x];
    partial[static_cast<int64_t>(blockIdx.x) * kNPar + threadIdx.x] = v;
  }
}

// Backward with four lanes per token: lane qd of a quad owns projections
// 8 qd .. 8 qd + 7, so lane 0 holds the eight sigmoid logits (h_pre, then
// h_post's) and lanes 1-3 eight softmax terms each (m = 8 (qd - 1) + u).
// Every lane evaluates one exponential and one division per value (lane 0:
// 1 / (1 + exp(-z)), the others exp(z - max) / sum), and the sums over a
// token's terms gather the quad's values with DPP moves and add them in the
// chain's order, so every per-token value is k2_bwd_small's bit for bit.
// grad_proj leaves as one 16-byte row piece per lane.  The workgroup's
// parameter partials add its tokens in order.
template <int THREADS, bool VEC>
__global__ __launch_bounds__(THREADS) void k2_bwd_quad(
    const uint16_t* __restrict__ proj, const K2Params P, const float* __restrict__ g_hpre,
    const float* __restrict__ g_hpost, const float* __restrict__ g_H, uint16_t* __restrict__ grad_proj,
    float* __restrict__ partial, int64_t T) {
#pragma clang fp contract(off)
  constexpr int kTok = THREADS / 4;
  __shared__ K2Smem sm;
  __shared__ float red[kTok][kNPar];
  const int qd = threadIdx.x & 3;
  const int slot = static_cast<int>(threadIdx.x) >> 2;
  const int64_t tq = static_cast<int64_t>(blockIdx.x) * kTok + slot;
  const bool valid = tq < T;
  const int64_t t = valid ? tq : T - 1;  // idle slots recompute the last token, store nothing

  // The token's operands are loaded before the parameters' barrier, so that
  // the two loads' latencies overlap.
  float p[8];
  if constexpr (VEC) {
    unpack8(*reinterpret_cast<const u32x4*>(proj + t * kDk + 8 * qd), p);
  } else {
#pragma unroll
    for (int u = 0; u < 8; ++u) p[u] = bf16_to_f32(proj[t * kDk + 8 * qd + u]);
  }
  float gH[kN * kN], gpost[kN], gpre[kN];
#pragma unroll
  for (int ij = 0; ij < kN * kN; ++ij) gH[ij] = g_H ? g_H[t * kN * kN + ij] : 0.f;
#pragma unroll
  for (int i = 0; i < kN; ++i) {
    gpost[i] = g_hpost ? g_hpost[t * kN + i] : 0.f;
    gpre[i] = g_hpre ? g_hpre[t * kN + i] : 0.f;
  }
  stage_params<THREADS>(P, sm);
  float gp[8], gz[8], s0, s1, s2;
  k2_bwd_quad_token(sm, qd, p, gH, gpost, gpre, gp, gz, s0, s1, s2);
  if (valid) {
    uint16_t* row = grad_proj + t * kDk + 8 * qd;
    if constexpr (VEC) {
      *reinterpret_cast<u32x4*>(row) = pack8(gp);
    } else {
#pragma unroll
      for (int u = 0; u < 8; ++u) row[u] = f32_to_bf16(gp[u]);
    }
  }
#pragma unroll
  for (int u = 0; u < 8; ++u) red[slot][3 + 8 * qd + u] = valid ? gz[u] : 0.f;
  if (qd == 0) {
    red[slot][0] = valid ? s0 : 0.f;
    red[slot][1] = valid ? s1 : 0.f;
    red[slot][2] = valid ? s2 : 0.f;
  }
  __syncthreads();
  // One partial per kK2PartTok tokens (the last workgroup's past T are not
  // written: ceil(T / kK2PartTok) partials in all).
  constexpr int kGroups = kTok / kK2PartTok;
  if (threadIdx.x < kNPar * kGroups) {
    const int g = static_cast<int>(threadIdx.x) / kNPar, k = static_cast<int>(threadIdx.x) % kNPar;
    const int64_t part = static_cast<int64_t>(blockIdx.x) * kGroups + g;
    if (part < (T + kK2PartTok - 1) / kK2PartTok) {
      float v = 0.f;
#pragma unroll
      for (int w = 0; w < kK2PartTok; ++w) v += red[g * kK2PartTok + w][k];
      partial[part * kNPar + k] = v;
    }
  }
}

// One workgroup per parameter gradient (k2_param_sum).
__global__ __launch_bounds__(kK2SumThreads) void k2_param_reduce(const K2ParamSums r) {
  k2_param_sum(r, static_cast<int>(blockIdx.x));
}

bool k2_bad(int64_t T, int64_t n) { return T < 0 || n != kN; }

// Workgroups (and parameter partials) of the backward: k2_bwd_small up to
// kK2BwdSmallT tokens, k2_bwd_quad (kK2QuadTok tokens each) above.
int64_t k2_bwd_blocks(int64_t T) {
  return T <= kK2BwdSmallT ? (T + kK2BwdTok - 1) / kK2BwdTok : (T + kK2PartTok - 1) / kK2PartTok;
}

}  // namespace

bool k2_params(const void* ap, const void* apo, const void* ar, const void* bias, const void* perm, int dtype,
               K2Params& P) {
  if (!ap || !apo || !ar || !bias || !perm || (dtype != FMHC_PARAM_F32 && dtype != FMHC_PARAM_BF16)) return false;
  P = K2Params{ap, apo, ar, bias, perm, dtype == FMHC_PARAM_BF16};
  return true;
}

int k2_fwd_launch(const uint16_t* proj, const K2Params& P, float* h_pre, float* h_post, float* H_merged, int64_t T,
                  ZeroWords z, hipStream_t s) {
  if (T <= kK2FwdSmallT) {
    k2_fwd_small<<<dim3(static_cast<unsigned>((T + 7) / 8)), kK2Threads, 0, s>>>(proj, P, h_pre, h_post,
                                                                                H_merged, T, z);
    return launch_status();
  }
  const dim3 grid(static_cast<unsigned>((T + kK2QuadTok - 1) / kK2QuadTok));
  if (aligned16(proj))
    k2_fwd_quad<true><<<grid, kK2Threads, 0, s>>>(proj, P, h_pre, h_post, H_merged, T, z);
  else
    k2_fwd_quad<false><<<grid, kK2Threads, 0, s>>>(proj, P, h_pre, h_post, H_merged, T, z);
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
    const dim3 grid(static_cast<unsigned>(T <= kK2BwdSmallT ? nblocks : (T + kK2QuadTok - 1) / kK2QuadTok));
    if (T <= kK2BwdSmallT)
      k2_bwd_small<<<grid, kK2Threads, 0, s>>>(proj, P, grad_h_pre, grad_h_post, grad_H_merged, grad_proj,
                                               partial, T);
    else if (aligned16(proj) && aligned16(grad_proj))
      k2_bwd_quad<kK2BwdQuadThreads, true><<<grid, kK2BwdQuadThreads, 0, s>>>(
          proj, P, grad_h_pre, grad_h_post, grad_H_merged, grad_proj, partial, T);
    else
      k2_bwd_quad<kK2BwdQuadThreads, false><<<grid, kK2BwdQuadThreads, 0, s>>>(
          proj, P, grad_h_pre, grad_h_post, grad_H_merged, grad_proj, partial, T);
    const int st = launch_status();
    if (st != FMHC_OK) return st;
  }
  // T == 0: the sums write zero gradients (nblocks = 0 partials).
  *sums = K2ParamSums{partial, T > 0 ? nblocks : 0, grad_alpha_pre, grad_alpha_post, grad_alpha_res, grad_bias,
                      P.bf16};
  return FMHC_OK;
}

void launch_k2_param_reduce(const K2ParamSums& sums, hipStream_t s) {
  k2_param_reduce<<<dim3(kNPar), kK2SumThreads, 0, s>>>(sums);
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
