// K3: pre-map of the n = 4 residual streams into the layer input, and its
// backward.
//
//   forward   out[t,c]        = bf16(sum_j h_pre[t,j] * x[t,j,c])       j = 0..3 in order
//   backward  grad_x[t,j,c]   = bf16(h_pre[t,j] * go[t,c])
//             grad_h_pre[t,j] = sum_c x[t,j,c] * go[t,c]                 (fp32)
//
// Follows src/flash_mhc/kernels.py:673-717 (forward) and :720-853 (fused
// backward) of the reference, written for gfx950:
//   * a group of LPT consecutive lanes owns one token: a wave64 holds 64 / LPT
//     tokens, or a token spans LPT / 64 waves (LPT = 128, 256: wide rows, few
//     tokens).  Each lane streams 16-byte vectors of all four stream rows, so
//     every x row is read once and every output row written once;
//   * the four per-token coefficients are wave-uniform when LPT >= 64 and then
//     live in SGPRs;
//   * the backward's four reductions over C finish with an in-wave butterfly
//     and, when a token spans several waves, an LDS sum over them in wave
//     order (no atomics), so grad_h_pre is deterministic.
#include <type_traits>

#include "fmhc_common.h"

namespace fmhc {

namespace {

constexpr int kBlock = 256;  // 4 waves per workgroup, or one token's LPT lanes when more

// Threads per workgroup for LPT lanes per token.
template <int LPT>
constexpr int block_of() {
  return LPT > kBlock ? LPT : kBlock;
}

// LPT <= 64: 64 / LPT tokens per wave.  LPT = 128 or 256: LPT / 64 waves per
// token; LPT a multiple of 64 above 256: one token per workgroup.
template <int LPT>
__device__ __forceinline__ int64_t token_of_lane(int lane) {
  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) >> 6);
  if constexpr (LPT > kWave) {
    return static_cast<int64_t>(blockIdx.x) * (block_of<LPT>() / LPT) + wave / (LPT / kWave);
  } else {
    constexpr int TPW = kWave / LPT;
    const int64_t first = (static_cast<int64_t>(blockIdx.x) * (kBlock / kWave) + wave) * TPW;
    return LPT == kWave ? first : first + lane / LPT;
  }
}

// Position of this lane among its token's LPT lanes.
template <int LPT>
__device__ __forceinline__ int sub_of_lane() {
  return static_cast<int>(threadIdx.x) % LPT;
}

template <int VEC, int LPT>
__global__ __launch_bounds__(block_of<LPT>()) void k3_fwd_kernel(const uint16_t* __restrict__ x,
                                                        const float* __restrict__ h_pre,
                                                        uint16_t* __restrict__ out,
                                                        int64_t T, int C) {
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t tok = token_of_lane<LPT>(lane);
  if (tok >= T) return;
  const int sub = sub_of_lane<LPT>();
  const float* hp = h_pre + tok * 4;
  const float h[4] = {hp[0], hp[1], hp[2], hp[3]};
  k3_token<VEC>(x + tok * 4 * C, h, out + tok * C, sub, LPT, C);
}

// GX = false: grad_h_pre only (the pre-map backward adds h_pre * go into K1's
// grad_x store instead of writing it here).  CANON (C a multiple of 128, at
// most kMaxSlices slices, 16-byte groups): grad_h_pre in the slice order of
// slice_sums_add (fmhc_common.h), which the pre-map backward's split kernel
// reproduces; otherwise one FMA chain per lane over its groups, then
// group_sum.
template <int VEC, int LPT, bool GX, bool CANON>
__global__ __launch_bounds__(block_of<LPT>()) void k3_bwd_kernel(const uint16_t* __restrict__ x,
                                                        const float* __restrict__ h_pre,
                                                        const uint16_t* __restrict__ go,
                                                        uint16_t* __restrict__ grad_x,
                                                        float* __restrict__ grad_h_pre,
                                                        int64_t T, int C) {
  static_assert(!CANON || (VEC == 8 && LPT >= 16), "slice order: 16-byte groups, whole 16-lane rows");
  constexpr int WPT = LPT > kWave ? LPT / kWave : 1;  // waves per token
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t tok = token_of_lane<LPT>(lane);
  // With several waves per token every wave reaches the barrier below.
  if constexpr (WPT == 1) {
    if (tok >= T) return;
  }
  const bool live = tok < T;
  const int sub = sub_of_lane<LPT>();
  const int ng = C / VEC;
  // CANON with several waves per token: slice sums by slice.
  __shared__ float slices[CANON && WPT > 1 ? kMaxSlices : 1][4];

  float s[4] = {0.f, 0.f, 0.f, 0.f};
  if (live) {
  const float* hp = h_pre + tok * 4;
  const float h0 = hp[0], h1 = hp[1], h2 = hp[2], h3 = hp[3];
  const uint16_t* x0 = x + tok * 4 * C;
  const uint16_t* x1 = x0 + C;
  const uint16_t* x2 = x1 + C;
  const uint16_t* x3 = x2 + C;
  const uint16_t* grow = go + tok * C;
  uint16_t* gx0 = grad_x + tok * 4 * C;
  uint16_t* gx1 = gx0 + C;
  uint16_t* gx2 = gx1 + C;
  uint16_t* gx3 = gx2 + C;

  auto round = [&](int g, float (&acc)[4]) {
    float q[VEC], a[VEC], b[VEC], c[VEC], d[VEC], o[VEC];
    Lanes<VEC>::load(grow, g, q);
    Lanes<VEC>::load(x0, g, a);
    Lanes<VEC>::load(x1, g, b);
    Lanes<VEC>::load(x2, g, c);
    Lanes<VEC>::load(x3, g, d);
    if constexpr (GX) {
#pragma unroll
      for (int e = 0; e < VEC; ++e) o[e] = h0 * q[e];
      Lanes<VEC>::store(gx0, g, o);
#pragma unroll
      for (int e = 0; e < VEC; ++e) o[e] = h1 * q[e];
      Lanes<VEC>::store(gx1, g, o);
#pragma unroll
      for (int e = 0; e < VEC; ++e) o[e] = h2 * q[e];
      Lanes<VEC>::store(gx2, g, o);
#pragma unroll
      for (int e = 0; e < VEC; ++e) o[e] = h3 * q[e];
      Lanes<VEC>::store(gx3, g, o);
    }
#pragma unroll
    for (int e = 0; e < VEC; ++e) {
      acc[0] = __builtin_fmaf(a[e], q[e], acc[0]);
      acc[1] = __builtin_fmaf(b[e], q[e], acc[1]);
      acc[2] = __builtin_fmaf(c[e], q[e], acc[2]);
      acc[3] = __builtin_fmaf(d[e], q[e], acc[3]);
    }
  };
  if constexpr (CANON) {
    // Rounds k < kCanonRounds: lane sub takes group sub + k LPT (slice
    // (sub + k LPT) / 16); whole 16-lane rows are inside or past the row.
    // All rounds' loads first, then the slice sums.
    const int ns = ng / 16;
    float e[kCanonRounds][4];
#pragma unroll
    for (int k = 0; k < kCanonRounds; ++k) {
#pragma unroll
      for (int j = 0; j < 4; ++j) e[k][j] = 0.f;
      if (sub + k * LPT < ng) round(sub + k * LPT, e[k]);
    }
#pragma unroll
    for (int k = 0; k < kCanonRounds; ++k) {
      if (k * LPT >= ng) break;  // uniform
      if constexpr (WPT == 1) {
        slice_sums_add<LPT>(e[k], s, k, ns, lane);
      } else {
        const int g = sub + k * LPT;
#pragma unroll
        for (int j = 0; j < 4; ++j) e[k][j] = row16_sum(e[k][j]);
        if ((sub & 15) == 0 && g < ng) {
#pragma unroll
          for (int j = 0; j < 4; ++j) slices[g >> 4][j] = e[k][j];
        }
      }
    }
  } else {
#pragma unroll 2
    for (int g = sub; g < ng; g += LPT) round(g, s);
  }
  }
  if constexpr (!CANON) {
    constexpr int GS = LPT < kWave ? LPT : kWave;
#pragma unroll
    for (int j = 0; j < 4; ++j) s[j] = group_sum<GS>(s[j]);
  }
  if constexpr (WPT > 1) {
    // The token's waves add their sums in wave order (deterministic), or
    // with CANON its slices in slice order.
    __shared__ float red[block_of<LPT>() / kWave][4];
    const int wave = static_cast<int>(threadIdx.x) >> 6;
    if (!CANON && lane == 0) {
#pragma unroll
      for (int j = 0; j < 4; ++j) red[wave][j] = s[j];
    }
    __syncthreads();
    if (live && sub == 0) {
      float t[4] = {0.f, 0.f, 0.f, 0.f};
      if constexpr (CANON) {
        const int ns = ng / 16;
#pragma unroll
        for (int j = 0; j < 4; ++j) t[j] = slices[0][j];
        for (int sg = 1; sg < ns; ++sg)
#pragma unroll
          for (int j = 0; j < 4; ++j) t[j] += slices[sg][j];
      } else {
#pragma unroll
        for (int w = 0; w < WPT; ++w)
#pragma unroll
          for (int k = 0; k < 4; ++k) t[k] += red[wave + w][k];
      }
      float* dst = grad_h_pre + tok * 4;
#pragma unroll
      for (int k = 0; k < 4; ++k) dst[k] = t[k];
    }
  } else if (sub == 0) {
    float* dst = grad_h_pre + tok * 4;
#pragma unroll
    for (int j = 0; j < 4; ++j) dst[j] = s[j];
  }
}

// Lanes per token: a full wave for wide rows, fewer lanes (more tokens per
// wave) when a row would leave most of a wave idle.  A full wave from one
// 8-element group per lane on: at C = 512 the backward kernels are 5% (K3)
// and 20% (K4) faster with 64 lanes than with 32.
template <int VEC>
int pick_lpt(int C) {
  const int groups = C / VEC;
  if (groups >= 64) return 64;
  if (groups >= 32) return 32;
  if (groups >= 16) return 16;
  return 8;
}

// Widest layout (16-byte path): a workgroup of exactly one 8-element group
// per lane and stream when a row's groups (a multiple of 64, from 320 to
// kMaxLpt) do not split evenly over 256 lanes: C = 2560, 3072, 3584.  With
// 256 lanes at C = 2560 (320 groups) a quarter of the lanes took a second
// group while the rest waited; 320 lanes took the six-kernel step at
// T = 65536 from 5677 to 6054 GB/s (K4 backward 5378 -> 6307).  C = 4096
// (512 groups, two per lane at 256) measured the same at 512 and 256 lanes
// (T = 65536 and 262144, within 2%) and keeps 256.
#ifndef FMHC_K34_MAX_LPT
#define FMHC_K34_MAX_LPT 512
#endif
constexpr int kMaxLpt = FMHC_K34_MAX_LPT;

template <int VEC>
int wide_lpt(int groups) {
  if constexpr (VEC == 8) {
    if (groups % kWave == 0 && groups % 256 != 0 && groups > 256 && groups <= kMaxLpt) return groups;
  }
  return 256;
}

// f(std::integral_constant<int, L>{}) for the lanes per token L the kernels
// are built for; threads per workgroup block_of<L>().
template <typename F>
void with_lpt(int lpt, F&& f) {
  switch (lpt) {
    case 512: f(std::integral_constant<int, 512>{}); break;
    case 448: f(std::integral_constant<int, 448>{}); break;
    case 384: f(std::integral_constant<int, 384>{}); break;
    case 320: f(std::integral_constant<int, 320>{}); break;
    case 256: f(std::integral_constant<int, 256>{}); break;
    case 128: f(std::integral_constant<int, 128>{}); break;
    case 64: f(std::integral_constant<int, 64>{}); break;
    case 32: f(std::integral_constant<int, 32>{}); break;
    case 16: f(std::integral_constant<int, 16>{}); break;
    default: f(std::integral_constant<int, 8>{}); break;
  }
}

// Tokens per workgroup with lpt lanes per token.
int64_t tokens_per_block(int lpt) {
  return lpt > kWave ? (lpt > kBlock ? 1 : kBlock / lpt) : (kBlock / kWave) * (kWave / lpt);
}

// The forward kernel spreads a token over more lanes (up to a workgroup),
// so that each lane has one or two 8-element groups per stream instead of a
// loop over them.  Measured at T x C = 64 Mi elements: with 256 lanes per
// token from C = 2048 on the kernel is 13-17% faster than with one wave;
// at C = 1024 K3 is 2% faster with one wave.  Few tokens always take the
// wide layout (latency, not bandwidth, bounds that regime).
template <int VEC>
int pick_lpt_fwd(int C, int64_t T) {
  const int lpt = pick_lpt<VEC>(C);
  const int groups = C / VEC;
  if (groups >= 256) return wide_lpt<VEC>(groups);
  if (groups >= 128) return T * lpt < int64_t{256} * kBlock ? 128 : lpt;
  return lpt;
}

template <int VEC>
int launch_k3_fwd(const uint16_t* x, const float* h_pre, uint16_t* out, int64_t T, int C,
                  hipStream_t s) {
  const int lpt = pick_lpt_fwd<VEC>(C, T);
  const dim3 grid(blocks_for(T, tokens_per_block(lpt)));
  with_lpt(lpt, [&](auto l) {
    constexpr int L = decltype(l)::value;
    // Residency cap (fmhc_common.h).
    static const unsigned lds =
        lds_reserve(reinterpret_cast<const void*>(&k3_fwd_kernel<VEC, L>), VEC == 8 && FMHC_LDS_CAP ? kLdsCapSix : 0u);
    k3_fwd_kernel<VEC, L><<<grid, block_of<L>(), lds, s>>>(x, h_pre, out, T, C);
  });
  return launch_status();
}

// Backward: a workgroup per token from C = 2048 on (the four per-token sums
// then finish across the waves in LDS): 14-24% faster there than one wave
// per token at T x C = 64 Mi elements.  At C = 1024 two waves per token are
// 16% slower than one, which stays the choice below C = 2048.
template <int VEC>
int pick_lpt_bwd(int C) {
  return C / VEC >= 256 ? wide_lpt<VEC>(C / VEC) : pick_lpt<VEC>(C);
}

template <int VEC, bool GX>
int launch_k3_bwd(const uint16_t* x, const float* h_pre, const uint16_t* go, uint16_t* grad_x,
                  float* grad_h_pre, int64_t T, int C, hipStream_t s) {
  const int lpt = pick_lpt_bwd<VEC>(C);
  const dim3 grid(blocks_for(T, tokens_per_block(lpt)));
  const bool canon = VEC == 8 && k3_canon(C, lpt);
  // Residency cap (fmhc_common.h): with grad_x, up to C = 2048.
  const unsigned cap = VEC == 8 && GX && FMHC_LDS_CAP && C <= 2048 ? kLdsCapFive : 0u;
  with_lpt(lpt, [&](auto l) {
    constexpr int L = decltype(l)::value;
    if constexpr (VEC == 8 && L >= 16) {
      if (canon) {
        static const unsigned lds =
            lds_reserve(reinterpret_cast<const void*>(&k3_bwd_kernel<VEC, L, GX, true>), kLdsCapFive);
        k3_bwd_kernel<VEC, L, GX, true><<<grid, block_of<L>(), cap ? lds : 0u, s>>>(x, h_pre, go, grad_x,
                                                                                  grad_h_pre, T, C);
        return;
      }
    }
    static const unsigned lds =
        lds_reserve(reinterpret_cast<const void*>(&k3_bwd_kernel<VEC, L, GX, false>), kLdsCapFive);
    k3_bwd_kernel<VEC, L, GX, false><<<grid, block_of<L>(), cap ? lds : 0u, s>>>(x, h_pre, go, grad_x, grad_h_pre,
                                                                               T, C);
  });
  return launch_status();
}

bool bad_sizes(int64_t T, int64_t C, int64_t n) {
  return T < 0 || C <= 0 || C > (int64_t{1} << 30) || n != 4;
}

}  // namespace

int k3_bwd_lanes8(int C) { return pick_lpt_bwd<8>(C); }
}  // namespace fmhc

extern "C" int fmhc_k3_fwd(const uint16_t* x, const float* h_pre, uint16_t* out, int64_t T,
                           int64_t C, int64_t n, void* stream) {
  using namespace fmhc;
  if (bad_sizes(T, C, n)) return FMHC_ERR_INVALID_ARGUMENT;
  if (T == 0) return FMHC_OK;
  if (!x || !h_pre || !out) return FMHC_ERR_INVALID_ARGUMENT;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int c = static_cast<int>(C);
  if (C % 8 == 0 && aligned16(x) && aligned16(out))
    return launch_k3_fwd<8>(x, h_pre, out, T, c, s);
  return launch_k3_fwd<1>(x, h_pre, out, T, c, s);
}

extern "C" int fmhc_k3_bwd(const uint16_t* x, const float* h_pre, const uint16_t* grad_out,
                           uint16_t* grad_x, float* grad_h_pre, int64_t T, int64_t C, int64_t n,
                           void* stream) {
  using namespace fmhc;
  if (bad_sizes(T, C, n)) return FMHC_ERR_INVALID_ARGUMENT;
  if (T == 0) return FMHC_OK;
  if (!x || !h_pre || !grad_out || !grad_h_pre) return FMHC_ERR_INVALID_ARGUMENT;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int c = static_cast<int>(C);
  const bool vec = C % 8 == 0 && aligned16(x) && aligned16(grad_out) && (!grad_x || aligned16(grad_x));
  if (!grad_x)  // grad_h_pre only
    return vec ? launch_k3_bwd<8, false>(x, h_pre, grad_out, nullptr, grad_h_pre, T, c, s)
               : launch_k3_bwd<1, false>(x, h_pre, grad_out, nullptr, grad_h_pre, T, c, s);
  return vec ? launch_k3_bwd<8, true>(x, h_pre, grad_out, grad_x, grad_h_pre, T, c, s)
             : launch_k3_bwd<1, true>(x, h_pre, grad_out, grad_x, grad_h_pre, T, c, s);
}
