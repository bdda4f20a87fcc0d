// K4: post-mixing (residual stream mix + post-weighted layer output) and its
// backward.
//
//   forward   out[t,i,c]    = bf16(h_post[t,i] * lo[t,c] + sum_j H[t,i,j] * x[t,j,c])
//   backward  grad_lo[t,c]  = bf16(sum_i h_post[t,i] * go[t,i,c])
//             grad_hp[t,i]  = sum_c go[t,i,c] * lo[t,c]           (fp32)
//             grad_H[t,i,j] = sum_c go[t,i,c] * x[t,j,c]          (fp32)
//             grad_x[t,j,c] = bf16(sum_i H[t,i,j] * go[t,i,c])
//
// Follows src/flash_mhc/kernels.py:384-481 (forward) and :487-665 (fused
// backward) of the reference, written for gfx950: a group of LPT consecutive
// lanes owns one token and streams 16-byte vectors of every row it touches, so
// each input row is read once and each output row written once per launch.
// The backward keeps its 20 per-token partial sums in registers and finishes
// them with an in-wave butterfly (and, when a token spans several waves, an
// LDS sum over them in wave order): no atomics, deterministic.
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
__global__ __launch_bounds__(block_of<LPT>()) void k4_fwd_kernel(const uint16_t* __restrict__ x,
                                                        const uint16_t* __restrict__ lo,
                                                        const float* __restrict__ H,
                                                        const float* __restrict__ h_post,
                                                        uint16_t* __restrict__ out,
                                                        int64_t T, int C) {
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t tok = token_of_lane<LPT>(lane);
  if (tok >= T) return;
  const int sub = sub_of_lane<LPT>();
  const int ng = C / VEC;

  float h[4][4], p[4];
  {
    const float* Ht = H + tok * 16;
    const float* pt = h_post + tok * 4;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      p[i] = pt[i];
#pragma unroll
      for (int j = 0; j < 4; ++j) h[i][j] = Ht[i * 4 + j];
    }
  }
  const uint16_t* xr[4];
  uint16_t* orow[4];
  xr[0] = x + tok * 4 * C;
  orow[0] = out + tok * 4 * C;
#pragma unroll
  for (int j = 1; j < 4; ++j) {
    xr[j] = xr[j - 1] + C;
    orow[j] = orow[j - 1] + C;
  }
  const uint16_t* lrow = lo + tok * C;

#pragma unroll 2
  for (int g = sub; g < ng; g += LPT) {
    float l[VEC], xv[4][VEC];
    Lanes<VEC>::load(lrow, g, l);
#pragma unroll
    for (int j = 0; j < 4; ++j) Lanes<VEC>::load(xr[j], g, xv[j]);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float o[VEC];
#pragma unroll
      for (int e = 0; e < VEC; ++e) {
        float acc = p[i] * l[e];
#pragma unroll
        for (int j = 0; j < 4; ++j) acc = __builtin_fmaf(h[i][j], xv[j][e], acc);
        o[e] = acc;
      }
      Lanes<VEC>::store(orow[i], g, o);
    }
  }
}

template <int VEC, int LPT, bool EARLY>
__global__ __launch_bounds__(block_of<LPT>()) void k4_bwd_kernel(const uint16_t* __restrict__ x,
                                                        const uint16_t* __restrict__ lo,
                                                        const float* __restrict__ H,
                                                        const float* __restrict__ h_post,
                                                        const uint16_t* __restrict__ go,
                                                        uint16_t* __restrict__ grad_x,
                                                        uint16_t* __restrict__ grad_lo,
                                                        float* __restrict__ grad_H,
                                                        float* __restrict__ grad_hp,
                                                        int64_t T, int C) {
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

  float shp[4] = {0.f, 0.f, 0.f, 0.f};
  float sH[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) sH[i][j] = 0.f;

  if (live) {
  float h[4][4], p[4];
  {
    const float* Ht = H + tok * 16;
    const float* pt = h_post + tok * 4;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      p[i] = pt[i];
#pragma unroll
      for (int j = 0; j < 4; ++j) h[i][j] = Ht[i * 4 + j];
    }
  }
  const uint16_t* xr[4];
  const uint16_t* gr[4];
  uint16_t* gxr[4];
  xr[0] = x + tok * 4 * C;
  gr[0] = go + tok * 4 * C;
  gxr[0] = grad_x + tok * 4 * C;
#pragma unroll
  for (int j = 1; j < 4; ++j) {
    xr[j] = xr[j - 1] + C;
    gr[j] = gr[j - 1] + C;
    gxr[j] = gxr[j - 1] + C;
  }
  const uint16_t* lrow = lo + tok * C;
  uint16_t* glrow = grad_lo + tok * C;

#pragma unroll 2
  for (int g = sub; g < ng; g += LPT) {
    float q[4][VEC], l[VEC];
#pragma unroll
    for (int i = 0; i < 4; ++i) Lanes<VEC>::load(gr[i], g, q[i]);
    Lanes<VEC>::load(lrow, g, l);

    // EARLY: the iteration's x rows load with grad_out and lo, before its
    // first store (the compiler keeps a load behind an earlier store).
    float xs[EARLY ? 4 : 1][VEC];
    if constexpr (EARLY) {
#pragma unroll
      for (int j = 0; j < 4; ++j) Lanes<VEC>::load(xr[j], g, xs[j]);
    }
    // grad_lo and the grad_h_post partial sums.
    {
      float o[VEC];
#pragma unroll
      for (int e = 0; e < VEC; ++e) {
        float acc = p[0] * q[0][e];
        acc = __builtin_fmaf(p[1], q[1][e], acc);
        acc = __builtin_fmaf(p[2], q[2][e], acc);
        o[e] = __builtin_fmaf(p[3], q[3][e], acc);
      }
      Lanes<VEC>::store(glrow, g, o);
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int e = 0; e < VEC; ++e) shp[i] = __builtin_fmaf(q[i][e], l[e], shp[i]);
    }

    // One x stream at a time: grad_H partial sums and grad_x.
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      float xl[VEC], o[VEC];
      const float* xv = xl;
      if constexpr (EARLY)
        xv = xs[j];
      else
        Lanes<VEC>::load(xr[j], g, xl);
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int e = 0; e < VEC; ++e) sH[i][j] = __builtin_fmaf(q[i][e], xv[e], sH[i][j]);
#pragma unroll
      for (int e = 0; e < VEC; ++e) {
        float acc = h[0][j] * q[0][e];
        acc = __builtin_fmaf(h[1][j], q[1][e], acc);
        acc = __builtin_fmaf(h[2][j], q[2][e], acc);
        o[e] = __builtin_fmaf(h[3][j], q[3][e], acc);
      }
      Lanes<VEC>::store(gxr[j], g, o);
    }
  }
  }

  constexpr int GS = LPT < kWave ? LPT : kWave;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    shp[i] = group_sum<GS>(shp[i]);
#pragma unroll
    for (int j = 0; j < 4; ++j) sH[i][j] = group_sum<GS>(sH[i][j]);
  }
  if constexpr (WPT > 1) {
    // The token's waves add their 20 sums in wave order (deterministic).
    __shared__ float red[block_of<LPT>() / kWave][20];
    const int wave = static_cast<int>(threadIdx.x) >> 6;
    if (lane == 0) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        red[wave][16 + i] = shp[i];
#pragma unroll
        for (int j = 0; j < 4; ++j) red[wave][i * 4 + j] = sH[i][j];
      }
    }
    __syncthreads();
    if (live && sub == 0) {
      float t[20];
#pragma unroll
      for (int k = 0; k < 20; ++k) t[k] = 0.f;
#pragma unroll
      for (int w = 0; w < WPT; ++w)
#pragma unroll
        for (int k = 0; k < 20; ++k) t[k] += red[wave + w][k];
      float* dH = grad_H + tok * 16;
      float* dp = grad_hp + tok * 4;
#pragma unroll
      for (int k = 0; k < 16; ++k) dH[k] = t[k];
#pragma unroll
      for (int i = 0; i < 4; ++i) dp[i] = t[16 + i];
    }
  } else if (sub == 0) {
    float* dH = grad_H + tok * 16;
    float* dp = grad_hp + tok * 4;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      dp[i] = shp[i];
#pragma unroll
      for (int j = 0; j < 4; ++j) dH[i * 4 + j] = sH[i][j];
    }
  }
}

// Lanes per token: a full wave from one 8-element group per lane on (at
// C = 512, 64 lanes make the backward 20% and the forward 4% faster than 32),
// fewer lanes (more tokens per wave) for narrower rows.
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
// token from C = 2048 on the kernel is 13-17% faster than with one wave, and
// at C = 1024 2% faster with 128 lanes; few tokens gain most (latency bounds
// that regime).
template <int VEC>
int pick_lpt_fwd(int C) {
  const int groups = C / VEC;
  if (groups >= 256) return wide_lpt<VEC>(groups);
  if (groups >= 128) return 128;
  return pick_lpt<VEC>(C);
}

// Backward: a workgroup per token from C = 2048 on (the 20 per-token sums
// then finish across the waves in LDS): 13% faster there than one wave per
// token at T x C = 64 Mi elements.  At C = 1024 two waves per token (one
// 16-byte group per lane) with the residency cap of launch_k4_bwd: at
// T = 65536 6389-6454 against 6270-6291 GB/s in the six-kernel step, 32768
// 6298-6330 against 6149-6150, 20000 6071-6121 against 5999-6008, 262144
// 6298-6369 against 6145-6233; below the cap's threshold two waves were
// already 1-4 us faster (T = 4096 22.1 -> 21.0 us).  Other widths below
// 2048 keep one wave (a second wave would leave lanes without a group).
template <int VEC>
int pick_lpt_bwd(int C) {
  if (VEC == 8 && C / VEC == 128) return 128;
  return C / VEC >= 256 ? wide_lpt<VEC>(C / VEC) : pick_lpt<VEC>(C);
}

template <int VEC>
int launch_k4_fwd(const uint16_t* x, const uint16_t* lo, const float* H, const float* hp,
                  uint16_t* out, int64_t T, int C, hipStream_t s) {
  const int lpt = pick_lpt_fwd<VEC>(C);
  const dim3 grid(blocks_for(T, tokens_per_block(lpt)));
  // Residency cap (fmhc_common.h) from 16 workgroups per CU on.
  const bool cap = VEC == 8 && FMHC_LDS_CAP && grid.x >= 16u * 256u;
  with_lpt(lpt, [&](auto l) {
    constexpr int L = decltype(l)::value;
    static const unsigned lds = lds_reserve(reinterpret_cast<const void*>(&k4_fwd_kernel<VEC, L>), kLdsCapFive);
    k4_fwd_kernel<VEC, L><<<grid, block_of<L>(), cap ? lds : 0u, s>>>(x, lo, H, hp, out, T, C);
  });
  return launch_status();
}

constexpr int64_t kK4EarlyLanes = int64_t{16384} * 64;

template <int VEC>
int launch_k4_bwd(const uint16_t* x, const uint16_t* lo, const float* H, const float* hp,
                  const uint16_t* go, uint16_t* gx, uint16_t* glo, float* gH, float* ghp,
                  int64_t T, int C, hipStream_t s) {
  const int lpt = pick_lpt_bwd<VEC>(C);
  const dim3 grid(blocks_for(T, tokens_per_block(lpt)));
  // Residency cap (fmhc_common.h): four workgroups per CU where each lane
  // has one 16-byte group (C = 512, 1024, 2048), from 16 workgroups per CU
  // on.  Six-kernel step, GB/s for K4 backward, no cap against four:
  // T = 65536, C = 512 6401-6416 against 6448-6455, C = 2048 6139-6169
  // against 6387-6395 (cold 6127-6155 against 6426-6467); T = 262144,
  // C = 512 6278-6295 against 6452-6485.  With two groups per lane a cap
  // lost (C = 1024 on one wave per token: 5949-5969 against 6242-6249;
  // C = 4096: 4742 against 5624); at C = 2560 and 3072 it changed nothing.
  const bool cap = VEC == 8 && FMHC_LDS_CAP && C / VEC == lpt && lpt <= 256 && grid.x >= 16u * 256u;
  // Few waves (up to 64 per CU): each iteration's loads go out before its
  // stores, so a wave waits for one round trip per iteration instead of five
  // (block step at C = 1024, HIP graph: T = 1024 96.5 -> 94.6 us, 6000 232.2
  // -> 228.5 us; K4 backward alone at T = 16384 81.1 -> 79.0 us).  With more
  // waves the extra registers (124 against 90: four waves per SIMD instead of
  // five) cost more than the latency they hide (T = 32768 150.8 -> 153.5 us,
  // 65536 302.2 -> 304.3 us).
  auto launch = [&](auto early) {
    constexpr bool E = decltype(early)::value;
    with_lpt(lpt, [&](auto l) {
      constexpr int L = decltype(l)::value;
      static const unsigned lds =
          lds_reserve(reinterpret_cast<const void*>(&k4_bwd_kernel<VEC, L, E && L >= kWave>), kLdsCapFour);
      k4_bwd_kernel<VEC, L, E && L >= kWave><<<grid, block_of<L>(), cap ? lds : 0u, s>>>(x, lo, H, hp, go, gx, glo,
                                                                                         gH, ghp, T, C);
    });
  };
  // Measured on the 16-byte path with a wave or more per token; narrower
  // tokens (C < 512) keep the loop as it is.
  if constexpr (VEC == 8) {
    if (lpt >= kWave && T * lpt <= kK4EarlyLanes) {
      launch(std::true_type{});
      return launch_status();
    }
  }
  launch(std::false_type{});
  return launch_status();
}

bool bad_sizes(int64_t T, int64_t C, int64_t n) {
  return T < 0 || C <= 0 || C > (int64_t{1} << 30) || n != 4;
}

}  // namespace
}  // namespace fmhc

extern "C" int fmhc_k4_fwd(const uint16_t* x, const uint16_t* lo, const float* H,
                           const float* h_post, uint16_t* out, int64_t T, int64_t C, int64_t n,
                           void* stream) {
  using namespace fmhc;
  if (bad_sizes(T, C, n)) return FMHC_ERR_INVALID_ARGUMENT;
  if (T == 0) return FMHC_OK;
  if (!x || !lo || !H || !h_post || !out) return FMHC_ERR_INVALID_ARGUMENT;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int c = static_cast<int>(C);
  if (C % 8 == 0 && aligned16(x) && aligned16(lo) && aligned16(out))
    return launch_k4_fwd<8>(x, lo, H, h_post, out, T, c, s);
  return launch_k4_fwd<1>(x, lo, H, h_post, out, T, c, s);
}

extern "C" int fmhc_k4_bwd(const uint16_t* x, const uint16_t* lo, const float* H,
                           const float* h_post, const uint16_t* grad_out, uint16_t* grad_x,
                           uint16_t* grad_lo, float* grad_H, float* grad_h_post, int64_t T,
                           int64_t C, int64_t n, void* stream) {
  using namespace fmhc;
  if (bad_sizes(T, C, n)) return FMHC_ERR_INVALID_ARGUMENT;
  if (T == 0) return FMHC_OK;
  if (!x || !lo || !H || !h_post || !grad_out || !grad_x || !grad_lo || !grad_H || !grad_h_post)
    return FMHC_ERR_INVALID_ARGUMENT;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int c = static_cast<int>(C);
  if (C % 8 == 0 && aligned16(x) && aligned16(lo) && aligned16(grad_out) && aligned16(grad_x) &&
      aligned16(grad_lo))
    return launch_k4_bwd<8>(x, lo, H, h_post, grad_out, grad_x, grad_lo, grad_H, grad_h_post, T,
                            c, s);
  return launch_k4_bwd<1>(x, lo, H, h_post, grad_out, grad_x, grad_lo, grad_H, grad_h_post, T, c,
                          s);
}
