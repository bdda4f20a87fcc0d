// Shared device helpers for the mHC-lite K1/K3/K4 HIP kernels (gfx950, wave64).
//
// Data conventions used by every kernel in this library:
//   * bf16 tensors arrive as uint16_t bit patterns, row-major and contiguous.
//   * fp32 accumulation everywhere; every bf16 output is rounded exactly once,
//     round-to-nearest-even, by the hardware v_cvt_pk_bf16_f32 conversion.
//   * The "vector" code paths move 16 bytes (8 bf16) per lane per memory
//     instruction; they need C % 8 == 0 and 16-byte aligned base pointers.
//     The "scalar" code paths move one element per lane and accept any C and
//     any 2-byte alignment.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/flash_mhc_hip.h"

namespace fmhc {

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

constexpr int kWave = 64;

// Streaming loads/stores.  Data that is read or written exactly once per
// launch carries the nontemporal hint so it does not evict the small,
// reused operands (W, coefficients) from the caches.
#ifndef FMHC_NT_LOADS
#define FMHC_NT_LOADS 1
#endif
#ifndef FMHC_NT_STORES
#define FMHC_NT_STORES 1
#endif

template <typename V>
__device__ __forceinline__ V ld_stream(const V* p) {
#if FMHC_NT_LOADS
  return __builtin_nontemporal_load(p);
#else
  return *p;
#endif
}

template <typename V>
__device__ __forceinline__ void st_stream(V* p, V v) {
#if FMHC_NT_STORES
  __builtin_nontemporal_store(v, p);
#else
  *p = v;
#endif
}

// bf16 bit pattern -> fp32 (exact).
__device__ __forceinline__ float bf_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf_hi(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }
__device__ __forceinline__ float bf16_to_f32(uint16_t h) {
  return __uint_as_float(static_cast<uint32_t>(h) << 16);
}

// Two fp32 -> packed bf16 pair, round-to-nearest-even (v_cvt_pk_bf16_f32).
__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
  bf16x2 r = {static_cast<__bf16>(a), static_cast<__bf16>(b)};
  return __builtin_bit_cast(uint32_t, r);
}
__device__ __forceinline__ uint16_t f32_to_bf16(float a) {
  return __builtin_bit_cast(uint16_t, static_cast<__bf16>(a));
}

__device__ __forceinline__ void unpack8(const u32x4 v, float f[8]) {
  f[0] = bf_lo(v.x); f[1] = bf_hi(v.x);
  f[2] = bf_lo(v.y); f[3] = bf_hi(v.y);
  f[4] = bf_lo(v.z); f[5] = bf_hi(v.z);
  f[6] = bf_lo(v.w); f[7] = bf_hi(v.w);
}

__device__ __forceinline__ u32x4 pack8(const float f[8]) {
  u32x4 v;
  v.x = pack_bf16x2(f[0], f[1]);
  v.y = pack_bf16x2(f[2], f[3]);
  v.z = pack_bf16x2(f[4], f[5]);
  v.w = pack_bf16x2(f[6], f[7]);
  return v;
}

// Element group moved by one lane per step: VEC = 8 (one 16-byte vector) or
// VEC = 1 (one bf16 scalar).  `idx` counts groups, so the element offset is
// idx * VEC.  raw() issues the load and keeps the packed bf16 bits; unpack()
// widens them to fp32; load() does both.
template <int VEC>
struct Lanes;

template <>
struct Lanes<8> {
  using Raw = u32x4;
  __device__ static __forceinline__ Raw raw(const uint16_t* __restrict__ row, int idx) {
    return ld_stream(reinterpret_cast<const u32x4*>(row) + idx);
  }
  __device__ static __forceinline__ void unpack(const Raw v, float f[8]) { unpack8(v, f); }
  __device__ static __forceinline__ void load(const uint16_t* __restrict__ row, int idx, float f[8]) {
    unpack8(raw(row, idx), f);
  }
  __device__ static __forceinline__ void store(uint16_t* __restrict__ row, int idx, const float f[8]) {
    st_stream(reinterpret_cast<u32x4*>(row) + idx, pack8(f));
  }
};

template <>
struct Lanes<1> {
  using Raw = uint32_t;
  __device__ static __forceinline__ Raw raw(const uint16_t* __restrict__ row, int idx) { return row[idx]; }
  __device__ static __forceinline__ void unpack(const Raw v, float f[1]) { f[0] = __uint_as_float(v << 16); }
  __device__ static __forceinline__ void load(const uint16_t* __restrict__ row, int idx, float f[1]) {
    unpack(raw(row, idx), f);
  }
  __device__ static __forceinline__ void store(uint16_t* __restrict__ row, int idx, const float f[1]) {
    row[idx] = f32_to_bf16(f[0]);
  }
};

// K3 forward of one token: out[c] = bf16(h0 x0[c] + h1 x1[c] + h2 x2[c] +
// h3 x3[c]), the products added in stream order with fused multiply-adds;
// element groups g = first, first + step, ... below C / VEC.  Shared by the
// K3 kernel and the pre-map's few-token kernel, which must agree bit for bit.
template <int VEC>
__device__ __forceinline__ void k3_token(const uint16_t* __restrict__ x0, const float h[4],
                                         uint16_t* __restrict__ orow, int first, int step, int C) {
  const uint16_t* x1 = x0 + C;
  const uint16_t* x2 = x1 + C;
  const uint16_t* x3 = x2 + C;
  const int ng = C / VEC;
#pragma unroll 2
  for (int g = first; g < ng; g += step) {
    float a[VEC], b[VEC], c[VEC], d[VEC], o[VEC];
    Lanes<VEC>::load(x0, g, a);
    Lanes<VEC>::load(x1, g, b);
    Lanes<VEC>::load(x2, g, c);
    Lanes<VEC>::load(x3, g, d);
#pragma unroll
    for (int e = 0; e < VEC; ++e) {
      float acc = h[0] * a[e];
      acc = __builtin_fmaf(h[1], b[e], acc);
      acc = __builtin_fmaf(h[2], c[e], acc);
      o[e] = __builtin_fmaf(h[3], d[e], acc);
    }
    Lanes<VEC>::store(orow, g, o);
  }
}

// Residency caps.  The K3 / K4 kernels use a few dozen VGPRs, so eight
// 4-wave workgroups could share a CU; several run faster with fewer (the
// host's launch reserves LDS the kernel does not use: the CU's 160 KiB hold
// six workgroups of kLdsCapSix, five of kLdsCapFive).  K1's backward dx
// likewise runs faster with one workgroup per CU than with two (k1.hip).
// Measured at T = 65536 (GB/s in the six-kernel step, eight workgroups per CU
// against the cap): K3 forward 6047-6092 against 6344-6405 with six (C =
// 1024; also 5.60-5.67 against 5.88-5.93 TB/s at T = 262144, C = 4096);
// K3 backward 6015-6070 against 6123-6175 with five at C = 1024 and
// 6195-6252 against 6436-6605 at C = 2048; K4 forward 6325-6368 against
// 6440-6478 with five at C = 1024, 6135-6175 against 6364-6420 at C = 2048.
// Where a cap lost it is not applied: K3 backward at C = 4096 (5.57 against
// 5.35-5.41 TB/s at T = 262144) and in the pre-map backward's reduce-only
// pass (C = 2048: 846 against 862-872 us; at C = 1024 five per CU changed
// nothing, 424-427 against 426-437 us at T = 65536), and K4 forward with few
// workgroups per CU (T = 4096, C = 1024: a second round of workgroups).
// Caps of five for K3 forward or six for K3 backward measured slower than
// none, so the effect is not simply fewer memory requests in flight.
#ifndef FMHC_LDS_CAP
#define FMHC_LDS_CAP 1
#endif
constexpr unsigned kLdsCapSix = 24 * 1024;
constexpr unsigned kLdsCapFive = 32 * 1024;
constexpr unsigned kLdsCapFour = 40 * 1024;  // K4 backward, one group per lane (k4.hip)
// One workgroup per CU (K1 backward dx, k1.hip).
constexpr unsigned kLdsCapOne = 96 * 1024;
constexpr unsigned kLdsPerCu = 160 * 1024;

// The reserve `dyn` for `kernel` if the kernel's own LDS plus dyn fit in a
// CU's LDS, else 0 (no cap): a launch asking for more LDS than the CU holds
// is not refused, and faults.  Callers keep the result in a static of the
// launch site's kernel instantiation.
inline unsigned lds_reserve(const void* kernel, unsigned dyn) {
  hipFuncAttributes a;
  if (dyn == 0 || hipFuncGetAttributes(&a, kernel) != hipSuccess) return 0u;
  return a.sharedSizeBytes + dyn <= kLdsPerCu ? dyn : 0u;
}

// Sum over the wave's 64 lanes, every lane receiving the total, with the
// pairs of group_sum<64>'s butterfly (lanes 32 apart first, then 16, 8, 4,
// 2, 1), so the same bits, on the VALU's cross-lane moves instead of LDS
// permutes.  Lanes 32 apart (v_permlane32_swap, which exchanges the two
// halves of its operands) and 16 apart (v_permlane16_swap: odd rows of one
// operand with even rows of the other); every 16-lane row then holds the same
// values, so a rotation by 8 within the row pairs lane j with j ^ 8, and, the
// values now repeating every 8 lanes, a rotation by 4 pairs j with a lane
// holding j ^ 4's value; quad permutations pair j ^ 2 and j ^ 1.  Every lane
// of the wave must be active.
__device__ __forceinline__ float wave_sum(float v) {
  const auto h = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = __uint_as_float(h[0]) + __uint_as_float(h[1]);
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = __uint_as_float(r[0]) + __uint_as_float(r[1]);
  // DPP controls: row_ror:8, row_ror:4, quad_perm [2,3,0,1], quad_perm [1,0,3,2].
  v += __uint_as_float(__builtin_amdgcn_update_dpp(0u, __float_as_uint(v), 0x128, 0xf, 0xf, false));
  v += __uint_as_float(__builtin_amdgcn_update_dpp(0u, __float_as_uint(v), 0x124, 0xf, 0xf, false));
  v += __uint_as_float(__builtin_amdgcn_update_dpp(0u, __float_as_uint(v), 0x4e, 0xf, 0xf, false));
  v += __uint_as_float(__builtin_amdgcn_update_dpp(0u, __float_as_uint(v), 0xb1, 0xf, 0xf, false));
  return v;
}

// Sum over the four lanes 16 apart (one per 16-lane row), in the order of the
// two shuffle steps v += v[lane ^ 16]; v += v[lane ^ 32]: v_permlane16_swap
// pairs each row with its neighbour, v_permlane32_swap the two halves.  Every
// lane of the wave must be active.
__device__ __forceinline__ float rows_sum(float v) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = __uint_as_float(r[0]) + __uint_as_float(r[1]);
  const auto h = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(h[0]) + __uint_as_float(h[1]);
}

// Sum over each 16-lane row, every lane of the row receiving the total: the
// butterfly lanes 1, 2, 4, 8 apart.  Quad permutations pair lane ^ 1 and
// lane ^ 2; the half-row mirror (lane j with 7 - j within each 8) then pairs
// the same values as lane ^ 4, since every quad holds one value by then, and
// the row mirror (j with 15 - j) those of lane ^ 8.  All 16 lanes of a row
// must be active.
__device__ __forceinline__ float row16_sum(float v) {
  // DPP controls: quad_perm [1,0,3,2], quad_perm [2,3,0,1], row_half_mirror, row_mirror.
  v += __uint_as_float(__builtin_amdgcn_update_dpp(0u, __float_as_uint(v), 0xb1, 0xf, 0xf, false));
  v += __uint_as_float(__builtin_amdgcn_update_dpp(0u, __float_as_uint(v), 0x4e, 0xf, 0xf, false));
  v += __uint_as_float(__builtin_amdgcn_update_dpp(0u, __float_as_uint(v), 0x141, 0xf, 0xf, false));
  v += __uint_as_float(__builtin_amdgcn_update_dpp(0u, __float_as_uint(v), 0x140, 0xf, 0xf, false));
  return v;
}

// Slice order of the per-token stream sums s_j = sum_c x[t, j, c] g[t, c]
// (K3's grad_h_pre) for rows with C a multiple of 128, shared by every kernel
// that produces them, so that each gives the same bits however it splits a
// row: each 8-element group's products as an FMA chain from zero, row16_sum
// over the 16 groups of each 128-column slice, then the C / 128 slice sums
// added in slice order (the first one taken as is).
constexpr int kSliceCols = 128;
constexpr int kMaxSlices = 64;  // C up to 8192 per stream
constexpr int kCanonRounds = 4;  // 16-byte groups per lane

// The slice order applies to a K3-backward layout of lpt lanes per token with
// 16-byte groups: C a multiple of 128, at most kMaxSlices slices, at least 16
// lanes per token and at most kCanonRounds groups per lane.
inline bool k3_canon(int64_t C, int lpt) {
  return C % kSliceCols == 0 && C / kSliceCols <= kMaxSlices && lpt >= 16 && C / 8 <= int64_t{kCanonRounds} * lpt;
}

// One round of a token held by LPT aligned lanes (16 <= LPT <= 64) whose lane
// sub holds group sub + k LPT of the row: e[j] is that group's FMA chain
// (zero past the row).  Adds slices k LPT / 16 ... of the round to s[j], in
// slice order; ns = C / 128.  Every lane of the token must be active.
template <int LPT>
__device__ __forceinline__ void slice_sums_add(float (&e)[4], float (&s)[4], int k, int ns, int lane) {
  static_assert(LPT >= 16 && LPT <= 64, "rows of 16 lanes within one wave");
#pragma unroll
  for (int j = 0; j < 4; ++j) e[j] = row16_sum(e[j]);
  const int tb = lane & ~(LPT - 1);
#pragma unroll
  for (int r = 0; r < LPT / 16; ++r) {
    const int sigma = k * (LPT / 16) + r;
    if (sigma < ns) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        // A whole wave per token: the row's sum is read as a scalar (no LDS).
        const float p = LPT == kWave ? __int_as_float(__builtin_amdgcn_readlane(__float_as_int(e[j]), 16 * r))
                                     : __shfl(e[j], tb + 16 * r, kWave);
        s[j] = sigma == 0 ? p : s[j] + p;
      }
    }
  }
}

// Sum over the LPT consecutive lanes that share one token (LPT a power of
// two <= 64): a butterfly, lanes LPT / 2 apart first.  Every lane of the
// group receives the total.  LPT = 64 runs wave_sum (same bits) and needs
// every lane of the wave active.
template <int LPT>
__device__ __forceinline__ float group_sum(float v) {
  if constexpr (LPT == kWave) {
    return wave_sum(v);
  } else {
#pragma unroll
    for (int m = LPT / 2; m >= 1; m >>= 1) v += __shfl_xor(v, m, kWave);
    return v;
  }
}

// Status helpers shared by the C entry points.
inline int hip_status(hipError_t e) {
  return e == hipSuccess ? FMHC_OK : FMHC_ERR_HIP_BASE + static_cast<int>(e);
}

inline int launch_status() { return hip_status(hipGetLastError()); }

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

inline unsigned int blocks_for(int64_t items, int64_t per_block) {
  return static_cast<unsigned int>((items + per_block - 1) / per_block);
}

}  // namespace fmhc
