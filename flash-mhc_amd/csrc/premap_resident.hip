// The pre-map forward (K1 -> K2 -> K3 of block.py:157-177 of alint77/flash-mHC)
// with one read of x, for rows of C = 512 or 1024 per stream: a workgroup per
// CU keeps all of W (32 x 4C bf16, 256 KiB at C = 1024) on its CU for the
// whole launch -- at C = 1024 half in registers, half in LDS; at C = 512 all
// in LDS -- and walks 16-token blocks of rows held in registers.  Each
// block's rows are read once: K1 runs on them (matrix cores), K2 on its 16
// projections, then K3 mixes the same registers into the layer input.  No
// other workgroup is involved, so nothing waits on another CU.
//
// Why W has to be on chip: the vector memory counter of gfx950 is in order,
// so a load issued after the next block's prefetch cannot be consumed before
// that prefetch lands.  Streaming W from L2 while x is prefetched a block
// ahead would wait for the prefetch at every k-step.  With W in registers and
// LDS the only global loads are the rows of x.
//
// Layout.  Four waves per workgroup (one per SIMD, up to 512 registers each);
// wave w owns columns w CPW .. + CPW of each of the four streams (CPW = C / 4),
// i.e. KS = C / 32 k-steps of the 16x16x32 MFMA.  A block is held as two
// halves of KS / 2 k-steps, each half the same 64-column chunks of all four
// streams.  x arrives as whole 128-byte lines: for chunk c0 .. c0 + 64 of
// stream j, one load gives lane l
//   x[t0 + (l >> 3), j, c0 + 8 (l & 7) + e]   (tokens 0-7; a second load 8-15)
// so every lane holds the same tokens and columns of all four streams: K3 is
// lane-local, with k3_token's arithmetic, and its stores are whole lines too.
// For K1 the two loads go through a wave-private LDS tile (swizzled, free of
// bank conflicts) into the MFMA layout of the chunk's two k-steps:
//   x  (MFMA B):  x[t0 + (l & 15), j, c0 + 32 s + 8 (l >> 4) + e]
//   W  (MFMA A):  W[d, j C + c0 + 32 s + 8 (l >> 4) + e], d = l & 15 and 16 + (l & 15)
// The sum of squares is the diagonal of x x^T, a third MFMA on the same
// operands (exact bf16 products, fp32 sums), as in K1's one-pass kernel.  The waves' partial sums are added in
// wave order through LDS.  K2 runs 16 lanes per token (k2_token16_lds: the
// chain's bits, its cross-lane values exchanged through LDS), and the block's
// K1 / K2 outputs are staged in LDS and stored as whole 16-byte pieces of
// contiguous rows (per-lane scattered stores of them cost 40 us at
// T = 65536).
//
// Outputs: proj, inv_rms, h_pre, h_post, H_merged and the layer input, the
// values of K1 -> K2 -> K3 up to K1's fp32 summation order (this kernel
// partitions the contraction over four waves of C columns each).
//
// Loading x in the MFMA layout directly (16 tokens x 64 bytes per load, two
// loads per line) took 150-153 us at T = 65536, C = 1024 against 145-146 us
// with whole lines and the LDS tile (C = 512: 86 against 84 us), with the same
// bits; with half lines the nontemporal hint cost 14% (each half fetched on
// its own), with whole lines it gained nothing.
//
// Measured at T = 65536 (each launch after a cache flush): C = 1024 136-139 us
// against 174 us for the tile kernel that re-reads x and 205 us for three
// kernels, 1.05x the region's algorithmic bytes past L2 against 1.74x;
// C = 512 72-73 against 94 us; T = 131072, C = 1024: 258 against 331 us.
// W (256 KiB) and one and a half blocks of rows (192 KiB) fill the CU's
// registers and LDS, so a block's second half is issued only once the
// previous block's first half is mixed, and the K1 phase that needs it
// waits for it.

#include <hip/hip_runtime.h>

#include "fmhc_common.h"
#include "k1_premap.h"
#include "k2_chain.h"

namespace fmhc {
namespace {

__device__ __forceinline__ bf16x8 as_bf(u32x4 v) { return __builtin_bit_cast(bf16x8, v); }
__device__ __forceinline__ f32x4 mfma(u32x4 a, u32x4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf(a), as_bf(b), c, 0, 0, 0);
}

// K2's exchanges within a token: its softmax exponentials and weights and its
// sigmoid values (h_pre 0-3, h_post 4-7), written by the lanes that compute
// them and read back by all 32 lanes of the token (broadcast reads).
struct K2Xchg {
  float e[16][kNF];
  float a[16][kNF];
  float y[16][2 * kN];
};

// A block's K1 and K2 outputs, staged for whole-row stores (h_pre: hp below).
struct K2Out {
  uint16_t pj[16][kDk];
  float inv[16];
  float hq[16][kN];
  float H[16][kN * kN];
};

// NW waves per workgroup, KS k-steps per wave, the first KR of them with W in
// registers, the rest in LDS.
template <int NW, int KS, int KR>
struct ResidentSmem {
  u32x4 w[NW][KS > KR ? KS - KR : 1][2][kWave];  // W A operands kept in LDS (rows 0-15, 16-31)
  union {
    struct {
      float red[NW][8][kWave];  // per-wave partial projections, MFMA D layout
      float red_ss[NW][16];     // per-wave partial sums of squares
    } r;
    K2Xchg x;  // used once the partial sums have been added
  } u;
  float tok[16][kDk + 1];    // a block's sums: projections [t][d], squares [t][32]
  float hp[16][kN];          // a block's h_pre, for K3 and its store
  K2Out out;
  float permT[kN * kN][kNF];  // perm transposed: H_res entry r, permutation m
  K2Smem k2;
};

// K2 forward of token tt with 16 lanes per token, so that four waves take a
// block's 16 tokens at once: lane r (0-15) computes logits r and 16 + r
// (r < 4: h_pre, r < 8: h_post, otherwise softmax terms r - 8 and 8 + r),
// and H_res / H_merged entry r.  Every value is k2_token32's expression in its
// order (logits, the maximum over the softmax logits, the softmax denominator
// added over m = 0..23, the weights, H_res added over m = 0..23, H_merged),
// with the values other lanes hold read from LDS instead of shuffled, so the
// results are the chain's bit for bit.  p0 / p1 are projections r and 16 + r
// as bf16 values.  Outputs go to the block's staging area, and h_pre to
// hp_out unless it is null.
__device__ __forceinline__ void k2_token16_lds(const K2Smem& k2, const float (&permT)[kN * kN][kNF], K2Xchg& xc,
                                               K2Out& out, float* hp_out, int tt, int r, float p0, float p1) {
#pragma clang fp contract(off)
  const float alpha0 = r < kN ? k2.sc[0] : (r < 2 * kN ? k2.sc[1] : k2.sc[2]);
  const float z0 = rb(rb(alpha0 * p0) + k2.sc[3 + r]);
  const float z1 = rb(rb(k2.sc[2] * p1) + k2.sc[3 + 16 + r]);
  const float y = r < 2 * kN ? rb(sigmoid_f32(z0)) : 0.f;  // h_pre (r < 4), sigmoid of the post logit
  const float hq = rb(2.f * y);                             // h_post for 4 <= r < 8
  float mx = r >= 2 * kN ? fmaxf(z0, z1) : z1;
#pragma unroll
  for (int o = 8; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, 16));
  const float e0 = r >= 2 * kN ? expf(z0 - mx) : 0.f;
  const float e1 = expf(z1 - mx);
  if (r >= 2 * kN) xc.e[tt][r - 2 * kN] = e0;
  xc.e[tt][8 + r] = e1;
  if (r < 2 * kN) xc.y[tt][r] = r < kN ? y : hq;
  // The 16-lane group is part of one wave: its LDS writes precede these reads.
  const f32x4* ev = reinterpret_cast<const f32x4*>(xc.e[tt]);
  float sum = 0.f;
#pragma unroll
  for (int m4 = 0; m4 < kNF / 4; ++m4) {
    const f32x4 v = ev[m4];
    sum = sum + v[0];
    sum = sum + v[1];
    sum = sum + v[2];
    sum = sum + v[3];
  }
  if (r >= 2 * kN) xc.a[tt][r - 2 * kN] = rb(e0 / sum);
  xc.a[tt][8 + r] = rb(e1 / sum);
  const f32x4* av = reinterpret_cast<const f32x4*>(xc.a[tt]);
  const f32x4* pv = reinterpret_cast<const f32x4*>(permT[r]);
  float acc = 0.f;
#pragma unroll
  for (int m4 = 0; m4 < kNF / 4; ++m4) {
    const f32x4 am = av[m4], pm = pv[m4];
    acc = acc + am[0] * pm[0];
    acc = acc + am[1] * pm[1];
    acc = acc + am[2] * pm[2];
    acc = acc + am[3] * pm[3];
  }
  const float hp_j = xc.y[tt][r & 3];
  const float hq_i = xc.y[tt][kN + (r >> 2)];
  out.H[tt][r] = rb(rb(acc) - rb(hq_i * hp_j));
  if (r < kN) {
    if (hp_out) hp_out[r] = y;
  } else if (r < 2 * kN) {
    out.hq[tt][r - kN] = hq;
  }
}

// h_pre alone, on lanes r < 4 of the token's 16: k2_token16_lds's first
// operations for those lanes, so the same bits.  K3 needs nothing else of K2.
__device__ __forceinline__ void k2_hpre16(const K2Smem& k2, float* hp_out, int r, float p0) {
#pragma clang fp contract(off)
  if (r < kN) hp_out[r] = rb(sigmoid_f32(rb(rb(k2.sc[0] * p0) + k2.sc[3 + r])));
}

template <int NW, int KS, int KR, bool K2LATE>
__global__ __launch_bounds__(NW * kWave) void premap_resident_fwd(const uint16_t* __restrict__ x,
                                                                 const uint16_t* __restrict__ W,
                                                                 uint16_t* __restrict__ proj,
                                                                 float* __restrict__ inv_rms, const PremapTile pt,
                                                                 int64_t T) {
  static_assert(NW == 4 && KS % 4 == 0 && KR <= KS, "four waves; k-steps come in groups of four streams");
  constexpr int HPS = KS / 4;      // k-steps per stream
  constexpr int CPW = 32 * HPS;    // columns per wave and stream
  constexpr int C = CPW * NW;
  constexpr int NC = 4 * C;
  constexpr int NT = NW * kWave;
  __shared__ ResidentSmem<NW, KS, KR> sm;
  __shared__ u32x4 xt[NW][16 * 8];  // per wave: a chunk's 16 tokens x 8 swizzled 16-byte slots

  const int lane = static_cast<int>(threadIdx.x) & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) >> 6);
  const int row = lane & 15;
  const int grp = lane >> 4;
  const int cbase = wave * CPW + 8 * grp;  // the lane's column within each stream, piece 0
  const int lt = lane >> 3, ls = lane & 7;  // line layout: token lt (and 8 + lt), 16-byte slot ls
  const int ccol = wave * CPW + 8 * ls;

  const int64_t nblocks = (T + 15) / 16;
  const int64_t g0 = blockIdx.x;
  const int64_t G = gridDim.x;
  const int nb = g0 < nblocks ? static_cast<int>((nblocks - 1 - g0) / G + 1) : 0;

  // A block is loaded in two halves of NP k-steps, each half the pieces of
  // all four streams: k-step q = NP half + HH j + p holds piece HH half + p
  // of stream j.  (Halves by stream, streams 0-1 then 2-3, put every CU's
  // requests on the same 4 KiB of its rows at a time: 3.6 TB/s.)
  constexpr int NP = KS / 2;
  constexpr int HH = HPS / 2;  // pieces per stream in a half
  static_assert(HPS % 2 == 0, "two halves of pieces");
  auto col_of = [](int q) {  // offset of k-step q within a token row, past the lane's cbase
    const int half = q / NP, j = (q % NP) / HH, p = (q % NP) % HH;
    return j * C + 32 * (HH * half + p);
  };

  // K2's parameters first, then W, loaded once: k-steps below KR stay in
  // registers, the others go to LDS.  Their loads are issued before the
  // first blocks of x, so waiting for them does not wait for x.
  K2ParamRegs<NT> prm;
  prm.load(pt.P);
  u32x4 wr[KR > 0 ? KR : 1][2];
  u32x4 wl[KS > KR ? KS - KR : 1][2];
#pragma unroll
  for (int q = 0; q < KS; ++q) {
    const int k = cbase + col_of(q);
    const u32x4 a = *reinterpret_cast<const u32x4*>(W + static_cast<int64_t>(row) * NC + k);
    const u32x4 b = *reinterpret_cast<const u32x4*>(W + static_cast<int64_t>(16 + row) * NC + k);
    if (q < KR) {
      wr[q][0] = a;
      wr[q][1] = b;
    } else {
      wl[q - KR][0] = a;
      wl[q - KR][1] = b;
    }
  }
  zero_words(pt.z);

  // Half `half` of block g0 + i G: tail rows re-read the last token (not
  // stored).  Blocks past the workgroup's last re-read that one: prefetches
  // are issued unconditionally, so that every path reaches a step with the
  // same loads in flight and the compiler's in-order wait counts stay exact
  // (with a conditional prefetch the wait for a block also waited for the
  // next one's loads).
  constexpr int PPH = HH / 2;  // 64-column chunks per stream in a half
  static_assert(HH % 2 == 0, "whole 64-column chunks");
  // Register q of a half: stream q / (2 PPH), chunk (q / 2) % PPH of the
  // half, tokens 0-7 (q even) or 8-15 (q odd).
  auto load_half = [&](u32x4 (&X)[NP], int i, int half) __attribute__((always_inline)) {
    const int ic = i < nb ? i : nb - 1;
    const int64_t t0 = (g0 + static_cast<int64_t>(ic) * G) * 16;
    const int64_t ta = t0 + lt < T ? t0 + lt : T - 1;
    const int64_t tb = t0 + 8 + lt < T ? t0 + 8 + lt : T - 1;
    const uint16_t* pa = x + ta * NC + ccol;
    const uint16_t* pb = x + tb * NC + ccol;
#pragma unroll
    for (int q = 0; q < NP; ++q) {
      const int j = q / (2 * PPH), pp = (q / 2) % PPH, th = q % 2;
      const int off = j * C + 64 * (PPH * half + pp);
      X[q] = *reinterpret_cast<const u32x4*>((th ? pb : pa) + off);
    }
  };

  // Three half-block buffers in rotation.  Block i + 1's second half is
  // loaded once block i's first half is mixed, its first half once block i's
  // K1 phase is done: that phase then waits only for block i's second half,
  // which is alone in flight.  Loading the first half two steps ahead instead
  // (when block i - 1's second half is mixed) shares the bandwidth between
  // the half that phase waits for and one it does not need yet.  Measured at
  // T = 65536, each launch after a cache flush: C = 1024 136-139 against
  // 143-146 us, C = 512 78-79 against 80-84 us; T = 32768 and 131072 at
  // C = 1024: 76.4 against 81.5 us, 258 against 274 us.
  u32x4 H0[NP], H1[NP], H2[NP];
  __builtin_amdgcn_sched_barrier(0);  // W's loads first: waiting for them does not wait for x
  load_half(H0, 0, 0);  // nb >= 1: the grid has at most one workgroup per block
  load_half(H1, 0, 1);
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int q = KR; q < KS; ++q) {
    sm.w[wave][q - KR][0][lane] = wl[q - KR][0];
    sm.w[wave][q - KR][1][lane] = wl[q - KR][1];
  }
  prm.store(sm.k2);
  __syncthreads();
  {
    const float* pf = reinterpret_cast<const float*>(sm.k2.perm);  // perm[m][r], 24 x 16
    for (int i = threadIdx.x; i < kNF * kN * kN; i += NT) sm.permT[i % (kN * kN)][i / (kN * kN)] = pf[i];
  }  // read after the first block's barriers

  // Block i with its first half in A and its second half in B; D is free
  // until the step loads block i + 1's first half into it.
  auto step = [&](u32x4 (&A)[NP], u32x4 (&B)[NP], u32x4 (&D)[NP], int i) __attribute__((always_inline)) {
    const int64_t t0 = (g0 + static_cast<int64_t>(i) * G) * 16;
    // K1: this wave's share of the 32 projections and of the sum of squares.
    f32x4 a0 = {0.f, 0.f, 0.f, 0.f}, a1 = a0, gm = a0;
    // Chunk by chunk through the wave's tile (slot s of token t at
    // 8 t + (s ^ ((t >> 1) & 7))); same-wave LDS operations complete in
    // order, so the tile needs no barrier.  The k-steps run in the order
    // q = 0 .. KS - 1 of the W registers.
    u32x4* tile = xt[wave];
    const int wlo = lt * 8 + (ls ^ ((lt >> 1) & 7));
    const int whi = (8 + lt) * 8 + (ls ^ (((8 + lt) >> 1) & 7));
    const int rd0 = row * 8 + (grp ^ ((row >> 1) & 7));
    const int rd1 = row * 8 + ((4 + grp) ^ ((row >> 1) & 7));
#pragma unroll
    for (int half = 0; half < 2; ++half)
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int pp = 0; pp < PPH; ++pp) {
          const int r0 = j * 2 * PPH + 2 * pp;
          tile[wlo] = half ? B[r0] : A[r0];
          tile[whi] = half ? B[r0 + 1] : A[r0 + 1];
          const u32x4 xs0 = tile[rd0], xs1 = tile[rd1];
#pragma unroll
          for (int sub = 0; sub < 2; ++sub) {
            const u32x4 xq = sub ? xs1 : xs0;
            const int q = half * NP + j * HH + 2 * pp + sub;
            const u32x4 wa = q < KR ? wr[q < KR ? q : 0][0] : sm.w[wave][q < KR ? 0 : q - KR][0][lane];
            const u32x4 wb = q < KR ? wr[q < KR ? q : 0][1] : sm.w[wave][q < KR ? 0 : q - KR][1][lane];
            a0 = mfma(wa, xq, a0);
            a1 = mfma(wb, xq, a1);
            gm = mfma(xq, xq, gm);
          }
        }
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      sm.u.r.red[wave][r][lane] = a0[r];
      sm.u.r.red[wave][4 + r][lane] = a1[r];
    }
    // The diagonal G[row][row] sits in lane row + 16 (row >> 2), register row & 3.
    if (grp == (row >> 2)) sm.u.r.red_ss[wave][row] = gm[row & 3];
    // Block i + 1's first half, now that the loads in flight are none but
    // its second half's.
    load_half(D, i + 1, 0);
    __builtin_amdgcn_sched_barrier(0);
    __syncthreads();
    // Thread (r, l) adds D element r of lane l over the waves, in wave order:
    // projection d = 4 (l >> 4) + (r & 3) + 16 (r >> 2) of token l & 15.
#pragma unroll
    for (int r = wave; r < 8; r += NW) {
      float v = 0.f;
#pragma unroll
      for (int w = 0; w < NW; ++w) v += sm.u.r.red[w][r][lane];
      sm.tok[lane & 15][4 * (lane >> 4) + (r & 3) + 16 * (r >> 2)] = v;
    }
    if (threadIdx.x < 16) {
      float s2 = 0.f;
#pragma unroll
      for (int w = 0; w < NW; ++w) s2 += sm.u.r.red_ss[w][threadIdx.x];
      sm.tok[threadIdx.x][kDk] = s2;
    }
    __syncthreads();
    // K1's outputs and h_pre on the block's 16 tokens at once, 16 lanes per
    // token (token 4 wave + (lane >> 4)).  Rows past T (the last block) hold
    // re-reads of token T - 1: computed, never stored.
    const int tt = 4 * wave + (lane >> 4);
    const int r = lane & 15;
    const float inv = rsqrtf(sm.tok[tt][kDk] / static_cast<float>(NC) + kRmsEps);
    const uint16_t pj0 = f32_to_bf16(sm.tok[tt][r] * inv);
    const uint16_t pj1 = f32_to_bf16(sm.tok[tt][16 + r] * inv);
    sm.out.pj[tt][r] = pj0;
    sm.out.pj[tt][16 + r] = pj1;
    if (r == 0) sm.out.inv[tt] = inv;
    // The block's K1 and K2 outputs, whole 16-byte pieces of contiguous rows.
    // The next step's LDS writes come after its first barrier, which every
    // wave reaches only after these reads.
    auto store_outputs = [&]() __attribute__((always_inline)) {
      if (wave == 0) {  // proj: token lane >> 2, projections 8 (lane & 3) .. + 8
        const int64_t t = t0 + (lane >> 2);
        if (t < T)
          *reinterpret_cast<u32x4*>(proj + t * kDk + 8 * (lane & 3)) =
              reinterpret_cast<const u32x4*>(sm.out.pj[lane >> 2])[lane & 3];
      } else if (wave == 1) {  // H_merged: token lane >> 2, row lane & 3
        const int64_t t = t0 + (lane >> 2);
        if (t < T)
          reinterpret_cast<f32x4*>(pt.H)[t * kN + (lane & 3)] =
              reinterpret_cast<const f32x4*>(sm.out.H[lane >> 2])[lane & 3];
      } else if (wave == 2) {  // h_pre (lanes 0-15), h_post (16-31), inv_rms (32-47)
        const int64_t t = t0 + (lane & 15);
        if (t < T) {
          if (lane < 16)
            reinterpret_cast<f32x4*>(pt.h_pre)[t] = *reinterpret_cast<const f32x4*>(sm.hp[lane]);
          else if (lane < 32)
            reinterpret_cast<f32x4*>(pt.h_post)[t] = *reinterpret_cast<const f32x4*>(sm.out.hq[lane & 15]);
          else if (lane < 48)
            inv_rms[t] = sm.out.inv[lane & 15];
        }
      }
    };
    // K2LATE: only h_pre stands between K1 and the mix, and the rest of K2
    // (h_post, H_merged) runs after the mix, while the next block's loads
    // are in flight.  Otherwise all of K2 and the outputs' stores come first.
    // At T = 65536, each launch after a cache flush: C = 512 77.3 -> 73.2 us
    // late; C = 1024 137.3 -> 143.3 us late (the next block's second half is
    // then issued while its first half is still in flight), so it stays
    // early there.
    if constexpr (K2LATE) {
      k2_hpre16(sm.k2, sm.hp[tt], r, bf16_to_f32(pj0));
    } else {
      k2_token16_lds(sm.k2, sm.permT, sm.u.x, sm.out, sm.hp[tt], tt, r, bf16_to_f32(pj0), bf16_to_f32(pj1));
    }
    __syncthreads();
    if constexpr (!K2LATE) store_outputs();
    // K3 on the rows still in registers, a half at a time: once the first
    // half is mixed its registers take block i + 1's second half.
    const int64_t ta = t0 + lt, tb = t0 + 8 + lt;
    const bool va = ta < T, vb = tb < T;
    float hh[2][4];
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) {
      hh[0][jj] = sm.hp[lt][jj];
      hh[1][jj] = sm.hp[8 + lt][jj];
    }
    uint16_t* oa = pt.layer_input + (va ? ta : 0) * C + ccol;
    uint16_t* ob = pt.layer_input + (vb ? tb : 0) * C + ccol;
    auto mix = [&](const u32x4 (&X)[NP], int half) __attribute__((always_inline)) {
#pragma unroll
      for (int p2 = 0; p2 < 2 * PPH; ++p2) {
        const int pp = p2 / 2, th = p2 % 2;
        float a[8], b[8], c[8], d[8], o[8];
        unpack8(X[0 * 2 * PPH + p2], a);
        unpack8(X[1 * 2 * PPH + p2], b);
        unpack8(X[2 * 2 * PPH + p2], c);
        unpack8(X[3 * 2 * PPH + p2], d);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          float acc = hh[th][0] * a[e];
          acc = __builtin_fmaf(hh[th][1], b[e], acc);
          acc = __builtin_fmaf(hh[th][2], c[e], acc);
          o[e] = __builtin_fmaf(hh[th][3], d[e], acc);
        }
        // Whole lines, ordinary stores (the nontemporal hint measured the
        // same or slower).
        uint16_t* dst = (th ? ob : oa) + 64 * (PPH * half + pp);
        if (th ? vb : va) *reinterpret_cast<u32x4*>(dst) = pack8(o);
      }
    };
    mix(A, 0);
    load_half(A, i + 1, 1);
    __builtin_amdgcn_sched_barrier(0);  // all of block i + 1 before block i + 2 (in-order wait counts)
    mix(B, 1);
    if constexpr (K2LATE) {
      // The rest of K2 (h_post, H_merged; its h_pre is the value above).
      k2_token16_lds(sm.k2, sm.permT, sm.u.x, sm.out, nullptr, tt, r, bf16_to_f32(pj0), bf16_to_f32(pj1));
      __syncthreads();
      store_outputs();
    }
  };

  // Block i in (H[2i % 3], H[(2i + 1) % 3]).  The loop body has no exit
  // between its steps: with a `break` after a step, the reload issued there
  // was dead on that path, and hipcc (ROCm 7.2) sank it into the next step,
  // where the scheduler placed it after that step's K1 phase, which then
  // waited for it.  The last one or two blocks run after the loop.
  int i = 0;
  for (; i + 3 <= nb; i += 3) {
    step(H0, H1, H2, i);
    step(H2, H0, H1, i + 1);
    step(H1, H2, H0, i + 2);
  }
  if (i < nb) {
    step(H0, H1, H2, i);
    if (i + 1 < nb) step(H2, H0, H1, i + 1);
  }
}

// Compute units of each device, looked up on the first launch there (a racing
// first lookup stores the same value).
constexpr int kMaxDevices = 64;
int g_cus[kMaxDevices];

int device_cus() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return 0;
  if (g_cus[dev] <= 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
    g_cus[dev] = n;
  }
  return g_cus[dev];
}

}  // namespace

// The resident kernel for rows of C = 512 or 1024 per stream; returns false
// (nothing launched) for other shapes, fewer than kResidentMinT tokens, no
// layer input or misaligned pointers.
bool premap_resident(const uint16_t* x, const uint16_t* W, uint16_t* proj, float* inv_rms, const PremapTile& pt,
                     int64_t T, int64_t C, hipStream_t s, int* status) {
  if (!(C == 1024 || C == 512) || T < kResidentMinT || !pt.layer_input || !aligned16(x) || !aligned16(W) ||
      !aligned16(pt.layer_input) || !aligned16(proj) || !aligned16(pt.h_pre) || !aligned16(pt.h_post) ||
      !aligned16(pt.H))
    return false;
  const int cus = device_cus();
  if (cus <= 0) return false;
  const int64_t nblocks = (T + 15) / 16;
  const unsigned grid = static_cast<unsigned>(nblocks < cus ? nblocks : cus);
  if (C == 1024)
    premap_resident_fwd<4, 32, 16, false><<<grid, 4 * kWave, 0, s>>>(x, W, proj, inv_rms, pt, T);
  else
    premap_resident_fwd<4, 16, 0, true><<<grid, 4 * kWave, 0, s>>>(x, W, proj, inv_rms, pt, T);
  *status = launch_status();
  return true;
}

}  // namespace fmhc
