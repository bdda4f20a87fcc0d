// The pre-map backward (K3's grad_h_pre, K2's backward, K1's backward with
// grad_W and the K3 term of grad_x; autograd through block.py:157-177 of
// alint77/flash-mHC) with one read of x.
//
// Each token's grad_proj depends on grad_h_pre, a sum over the token's whole
// row of x, and K1's backward needs grad_proj before it can use the row.
// K1's backward with grad_W keeps 32 x 128 fp32 accumulators per 128-column
// slice for a whole run of tokens, so a row cannot sit on one CU.  Here the
// waves of the slices of a row form a team (nslices / 4 workgroups, one per
// CU) that walks the runs of k1_bwd_mfma side by side, block by block:
//
//   1. each wave loads its slice of a 16-token block (x and go3), adds the
//      slice's share of grad_h_pre (the slice order of slice_sums_add), and
//      publishes the 16 values to the team's exchange ring; the block stays
//      in the wave's LDS;
//   2. one wave of the team (rotating over blocks and workgroups) gathers the
//      block's nslices x 16 values, adds them in slice order, runs K2's
//      backward on the 16 tokens (k2_bwd_quad_token, the four-lane kernel's
//      chain) and publishes their grad_proj;
//   3. kLag blocks later every wave takes the block's grad_proj and its slice
//      back from LDS and runs k1_bwd_mfma's pre-map step on it: dx, the K3
//      and incoming terms of grad_x, and the grad_W accumulators.
//
// x, go3, the incoming gradient and grad_x cross HBM once.  The values are
// those of K3's backward -> K2's backward -> K1's backward (premap.hip's
// three-kernel backward) bit for bit: the same grad_h_pre order, the same K2
// chain and 16-token parameter partials, and the same runs, block order and
// grad_W partials as k1_bwd_mfma.
//
// Exchange.  A ring word is 64 bits, the value in the low half and the
// block's sequence number + 1 in the high half, stored and loaded as one
// relaxed agent-scope atomic, so a word read is either old or the published
// value with its tag, and no fence is needed.  The caller's ring starts
// zeroed (split_ring_zero).  Every wait is bounded (spin polls): a wave that
// does not see a value in time computes it itself from HBM with the same
// code, so the result is the same and the kernel always finishes, whether or
// not the team's workgroups are resident together (the grid is one
// workgroup per CU, so normally they are).
#include <hip/hip_runtime.h>

#include <cstdlib>

#include "flash_mhc_hip.h"
#include "fmhc_common.h"
#include "k1_premap.h"
#include "k2_chain.h"

namespace fmhc {

namespace {

constexpr int kDout = 32;
constexpr int kLag = 3;           // blocks between a block's slice sums and its dx
constexpr int kStash = kLag + 1;  // LDS slots per wave
constexpr int kRing = 8;          // exchange slots per team
constexpr int kSplitWaves = 1024; // one wave per SIMD of 256 CUs
constexpr int kSpinDefault = 4096;

typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ bf16x8 as_bf16x8(u32x4 v) { return __builtin_bit_cast(bf16x8, v); }
__device__ __forceinline__ f32x4 mfma16(bf16x8 a, bf16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ void put_word(uint64_t* p, uint32_t v, uint32_t tag) {
  __hip_atomic_store(p, (static_cast<uint64_t>(tag) << 32) | v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint64_t get_word(uint64_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

struct SplitArgs {
  const uint16_t* x;        // (T, nC)
  const uint16_t* W;        // (32, nC)
  const uint16_t* proj;     // (T, 32)
  const float* inv_rms;     // (T)
  const uint16_t* go3;      // (T, C), the layer input's gradient
  const float* h_pre;       // (T, 4)
  const float* g_hpost;     // (T, 4) or null
  const float* g_H;         // (T, 16) or null
  const uint16_t* gi;       // (T, nC): x's incoming gradient (GI)
  uint16_t* gx;             // (T, nC)
  float* dw_partial;        // [nruns][nslices][8][2][4][64], as k1_bwd_mfma
  float* k2_partial;        // [nblocks][kNPar]: one partial per 16-token block
  uint64_t* ring;           // [nteams][kRing][ring_words]
  K2Params P;
  int64_t T, nblocks, nruns;
  int nC, C, nslices, ns, nteams, wpt, spin;
};

// Ring slot: nslices x 16 slice sums, then 16 tokens x 16 words of grad_proj.
__host__ __device__ __forceinline__ int64_t ring_words(int nslices) { return int64_t{nslices} * 16 + 16 * 16; }

// Fragment of one step: the slice of block i (first pass) and the step's
// operands of block i - kLag (dx).
template <bool GI>
struct SplitFrag {
  u32x4 xv[4];  // x of tokens 4 grp + q at the lane's 8 k
  u32x4 g3[4];  // go3 of those tokens at the lane's 8 c
  u32x4 pv;     // proj of token col, d = 8 grp .. + 8 (dx block)
  float inv[4]; // inv_rms of tokens 4 grp + q (dx block)
  float hp[4];  // their h_pre of the lane's stream (dx block)
  u32x4 gi[GI ? 4 : 1];
};

template <bool GI>
__global__ __launch_bounds__(256) void premap_bwd_split(const SplitArgs a) {
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) >> 6);
  const int col = lane & 15;  // token of the A / D rows, B / D column
  const int grp = lane >> 4;  // d group of A / B, 4-token group of D
  // Workgroups are dispatched round-robin over the 8 XCDs; logical ids run
  // XCD by XCD so that a team's workgroups share one L2 where they fit.
  const unsigned G = gridDim.x, bid = blockIdx.x;
  const unsigned lid = G % 8u == 0 ? (bid % 8u) * (G / 8u) + bid / 8u : bid;
  const int team = static_cast<int>(lid) / a.wpt;
  const int member = static_cast<int>(lid) % a.wpt;
  const int slice = member * 4 + wave;  // the wave's 128 columns of nC
  const int kl = slice * 128 + 8 * col;
  const int sj = slice * 128 / a.C;  // the slice's stream
  const uint32_t row_bytes = 2u * static_cast<uint32_t>(a.nC);
  const uint32_t kbytes = 2u * static_cast<uint32_t>(kl);
  const uint32_t c3bytes = 2u * static_cast<uint32_t>(kl - sj * a.C);

  __shared__ K2Smem sm;
  __shared__ u32x4 stash[4][kStash][8][kWave];  // per wave and slot: x (4 vectors), go3 (4)
  __shared__ uint32_t gtile[4][16 * 16];        // wave-private 16 tokens x 32 d bf16
  __shared__ float red[4][16][kNPar];           // K2's per-token parameter terms
  stage_params<256>(a.P, sm);

  // B tiles of dx: bfr[m] holds W[8 grp + e][kl + m], e = 0..7 (k1_bwd_mfma's).
  bf16x8 bfr[8];
  {
    u32x4 rows[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) rows[e] = *reinterpret_cast<const u32x4*>(a.W + static_cast<int64_t>(8 * grp + e) * a.nC + kl);
#pragma unroll
    for (int m = 0; m < 8; ++m) {
      uint32_t h[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const uint32_t w = rows[e][m >> 1];
        h[e] = (m & 1) ? (w >> 16) : (w & 0xffffu);
      }
      const u32x4 v = {h[0] | (h[1] << 16), h[2] | (h[3] << 16), h[4] | (h[5] << 16), h[6] | (h[7] << 16)};
      bfr[m] = as_bf16x8(v);
    }
  }

  // The team's blocks: runs r = team, team + nteams, ... (r < nruns), each
  // run's blocks tb = 0, 1, ... at token block r + tb nruns, in that order.
  const int64_t q = a.nblocks / a.nruns, rem = a.nblocks % a.nruns;
  const int64_t kq1 = rem > team ? (rem - team + a.nteams - 1) / a.nteams : 0;  // team runs with q + 1 blocks
  const int64_t nrun_team = team < a.nruns ? (a.nruns - team + a.nteams - 1) / a.nteams : 0;
  const int64_t S = nrun_team * q + (kq1 < nrun_team ? kq1 : nrun_team);
  if (S == 0) return;  // every team has a run (nteams <= nruns); kept for safety
  struct Blk {
    int64_t run, tbase;
    int rows;
    bool last;  // last block of its run
  };
  auto block_at = [&](int64_t s) {
    int64_t k, tb;
    if (s < kq1 * (q + 1)) {
      k = s / (q + 1);
      tb = s - k * (q + 1);
    } else {
      const int64_t s2 = s - kq1 * (q + 1);
      k = kq1 + s2 / q;
      tb = s2 - (s2 / q) * q;
    }
    Blk b;
    b.run = team + k * a.nteams;
    b.tbase = (b.run + tb * a.nruns) * 16;
    b.rows = static_cast<int>(a.T - b.tbase < 16 ? a.T - b.tbase : 16);
    const int64_t nb = q + (b.run < rem ? 1 : 0);
    b.last = tb == nb - 1;
    return b;
  };
  auto slot_of = [&](int64_t s) { return a.ring + (static_cast<int64_t>(team) * kRing + s % kRing) * ring_words(a.nslices); };
  // The wave that runs K2 for block s: consecutive blocks on different workgroups.
  auto k2_wave_of = [&](int64_t s) { return static_cast<int>((s % a.wpt) * 4 + (s / a.wpt) % 4); };

  // Loads of the first pass of block s1 and of the dx operands of block s3
  // (both clamped into the team's range, so that every step issues them).
  auto load = [&](SplitFrag<GI>& f, int64_t s1, int64_t s3) {
    {
      const Blk b = block_at(s1 < S ? s1 : S - 1);
      const int last = b.rows - 1;  // rows past the end re-read the last one
      const char* xb = reinterpret_cast<const char*>(a.x + b.tbase * a.nC);
      const char* g3b = reinterpret_cast<const char*>(a.go3 + b.tbase * a.C);
#pragma unroll
      for (int qq = 0; qq < 4; ++qq) {
        const int r0 = 4 * grp + qq;
        const uint32_t r = static_cast<uint32_t>(r0 < last ? r0 : last);
        f.xv[qq] = ld_stream(reinterpret_cast<const u32x4*>(xb + (r * row_bytes + kbytes)));
        // Ordinary load: the four streams' slices read the same go3 row.
        f.g3[qq] = *reinterpret_cast<const u32x4*>(g3b + (r * 2u * static_cast<uint32_t>(a.C) + c3bytes));
      }
    }
    {
      const Blk b = block_at(s3 < 0 ? 0 : (s3 < S ? s3 : S - 1));
      const int last = b.rows - 1;
      const int rg = col < last ? col : last;
      f.pv = *reinterpret_cast<const u32x4*>(a.proj + (b.tbase + rg) * kDout + 8 * grp);
#pragma unroll
      for (int qq = 0; qq < 4; ++qq) {
        const int r0 = 4 * grp + qq;
        const int64_t t = b.tbase + (r0 < last ? r0 : last);
        f.inv[qq] = a.inv_rms[t];
        f.hp[qq] = a.h_pre[t * 4 + sj];
        if constexpr (GI)
          f.gi[qq] = ld_stream(reinterpret_cast<const u32x4*>(reinterpret_cast<const char*>(a.gi + t * a.nC) + kbytes));
      }
    }
  };

  // Slice sums of the lane's four tokens (every lane of a 16-lane row holds
  // the row's four values); x and go3 as loaded for the first pass.
  auto slice_sums = [&](const u32x4 (&xv)[4], const u32x4 (&g3)[4], float (&e)[4]) {
#pragma unroll
    for (int qq = 0; qq < 4; ++qq) {
      float xf[8], gf[8];
      unpack8(xv[qq], xf);
      unpack8(g3[qq], gf);
      float acc = 0.f;
#pragma unroll
      for (int m = 0; m < 8; ++m) acc = __builtin_fmaf(xf[m], gf[m], acc);
      e[qq] = row16_sum(acc);
    }
  };

  // grad_h_pre of block s for the quad layout (lane: token lane >> 2, stream
  // lane & 3), summed in slice order from the ring, or, if a value does not
  // arrive within spin polls, from the block's rows in HBM (same values).
  const int ktok = lane >> 2, kqd = lane & 3;
  auto gather_gpre = [&](int64_t s) -> float {
    uint64_t* base = slot_of(s);
    const uint32_t tag = static_cast<uint32_t>(s + 1);
    for (int it = 0; a.spin >= 0; ++it) {  // spin < 0: no waiting at all (tests)
      int ok = 1;
      float acc = 0.f;
      for (int sg = 0; sg < a.ns; ++sg) {
        const uint64_t w = get_word(base + (kqd * a.ns + sg) * 16 + ktok);
        ok &= static_cast<uint32_t>(w >> 32) == tag;
        const float p = __uint_as_float(static_cast<uint32_t>(w));
        acc = sg == 0 ? p : acc + p;
      }
      if (__all(ok)) return acc;
      if (it >= a.spin) break;
      __builtin_amdgcn_s_sleep(2);
    }
    // Fallback: every slice from HBM, in slice order per stream.
    const Blk b = block_at(s);
    const int last = b.rows - 1;
    float acc = 0.f;
    for (int sl = 0; sl < a.nslices; ++sl) {
      const int klf = sl * 128 + 8 * col;
      const int sjf = sl * 128 / a.C;
      const char* xb = reinterpret_cast<const char*>(a.x + b.tbase * a.nC);
      const char* g3b = reinterpret_cast<const char*>(a.go3 + b.tbase * a.C);
      u32x4 xv[4], g3[4];
#pragma unroll
      for (int qq = 0; qq < 4; ++qq) {
        const int r0 = 4 * grp + qq;
        const uint32_t r = static_cast<uint32_t>(r0 < last ? r0 : last);
        xv[qq] = *reinterpret_cast<const u32x4*>(xb + (r * row_bytes + 2u * static_cast<uint32_t>(klf)));
        g3[qq] = *reinterpret_cast<const u32x4*>(g3b + (r * 2u * static_cast<uint32_t>(a.C) +
                                                         2u * static_cast<uint32_t>(klf - sjf * a.C)));
      }
      float e[4];
      slice_sums(xv, g3, e);
      // Token ktok's value sits in row ktok / 4, register ktok % 4.
      const int src = (ktok >> 2) * 16;
      const float v0 = __shfl(e[0], src, kWave), v1 = __shfl(e[1], src, kWave);
      const float v2 = __shfl(e[2], src, kWave), v3 = __shfl(e[3], src, kWave);
      const int qsel = ktok & 3;
      const float v = qsel == 0 ? v0 : (qsel == 1 ? v1 : (qsel == 2 ? v2 : v3));
      if (sjf == kqd) acc = sl == sjf * a.ns ? v : acc + v;
    }
    return acc;
  };

  // K2's backward of block s on the quad layout; gp: the lane's 8 grad_proj
  // values (token ktok, d = 8 kqd ..).  With `partial`, also the block's
  // parameter partial (16 tokens in order, idle tokens contributing zero).
  auto k2_block = [&](int64_t s, float G, float (&gp)[8], bool partial) {
    const Blk b = block_at(s);
    const bool valid = ktok < b.rows;
    const int64_t t = b.tbase + (valid ? ktok : b.rows - 1);
    float p[8];
    unpack8(*reinterpret_cast<const u32x4*>(a.proj + t * kDout + 8 * kqd), p);
    float gH[kN * kN], gpost[kN], gpre[kN];
#pragma unroll
    for (int ij = 0; ij < kN * kN; ++ij) gH[ij] = a.g_H ? a.g_H[t * kN * kN + ij] : 0.f;
#pragma unroll
    for (int i = 0; i < kN; ++i) gpost[i] = a.g_hpost ? a.g_hpost[t * kN + i] : 0.f;
    gpre[0] = quad_lane<0>(G);
    gpre[1] = quad_lane<1>(G);
    gpre[2] = quad_lane<2>(G);
    gpre[3] = quad_lane<3>(G);
    float gz[8], s0, s1, s2;
    k2_bwd_quad_token(sm, kqd, p, gH, gpost, gpre, gp, gz, s0, s1, s2);
    if (partial) {
      float* rw = red[wave][ktok];
#pragma unroll
      for (int u = 0; u < 8; ++u) rw[3 + 8 * kqd + u] = valid ? gz[u] : 0.f;
      if (kqd == 0) {
        rw[0] = valid ? s0 : 0.f;
        rw[1] = valid ? s1 : 0.f;
        rw[2] = valid ? s2 : 0.f;
      }
      // Same-wave LDS operations are performed in order.
      if (lane < kNPar) {
        float v = 0.f;
#pragma unroll
        for (int w = 0; w < 16; ++w) v += red[wave][w][lane];
        a.k2_partial[(b.tbase / 16) * kNPar + lane] = v;
      }
    }
  };

  // grad_proj of block s in the A layout (lane: token col, d = 8 grp .. + 8),
  // from the ring, or computed here if it does not arrive within spin polls.
  auto gather_gp = [&](int64_t s) -> u32x4 {
    uint64_t* base = slot_of(s) + static_cast<int64_t>(a.nslices) * 16 + col * 16 + grp * 4;
    const uint32_t tag = static_cast<uint32_t>(s + 1);
    for (int it = 0; a.spin >= 0; ++it) {  // spin < 0: no waiting at all (tests)
      uint64_t w[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) w[u] = get_word(base + u);
      int ok = 1;
#pragma unroll
      for (int u = 0; u < 4; ++u) ok &= static_cast<uint32_t>(w[u] >> 32) == tag;
      if (__all(ok))
        return u32x4{static_cast<uint32_t>(w[0]), static_cast<uint32_t>(w[1]), static_cast<uint32_t>(w[2]),
                     static_cast<uint32_t>(w[3])};
      if (it >= a.spin) break;
      __builtin_amdgcn_s_sleep(2);
    }
    float gp[8];
    k2_block(s, gather_gpre(s), gp, false);
    const u32x4 mine = pack8(gp);  // quad layout: token ktok, d group kqd
    const int src = col * 4 + grp;
    return u32x4{static_cast<uint32_t>(__shfl(static_cast<int>(mine[0]), src, kWave)),
                 static_cast<uint32_t>(__shfl(static_cast<int>(mine[1]), src, kWave)),
                 static_cast<uint32_t>(__shfl(static_cast<int>(mine[2]), src, kWave)),
                 static_cast<uint32_t>(__shfl(static_cast<int>(mine[3]), src, kWave))};
  };

  f32x4 dacc[8][2];
#pragma unroll
  for (int m = 0; m < 8; ++m) dacc[m][0] = dacc[m][1] = f32x4{0.f, 0.f, 0.f, 0.f};

  // dx step of block s (k1_bwd_mfma's compute with EPI): gv its grad_proj,
  // x and go3 from the stash, the other operands from f.
  auto dx_step = [&](const SplitFrag<GI>& f, int64_t s, const u32x4 gv) {
    const Blk b = block_at(s);
    const int rows = b.rows;
    const int st = static_cast<int>(s % kStash);
    u32x4 xv[4], g3v[4];
#pragma unroll
    for (int qq = 0; qq < 4; ++qq) {
      xv[qq] = stash[wave][st][qq][lane];
      g3v[qq] = stash[wave][st][4 + qq][lane];
    }
    float gf[8], pf[8];
    unpack8(gv, gf);
    unpack8(f.pv, pf);
    float dot = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) dot = __builtin_fmaf(gf[e], pf[e], dot);
    dot = rows_sum(dot);
    float scale[4];
#pragma unroll
    for (int qq = 0; qq < 4; ++qq) {
      const float d = __shfl(dot, 4 * grp + qq, kWave);
      scale[qq] = d * (f.inv[qq] * f.inv[qq]) / static_cast<float>(a.nC);
    }
    f32x4 acc[8];
    const bf16x8 av = as_bf16x8(gv);
#pragma unroll
    for (int m = 0; m < 8; ++m) acc[m] = mfma16(av, bfr[m], f32x4{0.f, 0.f, 0.f, 0.f});
    char* gxb = reinterpret_cast<char*>(a.gx + b.tbase * a.nC);
#pragma unroll
    for (int qq = 0; qq < 4; ++qq) {
      const int r = 4 * grp + qq;
      if (r < rows) {
        float xf[8], o[8], g3f[8];
        unpack8(xv[qq], xf);
        unpack8(g3v[qq], g3f);
#pragma unroll
        for (int m = 0; m < 8; ++m) {
          o[m] = __builtin_fmaf(f.inv[qq], acc[m][qq], -(scale[qq] * xf[m]));
          o[m] = bf16_to_f32(f32_to_bf16(f.hp[qq] * g3f[m])) + bf16_to_f32(f32_to_bf16(o[m]));
        }
        if constexpr (GI) {
          float gif[8];
          unpack8(f.gi[qq], gif);
#pragma unroll
          for (int m = 0; m < 8; ++m) o[m] = gif[m] + bf16_to_f32(f32_to_bf16(o[m]));
        }
        st_stream(reinterpret_cast<u32x4*>(gxb + (static_cast<uint32_t>(r) * row_bytes + kbytes)), pack8(o));
      }
    }
    // grad_W: D (16 k x 16 d) += x^T (A) G (B), G = bf16(go inv_rms) through LDS.
    uint32_t* tile = gtile[wave];
    *reinterpret_cast<u32x4*>(tile + col * 16 + grp * 4) = gv;
    const uint16_t* t16 = reinterpret_cast<const uint16_t*>(tile);
    uint32_t graw[2][4];
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int qq = 0; qq < 4; ++qq) graw[h][qq] = t16[(4 * grp + qq) * 32 + 16 * h + col];
    __builtin_amdgcn_sched_barrier(0);
    uint32_t bh[2][2];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      float gq[4];
#pragma unroll
      for (int qq = 0; qq < 4; ++qq) {
        const float g = __uint_as_float(graw[h][qq] << 16);
        gq[qq] = 4 * grp + qq < rows ? g * f.inv[qq] : 0.f;
      }
      bh[h][0] = pack_bf16x2(gq[0], gq[1]);
      bh[h][1] = pack_bf16x2(gq[2], gq[3]);
    }
#pragma unroll
    for (int m = 0; m < 8; ++m) {
      uint32_t e[4];
#pragma unroll
      for (int qq = 0; qq < 4; ++qq) {
        const uint32_t w = xv[qq][m >> 1];
        e[qq] = (m & 1) ? (w >> 16) : (w & 0xffffu);
      }
      const u32x2 avx = {e[0] | (e[1] << 16), e[2] | (e[3] << 16)};
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const u32x2 bv = {bh[h][0], bh[h][1]};
        dacc[m][h] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(bf16x4, avx),
                                                               __builtin_bit_cast(bf16x4, bv), dacc[m][h], 0, 0, 0);
      }
    }
    if (b.last) {
      // Run finished: its partial for this slice ([run][slice][m][h][r][lane]).
      float* dst = a.dw_partial + (b.run * a.nslices + slice) * (8 * 2 * 4 * kWave);
#pragma unroll
      for (int m = 0; m < 8; ++m)
#pragma unroll
        for (int h = 0; h < 2; ++h) {
#pragma unroll
          for (int r = 0; r < 4; ++r) dst[((m * 2 + h) * 4 + r) * kWave + lane] = dacc[m][h][r];
          dacc[m][h] = f32x4{0.f, 0.f, 0.f, 0.f};
        }
    }
  };

  // One step i: block i's first pass, K2 of block i - 1 if it is this
  // wave's, and block i - kLag's dx.  The waits come first (they also cover
  // cur, loaded in the previous step), then next's loads, then the compute.
  const int tw = slice;  // the wave's index in its team
  auto step = [&](SplitFrag<GI>& cur, SplitFrag<GI>& nxt, int64_t i) {
    const int64_t s3 = i - kLag, sd = i - 1;
    const bool do_k2 = sd >= 0 && sd < S && k2_wave_of(sd) == tw;
    const bool do_dx = s3 >= 0 && s3 < S;
    u32x4 gv = u32x4{0u, 0u, 0u, 0u};
    if (do_dx) gv = gather_gp(s3);
    float G = 0.f;
    if (do_k2) G = gather_gpre(sd);
    load(nxt, i + 1, i + 1 - kLag);
    __builtin_amdgcn_sched_barrier(0);
    if (i < S) {
      float e[4];
      slice_sums(cur.xv, cur.g3, e);
      const float mine = col == 0 ? e[0] : (col == 1 ? e[1] : (col == 2 ? e[2] : e[3]));
      if (col < 4) put_word(slot_of(i) + slice * 16 + 4 * grp + col, __float_as_uint(mine), static_cast<uint32_t>(i + 1));
      const int stn = static_cast<int>(i % kStash);
#pragma unroll
      for (int qq = 0; qq < 4; ++qq) {
        stash[wave][stn][qq][lane] = cur.xv[qq];
        stash[wave][stn][4 + qq][lane] = cur.g3[qq];
      }
    }
    if (do_k2) {
      float gp[8];
      k2_block(sd, G, gp, true);
      const u32x4 pk = pack8(gp);
      uint64_t* gpb = slot_of(sd) + static_cast<int64_t>(a.nslices) * 16 + ktok * 16 + kqd * 4;
      const uint32_t tag = static_cast<uint32_t>(sd + 1);
#pragma unroll
      for (int u = 0; u < 4; ++u) put_word(gpb + u, pk[u], tag);
    }
    if (do_dx) dx_step(cur, s3, gv);
  };

  const int64_t steps = S + kLag;
  SplitFrag<GI> fa, fb;
  if (S > 0) load(fa, 0, -kLag);
  for (int64_t i = 0; i < steps; i += 2) {
    step(fa, fb, i);
    if (i + 1 >= steps) break;
    step(fb, fa, i + 1);
  }
}

__global__ __launch_bounds__(256) void split_ring_zero(uint64_t* __restrict__ ring, int64_t n) {
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x; i < n; i += static_cast<int64_t>(gridDim.x) * 256)
    ring[i] = 0;
}

struct SplitShape {
  int nslices, ns, nteams, wpt;
  int64_t nruns, nblocks;
};

SplitShape split_shape(int64_t T, int64_t C) {
  SplitShape sh;
  const int64_t nC = 4 * C;
  sh.nslices = static_cast<int>(nC / 128);
  sh.ns = static_cast<int>(C / kSliceCols);
  const int fill = kSplitWaves / sh.nslices > 1 ? kSplitWaves / sh.nslices : 1;
  sh.nruns = k1_bwd_dw_runs(T, nC);
  sh.nteams = static_cast<int>(sh.nruns < fill ? sh.nruns : fill);
  sh.wpt = sh.nslices / 4;
  sh.nblocks = (T + 15) / 16;
  return sh;
}

// Polls per wait, FLASH_MHC_SPLIT_SPIN if set (read at each call): a negative
// value makes every wave compute every exchanged value itself (a test of the
// fallback; same results).
int split_spin() {
  const char* e = std::getenv("FLASH_MHC_SPLIT_SPIN");
  if (!e || !*e) return kSpinDefault;
  const long v = std::strtol(e, nullptr, 10);
  return v < 0 ? -1 : (v > (1 << 24) ? (1 << 24) : static_cast<int>(v));
}

}  // namespace

bool premap_split_ok(const void* x, const void* W, const void* proj, const void* inv_rms, const void* gx,
                     const void* go3, const void* gi, int64_t T, int64_t C) {
  if (T < kSplitMinT || C % kSliceCols != 0 || C / kSliceCols > kMaxSlices) return false;
  // The alignments and sizes of k1_bwd_mfma's pre-map path (its grad_proj operand is proj's alignment here).
  if (!k1_bwd_premap_fused(x, W, proj, proj, inv_rms, gx, go3, gi, C)) return false;
  // The slice order is K3's backward's for this shape.
  return k3_canon(C, k3_bwd_lanes8(static_cast<int>(C)));
}

int64_t premap_split_ring_bytes(int64_t T, int64_t C) {
  const SplitShape sh = split_shape(T, C);
  return int64_t{sh.nteams} * kRing * ring_words(sh.nslices) * 8;
}

int premap_bwd_split(const uint16_t* x, const uint16_t* W, const uint16_t* proj, const float* inv_rms,
                     const uint16_t* go3, const float* h_pre, const float* grad_h_post, const float* grad_H,
                     const uint16_t* grad_x_in, uint16_t* grad_x, uint16_t* grad_W, const K2Params& P,
                     void* grad_alpha_pre, void* grad_alpha_post, void* grad_alpha_res, void* grad_bias,
                     float* k2_partial, float* dw_partial, void* ring, int64_t T, int64_t C, hipStream_t s) {
  const SplitShape sh = split_shape(T, C);
  const int64_t words = int64_t{sh.nteams} * kRing * ring_words(sh.nslices);
  split_ring_zero<<<dim3(static_cast<unsigned>((words + 255) / 256 < 1024 ? (words + 255) / 256 : 1024)), 256, 0, s>>>(
      static_cast<uint64_t*>(ring), words);
  int st = launch_status();
  if (st != FMHC_OK) return st;
  SplitArgs a;
  a.x = x;
  a.W = W;
  a.proj = proj;
  a.inv_rms = inv_rms;
  a.go3 = go3;
  a.h_pre = h_pre;
  a.g_hpost = grad_h_post;
  a.g_H = grad_H;
  a.gi = grad_x_in;
  a.gx = grad_x;
  a.dw_partial = dw_partial;
  a.k2_partial = k2_partial;
  a.ring = static_cast<uint64_t*>(ring);
  a.P = P;
  a.T = T;
  a.nblocks = sh.nblocks;
  a.nruns = sh.nruns;
  a.nC = static_cast<int>(4 * C);
  a.C = static_cast<int>(C);
  a.nslices = sh.nslices;
  a.ns = sh.ns;
  a.nteams = sh.nteams;
  a.wpt = sh.wpt;
  a.spin = split_spin();
  const dim3 grid(static_cast<unsigned>(sh.nteams * sh.wpt));
  if (grad_x_in)
    premap_bwd_split<true><<<grid, 256, 0, s>>>(a);
  else
    premap_bwd_split<false><<<grid, 256, 0, s>>>(a);
  st = launch_status();
  if (st != FMHC_OK) return st;
  const K2ParamSums sums{k2_partial, sh.nblocks, grad_alpha_pre, grad_alpha_post, grad_alpha_res, grad_bias, P.bf16};
  return k1_dw_finish(dw_partial, grad_W, sh.nruns, sh.nslices, static_cast<int>(4 * C), sums, s);
}

}  // namespace fmhc
