// K1: fused RMSNorm over the flattened n*C stream + the D_out = 32 wide
// coefficient projection, and its backward.
//
// Kernels: k1_fwd_mfma (one pass over x per workgroup of 16-64 tokens, or, for
// few tokens, a column split whose partial sums k1_fwd_finish adds),
// k1_bwd_mfma (dx; with DW also grad_W's per-run partials, which
// k1_dw_reduce adds; with EPI / GI the pre-map backward's extra terms of
// grad_x in the same store), and element-wise kernels for shapes off the
// matrix-core path (nC % 8 != 0, unaligned pointers).
//
//   forward   inv_rms[t] = rsqrt(sum_k x[t,k]^2 / nC + 1e-6)
//             out[t,d]   = bf16(inv_rms[t] * sum_k x[t,k] * W[d,k])
//   backward  scale[t]    = (sum_d go[t,d] * proj_out[t,d]) * inv_rms[t]^2 / nC
//             grad_x[t,k] = bf16(inv_rms[t] * sum_d go[t,d] * W[d,k] - scale[t] * x[t,k])
//
// Follows src/flash_mhc/kernels.py:250-303 (forward: project first, then
// normalise, eps 1e-6) and :306-376 (dx from the stored bf16 projection, no
// second pass over x).  Both contractions run on the gfx950 matrix cores with
// v_mfma_f32_16x16x32_bf16.  Operand layout of that instruction, for lane l:
//   A (16 x 32): lane l holds A[l & 15][8 * (l >> 4) + e], e = 0..7
//   B (32 x 16): lane l holds B[8 * (l >> 4) + e][l & 15]
//   D (16 x 16): lane l, register q holds D[4 * (l >> 4) + q][l & 15]
// Because the contraction index may be permuted freely (as long as A and B
// agree), each lane's eight contraction values are eight consecutive bf16 in
// memory: one 16-byte load.
#include <type_traits>

#include "fmhc_common.h"
#include "k1_premap.h"
#include "k2_chain.h"

namespace fmhc {

namespace {

constexpr int kDout = 32;
constexpr float kEps = kRmsEps;

// Evidence build (build.py, variant "k1_valu"): the two K1 contractions run as
// fp32 FMAs on the VALU instead of on the matrix cores, with the same tiles,
// loads, LDS transposes and pipeline, so that the two can be timed against
// each other.  The product library is built with the matrix cores.
#ifndef FMHC_K1_VALU
#define FMHC_K1_VALU 0
#endif
constexpr bool kValu = FMHC_K1_VALU != 0;
// Evidence build switch: the pre-map's one-kernel forward (TILE) loads x with
// the nontemporal hint like the plain forward, so that K3's re-read of the
// tile cannot find it in the memory-side cache.  The product loads it with
// ordinary loads.
#ifndef FMHC_PREMAP_TILE_NT
#define FMHC_PREMAP_TILE_NT 0
#endif
constexpr bool kTileNt = FMHC_PREMAP_TILE_NT != 0;

__device__ __forceinline__ bf16x8 as_bf16x8(u32x4 v) { return __builtin_bit_cast(bf16x8, v); }
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ f32x4 mfma16(bf16x8 a, bf16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// ---------------------------------------------------------------------------
// K1 forward, matrix-core path (nC % 8 == 0, 16-byte aligned x / W / out).
//
// A workgroup owns 16*R consecutive tokens and SPLIT waves.  The nC axis is
// cut into 64-wide chunks; wave w accumulates chunks w, w + SPLIT, ... for all
// of the workgroup's tokens (so the waves of a workgroup read adjacent
// 128-byte pieces of the same x rows), then the SPLIT partial results are
// summed in LDS in a fixed order.  Per chunk and token block the MFMA is
//   D (32 d x 16 tokens) += W[:, chunk] (A, two 16-row halves) * x[tokens, chunk]^T (B)
// so D's layout gives every lane 4 consecutive d of one token.  The sum of
// squares also runs on the matrix cores: the same x registers are both A and
// B of a third MFMA, G (16 x 16) += x x^T, whose diagonal is sum_k x[t,k]^2
// in fp32 (the bf16 products are exact).
//
// The MFMA operand layout puts 16 tokens x 64 bytes in one register, i.e.
// half of each 128-byte line per load instruction.  Loading that layout
// directly from HBM is 3% slower than loading whole lines (8 tokens x 128
// bytes per instruction) and moving them into the MFMA layout through a
// wave-private LDS tile (16R tokens x 128 bytes).
// The pre-map tile epilogue's shared memory (TILE below).
template <int R>
struct TileSmem {
  K2Smem k2;
  float proj[16 * R][kDk];
  f32x4 hpre[16 * R];
};

template <int R>
struct FwdFrag {
  u32x4 wa[2], wb[2];  // W rows 0-15 / 16-31, two 32-wide k steps
  u32x4 xv[2][R];      // x of the R token blocks, two k steps
};

// K3 over one 16-token block of the tile by one wave (rows of C, a multiple
// of 1024: each lane takes groups lane, lane + 64, ... of every row), with
// k3_token's loads, arithmetic and stores.  Pieces of a token (two groups of
// the four streams, eight loads) follow each other token by token, and each
// piece's loads go out before the previous piece's stores: the compiler does
// not move a load above an earlier store, so k3_token called token by token
// waits for its loads once per group.  The last trip reloads the last piece
// (clamped, as every prefetch here) instead of branching.  The tile kernel
// takes it for rows of 4096 and 8192: the pre-map forward at C = 4096, each
// launch after a cache flush, T = 262144 3411 -> 3258 us, 131072 1684 ->
// 1600, 65536 813 -> 778, 32768 393 -> 381, 16384 186 either way (inside
// the eager training stack, 3136 against 3140 us at T = 262144).  With
// fewer pieces per token it lost (C = 2048, T = 65536: 343 -> 352 us;
// C = 1024, T = 16384: 51.1 -> 52.7 us).
__device__ __forceinline__ void k3_block_pipelined(const uint16_t* __restrict__ x, const f32x4* hpre,
                                                   uint16_t* __restrict__ out, int64_t tb, int64_t T, int C,
                                                   int lane) {
  const int np = C / 1024;  // pieces per token
  const int nu = 16 * np;   // pieces of the block, an even count
  auto load = [&](u32x4 (&v)[8], int u) __attribute__((always_inline)) {
    const int tt = u / np, p = u - tt * np;
    const int64_t t = tb + tt < T ? tb + tt : T - 1;  // rows past T re-read the last one
    const uint16_t* row = x + t * 4 * C;
#pragma unroll
    for (int s = 0; s < 2; ++s)
#pragma unroll
      for (int j = 0; j < 4; ++j) v[4 * s + j] = Lanes<8>::raw(row + j * C, lane + 128 * p + 64 * s);
  };
  auto mix_store = [&](const u32x4 (&v)[8], int u) __attribute__((always_inline)) {
    const int tt = u / np, p = u - tt * np;
    const int64_t t = tb + tt;
    if (t >= T) return;
    const f32x4 hv = hpre[tt];
    const float h[4] = {hv[0], hv[1], hv[2], hv[3]};
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      float a[8], b[8], c[8], d[8], o[8];
      Lanes<8>::unpack(v[4 * s], a);
      Lanes<8>::unpack(v[4 * s + 1], b);
      Lanes<8>::unpack(v[4 * s + 2], c);
      Lanes<8>::unpack(v[4 * s + 3], d);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        float acc = h[0] * a[e];
        acc = __builtin_fmaf(h[1], b[e], acc);
        acc = __builtin_fmaf(h[2], c[e], acc);
        o[e] = __builtin_fmaf(h[3], d[e], acc);
      }
      Lanes<8>::store(out + t * C, lane + 128 * p + 64 * s, o);
    }
  };
  u32x4 va[8], vb[8];
  load(va, 0);
  for (int u = 0; u < nu; u += 2) {
    load(vb, u + 1);
    __builtin_amdgcn_sched_barrier(0);
    mix_store(va, u);
    load(va, u + 2 < nu ? u + 2 : nu - 1);
    __builtin_amdgcn_sched_barrier(0);
    mix_store(vb, u + 1);
  }
}

// SPLITK (few tokens): blockIdx.y selects a range of cps chunks, and the
// workgroup writes its fp32 partial sums (32 projections + sum of squares per
// token) to part[t][33][S4] (S4 = gridDim.y rounded up to 4) instead of the
// outputs; k1_fwd_finish adds the gridDim.y partials in order.
// TILE (the pre-map region without the column split, premap.hip): after a
// tile's projections, the same workgroup runs K2 on the tile's tokens (four
// lanes per token, k2_token4) and then K3 (each wave its own blocks; with
// fewer blocks than waves, all waves over the tile), mixing the tile's
// streams into the layer input while L2 and the memory-side cache may still
// hold the rows it just read (its x loads are ordinary loads, which allocate
// there).  Same values as K1 -> K2 -> K3 launched separately.
template <int R, int SPLIT, bool SPLITK, bool TILE = false>
__global__ __launch_bounds__(kWave * SPLIT) void k1_fwd_mfma(const uint16_t* __restrict__ x,
                                                             const uint16_t* __restrict__ W,
                                                             uint16_t* __restrict__ out,
                                                             float* __restrict__ inv_rms,
                                                             float* __restrict__ part,
                                                             int64_t T, int nC, int cps,
                                                             const PremapTile pt = PremapTile{}) {
  static_assert(!TILE || !SPLITK, "the tile epilogue runs on the one-pass kernel");
  __shared__ float red_acc[SPLIT][R][8][kWave];
  __shared__ float red_ss[SPLIT][R][16];
  __shared__ u32x4 xs[SPLIT][16 * R * 8];  // per wave: 16R tokens x 8 swizzled 16-byte slots
  __shared__ u32x4 wts[kValu ? SPLIT : 1][kValu ? 32 * 8 : 1];  // VALU build: the W chunk, 32 rows x 8 slots
  // TILE: K2's parameters, the tile's stored projections and its h_pre.
  __shared__ std::conditional_t<TILE, TileSmem<R>, char> tile_sm;
  if constexpr (TILE) {
    zero_words(pt.z);
    stage_params<kWave * SPLIT>(pt.P, tile_sm.k2);
  }

  const int lane = threadIdx.x & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) >> 6);
  const int row = lane & 15;
  const int grp = lane >> 4;
  const int64_t t0 = static_cast<int64_t>(blockIdx.x) * (16 * R);

  // Full-line loads: instruction j (0 .. 2R-1) covers tokens 8j .. 8j+7 of the
  // workgroup, lane l the 16-byte slot l & 7 of token 8j + (l >> 3).  Tail
  // rows re-read the last token; their results are not stored.
  const uint16_t* xw = x + t0 * nC;
  const int64_t rem = T - 1 - t0;
  const int tmax = rem < 16 * R ? static_cast<int>(rem) : 16 * R - 1;
  uint32_t xoff[2 * R];
#pragma unroll
  for (int j = 0; j < 2 * R; ++j) {
    const int tl = 8 * j + (lane >> 3);
    xoff[j] = static_cast<uint32_t>(tl < tmax ? tl : tmax) * static_cast<uint32_t>(nC) + 8u * (lane & 7);
  }
  // LDS slots are swizzled (slot ^ ((token >> 1) & 7)) so that the row writes
  // and the MFMA-layout reads are free of bank conflicts.
  u32x4* xl = xs[wave];
  const int wr0 = (lane >> 3) * 8 + ((lane & 7) ^ (lane >> 4));
  const int wr1 = (lane >> 3) * 8 + ((lane & 7) ^ (4 + (lane >> 4)));
  const int rd0 = row * 8 + (grp ^ ((row >> 1) & 7));
  const int rd1 = row * 8 + ((4 + grp) ^ ((row >> 1) & 7));
  const uint16_t* w0 = W + static_cast<int64_t>(row) * nC + 8 * grp;
  const uint16_t* w1 = W + static_cast<int64_t>(16 + row) * nC + 8 * grp;

  f32x4 acc[2][R];
  f32x4 gram[R];
#pragma unroll
  for (int r = 0; r < R; ++r) {
    acc[0][r] = f32x4{0.f, 0.f, 0.f, 0.f};
    acc[1][r] = f32x4{0.f, 0.f, 0.f, 0.f};
    gram[r] = f32x4{0.f, 0.f, 0.f, 0.f};
  }

  // Full 64-wide chunks.  Wave w takes the chunks at positions w, w + SPLIT,
  // ... of a per-workgroup rotation of the chunk order (rotating spreads the
  // concurrent reads of all workgroups over the DRAM channels instead of every
  // workgroup hitting the same column of its 8 KiB-strided rows), and keeps
  // three chunks in flight: the next two chunks' fragments are loaded while
  // the MFMAs of the current one run.  x is read once per launch, so its loads carry the
  // nontemporal hint (8-10% faster than ordinary loads).  With SPLITK (few
  // tokens) they do not: the pre-map's few-token kernel reads the same x
  // again right after, from the caches.  With SPLITK the workgroup's chunks
  // are cbeg .. cbeg + nfull - 1 (no rotation: the workgroups of one token
  // block already cover different columns), and only the last split takes the
  // ragged chunk.
  const int nall = nC >> 6;
  const int cbeg = SPLITK ? static_cast<int>(blockIdx.y) * cps : 0;
  const int nfull = SPLITK ? (cps < nall - cbeg ? cps : nall - cbeg) : nall;
  const bool last_split = !SPLITK || blockIdx.y + 1 == gridDim.y;
  const int rot = !SPLITK && nfull > 0 ? static_cast<int>(blockIdx.x % static_cast<unsigned>(nfull)) : 0;
  FwdFrag<R> f0, f1;
  auto chunk_at = [&](int p) __attribute__((always_inline)) { return cbeg + (p + rot < nfull ? p + rot : p + rot - nfull); };
  auto load = [&](FwdFrag<R>& f, int p) __attribute__((always_inline)) {
    const int k = chunk_at(p) * 64;
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      f.wa[s] = *reinterpret_cast<const u32x4*>(w0 + k + 32 * s);
      f.wb[s] = *reinterpret_cast<const u32x4*>(w1 + k + 32 * s);
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const u32x4* px = reinterpret_cast<const u32x4*>(xw + xoff[s * R + r] + k);
        if constexpr (!SPLITK && (!TILE || kTileNt))
          f.xv[s][r] = __builtin_nontemporal_load(px);
        else
          f.xv[s][r] = *px;
      }
    }
  };
  // Token rows -> MFMA layout (lane: token row, 8 consecutive k) through the
  // wave's LDS tile.  Same-wave LDS operations complete in order, so the
  // next chunk's writes cannot overtake these reads.
  auto transpose = [&](FwdFrag<R>& f) __attribute__((always_inline)) {
#pragma unroll
    for (int j = 0; j < 2 * R; ++j) xl[64 * j + ((j & 1) ? wr1 : wr0)] = f.xv[j / R][j % R];
#pragma unroll
    for (int s = 0; s < 2; ++s)
#pragma unroll
      for (int r = 0; r < R; ++r) f.xv[s][r] = xl[128 * r + (s ? rd1 : rd0)];
  };
  auto compute_mfma = [&](const FwdFrag<R>& f) __attribute__((always_inline)) {
#pragma unroll
    for (int s = 0; s < 2; ++s) {
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const bf16x8 xb = as_bf16x8(f.xv[s][r]);
        acc[0][r] = mfma16(as_bf16x8(f.wa[s]), xb, acc[0][r]);
        acc[1][r] = mfma16(as_bf16x8(f.wb[s]), xb, acc[1][r]);
        gram[r] = mfma16(xb, xb, gram[r]);
      }
    }
  };
  // VALU build: lane (grp, row) accumulates, for token `row` of each block,
  // the outputs d = 4 grp + q and 16 + 4 grp + q (the matrix-core D layout)
  // over the chunk's 64 k, reading x from the wave's transpose tile and W
  // from a wave-private copy of the chunk; the sum of squares goes into the
  // diagonal slot of `gram` that the epilogue reads.
  float ssq[kValu ? R : 1];
#pragma unroll
  for (int r = 0; r < (kValu ? R : 1); ++r) ssq[r] = 0.f;
  auto compute_valu = [&](const FwdFrag<R>& f, bool mfma_layout) __attribute__((always_inline)) {
    u32x4* wl = wts[kValu ? wave : 0];
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      wl[row * 8 + 4 * s + grp] = f.wa[s];
      wl[(16 + row) * 8 + 4 * s + grp] = f.wb[s];
      if (mfma_layout) {  // x is in registers in the matrix-core layout: put it where the tile would hold it
#pragma unroll
        for (int r = 0; r < R; ++r) xl[128 * r + (s ? rd1 : rd0)] = f.xv[s][r];
      }
    }
    const int key = (row >> 1) & 7;
#pragma unroll 1
    for (int p = 0; p < 8; ++p) {
      float xv[R][8];
#pragma unroll
      for (int r = 0; r < R; ++r) {
        unpack8(xl[128 * r + row * 8 + (p ^ key)], xv[r]);
#pragma unroll
        for (int e = 0; e < 8; ++e) ssq[r] = __builtin_fmaf(xv[r][e], xv[r][e], ssq[r]);
      }
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        float w[8];
        unpack8(wl[(i < 4 ? 4 * grp + i : 12 + 4 * grp + i) * 8 + p], w);
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
          for (int e = 0; e < 8; ++e) acc[i >> 2][r][i & 3] = __builtin_fmaf(w[e], xv[r][e], acc[i >> 2][r][i & 3]);
      }
    }
  };
  auto compute = [&](const FwdFrag<R>& f, bool mfma_layout = false) __attribute__((always_inline)) {
    if constexpr (kValu)
      compute_valu(f, mfma_layout);
    else
      compute_mfma(f);
  };
  // n chunks for this wave (positions wave, wave + SPLIT, ...), three in
  // flight: f0, f1, f2 in rotation, each trip loading two chunks ahead of the
  // one it computes.  Every load of the steady loop is below n, so its wait
  // counts stay exact and no chunk is read twice (a clamped re-read of the
  // last chunk cost 3.5% more traffic under the nontemporal hint); the tail
  // finishes the last one to four chunks.
  const int n = nfull > wave ? (nfull - wave + SPLIT - 1) / SPLIT : 0;
  if (n > 0) {
    FwdFrag<R> f2;
    load(f0, wave);
    if (n > 1) load(f1, wave + SPLIT);
    int i = 0;
    for (; i + 4 < n; i += 3) {
      load(f2, wave + SPLIT * (i + 2));
      __builtin_amdgcn_sched_barrier(0);
      transpose(f0);
      compute(f0);
      load(f0, wave + SPLIT * (i + 3));
      __builtin_amdgcn_sched_barrier(0);
      transpose(f1);
      compute(f1);
      load(f1, wave + SPLIT * (i + 4));
      __builtin_amdgcn_sched_barrier(0);
      transpose(f2);
      compute(f2);
    }
    const int left = n - i;  // 1 .. 4: chunk i in f0, chunk i + 1 in f1
    if (left >= 3) load(f2, wave + SPLIT * (i + 2));
    transpose(f0);
    compute(f0);
    if (left >= 4) load(f0, wave + SPLIT * (i + 3));
    if (left >= 2) {
      transpose(f1);
      compute(f1);
    }
    if (left >= 3) {
      transpose(f2);
      compute(f2);
    }
    if (left >= 4) {
      transpose(f0);
      compute(f0);
    }
  }
  // Ragged last chunk (nC % 64 != 0): 16-byte pieces past nC contribute zero.
  if ((nC & 63) != 0 && last_split && wave == nfull % SPLIT) {
    const int k = nall * 64;
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      const bool ok = k + 32 * s + 8 * grp < nC;
      f0.wa[s] = f0.wb[s] = u32x4{0u, 0u, 0u, 0u};
#pragma unroll
      for (int r = 0; r < R; ++r) f0.xv[s][r] = u32x4{0u, 0u, 0u, 0u};
      if (ok) {
        f0.wa[s] = *reinterpret_cast<const u32x4*>(w0 + k + 32 * s);
        f0.wb[s] = *reinterpret_cast<const u32x4*>(w1 + k + 32 * s);
#pragma unroll
        for (int r = 0; r < R; ++r) {
          int64_t t = t0 + 16 * r + row;
          t = t < T ? t : T - 1;
          f0.xv[s][r] = *reinterpret_cast<const u32x4*>(x + t * nC + 8 * grp + k + 32 * s);
        }
      }
    }
    compute(f0, true);
  }

  if constexpr (kValu) {
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const int qd = row & 3;
      gram[r] = f32x4{qd == 0 ? ssq[r] : 0.f, qd == 1 ? ssq[r] : 0.f, qd == 2 ? ssq[r] : 0.f, qd == 3 ? ssq[r] : 0.f};
    }
  }
  // Diagonal G[row][row] sits in lane row + 16 * (row >> 2), register row & 3.
  const int q_diag = row & 3;
  const bool holds_diag = grp == (row >> 2);
#pragma unroll
  for (int r = 0; r < R; ++r) {
    const f32x4 gr = gram[r];
    const float diag = q_diag == 0 ? gr[0] : q_diag == 1 ? gr[1] : q_diag == 2 ? gr[2] : gr[3];
    if (holds_diag) red_ss[wave][r][row] = diag;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      red_acc[wave][r][q][lane] = acc[0][r][q];
      red_acc[wave][r][4 + q][lane] = acc[1][r][q];
    }
  }
  __syncthreads();

  for (int r = wave; r < R; r += SPLIT) {
    float a[8];
    float s2 = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) a[i] = 0.f;
#pragma unroll
    for (int w = 0; w < SPLIT; ++w) {
      s2 += red_ss[w][r][row];
#pragma unroll
      for (int i = 0; i < 8; ++i) a[i] += red_acc[w][r][i][lane];
    }
    const int64_t t = t0 + 16 * r + row;
    if constexpr (SPLITK) {
      if (t < T) {
        const int s4 = (static_cast<int>(gridDim.y) + 3) & ~3;
        float* pr = part + t * (kDout + 1) * s4 + blockIdx.y;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          pr[(4 * grp + q) * s4] = a[q];
          pr[(16 + 4 * grp + q) * s4] = a[4 + q];
        }
        if (grp == 0) pr[kDout * s4] = s2;
      }
    } else {
      const float inv = rsqrtf(s2 / static_cast<float>(nC) + kEps);
      if (t < T) {
        uint16_t* orow = out + t * kDout + 4 * grp;
        u32x2 lo2 = {pack_bf16x2(a[0] * inv, a[1] * inv), pack_bf16x2(a[2] * inv, a[3] * inv)};
        u32x2 hi2 = {pack_bf16x2(a[4] * inv, a[5] * inv), pack_bf16x2(a[6] * inv, a[7] * inv)};
        st_stream(reinterpret_cast<u32x2*>(orow), lo2);
        st_stream(reinterpret_cast<u32x2*>(orow + 16), hi2);
        if (grp == 0) inv_rms[t] = inv;
      }
      if constexpr (TILE) {
        // The stored (bf16) projections of token row, for the K2 lanes below.
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          tile_sm.proj[16 * r + row][4 * grp + q] = bf16_to_f32(f32_to_bf16(a[q] * inv));
          tile_sm.proj[16 * r + row][16 + 4 * grp + q] = bf16_to_f32(f32_to_bf16(a[4 + q] * inv));
        }
      }
    }
  }
  if constexpr (TILE) {
    // Wave w owns blocks w, w + SPLIT, ... (the blocks whose projections it
    // stored above) and runs K2 for their tokens, four lanes per token
    // (k2_token4; one lane per token measured 4-6 us slower per launch).
    // With at least a block per wave it also runs K3 over its blocks:
    // same-wave LDS operations are ordered, so those projections and the h_pre
    // written below need no barrier.  With fewer blocks than waves, every wave
    // takes a share of the tile's tokens in K3, after a barrier.
    for (int r = wave; r < R; r += SPLIT) {
    {
      const int i = lane >> 2, qd = lane & 3;
      const int64_t t = t0 + 16 * r + i;
      float hp, hq, hp_all[kN];
      f32x4 hrow;
      k2_token4(tile_sm.proj[16 * r + i], tile_sm.k2, qd, hp, hq, hrow, hp_all);
      if (t < T) {
        pt.h_pre[t * kN + qd] = hp;
        pt.h_post[t * kN + qd] = hq;
        reinterpret_cast<f32x4*>(pt.H)[t * kN + qd] = hrow;
      }
      if (qd == 0) tile_sm.hpre[16 * r + i] = f32x4{hp_all[0], hp_all[1], hp_all[2], hp_all[3]};
    }
    if (R >= SPLIT && pt.layer_input) {
      if (pt.C % 4096 == 0) {
        k3_block_pipelined(x, tile_sm.hpre + 16 * r, pt.layer_input, t0 + 16 * r, T, pt.C, lane);
      } else {
        for (int tt = 0; tt < 16; ++tt) {
          const int64_t t = t0 + 16 * r + tt;
          if (t >= T) break;
          const f32x4 hv = tile_sm.hpre[16 * r + tt];
          const float h[4] = {hv[0], hv[1], hv[2], hv[3]};
          k3_token<8>(x + t * 4 * pt.C, h, pt.layer_input + t * pt.C, lane, kWave, pt.C);
        }
      }
    }
    }
    if (R < SPLIT && pt.layer_input) {  // the same branch in every thread
      __syncthreads();
      for (int tt = wave; tt < 16 * R; tt += SPLIT) {
        const int64_t t = t0 + tt;
        if (t >= T) break;
        const f32x4 hv = tile_sm.hpre[tt];
        const float h[4] = {hv[0], hv[1], hv[2], hv[3]};
        k3_token<8>(x + t * 4 * pt.C, h, pt.layer_input + t * pt.C, lane, kWave, pt.C);
      }
    }
  }
}

// Second stage of the split K1 forward: one wave per token; lane v < 33 adds
// the S partials of value v (32 projections, then the sum of squares) in split
// order, so the result does not depend on scheduling.
__global__ __launch_bounds__(256) void k1_fwd_finish(const float* __restrict__ part,
                                                     uint16_t* __restrict__ out,
                                                     float* __restrict__ inv_rms, int64_t T, int nC,
                                                     int S) {
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t t = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (t >= T) return;
  const int s4 = (S + 3) & ~3;
  float v = 0.f;
  if (lane <= kDout) {
    const f32x4* p = reinterpret_cast<const f32x4*>(part + (t * (kDout + 1) + lane) * s4);
#pragma unroll 4
    for (int i = 0; i < s4 / 4; ++i) {
      const f32x4 q = p[i];
      v += q[0];  // 4 i < S always
      if (4 * i + 1 < S) v += q[1];
      if (4 * i + 2 < S) v += q[2];
      if (4 * i + 3 < S) v += q[3];
    }
  }
  const float inv = rsqrtf(__shfl(v, kDout, kWave) / static_cast<float>(nC) + kEps);
  if (lane < kDout) out[t * kDout + lane] = f32_to_bf16(v * inv);
  if (lane == kDout) inv_rms[t] = inv;
}

// ---------------------------------------------------------------------------
// K1 backward dx, matrix-core path (nC % 8 == 0, 16-byte aligned x / W / go /
// proj_out / inv_rms / grad_x).
//
// Each wave owns a 128-wide slice of the nC axis and walks one run of blocks
// of 16 tokens (strided by the number of runs, see below; the host picks the
// run count, k1_bwd_nruns).  Per token block, eight MFMAs (tiles m = 0..7) compute
//   D_m (16 tokens x 16 columns) = go[tokens, 0:32] (A) * W[0:32, cols_m] (B)
// i.e. the whole D_out = 32 contraction in one instruction per tile, where
// column j of tile m stands for k = k_slice + 8 * j + m.  With D's layout
// (lane l, register q holds D[4 * (l >> 4) + q][l & 15]) every lane then owns
// 8 consecutive k (tiles m = 0..7) of 4 tokens (q = 0..3): x is read and
// grad_x written as one 16-byte vector per lane and token, and each memory
// instruction covers 4 token rows x 256 contiguous bytes (whole cache lines).
// The B tiles depend only on the slice, so each wave builds them once: eight
// 16-byte loads of W rows and an 8 x 8 bf16 transpose in registers.
template <bool EPI, bool GI>
struct BwdFrag {
  u32x4 gv, pv;   // go / proj_out row of token tbase + col, d = 8 * grp .. + 8
  float inv[4];   // inv_rms of tokens tbase + 4 * grp + q
  u32x4 xv[4];    // x of those tokens, k = kl .. kl + 8
  u32x4 g3[EPI ? 4 : 1];  // EPI: the K3 output gradient of those tokens at the lane's c
  float hp[EPI ? 4 : 1];  // EPI: their h_pre of the lane's stream j
  u32x4 gi[GI ? 4 : 1];   // GI: x's incoming gradient at the lane's 8 k
};

// With DW = true the same pass also accumulates the weight gradient
//   grad_W[d, k] = sum_t bf16(go[t,d] * inv_rms[t]) * x[t,k]
// (ops.py:683-684 of the reference computes it as a separate matmul that reads
// x a second time).  The lane's x registers for one token block (4 tokens x 8
// consecutive k) are exactly the A operand of v_mfma_f32_16x16x16_bf16 with
// the contraction over tokens, so tile m of dW^T is
//   D (16 k x 16 d) += x[tokens, k_slice + 8 * i + m]^T (A) * G[tokens, 16 h + j] (B)
// with G = bf16(go * inv_rms).  G reaches the B layout through a 1 KiB
// wave-private LDS tile.  Each wave writes its fp32 partial dW for its slice;
// k1_dw_reduce sums the partials of all runs in a fixed order.
//
// With EPI = true (the pre-map backward) the store also adds the K3 term of
// x's gradient, grad_x = bf16(bf16(h_pre[t, j] go3[t, c]) + bf16(dx)), k = j C + c:
// the bf16 sum autograd forms when K3 and K1 are separate ops.  The B tiles
// then live in LDS so that the extra operands keep two waves per SIMD.
//
// With GI = true (EPI only) the store also adds an incoming gradient of x (the
// post-res op's H_merged^T grad_out): grad_x = bf16(gi + bf16(pre-map term)),
// the value autograd's accumulation of x's gradients gives.  The extra
// operand takes the kernel to one wave per SIMD; it is still bound by HBM
// (measured: +80 us at T=65536, C=1024 for the 512 MiB it reads, against
// 260 us for the separate accumulation pass it replaces).
template <bool DW, bool FULLK, bool EPI, bool GI, int NBUF>
__global__ __launch_bounds__(256) void k1_bwd_mfma(const uint16_t* __restrict__ x,
                                                   const uint16_t* __restrict__ W,
                                                   const uint16_t* __restrict__ go,
                                                   const uint16_t* __restrict__ proj,
                                                   const float* __restrict__ inv_rms,
                                                   uint16_t* __restrict__ gx,
                                                   float* __restrict__ dw_partial,
                                                   const uint16_t* __restrict__ go3,
                                                   const float* __restrict__ h_pre,
                                                   const uint16_t* __restrict__ gi,
                                                   int64_t T, int nC, int nslices, int64_t nruns, int C) {
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) >> 6);
  const int col = lane & 15;  // A row (token) for the loads of go, B/D column
  const int grp = lane >> 4;  // 8-wide d group of A/B; 4-token group of D
  // Wave -> (k slice, run): the four waves of a workgroup take four
  // consecutive slices (1 KiB of each x row) of the same run.  (Giving them
  // one slice and four runs, to sum their grad_W partials in LDS, measured
  // 8% slower.)
  // Workgroups are dispatched round-robin over the 8 XCDs.  Within each
  // group of 64, workgroup b takes the logical id 8 (b % 8) + (b % 64) / 8:
  // the workgroups of one run, which read the same go / proj rows, share one
  // XCD's L2 (8% less HBM traffic), and a group still covers 8 neighbouring
  // runs at a time.
  const unsigned bid = blockIdx.x;
  const unsigned full = gridDim.x & ~63u;
  const unsigned lid = bid < full ? (bid & ~63u) + 8u * (bid % 8u) + (bid % 64u) / 8u : bid;
  const int64_t wid = static_cast<int64_t>(lid) * 4 + wave;
  const int slice = static_cast<int>(wid % nslices);
  const int64_t run = wid / nslices;
  // Token blocks run, run + nruns, run + 2 * nruns, ...: the waves resident at
  // one time work on neighbouring blocks, so the concurrent reads and writes
  // cover contiguous memory instead of addresses a power-of-two apart.
  const int64_t nblocks = (T + 15) / 16;  // nruns <= nblocks
  if (run >= nruns) return;
  const int kl = slice * 128 + 8 * col;  // this lane's 8 consecutive k
  const bool kok = FULLK || kl < nC;     // nC % 8 == 0: all 8 valid or none
  // Addresses are a wave-uniform block base plus a 32-bit per-lane byte offset
  // (16 rows of x span 32 * nC bytes < 2^32, checked by the caller).
  const uint32_t row_bytes = 2u * static_cast<uint32_t>(nC);
  const uint32_t kbytes = 2u * static_cast<uint32_t>(kl);

  __shared__ uint32_t gtile[DW ? 4 : 1][16 * 16];  // wave-private 16 tokens x 32 d bf16
  __shared__ u32x4 btile[EPI ? 4 : 1][EPI ? 8 : 1][EPI ? kWave : 1];  // EPI: wave-private B tiles
  // VALU build: W[d][kl .. kl + 8) for d = 0..31 and the lane columns, and the token block's go rows.
  __shared__ u32x4 wvl[kValu ? 4 : 1][kValu ? 32 * 16 : 1];
  __shared__ u32x4 gvl[kValu ? 4 : 1][kValu ? 16 * 4 : 1];
  // EPI: the lane's stream j and position c (C % 8 == 0: k .. k + 7 stay in one stream).
  const int sj = EPI ? kl / C : 0;
  const uint32_t c3bytes = EPI ? 2u * static_cast<uint32_t>(kl - sj * C) : 0u;
  f32x4 dacc[DW ? 8 : 1][2];
#pragma unroll
  for (int m = 0; m < (DW ? 8 : 1); ++m) dacc[m][0] = dacc[m][1] = f32x4{0.f, 0.f, 0.f, 0.f};

  // B tiles: bfr[m] holds W[8 * grp + e][kl + m], e = 0..7.
  bf16x8 bfr[8];
  {
    u32x4 rows[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      rows[e] = u32x4{0u, 0u, 0u, 0u};
      if (kok) rows[e] = *reinterpret_cast<const u32x4*>(W + static_cast<int64_t>(8 * grp + e) * nC + kl);
    }
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
      if constexpr (EPI) btile[wave][m][lane] = v;
    }
    if constexpr (kValu) {
#pragma unroll
      for (int e = 0; e < 8; ++e) wvl[wave][(8 * grp + e) * 16 + col] = rows[e];
    }
  }
  // Same-wave LDS writes and reads are ordered: the tiles need no barrier.
  auto btile_at = [&](int m) -> bf16x8 {
    if constexpr (EPI)
      return as_bf16x8(btile[wave][m][lane]);
    else
      return bfr[m];
  };

  // Token blocks of this wave, NBUF fragments in rotation: the next blocks'
  // go / proj_out / inv_rms / x (and the pre-map operands) are in flight
  // while the current block computes.
  const int nb = static_cast<int>((nblocks - run + nruns - 1) / nruns);
  auto pos = [&](int i) { return i < nb ? i : nb - 1; };
  auto block_base = [&](int tb) { return (run + static_cast<int64_t>(tb) * nruns) * 16; };
  // Valid rows of the block starting at tbase (16 except in the last block).
  auto block_rows = [&](int64_t tbase) { return static_cast<int>(T - tbase < 16 ? T - tbase : 16); };
  auto load = [&](BwdFrag<EPI, GI>& f, int tb) {
    const int64_t tbase = block_base(tb);
    const int last = block_rows(tbase) - 1;  // rows past the end re-read the last one
    const int rg = col < last ? col : last;
    const uint32_t goff = static_cast<uint32_t>(rg) * (2u * kDout) + 16u * static_cast<uint32_t>(grp);
    f.gv = *reinterpret_cast<const u32x4*>(reinterpret_cast<const char*>(go + tbase * kDout) + goff);
    f.pv = *reinterpret_cast<const u32x4*>(reinterpret_cast<const char*>(proj + tbase * kDout) + goff);
    const char* ib = reinterpret_cast<const char*>(inv_rms + tbase);
    const char* xb = reinterpret_cast<const char*>(x + tbase * nC);
    // The lane's four tokens are consecutive: a full block reads their
    // inv_rms with one 16-byte load (the block-uniform branch below).
    if (last == 15) {
      const f32x4 iv = *reinterpret_cast<const f32x4*>(ib + 16u * static_cast<uint32_t>(grp));
#pragma unroll
      for (int q = 0; q < 4; ++q) f.inv[q] = iv[q];
    }
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const int r0 = 4 * grp + q;
      const uint32_t r = static_cast<uint32_t>(r0 < last ? r0 : last);
      if (last != 15) f.inv[q] = *reinterpret_cast<const float*>(ib + 4u * r);
      f.xv[q] = u32x4{0u, 0u, 0u, 0u};
      if (kok) f.xv[q] = ld_stream(reinterpret_cast<const u32x4*>(xb + (r * row_bytes + kbytes)));
      if constexpr (EPI) {
        f.hp[q] = 0.f;
        f.g3[q] = u32x4{0u, 0u, 0u, 0u};
        if (kok) {  // lanes past nC have no stream
          const char* g3b = reinterpret_cast<const char*>(go3 + tbase * C);
          f.hp[q] = *reinterpret_cast<const float*>(reinterpret_cast<const char*>(h_pre + tbase * 4) +
                                                    16u * r + 4u * static_cast<uint32_t>(sj));
          // Ordinary load: the four streams' slices read the same go3 row, and
          // the nontemporal hint kept it out of L2 between them (1.14x FETCH).
          f.g3[q] = *reinterpret_cast<const u32x4*>(g3b + (r * 2u * static_cast<uint32_t>(C) + c3bytes));
        }
      }
      if constexpr (GI) {
        f.gi[q] = u32x4{0u, 0u, 0u, 0u};
        if (kok)
          f.gi[q] = ld_stream(reinterpret_cast<const u32x4*>(reinterpret_cast<const char*>(gi + tbase * nC) +
                                                             (r * row_bytes + kbytes)));
      }
    }
  };
  auto compute = [&](const BwdFrag<EPI, GI>& f, int tb) {
    const int64_t tbase = block_base(tb);
    const int rows = block_rows(tbase);
    // dot(go, proj_out) of token tbase + col, over the four 8-wide d groups.
    float gf[8], pf[8];
    unpack8(f.gv, gf);
    unpack8(f.pv, pf);
    float dot = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) dot = __builtin_fmaf(gf[e], pf[e], dot);
    dot = rows_sum(dot);  // the wave is converged here
    float scale[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const float d = __shfl(dot, 4 * grp + q, kWave);  // token tbase + 4 * grp + q
      scale[q] = d * (f.inv[q] * f.inv[q]) / static_cast<float>(nC);
    }
    f32x4 acc[8];
    if constexpr (kValu) {
      // VALU build: acc[m][q] = sum_d go[token 4 grp + q][d] * W[d][kl + m] as
      // fp32 FMAs, go rows and W columns read from the wave's LDS copies.
      gvl[wave][col * 4 + grp] = f.gv;
#pragma unroll
      for (int m = 0; m < 8; ++m) acc[m] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll 1
      for (int j = 0; j < 4; ++j) {
        float g[4][8];
#pragma unroll
        for (int q = 0; q < 4; ++q) unpack8(gvl[wave][(4 * grp + q) * 4 + j], g[q]);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          float w[8];
          unpack8(wvl[wave][(8 * j + e) * 16 + col], w);
#pragma unroll
          for (int m = 0; m < 8; ++m)
#pragma unroll
            for (int q = 0; q < 4; ++q) acc[m][q] = __builtin_fmaf(g[q][e], w[m], acc[m][q]);
        }
      }
    } else {
      const bf16x8 a = as_bf16x8(f.gv);
#pragma unroll
      for (int m = 0; m < 8; ++m) acc[m] = mfma16(a, btile_at(m), f32x4{0.f, 0.f, 0.f, 0.f});
    }
    if (kok) {
      char* gxb = reinterpret_cast<char*>(gx + tbase * nC);
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int r = 4 * grp + q;
        if (r < rows) {
          float xf[8], o[8];
          unpack8(f.xv[q], xf);
#pragma unroll
          for (int m = 0; m < 8; ++m) o[m] = f.inv[q] * acc[m][q] - scale[q] * xf[m];
          if constexpr (EPI) {
            float g3f[8];
            unpack8(f.g3[q], g3f);
#pragma unroll
            for (int m = 0; m < 8; ++m)
              o[m] = bf16_to_f32(f32_to_bf16(f.hp[q] * g3f[m])) + bf16_to_f32(f32_to_bf16(o[m]));
            if constexpr (GI) {
              float gif[8];
              unpack8(f.gi[q], gif);
#pragma unroll
              for (int m = 0; m < 8; ++m) o[m] = gif[m] + bf16_to_f32(f32_to_bf16(o[m]));
            }
          }
          st_stream(reinterpret_cast<u32x4*>(gxb + (static_cast<uint32_t>(r) * row_bytes + kbytes)), pack8(o));
        }
      }
    }
    if constexpr (DW) {
      // go block -> LDS (lane (col, grp) holds go[tbase + col][8 grp .. + 8]),
      // then B operands G[tbase + 4 grp + q][16 h + col], q = 0..3, h = 0..1.
      uint32_t* tile = gtile[wave];
      *reinterpret_cast<u32x4*>(tile + col * 16 + grp * 4) = f.gv;
      // Same-wave LDS operations are performed in order: no wait is needed
      // between the write above and the reads below.
      const uint16_t* t16 = reinterpret_cast<const uint16_t*>(tile);
      uint32_t graw[2][4];
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int q = 0; q < 4; ++q) graw[h][q] = t16[(4 * grp + q) * 32 + 16 * h + col];
      __builtin_amdgcn_sched_barrier(0);  // issue all eight reads before converting
      uint32_t bh[2][2];
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        float gq[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const float g = __uint_as_float(graw[h][q] << 16);
          gq[q] = 4 * grp + q < rows ? g * f.inv[q] : 0.f;  // rows past the end contribute nothing
        }
        bh[h][0] = pack_bf16x2(gq[0], gq[1]);
        bh[h][1] = pack_bf16x2(gq[2], gq[3]);
      }
#pragma unroll
      for (int m = 0; m < 8; ++m) {
        // A: element m of the 4 tokens' x vectors.
        uint32_t e[4];
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          const uint32_t w = f.xv[q][m >> 1];
          e[q] = (m & 1) ? (w >> 16) : (w & 0xffffu);
        }
        const u32x2 av = {e[0] | (e[1] << 16), e[2] | (e[3] << 16)};
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const u32x2 bv = {bh[h][0], bh[h][1]};
          dacc[m][h] = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(
              __builtin_bit_cast(bf16x4, av), __builtin_bit_cast(bf16x4, bv), dacc[m][h], 0, 0, 0);
        }
      }
    }
  };
  // NBUF = 3: two blocks in flight while one computes (three rotating
  // fragments, three blocks per trip); NBUF = 2: one.
  BwdFrag<EPI, GI> f0, f1;
  if constexpr (NBUF == 3) {
    BwdFrag<EPI, GI> f2;
    load(f0, 0);
    load(f1, pos(1));
    int i = 0;
    for (; i + 2 < nb; i += 3) {
      load(f2, pos(i + 2));
      __builtin_amdgcn_sched_barrier(0);  // keep the prefetches ahead of the compute
      compute(f0, i);
      load(f0, pos(i + 3));
      __builtin_amdgcn_sched_barrier(0);
      compute(f1, i + 1);
      load(f1, pos(i + 4));
      __builtin_amdgcn_sched_barrier(0);
      compute(f2, i + 2);
    }
    if (i < nb) compute(f0, i);
    if (i + 1 < nb) compute(f1, i + 1);
  } else {
    load(f0, 0);
    int i = 0;
    for (; i + 1 < nb; i += 2) {
      load(f1, pos(i + 1));
      __builtin_amdgcn_sched_barrier(0);  // keep the prefetch ahead of the compute
      compute(f0, i);
      load(f0, pos(i + 2));
      __builtin_amdgcn_sched_barrier(0);
      compute(f1, i + 1);
    }
    if (i < nb) compute(f0, i);
  }

  if constexpr (DW) {
    // Partial layout [run][slice][m][h][r][lane]: one 256-byte row per store.
    float* dst = dw_partial + (run * nslices + slice) * (8 * 2 * 4 * kWave);
#pragma unroll
    for (int m = 0; m < 8; ++m)
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int r = 0; r < 4; ++r) dst[((m * 2 + h) * 4 + r) * kWave + lane] = dacc[m][h][r];
  }
}

// Sums the per-run partials of k1_bwd_mfma<true, ...> in run order and
// writes grad_W (32, nC) bf16.  Partial element
// i = (((slice * 8 + m) * 2 + h) * 4 + r) * 64 + lane stands for
// d = 16 h + (lane & 15), k = 128 slice + 8 (4 (lane >> 4) + r) + m; each
// thread sums four consecutive elements (16-byte loads, four parts per trip).
// Workgroups from dw_blocks on sum K2's parameter gradients instead, one
// workgroup per parameter (the pre-map backward; one launch fewer than K2's
// own reduce).
__global__ __launch_bounds__(256) void k1_dw_reduce(const float* __restrict__ partial,
                                                    uint16_t* __restrict__ dW, int64_t nparts,
                                                    int nslices, int nC, unsigned dw_blocks,
                                                    const K2ParamSums k2) {
  if (blockIdx.x >= dw_blocks) {  // one workgroup per K2 parameter
    k2_param_sum(k2, static_cast<int>(blockIdx.x - dw_blocks));
    return;
  }
  const int64_t per_part = static_cast<int64_t>(nslices) * (8 * 2 * 4 * kWave);
  const int64_t i0 = (static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x) * 4;
  if (i0 >= per_part) return;
  const f32x4* src = reinterpret_cast<const f32x4*>(partial + i0);
  const int64_t stride = per_part / 4;  // in 16-byte vectors
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  int64_t p = 0;
  for (; p + 4 <= nparts; p += 4) {
    const f32x4 v0 = src[(p + 0) * stride], v1 = src[(p + 1) * stride];
    const f32x4 v2 = src[(p + 2) * stride], v3 = src[(p + 3) * stride];
    acc += v0;
    acc += v1;
    acc += v2;
    acc += v3;
  }
  for (; p < nparts; ++p) acc += src[p * stride];
  const int lane0 = static_cast<int>(i0 % kWave);  // multiple of 4
  const int rr = static_cast<int>((i0 / kWave) % 4);
  const int h = static_cast<int>((i0 / (4 * kWave)) % 2);
  const int m = static_cast<int>((i0 / (8 * kWave)) % 8);
  const int slice = static_cast<int>(i0 / (64 * kWave));
  const int k = 128 * slice + 8 * (4 * (lane0 >> 4) + rr) + m;
  if (k >= nC) return;
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int d = 16 * h + ((lane0 + e) & 15);
    dW[static_cast<int64_t>(d) * nC + k] = f32_to_bf16(acc[e]);
  }
}

// grad_W of an empty batch (a kernel, not a memset, so the call can be captured
// in a graph).
__global__ __launch_bounds__(256) void k1_dw_zero(uint16_t* __restrict__ dW, int nC) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i < static_cast<int64_t>(kDout) * nC) dW[i] = 0;
}

// Element-wise weight gradient for shapes the matrix-core path does not take:
// one thread per (d, k), tokens summed in order.
__global__ __launch_bounds__(256) void k1_dw_scalar(const uint16_t* __restrict__ x,
                                                    const uint16_t* __restrict__ go,
                                                    const float* __restrict__ inv_rms,
                                                    uint16_t* __restrict__ dW, int64_t T, int nC) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i >= static_cast<int64_t>(kDout) * nC) return;
  const int d = static_cast<int>(i / nC);
  const int k = static_cast<int>(i % nC);
  float acc = 0.f;
  for (int64_t t = 0; t < T; ++t) {
    const float g = bf16_to_f32(f32_to_bf16(bf16_to_f32(go[t * kDout + d]) * inv_rms[t]));
    acc = __builtin_fmaf(g, bf16_to_f32(x[t * nC + k]), acc);
  }
  dW[i] = f32_to_bf16(acc);
}

// ---------------------------------------------------------------------------
// Element-wise paths for shapes or alignments the matrix-core paths do not
// take (nC % 8 != 0, or a base pointer not 16-byte aligned).  One wave per
// token; results agree with the matrix-core paths to fp32 summation order.
__global__ __launch_bounds__(256) void k1_fwd_scalar(const uint16_t* __restrict__ x,
                                                     const uint16_t* __restrict__ W,
                                                     uint16_t* __restrict__ out,
                                                     float* __restrict__ inv_rms,
                                                     int64_t T, int nC) {
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) >> 6);
  const int64_t t = static_cast<int64_t>(blockIdx.x) * 4 + wave;
  if (t >= T) return;
  const uint16_t* xr = x + t * nC;
  float acc[kDout];
#pragma unroll
  for (int d = 0; d < kDout; ++d) acc[d] = 0.f;
  float ss = 0.f;
  for (int k = lane; k < nC; k += kWave) {
    const float xv = bf16_to_f32(xr[k]);
    ss = __builtin_fmaf(xv, xv, ss);
#pragma unroll
    for (int d = 0; d < kDout; ++d)
      acc[d] = __builtin_fmaf(xv, bf16_to_f32(W[static_cast<int64_t>(d) * nC + k]), acc[d]);
  }
  ss = group_sum<kWave>(ss);
#pragma unroll
  for (int d = 0; d < kDout; ++d) acc[d] = group_sum<kWave>(acc[d]);
  const float inv = rsqrtf(ss / static_cast<float>(nC) + kEps);
  if (lane == 0) {
    inv_rms[t] = inv;
#pragma unroll
    for (int d = 0; d < kDout; ++d) out[t * kDout + d] = f32_to_bf16(acc[d] * inv);
  }
}

// ACC: grad_x already holds the pre-map's K3 term; store bf16(that + bf16(dx)),
// and with an incoming gradient gi (may be null) bf16(gi + bf16(that + bf16(dx))).
template <bool ACC>
__global__ __launch_bounds__(256) void k1_bwd_scalar(const uint16_t* __restrict__ x,
                                                     const uint16_t* __restrict__ W,
                                                     const uint16_t* __restrict__ go,
                                                     const uint16_t* __restrict__ proj,
                                                     const float* __restrict__ inv_rms,
                                                     uint16_t* __restrict__ gx,
                                                     const uint16_t* __restrict__ gi,
                                                     int64_t T, int nC) {
  const int lane = threadIdx.x & (kWave - 1);
  const int wave = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) >> 6);
  const int64_t t = static_cast<int64_t>(blockIdx.x) * 4 + wave;
  if (t >= T) return;
  float g[kDout];
  float dot = 0.f;
#pragma unroll
  for (int d = 0; d < kDout; ++d) {
    g[d] = bf16_to_f32(go[t * kDout + d]);
    dot = __builtin_fmaf(g[d], bf16_to_f32(proj[t * kDout + d]), dot);
  }
  const float inv = inv_rms[t];
  const float scale = dot * (inv * inv) / static_cast<float>(nC);
  const uint16_t* xr = x + t * nC;
  uint16_t* gr = gx + t * nC;
  for (int k = lane; k < nC; k += kWave) {
    float s = 0.f;
#pragma unroll
    for (int d = 0; d < kDout; ++d)
      s = __builtin_fmaf(g[d], bf16_to_f32(W[static_cast<int64_t>(d) * nC + k]), s);
    const float v = inv * s - scale * bf16_to_f32(xr[k]);
    if constexpr (ACC) {
      float u = bf16_to_f32(f32_to_bf16(bf16_to_f32(gr[k]) + bf16_to_f32(f32_to_bf16(v))));
      if (gi) u += bf16_to_f32(gi[t * nC + k]);
      gr[k] = f32_to_bf16(u);
    } else
      gr[k] = f32_to_bf16(v);
  }
}

constexpr int kFwdSplit = 4;  // waves per workgroup (split of the nC axis)
// One-pass forward: R blocks of 16 tokens per workgroup, the fewest that keep
// a launch to one round of workgroups on the 256 CUs, up to 4 (k1_fwd_blocks:
// R = 1 up to T = 4096, 2 up to 8192, 3 up to 12288, 4 beyond; where the
// column split below is not planned the pre-map forward is one kernel on the
// same tiles: against K1 -> K2 -> K3 at C = 1024, T = 4096 / 6000 / 8192
// 29.5 / 36.1 / 41.2 -> 27.1 / 34.5 / 37.2 us).  A workgroup too many
// puts a second one on some CUs, and those set the kernel's time.  K1 forward
// alone at C = 1024, against 32-token tiles below T = 16384 and 64 from there:
// T = 4096 14.3 -> 12.1 us, 12000 27.9 -> 18.1 us, 16000 30.5 -> 21.9 us; the
// pre-map forward at T = 9000 / 12000 / 16000 52.5 / 56.0 / 65.3 -> 35.8 /
// 38.9 / 50.1 us.  More blocks per workgroup than needed cost time (16-token
// blocks at T = 6000 15.3 -> 20.2 us: W is read from L2 once per 16 tokens).
// 5-7 blocks would suit 16385-28672 tokens in the op alone (T = 20000
// 37.6 -> 27.2 us), but not the pre-map tile kernel: it spills (119 us at
// T = 20000 against 71), is slower with its K2 chain in a separate function
// (81 us), and without spills (H_merged's LDS reads kept next to their use)
// runs one workgroup per CU, whose K3 part then has half the waves in flight
// (70 us at T = 20000, 80-86 against 71-76 us at T = 24576-28672).  The op
// keeps the tile's sizes so that the pre-map forward and K1 -> K2 -> K3 give
// the same bits.
// 64-token tiles run two workgroups per CU; 128-token tiles (one) measured
// equal at T = 65536 and 2% slower at T = 262144, C = 4096.
constexpr int kFwdR = 4;
constexpr int64_t kFwdCUs = 256;
// Split forward for few tokens: one 16-token block per workgroup and up to
// kSplitMax column ranges per block, aiming at kSplitTarget workgroups, each
// range at least one 64-wide chunk per wave of the workgroup (narrower ranges
// left waves idle: C = 1024, T = 1 ... 257 took 0.5-0.9 us longer); taken
// when the plan has at least kSplitMinS ranges (T <= 2720 from C = 128 on),
// twice that for rows of up to 64 chunks (C <= 1024: T <= 1024), whose
// one-pass waves walk at most 8 chunks each.  At C = 1024 the pre-map forward
// then takes 14.9 / 16.7 / 17.0 us at T = 1536 / 2048 / 2720 instead of
// 18.8 / 18.6 / 24.8 (the K1 op 11.6 / 11.8 / 12.0 against 10.7 / 10.9 /
// 13.7); at C = 4096 (32 chunks per wave) the split stays the faster form
// (T = 1536: pre-map 39.0 against 48.6 us), and at C = 2048 it is up to
// T = 2048 (K1 op 16.2 against 19.4 us at T = 1536, though 35.2 against
// 28.4 us for the pre-map at 2720).  Above these counts the one-pass
// kernel is faster (T = 3000 ... 6000: 20-40%).
constexpr int kSplitR = 1;
constexpr int64_t kSplitTarget = 512;
constexpr int64_t kSplitMax = 64;
constexpr int64_t kSplitMinS = 4;
// Runs of k1_bwd_mfma: up to kBwdNTB blocks of 16 tokens per run for dx
// alone, kBwdDwNTB with grad_W (fewer runs, fewer grad_W partials); with few
// tokens, runs as short as kBwdDwMinNTB blocks with grad_W (its partials then
// stay below x's bytes) or one block without.
constexpr int kBwdNTB = 8;
constexpr int kBwdDwNTB = 64;
// Fragments in flight in k1_bwd_mfma's block loop (two blocks load while one
// computes): the K1 op kernels, and the pre-map variants (EPI), whose extra
// operands leave no registers for a third buffer at two waves per SIMD.
constexpr int kBwdBufs = 3;
constexpr int kBwdEpiBufs = 2;
constexpr int kBwdDwMinNTB = 4;
constexpr int64_t kBwdFillWaves = 1024;  // one wave per SIMD of 256 CUs

bool bad_sizes(int64_t T, int64_t nC, int64_t D_out) {
  return T < 0 || nC <= 0 || nC > (int64_t{1} << 30) || D_out != kDout;
}

// The backward MFMA kernel addresses 16 rows of x with 32-bit byte offsets
// and reads inv_rms four tokens at a time.
bool k1_bwd_mfma_path(const void* x, const void* W, const void* go, const void* proj, const void* inv_rms,
                      const void* gx, int64_t nC) {
  return nC % 8 == 0 && nC <= (int64_t{1} << 26) && aligned16(x) && aligned16(W) && aligned16(go) &&
         aligned16(proj) && aligned16(inv_rms) && aligned16(gx);
}

// Column split of the forward for T tokens (S = 1: the one-pass kernel).
struct K1FwdSplit {
  int S = 1, cps = 0;
  int64_t bytes = 0;  // partial sums: T x 33 x S4 fp32
};

K1FwdSplit k1_fwd_split(int64_t T, int64_t nC) {
  K1FwdSplit p;
  const int64_t nall = nC >> 6;
  if (T <= 0 || nC % 8 != 0 || nC > (int64_t{1} << 24) || nall < 2) return p;
  const int64_t nblk = (T + 16 * kSplitR - 1) / (16 * kSplitR);
  int64_t S = (kSplitTarget + nblk - 1) / nblk;
  if (S < (nall <= 64 ? 2 * kSplitMinS : kSplitMinS)) return p;
  S = S < kSplitMax ? S : kSplitMax;
  S = S < nall / kFwdSplit ? S : nall / kFwdSplit;
  if (S < 2) return p;
  const int64_t cps = (nall + S - 1) / S;
  S = (nall + cps - 1) / cps;  // every split non-empty
  if (S < 2) return p;
  p.S = static_cast<int>(S);
  p.cps = static_cast<int>(cps);
  p.bytes = T * (kDout + 1) * ((S + 3) & ~int64_t{3}) * static_cast<int64_t>(sizeof(float));
  return p;
}

// Blocks of 16 tokens per workgroup of the one-pass forward for T tokens.
int k1_fwd_blocks(int64_t T) {
  const int64_t r = ((T + 15) / 16 + kFwdCUs - 1) / kFwdCUs;
  return r < 1 ? 1 : (r < kFwdR ? static_cast<int>(r) : kFwdR);
}

// Waves per workgroup of the one-pass forward with R blocks: 8 for tiles of
// 16 and 32 tokens, so that each wave walks half as many column chunks of
// its few rows (pre-map forward at C = 1024, T = 4096 / 6000 / 8192:
// 24.1 / 29.9 / 32.7 -> 22.6 / 28.7 / 32.0 us), 4 for larger tiles, whose
// LDS then leaves room for two workgroups per CU (eight waves on 64-token
// tiles, one workgroup per CU: K1 forward at T = 65536 84.3 -> 89.9 us, the
// pre-map forward 177 -> 183 us).
template <int R>
constexpr int fwd_waves() {
  return R <= 2 ? 8 : kFwdSplit;
}

// The one-pass forward with R blocks per workgroup (k1_fwd_blocks); TILE: the
// pre-map forward on the same tiles.
template <bool TILE>
void launch_k1_fwd_onepass(int R, const uint16_t* x, const uint16_t* W, uint16_t* out, float* inv_rms,
                           int64_t T, int nc, const PremapTile& pt, hipStream_t s) {
  const dim3 grid(blocks_for(T, 16 * R));
  auto launch = [&](auto r) {
    constexpr int kR = decltype(r)::value;
    constexpr int kS = fwd_waves<kR>();
    k1_fwd_mfma<kR, kS, false, TILE><<<grid, kWave * kS, 0, s>>>(x, W, out, inv_rms, nullptr, T, nc, 0, pt);
  };
  switch (R) {
    case 1: launch(std::integral_constant<int, 1>{}); break;
    case 2: launch(std::integral_constant<int, 2>{}); break;
    case 3: launch(std::integral_constant<int, 3>{}); break;
    default: launch(std::integral_constant<int, 4>{});
  }
}

// K1 forward; with a workspace of k1_fwd_split(T, nC).bytes (allow_split) few
// tokens take the column-split kernel.
int k1_fwd_run(const uint16_t* x_flat, const uint16_t* W, uint16_t* out, float* inv_rms, void* ws,
               int64_t ws_bytes, bool allow_split, int64_t T, int64_t nC, hipStream_t s) {
  const int nc = static_cast<int>(nC);
  // The MFMA kernel addresses a workgroup's 16 R rows of x with 32-bit
  // element offsets.
  if (nC % 8 == 0 && nC <= (int64_t{1} << 24) && aligned16(x_flat) && aligned16(W) && aligned16(out)) {
    const K1FwdSplit p = allow_split ? k1_fwd_split(T, nC) : K1FwdSplit{};
    if (p.S > 1) {
      if (!ws || ws_bytes < p.bytes || !aligned16(ws)) return FMHC_ERR_INVALID_ARGUMENT;
      float* part = static_cast<float*>(ws);
      const dim3 grid(blocks_for(T, 16 * kSplitR), p.S);
      k1_fwd_mfma<kSplitR, kFwdSplit, true><<<grid, kWave * kFwdSplit, 0, s>>>(x_flat, W, out, inv_rms, part,
                                                                              T, nc, p.cps);
      const int st = launch_status();
      if (st != FMHC_OK) return st;
      k1_fwd_finish<<<dim3(blocks_for(T, 4)), 256, 0, s>>>(part, out, inv_rms, T, nc, p.S);
    } else {
      launch_k1_fwd_onepass<false>(k1_fwd_blocks(T), x_flat, W, out, inv_rms, T, nc, PremapTile{}, s);
    }
  } else {
    const dim3 grid(blocks_for(T, 4));
    k1_fwd_scalar<<<grid, 256, 0, s>>>(x_flat, W, out, inv_rms, T, nc);
  }
  return launch_status();
}

// Number of runs of k1_bwd_mfma for T tokens (nblocks blocks of 16) and
// nC / 128 slices: ceil(nblocks / max_blocks) runs, or, when those leave SIMDs
// without a wave, more and shorter runs (down to min_blocks blocks) until
// there is one wave per SIMD (kBwdFillWaves).  Measured with grad_W: T = 1024,
// C = 1024 63 -> 14 us, T = 8192 70 -> 40 us; dx alone at T = 1024 16 -> 6 us.
// Filling two waves per SIMD instead, or rounding large run counts to whole
// rounds of resident waves, was slower at C = 4096; two waves per SIMD also
// at C = 1024 (block step at T = 4096 / 6000: 170 -> 178 / 230 -> 236 us).
int64_t k1_bwd_nruns(int64_t T, int64_t nC, int64_t max_blocks, int64_t min_blocks) {
  const int64_t nblocks = (T + 15) / 16;
  if (nblocks <= 0) return 1;
  const int64_t nslices = (nC + 127) / 128;
  const int64_t fill = kBwdFillWaves / nslices > 1 ? kBwdFillWaves / nslices : 1;
  const int64_t nmin = (nblocks + max_blocks - 1) / max_blocks;
  int64_t n = nblocks / min_blocks;
  n = n < fill ? n : fill;
  return n > nmin ? n : nmin;
}

template <bool DW, bool EPI = false, bool GI = false>
void launch_k1_bwd_mfma(hipStream_t s, const uint16_t* x, const uint16_t* W, const uint16_t* go,
                        const uint16_t* proj, const float* inv_rms, uint16_t* gx, float* partial, int64_t T, int nC,
                        int nslices, int64_t nruns, const uint16_t* go3 = nullptr, const float* h_pre = nullptr,
                        int C = 1, const uint16_t* gi = nullptr) {
  const dim3 grid(blocks_for(nruns * nslices, 4));
  constexpr int nbuf = EPI ? kBwdEpiBufs : kBwdBufs;
  // dx alone: one workgroup per CU (LDS reserved that the kernel does not
  // use; its registers allow two) up to C = 2560 per stream.  Measured in
  // the six-kernel step (GB/s, two workgroups per CU against one): T = 65536,
  // C = 1024 6185-6222 against 6436-6440 (cold 6129 against 6315-6355);
  // C = 512 5864 against 6162; C = 2560 5599 against 5789; T = 16384 /
  // 262144, C = 1024 5588 / 6183 against 5724 / 6577; at C = 4096 1-3%
  // slower (T = 65536 and 262144).  With grad_W it changed nothing
  // (202.7-203.1 against 201.8-203.3 us at T = 65536, C = 1024).
  const bool cap = !DW && !EPI && FMHC_LDS_CAP && nC <= 4 * 2560;
  if (nC % 128 == 0) {
    static const unsigned lds =
        lds_reserve(reinterpret_cast<const void*>(&k1_bwd_mfma<DW, true, EPI, GI, nbuf>), kLdsCapOne);
    k1_bwd_mfma<DW, true, EPI, GI, nbuf><<<grid, 256, cap ? lds : 0u, s>>>(x, W, go, proj, inv_rms, gx, partial,
                                                                          go3, h_pre, gi, T, nC, nslices, nruns, C);
  } else {
    static const unsigned lds =
        lds_reserve(reinterpret_cast<const void*>(&k1_bwd_mfma<DW, false, EPI, GI, nbuf>), kLdsCapOne);
    k1_bwd_mfma<DW, false, EPI, GI, nbuf><<<grid, 256, cap ? lds : 0u, s>>>(x, W, go, proj, inv_rms, gx, partial,
                                                                           go3, h_pre, gi, T, nC, nslices, nruns,
                                                                           C);
  }
}

}  // namespace
}  // namespace fmhc

extern "C" int fmhc_k1_fwd(const uint16_t* x_flat, const uint16_t* W, uint16_t* out,
                           float* inv_rms, int64_t T, int64_t nC, int64_t D_out, void* stream) {
  using namespace fmhc;
  if (bad_sizes(T, nC, D_out)) return FMHC_ERR_INVALID_ARGUMENT;
  if (T == 0) return FMHC_OK;
  if (!x_flat || !W || !out || !inv_rms) return FMHC_ERR_INVALID_ARGUMENT;
  return k1_fwd_run(x_flat, W, out, inv_rms, nullptr, 0, false, T, nC, static_cast<hipStream_t>(stream));
}

extern "C" int64_t fmhc_k1_fwd_workspace_bytes(int64_t T, int64_t nC) {
  return fmhc::k1_fwd_split(T, nC).bytes;
}

extern "C" int fmhc_k1_fwd_ws(const uint16_t* x_flat, const uint16_t* W, uint16_t* out, float* inv_rms,
                              void* workspace, int64_t workspace_bytes, int64_t T, int64_t nC, int64_t D_out,
                              void* stream) {
  using namespace fmhc;
  if (bad_sizes(T, nC, D_out)) return FMHC_ERR_INVALID_ARGUMENT;
  if (T == 0) return FMHC_OK;
  if (!x_flat || !W || !out || !inv_rms) return FMHC_ERR_INVALID_ARGUMENT;
  return k1_fwd_run(x_flat, W, out, inv_rms, workspace, workspace_bytes, true, T, nC,
                    static_cast<hipStream_t>(stream));
}

extern "C" int fmhc_k1_bwd_dx(const uint16_t* x_flat, const uint16_t* W, const uint16_t* grad_out,
                              const uint16_t* proj_out, const float* inv_rms, uint16_t* grad_x,
                              int64_t T, int64_t nC, int64_t D_out, void* stream) {
  using namespace fmhc;
  if (bad_sizes(T, nC, D_out)) return FMHC_ERR_INVALID_ARGUMENT;
  if (T == 0) return FMHC_OK;
  if (!x_flat || !W || !grad_out || !proj_out || !inv_rms || !grad_x)
    return FMHC_ERR_INVALID_ARGUMENT;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int nc = static_cast<int>(nC);
  if (k1_bwd_mfma_path(x_flat, W, grad_out, proj_out, inv_rms, grad_x, nC)) {
    const int nslices = static_cast<int>((nC + 127) / 128);
    const int64_t nruns = k1_bwd_nruns(T, nC, kBwdNTB, 1);
    launch_k1_bwd_mfma<false>(s, x_flat, W, grad_out, proj_out, inv_rms, grad_x, nullptr, T, nc, nslices, nruns);
  } else {
    const dim3 grid(blocks_for(T, 4));
    k1_bwd_scalar<false><<<grid, 256, 0, s>>>(x_flat, W, grad_out, proj_out, inv_rms, grad_x, nullptr, T, nc);
  }
  return launch_status();
}

namespace fmhc {
namespace {
// Runs with grad_W fused.
// Runs of the backward with grad_W.  Beyond one run per wave slot the count
// is rounded up to a multiple of kBwdFillWaves / nslices, the run groups the
// pre-map backward's split kernel walks side by side (premap_split.hip), so
// that each group takes the same number of runs; it shares these runs, and so
// grad_W's partial sums, with this kernel.
int64_t k1_bwd_runs(int64_t T, int64_t nC) {
  const int64_t n = k1_bwd_nruns(T, nC, kBwdDwNTB, kBwdDwMinNTB);
  const int64_t nslices = (nC + 127) / 128;
  const int64_t fill = kBwdFillWaves / nslices > 1 ? kBwdFillWaves / nslices : 1;
  const int64_t nblocks = (T + 15) / 16;
  if (n <= fill) return n;
  const int64_t r = (n + fill - 1) / fill * fill;
  return r < nblocks ? r : nblocks;
}
}  // namespace
}  // namespace fmhc

extern "C" int64_t fmhc_k1_bwd_workspace_bytes(int64_t T, int64_t nC) {
  using namespace fmhc;
  if (T <= 0 || nC <= 0 || nC % 8 != 0 || nC > (int64_t{1} << 26)) return 0;  // no MFMA path: no workspace
  const int64_t nslices = (nC + 127) / 128;
  return k1_bwd_runs(T, nC) * nslices * (8 * 2 * 4 * kWave) * static_cast<int64_t>(sizeof(float));
}

extern "C" int fmhc_k1_bwd(const uint16_t* x_flat, const uint16_t* W, const uint16_t* grad_out,
                           const uint16_t* proj_out, const float* inv_rms, uint16_t* grad_x,
                           uint16_t* grad_W, void* workspace, int64_t workspace_bytes, int64_t T,
                           int64_t nC, int64_t D_out, void* stream) {
  using namespace fmhc;
  if (bad_sizes(T, nC, D_out)) return FMHC_ERR_INVALID_ARGUMENT;
  if (!grad_W) return FMHC_ERR_INVALID_ARGUMENT;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int nc = static_cast<int>(nC);
  if (T == 0) {  // grad_W of an empty batch is zero
    k1_dw_zero<<<dim3(blocks_for(static_cast<int64_t>(kDout) * nC, 256)), 256, 0, s>>>(grad_W, nC);
    return launch_status();
  }
  if (!x_flat || !W || !grad_out || !proj_out || !inv_rms || !grad_x) return FMHC_ERR_INVALID_ARGUMENT;
  if (k1_bwd_mfma_path(x_flat, W, grad_out, proj_out, inv_rms, grad_x, nC)) {
    const int64_t need = fmhc_k1_bwd_workspace_bytes(T, nC);
    if (!workspace || workspace_bytes < need || !aligned16(workspace)) return FMHC_ERR_INVALID_ARGUMENT;
    const int nslices = static_cast<int>((nC + 127) / 128);
    const int64_t nruns = k1_bwd_runs(T, nC);
    float* partial = static_cast<float*>(workspace);
    launch_k1_bwd_mfma<true>(s, x_flat, W, grad_out, proj_out, inv_rms, grad_x, partial, T, nc, nslices, nruns);
    const int st = launch_status();
    if (st != FMHC_OK) return st;
    const int64_t per_part = static_cast<int64_t>(nslices) * (8 * 2 * 4 * kWave);
    const unsigned nb = blocks_for(per_part / 4, 256);
    k1_dw_reduce<<<dim3(nb), 256, 0, s>>>(partial, grad_W, nruns, nslices, nc, nb, K2ParamSums{});
    return launch_status();
  }
  const int st = fmhc_k1_bwd_dx(x_flat, W, grad_out, proj_out, inv_rms, grad_x, T, nC, D_out, stream);
  if (st != FMHC_OK) return st;
  k1_dw_scalar<<<dim3(blocks_for(static_cast<int64_t>(kDout) * nC, 256)), 256, 0, s>>>(
      x_flat, grad_out, inv_rms, grad_W, T, nc);
  return launch_status();
}

namespace fmhc {

bool k1_premap_tile(const uint16_t* x, const uint16_t* W, uint16_t* proj, float* inv_rms, const PremapTile& pt,
                    int64_t T, int64_t C, hipStream_t s, int* status) {
  const int64_t nC = 4 * C;
  // Where K1's column split is planned (few tokens) the pre-map forward takes
  // it and its second stage fused with K2 and K3 (premap.hip) instead.
  if (T <= 0 || k1_fwd_split(T, nC).S > 1 || C % 8 != 0 || nC > (int64_t{1} << 24) || !aligned16(x) || !aligned16(W) ||
      !aligned16(proj) || (pt.layer_input && !aligned16(pt.layer_input)))
    return false;
  launch_k1_fwd_onepass<true>(k1_fwd_blocks(T), x, W, proj, inv_rms, T, static_cast<int>(nC), pt, s);
  *status = launch_status();
  return true;
}

int k1_fwd_partials(const uint16_t* x_flat, const uint16_t* W, void* ws, int64_t ws_bytes, int64_t T,
                    int64_t nC, hipStream_t s) {
  if (!(nC % 8 == 0 && nC <= (int64_t{1} << 24) && aligned16(x_flat) && aligned16(W))) return 0;
  const K1FwdSplit p = k1_fwd_split(T, nC);
  if (p.S < 2) return 0;
  if (!ws || ws_bytes < p.bytes || !aligned16(ws)) return -FMHC_ERR_INVALID_ARGUMENT;
  const dim3 grid(blocks_for(T, 16 * kSplitR), p.S);
  k1_fwd_mfma<kSplitR, kFwdSplit, true><<<grid, kWave * kFwdSplit, 0, s>>>(
      x_flat, W, nullptr, nullptr, static_cast<float*>(ws), T, static_cast<int>(nC), p.cps);
  const int st = launch_status();
  return st == FMHC_OK ? p.S : -st;
}

int64_t k1_bwd_dw_runs(int64_t T, int64_t nC) { return k1_bwd_runs(T, nC); }

int k1_dw_finish(const float* partial, uint16_t* grad_W, int64_t nruns, int nslices, int nC,
                 const K2ParamSums& sums, hipStream_t s) {
  const int64_t per_part = static_cast<int64_t>(nslices) * (8 * 2 * 4 * kWave);
  const unsigned nb = blocks_for(per_part / 4, 256);
  static_assert(kK2SumThreads == 256, "K2's parameter sums share the reduce's workgroups");
  k1_dw_reduce<<<dim3(nb + kNPar), 256, 0, s>>>(partial, grad_W, nruns, nslices, nC, nb, sums);
  return launch_status();
}

// K1 backward of the pre-map region (premap.hip): grad_W as fmhc_k1_bwd and
// grad_x = bf16(bf16(h_pre[t, j] go3[t, c]) + bf16(dx)).  On the MFMA path the
// K3 term is computed in the store; otherwise grad_x must already hold it
// (fmhc_k3_bwd's grad_x) and the element-wise kernel adds dx to it.
bool k1_bwd_premap_fused(const void* x, const void* W, const void* go, const void* proj, const void* inv_rms,
                         const void* gx, const void* go3, const void* gi, int64_t C) {
  return C % 8 == 0 && k1_bwd_mfma_path(x, W, go, proj, inv_rms, gx, 4 * C) && aligned16(go3) && aligned16(gi);
}

int k1_bwd_premap(const uint16_t* x_flat, const uint16_t* W, const uint16_t* grad_proj,
                  const uint16_t* proj, const float* inv_rms, const uint16_t* go3, const float* h_pre,
                  const uint16_t* grad_x_in, uint16_t* grad_x, uint16_t* grad_W, void* workspace,
                  int64_t workspace_bytes, int64_t T, int64_t C, const K2ParamSums& k2_sums, hipStream_t s) {
  const int64_t nC = 4 * C;
  const int nc = static_cast<int>(nC);
  if (T == 0) {
    k1_dw_zero<<<dim3(blocks_for(static_cast<int64_t>(kDout) * nC, 256)), 256, 0, s>>>(grad_W, nc);
    launch_k2_param_reduce(k2_sums, s);
    return launch_status();
  }
  if (k1_bwd_premap_fused(x_flat, W, grad_proj, proj, inv_rms, grad_x, go3, grad_x_in, C)) {
    if (!workspace || workspace_bytes < fmhc_k1_bwd_workspace_bytes(T, nC) || !aligned16(workspace))
      return FMHC_ERR_INVALID_ARGUMENT;
    const int nslices = static_cast<int>((nC + 127) / 128);
    const int64_t nruns = k1_bwd_runs(T, nC);
    float* partial = static_cast<float*>(workspace);
    if (grad_x_in)
      launch_k1_bwd_mfma<true, true, true>(s, x_flat, W, grad_proj, proj, inv_rms, grad_x, partial, T, nc, nslices,
                                           nruns, go3, h_pre, static_cast<int>(C), grad_x_in);
    else
      launch_k1_bwd_mfma<true, true>(s, x_flat, W, grad_proj, proj, inv_rms, grad_x, partial, T, nc, nslices,
                                     nruns, go3, h_pre, static_cast<int>(C));
    const int st = launch_status();
    if (st != FMHC_OK) return st;
    return k1_dw_finish(partial, grad_W, nruns, nslices, nc, k2_sums, s);
  }
  k1_bwd_scalar<true><<<dim3(blocks_for(T, 4)), 256, 0, s>>>(x_flat, W, grad_proj, proj, inv_rms, grad_x,
                                                             grad_x_in, T, nc);
  const int st = launch_status();
  if (st != FMHC_OK) return st;
  k1_dw_scalar<<<dim3(blocks_for(static_cast<int64_t>(kDout) * nC, 256)), 256, 0, s>>>(
      x_flat, grad_proj, inv_rms, grad_W, T, nc);
  launch_k2_param_reduce(k2_sums, s);
  return launch_status();
}

}  // namespace fmhc
