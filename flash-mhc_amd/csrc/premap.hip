// The pre-map region of an mHC-lite block (K1, K2, K3 of block.py:157-177 of
// alint77/flash-mHC) behind one entry point per direction.
//
// Backward: x receives two gradients here, K3's h_pre[j] go3 and K1's dx;
// with separate ops autograd writes both (2 x T x nC bf16) and adds them in a
// third pass.  Here K3's backward only reduces grad_h_pre (x and go3 read, no
// grad_x written), K2's backward gives K1's grad_out, and K1's backward
// (with grad_W) adds bf16(h_pre go3) to bf16(dx) in its store: one grad_x
// write, the same bf16 sum.  x's third gradient in a block, post-res's
// H_merged^T grad_out, can come in as grad_x_in: K1's store then adds it too
// (bf16(grad_x_in + pre-map gradient), autograd's sum), which replaces
// autograd's separate accumulation pass (1.5 x T x nC x 2 bytes).
//
// Forward.  Rows of C = 512 or 1024 per stream with at least 16384 tokens
// and a layer input: the single-read kernel (premap_resident.hip), which
// keeps W on each CU and reads every row of x once.  Other shapes from the
// token count where K1 runs one pass (no column split; T > 1024 up to
// C = 1024, T > 2720 above): one tile kernel (k1_premap_tile, k1.hip).  Each
// workgroup runs K1 on its tile (16, 32, 48 or 64 tokens, the fewest that
// keep the launch to one round on the CUs) with ordinary loads of x, then K2
// on the tile's tokens (four lanes per token) and K3 on the tile.  K3's
// re-read of the tile misses L2: past L2 the kernel moves x twice (FETCH_SIZE
// 2 x x), as three kernels do, in 15% less time (T = 65536, C = 1024: 174
// against 209 us cold), and the same kernel with nontemporal K1 loads is no
// faster than three kernels, which places the gain in the re-read.  Fewer
// tokens, and shapes off the matrix-core path: K1 -> K2 -> K3, the kernels of
// k1.hip, k2.hip, k3.hip; for few tokens K1 is split over the columns
// (partial sums in the caller's workspace), and its second stage runs inside
// the K2 kernel (k1_finish_k2; with K3 too when the layer input is wanted,
// k1_finish_k2_k3).

#include <hip/hip_runtime.h>

#include <mutex>
#include <type_traits>

#include "flash_mhc_hip.h"
#include "fmhc_common.h"
#include "k1_premap.h"
#include "k2_chain.h"

// 1 (an evidence build): the backward of many tokens at C a multiple of 128
// reads x once (premap_split.hip); 0: K3's reduce pass, K2's backward and K1's
// backward, each reading x, which is faster (the split kernel waits on its
// team's exchange).
#ifndef FMHC_PREMAP_SPLIT
#define FMHC_PREMAP_SPLIT 0
#endif

// 1: the forward without K1's column split runs as one kernel, K1 with K2
// and K3 on each tile (k1_premap_tile); 0 (an evidence build): K1, K2 and K3
// as three kernels, each reading x from HBM.
#ifndef FMHC_PREMAP_TILE
#define FMHC_PREMAP_TILE 1
#endif
// 1: rows of C = 512 or 1024 per stream and many tokens take the kernel that
// keeps W and the rows on chip (premap_resident.hip, x read once); 0 (an
// evidence build): they take the tile kernel, whose K3 part re-reads x.
#ifndef FMHC_PREMAP_RESIDENT
#define FMHC_PREMAP_RESIDENT 1
#endif

namespace {

using namespace fmhc;

constexpr int64_t kAlign = 256;
int64_t round_up(int64_t v) { return (v + kAlign - 1) / kAlign * kAlign; }

// Checked before the first launch, so that a bad dtype leaves no partial outputs.
bool param_dtype_ok(int d) { return d == FMHC_PARAM_F32 || d == FMHC_PARAM_BF16; }

constexpr int kFinishThreads = 256;  // 8 tokens of 32 lanes

// Few tokens: K1's second stage and K2 in one kernel, 32 lanes per token.
// Lane q adds the S partials of projection q and those of the sum of squares
// in split order (as k1_fwd_finish does), stores proj[t, q] =
// bf16(sum * inv_rms) and inv_rms, then runs K2 on that bf16 value
// (k2_token32): the same values as K1's finish kernel followed by K2.
// K1's second stage for token t in 32 lanes: lane q adds the S partials of
// projection q and of the sum of squares in split order, stores proj[t, q]
// and (lane 0) inv_rms[t], and returns the stored bf16 projection as fp32.
__device__ __forceinline__ float finish_token32(const float* __restrict__ part, int S, int nC, int q, int64_t t,
                                                uint16_t* __restrict__ proj, float* __restrict__ inv_rms) {
  // The loads of both sums run ahead together.
  const int s4 = (S + 3) & ~3;
  const f32x4* pv = reinterpret_cast<const f32x4*>(part + (t * (kDk + 1) + q) * s4);
  const f32x4* ps = reinterpret_cast<const f32x4*>(part + (t * (kDk + 1) + kDk) * s4);
  float v = 0.f, ss = 0.f;
#pragma unroll 8
  for (int i = 0; i < s4 / 4; ++i) {
    const f32x4 a = pv[i], b = ps[i];
    v += a[0];  // 4 i < S always
    ss += b[0];
    if (4 * i + 1 < S) {
      v += a[1];
      ss += b[1];
    }
    if (4 * i + 2 < S) {
      v += a[2];
      ss += b[2];
    }
    if (4 * i + 3 < S) {
      v += a[3];
      ss += b[3];
    }
  }
  const float inv = rsqrtf(ss / static_cast<float>(nC) + kRmsEps);
  const uint16_t pj = f32_to_bf16(v * inv);
  proj[t * kDk + q] = pj;
  if (q == 0) inv_rms[t] = inv;
  return bf16_to_f32(pj);
}

__global__ __launch_bounds__(kFinishThreads) void k1_finish_k2(
    const float* __restrict__ part, int S, int nC, const K2Params P, uint16_t* __restrict__ proj,
    float* __restrict__ inv_rms, float* __restrict__ h_pre, float* __restrict__ h_post, float* __restrict__ H,
    int64_t T, const ZeroWords z) {
  __shared__ K2Smem sm;
  zero_words(z);
  stage_params<kFinishThreads>(P, sm);
  const int q = threadIdx.x & 31;
  const int64_t t = static_cast<int64_t>(blockIdx.x) * (kFinishThreads / 32) + (threadIdx.x >> 5);
  if (t >= T) return;  // a whole 32-lane group leaves together
  const float p = finish_token32(part, S, nC, q, t, proj, inv_rms);
  k2_token32(sm, p, q, t, h_pre, h_post, H);
}

// The same with K3 fused, one token per workgroup (blockIdx.x): its first 32
// lanes finish K1 and run K2 and leave h_pre in LDS; after the barrier all
// 256 lanes mix the token's streams into layer_input with those values
// (k3_token's arithmetic, so the results are those of the separate K3 kernel
// reading the stored h_pre).  Saves K3's launch for few tokens.  Up to
// C = 4096 (two 16-byte groups per lane) every lane loads its x vectors
// before K1's partial sums and K2's chain run, so their latency overlaps.
template <int VEC>
__global__ __launch_bounds__(kFinishThreads) void k1_finish_k2_k3(
    const float* __restrict__ part, int S, int nC, const K2Params P, uint16_t* __restrict__ proj,
    float* __restrict__ inv_rms, float* __restrict__ h_pre, float* __restrict__ h_post, float* __restrict__ H,
    const ZeroWords z, const uint16_t* __restrict__ x, uint16_t* __restrict__ layer_input, int C) {
  __shared__ K2Smem sm;
  __shared__ float hsh[kN];  // the token's h_pre, handed from the K2 lanes to all
  constexpr int kPre = 2;    // 16-byte groups per lane and stream loaded ahead
  const int64_t t = blockIdx.x;
  const int lane = static_cast<int>(threadIdx.x);
  const uint16_t* x0 = x + t * 4 * C;
  const int ng = C / 8;
  const bool pre = VEC == 8 && ng <= kPre * kFinishThreads;
  u32x4 xv[kPre][4];
  if (pre) {
#pragma unroll
    for (int it = 0; it < kPre; ++it) {
      const int g = lane + it * kFinishThreads;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        xv[it][j] = u32x4{0u, 0u, 0u, 0u};
        if (g < ng) xv[it][j] = ld_stream(reinterpret_cast<const u32x4*>(x0 + j * C) + g);
      }
    }
  }
  zero_words(z);
  stage_params<kFinishThreads>(P, sm);
  if (threadIdx.x < 32) {
    const int q = lane;
    const float p = finish_token32(part, S, nC, q, t, proj, inv_rms);
    const float y = k2_token32(sm, p, q, t, h_pre, h_post, H);
    if (q < kN) hsh[q] = y;
  }
  __syncthreads();
  const float h[4] = {hsh[0], hsh[1], hsh[2], hsh[3]};
  if (!pre) {
    k3_token<VEC>(x0, h, layer_input + t * C, lane, kFinishThreads, C);
    return;
  }
#pragma unroll
  for (int it = 0; it < kPre; ++it) {
    const int g = lane + it * kFinishThreads;
    if (g < ng) {
      float a[8], b[8], c[8], d[8], o[8];
      unpack8(xv[it][0], a);
      unpack8(xv[it][1], b);
      unpack8(xv[it][2], c);
      unpack8(xv[it][3], d);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        float acc = h[0] * a[e];
        acc = __builtin_fmaf(h[1], b[e], acc);
        acc = __builtin_fmaf(h[2], c[e], acc);
        o[e] = __builtin_fmaf(h[3], d[e], acc);
      }
      Lanes<8>::store(layer_input + t * C, g, o);
    }
  }
}

// Backward, few tokens (T <= kK2BwdSmallT) where K3's backward runs 32 or 64
// lanes per token: K3's reduce-only pass and K2's backward in one kernel,
// kK2BwdTok tokens per workgroup.  A token's four grad_h_pre sums are
// k3_bwd_kernel's (the same lanes, loop order and group sums) and stay in
// registers; the token's first 32 lanes then run k2_bwd_token32 as
// k2_bwd_small does, and the workgroup adds its tokens' parameter terms in
// token order.  grad_proj and the parameter partials are those of K3's
// backward followed by k2_bwd_small, bit for bit, with one launch and one
// chain of load latencies fewer.
template <int LPT, bool CANON>
__global__ __launch_bounds__(kK2BwdTok * LPT) void k3_reduce_k2_bwd(
    const uint16_t* __restrict__ x, const uint16_t* __restrict__ go3, const uint16_t* __restrict__ proj,
    const K2Params P, const float* __restrict__ g_hpost, const float* __restrict__ g_H,
    uint16_t* __restrict__ grad_proj, float* __restrict__ partial, int64_t T, int C) {
  static_assert(LPT == 32 || LPT == 64, "half a wave or one wave per token");
  constexpr int kThreads = kK2BwdTok * LPT;
  __shared__ K2Smem sm;
  __shared__ float red[kK2BwdTok][kNPar];
  const int slot = static_cast<int>(threadIdx.x) / LPT;
  const int sub = static_cast<int>(threadIdx.x) % LPT;
  const int q = sub & 31;
  const int64_t tq = static_cast<int64_t>(blockIdx.x) * kK2BwdTok + slot;
  const bool valid = tq < T;
  const int64_t t = valid ? tq : T - 1;  // idle slots recompute the last token, store nothing
  // K2's operands and the parameters are loaded before K3's loop.
  const float p = bf16_to_f32(proj[t * kDk + q]);
  const float gh_in = (q < kN * kN && g_H) ? g_H[t * kN * kN + q] : 0.f;
  const float gpost = g_hpost ? g_hpost[t * kN + ((q - kN) & 3)] : 0.f;
  K2ParamRegs<kThreads> regs;
  regs.load(P);

  // K3's reduce-only backward of the token: s_j = sum_c x[t, j, c] go3[t, c],
  // in k3_bwd_kernel's order (with CANON the slice order of slice_sums_add).
  float s[4] = {0.f, 0.f, 0.f, 0.f};
  const int ng = C / 8;
  const uint16_t* x0 = x + t * 4 * C;
  const uint16_t* x1 = x0 + C;
  const uint16_t* x2 = x1 + C;
  const uint16_t* x3 = x2 + C;
  const uint16_t* grow = go3 + t * C;
  auto round = [&](int g, float (&acc)[4]) {
    float gq[8], a[8], b[8], c[8], d[8];
    Lanes<8>::load(grow, g, gq);
    Lanes<8>::load(x0, g, a);
    Lanes<8>::load(x1, g, b);
    Lanes<8>::load(x2, g, c);
    Lanes<8>::load(x3, g, d);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      acc[0] = __builtin_fmaf(a[e], gq[e], acc[0]);
      acc[1] = __builtin_fmaf(b[e], gq[e], acc[1]);
      acc[2] = __builtin_fmaf(c[e], gq[e], acc[2]);
      acc[3] = __builtin_fmaf(d[e], gq[e], acc[3]);
    }
  };
  if constexpr (CANON) {
    // Every slot computes (idle ones on the last token), so the slot's lanes
    // are all active for the row sums.
    constexpr int kRounds = LPT == 64 ? 4 : 2;  // fewer than 256 (64) groups for 64 (32) lanes
    float e[kRounds][4];
#pragma unroll
    for (int k = 0; k < kRounds; ++k) {
#pragma unroll
      for (int j = 0; j < 4; ++j) e[k][j] = 0.f;
      if (sub + k * LPT < ng) round(sub + k * LPT, e[k]);
    }
    const int lane = static_cast<int>(threadIdx.x) & (kWave - 1);
#pragma unroll
    for (int k = 0; k < kRounds; ++k) {
      if (k * LPT >= ng) break;  // uniform
      slice_sums_add<LPT>(e[k], s, k, ng / 16, lane);
    }
  } else {
    if (valid) {
#pragma unroll 2
      for (int g = sub; g < ng; g += LPT) round(g, s);
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) s[j] = group_sum<LPT>(s[j]);
  }
  const float s0 = s[0], s1 = s[1], s2 = s[2], s3 = s[3];

  regs.store(sm);
  __syncthreads();
  const int j4 = q & 3;
  const float gpre = j4 == 0 ? s0 : (j4 == 1 ? s1 : (j4 == 2 ? s2 : s3));
  // With 64 lanes per token, lanes 32-63 repeat lanes 0-31 and store nothing.
  const bool first = sub < 32;
  k2_bwd_token32(sm, q, t, valid && first, first, p, gh_in, gpost, gpre, grad_proj, red[slot]);
  __syncthreads();
  if (threadIdx.x < kNPar) {
    float v = 0.f;
#pragma unroll
    for (int w = 0; w < kK2BwdTok; ++w) v += red[w][threadIdx.x];
    partial[static_cast<int64_t>(blockIdx.x) * kNPar + threadIdx.x] = v;
  }
}

struct PremapWs {
  int64_t gh, gp, k2, k1, ring, total;  // byte offsets / sizes
};

PremapWs premap_ws(int64_t T, int64_t C) {
  PremapWs w;
  w.gh = 0;                                     // grad_h_pre (T, 4) fp32
  w.gp = round_up(T * 4 * 4);                   // grad_proj (T, 32) bf16
  w.k2 = w.gp + round_up(T * 32 * 2);           // K2 parameter partials
  w.k1 = w.k2 + round_up(fmhc_k2_bwd_workspace_bytes(T));  // K1 grad_W partials
  w.ring = w.k1 + round_up(fmhc_k1_bwd_workspace_bytes(T, 4 * C));  // the split backward's exchange ring
  w.total = w.ring + (T > 0 && C % kSliceCols == 0 ? round_up(premap_split_ring_bytes(T, C)) : 0);
  return w;
}

}  // namespace

extern "C" int64_t fmhc_premap_fwd_workspace_bytes(int64_t T, int64_t C) {
  if (T <= 0 || C <= 0) return 0;
  return fmhc_k1_fwd_workspace_bytes(T, 4 * C);
}

namespace {

// The forward of fmhc_premap_fwd with its workspace already in hand.
int premap_fwd_run(const uint16_t* x, const uint16_t* W, const void* alpha_pre, const void* alpha_post,
                   const void* alpha_res, const void* bias, const void* perm, int param_dtype,
                   uint16_t* layer_input, uint16_t* proj, float* inv_rms, float* h_pre, float* h_post,
                   float* H_merged, uint16_t* zero_word_a, uint16_t* zero_word_b, void* workspace,
                   int64_t workspace_bytes, int64_t T, int64_t C, int64_t n, void* stream) {
  if (T < 0 || C <= 0 || C > (int64_t{1} << 24) || n != 4 || !param_dtype_ok(param_dtype))
    return FMHC_ERR_INVALID_ARGUMENT;
  if (T == 0) return FMHC_OK;
  if (!x || !W || !alpha_pre || !alpha_post || !alpha_res || !bias || !perm || !proj || !inv_rms || !h_pre ||
      !h_post || !H_merged)
    return FMHC_ERR_INVALID_ARGUMENT;
  if (!aligned16(h_pre) || !aligned16(h_post) || !aligned16(H_merged)) return FMHC_ERR_INVALID_ARGUMENT;
  fmhc::K2Params P;
  if (!fmhc::k2_params(alpha_pre, alpha_post, alpha_res, bias, perm, param_dtype, P))
    return FMHC_ERR_INVALID_ARGUMENT;
  const fmhc::ZeroWords z{zero_word_a, zero_word_b};
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (FMHC_PREMAP_TILE) {
    fmhc::PremapTile pt;
    pt.P = P;
    pt.h_pre = h_pre;
    pt.h_post = h_post;
    pt.H = H_merged;
    pt.layer_input = layer_input;
    pt.C = static_cast<int>(C);
    pt.z = z;
    int st = FMHC_OK;
    if (FMHC_PREMAP_RESIDENT && fmhc::premap_resident(x, W, proj, inv_rms, pt, T, C, s, &st)) return st;
    if (fmhc::k1_premap_tile(x, W, proj, inv_rms, pt, T, C, s, &st)) return st;
  }
  const int S = fmhc::k1_fwd_partials(x, W, workspace, workspace_bytes, T, n * C, s);
  if (S < 0) return -S;
  int st = FMHC_OK;
  const float* part = static_cast<const float*>(workspace);
  const int nc = static_cast<int>(n * C);
  if (S >= 2 && layer_input) {
    const dim3 grid(static_cast<unsigned>(T));
    const int c = static_cast<int>(C);
    if (C % 8 == 0 && aligned16(x) && aligned16(layer_input))
      k1_finish_k2_k3<8><<<grid, kFinishThreads, 0, s>>>(part, S, nc, P, proj, inv_rms, h_pre, h_post, H_merged,
                                                          z, x, layer_input, c);
    else
      k1_finish_k2_k3<1><<<grid, kFinishThreads, 0, s>>>(part, S, nc, P, proj, inv_rms, h_pre, h_post, H_merged,
                                                          z, x, layer_input, c);
    return fmhc::launch_status();
  }
  if (S >= 2) {
    k1_finish_k2<<<dim3(static_cast<unsigned>((T + 7) / 8)), kFinishThreads, 0, s>>>(
        part, S, nc, P, proj, inv_rms, h_pre, h_post, H_merged, T, z);
    st = fmhc::launch_status();
  } else {
    st = fmhc_k1_fwd_ws(x, W, proj, inv_rms, workspace, workspace_bytes, T, n * C, 32, stream);
    if (st == FMHC_OK) st = fmhc::k2_fwd_launch(proj, P, h_pre, h_post, H_merged, T, z, s);
  }
  if (st == FMHC_OK && layer_input) st = fmhc_k3_fwd(x, h_pre, layer_input, T, C, n, stream);
  return st;
}

// Scratch of fmhc_premap_fwd_noalloc: the column-split forward's partial sums
// (T x 33 x S4 fp32 for T <= 2720 tokens; at most 2,145,792 bytes over every
// (T, C), at T = 2032, C = 1040).  Each device holds its own copy for the life
// of the process.  In host code `scratch` names a host-side stand-in, so its
// device address is looked up once per device (scratch_on_device) and only
// that address is used.
constexpr int64_t kNoAllocScratchBytes = int64_t{4} << 20;
__device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex scratch_mu;
void* scratch_addr[kMaxDevices];  // per device; guarded by scratch_mu

// Device address of `scratch` on the device that runs `stream` (which must be
// the current device), looked up on the first call on that device.
int scratch_on_device(void* stream, void** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return fmhc::hip_status(e);
  if (stream) {
    int sdev = 0;
    e = hipStreamGetDevice(static_cast<hipStream_t>(stream), &sdev);
    if (e != hipSuccess) return fmhc::hip_status(e);
    if (sdev != dev) return FMHC_ERR_INVALID_ARGUMENT;
  }
  if (dev < 0 || dev >= kMaxDevices) return FMHC_ERR_INVALID_ARGUMENT;
  std::lock_guard<std::mutex> lock(scratch_mu);
  if (!scratch_addr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return fmhc::hip_status(e);
    if (!p) return FMHC_ERR_HIP_BASE + static_cast<int>(hipErrorInvalidSymbol);
    scratch_addr[dev] = p;
  }
  *out = scratch_addr[dev];
  return FMHC_OK;
}

}  // namespace

extern "C" int fmhc_premap_fwd(const uint16_t* x, const uint16_t* W, const void* alpha_pre,
                               const void* alpha_post, const void* alpha_res, const void* bias,
                               const void* perm, int param_dtype, uint16_t* layer_input, uint16_t* proj,
                               float* inv_rms, float* h_pre, float* h_post, float* H_merged,
                               uint16_t* zero_word_a, uint16_t* zero_word_b, void* workspace,
                               int64_t workspace_bytes, int64_t T, int64_t C, int64_t n, void* stream) {
  return premap_fwd_run(x, W, alpha_pre, alpha_post, alpha_res, bias, perm, param_dtype, layer_input, proj,
                        inv_rms, h_pre, h_post, H_merged, zero_word_a, zero_word_b, workspace, workspace_bytes,
                        T, C, n, stream);
}

extern "C" int fmhc_premap_fwd_noalloc(const uint16_t* x, const uint16_t* W, const void* alpha_pre,
                                       const void* alpha_post, const void* alpha_res, const void* bias,
                                       const void* perm, int param_dtype, uint16_t* layer_input,
                                       uint16_t* proj, float* inv_rms, float* h_pre, float* h_post,
                                       float* H_merged, uint16_t* zero_word_a, uint16_t* zero_word_b,
                                       int64_t T, int64_t C, int64_t n, void* stream) {
  if (T < 0 || C <= 0 || n != 4) return FMHC_ERR_INVALID_ARGUMENT;
  if (T == 0) return FMHC_OK;
  const int64_t need = fmhc_premap_fwd_workspace_bytes(T, C);
  if (need > kNoAllocScratchBytes) return FMHC_ERR_SCRATCH_LIMIT;
  void* ws = nullptr;
  if (need > 0) {
    const int st = scratch_on_device(stream, &ws);
    if (st != FMHC_OK) return st;
  }
  return premap_fwd_run(x, W, alpha_pre, alpha_post, alpha_res, bias, perm, param_dtype, layer_input, proj,
                        inv_rms, h_pre, h_post, H_merged, zero_word_a, zero_word_b, ws,
                        need > 0 ? kNoAllocScratchBytes : 0, T, C, n, stream);
}

extern "C" int64_t fmhc_premap_bwd_workspace_bytes(int64_t T, int64_t C) {
  if (T <= 0 || C <= 0) return 0;
  return premap_ws(T, C).total;
}

extern "C" int fmhc_premap_bwd(const uint16_t* x, const uint16_t* W, const void* alpha_pre,
                               const void* alpha_post, const void* alpha_res, const void* bias,
                               const void* perm, int param_dtype, const float* h_pre, const uint16_t* proj,
                               const float* inv_rms, const uint16_t* grad_layer_input,
                               const float* grad_h_post, const float* grad_H_merged,
                               const uint16_t* grad_x_in, uint16_t* grad_x,
                               uint16_t* grad_W, void* grad_alpha_pre, void* grad_alpha_post,
                               void* grad_alpha_res, void* grad_bias, void* workspace,
                               int64_t workspace_bytes, int64_t T, int64_t C, int64_t n, void* stream) {
  using namespace fmhc;
  if (T < 0 || C <= 0 || C > (int64_t{1} << 24) || n != 4 || !param_dtype_ok(param_dtype))
    return FMHC_ERR_INVALID_ARGUMENT;
  if (!W || !alpha_pre || !alpha_post || !alpha_res || !bias || !perm || !grad_W || !grad_alpha_pre ||
      !grad_alpha_post || !grad_alpha_res || !grad_bias)
    return FMHC_ERR_INVALID_ARGUMENT;
  if (T > 0 && (!x || !h_pre || !proj || !inv_rms || !grad_layer_input || !grad_x)) return FMHC_ERR_INVALID_ARGUMENT;
  if (T > 0 && grad_x_in) {  // grad_x_in is read while grad_x is written: no overlap
    const auto a = reinterpret_cast<uintptr_t>(grad_x_in), b = reinterpret_cast<uintptr_t>(grad_x);
    const auto bytes = static_cast<uintptr_t>(T * n * C * 2);
    if (a < b + bytes && b < a + bytes) return FMHC_ERR_INVALID_ARGUMENT;
  }
  const PremapWs w = premap_ws(T, C);
  if (T > 0 && (!workspace || workspace_bytes < w.total || !aligned16(workspace))) return FMHC_ERR_INVALID_ARGUMENT;
  char* ws = static_cast<char*>(workspace);
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (FMHC_PREMAP_SPLIT && premap_split_ok(x, W, proj, inv_rms, grad_x, grad_layer_input, grad_x_in, T, C)) {
    K2Params P;
    if (!k2_params(alpha_pre, alpha_post, alpha_res, bias, perm, param_dtype, P)) return FMHC_ERR_INVALID_ARGUMENT;
    return premap_bwd_split(x, W, proj, inv_rms, grad_layer_input, h_pre, grad_h_post, grad_H_merged, grad_x_in,
                            grad_x, grad_W, P, grad_alpha_pre, grad_alpha_post, grad_alpha_res, grad_bias,
                            reinterpret_cast<float*>(ws + w.k2), reinterpret_cast<float*>(ws + w.k1), ws + w.ring, T,
                            C, s);
  }
  float* gh = T > 0 ? reinterpret_cast<float*>(ws + w.gh) : nullptr;
  uint16_t* gp = T > 0 ? reinterpret_cast<uint16_t*>(ws + w.gp) : nullptr;
  int st = FMHC_OK;
  const bool fused = T > 0 && k1_bwd_premap_fused(x, W, gp, proj, inv_rms, grad_x, grad_layer_input, grad_x_in, C);
  K2Params P;
  if (!k2_params(alpha_pre, alpha_post, alpha_res, bias, perm, param_dtype, P)) return FMHC_ERR_INVALID_ARGUMENT;
  // K2's backward, whose parameter partials K1's grad_W reduce also sums.
  K2ParamSums sums;
  const int lanes = C % 8 == 0 ? k3_bwd_lanes8(static_cast<int>(C)) : 0;
  if (fused && T <= kK2BwdSmallT && (lanes == 32 || lanes == 64) && aligned16(x) && aligned16(grad_layer_input)) {
    // Few tokens: K3's reduce-only pass and K2's backward as one kernel.
    float* partial = reinterpret_cast<float*>(ws + w.k2);
    const dim3 grid(static_cast<unsigned>((T + kK2BwdTok - 1) / kK2BwdTok));
    const bool canon = k3_canon(C, lanes);
    auto launch = [&](auto lpt_c, auto canon_c) {
      constexpr int L = decltype(lpt_c)::value;
      k3_reduce_k2_bwd<L, decltype(canon_c)::value><<<grid, kK2BwdTok * L, 0, s>>>(
          x, grad_layer_input, proj, P, grad_h_post, grad_H_merged, gp, partial, T, static_cast<int>(C));
    };
    using I64 = std::integral_constant<int, 64>;
    using I32 = std::integral_constant<int, 32>;
    if (lanes == 64)
      canon ? launch(I64{}, std::true_type{}) : launch(I64{}, std::false_type{});
    else
      canon ? launch(I32{}, std::true_type{}) : launch(I32{}, std::false_type{});
    st = launch_status();
    sums = K2ParamSums{partial, static_cast<int64_t>(grid.x), grad_alpha_pre, grad_alpha_post, grad_alpha_res,
                       grad_bias, P.bf16};
  } else {
    if (T > 0) st = fmhc_k3_bwd(x, h_pre, grad_layer_input, fused ? nullptr : grad_x, gh, T, C, n, stream);
    if (st == FMHC_OK)
      st = k2_bwd_partials(proj, P, gh, grad_h_post, grad_H_merged, gp, grad_alpha_pre, grad_alpha_post,
                           grad_alpha_res, grad_bias, T > 0 ? ws + w.k2 : nullptr, T > 0 ? w.k1 - w.k2 : 0, T, s,
                           &sums);
  }
  if (st == FMHC_OK)
    st = k1_bwd_premap(x, W, gp, proj, inv_rms, grad_layer_input, h_pre, grad_x_in, grad_x, grad_W,
                       T > 0 ? ws + w.k1 : nullptr, T > 0 ? w.total - w.k1 : 0, T, C, sums, s);
  return st;
}
