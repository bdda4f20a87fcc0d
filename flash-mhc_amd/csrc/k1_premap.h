// K1 and K2 pieces used by the pre-map region (premap.hip); defined in k1.hip and k2.hip.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "k2_chain.h"

namespace fmhc {

constexpr float kRmsEps = 1e-6f;  // K1's RMSNorm epsilon (kernels.py:296 of the reference)

// The first kernel of K1's column-split forward alone: when T tokens take that
// path (few tokens, MFMA-eligible pointers) it writes the fp32 partial sums to
// `ws` as part[t][33][S4] (32 projections, then the sum of squares; S4 = S
// rounded up to 4) and returns the number of splits S >= 2; it returns 0 when
// the tokens do not take that path and -status on an error.  The second stage
// (k1_fwd_finish in k1.hip) adds the S partials of each value in split order.
// Outputs of the pre-map tile kernel beyond K1's (k1_fwd_mfma with TILE):
// K2's parameters and outputs, and the layer input (null: K1 + K2 only).
struct PremapTile {
  K2Params P{};
  float* h_pre = nullptr;
  float* h_post = nullptr;
  float* H = nullptr;
  uint16_t* layer_input = nullptr;
  int C = 0;
  ZeroWords z{};
};

// The pre-map forward as one kernel, when T takes K1's one-pass forward (no
// column split planned) and the shapes allow (C % 8 == 0, 16-byte aligned x /
// W / proj / layer_input): K1 on tiles of 16 to 64 tokens, then K2 and K3 on
// each tile by the same workgroup.  Returns false (nothing launched) when
// they do not; otherwise launches and returns true with *status set.
bool k1_premap_tile(const uint16_t* x, const uint16_t* W, uint16_t* proj, float* inv_rms, const PremapTile& pt,
                    int64_t T, int64_t C, hipStream_t s, int* status);

// The pre-map forward with one read of x for rows of C = 512 or 1024 per
// stream (premap_resident.hip): W resident on each CU, a 16-token block of
// rows in registers from K1 to K3.  Returns false (nothing launched) when the
// shape, token count (below kResidentMinT), layer input or alignment does not
// allow it.  Against the tile kernel, each launch after a cache flush:
// C = 1024, T = 16384 47-48 against 51 us, 24576 61 against 72-73, 32768
// 76.4 against 91.2, 65536 136-139 against 174, 131072 258 against 335;
// C = 512, T = 16384 27.6 against 31.5, 24576 35.0 against 42.9, 65536 72-73
// against 94.  At T = 8192 it loses (31.1 against 30.0 us at C = 1024): too
// few blocks per CU to pay for loading W.
constexpr int64_t kResidentMinT = 16384;
bool premap_resident(const uint16_t* x, const uint16_t* W, uint16_t* proj, float* inv_rms, const PremapTile& pt,
                     int64_t T, int64_t C, hipStream_t s, int* status);

int k1_fwd_partials(const uint16_t* x_flat, const uint16_t* W, void* ws, int64_t ws_bytes, int64_t T,
                    int64_t nC, hipStream_t s);

// True when k1_bwd_premap computes the K3 term of grad_x itself (MFMA path);
// otherwise grad_x must hold it on entry.  gi: the incoming gradient or null.
bool k1_bwd_premap_fused(const void* x, const void* W, const void* go, const void* proj, const void* inv_rms,
                         const void* gx, const void* go3, const void* gi, int64_t C);

// grad_W (32, 4C) and grad_x = bf16(bf16(h_pre[t, j] go3[t, c]) + bf16(dx)) of
// K1 for x (T, 4, C); with grad_x_in (may be null, must not overlap grad_x)
// grad_x = bf16(grad_x_in + that).  `workspace` as fmhc_k1_bwd
// (fmhc_k1_bwd_workspace_bytes(T, 4C)).  K2's parameter gradients
// (k2_bwd_partials) are summed by the same launch as grad_W's partials.
int k1_bwd_premap(const uint16_t* x_flat, const uint16_t* W, const uint16_t* grad_proj,
                  const uint16_t* proj, const float* inv_rms, const uint16_t* go3, const float* h_pre,
                  const uint16_t* grad_x_in, uint16_t* grad_x, uint16_t* grad_W, void* workspace,
                  int64_t workspace_bytes, int64_t T, int64_t C, const K2ParamSums& k2_sums, hipStream_t s);

// fmhc_k2_bwd without its last launch: K2's backward writes grad_proj and the
// per-workgroup parameter partials, and *sums describes what remains to sum
// (k2_param_sum; launch_k2_param_reduce, or folded into another launch).
int k2_bwd_partials(const uint16_t* proj, const K2Params& P, const float* grad_h_pre, const float* grad_h_post,
                    const float* grad_H_merged, uint16_t* grad_proj, void* grad_alpha_pre, void* grad_alpha_post,
                    void* grad_alpha_res, void* grad_bias, void* workspace, int64_t workspace_bytes, int64_t T,
                    hipStream_t s, K2ParamSums* sums);
void launch_k2_param_reduce(const K2ParamSums& sums, hipStream_t s);

// Lanes per token of K3's backward (fmhc_k3_bwd) on its 16-byte path.
int k3_bwd_lanes8(int C);

// The grad_W backward's runs (k1_bwd_mfma<true, ...>) for T tokens and nC
// columns, and the reduce of its per-run partials into grad_W (32, nC) bf16
// plus, in extra workgroups, K2's parameter gradients from `sums`
// (k1_dw_reduce, k1.hip).
int64_t k1_bwd_dw_runs(int64_t T, int64_t nC);
int k1_dw_finish(const float* partial, uint16_t* grad_W, int64_t nruns, int nslices, int nC,
                 const K2ParamSums& sums, hipStream_t s);

// The pre-map backward with one read of x (premap_split.hip), for many tokens
// (T >= kSplitMinT) and C a multiple of 128 with the MFMA path's alignments.
constexpr int64_t kSplitMinT = 16384;
bool premap_split_ok(const void* x, const void* W, const void* proj, const void* inv_rms, const void* gx,
                     const void* go3, const void* gi, int64_t T, int64_t C);
// Bytes of its exchange ring (zeroed by the call itself).
int64_t premap_split_ring_bytes(int64_t T, int64_t C);
// grad_x, grad_W and K2's parameter gradients as the three-kernel backward
// gives them.  k2_partial: ceil(T / 16) x kNPar floats; dw_partial:
// fmhc_k1_bwd_workspace_bytes(T, 4 C) bytes; ring: premap_split_ring_bytes.
int premap_bwd_split(const uint16_t* x, const uint16_t* W, const uint16_t* proj, const float* inv_rms,
                     const uint16_t* go3, const float* h_pre, const float* grad_h_post, const float* grad_H,
                     const uint16_t* grad_x_in, uint16_t* grad_x, uint16_t* grad_W, const K2Params& P,
                     void* grad_alpha_pre, void* grad_alpha_post, void* grad_alpha_res, void* grad_bias,
                     float* k2_partial, float* dw_partial, void* ring, int64_t T, int64_t C, hipStream_t s);

}  // namespace fmhc
