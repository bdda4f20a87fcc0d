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
// Forward: K1 -> K2 -> K3, the three kernels of k1.hip, k2.hip, k3.hip (K1
// split over the columns for few tokens, with the caller's workspace).  A
// one-pass variant that kept each token tile of x in LDS between K1 and K3
// (saving K3's read of x) was built and measured slower on gfx950 at
// C <= 1024: with tiles of 8-16 tokens every tile re-reads the whole of W
// (32 x nC) from L2, and holding a wave's share of W in registers instead
// does not fit beside the tile pipeline (register spills), whereas K1
// amortises W over 128 tokens per workgroup.

#include <hip/hip_runtime.h>

#include "flash_mhc_hip.h"
#include "fmhc_common.h"
#include "k1_premap.h"

namespace {

constexpr int64_t kAlign = 256;
int64_t round_up(int64_t v) { return (v + kAlign - 1) / kAlign * kAlign; }

// Checked before the first launch, so that a bad dtype leaves no partial outputs.
bool param_dtype_ok(int d) { return d == FMHC_PARAM_F32 || d == FMHC_PARAM_BF16; }

struct PremapWs {
  int64_t gh, gp, k2, k1, total;  // byte offsets / sizes
};

PremapWs premap_ws(int64_t T, int64_t C) {
  PremapWs w;
  w.gh = 0;                                     // grad_h_pre (T, 4) fp32
  w.gp = round_up(T * 4 * 4);                   // grad_proj (T, 32) bf16
  w.k2 = w.gp + round_up(T * 32 * 2);           // K2 parameter partials
  w.k1 = w.k2 + round_up(fmhc_k2_bwd_workspace_bytes(T));  // K1 grad_W partials
  w.total = w.k1 + round_up(fmhc_k1_bwd_workspace_bytes(T, 4 * C));
  return w;
}

}  // namespace

extern "C" int64_t fmhc_premap_fwd_workspace_bytes(int64_t T, int64_t C) {
  if (T <= 0 || C <= 0) return 0;
  return fmhc_k1_fwd_workspace_bytes(T, 4 * C);
}

extern "C" int fmhc_premap_fwd(const uint16_t* x, const uint16_t* W, const void* alpha_pre,
                               const void* alpha_post, const void* alpha_res, const void* bias,
                               const void* perm, int param_dtype, uint16_t* layer_input, uint16_t* proj,
                               float* inv_rms, float* h_pre, float* h_post, float* H_merged,
                               void* workspace, int64_t workspace_bytes, int64_t T, int64_t C, int64_t n,
                               void* stream) {
  if (T < 0 || C <= 0 || n != 4 || !param_dtype_ok(param_dtype)) return FMHC_ERR_INVALID_ARGUMENT;
  if (T == 0) return FMHC_OK;
  if (!x || !W || !alpha_pre || !alpha_post || !alpha_res || !bias || !perm || !layer_input || !proj ||
      !inv_rms || !h_pre || !h_post || !H_merged)
    return FMHC_ERR_INVALID_ARGUMENT;
  int st = fmhc_k1_fwd_ws(x, W, proj, inv_rms, workspace, workspace_bytes, T, n * C, 32, stream);
  if (st == FMHC_OK)
    st = fmhc_k2_fwd(proj, alpha_pre, alpha_post, alpha_res, bias, perm, param_dtype, h_pre, h_post, H_merged, T,
                     n, stream);
  if (st == FMHC_OK) st = fmhc_k3_fwd(x, h_pre, layer_input, T, C, n, stream);
  return st;
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
  float* gh = T > 0 ? reinterpret_cast<float*>(ws + w.gh) : nullptr;
  uint16_t* gp = T > 0 ? reinterpret_cast<uint16_t*>(ws + w.gp) : nullptr;
  int st = FMHC_OK;
  const bool fused = T > 0 && k1_bwd_premap_fused(x, W, gp, proj, grad_x, grad_layer_input, grad_x_in, C);
  if (T > 0) st = fmhc_k3_bwd(x, h_pre, grad_layer_input, fused ? nullptr : grad_x, gh, T, C, n, stream);
  if (st == FMHC_OK)
    st = fmhc_k2_bwd(proj, alpha_pre, alpha_post, alpha_res, bias, perm, param_dtype, gh, grad_h_post,
                     grad_H_merged, gp,
                     grad_alpha_pre, grad_alpha_post, grad_alpha_res, grad_bias, T > 0 ? ws + w.k2 : nullptr,
                     T > 0 ? w.k1 - w.k2 : 0, T, n, stream);
  if (st == FMHC_OK)
    st = k1_bwd_premap(x, W, gp, proj, inv_rms, grad_layer_input, h_pre, grad_x_in, grad_x, grad_W,
                       T > 0 ? ws + w.k1 : nullptr, T > 0 ? w.total - w.k1 : 0, T, C, s);
  return st;
}
