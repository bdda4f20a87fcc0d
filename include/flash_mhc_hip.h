/*
 * flash_mhc_hip.h -- C ABI of the MI355X (gfx950) mHC-lite K1/K3/K4 kernels.
 *
 * Each entry point replaces one Triton launch of the reference
 * (alint77/flash-mHC).  The Python layer (flash_mhc/ops.py) keeps the
 * reference's torch.library op names, schemas and autograd formulas and calls
 * these functions with raw device pointers.
 *
 * Conventions shared by every entry point:
 *   - Pointers are device pointers into contiguous, row-major buffers.
 *     bf16 tensors are passed as uint16_t bit patterns; fp32 as float.
 *   - Sizes are int64_t.  T == 0 is valid and launches nothing.
 *   - `stream` is a hipStream_t (NULL = the legacy default stream).  Work is
 *     enqueued asynchronously; nothing blocks the host.
 *   - The library allocates no memory.  It keeps no state between calls,
 *     except fmhc_premap_fwd_noalloc's static scratch array (below).
 *     Every element of every output is written.
 *   - n (streams per token) must be 4 and D_out (K1 projection width) must be
 *     32, matching the reference's n = 4 specialisation.
 *   - Fast paths move 16 bytes per lane and are taken when C % 8 == 0 and
 *     the bf16 pointers (for K1's backward also inv_rms) are 16-byte aligned;
 *     any other C or alignment takes an element-wise path, which gives the
 *     same values up to the order of fp32 sums.
 *   - Return value: FMHC_OK (0), or an FMHC_ERR_* code; for HIP runtime
 *     failures FMHC_ERR_HIP_BASE + hipError_t.  fmhc_error_string() names it.
 */
#ifndef FLASH_MHC_HIP_H_
#define FLASH_MHC_HIP_H_

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define FMHC_OK 0
#define FMHC_ERR_INVALID_ARGUMENT 1 /* negative size, n != 4, D_out != 32, null pointer */
#define FMHC_ERR_SCRATCH_LIMIT 2    /* fmhc_premap_fwd_noalloc: shape needs more than its scratch */
#define FMHC_ERR_HIP_BASE 1000      /* + hipError_t from the launch */

#define FMHC_ABI_VERSION 7

/* Storage dtype of the block parameters K2 reads (alpha_pre, alpha_post,
 * alpha_res, bias, perm: all five the same) and of their gradients. */
#define FMHC_PARAM_F32 0
#define FMHC_PARAM_BF16 1

/* K1 forward: fused RMSNorm + projection.
 *   inv_rms[t] = rsqrt(sum_k x[t,k]^2 / nC + 1e-6)
 *   out[t,d]   = bf16(inv_rms[t] * sum_k x[t,k] * W[d,k])   (fp32 accumulation)
 * x_flat (T, nC) bf16; W (D_out, nC) bf16; out (T, D_out) bf16; inv_rms (T,) fp32.
 * Replaces: src/flash_mhc/ops.py:205-264 (_fused_rmsnorm_project_cuda) launching
 *           src/flash_mhc/kernels.py:250-303 (_fused_rmsnorm_project_fwd_kernel). */
int fmhc_k1_fwd(const uint16_t* x_flat, const uint16_t* W, uint16_t* out, float* inv_rms,
                int64_t T, int64_t nC, int64_t D_out, void* stream);
/* fmhc_k1_fwd with a workspace: for few tokens (T <= 1024 up to nC = 4096,
 * T <= 2720 above) the nC axis is split
 * over up to 64 workgroups per 16-token block, whose fp32 partial sums (in
 * `workspace`) a second kernel adds in a fixed order.  `workspace`: at least
 * fmhc_k1_fwd_workspace_bytes(T, nC) bytes, 16-byte aligned (may be NULL when
 * that is 0).  Results equal fmhc_k1_fwd's up to fp32 summation order.  No
 * counterpart in the reference (its kernel has one program per token tile). */
int fmhc_k1_fwd_ws(const uint16_t* x_flat, const uint16_t* W, uint16_t* out, float* inv_rms,
                   void* workspace, int64_t workspace_bytes, int64_t T, int64_t nC, int64_t D_out,
                   void* stream);
int64_t fmhc_k1_fwd_workspace_bytes(int64_t T, int64_t nC);

/* K1 backward, grad of x_flat:
 *   scale[t]    = (sum_d go[t,d] * proj_out[t,d]) * inv_rms[t]^2 / nC
 *   grad_x[t,k] = bf16(inv_rms[t] * sum_d go[t,d] * W[d,k] - scale[t] * x[t,k])
 * grad_out, proj_out (T, D_out) bf16; inv_rms (T,) fp32; grad_x (T, nC) bf16.
 * Replaces: src/flash_mhc/ops.py:267-344 (_fused_rmsnorm_project_bwd_dx_cuda) launching
 *           src/flash_mhc/kernels.py:306-376 (_fused_rmsnorm_project_bwd_dx_kernel). */
int fmhc_k1_bwd_dx(const uint16_t* x_flat, const uint16_t* W, const uint16_t* grad_out,
                   const uint16_t* proj_out, const float* inv_rms, uint16_t* grad_x,
                   int64_t T, int64_t nC, int64_t D_out, void* stream);

/* K1 backward, grad of x_flat and of W in one pass over x:
 *   grad_x as fmhc_k1_bwd_dx;
 *   grad_W[d,k] = bf16(sum_t bf16(go[t,d] * inv_rms[t]) * x[t,k])   (fp32 accumulation)
 * grad_W (D_out, nC) bf16.  `workspace` is device memory of at least
 * fmhc_k1_bwd_workspace_bytes(T, nC) bytes, 16-byte aligned, for per-wave
 * partial sums (summed in a fixed order: results are deterministic).
 * Replaces: src/flash_mhc/ops.py:678-685 (_fused_rmsnorm_project_backward:
 *           the bwd_dx launch plus the grad_W torch.matmul, which reads x again). */
int fmhc_k1_bwd(const uint16_t* x_flat, const uint16_t* W, const uint16_t* grad_out,
                const uint16_t* proj_out, const float* inv_rms, uint16_t* grad_x, uint16_t* grad_W,
                void* workspace, int64_t workspace_bytes, int64_t T, int64_t nC, int64_t D_out,
                void* stream);

/* Workspace bytes fmhc_k1_bwd needs for (T, nC); 0 when none is needed.
 * No counterpart in the reference. */
int64_t fmhc_k1_bwd_workspace_bytes(int64_t T, int64_t nC);

/* K2 forward, the coefficient math of the fused path with the reference's bf16
 * rounding points (every intermediate rounded to bf16, as the reference's chain
 * of bf16 tensor ops does), per token t:
 *   h_pre[t,j]    = bf16(sigmoid(bf16(bf16(a_pre  * p[j])     + b[j])))
 *   h_post[t,j]   = bf16(2 * bf16(sigmoid(bf16(bf16(a_post * p[4+j]) + b[4+j]))))
 *   a[m]          = bf16(softmax_m(bf16(bf16(a_res * p[8+m]) + b[8+m])))
 *   H_merged[t,i,j] = bf16(bf16(sum_m a[m] perm[m, 4i+j]) - bf16(h_post[t,i] h_pre[t,j]))
 * with p = proj[t,:] (T, 32) bf16, a_* = bf16(alpha_*[0]), b = bf16(bias) (32,),
 * perm (24, 16) (the block's perm_mat), the five parameters in param_dtype
 * (FMHC_PARAM_F32 or FMHC_PARAM_BF16; rounded to bf16 on use either way, as
 * the reference's .to(bf16) does).  Outputs are fp32 (the values are
 * bf16), 16-byte aligned: h_pre (T, 4), h_post (T, 4), H_merged (T, 4, 4).
 * n must be 4.
 * Replaces: src/flash_mhc/block.py:161-170 (_mhc_coeffs_triton's PyTorch ops)
 *           and the .float() casts of block.py:176-177. */
int fmhc_k2_fwd(const uint16_t* proj, const void* alpha_pre, const void* alpha_post,
                const void* alpha_res, const void* bias, const void* perm, int param_dtype,
                float* h_pre, float* h_post, float* H_merged, int64_t T, int64_t n, void* stream);
/* K2 backward: autograd of the chain above with the rounding points of
 * PyTorch's GPU kernels (the incoming fp32 gradients are rounded to bf16 first,
 * as the .float() casts' backward does; the sigmoid and softmax backward steps
 * round their intermediate products to bf16 as the bf16 GPU kernels do:
 * rb(rb(g rb(1 - y)) y) and rb(gy - y sum(gy)), gy = rb(g y)).  grad_h_pre / grad_h_post / grad_H_merged may be NULL
 * (zero).  Writes grad_proj (T, 32) bf16 and the parameter gradients
 * grad_alpha_pre, grad_alpha_post, grad_alpha_res (one each) and grad_bias
 * (32), in param_dtype: sums over tokens, accumulated in fp32 in a fixed order
 * and rounded once to bf16.  `workspace`: at least
 * fmhc_k2_bwd_workspace_bytes(T) bytes of device memory for per-block partials.
 * Replaces: autograd through src/flash_mhc/block.py:161-170 and :176-177. */
int fmhc_k2_bwd(const uint16_t* proj, const void* alpha_pre, const void* alpha_post,
                const void* alpha_res, const void* bias, const void* perm, int param_dtype,
                const float* grad_h_pre, const float* grad_h_post, const float* grad_H_merged,
                uint16_t* grad_proj, void* grad_alpha_pre, void* grad_alpha_post,
                void* grad_alpha_res, void* grad_bias, void* workspace, int64_t workspace_bytes,
                int64_t T, int64_t n, void* stream);
/* Workspace bytes fmhc_k2_bwd needs for T tokens.  No counterpart in the reference. */
int64_t fmhc_k2_bwd_workspace_bytes(int64_t T);
/* Pre-map forward: K1, K2 and K3 of the same tokens (fmhc_k1_fwd_ws, fmhc_k2_fwd,
 * fmhc_k3_fwd in order, on `stream`; `workspace` as fmhc_k1_fwd_ws for n C).  Outputs: layer_input (T, C) bf16,
 * proj (T, 32) bf16, inv_rms (T,) fp32, h_pre, h_post (T, 4) and
 * H_merged (T, 4, 4) fp32 (16-byte aligned).  x (T, n, C) bf16, W (32, n C)
 * bf16, alphas / bias / perm / param_dtype as fmhc_k2_fwd; n must be 4.
 * layer_input may be NULL: K1 and K2 only (the coefficients), K3 skipped.
 * zero_word_a, zero_word_b: NULL, or 16-bit words the call also sets to zero
 * (inside K2's launch, for T > 0): the single stored element of a caller's
 * zero-stride placeholder tensor, which would otherwise need a fill of its own.
 * Replaces: src/flash_mhc/block.py:157-177 (_mhc_pre_map_triton: the K1 launch,
 *           the K2 PyTorch ops and the K3 launch). */
int fmhc_premap_fwd(const uint16_t* x, const uint16_t* W, const void* alpha_pre,
                    const void* alpha_post, const void* alpha_res, const void* bias,
                    const void* perm, int param_dtype, uint16_t* layer_input, uint16_t* proj,
                    float* inv_rms, float* h_pre, float* h_post, float* H_merged,
                    uint16_t* zero_word_a, uint16_t* zero_word_b, void* workspace,
                    int64_t workspace_bytes, int64_t T, int64_t C, int64_t n, void* stream);
/* Workspace bytes fmhc_premap_fwd needs (fmhc_k1_fwd_workspace_bytes(T, 4 C);
 * 0: workspace may be NULL).  No counterpart in the reference. */
int64_t fmhc_premap_fwd_workspace_bytes(int64_t T, int64_t C);
/* fmhc_premap_fwd without a workspace argument, allocating nothing: no
 * hipMalloc / hipFree or allocating library call on any path.  No counterpart
 * in the reference; it is for callers that cannot allocate device memory
 * (code under HIP graph capture, tight serving loops, harnesses that forbid
 * allocation).  The few-token forward's partial sums go to a static 4 MiB
 * device array of the library (one per device, held until the process ends),
 * which covers every shape (at most 2,145,792 bytes are needed, at T = 2032,
 * C = 1040); a shape needing more returns FMHC_ERR_SCRATCH_LIMIT.  The array's
 * device address is looked up on the first call on each device.  `stream`
 * must belong to the current device (else FMHC_ERR_INVALID_ARGUMENT).  Every
 * call on a device shares that device's array and overwrites what the last
 * call left there (every partial it reads was written by the same call, so
 * nothing needs clearing): calls that overlap on one device (on different
 * streams, or from several host threads without ordering) race.  Outputs
 * are bit-identical to fmhc_premap_fwd's. */
int fmhc_premap_fwd_noalloc(const uint16_t* x, const uint16_t* W, const void* alpha_pre,
                            const void* alpha_post, const void* alpha_res, const void* bias,
                            const void* perm, int param_dtype, uint16_t* layer_input, uint16_t* proj,
                            float* inv_rms, float* h_pre, float* h_post, float* H_merged,
                            uint16_t* zero_word_a, uint16_t* zero_word_b, int64_t T, int64_t C,
                            int64_t n, void* stream);
/* Pre-map backward: the gradients of fmhc_premap_fwd's inputs from those of
 * layer_input (T, C) bf16, h_post (T, 4) and H_merged (T, 4, 4) fp32 (the
 * latter two may be NULL: zero):
 *   grad_x = bf16(K3's h_pre[t,j] * grad_layer_input[t,c] + K1's dx)
 *            (each term rounded to bf16 first, as autograd sums them),
 *   grad_W (32, n C) bf16 as fmhc_k1_bwd, the alpha / bias gradients as
 *   fmhc_k2_bwd (in param_dtype).
 * grad_x_in (T, n, C) bf16 may be NULL; otherwise it is a further gradient of
 * x (in a block: post-res's H_merged^T grad_out) and
 *   grad_x = bf16(grad_x_in + the bf16 value above)
 * (autograd's sum of x's gradients).  It must not overlap grad_x.
 * h_pre, proj, inv_rms are fmhc_premap_fwd's outputs.  `workspace`: at least
 * fmhc_premap_bwd_workspace_bytes(T, C) bytes, 16-byte aligned.
 * Replaces: autograd through src/flash_mhc/block.py:157-177 (the K3, K2 and K1
 *           backward launches, and the addition of x's gradients). */
int fmhc_premap_bwd(const uint16_t* x, const uint16_t* W, const void* alpha_pre,
                    const void* alpha_post, const void* alpha_res, const void* bias,
                    const void* perm, int param_dtype, const float* h_pre, const uint16_t* proj,
                    const float* inv_rms, const uint16_t* grad_layer_input, const float* grad_h_post,
                    const float* grad_H_merged, const uint16_t* grad_x_in, uint16_t* grad_x,
                    uint16_t* grad_W, void* grad_alpha_pre, void* grad_alpha_post, void* grad_alpha_res,
                    void* grad_bias, void* workspace, int64_t workspace_bytes, int64_t T, int64_t C,
                    int64_t n, void* stream);
/* Workspace bytes fmhc_premap_bwd needs.  No counterpart in the reference. */
int64_t fmhc_premap_bwd_workspace_bytes(int64_t T, int64_t C);
/* K3 forward: out[t,c] = bf16(sum_j h_pre[t,j] * x[t,j,c]), j = 0..3 in order.
 * x (T, n, C) bf16; h_pre (T, n) fp32; out (T, C) bf16.
 * Replaces: src/flash_mhc/ops.py:347-414 (_fused_pre_map_cuda) launching
 *           src/flash_mhc/kernels.py:673-717 (_fused_pre_map_fwd_kernel). */
int fmhc_k3_fwd(const uint16_t* x, const float* h_pre, uint16_t* out,
                int64_t T, int64_t C, int64_t n, void* stream);

/* K3 backward:
 *   grad_x[t,j,c]   = bf16(h_pre[t,j] * go[t,c])
 *   grad_h_pre[t,j] = sum_c x[t,j,c] * go[t,c]              (fp32)
 * grad_out (T, C) bf16; grad_x (T, n, C) bf16; grad_h_pre (T, n) fp32.
 * grad_x may be NULL: then only grad_h_pre is computed (no counterpart in the
 * reference; the pre-map backward folds h_pre * go into K1's grad_x store).
 * Replaces: src/flash_mhc/ops.py:417-493 (_fused_pre_map_backward_cuda) launching
 *           src/flash_mhc/kernels.py:720-853 (_fused_pre_map_bwd_fused_kernel_n4). */
int fmhc_k3_bwd(const uint16_t* x, const float* h_pre, const uint16_t* grad_out,
                uint16_t* grad_x, float* grad_h_pre,
                int64_t T, int64_t C, int64_t n, void* stream);

/* K4 forward:
 *   out[t,i,c] = bf16(h_post[t,i] * lo[t,c] + sum_j H[t,i,j] * x[t,j,c])
 * x (T, n, C) bf16; lo (T, C) bf16; H (T, n, n) fp32; h_post (T, n) fp32;
 * out (T, n, C) bf16.
 * Replaces: src/flash_mhc/ops.py:496-567 (_fused_post_res_cuda) launching
 *           src/flash_mhc/kernels.py:384-481 (_fused_post_res_fwd_kernel_n4). */
int fmhc_k4_fwd(const uint16_t* x, const uint16_t* lo, const float* H, const float* h_post,
                uint16_t* out, int64_t T, int64_t C, int64_t n, void* stream);

/* K4 backward:
 *   grad_lo[t,c]   = bf16(sum_i h_post[t,i] * go[t,i,c])
 *   grad_hp[t,i]   = sum_c go[t,i,c] * lo[t,c]              (fp32)
 *   grad_H[t,i,j]  = sum_c go[t,i,c] * x[t,j,c]             (fp32)
 *   grad_x[t,j,c]  = bf16(sum_i H[t,i,j] * go[t,i,c])
 * grad_out (T, n, C) bf16; grad_x (T, n, C) bf16; grad_lo (T, C) bf16;
 * grad_H (T, n, n) fp32; grad_h_post (T, n) fp32.
 * Replaces: src/flash_mhc/ops.py:570-667 (_fused_post_res_backward_cuda) launching
 *           src/flash_mhc/kernels.py:487-665 (_fused_post_res_bwd_fused_kernel_n4). */
int fmhc_k4_bwd(const uint16_t* x, const uint16_t* lo, const float* H, const float* h_post,
                const uint16_t* grad_out, uint16_t* grad_x, uint16_t* grad_lo,
                float* grad_H, float* grad_h_post,
                int64_t T, int64_t C, int64_t n, void* stream);

/* Human-readable text for a status code.  Never returns NULL.
 * No counterpart in the reference (Triton raises Python exceptions). */
const char* fmhc_error_string(int status);

/* FMHC_ABI_VERSION of the built library.  No counterpart in the reference. */
int fmhc_abi_version(void);

#ifdef __cplusplus
}
#endif

#endif /* FLASH_MHC_HIP_H_ */
