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
 *   - The library allocates no memory and keeps no state between calls.
 *     Every element of every output is written.
 *   - n (streams per token) must be 4 and D_out (K1 projection width) must be
 *     32, matching the reference's n = 4 specialisation.
 *   - Fast paths move 16 bytes per lane and are taken when C % 8 == 0 and
 *     the bf16 pointers are 16-byte aligned; any other C or alignment takes an
 *     element-wise path with identical results.
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
#define FMHC_ERR_HIP_BASE 1000      /* + hipError_t from the launch */

#define FMHC_ABI_VERSION 1

/* K1 forward: fused RMSNorm + projection.
 *   inv_rms[t] = rsqrt(sum_k x[t,k]^2 / nC + 1e-6)
 *   out[t,d]   = bf16(inv_rms[t] * sum_k x[t,k] * W[d,k])   (fp32 accumulation)
 * x_flat (T, nC) bf16; W (D_out, nC) bf16; out (T, D_out) bf16; inv_rms (T,) fp32.
 * Replaces: src/flash_mhc/ops.py:205-264 (_fused_rmsnorm_project_cuda) launching
 *           src/flash_mhc/kernels.py:250-303 (_fused_rmsnorm_project_fwd_kernel). */
int fmhc_k1_fwd(const uint16_t* x_flat, const uint16_t* W, uint16_t* out, float* inv_rms,
                int64_t T, int64_t nC, int64_t D_out, void* stream);

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
