/*
 * nanonemo_rmsnorm.h — C ABI of the MI355X (gfx950) fused residual add + RMSNorm
 * (libnanonemo_fa.so, built from nanonemo_amd/csrc/rmsnorm.hip).
 *
 * The normalisation on either side of attention in every block: /root/reference/nanonemo/model/
 * layers.py:19-56 (RMSNorm, AddRMSNorm) and the reference's fused kernel
 * /root/reference/nanonemo/kernels/cuda/rmsnorm.cu (fwd :183-218, bwd :222-271), whose pybind
 * entry points these replace:
 *     h = x + delta (rounded to h's dtype),  y = (h * rstd) * w,  rstd = 1 / sqrt(mean(h^2) + eps)
 * backward, with n = h * rstd and dn = dy * w:
 *     dx = ddelta = rstd * (dn - n * mean(dn * n)) + dh,   dw = sum over rows of dy * n.
 *
 *   - x, delta, y, h, dy, dh, dx, ddelta: dense row-major [M][N]; weight, dw: fp32 [N]; rstd: fp32 [M].
 *   - dtype codes: 0 = fp16, 1 = bf16, 2 = fp32 (the reference takes fp32 / fp16; bf16 is added).
 *     h's dtype is the promotion of x's and delta's: fp32 if either is fp32 or they differ, else theirs.
 *   - delta == NULL: y = rmsnorm(x) and h is not written (the residual is x itself); in the backward,
 *     dh == NULL and ddelta is not written, and h is x.
 *   - N a multiple of 8 up to 4096 (pointers 16-byte aligned), or any N up to 1024 (the reference's limits).
 *   - Enqueued on `stream` (a hipStream_t); nothing is allocated, synchronised or read back, and no
 *     memset is issued, so calls may be captured into a HIP graph.
 *   - Returns 0 on success, non-zero on an argument error or a failed launch; the message is in
 *     nn_rmsnorm_last_error() (thread-local).
 */
#ifndef NANONEMO_RMSNORM_H
#define NANONEMO_RMSNORM_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Forward: (y, h, rstd). Replaces fwd(x, delta, weight, eps, out_dtype) of rmsnorm.cu:183-218,
 * bound as nanonemo::cuda_add_rms_norm_fwd at /root/reference/nanonemo/kernels/cuda/rmsnorm.py:17-22. */
int nn_add_rmsnorm_fwd(const void* x, const void* delta, const float* weight,
                       void* y, void* h, float* rstd,
                       int64_t M, int64_t N, float eps,
                       int x_dtype, int delta_dtype, int y_dtype, void* stream);

/* Bytes of fp32 workspace the backward needs for its per-block dw partials. */
size_t nn_add_rmsnorm_bwd_workspace_size(int64_t M, int64_t N);

/* Backward: dx (and ddelta, the same values in its dtype) and dw, written (not accumulated).
 * Replaces bwd(dy, dh, h, weight, rstd, dx_dtype, ddelta_dtype) of rmsnorm.cu:222-271 (with its
 * host-side dw_partial.sum(0)), bound as nanonemo::cuda_add_rms_norm_bwd at rmsnorm.py:31-38.
 * M == 0 writes dw = 0. */
int nn_add_rmsnorm_bwd(const void* dy, const void* dh, const void* h, const float* weight, const float* rstd,
                       void* dx, void* ddelta, float* dw, void* workspace, size_t workspace_bytes,
                       int64_t M, int64_t N, int dy_dtype, int h_dtype, int dx_dtype, int ddelta_dtype,
                       void* stream);

/* Message of the last failed call on this thread ("" if none). */
const char* nn_rmsnorm_last_error(void);

#ifdef __cplusplus
}
#endif

#endif /* NANONEMO_RMSNORM_H */
