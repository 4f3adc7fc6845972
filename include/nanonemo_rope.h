/*
 * nanonemo_rope.h — C ABI of the MI355X (gfx950) rotary-position-embedding kernel for q and k
 * (libnanonemo_fa.so, built from nanonemo_amd/csrc/rope.hip).
 *
 * Rotate-half RoPE of /root/reference/nanonemo/model/layers.py:67-74 (apply_rope), applied to q and
 * k in one launch in the (B, T, heads, head_dim) projection layout, as the reference's fused Triton
 * kernel does (/root/reference/nanonemo/kernels/triton/rope.py). For row x at position t and
 * i < D/2:  y[i] = x[i] cos[t][i] - x[i + D/2] sin[t][i],  y[i + D/2] = x[i] sin[t][i] + x[i + D/2] cos[t][i],
 * in fp32 with one rounding per product and per sum (bit-identical to the reference's torch ops),
 * rounded once to the tensor's dtype.
 *
 *   - q: [B][T][H][D], k: [B][T][KVH][D] views with element strides {batch, position, head}
 *     (positive multiples of 8) and unit D stride, 16-byte aligned; outputs use the same strides as
 *     their inputs (in place is allowed: out == in). D is a multiple of 16.
 *   - cos_table, sin_table: dense fp32 [table_rows][D/2], table_rows >= T, 16-byte aligned.
 *   - dtype: 0 = fp16, 1 = bf16, 2 = fp32; q and k share it.
 *   - Enqueued on `stream` (a hipStream_t); nothing is allocated, synchronised or read back.
 *   - Returns 0 on success, non-zero on an argument error or a failed launch; the message is in
 *     nn_rope_last_error() (thread-local).
 */
#ifndef NANONEMO_ROPE_H
#define NANONEMO_ROPE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Forward rotation. Replaces apply_rope (layers.py:67-74) on q and k, and the reference's fused
 * Triton apply_rope_qk (nanonemo/kernels/triton/rope.py) used at layers.py:99-101. */
int nn_rope_qk(const void* q, void* q_out, const void* k, void* k_out,
               const float* cos_table, const float* sin_table,
               int64_t B, int64_t T, int64_t H, int64_t KVH, int64_t D,
               const int64_t q_strides[3], const int64_t k_strides[3], int64_t table_rows,
               int dtype, void* stream);

/* Backward: the gradient of the rotation, i.e. the rotation by -theta of the incoming gradients
 * (the autograd of apply_rope in the reference). */
int nn_rope_qk_bwd(const void* dq_out, void* dq, const void* dk_out, void* dk,
                   const float* cos_table, const float* sin_table,
                   int64_t B, int64_t T, int64_t H, int64_t KVH, int64_t D,
                   const int64_t q_strides[3], const int64_t k_strides[3], int64_t table_rows,
                   int dtype, void* stream);

/* Message of the last failed call on this thread ("" if none). */
const char* nn_rope_last_error(void);

#ifdef __cplusplus
}
#endif

#endif /* NANONEMO_ROPE_H */
