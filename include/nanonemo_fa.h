/*
 * nanonemo_fa.h — C ABI of the MI355X (gfx950) causal grouped-query FlashAttention-2 library
 * (libnanonemo_fa.so, built from nanonemo_amd/csrc/flash_attn.hip).
 *
 * Contract shared by every entry point:
 *   - Tensors are dense, contiguous, row-major device buffers:
 *       q, o, dO, dq   [B, H,   T, D]   16-bit (dtype code below)
 *       k, v, dk, dv   [B, KVH, T, D]   16-bit
 *       lse            [B, H,   T]      fp32, natural-log logsumexp of the scaled scores
 *   - Query head h reads KV head h / (H / KVH) (the order of repeat_interleave over heads).
 *   - Causal, top-left aligned, square: key j is visible to query i iff j <= i.
 *   - dtype: 0 = fp16, 1 = bf16. Operands are multiplied on MFMA with fp32 accumulation;
 *     softmax statistics are fp32.
 *   - D must be 32 or 64; H % KVH == 0; every pointer 16-byte aligned.
 *   - `stream` is a hipStream_t (may be NULL for the default stream). Work is only enqueued:
 *     no entry point allocates, frees, synchronises or reads device memory back to the host,
 *     so every call may be captured into a HIP graph.
 *   - Return value: 0 on success. Non-zero is an argument error (-1) or the hipError_t of a
 *     failed launch; nn_fa_last_error() then returns the message (thread-local).
 */
#ifndef NANONEMO_FA_H
#define NANONEMO_FA_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Forward: o = softmax(scale * q k^T + causal mask) v and lse per query row.
 * Replaces the pybind `fwd(q, k, v) -> (o, lse)` of
 * /root/reference/nanonemo/kernels/cuda/flash_attn.cu:362-379 (kernel :52-174),
 * bound at /root/reference/nanonemo/kernels/cuda/flash_attn.py:18-22. */
int nn_fa_fwd(const void* q, const void* k, const void* v, void* o, float* lse,
              int64_t B, int64_t H, int64_t KVH, int64_t T, int64_t D,
              int dtype, float scale, void* stream);

/* Forward on strided views: as nn_fa_fwd, but q and o are read / written through the element
 * strides qo_strides = {batch, head, row} of a [B, H, T, D] view, and k, v through kv_strides of
 * a [B, KVH, T, D] view (the D stride is 1 in both). Every stride is a positive multiple of 8
 * elements and rows are at least D apart. With the (B, T, heads, D) layout that the model's
 * projections produce ({T*H*D, D, H*D} and {T*KVH*D, D, KVH*D}), q, k and v are consumed and o is
 * produced in place, so the transposes and .contiguous() copies of
 * /root/reference/nanonemo/model/layers.py:97-104,116 and
 * /root/reference/nanonemo/kernels/cuda/flash_attn.py:20 disappear. lse stays dense [B, H, T]. */
int nn_fa_fwd_strided(const void* q, const void* k, const void* v, void* o, float* lse,
                      int64_t B, int64_t H, int64_t KVH, int64_t T, int64_t D,
                      const int64_t qo_strides[3], const int64_t kv_strides[3],
                      int dtype, float scale, void* stream);

/* Bytes of device workspace the backward needs: -rowsum(dO * o) and -lse / scale, one fp32 each
 * per query row, and, for shapes whose B * KVH * ceil(T / 128) dK/dV work units are too few to fill
 * the chip (under 256), split partials of dk and dv: S * 2 * B * KVH * T * D fp32 with
 * S = min(16, ceil(256 / units), (H / KVH) * (ceil(T / 64) + 1) / 8) and S >= 1 (every split keeps
 * at least 8 of a unit pair's iterations), or S = 1 when (H / KVH) * ceil(T / 64) * 16 reaches 2^31.
 * The caller allocates the size returned here, 256-byte aligned; its contents on entry do not matter. */
size_t nn_fa_bwd_workspace_size(int64_t B, int64_t H, int64_t KVH, int64_t T, int64_t D);

/* Backward: (dq, dk, dv) in the input dtype, contiguous. dk/dv hold the sum over the
 * H / KVH query heads that share each KV head. Runs nn_fa_bwd_dq (which also performs the
 * preprocessing pass into the workspace) and then nn_fa_bwd_dkdv on `stream`. Deterministic:
 * no atomics.
 * Replaces the pybind `bwd(d_o, q, k, v, o, lse) -> (dq, dk, dv)` of
 * /root/reference/nanonemo/kernels/cuda/flash_attn.cu:381-405 (kernel :176-340),
 * bound at /root/reference/nanonemo/kernels/cuda/flash_attn.py:31-35. */
int nn_fa_bwd(const void* dO, const void* q, const void* k, const void* v, const void* o,
              const float* lse, void* dq, void* dk, void* dv,
              void* workspace, size_t workspace_bytes,
              int64_t B, int64_t H, int64_t KVH, int64_t T, int64_t D,
              int dtype, float scale, void* stream);

/* Backward on strided views: as nn_fa_bwd, with dO, q, o and dq through qo_strides and k, v, dk
 * and dv through kv_strides (see nn_fa_fwd_strided). Replaces the .contiguous() copies of
 * /root/reference/nanonemo/kernels/cuda/flash_attn.py:33 and the transposes of the gradients. */
int nn_fa_bwd_strided(const void* dO, const void* q, const void* k, const void* v, const void* o,
                      const float* lse, void* dq, void* dk, void* dv,
                      void* workspace, size_t workspace_bytes,
                      int64_t B, int64_t H, int64_t KVH, int64_t T, int64_t D,
                      const int64_t qo_strides[3], const int64_t kv_strides[3],
                      int dtype, float scale, void* stream);

/* Forward with the rotary position embedding of q folded in: as nn_fa_fwd_strided, with q holding the
 * projections *before* RoPE. Each query row is rotated in registers (rotate-half, dimension i paired with
 * i + D/2, angle of the row's position: y[i] = x[i] cos - x[i+D/2] sin, y[i+D/2] = x[i] sin + x[i+D/2] cos,
 * one fp32 rounding per product and sum, then one to the 16-bit type), used for the scores, and written to
 * q_rot (q's layout) for the backward. cos_table / sin_table are dense fp32 [table_rows][D/2] with
 * table_rows >= T, 16-byte aligned. k must already be rotated (nn_rope_qk with H = 0 rotates k alone).
 * o, lse and q_rot are bit-identical to nn_rope_qk followed by nn_fa_fwd_strided. Replaces the q half of
 * the RoPE call beside the op, /root/reference/nanonemo/model/layers.py:99-101 (apply_rope_qk of
 * nanonemo/kernels/triton/rope.py), and the op's forward, flash_attn.py:18-22. */
int nn_fa_fwd_rope_strided(const void* q, const void* k, const void* v, void* o, float* lse, void* q_rot,
                           const float* cos_table, const float* sin_table, int64_t table_rows,
                           int64_t B, int64_t H, int64_t KVH, int64_t T, int64_t D,
                           const int64_t qo_strides[3], const int64_t kv_strides[3],
                           int dtype, float scale, void* stream);

/* Backward of nn_fa_fwd_rope_strided: as nn_fa_bwd_strided on q_rot, except that dq is the gradient of the
 * *unrotated* q: the gradient reaching q_rot, rounded to the 16-bit type, rotated by -theta in the dQ kernel
 * before its store. dk and dv are the gradients of the rotated k and of v. Bit-identical to
 * nn_fa_bwd_strided followed by nn_rope_qk_bwd on dq. Replaces the op's backward (flash_attn.py:31-35) and
 * the q half of RoPE's backward. */
int nn_fa_bwd_rope_strided(const void* dO, const void* q_rot, const void* k, const void* v, const void* o,
                           const float* lse, void* dq, void* dk, void* dv,
                           void* workspace, size_t workspace_bytes,
                           const float* cos_table, const float* sin_table, int64_t table_rows,
                           int64_t B, int64_t H, int64_t KVH, int64_t T, int64_t D,
                           const int64_t qo_strides[3], const int64_t kv_strides[3],
                           int dtype, float scale, void* stream);

/* Backward preprocessing alone: -D = -rowsum(dO * o) and -lse / scale, fp32, into the workspace.
 * Replaces the ATen preprocessing inside flash_bwd, flash_attn.cu:387-391. nn_fa_bwd does not call
 * it (nn_fa_bwd_dq performs the same pass in its prologue); it prepares the workspace for a caller
 * that runs nn_fa_bwd_dkdv on its own. */
int nn_fa_bwd_pre(const void* o, const void* dO, const float* lse, void* workspace, size_t workspace_bytes,
                  int64_t B, int64_t H, int64_t KVH, int64_t T, int64_t D, int dtype, float scale,
                  void* stream);

/* Backward, dk and dv (keys outer; recomputes P from the workspace's -lse/scale and uses its -D).
 * Needs the workspace prepared by nn_fa_bwd_dq or nn_fa_bwd_pre. When the shape splits the dK/dV
 * work (see nn_fa_bwd_workspace_size), it writes the split partials into the workspace and sums them
 * in a fixed order (deterministic). Together with nn_fa_bwd_dq it replaces bwd_kernel<HD>,
 * flash_attn.cu:176-340 with its launch at :393-401 and the casts at :404. */
int nn_fa_bwd_dkdv(const void* q, const void* k, const void* v, const void* dO,
                   void* workspace, size_t workspace_bytes, void* dk, void* dv,
                   int64_t B, int64_t H, int64_t KVH, int64_t T, int64_t D,
                   int dtype, float scale, void* stream);

/* Backward, dq (queries outer). Also computes -D = -rowsum(dO * o) and -lse / scale for its rows
 * and writes them into the workspace (the preprocessing pass of flash_attn.cu:387-391, fused), so
 * nn_fa_bwd_dkdv can run after it. */
int nn_fa_bwd_dq(const void* q, const void* k, const void* v, const void* o, const void* dO,
                 const float* lse, void* workspace, size_t workspace_bytes, void* dq,
                 int64_t B, int64_t H, int64_t KVH, int64_t T, int64_t D,
                 int dtype, float scale, void* stream);

/* Backward that allocates nothing: as nn_fa_bwd, with the workspace taken from a 32 MiB device array
 * inside the library (one per GPU, held until the process ends) instead of a caller buffer. No
 * counterpart in the reference: it is for callers that cannot allocate (code under HIP-graph capture,
 * tight serving loops, harnesses that forbid hipMalloc). Shapes whose nn_fa_bwd_workspace_size exceeds
 * 32 MiB (33554432 bytes; e.g. B * H * T above 4M query rows) are rejected with an error. The current
 * device must own `stream`; the first call on a device looks the array up (hipGetSymbolAddress, which may
 * load the library's code object), no call allocates or frees. Code that captures it into a HIP graph
 * makes one non-empty call on that device before the capture begins (an empty call, B = 0 or T = 0,
 * returns before the lookup). Calls that overlap on one GPU (other streams or threads) share the array
 * and race; calls in one stream's order do not. */
int nn_fa_bwd_noalloc(const void* dO, const void* q, const void* k, const void* v, const void* o,
                      const float* lse, void* dq, void* dk, void* dv,
                      int64_t B, int64_t H, int64_t KVH, int64_t T, int64_t D,
                      int dtype, float scale, void* stream);

/* The backward's dK/dV launch plan for a shape, computed on the host (no GPU, no allocation), for inspection
 * and tests: *nsplit blocks share each unit pair's iterations (above 1: fp32 partials in the workspace and a
 * sum kernel), *waves waves share a pair (or a unit), *paired is 1 when a block takes a pair of 64-key
 * units (j and nkb - 1 - j) and 0 when it takes single units (small unsplit problems), *blocks is the grid.
 * Returns 0, or nonzero with nn_fa_last_error set for sizes the library rejects. No counterpart in the
 * reference (its backward launch, flash_attn.cu:393-401, has one fixed grid). */
int nn_fa_bwd_plan(int64_t B, int64_t H, int64_t KVH, int64_t T, int* nsplit, int* waves, int* paired,
                   int64_t* blocks);

/* Message of the last failed call on this thread ("" if none). Replaces the TORCH_CHECK
 * messages of flash_attn.cu:342-356 and :383-385. */
const char* nn_fa_last_error(void);

/* ABI version of this header (bumped on any signature change). */
int nn_fa_abi_version(void);

#ifdef __cplusplus
}
#endif

#endif /* NANONEMO_FA_H */
