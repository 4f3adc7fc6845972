// Causal grouped-query FlashAttention-2, forward and backward, for MI355X (gfx950, CDNA4).
//
// Semantics follow /root/reference/nanonemo/kernels/cuda/flash_attn.cu (fwd_kernel :52-174,
// bwd_kernel :176-340, host wrappers :342-405); the design is written for CDNA4 wave64 + MFMA:
//
//   * All products run on v_mfma_f32_32x32x16_{bf16,f16} with fp32 accumulators in VGPRs. One
//     wave owns a 32-wide slab of the sequence dimension; LDS holds tiles shared by the block.
//   * Tiles move global -> LDS with buffer_load_dwordx4 ... lds (no staging registers; the scalar
//     buffer descriptor ends at row T - 1, so rows past it read as zeros) into row-major tiles
//     whose 16-byte chunks are XOR-swizzled by row. Operands that need a
//     row of a tile are read with ds_read_b128; operands that need a column (the transposed
//     products) are read with ds_read_b64_tr_b16, so no transposed copy is ever stored.
//   * Forward computes S^T = K Q^T so that each lane owns one query row (lane % 32) and the
//     keys sit in its accumulator registers: the row max/sum are in-lane reductions plus one
//     exchange with the other half-wave, and P^T feeds O^T += V^T P^T straight from registers.
//     The running max is only moved when a row's 16-bit p of one sub-tile sum past 2^28 (or one
//     of them overflows the 16-bit format), so most tiles skip rescaling O; the row sum adds the
//     16-bit P that the product actually uses.
//   * Backward in two deterministic kernels with no atomics. dK/dV: keys outer; a block owns a
//     64-key block, its waves walk the group's query heads x query tiles, S = Q K^T and
//     dP = dO V^T land with the key on the lane, so P and dS feed dV^T += dO^T P and
//     dK^T += Q^T dS as B operands, and dK/dV are summed over the group's query heads in
//     registers and LDS, then stored once. dQ: queries outer, shaped like the forward;
//     dQ^T += K^T dS^T takes dS^T straight from registers and is stored once.
//   * Softmax runs in base 2: exp2(s * scale * log2(e) - m'), with lse stored in natural log.
//
// MFMA 32x32x16 register layouts used throughout (lane l, l32 = l % 32, hh = l / 32):
//   A (32x16, M x K): lane l supplies A[l32][8*hh + j], j = 0..7
//   B (16x32, K x N): lane l supplies B[8*hh + j][l32]
//   C (32x32):        lane l holds C[(i/4)*8 + 4*hh + (i%4)][l32] in element i = 0..15
// A and B agree on which (half-wave, element) carries which k, so a product may permute the
// contraction index freely as long as both operands use the same permutation.
//
// ds_read_b64_tr_b16 (per 16-lane group, lane i, result element j) returns element i%4 of the
// 4-element vector addressed by lane 4j + i/4 of the same group. If lane i' of a group
// addresses row r0 + i'/4, columns c0 + 4*(i'%4) .. +3 of a row-major tile, lane i receives
// rows r0..r0+3 of column c0 + i: a column operand for the MFMA.
#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <algorithm>
#include <mutex>
#include <string>
#include <type_traits>

#include "nanonemo_fa.h"

#define NNFA_API extern "C" __attribute__((visibility("default")))

namespace {

using u16 = unsigned short;
typedef u16 u16x8 __attribute__((ext_vector_type(8)));
typedef u16 u16x4 __attribute__((ext_vector_type(4)));
typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// Block timelines, in diagnostic builds only (NN_TIMELINE=1: libnanonemo_fa_timeline.so, which
// `bench.py --timeline` loads; in the product library every stamp compiles to nothing). One lane records
// clock readings into a file-scope device array, one record of kTlWords 64-bit words per (kernel, block):
// the 100 MHz constant clock (s_memrealtime) at the block's start and end, comparable across CUs, the
// shader clock (s_memtime) at its phase boundaries, for cycle counts within the block, and the XCD and
// hardware id of the wave that ran it. Block-level words come from wave 0; per-wave words from each wave.
#ifndef NN_TIMELINE
#define NN_TIMELINE 0
#endif
enum TlKernel { kTlFwd = 0, kTlDq = 1, kTlDkdv = 2, kTlKernels = 3 };
// Words of a record. Forward and dQ: kTlExtra = dQ's prologue end (rows loaded, -D and -lse/scale
// written), kTlExtra + 1 = the block's count of 128-key tiles. dK/dV: kTlExtra + 4 u + w = wave w's loop
// end in the block's unit u (0, 1); kTlExtra + 8 = wave 0 after the first unit's reduction.
enum TlWord { kTlRtStart = 0, kTlRtEnd = 1, kTlMtStart = 2, kTlMtReady = 3, kTlMtEnd = 4, kTlHw = 5, kTlExtra = 6 };
constexpr int kTlBlocks = 16384, kTlWords = 16;
#if NN_TIMELINE
__device__ __align__(256) unsigned long long nn_timeline[kTlKernels * kTlBlocks * kTlWords];
__device__ __forceinline__ void tl_word(int kern, int word, unsigned long long v) {
    if (blockIdx.x < kTlBlocks) nn_timeline[((size_t)kern * kTlBlocks + blockIdx.x) * kTlWords + word] = v;
}
__device__ __forceinline__ unsigned long long tl_hw() {
    // HW_REG_XCC_ID (20), bits 3:0, and HW_REG_HW_ID (4), all 32 bits (CU id in bits 11:8, SE id in 15:13).
    const unsigned xcc = __builtin_amdgcn_s_getreg((3 << 11) | 20), hw = __builtin_amdgcn_s_getreg((31 << 11) | 4);
    return ((unsigned long long)xcc << 32) | hw;
}
#define NN_TL_BLOCK(kern, word, expr) \
    do { if (threadIdx.x == 0) tl_word(kern, word, (expr)); } while (0)
#define NN_TL_WAVE(kern, word, expr) \
    do { if ((threadIdx.x & 63) == 0) tl_word(kern, word, (expr)); } while (0)
#define NN_TL_START(kern)                                                                 \
    do {                                                                                  \
        NN_TL_BLOCK(kern, kTlRtStart, __builtin_amdgcn_s_memrealtime());                  \
        NN_TL_BLOCK(kern, kTlMtStart, __builtin_amdgcn_s_memtime());                      \
        NN_TL_BLOCK(kern, kTlHw, tl_hw());                                                \
    } while (0)
#define NN_TL_END(kern)                                                                   \
    do {                                                                                  \
        NN_TL_BLOCK(kern, kTlMtEnd, __builtin_amdgcn_s_memtime());                        \
        NN_TL_BLOCK(kern, kTlRtEnd, __builtin_amdgcn_s_memrealtime());                    \
    } while (0)
#else
#define NN_TL_BLOCK(kern, word, expr) ((void)0)
#define NN_TL_WAVE(kern, word, expr) ((void)0)
#define NN_TL_START(kern) ((void)0)
#define NN_TL_END(kern) ((void)0)
#endif

constexpr int kF16 = 0;
constexpr int kBF16 = 1;
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;
// The forward keeps a stale running max m until a row's exponentials exp2(s - m) grow past this
// bound (base-2 units): p <= 2^24 stays within the exponent range of fp32 and bf16, and a row's 16
// values of a sub-tile then sum to at most 2^28. In fp16, whose largest value is 65504, a p that large
// packs to inf, and that inf in the row sum triggers the rescale as well.
constexpr float kGrowLog2 = 24.0f;
constexpr float kPsumMax = 16.0f * 16777216.0f;  // 16 * 2^kGrowLog2

#define LDS_AS(T, p) ((__attribute__((address_space(3))) T*)(p))

template <int DT>
struct Elem;

template <>
struct Elem<kBF16> {
    __device__ static inline f32x16 mfma(u16x8 a, u16x8 b, f32x16 c) {
        return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b),
                                                       c, 0, 0, 0);
    }
    // Round-to-nearest-even conversion of two fp32 values into one packed dword (lo first).
    __device__ static inline uint32_t pack2(float lo, float hi) {
        bf16x2 v = {(__bf16)lo, (__bf16)hi};
        return __builtin_bit_cast(uint32_t, v);
    }
    // acc + lo + hi of a packed pair.
    __device__ static inline float add_pair(uint32_t pair, float acc) {
        const bf16x2 one = {(__bf16)1.0f, (__bf16)1.0f};
        return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, pair), one, acc, false);
    }
    __device__ static inline float to_f32(u16 x) { return __uint_as_float((uint32_t)x << 16); }
};

template <>
struct Elem<kF16> {
    __device__ static inline f32x16 mfma(u16x8 a, u16x8 b, f32x16 c) {
        return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0,
                                                      0, 0);
    }
    __device__ static inline uint32_t pack2(float lo, float hi) {
        f16x2 v = {(_Float16)lo, (_Float16)hi};
        return __builtin_bit_cast(uint32_t, v);
    }
    __device__ static inline float add_pair(uint32_t pair, float acc) {
        const f16x2 one = {(_Float16)1.0f, (_Float16)1.0f};
        return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, pair), one, acc, false);
    }
    __device__ static inline float to_f32(u16 x) { return (float)__builtin_bit_cast(_Float16, x); }
};

// Elements [base, base+8) of an accumulator, rounded to 16 bits and packed as an MFMA operand.
template <int DT>
__device__ inline u16x8 pack8(const f32x16& a, int base) {
    u32x4 r = {Elem<DT>::pack2(a[base + 0], a[base + 1]), Elem<DT>::pack2(a[base + 2], a[base + 3]),
               Elem<DT>::pack2(a[base + 4], a[base + 5]), Elem<DT>::pack2(a[base + 6], a[base + 7])};
    return __builtin_bit_cast(u16x8, r);
}

__device__ inline u16x8 cat4(u16x4 a, u16x4 b) { return __builtin_shufflevector(a, b, 0, 1, 2, 3, 4, 5, 6, 7); }
typedef float f32x8 __attribute__((ext_vector_type(8)));
__device__ inline f32x16 cat16(f32x4 a, f32x4 b, f32x4 c, f32x4 d) {
    const f32x8 ab = __builtin_shufflevector(a, b, 0, 1, 2, 3, 4, 5, 6, 7);
    const f32x8 cd = __builtin_shufflevector(c, d, 0, 1, 2, 3, 4, 5, 6, 7);
    return __builtin_shufflevector(ab, cd, 0, 1, 2, 3, 4, 5, 6, 7, 8, 9, 10, 11, 12, 13, 14, 15);
}
__device__ inline u16x8 ld8(const u16* p) { return *reinterpret_cast<const u16x8*>(p); }

// Row-major LDS tiles of W 16-bit columns store 16-byte chunk c of row r at chunk position
// swz_chunk(r, c). The XOR pattern depends only on row bits 1..3 (W = 64) or 2..3 (W = 32), so
// it repeats every 16 rows, and it keeps both access patterns free of bank conflicts:
//   * ds_read_b128 of one logical chunk from 16 consecutive rows (row operands);
//   * ds_read_b64_tr_b16 of 4 consecutive rows x 4 aligned chunks per 32 lanes (column operands).
// It is an involution, so the DMA uses the same map to place chunks.
template <int W>
__device__ inline int swz_chunk(int row, int c) {
    static_assert(W == 64 || W == 32, "tile width");
    if constexpr (W == 64)
        return c ^ ((((row >> 1) & 1) << 2) | ((row >> 2) & 3));
    else
        return c ^ ((row >> 2) & 3);
}
template <int W>
__device__ inline int swz(int row, int col) {
    return row * W + (swz_chunk<W>(row, col >> 3) << 3) + (col & 7);
}

// Per-lane offset of a row operand: 8 columns col0 + 8*hh .. of row `row` (rows 16k + row read
// the same chunk positions, so callers add 16k * W).
template <int W>
__device__ inline int row_off(int row, int col) { return swz<W>(row, col); }

// Per-lane offset of a column operand for ds_read_b64_tr_b16: lane i (of its 16-lane group)
// addresses row r0 + i/4, columns c0 + 4*(i%4) .. +3, and receives rows r0..r0+3 of column
// c0 + i. r0 % 4 == 0 and c0 % 16 == 0; rows 16k + r0 reuse the offset plus 16k * W.
template <int W>
__device__ inline int col_off(int r0, int c0, int lane) {
    const int i = lane & 15;
    return swz<W>(r0 + (i >> 2), c0 + 4 * (i & 3));
}
__device__ inline u16x4 ld_tr(const u16* p) {
    return __builtin_bit_cast(u16x4, __builtin_amdgcn_ds_read_tr16_b64_v4i16(LDS_AS(s16x4, const_cast<u16*>(p))));
}

// Per-lane part of the DMA addressing of a W-column tile (computed once per kernel): the lane's
// row within one copy instruction (a copy instruction moves 64 chunks of 16 bytes, i.e.
// 64 / (W / 8) rows) and its swizzled chunk byte offset. An instruction's rows start at a
// multiple of 64 / (W / 8); the swizzle reads row bits 1..3 (W = 64), of which that start
// contributes only bit 3 (cB1 applies to odd instructions), or bits 2..3 (W = 32), which it never
// touches.
struct DmaLane {
    uint32_t rl, cB0, cB1;
};
template <int W>
__device__ inline DmaLane dma_lane(int lane) {
    constexpr int CH = W / 8;
    const int rl = lane / CH, cl = lane % CH;
    return {(uint32_t)rl, (uint32_t)swz_chunk<W>(rl, cl) * 16, (uint32_t)swz_chunk<W>(rl + 8, cl) * 16};
}

// Per-lane byte offsets of the copy instructions (this wave's share) of a [ROWS][W] tile with row
// stride `ld` elements, relative to the tile's first row: computed once per kernel, so that a copy
// of a tile that does not reach past row T - 1 costs no per-lane address arithmetic.
template <int W, int ROWS, int NW>
struct DmaOffs {
    static constexpr int N = ROWS * (W / 8) / (64 * NW);
    uint32_t o[N];
};
template <int W, int ROWS, int NW>
__device__ inline DmaOffs<W, ROWS, NW> dma_offsets(int lane, int wave, int ld) {
    constexpr int CH = W / 8;
    const DmaLane dl = dma_lane<W>(lane);
    DmaOffs<W, ROWS, NW> r;
#pragma unroll
    for (int it = 0; it < DmaOffs<W, ROWS, NW>::N; ++it) {
        const int k = it * NW + wave;  // copy instruction index within the tile
        r.o[it] = (dl.rl + (uint32_t)(k * (64 / CH))) * (uint32_t)ld * 2 + ((W == 64 && (k & 1)) ? dl.cB1 : dl.cB0);
    }
    return r;
}

// Buffer resource word 3 for raw (unswizzled, stride 0) buffer access on gfx9-family parts.
constexpr int kBufWord3 = 0x00020000;

// Copies rows [r0, r0 + ROWS) of a [T][W] global matrix with row stride `ld` elements into a
// swizzled row-major LDS tile, 16 bytes per lane. `g`, `ld`, `r0`, `T`, `lds` and `wave` are
// wave-uniform, and `fo` holds this lane's offsets for stride `ld` (dma_offsets). The copies are
// buffer loads: the tile's base and extent live in a scalar buffer descriptor and each lane adds its
// 32-bit offset, so they cost no per-lane address arithmetic. The descriptor's extent ends at row
// T - 1, so rows past it read as zeros (their results are masked by the callers). The LDS
// destination of a copy is the uniform base + 16 * lane.
template <int W, int ROWS, int NW>
__device__ inline void dma_rows(const u16* __restrict__ g, int ld, int r0, int T, u16* lds, int wave,
                                const DmaOffs<W, ROWS, NW>& fo) {
    constexpr int CH = W / 8, NCH = ROWS * CH;
    static_assert(NCH % (64 * NW) == 0 && 64 % CH == 0, "tile must split evenly over the block's waves");
#if defined(__HIP_DEVICE_COMPILE__)  // the buffer descriptor type exists in the device pass only
    const int wu = __builtin_amdgcn_readfirstlane(wave);
    // readfirstlane yields an int: each half goes through uint32_t before widening, or a low word with
    // bit 31 set would sign-extend into the high word.
    const uint64_t ga = reinterpret_cast<uint64_t>(g + (size_t)r0 * ld);
    const uint32_t ghi = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(ga >> 32));
    const uint32_t glo = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)ga);
    void* gt = reinterpret_cast<void*>(((uint64_t)ghi << 32) | glo);
    const int nbytes = __builtin_amdgcn_readfirstlane(min(T - r0, ROWS) * ld * 2);
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(gt, 0, nbytes, kBufWord3);
#pragma unroll
    for (int it = 0; it < NCH / (64 * NW); ++it) {
        const int k = it * NW + wu;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, LDS_AS(void, lds + k * 64 * 8), 16, fo.o[it], 0, 0, 0);
    }
#endif
}

// 64 consecutive fp32 values g[0 .. 63] into LDS (lane l's value at lds[l]) by one buffer-load DMA, lane l
// reading g[off_l / 4] (off_l in bytes, below 256). A buffer load, like the tiles' copies, rather than a global
// one: the compiler counts a global load to LDS also among the LDS operations, whose waits it then cannot count
// per instruction, and every LDS wait after one (through the next loop iteration) becomes a wait for all.
__device__ inline void dma_vec64(const float* __restrict__ g, uint32_t off, float* lds) {
#if defined(__HIP_DEVICE_COMPILE__)
    const uint64_t ga = reinterpret_cast<uint64_t>(g);
    const uint32_t ghi = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(ga >> 32));
    const uint32_t glo = (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)ga);
    void* gt = reinterpret_cast<void*>(((uint64_t)ghi << 32) | glo);
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(gt, 0, 256, kBufWord3);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, LDS_AS(void, lds), 4, off, 0, 0, 0);
#endif
}

// Block -> (batch * H + head, query block) for the forward and dQ grids of nqb * BH blocks: heaviest
// query blocks first (the causal work of a block grows with its index). Blocks are dispatched to the
// 8 XCDs round-robin (block i to XCD i % 8), and each XCD has its own L2. When the B * KVH head groups
// divide evenly over the XCDs, the blocks of every query head of one group go to the same XCD
// (group g to XCD g % 8, heaviest first within the XCD), so that the group's K / V tiles are fetched
// into one L2 instead of H / KVH of them. Otherwise blocks of one (batch, head) still share an XCD
// when BH % 8 == 0.
struct QBlk {
    int bh, qb;
};
__device__ inline QBlk qblock_of(int bid, int BH, int group, int nqb) {
    const int G = BH / group;  // (batch, KV head) groups
    if (G % 8 == 0) {
        const int x = bid & 7, slot = bid >> 3;
        const int per = (G >> 3) * group;  // blocks of one query-block index on one XCD
        const int qi = slot / per, r = slot - qi * per;
        const int gi = r / group, hq = r - gi * group;
        return {(gi * 8 + x) * group + hq, nqb - 1 - qi};
    }
    return {bid % BH, nqb - 1 - bid / BH};
}

// Element strides of a [B][heads][T][D] tensor view whose D stride is 1: batch, head and row
// (sequence position). Q, O, dO and dQ share one layout; K, V, dK and dV another.
struct Lay {
    long long sb, sh;
    int st;
    __device__ size_t at(int b, int h) const { return (size_t)b * sb + (size_t)h * sh; }
};

// Wait until this wave's vector-memory operations (including LDS DMA) have completed.
__device__ inline void wait_vmem() { __builtin_amdgcn_s_waitcnt(0x0F70); }
// Wait until at most N of this wave's vector-memory operations are outstanding (they complete in
// issue order, so everything issued before the last N has landed). gfx9 encoding: vmcnt in bits
// 3:0 and 15:14; expcnt and lgkmcnt left at their maxima.
template <int N>
__device__ inline void wait_vmem_keep() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}

// Block barrier that orders LDS only: this wave's LDS accesses complete, then s_barrier. Vector-memory
// operations (global loads and stores, LDS DMA) may stay in flight across it, so it must only be used
// where no wave reads, before its own vmcnt wait, LDS that such an operation writes. (__syncthreads
// also waits for every vector-memory operation.) The memory clobber keeps the compiler from moving
// memory accesses across it.
__device__ inline void barrier_lds() { __asm__ volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// The other half-wave's value combined with this lane's: v_permlane32_swap exchanges the two
// 32-lane halves, and its two results hold this lane's value and its partner's (lane ^ 32).
__device__ inline float pair_max(float x) {
    const unsigned u = __float_as_uint(x);
    const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ inline float pair_sum(float x) {
    const unsigned u = __float_as_uint(x);
    const auto r = __builtin_amdgcn_permlane32_swap(u, u, false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

__device__ inline float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }
__device__ inline float fast_log2(float x) { return __builtin_amdgcn_logf(x); }

// Rotary position embedding folded into the attention (rotate-half, dimension i pairs with i + HD/2):
//     y[i] = x[i] cos - x[i + HD/2] sin,   y[i + HD/2] = x[i] sin + x[i + HD/2] cos   at the row's position,
// with one fp32 rounding per product and per sum (no contraction into fma) and one rounding to the 16-bit
// type, so that it equals the standalone RoPE kernel's result bit for bit. The forward rotates its raw Q
// rows and also writes them out (the backward's dK/dV kernel reads rotated Q); the dQ kernel applies the
// inverse rotation (angle -theta) to its output. cos / sin are dense fp32 [table rows][HD/2] tables.
struct RopeArgs {
    const float* cosT;
    const float* sinT;
    u16* qrot;  // forward only: rotated Q, written with Q's layout
};
__device__ inline float mul_rn(float a, float b) {
#pragma clang fp contract(off)
    return a * b;
}
__device__ inline float add_rn(float a, float b) {
#pragma clang fp contract(off)
    return a + b;
}
__device__ inline float sub_rn(float a, float b) {
#pragma clang fp contract(off)
    return a - b;
}

// ------------------------------------------------------------------------------------------
// Forward. Block = 4 waves = 128 query rows of one (batch, head); 128-key tiles of K and V,
// double-buffered in LDS by DMA. Q stays in registers for the whole block.
// ------------------------------------------------------------------------------------------
template <int HD, int DT, bool ROPE>
__global__ __launch_bounds__(256, 2) void fa_fwd_kernel(const u16* __restrict__ Q, const u16* __restrict__ K,
                                                        const u16* __restrict__ V, u16* __restrict__ O,
                                                        float* __restrict__ LSE, int BH, int H, int KVH, int T,
                                                        int nqb, float sl2, Lay lq, Lay lk, RopeArgs ra) {
    using E = Elem<DT>;
    NN_TL_START(kTlFwd);
    constexpr int BM = 128, BN = 128, NW = 4;
    constexpr int NS = HD / 16;  // k-steps of Q K^T
    constexpr int ND = HD / 32;  // 32-wide head_dim tiles of O^T
    constexpr int NT = BN / 32;  // 32-key tiles of S^T
    constexpr int TILE = BN * HD;
    __shared__ __attribute__((aligned(16))) u16 kA[TILE];
    __shared__ __attribute__((aligned(16))) u16 vA[TILE];
    __shared__ __attribute__((aligned(16))) u16 kB[TILE];
    __shared__ __attribute__((aligned(16))) u16 vB[TILE];

    const QBlk blk = qblock_of(blockIdx.x, BH, H / KVH, nqb);
    const int bh = blk.bh, qb = blk.qb;
    const int b = bh / H, h = bh - b * H;
    const int kvh = h / (H / KVH);
    const size_t qoff = lq.at(b, h);
    const size_t kvoff = lk.at(b, kvh);
    const u16* Kp = K + kvoff;
    const u16* Vp = V + kvoff;

    const int tid = threadIdx.x, lane = tid & 63, l32 = lane & 31, hh = lane >> 5;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const DmaOffs<HD, BN, NW> dfo = dma_offsets<HD, BN, NW>(lane, wave, lk.st);
    const int g16 = (lane >> 4) & 1;  // which 16-column half of a 32-wide MFMA tile this lane reads
    const int q0 = qb * BM, qw = q0 + wave * 32, qrow = qw + l32;

    const int ntiles = (min(q0 + BM, T) + BN - 1) / BN;
    NN_TL_BLOCK(kTlFwd, kTlExtra + 1, (unsigned long long)ntiles);
    auto issue = [&](int it, u16* kb, u16* vb) {
        dma_rows<HD, BN, NW>(Kp, lk.st, it * BN, T, kb, wave, dfo);
        dma_rows<HD, BN, NW>(Vp, lk.st, it * BN, T, vb, wave, dfo);
    };
    // Per-lane LDS offsets of a row operand (row l32 of a 32-row slice, columns 16ks + 8hh; add 32t*HD).
    int koff[NS];
#pragma unroll
    for (int ks = 0; ks < NS; ++ks) koff[ks] = row_off<HD>(l32, 16 * ks + 8 * hh);
    // This wave's 32 Q rows by DMA into its slice of the second K tile buffer, which the loop's first copy
    // overwrites only after the block barrier (whole 128-byte rows per 8 lanes; loaded per lane in the operand
    // layout, each load instruction would touch 32 rows 32 bytes at a time), then the first K / V tile. Rows past
    // T read as zeros: their scores stay finite and nothing of theirs is stored. Copies complete in issue order,
    // so the wave waits for its rows (and, with RoPE, the row's cos / sin) with the tile still in flight, and
    // reads its Q operands (and rotates them) during the tile's flight; the loop's first wait takes the tile.
    // (Tile first and one wait for both: the forward 1-3 % slower.)
    constexpr int kTileOps = 2 * (BN * HD / 8) / (64 * NW);  // vector-memory instructions per issue()
    if (qw < T) {
        const DmaOffs<HD, 32, 1> rfo = dma_offsets<HD, 32, 1>(lane, 0, lq.st);
        dma_rows<HD, 32, 1>(Q + qoff, lq.st, qw, T, kB + 32 * wave * HD, 0, rfo);
    }
    u16x8 qf[NS];
    if constexpr (ROPE) {
        // The row's cos / sin values are loaded with the Q rows, before the first K / V tile and the rotation,
        // so that the latencies overlap. The rotated rows are stored to q_rot at the end, with O: vector-memory
        // counts complete in order, so a store issued earlier would make the next tile's wait wait for it.
        // qf[s] holds columns 16 s + 8 hh .. + 7 of the row, so qf[s] and qf[s + NS / 2] are the two halves of
        // the same rotation pairs (columns c and c + HD / 2, c < HD / 2).
        constexpr int HALF = HD / 2;
        f32x4 cs[NS / 2][2], sn[NS / 2][2];
        const float* cr = ra.cosT + (size_t)min(qrow, T - 1) * HALF;
        const float* sr = ra.sinT + (size_t)min(qrow, T - 1) * HALF;
#pragma unroll
        for (int s = 0; s < NS / 2; ++s)
#pragma unroll
            for (int x = 0; x < 2; ++x) {
                cs[s][x] = *reinterpret_cast<const f32x4*>(cr + 16 * s + 8 * hh + 4 * x);
                sn[s][x] = *reinterpret_cast<const f32x4*>(sr + 16 * s + 8 * hh + 4 * x);
            }
        issue(0, kA, vA);
        wait_vmem_keep<kTileOps>();
#pragma unroll
        for (int s = 0; s < NS; ++s) qf[s] = ld8(kB + 32 * wave * HD + koff[s]);
        {
#pragma unroll
            for (int s = 0; s < NS / 2; ++s) {
                float y1[8], y2[8];
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    const float c = cs[s][j >> 2][j & 3], si = sn[s][j >> 2][j & 3];
                    const float x1 = E::to_f32(qf[s][j]), x2 = E::to_f32(qf[s + NS / 2][j]);
                    y1[j] = sub_rn(mul_rn(x1, c), mul_rn(x2, si));
                    y2[j] = add_rn(mul_rn(x1, si), mul_rn(x2, c));
                }
                const u32x4 w1 = {E::pack2(y1[0], y1[1]), E::pack2(y1[2], y1[3]), E::pack2(y1[4], y1[5]), E::pack2(y1[6], y1[7])};
                const u32x4 w2 = {E::pack2(y2[0], y2[1]), E::pack2(y2[2], y2[3]), E::pack2(y2[4], y2[5]), E::pack2(y2[6], y2[7])};
                qf[s] = __builtin_bit_cast(u16x8, w1);
                qf[s + NS / 2] = __builtin_bit_cast(u16x8, w2);
            }
        }
    } else {
        issue(0, kA, vA);
        wait_vmem_keep<kTileOps>();
#pragma unroll
        for (int s = 0; s < NS; ++s) qf[s] = ld8(kB + 32 * wave * HD + koff[s]);
    }

    f32x16 oacc[ND];
#pragma unroll
    for (int dt = 0; dt < ND; ++dt) oacc[dt] = f32x16{};
    float mb = -INFINITY, lsum = 0.f;
    bool first = true;  // wave-uniform: no sub-tile processed yet

    // Per-lane LDS offsets of a V^T column operand (keys 16c + 8x + 4hh.., column 32dt + l32; add 16c*HD); K row
    // operands (key l32 + 32t) use koff.
    int voff[ND][2];
#pragma unroll
    for (int dt = 0; dt < ND; ++dt)
#pragma unroll
        for (int x = 0; x < 2; ++x) voff[dt][x] = col_off<HD>(8 * x + 4 * hh, 32 * dt + 16 * g16, lane);

    // One 128-key tile as four 32-key sub-tiles, software-pipelined so that the matrix unit and the
    // VALU have independent work in the same stretch of straight-line code:
    //   * K operands of sub-tile t+2 are read from LDS while sub-tile t is processed, so the S^T
    //     MFMAs of sub-tile t+1, issued at the top of step t, never wait on LDS;
    //   * the V^T operands of step t are read before its exponentials;
    //   * no max is taken per sub-tile: p = exp2(s * sl2 - mb) against the stale running max mb,
    //     and the row sums of p, which P V needs anyway, show when a row has outgrown mb. Then (rare:
    //     a row's first sub-tile, where mb = -inf, and large jumps of its max) the wave takes the
    //     true max, rescales the row sum and O, and recomputes p, just before the P V MFMAs.
    // MASK: the tile crosses the diagonal or T.
    auto tile = [&](auto mask_tag, int k0, const u16* kb, const u16* vb) {
        constexpr bool MASK = decltype(mask_tag)::value;
        const int lim = min(qrow, T - 1) - k0 - 4 * hh;  // key offsets beyond this are masked
        const int nt = MASK ? min(NT, (qw + 31 - k0) / 32 + 1) : NT;  // sub-tiles with a visible key
        // The wave's smallest lim (lane 32: row qw, hh = 1): sub-tiles whose last key offset (32t + 27)
        // does not exceed it are visible to every lane and skip the per-element selects.
        const int lim_w = min(qw, T - 1) - k0 - 4;
        auto kops = [&](int t, u16x8* kq) {
#pragma unroll
            for (int ks = 0; ks < NS; ++ks) kq[ks] = ld8(kb + 32 * t * HD + koff[ks]);
        };
        auto scores = [&](const u16x8* kq) {
            f32x16 a = f32x16{};
#pragma unroll
            for (int ks = 0; ks < NS; ++ks) a = E::mfma(kq[ks], qf[ks], a);
            return a;
        };
        u16x8 kq0[NS], kq1[NS];
        kops(0, kq0);
        f32x16 cur = scores(kq0);
        if (!MASK || nt > 1) kops(1, kq1);
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            if (MASK && t >= nt) break;
            u16x8* kn = (t & 1) ? kq0 : kq1;  // operands of sub-tile t+1, read one step ago
            f32x16 nxt = f32x16{};
            if (t + 1 < NT && (!MASK || t + 1 < nt)) nxt = scores(kn);
            if (t + 2 < NT && (!MASK || t + 2 < nt)) kops(t + 2, (t & 1) ? kq1 : kq0);
            u16x8 va[2][ND];
#pragma unroll
            for (int half = 0; half < 2; ++half)
#pragma unroll
                for (int dt = 0; dt < ND; ++dt) {
                    const u16* vc = vb + 16 * (2 * t + half) * HD;
                    va[half][dt] = cat4(ld_tr(vc + voff[dt][0]), ld_tr(vc + voff[dt][1]));
                }
            // cur[i] = score of query qrow against key k0 + 32t + (i/4)*8 + 4hh + i%4.
            if (MASK && 32 * t + 27 > lim_w) {
#pragma unroll
                for (int i = 0; i < 16; ++i) cur[i] = (32 * t + (i >> 2) * 8 + (i & 3) > lim) ? -INFINITY : cur[i];
            }
            // p against the stale max; a lane's 16 values sum to psum (of the 16-bit p that P V uses).
            f32x16 pv;
            u16x8 pf[2];
            float psum = 0.f;
            auto exps = [&]() {
#pragma unroll
                for (int i = 0; i < 16; ++i) pv[i] = fast_exp2(fmaf(cur[i], sl2, -mb));
                psum = 0.f;
#pragma unroll
                for (int half = 0; half < 2; ++half) {
                    pf[half] = pack8<DT>(pv, 8 * half);  // P^T chunk 2t+half: keys 16(2t+half) + (j/4)*8 + 4hh + j%4
                    const u32x4 pw = __builtin_bit_cast(u32x4, pf[half]);
                    psum = E::add_pair(pw[0], psum);
                    psum = E::add_pair(pw[1], psum);
                    psum = E::add_pair(pw[2], psum);
                    psum = E::add_pair(pw[3], psum);
                }
            };
            // The row's true max sets the new mb (both half-waves agree through pair_max); the row sum
            // and O are rescaled by 2^(old - new), and p is (re)computed.
            auto rescale = [&]() {
                float mx = cur[0];
#pragma unroll
                for (int i = 1; i < 16; ++i) mx = fmaxf(mx, cur[i]);
                mx = pair_max(mx);
                const float mnew = fmaxf(mb, mx * sl2);
                const float corr = fast_exp2(mb - mnew);
                mb = mnew;
                lsum *= corr;
#pragma unroll
                for (int dt = 0; dt < ND; ++dt) oacc[dt] *= corr;
                exps();
            };
            if (first) {
                // This wave's first sub-tile (keys 0..31, which hold key 0 for every row, so every
                // row's max is finite): mb = -inf until here, so the max is taken directly.
                rescale();
                first = false;
            } else {
                exps();
                // Rare: some row outgrew mb (its psum past the bound, or inf).
                if (__builtin_amdgcn_ballot_w64(psum > kPsumMax)) rescale();
            }
            lsum += psum;
#pragma unroll
            for (int half = 0; half < 2; ++half)
#pragma unroll
                for (int dt = 0; dt < ND; ++dt) oacc[dt] = E::mfma(va[half][dt], pf[half], oacc[dt]);
            cur = nxt;
        }
    };
    auto step = [&](int it, const u16* kb, const u16* vb) {
        const int k0 = it * BN;
        if (qw >= T || k0 > qw + 31) return;  // no visible key in this tile for this wave
        if (k0 + BN - 1 > qw || k0 + BN > T)
            tile(std::true_type{}, k0, kb, vb);
        else
            tile(std::false_type{}, k0, kb, vb);
    };

    for (int it = 0; it < ntiles; it += 2) {
        wait_vmem();
        __syncthreads();
        if (it == 0) NN_TL_BLOCK(kTlFwd, kTlMtReady, __builtin_amdgcn_s_memtime());
        if (it + 1 < ntiles) issue(it + 1, kB, vB);
        step(it, kA, vA);
        if (it + 1 >= ntiles) break;
        wait_vmem();
        __syncthreads();
        if (it + 2 < ntiles) issue(it + 2, kA, vA);
        step(it + 1, kB, vB);
    }

    const float ltot = pair_sum(lsum);
    if (qrow < T) {
        if constexpr (ROPE) {  // the rotated rows, stored with O (a store inside the loop would hold up tile waits)
            u16* qo = ra.qrot + qoff + (size_t)qrow * lq.st;
#pragma unroll
            for (int s = 0; s < NS; ++s) *reinterpret_cast<u16x8*>(qo + 16 * s + 8 * hh) = qf[s];
        }
        const float inv = 1.f / ltot;
        u16* op = O + qoff + (size_t)qrow * lq.st;
#pragma unroll
        for (int dt = 0; dt < ND; ++dt)
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const f32x16& a = oacc[dt];
                u32x2 w = {E::pack2(a[4 * g] * inv, a[4 * g + 1] * inv), E::pack2(a[4 * g + 2] * inv, a[4 * g + 3] * inv)};
                *reinterpret_cast<u32x2*>(op + 32 * dt + 8 * g + 4 * hh) = w;
            }
        if (hh == 0) LSE[(size_t)bh * T + qrow] = (mb + fast_log2(ltot)) * kLn2;
    }
    NN_TL_END(kTlFwd);
}

// ------------------------------------------------------------------------------------------
// Backward, preprocessing, one pass over dO and O: nD = -rowsum(dO * O) and nL = -lse / scale, fp32.
// Both enter the backward products as accumulator initial values: S - lse/scale and dP - D come
// straight out of the MFMAs, so P = exp2((S - lse/scale) * scale * log2(e)) and dS = P (dP - D).
// ------------------------------------------------------------------------------------------
template <int HD, int DT>
__global__ __launch_bounds__(256) void fa_bwd_pre_kernel(const u16* __restrict__ O, const u16* __restrict__ dO,
                                                         const float* __restrict__ LSE, float* __restrict__ nDvec,
                                                         float* __restrict__ nLvec, int64_t rows, int H, int T,
                                                         float inv_scale, Lay lq) {
    using E = Elem<DT>;
    constexpr int TPR = HD / 8;  // threads per row
    const int64_t gtid = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int64_t row = gtid / TPR;  // (batch, head, position) in [B][H][T] order
    const int c = (int)(gtid % TPR);
    float acc = 0.f;
    if (row < rows) {
        const int64_t bh = row / T;
        const int t = (int)(row - bh * T), b = (int)(bh / H), h = (int)(bh - (int64_t)b * H);
        const size_t off = lq.at(b, h) + (size_t)t * lq.st + 8 * c;
        const u16x8 o = ld8(O + off), g = ld8(dO + off);
#pragma unroll
        for (int j = 0; j < 8; ++j) acc = fmaf(E::to_f32(o[j]), E::to_f32(g[j]), acc);
    }
#pragma unroll
    for (int off = TPR / 2; off > 0; off >>= 1) acc += __shfl_xor(acc, off);
    if (row < rows && c == 0) {
        nDvec[row] = -acc;
        nLvec[row] = -LSE[row] * inv_scale;
    }
}

// ------------------------------------------------------------------------------------------
// Backward, dK / dV. Block = 4 waves, one per SIMD, and one block per CU, so each wave has the
// SIMD's whole register file (up to 512 registers). The block owns a 64-key block ("unit"); every
// wave holds all 64 keys: K and V as B operands and its own partial dK^T, dV^T accumulators.
// The 4 waves split the unit's (query head, 64-row query tile) iterations round-robin and each
// streams its own Q / dO tiles and -lse/scale, -D vectors through a private double-buffered LDS
// slot by DMA, so the loop needs no block barrier, and every Q / dO operand read from LDS feeds
// both 32-key slabs. The GQA sum over the H/KVH query heads of a KV head happens in the
// accumulators. At the end of a unit the 4 partial dK / dV are summed through LDS and stored once
// in the output dtype (no atomics, no fp32 round trip through HBM). A block takes unit j and unit
// nkb-1-j, so every block carries the same causal work; small unsplit problems (paired = 0, see
// dkdv_mode) take single units instead: one per block, or two per block with two waves each, so that no
// block carries a second unit's loads, iterations and reduction after its first. When the pairs are too
// few to fill the chip, nsplit > 1 blocks share each pair: block s takes iterations [s n / nsplit, (s+1) n / nsplit)
// of each unit (n of them) and stores its fp32 partial sums into `part` instead, which
// fa_bwd_dkdv_sum_kernel adds in split order. Per 32-query step and 32-key slab:
//   S' = Q K^T - lse/scale, dP' = dO V^T - D   (A = Q / dO rows from LDS, B = K / V registers;
//                                              the accumulators start from -lse/scale and -D)
//   P = exp2(S' * sl2), dS = P dP'
//   dV^T += dO^T P, dK^T += Q^T dS             (A = columns of the Q / dO tiles, B = P / dS registers)
// ------------------------------------------------------------------------------------------
// KVL: with four waves on one unit pair (WPP = 4), the block copies each unit's K and V rows once into LDS
// (each wave a quarter, by DMA), and every wave reads its K / V operands from there, instead of each wave
// loading all 64 rows from memory; the second unit's rows are copied a whole unit ahead, while the first
// unit's loop runs, so its unit change carries only the first tiles' copies.
template <int HD, int DT, int WPP, bool KVL>
__global__ __launch_bounds__(256, 1) void fa_bwd_dkdv_kernel(
    const u16* __restrict__ Q, const u16* __restrict__ K, const u16* __restrict__ V, const u16* __restrict__ dO,
    const float* __restrict__ nLvec, const float* __restrict__ nDvec, u16* __restrict__ dK, u16* __restrict__ dV,
    int BKV, int H, int KVH, int T, int nkb, int nqt, float sl2, float scale, Lay lq, Lay lk, int nsplit,
    float* __restrict__ part, int paired) {
    using E = Elem<DT>;
    NN_TL_START(kTlDkdv);
    constexpr int BNK = 64, BM = 64, NW = 4, NSL = BNK / 32;
    constexpr int PPB = NW / WPP;  // unit pairs per block: waves WPP p .. WPP p + WPP - 1 share pair p
    static_assert(WPP == 1 || WPP == 2 || WPP == 4, "waves per unit pair");
    constexpr int NS = HD / 16;
    constexpr int ND = HD / 32;
    constexpr int QT = BM * HD;  // elements of one Q or dO tile
    static_assert(BNK == BM, "a unit's first query tile is its own index");
    __shared__ __attribute__((aligned(16))) u16 qA[NW * QT];
    __shared__ __attribute__((aligned(16))) u16 oA[NW * QT];
    __shared__ __attribute__((aligned(16))) u16 qB[NW * QT];
    __shared__ __attribute__((aligned(16))) u16 oB[NW * QT];
    __shared__ __attribute__((aligned(16))) float lA[NW * 2 * BM];  // per wave: -lse/scale | -D
    __shared__ __attribute__((aligned(16))) float lB[NW * 2 * BM];
    static_assert(!KVL || WPP == NW, "K / V through LDS needs the block's four waves on one pair");
    __shared__ __attribute__((aligned(16))) u16 kvS[KVL ? 2 * BNK * HD : 8];  // a unit's K rows, then its V rows

    const int nbk = (BKV + PPB - 1) / PPB;   // blocks per unit-pair index (and split)
    const int nbase = nbk * (paired ? (nkb + 1) / 2 : nkb);  // blocks of one split
    const int sidx = blockIdx.x / nbase;      // this block's split
    const int bid = blockIdx.x - sidx * nbase;
    const int bgrp = bid % nbk;               // the block's pairs are (batch, KV head) bgrp PPB .. + PPB - 1
    const int pj = bid / nbk;  // the pair's first unit (the block's only unit when unpaired)
    const int tid = threadIdx.x, lane = tid & 63, l32 = lane & 31, hh = lane >> 5;
    const int wave = tid >> 6;  // a uniform copy in an SGPR costs this kernel more than it saves
    const int wp = wave % WPP;  // this wave's place among its pair's waves
    // This wave's (batch, KV head); past BKV in the last block (the wave idles but keeps the barriers). It is
    // wave-uniform and kept in a scalar register (with every wave on one pair it is the block's), so that the
    // tile copies' addressing stays in SALU. (With one wave per pair the scalar form breaks the compiler's
    // AGPR-copy rewrite pass.)
    const int bk = WPP == NW ? bgrp : WPP == 2 ? __builtin_amdgcn_readfirstlane(bgrp * PPB + wave / WPP) : bgrp * PPB + wave / WPP;
    const bool active = bk < BKV;
    const int b = bk / KVH, kvh = bk - b * KVH, group = H / KVH;
    const DmaOffs<HD, BM, 1> dfo = dma_offsets<HD, BM, 1>(lane, 0, lq.st);
    // This split's iterations [first, end) of a unit with n of them.
    // 32-bit: the host splits only units whose (sidx + 1) n stays below 2^31 (dkdv_split).
    const uint32_t su = __builtin_amdgcn_readfirstlane(sidx), nsu = __builtin_amdgcn_readfirstlane(nsplit);
    auto first_of = [&](int n) { return (int)(su * (uint32_t)n / nsu); };
    auto end_of = [&](int n) { return (int)((su + 1) * (uint32_t)n / nsu); };
    const int g16 = (lane >> 4) & 1;
    const size_t kvoff = lk.at(b, kvh);

    int qroff[NS], qcoff[ND][2];
#pragma unroll
    for (int ks = 0; ks < NS; ++ks) qroff[ks] = row_off<HD>(l32, 16 * ks + 8 * hh);
#pragma unroll
    for (int dt = 0; dt < ND; ++dt)
#pragma unroll
        for (int x = 0; x < 2; ++x) qcoff[dt][x] = col_off<HD>(8 * x + 4 * hh, 32 * dt + 16 * g16, lane);

    // A unit's K / V operands (every wave holds all 64 keys).
    u16x8 kf[NSL][NS], vf[NSL][NS];
    auto load_kv = [&](int kb0_) {
#pragma unroll
        for (int sl = 0; sl < NSL; ++sl) {
            const int key = min(kb0_ + 32 * sl + l32, T - 1);  // keys past T are masked below
#pragma unroll
            for (int s = 0; s < NS; ++s) {
                kf[sl][s] = ld8(K + kvoff + (size_t)key * lk.st + 16 * s + 8 * hh);
                vf[sl][s] = ld8(V + kvoff + (size_t)key * lk.st + 16 * s + 8 * hh);
            }
        }
    };
    // KVL: this wave's quarter of a unit's K and V rows into kvS (swizzled like the Q / dO tiles), and every
    // wave's operands from there.
    const DmaOffs<HD, BNK, NW> kvo = dma_offsets<HD, BNK, NW>(lane, wave, lk.st);
    auto issue_kv = [&](int kb0_) {
        dma_rows<HD, BNK, NW>(K + kvoff, lk.st, kb0_, T, kvS, wave, kvo);
        dma_rows<HD, BNK, NW>(V + kvoff, lk.st, kb0_, T, kvS + BNK * HD, wave, kvo);
    };
    auto read_kv = [&]() {
#pragma unroll
        for (int sl = 0; sl < NSL; ++sl)
#pragma unroll
            for (int s = 0; s < NS; ++s) {
                kf[sl][s] = ld8(kvS + 32 * sl * HD + qroff[s]);
                vf[sl][s] = ld8(kvS + BNK * HD + 32 * sl * HD + qroff[s]);
            }
    };
    // Iteration itn of unit qtf (whose query tiles run from qtf to nqt - 1): query head iter_head of the group,
    // query tile iter_tile. Head-minor, so that the group's diagonal iterations, which carry the mask, go to
    // different waves. The pair's first unit (pj, the longer) walks its tiles down from the last one, the second
    // (nkb - 1 - pj) up from its own: at the pair's i-th iteration every pair of the (batch, KV head) is then on
    // tile nqt - 1 - i / group in its first unit or on tile i / group - 1 in its second, whichever pair it is. The
    // pairs' blocks of one (batch, KV head) run on one XCD and start together, so they ask for the same Q / dO
    // tiles at about the same time and share them in that XCD's L2 (at most two tiles per head in flight).
    auto iter_head = [&](int itn, int qtf) { (void)qtf; return itn % group; };
    auto iter_tile = [&](int itn, int qtf) { return qtf == pj ? nqt - 1 - itn / group : qtf + itn / group; };
    // DMA iteration itn into this wave's slot: the Q / dO tiles and the -lse/scale, -D vectors.
    auto issue_it = [&](int itn, int qtf, u16* qs, u16* os, float* ls) {
        // Wave-uniform in fact; made uniform for the compiler only here, so that the tile addressing is
        // scalar without keeping scalar copies alive across the whole kernel.
        const int itu = __builtin_amdgcn_readfirstlane(itn), wu = __builtin_amdgcn_readfirstlane(wave);
        const int bu = __builtin_amdgcn_readfirstlane(b), ku = __builtin_amdgcn_readfirstlane(kvh);
        const int hq = ku * group + iter_head(itu, qtf);
        const size_t ro = ((size_t)bu * H + hq) * T;  // first row of the head's [T] vectors
        const size_t qo = lq.at(bu, hq);
        const int q0 = iter_tile(itu, qtf) * BM;
        dma_rows<HD, BM, 1>(Q + qo, lq.st, q0, T, qs + wu * QT, 0, dfo);
        dma_rows<HD, BM, 1>(dO + qo, lq.st, q0, T, os + wu * QT, 0, dfo);
        const uint32_t lo = (uint32_t)min(lane, T - 1 - q0) * 4;  // rows past T repeat row T - 1
        dma_vec64(nLvec + ro + q0, lo, ls + wu * 2 * BM);
        dma_vec64(nDvec + ro + q0, lo, ls + wu * 2 * BM + BM);
    };
    constexpr int kDmaOps = 2 * (QT / 8 / 64) + 2;  // vector-memory instructions per issue_it()
    // The first unit's K / V and first tiles; each later unit's are issued before the previous unit's
    // reduction, so that their latency overlaps it. With KVL the first unit's rows go through kvS and, with two
    // units, once every wave has read them the second unit's rows are copied there, in flight during the first
    // unit's loop; rows past T read as zeros, where the direct loads repeat row T - 1 (both are future keys of
    // every row, masked below). KVL takes kvS for a single unit too: then no register the loops read comes
    // from a global load, which would make the compiler wait for every copy in flight (the second unit's K / V
    // included) before it enters the unit loop.
    const int nunits = paired && nkb - 1 - pj > pj ? 2 : 1;  // an odd unit count leaves the middle unit alone
    const bool kvl = KVL && nunits == 2;  // block-uniform (with WPP = 4 the block's waves share one pair)
    // The partial dK^T / dV^T of the current unit, cleared once before the unit loop and again after each unit's
    // reduction. (Declared and cleared at the top of the unit loop, they cost about twice as many register moves
    // there: dK/dV 2-4 % slower.) Each accumulator is cleared by an MFMA of zero operands onto a zero C, one
    // instruction per 16 registers on the matrix pipe; the empty asm statements keep the compiler from seeing
    // the operands as constants, which would let it compute one zero tile and copy it 16 registers at a time.
    f32x16 dk[NSL][ND], dv[NSL][ND];
    auto clear_acc = [&]() {
#pragma unroll
        for (int sl = 0; sl < NSL; ++sl)
#pragma unroll
            for (int dt = 0; dt < ND; ++dt) {
                u16x8 zk = {}, zv = {};
                __asm__ volatile("" : "+v"(zk));
                __asm__ volatile("" : "+v"(zv));
                dk[sl][dt] = E::mfma(zk, zk, f32x16{});
                dv[sl][dt] = E::mfma(zv, zv, f32x16{});
            }
    };
    if constexpr (KVL) {
        bool tile0 = false;  // wave-uniform: this wave's first tiles were issued after its K / V copies
        if (active) {
            issue_kv(pj * BNK);
            const int n0 = group * (nqt - pj), i0 = first_of(n0);
            if (wp < end_of(n0) - i0) {
                issue_it(i0 + wp, pj, qA, oA, lA);
                tile0 = true;
            }
        }
        clear_acc();
        // This wave's K / V copies have landed (copies complete in issue order; its first tiles may stay in
        // flight), and after the barrier every wave's have. An LDS-only barrier: __syncthreads would wait for the
        // tiles too.
        if (tile0)
            wait_vmem_keep<kDmaOps>();
        else
            wait_vmem();
        barrier_lds();
        if (active) read_kv();
        if (kvl) {
            barrier_lds();  // every wave's reads of kvS are done before the second unit's copies overwrite it
            if (active) issue_kv((nkb - 1 - pj) * BNK);
        }
    } else {
        if (active) {
            load_kv(pj * BNK);
            const int n0 = group * (nqt - pj), i0 = first_of(n0);
            if (wp < end_of(n0) - i0) issue_it(i0 + wp, pj, qA, oA, lA);
        }
        clear_acc();
    }

    for (int ui = 0; ui < nunits; ++ui) {
        const int unit = ui == 0 ? pj : nkb - 1 - pj;
        const int kb0 = unit * BNK;
        // The second unit's rows, copied during the first unit's loop, into registers. With KVL a second unit
        // implies kvl; the test is on KVL and ui > 0 so that the compiler sees every later unit redefine the K / V
        // registers, and does not keep the previous unit's alive through its reduction.
        if (KVL && ui > 0) {
            wait_vmem();
            __syncthreads();
            if (active) read_kv();
        }
        const int qt_first = unit, nq = nqt - qt_first, niter = group * nq;
        const int ifirst = first_of(niter), nsp = end_of(niter) - ifirst;  // this split's iterations
        const int nmine = active && wp < nsp ? (nsp - wp + WPP - 1) / WPP : 0;  // iterations ifirst + wp + WPP j


        // Iteration itn -> 64-row query tile.
        auto qbase_of = [&](int itn) { return iter_tile(itn, qt_first) * BM; };
        auto issue = [&](int itn, u16* qs, u16* os, float* ls) { issue_it(itn, qt_first, qs, os, ls); };
        // Operands of one 32-query step: Q / dO rows (A operands) and -lse/scale, -D as the
        // accumulators' initial values (element i: query 32qh + (i/4)*8 + 4hh + i%4, the same for
        // every key); and the Q^T / dO^T columns of its two 16-query chunks.
        struct RowOps {
            u16x8 qa[NS], oa[NS];
            f32x16 s0, d0;
        };
        struct ColOps {
            u16x8 gcol[2][ND], qcol[2][ND];
        };
        auto load_rows = [&](int qh, const u16* qb_, const u16* ob_, const float* lb_, RowOps& r) {
#pragma unroll
            for (int ks = 0; ks < NS; ++ks) {
                r.qa[ks] = ld8(qb_ + 32 * qh * HD + qroff[ks]);
                r.oa[ks] = ld8(ob_ + 32 * qh * HD + qroff[ks]);
            }
            const f32x4* lv = reinterpret_cast<const f32x4*>(lb_ + 32 * qh + 4 * hh);
            const f32x4* dv4 = reinterpret_cast<const f32x4*>(lb_ + BM + 32 * qh + 4 * hh);
            r.s0 = cat16(lv[0], lv[2], lv[4], lv[6]);  // +8 floats per group of 4 rows
            r.d0 = cat16(dv4[0], dv4[2], dv4[4], dv4[6]);
        };
        auto load_cols = [&](int qh, const u16* qb_, const u16* ob_, ColOps& c) {
#pragma unroll
            for (int half = 0; half < 2; ++half) {
                const u16* oc = ob_ + 16 * (2 * qh + half) * HD;
                const u16* qc = qb_ + 16 * (2 * qh + half) * HD;
#pragma unroll
                for (int dt = 0; dt < ND; ++dt) {
                    c.gcol[half][dt] = cat4(ld_tr(oc + qcoff[dt][0]), ld_tr(oc + qcoff[dt][1]));
                    c.qcol[half][dt] = cat4(ld_tr(qc + qcoff[dt][0]), ld_tr(qc + qcoff[dt][1]));
                }
            }
        };
        // One 64-query iteration: two 32-query steps, each against both 32-key slabs. The second
        // step's operands are read from LDS while the first step's products run.
        // MASK: the iteration crosses the diagonal (a separate instantiation, so that unmasked iterations
        // carry no per-element selects).
        // DMA: the next iteration's tiles (iteration nitn into nqs / nos / nls) are copied during this
        // one, their copy instructions spread over the MFMAs (the CU's copy path accepts them only so
        // fast, and an in-order wave that issued them back to back would stall on it with its MFMA
        // pipe idle).
        auto compute = [&](auto mask_tag, auto dma_tag, int qbase, const u16* qs, const u16* os, const float* ls,
                           int nitn, u16* nqs, u16* nos, float* nls) {
            constexpr bool MASK = decltype(mask_tag)::value;
            constexpr bool DMA = decltype(dma_tag)::value;
            if constexpr (DMA) issue(nitn, nqs, nos, nls);
            const u16* qb_ = qs + wave * QT;
            const u16* ob_ = os + wave * QT;
            const float* lb_ = ls + wave * 2 * BM;
            RowOps r[2];
            ColOps c[2];
            load_rows(0, qb_, ob_, lb_, r[0]);
            load_cols(0, qb_, ob_, c[0]);
#pragma unroll
            for (int qh = 0; qh < 2; ++qh) {
                // A masked iteration sits on the diagonal (its query tile is the unit: qbase == kb0), so
                // slab sl against step qh is wholly future for sl > qh (no products at all: p = 0),
                // wholly visible for sl < qh, and only sl == qh needs the per-element mask.
                f32x16 s[NSL], dp[NSL];
#pragma unroll
                for (int sl = 0; sl < NSL; ++sl) {
                    if (MASK && sl > qh) continue;
                    s[sl] = r[qh].s0;
                    dp[sl] = r[qh].d0;
#pragma unroll
                    for (int ks = 0; ks < NS; ++ks) {
                        s[sl] = E::mfma(r[qh].qa[ks], kf[sl][ks], s[sl]);
                        dp[sl] = E::mfma(r[qh].oa[ks], vf[sl][ks], dp[sl]);
                    }
                }
                if (qh == 0) {
                    load_rows(1, qb_, ob_, lb_, r[1]);
                    load_cols(1, qb_, ob_, c[1]);
                }
#pragma unroll
                for (int sl = 0; sl < NSL; ++sl) {
                    if (MASK && sl > qh) continue;
                    // Future keys (key > q) get the score -inf, so p = 0 and dS = 0. Keys past T (loaded as
                    // key T - 1, and only in the last unit, whose one query tile is its diagonal) are future
                    // keys of every row before T, and their columns are never stored. Rows past T start
                    // from -inf (see below), so their p is 0 too.
                    if (MASK && sl == qh) {
                        const int key = kb0 + 32 * sl + l32;
                        const int qlo = key - qbase - 32 * qh - 4 * hh;  // offsets below this: future
#pragma unroll
                        for (int i = 0; i < 16; ++i)
                            s[sl][i] = (i >> 2) * 8 + (i & 3) >= qlo ? s[sl][i] : -INFINITY;
                    }
#pragma unroll
                    for (int i = 0; i < 16; ++i) {
                        const float p = fast_exp2(s[sl][i] * sl2);
                        dp[sl][i] *= p;
                        s[sl][i] = p;
                    }
#pragma unroll
                    for (int half = 0; half < 2; ++half) {
                        // 16-query chunk 2qh + half: queries 16(2qh+half) + (j/4)*8 + 4hh + j%4
                        const u16x8 pf = pack8<DT>(s[sl], 8 * half);
                        const u16x8 sf = pack8<DT>(dp[sl], 8 * half);
#pragma unroll
                        for (int dt = 0; dt < ND; ++dt) {
                            dv[sl][dt] = E::mfma(c[qh].gcol[half][dt], pf, dv[sl][dt]);
                            dk[sl][dt] = E::mfma(c[qh].qcol[half][dt], sf, dk[sl][dt]);
                        }
                    }
                }
            }
            if constexpr (DMA) {  // three MFMAs (two in a masked iteration, which has 48), then one copy
                                  // instruction, kDmaOps times (denser stalls on the copy path, sparser
                                  // leaves the last copies' latency exposed)
#pragma unroll
                for (int k = 0; k < kDmaOps; ++k) {
                    __builtin_amdgcn_sched_group_barrier(0x008, MASK ? 2 : 3, 0);
                    __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);
                }
            }
        };
        auto run = [&](auto dma_tag, int itn, const u16* qs, const u16* os, float* ls, int nitn, u16* nqs,
                       u16* nos, float* nls) {
            const int qbase = qbase_of(itn);
            // Rows past T (zero Q and dO rows; their -lse is row T - 1's, which with a zero score could
            // overflow p) start their scores from -inf instead, so their p is 0: patched in this wave's
            // copy of the -lse vector, which has landed.
            if (qbase + BM > T && lane >= T - qbase) ls[wave * 2 * BM + lane] = -INFINITY;
            if (kb0 + BNK - 1 > qbase)
                compute(std::true_type{}, dma_tag, qbase, qs, os, ls, nitn, nqs, nos, nls);
            else
                compute(std::false_type{}, dma_tag, qbase, qs, os, ls, nitn, nqs, nos, nls);
        };
        // Double-buffered: this wave's iteration j uses buffer j % 2 while j + 1 streams into the other.
        // The DMA into a buffer is issued only after this wave's own reads of it (iteration j - 1)
        // have returned, which their use by the MFMAs guarantees.
        for (int j = 0; j < nmine; j += 2) {  // iteration ifirst + wp is already in flight into buffer A
            const int itn = ifirst + wp + WPP * j;
            // This iteration's tiles, copied during the previous one. The first time with KVL, the second unit's K / V
            // copies, issued after the tiles, stay in flight.
            constexpr int kKvOps = 2 * (BNK * HD / 8) / (64 * NW);
            if (kvl && ui == 0 && j == 0)
                wait_vmem_keep<kKvOps>();
            else
                wait_vmem();
            if (ui == 0 && j == 0) NN_TL_BLOCK(kTlDkdv, kTlMtReady, __builtin_amdgcn_s_memtime());
            if (j + 1 < nmine)
                run(std::true_type{}, itn, qA, oA, lA, itn + WPP, qB, oB, lB);
            else
                run(std::false_type{}, itn, qA, oA, lA, 0, qB, oB, lB);
            if (j + 1 >= nmine) break;
            wait_vmem();
            if (j + 2 < nmine)
                run(std::true_type{}, itn + WPP, qB, oB, lB, itn + 2 * WPP, qA, oA, lA);
            else
                run(std::false_type{}, itn + WPP, qB, oB, lB, 0, qA, oA, lA);
        }

        // This wave is done with its tiles, its copies have landed (its last iteration issued none) and
        // its K / V registers are free: it issues the next unit's K / V loads (with KVL: already in kvS) and
        // first tiles (into its A slots) now, while it waits for the slower waves, and they stay in flight
        // through the reduction, which uses only the B buffers. The next unit's loop waits for them (vmcnt)
        // before reading either.
        if (ui < 2) NN_TL_WAVE(kTlDkdv, kTlExtra + 4 * ui + wave, __builtin_amdgcn_s_memtime());
        if (ui + 1 < nunits && active) {
            const int un = nkb - 1 - pj;
            // With KVL a unit change implies two units, i.e. kvl: the next unit's K / V are in kvS already.
            // (Compile-time, so that the K / V registers are free through the reduction.)
            if constexpr (!KVL) load_kv(un * BNK);
            const int n1 = group * (nqt - un), i1 = first_of(n1);
            if (wp < end_of(n1) - i1) issue_it(i1 + wp, un, qA, oA, lA);
        }
        // Sum each pair's WPP partial dK^T, then dV^T, and store the sums. A wave's partial is NCK chunks of
        // 1 KB: chunk c = (sl, dt, g) holds accumulator elements 4g .. 4g + 3 of acc[sl][dt] in every lane
        // (lane = key 32 sl + l32, element 4g + e = column 32 dt + 8g + 4hh + e). Chunk (sl, dt, g) belongs
        // to wave g % WPP of the pair: the pair's other waves stage their copies of it in their LDS slots,
        // and the owner adds them and its own in wave order. Each wave's slots are its own B tile slots,
        // which only it used in its loop and the next unit's first tiles leave alone: a wave stages as soon
        // as its loop is done, and with one wave per pair no wave waits for another. The LDS-only barriers
        // leave the next unit's loads in flight.
        // Without a split and with four waves on the pair, the owner rounds its sums to 16 bits and stores them
        // straight from registers (each store instruction covers 16 bytes of 32 gradient rows; measured 1-3 %
        // faster than the transpose below, which costs an LDS round trip and a barrier). With fewer waves per
        // pair a wave owns more chunks, and the transpose pays (direct stores: 2-4 % slower there): the owner
        // writes its 16-bit sums back into its own slot of the chunk (dK in the first half, dV in the second:
        // 32 rows of 16 bytes, row r at 16-byte group (r + j) % 32 with j = the chunk's 16-byte column group,
        // so that the groups of one gradient row fall in different banks); then the pair's waves store whole
        // gradient rows, 16 bytes per lane. With a split the owner stores its fp32 sums into the split's partial
        // directly.
        constexpr int NCK = NSL * ND * 4;
        constexpr int NG = HD / 8;  // 16-byte (8-column) groups per 16-bit gradient row
        static_assert(NCK / 2 * 1024 == QT * 2, "a wave's chunks fill its two B tile slots");
        auto slot = [&](int w, int c) {  // wave w's 1 KB slot for chunk c: half in its qB slot, half in oB
            return reinterpret_cast<char*>((c < NCK / 2 ? qB : oB) + w * QT) + (c % (NCK / 2)) * 1024;
        };
        auto row16 = [&](int w, int c, int which, int r) {  // 16-bit sums of row r (0..31) of chunk c
            return reinterpret_cast<u32x4*>(slot(w, c) + which * 512) + ((r + c % (4 * ND)) & 31);
        };
        auto reduce = [&](const f32x16 (&acc)[NSL][ND], float mul, int which) {
            auto chunk = [&](int c) {
                const f32x16& a = acc[c / (4 * ND)][c / 4 % ND];
                const int g = c % 4;
                return f32x4{a[4 * g], a[4 * g + 1], a[4 * g + 2], a[4 * g + 3]};
            };
            // P: this wave's place in its pair (a compile-time value per branch, so that the chunks it owns
            // are fixed registers).
            auto body = [&](auto p_tag) {
                constexpr int P = decltype(p_tag)::value;
                if constexpr (WPP > 1) {
#pragma unroll
                    for (int c = 0; c < NCK; ++c)
                        if (c % 4 % WPP != P) reinterpret_cast<f32x4*>(slot(wave, c))[lane] = chunk(c);
                    barrier_lds();
                }
                // The owned chunks: c = 4 i + P + WPP j (j < 4 / WPP). Every staged copy they need is read first,
                // then all the sums are formed, then stored: one block of code with no branch, so that the LDS
                // reads are in flight together and wait once. (Read and summed chunk by chunk between the stores,
                // whose bounds tests are branches, every read waited alone: dK/dV 1-5 % slower.)
                constexpr int GPW = 4 / WPP, NO = NCK / WPP;
                auto owned = [](int k) { return 4 * (k / GPW) + P + WPP * (k % GPW); };
                f32x4 copy[NO][WPP];
#pragma unroll
                for (int k = 0; k < NO; ++k)
#pragma unroll
                    for (int m = 0; m < WPP; ++m)
                        if (m != P) copy[k][m] = reinterpret_cast<const f32x4*>(slot(wave - P + m, owned(k)))[lane];
                f32x4 sum[NO];
#pragma unroll
                for (int k = 0; k < NO; ++k) {
                    // In wave order, starting from the pair's first wave's partial (0 + x is x: the partials are
                    // never -0, an MFMA chain from +0 cannot produce it).
                    sum[k] = P == 0 ? chunk(owned(k)) : copy[k][0];
#pragma unroll
                    for (int m = 1; m < WPP; ++m) sum[k] += m == P ? chunk(owned(k)) : copy[k][m];
                    sum[k] *= mul;
                }
                auto col_of = [&](int c) { return 32 * (c / 4 % ND) + 8 * (c % 4) + 4 * hh; };
                if (nsplit == 1 && WPP == NW) {  // the owner stores its 16-bit sums straight from registers
#pragma unroll
                    for (int sl = 0; sl < NSL; ++sl) {
                        const int key = kb0 + 32 * sl + l32;
                        if (active && key < T) {
                            u16* row = (which == 0 ? dK : dV) + kvoff + (size_t)key * lk.st;
#pragma unroll
                            for (int k = 0; k < NO; ++k)
                                if (owned(k) / (4 * ND) == sl)
                                    *reinterpret_cast<u32x2*>(row + col_of(owned(k))) =
                                        u32x2{E::pack2(sum[k][0], sum[k][1]), E::pack2(sum[k][2], sum[k][3])};
                        }
                    }
                } else if (nsplit == 1) {
#pragma unroll
                    for (int k = 0; k < NO; ++k)
                        reinterpret_cast<u32x2*>(row16(wave, owned(k), which, l32))[hh] =
                            u32x2{E::pack2(sum[k][0], sum[k][1]), E::pack2(sum[k][2], sum[k][3])};
                } else {  // this split's partial: part[split][dK | dV][bk][key][HD]
#pragma unroll
                    for (int sl = 0; sl < NSL; ++sl) {
                        const int key = kb0 + 32 * sl + l32;
                        if (active && key < T) {
                            float* row = part + (((size_t)sidx * 2 + which) * BKV + bk) * T * HD + (size_t)key * HD;
#pragma unroll
                            for (int k = 0; k < NO; ++k)
                                if (owned(k) / (4 * ND) == sl) *reinterpret_cast<f32x4*>(row + col_of(owned(k))) = sum[k];
                        }
                    }
                }
                if constexpr (WPP > 1) barrier_lds();  // staged copies read, 16-bit sums written
            };
            if constexpr (WPP == 1) {
                body(std::integral_constant<int, 0>{});
            } else {
                const int pu = __builtin_amdgcn_readfirstlane(wp);
                if (pu == 0) body(std::integral_constant<int, 0>{});
                else if (WPP == 2 || pu == 1) body(std::integral_constant<int, 1>{});
                else if constexpr (WPP == 4) {
                    if (pu == 2) body(std::integral_constant<int, 2>{});
                    else body(std::integral_constant<int, 3>{});
                }
            }
        };
        reduce(dk, scale, 0);
        reduce(dv, 1.f, 1);
        if (nsplit == 1 && WPP != NW) {
            // The pair's 64 x HD sums of each gradient: 64 NG groups of 16 bytes, 64 NG / WPP per wave.
#pragma unroll
            for (int k = 0; k < NG / WPP; ++k) {
                const int G = (wp * (NG / WPP) + k) * 64 + lane;  // group G: row G / NG, column group G % NG
                const int r = G / NG, j = G % NG;
                const int c = r / 32 * 4 * ND + j;  // the chunk holding it, and its owner
                const int ow = wave - wp + c % 4 % WPP;
                const u32x4 vk = *row16(ow, c, 0, r & 31), vv = *row16(ow, c, 1, r & 31);
                if (active && kb0 + r < T) {
                    const size_t off = kvoff + (size_t)(kb0 + r) * lk.st + 8 * j;
                    *reinterpret_cast<u32x4*>(dK + off) = vk;
                    *reinterpret_cast<u32x4*>(dV + off) = vv;
                }
            }
            if constexpr (WPP > 1) barrier_lds();  // the B buffers are free for the next unit
        }
        if (ui == 0) NN_TL_BLOCK(kTlDkdv, kTlExtra + 8, __builtin_amdgcn_s_memtime());
        if (ui + 1 < nunits) clear_acc();
    }
    NN_TL_END(kTlDkdv);
}

// ------------------------------------------------------------------------------------------
// Backward, dK / dV with nsplit > 1: dK, dV = the sum over splits s = 0, 1, ... (in that order) of
// part[s][dK | dV][bk][key][HD] (fp32, dK already scaled), rounded once to the output dtype. One
// thread per 4 consecutive columns; grid-stride.
// ------------------------------------------------------------------------------------------
template <int DT>
__global__ __launch_bounds__(256) void fa_bwd_dkdv_sum_kernel(const float* __restrict__ part, u16* __restrict__ dK,
                                                              u16* __restrict__ dV, int nsplit, int BKV, int KVH,
                                                              int T, int HD, Lay lk) {
    using E = Elem<DT>;
    const int64_t per = (int64_t)BKV * T * HD;  // elements of one gradient
    const int64_t n4 = 2 * per / 4;
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n4; i += (int64_t)gridDim.x * 256) {
        const int64_t e = 4 * i;
        const int which = (int)(e / per);
        const int64_t r = e - which * per;
        const int bk = (int)(r / ((int64_t)T * HD));
        const int64_t r2 = r - (int64_t)bk * T * HD;
        const int key = (int)(r2 / HD), col = (int)(r2 - (int64_t)key * HD);
        f32x4 acc = *reinterpret_cast<const f32x4*>(part + e);
        for (int s = 1; s < nsplit; ++s) acc += *reinterpret_cast<const f32x4*>(part + (int64_t)s * 2 * per + e);
        const int b = bk / KVH, kvh = bk - b * KVH;
        u16* dst = (which == 0 ? dK : dV) + lk.at(b, kvh) + (size_t)key * lk.st + col;
        *reinterpret_cast<u32x2*>(dst) = u32x2{E::pack2(acc[0], acc[1]), E::pack2(acc[2], acc[3])};
    }
}

// ------------------------------------------------------------------------------------------
// Backward, dQ. Shaped like the forward: block = 4 waves = 128 query rows of one (batch, head),
// 128-key tiles of K and V double-buffered in LDS by DMA and processed in 64-key halves, Q and dO rows
// in registers, lse and D per lane. Per 64-key half:
//   S^T = K Q^T, dP^T = V dO^T          (A = K / V rows from LDS, B = Q / dO registers)
//   dS^T = exp2((S^T - lse/scale) * sl2) (dP^T - D)
//   dQ^T += K^T dS^T                    (A = columns of the K tile, B = dS^T registers)
// dQ stays in registers for the whole key loop and is stored once, scaled, in the output dtype.
// ------------------------------------------------------------------------------------------
template <int HD, int DT, bool ROPE>
__global__ __launch_bounds__(256, 2) void fa_bwd_dq_kernel(const u16* __restrict__ Q, const u16* __restrict__ K,
                                                           const u16* __restrict__ V, const u16* __restrict__ O,
                                                           const u16* __restrict__ dO, const float* __restrict__ LSE,
                                                           float* __restrict__ nLvec, float* __restrict__ nDvec,
                                                           u16* __restrict__ dQ, int BH, int H, int KVH, int T, int nqb,
                                                           float sl2, float scale, Lay lq, Lay lk, RopeArgs ra) {
    using E = Elem<DT>;
    NN_TL_START(kTlDq);
    // LDS tiles of BT = 128 keys (one barrier and one tile wait per 128 keys), each processed as two BN = 64-key
    // halves (the register working set of a 64-key step).
    constexpr int BM = 128, BN = 64, NW = 4, BT = 128;
    constexpr int NS = HD / 16;
    constexpr int ND = HD / 32;
    constexpr int NT = BN / 32;
    constexpr int TILE = BT * HD;
    __shared__ __attribute__((aligned(16))) u16 kA[TILE];
    __shared__ __attribute__((aligned(16))) u16 vA[TILE];
    __shared__ __attribute__((aligned(16))) u16 kB[TILE];
    __shared__ __attribute__((aligned(16))) u16 vB[TILE];
    __shared__ __attribute__((aligned(16))) u16 oS[BM * HD];  // the block's O rows (for D)

    const QBlk blk = qblock_of(blockIdx.x, BH, H / KVH, nqb);
    const int bh = blk.bh, qb = blk.qb;
    const int b = bh / H, h = bh - b * H;
    const int kvh = h / (H / KVH);
    const size_t qoff = lq.at(b, h);
    const size_t kvoff = lk.at(b, kvh);
    const u16* Kp = K + kvoff;
    const u16* Vp = V + kvoff;

    const int tid = threadIdx.x, lane = tid & 63, l32 = lane & 31, hh = lane >> 5;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const DmaOffs<HD, BT, NW> dfo = dma_offsets<HD, BT, NW>(lane, wave, lk.st);
    const int g16 = (lane >> 4) & 1;
    const int q0 = qb * BM, qw = q0 + wave * 32, qrow = qw + l32;
    const int qc_ = min(qrow, T - 1);

    int koff[NS], kcol[ND][2];
#pragma unroll
    for (int ks = 0; ks < NS; ++ks) koff[ks] = row_off<HD>(l32, 16 * ks + 8 * hh);
#pragma unroll
    for (int dt = 0; dt < ND; ++dt)
#pragma unroll
        for (int x = 0; x < 2; ++x) kcol[dt][x] = col_off<HD>(8 * x + 4 * hh, 32 * dt + 16 * g16, lane);
    auto issue = [&](int it, u16* kb, u16* vb) {
        dma_rows<HD, BT, NW>(Kp, lk.st, it * BT, T, kb, wave, dfo);
        dma_rows<HD, BT, NW>(Vp, lk.st, it * BT, T, vb, wave, dfo);
    };
    // The first K / V tile, then this wave's 32 Q, dO and O rows by DMA (whole 128-byte rows per 8 lanes;
    // loaded per lane in the operand layout, each load instruction would touch 32 rows 32 bytes at a time):
    // Q and dO into its slices of the second tile buffers, which the loop's first copy overwrites only after
    // the block barrier, O into oS. Rows past T read as zeros.
    issue(0, kA, vA);
    const float lse = LSE[(size_t)bh * T + qc_];
    if (qw < T) {
        const DmaOffs<HD, 32, 1> rfo = dma_offsets<HD, 32, 1>(lane, 0, lq.st);
        dma_rows<HD, 32, 1>(Q + qoff, lq.st, qw, T, kB + 32 * wave * HD, 0, rfo);
        dma_rows<HD, 32, 1>(dO + qoff, lq.st, qw, T, vB + 32 * wave * HD, 0, rfo);
        dma_rows<HD, 32, 1>(O + qoff, lq.st, qw, T, oS + 32 * wave * HD, 0, rfo);
    }
    wait_vmem();
    // The preprocessing pass, for this block's rows: D = rowsum(dO * O) from the 16-bit O (each half-wave
    // holds half of a row; one exchange completes it), and -lse/scale. Every query row belongs to exactly
    // one dQ block, which also writes both into the workspace for the dK/dV kernel that runs next.
    u16x8 qf[NS], gf[NS];
    float dacc = 0.f;
#pragma unroll
    for (int s = 0; s < NS; ++s) {
        qf[s] = ld8(kB + 32 * wave * HD + koff[s]);
        gf[s] = ld8(vB + 32 * wave * HD + koff[s]);
        const u16x8 of = ld8(oS + 32 * wave * HD + koff[s]);
#pragma unroll
        for (int j = 0; j < 8; ++j) dacc = fmaf(E::to_f32(gf[s][j]), E::to_f32(of[j]), dacc);
    }
    const float nd = -pair_sum(dacc);
    const float nl2 = -lse * kLog2e;  // (-lse/scale) * sl2
    if (hh == 0 && qrow < T) {
        nDvec[(size_t)bh * T + qrow] = nd;
        nLvec[(size_t)bh * T + qrow] = -lse / scale;
    }
    NN_TL_BLOCK(kTlDq, kTlExtra, __builtin_amdgcn_s_memtime());

    f32x16 dq[ND];
#pragma unroll
    for (int dt = 0; dt < ND; ++dt) dq[dt] = f32x16{};

    const int ntiles = (min(q0 + BM, T) + BT - 1) / BT;
    NN_TL_BLOCK(kTlDq, kTlExtra + 1, (unsigned long long)ntiles);
    // -D enters as the initial value of every dP^T accumulator (the same for all of a lane's keys).
    f32x16 ndv;
#pragma unroll
    for (int i = 0; i < 16; ++i) ndv[i] = nd;
    // MASK: the tile crosses the diagonal or T (a separate instantiation, so that unmasked tiles
    // carry no per-element selects).
    // At head_dim 64 the dQ products of a half run after the masked / unmasked branch, in one copy for both
    // paths: with a copy inside each path, the two paths left dq in different registers and every half paid a
    // 16-instruction register copy (32 for masked halves) where they joined (dQ 2-7 % faster at configs 2 and 3
    // and the small shapes, flat at T = 8192, up to 4-5 % slower for B * T = 8192 at T >= 4096; slower at
    // head_dim 32, which keeps the products inside each path).
    constexpr bool kJoinDq = HD == 64;
    auto dq_products = [&](const u16* kb, const u16x8* sf) __attribute__((always_inline)) {
#pragma unroll
        for (int c = 0; c < BN / 16; ++c) {
            const u16* kc = kb + 16 * c * HD;
#pragma unroll
            for (int dt = 0; dt < ND; ++dt)
                dq[dt] = E::mfma(cat4(ld_tr(kc + kcol[dt][0]), ld_tr(kc + kcol[dt][1])), sf[c], dq[dt]);
        }
    };
    // sfo: this half's 16-bit dS^T operands (chunk c: keys 16c + (j/4)*8 + 4hh + j%4), with kJoinDq.
    auto tile = [&](auto mask_tag, int k0, const u16* kb, const u16* vb, u16x8* sfo) __attribute__((always_inline)) {
        constexpr bool MASK = decltype(mask_tag)::value;
        u16x8 ka[NT][NS], va[NT][NS];
#pragma unroll
        for (int t = 0; t < NT; ++t)
#pragma unroll
            for (int ks = 0; ks < NS; ++ks) {
                ka[t][ks] = ld8(kb + 32 * t * HD + koff[ks]);
                va[t][ks] = ld8(vb + 32 * t * HD + koff[ks]);
            }
        f32x16 s[NT], dp[NT];
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            s[t] = f32x16{};
            dp[t] = ndv;
#pragma unroll
            for (int ks = 0; ks < NS; ++ks) {
                s[t] = E::mfma(ka[t][ks], qf[ks], s[t]);
                dp[t] = E::mfma(va[t][ks], gf[ks], dp[t]);
            }
        }
        // s[t][i]: key k0 + 32t + (i/4)*8 + 4hh + i%4 against query qrow; dp[t][i] already holds dP - D.
        const int lim = min(qrow, T - 1) - k0 - 4 * hh;
        // The wave's smallest lim (lane 32: row qw, hh = 1): sub-tiles whose last key offset (32t + 27)
        // does not exceed it are visible to every lane and skip the per-element selects.
        const int lim_w = min(qw, T - 1) - k0 - 4;
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            if (MASK && 32 * t + 27 > lim_w) {  // masked scores become -inf, so their dS is 0
#pragma unroll
                for (int i = 0; i < 16; ++i) s[t][i] = 32 * t + (i >> 2) * 8 + (i & 3) > lim ? -INFINITY : s[t][i];
            }
#pragma unroll
            for (int i = 0; i < 16; ++i) dp[t][i] = fast_exp2(fmaf(s[t][i], sl2, nl2)) * dp[t][i];
        }
#pragma unroll
        for (int c = 0; c < BN / 16; ++c) sfo[c] = pack8<DT>(dp[c >> 1], 8 * (c & 1));  // keys 16c + (j/4)*8 + 4hh + j%4
        if constexpr (!kJoinDq) dq_products(kb, sfo);
    };
    auto half = [&](int k0, const u16* kb, const u16* vb) __attribute__((always_inline)) {
        if (qw >= T || k0 > qw + 31) return;  // no visible key in this half for this wave
        u16x8 sf[BN / 16];
        if (k0 + BN - 1 > qw || k0 + BN > T)
            tile(std::true_type{}, k0, kb, vb, sf);
        else
            tile(std::false_type{}, k0, kb, vb, sf);
        if constexpr (kJoinDq) dq_products(kb, sf);
    };
    auto step = [&](int it, const u16* kb, const u16* vb) __attribute__((always_inline)) {
        half(it * BT, kb, vb);
        half(it * BT + BN, kb + BN * HD, vb + BN * HD);
    };

    for (int it = 0; it < ntiles; it += 2) {
        wait_vmem();
        __syncthreads();
        if (it == 0) NN_TL_BLOCK(kTlDq, kTlMtReady, __builtin_amdgcn_s_memtime());
        if (it + 1 < ntiles) issue(it + 1, kB, vB);
        step(it, kA, vA);
        if (it + 1 >= ntiles) break;
        wait_vmem();
        __syncthreads();
        if (it + 2 < ntiles) issue(it + 2, kA, vA);
        step(it + 1, kB, vB);
    }

    if (qrow < T) {
        u16* dst = dQ + qoff + (size_t)qrow * lq.st;
        if constexpr (ROPE) {
            // The gradient reaching the rotated Q, rounded to the 16-bit type as a stored dQ would be, then the
            // rotation by -theta. Element i of dq[dt] is column c = 32 dt + (i / 4) * 8 + 4 hh + i % 4; its pair
            // (c + HD / 2) is element i of dq[1] (HD = 64) or element i + 8 of dq[0] (HD = 32).
            constexpr int HALF = HD / 2;
            const float* cr = ra.cosT + (size_t)qrow * HALF;
            const float* sr = ra.sinT + (size_t)qrow * HALF;
            float y[ND * 16];
#pragma unroll
            for (int dt = 0; dt < ND; ++dt)
#pragma unroll
                for (int i = 0; i < 16; ++i) {
                    const uint32_t w = E::pack2(dq[dt][i] * scale, 0.f);
                    y[dt * 16 + i] = E::to_f32((u16)(w & 0xFFFFu));
                }
            // Groups g of 4 consecutive low-half columns c0 = 8 g + 4 hh .. + 3: elements 4 g .. 4 g + 3 of y, and
            // their partners at y[16 + 4 g ..] (HD = 64, in dq[1]) or y[4 g + 8 ..] (HD = 32).
#pragma unroll
            for (int g = 0; g < ND * 2; ++g) {
                const int c0 = 8 * g + 4 * hh;
                const f32x4 cs = *reinterpret_cast<const f32x4*>(cr + c0), sn = *reinterpret_cast<const f32x4*>(sr + c0);
                const int lo = 4 * g, hi = HD == 64 ? 16 + 4 * g : 4 * g + 8;
                float r1[4], r2[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const float y1 = y[lo + e], y2 = y[hi + e];
                    r1[e] = add_rn(mul_rn(y1, cs[e]), mul_rn(y2, sn[e]));
                    r2[e] = sub_rn(mul_rn(y2, cs[e]), mul_rn(y1, sn[e]));
                }
                const int clo = c0, chi = c0 + HALF;
                *reinterpret_cast<u32x2*>(dst + clo) = u32x2{E::pack2(r1[0], r1[1]), E::pack2(r1[2], r1[3])};
                *reinterpret_cast<u32x2*>(dst + chi) = u32x2{E::pack2(r2[0], r2[1]), E::pack2(r2[2], r2[3])};
            }
        } else {
#pragma unroll
            for (int dt = 0; dt < ND; ++dt)
#pragma unroll
                for (int g = 0; g < 4; ++g) {
                    const f32x16& a = dq[dt];
                    u32x2 w = {E::pack2(a[4 * g] * scale, a[4 * g + 1] * scale), E::pack2(a[4 * g + 2] * scale, a[4 * g + 3] * scale)};
                    *reinterpret_cast<u32x2*>(dst + 32 * dt + 8 * g + 4 * hh) = w;
                }
        }
    }
    NN_TL_END(kTlDq);
}

// ------------------------------------------------------------------------------------------
// Host side.
// ------------------------------------------------------------------------------------------
thread_local std::string g_last_error;

int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
int fail(int code, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_last_error = buf;
    return code;
}

int launch_status(const char* what) {
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail((int)e, "%s launch failed: %s", what, hipGetErrorString(e));
    return 0;
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

int check_dims(int64_t B, int64_t H, int64_t KVH, int64_t T, int64_t D, int dtype) {
    if (B < 0 || H <= 0 || KVH <= 0 || T < 0)
        return fail(-1, "invalid sizes B=%lld H=%lld KVH=%lld T=%lld", (long long)B, (long long)H, (long long)KVH,
                    (long long)T);
    if (D != 32 && D != 64) return fail(-1, "head_dim must be 32 or 64");
    if (H % KVH != 0) return fail(-1, "query heads must group evenly over KV heads");
    if (dtype != kF16 && dtype != kBF16) return fail(-1, "inputs must be float16 or bfloat16");
    if (B * H * T * D >= ((int64_t)1 << 40) || T >= ((int64_t)1 << 30) || B * H >= ((int64_t)1 << 30))
        return fail(-1, "sizes too large");
    return 0;
}

// Backward workspace: nD = -rowsum(dO * o) and nL = -lse / scale, one fp32 per query row each.
struct Workspace {
    float* nD;
    float* nL;
    float* part;  // dK / dV split partials (nsplit > 1 only)
    int nsplit;
    size_t bytes;
};

size_t round256(size_t n) { return (n + 255) & ~(size_t)255; }

// Splits of the dK/dV work: one block per CU (256 on MI355X) is what fills the chip; below that, each
// block's work is shared by up to 16 blocks whose fp32 partials are summed afterwards, as long as
// every split keeps at least 8 of the pair's (query head, query tile) iterations (two per wave: a
// block's fixed cost is about that much work).
constexpr int64_t kDkdvFill = 256, kDkdvMaxSplit = 16, kDkdvMinIters = 8;
int dkdv_split(int64_t B, int64_t H, int64_t KVH, int64_t T) {
    if (B <= 0 || KVH <= 0 || H < KVH || T <= 0) return 1;
    const int64_t nkb = (T + 63) / 64, base = B * KVH * ((nkb + 1) / 2);
    if (base >= kDkdvFill) return 1;
    if ((H / KVH) * nkb * kDkdvMaxSplit >= ((int64_t)1 << 31)) return 1;  // the kernel's 32-bit split bounds
    const int64_t by_fill = (kDkdvFill + base - 1) / base, by_work = (H / KVH) * (nkb + 1) / kDkdvMinIters;
    return (int)std::max<int64_t>(1, std::min({kDkdvMaxSplit, by_fill, by_work}));
}

// Waves sharing one unit pair (1, 2 or 4; see dkdv_impl). Splitting (dkdv_split > 1) needs 4. Fewer waves
// per pair pay off while a pair's (query head, query tile) iterations are few enough that its fixed costs
// weigh (measured: 8-24 % faster at up to about 200 iterations); long pairs amortise those costs anyway,
// and four waves on one pair keep its Q / dO tiles in L2 (B=1, T=16384: two waves per pair 8 % slower).
constexpr int64_t kDkdvFewWavesMaxIters = 300;
int dkdv_waves_per_pair(int64_t B, int64_t H, int64_t KVH, int64_t T) {
    if (B <= 0 || KVH <= 0 || H < KVH || T <= 0) return 4;
    const int64_t nkb = (T + 63) / 64, pairs = B * KVH * ((nkb + 1) / 2);
    if ((H / KVH) * (nkb + 1) > kDkdvFewWavesMaxIters) return 4;
    return pairs >= 3 * kDkdvFill ? 1 : (pairs >= 2 * kDkdvFill ? 2 : 4);
}

// Units per dK/dV block and waves per unit. A block normally takes a unit pair; when the work is not split
// and four waves share each pair, small problems take single units instead, because a pair's second unit
// only lengthens the block that carries it (its loads, iterations and reduction come after the first's)
// while CUs sit idle:
//   * all the units fit in one block per CU (B=1, T=256): one unit per block, four waves on it;
//   * they fit in two (B=32, T=256): two units per block, two waves on each, as long as a wave's share
//     of the heaviest unit, ceil(g nqt / 2) iterations (g query heads per KV head), stays below a pair
//     wave's share, about ceil(g (nqt + 1) / 4), plus the unit change between the pair's units, which
//     costs about kDkdvUnitChangeIters iterations' time (its loop-end spread and reduction). Measured:
//     10-23 % faster at T <= 256, 9 % slower at B=16, T=512, where the rule keeps pairs.
struct DkdvMode {
    bool paired;
    int wpp;  // waves per pair, or per unit when unpaired
};
constexpr int64_t kDkdvUnitChangeIters = 3;
// The dK/dV grid: blocks of 4 waves, each wave on the (batch, KV head) of its pair or unit (4 / wpp of them per
// block), times the pairs or units of one (batch, KV head), times the splits.
int64_t dkdv_blocks(int64_t B, int64_t KVH, int64_t T, DkdvMode mode, int nsplit) {
    const int64_t nkb = (T + 63) / 64, ppb = 4 / mode.wpp, nbk = (B * KVH + ppb - 1) / ppb;
    return nbk * (mode.paired ? (nkb + 1) / 2 : nkb) * nsplit;
}
DkdvMode dkdv_mode(int64_t B, int64_t H, int64_t KVH, int64_t T) {
    const int wpp = dkdv_waves_per_pair(B, H, KVH, T);
    if (B <= 0 || KVH <= 0 || H < KVH || T <= 0 || dkdv_split(B, H, KVH, T) != 1 || wpp != 4) return {true, wpp};
    const int64_t nkb = (T + 63) / 64, units = B * KVH * nkb, g = H / KVH;
    if (units <= kDkdvFill) return {false, 4};
    if (units <= 2 * kDkdvFill && (g * nkb + 1) / 2 < (g * (nkb + 1) + 3) / 4 + kDkdvUnitChangeIters) return {false, 2};
    return {true, 4};
}

Workspace carve(void* base, int64_t B, int64_t H, int64_t KVH, int64_t T, int64_t D) {
    const size_t vec = round256(4 * (size_t)B * H * T);
    Workspace w;
    w.nsplit = dkdv_split(B, H, KVH, T);
    w.nD = (float*)base;
    w.nL = (float*)((char*)base + vec);
    w.part = w.nsplit > 1 ? (float*)((char*)base + 2 * vec) : nullptr;
    w.bytes = 2 * vec + (w.nsplit > 1 ? round256((size_t)w.nsplit * 2 * 4 * B * KVH * T * D) : 0);
    return w;
}

template <int HD, int DT>
int fwd_impl(const void* q, const void* k, const void* v, void* o, float* lse, int64_t B, int64_t H, int64_t KVH,
             int64_t T, float scale, Lay lq, Lay lk, RopeArgs ra, hipStream_t st) {
    const int nqb = (int)((T + 127) / 128);
    const int BH = (int)(B * H);
    auto launch = [&](auto kern) {
        kern<<<dim3(nqb * BH), dim3(256), 0, st>>>((const u16*)q, (const u16*)k, (const u16*)v, (u16*)o, lse, BH, (int)H,
                                                   (int)KVH, (int)T, nqb, scale * kLog2e, lq, lk, ra);
    };
    if (ra.cosT)
        launch(fa_fwd_kernel<HD, DT, true>);
    else
        launch(fa_fwd_kernel<HD, DT, false>);
    return launch_status("fa_fwd_kernel");
}

template <int HD, int DT>
int pre_impl(const void* o, const void* dO, const float* lse, const Workspace& w, int64_t B, int64_t H, int64_t KVH,
             int64_t T, float scale, Lay lq, hipStream_t st) {
    (void)KVH;
    const int64_t rows = B * H * T;
    const int64_t blocks = (rows * (HD / 8) + 255) / 256;
    fa_bwd_pre_kernel<HD, DT><<<dim3((unsigned)blocks), dim3(256), 0, st>>>(
        (const u16*)o, (const u16*)dO, lse, w.nD, w.nL, rows, (int)H, (int)T, 1.0f / scale, lq);
    return launch_status("fa_bwd_pre_kernel");
}

template <int HD, int DT>
int dkdv_impl(const void* q, const void* k, const void* v, const void* dO, const Workspace& w, void* dk, void* dv,
              int64_t B, int64_t H, int64_t KVH, int64_t T, float scale, Lay lq, Lay lk, hipStream_t st) {
    const int nkb = (int)((T + 63) / 64);  // 64-key units
    const int nqt = nkb;                   // 64-row query tiles
    const int npairs = (nkb + 1) / 2;
    const int BKV = (int)(B * KVH);
    // Waves per unit pair: 4 while the pairs do not fill two blocks per CU; with more pairs, fewer waves
    // share each pair (a block then hosts 2 or 4 pairs), so that the per-unit costs (loads, barrier,
    // reduction) are paid by fewer, longer blocks.
    const DkdvMode mode = dkdv_mode(B, H, KVH, T);
    const int wpp = mode.wpp;
    const bool paired = mode.paired;
    auto launch = [&](auto kern, int ppb) {
        kern<<<dim3((unsigned)dkdv_blocks(B, KVH, T, mode, w.nsplit)), dim3(256), 0, st>>>(
            (const u16*)q, (const u16*)k, (const u16*)v, (const u16*)dO, w.nL, w.nD, (u16*)dk, (u16*)dv, BKV, (int)H,
            (int)KVH, (int)T, nkb, nqt, scale * kLog2e, scale, lq, lk, w.nsplit, w.part, paired ? 1 : 0);
    };
    // K / V through LDS (KVL) for pairs at head_dim 64 up to T = 2048: measured 1-3.4 % faster there (config 2:
    // -3 %), within noise or slower at T >= 4096 and at head_dim 32, where the direct loads stay.
    if (wpp == 1)
        launch(fa_bwd_dkdv_kernel<HD, DT, 1, false>, 4);
    else if (wpp == 2)
        launch(fa_bwd_dkdv_kernel<HD, DT, 2, false>, 2);
    else if (HD == 64 && paired && nkb <= 32)
        launch(fa_bwd_dkdv_kernel<HD, DT, 4, true>, 1);
    else
        launch(fa_bwd_dkdv_kernel<HD, DT, 4, false>, 1);
    (void)npairs;
    if (int e = launch_status("fa_bwd_dkdv_kernel")) return e;
    if (w.nsplit == 1) return 0;
    const int64_t n4 = 2 * (int64_t)BKV * T * HD / 4;
    const int blocks = (int)std::min<int64_t>((n4 + 255) / 256, 2048);
    fa_bwd_dkdv_sum_kernel<DT><<<dim3(blocks), dim3(256), 0, st>>>(w.part, (u16*)dk, (u16*)dv, w.nsplit, BKV, (int)KVH,
                                                                   (int)T, HD, lk);
    return launch_status("fa_bwd_dkdv_sum_kernel");
}

template <int HD, int DT>
int dq_impl(const void* q, const void* k, const void* v, const void* o, const void* dO, const float* lse,
            const Workspace& w, void* dq, int64_t B, int64_t H, int64_t KVH, int64_t T, float scale, Lay lq, Lay lk,
            RopeArgs ra, hipStream_t st) {
    const int nqb = (int)((T + 127) / 128);
    const int BH = (int)(B * H);
    auto launch = [&](auto kern) {
        kern<<<dim3(nqb * BH), dim3(256), 0, st>>>((const u16*)q, (const u16*)k, (const u16*)v, (const u16*)o,
                                                   (const u16*)dO, lse, w.nL, w.nD, (u16*)dq, BH, (int)H, (int)KVH,
                                                   (int)T, nqb, scale * kLog2e, scale, lq, lk, ra);
    };
    if (ra.cosT)
        launch(fa_bwd_dq_kernel<HD, DT, true>);
    else
        launch(fa_bwd_dq_kernel<HD, DT, false>);
    return launch_status("fa_bwd_dq_kernel");
}

// Dense [B][heads][T][D] layout.
Lay contiguous(int64_t heads, int64_t T, int64_t D) { return Lay{(long long)(heads * T * D), (long long)(T * D), (int)D}; }

// Validates caller-given element strides {batch, head, row} of a [B][heads][T][D] view with unit D
// stride: every stride a positive multiple of 8 elements (16-byte rows, so tiles move 16 bytes
// per lane), rows at least D apart, and row offsets inside one (batch, head) slice below 2^30.
int take_layout(const int64_t* strides, int64_t heads, int64_t T, int64_t D, const char* what, Lay* out) {
    if (!strides) return fail(-1, "null %s strides", what);
    const int64_t sb = strides[0], sh = strides[1], st = strides[2];
    if (sb <= 0 || sh <= 0 || st <= 0 || sb % 8 || sh % 8 || st % 8)
        return fail(-1, "%s strides must be positive multiples of 8 elements", what);
    if (st < D) return fail(-1, "%s row stride is smaller than head_dim", what);
    if (T * st >= ((int64_t)1 << 30) || sb >= ((int64_t)1 << 40) || sh * heads >= ((int64_t)1 << 40))
        return fail(-1, "%s strides too large", what);
    *out = Lay{(long long)sb, (long long)sh, (int)st};
    return 0;
}

int check_ws(void* workspace, size_t workspace_bytes, int64_t B, int64_t H, int64_t KVH, int64_t T, int64_t D) {
    if (!workspace) return fail(-1, "null workspace");
    if (((uintptr_t)workspace & 255u) != 0) return fail(-1, "workspace must be 256-byte aligned");
    const size_t need = carve(nullptr, B, H, KVH, T, D).bytes;
    if (workspace_bytes < need) return fail(-1, "workspace too small: %zu bytes given, %zu needed", workspace_bytes, need);
    return 0;
}

}  // namespace

// Dispatch on (head_dim, dtype) for the templated stages.
#define NNFA_DISPATCH(FN, D, DT, ...)                                 \
    ((D) == 64 ? ((DT) == kBF16 ? FN<64, kBF16>(__VA_ARGS__)          \
                                : FN<64, kF16>(__VA_ARGS__))          \
               : ((DT) == kBF16 ? FN<32, kBF16>(__VA_ARGS__)          \
                                : FN<32, kF16>(__VA_ARGS__)))

NNFA_API const char* nn_fa_last_error(void) { return g_last_error.c_str(); }

NNFA_API int nn_fa_abi_version(void) { return 10; }

NNFA_API size_t nn_fa_bwd_workspace_size(int64_t B, int64_t H, int64_t KVH, int64_t T, int64_t D) {
    if (B < 0 || H < 0 || KVH < 0 || T < 0 || D < 0) return 0;
    return carve(nullptr, B, H, KVH, T, D).bytes;
}

NNFA_API int nn_fa_bwd_plan(int64_t B, int64_t H, int64_t KVH, int64_t T, int* nsplit, int* waves, int* paired,
                            int64_t* blocks) {
    g_last_error.clear();
    if (!nsplit || !waves || !paired || !blocks) return fail(-1, "nn_fa_bwd_plan: null output pointer");
    if (int e = check_dims(B, H, KVH, T, 64, kBF16)) return e;
    const DkdvMode mode = dkdv_mode(B, H, KVH, T);
    *nsplit = dkdv_split(B, H, KVH, T);
    *waves = mode.wpp;
    *paired = mode.paired ? 1 : 0;
    *blocks = B == 0 || T == 0 ? 0 : dkdv_blocks(B, KVH, T, mode, *nsplit);
    return 0;
}

namespace {

// The RoPE tables of the rope-fused entry points: non-null, 16-byte aligned, at least T rows.
int check_rope(const float* cos_table, const float* sin_table, int64_t table_rows, int64_t T) {
    if (!cos_table || !sin_table) return fail(-1, "null RoPE table");
    if (((uintptr_t)cos_table & 15u) || ((uintptr_t)sin_table & 15u)) return fail(-1, "RoPE tables must be 16-byte aligned");
    if (table_rows < T)
        return fail(-1, "sequence length %lld exceeds the %lld rows of the RoPE tables", (long long)T, (long long)table_rows);
    return 0;
}

int fwd_entry(const void* q, const void* k, const void* v, void* o, float* lse, int64_t B, int64_t H, int64_t KVH,
              int64_t T, int64_t D, int dtype, float scale, const int64_t* qo_strides, const int64_t* kv_strides,
              void* stream, RopeArgs ra = {}, int64_t table_rows = 0) {
    g_last_error.clear();
    if (int e = check_dims(B, H, KVH, T, D, dtype)) return e;
    if (B == 0 || T == 0) return 0;
    if (!q || !k || !v || !o || !lse) return fail(-1, "null pointer argument");
    if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(o)) return fail(-1, "inputs must be 16-byte aligned");
    if (ra.cosT || ra.sinT || ra.qrot) {
        if (int e = check_rope(ra.cosT, ra.sinT, table_rows, T)) return e;
        if (!ra.qrot || !aligned16(ra.qrot)) return fail(-1, "q_rot must be a 16-byte aligned buffer");
    }
    Lay lq = contiguous(H, T, D), lk = contiguous(KVH, T, D);
    if (qo_strides)
        if (int e = take_layout(qo_strides, H, T, D, "q/o", &lq)) return e;
    if (kv_strides)
        if (int e = take_layout(kv_strides, KVH, T, D, "k/v", &lk)) return e;
    return NNFA_DISPATCH(fwd_impl, D, dtype, q, k, v, o, lse, B, H, KVH, T, scale, lq, lk, ra, (hipStream_t)stream);
}

// Shared argument checks of the backward stages; fills the workspace view and the two layouts.
int bwd_prologue(const void* workspace, size_t workspace_bytes, int64_t B, int64_t H, int64_t KVH, int64_t T,
                 int64_t D, int dtype, const int64_t* qo_strides, const int64_t* kv_strides, Workspace* w, Lay* lq,
                 Lay* lk) {
    g_last_error.clear();
    if (int e = check_dims(B, H, KVH, T, D, dtype)) return e;
    if (B == 0 || T == 0) return 1;  // nothing to do
    if (int e = check_ws((void*)workspace, workspace_bytes, B, H, KVH, T, D)) return e;
    *w = carve((void*)workspace, B, H, KVH, T, D);
    *lq = contiguous(H, T, D);
    *lk = contiguous(KVH, T, D);
    if (qo_strides)
        if (int e = take_layout(qo_strides, H, T, D, "q/o", lq)) return e;
    if (kv_strides)
        if (int e = take_layout(kv_strides, KVH, T, D, "k/v", lk)) return e;
    return 0;
}

int pre_entry(const void* o, const void* dO, const float* lse, void* workspace, size_t workspace_bytes, int64_t B,
              int64_t H, int64_t KVH, int64_t T, int64_t D, int dtype, float scale, const int64_t* qo_strides,
              void* stream) {
    Workspace w;
    Lay lq, lk;
    if (int e = bwd_prologue(workspace, workspace_bytes, B, H, KVH, T, D, dtype, qo_strides, nullptr, &w, &lq, &lk))
        return e > 0 ? 0 : e;
    if (!o || !dO || !lse) return fail(-1, "null pointer argument");
    if (!aligned16(o) || !aligned16(dO)) return fail(-1, "inputs must be 16-byte aligned");
    if (!(scale > 0.f)) return fail(-1, "scale must be positive");
    return NNFA_DISPATCH(pre_impl, D, dtype, o, dO, lse, w, B, H, KVH, T, scale, lq, (hipStream_t)stream);
}

int dkdv_entry(const void* q, const void* k, const void* v, const void* dO, void* workspace,
               size_t workspace_bytes, void* dk, void* dv, int64_t B, int64_t H, int64_t KVH, int64_t T, int64_t D,
               int dtype, float scale, const int64_t* qo_strides, const int64_t* kv_strides, void* stream) {
    Workspace w;
    Lay lq, lk;
    if (int e = bwd_prologue(workspace, workspace_bytes, B, H, KVH, T, D, dtype, qo_strides, kv_strides, &w, &lq, &lk))
        return e > 0 ? 0 : e;
    if (!q || !k || !v || !dO || !dk || !dv) return fail(-1, "null pointer argument");
    if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(dO) || !aligned16(dk) || !aligned16(dv))
        return fail(-1, "inputs must be 16-byte aligned");
    return NNFA_DISPATCH(dkdv_impl, D, dtype, q, k, v, dO, w, dk, dv, B, H, KVH, T, scale, lq, lk, (hipStream_t)stream);
}

int dq_entry(const void* q, const void* k, const void* v, const void* o, const void* dO, const float* lse,
             void* workspace, size_t workspace_bytes, void* dq, int64_t B, int64_t H, int64_t KVH, int64_t T,
             int64_t D, int dtype, float scale, const int64_t* qo_strides, const int64_t* kv_strides, void* stream,
             RopeArgs ra = {}, int64_t table_rows = 0) {
    Workspace w;
    Lay lq, lk;
    if (int e = bwd_prologue(workspace, workspace_bytes, B, H, KVH, T, D, dtype, qo_strides, kv_strides, &w, &lq, &lk))
        return e > 0 ? 0 : e;
    if (!q || !k || !v || !o || !dO || !lse || !dq) return fail(-1, "null pointer argument");
    if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(o) || !aligned16(dO) || !aligned16(dq))
        return fail(-1, "inputs must be 16-byte aligned");
    if (!(scale > 0.f)) return fail(-1, "scale must be positive");
    if (ra.cosT || ra.sinT)
        if (int e = check_rope(ra.cosT, ra.sinT, table_rows, T)) return e;
    return NNFA_DISPATCH(dq_impl, D, dtype, q, k, v, o, dO, lse, w, dq, B, H, KVH, T, scale, lq, lk, ra,
                         (hipStream_t)stream);
}

int bwd_entry(const void* dO, const void* q, const void* k, const void* v, const void* o, const float* lse, void* dq,
              void* dk, void* dv, void* workspace, size_t workspace_bytes, int64_t B, int64_t H, int64_t KVH,
              int64_t T, int64_t D, int dtype, float scale, const int64_t* qo_strides, const int64_t* kv_strides,
              void* stream, RopeArgs ra = {}, int64_t table_rows = 0) {
    // Every argument of the three stages is checked before the first launch.
    Workspace w;
    Lay lq, lk;
    if (int e = bwd_prologue(workspace, workspace_bytes, B, H, KVH, T, D, dtype, qo_strides, kv_strides, &w, &lq, &lk))
        return e > 0 ? 0 : e;
    if (!dO || !q || !k || !v || !o || !lse || !dq || !dk || !dv) return fail(-1, "null pointer argument");
    if (!aligned16(dO) || !aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(o) || !aligned16(dq) ||
        !aligned16(dk) || !aligned16(dv))
        return fail(-1, "inputs must be 16-byte aligned");
    if (!(scale > 0.f)) return fail(-1, "scale must be positive");
    if (ra.cosT || ra.sinT)
        if (int e = check_rope(ra.cosT, ra.sinT, table_rows, T)) return e;
    // dQ first: it also computes -D and -lse/scale for its rows into the workspace (the preprocessing
    // pass, fused), which the dK/dV kernel reads.
    if (int e = dq_entry(q, k, v, o, dO, lse, workspace, workspace_bytes, dq, B, H, KVH, T, D, dtype, scale, qo_strides,
                         kv_strides, stream, ra, table_rows))
        return e;
    return dkdv_entry(q, k, v, dO, workspace, workspace_bytes, dk, dv, B, H, KVH, T, D, dtype, scale, qo_strides,
                      kv_strides, stream);
}

}  // namespace

NNFA_API int nn_fa_fwd(const void* q, const void* k, const void* v, void* o, float* lse, int64_t B, int64_t H,
                       int64_t KVH, int64_t T, int64_t D, int dtype, float scale, void* stream) {
    return fwd_entry(q, k, v, o, lse, B, H, KVH, T, D, dtype, scale, nullptr, nullptr, stream);
}

NNFA_API int nn_fa_fwd_strided(const void* q, const void* k, const void* v, void* o, float* lse, int64_t B, int64_t H,
                               int64_t KVH, int64_t T, int64_t D, const int64_t* qo_strides, const int64_t* kv_strides,
                               int dtype, float scale, void* stream) {
    if (!qo_strides || !kv_strides) return fail(-1, "null strides");
    return fwd_entry(q, k, v, o, lse, B, H, KVH, T, D, dtype, scale, qo_strides, kv_strides, stream);
}

NNFA_API int nn_fa_bwd_pre(const void* o, const void* dO, const float* lse, void* workspace, size_t workspace_bytes,
                           int64_t B, int64_t H, int64_t KVH, int64_t T, int64_t D, int dtype, float scale,
                           void* stream) {
    return pre_entry(o, dO, lse, workspace, workspace_bytes, B, H, KVH, T, D, dtype, scale, nullptr, stream);
}

NNFA_API int nn_fa_bwd_dkdv(const void* q, const void* k, const void* v, const void* dO, void* workspace,
                            size_t workspace_bytes, void* dk, void* dv, int64_t B, int64_t H, int64_t KVH, int64_t T,
                            int64_t D, int dtype, float scale, void* stream) {
    return dkdv_entry(q, k, v, dO, workspace, workspace_bytes, dk, dv, B, H, KVH, T, D, dtype, scale, nullptr, nullptr,
                      stream);
}

NNFA_API int nn_fa_bwd_dq(const void* q, const void* k, const void* v, const void* o, const void* dO, const float* lse,
                          void* workspace, size_t workspace_bytes, void* dq, int64_t B, int64_t H, int64_t KVH,
                          int64_t T, int64_t D, int dtype, float scale, void* stream) {
    return dq_entry(q, k, v, o, dO, lse, workspace, workspace_bytes, dq, B, H, KVH, T, D, dtype, scale, nullptr,
                    nullptr, stream);
}

NNFA_API int nn_fa_bwd(const void* dO, const void* q, const void* k, const void* v, const void* o, const float* lse,
                       void* dq, void* dk, void* dv, void* workspace, size_t workspace_bytes, int64_t B, int64_t H,
                       int64_t KVH, int64_t T, int64_t D, int dtype, float scale, void* stream) {
    return bwd_entry(dO, q, k, v, o, lse, dq, dk, dv, workspace, workspace_bytes, B, H, KVH, T, D, dtype, scale,
                     nullptr, nullptr, stream);
}

NNFA_API int nn_fa_bwd_strided(const void* dO, const void* q, const void* k, const void* v, const void* o,
                               const float* lse, void* dq, void* dk, void* dv, void* workspace, size_t workspace_bytes,
                               int64_t B, int64_t H, int64_t KVH, int64_t T, int64_t D, const int64_t* qo_strides,
                               const int64_t* kv_strides, int dtype, float scale, void* stream) {
    if (!qo_strides || !kv_strides) return fail(-1, "null strides");
    return bwd_entry(dO, q, k, v, o, lse, dq, dk, dv, workspace, workspace_bytes, B, H, KVH, T, D, dtype, scale,
                     qo_strides, kv_strides, stream);
}

NNFA_API int nn_fa_fwd_rope_strided(const void* q, const void* k, const void* v, void* o, float* lse, void* q_rot,
                                    const float* cos_table, const float* sin_table, int64_t table_rows, int64_t B,
                                    int64_t H, int64_t KVH, int64_t T, int64_t D, const int64_t* qo_strides,
                                    const int64_t* kv_strides, int dtype, float scale, void* stream) {
    if (!qo_strides || !kv_strides) return fail(-1, "null strides");
    const RopeArgs ra{cos_table, sin_table, (u16*)q_rot};
    if (!cos_table || !sin_table || !q_rot) return fail(-1, "null RoPE table or q_rot");
    return fwd_entry(q, k, v, o, lse, B, H, KVH, T, D, dtype, scale, qo_strides, kv_strides, stream, ra, table_rows);
}

NNFA_API int nn_fa_bwd_rope_strided(const void* dO, const void* q_rot, const void* k, const void* v, const void* o,
                                    const float* lse, void* dq, void* dk, void* dv, void* workspace,
                                    size_t workspace_bytes, const float* cos_table, const float* sin_table,
                                    int64_t table_rows, int64_t B, int64_t H, int64_t KVH, int64_t T, int64_t D,
                                    const int64_t* qo_strides, const int64_t* kv_strides, int dtype, float scale,
                                    void* stream) {
    if (!qo_strides || !kv_strides) return fail(-1, "null strides");
    if (!cos_table || !sin_table) return fail(-1, "null RoPE table");
    const RopeArgs ra{cos_table, sin_table, nullptr};
    return bwd_entry(dO, q_rot, k, v, o, lse, dq, dk, dv, workspace, workspace_bytes, B, H, KVH, T, D, dtype, scale,
                     qo_strides, kv_strides, stream, ra, table_rows);
}

// ------------------------------------------------------------------------------------------
// Backward with no allocation at all: the workspace of nn_fa_bwd (-D, -lse/scale and, for split shapes,
// the dK/dV partials) lives in this file-scope device array instead of a caller buffer. Each GPU the
// library runs on holds its own copy for the life of the process. Every call on one GPU uses that GPU's
// copy, so calls that overlap on one GPU (concurrent streams, or threads) race on it; calls in stream
// order do not. Nothing in it needs to start at zero: the dQ kernel writes every -D / -lse/scale entry
// before the dK/dV kernel reads it, and every split partial is written before the sum kernel reads it.
// ------------------------------------------------------------------------------------------
constexpr size_t kNoAllocScratchBytes = (size_t)32 << 20;
static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices];  // device address of `scratch` on each device, looked up once per device

// The device address of `scratch` on the current device (which must own `stream`). In host code the
// array's name is only a host-side handle; hipGetSymbolAddress, with the device current, gives that
// device's copy. Looked up on the first call on each device and kept.
int scratch_ptr(void* stream, void** out) {
    int dev = -1;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return fail((int)e, "hipGetDevice failed: %s", hipGetErrorString(e));
    if (dev < 0 || dev >= kMaxDevices) return fail(-1, "device %d is out of the supported range", dev);
    if (stream) {
        int sdev = -1;
        e = hipStreamGetDevice((hipStream_t)stream, &sdev);
        if (e != hipSuccess) return fail((int)e, "hipStreamGetDevice failed: %s", hipGetErrorString(e));
        if (sdev != dev) return fail(-1, "the stream belongs to device %d but device %d is current", sdev, dev);
    }
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p)
            return fail(e != hipSuccess ? (int)e : -1, "hipGetSymbolAddress(scratch) failed on device %d: %s", dev,
                        hipGetErrorString(e));
        g_scratch_ptr[dev] = p;
    }
    *out = g_scratch_ptr[dev];
    return 0;
}

}  // namespace

NNFA_API int nn_fa_bwd_noalloc(const void* dO, const void* q, const void* k, const void* v, const void* o,
                               const float* lse, void* dq, void* dk, void* dv, int64_t B, int64_t H, int64_t KVH,
                               int64_t T, int64_t D, int dtype, float scale, void* stream) {
    g_last_error.clear();
    if (int e = check_dims(B, H, KVH, T, D, dtype)) return e;
    if (B == 0 || T == 0) return 0;
    const size_t need = carve(nullptr, B, H, KVH, T, D).bytes;
    if (need > kNoAllocScratchBytes)
        return fail(-1, "nn_fa_bwd_noalloc: this shape needs %zu bytes of workspace, more than the %zu-byte scratch; "
                    "use nn_fa_bwd with a caller workspace", need, kNoAllocScratchBytes);
    void* ws = nullptr;
    if (int e = scratch_ptr(stream, &ws)) return e;
    return bwd_entry(dO, q, k, v, o, lse, dq, dk, dv, ws, kNoAllocScratchBytes, B, H, KVH, T, D, dtype, scale, nullptr,
                     nullptr, stream);
}

#if NN_TIMELINE
// ------------------------------------------------------------------------------------------
// Diagnostic build only: access to the block timelines (see NN_TL_START). Not part of the C ABI in
// include/nanonemo_fa.h; bench.py --timeline is the one caller. Both functions synchronise the device.
// ------------------------------------------------------------------------------------------
namespace {
int timeline_ptr(unsigned long long** out) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(nn_timeline));
    if (e != hipSuccess || !p)
        return fail(e != hipSuccess ? (int)e : -1, "hipGetSymbolAddress(nn_timeline) failed: %s", hipGetErrorString(e));
    *out = static_cast<unsigned long long*>(p);
    return 0;
}
}  // namespace

// Record layout: kTlKernels kernels x kTlBlocks blocks x kTlWords words (see TlWord).
NNFA_API int nn_fa_timeline_dims(int* kernels, int* blocks, int* words) {
    *kernels = kTlKernels;
    *blocks = kTlBlocks;
    *words = kTlWords;
    return 0;
}

// Zero every record on the current device.
NNFA_API int nn_fa_timeline_clear(void) {
    g_last_error.clear();
    unsigned long long* p = nullptr;
    if (int e = timeline_ptr(&p)) return e;
    hipError_t e = hipDeviceSynchronize();
    if (e == hipSuccess) e = hipMemset(p, 0, sizeof(unsigned long long) * kTlKernels * kTlBlocks * kTlWords);
    if (e == hipSuccess) e = hipDeviceSynchronize();
    return e == hipSuccess ? 0 : fail((int)e, "timeline clear failed: %s", hipGetErrorString(e));
}

// Copy the records of kernel `kernel` (a TlKernel), blocks 0 .. nblocks - 1, to host memory `out`.
NNFA_API int nn_fa_timeline_read(int kernel, unsigned long long* out, int nblocks) {
    g_last_error.clear();
    if (kernel < 0 || kernel >= kTlKernels || nblocks < 0 || nblocks > kTlBlocks || !out)
        return fail(-1, "nn_fa_timeline_read: invalid arguments");
    unsigned long long* p = nullptr;
    if (int e = timeline_ptr(&p)) return e;
    hipError_t e = hipDeviceSynchronize();
    if (e == hipSuccess)
        e = hipMemcpy(out, p + (size_t)kernel * kTlBlocks * kTlWords, sizeof(unsigned long long) * nblocks * kTlWords,
                      hipMemcpyDeviceToHost);
    return e == hipSuccess ? 0 : fail((int)e, "timeline read failed: %s", hipGetErrorString(e));
}
#endif
