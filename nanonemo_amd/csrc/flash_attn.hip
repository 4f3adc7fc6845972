// Causal grouped-query FlashAttention-2, forward and backward, for MI355X (gfx950, CDNA4).
//
// Semantics follow /root/reference/nanonemo/kernels/cuda/flash_attn.cu (fwd_kernel :52-174,
// bwd_kernel :176-340, host wrappers :342-405); the design is written for CDNA4 wave64 + MFMA:
//
//   * All products run on v_mfma_f32_32x32x16_{bf16,f16} with fp32 accumulators in VGPRs. One
//     wave owns a 32-wide slab of the sequence dimension; LDS holds tiles shared by the block.
//   * Tiles move global -> LDS with global_load_lds_dwordx4 (no staging registers) into
//     row-major tiles whose 16-byte chunks are XOR-swizzled by row. Operands that need a
//     row of a tile are read with ds_read_b128; operands that need a column (the transposed
//     products) are read with ds_read_b64_tr_b16, so no transposed copy is ever stored.
//   * Forward computes S^T = K Q^T so that each lane owns one query row (lane % 32) and the
//     keys sit in its accumulator registers: the row max/sum are in-lane reductions plus one
//     exchange with the other half-wave, and P^T feeds O^T += V^T P^T straight from registers.
//     The running max is only moved when it grows by more than 2^8 (in base 2), so most tiles
//     skip rescaling O; the row sum adds the 16-bit P that the product actually uses.
//   * Backward: one block per (batch, KV head, 128-key block, chunk of query tiles). It loops
//     over the H/KVH query heads of the group, so dK/dV of the group are summed in registers.
//     S = Q K^T and dP = dO V^T land with the key on the lane, so P and dS feed
//     dV^T += dO^T P and dK^T += Q^T dS as B operands; dS^T goes to LDS for dQ = dS K, which
//     is accumulated in fp32 with atomics. dK/dV leave through LDS as coalesced fp32 atomics.
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

#include <string>

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

constexpr int kF16 = 0;
constexpr int kBF16 = 1;
constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;
// The forward keeps a stale running max until a row's max grows by more than this (base-2
// units): p = exp2(s - m) then stays <= 2^8, far inside fp32 and the 16-bit formats.
constexpr float kRescaleLog2 = 8.0f;

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
__device__ inline u16x8 ld8(const u16* p) { return *reinterpret_cast<const u16x8*>(p); }

// Element offset of (row, col) in a row-major LDS tile of W 16-bit columns whose 16-byte chunks
// are XOR-swizzled by the row index (spreads column reads of consecutive rows over the banks).
template <int W>
__device__ inline int swz(int row, int col) {
    constexpr int CH = W / 8;
    return row * W + ((((col >> 3) ^ row) & (CH - 1)) << 3) + (col & 7);
}

// Column operand: rows r0..r0+3 of column c0 + lane%16 of a swizzled row-major tile
// (ds_read_b64_tr_b16; r0 and c0 must be the same across each 16-lane group, c0 % 4 == 0).
template <int W>
__device__ inline u16x4 ld_col4(const u16* tile, int r0, int c0, int lane) {
    const int i = lane & 15;
    const u16* p = tile + swz<W>(r0 + (i >> 2), c0 + 4 * (i & 3));
    return __builtin_bit_cast(u16x4, __builtin_amdgcn_ds_read_tr16_b64_v4i16(LDS_AS(s16x4, const_cast<u16*>(p))));
}

// Copies rows [r0, r0 + ROWS) of a row-major [T][W] global matrix (rows past T - 1 repeat row
// T - 1; their results are masked by the callers) into a swizzled LDS tile, 16 bytes per lane.
template <int W, int ROWS, int NW>
__device__ inline void dma_rows(const u16* __restrict__ g, int r0, int T, u16* lds, int wave, int lane) {
    constexpr int CH = W / 8, NCH = ROWS * CH;
    static_assert(NCH % (64 * NW) == 0, "tile must split evenly over the block's waves");
#pragma unroll
    for (int it = 0; it < NCH / (64 * NW); ++it) {
        const int p0 = (it * NW + wave) * 64;  // first chunk written by this wave instruction
        const int p = p0 + lane;
        const int row = p / CH;
        const int c = (p % CH) ^ (row & (CH - 1));
        const int gr = min(r0 + row, T - 1);
        __builtin_amdgcn_global_load_lds(reinterpret_cast<const void*>(g + (size_t)gr * W + c * 8),
                                         LDS_AS(void, lds + p0 * 8), 16, 0, 0);
    }
}

// Wait until this wave's vector-memory operations (including LDS DMA) have completed.
__device__ inline void wait_vmem() { __builtin_amdgcn_s_waitcnt(0x0F70); }

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

// ------------------------------------------------------------------------------------------
// Forward. Block = 4 waves = 128 query rows of one (batch, head); 128-key tiles of K and V,
// double-buffered in LDS by DMA. Q stays in registers for the whole block.
// ------------------------------------------------------------------------------------------
template <int HD, int DT>
__global__ __launch_bounds__(256, 2) void fa_fwd_kernel(const u16* __restrict__ Q, const u16* __restrict__ K,
                                                        const u16* __restrict__ V, u16* __restrict__ O,
                                                        float* __restrict__ LSE, int BH, int H, int KVH, int T,
                                                        int nqb, float sl2) {
    using E = Elem<DT>;
    constexpr int BM = 128, BN = 128, NW = 4;
    constexpr int NS = HD / 16;  // k-steps of Q K^T
    constexpr int ND = HD / 32;  // 32-wide head_dim tiles of O^T
    constexpr int NT = BN / 32;  // 32-key tiles of S^T
    constexpr int TILE = BN * HD;
    __shared__ __attribute__((aligned(16))) u16 kA[TILE];
    __shared__ __attribute__((aligned(16))) u16 vA[TILE];
    __shared__ __attribute__((aligned(16))) u16 kB[TILE];
    __shared__ __attribute__((aligned(16))) u16 vB[TILE];

    // Heaviest query blocks first; blocks of one (batch, head) share an XCD when BH % 8 == 0.
    const int bid = blockIdx.x;
    const int bh = bid % BH;
    const int qb = nqb - 1 - bid / BH;
    const int b = bh / H, h = bh - b * H;
    const int kvh = h / (H / KVH);
    const size_t qoff = (size_t)bh * T * HD;
    const size_t kvoff = ((size_t)b * KVH + kvh) * T * HD;
    const u16* Kp = K + kvoff;
    const u16* Vp = V + kvoff;

    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, l32 = lane & 31, hh = lane >> 5;
    const int g16 = (lane >> 4) & 1;  // which 16-column half of a 32-wide MFMA tile this lane reads
    const int q0 = qb * BM, qw = q0 + wave * 32, qrow = qw + l32;

    u16x8 qf[NS];
#pragma unroll
    for (int s = 0; s < NS; ++s) qf[s] = qrow < T ? ld8(Q + qoff + (size_t)qrow * HD + 16 * s + 8 * hh) : u16x8{};

    f32x16 oacc[ND];
#pragma unroll
    for (int dt = 0; dt < ND; ++dt) oacc[dt] = f32x16{};
    float m = -INFINITY, lsum = 0.f;

    const int ntiles = (min(q0 + BM, T) + BN - 1) / BN;
    auto issue = [&](int it, u16* kb, u16* vb) {
        dma_rows<HD, BN, NW>(Kp, it * BN, T, kb, wave, lane);
        dma_rows<HD, BN, NW>(Vp, it * BN, T, vb, wave, lane);
    };
    auto step = [&](int it, const u16* kb, const u16* vb) {
        const int k0 = it * BN;
        if (qw >= T || k0 > qw + 31) return;  // no visible key in this tile for this wave
        f32x16 s[NT];
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            s[t] = f32x16{};
#pragma unroll
            for (int ks = 0; ks < NS; ++ks)
                s[t] = E::mfma(ld8(kb + swz<HD>(32 * t + l32, 16 * ks + 8 * hh)), qf[ks], s[t]);
        }
        // s[t][i] = score of query qrow against key k0 + 32t + (i/4)*8 + 4hh + i%4.
        if (k0 + BN - 1 > qw || k0 + BN > T) {
            const int lim = min(qrow, T - 1) - k0 - 4 * hh;
#pragma unroll
            for (int t = 0; t < NT; ++t)
#pragma unroll
                for (int i = 0; i < 16; ++i)
                    if (32 * t + (i >> 2) * 8 + (i & 3) > lim) s[t][i] = -INFINITY;
        }
        float mx = -INFINITY;
#pragma unroll
        for (int t = 0; t < NT; ++t)
#pragma unroll
            for (int i = 0; i < 16; ++i) mx = fmaxf(mx, s[t][i]);
        mx = pair_max(mx);
        const bool grow = (mx - m) * sl2 > kRescaleLog2;  // always true while m = -inf
        if (__builtin_amdgcn_ballot_w64(grow)) {
            const float mnew = grow ? mx : m;
            const float corr = fast_exp2((m - mnew) * sl2);  // 0 on the first tile, 1 where m is kept
            lsum *= corr;
#pragma unroll
            for (int dt = 0; dt < ND; ++dt) oacc[dt] *= corr;
            m = mnew;
        }
        const float mb = m * sl2;
#pragma unroll
        for (int c = 0; c < BN / 16; ++c) {
            f32x16& st = s[c >> 1];
            const int base = 8 * (c & 1);
#pragma unroll
            for (int j = 0; j < 8; ++j) st[base + j] = fast_exp2(fmaf(st[base + j], sl2, -mb));
            const u16x8 pf = pack8<DT>(st, base);
            const u32x4 pw = __builtin_bit_cast(u32x4, pf);
            lsum = E::add_pair(pw[0], lsum);
            lsum = E::add_pair(pw[1], lsum);
            lsum = E::add_pair(pw[2], lsum);
            lsum = E::add_pair(pw[3], lsum);
            // P^T chunk c holds keys 16c + (j/4)*8 + 4hh + j%4; V^T must use the same order.
#pragma unroll
            for (int dt = 0; dt < ND; ++dt) {
                const u16x8 va = cat4(ld_col4<HD>(vb, 16 * c + 4 * hh, 32 * dt + 16 * g16, lane),
                                      ld_col4<HD>(vb, 16 * c + 8 + 4 * hh, 32 * dt + 16 * g16, lane));
                oacc[dt] = E::mfma(va, pf, oacc[dt]);
            }
        }
    };

    issue(0, kA, vA);
    for (int it = 0; it < ntiles; it += 2) {
        wait_vmem();
        __syncthreads();
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
        const float inv = 1.f / ltot;
        u16* op = O + qoff + (size_t)qrow * HD;
#pragma unroll
        for (int dt = 0; dt < ND; ++dt)
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const f32x16& a = oacc[dt];
                u32x2 w = {E::pack2(a[4 * g] * inv, a[4 * g + 1] * inv), E::pack2(a[4 * g + 2] * inv, a[4 * g + 3] * inv)};
                *reinterpret_cast<u32x2*>(op + 32 * dt + 8 * g + 4 * hh) = w;
            }
        if (hh == 0) LSE[(size_t)bh * T + qrow] = (m * sl2 + fast_log2(ltot)) * kLn2;
    }
}

// ------------------------------------------------------------------------------------------
// Backward stage 1: D = rowsum(dO * O) and lse2 = lse * log2(e) in fp32, and zero the fp32
// dQ/dK/dV accumulators.
// ------------------------------------------------------------------------------------------
template <int HD, int DT>
__global__ __launch_bounds__(256) void fa_bwd_pre_kernel(const u16* __restrict__ O, const u16* __restrict__ dO,
                                                         const float* __restrict__ LSE, float* __restrict__ Dvec,
                                                         float* __restrict__ Lse2, int64_t rows,
                                                         f32x4* __restrict__ zero, int64_t nzero4) {
    using E = Elem<DT>;
    constexpr int TPR = HD / 8;  // threads per row
    const int64_t gtid = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int64_t row = gtid / TPR;
    const int c = (int)(gtid % TPR);
    float acc = 0.f;
    if (row < rows) {
        const u16x8 o = ld8(O + row * HD + 8 * c), g = ld8(dO + row * HD + 8 * c);
#pragma unroll
        for (int j = 0; j < 8; ++j) acc = fmaf(E::to_f32(o[j]), E::to_f32(g[j]), acc);
    }
#pragma unroll
    for (int off = TPR / 2; off > 0; off >>= 1) acc += __shfl_xor(acc, off);
    if (row < rows && c == 0) {
        Dvec[row] = acc;
        Lse2[row] = LSE[row] * kLog2e;
    }
    const int64_t stride = (int64_t)gridDim.x * 256;
    for (int64_t i = gtid; i < nzero4; i += stride) zero[i] = f32x4{};
}

// ------------------------------------------------------------------------------------------
// Backward stage 2. Block = 4 waves = 128 keys of one (batch, KV head); wave w owns keys
// kb0 + 32w .. +31 and keeps K, V (B operands) and its dK^T, dV^T accumulators in registers.
// The block walks the group's query heads x a chunk of 64-row query tiles; per tile:
//   S = Q K^T, dP = dO V^T             (A = Q / dO rows, LDS; B = K / V, registers)
//   P = exp2(S*sl2 - lse2), dS = P (dP - D)
//   dV^T += dO^T P, dK^T += Q^T dS     (A = columns of the Q / dO tiles; B = P / dS registers)
//   dQ += dS K                         (A = columns of dS^T in LDS, B = columns of K in LDS)
// Q/dO tiles of the next iteration stream in by DMA while the current one is computed, and each
// tile's dQ partial is added to the fp32 accumulator with atomics. The softmax scale is folded
// into the final dQ/dK conversion (stage 3).
// ------------------------------------------------------------------------------------------
template <int HD, int DT>
__global__ __launch_bounds__(256, 2) void fa_bwd_main_kernel(
    const u16* __restrict__ Q, const u16* __restrict__ K, const u16* __restrict__ V, const u16* __restrict__ dO,
    const float* __restrict__ Lse2, const float* __restrict__ Dvec, float* __restrict__ dQa, float* __restrict__ dKa,
    float* __restrict__ dVa, int BKV, int H, int KVH, int T, int nkb, int nqt, int qchunk, float sl2) {
    using E = Elem<DT>;
    constexpr int BN = 128, BM = 64, NW = 4;
    constexpr int NS = HD / 16;
    constexpr int ND = HD / 32;
    constexpr int QT = BM * HD;  // elements of one Q or dO tile
    __shared__ __attribute__((aligned(16))) u16 qA[QT];
    __shared__ __attribute__((aligned(16))) u16 oA[QT];
    __shared__ __attribute__((aligned(16))) u16 qB[QT];
    __shared__ __attribute__((aligned(16))) u16 oB[QT];
    __shared__ __attribute__((aligned(16))) u16 kS[BN * HD];   // K rows of the block (dQ's B operand)
    __shared__ __attribute__((aligned(16))) u16 dsT[BN * BM];  // dS^T [key][query]
    __shared__ __attribute__((aligned(16))) float lA[2 * BM];  // lse2 | D of the tile in qA/oA
    __shared__ __attribute__((aligned(16))) float lB[2 * BM];

    const int bid = blockIdx.x;
    const int bk = bid % BKV;
    const int item = bid / BKV;
    const int c = item / nkb, j = item - (item / nkb) * nkb;
    const int qt_first = (j * BN) / BM;
    const int qt_hi = nqt - c * qchunk;
    if (qt_hi <= qt_first) return;  // this (key block, chunk) pair has no work
    const int qt_lo = max(qt_first, qt_hi - qchunk);
    const int nq = qt_hi - qt_lo;

    const int b = bk / KVH, kvh = bk - b * KVH, group = H / KVH;
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, l32 = lane & 31, hh = lane >> 5;
    const int g16 = (lane >> 4) & 1;
    const int kb0 = j * BN, kw = kb0 + 32 * wave, key = kw + l32;
    const size_t kvoff = (size_t)bk * T * HD;

    u16x8 kf[NS], vf[NS];
#pragma unroll
    for (int s = 0; s < NS; ++s) {
        kf[s] = key < T ? ld8(K + kvoff + (size_t)key * HD + 16 * s + 8 * hh) : u16x8{};
        vf[s] = key < T ? ld8(V + kvoff + (size_t)key * HD + 16 * s + 8 * hh) : u16x8{};
    }
    dma_rows<HD, BN, NW>(K + kvoff, kb0, T, kS, wave, lane);

    f32x16 dk[ND], dv[ND];
#pragma unroll
    for (int dt = 0; dt < ND; ++dt) dk[dt] = dv[dt] = f32x16{};

    // dQ tile of this wave: query rows 32*dq_qh.., head_dim columns 32*dq_dt.. of the 64 x HD tile.
    const bool dq_wave = wave < 2 * ND;
    const int dq_qh = wave / ND, dq_dt = wave - (wave / ND) * ND;

    const int niter = group * nq;
    float lse_r = 0.f, d_r = 0.f;
    auto issue = [&](int itn, u16* qb_, u16* ob_) {
        const int g = itn / nq, qt = qt_lo + itn - g * nq;
        const int hq = kvh * group + g;
        const size_t qoff = ((size_t)b * H + hq) * T * HD;
        dma_rows<HD, BM, NW>(Q + qoff, qt * BM, T, qb_, wave, lane);
        dma_rows<HD, BM, NW>(dO + qoff, qt * BM, T, ob_, wave, lane);
        if (tid < 2 * BM) {
            const int q = min(qt * BM + (tid & (BM - 1)), T - 1);
            const size_t ro = ((size_t)b * H + hq) * T + q;
            if (tid < BM) lse_r = Lse2[ro];
            else d_r = Dvec[ro];
        }
    };
    // One query tile. On entry the tile's Q / dO rows (qb_, ob_) and lse2 / D (lb_) are in LDS
    // for this wave; the next tile is fetched into (qn_, on_, ln_) while this one is computed.
    auto step = [&](int itn, const u16* qb_, const u16* ob_, const float* lb_, u16* qn_, u16* on_, float* ln_) {
        const int g = itn / nq, qt = qt_lo + itn - g * nq;
        const int hq = kvh * group + g;
        const int qbase = qt * BM;
        __syncthreads();
        const bool more = itn + 1 < niter;
        if (more) issue(itn + 1, qn_, on_);

        if (kw <= qbase + BM - 1 && kw < T) {
            const bool need_mask = (kw + 31 > qbase) || (qbase + BM > T) || (kw + 32 > T);
            const int qlim = key - qbase - 4 * hh;  // query offsets below this are in the future of the key
            // One 32-query half at a time keeps S, dP and their 16-bit forms for 32 queries live.
#pragma unroll 1
            for (int qh = 0; qh < 2; ++qh) {
                f32x16 s = f32x16{}, dp = f32x16{};
#pragma unroll
                for (int ks = 0; ks < NS; ++ks) {
                    s = E::mfma(ld8(qb_ + swz<HD>(32 * qh + l32, 16 * ks + 8 * hh)), kf[ks], s);
                    dp = E::mfma(ld8(ob_ + swz<HD>(32 * qh + l32, 16 * ks + 8 * hh)), vf[ks], dp);
                }
                // s[i]: query qbase + 32qh + (i/4)*8 + 4hh + i%4 against this lane's key.
#pragma unroll
                for (int g4 = 0; g4 < 4; ++g4) {
                    const int ql = 32 * qh + 8 * g4 + 4 * hh;
                    const f32x4 L = *reinterpret_cast<const f32x4*>(&lb_[ql]);
                    const f32x4 Dd = *reinterpret_cast<const f32x4*>(&lb_[BM + ql]);
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const int i = 4 * g4 + r;
                        float p = fast_exp2(fmaf(s[i], sl2, -L[r]));
                        float ds = p * (dp[i] - Dd[r]);
                        // visible iff key <= q, q < T and key < T
                        if (need_mask && (32 * qh + 8 * g4 + r < qlim || qbase + ql + r >= T || key >= T)) p = ds = 0.f;
                        s[i] = p;
                        dp[i] = ds;
                    }
                }
#pragma unroll
                for (int half = 0; half < 2; ++half) {
                    const int qc = 2 * qh + half;  // 16-query chunk: queries 16qc + (j/4)*8 + 4hh + j%4
                    const u16x8 pf = pack8<DT>(s, 8 * half);
                    const u16x8 sf = pack8<DT>(dp, 8 * half);
#pragma unroll
                    for (int dt = 0; dt < ND; ++dt) {
                        const int c0 = 32 * dt + 16 * g16;
                        const u16x8 ga = cat4(ld_col4<HD>(ob_, 16 * qc + 4 * hh, c0, lane),
                                              ld_col4<HD>(ob_, 16 * qc + 8 + 4 * hh, c0, lane));
                        dv[dt] = E::mfma(ga, pf, dv[dt]);
                        const u16x8 qa = cat4(ld_col4<HD>(qb_, 16 * qc + 4 * hh, c0, lane),
                                              ld_col4<HD>(qb_, 16 * qc + 8 + 4 * hh, c0, lane));
                        dk[dt] = E::mfma(qa, sf, dk[dt]);
                    }
                    // dS^T row (this lane's key): 4 consecutive queries per 8-byte store.
                    const u32x4 w = __builtin_bit_cast(u32x4, sf);
                    const int qa0 = 16 * qc + 4 * hh;
                    *reinterpret_cast<u32x2*>(dsT + swz<BM>(32 * wave + l32, qa0)) = u32x2{w[0], w[1]};
                    *reinterpret_cast<u32x2*>(dsT + swz<BM>(32 * wave + l32, qa0 + 8)) = u32x2{w[2], w[3]};
                }
            }
        }
        __syncthreads();

        // dQ tile over the keys that can be visible (every other dS^T row is never read).
        int kvis = min(BN, qbase + BM - kb0);
        kvis = min(kvis, T - kb0);
        const int nks = (kvis + 15) / 16;
        f32x16 dqacc = f32x16{};
        if (dq_wave) {
            const int cq = 32 * dq_qh + 16 * g16, cd = 32 * dq_dt + 16 * g16;
            for (int ks = 0; ks < nks; ++ks) {
                const u16x8 a = cat4(ld_col4<BM>(dsT, 16 * ks + 8 * hh, cq, lane),
                                     ld_col4<BM>(dsT, 16 * ks + 8 * hh + 4, cq, lane));
                const u16x8 bb = cat4(ld_col4<HD>(kS, 16 * ks + 8 * hh, cd, lane),
                                      ld_col4<HD>(kS, 16 * ks + 8 * hh + 4, cd, lane));
                dqacc = E::mfma(a, bb, dqacc);
            }
        }
        // The next tile's DMA and lse2 / D loads (and the previous dQ atomics) are done after this.
        wait_vmem();
        if (more && tid < 2 * BM) ln_[tid] = tid < BM ? lse_r : d_r;
        if (dq_wave) {
            float* dst = dQa + (((size_t)b * H + hq) * T + qbase) * HD + 32 * dq_dt + l32;
            const int rows = min(BM, T - qbase);
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const int r = 32 * dq_qh + (i >> 2) * 8 + 4 * hh + (i & 3);
                if (r < rows) unsafeAtomicAdd(dst + (size_t)r * HD, dqacc[i]);
            }
        }
    };

    issue(0, qA, oA);
    wait_vmem();
    if (tid < 2 * BM) lA[tid] = tid < BM ? lse_r : d_r;
    for (int itn = 0; itn < niter; itn += 2) {
        step(itn, qA, oA, lA, qB, oB, lB);
        if (itn + 1 >= niter) break;
        step(itn + 1, qB, oB, lB, qA, oA, lA);
    }

    // dK^T / dV^T accumulators (lane = key, element i = column 32dt + (i/4)*8 + 4hh + i%4) leave
    // through LDS so that each atomic instruction covers 64 consecutive floats of one tensor.
    float* stage = reinterpret_cast<float*>(dsT);  // 128 keys x 32 columns fp32 = the dS^T tile's bytes
    static_assert(BN * 32 * 4 == BN * BM * 2, "staging must fit the dS^T tile");
#pragma unroll
    for (int which = 0; which < 2; ++which)
#pragma unroll
        for (int dt = 0; dt < ND; ++dt) {
            __syncthreads();
            const f32x16& a = which == 0 ? dk[dt] : dv[dt];
            const int r = 32 * wave + l32;
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                const int col = 8 * g + 4 * hh;  // 4 consecutive columns
                *reinterpret_cast<f32x4*>(stage + r * 32 + (((col >> 2) ^ (r & 7)) << 2)) =
                    f32x4{a[4 * g], a[4 * g + 1], a[4 * g + 2], a[4 * g + 3]};
            }
            __syncthreads();
            float* dst = (which == 0 ? dKa : dVa) + kvoff + 32 * dt;
#pragma unroll
            for (int k = 0; k < BN * 32 / 256; ++k) {
                const int f = tid + 256 * k;
                const int row = f >> 5, col = f & 31;
                if (kb0 + row < T)
                    unsafeAtomicAdd(dst + (size_t)(kb0 + row) * HD + col,
                                    stage[row * 32 + ((((col >> 2) ^ (row & 7)) << 2) | (col & 3))]);
            }
        }
}

// ------------------------------------------------------------------------------------------
// Backward stage 3: dq = dQacc * scale, dk = dKacc * scale, dv = dVacc, rounded to 16 bits.
// ------------------------------------------------------------------------------------------
template <int DT>
__global__ __launch_bounds__(256) void fa_bwd_post_kernel(const f32x4* __restrict__ dQa, const f32x4* __restrict__ dKa,
                                                          const f32x4* __restrict__ dVa, u32x2* __restrict__ dq,
                                                          u32x2* __restrict__ dk, u32x2* __restrict__ dv, int64_t nq4,
                                                          int64_t nk4, float scale) {
    using E = Elem<DT>;
    const int64_t stride = (int64_t)gridDim.x * 256;
    const int64_t total = nq4 + 2 * nk4;
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < total; i += stride) {
        f32x4 x;
        float s;
        u32x2* dst;
        if (i < nq4) {
            x = dQa[i], s = scale, dst = dq + i;
        } else if (i < nq4 + nk4) {
            x = dKa[i - nq4], s = scale, dst = dk + (i - nq4);
        } else {
            x = dVa[i - nq4 - nk4], s = 1.f, dst = dv + (i - nq4 - nk4);
        }
        *dst = u32x2{E::pack2(x[0] * s, x[1] * s), E::pack2(x[2] * s, x[3] * s)};
    }
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
    if (B < 0 || H <= 0 || KVH <= 0 || T < 0) return fail(-1, "invalid sizes B=%lld H=%lld KVH=%lld T=%lld",
                                                          (long long)B, (long long)H, (long long)KVH, (long long)T);
    if (D != 32 && D != 64) return fail(-1, "head_dim must be 32 or 64");
    if (H % KVH != 0) return fail(-1, "query heads must group evenly over KV heads");
    if (dtype != kF16 && dtype != kBF16) return fail(-1, "inputs must be float16 or bfloat16");
    if (B * H * T * D >= ((int64_t)1 << 40) || T >= ((int64_t)1 << 30) || B * H >= ((int64_t)1 << 30))
        return fail(-1, "sizes too large");
    return 0;
}

struct Workspace {
    float* dq;
    float* dk;
    float* dv;
    float* D;
    float* lse2;
    size_t bytes;
};

size_t round256(size_t n) { return (n + 255) & ~(size_t)255; }

Workspace carve(void* base, int64_t B, int64_t H, int64_t KVH, int64_t T, int64_t D) {
    const size_t nq = (size_t)B * H * T * D, nk = (size_t)B * KVH * T * D, nr = (size_t)B * H * T;
    char* p = (char*)base;
    Workspace w;
    w.dq = (float*)p;
    w.dk = w.dq + nq;  // dQ, dK, dV accumulators are adjacent so one pass can zero them
    w.dv = w.dk + nk;
    const size_t acc = round256(4 * (nq + 2 * nk)), vec = round256(4 * nr);
    w.D = (float*)(p + acc);
    w.lse2 = (float*)(p + acc + vec);
    w.bytes = acc + 2 * vec;
    return w;
}

int env_int(const char* name, int dflt) {
    const char* s = getenv(name);
    if (!s || !*s) return dflt;
    const int v = atoi(s);
    return v > 0 ? v : dflt;
}

template <int HD, int DT>
int fwd_impl(const void* q, const void* k, const void* v, void* o, float* lse, int64_t B, int64_t H, int64_t KVH,
             int64_t T, float scale, hipStream_t st) {
    const int nqb = (int)((T + 127) / 128);
    const int BH = (int)(B * H);
    fa_fwd_kernel<HD, DT><<<dim3(nqb * BH), dim3(256), 0, st>>>(
        (const u16*)q, (const u16*)k, (const u16*)v, (u16*)o, lse, BH, (int)H, (int)KVH, (int)T, nqb, scale * kLog2e);
    return launch_status("fa_fwd_kernel");
}

template <int HD, int DT>
int pre_impl(const void* o, const void* dO, const float* lse, const Workspace& w, int64_t B, int64_t H, int64_t KVH,
             int64_t T, hipStream_t st) {
    const int64_t rows = B * H * T;
    const int64_t threads = rows * (HD / 8);
    const int64_t nzero4 = (B * H * T * HD + 2 * B * KVH * T * HD) / 4;
    int64_t blocks = (threads + 255) / 256;
    if (blocks < 1) blocks = 1;
    fa_bwd_pre_kernel<HD, DT><<<dim3((unsigned)blocks), dim3(256), 0, st>>>((const u16*)o, (const u16*)dO, lse, w.D,
                                                                           w.lse2, rows, (f32x4*)w.dq, nzero4);
    return launch_status("fa_bwd_pre_kernel");
}

template <int HD, int DT>
int main_impl(const void* q, const void* k, const void* v, const void* dO, const Workspace& w, int64_t B, int64_t H,
              int64_t KVH, int64_t T, float scale, hipStream_t st) {
    const int nkb = (int)((T + 127) / 128);
    const int nqt = (int)((T + 63) / 64);
    static const int qchunk = env_int("NNFA_BWD_QCHUNK", 4);
    const int nch = (nqt + qchunk - 1) / qchunk;
    const int BKV = (int)(B * KVH);
    fa_bwd_main_kernel<HD, DT><<<dim3(nch * nkb * BKV), dim3(256), 0, st>>>(
        (const u16*)q, (const u16*)k, (const u16*)v, (const u16*)dO, w.lse2, w.D, w.dq, w.dk, w.dv, BKV, (int)H,
        (int)KVH, (int)T, nkb, nqt, qchunk, scale * kLog2e);
    return launch_status("fa_bwd_main_kernel");
}

template <int DT>
int post_impl(const Workspace& w, void* dq, void* dk, void* dv, int64_t B, int64_t H, int64_t KVH, int64_t T,
              int64_t D, float scale, hipStream_t st) {
    const int64_t nq4 = B * H * T * D / 4, nk4 = B * KVH * T * D / 4;
    int64_t blocks = (nq4 + 2 * nk4 + 255) / 256;
    if (blocks > 8192) blocks = 8192;
    if (blocks < 1) blocks = 1;
    fa_bwd_post_kernel<DT><<<dim3((unsigned)blocks), dim3(256), 0, st>>>(
        (const f32x4*)w.dq, (const f32x4*)w.dk, (const f32x4*)w.dv, (u32x2*)dq, (u32x2*)dk, (u32x2*)dv, nq4, nk4,
        scale);
    return launch_status("fa_bwd_post_kernel");
}

}  // namespace

// Dispatch on (head_dim, dtype) for the four templated stages.
#define NNFA_DISPATCH(FN, D, DT, ...)                                 \
    ((D) == 64 ? ((DT) == kBF16 ? FN<64, kBF16>(__VA_ARGS__)          \
                                : FN<64, kF16>(__VA_ARGS__))          \
               : ((DT) == kBF16 ? FN<32, kBF16>(__VA_ARGS__)          \
                                : FN<32, kF16>(__VA_ARGS__)))

NNFA_API const char* nn_fa_last_error(void) { return g_last_error.c_str(); }

NNFA_API int nn_fa_abi_version(void) { return 2; }

NNFA_API size_t nn_fa_bwd_workspace_size(int64_t B, int64_t H, int64_t KVH, int64_t T, int64_t D) {
    if (B < 0 || H < 0 || KVH < 0 || T < 0 || D < 0) return 0;
    return carve(nullptr, B, H, KVH, T, D).bytes;
}

NNFA_API int nn_fa_fwd(const void* q, const void* k, const void* v, void* o, float* lse, int64_t B, int64_t H,
                       int64_t KVH, int64_t T, int64_t D, int dtype, float scale, void* stream) {
    g_last_error.clear();
    if (int e = check_dims(B, H, KVH, T, D, dtype)) return e;
    if (B == 0 || T == 0) return 0;
    if (!q || !k || !v || !o || !lse) return fail(-1, "null pointer argument");
    if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(o)) return fail(-1, "inputs must be 16-byte aligned");
    return NNFA_DISPATCH(fwd_impl, D, dtype, q, k, v, o, lse, B, H, KVH, T, scale, (hipStream_t)stream);
}

static int check_ws(void* workspace, size_t workspace_bytes, int64_t B, int64_t H, int64_t KVH, int64_t T, int64_t D) {
    if (!workspace) return fail(-1, "null workspace");
    if (((uintptr_t)workspace & 255u) != 0) return fail(-1, "workspace must be 256-byte aligned");
    const size_t need = nn_fa_bwd_workspace_size(B, H, KVH, T, D);
    if (workspace_bytes < need)
        return fail(-1, "workspace too small: %zu bytes given, %zu needed", workspace_bytes, need);
    return 0;
}

NNFA_API int nn_fa_bwd_pre(const void* o, const void* dO, const float* lse, void* workspace, size_t workspace_bytes,
                           int64_t B, int64_t H, int64_t KVH, int64_t T, int64_t D, int dtype, void* stream) {
    g_last_error.clear();
    if (int e = check_dims(B, H, KVH, T, D, dtype)) return e;
    if (B == 0 || T == 0) return 0;
    if (int e = check_ws(workspace, workspace_bytes, B, H, KVH, T, D)) return e;
    if (!o || !dO || !lse) return fail(-1, "null pointer argument");
    if (!aligned16(o) || !aligned16(dO)) return fail(-1, "inputs must be 16-byte aligned");
    const Workspace w = carve(workspace, B, H, KVH, T, D);
    return NNFA_DISPATCH(pre_impl, D, dtype, o, dO, lse, w, B, H, KVH, T, (hipStream_t)stream);
}

NNFA_API int nn_fa_bwd_main(const void* q, const void* k, const void* v, const void* dO, void* workspace,
                            size_t workspace_bytes, int64_t B, int64_t H, int64_t KVH, int64_t T, int64_t D, int dtype,
                            float scale, void* stream) {
    g_last_error.clear();
    if (int e = check_dims(B, H, KVH, T, D, dtype)) return e;
    if (B == 0 || T == 0) return 0;
    if (int e = check_ws(workspace, workspace_bytes, B, H, KVH, T, D)) return e;
    if (!q || !k || !v || !dO) return fail(-1, "null pointer argument");
    if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(dO))
        return fail(-1, "inputs must be 16-byte aligned");
    const Workspace w = carve(workspace, B, H, KVH, T, D);
    return NNFA_DISPATCH(main_impl, D, dtype, q, k, v, dO, w, B, H, KVH, T, scale, (hipStream_t)stream);
}

NNFA_API int nn_fa_bwd_post(const void* workspace, size_t workspace_bytes, void* dq, void* dk, void* dv, int64_t B,
                            int64_t H, int64_t KVH, int64_t T, int64_t D, int dtype, float scale, void* stream) {
    g_last_error.clear();
    if (int e = check_dims(B, H, KVH, T, D, dtype)) return e;
    if (B == 0 || T == 0) return 0;
    if (int e = check_ws((void*)workspace, workspace_bytes, B, H, KVH, T, D)) return e;
    if (!dq || !dk || !dv) return fail(-1, "null pointer argument");
    if (!aligned16(dq) || !aligned16(dk) || !aligned16(dv)) return fail(-1, "outputs must be 16-byte aligned");
    const Workspace w = carve((void*)workspace, B, H, KVH, T, D);
    hipStream_t st = (hipStream_t)stream;
    return dtype == kBF16 ? post_impl<kBF16>(w, dq, dk, dv, B, H, KVH, T, D, scale, st)
                          : post_impl<kF16>(w, dq, dk, dv, B, H, KVH, T, D, scale, st);
}

NNFA_API int nn_fa_bwd(const void* dO, const void* q, const void* k, const void* v, const void* o, const float* lse,
                       void* dq, void* dk, void* dv, void* workspace, size_t workspace_bytes, int64_t B, int64_t H,
                       int64_t KVH, int64_t T, int64_t D, int dtype, float scale, void* stream) {
    if (int e = nn_fa_bwd_pre(o, dO, lse, workspace, workspace_bytes, B, H, KVH, T, D, dtype, stream)) return e;
    if (int e = nn_fa_bwd_main(q, k, v, dO, workspace, workspace_bytes, B, H, KVH, T, D, dtype, scale, stream))
        return e;
    return nn_fa_bwd_post(workspace, workspace_bytes, dq, dk, dv, B, H, KVH, T, D, dtype, scale, stream);
}
