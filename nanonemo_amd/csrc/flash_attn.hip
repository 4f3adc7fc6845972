// Causal grouped-query FlashAttention-2, forward and backward, for MI355X (gfx950, CDNA4).
//
// Semantics follow /root/reference/nanonemo/kernels/cuda/flash_attn.cu (fwd_kernel :52-174,
// bwd_kernel :176-340, host wrappers :342-405); the design is written for CDNA4 wave64 + MFMA:
//
//   * All products run on v_mfma_f32_32x32x16_{bf16,f16}. One wave owns a 32-wide slab of the
//     sequence dimension; LDS holds tiles shared by the waves of a block.
//   * Forward computes S^T = K Q^T so that each lane owns one query row (lane % 32) and the
//     keys sit in its accumulator registers. Row max/sum are then in-lane reductions plus one
//     exchange with the other half-wave, and P^T feeds the P·V MFMA straight from registers
//     as the B operand (O^T = V^T P^T). V is staged transposed in LDS for that product.
//   * Backward: one block per (batch, KV head, 128-key block, chunk of query tiles). It loops
//     over the H/KVH query heads of the group, so dK/dV of the group are summed in registers;
//     S = Q K^T and dP = dO V^T land with the key on the lane, so P and dS feed dV^T += dO^T P
//     and dK^T += Q^T dS as B operands without transposes; dQ = dS K goes through LDS and is
//     accumulated in fp32 with atomics.
//   * Softmax runs in base 2: exp2(s * scale * log2(e) - m'), with lse stored in natural log.
//
// MFMA 32x32x16 register layouts used throughout (lane l, l32 = l % 32, hh = l / 32):
//   A (32x16, M x K): lane l supplies A[l32][8*hh + j], j = 0..7
//   B (16x32, K x N): lane l supplies B[8*hh + j][l32]
//   C (32x32):        lane l holds C[(i/4)*8 + 4*hh + (i%4)][l32] in element i = 0..15
// A and B agree on which (half-wave, element) carries which k, so a product may permute the
// contraction index freely as long as both operands use the same permutation.
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
__device__ inline u16x4 ld4(const u16* p) { return *reinterpret_cast<const u16x4*>(p); }
__device__ inline void st8(u16* p, u16x8 v) { *reinterpret_cast<u16x8*>(p) = v; }
__device__ inline void st_u32(u16* p, uint32_t v) { *reinterpret_cast<uint32_t*>(p) = v; }

__device__ inline float xhalf(float x) { return __shfl_xor(x, 32); }  // value of the other half-wave

__device__ inline float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }
__device__ inline float fast_log2(float x) { return __builtin_amdgcn_logf(x); }

// ------------------------------------------------------------------------------------------
// Forward. Block = 4 waves = 128 query rows of one (batch, head); 64-key tiles, double-buffered
// in LDS (K row-major for the A operand of S^T = K Q^T, V transposed for the A operand of
// O^T = V^T P^T). Q stays in registers for the whole block.
// ------------------------------------------------------------------------------------------
template <int HD, int DT>
__global__ __launch_bounds__(256) void fa_fwd_kernel(const u16* __restrict__ Q, const u16* __restrict__ K,
                                                     const u16* __restrict__ V, u16* __restrict__ O,
                                                     float* __restrict__ LSE, int BH, int H, int KVH, int T,
                                                     int nqb, float sl2) {
    using E = Elem<DT>;
    constexpr int BM = 128, BN = 64;
    constexpr int KP = HD + 8;  // K tile row pitch (elements); 16-byte aligned rows
    constexpr int VP = BN + 4;  // V^T tile row pitch (elements); 8-byte aligned rows
    constexpr int NS = HD / 16;
    constexpr int ND = HD / 32;
    constexpr int KCH = BN * HD / 8;         // 16-byte chunks per K tile
    constexpr int KPT = KCH / 256;           // ... per thread
    constexpr int VIT = (BN / 2) * (HD / 8);  // (key pair, 8-column chunk) items per V tile
    static_assert(KCH % 256 == 0, "K tile must split evenly over the block");
    __shared__ __attribute__((aligned(16))) u16 Ks[2][BN * KP];
    __shared__ __attribute__((aligned(16))) u16 Vts[2][HD * VP];

    // Heaviest query blocks first; blocks of one (batch, head) share an XCD when BH % 8 == 0.
    const int bid = blockIdx.x;
    const int bh = bid % BH;
    const int qb = nqb - 1 - bid / BH;
    const int b = bh / H, h = bh - b * H;
    const int kvh = h / (H / KVH);
    const size_t qoff = (size_t)bh * T * HD;
    const size_t kvoff = ((size_t)b * KVH + kvh) * T * HD;
    const u16* Qp = Q + qoff;
    const u16* Kp = K + kvoff;
    const u16* Vp = V + kvoff;

    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, l32 = lane & 31, hh = lane >> 5;
    const int q0 = qb * BM, qw = q0 + wave * 32, qrow = qw + l32;

    u16x8 kreg[KPT], vreg0 = {}, vreg1 = {};
    auto gload = [&](int k0) {
#pragma unroll
        for (int r = 0; r < KPT; ++r) {
            const int c = tid + 256 * r, row = c / (HD / 8), col = (c % (HD / 8)) * 8;
            const int key = k0 + row;
            kreg[r] = key < T ? ld8(Kp + (size_t)key * HD + col) : u16x8{};
        }
        if (tid < VIT) {
            const int col = (tid % (HD / 8)) * 8, key = k0 + 2 * (tid / (HD / 8));
            vreg0 = key < T ? ld8(Vp + (size_t)key * HD + col) : u16x8{};
            vreg1 = key + 1 < T ? ld8(Vp + (size_t)(key + 1) * HD + col) : u16x8{};
        }
    };
    auto sstore = [&](int buf) {
#pragma unroll
        for (int r = 0; r < KPT; ++r) {
            const int c = tid + 256 * r, row = c / (HD / 8), col = (c % (HD / 8)) * 8;
            st8(&Ks[buf][row * KP + col], kreg[r]);
        }
        if (tid < VIT) {
            const int col = (tid % (HD / 8)) * 8, kp = tid / (HD / 8);
#pragma unroll
            for (int j = 0; j < 8; ++j)
                st_u32(&Vts[buf][(col + j) * VP + 2 * kp], (uint32_t)vreg0[j] | ((uint32_t)vreg1[j] << 16));
        }
    };

    u16x8 qf[NS];
#pragma unroll
    for (int s = 0; s < NS; ++s) qf[s] = qrow < T ? ld8(Qp + (size_t)qrow * HD + 16 * s + 8 * hh) : u16x8{};

    f32x16 oacc[ND];
#pragma unroll
    for (int dt = 0; dt < ND; ++dt) oacc[dt] = f32x16{};
    float m = -INFINITY, lsum = 0.f;

    const int kend = min(q0 + BM, T);
    const int ntiles = (kend + BN - 1) / BN;
    gload(0);
    sstore(0);
    __syncthreads();
    for (int it = 0; it < ntiles; ++it) {
        const int k0 = it * BN, buf = it & 1;
        const bool nxt = it + 1 < ntiles;
        if (nxt) gload(k0 + BN);
        if (qw < T && k0 <= qw + 31) {
            f32x16 s[BN / 32];
#pragma unroll
            for (int t = 0; t < BN / 32; ++t) {
                s[t] = f32x16{};
#pragma unroll
                for (int ks = 0; ks < NS; ++ks)
                    s[t] = E::mfma(ld8(&Ks[buf][(32 * t + l32) * KP + 16 * ks + 8 * hh]), qf[ks], s[t]);
            }
            // s[t][i] = score of query qrow against key k0 + 32t + (i/4)*8 + 4hh + i%4.
            if (k0 + BN - 1 > qw || k0 + BN > T) {
#pragma unroll
                for (int t = 0; t < BN / 32; ++t)
#pragma unroll
                    for (int i = 0; i < 16; ++i) {
                        const int key = k0 + 32 * t + (i >> 2) * 8 + 4 * hh + (i & 3);
                        if (key > qrow || key >= T) s[t][i] = -INFINITY;
                    }
            }
            float mx = s[0][0];
#pragma unroll
            for (int t = 0; t < BN / 32; ++t)
#pragma unroll
                for (int i = 0; i < 16; ++i) mx = fmaxf(mx, s[t][i]);
            mx = fmaxf(mx, xhalf(mx));
            const float mnew = fmaxf(m, mx);
            const float corr = fast_exp2((m - mnew) * sl2);
            const float mb = mnew * sl2;
            float ps = 0.f;
#pragma unroll
            for (int t = 0; t < BN / 32; ++t)
#pragma unroll
                for (int i = 0; i < 16; ++i) {
                    const float p = fast_exp2(fmaf(s[t][i], sl2, -mb));
                    s[t][i] = p;
                    ps += p;
                }
            lsum = lsum * corr + ps;
            m = mnew;
#pragma unroll
            for (int dt = 0; dt < ND; ++dt) oacc[dt] *= corr;
#pragma unroll
            for (int c = 0; c < BN / 16; ++c) {
                const u16x8 pf = pack8<DT>(s[c >> 1], 8 * (c & 1));
#pragma unroll
                for (int dt = 0; dt < ND; ++dt) {
                    const u16* vr = &Vts[buf][(32 * dt + l32) * VP + 16 * c + 4 * hh];
                    oacc[dt] = E::mfma(cat4(ld4(vr), ld4(vr + 8)), pf, oacc[dt]);
                }
            }
        }
        if (nxt) sstore(buf ^ 1);
        __syncthreads();
    }

    const float ltot = lsum + xhalf(lsum);
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
// Backward stage 1: D = rowsum(dO * O) in fp32, and zero the fp32 accumulators.
// ------------------------------------------------------------------------------------------
template <int HD, int DT>
__global__ __launch_bounds__(256) void fa_bwd_pre_kernel(const u16* __restrict__ O, const u16* __restrict__ dO,
                                                         float* __restrict__ Dvec, int64_t rows,
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
    if (row < rows && c == 0) Dvec[row] = acc;
    const int64_t stride = (int64_t)gridDim.x * 256;
    for (int64_t i = gtid; i < nzero4; i += stride) zero[i] = f32x4{};
}

// ------------------------------------------------------------------------------------------
// Backward stage 2. Block = 4 waves = 128 keys of one (batch, KV head); wave w owns keys
// kb0 + 32w .. +31 and keeps K, V (B operands) and its dK^T, dV^T accumulators in registers.
// The block walks the group's query heads x a chunk of 64-row query tiles; per tile:
//   S = Q K^T, dP = dO V^T             (A = Q / dO rows from LDS, B = K / V registers)
//   P = exp2(S*sl2 - lse2), dS = P (dP - D)
//   dV^T += dO^T P, dK^T += Q^T dS     (A = transposed Q / dO tiles in LDS, B = P / dS registers)
//   dQ += dS K                         (A = dS via LDS, B = K^T in LDS), fp32 atomics
// The softmax scale is folded into the final dQ/dK conversion (stage 3).
// ------------------------------------------------------------------------------------------
template <int HD, int DT>
__global__ __launch_bounds__(256) void fa_bwd_main_kernel(const u16* __restrict__ Q, const u16* __restrict__ K,
                                                          const u16* __restrict__ V, const u16* __restrict__ dO,
                                                          const float* __restrict__ LSE,
                                                          const float* __restrict__ Dvec, float* __restrict__ dQa,
                                                          float* __restrict__ dKa, float* __restrict__ dVa, int BKV,
                                                          int H, int KVH, int T, int nkb, int nqt, int qchunk,
                                                          float sl2) {
    using E = Elem<DT>;
    constexpr int BN = 128, BM = 64;
    constexpr int QP = HD + 8;   // row-major Q / dO tile pitch
    constexpr int TP = BM + 4;   // transposed Q / dO tile pitch (query contiguous)
    constexpr int KTP = BN + 8;  // transposed K tile pitch (key contiguous)
    constexpr int SP = BN + 8;   // dS tile pitch (key contiguous)
    constexpr int NS = HD / 16;
    constexpr int ND = HD / 32;
    constexpr int LIT = (BM / 2) * (HD / 8);  // (row pair, 8-column chunk) items per Q / dO tile
    __shared__ __attribute__((aligned(16))) u16 Qs[BM * QP];
    __shared__ __attribute__((aligned(16))) u16 dOs[BM * QP];
    __shared__ __attribute__((aligned(16))) u16 Qts[HD * TP];
    __shared__ __attribute__((aligned(16))) u16 dOts[HD * TP];
    __shared__ __attribute__((aligned(16))) u16 Kts[HD * KTP];
    __shared__ __attribute__((aligned(16))) u16 dSs[BM * SP];
    __shared__ __attribute__((aligned(16))) float lse2s[BM];
    __shared__ __attribute__((aligned(16))) float Ds[BM];

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
    const int kb0 = j * BN, kw = kb0 + 32 * wave, key = kw + l32;
    const size_t kvoff = (size_t)bk * T * HD;

    u16x8 kf[NS], vf[NS];
#pragma unroll
    for (int s = 0; s < NS; ++s) {
        kf[s] = key < T ? ld8(K + kvoff + (size_t)key * HD + 16 * s + 8 * hh) : u16x8{};
        vf[s] = key < T ? ld8(V + kvoff + (size_t)key * HD + 16 * s + 8 * hh) : u16x8{};
    }
    for (int it = tid; it < (BN / 2) * (HD / 8); it += 256) {
        const int col = (it % (HD / 8)) * 8, kp = it / (HD / 8), k2 = kb0 + 2 * kp;
        const u16x8 a = k2 < T ? ld8(K + kvoff + (size_t)k2 * HD + col) : u16x8{};
        const u16x8 bb = k2 + 1 < T ? ld8(K + kvoff + (size_t)(k2 + 1) * HD + col) : u16x8{};
#pragma unroll
        for (int jj = 0; jj < 8; ++jj) st_u32(&Kts[(col + jj) * KTP + 2 * kp], (uint32_t)a[jj] | ((uint32_t)bb[jj] << 16));
    }

    f32x16 dk[ND], dv[ND];
#pragma unroll
    for (int dt = 0; dt < ND; ++dt) dk[dt] = dv[dt] = f32x16{};

    u16x8 qa = {}, qb = {}, ga = {}, gb = {};
    float lse_r = 0.f, d_r = 0.f;
    auto gload = [&](int itn) {
        const int g = itn / nq, qt = qt_lo + itn - g * nq;
        const int hq = kvh * group + g;
        const size_t qoff = ((size_t)b * H + hq) * T * HD;
        const int qbase = qt * BM;
        if (tid < LIT) {
            const int col = (tid % (HD / 8)) * 8, r0 = qbase + 2 * (tid / (HD / 8));
            qa = r0 < T ? ld8(Q + qoff + (size_t)r0 * HD + col) : u16x8{};
            qb = r0 + 1 < T ? ld8(Q + qoff + (size_t)(r0 + 1) * HD + col) : u16x8{};
            ga = r0 < T ? ld8(dO + qoff + (size_t)r0 * HD + col) : u16x8{};
            gb = r0 + 1 < T ? ld8(dO + qoff + (size_t)(r0 + 1) * HD + col) : u16x8{};
        }
        if (tid < BM) {
            const int q = qbase + tid;
            const size_t ro = ((size_t)b * H + hq) * T + q;
            lse_r = q < T ? LSE[ro] : 0.f;
            d_r = q < T ? Dvec[ro] : 0.f;
        }
    };
    auto sstore = [&]() {
        if (tid < LIT) {
            const int col = (tid % (HD / 8)) * 8, rp = tid / (HD / 8);
            st8(&Qs[(2 * rp) * QP + col], qa);
            st8(&Qs[(2 * rp + 1) * QP + col], qb);
            st8(&dOs[(2 * rp) * QP + col], ga);
            st8(&dOs[(2 * rp + 1) * QP + col], gb);
#pragma unroll
            for (int jj = 0; jj < 8; ++jj) {
                st_u32(&Qts[(col + jj) * TP + 2 * rp], (uint32_t)qa[jj] | ((uint32_t)qb[jj] << 16));
                st_u32(&dOts[(col + jj) * TP + 2 * rp], (uint32_t)ga[jj] | ((uint32_t)gb[jj] << 16));
            }
        }
        if (tid < BM) {
            lse2s[tid] = lse_r * kLog2e;
            Ds[tid] = d_r;
        }
    };

    const int niter = group * nq;
    gload(0);
    for (int itn = 0; itn < niter; ++itn) {
        const int g = itn / nq, qt = qt_lo + itn - g * nq;
        const int hq = kvh * group + g;
        const int qbase = qt * BM;
        sstore();
        __syncthreads();
        if (itn + 1 < niter) gload(itn + 1);

        if (kw <= qbase + BM - 1 && kw < T) {
            f32x16 s[2], dp[2];
#pragma unroll
            for (int qh = 0; qh < 2; ++qh) {
                s[qh] = f32x16{};
                dp[qh] = f32x16{};
#pragma unroll
                for (int ks = 0; ks < NS; ++ks) {
                    s[qh] = E::mfma(ld8(&Qs[(32 * qh + l32) * QP + 16 * ks + 8 * hh]), kf[ks], s[qh]);
                    dp[qh] = E::mfma(ld8(&dOs[(32 * qh + l32) * QP + 16 * ks + 8 * hh]), vf[ks], dp[qh]);
                }
            }
            // s[qh][i]: query qbase + 32qh + (i/4)*8 + 4hh + i%4 against this lane's key.
            const bool need_mask = (kw + 31 > qbase) || (qbase + BM > T) || (kw + 32 > T);
#pragma unroll
            for (int qh = 0; qh < 2; ++qh)
#pragma unroll
                for (int g4 = 0; g4 < 4; ++g4) {
                    const int ql = 32 * qh + 8 * g4 + 4 * hh;
                    const f32x4 L = *reinterpret_cast<const f32x4*>(&lse2s[ql]);
                    const f32x4 Dd = *reinterpret_cast<const f32x4*>(&Ds[ql]);
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const int i = 4 * g4 + r;
                        float p = fast_exp2(fmaf(s[qh][i], sl2, -L[r]));
                        if (need_mask) {
                            const int q = qbase + ql + r;
                            if (key > q || q >= T || key >= T) p = 0.f;
                        }
                        s[qh][i] = p;
                        dp[qh][i] = p * (dp[qh][i] - Dd[r]);
                    }
                }
            u16x8 pf[4], sf[4];
#pragma unroll
            for (int qc = 0; qc < 4; ++qc) {
                pf[qc] = pack8<DT>(s[qc >> 1], 8 * (qc & 1));
                sf[qc] = pack8<DT>(dp[qc >> 1], 8 * (qc & 1));
            }
#pragma unroll
            for (int dt = 0; dt < ND; ++dt)
#pragma unroll
                for (int qc = 0; qc < 4; ++qc) {
                    const u16* gr = &dOts[(32 * dt + l32) * TP + 16 * qc + 4 * hh];
                    dv[dt] = E::mfma(cat4(ld4(gr), ld4(gr + 8)), pf[qc], dv[dt]);
                    const u16* qr = &Qts[(32 * dt + l32) * TP + 16 * qc + 4 * hh];
                    dk[dt] = E::mfma(cat4(ld4(qr), ld4(qr + 8)), sf[qc], dk[dt]);
                }
            // dS into LDS as [query][key]: element jj of chunk qc is query 16qc + (jj/4)*8 + 4hh + jj%4.
#pragma unroll
            for (int qc = 0; qc < 4; ++qc)
#pragma unroll
                for (int jj = 0; jj < 8; ++jj)
                    dSs[(16 * qc + (jj >> 2) * 8 + 4 * hh + (jj & 3)) * SP + 32 * wave + l32] = sf[qc][jj];
        }
        __syncthreads();

        // dQ tile rows 32*qh.., columns 32*dt..; contraction over the keys that can be visible.
        int kvis = min(BN, qbase + BM - kb0);
        kvis = min(kvis, T - kb0);
        const int nks = (kvis + 15) / 16;
        for (int tile = wave; tile < 2 * ND; tile += 4) {
            const int qh = tile / ND, dt = tile - qh * ND;
            f32x16 acc = f32x16{};
            for (int ks = 0; ks < nks; ++ks)
                acc = E::mfma(ld8(&dSs[(32 * qh + l32) * SP + 16 * ks + 8 * hh]),
                              ld8(&Kts[(32 * dt + l32) * KTP + 16 * ks + 8 * hh]), acc);
            float* dst = dQa + (((size_t)b * H + hq) * T) * HD + 32 * dt + l32;
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const int q = qbase + 32 * qh + (i >> 2) * 8 + 4 * hh + (i & 3);
                if (q < T) unsafeAtomicAdd(dst + (size_t)q * HD, acc[i]);
            }
        }
    }

    // dK^T / dV^T accumulators: lane = key, element i = head_dim column 32dt + (i/4)*8 + 4hh + i%4.
    if (key < T) {
        float* dkp = dKa + kvoff + (size_t)key * HD;
        float* dvp = dVa + kvoff + (size_t)key * HD;
#pragma unroll
        for (int dt = 0; dt < ND; ++dt)
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const int d = 32 * dt + (i >> 2) * 8 + 4 * hh + (i & 3);
                unsafeAtomicAdd(dkp + d, dk[dt][i]);
                unsafeAtomicAdd(dvp + d, dv[dt][i]);
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
    w.D = (float*)(p + round256(4 * (nq + 2 * nk)));
    w.bytes = round256(4 * (nq + 2 * nk)) + round256(4 * nr);
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
int pre_impl(const void* o, const void* dO, const Workspace& w, int64_t B, int64_t H, int64_t KVH, int64_t T,
             hipStream_t st) {
    const int64_t rows = B * H * T;
    const int64_t threads = rows * (HD / 8);
    const int64_t nzero4 = (B * H * T * HD + 2 * B * KVH * T * HD) / 4;
    int64_t blocks = (threads + 255) / 256;
    if (blocks < 1) blocks = 1;
    fa_bwd_pre_kernel<HD, DT><<<dim3((unsigned)blocks), dim3(256), 0, st>>>((const u16*)o, (const u16*)dO, w.D, rows,
                                                                           (f32x4*)w.dq, nzero4);
    return launch_status("fa_bwd_pre_kernel");
}

template <int HD, int DT>
int main_impl(const void* q, const void* k, const void* v, const void* dO, const float* lse, const Workspace& w,
              int64_t B, int64_t H, int64_t KVH, int64_t T, float scale, hipStream_t st) {
    const int nkb = (int)((T + 127) / 128);
    const int nqt = (int)((T + 63) / 64);
    static const int qchunk = env_int("NNFA_BWD_QCHUNK", 4);
    const int nch = (nqt + qchunk - 1) / qchunk;
    const int BKV = (int)(B * KVH);
    fa_bwd_main_kernel<HD, DT><<<dim3(nch * nkb * BKV), dim3(256), 0, st>>>(
        (const u16*)q, (const u16*)k, (const u16*)v, (const u16*)dO, lse, w.D, w.dq, w.dk, w.dv, BKV, (int)H,
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

NNFA_API int nn_fa_abi_version(void) { return 1; }

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

NNFA_API int nn_fa_bwd_pre(const void* o, const void* dO, void* workspace, size_t workspace_bytes, int64_t B,
                           int64_t H, int64_t KVH, int64_t T, int64_t D, int dtype, void* stream) {
    g_last_error.clear();
    if (int e = check_dims(B, H, KVH, T, D, dtype)) return e;
    if (B == 0 || T == 0) return 0;
    if (int e = check_ws(workspace, workspace_bytes, B, H, KVH, T, D)) return e;
    if (!o || !dO) return fail(-1, "null pointer argument");
    if (!aligned16(o) || !aligned16(dO)) return fail(-1, "inputs must be 16-byte aligned");
    const Workspace w = carve(workspace, B, H, KVH, T, D);
    return NNFA_DISPATCH(pre_impl, D, dtype, o, dO, w, B, H, KVH, T, (hipStream_t)stream);
}

NNFA_API int nn_fa_bwd_main(const void* q, const void* k, const void* v, const void* dO, const float* lse,
                            void* workspace, size_t workspace_bytes, int64_t B, int64_t H, int64_t KVH, int64_t T,
                            int64_t D, int dtype, float scale, void* stream) {
    g_last_error.clear();
    if (int e = check_dims(B, H, KVH, T, D, dtype)) return e;
    if (B == 0 || T == 0) return 0;
    if (int e = check_ws(workspace, workspace_bytes, B, H, KVH, T, D)) return e;
    if (!q || !k || !v || !dO || !lse) return fail(-1, "null pointer argument");
    if (!aligned16(q) || !aligned16(k) || !aligned16(v) || !aligned16(dO))
        return fail(-1, "inputs must be 16-byte aligned");
    const Workspace w = carve(workspace, B, H, KVH, T, D);
    return NNFA_DISPATCH(main_impl, D, dtype, q, k, v, dO, lse, w, B, H, KVH, T, scale, (hipStream_t)stream);
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
    if (int e = nn_fa_bwd_pre(o, dO, workspace, workspace_bytes, B, H, KVH, T, D, dtype, stream)) return e;
    if (int e = nn_fa_bwd_main(q, k, v, dO, lse, workspace, workspace_bytes, B, H, KVH, T, D, dtype, scale, stream))
        return e;
    return nn_fa_bwd_post(workspace, workspace_bytes, dq, dk, dv, B, H, KVH, T, D, dtype, scale, stream);
}
