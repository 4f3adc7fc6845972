// Fused residual add + RMSNorm, forward and backward, for MI355X (gfx950).
//
// What it computes (the plain-PyTorch blocks of /root/reference/nanonemo/model/layers.py:19-56 and the
// reference's fused op, kernels/cuda/rmsnorm.py):
//     h = x + delta, rounded to h's dtype (the promotion of x's and delta's); h is x when there is no delta
//     r = 1 / sqrt(mean(h^2) + eps),   y = (h * r) * w          (fp32 arithmetic, y rounded once)
// and its gradient, with g = dy * w:
//     dh_total = r * g - h * (r^3 * sum(g * h) / N)  (+ dh, the gradient reaching h from the residual)
//     dw = sum over rows of dy * h * r
// (the derivative of y with respect to h: r g minus the projection of r g on h's direction).
//
// Work decomposition. A row is owned by a *team* of R lanes: in the backward R = 32 for up to 128 16-byte
// vectors per row (N <= 1024) and R = 64 above (N <= 4096); the forward uses R = 64 throughout. A wave holds
// 64 / R rows. Lane t of a team owns the vectors t, t + R, ..., t + (K - 1) R of its row (K = ceil(vectors /
// R), from a small set of counts; a vector past the row's end is never loaded or stored), so each load
// instruction of a team reads R consecutive 16-byte vectors and the row sits in registers from its loads to
// its stores. At the model's width (N = 768: 96 vectors) a backward team of 32 lanes holds exactly 3 vectors
// per lane and a wave 2 rows.
// Widths that are not a multiple of 8 (up to 1024) use a 64-lane team of single elements.
// Team sums are xor-butterflies over the team's lanes (deterministic). Every load a row needs (and the
// weight, first) is issued before its first use, so one memory latency covers the row.
//
// Backward. A fixed grid of at most kBwdBlocks blocks of 8 waves; every team walks rows team_id,
// team_id + teams, ... and keeps its lanes' dw contributions in registers across all of them. At the
// end the teams of a wave are summed by an xor-butterfly over their lane groups, the block's waves in
// LDS in wave order into one fp32 partial row per block, and colsum_kernel adds the partial rows in
// block order (16 waves per 64 columns, each wave a fixed stride of rows, then the 16 wave sums in
// order): dw without atomics, bit-reproducible, and no memset (M = 0 writes zeros).
//
// Element types are runtime codes (0 fp16, 1 bf16, 2 fp32), uniform per launch, converted to fp32 at
// the load and rounded at the store: the kernels are HBM-bound, so a uniform branch per vector is free.
#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>

#include <string>
#include <type_traits>

#include "nanonemo_rmsnorm.h"

#define NNRMS_API extern "C" __attribute__((visibility("default")))

namespace {

using u16 = unsigned short;
typedef u16 u16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

constexpr int kF16 = 0, kBF16 = 1, kF32 = 2;
constexpr int kWaves = 4;         // waves per block of the forward
constexpr int kBwdWaves = 8;      // waves per block of the backward (4 for the widest rows, see bwd_waves)
constexpr int kBwdBlocks = 512;   // most blocks of the backward (each then owns one dw partial row)
constexpr int kSumWaves = 16;     // waves of a column-sum block

__host__ __device__ inline int elem_bytes(int dt) { return dt == kF32 ? 4 : 2; }

// Vector j (8 elements) of a row-major array of element type dt, widened to fp32.
__device__ inline f32x8 load_vec(const void* base, long long j, int dt) {
    if (dt == kF32) {
        const f32x4* p = reinterpret_cast<const f32x4*>(base) + 2 * j;
        const f32x4 a = p[0], b = p[1];
        return f32x8{a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
    }
    const u16x8 raw = reinterpret_cast<const u16x8*>(base)[j];
    f32x8 v;
    if (dt == kBF16) {
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = __uint_as_float((uint32_t)raw[e] << 16);
    } else {
        const f16x8 hv = __builtin_bit_cast(f16x8, raw);
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = (float)hv[e];
    }
    return v;
}

// Vector j of a row-major array of type dt from fp32, rounded to nearest even.
__device__ inline void store_vec(void* base, long long j, int dt, const f32x8& v) {
    if (dt == kF32) {
        f32x4* p = reinterpret_cast<f32x4*>(base) + 2 * j;
        p[0] = f32x4{v[0], v[1], v[2], v[3]};
        p[1] = f32x4{v[4], v[5], v[6], v[7]};
    } else if (dt == kBF16) {
        bf16x8 r;
#pragma unroll
        for (int e = 0; e < 8; ++e) r[e] = (__bf16)v[e];
        reinterpret_cast<u16x8*>(base)[j] = __builtin_bit_cast(u16x8, r);
    } else {
        f16x8 r;
#pragma unroll
        for (int e = 0; e < 8; ++e) r[e] = (_Float16)v[e];
        reinterpret_cast<u16x8*>(base)[j] = __builtin_bit_cast(u16x8, r);
    }
}

__device__ inline float load_one(const void* base, long long i, int dt) {
    if (dt == kF32) return reinterpret_cast<const float*>(base)[i];
    const u16 raw = reinterpret_cast<const u16*>(base)[i];
    return dt == kBF16 ? __uint_as_float((uint32_t)raw << 16) : (float)__builtin_bit_cast(_Float16, raw);
}

__device__ inline void store_one(void* base, long long i, int dt, float v) {
    if (dt == kF32)
        reinterpret_cast<float*>(base)[i] = v;
    else if (dt == kBF16)
        reinterpret_cast<__bf16*>(base)[i] = (__bf16)v;
    else
        reinterpret_cast<_Float16*>(base)[i] = (_Float16)v;
}

// The value a store to dtype dt would keep.
__device__ inline float keep_as(float v, int dt) {
    return dt == kBF16 ? (float)(__bf16)v : dt == kF16 ? (float)(_Float16)v : v;
}

// Sum over the R lanes of a team (R a power of two, teams aligned to R lanes).
template <int R>
__device__ inline float team_sum(float v) {
#pragma unroll
    for (int m = R / 2; m > 0; m >>= 1) v += __shfl_xor(v, m);
    return v;
}

// A row's slice held by one lane: K units of W elements (W = 8: 16-byte vectors; W = 1: single
// elements); unit k is the row's unit t + k R.
template <int W, int K>
struct Slice {
    float v[K][W];
};

template <int W, int K, int R>
__device__ inline void load_slice(const void* row, int dt, int t, int units, Slice<W, K>& s) {
#pragma unroll
    for (int k = 0; k < K; ++k) {
        const int u = t + k * R;
        if constexpr (W == 8) {
            const f32x8 x = u < units ? load_vec(row, u, dt) : f32x8{};
#pragma unroll
            for (int e = 0; e < 8; ++e) s.v[k][e] = x[e];
        } else {
            s.v[k][0] = u < units ? load_one(row, u, dt) : 0.f;
        }
    }
}

template <int W, int K, int R>
__device__ inline void store_slice(void* row, int dt, int t, int units, const Slice<W, K>& s) {
#pragma unroll
    for (int k = 0; k < K; ++k) {
        const int u = t + k * R;
        if (u >= units) continue;
        if constexpr (W == 8) {
            f32x8 x;
#pragma unroll
            for (int e = 0; e < 8; ++e) x[e] = s.v[k][e];
            store_vec(row, u, dt, x);
        } else {
            store_one(row, u, dt, s.v[k][0]);
        }
    }
}

// The weight's units of this lane (fp32 [N]).
template <int W, int K, int R>
__device__ inline void load_weight(const float* w, int t, int units, Slice<W, K>& s) {
    load_slice<W, K, R>(w, kF32, t, units, s);
}

// ------------------------------------------------------------------------------------------
// Forward: one row per team, 4 waves per block.
// ------------------------------------------------------------------------------------------
template <int W, int K, int R, bool DELTA>
__global__ __launch_bounds__(64 * kWaves) void add_rmsnorm_fwd_kernel(const void* __restrict__ x,
                                                                       const void* __restrict__ delta,
                                                                       const float* __restrict__ w,
                                                                       void* __restrict__ y, void* __restrict__ h,
                                                                       float* __restrict__ rstd, long long M, int N,
                                                                       float eps, int xdt, int ddt, int hdt, int ydt) {
    constexpr int TPB = 64 * kWaves / R;  // teams (rows) per block
    const int team = threadIdx.x / R, t = threadIdx.x % R;
    const long long row = (long long)blockIdx.x * TPB + team;
    if (row >= M) return;  // a whole team leaves together (teams never straddle a row)
    const int units = N / W;
    const long long off = row * N;  // element offset of the row
    const int xb = elem_bytes(xdt);

    Slice<W, K> hv, wv, dv;
    load_weight<W, K, R>(w, t, units, wv);
    load_slice<W, K, R>((const char*)x + off * xb, xdt, t, units, hv);
    if constexpr (DELTA) load_slice<W, K, R>((const char*)delta + off * elem_bytes(ddt), ddt, t, units, dv);
    if constexpr (DELTA) {
#pragma unroll
        for (int k = 0; k < K; ++k)
#pragma unroll
            for (int e = 0; e < W; ++e) hv.v[k][e] = keep_as(hv.v[k][e] + dv.v[k][e], hdt);
        store_slice<W, K, R>((char*)h + off * elem_bytes(hdt), hdt, t, units, hv);
    }
    float ss = 0.f;
#pragma unroll
    for (int k = 0; k < K; ++k)
#pragma unroll
        for (int e = 0; e < W; ++e) ss = fmaf(hv.v[k][e], hv.v[k][e], ss);
    const float r = rsqrtf(team_sum<R>(ss) / (float)N + eps);
#pragma unroll
    for (int k = 0; k < K; ++k)
#pragma unroll
        for (int e = 0; e < W; ++e) hv.v[k][e] = (hv.v[k][e] * r) * wv.v[k][e];
    store_slice<W, K, R>((char*)y + off * elem_bytes(ydt), ydt, t, units, hv);
    if (t == 0) rstd[row] = r;
}

// ------------------------------------------------------------------------------------------
// Backward: a fixed grid; each team walks rows team_id + i * teams, keeping dw in registers; then the
// teams of a wave are summed over their lane groups and the block's waves in LDS into partial row
// blockIdx.x.
// ------------------------------------------------------------------------------------------
template <int W, int K, int R, bool DELTA, int NWV, bool PIPE>
__global__ __launch_bounds__(64 * NWV) void add_rmsnorm_bwd_kernel(
    const void* __restrict__ dy, const void* __restrict__ dh, const void* __restrict__ h, const float* __restrict__ w,
    const float* __restrict__ rstd, void* __restrict__ dx, void* __restrict__ ddelta, float* __restrict__ dw_part,
    long long M, int N, int dydt, int hdt, int dxdt, int dddt) {
    constexpr int TPB = 64 * NWV / R;
    // Wide rows (more than 32 values per lane) take two passes over the row per team: the first sums g * h and
    // dw, the second re-reads the row (now in cache) for dx, so that only dw stays resident across rows.
    constexpr bool TWO_PASS = W * K > 32;
    // PIPE: one pass per row, software-pipelined over the team's rows (two rows' values in registers beside dw and
    // the weight); the host selects it where it measured faster (see bwd_pipelined). Otherwise rows of up to 32
    // values per lane take one pass, a row at a time.
    static_assert(!PIPE || W * K <= 24, "two rows of this width do not fit in registers");
    __shared__ float red[NWV][R * W];  // one unit's dw per wave, per lane position
    const int team = threadIdx.x / R, t = threadIdx.x % R, wave = threadIdx.x >> 6;
    const int units = N / W;
    const long long teams = (long long)gridDim.x * TPB;
    const int dyb = elem_bytes(dydt), hb = elem_bytes(hdt);

    Slice<W, K> wv, acc;
    if constexpr (!TWO_PASS) load_weight<W, K, R>(w, t, units, wv);
#pragma unroll
    for (int k = 0; k < K; ++k)
#pragma unroll
        for (int e = 0; e < W; ++e) acc.v[k][e] = 0.f;

    // Unit k of this lane of tensor p (dtype dt) at row offset off, widened to fp32 (zeros past the row).
    auto unit = [&](const void* p, int dt, long long off, int k, float* v) {
        const int u = t + k * R;
        if constexpr (W == 8) {
            const f32x8 x = u < units ? load_vec((const char*)p + off * elem_bytes(dt), u, dt) : f32x8{};
#pragma unroll
            for (int e = 0; e < 8; ++e) v[e] = x[e];
        } else {
            v[0] = u < units ? load_one((const char*)p + off * elem_bytes(dt), u, dt) : 0.f;
        }
    };

    if constexpr (PIPE) {
        // The next row's loads are issued before this row's arithmetic and stores, so that the grid's reads and
        // writes overlap (the host gives every team at least two rows where the rows allow it).
        auto fetch = [&](long long rw, Slice<W, K>& g, Slice<W, K>& hv, Slice<W, K>& res, float& r) {
            const long long off = rw * N;
            r = rstd[rw];
            load_slice<W, K, R>((const char*)dy + off * dyb, dydt, t, units, g);
            load_slice<W, K, R>((const char*)h + off * hb, hdt, t, units, hv);
            if constexpr (DELTA) load_slice<W, K, R>((const char*)dh + off * hb, hdt, t, units, res);
        };
        Slice<W, K> gv, hv, res;  // this row: dy (then g, then the gradient), h, and dh
        float r = 0.f;
        long long row = (long long)blockIdx.x * TPB + team;
        if (row < M) fetch(row, gv, hv, res, r);
        for (; row < M; row += teams) {
            Slice<W, K> ng, nh, nres;
            float nr = 0.f;
            if (row + teams < M) fetch(row + teams, ng, nh, nres, nr);
            const long long off = row * N;
            float s = 0.f;
#pragma unroll
            for (int k = 0; k < K; ++k)
#pragma unroll
                for (int e = 0; e < W; ++e) {
                    acc.v[k][e] = fmaf(gv.v[k][e], hv.v[k][e] * r, acc.v[k][e]);  // dw += dy * (h r)
                    gv.v[k][e] *= wv.v[k][e];                                     // g = dy * w
                    s = fmaf(gv.v[k][e], hv.v[k][e], s);
                }
            const float c = r * r * r * team_sum<R>(s) / (float)N;
#pragma unroll
            for (int k = 0; k < K; ++k)
#pragma unroll
                for (int e = 0; e < W; ++e) {
                    const float d = gv.v[k][e] * r - hv.v[k][e] * c;
                    gv.v[k][e] = DELTA ? d + res.v[k][e] : d;
                }
            store_slice<W, K, R>((char*)dx + off * elem_bytes(dxdt), dxdt, t, units, gv);
            if constexpr (DELTA) store_slice<W, K, R>((char*)ddelta + off * elem_bytes(dddt), dddt, t, units, gv);
            gv = ng;
            hv = nh;
            if constexpr (DELTA) res = nres;
            r = nr;
        }
    }
    for (long long row = (long long)blockIdx.x * TPB + team; !PIPE && row < M; row += teams) {
        const long long off = row * N;
        const float r = rstd[row];
        if constexpr (TWO_PASS) {
            float s = 0.f;
#pragma unroll
            for (int k = 0; k < K; ++k) {
                float g[W], hv[W], wk[W];
                unit(dy, dydt, off, k, g);
                unit(h, hdt, off, k, hv);
                unit(w, kF32, 0, k, wk);
#pragma unroll
                for (int e = 0; e < W; ++e) {
                    acc.v[k][e] = fmaf(g[e], hv[e] * r, acc.v[k][e]);  // dw += dy * (h r)
                    s = fmaf(g[e] * wk[e], hv[e], s);                   // g = dy * w
                }
                __builtin_amdgcn_sched_barrier(0);  // keep each unit's loads next to their use (registers)
            }
            const float c = r * r * r * team_sum<R>(s) / (float)N;
            // the second pass re-reads the row from cache: without this the compiler keeps the first pass's loaded
            // values live instead (the same addresses), which is what this form avoids
            __asm__ volatile("" ::: "memory");
#pragma unroll
            for (int k = 0; k < K; ++k) {
                const int u = t + k * R;
                if (u >= units) continue;
                float g[W], hv[W], wk[W], res[W];
                unit(dy, dydt, off, k, g);
                unit(h, hdt, off, k, hv);
                unit(w, kF32, 0, k, wk);
                if constexpr (DELTA) unit(dh, hdt, off, k, res);
                f32x8 d8;
#pragma unroll
                for (int e = 0; e < W; ++e) {
                    const float d = (g[e] * wk[e]) * r - hv[e] * c;
                    g[e] = DELTA ? d + res[e] : d;
                    if constexpr (W == 8) d8[e] = g[e];
                }
                if constexpr (W == 8) {
                    store_vec((char*)dx + off * elem_bytes(dxdt), u, dxdt, d8);
                    if constexpr (DELTA) store_vec((char*)ddelta + off * elem_bytes(dddt), u, dddt, d8);
                } else {
                    store_one((char*)dx + off * elem_bytes(dxdt), u, dxdt, g[0]);
                    if constexpr (DELTA) store_one((char*)ddelta + off * elem_bytes(dddt), u, dddt, g[0]);
                }
                __builtin_amdgcn_sched_barrier(0);
            }
        } else {
            Slice<W, K> gv, hv, res;  // dy (then g, then the gradient), h, and dh
            load_slice<W, K, R>((const char*)dy + off * dyb, dydt, t, units, gv);
            load_slice<W, K, R>((const char*)h + off * hb, hdt, t, units, hv);
            if constexpr (DELTA) load_slice<W, K, R>((const char*)dh + off * hb, hdt, t, units, res);
            float s = 0.f;
#pragma unroll
            for (int k = 0; k < K; ++k)
#pragma unroll
                for (int e = 0; e < W; ++e) {
                    acc.v[k][e] = fmaf(gv.v[k][e], hv.v[k][e] * r, acc.v[k][e]);  // dw += dy * (h r)
                    gv.v[k][e] *= wv.v[k][e];                                     // g = dy * w
                    s = fmaf(gv.v[k][e], hv.v[k][e], s);
                }
            const float c = r * r * r * team_sum<R>(s) / (float)N;
#pragma unroll
            for (int k = 0; k < K; ++k)
#pragma unroll
                for (int e = 0; e < W; ++e) {
                    const float d = gv.v[k][e] * r - hv.v[k][e] * c;
                    gv.v[k][e] = DELTA ? d + res.v[k][e] : d;
                }
            store_slice<W, K, R>((char*)dx + off * elem_bytes(dxdt), dxdt, t, units, gv);
            if constexpr (DELTA) store_slice<W, K, R>((char*)ddelta + off * elem_bytes(dddt), dddt, t, units, gv);
        }
    }

    // Unit by unit: the wave's teams hold the same columns in lanes t, t + R, ... (an xor-butterfly over those lane
    // groups leaves every lane with the wave's sum), then the block's waves are added in wave order.
#pragma unroll
    for (int k = 0; k < K; ++k) {
#pragma unroll
        for (int e = 0; e < W; ++e) {
            float a = acc.v[k][e];
#pragma unroll
            for (int m = R; m < 64; m <<= 1) a += __shfl_xor(a, m);
            if ((threadIdx.x & 63) < R) red[wave][t * W + e] = a;
        }
        __syncthreads();
        // element t W + e of a wave's slot is column (t + k R) W + e
        for (int i = threadIdx.x; i < R * W; i += 64 * NWV) {
            const int col = (i / W + k * R) * W + i % W;
            if (col < N) {
                float sum = 0.f;
#pragma unroll
                for (int m = 0; m < NWV; ++m) sum += red[m][i];
                dw_part[(long long)blockIdx.x * N + col] = sum;
            }
        }
        __syncthreads();
    }
}

// dw[c] = sum over p = 0 .. P-1 of part[p][c], in a fixed order: a block of 16 waves owns 64 columns; wave v
// loads rows v, v + 16, ..., v + 16 * 31 at once (P <= kBwdBlocks = 512, so one round trip to memory) and adds
// them as a fixed pairwise tree, and the 16 wave sums are then added in wave order. P = 0 writes zeros.
__global__ __launch_bounds__(64 * kSumWaves) void colsum_kernel(const float* __restrict__ part,
                                                                float* __restrict__ dw, int P, int N) {
    static_assert(kBwdBlocks <= 32 * kSumWaves, "a wave sums at most 32 partial rows");
    __shared__ float red[kSumWaves][64];
    const int v = threadIdx.x >> 6, l = threadIdx.x & 63;
    const int c = blockIdx.x * 64 + l;
    float x[32];
#pragma unroll
    for (int u = 0; u < 32; ++u) {
        const int p = v + u * kSumWaves;
        x[u] = c < N && p < P ? part[(long long)p * N + c] : 0.f;
    }
#pragma unroll
    for (int w = 16; w > 0; w >>= 1)
#pragma unroll
        for (int u = 0; u < w; ++u) x[u] += x[u + w];
    const float acc = x[0];
    red[v][l] = acc;
    __syncthreads();
    if (v == 0 && c < N) {
        float s = 0.f;
#pragma unroll
        for (int m = 0; m < kSumWaves; ++m) s += red[m][l];
        dw[c] = s;
    }
}

// ------------------------------------------------------------------------------------------
// Host side.
// ------------------------------------------------------------------------------------------
thread_local std::string g_err;

int fail(const char* fmt, ...) __attribute__((format(printf, 1, 2)));
int fail(const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_err = buf;
    return -1;
}

int launched(const char* what) {
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        g_err = std::string(what) + " launch failed: " + hipGetErrorString(e);
        return (int)e;
    }
    return 0;
}

bool valid_dt(int dt) { return dt == kF16 || dt == kBF16 || dt == kF32; }
bool aligned(const void* p, int a) { return ((uintptr_t)p & (uintptr_t)(a - 1)) == 0; }

// The residual's dtype: fp32 if either is fp32 or they differ (fp16 + bf16), else their common type.
int promote(int a, int b) { return a == b ? a : kF32; }

// The team layout for a width: (W, R, K). 16-byte vectors (W = 8) when N is a multiple of 8 up to 4096;
// single elements (W = 1, one 64-lane team, up to 16 per lane) for other widths up to 1024.
struct Layout {
    int W, R, K;
};
// The forward uses 64-lane teams up to 128 vectors as well (one row per wave, 2 vectors per lane at most):
// measured faster than 32-lane teams for its single pass (14.6 against 14.8 us at 8192 x 768, 57.3 against
// 61.5 us at 32768 x 768); the backward keeps 32-lane teams (two rows per wave, 3 vectors per lane at 768).
int pick_layout(long long N, Layout* L, bool fwd = false) {
    if (N % 8 == 0 && N >= 8 && N <= 4096) {
        const int units = (int)(N / 8);
        L->W = 8;
        L->R = units <= 128 && !fwd ? 32 : 64;
        const int k = (units + L->R - 1) / L->R;
        L->K = L->R == 32 ? k : L->R == 64 && units <= 128 ? 2 : (k <= 4 ? 4 : k <= 6 ? 6 : 8);
        return 0;
    }
    if (N >= 1 && N <= 1024) {
        L->W = 1;
        L->R = 64;
        L->K = 16;
        return 0;
    }
    return fail("hidden size must be <= 1024, or a multiple of 8 and <= 4096; got %lld", N);
}

template <typename F>
int with_layout(const Layout& L, bool delta, F&& f) {
#define NNRMS_CASE(W_, R_, K_)                                                                    \
    if (L.W == W_ && L.R == R_ && L.K == K_)                                                      \
        return delta ? f(std::integral_constant<int, W_>{}, std::integral_constant<int, K_>{},    \
                         std::integral_constant<int, R_>{}, std::true_type{})                     \
                     : f(std::integral_constant<int, W_>{}, std::integral_constant<int, K_>{},    \
                         std::integral_constant<int, R_>{}, std::false_type{});
    NNRMS_CASE(8, 32, 1)
    NNRMS_CASE(8, 32, 2)
    NNRMS_CASE(8, 32, 3)
    NNRMS_CASE(8, 32, 4)
    NNRMS_CASE(8, 64, 2)
    NNRMS_CASE(8, 64, 4)
    NNRMS_CASE(8, 64, 6)
    NNRMS_CASE(8, 64, 8)
    NNRMS_CASE(1, 64, 16)
#undef NNRMS_CASE
    return fail("internal: no layout variant for W=%d R=%d K=%d", L.W, L.R, L.K);
}

long long rows_per_block(const Layout& L) { return 64LL * kWaves / L.R; }

// Waves per backward block: 8, or 4 for rows of more than 48 values per lane, whose resident dw alone is 64
// values (4 waves leave a wave up to 512 registers; 8 cap it at 256, which such a row exceeds).
template <int W, int K>
constexpr int bwd_waves() { return W * K > 48 ? 4 : kBwdWaves; }
int bwd_waves_of(const Layout& L) { return L.W * L.K > 48 ? 4 : kBwdWaves; }

// The pipelined backward, with two rows per team, for rows of three 8-element units per lane (N = 520 .. 768 in
// 32-lane teams, the 114 M model's width) where two rows per team give 256 to 512 blocks. Measured against a row
// at a time (interleaved A/B): 22.9 against 27.5 us at 8192 x 768, 40.8 against 43.2 at 16384 x 768; with fewer
// blocks than CUs, with teams walking more rows (32768 x 768: +2.6 %) or at other widths (8192 x 512: +3 %,
// 16384 x 512: +9 %) it is slower, and those shapes keep the row-at-a-time kernel.
constexpr long long kBwdFillBlocks = 256;
bool bwd_pipelined(long long M, const Layout& L) {
    const long long per = 64LL * bwd_waves_of(L) / L.R;  // teams per block
    const long long b2 = (M + 2 * per - 1) / (2 * per);
    return L.W == 8 && L.K == 3 && b2 >= kBwdFillBlocks && b2 <= kBwdBlocks;
}

// Backward grid: one row per team (two when pipelined), at most kBwdBlocks blocks, whose teams then walk further rows.
long long bwd_blocks(long long M, const Layout& L) {
    const long long per = 64LL * bwd_waves_of(L) / L.R * (bwd_pipelined(M, L) ? 2 : 1);
    const long long b = (M + per - 1) / per;
    return b < kBwdBlocks ? b : kBwdBlocks;
}

}  // namespace

NNRMS_API const char* nn_rmsnorm_last_error(void) { return g_err.c_str(); }

NNRMS_API int nn_add_rmsnorm_fwd(const void* x, const void* delta, const float* weight, void* y, void* h, float* rstd,
                                 int64_t M, int64_t N, float eps, int x_dtype, int delta_dtype, int y_dtype,
                                 void* stream) {
    g_err.clear();
    if (M < 0 || N < 1) return fail("invalid sizes M=%lld N=%lld", (long long)M, (long long)N);
    if (!valid_dt(x_dtype) || !valid_dt(y_dtype) || (delta && !valid_dt(delta_dtype)))
        return fail("dtype must be float16, bfloat16 or float32");
    if (!(eps >= 0.f)) return fail("eps must be non-negative");
    Layout L;
    if (int e = pick_layout(N, &L, true)) return e;
    if (M == 0) return 0;
    if (!x || !weight || !y || !rstd || (delta && !h)) return fail("null pointer argument");
    const int hdt = delta ? promote(x_dtype, delta_dtype) : x_dtype;
    auto al = [&](const void* p, int dt) { return aligned(p, L.W == 8 ? 16 : elem_bytes(dt)); };
    if (!al(x, x_dtype) || !al(y, y_dtype) || !al(weight, kF32) || (delta && (!al(delta, delta_dtype) || !al(h, hdt))))
        return fail("tensors must be 16-byte aligned");
    const long long blocks = (M + rows_per_block(L) - 1) / rows_per_block(L);
    if (blocks >= (1LL << 31)) return fail("too many rows");
    hipStream_t st = (hipStream_t)stream;
    return with_layout(L, delta != nullptr, [&](auto w_, auto k_, auto r_, auto d_) {
        add_rmsnorm_fwd_kernel<decltype(w_)::value, decltype(k_)::value, decltype(r_)::value, decltype(d_)::value>
            <<<dim3((unsigned)blocks), dim3(64 * kWaves), 0, st>>>(x, delta, weight, y, h, rstd, (long long)M, (int)N,
                                                                    eps, x_dtype, delta ? delta_dtype : x_dtype, hdt,
                                                                    y_dtype);
        return launched("add_rmsnorm_fwd_kernel");
    });
}

NNRMS_API size_t nn_add_rmsnorm_bwd_workspace_size(int64_t M, int64_t N) {
    Layout L;
    if (M <= 0 || N <= 0 || pick_layout(N, &L)) return 0;
    return (size_t)bwd_blocks(M, L) * (size_t)N * 4;
}

NNRMS_API int nn_add_rmsnorm_bwd(const void* dy, const void* dh, const void* h, const float* weight, const float* rstd,
                                 void* dx, void* ddelta, float* dw, void* workspace, size_t workspace_bytes, int64_t M,
                                 int64_t N, int dy_dtype, int h_dtype, int dx_dtype, int ddelta_dtype, void* stream) {
    g_err.clear();
    if (M < 0 || N < 1) return fail("invalid sizes M=%lld N=%lld", (long long)M, (long long)N);
    if (!valid_dt(dy_dtype) || !valid_dt(h_dtype) || !valid_dt(dx_dtype) || (dh && !valid_dt(ddelta_dtype)))
        return fail("dtype must be float16, bfloat16 or float32");
    Layout L;
    if (int e = pick_layout(N, &L)) return e;
    if (!dw || !weight) return fail("null pointer argument");
    hipStream_t st = (hipStream_t)stream;
    const unsigned cblocks = (unsigned)((N + 63) / 64);
    if (M == 0) {  // no rows: dw = 0, written by the column sum over no partial rows (a kernel, not a memset)
        colsum_kernel<<<dim3(cblocks), dim3(64 * kSumWaves), 0, st>>>(nullptr, dw, 0, (int)N);
        return launched("colsum_kernel");
    }
    if (!dy || !h || !rstd || !dx || (dh && !ddelta)) return fail("null pointer argument");
    const size_t need = nn_add_rmsnorm_bwd_workspace_size(M, N);
    if (!workspace) return fail("null workspace");
    if (workspace_bytes < need) return fail("workspace too small: %zu bytes given, %zu needed", workspace_bytes, need);
    auto al = [&](const void* p, int dt) { return aligned(p, L.W == 8 ? 16 : elem_bytes(dt)); };
    if (!al(dy, dy_dtype) || !al(h, h_dtype) || !al(dx, dx_dtype) || !aligned(weight, L.W == 8 ? 16 : 4) ||
        !aligned(workspace, 16) || !aligned(dw, 4) || (dh && (!al(dh, h_dtype) || !al(ddelta, ddelta_dtype))))
        return fail("tensors must be 16-byte aligned");
    const long long P = bwd_blocks(M, L);
    const bool pipe = bwd_pipelined(M, L);
    int rc = with_layout(L, dh != nullptr, [&](auto w_, auto k_, auto r_, auto d_) {
        constexpr int W = decltype(w_)::value, K = decltype(k_)::value, R = decltype(r_)::value;
        constexpr bool D = decltype(d_)::value;
        constexpr int NWV = bwd_waves<W, K>();
        auto go = [&](auto kern) {
            kern<<<dim3((unsigned)P), dim3(64 * NWV), 0, st>>>(dy, dh, h, weight, rstd, dx, ddelta, (float*)workspace,
                                                                (long long)M, (int)N, dy_dtype, h_dtype, dx_dtype,
                                                                dh ? ddelta_dtype : dx_dtype);
            return launched("add_rmsnorm_bwd_kernel");
        };
        if constexpr (W == 8 && K == 3) {
            if (pipe) return go(add_rmsnorm_bwd_kernel<W, K, R, D, NWV, true>);
        }
        return go(add_rmsnorm_bwd_kernel<W, K, R, D, NWV, false>);
    });
    if (rc) return rc;
    colsum_kernel<<<dim3(cblocks), dim3(64 * kSumWaves), 0, st>>>((const float*)workspace, dw, (int)P, (int)N);
    return launched("colsum_kernel");
}
