// Fused residual add + RMSNorm, forward and backward, for MI355X (gfx950).
//
// Semantics of the reference's fused kernel (/root/reference/nanonemo/kernels/cuda/rmsnorm.cu, op
// wrapper rmsnorm.py) and of the plain-PyTorch blocks it replaces (nanonemo/model/layers.py:19-56):
//     h = x + delta (rounded to h's dtype, the promotion of x's and delta's),
//     y = (h * rstd) * w,   rstd = 1 / sqrt(mean(h^2) + eps)            (fp32, rounded once to y's dtype)
// and, with n = h * rstd and dn = dy * w,
//     dh = rstd * (dn - n * mean(dn * n)) + dh_residual,   dw = sum over rows of dy * n.
// delta may be absent (y = rmsnorm(x); h is then x itself and is not written).
//
// Layout: M rows of N contiguous elements. One wave64 per row (4 rows per 256-thread block); a lane
// owns 8-element chunks lane, lane + 64, ... (16-byte loads for the 16-bit types, two for fp32) and
// keeps its row in registers between the reduction and the write, so every input is read once and
// every output written once (N a multiple of 8 up to 4096; any other N up to 1024 takes single
// elements instead). The backward walks two rows per wave at a time where they fit (N <= 2048). The
// sums of squares and of dn * n are butterfly reductions over the wave (deterministic). The
// backward's dw is reduced per block (its 4 waves through LDS) into a [blocks][N] fp32 workspace,
// then summed over blocks in a fixed order by a second kernel: no atomics, bit-reproducible.
//
// Element types are a launch-uniform runtime code (0 fp16, 1 bf16, 2 fp32) resolved inside the
// load / store helpers: the kernel is HBM-bound, and the switch is a scalar branch per chunk.
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
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

constexpr int kF16 = 0, kBF16 = 1, kF32 = 2;
constexpr int kRows = 4;          // rows (waves) per block
constexpr int kBwdBlocks = 1024;  // most blocks of the backward; each owns a range of rows

__host__ __device__ inline int elem_bytes(int dt) { return dt == kF32 ? 4 : 2; }

// V consecutive elements at element index i of a row-major array of type dt, to / from fp32.
template <int V>
__device__ inline void load(const char* base, long long i, int dt, float* v) {
    if constexpr (V == 8) {
        if (dt == kF32) {
            const f32x4* p = reinterpret_cast<const f32x4*>(base + i * 4);
            const f32x4 a = p[0], b = p[1];
#pragma unroll
            for (int j = 0; j < 4; ++j) v[j] = a[j], v[j + 4] = b[j];
        } else {
            const u16x8 w = *reinterpret_cast<const u16x8*>(base + i * 2);
            if (dt == kBF16) {
#pragma unroll
                for (int j = 0; j < 8; ++j) v[j] = __uint_as_float((uint32_t)w[j] << 16);
            } else {
                const f16x8 hv = __builtin_bit_cast(f16x8, w);
#pragma unroll
                for (int j = 0; j < 8; ++j) v[j] = (float)hv[j];
            }
        }
    } else {
        if (dt == kF32)
            v[0] = reinterpret_cast<const float*>(base)[i];
        else if (dt == kBF16)
            v[0] = __uint_as_float((uint32_t)reinterpret_cast<const u16*>(base)[i] << 16);
        else
            v[0] = (float)reinterpret_cast<const _Float16*>(base)[i];
    }
}

template <int V>
__device__ inline void store(char* base, long long i, int dt, const float* v) {  // round to nearest even
    if constexpr (V == 8) {
        if (dt == kF32) {
            f32x4* p = reinterpret_cast<f32x4*>(base + i * 4);
            p[0] = f32x4{v[0], v[1], v[2], v[3]};
            p[1] = f32x4{v[4], v[5], v[6], v[7]};
        } else if (dt == kBF16) {
            bf16x8 r;
#pragma unroll
            for (int j = 0; j < 8; ++j) r[j] = (__bf16)v[j];
            *reinterpret_cast<u16x8*>(base + i * 2) = __builtin_bit_cast(u16x8, r);
        } else {
            f16x8 r;
#pragma unroll
            for (int j = 0; j < 8; ++j) r[j] = (_Float16)v[j];
            *reinterpret_cast<u16x8*>(base + i * 2) = __builtin_bit_cast(u16x8, r);
        }
    } else {
        if (dt == kF32)
            reinterpret_cast<float*>(base)[i] = v[0];
        else if (dt == kBF16)
            reinterpret_cast<__bf16*>(base)[i] = (__bf16)v[0];
        else
            reinterpret_cast<_Float16*>(base)[i] = (_Float16)v[0];
    }
}

// fp32 value rounded to dtype dt and widened back (the value a store of dt would hold).
__device__ inline float round_to(float x, int dt) {
    if (dt == kBF16) return (float)(__bf16)x;
    if (dt == kF16) return (float)(_Float16)x;
    return x;
}

__device__ inline float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
    return v;
}

// y, h, rstd of rows blockIdx.x * 4 + wave. Chunk i of a lane: elements (lane + 64 i) * V ...
template <int V, int MAXC, bool HAS_DELTA>
__global__ __launch_bounds__(256) void add_rmsnorm_fwd_kernel(const char* __restrict__ x, const char* __restrict__ d,
                                                              const float* __restrict__ w, char* __restrict__ y,
                                                              char* __restrict__ h, float* __restrict__ rstd_out,
                                                              long long M, int N, float eps, int xdt, int ddt, int hdt,
                                                              int ydt) {
    const long long row = (long long)blockIdx.x * kRows + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (row >= M) return;  // the whole wave
    const int chunks = N / V;
    float v[MAXC][V];
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < MAXC; ++i) {
        const int c = lane + 64 * i;
        if (c >= chunks) break;
        const long long off = row * N + (long long)c * V;
        load<V>(x, off, xdt, v[i]);
        if constexpr (HAS_DELTA) {
            float dv[V];
            load<V>(d, off, ddt, dv);
#pragma unroll
            for (int j = 0; j < V; ++j) v[i][j] = round_to(v[i][j] + dv[j], hdt);  // the residual as stored
            store<V>(h, off, hdt, v[i]);
        }
#pragma unroll
        for (int j = 0; j < V; ++j) ss += v[i][j] * v[i][j];
    }
    const float rstd = 1.f / sqrtf(wave_sum(ss) / (float)N + eps);
    if (lane == 0) rstd_out[row] = rstd;
#pragma unroll
    for (int i = 0; i < MAXC; ++i) {
        const int c = lane + 64 * i;
        if (c >= chunks) break;
        float o[V];
        load<V>(reinterpret_cast<const char*>(w), (long long)c * V, kF32, o);
#pragma unroll
        for (int j = 0; j < V; ++j) o[j] *= v[i][j] * rstd;
        store<V>(y, row * N + (long long)c * V, ydt, o);
    }
}

// Rows [blockIdx.x * rpb, +rpb) of the backward, wave w taking rows w, w + 4, ... in groups of R rows
// (R = 2 while a row's operands fit in registers twice): every load of a group (h, dy and dh of its
// rows) is issued before the group's reductions, so one memory latency covers them. The dw partial of
// the block (its 4 waves summed through LDS) goes to dw_part[blockIdx.x][N].
template <int V, int MAXC, bool HAS_DELTA>
__global__ __launch_bounds__(256) void add_rmsnorm_bwd_kernel(const char* __restrict__ dy, const char* __restrict__ dh,
                                                              const char* __restrict__ h, const float* __restrict__ w,
                                                              const float* __restrict__ rstd, char* __restrict__ dx,
                                                              char* __restrict__ dd, float* __restrict__ dw_part,
                                                              long long M, int N, long long rpb, int dydt, int hdt,
                                                              int dxdt, int dddt) {
    constexpr int R = V == 8 && MAXC <= 4 ? 2 : 1;  // as bwd_rows_per_group
    __shared__ float red[2][MAXC * 64 * V];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int chunks = N / V;
    float wv[MAXC][V], dw[MAXC][V];
#pragma unroll
    for (int i = 0; i < MAXC; ++i) {
        const int c = lane + 64 * i;
        if (c < chunks) load<V>(reinterpret_cast<const char*>(w), (long long)c * V, kF32, wv[i]);
#pragma unroll
        for (int j = 0; j < V; ++j) dw[i][j] = 0.f;
    }
    const long long r0 = (long long)blockIdx.x * rpb;
    const long long r1 = r0 + rpb < M ? r0 + rpb : M;
    for (long long row0 = r0 + wave; row0 < r1; row0 += R * kRows) {
        float n[R][MAXC][V], g[R][MAXC][V], res[R][MAXC][V];
        bool live[R];
#pragma unroll
        for (int k = 0; k < R; ++k) {
            const long long row = row0 + k * kRows;
            live[k] = row < r1;
            if (!live[k]) continue;
#pragma unroll
            for (int i = 0; i < MAXC; ++i) {
                const int c = lane + 64 * i;
                if (c >= chunks) break;
                const long long off = row * N + (long long)c * V;
                load<V>(h, off, hdt, n[k][i]);
                load<V>(dy, off, dydt, g[k][i]);
                if constexpr (HAS_DELTA) load<V>(dh, off, hdt, res[k][i]);
            }
        }
#pragma unroll
        for (int k = 0; k < R; ++k) {
            if (!live[k]) continue;
            const long long row = row0 + k * kRows;
            const float r = rstd[row];
            float dot = 0.f;
#pragma unroll
            for (int i = 0; i < MAXC; ++i) {
                const int c = lane + 64 * i;
                if (c >= chunks) break;
#pragma unroll
                for (int j = 0; j < V; ++j) {
                    n[k][i][j] *= r;  // n = h * rstd
                    dw[i][j] += g[k][i][j] * n[k][i][j];
                    g[k][i][j] *= wv[i][j];  // dn = dy * w
                    dot += g[k][i][j] * n[k][i][j];
                }
            }
            const float mean = wave_sum(dot) / (float)N;
#pragma unroll
            for (int i = 0; i < MAXC; ++i) {
                const int c = lane + 64 * i;
                if (c >= chunks) break;
                const long long off = row * N + (long long)c * V;
                float o[V];
#pragma unroll
                for (int j = 0; j < V; ++j) {
                    const float gj = (g[k][i][j] - n[k][i][j] * mean) * r;
                    o[j] = HAS_DELTA ? res[k][i][j] + gj : gj;
                }
                store<V>(dx, off, dxdt, o);
                if constexpr (HAS_DELTA) store<V>(dd, off, dddt, o);
            }
        }
    }
    // Waves 2, 3 hand their partials to waves 0, 1; wave 1 then hands the pair sum to wave 0.
    if (wave >= 2) {
#pragma unroll
        for (int i = 0; i < MAXC; ++i)
#pragma unroll
            for (int j = 0; j < V; ++j) red[wave - 2][(i * 64 + lane) * V + j] = dw[i][j];
    }
    __syncthreads();
    if (wave < 2) {
#pragma unroll
        for (int i = 0; i < MAXC; ++i)
#pragma unroll
            for (int j = 0; j < V; ++j) dw[i][j] += red[wave][(i * 64 + lane) * V + j];
    }
    __syncthreads();
    if (wave == 1) {
#pragma unroll
        for (int i = 0; i < MAXC; ++i)
#pragma unroll
            for (int j = 0; j < V; ++j) red[0][(i * 64 + lane) * V + j] = dw[i][j];
    }
    __syncthreads();
    if (wave == 0) {
        float* out = dw_part + (long long)blockIdx.x * N;
#pragma unroll
        for (int i = 0; i < MAXC; ++i) {
            const int c = lane + 64 * i;
            if (c >= chunks) break;
            float s[V];
#pragma unroll
            for (int j = 0; j < V; ++j) s[j] = dw[i][j] + red[0][(i * 64 + lane) * V + j];
            store<V>(reinterpret_cast<char*>(out), (long long)c * V, kF32, s);
        }
    }
}

// Column sums of a [P][N] fp32 array over row slices: block (cb, sl) sums rows [sl * rps, +rps) of
// columns cb * 64 .. +63 into out[sl][N]. Its 4 waves take every 4th row of the slice, each with 4
// independent accumulators (so 4 loads are in flight per wave), and are then summed in wave order:
// a fixed order, so the result is bit-reproducible. The backward's dw is two of these passes: the
// per-block partials (at most 1024 rows) into slices of kSliceRows rows, then the slices into dw.
constexpr int kSliceRows = 64;
__global__ __launch_bounds__(256) void colsum_kernel(const float* __restrict__ part, float* __restrict__ out, int P,
                                                     int N, int rps) {
    __shared__ float red[kRows][64];
    const int g = threadIdx.x >> 6, l = threadIdx.x & 63;
    const int c = blockIdx.x * 64 + l;
    const int p0 = blockIdx.y * rps;
    const int p1 = p0 + rps < P ? p0 + rps : P;
    float a0 = 0.f, a1 = 0.f, a2 = 0.f, a3 = 0.f;
    if (c < N) {
        int p = p0 + g;
        for (; p + 12 < p1; p += 16) {
            a0 += part[(long long)p * N + c];
            a1 += part[(long long)(p + 4) * N + c];
            a2 += part[(long long)(p + 8) * N + c];
            a3 += part[(long long)(p + 12) * N + c];
        }
        for (; p < p1; p += 4) a0 += part[(long long)p * N + c];
    }
    red[g][l] = (a0 + a1) + (a2 + a3);
    __syncthreads();
    if (g == 0 && c < N) out[(long long)blockIdx.y * N + c] = (red[0][l] + red[1][l]) + (red[2][l] + red[3][l]);
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

// The shape variant: 16-byte chunks for N % 8 == 0 (up to 4096 elements, the reference's limit, where
// the backward's row still fits in registers), single elements up to 1024.
struct Shape {
    int V, MAXC;
};
int pick_shape(long long N, Shape* s) {
    if (N % 8 == 0 && N <= 4096) {
        const int chunks = (int)(N / 8);
        s->V = 8;
        s->MAXC = chunks <= 128 ? 2 : chunks <= 256 ? 4 : 8;
        return 0;
    }
    if (N >= 1 && N <= 1024) {
        s->V = 1;
        s->MAXC = 16;
        return 0;
    }
    return fail("hidden size must be <= 1024, or a multiple of 8 and <= 4096; got %lld", N);
}

// Backward grid: R rows per wave and group (2 for N <= 2048, where a row group fits in registers),
// a block's row range a multiple of 4R rows, at most kBwdBlocks blocks.
int bwd_rows_per_group(long long N) { return N % 8 == 0 && N <= 2048 ? 2 : 1; }
long long bwd_blocks(long long M, long long N) {
    const long long per = kRows * bwd_rows_per_group(N);
    const long long b = (M + per - 1) / per;
    return b < kBwdBlocks ? b : kBwdBlocks;
}

template <typename F>
int with_shape(const Shape& s, bool delta, F&& f) {
#define NNRMS_CASE(V_, C_)                                                                     \
    if (s.V == V_ && s.MAXC == C_)                                                             \
        return delta ? f(std::integral_constant<int, V_>{}, std::integral_constant<int, C_>{}, \
                         std::true_type{})                                                     \
                     : f(std::integral_constant<int, V_>{}, std::integral_constant<int, C_>{}, \
                         std::false_type{});
    NNRMS_CASE(8, 2)
    NNRMS_CASE(8, 4)
    NNRMS_CASE(8, 8)
    NNRMS_CASE(1, 16)
#undef NNRMS_CASE
    return fail("internal: no shape variant");
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
    Shape s;
    if (int e = pick_shape(N, &s)) return e;
    if (M == 0) return 0;
    if (!x || !weight || !y || !rstd || (delta && !h)) return fail("null pointer argument");
    const int hdt = delta ? promote(x_dtype, delta_dtype) : x_dtype;
    auto al = [&](const void* p, int dt) { return aligned(p, s.V == 8 ? 16 : elem_bytes(dt)); };
    if (!al(x, x_dtype) || !al(y, y_dtype) || !al(weight, kF32) || (delta && (!al(delta, delta_dtype) || !al(h, hdt))))
        return fail("tensors must be 16-byte aligned");
    const long long blocks = (M + kRows - 1) / kRows;
    if (blocks >= (1LL << 31)) return fail("too many rows");
    hipStream_t st = (hipStream_t)stream;
    return with_shape(s, delta != nullptr, [&](auto v, auto c, auto has_delta) {
        add_rmsnorm_fwd_kernel<decltype(v)::value, decltype(c)::value, decltype(has_delta)::value>
            <<<dim3((unsigned)blocks), dim3(256), 0, st>>>((const char*)x, (const char*)delta, weight, (char*)y,
                                                           (char*)h, rstd, (long long)M, (int)N, eps, x_dtype,
                                                           delta ? delta_dtype : x_dtype, hdt, y_dtype);
        return launched("add_rmsnorm_fwd_kernel");
    });
}

// The dw reduction's passes: the per-block partial rows, and their slice sums when there are more than
// one slice's worth.
int dw_slices(long long P) { return P <= kSliceRows ? 1 : (int)((P + kSliceRows - 1) / kSliceRows); }

NNRMS_API size_t nn_add_rmsnorm_bwd_workspace_size(int64_t M, int64_t N) {
    if (M <= 0 || N <= 0) return 0;
    const long long P = bwd_blocks(M, N);
    const int S = dw_slices(P);
    return (size_t)(P + (S > 1 ? S : 0)) * (size_t)N * 4;
}

NNRMS_API int nn_add_rmsnorm_bwd(const void* dy, const void* dh, const void* h, const float* weight, const float* rstd,
                                 void* dx, void* ddelta, float* dw, void* workspace, size_t workspace_bytes, int64_t M,
                                 int64_t N, int dy_dtype, int h_dtype, int dx_dtype, int ddelta_dtype, void* stream) {
    g_err.clear();
    if (M < 0 || N < 1) return fail("invalid sizes M=%lld N=%lld", (long long)M, (long long)N);
    if (!valid_dt(dy_dtype) || !valid_dt(h_dtype) || !valid_dt(dx_dtype) || (dh && !valid_dt(ddelta_dtype)))
        return fail("dtype must be float16, bfloat16 or float32");
    Shape s;
    if (int e = pick_shape(N, &s)) return e;
    if (!dw || !weight) return fail("null pointer argument");
    hipStream_t st = (hipStream_t)stream;
    if (M == 0) {  // no rows: dw = 0, written by the column sum over no partials (a kernel, not a memset)
        colsum_kernel<<<dim3((unsigned)((N + 63) / 64), 1), dim3(256), 0, st>>>(nullptr, dw, 0, (int)N, 1);
        return launched("colsum_kernel");
    }
    if (!dy || !h || !rstd || !dx || (dh && !ddelta)) return fail("null pointer argument");
    const size_t need = nn_add_rmsnorm_bwd_workspace_size(M, N);
    if (!workspace) return fail("null workspace");
    if (workspace_bytes < need) return fail("workspace too small: %zu bytes given, %zu needed", workspace_bytes, need);
    auto al = [&](const void* p, int dt) { return aligned(p, s.V == 8 ? 16 : elem_bytes(dt)); };
    if (!al(dy, dy_dtype) || !al(h, h_dtype) || !al(dx, dx_dtype) || !aligned(weight, s.V == 8 ? 16 : 4) ||
        !aligned(workspace, 16) || !aligned(dw, 4) || (dh && (!al(dh, h_dtype) || !al(ddelta, ddelta_dtype))))
        return fail("tensors must be 16-byte aligned");
    const long long P = bwd_blocks(M, N);
    const long long per = kRows * bwd_rows_per_group(N);
    const long long rpb = ((M + P - 1) / P + per - 1) / per * per;  // rows per block, a multiple of 4R
    const long long P_used = (M + rpb - 1) / rpb;
    int rc = with_shape(s, dh != nullptr, [&](auto v, auto c, auto has_delta) {
        add_rmsnorm_bwd_kernel<decltype(v)::value, decltype(c)::value, decltype(has_delta)::value>
            <<<dim3((unsigned)P_used), dim3(256), 0, st>>>((const char*)dy, (const char*)dh, (const char*)h, weight,
                                                           rstd, (char*)dx, (char*)ddelta, (float*)workspace,
                                                           (long long)M, (int)N, rpb, dy_dtype, h_dtype, dx_dtype,
                                                           dh ? ddelta_dtype : dx_dtype);
        return launched("add_rmsnorm_bwd_kernel");
    });
    if (rc) return rc;
    const unsigned cb = (unsigned)((N + 63) / 64);
    const int S = dw_slices(P_used);
    if (S == 1) {
        colsum_kernel<<<dim3(cb, 1), dim3(256), 0, st>>>((const float*)workspace, dw, (int)P_used, (int)N, (int)P_used);
        return launched("colsum_kernel");
    }
    float* slices = (float*)workspace + P_used * N;  // P_used <= P, so the slices fit where the size promised
    colsum_kernel<<<dim3(cb, (unsigned)S), dim3(256), 0, st>>>((const float*)workspace, slices, (int)P_used, (int)N,
                                                               kSliceRows);
    if (int e = launched("colsum_kernel")) return e;
    colsum_kernel<<<dim3(cb, 1), dim3(256), 0, st>>>(slices, dw, S, (int)N, S);
    return launched("colsum_kernel");
}
