// Rotary position embedding (rotate-half) of q and k in one launch, for MI355X (gfx950).
//
// Semantics of /root/reference/nanonemo/model/layers.py:67-74 (apply_rope) and the reference's
// fused Triton version (nanonemo/kernels/triton/rope.py, which rotates Q and K in one launch in the
// (B, T, heads, hd) layout): for each row x of head_dim D at sequence position t, with half = D/2,
//     y[i]        = x[i] * cos[t][i] - x[i + half] * sin[t][i]
//     y[i + half] = x[i] * sin[t][i] + x[i + half] * cos[t][i]        (i < half)
// computed in fp32 with one rounding per product and per sum (the order of the reference's
// elementwise torch ops, so the result is bit-identical to it) and rounded once to the output dtype.
// The backward applies the inverse rotation (angle -theta) to the incoming gradient.
//
// Layout: x is a [B][T][heads][D] view with element strides {batch, row (position), head} and unit D
// stride; q and k may have different head counts and strides; outputs are written with the same
// strides as their inputs. The tables are dense fp32 [T_max][half]. The kernel is HBM-bound: each
// thread moves 8 pairs (two 16-byte loads and two 16-byte stores of 16-bit data).
#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>

#include <string>

#include "nanonemo_rope.h"

#define NNROPE_API extern "C" __attribute__((visibility("default")))

namespace {

using u16 = unsigned short;
typedef u16 u16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

constexpr int kF16 = 0, kBF16 = 1, kF32 = 2;

// 8 consecutive elements of a row, converted to / from fp32 (16 bytes for the 16-bit types).
template <int DT>
struct Vec8 {
    __device__ static void load(const char* p, float* v) {
        if constexpr (DT == kF32) {
            const f32x4 a = *reinterpret_cast<const f32x4*>(p), b = *reinterpret_cast<const f32x4*>(p + 16);
#pragma unroll
            for (int j = 0; j < 4; ++j) v[j] = a[j], v[j + 4] = b[j];
        } else {
            const u16x8 w = *reinterpret_cast<const u16x8*>(p);
            if constexpr (DT == kBF16) {
#pragma unroll
                for (int j = 0; j < 8; ++j) v[j] = __uint_as_float((uint32_t)w[j] << 16);
            } else {
                // whole-vector bit cast (a bit cast of one subscripted element came out as element 0)
                const f16x8 hv = __builtin_bit_cast(f16x8, w);
#pragma unroll
                for (int j = 0; j < 8; ++j) v[j] = (float)hv[j];
            }
        }
    }
    __device__ static void store(char* p, const float* v) {  // round to nearest even
        if constexpr (DT == kF32) {
            *reinterpret_cast<f32x4*>(p) = f32x4{v[0], v[1], v[2], v[3]};
            *reinterpret_cast<f32x4*>(p + 16) = f32x4{v[4], v[5], v[6], v[7]};
        } else if constexpr (DT == kBF16) {
            bf16x8 r;
#pragma unroll
            for (int j = 0; j < 8; ++j) r[j] = (__bf16)v[j];
            *reinterpret_cast<u16x8*>(p) = __builtin_bit_cast(u16x8, r);
        } else {
            f16x8 r;
#pragma unroll
            for (int j = 0; j < 8; ++j) r[j] = (_Float16)v[j];
            *reinterpret_cast<u16x8*>(p) = __builtin_bit_cast(u16x8, r);
        }
    }
    static constexpr int bytes = DT == kF32 ? 4 : 2;
};

struct Side {  // one of q / k
    const char* x;
    char* y;
    long long sb, st, sh;  // element strides: batch, position, head
};

// One rounding per product and per sum, as the reference's separate torch ops do: no contraction
// into fma (which the compiler otherwise forms even from __fmul_rn / __fsub_rn).
__device__ inline float mul(float a, float b) {
#pragma clang fp contract(off)
    return a * b;
}
__device__ inline float add(float a, float b) {
#pragma clang fp contract(off)
    return a + b;
}
__device__ inline float sub(float a, float b) {
#pragma clang fp contract(off)
    return a - b;
}

// Thread = 8 consecutive pairs (i0 .. i0+7 with their partners i + half) of one row. Threads are
// ordered (batch, position, head, chunk) with the H q heads before the KVH k heads of a position, so
// consecutive threads cover the contiguous q row block and then the k row block of one position.
// 32-bit index arithmetic (the host checks that the thread count fits).
template <int DT, bool INVERSE>
__global__ __launch_bounds__(256) void rope_qk_kernel(Side q, Side k, const float* __restrict__ cosT,
                                                      const float* __restrict__ sinT, int T, int H, int heads,
                                                      int half, int cpr, int nthreads) {
    using V = Vec8<DT>;
    const int gid = blockIdx.x * 256 + threadIdx.x;
    if (gid >= nthreads) return;
    const int row = gid / cpr;  // (b, t, head) in [B][T][H + KVH] order
    const int i0 = (gid - row * cpr) * 8;
    const int bt = row / heads;
    const int hh = row - bt * heads;
    const int b = bt / T, t = bt - b * T;
    // field by field (not a reference to either parameter, which would take its address)
    const bool isq = hh < H;
    const int h = isq ? hh : hh - H;
    const char* xp = isq ? q.x : k.x;
    char* yp = isq ? q.y : k.y;
    const long long off = b * (isq ? q.sb : k.sb) + (long long)t * (isq ? q.st : k.st) +
                          (long long)h * (isq ? q.sh : k.sh) + i0;
    float x1[8], x2[8], c[8], sn[8], y1[8], y2[8];
    V::load(xp + off * V::bytes, x1);
    V::load(xp + (off + half) * V::bytes, x2);
    const f32x4* cp = reinterpret_cast<const f32x4*>(cosT + t * half + i0);
    const f32x4* sp = reinterpret_cast<const f32x4*>(sinT + t * half + i0);
#pragma unroll
    for (int j = 0; j < 4; ++j) c[j] = cp[0][j], c[j + 4] = cp[1][j], sn[j] = sp[0][j], sn[j + 4] = sp[1][j];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        if (!INVERSE) {
            y1[j] = sub(mul(x1[j], c[j]), mul(x2[j], sn[j]));
            y2[j] = add(mul(x1[j], sn[j]), mul(x2[j], c[j]));
        } else {  // rotation by -theta: the transpose of the forward rotation
            y1[j] = add(mul(x1[j], c[j]), mul(x2[j], sn[j]));
            y2[j] = sub(mul(x2[j], c[j]), mul(x1[j], sn[j]));
        }
    }
    V::store(yp + off * V::bytes, y1);
    V::store(yp + (off + half) * V::bytes, y2);
}

thread_local std::string g_err;
int fail(const char* fmt, ...) __attribute__((format(printf, 1, 2)));
int fail(const char* fmt, ...) {
    char buf[256];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_err = buf;
    return -1;
}

bool aligned(const void* p, int n) { return ((uintptr_t)p % n) == 0; }

int check_side(const void* x, const void* y, int64_t heads, const int64_t* strides, int64_t D, int esize,
               const char* what) {
    if (heads < 0) return fail("invalid %s head count", what);
    if (heads == 0) return 0;
    if (!x || !y || !strides) return fail("null %s argument", what);
    for (int i = 0; i < 3; ++i)
        if (strides[i] <= 0 || strides[i] % 8) return fail("%s strides must be positive multiples of 8 elements", what);
    if (!aligned(x, 16) || !aligned(y, 16)) return fail("%s must be 16-byte aligned", what);
    (void)D;
    return 0;
}

template <int DT>
int launch(const Side& q, const Side& k, const float* cosT, const float* sinT, int T, int H, int KVH, int half,
           long long rows, bool inverse, hipStream_t st) {
    const int cpr = half / 8;
    const long long n = rows * cpr;
    if (n == 0) return 0;
    const unsigned blocks = (unsigned)((n + 255) / 256);
    if (inverse)
        rope_qk_kernel<DT, true><<<dim3(blocks), dim3(256), 0, st>>>(q, k, cosT, sinT, T, H, H + KVH, half, cpr, (int)n);
    else
        rope_qk_kernel<DT, false><<<dim3(blocks), dim3(256), 0, st>>>(q, k, cosT, sinT, T, H, H + KVH, half, cpr, (int)n);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        g_err = std::string("rope_qk_kernel launch failed: ") + hipGetErrorString(e);
        return (int)e;
    }
    return 0;
}

int rope_entry(const void* q, void* q_out, const void* k, void* k_out, const float* cos_table, const float* sin_table,
               int64_t B, int64_t T, int64_t H, int64_t KVH, int64_t D, const int64_t* q_strides,
               const int64_t* k_strides, int64_t table_rows, int dtype, bool inverse, void* stream) {
    g_err.clear();
    if (B < 0 || T < 0 || D <= 0) return fail("invalid sizes");
    if (D % 16) return fail("head_dim must be a multiple of 16");
    if (dtype != kF16 && dtype != kBF16 && dtype != kF32) return fail("dtype must be float16, bfloat16 or float32");
    if (T > table_rows) return fail("sequence length %lld exceeds the %lld rows of the tables", (long long)T, (long long)table_rows);
    if (B == 0 || T == 0 || (H == 0 && KVH == 0)) return 0;
    if (!cos_table || !sin_table) return fail("null table");
    if (!aligned(cos_table, 16) || !aligned(sin_table, 16)) return fail("tables must be 16-byte aligned");
    const int es = dtype == kF32 ? 4 : 2;
    if (int e = check_side(q, q_out, H, q_strides, D, es, "q")) return e;
    if (int e = check_side(k, k_out, KVH, k_strides, D, es, "k")) return e;
    const long long rows = (long long)B * T * (H + KVH);
    if (rows * (D / 16) >= ((int64_t)1 << 31) || T * (D / 2) >= ((int64_t)1 << 31)) return fail("sizes too large");
    Side sq{(const char*)q, (char*)q_out, H ? q_strides[0] : 0, H ? q_strides[1] : 0, H ? q_strides[2] : 0};
    Side sk{(const char*)k, (char*)k_out, KVH ? k_strides[0] : 0, KVH ? k_strides[1] : 0, KVH ? k_strides[2] : 0};
    const int half = (int)(D / 2);
    const hipStream_t st = (hipStream_t)stream;
    switch (dtype) {
        case kBF16: return launch<kBF16>(sq, sk, cos_table, sin_table, (int)T, (int)H, (int)KVH, half, rows, inverse, st);
        case kF16: return launch<kF16>(sq, sk, cos_table, sin_table, (int)T, (int)H, (int)KVH, half, rows, inverse, st);
        default: return launch<kF32>(sq, sk, cos_table, sin_table, (int)T, (int)H, (int)KVH, half, rows, inverse, st);
    }
}

}  // namespace

NNROPE_API int nn_rope_qk(const void* q, void* q_out, const void* k, void* k_out, const float* cos_table,
                          const float* sin_table, int64_t B, int64_t T, int64_t H, int64_t KVH, int64_t D,
                          const int64_t* q_strides, const int64_t* k_strides, int64_t table_rows, int dtype,
                          void* stream) {
    return rope_entry(q, q_out, k, k_out, cos_table, sin_table, B, T, H, KVH, D, q_strides, k_strides, table_rows,
                      dtype, false, stream);
}

NNROPE_API int nn_rope_qk_bwd(const void* dq_out, void* dq, const void* dk_out, void* dk, const float* cos_table,
                              const float* sin_table, int64_t B, int64_t T, int64_t H, int64_t KVH, int64_t D,
                              const int64_t* q_strides, const int64_t* k_strides, int64_t table_rows, int dtype,
                              void* stream) {
    return rope_entry(dq_out, dq, dk_out, dk, cos_table, sin_table, B, T, H, KVH, D, q_strides, k_strides, table_rows,
                      dtype, true, stream);
}

NNROPE_API const char* nn_rope_last_error(void) { return g_err.c_str(); }
