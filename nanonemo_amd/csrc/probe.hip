// Measurement probes behind `python bench.py --probes`: not part of the attention library's ABI.
//
// nn_probe_coissue: how much VALU work a SIMD absorbs beside 32x32x16 bf16 MFMAs. Every wave runs n steps of
//   4 MFMAs (4 independent accumulators), each followed by K independent fp32 FMAs (8 independent chains), so
//   the time per MFMA as a function of K and of the waves resident per SIMD (blocks of 256 threads: 256 blocks
//   put one wave on each SIMD of a 256-CU chip, 1024 blocks four) gives the co-issue budget the attention
//   kernels' softmax VALU runs against.
// nn_probe_clock: the shader clock under a load. Every wave stamps s_memtime (shader clock) and s_memrealtime
//   (fixed 100 MHz) before and after n steps of back-to-back MFMAs (mode 0) or FMAs only (mode 1); the host
//   divides the two intervals.
//
// Values are not checked (timing probes), but every wave's result is stored, so that the loops are kept.
// Every store is a vector store of lane 0 or of every lane into buffers the host sizes from the grid.
#include <hip/hip_runtime.h>

#include <cstdint>
#include <string>

namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

thread_local std::string g_probe_error;

template <int K>
__global__ __launch_bounds__(256) void coissue_kernel(float* out, int n) {
    bf16x8 a, b;
    for (int j = 0; j < 8; ++j) {
        a[j] = (__bf16)(threadIdx.x * 1e-3f);
        b[j] = (__bf16)(j * 1e-3f);
    }
    f32x16 c0 = {}, c1 = {}, c2 = {}, c3 = {};
    float x[8];
    for (int j = 0; j < 8; ++j) x[j] = threadIdx.x * 1e-4f + j;
    for (int i = 0; i < n; ++i) {
#define NN_PROBE_STEP(c)                                                                 \
    c = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);                      \
    _Pragma("unroll") for (int k = 0; k < K; ++k) x[k % 8] = __builtin_fmaf(x[k % 8], 0.999f, 0.5f); \
    __builtin_amdgcn_sched_barrier(0);
        NN_PROBE_STEP(c0)
        NN_PROBE_STEP(c1)
        NN_PROBE_STEP(c2)
        NN_PROBE_STEP(c3)
#undef NN_PROBE_STEP
    }
    float s = 0.f;
    for (int j = 0; j < 16; ++j) s += c0[j] + c1[j] + c2[j] + c3[j];
    for (int j = 0; j < 8; ++j) s += x[j];
    out[blockIdx.x * 256 + threadIdx.x] = s;
}

template <int MODE>
__global__ __launch_bounds__(256) void clock_kernel(unsigned long long* stamps, float* sink, int n) {
    bf16x8 a, b;
    for (int j = 0; j < 8; ++j) {
        a[j] = (__bf16)(threadIdx.x * 1e-3f);
        b[j] = (__bf16)(j * 1e-3f);
    }
    f32x16 c0 = {}, c1 = {}, c2 = {}, c3 = {};
    float x[8];
    for (int j = 0; j < 8; ++j) x[j] = threadIdx.x * 1e-4f + j;
    const unsigned long long t0 = __builtin_amdgcn_s_memtime(), r0 = __builtin_amdgcn_s_memrealtime();
    for (int i = 0; i < n; ++i) {
        if constexpr (MODE == 0) {
            c0 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c0, 0, 0, 0);
            c1 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c1, 0, 0, 0);
            c2 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c2, 0, 0, 0);
            c3 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c3, 0, 0, 0);
        } else {
#pragma unroll
            for (int k = 0; k < 32; ++k) x[k % 8] = __builtin_fmaf(x[k % 8], 0.999f, 0.5f);
        }
    }
    const unsigned long long t1 = __builtin_amdgcn_s_memtime(), r1 = __builtin_amdgcn_s_memrealtime();
    float s = 0.f;
    for (int j = 0; j < 16; ++j) s += c0[j] + c1[j] + c2[j] + c3[j];
    for (int j = 0; j < 8; ++j) s += x[j];
    sink[blockIdx.x * 256 + threadIdx.x] = s;
    if ((threadIdx.x & 63) == 0) {
        unsigned long long* o = stamps + ((size_t)blockIdx.x * 4 + (threadIdx.x >> 6)) * 4;
        o[0] = t0;
        o[1] = t1;
        o[2] = r0;
        o[3] = r1;
    }
}

int fail(const char* msg) {
    g_probe_error = msg;
    return -1;
}

int status() {
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        g_probe_error = hipGetErrorString(e);
        return (int)e;
    }
    return 0;
}

}  // namespace

extern "C" {

// out: blocks * 256 floats. k in {0, 4, 8, 12, 16}.
int nn_probe_coissue(int k, int blocks, int n, float* out, void* stream) {
    if (blocks <= 0 || blocks > 65536 || n <= 0 || !out) return fail("invalid probe arguments");
    hipStream_t s = (hipStream_t)stream;
    switch (k) {
        case 0: coissue_kernel<0><<<blocks, 256, 0, s>>>(out, n); break;
        case 4: coissue_kernel<4><<<blocks, 256, 0, s>>>(out, n); break;
        case 8: coissue_kernel<8><<<blocks, 256, 0, s>>>(out, n); break;
        case 12: coissue_kernel<12><<<blocks, 256, 0, s>>>(out, n); break;
        case 16: coissue_kernel<16><<<blocks, 256, 0, s>>>(out, n); break;
        default: return fail("k must be 0, 4, 8, 12 or 16");
    }
    return status();
}

// stamps: blocks * 4 waves * 4 uint64 (shader clock start, end; 100 MHz clock start, end); sink: blocks * 256
// floats. mode 0: MFMAs only, mode 1: FMAs only.
int nn_probe_clock(int mode, int blocks, int n, unsigned long long* stamps, float* sink, void* stream) {
    if (blocks <= 0 || blocks > 65536 || n <= 0 || !stamps || !sink) return fail("invalid probe arguments");
    hipStream_t s = (hipStream_t)stream;
    if (mode == 0)
        clock_kernel<0><<<blocks, 256, 0, s>>>(stamps, sink, n);
    else if (mode == 1)
        clock_kernel<1><<<blocks, 256, 0, s>>>(stamps, sink, n);
    else
        return fail("mode must be 0 (MFMA) or 1 (FMA)");
    return status();
}

const char* nn_probe_last_error(void) { return g_probe_error.c_str(); }

}  // extern "C"
