// Hardware floors for the measurement section (bench.py --suite floors): the rates the kernels
// in libqlin are compared against, measured on the device rather than taken from a data sheet.
// Built into libqlin_floors.so, a library of its own: nothing in libqlin calls it.
//
//   * qlin_floor_mfma: issue rate of one MFMA shape.  Every wave runs `iters` rounds of
//     independent MFMAs (8 accumulators for 16 x 16 shapes, 4 for 32 x 32) on register operands,
//     so the result is the matrix core's throughput with no memory traffic.
//   * qlin_floor_read: a streaming read of `bytes` (16-byte loads, grid-stride, one XOR-reduced
//     word per thread written at the end): the time any kernel needs to bring that many bytes in.
//   * qlin_floor_copy: a streaming copy (read + write) of `bytes`.
//   * qlin_floor_empty: a launch whose workgroups do nothing: the fixed cost of a kernel.
#include <hip/hip_runtime.h>

#include <cstdint>

namespace {

typedef _Float16 f16;
typedef f16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef int i32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// KIND 0: v_mfma_f32_32x32x16_f16, 1: v_mfma_f32_16x16x32_f16, 2: v_mfma_i32_32x32x32_i8,
// 3: v_mfma_i32_16x16x64_i8.
template <int KIND>
__global__ __launch_bounds__(256) void mfma_rate_kernel(float* out, int iters) {
    const int t = threadIdx.x;
    f16x8 a, b;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        a[i] = (f16)(0.001f * (float)(t + i));
        b[i] = (f16)(0.002f * (float)(t - i));
    }
    const i32x4 ai = {t, t + 1, t + 2, t + 3}, bi = {3 * t, 5 * t, 7, 9};
    float s = 0.0f;
    if constexpr (KIND == 0) {
        f32x16 c[4] = {};
        for (int it = 0; it < iters; ++it)
#pragma unroll
            for (int j = 0; j < 4; ++j) c[j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c[j], 0, 0, 0);
#pragma unroll
        for (int j = 0; j < 4; ++j) s += c[j][0] + c[j][15];
    } else if constexpr (KIND == 1) {
        f32x4 c[8] = {};
        for (int it = 0; it < iters; ++it)
#pragma unroll
            for (int j = 0; j < 8; ++j) c[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c[j], 0, 0, 0);
#pragma unroll
        for (int j = 0; j < 8; ++j) s += c[j][0] + c[j][3];
    } else if constexpr (KIND == 2) {
        i32x16 c[4] = {};
        for (int it = 0; it < iters; ++it)
#pragma unroll
            for (int j = 0; j < 4; ++j) c[j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(ai, bi, c[j], 0, 0, 0);
#pragma unroll
        for (int j = 0; j < 4; ++j) s += (float)(c[j][0] + c[j][15]);
    } else {
        i32x4 c[8] = {};
        for (int it = 0; it < iters; ++it)
#pragma unroll
            for (int j = 0; j < 8; ++j) c[j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(ai, bi, c[j], 0, 0, 0);
#pragma unroll
        for (int j = 0; j < 8; ++j) s += (float)(c[j][0] + c[j][3]);
    }
    out[blockIdx.x * 256 + t] = s;
}

__global__ __launch_bounds__(256) void read_kernel(const u32x4* __restrict__ src, int64_t n16, uint32_t* out) {
    const int64_t stride = (int64_t)gridDim.x * 256;
    uint32_t acc = 0;
    int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    for (; i + 3 * stride < n16; i += 4 * stride) {
        const u32x4 v0 = src[i], v1 = src[i + stride], v2 = src[i + 2 * stride], v3 = src[i + 3 * stride];
        acc ^= v0.x ^ v1.y ^ v2.z ^ v3.w;
    }
    for (; i < n16; i += stride) acc ^= src[i].x;
    out[blockIdx.x * 256 + threadIdx.x] = acc;
}

__global__ __launch_bounds__(256) void copy_kernel(const u32x4* __restrict__ src, u32x4* __restrict__ dst, int64_t n16) {
    const int64_t stride = (int64_t)gridDim.x * 256;
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n16; i += stride) dst[i] = src[i];
}

__global__ __launch_bounds__(256) void empty_kernel(uint32_t* out, int flag) {
    if (flag == 12345) out[threadIdx.x] = 0;  // never true: the workgroups do nothing
}

}  // namespace

extern "C" {

// Launch `blocks` workgroups of 256 threads running `iters` rounds of MFMA shape `kind` (0..3).
// `out` holds blocks * 256 floats.
int qlin_floor_mfma(int kind, int blocks, int iters, float* out, hipStream_t st) {
    if (blocks < 1 || iters < 1 || !out) return (int)hipErrorInvalidValue;
    switch (kind) {
        case 0: hipLaunchKernelGGL(mfma_rate_kernel<0>, dim3(blocks), dim3(256), 0, st, out, iters); break;
        case 1: hipLaunchKernelGGL(mfma_rate_kernel<1>, dim3(blocks), dim3(256), 0, st, out, iters); break;
        case 2: hipLaunchKernelGGL(mfma_rate_kernel<2>, dim3(blocks), dim3(256), 0, st, out, iters); break;
        case 3: hipLaunchKernelGGL(mfma_rate_kernel<3>, dim3(blocks), dim3(256), 0, st, out, iters); break;
        default: return (int)hipErrorInvalidValue;
    }
    return (int)hipGetLastError();
}

// Read `bytes` (a multiple of 16, 16-byte aligned) with `blocks` workgroups; `out` holds
// blocks * 256 words.
int qlin_floor_read(const void* src, int64_t bytes, int blocks, uint32_t* out, hipStream_t st) {
    if (!src || !out || bytes < 16 || bytes % 16 || (uintptr_t)src % 16 || blocks < 1) return (int)hipErrorInvalidValue;
    hipLaunchKernelGGL(read_kernel, dim3(blocks), dim3(256), 0, st, (const u32x4*)src, bytes / 16, out);
    return (int)hipGetLastError();
}

// Copy `bytes` (a multiple of 16, both pointers 16-byte aligned) with `blocks` workgroups.
int qlin_floor_copy(const void* src, void* dst, int64_t bytes, int blocks, hipStream_t st) {
    if (!src || !dst || bytes < 16 || bytes % 16 || (uintptr_t)src % 16 || (uintptr_t)dst % 16 || blocks < 1)
        return (int)hipErrorInvalidValue;
    hipLaunchKernelGGL(copy_kernel, dim3(blocks), dim3(256), 0, st, (const u32x4*)src, (u32x4*)dst, bytes / 16);
    return (int)hipGetLastError();
}

// `blocks` workgroups of 256 threads that return at once.
int qlin_floor_empty(int blocks, uint32_t* out, hipStream_t st) {
    if (blocks < 1 || !out) return (int)hipErrorInvalidValue;
    hipLaunchKernelGGL(empty_kernel, dim3(blocks), dim3(256), 0, st, out, 0);
    return (int)hipGetLastError();
}

}  // extern "C"
