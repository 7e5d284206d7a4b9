// Residual epilogue: y[m, n] = dtype(residual[m, n] + residual_scale[n] * base[m, n]), with base
// the linear's fp32 output (bias and LoRA already added) -- the bias first, then the scaled
// residual add, as the reference's fused epilogue orders them
// (roblennon/mac-kernels-public docs/upstream/comfy-kitchen-mps-backend.md:52;
// tests/test_lora_sidepath.py:378-386), in fp32 with one rounding.
// Eight outputs per thread, 16-byte loads and stores where rows allow them.
#include "qlin_internal.h"

namespace qlin {
namespace {

__global__ __launch_bounds__(256) void residual_kernel(ResidualArgs a) {
    const int64_t cpr = (a.N + 7) / 8;  // 8-output chunks per row
    const int64_t c = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (c >= a.M * cpr) return;
    const int64_t m = c / cpr, n = (c % cpr) * 8;
    const int cnt = (int)min<int64_t>(8, a.N - n);
    const bool bvec = cnt == 8 && a.ldb % 4 == 0 && (uintptr_t)a.base % 16 == 0;
    float b[8];
    if (bvec) {
        const f32x4* p = reinterpret_cast<const f32x4*>(a.base + m * a.ldb + n);
        const f32x4 u = p[0], v = p[1];
        b[0] = u.x; b[1] = u.y; b[2] = u.z; b[3] = u.w; b[4] = v.x; b[5] = v.y; b[6] = v.z; b[7] = v.w;
    } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) b[e] = e < cnt ? a.base[m * a.ldb + n + e] : 0.0f;
    }
    float o[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        const int64_t nn = min(n + e, a.N - 1);
        const float r = load_rt(a.res, a.res_dt, m * a.ldr + nn);
        const float s = a.rscale ? load_rt(a.rscale, a.rscale_dt, nn) : 1.0f;
        o[e] = __builtin_fmaf(s, b[e], r);
    }
    const bool yvec = a.ldy % 8 == 0 && (uintptr_t)a.y % 16 == 0;
    store8_rt(a.y, a.y_dt, m * a.ldy + n, o, cnt, yvec);
}

}  // namespace

hipError_t run_residual(const ResidualArgs& a, hipStream_t st) {
    if (a.M == 0 || a.N == 0) return hipSuccess;
    if (a.y_dt != DT_F32 && a.y_dt != DT_F16 && a.y_dt != DT_BF16) return hipErrorInvalidValue;
    const int64_t chunks = a.M * ((a.N + 7) / 8);
    hipLaunchKernelGGL(residual_kernel, dim3((unsigned)((chunks + 255) / 256)), dim3(256), 0, st, a);
    return hipGetLastError();
}

}  // namespace qlin
