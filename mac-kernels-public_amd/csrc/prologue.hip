// Activation prologue: per-row ConvRot rotation, then either
//   * weight-only mode: x' = rot(x) * 2^-E (E = frexp exponent of the row's max |rot(x)|),
//     rounded once to fp16, plus E -- the range-safe operand of the fp16 MFMA GEMMs; or
//   * A8 mode: quantize_int8_rowwise of rot(x) in x's dtype (roblennon/mac-kernels-public
//     modal/weight_error_app.py:109-115): scale = max(absmax/127, 1e-30) in fp32,
//     s = dtype(scale) (0 -> dtype tiny), q = clamp(rne(dtype(x / s)), -128, 127); or
//   * rotate-only mode (fp32 rows in, fp32 rows out), used to bring decoded weights back to the
//     original basis.
// One workgroup per row, of NT threads (a multiple of 64, chosen with SLOTS so that NT x SLOTS x 16
// just covers the row); each thread holds 16 consecutive elements per (16 NT)-element slot, so a
// rotation group (<= 256 elements) lives in one 16-lane DPP row.
#include "prologue_dev.h"

namespace qlin {

template <typename TIn, int MODE, int G, int SLOTS>
__global__ __launch_bounds__(prologue_max_threads(SLOTS), SLOTS <= 2 ? 6 : 1) void prologue_kernel(const TIn* __restrict__ x, int64_t ldx, int K,
                                                       bool vec_ok, f16* __restrict__ xo, int64_t ldo,
                                                       int32_t* __restrict__ eo, int8_t* __restrict__ qo,
                                                       float* __restrict__ so, TIn* __restrict__ xr,
                                                       float* __restrict__ fo) {
    prologue_row<TIn, MODE, G, SLOTS>(blockIdx.x, (int)blockDim.x, x, ldx, K, vec_ok, xo, ldo, eo, qo, so, xr, fo);
}

// Rows longer than one workgroup's registers hold (K > 32768): the row is processed in chunks of
// WIDE_CAP values, twice -- the first pass rotates each chunk only for the row's max |value|, the
// second rotates it again (same arithmetic, same values) and writes the outputs.  Rotate-only
// rows need no max and take one pass.
constexpr int WIDE_NT = 512, WIDE_SLOTS = 4, WIDE_CAP = WIDE_NT * WIDE_SLOTS * 16;

template <typename TIn, int MODE, int G>
__global__ __launch_bounds__(WIDE_NT) void prologue_wide_kernel(const TIn* __restrict__ x, int64_t ldx, int K,
                                                             bool vec_ok, f16* __restrict__ xo, int64_t ldo,
                                                             int32_t* __restrict__ eo, int8_t* __restrict__ qo,
                                                             float* __restrict__ so, TIn* __restrict__ xr,
                                                             float* __restrict__ fo) {
    __shared__ float red[16];
    const int m = blockIdx.x;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const TIn* row = x + (int64_t)m * ldx;
    float amax = 0.0f;
    if constexpr (MODE != 2) {
        for (int64_t c0 = 0; c0 < K; c0 += WIDE_CAP) {
#pragma unroll
            for (int s = 0; s < WIDE_SLOTS; ++s) {
                float v[16];
                rotate_unit<TIn, MODE, G>(row, c0 + ((int64_t)s * WIDE_NT + tid) * 16, K, vec_ok, lane, v);
#pragma unroll
                for (int i = 0; i < 16; ++i) amax = fmaxf(amax, fabsf(v[i]));
            }
        }
        amax = block_max(amax, red, WIDE_NT, lane, wave);
    }
    int E = 0;
    float scale = 0.0f, st = 1.0f;
    if constexpr (MODE == 0) E = frexp_exp(amax);
    if constexpr (MODE == 1) a8_scale<TIn>(amax, scale, st);
    const bool fast = MODE == 1 && sizeof(TIn) == 2 && st >= 0x1p-126f && st <= 0x1.fffffep127f;
    const float y = 1.0f / st;
    for (int64_t c0 = 0; c0 < K; c0 += WIDE_CAP) {
#pragma unroll
        for (int s = 0; s < WIDE_SLOTS; ++s) {
            const int64_t e0 = c0 + ((int64_t)s * WIDE_NT + tid) * 16;
            float v[16];
            rotate_unit<TIn, MODE, G>(row, e0, K, vec_ok, lane, v);
            if (e0 >= K) continue;
            if constexpr (MODE == 0) {
                emit_wo(v, E, e0, K, vec_ok, xo + (int64_t)m * ldo + e0);
            } else if constexpr (MODE == 1) {
                int8_t* dst = qo + (int64_t)m * ldo + e0;
                TIn* xd = xr ? xr + (int64_t)m * ldo + e0 : nullptr;
                if (fast) emit_a8<TIn, true>(v, st, y, e0, K, vec_ok, dst, xd);
                else emit_a8<TIn, false>(v, st, y, e0, K, vec_ok, dst, xd);
            } else {
                emit_f32(v, e0, K, fo + (int64_t)m * ldo + e0);
            }
        }
    }
    if (tid == 0) {
        if constexpr (MODE == 0) eo[m] = E;
        if constexpr (MODE == 1) so[m] = scale;
    }
}

template <typename TIn, int MODE>
static hipError_t launch_prologue(const PrologueArgs& a, hipStream_t st) {
    int nt = 0, slots = 0;
    prologue_shape(a.K, nt, slots);
    const bool vec_ok = (a.K % 16 == 0) && (a.ldx % 16 == 0) && (a.ldo % 16 == 0) &&
                        ((uintptr_t)a.x % 64 == 0);
    bool ok = false;
    const bool wide = a.K > PROLOGUE_ROW_MAX;
    if (wide) nt = WIDE_NT;
    auto go = [&]<int G>() {
        auto launch = [&](auto kern) {
            hipLaunchKernelGGL(kern, dim3((unsigned)a.M), dim3((unsigned)nt), 0, st, (const TIn*)a.x, a.ldx, a.K,
                               vec_ok, a.xo, a.ldo, a.eo, a.qo, a.so, (TIn*)a.xr, a.fo);
            ok = true;
        };
        if (wide) launch(prologue_wide_kernel<TIn, MODE, G>);
        else if (slots <= 1) launch(prologue_kernel<TIn, MODE, G, 1>);
        else if (slots <= 2) launch(prologue_kernel<TIn, MODE, G, 2>);
        else if (slots <= 4) launch(prologue_kernel<TIn, MODE, G, 4>);
        else if (slots <= 8) launch(prologue_kernel<TIn, MODE, G, 8>);
    };
    if (!dispatch_group(a.G, go) || !ok) return hipErrorInvalidValue;
    return hipGetLastError();
}

hipError_t run_prologue(const PrologueArgs& a, hipStream_t st) {
    if (a.M == 0) return hipSuccess;
    if (a.K > (a.mode == PROLOGUE_A8 ? QLIN_MAX_K : QLIN_MAX_K_WO)) return hipErrorInvalidValue;
    switch (a.mode) {
        case PROLOGUE_WO:
            if (a.x_dtype == DT_F16) return launch_prologue<f16, 0>(a, st);
            if (a.x_dtype == DT_BF16) return launch_prologue<bf16_t, 0>(a, st);
            if (a.x_dtype == DT_F32) return launch_prologue<float, 0>(a, st);
            break;
        case PROLOGUE_A8:
            if (a.x_dtype == DT_F16) return launch_prologue<f16, 1>(a, st);
            if (a.x_dtype == DT_BF16) return launch_prologue<bf16_t, 1>(a, st);
            if (a.x_dtype == DT_F32) return launch_prologue<float, 1>(a, st);
            break;
        case PROLOGUE_ROT_F32:
            if (a.x_dtype == DT_F32) return launch_prologue<float, 2>(a, st);
            break;
    }
    return hipErrorInvalidValue;
}

}  // namespace qlin
