// Device code of the activation prologue, shared by its own kernels (prologue.hip) and the A8
// pre-pass that runs it beside the weight-grid decode (gemm_i8.hip).
// The modes (weight-only, A8, rotate-only) and the row layout are described in prologue.hip.
#pragma once
#include "qlin_internal.h"
#include "hadamard.h"

namespace qlin {

template <typename TIn>
__device__ __forceinline__ void load16(const TIn* row, int64_t e0, int K, bool vec_ok, float* v) {
    if (vec_ok && e0 + 16 <= K) {
        if constexpr (sizeof(TIn) == 2) {
            const u32x4* p = reinterpret_cast<const u32x4*>(row + e0);
            u32x4 a = p[0], b = p[1];
            uint32_t w[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                TIn lo, hi;
                uint16_t l16 = (uint16_t)(w[i] & 0xFFFFu), h16 = (uint16_t)(w[i] >> 16);
                __builtin_memcpy(&lo, &l16, 2);
                __builtin_memcpy(&hi, &h16, 2);
                v[2 * i] = dtype_traits<TIn>::to_f32(lo);
                v[2 * i + 1] = dtype_traits<TIn>::to_f32(hi);
            }
        } else {
            const f32x4* p = reinterpret_cast<const f32x4*>(row + e0);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                f32x4 a = p[i];
                v[4 * i] = a.x; v[4 * i + 1] = a.y; v[4 * i + 2] = a.z; v[4 * i + 3] = a.w;
            }
        }
    } else {
#pragma unroll
        for (int i = 0; i < 16; ++i) v[i] = (e0 + i < K) ? dtype_traits<TIn>::to_f32(row[e0 + i]) : 0.0f;
    }
}

// Largest workgroup per slot count (keeps 16 x SLOTS row values in registers without spilling).
constexpr int prologue_max_threads(int slots) { return slots <= 2 ? 1024 : slots == 4 ? 512 : 256; }

// One 16-value unit of a row: load, rotate by the normalized Hadamard, and for A8 round to the
// input dtype (the value a rotated x.dtype tensor holds).
template <typename TIn, int MODE, int G>
__device__ __forceinline__ void rotate_unit(const TIn* row, int64_t e0, int K, bool vec_ok, int lane, float* v) {
    load16<TIn>(row, e0, K, vec_ok, v);
    if constexpr (G > 0) {
        hadamard16<G>(v, lane);
        const float nrm = hadamard_norm<G>();
#pragma unroll
        for (int i = 0; i < 16; ++i) v[i] *= nrm;
    }
    if constexpr (MODE == 1) {
#pragma unroll
        for (int i = 0; i < 16; ++i) v[i] = round_to<TIn>(v[i]);
    }
}

// Largest |value| over the workgroup (every thread gets it); red holds one float per wave.
__device__ __forceinline__ float block_max(float amax, float* red, int NT, int lane, int wave) {
    amax = wave_max(amax);
    if (lane == 0) red[wave] = amax;
    __syncthreads();
    amax = red[0];
    for (int w = 1; w < NT / 64; ++w) amax = fmaxf(amax, red[w]);
    return amax;
}

// Weight-only output of one unit: fp16(v * 2^-E), 16-byte stores where the row allows.
__device__ __forceinline__ void emit_wo(const float* v, int E, int64_t e0, int K, bool vec_ok, f16* dst) {
    f16 h[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) h[i] = (f16)__builtin_ldexpf(v[i], -E);
    if (e0 + 16 <= K && vec_ok) {
        uint32_t w[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            w[i] = (uint32_t)__builtin_bit_cast(uint16_t, h[2 * i]) |
                   ((uint32_t)__builtin_bit_cast(uint16_t, h[2 * i + 1]) << 16);
        }
        u32x4* d = reinterpret_cast<u32x4*>(dst);
        d[0] = u32x4{w[0], w[1], w[2], w[3]};
        d[1] = u32x4{w[4], w[5], w[6], w[7]};
    } else {
        for (int i = 0; i < 16; ++i)
            if (e0 + i < K) dst[i] = h[i];
    }
}

// A8 row scale from the row's max |value| (quantize_int8_rowwise): scale = max(amax / 127, 1e-30)
// in fp32, st = dtype(scale), 0 -> the dtype's smallest normal.
template <typename TIn>
__device__ __forceinline__ void a8_scale(float amax, float& scale, float& st) {
    scale = amax / 127.0f;
    if (!(scale >= 1e-30f)) scale = (scale != scale) ? scale : 1e-30f;
    st = round_to<TIn>(scale);
    if (st == 0.0f) st = dtype_traits<TIn>::tiny();
}

// A8 output of one unit: q = clamp(rne(dtype(x / st)), -128, 127).  x / st: for 16-bit inputs and a
// finite normal st, the reciprocal y = 1/st with one residual correction, q = fma(fma(-x y, st, x),
// y, x y) (Markstein).  Checked against the IEEE quotient for every pair of finite fp16 (bf16)
// values x, st with |x| <= 130 st (tests/quotient_check.c): identical fp32 quotients for fp16,
// identical int8 results for bf16.  Otherwise (fp32 inputs, subnormal or infinite st) the IEEE
// division.  xd (optional) receives the rotated values in x's dtype.
template <typename TIn, bool FAST>
__device__ __forceinline__ void emit_a8(const float* v, float st, float y, int64_t e0, int K, bool vec_ok,
                                        int8_t* dst, TIn* xd) {
    // q = clamp(t, -128, 127) with t = rne(dtype(x / st)) integer-valued: t + 128 (exact) goes to an
    // unsigned byte through v_cvt_pk_u8_f32, which saturates to [0, 255] (and gives 0 for a NaN,
    // the -128 the float clamp gives), packed four to a word; XOR 0x80 restores the signed byte.
    uint32_t w[4] = {0u, 0u, 0u, 0u};
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        float qt;
        {
#pragma clang fp contract(off)
            if constexpr (FAST) {
                const float q0 = v[i] * y;
                qt = __builtin_fmaf(__builtin_fmaf(-q0, st, v[i]), y, q0);
            } else {
                qt = v[i] / st;
            }
        }
        const float t = __builtin_rintf(round_to<TIn>(qt));
        w[i / 4] = __builtin_amdgcn_cvt_pk_u8_f32(t + 128.0f, (uint32_t)(i % 4), w[i / 4]);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) w[i] ^= 0x80808080u;
    if (e0 + 16 <= K && vec_ok) {
        *reinterpret_cast<u32x4*>(dst) = u32x4{w[0], w[1], w[2], w[3]};
    } else {
        for (int i = 0; i < 16; ++i)
            if (e0 + i < K) dst[i] = (int8_t)(w[i / 4] >> (8 * (i % 4)));
    }
    if (xd) {
        for (int i = 0; i < 16; ++i)
            if (e0 + i < K) xd[i] = dtype_traits<TIn>::from_f32(v[i]);
    }
}

__device__ __forceinline__ void emit_f32(const float* v, int64_t e0, int K, float* dst) {
    for (int i = 0; i < 16; ++i)
        if (e0 + i < K) dst[i] = v[i];
}

// One row m of the one-pass kernel, computed by a workgroup of NT threads; every thread of the
// workgroup calls it (the row max is a workgroup reduction).
template <typename TIn, int MODE, int G, int SLOTS>
__device__ __forceinline__ void prologue_row(int64_t m, int NT, const TIn* __restrict__ x, int64_t ldx, int K,
                                             bool vec_ok, f16* __restrict__ xo, int64_t ldo,
                                             int32_t* __restrict__ eo, int8_t* __restrict__ qo,
                                             float* __restrict__ so, TIn* __restrict__ xr,
                                             float* __restrict__ fo) {
    __shared__ float red[16];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const TIn* row = x + (int64_t)m * ldx;
    float v[SLOTS][16];
    float amax = 0.0f;
#pragma unroll
    for (int s = 0; s < SLOTS; ++s) {
        rotate_unit<TIn, MODE, G>(row, ((int64_t)s * NT + tid) * 16, K, vec_ok, lane, v[s]);
#pragma unroll
        for (int i = 0; i < 16; ++i) amax = fmaxf(amax, fabsf(v[s][i]));
    }
    if constexpr (MODE != 2) amax = block_max(amax, red, NT, lane, wave);

    if constexpr (MODE == 0) {
        const int E = frexp_exp(amax);
#pragma unroll
        for (int s = 0; s < SLOTS; ++s) {
            const int64_t e0 = ((int64_t)s * NT + tid) * 16;
            if (e0 >= K) break;
            emit_wo(v[s], E, e0, K, vec_ok, xo + (int64_t)m * ldo + e0);
        }
        if (tid == 0) eo[m] = E;
    } else if constexpr (MODE == 1) {
        float scale, st;
        a8_scale<TIn>(amax, scale, st);
        const bool fast = sizeof(TIn) == 2 && st >= 0x1p-126f && st <= 0x1.fffffep127f;
        const float y = 1.0f / st;
        // the row-uniform choice is made once, outside the element loops
        auto quantize_row = [&]<bool FAST>() {
#pragma unroll
            for (int s = 0; s < SLOTS; ++s) {
                const int64_t e0 = ((int64_t)s * NT + tid) * 16;
                if (e0 >= K) break;
                emit_a8<TIn, FAST>(v[s], st, y, e0, K, vec_ok, qo + (int64_t)m * ldo + e0,
                                   xr ? xr + (int64_t)m * ldo + e0 : nullptr);
            }
        };
        if (fast) quantize_row.template operator()<true>();
        else quantize_row.template operator()<false>();
        if (tid == 0) so[m] = scale;
    } else {
#pragma unroll
        for (int s = 0; s < SLOTS; ++s) {
            const int64_t e0 = ((int64_t)s * NT + tid) * 16;
            if (e0 >= K) break;
            emit_f32(v[s], e0, K, fo + (int64_t)m * ldo + e0);
        }
    }
}

// Threads per row and slots per thread: one or two slots whenever the workgroup allows (four and
// eight hold 200+ registers per thread, which leaves two waves per SIMD), then the fewest idle
// 16-element units (NT x SLOTS x 16 - K), then the thread count nearest 384.
inline void prologue_shape(int K, int& nt, int& slots) {
    const int units = (K + 15) / 16;
    bool have = false;
    int bk0 = 0, bk1 = 0, bk2 = 0;
    for (int sl : {1, 2, 4, 8}) {
        const int n = ((units + sl - 1) / sl + 63) / 64 * 64;
        if (n > prologue_max_threads(sl)) continue;
        const int k0 = sl > 2, k1 = n * sl - units, k2 = n > 384 ? n - 384 : 384 - n;
        if (!have || k0 < bk0 || (k0 == bk0 && (k1 < bk1 || (k1 == bk1 && k2 < bk2)))) {
            nt = n; slots = sl; bk0 = k0; bk1 = k1; bk2 = k2; have = true;
        }
    }
}

// Longest row one workgroup holds in registers (the one-pass kernel).
constexpr int PROLOGUE_ROW_MAX = 32768;

}  // namespace qlin
