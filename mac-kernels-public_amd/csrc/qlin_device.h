// Device-side helpers shared by the qlin kernels (gfx950 / CDNA4, wave64).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace qlin {

typedef _Float16 f16;
typedef f16 f16x2 __attribute__((ext_vector_type(2)));
typedef f16 f16x4 __attribute__((ext_vector_type(4)));
typedef f16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef int i32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

struct bf16_t { uint16_t bits; };

// ---------------------------------------------------------------------------------------------
// Scalar conversions.  All exact or correctly rounded (round to nearest even).
// ---------------------------------------------------------------------------------------------
__device__ __forceinline__ float f16_bits_to_f32(uint16_t h) {
    // v_cvt_f32_f16 is exact for every fp16 input (denormals are kept: HIP's default fp16 mode).
    return (float)__builtin_bit_cast(f16, h);
}
__device__ __forceinline__ float bf16_bits_to_f32(uint16_t b) { return __uint_as_float((uint32_t)b << 16); }

// f32 -> bf16 bits, round to nearest even; a NaN keeps its top payload bits and becomes quiet.
// gfx950's v_cvt_pk_bf16_f32 rounds to nearest even with denormals kept; it gives the integer
// rounding (u + 0x7FFF + ((u >> 16) & 1)) >> 16 for every non-NaN fp32 input (all 2^32 bit
// patterns compared on the device).  The NaN case is a select, so the conversion is branch-free.
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
    const uint32_t u = __float_as_uint(f);
    const uint32_t hw = __builtin_bit_cast(uint16_t, (__bf16)f);
    const uint32_t qnan = (u >> 16) | 0x40u;
    return (uint16_t)((u & 0x7FFFFFFFu) > 0x7F800000u ? qnan : hw);
}

// f32 -> IEEE fp16 bits, round to nearest even, overflow to inf, subnormals kept; computed with
// integer operations so the result does not depend on the hardware conversion's mode bits.
__device__ __forceinline__ uint16_t f32_to_f16_bits_rne(float f) {
    const uint32_t u = __float_as_uint(f);
    const uint32_t sign = (u >> 16) & 0x8000u;
    const uint32_t a = u & 0x7FFFFFFFu;
    if (a > 0x7F800000u) return (uint16_t)(sign | 0x7E00u | ((a >> 13) & 0x3FFu));
    if (a >= 0x477FF000u) return (uint16_t)(sign | 0x7C00u);
    if (a < 0x38800000u) {  // fp16 subnormal or zero: quantum 2^-24
        if (a < 0x33000000u) return (uint16_t)sign;
        const uint32_t e = a >> 23, m = (a & 0x7FFFFFu) | 0x800000u;
        const uint32_t sh = 126u - e;
        uint32_t q = m >> sh;
        const uint32_t rem = m & ((1u << sh) - 1u), half = 1u << (sh - 1u);
        if (rem > half || (rem == half && (q & 1u))) ++q;
        return (uint16_t)(sign | q);
    }
    uint32_t q = (((a >> 23) - 112u) << 10) | ((a & 0x7FFFFFu) >> 13);
    const uint32_t rem = a & 0x1FFFu;
    if (rem > 0x1000u || (rem == 0x1000u && (q & 1u))) ++q;
    return (uint16_t)(sign | q);
}

// float8_e4m3fn -> f32 (bias 7, no infinities, S.1111.111 = NaN).
__device__ __forceinline__ float e4m3_to_f32(uint8_t v) {
    uint32_t sign = (uint32_t)(v & 0x80u) << 24;
    uint32_t e = (v >> 3) & 0xFu, m = v & 7u;
    if (e == 15u && m == 7u) return __uint_as_float(sign | 0x7FC00000u);
    if (e == 0u) {
        float x = (float)m * 0.001953125f;
        return sign ? -x : x;
    }
    return __uint_as_float(sign | ((e + 120u) << 23) | (m << 20));
}

template <typename T> struct dtype_traits;
template <> struct dtype_traits<float> {
    static __device__ __forceinline__ float to_f32(float v) { return v; }
    static __device__ __forceinline__ float from_f32(float v) { return v; }
    static __device__ __forceinline__ float tiny() { return 1.17549435e-38f; }
};
template <> struct dtype_traits<f16> {
    static __device__ __forceinline__ float to_f32(f16 v) { return (float)v; }
    static __device__ __forceinline__ f16 from_f32(float v) { return (f16)v; }
    static __device__ __forceinline__ float tiny() { return 6.103515625e-05f; }
};
template <> struct dtype_traits<bf16_t> {
    static __device__ __forceinline__ float to_f32(bf16_t v) { return bf16_bits_to_f32(v.bits); }
    static __device__ __forceinline__ bf16_t from_f32(float v) { return bf16_t{f32_to_bf16_bits(v)}; }
    static __device__ __forceinline__ float tiny() { return 1.17549435e-38f; }
};

// Round a float to the storage type T and back (the value an x.dtype tensor would hold).
template <typename T>
__device__ __forceinline__ float round_to(float v) { return dtype_traits<T>::to_f32(dtype_traits<T>::from_f32(v)); }
// bf16: the hardware conversion and a shift (a NaN stays a NaN; only its payload is not kept).
template <>
__device__ __forceinline__ float round_to<bf16_t>(float v) { return (float)(__bf16)v; }

// ---------------------------------------------------------------------------------------------
// Cross-lane helpers.
// ---------------------------------------------------------------------------------------------
// xor-shuffle within groups of 32 lanes through ds_swizzle (bit mode), for masks < 32.
template <int MASK>
__device__ __forceinline__ float swz_xor(float v) {
    static_assert(MASK > 0 && MASK < 32, "ds_swizzle bit mode reaches 32 lanes");
    constexpr int pattern = 0x1F | (MASK << 10);
    return __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(v), pattern));
}

// DPP quad permutation (lane r of each quad reads lane SEL[r]).  Every lane is written and every
// source lane exists, so the old value (0) and bound_ctrl never show; with them in this form the
// compiler folds the permutation into the consuming add (v_add_f32 with a DPP source).
template <int A, int B, int C, int D>
__device__ __forceinline__ float dpp_quad(float v) {
    constexpr int ctrl = A | (B << 2) | (C << 4) | (D << 6);
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), ctrl, 0xF, 0xF, true));
}

template <int MASK>
__device__ __forceinline__ float lane_xor(float v) {
    if constexpr (MASK == 1) return dpp_quad<1, 0, 3, 2>(v);
    else if constexpr (MASK == 2) return dpp_quad<2, 3, 0, 1>(v);
    else if constexpr (MASK == 3) return dpp_quad<3, 2, 1, 0>(v);
    else if constexpr (MASK < 32) return swz_xor<MASK>(v);
    else return __shfl_xor(v, MASK, 64);
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int m = 1; m < 64; m <<= 1) v = fmaxf(v, __shfl_xor(v, m, 64));
    return v;
}
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int m = 1; m < 64; m <<= 1) v += __shfl_xor(v, m, 64);
    return v;
}

// Exponent E with |v| = mant * 2^E, mant in [0.5, 1) (frexp); 0 for zero / non-finite.
__device__ __forceinline__ int frexp_exp(float v) {
    if (!(v != 0.0f) || !__builtin_isfinite(v)) return 0;
    return __builtin_amdgcn_frexp_expf(v);
}

// Unaligned 32-bit read from a 4-byte aligned base: bytes [off, off+4).
__device__ __forceinline__ uint32_t ld_u32(const uint8_t* base, int off) {
    const uint32_t* p = reinterpret_cast<const uint32_t*>(base + (off & ~3));
    const int sh = off & 3;
    if (sh == 0) return p[0];
    return __builtin_amdgcn_alignbyte(p[1], p[0], sh);  // shift is in bytes
}
__device__ __forceinline__ uint16_t ld_u16(const uint8_t* base, int off) {
    return (uint16_t)(ld_u32(base, off) & 0xFFFFu);
}

// Output stores for the supported output dtypes.
__device__ __forceinline__ void store_out(float* p, float v) { *p = v; }
__device__ __forceinline__ void store_out(f16* p, float v) { *p = (f16)v; }
__device__ __forceinline__ void store_out(bf16_t* p, float v) { p->bits = f32_to_bf16_bits(v); }

// Runtime-typed output store / bias load (the dtype is uniform across the launch, so the branch
// costs one scalar compare).
__device__ __forceinline__ void store_rt(void* base, int dtype, int64_t idx, float v) {
    if (dtype == 0) reinterpret_cast<float*>(base)[idx] = v;
    else if (dtype == 1) reinterpret_cast<f16*>(base)[idx] = (f16)v;
    else reinterpret_cast<uint16_t*>(base)[idx] = f32_to_bf16_bits(v);
}
// Eight consecutive outputs v[0..7] at element idx of an output of runtime dtype.  `vec`: the
// caller has checked that base + idx is 16-byte aligned for this dtype; `count` < 8 stores a
// ragged row end element by element.
__device__ __forceinline__ void store8_rt(void* base, int dtype, int64_t idx, const float* v, int count, bool vec) {
    if (vec && count == 8) {
        if (dtype == 0) {
            float* p = reinterpret_cast<float*>(base) + idx;
            *reinterpret_cast<f32x4*>(p) = f32x4{v[0], v[1], v[2], v[3]};
            *reinterpret_cast<f32x4*>(p + 4) = f32x4{v[4], v[5], v[6], v[7]};
        } else if (dtype == 1) {
            f16x8 h;
#pragma unroll
            for (int e = 0; e < 8; ++e) h[e] = (f16)v[e];
            *reinterpret_cast<f16x8*>(reinterpret_cast<f16*>(base) + idx) = h;
        } else {
            u32x4 b;
#pragma unroll
            for (int e = 0; e < 4; ++e)
                b[e] = (uint32_t)f32_to_bf16_bits(v[2 * e]) | ((uint32_t)f32_to_bf16_bits(v[2 * e + 1]) << 16);
            *reinterpret_cast<u32x4*>(reinterpret_cast<uint16_t*>(base) + idx) = b;
        }
        return;
    }
    for (int e = 0; e < count; ++e) store_rt(base, dtype, idx + e, v[e]);
}
// The same for 4 consecutive outputs (8-byte stores for f16/bf16, 16-byte for f32; the caller has
// checked the alignment).
__device__ __forceinline__ void store4_rt(void* base, int dtype, int64_t idx, const float* v, int count, bool vec) {
    if (vec && count == 4) {
        if (dtype == 0) {
            *reinterpret_cast<f32x4*>(reinterpret_cast<float*>(base) + idx) = f32x4{v[0], v[1], v[2], v[3]};
        } else if (dtype == 1) {
            f16x4 h;
#pragma unroll
            for (int e = 0; e < 4; ++e) h[e] = (f16)v[e];
            *reinterpret_cast<f16x4*>(reinterpret_cast<f16*>(base) + idx) = h;
        } else {
            u32x2 b;
            b[0] = (uint32_t)f32_to_bf16_bits(v[0]) | ((uint32_t)f32_to_bf16_bits(v[1]) << 16);
            b[1] = (uint32_t)f32_to_bf16_bits(v[2]) | ((uint32_t)f32_to_bf16_bits(v[3]) << 16);
            *reinterpret_cast<u32x2*>(reinterpret_cast<uint16_t*>(base) + idx) = b;
        }
        return;
    }
    for (int e = 0; e < count; ++e) store_rt(base, dtype, idx + e, v[e]);
}
__device__ __forceinline__ float load_rt(const void* base, int dtype, int64_t idx) {
    if (dtype == 0) return reinterpret_cast<const float*>(base)[idx];
    if (dtype == 1) return (float)reinterpret_cast<const f16*>(base)[idx];
    return bf16_bits_to_f32(reinterpret_cast<const uint16_t*>(base)[idx]);
}

// Raw bits of element idx (for an early load whose conversion happens at the point of use:
// keeps the load from waiting on everything issued before it).
__device__ __forceinline__ uint32_t load_bits_rt(const void* base, int dtype, int64_t idx) {
    if (dtype == 0) return reinterpret_cast<const uint32_t*>(base)[idx];
    return reinterpret_cast<const uint16_t*>(base)[idx];
}
__device__ __forceinline__ float bits_to_f32_rt(uint32_t bits, int dtype) {
    if (dtype == 0) return __uint_as_float(bits);
    if (dtype == 1) return f16_bits_to_f32((uint16_t)bits);
    return bf16_bits_to_f32((uint16_t)bits);
}

// Wait until at most n vector-memory operations of this wave are outstanding (an LDS DMA counts as
// one); the other counters are left alone.
template <int n>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(n >= 0 && n < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((n & 15) | (7 << 4) | (15 << 8) | ((n >> 4) << 14));
}

// Wait until this wave's LDS reads and writes (and scalar loads) have completed; the vector-memory
// counter is left alone.
__device__ __forceinline__ void wait_lgkmcnt0() { __builtin_amdgcn_s_waitcnt((15) | (7 << 4) | (0 << 8) | (3 << 14)); }

// 16 bytes per lane from global memory straight into LDS at lds + 16 * lane (lds wave-uniform).
__device__ __forceinline__ void lds_dma16(const void* g, void* lds) {
    __builtin_amdgcn_global_load_lds(g, lds, 16, 0, 0);
}

// 4 bytes per lane into LDS at lds + 4 * lane: used to pull cache lines into L2 ahead of their
// 16-byte DMA (the LDS destination is a sink nobody reads).
__device__ __forceinline__ void lds_dma4(const void* g, void* lds) {
    __builtin_amdgcn_global_load_lds(g, lds, 4, 0, 0);
}

__device__ __forceinline__ float load_f(const float* p) { return *p; }
__device__ __forceinline__ float load_f(const f16* p) { return (float)*p; }
__device__ __forceinline__ float load_f(const bf16_t* p) { return bf16_bits_to_f32(p->bits); }

// Workgroup barrier that orders LDS only: waits for this wave's LDS operations, not for its global
// loads in flight (a plain __syncthreads also waits for every global load).  Data that reaches LDS
// through global loads (LDS DMA) needs its own vmcnt wait first.
__device__ __forceinline__ void lds_barrier() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

}  // namespace qlin
