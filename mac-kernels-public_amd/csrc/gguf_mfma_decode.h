// GGUF decode policies for the MFMA kernels (gguf_smallm.hip, gguf_split.hip): each lane turns
// its slice of a packed block, staged in LDS, into the fp16 B operand of an fp16 MFMA, in one of
// two forms:
//   * get(): exact small integers, with the block's scales returned in fp32 for the caller to
//     apply to the MFMA results (no rounding of the weight at all);
//   * getf(): the whole weight w times a power of two f, rounded to fp16 (the range-safe fp16
//     operand of the large-M path, with f per weight row and K range instead of per row).  The
//     caller picks f from bound(), an upper bound on |w| over a block, so that every |w * f| stays
//     below 2^15.  Where the block scales are fp16 values (d, m) the product is formed in packed
//     fp16 with one rounding.  Where a scale has more significant bits (d * sc for Q6_K and
//     IQ4_XS) it is rounded to fp16 first, two roundings of the same product.  The K-quants with
//     minima (Q2_K, Q4_K, Q5_K) subtract dmin * m, which can be much larger than w: their operand
//     is formed in fp32 (v_fma_mix) and rounded once.
#pragma once
#include "qlin_internal.h"
#include "gguf_exact.h"

namespace qlin {
namespace gguf_mfma {

template <int VPL> struct FragT;
template <> struct FragT<8> { typedef f16x8 type; typedef u32x4 bits; };
template <> struct FragT<4> { typedef f16x4 type; typedef u32x2 bits; };

template <int VPL>
__device__ __forceinline__ f32x4 mfma16(typename FragT<VPL>::type a, typename FragT<VPL>::type b, f32x4 c) {
    if constexpr (VPL == 8) return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
    else return __builtin_amdgcn_mfma_f32_16x16x16f16(a, b, c, 0, 0, 0);
}

// --------------------------------------------------------------------------------------------
// Byte -> fp16 helpers.  `t` holds four bytes b0..b3 (each < 1024 - 1024 offset fits 10 bits);
// perm64 pairs them with 0x64 high bytes: fp16 (1024 + b0, 1024 + b1) and (1024 + b2, 1024 + b3).
// --------------------------------------------------------------------------------------------
__device__ __forceinline__ uint32_t perm64_lo(uint32_t t) { return __builtin_amdgcn_perm(0x64646464u, t, 0x04010400u); }
__device__ __forceinline__ uint32_t perm64_hi(uint32_t t) { return __builtin_amdgcn_perm(0x64646464u, t, 0x04030402u); }

__device__ __forceinline__ f16x2 as_h2(uint32_t u) { return __builtin_bit_cast(f16x2, u); }
__device__ __forceinline__ uint32_t as_u(f16x2 h) { return __builtin_bit_cast(uint32_t, h); }

// 8 bytes (< 256 each, as two dwords) -> 8 fp16 (1024 + byte) + off, exactly.
__device__ __forceinline__ f16x8 bytes_to_f16x8(uint32_t t0, uint32_t t1, f16 off) {
    const f16x2 o = {off, off};
    u32x4 r;
    r.x = as_u(as_h2(perm64_lo(t0)) + o);
    r.y = as_u(as_h2(perm64_hi(t0)) + o);
    r.z = as_u(as_h2(perm64_lo(t1)) + o);
    r.w = as_u(as_h2(perm64_hi(t1)) + o);
    return __builtin_bit_cast(f16x8, r);
}
// Same, scaled: ((1024 + byte) * s - 1024 * s) = byte * s with one fp16 rounding of an exact
// integer result (callers keep |byte * s| <= 2048).
__device__ __forceinline__ f16x8 bytes_to_f16x8_scaled(uint32_t t0, uint32_t t1, f16 s, f16 off) {
    const f16x2 sv = {s, s}, o = {off, off};
    u32x4 r;
    r.x = as_u(__builtin_elementwise_fma(as_h2(perm64_lo(t0)), sv, o));
    r.y = as_u(__builtin_elementwise_fma(as_h2(perm64_hi(t0)), sv, o));
    r.z = as_u(__builtin_elementwise_fma(as_h2(perm64_lo(t1)), sv, o));
    r.w = as_u(__builtin_elementwise_fma(as_h2(perm64_hi(t1)), sv, o));
    return __builtin_bit_cast(f16x8, r);
}
__device__ __forceinline__ f16x4 bytes_to_f16x4(uint32_t t, f16 off) {
    const f16x2 o = {off, off};
    u32x2 r;
    r.x = as_u(as_h2(perm64_lo(t)) + o);
    r.y = as_u(as_h2(perm64_hi(t)) + o);
    return __builtin_bit_cast(f16x4, r);
}
__device__ __forceinline__ f16x4 bytes_to_f16x4_scaled(uint32_t t, f16 s, f16 off) {
    const f16x2 sv = {s, s}, o = {off, off};
    u32x2 r;
    r.x = as_u(__builtin_elementwise_fma(as_h2(perm64_lo(t)), sv, o));
    r.y = as_u(__builtin_elementwise_fma(as_h2(perm64_hi(t)), sv, o));
    return __builtin_bit_cast(f16x4, r);
}

// Folded operands.  fold8/fold4: exact integers q times rne16(a * f) (+ rne16(b * f)), one
// rounding of the product when a and b are fp16 values (a * f, b * f are then exact).  fold8x/fold4x:
// raw values r = 1024 + byte (as perm64 leaves them, no offset removed) -> r * A + B in fp32
// (v_fma_mix reads the fp16 halves directly), then rounded to fp16; B carries the offset
// (-1024 A - ...), whose own fp32 rounding is below 2^-14 |A|.
__device__ __forceinline__ f16x8 fold8(f16x8 q, float a, float f) {
    const f16 A = (f16)(a * f);
    return q * (f16x8){A, A, A, A, A, A, A, A};
}
__device__ __forceinline__ f16x8 fold8(f16x8 q, float a, float b, float f) {
    const f16 A = (f16)(a * f), B = (f16)(b * f);
    return __builtin_elementwise_fma(q, (f16x8){A, A, A, A, A, A, A, A}, (f16x8){B, B, B, B, B, B, B, B});
}
__device__ __forceinline__ f16x4 fold4(f16x4 q, float a, float f) {
    const f16 A = (f16)(a * f);
    return q * (f16x4){A, A, A, A};
}
__device__ __forceinline__ f16x4 fold4(f16x4 q, float a, float b, float f) {
    const f16 A = (f16)(a * f), B = (f16)(b * f);
    return __builtin_elementwise_fma(q, (f16x4){A, A, A, A}, (f16x4){B, B, B, B});
}
__device__ __forceinline__ f16x8 raw8(uint32_t t0, uint32_t t1) {
    return __builtin_bit_cast(f16x8, (u32x4){perm64_lo(t0), perm64_hi(t0), perm64_lo(t1), perm64_hi(t1)});
}
__device__ __forceinline__ f16x4 raw4(uint32_t t) {
    return __builtin_bit_cast(f16x4, (u32x2){perm64_lo(t), perm64_hi(t)});
}
__device__ __forceinline__ f16x8 fold8x(f16x8 r, float A, float B) {
    f16x8 o;
#pragma unroll
    for (int i = 0; i < 8; ++i) o[i] = (f16)__builtin_fmaf((float)r[i], A, B);
    return o;
}
__device__ __forceinline__ f16x4 fold4x(f16x4 r, float A, float B) {
    f16x4 o;
#pragma unroll
    for (int i = 0; i < 4; ++i) o[i] = (f16)__builtin_fmaf((float)r[i], A, B);
    return o;
}

// Spread bits 0..3 of x to bit 0 of bytes 0..3.
__device__ __forceinline__ uint32_t spread4(uint32_t x) { return ((x & 0xFu) * 0x00204081u) & 0x01010101u; }

// IQ4_NL levels + 128 as bytes: lut(i) for 4 nibble bytes at once (two 8-entry v_perm lookups and
// a byte select on bit 3).
__device__ __forceinline__ uint32_t iq4_lut4(uint32_t idx) {
    const uint32_t L0 = 0x3F2D1801u;  // -127..-65 + 128:  1, 24, 45, 63
    const uint32_t L1 = 0x766A5D4Fu;  // -49..-10 + 128:  79, 93, 106, 118
    const uint32_t L2 = 0xA6998D81u;  // 1..38 + 128:   129, 141, 153, 166
    const uint32_t L3 = 0xF1D9C5B5u;  // 53..113 + 128: 181, 197, 217, 241
    const uint32_t sel = idx & 0x07070707u;
    const uint32_t lo = __builtin_amdgcn_perm(L1, L0, sel);
    const uint32_t hi = __builtin_amdgcn_perm(L3, L2, sel);
    const uint32_t m8 = idx & 0x08080808u;
    const uint32_t mask = (m8 << 5) - (m8 >> 3);
    return (hi & mask) | (lo & ~mask);
}

// --------------------------------------------------------------------------------------------
// Format policies.  KIND 0: one fp32 scale (and offset) per unit; KIND 1: sub-scales folded,
// fp32 d (dmin) per block.  get() decodes this lane's VPL values of the unit starting at value v0
// of the block at byte offset o of the LDS stage row s.
// --------------------------------------------------------------------------------------------
template <int T> struct SM;

__device__ __forceinline__ float lds_f16(const uint8_t* s, int off) { return f16_bits_to_f32(ld_u16(s, off)); }

template <> struct SM<gguf::Q8_0> {
    static constexpr int QK = 32, TS = 34, UNIT = 32, SBLK = 8, KIND = 0;
    static constexpr bool MIN = false;
    __device__ static f16x8 get(const uint8_t* s, int o, int v0, float& a, float& b) {
        a = lds_f16(s, o);
        b = 0.0f;
        const uint32_t w0 = ld_u32(s, o + 2 + v0) ^ 0x80808080u, w1 = ld_u32(s, o + 6 + v0) ^ 0x80808080u;
        return bytes_to_f16x8(w0, w1, (f16)-1152.0f);
    }
    __device__ static float bound(const uint8_t* s, int o) { return fabsf(lds_f16(s, o)) * 128.0f; }
    __device__ static f16x8 getf(const uint8_t* s, int o, int v0, float f) {
        float a, b;
        const f16x8 q = get(s, o, v0, a, b);
        return fold8(q, a, f);
    }
};

// INT8 weight rows (INT8_ROWS): 256-value "blocks" of raw int8 codes with no stored scale; the
// codes become exact fp16 (q + 1152 - 1152) and the per-row scale joins the epilogue.
template <> struct SM<INT8_ROWS> {
    static constexpr int QK = 256, TS = 256, UNIT = 32, SBLK = 1, KIND = 1;
    static constexpr bool MIN = false;
    __device__ static void block(const uint8_t*, int, float& d, float& dmin) {
        d = 1.0f;
        dmin = 0.0f;
    }
    __device__ static f16x8 get(const uint8_t* s, int o, int v0, f16& mv) {
        mv = (f16)0.0f;
        const uint32_t w0 = ld_u32(s, o + v0) ^ 0x80808080u, w1 = ld_u32(s, o + v0 + 4) ^ 0x80808080u;
        return bytes_to_f16x8(w0, w1, (f16)-1152.0f);
    }
};

template <int T> struct SMNib32 {
    static constexpr int QK = 32, TS = (T == gguf::Q4_1) ? 20 : 18, UNIT = 32, SBLK = 8, KIND = 0;
    static constexpr bool MIN = (T == gguf::Q4_1);
    __device__ static f16x8 get(const uint8_t* s, int o, int v0, float& a, float& b) {
        constexpr int qo = (T == gguf::Q4_1) ? 4 : 2;
        a = lds_f16(s, o);
        b = MIN ? lds_f16(s, o + 2) : 0.0f;
        const int sh = (v0 >> 4) * 4;
        uint32_t t0 = (ld_u32(s, o + qo + (v0 & 15)) >> sh) & 0x0F0F0F0Fu;
        uint32_t t1 = (ld_u32(s, o + qo + (v0 & 15) + 4) >> sh) & 0x0F0F0F0Fu;
        if constexpr (T == gguf::IQ4_NL) {
            t0 = iq4_lut4(t0);
            t1 = iq4_lut4(t1);
            return bytes_to_f16x8(t0, t1, (f16)-1152.0f);
        }
        return bytes_to_f16x8(t0, t1, (f16)((T == gguf::Q4_0) ? -1032.0f : -1024.0f));
    }
    // |w| <= |d| * max|q| (+ |m|): Q4_0 q - 8 in -8..7, Q4_1 q in 0..15, IQ4_NL levels in -127..113
    __device__ static float bound(const uint8_t* s, int o) {
        if constexpr (T == gguf::Q4_1) return fabsf(lds_f16(s, o)) * 15.0f + fabsf(lds_f16(s, o + 2));
        return fabsf(lds_f16(s, o)) * (T == gguf::IQ4_NL ? 127.0f : 8.0f);
    }
    __device__ static f16x8 getf(const uint8_t* s, int o, int v0, float f) {
        float a, b;
        const f16x8 q = get(s, o, v0, a, b);
        if constexpr (MIN) return fold8(q, a, b, f);
        else return fold8(q, a, f);
    }
};
template <> struct SM<gguf::Q4_0> : SMNib32<gguf::Q4_0> {};
template <> struct SM<gguf::Q4_1> : SMNib32<gguf::Q4_1> {};
template <> struct SM<gguf::IQ4_NL> : SMNib32<gguf::IQ4_NL> {};

template <int T> struct SMQ5 {
    static constexpr int QK = 32, TS = (T == gguf::Q5_0) ? 22 : 24, UNIT = 32, SBLK = 8, KIND = 0;
    static constexpr bool MIN = (T == gguf::Q5_1);
    __device__ static f16x8 get(const uint8_t* s, int o, int v0, float& a, float& b) {
        constexpr int ho = (T == gguf::Q5_0) ? 2 : 4;
        a = lds_f16(s, o);
        b = MIN ? lds_f16(s, o + 2) : 0.0f;
        const uint32_t qh = ld_u32(s, o + ho) >> v0;  // bits of values v0..v0+7
        const int sh = (v0 >> 4) * 4;
        const uint32_t t0 = ((ld_u32(s, o + ho + 4 + (v0 & 15)) >> sh) & 0x0F0F0F0Fu) | (spread4(qh) << 4);
        const uint32_t t1 = ((ld_u32(s, o + ho + 8 + (v0 & 15)) >> sh) & 0x0F0F0F0Fu) | (spread4(qh >> 4) << 4);
        return bytes_to_f16x8(t0, t1, (f16)((T == gguf::Q5_0) ? -1040.0f : -1024.0f));
    }
    // Q5_0 q - 16 in -16..15, Q5_1 q in 0..31 plus m
    __device__ static float bound(const uint8_t* s, int o) {
        if constexpr (MIN) return fabsf(lds_f16(s, o)) * 31.0f + fabsf(lds_f16(s, o + 2));
        return fabsf(lds_f16(s, o)) * 16.0f;
    }
    __device__ static f16x8 getf(const uint8_t* s, int o, int v0, float f) {
        float a, b;
        const f16x8 q = get(s, o, v0, a, b);
        if constexpr (MIN) return fold8(q, a, b, f);
        else return fold8(q, a, f);
    }
};
template <> struct SM<gguf::Q5_0> : SMQ5<gguf::Q5_0> {};
template <> struct SM<gguf::Q5_1> : SMQ5<gguf::Q5_1> {};

template <> struct SM<gguf::IQ4_XS> {
    static constexpr int QK = 256, TS = 136, UNIT = 32, SBLK = 1, KIND = 0;
    static constexpr bool MIN = false;
    // d * (ls - 32) of the sub-block of v0, and its levels + 128 as bytes
    __device__ static float scale(const uint8_t* s, int o, int v0) {
        const int sb = v0 >> 5;
        const uint32_t hdr = ld_u32(s, o), sl = ld_u32(s, o + 4);
        const int ls = ((sl >> (8 * (sb >> 1) + 4 * (sb & 1))) & 0xF) | (int)(((hdr >> (16 + 2 * sb)) & 3u) << 4);
        return f16_bits_to_f32((uint16_t)(hdr & 0xFFFFu)) * (float)(ls - 32);
    }
    __device__ static void codes(const uint8_t* s, int o, int v0, uint32_t& t0, uint32_t& t1) {
        const int sb = v0 >> 5, i = v0 & 31, sh = (i >> 4) * 4;
        t0 = iq4_lut4((ld_u32(s, o + 8 + 16 * sb + (i & 15)) >> sh) & 0x0F0F0F0Fu);
        t1 = iq4_lut4((ld_u32(s, o + 12 + 16 * sb + (i & 15)) >> sh) & 0x0F0F0F0Fu);
    }
    __device__ static f16x8 get(const uint8_t* s, int o, int v0, float& a, float& b) {
        a = scale(s, o, v0);
        b = 0.0f;
        uint32_t t0, t1;
        codes(s, o, v0, t0, t1);
        return bytes_to_f16x8(t0, t1, (f16)-1152.0f);
    }
    // sub-block scale ls - 32 in -32..31, levels in -127..113
    __device__ static float bound(const uint8_t* s, int o) { return fabsf(lds_f16(s, o)) * (32.0f * 127.0f); }
    __device__ static f16x8 getf(const uint8_t* s, int o, int v0, float f) {
        uint32_t t0, t1;
        codes(s, o, v0, t0, t1);
        return fold8(bytes_to_f16x8(t0, t1, (f16)-1152.0f), scale(s, o, v0), f);
    }
};

template <> struct SM<gguf::Q6_K> {
    static constexpr int QK = 256, TS = 210, UNIT = 16, SBLK = 2, KIND = 0;
    static constexpr bool MIN = false;
    // d * sc of the 16 values from v0, and their codes q (0..63) as bytes
    __device__ static float scale(const uint8_t* s, int o, int v0) {
        return lds_f16(s, o + 208) * (float)(int)(int8_t)(ld_u32(s, o + 192 + (v0 >> 4)) & 0xFFu);
    }
    __device__ static uint32_t codes(const uint8_t* s, int o, int v0) {
        const int h = v0 >> 7, r = v0 & 127;
        const uint32_t lo = (ld_u32(s, o + 64 * h + (r & 63)) >> (4 * (r >> 6))) & 0x0F0F0F0Fu;
        const uint32_t hi = (ld_u32(s, o + 128 + 32 * h + (r & 31)) >> (2 * (r >> 5))) & 0x03030303u;
        return lo | (hi << 4);
    }
    __device__ static f16x4 get(const uint8_t* s, int o, int v0, float& a, float& b) {
        a = scale(s, o, v0);
        b = 0.0f;
        return bytes_to_f16x4(codes(s, o, v0), (f16)-1056.0f);
    }
    // int8 sub-scales, q - 32 in -32..31
    __device__ static float bound(const uint8_t* s, int o) { return fabsf(lds_f16(s, o + 208)) * (128.0f * 32.0f); }
    __device__ static f16x4 getf(const uint8_t* s, int o, int v0, float f) {
        return fold4(bytes_to_f16x4(codes(s, o, v0), (f16)-1056.0f), scale(s, o, v0), f);
    }
};

// K-quants with folded sub-scales.  get() returns the operand sc*q for this lane and the
// sub-block minimum (fp16, exact) for the second MFMA; block() returns the fp32 d, dmin.
template <int T> struct SMK45 {
    static constexpr int QK = 256, TS = (T == gguf::Q4_K) ? 144 : 176, UNIT = 32, SBLK = 1, KIND = 1;
    static constexpr bool MIN = true;
    __device__ static void block(const uint8_t* s, int o, float& d, float& dmin) {
        const uint32_t h = ld_u32(s, o);
        d = f16_bits_to_f32((uint16_t)(h & 0xFFFFu));
        dmin = f16_bits_to_f32((uint16_t)(h >> 16));
    }
    // 6-bit scale and minimum of sub-block sb
    __device__ static void subscales(const uint8_t* s, int o, int sb, int& sc, int& mn) {
        const uint32_t s0 = ld_u32(s, o + 4), s1 = ld_u32(s, o + 8), s2 = ld_u32(s, o + 12);
        if (sb < 4) {
            sc = (s0 >> (8 * sb)) & 63;
            mn = (s1 >> (8 * sb)) & 63;
        } else {
            const int j = sb - 4;
            sc = ((s2 >> (8 * j)) & 0xF) | (((s0 >> (8 * j + 6)) & 3) << 4);
            mn = ((s2 >> (8 * j + 4)) & 0xF) | (((s1 >> (8 * j + 6)) & 3) << 4);
        }
    }
    // codes q (0..15, or 0..31 with Q5_K's fifth bit) of values v0..v0+7 as bytes
    __device__ static void codes(const uint8_t* s, int o, int v0, uint32_t& t0, uint32_t& t1) {
        const int sb = v0 >> 5;
        constexpr int qs = (T == gguf::Q4_K) ? 16 : 48;
        const int i = v0 & 31, sh = (sb & 1) * 4;
        t0 = (ld_u32(s, o + qs + 32 * (sb >> 1) + i) >> sh) & 0x0F0F0F0Fu;
        t1 = (ld_u32(s, o + qs + 32 * (sb >> 1) + i + 4) >> sh) & 0x0F0F0F0Fu;
        if constexpr (T == gguf::Q5_K) {
            t0 |= ((ld_u32(s, o + 16 + i) >> sb) & 0x01010101u) << 4;
            t1 |= ((ld_u32(s, o + 20 + i) >> sb) & 0x01010101u) << 4;
        }
    }
    __device__ static f16x8 get(const uint8_t* s, int o, int v0, f16& mv) {
        int sc, mn;
        subscales(s, o, v0 >> 5, sc, mn);
        mv = (f16)(float)mn;
        uint32_t t0, t1;
        codes(s, o, v0, t0, t1);
        const f16 scv = (f16)(float)sc;
        return bytes_to_f16x8_scaled(t0, t1, scv, (f16)(-1024.0f * (float)sc));
    }
    // w = d * sc * q - dmin * mn with 6-bit sc, mn
    __device__ static float bound(const uint8_t* s, int o) {
        float d, dmin;
        block(s, o, d, dmin);
        return fabsf(d) * (63.0f * (T == gguf::Q4_K ? 15.0f : 31.0f)) + fabsf(dmin) * 63.0f;
    }
    __device__ static f16x8 getf(const uint8_t* s, int o, int v0, float f) {
        float d, dmin;
        block(s, o, d, dmin);
        int sc, mn;
        subscales(s, o, v0 >> 5, sc, mn);
        uint32_t t0, t1;
        codes(s, o, v0, t0, t1);
        const float A = d * (float)sc * f;
        return fold8x(raw8(t0, t1), A, -1024.0f * A - dmin * (float)mn * f);
    }
};
template <> struct SM<gguf::Q4_K> : SMK45<gguf::Q4_K> {};
template <> struct SM<gguf::Q5_K> : SMK45<gguf::Q5_K> {};

template <> struct SM<gguf::Q2_K> {
    static constexpr int QK = 256, TS = 84, UNIT = 16, SBLK = 1, KIND = 1;
    static constexpr bool MIN = true;
    __device__ static void block(const uint8_t* s, int o, float& d, float& dmin) {
        const uint32_t h = ld_u32(s, o + 80);
        d = f16_bits_to_f32((uint16_t)(h & 0xFFFFu));
        dmin = f16_bits_to_f32((uint16_t)(h >> 16));
    }
    __device__ static f16x4 get(const uint8_t* s, int o, int v0, f16& mv) {
        const uint32_t scb = ld_u32(s, o + (v0 >> 4)) & 0xFFu;
        mv = (f16)(float)(scb >> 4);
        const int sc = scb & 0xF;
        const int h = v0 >> 7, t2 = (v0 >> 5) & 3, i0 = v0 & 31;
        const uint32_t t = (ld_u32(s, o + 16 + 32 * h + i0) >> (2 * t2)) & 0x03030303u;
        return bytes_to_f16x4_scaled(t, (f16)(float)sc, (f16)(-1024.0f * (float)sc));
    }
    // w = d * sc * q - dmin * m with 4-bit sc, m and q in 0..3
    __device__ static float bound(const uint8_t* s, int o) {
        float d, dmin;
        block(s, o, d, dmin);
        return fabsf(d) * 45.0f + fabsf(dmin) * 15.0f;
    }
    __device__ static f16x4 getf(const uint8_t* s, int o, int v0, float f) {
        float d, dmin;
        block(s, o, d, dmin);
        const uint32_t scb = ld_u32(s, o + (v0 >> 4)) & 0xFFu;
        const int h = v0 >> 7, t2 = (v0 >> 5) & 3, i0 = v0 & 31;
        const uint32_t t = (ld_u32(s, o + 16 + 32 * h + i0) >> (2 * t2)) & 0x03030303u;
        const float A = d * (float)(int)(scb & 0xF) * f;
        return fold4x(raw4(t), A, -1024.0f * A - dmin * (float)(int)(scb >> 4) * f);
    }
};

template <> struct SM<gguf::Q3_K> {
    // value = (d * s6) * q with q = q2 - 4 * (1 - hbit) in -4..3.  The operand carries t = q + 4
    // (0..7) scaled by s6 exactly, and the second MFMA removes 4 * s6 (dmin = d).
    static constexpr int QK = 256, TS = 110, UNIT = 16, SBLK = 2, KIND = 1;
    static constexpr bool MIN = true;
    __device__ static void block(const uint8_t* s, int o, float& d, float& dmin) {
        d = lds_f16(s, o + 108);
        dmin = d;
    }
    __device__ static f16x4 get(const uint8_t* s, int o, int v0, f16& mv) {
        const int si = v0 >> 4;
        const int lo = (ld_u32(s, o + 96 + (si & 7)) >> (4 * (si >> 3))) & 0xF;
        const int hs = (ld_u32(s, o + 104 + (si & 3)) >> (2 * (si >> 2))) & 3;
        const int s6 = (lo | (hs << 4)) - 32;
        mv = (f16)(float)(4 * s6);
        const int h = v0 >> 7, t2 = (v0 >> 5) & 3, i0 = v0 & 31, hb = v0 >> 5;
        const uint32_t q2 = (ld_u32(s, o + 32 + 32 * h + i0) >> (2 * t2)) & 0x03030303u;
        const uint32_t hm = (ld_u32(s, o + i0) >> hb) & 0x01010101u;
        const uint32_t t = q2 | (hm << 2);  // q + 4
        return bytes_to_f16x4_scaled(t, (f16)(float)s6, (f16)(-1024.0f * (float)s6));
    }
    // w = d * s6 * q with s6 in -32..31, q in -4..3
    __device__ static float bound(const uint8_t* s, int o) { return fabsf(lds_f16(s, o + 108)) * 128.0f; }
    __device__ static f16x4 getf(const uint8_t* s, int o, int v0, float f) {
        f16 mv;
        const f16x4 st = get(s, o, v0, mv);  // s6 * (q + 4), exact
        // s6 * q = s6 * (q + 4) - 4 * s6 is exact in fp16 (|s6 * q| <= 128); then the scale d
        const f16x4 sq = st - (f16x4){mv, mv, mv, mv};
        return fold4(sq, lds_f16(s, o + 108), f);
    }
};

}  // namespace gguf_mfma
}  // namespace qlin
