// GGUF decode policies for the small-M MFMA kernel (gguf_smallm.hip): each lane turns
// its slice of a packed block, staged in LDS, into the fp16 B operand of v_mfma_f32_16x16x{32,16}_f16
// as exact small integers, with the block's scales returned in fp32.
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
};
template <> struct SM<gguf::Q5_0> : SMQ5<gguf::Q5_0> {};
template <> struct SM<gguf::Q5_1> : SMQ5<gguf::Q5_1> {};

template <> struct SM<gguf::IQ4_XS> {
    static constexpr int QK = 256, TS = 136, UNIT = 32, SBLK = 1, KIND = 0;
    static constexpr bool MIN = false;
    __device__ static f16x8 get(const uint8_t* s, int o, int v0, float& a, float& b) {
        const int sb = v0 >> 5;
        const uint32_t hdr = ld_u32(s, o), sl = ld_u32(s, o + 4);
        const int ls = ((sl >> (8 * (sb >> 1) + 4 * (sb & 1))) & 0xF) | (int)(((hdr >> (16 + 2 * sb)) & 3u) << 4);
        a = f16_bits_to_f32((uint16_t)(hdr & 0xFFFFu)) * (float)(ls - 32);
        b = 0.0f;
        const int i = v0 & 31, sh = (i >> 4) * 4;
        const uint32_t t0 = iq4_lut4((ld_u32(s, o + 8 + 16 * sb + (i & 15)) >> sh) & 0x0F0F0F0Fu);
        const uint32_t t1 = iq4_lut4((ld_u32(s, o + 12 + 16 * sb + (i & 15)) >> sh) & 0x0F0F0F0Fu);
        return bytes_to_f16x8(t0, t1, (f16)-1152.0f);
    }
};

template <> struct SM<gguf::Q6_K> {
    static constexpr int QK = 256, TS = 210, UNIT = 16, SBLK = 2, KIND = 0;
    static constexpr bool MIN = false;
    __device__ static f16x4 get(const uint8_t* s, int o, int v0, float& a, float& b) {
        a = lds_f16(s, o + 208) * (float)(int)(int8_t)(ld_u32(s, o + 192 + (v0 >> 4)) & 0xFFu);
        b = 0.0f;
        const int h = v0 >> 7, r = v0 & 127;
        const uint32_t lo = (ld_u32(s, o + 64 * h + (r & 63)) >> (4 * (r >> 6))) & 0x0F0F0F0Fu;
        const uint32_t hi = (ld_u32(s, o + 128 + 32 * h + (r & 31)) >> (2 * (r >> 5))) & 0x03030303u;
        return bytes_to_f16x4(lo | (hi << 4), (f16)-1056.0f);
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
    __device__ static f16x8 get(const uint8_t* s, int o, int v0, f16& mv) {
        const int sb = v0 >> 5;
        const uint32_t s0 = ld_u32(s, o + 4), s1 = ld_u32(s, o + 8), s2 = ld_u32(s, o + 12);
        int sc, mn;
        if (sb < 4) {
            sc = (s0 >> (8 * sb)) & 63;
            mn = (s1 >> (8 * sb)) & 63;
        } else {
            const int j = sb - 4;
            sc = ((s2 >> (8 * j)) & 0xF) | (((s0 >> (8 * j + 6)) & 3) << 4);
            mn = ((s2 >> (8 * j + 4)) & 0xF) | (((s1 >> (8 * j + 6)) & 3) << 4);
        }
        mv = (f16)(float)mn;
        constexpr int qs = (T == gguf::Q4_K) ? 16 : 48;
        const int i = v0 & 31, sh = (sb & 1) * 4;
        uint32_t t0 = (ld_u32(s, o + qs + 32 * (sb >> 1) + i) >> sh) & 0x0F0F0F0Fu;
        uint32_t t1 = (ld_u32(s, o + qs + 32 * (sb >> 1) + i + 4) >> sh) & 0x0F0F0F0Fu;
        if constexpr (T == gguf::Q5_K) {
            t0 |= ((ld_u32(s, o + 16 + i) >> sb) & 0x01010101u) << 4;
            t1 |= ((ld_u32(s, o + 20 + i) >> sb) & 0x01010101u) << 4;
        }
        const f16 scv = (f16)(float)sc;
        return bytes_to_f16x8_scaled(t0, t1, scv, (f16)(-1024.0f * (float)sc));
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
};

}  // namespace gguf_mfma
}  // namespace qlin
