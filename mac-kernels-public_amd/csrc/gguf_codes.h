// GGUF block -> MFMA operand decode for the small-M kernels.
//
// A "unit" is one scale group of a block (32 values, or 16 for Q2_K/Q3_K/Q6_K).  For lane
// group g (lane / 16) the decoder returns the VPL = UNIT/4 consecutive values starting at
// VPL*g as exact small integers q (|q| <= 127) plus the unit's fp32 scale a and offset b, so
// that value = a*q + b.  The kernel feeds q to the fp16 MFMA (exact) and applies a, b in fp32:
//     sum_k x_k * value_k = a * sum_k x_k q_k + b * sum_k x_k.
// Bytes are read from a staged copy of the block row in LDS (`s`: LDS base of the stage row,
// `o`: byte offset of the block inside the stage).  Layouts follow
// docs/research/2026-10-03-gguf-on-metal.md:18-36 (roblennon/mac-kernels-public).
#pragma once
#include "gguf_exact.h"

namespace qlin {
namespace gguf {

template <int T> struct Codes;

__device__ __forceinline__ float lds_half(const uint8_t* s, int off) { return f16_bits_to_f32(ld_u16(s, off)); }
__device__ __forceinline__ uint32_t lds_byte(const uint8_t* s, int off) { return ld_u32(s, off) & 0xFFu; }

// Eight consecutive bytes starting at `off` (any alignment) as two dwords.
__device__ __forceinline__ void lds_bytes8(const uint8_t* s, int off, uint32_t& w0, uint32_t& w1) {
    w0 = ld_u32(s, off);
    w1 = ld_u32(s, off + 4);
}

template <> struct Codes<Q8_0> {
    static constexpr int QK = 32, TS = 34, UNIT = 32;
    static constexpr bool MIN = false;
    __device__ static void get(const uint8_t* s, int o, int v0, int* q, float& a, float& b) {
        a = lds_half(s, o);
        b = 0.0f;
        uint32_t w0, w1;
        lds_bytes8(s, o + 2 + v0, w0, w1);
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            q[t] = (int)(int8_t)(w0 >> (8 * t));
            q[t + 4] = (int)(int8_t)(w1 >> (8 * t));
        }
    }
};

// Q4_0 / IQ4_NL share the byte layout: f16 d, qs[16]; value j<16 = lo(qs[j]), j>=16 = hi(qs[j-16]).
template <int T> struct Codes32Nib {
    static constexpr int QK = 32, TS = 18, UNIT = 32;
    static constexpr bool MIN = false;
    __device__ static void get(const uint8_t* s, int o, int v0, int* q, float& a, float& b) {
        a = lds_half(s, o);
        b = 0.0f;
        uint32_t w0, w1;
        lds_bytes8(s, o + 2 + (v0 & 15), w0, w1);
        const int sh = (v0 >> 4) * 4;
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            int n0 = (w0 >> (8 * t + sh)) & 0xF, n1 = (w1 >> (8 * t + sh)) & 0xF;
            if constexpr (T == Q4_0) {
                q[t] = n0 - 8;
                q[t + 4] = n1 - 8;
            } else {
                q[t] = iq4nl_level(n0);
                q[t + 4] = iq4nl_level(n1);
            }
        }
    }
};
template <> struct Codes<Q4_0> : Codes32Nib<Q4_0> {};
template <> struct Codes<IQ4_NL> : Codes32Nib<IQ4_NL> {};

template <> struct Codes<Q4_1> {
    static constexpr int QK = 32, TS = 20, UNIT = 32;
    static constexpr bool MIN = true;
    __device__ static void get(const uint8_t* s, int o, int v0, int* q, float& a, float& b) {
        a = lds_half(s, o);
        b = lds_half(s, o + 2);
        uint32_t w0, w1;
        lds_bytes8(s, o + 4 + (v0 & 15), w0, w1);
        const int sh = (v0 >> 4) * 4;
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            q[t] = (w0 >> (8 * t + sh)) & 0xF;
            q[t + 4] = (w1 >> (8 * t + sh)) & 0xF;
        }
    }
};

template <int T> struct Codes5 {
    static constexpr int QK = 32, TS = (T == Q5_0) ? 22 : 24, UNIT = 32;
    static constexpr bool MIN = (T == Q5_1);
    __device__ static void get(const uint8_t* s, int o, int v0, int* q, float& a, float& b) {
        constexpr int qo = (T == Q5_0) ? 2 : 4;
        a = lds_half(s, o);
        b = (T == Q5_1) ? lds_half(s, o + 2) : 0.0f;
        const uint32_t qh = ld_u32(s, o + qo);
        uint32_t w0, w1;
        lds_bytes8(s, o + qo + 4 + (v0 & 15), w0, w1);
        const int sh = (v0 >> 4) * 4;
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            int n0 = ((w0 >> (8 * t + sh)) & 0xF) | (int)(((qh >> (v0 + t)) & 1u) << 4);
            int n1 = ((w1 >> (8 * t + sh)) & 0xF) | (int)(((qh >> (v0 + 4 + t)) & 1u) << 4);
            q[t] = (T == Q5_0) ? n0 - 16 : n0;
            q[t + 4] = (T == Q5_0) ? n1 - 16 : n1;
        }
    }
};
template <> struct Codes<Q5_0> : Codes5<Q5_0> {};
template <> struct Codes<Q5_1> : Codes5<Q5_1> {};

__device__ __forceinline__ void kq_scale_min_lds(const uint8_t* s, int o, int j, int& sc, int& mn) {
    // scales[12] at o: low 6 bits of bytes 0-3 / 4-7 for j < 4; nibble of bytes 8-11 plus the
    // top 2 bits of bytes 0-3 / 4-7 for j >= 4.
    const uint32_t s0 = ld_u32(s, o), s1 = ld_u32(s, o + 4), s2 = ld_u32(s, o + 8);
    if (j < 4) {
        sc = (s0 >> (8 * j)) & 63;
        mn = (s1 >> (8 * j)) & 63;
    } else {
        const int jj = j - 4;
        sc = ((s2 >> (8 * jj)) & 0xF) | (((s0 >> (8 * jj + 6)) & 3) << 4);
        mn = ((s2 >> (8 * jj + 4)) & 0xF) | (((s1 >> (8 * jj + 6)) & 3) << 4);
    }
}

template <int T> struct CodesK45 {
    static constexpr int QK = 256, TS = (T == Q4_K) ? 144 : 176, UNIT = 32;
    static constexpr bool MIN = true;
    __device__ static void get(const uint8_t* s, int o, int v0, int* q, float& a, float& b) {
        const float d = lds_half(s, o), dmin = lds_half(s, o + 2);
        const int sb = v0 >> 5;
        int sc, mn;
        kq_scale_min_lds(s, o + 4, sb, sc, mn);
        a = d * (float)sc;
        b = -(dmin * (float)mn);
        constexpr int qs = (T == Q4_K) ? 16 : 48;
        uint32_t w0, w1;
        lds_bytes8(s, o + qs + 32 * (sb >> 1) + (v0 & 31), w0, w1);
        const int sh = (sb & 1) * 4;
        uint32_t h0 = 0, h1 = 0;
        if constexpr (T == Q5_K) lds_bytes8(s, o + 16 + (v0 & 31), h0, h1);
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            int n0 = (w0 >> (8 * t + sh)) & 0xF, n1 = (w1 >> (8 * t + sh)) & 0xF;
            if constexpr (T == Q5_K) {
                n0 |= ((h0 >> (8 * t + sb)) & 1) << 4;
                n1 |= ((h1 >> (8 * t + sb)) & 1) << 4;
            }
            q[t] = n0;
            q[t + 4] = n1;
        }
    }
};
template <> struct Codes<Q4_K> : CodesK45<Q4_K> {};
template <> struct Codes<Q5_K> : CodesK45<Q5_K> {};

template <> struct Codes<IQ4_XS> {
    static constexpr int QK = 256, TS = 136, UNIT = 32;
    static constexpr bool MIN = false;
    __device__ static void get(const uint8_t* s, int o, int v0, int* q, float& a, float& b) {
        const float d = lds_half(s, o);
        const int sb = v0 >> 5;
        const uint32_t hdr = ld_u32(s, o);            // d (16 bits) | scales_h (16 bits)
        const uint32_t sl = ld_u32(s, o + 4);         // scales_l[4]
        const int ls = ((sl >> (8 * (sb >> 1) + 4 * (sb & 1))) & 0xF) | (int)(((hdr >> (16 + 2 * sb)) & 3u) << 4);
        a = d * (float)(ls - 32);
        b = 0.0f;
        const int i = v0 & 31;
        uint32_t w0, w1;
        lds_bytes8(s, o + 8 + 16 * sb + (i & 15), w0, w1);
        const int sh = (i >> 4) * 4;
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            q[t] = iq4nl_level((w0 >> (8 * t + sh)) & 0xF);
            q[t + 4] = iq4nl_level((w1 >> (8 * t + sh)) & 0xF);
        }
    }
};

// Units of 16 values: the decoder returns 4 values starting at v0.
template <> struct Codes<Q6_K> {
    static constexpr int QK = 256, TS = 210, UNIT = 16;
    static constexpr bool MIN = false;
    __device__ static void get(const uint8_t* s, int o, int v0, int* q, float& a, float& b) {
        const float d = lds_half(s, o + 208);
        a = d * (float)(int)(int8_t)lds_byte(s, o + 192 + (v0 >> 4));
        b = 0.0f;
        const int h = v0 >> 7, r = v0 & 127;
        const uint32_t l = ld_u32(s, o + 64 * h + (r & 63));
        const uint32_t hh = ld_u32(s, o + 128 + 32 * h + (r & 31));
        const int lsh = 4 * (r >> 6), hsh = 2 * (r >> 5);
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            int lo = (l >> (8 * t + lsh)) & 0xF;
            int hi = (hh >> (8 * t + hsh)) & 3;
            q[t] = (lo | (hi << 4)) - 32;
        }
    }
};

template <> struct Codes<Q3_K> {
    static constexpr int QK = 256, TS = 110, UNIT = 16;
    static constexpr bool MIN = false;
    __device__ static void get(const uint8_t* s, int o, int v0, int* q, float& a, float& b) {
        const float d = lds_half(s, o + 108);
        const int sidx = v0 >> 4;
        const int lo = (lds_byte(s, o + 96 + (sidx & 7)) >> (4 * (sidx >> 3))) & 0xF;
        const int hs = (lds_byte(s, o + 104 + (sidx & 3)) >> (2 * (sidx >> 2))) & 3;
        a = d * (float)((lo | (hs << 4)) - 32);
        b = 0.0f;
        const int h = v0 >> 7, t2 = (v0 >> 5) & 3, i0 = v0 & 31, hb = v0 >> 5;
        const uint32_t qq = ld_u32(s, o + 32 + 32 * h + i0);
        const uint32_t hm = ld_u32(s, o + i0);
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            int q2 = (qq >> (8 * t + 2 * t2)) & 3;
            int hbit = (hm >> (8 * t + hb)) & 1;
            q[t] = q2 - ((hbit ^ 1) << 2);
        }
    }
};

template <> struct Codes<Q2_K> {
    static constexpr int QK = 256, TS = 84, UNIT = 16;
    static constexpr bool MIN = true;
    __device__ static void get(const uint8_t* s, int o, int v0, int* q, float& a, float& b) {
        const float d = lds_half(s, o + 80), dmin = lds_half(s, o + 82);
        const uint32_t sc = lds_byte(s, o + (v0 >> 4));
        a = d * (float)(sc & 0xF);
        b = -(dmin * (float)(sc >> 4));
        const int h = v0 >> 7, t2 = (v0 >> 5) & 3, i0 = v0 & 31;
        const uint32_t qq = ld_u32(s, o + 16 + 32 * h + i0);
#pragma unroll
        for (int t = 0; t < 4; ++t) q[t] = (qq >> (8 * t + 2 * t2)) & 3;
    }
};

}  // namespace gguf
}  // namespace qlin
