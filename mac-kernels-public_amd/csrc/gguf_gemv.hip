// GGUF linear for a single activation row (M = 1): a VALU matrix-vector product.
//
// With one activation row the MFMA's 16-row tile would run 1/16 full while every lane still paid
// the decode, so this path decodes straight into packed fp16 pairs and uses v_dot2_f32_f16:
//   * each lane owns one contiguous "chunk" of a weight row (64 or 128 values: a run of whole
//     32-value blocks, or part of a 256-value super-block) and loads it with 16-byte global loads
//     (only 4-byte alignment is needed); a row is covered by 16..64 lanes, a wave covers 1..4 rows,
//     and the grid has one wave per such group of rows (its loads issued before anything else);
//   * the activation row is read once per workgroup with coalesced loads and staged in LDS in a
//     swizzled order (a lane's own chunk, read with a 256-byte lane stride straight from global
//     memory, would touch a different cache line per lane and per load); each lane keeps its
//     chunk in registers as fp16 pairs permuted to match the decode order, plus fp32 sums over
//     each scale group (needed by the offsets below);
//   * 4-bit codes: nibble pairs become fp16 (1024 + q) with one v_and_or_b32 ("0x6400 | nibble");
//     the 1024 (and any format offset) is removed in fp32 through the group sums:
//         sum_k x_k * (a * q_k + b) = a * (S - 1024 * sum x) + b * sum x,  S = sum x_k (1024 + q_k);
//     IQ4_NL / IQ4_XS / Q4_0 instead read a 256-entry LDS table byte -> (value(lo), value(hi)) and
//     pair it with (x_j, x_j+16);
//   * per lane fp32 partials are reduced across the row's lanes with xor shuffles.
// Everything after the fp16 operands is fp32; no weight is rounded to fp16.
#include <utility>

#include "qlin_internal.h"
#include "gguf_exact.h"

namespace qlin {
namespace {

// Compile-time loop: f(std::integral_constant<int, I>{}) for I in [0, N).
template <int N, typename F, int... I>
__device__ __forceinline__ void static_for_impl(F&& f, std::integer_sequence<int, I...>) {
    (f(std::integral_constant<int, I>{}), ...);
}
template <int N, typename F>
__device__ __forceinline__ void static_for(F&& f) {
    static_for_impl<N>(f, std::make_integer_sequence<int, N>{});
}

constexpr int GV_THREADS = 256;
constexpr int GV_MAX_K = 8192;

typedef uint32_t u32x4a __attribute__((ext_vector_type(4), aligned(4)));

__device__ __forceinline__ f16x2 h2(uint32_t u) { return __builtin_bit_cast(f16x2, u); }
__device__ __forceinline__ float dot2(uint32_t a, uint32_t b, float c) {
    return __builtin_amdgcn_fdot2(h2(a), h2(b), c, false);
}
// s + x.lo + x.hi for an fp16 pair x: one v_dot2_f32_f16 against (1, 1) (the products are exact)
__device__ __forceinline__ float pair_sum(uint32_t x, float s) { return dot2(x, 0x3C003C00u, s); }
// (x & 0x000F000F) | 0x64006400: fp16 pair (1024 + low nibble of byte 0, 1024 + low nibble of byte 2)
__device__ __forceinline__ uint32_t nib_pair(uint32_t w) { return (w & 0x000F000Fu) | 0x64006400u; }
// (x & 0x00F000F0) | 0x64006400: fp16 pair (1024 + 16 * high nibble of byte 0, of byte 2), exact
__device__ __forceinline__ uint32_t nib16_pair(uint32_t w) { return (w & 0x00F000F0u) | 0x64006400u; }
// bytes 0 and 2 (< 256) -> fp16 pair (1024 + b0, 1024 + b2)
__device__ __forceinline__ uint32_t byte_pair(uint32_t w) { return (w & 0x00FF00FFu) | 0x64006400u; }
// bytes 1 and 3 -> fp16 pair (1024 + b1, 1024 + b3): one v_perm against 0x64 bytes (no shift)
__device__ __forceinline__ uint32_t byte_pair_hi(uint32_t w) { return __builtin_amdgcn_perm(0x64646464u, w, 0x04030401u); }

// Interleave two fp16 pairs (a0, a1), (b0, b1) -> (a0, b0) and (a1, b1).
__device__ __forceinline__ uint32_t lo_lo(uint32_t a, uint32_t b) { return __builtin_amdgcn_perm(b, a, 0x05040100u); }
__device__ __forceinline__ uint32_t hi_hi(uint32_t a, uint32_t b) { return __builtin_amdgcn_perm(b, a, 0x07060302u); }

template <int N>
__device__ __forceinline__ void load_dwords(const uint8_t* p, uint32_t* r) {
    // p is 4-byte aligned; 16-byte loads need only dword alignment on gfx950.
#pragma unroll
    for (int i = 0; i + 4 <= N; i += 4) {
        const u32x4a v = *reinterpret_cast<const u32x4a*>(p + 4 * i);
        r[i] = v.x; r[i + 1] = v.y; r[i + 2] = v.z; r[i + 3] = v.w;
    }
#pragma unroll
    for (int i = (N / 4) * 4; i < N; ++i) r[i] = reinterpret_cast<const uint32_t*>(p)[i];
}

// Byte offset `off` (compile-time) of a dword array -> the dword starting there.
template <int OFF>
__device__ __forceinline__ uint32_t dw_at(const uint32_t* r) {
    if constexpr (OFF % 4 == 0) return r[OFF / 4];
    else return __builtin_amdgcn_alignbyte(r[OFF / 4 + 1], r[OFF / 4], OFF % 4);
}
template <int OFF>
__device__ __forceinline__ float half_at(const uint32_t* r) {
    const uint32_t w = (OFF % 4 == 0) ? r[OFF / 4] : (r[OFF / 4] >> 16);
    return f16_bits_to_f32((uint16_t)(w & 0xFFFFu));
}

// --------------------------------------------------------------------------------------------
// Format policies.  VC = values per lane chunk, LD = dwords loaded per chunk, CB = chunk byte
// offset inside a row for chunk c.  prep_x() turns the chunk's VC fp16 activations (natural order,
// as VC/2 pairs) into the operand order and the group sums; dot() returns the chunk's fp32 sum.
// --------------------------------------------------------------------------------------------
template <int T> struct GV;

// K-quants Q4_K / Q5_K: chunk = half super-block (sub-blocks 4h..4h+3, 128 values).
template <int T> struct GVK45 {
    static constexpr int QK = 256, TS = (T == gguf::Q4_K) ? 144 : 176, VC = 128;
    static constexpr int XP = 64;     // fp16 pairs kept per lane
    static constexpr int NG = 4;      // scale groups per chunk
    static constexpr int LD = (T == gguf::Q4_K) ? 20 : 28;
    static constexpr bool LUT = false;
    __device__ static int64_t chunk_off(int c) { return (int64_t)(c >> 1) * TS; }
    __device__ static void load(const uint8_t* row, int c, uint32_t* r) {
        const uint8_t* b = row + (int64_t)(c >> 1) * TS;
        const int h = c & 1;
        load_dwords<4>(b, r);                                  // d, dmin, scales[12]
        if constexpr (T == gguf::Q5_K) {
            load_dwords<8>(b + 16, r + 4);                     // qh[32]
            load_dwords<16>(b + 48 + 64 * h, r + 12);          // qs for sub-blocks 4h..4h+3
        } else {
            load_dwords<16>(b + 16 + 64 * h, r + 4);
        }
    }
    // natural pairs xn[v/2] = (x_v, x_v+1), v in [0,128): qs dword j (j<16) covers, for its low
    // nibbles, values v = 64*(j/8) + 4*(j%8) + t and for its high nibbles v + 32.
    __device__ static void prep_x(const uint32_t* xn, uint32_t* xp, float* xs) {
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            const int vlo = 64 * (j / 8) + 4 * (j % 8), vhi = vlo + 32;
            const uint32_t a = xn[vlo / 2], b = xn[vlo / 2 + 1], c = xn[vhi / 2], d = xn[vhi / 2 + 1];
            xp[4 * j + 0] = lo_lo(a, b);  // (x0, x2) low
            xp[4 * j + 1] = hi_hi(a, b);  // (x1, x3) low
            xp[4 * j + 2] = lo_lo(c, d);  // high
            xp[4 * j + 3] = hi_hi(c, d);
        }
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            float s = 0.0f;
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                s = pair_sum(xn[16 * g + i], s);
            }
            xs[g] = s;
        }
    }
    __device__ static float dot(const uint32_t* r, int c, const uint32_t* xp, const float* xs) {
        const int h = c & 1;
        const float d = f16_bits_to_f32((uint16_t)(r[0] & 0xFFFFu)), dmin = f16_bits_to_f32((uint16_t)(r[0] >> 16));
        const uint32_t s0 = r[1], s1 = r[2], s2 = r[3];
        constexpr int QB = (T == gguf::Q4_K) ? 4 : 12;
        float S[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            const uint32_t w = r[QB + j];
            const int pair = j / 8;               // sub-blocks 2*pair (low), 2*pair+1 (high)
            uint32_t lo = w, hi = w >> 4;
            if constexpr (T == gguf::Q5_K) {
                const uint32_t qh = r[4 + (j % 8)];
                const int sbl = 4 * h + 2 * pair;  // sub-block of the low nibbles
                lo = (w & 0x0F0F0F0Fu) | (((qh >> sbl) & 0x01010101u) << 4);
                hi = ((w >> 4) & 0x0F0F0F0Fu) | (((qh >> (sbl + 1)) & 0x01010101u) << 4);
                S[2 * pair] = dot2(byte_pair(lo), xp[4 * j], S[2 * pair]);
                S[2 * pair] = dot2(byte_pair_hi(lo), xp[4 * j + 1], S[2 * pair]);
                S[2 * pair + 1] = dot2(byte_pair(hi), xp[4 * j + 2], S[2 * pair + 1]);
                S[2 * pair + 1] = dot2(byte_pair_hi(hi), xp[4 * j + 3], S[2 * pair + 1]);
            } else {
                // high nibbles as 1024 + 16 q (no shift): their sums carry 16x the code term
                (void)hi;
                S[2 * pair] = dot2(nib_pair(lo), xp[4 * j], S[2 * pair]);
                S[2 * pair] = dot2(nib_pair(lo >> 8), xp[4 * j + 1], S[2 * pair]);
                S[2 * pair + 1] = dot2(nib16_pair(w), xp[4 * j + 2], S[2 * pair + 1]);
                S[2 * pair + 1] = dot2(nib16_pair(w >> 8), xp[4 * j + 3], S[2 * pair + 1]);
            }
        }
        float acc = 0.0f;
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const int sb = 4 * h + g;
            int sc, mn;
            if (h == 0) {
                sc = (s0 >> (8 * g)) & 63;
                mn = (s1 >> (8 * g)) & 63;
            } else {
                sc = ((s2 >> (8 * g)) & 0xF) | (((s0 >> (8 * g + 6)) & 3) << 4);
                mn = ((s2 >> (8 * g + 4)) & 0xF) | (((s1 >> (8 * g + 6)) & 3) << 4);
            }
            (void)sb;
            const float a = d * (float)sc, b = dmin * (float)mn;
            if (T == gguf::Q4_K && (g & 1)) acc += (0.0625f * a) * S[g] - (64.0f * a + b) * xs[g];
            else acc += a * S[g] - (1024.0f * a + b) * xs[g];
        }
        return acc;
    }
};
template <> struct GV<gguf::Q4_K> : GVK45<gguf::Q4_K> {};
template <> struct GV<gguf::Q5_K> : GVK45<gguf::Q5_K> {};

// Q8_0: chunk = 2 blocks (68 bytes, 64 values).
template <> struct GV<gguf::Q8_0> {
    static constexpr int VC = 64, XP = 32, NG = 2, LD = 17;
    static constexpr bool LUT = false;
    __device__ static void load(const uint8_t* row, int c, uint32_t* r) { load_dwords<17>(row + (int64_t)c * 68, r); }
    __device__ static void prep_x(const uint32_t* xn, uint32_t* xp, float* xs) {
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            xp[2 * j] = lo_lo(xn[2 * j], xn[2 * j + 1]);
            xp[2 * j + 1] = hi_hi(xn[2 * j], xn[2 * j + 1]);
        }
#pragma unroll
        for (int g = 0; g < 2; ++g) {
            float s = 0.0f;
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                s = pair_sum(xn[16 * g + i], s);
            }
            xs[g] = s;
        }
    }
    template <int B>
    __device__ static float block(const uint32_t* r, const uint32_t* xp, float xsum) {
        constexpr int o = 34 * B;
        const float d = half_at<o>(r);
        float S = 0.0f;
        static_for<8>([&](auto J) {
            constexpr int j = decltype(J)::value;
            const uint32_t w = dw_at<o + 2 + 4 * j>(r) ^ 0x80808080u;
            S = dot2(byte_pair(w), xp[16 * B + 2 * j], S);
            S = dot2(byte_pair_hi(w), xp[16 * B + 2 * j + 1], S);
        });
        return d * (S - 1152.0f * xsum);
    }
    __device__ static float dot(const uint32_t* r, int, const uint32_t* xp, const float* xs) {
        return block<0>(r, xp, xs[0]) + block<1>(r, xp, xs[1]);
    }
};

// Table formats: a 256-entry LDS table maps one code byte to the fp16 pair (value(lo), value(hi));
// the pair multiplies (x_j, x_j+16).
// Q4_0 / IQ4_NL: chunk = 4 blocks (72 bytes, 128 values).
template <int T> struct GVTab32 {
    static constexpr int QK = 32, TS = 18, VC = 128, XP = 64, NG = 4, LD = 18;
    static constexpr bool LUT = true;
    __device__ static void load(const uint8_t* row, int c, uint32_t* r) { load_dwords<18>(row + (int64_t)c * 72, r); }
    // block b (32 values): byte j (j<16) holds values j (lo) and j+16 (hi): pair (x_j, x_j+16)
    __device__ static void prep_x(const uint32_t* xn, uint32_t* xp, float* xs) {
#pragma unroll
        for (int b = 0; b < 4; ++b) {
#pragma unroll
            for (int j = 0; j < 16; j += 2) {
                const uint32_t lo = xn[16 * b + j / 2], hi = xn[16 * b + 8 + j / 2];
                xp[16 * b + j] = lo_lo(lo, hi);
                xp[16 * b + j + 1] = hi_hi(lo, hi);
            }
            float s = 0.0f;
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                s = pair_sum(xn[16 * b + i], s);
            }
            xs[b] = s;
        }
    }
    template <int B>
    __device__ static float block(const uint32_t* r, const uint32_t* xp, const uint32_t* tab) {
        constexpr int o = 18 * B;
        const float d = half_at<o>(r);
        float S = 0.0f;
        static_for<4>([&](auto Q) {
            constexpr int q = decltype(Q)::value;
            const uint32_t w = dw_at<o + 2 + 4 * q>(r);
#pragma unroll
            for (int t = 0; t < 4; ++t) S = dot2(tab[(w >> (8 * t)) & 0xFFu], xp[16 * B + 4 * q + t], S);
        });
        return d * S;
    }
    __device__ static float dot(const uint32_t* r, int, const uint32_t* xp, const float* xs, const uint32_t* tab) {
        (void)xs;
        return block<0>(r, xp, tab) + block<1>(r, xp, tab) + block<2>(r, xp, tab) + block<3>(r, xp, tab);
    }
};
template <> struct GV<gguf::Q4_0> : GVTab32<gguf::Q4_0> {};
template <> struct GV<gguf::IQ4_NL> : GVTab32<gguf::IQ4_NL> {};

// IQ4_XS: chunk = half super-block (sub-blocks 4h..4h+3, 128 values).
template <> struct GV<gguf::IQ4_XS> {
    static constexpr int TS = 136, VC = 128, XP = 64, NG = 4, LD = 18;
    static constexpr bool LUT = true;
    __device__ static void load(const uint8_t* row, int c, uint32_t* r) {
        const uint8_t* b = row + (int64_t)(c >> 1) * TS;
        load_dwords<2>(b, r);                          // d, scales_h, scales_l
        load_dwords<16>(b + 8 + 64 * (c & 1), r + 2);  // qs of the four sub-blocks
    }
    __device__ static void prep_x(const uint32_t* xn, uint32_t* xp, float* xs) {
        GVTab32<gguf::IQ4_NL>::prep_x(xn, xp, xs);  // same (x_j, x_j+16) pairing per 32 values
    }
    __device__ static float dot(const uint32_t* r, int c, const uint32_t* xp, const float* xs, const uint32_t* tab) {
        (void)xs;
        const int h = c & 1;
        const float d = f16_bits_to_f32((uint16_t)(r[0] & 0xFFFFu));
        const uint32_t sh = r[0] >> 16, sl = r[1];
        float acc = 0.0f;
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const int s = 4 * h + g;
            const int ls = ((sl >> (8 * (s >> 1) + 4 * (s & 1))) & 0xF) | (int)(((sh >> (2 * s)) & 3u) << 4);
            float S = 0.0f;
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const uint32_t w = r[2 + 4 * g + q];
#pragma unroll
                for (int t = 0; t < 4; ++t) S = dot2(tab[(w >> (8 * t)) & 0xFFu], xp[16 * g + 4 * q + t], S);
            }
            acc += (d * (float)(ls - 32)) * S;
        }
        return acc;
    }
};

// Q6_K: chunk = half super-block (128 values): ql[64h..+64], qh[32h..+32], scales[8h..+8], d.
// Blocks are 210 bytes, so a block may start 2 bytes off a dword boundary; each region is loaded
// from the dword below it and realigned with v_alignbyte.
template <> struct GV<gguf::Q6_K> {
    static constexpr int TS = 210, VC = 128, XP = 64, NG = 8, LD = 17 + 9 + 3 + 1 + 1;
    static constexpr bool LUT = false;
    // raw dwords as loaded (realigned in dot(), so that no loaded value is used before the
    // activation staging); r[30] = the block's byte offset from a dword boundary (0 or 2)
    __device__ static void load(const uint8_t* row, int c, uint32_t* r) {
        const int h = c & 1;
        const uint8_t* b = row + (int64_t)(c >> 1) * TS;
        const int sh = (int)((uintptr_t)b & 3);  // 0 or 2
        const uint8_t* a = b - sh;
        // ql and qh halves end at least 14 bytes before the block end: the extra dword stays inside
        load_dwords<17>(a + 64 * h, r);            // ql half
        load_dwords<9>(a + 128 + 32 * h, r + 17);  // qh half
        // scales and d sit at the end of the block: read no byte past it.  The third scale dword
        // is needed only when sh = 2; with sh = 0 it re-reads the second (and is shifted out).
        const uint32_t* sc = reinterpret_cast<const uint32_t*>(a + 192 + 8 * h);
        r[26] = sc[0];
        r[27] = sc[1];
        r[28] = sc[sh ? 2 : 1];
        r[29] = *reinterpret_cast<const uint16_t*>(b + 208);
        r[30] = (uint32_t)sh;
    }
    // alignbyte with shift 0 returns its low operand: the same code serves both alignments
    __device__ static void realign(const uint32_t* r, uint32_t* q) {
        const uint32_t sh = r[30];
#pragma unroll
        for (int i = 0; i < 16; ++i) q[i] = __builtin_amdgcn_alignbyte(r[i + 1], r[i], sh);
#pragma unroll
        for (int i = 17; i < 25; ++i) q[i] = __builtin_amdgcn_alignbyte(r[i + 1], r[i], sh);
        q[26] = __builtin_amdgcn_alignbyte(r[27], r[26], sh);
        q[27] = __builtin_amdgcn_alignbyte(r[28], r[27], sh);
        q[29] = r[29];
    }
    // ql dword j: low nibbles -> values 4j..4j+3, high nibbles -> 64 + 4j..; natural pairing (x0,x2),(x1,x3)
    __device__ static void prep_x(const uint32_t* xn, uint32_t* xp, float* xs) {
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            const int vlo = 4 * j, vhi = 64 + 4 * j;
            xp[4 * j + 0] = lo_lo(xn[vlo / 2], xn[vlo / 2 + 1]);
            xp[4 * j + 1] = hi_hi(xn[vlo / 2], xn[vlo / 2 + 1]);
            xp[4 * j + 2] = lo_lo(xn[vhi / 2], xn[vhi / 2 + 1]);
            xp[4 * j + 3] = hi_hi(xn[vhi / 2], xn[vhi / 2 + 1]);
        }
#pragma unroll
        for (int g = 0; g < 8; ++g) {
            float s = 0.0f;
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                s = pair_sum(xn[8 * g + i], s);
            }
            xs[g] = s;
        }
    }
    __device__ static float dot(const uint32_t* raw, int, const uint32_t* xp, const float* xs) {
        uint32_t r[30];
        realign(raw, r);
        const float d = f16_bits_to_f32((uint16_t)(r[29] & 0xFFFFu));
        float S[8];
#pragma unroll
        for (int g = 0; g < 8; ++g) S[g] = 0.0f;
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            const uint32_t ql = r[j], qh = r[17 + (j % 8)];
            const int sl = 2 * (j / 8);  // qh shift for the low-nibble values (v = 4j < 64)
            const uint32_t lo = (ql & 0x0F0F0F0Fu) | (((qh >> sl) & 0x03030303u) << 4);
            const uint32_t hi = ((ql >> 4) & 0x0F0F0F0Fu) | (((qh >> (sl + 4)) & 0x03030303u) << 4);
            const int glo = j / 4, ghi = 4 + j / 4;  // 16-value groups of v = 4j and 64 + 4j
            S[glo] = dot2(byte_pair(lo), xp[4 * j], S[glo]);
            S[glo] = dot2(byte_pair_hi(lo), xp[4 * j + 1], S[glo]);
            S[ghi] = dot2(byte_pair(hi), xp[4 * j + 2], S[ghi]);
            S[ghi] = dot2(byte_pair_hi(hi), xp[4 * j + 3], S[ghi]);
        }
        float acc = 0.0f;
#pragma unroll
        for (int g = 0; g < 8; ++g) {
            const int sc = (int)(int8_t)(r[26 + g / 4] >> (8 * (g % 4)));
            const float a = d * (float)sc;
            acc += a * (S[g] - 1056.0f * xs[g]);
        }
        return acc;
    }
};

template <int T>
__device__ __forceinline__ uint32_t table_entry(int b) {
    // fp16 pair (value(lo nibble), value(hi nibble)) for code byte b
    float lo, hi;
    if constexpr (T == gguf::Q4_0) {
        lo = (float)((b & 0xF) - 8);
        hi = (float)((b >> 4) - 8);
    } else {
        lo = (float)gguf::iq4nl_level(b & 0xF);
        hi = (float)gguf::iq4nl_level(b >> 4);
    }
    return (uint32_t)__builtin_bit_cast(uint16_t, (f16)lo) | ((uint32_t)__builtin_bit_cast(uint16_t, (f16)hi) << 16);
}

// LPR lanes per row (a power of two <= 64); RPP = 64 / LPR rows per pass of a wave.
// Order of work: the activation row (coalesced), then each wave's weight chunks for two passes --
// so every load is in flight before the first wait -- then the LDS staging of the activations
// (and the table, for formats with one) and the prep of the activation pairs while the weights
// arrive.  No load sits behind a lane-dependent branch: rows past N re-read row N - 1 and are
// not stored.
template <int T, int LPR>
__global__ __launch_bounds__(GV_THREADS) void gguf_gemv_kernel(const f16* __restrict__ x, const int32_t* __restrict__ xexp,
                                                               const uint8_t* __restrict__ w,
                                                               int64_t row_bytes, int N, int K,
                                                               const void* __restrict__ bias, int bias_dt,
                                                               void* __restrict__ y, int y_dt) {
    using F = GV<T>;
    constexpr int VC = F::VC;
    constexpr int RPP = 64 / LPR;  // rows per pass of a wave
    constexpr int NU = VC / 8;     // 16-byte activation units per chunk
    __shared__ uint32_t tab_all[F::LUT ? GV_THREADS / 64 : 1][F::LUT ? 256 : 1];
    __shared__ __attribute__((aligned(16))) u32x4 xs_lds[GV_MAX_K / 8];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int c = lane % LPR, rp = lane / LPR;

    const int waves_total = gridDim.x * (GV_THREADS / 64);
    const int gw = blockIdx.x * (GV_THREADS / 64) + wave;
    const int passes = (N + RPP - 1) / RPP;
    const int KU = K / 8;

    // 1. the activation row, with fully coalesced loads (consecutive lanes, consecutive 16 bytes).
    //    Without branches: units past the row re-read (and below re-write) its last unit.
    u32x4 xst[GV_MAX_K / 8 / GV_THREADS];
#pragma unroll
    for (int j = 0; j < GV_MAX_K / 8 / GV_THREADS; ++j)
        xst[j] = reinterpret_cast<const u32x4*>(x)[min(tid + GV_THREADS * j, KU - 1)];
    // 2. the weight chunks of this wave's first pass (rows past N re-read row N - 1)
    auto row_of = [&](int p) { return min(p * RPP + rp, N - 1); };
    int p = gw;
    uint32_t r0[F::LD];
    __builtin_amdgcn_sched_barrier(0);
    F::load(w + (int64_t)row_of(p) * row_bytes, c, r0);
    // epilogue operands, fetched now rather than after the reduction
    const int xe = xexp ? xexp[0] : 0;
    uint32_t bv0 = 0;  // raw bits (0 reads as +0 in every dtype)
    if (bias) bv0 = load_bits_rt(bias, bias_dt, row_of(p));
    __builtin_amdgcn_sched_barrier(0);
    // 3. activations into LDS: unit i of chunk c at i * LPR + (c ^ i), so that the per-lane reads
    //    below (fixed i, consecutive c) and these writes both spread over the banks.  The fences
    //    order LDS only: the weight loads stay in flight across the barrier.
#pragma unroll
    for (int j = 0; j < GV_MAX_K / 8 / GV_THREADS; ++j) {
        const int u = min(tid + GV_THREADS * j, KU - 1);
        const int cc = u / NU, i = u % NU;
        xs_lds[i * LPR + (cc ^ i)] = xst[j];
    }
    uint32_t* tab = tab_all[F::LUT ? wave : 0];
    if constexpr (F::LUT) {
#pragma unroll
        for (int i = 0; i < 4; ++i) tab[lane + 64 * i] = table_entry<T>(lane + 64 * i);
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
    __builtin_amdgcn_sched_barrier(0);  // nothing that needs a weight value moves above this point
    uint32_t xn[VC / 2];
#pragma unroll
    for (int i = 0; i < NU; ++i) {
        const u32x4 v = xs_lds[i * LPR + (c ^ i)];
        xn[4 * i] = v.x; xn[4 * i + 1] = v.y; xn[4 * i + 2] = v.z; xn[4 * i + 3] = v.w;
    }
    uint32_t xp[F::XP];
    float xsum[F::NG];
    F::prep_x(xn, xp, xsum);

    auto finish = [&](const uint32_t* r, int pp, uint32_t bv) {
        const int n = pp * RPP + rp;
        float v;
        if constexpr (F::LUT) v = F::dot(r, c, xp, xsum, tab);
        else v = F::dot(r, c, xp, xsum);
#pragma unroll
        for (int m = 1; m < LPR; m <<= 1) v += __shfl_xor(v, m, 64);
        if (c == 0 && n < N) store_rt(y, y_dt, n, __builtin_ldexpf(v, xe) + bits_to_f32_rt(bv, bias_dt));
    };
    // The first pass is computed unconditionally (its store is guarded), so its loads are not
    // moved into a branch behind the barrier; the launch sizes the grid so that it is all there is.
    for (;;) {
        finish(r0, p, bv0);
        p += waves_total;
        if (p >= passes) break;
        F::load(w + (int64_t)row_of(p) * row_bytes, c, r0);
        if (bias) bv0 = load_bits_rt(bias, bias_dt, row_of(p));
    }
}

template <int T>
hipError_t launch(const GgufGemvArgs& a, hipStream_t st) {
    using F = GV<T>;
    const int lpr = a.K / F::VC;
    const int rpp = 64 / lpr;
    const int passes = (a.N + rpp - 1) / rpp;
    // One pass per wave, every wave's loads issued up front.  Two passes per wave (half the
    // waves, the second pass's loads also up front) measured 5-14% slower at K = N = 4096: with
    // eight waves per CU instead of four, one wave's decode overlaps another's loads.
    int waves = passes;
    int blocks = (waves + 3) / 4;
    if (blocks < 1) blocks = 1;
    dim3 grid((unsigned)blocks), block(GV_THREADS);
#define QLIN_GV(L)                                                                                      \
    hipLaunchKernelGGL((gguf_gemv_kernel<T, L>), grid, block, 0, st, a.x, a.xexp, a.w, a.row_bytes, a.N, a.K, a.bias, \
                       a.bias_dtype, a.y, a.y_dtype)
    switch (lpr) {
        case 16: QLIN_GV(16); break;
        case 32: QLIN_GV(32); break;
        case 64: QLIN_GV(64); break;
        default: return hipErrorInvalidValue;
    }
#undef QLIN_GV
    return hipGetLastError();
}

template <typename Fn>
bool dispatch_gemv(int t, Fn&& f) {
    switch (t) {
        case gguf::Q4_0: f.template operator()<gguf::Q4_0>(); return true;
        case gguf::Q8_0: f.template operator()<gguf::Q8_0>(); return true;
        case gguf::Q4_K: f.template operator()<gguf::Q4_K>(); return true;
        case gguf::Q5_K: f.template operator()<gguf::Q5_K>(); return true;
        case gguf::Q6_K: f.template operator()<gguf::Q6_K>(); return true;
        case gguf::IQ4_NL: f.template operator()<gguf::IQ4_NL>(); return true;
        case gguf::IQ4_XS: f.template operator()<gguf::IQ4_XS>(); return true;
        default: return false;
    }
}

}  // namespace

bool gguf_gemv_supported(int type, int64_t M, int64_t K, int64_t row_bytes, const void* w, const void* x) {
    if (M != 1 || K > GV_MAX_K || (uintptr_t)w % 4 || (uintptr_t)x % 16 || row_bytes % 4) return false;
    bool ok = false;
    dispatch_gemv(type, [&]<int T>() {
        const int64_t vc = GV<T>::VC;
        if (K % vc) return;
        const int64_t lpr = K / vc;
        ok = (lpr == 16 || lpr == 32 || lpr == 64);
    });
    return ok;
}

hipError_t run_gguf_gemv(const GgufGemvArgs& a, hipStream_t st) {
    if (a.y_dtype != DT_F32 && a.y_dtype != DT_F16 && a.y_dtype != DT_BF16) return hipErrorInvalidValue;
    hipError_t err = hipErrorInvalidValue;
    bool ok = dispatch_gemv(a.type, [&]<int T>() { err = launch<T>(a, st); });
    return ok ? err : hipErrorInvalidValue;
}

}  // namespace qlin
