// Exact GGUF block decode on the GPU: eight consecutive values of one block, computed in fp32
// with separately rounded multiplies and adds in the order gguf-py 0.19.0 uses, so the result
// is bit-identical to the reference decode (layouts: docs/research/2026-10-03-gguf-on-metal.md
// :18-36 of roblennon/mac-kernels-public).  `b` points at the block, `j` is the index of the
// first value (a multiple of 8), and the eight values always share one scale group.
#pragma once
#include "qlin_device.h"

namespace qlin {
namespace gguf {

enum Type : int {
    Q4_0 = 2, Q4_1 = 3, Q5_0 = 6, Q5_1 = 7, Q8_0 = 8, Q2_K = 10, Q3_K = 11,
    Q4_K = 12, Q5_K = 13, Q6_K = 14, IQ4_NL = 20, IQ4_XS = 23,
};

template <int T> struct Info;
template <> struct Info<Q4_0>   { static constexpr int QK = 32,  TS = 18;  };
template <> struct Info<Q4_1>   { static constexpr int QK = 32,  TS = 20;  };
template <> struct Info<Q5_0>   { static constexpr int QK = 32,  TS = 22;  };
template <> struct Info<Q5_1>   { static constexpr int QK = 32,  TS = 24;  };
template <> struct Info<Q8_0>   { static constexpr int QK = 32,  TS = 34;  };
template <> struct Info<Q2_K>   { static constexpr int QK = 256, TS = 84;  };
template <> struct Info<Q3_K>   { static constexpr int QK = 256, TS = 110; };
template <> struct Info<Q4_K>   { static constexpr int QK = 256, TS = 144; };
template <> struct Info<Q5_K>   { static constexpr int QK = 256, TS = 176; };
template <> struct Info<Q6_K>   { static constexpr int QK = 256, TS = 210; };
template <> struct Info<IQ4_NL> { static constexpr int QK = 32,  TS = 18;  };
template <> struct Info<IQ4_XS> { static constexpr int QK = 256, TS = 136; };

// ggml's IQ4_NL level table (public ggml, ggml-common.h kvalues_iq4nl; used by gguf-py for
// IQ4_NL and IQ4_XS).
__device__ __forceinline__ int iq4nl_level(int i) {
    // Packed as 16 signed bytes in four dwords; selecting one byte keeps the table in SGPRs.
    const uint32_t t0 = 0xBFAD9881u;  // -127,-104,-83,-65
    const uint32_t t1 = 0xF6EADDCFu;  // -49,-35,-22,-10
    const uint32_t t2 = 0x26190D01u;  // 1,13,25,38
    const uint32_t t3 = 0x71594535u;  // 53,69,89,113
    uint32_t w = (i < 8) ? ((i < 4) ? t0 : t1) : ((i < 12) ? t2 : t3);
    return (int)(int8_t)(uint8_t)(w >> (8 * (i & 3)));
}

__device__ __forceinline__ float rd_half(const uint8_t* p) {
    return f16_bits_to_f32((uint16_t)(p[0] | (p[1] << 8)));
}

__device__ __forceinline__ void kq_scale_min(const uint8_t* s, int j, int& sc, int& mn) {
    if (j < 4) {
        sc = s[j] & 63;
        mn = s[j + 4] & 63;
    } else {
        sc = (s[j + 4] & 0xF) | ((s[j - 4] >> 6) << 4);
        mn = (s[j + 4] >> 4) | ((s[j] >> 6) << 4);
    }
}

template <int T>
__device__ __forceinline__ void decode8(const uint8_t* b, int j, float* y) {
#pragma clang fp contract(off)
    if constexpr (T == Q4_0 || T == IQ4_NL) {
        const float d = rd_half(b);
        const int hi = j >= 16;
        const int j0 = j & 15;
#pragma unroll
        for (int t = 0; t < 8; ++t) {
            int nib = (b[2 + j0 + t] >> (4 * hi)) & 0xF;
            if constexpr (T == Q4_0) y[t] = d * (float)(nib - 8);
            else y[t] = d * (float)iq4nl_level(nib);
        }
    } else if constexpr (T == Q4_1) {
        const float d = rd_half(b), m = rd_half(b + 2);
        const int hi = j >= 16, j0 = j & 15;
#pragma unroll
        for (int t = 0; t < 8; ++t) {
            float p = d * (float)((b[4 + j0 + t] >> (4 * hi)) & 0xF);
            y[t] = p + m;
        }
    } else if constexpr (T == Q5_0 || T == Q5_1) {
        constexpr int o = (T == Q5_0) ? 2 : 4;
        const float d = rd_half(b);
        const float m = (T == Q5_1) ? rd_half(b + 2) : 0.0f;
        const uint32_t qh = (uint32_t)b[o] | ((uint32_t)b[o + 1] << 8) | ((uint32_t)b[o + 2] << 16) |
                            ((uint32_t)b[o + 3] << 24);
        const int hi = j >= 16, j0 = j & 15;
#pragma unroll
        for (int t = 0; t < 8; ++t) {
            int q = ((b[o + 4 + j0 + t] >> (4 * hi)) & 0xF) | (int)(((qh >> (j + t)) & 1u) << 4);
            if constexpr (T == Q5_0) {
                y[t] = d * (float)(q - 16);
            } else {
                float p = d * (float)q;
                y[t] = p + m;
            }
        }
    } else if constexpr (T == Q8_0) {
        const float d = rd_half(b);
#pragma unroll
        for (int t = 0; t < 8; ++t) y[t] = (float)(int8_t)b[2 + j + t] * d;
    } else if constexpr (T == Q2_K) {
        const float d = rd_half(b + 80), dmin = rd_half(b + 82);
        const int s = j >> 4;
        const float dl = d * (float)(b[s] & 0xF);
        const float ml = dmin * (float)(b[s] >> 4);
        const int h = j >> 7, t2 = (j >> 5) & 3, i0 = j & 31;
#pragma unroll
        for (int t = 0; t < 8; ++t) {
            int q = (b[16 + 32 * h + i0 + t] >> (2 * t2)) & 3;
            float p = dl * (float)q;
            y[t] = p - ml;
        }
    } else if constexpr (T == Q3_K) {
        const float d = rd_half(b + 108);
        const int s = j >> 4;
        const int lo = (b[96 + (s & 7)] >> (4 * (s >> 3))) & 0xF;
        const int hs = (b[96 + 8 + (s & 3)] >> (2 * (s >> 2))) & 3;
        const float dl = d * (float)((lo | (hs << 4)) - 32);
        const int h = j >> 7, t2 = (j >> 5) & 3, i0 = j & 31, hb = j >> 5;
#pragma unroll
        for (int t = 0; t < 8; ++t) {
            int q2 = (b[32 + 32 * h + i0 + t] >> (2 * t2)) & 3;
            int hbit = (b[i0 + t] >> hb) & 1;
            y[t] = dl * (float)(q2 - ((hbit ^ 1) << 2));
        }
    } else if constexpr (T == Q4_K || T == Q5_K) {
        const float d = rd_half(b), dmin = rd_half(b + 2);
        const int sb = j >> 5;
        int sc, mn;
        kq_scale_min(b + 4, sb, sc, mn);
        const float dl = d * (float)sc;
        const float ml = dmin * (float)mn;
        constexpr int qs_off = (T == Q4_K) ? 16 : 48;
        const int c = sb >> 1, sh = (sb & 1) * 4, i0 = j & 31;
#pragma unroll
        for (int t = 0; t < 8; ++t) {
            int q = (b[qs_off + 32 * c + i0 + t] >> sh) & 0xF;
            if constexpr (T == Q5_K) q |= ((b[16 + i0 + t] >> sb) & 1) << 4;
            float p = dl * (float)q;
            y[t] = p - ml;
        }
    } else if constexpr (T == Q6_K) {
        const float d = rd_half(b + 208);
        const float dl = d * (float)(int8_t)b[192 + (j >> 4)];
        const int h = j >> 7, r0 = j & 127;
#pragma unroll
        for (int t = 0; t < 8; ++t) {
            const int r = r0 + t;
            int lo = (b[64 * h + (r & 63)] >> (4 * (r >> 6))) & 0xF;
            int hi = (b[128 + 32 * h + (r & 31)] >> (2 * (r >> 5))) & 3;
            y[t] = dl * (float)((lo | (hi << 4)) - 32);
        }
    } else if constexpr (T == IQ4_XS) {
        const float d = rd_half(b);
        const uint32_t sh = (uint32_t)b[2] | ((uint32_t)b[3] << 8);
        const int s = j >> 5;
        const int ls = ((b[4 + (s >> 1)] >> (4 * (s & 1))) & 0xF) | (int)(((sh >> (2 * s)) & 3u) << 4);
        const float dl = d * (float)(ls - 32);
        const int i = j & 31, hi = i >= 16, i0 = i & 15;
#pragma unroll
        for (int t = 0; t < 8; ++t) {
            int nib = (b[8 + 16 * s + i0 + t] >> (4 * hi)) & 0xF;
            y[t] = dl * (float)iq4nl_level(nib);
        }
    }
}

// Dispatch helper: call F.template operator()<T>() for a runtime ggml type id.
template <typename F>
__host__ inline bool dispatch_type(int t, F&& f) {
    switch (t) {
        case Q4_0: f.template operator()<Q4_0>(); return true;
        case Q4_1: f.template operator()<Q4_1>(); return true;
        case Q5_0: f.template operator()<Q5_0>(); return true;
        case Q5_1: f.template operator()<Q5_1>(); return true;
        case Q8_0: f.template operator()<Q8_0>(); return true;
        case Q2_K: f.template operator()<Q2_K>(); return true;
        case Q3_K: f.template operator()<Q3_K>(); return true;
        case Q4_K: f.template operator()<Q4_K>(); return true;
        case Q5_K: f.template operator()<Q5_K>(); return true;
        case Q6_K: f.template operator()<Q6_K>(); return true;
        case IQ4_NL: f.template operator()<IQ4_NL>(); return true;
        case IQ4_XS: f.template operator()<IQ4_XS>(); return true;
        default: return false;
    }
}

__host__ inline bool type_info(int t, int& qk, int& ts) {
    switch (t) {
        case Q4_0: qk = 32; ts = 18; return true;
        case Q4_1: qk = 32; ts = 20; return true;
        case Q5_0: qk = 32; ts = 22; return true;
        case Q5_1: qk = 32; ts = 24; return true;
        case Q8_0: qk = 32; ts = 34; return true;
        case Q2_K: qk = 256; ts = 84; return true;
        case Q3_K: qk = 256; ts = 110; return true;
        case Q4_K: qk = 256; ts = 144; return true;
        case Q5_K: qk = 256; ts = 176; return true;
        case Q6_K: qk = 256; ts = 210; return true;
        case IQ4_NL: qk = 32; ts = 18; return true;
        case IQ4_XS: qk = 256; ts = 136; return true;
        default: return false;
    }
}

}  // namespace gguf
}  // namespace qlin
