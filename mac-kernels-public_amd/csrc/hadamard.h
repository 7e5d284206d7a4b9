// Block Hadamard rotation of 16-element runs held in registers, across the lanes of a wave.
//
// H_G = H4^(x)p / sqrt(G) for G = 4^p, with H4 = [[1,1,1,-1],[1,1,-1,1],[1,-1,1,1],[-1,1,1,1]]
// (roblennon/mac-kernels-public modal/weight_error_app.py:90-98); for G = 2*4^p the extra H2
// factor is the most significant digit.  H4[i][j] = -1 iff i + j == 3, so one radix-4 butterfly
// on (a0..a3) is y_i = S - 2*a_{3-i} with S = a0+a1+a2+a3.
//
// Layout: each lane holds 16 consecutive elements; lane l's run starts at element 16*l within
// its rotation group, so digits 0-1 of the element index are register bits and the higher
// digits are lane bits (G <= 256 keeps a group inside one 16-lane DPP row).
#pragma once
#include "qlin_device.h"

namespace qlin {

__device__ __forceinline__ void bfly4_reg(float& a0, float& a1, float& a2, float& a3) {
    const float s = (a0 + a1) + (a2 + a3);
    const float y0 = s - 2.0f * a3, y1 = s - 2.0f * a2, y2 = s - 2.0f * a1, y3 = s - 2.0f * a0;
    a0 = y0; a1 = y1; a2 = y2; a3 = y3;
}

// Radix-4 stage on register index bits (B, B+1).
template <int B>
__device__ __forceinline__ void stage4_reg(float* v) {
    constexpr int st = 1 << B;
#pragma unroll
    for (int base = 0; base < 16; ++base) {
        if ((base >> B) & 3) continue;
        bfly4_reg(v[base], v[base + st], v[base + 2 * st], v[base + 3 * st]);
    }
}

// Radix-2 stage on register index bit B.
template <int B>
__device__ __forceinline__ void stage2_reg(float* v) {
    constexpr int st = 1 << B;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        if ((i >> B) & 1) continue;
        const float a = v[i], b = v[i + st];
        v[i] = a + b;
        v[i + st] = a - b;
    }
}

// Lane exchanges: DPP quad permutes within quads, ds_swizzle (the LDS crossbar) beyond -- the
// measured best split of the rotation's work between the VALU and the LDS pipe.
template <int MASK>
__device__ __forceinline__ float hx(float v) { return lane_xor<MASK>(v); }

// Radix-4 stage on lane bits (C, C+1): every lane of the 4-lane group computes the same S.
// Lane L forms t = a_L + a_(L^u) and adds the partner pair's t from lane L^2u, so
// S = (a_L + a_(L^u)) + (a_(L^2u) + a_(L^3u)) -- the same rounded sum in all four lanes
// (commutativity).
template <int C>
__device__ __forceinline__ void stage4_lane(float* v) {
    constexpr int u = 1 << C;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const float a = v[i];
        const float p1 = hx<u>(a);
        const float t = a + p1;
        const float s = t + hx<2 * u>(t);
        v[i] = s - 2.0f * hx<3 * u>(a);
    }
}

// Radix-2 stage on lane bit C: lane with the bit clear gets a + b, the other a - b.
template <int C>
__device__ __forceinline__ void stage2_lane(float* v, int lane) {
    constexpr int u = 1 << C;
    const bool upper = (lane >> C) & 1;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const float p = hx<u>(v[i]);
        v[i] = upper ? (p - v[i]) : (v[i] + p);
    }
}

// Unnormalized +-1 Hadamard of size G on the 16-element runs (G in {4,8,...,256}).
template <int G>
__device__ __forceinline__ void hadamard16(float* v, int lane) {
    static_assert(G == 4 || G == 8 || G == 16 || G == 32 || G == 64 || G == 128 || G == 256, "G");
    stage4_reg<0>(v);
    if constexpr (G == 8) stage2_reg<2>(v);
    if constexpr (G >= 16) stage4_reg<2>(v);
    if constexpr (G == 32) stage2_lane<0>(v, lane);
    if constexpr (G >= 64) stage4_lane<0>(v);
    if constexpr (G == 128) stage2_lane<2>(v, lane);
    if constexpr (G == 256) stage4_lane<2>(v);
}

template <int G>
__device__ __forceinline__ float hadamard_norm() {
    if constexpr (G == 4) return 0.5f;
    else if constexpr (G == 16) return 0.25f;
    else if constexpr (G == 64) return 0.125f;
    else if constexpr (G == 256) return 0.0625f;
    else if constexpr (G == 8) return 0.35355339059327373f;
    else if constexpr (G == 32) return 0.17677669529663687f;
    else return 0.088388347648318433f;  // 128
}

// Runtime -> compile-time dispatch for the supported group sizes (0 = identity).
template <typename F>
__host__ inline bool dispatch_group(int g, F&& f) {
    switch (g) {
        case 0: f.template operator()<0>(); return true;
        case 4: f.template operator()<4>(); return true;
        case 8: f.template operator()<8>(); return true;
        case 16: f.template operator()<16>(); return true;
        case 32: f.template operator()<32>(); return true;
        case 64: f.template operator()<64>(); return true;
        case 128: f.template operator()<128>(); return true;
        case 256: f.template operator()<256>(); return true;
        default: return false;
    }
}

}  // namespace qlin
