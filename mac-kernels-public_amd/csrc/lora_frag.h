// LoRA operand fragments for v_mfma_f32_32x32x16_bf16: raw 8-value loads of f32 / f16 / bf16 rows and
// the exact bf16 split of every operand that is not already bf16 (hi = bf16(v), lo = bf16(v - hi);
// bf16 x bf16 products are exact in fp32, hi + lo carries 16 significand bits, the lo x lo term is
// dropped).  Shared by the LoRA kernels (lora.hip) and the GEMM epilogues that add the LoRA term of
// their own output tile (gemm_f16.hip, gemm_i8.hip).
#pragma once
#include <utility>

#include "qlin_internal.h"

namespace qlin {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

__device__ __forceinline__ __bf16 to_bf16(float f) { return __builtin_bit_cast(__bf16, f32_to_bf16_bits(f)); }

// hi = bf16(v), lo = bf16(v - hi) (v - hi is exact in fp32)
__device__ __forceinline__ void split8(const float* v, bf16x8& hi, bf16x8& lo) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const uint16_t hb = f32_to_bf16_bits(v[i]);
        hi[i] = __builtin_bit_cast(__bf16, hb);
        lo[i] = to_bf16(v[i] - bf16_bits_to_f32(hb));
    }
}

// Raw storage of 8 consecutive values of one operand (16 bytes for f16/bf16, 32 for f32), loaded
// ahead of use so that several steps of loads are in flight.
template <int DT>
struct Raw8 {
    u32x4 v[DT == DT_F32 ? 2 : 1];
};

// VEC (16-byte loads) requires cols % 8 == 0 and cols >= 8, so with k a multiple of 8 a piece is
// either wholly inside the row or wholly past its end: the load is issued unconditionally from a
// clamped column, and the caller zeroes a past-the-end piece when it uses it (a load behind a
// lane-dependent branch, or a select right after it, would be waited for on the spot).
template <int DT, bool VEC>
__device__ __forceinline__ Raw8<DT> raw_load(const void* base, int64_t ld, int64_t row, int64_t k, int64_t cols) {
    Raw8<DT> r;
    if constexpr (VEC) {
        const int64_t kc = min(k, cols - 8);
        if constexpr (DT == DT_F32) {
            const u32x4* p = reinterpret_cast<const u32x4*>(reinterpret_cast<const float*>(base) + row * ld + kc);
            r.v[0] = p[0];
            r.v[1] = p[1];
        } else {
            r.v[0] = *reinterpret_cast<const u32x4*>(reinterpret_cast<const uint16_t*>(base) + row * ld + kc);
        }
        return r;  // a piece past the end holds the row's last 8 values: the caller zeroes it at use
    } else {
    float f[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) f[i] = k + i < cols ? load_rt(base, DT, row * ld + k + i) : 0.0f;
    if constexpr (DT == DT_F32) {
        r.v[0] = u32x4{__float_as_uint(f[0]), __float_as_uint(f[1]), __float_as_uint(f[2]), __float_as_uint(f[3])};
        r.v[1] = u32x4{__float_as_uint(f[4]), __float_as_uint(f[5]), __float_as_uint(f[6]), __float_as_uint(f[7])};
    } else {
        uint32_t w[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t lo = DT == DT_F16 ? (uint32_t)__builtin_bit_cast(uint16_t, (f16)f[2 * i])
                                             : (uint32_t)f32_to_bf16_bits(f[2 * i]);
            const uint32_t hi = DT == DT_F16 ? (uint32_t)__builtin_bit_cast(uint16_t, (f16)f[2 * i + 1])
                                             : (uint32_t)f32_to_bf16_bits(f[2 * i + 1]);
            w[i] = lo | (hi << 16);  // the loaded values are exact in the storage type
        }
        r.v[0] = u32x4{w[0], w[1], w[2], w[3]};
    }
    return r;
    }
}

template <int DT>
__device__ __forceinline__ Raw8<DT> zero_unless(const Raw8<DT>& r, bool keep) {
    Raw8<DT> z;
#pragma unroll
    for (int j = 0; j < (DT == DT_F32 ? 2 : 1); ++j) z.v[j] = keep ? r.v[j] : u32x4{0u, 0u, 0u, 0u};
    return z;
}

template <int DT>
__device__ __forceinline__ void raw_to_f32(const Raw8<DT>& r, float* f) {
    if constexpr (DT == DT_F32) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            f[i] = __uint_as_float(r.v[0][i]);
            f[4 + i] = __uint_as_float(r.v[1][i]);
        }
    } else {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            f[2 * i] = bits_to_f32_rt(r.v[0][i] & 0xFFFFu, DT);
            f[2 * i + 1] = bits_to_f32_rt(r.v[0][i] >> 16, DT);
        }
    }
}

// acc += A . B over one 16-value step from raw loads; bf16 operands are used as loaded.
template <int DA, int DB>
__device__ __forceinline__ void mfma_raw(const Raw8<DA>& ra, const Raw8<DB>& rb, f32x16& acc) {
    constexpr bool SA = DA != DT_BF16, SB = DB != DT_BF16;
    bf16x8 ah, al, bh, bl;
    if constexpr (SA) {
        float f[8];
        raw_to_f32(ra, f);
        split8(f, ah, al);
    } else {
        ah = __builtin_bit_cast(bf16x8, ra.v[0]);
    }
    if constexpr (SB) {
        float f[8];
        raw_to_f32(rb, f);
        split8(f, bh, bl);
    } else {
        bh = __builtin_bit_cast(bf16x8, rb.v[0]);
    }
    acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ah, bh, acc, 0, 0, 0);
    if constexpr (SA) acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(al, bh, acc, 0, 0, 0);
    if constexpr (SB) acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ah, bl, acc, 0, 0, 0);
}

// LoRA term of a GEMM workgroup's BMT x BNT output tile, added by its waves to accumulators that
// already hold their fp32 base values (after bias).  The whole rank (R <= RC) is staged at once: all
// NT threads load the tile's t rows [BMT x RC] (fp32) and up rows [BNT x RC] together (every load in
// flight at once, zeros past R; with PARTS, t's K-split partials summed in split order and scaled
// by 2^t_exp[m] as L asks).  t is multiplied by L.scale and split into bf16 hi and lo on its
// way into LDS, once per workgroup; up goes in as loaded.  Each wave then takes its TJ column blocks
// in turn: it reads (and, for f16 / f32, splits) the up fragments of the block once, and runs the
// bf16 MFMAs hi.hi, lo.hi (and hi.lo) of (scale t) . up^T for each of its TI row blocks straight into
// acc[i][j] (fp32 values, or their bits in int32 registers), so the base value is the MFMAs'
// accumulator input.  A wave's sub-tile (i, j) covers tile rows wr0 + 32 i .. + 31 and columns
// wc0 + 32 j .. + 31, in the MFMA C layout (lane l, register r: row 8 (r / 4) + 4 (l / 32) + r % 4,
// column l % 32).  LDS rows are unpadded; their 16-byte chunks are XOR-swizzled (lora_chunk) so the
// 32 rows of a fragment read spread over the banks.  Requires 8 <= R <= RC, R % 8 == 0 and 16-byte
// aligned t and up rows (t row stride R); lds must hold lora_lds_bytes<DU, BMT, BNT, RC>().  No loop
// here has a run-time trip count, so the caller's accumulators stay in registers.  Starts and ends
// with a workgroup barrier.
template <int DU, int BMT, int BNT, int RC>
constexpr int lora_lds_bytes() {
    return BMT * RC * 4 + BNT * RC * (DU == DT_F32 ? 4 : 2);  // t as bf16 hi + lo, up as stored
}

// Ranks a GEMM epilogue with `lds_bytes` of LDS (less what it keeps for itself) can stage at once.
template <int DU, int BMT, int BNT>
constexpr int lora_max_rank(int lds_bytes) {
    return lora_lds_bytes<DU, BMT, BNT, 64>() <= lds_bytes ? 64 : lora_lds_bytes<DU, BMT, BNT, 32>() <= lds_bytes ? 32 : 0;
}

// Byte offset of 16-byte chunk c of row `row` in an unpadded LDS array of BPR-byte rows: the chunk
// index is XOR-ed with the row's position among the rows that share a 128-byte bank line, so the
// same chunk of 8 consecutive rows lands on 8 different 16-byte bank groups.
template <int BPR>
__device__ __forceinline__ int lora_chunk(int row, int c) {
    constexpr int CPR = BPR / 16, RPL = CPR >= 8 ? 1 : 8 / CPR, SW = CPR >= 8 ? 8 : CPR;
    static_assert(BPR % 16 == 0 && CPR >= 2, "rows of whole 16-byte chunks");
    return row * BPR + 16 * (c ^ ((row / RPL) % SW));
}

template <int DU, int BMT, int BNT, int RC, int NT, int TI, int TJ, bool PARTS, typename AccT>
__device__ __forceinline__ void lora_tile_epilogue(const LoraTile& L, uint8_t* lds, int64_t m0, int64_t n0, int64_t M,
                                                   int64_t N, int wr0, int wc0, int tid, int lane, AccT (&acc)[TI][TJ]) {
    static_assert(sizeof(AccT) == sizeof(f32x16), "32 x 32 accumulators: fp32 values or their int32 bits");
    static_assert(RC % 16 == 0, "whole MFMA steps");
    constexpr int ES = DU == DT_F32 ? 4 : 2, UPP = 16 / ES;   // up element size, elements per 16 bytes
    constexpr int TBPR = RC * 2, UBPR = RC * ES;             // bytes per LDS row: t hi (or lo), up
    constexpr int TP = BMT * RC / 8 / NT, UP = BNT * RC / UPP / NT;  // pieces per thread: 8 t, 16 B of up
    static_assert(TP * 8 * NT == BMT * RC && UP * UPP * NT == BNT * RC, "rank must split into whole rounds");
    constexpr bool SU = DU != DT_BF16;  // up is split into hi and lo too
    uint8_t* th = lds;
    uint8_t* tl = lds + BMT * TBPR;
    uint8_t* us = lds + 2 * BMT * TBPR;
    const int r32 = lane & 31, h = lane >> 5;
    float tv[TP][8];
    u32x4 uv[UP];
    const int64_t ldt = L.ld_t ? L.ld_t : L.R;
#pragma unroll
    for (int i = 0; i < TP; ++i) {
        const int p = tid + NT * i, row = p / (RC / 8), c = 8 * (p % (RC / 8));
        const int64_t m = min(m0 + row, M - 1), k = min<int64_t>(c, L.R - 8);
        const float* tp = L.t + m * ldt + k;
        const u32x4 a0 = *reinterpret_cast<const u32x4*>(tp), a1 = *reinterpret_cast<const u32x4*>(tp + 4);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            tv[i][e] = __uint_as_float(a0[e]);
            tv[i][4 + e] = __uint_as_float(a1[e]);
        }
        if constexpr (PARTS) {
            // K-split partials 1 .. t_parts - 1 of t, added in split order, then 2^t_exp[m]
            for (int sp = 1; sp < L.t_parts; ++sp) {
                const u32x4 b0 = *reinterpret_cast<const u32x4*>(tp + sp * L.t_stride);
                const u32x4 b1 = *reinterpret_cast<const u32x4*>(tp + sp * L.t_stride + 4);
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    tv[i][e] += __uint_as_float(b0[e]);
                    tv[i][4 + e] += __uint_as_float(b1[e]);
                }
            }
            if (L.t_exp) {
                const int e = L.t_exp[m];
#pragma unroll
                for (int q = 0; q < 8; ++q) tv[i][q] = __builtin_ldexpf(tv[i][q], e);
            }
        }
    }
#pragma unroll
    for (int i = 0; i < UP; ++i) {
        const int p = tid + NT * i, row = p / (RC / UPP), c = UPP * (p % (RC / UPP));
        const int64_t n = min(n0 + row, N - 1), k = min<int64_t>(c, L.R - UPP);
        uv[i] = *reinterpret_cast<const u32x4*>(reinterpret_cast<const uint8_t*>(L.up) + (n * L.ld_up + k) * ES);
    }
    __syncthreads();  // every wave is done with the LDS the staging overwrites
#pragma unroll
    for (int i = 0; i < TP; ++i) {
        const int p = tid + NT * i, row = p / (RC / 8), c = 8 * (p % (RC / 8));
        float v[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) v[e] = c < L.R ? tv[i][e] * L.scale : 0.f;
        bf16x8 hi, lo;
        split8(v, hi, lo);
        *reinterpret_cast<bf16x8*>(th + lora_chunk<TBPR>(row, c / 8)) = hi;
        *reinterpret_cast<bf16x8*>(tl + lora_chunk<TBPR>(row, c / 8)) = lo;
    }
#pragma unroll
    for (int i = 0; i < UP; ++i) {
        const int p = tid + NT * i, row = p / (RC / UPP), c = UPP * (p % (RC / UPP));
        *reinterpret_cast<u32x4*>(us + lora_chunk<UBPR>(row, c / UPP)) = c < L.R ? uv[i] : u32x4{0u, 0u, 0u, 0u};
    }
    __syncthreads();
    // compile-time block indices, so that every access to the caller's accumulators is constant
    auto col = [&]<int J>() {
        __builtin_amdgcn_sched_barrier(0);
        const int un = wc0 + 32 * J + r32;
        bf16x8 bh[RC / 16], bl[RC / 16];
#pragma unroll
        for (int q = 0; q < RC / 16; ++q) {
            Raw8<DU> rb;
            if constexpr (DU == DT_F32) {
                rb.v[0] = *reinterpret_cast<const u32x4*>(us + lora_chunk<UBPR>(un, 4 * q + 2 * h));
                rb.v[1] = *reinterpret_cast<const u32x4*>(us + lora_chunk<UBPR>(un, 4 * q + 2 * h + 1));
            } else {
                rb.v[0] = *reinterpret_cast<const u32x4*>(us + lora_chunk<UBPR>(un, 2 * q + h));
            }
            if constexpr (SU) {
                float f[8];
                raw_to_f32(rb, f);
                split8(f, bh[q], bl[q]);
            } else {
                bh[q] = __builtin_bit_cast(bf16x8, rb.v[0]);
            }
        }
        auto row = [&]<int I>() {
            __builtin_amdgcn_sched_barrier(0);
            const int tm = wr0 + 32 * I + r32;
            f32x16 c = __builtin_bit_cast(f32x16, acc[I][J]);
#pragma unroll
            for (int q = 0; q < RC / 16; ++q) {
                const bf16x8 ah = *reinterpret_cast<const bf16x8*>(th + lora_chunk<TBPR>(tm, 2 * q + h));
                const bf16x8 al = *reinterpret_cast<const bf16x8*>(tl + lora_chunk<TBPR>(tm, 2 * q + h));
                c = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ah, bh[q], c, 0, 0, 0);
                c = __builtin_amdgcn_mfma_f32_32x32x16_bf16(al, bh[q], c, 0, 0, 0);
                if constexpr (SU) c = __builtin_amdgcn_mfma_f32_32x32x16_bf16(ah, bl[q], c, 0, 0, 0);
            }
            acc[I][J] = __builtin_bit_cast(AccT, c);
        };
        [&]<int... I>(std::integer_sequence<int, I...>) {
            (row.template operator()<I>(), ...);
        }(std::make_integer_sequence<int, TI>{});
    };
    [&]<int... J>(std::integer_sequence<int, J...>) {
        (col.template operator()<J>(), ...);
    }(std::make_integer_sequence<int, TJ>{});
    __syncthreads();  // LDS free for the caller's staging
}

// The same for ranks up to 2 RC: ranks 0 .. RC - 1 first, then the rest, each pass staged on its
// own; the second pass continues the MFMA chain of the first on the same accumulators, so the
// terms are added in rank order.  Requires R % 8 == 0 and 8 <= R <= 2 RC.
template <int DU, int BMT, int BNT, int RC, int NT, int TI, int TJ, bool PARTS = false, typename AccT>
__device__ __forceinline__ void lora_tile_epilogue_ranks(const LoraTile& L, uint8_t* lds, int64_t m0, int64_t n0,
                                                         int64_t M, int64_t N, int wr0, int wc0, int tid, int lane,
                                                         AccT (&acc)[TI][TJ]) {
    LoraTile p = L;
    p.ld_t = L.R;
    p.R = L.R < RC ? L.R : RC;
    lora_tile_epilogue<DU, BMT, BNT, RC, NT, TI, TJ, PARTS>(p, lds, m0, n0, M, N, wr0, wc0, tid, lane, acc);
    if (L.R > RC) {
        p.t = L.t + RC;
        p.up = reinterpret_cast<const uint8_t*>(L.up) + RC * (DU == DT_F32 ? 4 : 2);
        p.R = L.R - RC;
        lora_tile_epilogue<DU, BMT, BNT, RC, NT, TI, TJ, PARTS>(p, lds, m0, n0, M, N, wr0, wc0, tid, lane, acc);
    }
}

}  // namespace qlin
