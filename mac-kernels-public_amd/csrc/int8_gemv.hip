// INT8 weight-only linear for one or two activation rows: a VALU matrix-vector product.
//
// With so few activation rows an MFMA tile would be mostly padding, and the call is bound by
// streaming the int8 weights from HBM.  So:
//   * each weight row is read with fully coalesced 16-byte loads: lane l of a wave takes the
//     16-value units l, l + 64, l + 128, ... of its part of the row, so one load instruction
//     covers 1 KB of one row; KS waves of a workgroup split a row's K range, and a wave works on
//     RW rows at once, with every one of their loads issued before the first use;
//   * the lane's activation units (the prologue's normalized fp16 rows) are loaded once per
//     workgroup into registers, the same units for every weight row;
//   * the int8 codes become exact fp16 (one byte permute and one packed add per four codes) and
//     v_dot2_f32_f16 accumulates code * activation products in fp32;
//   * lane partials are added with xor shuffles, the KS wave partials through LDS in a fixed order,
//     and y[m, n] = ldexp(sum, xexp[m]) * scale[n] + bias[n] is rounded once.
// Fused prologue (fp16 or bf16 rows, ConvRot group 64, 128 or 256, K <= 8192): instead of reading
// the prologue kernel's output, every workgroup rotates and normalizes the activation rows itself
// with the prologue's arithmetic (hadamard16 on 16-value units, x 1/sqrt(G), E = frexp exponent
// of the row's max |value|, one rounding of x * 2^-E to fp16), so the operand is bit-identical to
// the prologue's and one launch is saved.  The rows are requested before the weights and the
// rotation runs while the weight loads are in flight; the normalized units go to LDS in two
// 16-byte planes (first and second half of every unit), which the dot-product lanes read without
// bank conflicts.
// No load sits behind a lane-dependent branch: units past the K range re-read the last unit with
// a zero activation, rows past N re-read row N - 1 (never stored).
#include "qlin_internal.h"
#include "hadamard.h"

namespace qlin {
namespace {

constexpr int IG_THREADS = 256, IG_WAVES = IG_THREADS / 64;

__device__ __forceinline__ float dot2h(uint32_t a, uint32_t b, float c) {
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2, a), __builtin_bit_cast(f16x2, b), c, false);
}

// 4 int8 codes (one dword) -> 4 exact fp16 (two dwords): bytes q + 128 under a 0x64 exponent
// byte are 1024 + 128 + q exactly, minus 1152.
__device__ __forceinline__ void codes_to_f16(uint32_t w, uint32_t& lo, uint32_t& hi) {
    const uint32_t u = w ^ 0x80808080u;
    const f16x2 off = {(f16)-1152.0f, (f16)-1152.0f};
    lo = __builtin_bit_cast(uint32_t, __builtin_bit_cast(f16x2, __builtin_amdgcn_perm(0x64646464u, u, 0x04010400u)) + off);
    hi = __builtin_bit_cast(uint32_t, __builtin_bit_cast(f16x2, __builtin_amdgcn_perm(0x64646464u, u, 0x04030402u)) + off);
}

// Rows a wave keeps in flight: about eight 16-byte loads per lane.
constexpr int ig_rows(int upl) { return upl >= 3 ? 2 : 8 / upl; }

// Fused-prologue variants: activation dtype and ConvRot group (PRE 0: the prologue kernel's rows).
constexpr int IG_FUSED_MAX_UNITS = 512;  // K <= 8192
template <int PRE> struct ig_pre;
template <> struct ig_pre<1> { using T = f16; static constexpr int G = 64; };
template <> struct ig_pre<2> { using T = f16; static constexpr int G = 128; };
template <> struct ig_pre<3> { using T = f16; static constexpr int G = 256; };
template <> struct ig_pre<4> { using T = bf16_t; static constexpr int G = 64; };
template <> struct ig_pre<5> { using T = bf16_t; static constexpr int G = 128; };
template <> struct ig_pre<6> { using T = bf16_t; static constexpr int G = 256; };

template <int MR, int UPL, int PRE>
__global__ __launch_bounds__(IG_THREADS) void int8_gemv_kernel(Int8GemvArgs a, int KS) {
    constexpr int RW = ig_rows(UPL);
    constexpr bool FUSED = PRE > 0;
    __shared__ float red[IG_WAVES][MR][RW];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int kq = wave % KS, rg = wave / KS;
    const int units = (int)(a.K / 16);
    const int u0 = (units * kq) / KS, u1 = (units * (kq + 1)) / KS;  // this wave's unit range
    const int groups = IG_WAVES / KS;
    const int64_t n0 = ((int64_t)blockIdx.x * groups + rg) * RW;

    // 0. fused prologue: each thread's 16-value units of the raw rows (thread t: units t, t + 256),
    //    requested before the weights so that waiting for them leaves the weight loads in flight
    constexpr int SLOTS = FUSED ? (MR == 1 ? 2 : 1) : 1;  // K <= 8192 (one row) or 4096 (two)
    __shared__ __attribute__((aligned(16))) u32x4 xs[FUSED ? MR : 1][2][FUSED ? IG_FUSED_MAX_UNITS / (MR == 1 ? 1 : 2) : 1];
    __shared__ int xe[MR];
    __shared__ float xmax[IG_WAVES][MR];
    u32x4 raw[FUSED ? MR : 1][SLOTS][2];
    if constexpr (FUSED) {
#pragma unroll
        for (int m = 0; m < MR; ++m) {
            const auto* xrow = reinterpret_cast<const typename ig_pre<PRE>::T*>(a.xraw) + (int64_t)min(m, (int)a.M - 1) * a.ldx;
#pragma unroll
            for (int s = 0; s < SLOTS; ++s) {
                const int u = min(tid + IG_THREADS * s, units - 1);  // past the row: a valid unit, not stored
                const u32x4* p = reinterpret_cast<const u32x4*>(xrow + 16 * (int64_t)u);
                raw[m][s][0] = p[0];
                raw[m][s][1] = p[1];
            }
        }
        __builtin_amdgcn_sched_barrier(0);
    }

    // 1. the weight units of this wave's RW rows
    u32x4 wr[RW][UPL];
#pragma unroll
    for (int r = 0; r < RW; ++r) {
        const int8_t* row = a.w + min(n0 + r, a.N - 1) * a.ldw;
#pragma unroll
        for (int i = 0; i < UPL; ++i) {
            const int u = min(u0 + lane + 64 * i, u1 - 1);
            wr[r][i] = *reinterpret_cast<const u32x4*>(row + 16 * (int64_t)u);
        }
    }
    // epilogue operands as raw bits, requested with the weights: a value conversion at the load
    // would wait for every load in flight, a memory round trip after the weights have arrived
    uint32_t csb[RW], bvb[RW];
#pragma unroll
    for (int r = 0; r < RW; ++r) {
        const int64_t n = min(n0 + r, a.N - 1);
        csb[r] = load_bits_rt(a.scale, a.scale_dtype, n * a.scale_stride);
        bvb[r] = a.bias ? load_bits_rt(a.bias, a.bias_dtype, n) : 0u;
    }
    // 2. the activation units, as two registers of 8 values each (zero past the range or past M)
    u32x4 xr[MR][UPL], xh[MR][UPL];
    if constexpr (FUSED) {
        __builtin_amdgcn_sched_barrier(0);
        using T = typename ig_pre<PRE>::T;
        constexpr int G = ig_pre<PRE>::G;
        // rotate (16-value units on lane bits, as the prologue kernel), scale by 1/sqrt(G), row max
        float v[MR][SLOTS][16];
        float amax[MR];
#pragma unroll
        for (int m = 0; m < MR; ++m) {
            amax[m] = 0.0f;
#pragma unroll
            for (int s = 0; s < SLOTS; ++s) {
                const uint32_t wd[8] = {raw[m][s][0].x, raw[m][s][0].y, raw[m][s][0].z, raw[m][s][0].w,
                                        raw[m][s][1].x, raw[m][s][1].y, raw[m][s][1].z, raw[m][s][1].w};
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    T lo, hi;
                    const uint16_t l16 = (uint16_t)(wd[i] & 0xFFFFu), h16 = (uint16_t)(wd[i] >> 16);
                    __builtin_memcpy(&lo, &l16, 2);
                    __builtin_memcpy(&hi, &h16, 2);
                    v[m][s][2 * i] = dtype_traits<T>::to_f32(lo);
                    v[m][s][2 * i + 1] = dtype_traits<T>::to_f32(hi);
                }
                hadamard16<G>(v[m][s], lane);
                const float nrm = hadamard_norm<G>();
                const bool in = tid + IG_THREADS * s < units;
#pragma unroll
                for (int i = 0; i < 16; ++i) {
                    v[m][s][i] *= nrm;
                    if (in) amax[m] = fmaxf(amax[m], fabsf(v[m][s][i]));
                }
            }
            amax[m] = wave_max(amax[m]);
            if (lane == 0) xmax[wave][m] = amax[m];
        }
        lds_barrier();
#pragma unroll
        for (int m = 0; m < MR; ++m) {
            float mx = xmax[0][m];
#pragma unroll
            for (int w = 1; w < IG_WAVES; ++w) mx = fmaxf(mx, xmax[w][m]);
            const int E = frexp_exp(mx);
            if (tid == 0) xe[m] = E;
#pragma unroll
            for (int s = 0; s < SLOTS; ++s) {
                const int u = tid + IG_THREADS * s;
                if (u >= units) continue;
                uint32_t h[8];
#pragma unroll
                for (int i = 0; i < 8; ++i)
                    h[i] = (uint32_t)__builtin_bit_cast(uint16_t, (f16)__builtin_ldexpf(v[m][s][2 * i], -E)) |
                           ((uint32_t)__builtin_bit_cast(uint16_t, (f16)__builtin_ldexpf(v[m][s][2 * i + 1], -E)) << 16);
                xs[m][0][u] = u32x4{h[0], h[1], h[2], h[3]};
                xs[m][1][u] = u32x4{h[4], h[5], h[6], h[7]};
            }
        }
        lds_barrier();
#pragma unroll
        for (int m = 0; m < MR; ++m)
#pragma unroll
            for (int i = 0; i < UPL; ++i) {
                const int u = u0 + lane + 64 * i;
                const int uc = min(u, u1 - 1);
                const u32x4 v0 = xs[m][0][uc], v1 = xs[m][1][uc];
                const bool ok = u < u1 && m < a.M;
                xr[m][i] = ok ? v0 : u32x4{0u, 0u, 0u, 0u};
                xh[m][i] = ok ? v1 : u32x4{0u, 0u, 0u, 0u};
            }
    } else {
#pragma unroll
        for (int m = 0; m < MR; ++m) {
            const f16* xrow = a.x + (int64_t)min(m, (int)a.M - 1) * a.ldx;
#pragma unroll
            for (int i = 0; i < UPL; ++i) {
                const int u = u0 + lane + 64 * i;
                const u32x4* p = reinterpret_cast<const u32x4*>(xrow + 16 * (int64_t)min(u, u1 - 1));
                const u32x4 v0 = p[0], v1 = p[1];
                const bool ok = u < u1 && m < a.M;
                xr[m][i] = ok ? v0 : u32x4{0u, 0u, 0u, 0u};
                xh[m][i] = ok ? v1 : u32x4{0u, 0u, 0u, 0u};
            }
        }
    }

    // 3. code x activation dot products, fp32
    float acc[MR][RW];
#pragma unroll
    for (int m = 0; m < MR; ++m)
#pragma unroll
        for (int r = 0; r < RW; ++r) acc[m][r] = 0.0f;
#pragma unroll
    for (int r = 0; r < RW; ++r)
#pragma unroll
        for (int i = 0; i < UPL; ++i) {
            uint32_t q[8];
            codes_to_f16(wr[r][i].x, q[0], q[1]);
            codes_to_f16(wr[r][i].y, q[2], q[3]);
            codes_to_f16(wr[r][i].z, q[4], q[5]);
            codes_to_f16(wr[r][i].w, q[6], q[7]);
#pragma unroll
            for (int m = 0; m < MR; ++m) {
                float s = acc[m][r];
                s = dot2h(q[0], xr[m][i].x, s);
                s = dot2h(q[1], xr[m][i].y, s);
                s = dot2h(q[2], xr[m][i].z, s);
                s = dot2h(q[3], xr[m][i].w, s);
                s = dot2h(q[4], xh[m][i].x, s);
                s = dot2h(q[5], xh[m][i].y, s);
                s = dot2h(q[6], xh[m][i].z, s);
                s = dot2h(q[7], xh[m][i].w, s);
                acc[m][r] = s;
            }
        }
    // 4. lane partials, then the KS wave partials in order
#pragma unroll
    for (int m = 0; m < MR; ++m)
#pragma unroll
        for (int r = 0; r < RW; ++r) {
            float v = acc[m][r];
#pragma unroll
            for (int s = 1; s < 64; s <<= 1) v += __shfl_xor(v, s, 64);
            acc[m][r] = v;
        }
    if (KS > 1) {
        if (lane == 0) {
#pragma unroll
            for (int m = 0; m < MR; ++m)
#pragma unroll
                for (int r = 0; r < RW; ++r) red[wave][m][r] = acc[m][r];
        }
        __syncthreads();
        if (kq != 0) return;
#pragma unroll
        for (int m = 0; m < MR; ++m)
#pragma unroll
            for (int r = 0; r < RW; ++r) {
                float v = red[wave][m][r];
                for (int j = 1; j < KS; ++j) v += red[wave + j][m][r];
                acc[m][r] = v;
            }
    }
    // 5. lanes (m, r) of the first wave of the row group store
#pragma unroll
    for (int m = 0; m < MR; ++m)
#pragma unroll
        for (int r = 0; r < RW; ++r) {
            const int64_t n = n0 + r;
            if (lane == m * RW + r && m < a.M && n < a.N) {
                const int e = FUSED ? xe[m] : a.xexp ? a.xexp[m] : 0;
                const float bv = a.bias ? bits_to_f32_rt(bvb[r], a.bias_dtype) : 0.0f;
                store_rt(a.y, a.y_dtype, m * a.ldy + n,
                         __builtin_ldexpf(acc[m][r], e) * bits_to_f32_rt(csb[r], a.scale_dtype) + bv);
            }
        }
}

// waves per row and units per lane for K: the fewest waves per row with at most four units per
// lane and at most eight activation units per lane in registers
bool ig_shape(int64_t M, int64_t K, int& mr, int& ks, int& upl) {
    if (M < 1 || M > 2 || K % 16 || K < 1024) return false;
    mr = (int)M;
    const int64_t units = K / 16;
    for (int k : {1, 2, 4}) {
        const int64_t u = ((units + k - 1) / k + 63) / 64;  // units per lane of the longest wave range
        if (u <= 4 && mr * u <= 8) {
            ks = k;
            upl = (int)u;
            return true;
        }
    }
    return false;
}

template <int MR, int UPL, int PRE>
hipError_t launch_ig(const Int8GemvArgs& a, int ks, hipStream_t st) {
    const int64_t rows_per_block = (int64_t)(IG_WAVES / ks) * ig_rows(UPL);
    const dim3 grid((unsigned)((a.N + rows_per_block - 1) / rows_per_block)), block(IG_THREADS);
    hipLaunchKernelGGL((int8_gemv_kernel<MR, UPL, PRE>), grid, block, 0, st, a, ks);
    return hipGetLastError();
}

// The fused-prologue variant for these raw rows, 0 when the prologue kernel must run first.
int ig_fused_pre(const Int8GemvArgs& a) {
    if (!a.xraw || (a.x_dtype != DT_F16 && a.x_dtype != DT_BF16)) return 0;
    if (a.G != 64 && a.G != 128 && a.G != 256) return 0;
    if (a.K / 16 > IG_FUSED_MAX_UNITS / a.M || a.ldx % 8 || (uintptr_t)a.xraw % 16) return 0;
    const int g = a.G == 64 ? 1 : a.G == 128 ? 2 : 3;
    return a.x_dtype == DT_F16 ? g : g + 3;
}

template <int MR, int UPL>
hipError_t launch_ig_pre(const Int8GemvArgs& a, int ks, int pre, hipStream_t st) {
    switch (pre) {
        case 0: return launch_ig<MR, UPL, 0>(a, ks, st);
        case 1: return launch_ig<MR, UPL, 1>(a, ks, st);
        case 2: return launch_ig<MR, UPL, 2>(a, ks, st);
        case 3: return launch_ig<MR, UPL, 3>(a, ks, st);
        case 4: return launch_ig<MR, UPL, 4>(a, ks, st);
        case 5: return launch_ig<MR, UPL, 5>(a, ks, st);
        case 6: return launch_ig<MR, UPL, 6>(a, ks, st);
    }
    return hipErrorInvalidValue;
}

}  // namespace

bool int8_gemv_supported(const Int8GemvArgs& a) {
    int mr, ks, upl;
    if (!ig_shape(a.M, a.K, mr, ks, upl) || a.ldw % 16 || (uintptr_t)a.w % 16) return false;
    if (a.xraw) return ig_fused_pre(a) > 0;
    return a.ldx % 8 == 0 && (uintptr_t)a.x % 16 == 0;
}

hipError_t run_int8_gemv(const Int8GemvArgs& a, hipStream_t st) {
    if (a.y_dtype != DT_F32 && a.y_dtype != DT_F16 && a.y_dtype != DT_BF16) return hipErrorInvalidValue;
    int mr, ks, upl;
    if (!int8_gemv_supported(a) || !ig_shape(a.M, a.K, mr, ks, upl)) return hipErrorInvalidValue;
    const int pre = a.xraw ? ig_fused_pre(a) : 0;
    // (mr, upl) pairs with mr * upl <= 8 (ig_shape never picks another)
    switch (mr * 8 + upl) {
        case 9: return launch_ig_pre<1, 1>(a, ks, pre, st);
        case 10: return launch_ig_pre<1, 2>(a, ks, pre, st);
        case 11: return launch_ig_pre<1, 3>(a, ks, pre, st);
        case 12: return launch_ig_pre<1, 4>(a, ks, pre, st);
        case 17: return launch_ig_pre<2, 1>(a, ks, pre, st);
        case 18: return launch_ig_pre<2, 2>(a, ks, pre, st);
        case 19: return launch_ig_pre<2, 3>(a, ks, pre, st);
        case 20: return launch_ig_pre<2, 4>(a, ks, pre, st);
    }
    return hipErrorInvalidValue;
}

}  // namespace qlin
