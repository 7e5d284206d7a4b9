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
// No load sits behind a lane-dependent branch: units past the K range re-read the last unit with
// a zero activation, rows past N re-read row N - 1 (never stored).
#include "qlin_internal.h"

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

template <int MR, int UPL>
__global__ __launch_bounds__(IG_THREADS) void int8_gemv_kernel(Int8GemvArgs a, int KS) {
    constexpr int RW = ig_rows(UPL);
    __shared__ float red[IG_WAVES][MR][RW];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int kq = wave % KS, rg = wave / KS;
    const int units = (int)(a.K / 16);
    const int u0 = (units * kq) / KS, u1 = (units * (kq + 1)) / KS;  // this wave's unit range
    const int groups = IG_WAVES / KS;
    const int64_t n0 = ((int64_t)blockIdx.x * groups + rg) * RW;

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
    // 2. the activation units, as two registers of 8 values each (zero past the range or past M)
    u32x4 xr[MR][UPL], xh[MR][UPL];
#pragma unroll
    for (int m = 0; m < MR; ++m) {
        const f16* xrow = a.x + (int64_t)min(m, a.M - 1) * a.ldx;
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
    // epilogue operands, fetched before the arithmetic
    float cs[RW], bv[RW];
#pragma unroll
    for (int r = 0; r < RW; ++r) {
        const int64_t n = min(n0 + r, a.N - 1);
        cs[r] = load_rt(a.scale, a.scale_dtype, n * a.scale_stride);
        bv[r] = a.bias ? load_rt(a.bias, a.bias_dtype, n) : 0.0f;
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
                const int e = a.xexp ? a.xexp[m] : 0;
                store_rt(a.y, a.y_dtype, m * a.ldy + n, __builtin_ldexpf(acc[m][r], e) * cs[r] + bv[r]);
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

template <int MR, int UPL>
hipError_t launch_ig(const Int8GemvArgs& a, int ks, hipStream_t st) {
    const int64_t rows_per_block = (int64_t)(IG_WAVES / ks) * ig_rows(UPL);
    const dim3 grid((unsigned)((a.N + rows_per_block - 1) / rows_per_block)), block(IG_THREADS);
    hipLaunchKernelGGL((int8_gemv_kernel<MR, UPL>), grid, block, 0, st, a, ks);
    return hipGetLastError();
}

}  // namespace

bool int8_gemv_supported(const Int8GemvArgs& a) {
    int mr, ks, upl;
    return ig_shape(a.M, a.K, mr, ks, upl) && a.ldw % 16 == 0 && (uintptr_t)a.w % 16 == 0 && a.ldx % 8 == 0 &&
           (uintptr_t)a.x % 16 == 0;
}

hipError_t run_int8_gemv(const Int8GemvArgs& a, hipStream_t st) {
    if (a.y_dtype != DT_F32 && a.y_dtype != DT_F16 && a.y_dtype != DT_BF16) return hipErrorInvalidValue;
    int mr, ks, upl;
    if (!int8_gemv_supported(a) || !ig_shape(a.M, a.K, mr, ks, upl)) return hipErrorInvalidValue;
    // (mr, upl) pairs with mr * upl <= 8 (ig_shape never picks another)
    switch (mr * 8 + upl) {
        case 9: return launch_ig<1, 1>(a, ks, st);
        case 10: return launch_ig<1, 2>(a, ks, st);
        case 11: return launch_ig<1, 3>(a, ks, st);
        case 12: return launch_ig<1, 4>(a, ks, st);
        case 17: return launch_ig<2, 1>(a, ks, st);
        case 18: return launch_ig<2, 2>(a, ks, st);
        case 19: return launch_ig<2, 3>(a, ks, st);
        case 20: return launch_ig<2, 4>(a, ks, st);
    }
    return hipErrorInvalidValue;
}

}  // namespace qlin
