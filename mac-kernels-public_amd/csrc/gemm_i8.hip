// A8 linear over AsymW4A8Int8 weights on the int8 MFMA (v_mfma_i32_16x16x64_i8).
//
// Activations arrive as the prologue's per-token int8 rows xq[m,:] with fp32 scales sx[m]
// (quantize_int8_rowwise of the rotated activation).  The packed weight tile is decoded in the
// load stage to the int8 grid the reference's decoder defines (roblennon/mac-kernels-public
// modal/weight_error_app.py:326-337):
//     level = codebook[code] or (code - 2^(bits-1)),  w8 = clamp(rne(level * s_rel[n, k/gs]), -127, 127)
// computed in fp32 (one rounding of the product, then round-half-even), so the int32 accumulators
// equal the exact integer products.  Epilogue: y = (f32(acc) * sx[m]) * s_channel[n] + bias[n].
// Tile 128 x 128 x 128 (int8), 256 threads = 2x2 waves of 64x64, LDS double-buffered through
// registers.  4-bit codes: nibble plane [N, K/2]; 6-bit: the same plane plus a 2-bit plane
// [N, K/4] (byte j holds bits 4-5 of codes 4j..4j+3).
#include "qlin_internal.h"

namespace qlin {
namespace {

constexpr int BM = 128, BN = 128, BK = 128, LDB = BK + 16;  // LDS row stride in bytes

struct Regs {
    u32x4 a[4];  // 64 int8 of one activation row half
    u32x4 b[4];  // 64 decoded int8 of one weight row half
};

template <typename TSrel>
__device__ __forceinline__ float srel_at(const void* s, int64_t i) {
    if constexpr (sizeof(TSrel) == 1) return e4m3_to_f32(((const uint8_t*)s)[i]);
    else return load_f((const TSrel*)s + i);
}

// Decode 8 codes packed as nibbles in w (code i = nibble i) [+ 2-bit high parts in hi8, bits
// 2i..2i+1] to the int8 grid; returns two dwords of int8.
template <int BITS, bool CB>
__device__ __forceinline__ void decode8_i8(uint32_t w, uint32_t hi8, float s, const float* cb, uint32_t& o0,
                                           uint32_t& o1) {
    int8_t r[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        int code = (w >> (4 * i)) & 0xF;
        if constexpr (BITS == 6) code |= ((hi8 >> (2 * i)) & 3) << 4;
        float level;
        if constexpr (CB) level = cb[code];
        else level = (float)(code - (1 << (BITS - 1)));
        float t = __builtin_rintf(level * s);
        t = fminf(fmaxf(t, -127.0f), 127.0f);
        r[i] = (int8_t)(int)t;
    }
    o0 = (uint32_t)(uint8_t)r[0] | ((uint32_t)(uint8_t)r[1] << 8) | ((uint32_t)(uint8_t)r[2] << 16) |
         ((uint32_t)(uint8_t)r[3] << 24);
    o1 = (uint32_t)(uint8_t)r[4] | ((uint32_t)(uint8_t)r[5] << 8) | ((uint32_t)(uint8_t)r[6] << 16) |
         ((uint32_t)(uint8_t)r[7] << 24);
}

template <int BITS, bool CB, typename TSrel>
__device__ __forceinline__ void load_tiles(const GemmI8Args& p, const float* cb, int64_t m0, int64_t n0, int64_t k0,
                                           int tid, bool vec_ok, Regs& R) {
    const int r = tid >> 1, h = tid & 1;
    // A: 64 int8 of row m0 + r from column k0 + 64h
    {
        const int64_t m = m0 + r, k = k0 + 64 * h;
        if (m < p.M && vec_ok && k + 64 <= p.K) {
            const u32x4* src = reinterpret_cast<const u32x4*>(p.xq + m * p.ldx + k);
#pragma unroll
            for (int i = 0; i < 4; ++i) R.a[i] = src[i];
        } else {
            uint32_t w[16];
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                uint32_t v = 0;
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    const int64_t kk = k + 4 * i + t;
                    if (m < p.M && kk < p.K) v |= (uint32_t)(uint8_t)p.xq[m * p.ldx + kk] << (8 * t);
                }
                w[i] = v;
            }
#pragma unroll
            for (int i = 0; i < 4; ++i) R.a[i] = u32x4{w[4 * i], w[4 * i + 1], w[4 * i + 2], w[4 * i + 3]};
        }
    }
    // B: 64 decoded values of weight row n0 + r from column k0 + 64h (K % 64 == 0 is required).
    {
        const int64_t n = n0 + r, k = k0 + 64 * h;
        if (n < p.N && k < p.K) {
            const uint8_t* row = p.q + n * p.ldq;
            const u32x4* lo = reinterpret_cast<const u32x4*>(row + k / 2);
            const u32x4 l0 = lo[0], l1 = lo[1];
            uint32_t nib[8] = {l0.x, l0.y, l0.z, l0.w, l1.x, l1.y, l1.z, l1.w};
            uint32_t hi[4] = {0u, 0u, 0u, 0u};
            if constexpr (BITS == 6) {
                const u32x4 hv = *reinterpret_cast<const u32x4*>(row + p.K / 2 + k / 4);
                hi[0] = hv.x; hi[1] = hv.y; hi[2] = hv.z; hi[3] = hv.w;
            }
            const int gs = p.group_size;
            uint32_t out[16];
#pragma unroll
            for (int c = 0; c < 8; ++c) {  // 8 codes per dword of the nibble plane
                const int64_t kc = k + 8 * c;
                const float s = srel_at<TSrel>(p.s_rel, n * p.ld_srel + kc / gs);
                const uint32_t h8 = (BITS == 6) ? ((hi[c >> 1] >> (16 * (c & 1))) & 0xFFFFu) : 0u;
                decode8_i8<BITS, CB>(nib[c], h8, s, cb, out[2 * c], out[2 * c + 1]);
            }
#pragma unroll
            for (int i = 0; i < 4; ++i) R.b[i] = u32x4{out[4 * i], out[4 * i + 1], out[4 * i + 2], out[4 * i + 3]};
        } else {
#pragma unroll
            for (int i = 0; i < 4; ++i) R.b[i] = u32x4{0u, 0u, 0u, 0u};
        }
    }
}

__device__ __forceinline__ void store_regs(uint8_t* As, uint8_t* Bs, int tid, const Regs& R) {
    const int r = tid >> 1, h = tid & 1;
    u32x4* pa = reinterpret_cast<u32x4*>(As + r * LDB + 64 * h);
    u32x4* pb = reinterpret_cast<u32x4*>(Bs + r * LDB + 64 * h);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        pa[i] = R.a[i];
        pb[i] = R.b[i];
    }
}

template <int BITS, bool CB, typename TSrel>
__global__ __launch_bounds__(256) void gemm_i8_kernel(GemmI8Args p) {
    __shared__ __attribute__((aligned(16))) uint8_t smem[2][2][BM * LDB];
    __shared__ float cb_s[16];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int64_t n0 = (int64_t)blockIdx.x * BN, m0 = (int64_t)blockIdx.y * BM;
    const bool vec_ok = (p.ldx % 16 == 0) && ((uintptr_t)p.xq % 16 == 0);
    const int ktiles = (int)((p.K + BK - 1) / BK);
    if constexpr (CB) {
        if (tid < 16) cb_s[tid] = p.codebook[tid];
        __syncthreads();
    }
    const float* cb = CB ? cb_s : nullptr;

    i32x4 acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = i32x4{0, 0, 0, 0};

    Regs R;
    load_tiles<BITS, CB, TSrel>(p, cb, m0, n0, 0, tid, vec_ok, R);
    store_regs(smem[0][0], smem[0][1], tid, R);
    __syncthreads();
    const int r16 = lane & 15, g = lane >> 4;
    for (int kt = 0; kt < ktiles; ++kt) {
        const int buf = kt & 1;
        if (kt + 1 < ktiles) load_tiles<BITS, CB, TSrel>(p, cb, m0, n0, (int64_t)(kt + 1) * BK, tid, vec_ok, R);
        const uint8_t* As = smem[buf][0];
        const uint8_t* Bs = smem[buf][1];
#pragma unroll
        for (int kk = 0; kk < BK / 64; ++kk) {
            i32x4 af[4], bf[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                af[i] = *reinterpret_cast<const i32x4*>(As + (wm * 64 + i * 16 + r16) * LDB + kk * 64 + 16 * g);
                bf[i] = *reinterpret_cast<const i32x4*>(Bs + (wn * 64 + i * 16 + r16) * LDB + kk * 64 + 16 * g);
            }
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(af[i], bf[j], acc[i][j], 0, 0, 0);
        }
        if (kt + 1 < ktiles) store_regs(smem[buf ^ 1][0], smem[buf ^ 1][1], tid, R);
        __syncthreads();
    }

    // Epilogue rounds each operation separately (no fused multiply-add), so the output is exactly
    // fp(((f32(acc) * sx[m]) * s_channel[n]) + bias[n]).
    {
#pragma clang fp contract(off)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int64_t n = n0 + wn * 64 + 16 * j + r16;
        if (n >= p.N) continue;
        const float sc = p.s_ch[n];
        const float bv = p.bias ? load_rt(p.bias, p.bias_dtype, n) : 0.0f;
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const int64_t m = m0 + wm * 64 + 16 * i + 4 * g + v;
                if (m >= p.M) continue;
                float val = (float)acc[i][j][v] * p.sx[m];
                val = val * sc;
                if (p.bias) val = val + bv;
                store_rt(p.y, p.y_dtype, m * p.ldy + n, val);
            }
    }
    }
}

template <int BITS, bool CB, typename TSrel>
hipError_t launch_o(const GemmI8Args& p, hipStream_t st) {
    if (p.y_dtype != DT_F32 && p.y_dtype != DT_F16 && p.y_dtype != DT_BF16) return hipErrorInvalidValue;
    dim3 grid((unsigned)((p.N + BN - 1) / BN), (unsigned)((p.M + BM - 1) / BM)), block(256);
    hipLaunchKernelGGL((gemm_i8_kernel<BITS, CB, TSrel>), grid, block, 0, st, p);
    return hipGetLastError();
}

template <int BITS, bool CB>
hipError_t launch_s(const GemmI8Args& p, hipStream_t st) {
    switch (p.s_rel_dtype) {
        case DT_E4M3: return launch_o<BITS, CB, uint8_t>(p, st);
        case DT_F16: return launch_o<BITS, CB, f16>(p, st);
        case DT_BF16: return launch_o<BITS, CB, bf16_t>(p, st);
        case DT_F32: return launch_o<BITS, CB, float>(p, st);
    }
    return hipErrorInvalidValue;
}

}  // namespace

hipError_t run_gemm_i8(const GemmI8Args& p, hipStream_t st) {
    if (p.M == 0 || p.N == 0) return hipSuccess;
    if (p.K % 64 != 0) return hipErrorInvalidValue;
    if (p.bits == 4) return p.codebook ? launch_s<4, true>(p, st) : launch_s<4, false>(p, st);
    if (p.bits == 6) return launch_s<6, false>(p, st);
    return hipErrorInvalidValue;
}

}  // namespace qlin
