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
#include "lora_frag.h"
#include "prologue_dev.h"

namespace qlin {
namespace {

constexpr int BM = 128, BN = 128, BK = 128, LDB = BK + 16;  // LDS row stride in bytes

struct Regs {
    u32x4 a[4];  // 64 int8 of one activation row half
    u32x4 b[4];  // 64 decoded int8 of one weight row half
};

// Raw bits of s_rel[i] (converted at the point of use, so the load does not force an early wait)
template <typename TSrel>
__device__ __forceinline__ uint32_t srel_bits(const void* s, int64_t i) {
    if constexpr (sizeof(TSrel) == 1) return ((const uint8_t*)s)[i];
    else if constexpr (sizeof(TSrel) == 2) return ((const uint16_t*)s)[i];
    else return ((const uint32_t*)s)[i];
}
template <typename TSrel>
__device__ __forceinline__ float srel_from_bits(uint32_t b) {
    if constexpr (sizeof(TSrel) == 1) return e4m3_to_f32((uint8_t)b);
    else if constexpr (sizeof(TSrel) == 4) return __uint_as_float(b);
    else if constexpr (__is_same(TSrel, bf16_t)) return bf16_bits_to_f32((uint16_t)b);
    else return f16_bits_to_f32((uint16_t)b);
}

template <typename TSrel>
__device__ __forceinline__ float srel_at(const void* s, int64_t i) {
    if constexpr (sizeof(TSrel) == 1) return e4m3_to_f32(((const uint8_t*)s)[i]);
    else return load_f((const TSrel*)s + i);
}

// The grid value clamp(rne(v), -127, 127) of an fp32 v, as the low byte of the result: adding
// 1.5 * 2^23 rounds v to an integer in the low mantissa bits (ties to even; |v| < 2^22), the float
// clamp keeps it within +-127 (any larger v, infinities included, lands on a bound), and the low
// byte of M + w8 is w8 in two's complement (M's low byte is 0).  tests/grid_decode_check.c checks
// this against clamp(rne(fp32(level * s))) for every code and every 16-bit scale.
constexpr float GRID_MAGIC = 12582912.0f;
__device__ __forceinline__ uint32_t grid_bits(float v) {
#pragma clang fp contract(off)
    return __float_as_uint(__builtin_amdgcn_fmed3f(v + GRID_MAGIC, GRID_MAGIC - 127.0f, GRID_MAGIC + 127.0f));
}
__device__ __forceinline__ uint32_t grid_byte(float level, float s) {
#pragma clang fp contract(off)
    return grid_bits(level * s) & 0xFFu;  // the product rounded to fp32 first
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
        r[i] = (int8_t)grid_byte(level, s);
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
    // fp(((f32(acc) * sx[m]) * s_channel[n]) + bias[n]).  Its operands are loaded before the first
    // store: a load between stores would wait for the stores before it.
    float sxv[4][4], scv[4];
    uint32_t bvb[4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int v = 0; v < 4; ++v) sxv[i][v] = p.sx[min(m0 + wm * 64 + 16 * i + 4 * g + v, p.M - 1)];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int64_t n = min(n0 + wn * 64 + 16 * j + r16, p.N - 1);
        scv[j] = p.s_ch[n];
        bvb[j] = p.bias ? load_bits_rt(p.bias, p.bias_dtype, n) : 0u;
    }
    // every output first, then (per output dtype) its stored bits in a register of its own and the
    // stores: rewriting the data register of a store in flight would wait for it
    float out[4][4][4];
    {
#pragma clang fp contract(off)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const float bv = p.bias ? bits_to_f32_rt(bvb[j], p.bias_dtype) : 0.0f;
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                float val = (float)acc[i][j][v] * sxv[i][v];
                val = val * scv[j];
                if (p.bias) val = val + bv;
                out[i][j][v] = val;
            }
    }
    }
    auto at = [&](int i, int j, int v, int64_t& idx) {
        const int64_t m = m0 + wm * 64 + 16 * i + 4 * g + v, n = n0 + wn * 64 + 16 * j + r16;
        idx = m * p.ldy + n;
        return m < p.M && n < p.N;
    };
    if (p.y_dtype == DT_F32) {
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int v = 0; v < 4; ++v) {
                    int64_t idx;
                    if (at(i, j, v, idx)) reinterpret_cast<float*>(p.y)[idx] = out[i][j][v];
                }
    } else {
        uint32_t hb[4][4][4];
        const bool h16 = p.y_dtype == DT_F16;
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int v = 0; v < 4; ++v)
                    hb[i][j][v] = h16 ? (uint32_t)__builtin_bit_cast(uint16_t, (f16)out[i][j][v])
                                      : (uint32_t)f32_to_bf16_bits(out[i][j][v]);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int v = 0; v < 4; ++v) {
                    int64_t idx;
                    if (at(i, j, v, idx)) reinterpret_cast<uint16_t*>(p.y)[idx] = (uint16_t)hb[i][j][v];
                }
    }
}


// ------------------------------------------------------------------------------------------------
// Large-tile A8 kernel: 512 threads, tile 256 x 256 x 128 (int8), waves 4 x 2 of 64 x 128 (two
// waves per SIMD, so one wave's MFMAs cover the other's memory waits).
// Each decoded weight value feeds 2 * BM MFMA ops, so the decode must stay near 2-4 VALU per value:
//   * 4-bit codes (uniform or codebook): per weight row and k-tile one 16-entry int8 table
//     T[c] = clamp(rne(level[c] * s), -127, 127), built by the two threads that decode the row,
//     then two v_perm lookups (the low and high eight entries) and a byte select on bit 3 per four
//     codes -- the same int8 grid as decode8_i8;
//   * 6-bit codes: (c - 32) * s is exact in fp32 for fp16 / e4m3 / bf16 scales (a 6-bit integer
//     times an 11-bit significand), so rint + one med3 clamp gives the grid value directly.
// The next k-tile's loads are issued before the current tile's MFMAs and decoded after them in the
// same basic block.  Requires K % 128 == 0 and group_size % 64 == 0 (one scale per 64-value half).
// ------------------------------------------------------------------------------------------------

// Byte-wise lookup of four 4-bit indices (one per byte) in a 16-byte table t0..t3.
__device__ __forceinline__ uint32_t lut16(uint32_t idx, uint32_t t0, uint32_t t1, uint32_t t2, uint32_t t3) {
    const uint32_t sel = idx & 0x07070707u;
    const uint32_t lo = __builtin_amdgcn_perm(t1, t0, sel);
    const uint32_t hi = __builtin_amdgcn_perm(t3, t2, sel);
    const uint32_t m8 = idx & 0x08080808u;
    const uint32_t mask = (m8 << 5) - (m8 >> 3);  // 0xFF in every byte whose index has bit 3
    return (hi & mask) | (lo & ~mask);
}

// 64 codes of one weight row (nibble dwords nib[0..7], 2-bit plane hi2[0..3] for 6-bit) -> 64
// int8 grid values in out[0..15].  4-bit: a 16-entry table per scale.  When the thread pair that
// shares the row also shares the scale (`pair`, wave-uniform), each builds half of it (entries
// 8h .. 8h+7) and the halves are swapped with one lane shuffle; otherwise each builds all 16.
template <int BITS, bool CB>
__device__ __forceinline__ void decode64(const uint32_t* nib, const uint32_t* hi2, float s, const float* cb, int h,
                                         bool pair, uint32_t* out) {
#pragma clang fp contract(off)
    if constexpr (BITS == 4) {
        auto entries = [&](int c0) {
            uint32_t v = 0;
#pragma unroll
            for (int b = 0; b < 4; ++b) {
                const int c = c0 + b;
                const float level = CB ? cb[c] : (float)(c - 8);
                v |= grid_byte(level, s) << (8 * b);
            }
            return v;
        };
        uint32_t t0, t1, t2, t3;
        if (pair) {
            const uint32_t mine0 = entries(8 * h), mine1 = entries(8 * h + 4);
            const uint32_t other0 = (uint32_t)__shfl_xor((int)mine0, 1, 64);
            const uint32_t other1 = (uint32_t)__shfl_xor((int)mine1, 1, 64);
            t0 = h ? other0 : mine0; t1 = h ? other1 : mine1;
            t2 = h ? mine0 : other0; t3 = h ? mine1 : other1;
        } else {
            t0 = entries(0); t1 = entries(4); t2 = entries(8); t3 = entries(12);
        }
#pragma unroll
        for (int d = 0; d < 8; ++d) {  // nibble dword d: codes 8d .. 8d+7
            const uint32_t w = nib[d];
            const uint32_t ev = lut16(w & 0x0F0F0F0Fu, t0, t1, t2, t3);         // codes 0, 2, 4, 6
            const uint32_t od = lut16((w >> 4) & 0x0F0F0F0Fu, t0, t1, t2, t3);  // codes 1, 3, 5, 7
            out[2 * d] = __builtin_amdgcn_perm(od, ev, 0x05010400u);
            out[2 * d + 1] = __builtin_amdgcn_perm(od, ev, 0x07030602u);
        }
    } else {
        (void)h;
        // (c - 32) * s as fma(c, s, -32 s): the exact product rounded once, the reference's fp32
        // product; s clamped to +-2^20 (every clamped grid value is unchanged, -32 s stays finite)
        const float sc = __builtin_amdgcn_fmed3f(s, -0x1p20f, 0x1p20f), off = -32.0f * sc;
#pragma unroll
        for (int d = 0; d < 8; ++d) {
            const uint32_t w = nib[d];
            const uint32_t h16 = (hi2[d >> 1] >> (16 * (d & 1))) & 0xFFFFu;  // 2 bits per code
            uint32_t o0 = 0, o1 = 0;
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const uint32_t code = ((w >> (4 * i)) & 0xFu) | (((h16 >> (2 * i)) & 3u) << 4);
                const uint32_t bb = grid_bits(__builtin_fmaf((float)code, sc, off)) & 0xFFu;
                if (i < 4) o0 |= bb << (8 * i);
                else o1 |= bb << (8 * (i - 4));
            }
            out[2 * d] = o0;
            out[2 * d + 1] = o1;
        }
    }
}

// Tile order for an 8-XCD part: block b runs on XCD b % 8, so each XCD is given a contiguous run
// of the tile sequence, and the sequence walks groups of 4 M-tiles across all N-tiles.  Tiles
// resident at the same time on one XCD then share activation and weight panels in its L2.
__device__ __forceinline__ void xcd_tile(int b, int nblocks, int n_m, int n_n, int& mt, int& nt) {
    constexpr int XCD = 8, GROUP_M = 4;
    const int per = nblocks / XCD;  // the last nblocks % 8 blocks keep the plain order
    const int t = b < XCD * per ? (b % XCD) * per + b / XCD : b;
    const int group = t / (GROUP_M * n_n);
    const int first_m = group * GROUP_M;
    const int gm = min(n_m - first_m, GROUP_M);
    mt = first_m + (t % (GROUP_M * n_n)) % gm;
    nt = (t % (GROUP_M * n_n)) / gm;
}

// 512 threads = 8 waves, 4 (M) x 2 (N) of 64 x 128; tile 256 x 256 x 128 (int8).
constexpr int BKA = 128, LDAA = BKA + 16;  // k-tile and LDS row stride (bytes)

template <int BITS, bool CB, typename TSrel, bool PAIR>
__global__ __launch_bounds__(512) void gemm_a8_kernel(GemmI8Args p) {
    constexpr int BMT = 256, BNT = 256, NT = 512;
    // v_mfma_i32_32x32x32_i8 sub-tiles (about 1.6x the throughput of the 16x16x64 form here)
    constexpr int WM = 64, WN = 128, TI = WM / 32, TJ = WN / 32;
    constexpr int NA = BMT * (BKA / 16) / NT;  // 16-byte activation chunks per thread and k-tile
    constexpr int ASZ = BMT * BKA;             // activation tile bytes (rows of 128 bytes, swizzled)
    // one LDS block: double-buffered operands in the loop, then the output staging of the epilogue
    __shared__ __attribute__((aligned(16))) uint8_t smem[2 * ASZ + 2 * BNT * LDAA];
    uint8_t (*As)[ASZ] = reinterpret_cast<uint8_t (*)[ASZ]>(smem);
    uint8_t (*Bs)[BNT * LDAA] = reinterpret_cast<uint8_t (*)[BNT * LDAA]>(smem + 2 * ASZ);
    __shared__ float cb_s[16];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int r32 = lane & 31, h = lane >> 5;
    int mt, nt;
    xcd_tile(blockIdx.x, (int)gridDim.x, (int)((p.M + BMT - 1) / BMT), (int)((p.N + BNT - 1) / BNT), mt, nt);
    const int64_t n0 = (int64_t)nt * BNT, m0 = (int64_t)mt * BMT;
    const int ktiles = (int)(p.K / BKA);
    if constexpr (CB) {
        if (tid < 16) cb_s[tid] = p.codebook[tid];
        __syncthreads();
    }
    const float* cb = CB ? cb_s : nullptr;

    // weight row r = tid / 2 of the tile, codes 64h .. 64h+63 of each k-tile (rows past N re-read
    // row N - 1 and are never stored)
    const int br = tid >> 1, bh = tid & 1;
    const int64_t nrow = min(n0 + br, p.N - 1);
    const uint8_t* wrow = p.q + nrow * p.ldq;
    const int gsh = p.group_size / 64;  // 64-value halves per scale group
    const void* srow = nullptr;
    if constexpr (sizeof(TSrel) == 1) srow = (const uint8_t*)p.s_rel + nrow * p.ld_srel;
    else srow = (const TSrel*)p.s_rel + nrow * p.ld_srel;

    // Activation tile: LDS DMA (global_load_lds, 16 bytes per lane) into rows of 128 bytes whose
    // 16-byte chunks are XOR-swizzled by (row / 2) % 8, so that the 32-row fragment reads below hit
    // 16 different bank groups per 16 lanes.  DMA instruction i of wave w fills physical chunks
    // 512 i + 64 w + lane, i.e. row 64 i + 8 w + lane / 8, physical chunk lane % 8, which holds
    // logical chunk (lane % 8) ^ ((4 w + lane / 16) % 8).  Rows past M re-read row M - 1.
    const int8_t* asrc[NA];
#pragma unroll
    for (int i = 0; i < NA; ++i) {
        const int row = 64 * i + 8 * wave + (lane >> 3);
        const int c = (lane & 7) ^ ((4 * wave + (lane >> 4)) & 7);
        asrc[i] = p.xq + min(m0 + row, p.M - 1) * p.ldx + 16 * c;
    }
    auto fetch_a = [&](int kt, int buf) {
        const int k0 = min(kt, ktiles - 1) * BKA;
#pragma unroll
        for (int i = 0; i < NA; ++i)
            __builtin_amdgcn_global_load_lds(asrc[i] + k0, &As[buf][16 * (512 * i + 64 * wave)], 16, 0, 0);
    };
    struct Regs {
        uint32_t n[8], hh[4], s;
    };
    constexpr int NB = (BITS == 6) ? 4 : 3;  // vector-memory operations per fetch_b
    auto fetch_b = [&](int kt, Regs& R) {
        kt = min(kt, ktiles - 1);  // past the end: re-reads the last tile (never staged for use)
        const int k0 = kt * BKA;
        const uint8_t* pn = wrow + k0 / 2 + 32 * bh;
        const u32x4 n_0 = *reinterpret_cast<const u32x4*>(pn), n_1 = *reinterpret_cast<const u32x4*>(pn + 16);
        R.n[0] = n_0.x; R.n[1] = n_0.y; R.n[2] = n_0.z; R.n[3] = n_0.w;
        R.n[4] = n_1.x; R.n[5] = n_1.y; R.n[6] = n_1.z; R.n[7] = n_1.w;
        if constexpr (BITS == 6) {
            const u32x4 hv = *reinterpret_cast<const u32x4*>(wrow + p.K / 2 + k0 / 4 + 16 * bh);
            R.hh[0] = hv.x; R.hh[1] = hv.y; R.hh[2] = hv.z; R.hh[3] = hv.w;
        }
        R.s = srel_bits<TSrel>(srow, (unsigned)(2 * kt + bh) / (unsigned)gsh);
    };
    auto stage_b = [&](int buf, const Regs& R) {
        uint32_t o[16];
        decode64<BITS, CB>(R.n, R.hh, srel_from_bits<TSrel>(R.s), cb, bh, PAIR, o);
        u32x4* pb = reinterpret_cast<u32x4*>(&Bs[buf][br * LDAA + 64 * bh]);
#pragma unroll
        for (int i = 0; i < 4; ++i) pb[i] = u32x4{o[4 * i], o[4 * i + 1], o[4 * i + 2], o[4 * i + 3]};
    };

    i32x16 acc[TI][TJ];
#pragma unroll
    for (int i = 0; i < TI; ++i)
#pragma unroll
        for (int j = 0; j < TJ; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0;
    // A / B fragment of a 32 x 32 x 32 step: lane l holds row (column) l % 32 and the 16
    // consecutive k values 16 (l / 32) .. + 15 of the step, in both operands alike
    const int asw = (r32 >> 1) & 7;  // swizzle of this lane's activation rows
    auto mfmas = [&](int buf) {
        const uint8_t* as = &As[buf][(wm * WM + r32) * BKA];
        const uint8_t* bs = &Bs[buf][(wn * WN + r32) * LDAA + 16 * h];
#pragma unroll
        for (int kk = 0; kk < BKA / 32; ++kk) {
            i32x4 bf[TJ];
#pragma unroll
            for (int j = 0; j < TJ; ++j) bf[j] = *reinterpret_cast<const i32x4*>(bs + 32 * j * LDAA + 32 * kk);
            const int ac = 16 * ((2 * kk + h) ^ asw);
#pragma unroll
            for (int i = 0; i < TI; ++i) {
                const i32x4 af = *reinterpret_cast<const i32x4*>(as + 32 * i * BKA + ac);
#pragma unroll
                for (int j = 0; j < TJ; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(af, bf[j], acc[i][j], 0, 0, 0);
            }
        }
    };
    // Schedule of one k-tile: the first fragment reads, then each MFMA followed by seven VALU
    // instructions (the next tile's weight decode), the next 32-k step's fragment reads spread over
    // the MFMAs, the LDS writes last.
    auto interleave = [&]() {
        constexpr int FR = TI + TJ;  // fragment reads per 32-k step
        __builtin_amdgcn_sched_group_barrier(0x100, FR, 0);
#pragma unroll
        for (int kk = 0; kk < BKA / 32; ++kk)
#pragma unroll
            for (int m = 0; m < TI * TJ; ++m) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                __builtin_amdgcn_sched_group_barrier(0x002, 7, 0);
                if (kk + 1 < BKA / 32 && m < FR) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
            }
        __builtin_amdgcn_sched_group_barrier(0x200, 4, 0);
    };

    // Iteration kt: the activation DMA of tile kt + 1 and the weight loads of tile kt + 2 go out
    // first; tile kt's MFMAs share a basic block with the decode of tile kt + 1's weights (loaded one
    // iteration earlier); the barrier waits for the DMA only.  Two weight register sets alternate
    // (the loop is unrolled by two).
    Regs R0, R1;
    fetch_a(0, 0);
    fetch_b(0, R0);
    fetch_b(1, R1);
    wait_vmcnt<NB>();  // tile 0 (DMA and weights) has landed
    stage_b(0, R0);
    __syncthreads();
    for (int kt = 0; kt < ktiles; kt += 2) {
        fetch_a(kt + 1, 1);
        __builtin_amdgcn_sched_barrier(0);  // the DMA is older than the weight loads (wait_vmcnt<NB>)
        fetch_b(kt + 2, R0);  // R0's tile is staged already
        __builtin_amdgcn_sched_barrier(0);
        mfmas(0);
        stage_b(1, R1);
        interleave();
        wait_vmcnt<NB>();
        lds_barrier();
        if (kt + 1 < ktiles) {  // uniform
            fetch_a(kt + 2, 0);
            __builtin_amdgcn_sched_barrier(0);
            fetch_b(kt + 3, R1);
            __builtin_amdgcn_sched_barrier(0);
            mfmas(1);
            stage_b(0, R0);
            interleave();
            wait_vmcnt<NB>();
            lds_barrier();
        }
    }

    // Epilogue: y = fp(((f32(acc) * sx[m]) * s_channel[n]) + bias[n]), each operation rounded on its
    // own.  The int32 tile goes through LDS in four passes of 64 rows, one wave row each (row stride
    // 264 words: rows 4 apart fall 32 banks apart), then every thread writes 8 consecutive outputs
    // of a row with 16-byte stores.  Lane l, register r of a 32 x 32 sub-tile holds row 8 (r / 4) +
    // 4 (l / 32) + r % 4, column l % 32.  Every operand of the epilogue is requested before the
    // first store (the tile's activation scales go to LDS): a global load between the stores would
    // wait for the stores before it.  Each pass computes all of a thread's outputs before its
    // stores; the passes synchronize LDS only.
    constexpr int ORW = BNT + 8, CPR = BNT / 8, RP = WM, Q = RP * CPR / NT;
    static_assert(RP * ORW * 4 + BMT * 4 <= (int)sizeof(smem), "output staging must fit in the operand buffers");
    static_assert((RP * CPR) % NT == 0, "chunks must split evenly");
    int32_t* ot = reinterpret_cast<int32_t*>(smem);
    float* sxs = reinterpret_cast<float*>(reinterpret_cast<uint8_t*>(smem) + sizeof(smem) - BMT * 4);
    const int cc = tid % CPR;                    // this thread's 8-column chunk (the same in every pass)
    const int64_t nc = n0 + 8 * cc;
    const int ncount = (int)max<int64_t>(0, min<int64_t>(8, p.N - nc));
    const float sxr = p.sx[min(m0 + min(tid, BMT - 1), (int64_t)p.M - 1)];
    float sc[8];
    uint32_t bvb[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        const int64_t n = min(nc + e, p.N - 1);
        sc[e] = p.s_ch[n];
        bvb[e] = p.bias ? load_bits_rt(p.bias, p.bias_dtype, n) : 0u;
    }
    uint32_t rsb[8];
    residual_scale_bits8(p.res, nc, p.N, rsb);
    float bv[8], rsv[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) bv[e] = p.bias ? bits_to_f32_rt(bvb[e], p.bias_dtype) : 0.0f;
    residual_scales8(p.res, rsb, rsv);
    const bool vec = (p.ldy % 8 == 0) && ((uintptr_t)p.y % 16 == 0);
#pragma unroll
    for (int pass = 0; pass < BMT / RP; ++pass) {
        lds_barrier();  // the operand buffers (or the previous pass) are no longer read
        if (pass == 0 && tid < BMT) sxs[tid] = sxr;
        if (wm == pass) {
#pragma unroll
            for (int i = 0; i < TI; ++i)
#pragma unroll
                for (int j = 0; j < TJ; ++j)
#pragma unroll
                    for (int r = 0; r < 16; ++r)
                        ot[(32 * i + 8 * (r / 4) + 4 * h + r % 4) * ORW + wn * WN + 32 * j + r32] = acc[i][j][r];
        }
        lds_barrier();
        float v[Q][8];
#pragma unroll
        for (int q = 0; q < Q; ++q) {
            const int row = tid / CPR + (NT / CPR) * q;
            const i32x4 a0 = *reinterpret_cast<const i32x4*>(ot + row * ORW + 8 * cc);
            const i32x4 a1 = *reinterpret_cast<const i32x4*>(ot + row * ORW + 8 * cc + 4);
            const float sxm = sxs[RP * pass + row];
            {
#pragma clang fp contract(off)
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    float val = (float)(e < 4 ? a0[e] : a1[e - 4]) * sxm;
                    val = val * sc[e];
                    if (p.bias) val = val + bv[e];
                    v[q][e] = val;
                }
            }
        }
        int64_t mq[Q];
#pragma unroll
        for (int q = 0; q < Q; ++q) mq[q] = m0 + RP * pass + tid / CPR + (NT / CPR) * q;
        if (p.res.r) residual_apply8<Q>(p.res, mq, nc, p.M, p.N, rsv, v);
#pragma unroll
        for (int q = 0; q < Q; ++q) {
            const int64_t m = mq[q];
            if (m < p.M && ncount > 0) store8_rt(p.y, p.y_dtype, m * p.ldy + nc, v[q], ncount, vec);
        }
    }
}

// ------------------------------------------------------------------------------------------------
// Decode-once path for many activation rows (M >= 1024): the int8 weight grid is decoded once
// into the workspace (the same decode64 as the fused kernel), then a plain int8 x int8 GEMM reads
// both operands with LDS DMA.  The fused kernel decodes every weight once per 256-row M-tile;
// here the decode VALU work leaves the GEMM loop, whose MFMAs interleave with fragment reads only.
// ------------------------------------------------------------------------------------------------

// Four threads per (weight row, 64-code segment): thread q of a quad writes w8[n][64 s + 16 q ..
// + 15], so the lanes of a wave load contiguous runs (8 bytes of nibbles and, for 6 bits, 4 bytes
// of high bits each) and store 16 contiguous bytes each.  The 4-bit level table (one grid byte per
// code) is built a quarter per thread and exchanged within the quad.  Needs group_size % 64 == 0.
// Thread t of the decode (quads of consecutive t share a segment; t % 4 == threadIdx.x % 4).
template <int BITS, bool CB, typename TSrel>
__device__ __forceinline__ void a8_grid_quad(const GemmI8Args& p, int8_t* __restrict__ w8, uint32_t t) {
#pragma clang fp contract(off)
    // 32-bit indices: the launchers refuse grids of 2^32 threads or more (4 per 64-code segment)
    const uint32_t segs = (uint32_t)p.K / 64u, total = (uint32_t)p.N * segs;
    const uint32_t u = t >> 2;
    const int q = (int)(t & 3u);
    // Threads past the end work on the last segment (all four lanes of a quad take part in the
    // table exchange) and skip only the store.
    const bool live = u < total;
    const uint32_t uu = live ? u : total - 1;
    const uint32_t n32 = uu / segs;
    const int sg = (int)(uu - n32 * segs);
    const int64_t n = n32;
    const uint8_t* row = p.q + n * p.ldq;
    const u32x2 nv = *reinterpret_cast<const u32x2*>(row + 32 * sg + 8 * q);  // codes 16 q .. 16 q + 15
    const void* srow;
    if constexpr (sizeof(TSrel) == 1) srow = (const uint8_t*)p.s_rel + n * p.ld_srel;
    else srow = (const TSrel*)p.s_rel + n * p.ld_srel;
    const float s = srel_from_bits<TSrel>(srel_bits<TSrel>(srow, (unsigned)(64 * sg) / (unsigned)p.group_size));
    uint32_t o[4];
    if constexpr (BITS == 4) {
        uint32_t mine = 0;  // grid bytes of codes 4 q .. 4 q + 3
#pragma unroll
        for (int b = 0; b < 4; ++b) {
            const int c = 4 * q + b;
            const float level = CB ? p.codebook[c] : (float)(c - 8);
            mine |= grid_byte(level, s) << (8 * b);
        }
        const uint32_t t0 = (uint32_t)__builtin_amdgcn_mov_dpp((int)mine, 0x00, 0xF, 0xF, false);
        const uint32_t t1 = (uint32_t)__builtin_amdgcn_mov_dpp((int)mine, 0x55, 0xF, 0xF, false);
        const uint32_t t2 = (uint32_t)__builtin_amdgcn_mov_dpp((int)mine, 0xAA, 0xF, 0xF, false);
        const uint32_t t3 = (uint32_t)__builtin_amdgcn_mov_dpp((int)mine, 0xFF, 0xF, 0xF, false);
#pragma unroll
        for (int d = 0; d < 2; ++d) {  // nibble dword d: codes 16 q + 8 d .. + 7
            const uint32_t w = nv[d];
            const uint32_t ev = lut16(w & 0x0F0F0F0Fu, t0, t1, t2, t3);         // codes 0, 2, 4, 6
            const uint32_t od = lut16((w >> 4) & 0x0F0F0F0Fu, t0, t1, t2, t3);  // codes 1, 3, 5, 7
            o[2 * d] = __builtin_amdgcn_perm(od, ev, 0x05010400u);
            o[2 * d + 1] = __builtin_amdgcn_perm(od, ev, 0x07030602u);
        }
    } else {
        const uint32_t hv = *reinterpret_cast<const uint32_t*>(row + p.K / 2 + 16 * sg + 4 * q);
        // (c - 32) * s as fma(c, s, -32 s): the exact product rounded once, the reference's fp32
        // product; s clamped to +-2^20 (every clamped grid value is unchanged, -32 s stays finite)
        const float sc = __builtin_amdgcn_fmed3f(s, -0x1p20f, 0x1p20f), off = -32.0f * sc;
#pragma unroll
        for (int d = 0; d < 2; ++d) {
            const uint32_t w = nv[d];
            const uint32_t h16 = (hv >> (16 * d)) & 0xFFFFu;  // 2 bits per code
            uint32_t o0 = 0, o1 = 0;
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const uint32_t code = ((w >> (4 * i)) & 0xFu) | (((h16 >> (2 * i)) & 3u) << 4);
                const uint32_t bb = grid_bits(__builtin_fmaf((float)code, sc, off)) & 0xFFu;
                if (i < 4) o0 |= bb << (8 * i);
                else o1 |= bb << (8 * (i - 4));
            }
            o[2 * d] = o0;
            o[2 * d + 1] = o1;
        }
    }
    if (live) *reinterpret_cast<u32x4*>(w8 + n * p.K + 64 * sg + 16 * q) = u32x4{o[0], o[1], o[2], o[3]};
}

template <int BITS, bool CB, typename TSrel>
__global__ __launch_bounds__(256) void a8_grid_kernel(GemmI8Args p, int8_t* __restrict__ w8) {
    a8_grid_quad<BITS, CB, TSrel>(p, w8, blockIdx.x * 256u + threadIdx.x);
}

// The s_rel dtype and the codebook choice of a8_grid_quad, made at run time (uniform per launch).
template <int BITS>
__device__ __forceinline__ void a8_grid_quad_rt(const GemmI8Args& p, int8_t* __restrict__ w8, uint32_t t) {
    auto by_srel = [&]<bool CB>() {
        switch (p.s_rel_dtype) {
            case DT_E4M3: a8_grid_quad<BITS, CB, uint8_t>(p, w8, t); break;
            case DT_F16: a8_grid_quad<BITS, CB, f16>(p, w8, t); break;
            case DT_BF16: a8_grid_quad<BITS, CB, bf16_t>(p, w8, t); break;
            default: a8_grid_quad<BITS, CB, float>(p, w8, t); break;
        }
    };
    if (BITS == 4 && p.codebook) by_srel.template operator()<true>();
    else by_srel.template operator()<false>();
}

// The A8 pre-pass in one launch: workgroups 0 .. M - 1 are the activation prologue's rows, the rest
// decode the weight grid (workgroup M + j: threads j NT .. j NT + NT - 1 of a8_grid_kernel's
// decode).  Both roles compute exactly what their own kernels compute.  In one launch the decode
// takes each CU as the prologue's last rows there finish, instead of after the whole prologue
// (same process: W6A8 M9504 K13824 N5120 780 -> 739 us per call, M9504 K5120 N13824 773 -> 741,
// W4A8 M4096 K3072 N12288 196 -> 183; at M1024 0.8-3.3 us slower, so fewer than A8_PREPASS_ROWS rows
// keep two launches).  The two roles side by side were slower than in sequence: interleaved through
// the grid 157 against 134 us (W6A8 M1024 K13824), and the two kernels on two streams 67 against
// 50 us for the pair alone.
struct A8PrepassArgs {
    const void* x;
    int64_t ldx;
    bool vec_ok;
    int8_t* qo;
    float* so;
};
template <typename TIn, int G, int SLOTS, int BITS>
__global__ __launch_bounds__(prologue_max_threads(SLOTS), SLOTS <= 2 ? 6 : 1) void a8_prepass_kernel(A8PrepassArgs a,
                                                                                                     GemmI8Args p) {
    const uint32_t b = blockIdx.x, rows = (uint32_t)p.M;
    if (b < rows) {
        prologue_row<TIn, PROLOGUE_A8, G, SLOTS>(b, (int)blockDim.x, (const TIn*)a.x, a.ldx, (int)p.K, a.vec_ok, nullptr,
                                                 p.ldx, nullptr, a.qo, a.so, nullptr, nullptr);
        return;
    }
    a8_grid_quad_rt<BITS>(p, p.w8, (b - rows) * blockDim.x + threadIdx.x);
}

// int8 GEMM y = epilogue(xq[M, K] . w8[N, K]^T), tile BMT x BNT x BK, 8 waves 4 (M) x 2 (N),
// v_mfma_i32_32x32x32_i8.  Both operand tiles arrive by LDS DMA into rows of BK bytes whose 16-byte
// chunks are XOR-swizzled (so that the 16 rows a fragment read touches fall in 16 bank groups),
// in STAGES buffers: the DMA of k-tile kt + STAGES - 1 goes out before tile kt's MFMAs, and each
// step waits only for the oldest DMA in flight.  L2PF: one step earlier still, every 64-byte half
// line of k-tile kt + STAGES is touched with a 4-byte DMA into a sink, so that the tile's own DMA
// finds it in L2 (a second tile of look-ahead for the price of two instructions per thread).
// LDU >= 0: the LoRA term of p.lora (up of dtype LDU) joins the epilogue: the accumulators become
// (the bits of) their fp32 base values, formed as below, then base + lora_scale * t up^T with t and
// up staged through LDS (lora_tile_epilogue); the staged values are final, so the output is rounded
// once.
// Largest LoRA rank every decode-once DMA tile shape (256 x 256, 128 x 256, 128 x 128; 2 stages of
// 128-value k-tiles) stages in its LDS, the row scales aside.
template <int DU>
constexpr int i8dma_lora_rank_t() {
    constexpr int a = lora_max_rank<DU, 256, 256>(2 * (256 * 128 + 256 * 128) - 256 * 4);
    constexpr int b = lora_max_rank<DU, 128, 256>(2 * (128 * 128 + 256 * 128) - 128 * 4);
    constexpr int c = lora_max_rank<DU, 128, 128>(2 * (128 * 128 + 128 * 128) - 128 * 4);
    return a < b ? (a < c ? a : c) : (b < c ? b : c);
}
constexpr int i8dma_lora_rank(int du) {
    return du == DT_F32 ? i8dma_lora_rank_t<DT_F32>() : i8dma_lora_rank_t<DT_BF16>();
}

// WVM x WVN waves (default 4 x 2) of (BMT / WVM) x (BNT / WVN).  With other wave grids (2 x 5 for
// 128 x 160 tiles: M1024 N5120 makes 256 of them, one round on 256 CUs, where 128 x 256 tiles leave
// 96 CUs idle) the DMA instructions of a k-tile do not split evenly over the waves: instruction j
// (1 KiB of one operand) is issued by wave j % waves, and two stages without the prefetch wait for
// all of a wave's copies, whatever their count.
template <int WVM, int WVN>
constexpr int i8dma_threads() { return 64 * WVM * WVN; }
template <int BMT, int BNT, int BK, int STAGES, bool L2PF, int LDU = -1, int WVM = 4, int WVN = 2>
__global__ __launch_bounds__(64 * WVM * WVN) void gemm_i8dma_kernel(GemmI8Args p, const int8_t* __restrict__ w8) {
    constexpr int NT = i8dma_threads<WVM, WVN>(), NW = WVM * WVN;
    constexpr int WM = BMT / WVM, WN = BNT / WVN, TI = WM / 32, TJ = WN / 32;
    static_assert(TI >= 1 && TJ >= 1 && WM % 32 == 0 && WN % 32 == 0 && (BK == 64 || BK == 128), "tile shape");
    constexpr int CPRW = BK / 16;                   // 16-byte chunks per row
    constexpr int RPS = 16 / CPRW;                  // rows per swizzle step
    constexpr int ASZ = BMT * BK, BSZ = BNT * BK;   // bytes per buffer
    constexpr bool EVEN = NT == 512;                // every wave issues the same DMAs (the 4 x 2 grid)
    constexpr int NIA = ASZ / 1024, NIB = BSZ / 1024, NIT = NIA + NIB;  // 1 KiB DMA instructions per k-tile
    constexpr int NA = EVEN ? ASZ / 16 / NT : 0, NB = EVEN ? BSZ / 16 / NT : 0;  // per thread and k-tile
    constexpr int NIW = EVEN ? 1 : (NIT + NW - 1) / NW;  // uneven grids: instructions per wave (at most)
    static_assert(!EVEN || (NA * 16 * NT == ASZ && NB * 16 * NT == BSZ), "tile must split into whole DMA rounds");
    static_assert(EVEN || (ASZ % 1024 == 0 && BSZ % 1024 == 0 && STAGES == 2 && !L2PF && LDU < 0),
                  "uneven wave grids: whole 1 KiB instructions, two stages, no prefetch, no LoRA");
    // operand buffers, then (L2PF) a 4-byte-per-thread sink for the prefetch DMAs; one LDS object,
    // so that the compiler's alias tracking does not make fragment reads wait for the prefetches
    constexpr int SINK = L2PF ? NT * 4 : 0;
    __shared__ __attribute__((aligned(16))) uint8_t smem[STAGES * (ASZ + BSZ) + SINK];
    uint8_t (*buf_of)[ASZ + BSZ] = reinterpret_cast<uint8_t (*)[ASZ + BSZ]>(smem);  // [buffer][A | B]
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave / WVN, wn = wave % WVN;
    const int r32 = lane & 31, h = lane >> 5;
    int mt, nt;
    xcd_tile(blockIdx.x, (int)gridDim.x, (int)((p.M + BMT - 1) / BMT), (int)((p.N + BNT - 1) / BNT), mt, nt);
    const int64_t n0 = (int64_t)nt * BNT, m0 = (int64_t)mt * BMT;
    const int ktiles = (int)(p.K / BK);

    // DMA instruction i of wave w fills physical chunks 512 i + 64 w + lane of a buffer: row
    // (512 i + 64 w + lane) / CPRW, physical chunk lane % CPRW, which holds logical chunk
    // (lane % CPRW) ^ ((row / RPS) % CPRW) -- the same for every i.  Rows past M (N) re-read row
    // M - 1 (N - 1) and are never stored.
    const int c_l = (lane % CPRW) ^ (((64 * wave + lane) / CPRW / RPS) % CPRW);
    const int8_t* asrc[NA > 0 ? NA : 1];
    const int8_t* bsrc[NB > 0 ? NB : 1];
#pragma unroll
    for (int i = 0; i < NA; ++i)
        asrc[i] = p.xq + min(m0 + (512 * i + 64 * wave + lane) / CPRW, p.M - 1) * p.ldx + 16 * c_l;
#pragma unroll
    for (int i = 0; i < NB; ++i)
        bsrc[i] = w8 + min(n0 + (512 * i + 64 * wave + lane) / CPRW, p.N - 1) * p.K + 16 * c_l;
    // uneven grids: instruction j = wave + NW i fills chunks u = 64 j' + lane of its operand (j' its
    // index there), row u / CPRW, physical chunk u % CPRW holding logical chunk u % CPRW ^ swizzle
    const int8_t* usrc[NIW];
    int udst[NIW];
#pragma unroll
    for (int i = 0; i < NIW; ++i) {
        const int j = min(wave + NW * i, NIT - 1), ja = j < NIA ? j : j - NIA;
        const int u = 64 * ja + lane, row = u / CPRW, c = (u % CPRW) ^ ((row / RPS) % CPRW);
        usrc[i] = j < NIA ? p.xq + min(m0 + row, p.M - 1) * p.ldx + 16 * c : w8 + min(n0 + row, p.N - 1) * p.K + 16 * c;
        udst[i] = j < NIA ? 1024 * ja : ASZ + 1024 * ja;
    }
    auto dma = [&](int kt, int buf) {
        const int k0 = min(kt, ktiles - 1) * BK;
        if constexpr (EVEN) {
#pragma unroll
            for (int i = 0; i < NA; ++i) lds_dma16(asrc[i] + k0, &buf_of[buf][16 * (512 * i + 64 * wave)]);
#pragma unroll
            for (int i = 0; i < NB; ++i) lds_dma16(bsrc[i] + k0, &buf_of[buf][ASZ + 16 * (512 * i + 64 * wave)]);
        } else {
#pragma unroll
            for (int i = 0; i < NIW; ++i)
                if (wave + NW * i < NIT) lds_dma16(usrc[i] + k0, &buf_of[buf][udst[i]]);
        }
    };
    // L2 prefetch: half line u = tid + NT i of a k-tile is row u / HPR (A rows, then B rows), half
    // u % HPR; rows past M (N) touch row M - 1 (N - 1)
    constexpr int HPR = BK / 64, PFN = L2PF ? (BMT + BNT) * HPR / NT : 0;
    static_assert(!L2PF || PFN * NT == (BMT + BNT) * HPR, "prefetch must split into whole rounds");
    const int8_t* pfsrc[PFN > 0 ? PFN : 1];
#pragma unroll
    for (int i = 0; i < PFN; ++i) {
        const int u = tid + NT * i, row = u / HPR;
        pfsrc[i] = (row < BMT ? p.xq + min<int64_t>(m0 + row, p.M - 1) * p.ldx
                              : w8 + min<int64_t>(n0 + row - BMT, p.N - 1) * p.K) + 64 * (u % HPR);
    }
    auto l2pf = [&](int kt) {
        const int k0 = min(kt, ktiles - 1) * BK;
#pragma unroll
        for (int i = 0; i < PFN; ++i) lds_dma4(pfsrc[i] + k0, smem + STAGES * (ASZ + BSZ) + 256 * wave);
    };

    i32x16 acc[TI][TJ];
#pragma unroll
    for (int i = 0; i < TI; ++i)
#pragma unroll
        for (int j = 0; j < TJ; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0;
    // fragments: lane l holds row (column) l % 32 and k 16 (l / 32) .. + 15 of a 32-k step in both
    // operands; rows wm * WM + 32 i + l % 32 share the swizzle (l % 32 / RPS) % CPRW
    const int sw = (r32 / RPS) % CPRW;
    auto mfmas = [&](int buf) {
        const uint8_t* as = &buf_of[buf][(wm * WM + r32) * BK];
        const uint8_t* bs = &buf_of[buf][ASZ + (wn * WN + r32) * BK];
#pragma unroll
        for (int kk = 0; kk < BK / 32; ++kk) {
            const int c = 16 * ((2 * kk + h) ^ sw);
            i32x4 bf[TJ];
#pragma unroll
            for (int j = 0; j < TJ; ++j) bf[j] = *reinterpret_cast<const i32x4*>(bs + 32 * j * BK + c);
#pragma unroll
            for (int i = 0; i < TI; ++i) {
                const i32x4 af = *reinterpret_cast<const i32x4*>(as + 32 * i * BK + c);
#pragma unroll
                for (int j = 0; j < TJ; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(af, bf[j], acc[i][j], 0, 0, 0);
            }
        }
        // the first step's fragments, then each MFMA with one of the next step's fragment reads
        constexpr int FR = TI + TJ;
        __builtin_amdgcn_sched_group_barrier(0x100, FR, 0);
#pragma unroll
        for (int kk = 0; kk < BK / 32; ++kk)
#pragma unroll
            for (int m = 0; m < TI * TJ; ++m) {
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                if (kk + 1 < BK / 32 && m < FR) __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
            }
    };

    // Barrier without a memory fence: the DMA data this wave needs is covered by wait_vmcnt, and
    // the loop writes LDS only by DMA.  Each step issues its tile DMA, then the prefetch of the
    // tile after it; a step may leave the prefetch and the DMAs of later tiles in flight.
    constexpr int ND = NA + NB;  // DMA instructions per k-tile and thread (uneven grids: STAGES = 2, no wait count)
    constexpr int INFLIGHT = PFN + (STAGES - 2) * (ND + PFN);
#pragma unroll
    for (int st = 0; st < STAGES - 1; ++st) {
        dma(st, st);
        l2pf(st + 1);
    }
    wait_vmcnt<INFLIGHT>();
    __builtin_amdgcn_s_barrier();
    // unrolled by STAGES: every stage buffer index is a constant (1-2% faster on the A8 configs)
    for (int k0 = 0; k0 < ktiles; k0 += STAGES) {
#pragma unroll
        for (int s = 0; s < STAGES; ++s) {
            const int kt = k0 + s;
            if (kt >= ktiles) break;
            // past the end: re-reads the last tile into a buffer no step reads
            dma(kt + STAGES - 1, (s + STAGES - 1) % STAGES);
            l2pf(kt + STAGES);
            __builtin_amdgcn_sched_barrier(0);
            mfmas(s);
            // this wave's fragment reads of buffer s are complete before the barrier, after which
            // the next step's DMA may overwrite it; tile kt + 1 has landed
            wait_lgkmcnt0();
            wait_vmcnt<INFLIGHT>();
            __builtin_amdgcn_s_barrier();
        }
    }
    wait_vmcnt<0>();

    // Epilogue: y = fp(((f32(acc) * sx[m]) * s_channel[n]) + bias[n]), each operation rounded on its
    // own, staged through LDS in passes of RP rows and written as 16-byte row pieces.  Lane l,
    // register r of a 32 x 32 sub-tile holds row 8 (r / 4) + 4 (l / 32) + r % 4, column l % 32.
    // Every operand of the epilogue is requested before the first store, the tile's activation
    // scales go to LDS: a global load between the stores would wait for the stores before it (one
    // counter counts both), a memory round trip per stored row.  The passes synchronize LDS only.
    constexpr int ORW = BNT + 8, SRB = BMT * 4;
    constexpr int RP = (BMT * ORW * 4 + SRB <= (int)sizeof(smem)) ? BMT
                       : (BMT / 2 * ORW * 4 + SRB <= (int)sizeof(smem)) ? BMT / 2 : BMT / 4;
    static_assert(RP * ORW * 4 + SRB <= (int)sizeof(smem) && RP % WM == 0, "output staging must fit");
    constexpr int CPR = BNT / 8;
    static_assert(NT % CPR == 0 && (RP * CPR) % NT == 0, "chunks must split evenly");
    int32_t* ot = reinterpret_cast<int32_t*>(smem);
    float* srow = reinterpret_cast<float*>(smem + sizeof(smem) - SRB);
    const int cc = tid % CPR;
    const int64_t nc = n0 + 8 * cc;
    const int ncount = (int)max<int64_t>(0, min<int64_t>(8, p.N - nc));
    // row scale of thread tid (threads past the tile re-read its last row; only tid < BMT stores it)
    const float sxr = p.sx[min(m0 + min(tid, BMT - 1), (int64_t)p.M - 1)];
    // the store loop's scales and bias (with a LoRA term the staged values are final)
    constexpr int CB8 = LDU >= 0 ? 1 : 8;
    float sc[CB8];
    uint32_t bvb[CB8];
    if constexpr (LDU < 0) {
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const int64_t n = min(nc + e, p.N - 1);
            sc[e] = p.s_ch[n];
            bvb[e] = p.bias ? load_bits_rt(p.bias, p.bias_dtype, n) : 0u;
        }
    }
    uint32_t rsb[8];
    residual_scale_bits8(p.res, nc, p.N, rsb);
    const bool vec = (p.ldy % 8 == 0) && ((uintptr_t)p.y % 16 == 0);
    if constexpr (LDU >= 0) {
        // the tile's activation scales at the end of LDS, past the LoRA chunks
        constexpr int RC = lora_max_rank<LDU, BMT, BNT>((int)sizeof(smem) - BMT * 4);
        static_assert(RC >= i8dma_lora_rank(LDU), "the host's rank limit must fit every tile shape");
        float scn[TJ];
        uint32_t bvj[TJ];
#pragma unroll
        for (int j = 0; j < TJ; ++j) {
            const int64_t n = min(n0 + wn * WN + 32 * j + r32, p.N - 1);
            scn[j] = p.s_ch[n];
            bvj[j] = p.bias ? load_bits_rt(p.bias, p.bias_dtype, n) : 0u;
        }
        lds_barrier();  // every wave is past the main loop: the operand buffers are free
        if (tid < BMT) srow[tid] = sxr;
        lds_barrier();
#pragma unroll
        for (int j = 0; j < TJ; ++j) {
            const float bvn = p.bias ? bits_to_f32_rt(bvj[j], p.bias_dtype) : 0.0f;
#pragma unroll
            for (int i = 0; i < TI; ++i)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
#pragma clang fp contract(off)
                    float base = (float)acc[i][j][r] * srow[wm * WM + 32 * i + 8 * (r / 4) + 4 * h + r % 4];
                    base = base * scn[j];
                    if (p.bias) base = base + bvn;
                    acc[i][j][r] = __float_as_int(base);
                }
        }
        lora_tile_epilogue_ranks<LDU, BMT, BNT, RC, NT, TI, TJ>(p.lora, smem, m0, n0, p.M, p.N, wm * WM, wn * WN, tid, lane, acc);
    }
    float bv[CB8], rsv[8];
    residual_scales8(p.res, rsb, rsv);
    if constexpr (LDU < 0) {
#pragma unroll
        for (int e = 0; e < 8; ++e) bv[e] = p.bias ? bits_to_f32_rt(bvb[e], p.bias_dtype) : 0.0f;
    }
#pragma unroll
    for (int pass = 0; pass < BMT / RP; ++pass) {
        lds_barrier();  // the operand buffers (or the previous pass) are no longer read
        if constexpr (LDU < 0)
            if (pass == 0 && tid < BMT) srow[tid] = sxr;
        if ((wm * WM) / RP == pass) {
            const int rw = wm * WM - pass * RP;
#pragma unroll
            for (int i = 0; i < TI; ++i)
#pragma unroll
                for (int j = 0; j < TJ; ++j)
#pragma unroll
                    for (int r = 0; r < 16; ++r)
                        ot[(rw + 32 * i + 8 * (r / 4) + 4 * h + r % 4) * ORW + wn * WN + 32 * j + r32] = acc[i][j][r];
        }
        lds_barrier();
        // all of the pass's outputs of this thread first, then all of its stores: a register that
        // feeds a store in flight is not rewritten until the next pass
        constexpr int Q = RP * CPR / NT;
        float v[Q][8];
#pragma unroll
        for (int q = 0; q < Q; ++q) {
            const int row = tid / CPR + (NT / CPR) * q;
            const i32x4 a0 = *reinterpret_cast<const i32x4*>(ot + row * ORW + 8 * cc);
            const i32x4 a1 = *reinterpret_cast<const i32x4*>(ot + row * ORW + 8 * cc + 4);
            if constexpr (LDU >= 0) {  // staged final values
#pragma unroll
                for (int e = 0; e < 8; ++e) v[q][e] = __int_as_float(e < 4 ? a0[e] : a1[e - 4]);
            } else {
#pragma clang fp contract(off)
                const float sxm = srow[pass * RP + row];
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    float val = (float)(e < 4 ? a0[e] : a1[e - 4]) * sxm;
                    val = val * sc[e];
                    if (p.bias) val = val + bv[e];
                    v[q][e] = val;
                }
            }
        }
        int64_t mq[Q];
#pragma unroll
        for (int q = 0; q < Q; ++q) mq[q] = m0 + pass * RP + tid / CPR + (NT / CPR) * q;
        if (p.res.r) residual_apply8<Q>(p.res, mq, nc, p.M, p.N, rsv, v);
#pragma unroll
        for (int q = 0; q < Q; ++q) {
            const int64_t m = mq[q];
            if (m < p.M && ncount > 0) store8_rt(p.y, p.y_dtype, m * p.ldy + nc, v[q], ncount, vec);
        }
    }
}

// A8 linear for few activation rows (up to 32): weight streaming, the decode in the load stage.
// One 512-thread workgroup per 16 weight rows; the K range is split across the 8 waves in stages
// of 256 values.  In a stage, lane l decodes the 64 codes k = 64 (l / 16) .. + 63 of weight row
// n0 + l % 16 (read with 16-byte loads: 32 bytes of nibbles, and for 6 bits 16 bytes of the 2-bit
// plane; the four lanes of a row cover its stage contiguously) straight into the B operand of four
// v_mfma_i32_16x16x64_i8 steps: step j takes the lane's values 16 j .. 16 j + 15, and the A
// operand (the int8 activation rows, lane l holding row l % 16) is read in the same k order, so
// both operands pair the same k values.  The next stage's codes, scales and activations are
// requested before the current stage is decoded.  The int32 sums are exact; the waves' sums are
// added through LDS and the epilogue is y = (f32(acc) * sx[m]) * s_channel[n] + bias[n].
template <int BITS, bool CB, typename TSrel, int MT>
__global__ __launch_bounds__(512) void a8_smallm_kernel(GemmI8Args p) {
    constexpr int NH = BITS == 6 ? 1 : 0;   // 16-byte loads of the 2-bit plane per lane and stage
    __shared__ int red[8][MT][4][64];
    __shared__ float cb_s[16];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int nl = lane & 15, g = lane >> 4;
    const int64_t n0 = (int64_t)blockIdx.x * 16;
    const int64_t n = min(n0 + nl, p.N - 1);   // rows past N re-read row N - 1 (never stored)
    const int stages = (int)(p.K / 256);
    const int st0 = (stages * wave) / 8, st1 = (stages * (wave + 1)) / 8;
    const int last = max(st1 - 1, st0);
    const uint8_t* qrow = p.q + n * p.ldq;
    const uint8_t* hrow = qrow + p.K / 2;
    const int gs = p.group_size;
    if (CB && tid < 16) cb_s[tid] = p.codebook[tid];
    const int8_t* xrow[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) xrow[mt] = p.xq + (int64_t)min(16 * mt + nl, (int)p.M - 1) * p.ldx;
    // the epilogue's operands for this thread's outputs e = tid + 512 j, requested now so that the
    // epilogue needs no memory round trip
    constexpr int EPT = (MT * 256 + 511) / 512;
    float esx[EPT], esc[EPT];
    uint32_t ebv[EPT];
#pragma unroll
    for (int j = 0; j < EPT; ++j) {
        const int e = min(tid + 512 * j, MT * 256 - 1), em = 16 * (e >> 8) + 4 * ((e & 63) >> 4) + ((e & 255) >> 6);
        const int64_t enn = min(n0 + (e & 15), p.N - 1);
        esx[j] = p.sx[min(em, (int)p.M - 1)];
        esc[j] = p.s_ch[enn];
        ebv[j] = p.bias ? load_bits_rt(p.bias, p.bias_dtype, enn) : 0u;
    }

    struct Stage {
        u32x4 nib[2];
        u32x4 hi[NH > 0 ? NH : 1];
        uint32_t sb[4];        // raw bits of the scales of the lane's 16-value runs
        i32x4 x[MT][4];
    };
    auto fetch = [&](int st, Stage& S) {
        st = min(st, last);
        const int64_t k0 = (int64_t)st * 256 + 64 * g;
        const u32x4* qp = reinterpret_cast<const u32x4*>(qrow + k0 / 2);
        S.nib[0] = qp[0];
        S.nib[1] = qp[1];
        if constexpr (NH > 0) S.hi[0] = *reinterpret_cast<const u32x4*>(hrow + k0 / 4);
#pragma unroll
        for (int r = 0; r < 4; ++r) S.sb[r] = srel_bits<TSrel>(p.s_rel, n * p.ld_srel + (k0 + 16 * r) / gs);
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
            for (int j = 0; j < 4; ++j) S.x[mt][j] = *reinterpret_cast<const i32x4*>(xrow[mt] + k0 + 16 * j);
    };

    i32x4 acc[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) acc[mt] = i32x4{0, 0, 0, 0};
    if (CB) __syncthreads();
    const float* cb = CB ? cb_s : nullptr;
    Stage cur, nxt;
    if (st0 < st1) {
        fetch(st0, cur);
        for (int st = st0; st < st1; ++st) {
            fetch(st + 1, nxt);
            __builtin_amdgcn_sched_barrier(0);
            const uint32_t nib[8] = {cur.nib[0].x, cur.nib[0].y, cur.nib[0].z, cur.nib[0].w,
                                     cur.nib[1].x, cur.nib[1].y, cur.nib[1].z, cur.nib[1].w};
            uint32_t hi2[4] = {0u, 0u, 0u, 0u};
            if constexpr (NH > 0) {
                hi2[0] = cur.hi[0].x; hi2[1] = cur.hi[0].y; hi2[2] = cur.hi[0].z; hi2[3] = cur.hi[0].w;
            }
            uint32_t w8[16];
            if (gs % 64 == 0) {
                decode64<BITS, CB>(nib, hi2, srel_from_bits<TSrel>(cur.sb[0]), cb, 0, false, w8);
            } else {
#pragma unroll
                for (int d = 0; d < 8; ++d)  // 8 codes with the scale of their 16-value run
                    decode8_i8<BITS, CB>(nib[d], (hi2[d >> 1] >> (16 * (d & 1))) & 0xFFFFu,
                                         srel_from_bits<TSrel>(cur.sb[d >> 1]), cb, w8[2 * d], w8[2 * d + 1]);
            }
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const i32x4 bf = i32x4{(int)w8[4 * j], (int)w8[4 * j + 1], (int)w8[4 * j + 2], (int)w8[4 * j + 3]};
#pragma unroll
                for (int mt = 0; mt < MT; ++mt)
                    acc[mt] = __builtin_amdgcn_mfma_i32_16x16x64_i8(cur.x[mt][j], bf, acc[mt], 0, 0, 0);
            }
            cur = nxt;
        }
    }
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int i = 0; i < 4; ++i) red[wave][mt][i][lane] = acc[mt][i];
    __syncthreads();
    // 16 x 16 outputs per m-tile: lane l, register i of a wave holds row 4 (l / 16) + i, column l % 16
    {
#pragma clang fp contract(off)
#pragma unroll
    for (int j = 0; j < EPT; ++j) {
        const int e = tid + 512 * j;
        const int mt = e >> 8, rem = e & 255, i = rem >> 6, sl = rem & 63;
        const int64_t m = 16 * mt + 4 * (sl >> 4) + i, nn = n0 + (sl & 15);
        if (e >= MT * 256 || m >= p.M || nn >= p.N) continue;
        int sum = 0;
#pragma unroll
        for (int w = 0; w < 8; ++w) sum += red[w][mt][i][sl];
        float val = (float)sum * esx[j];
        val = val * esc[j];
        if (p.bias) val = val + bits_to_f32_rt(ebv[j], p.bias_dtype);
        store_rt(p.y, p.y_dtype, m * p.ldy + nn, val);
    }
    }
}

inline bool a8_smallm_ok(const GemmI8Args& p) {
    return p.M <= 32 && p.K % 256 == 0 && p.group_size % 16 == 0 && p.ldq % 16 == 0 && (uintptr_t)p.q % 16 == 0 &&
           p.ldx % 16 == 0 && (uintptr_t)p.xq % 16 == 0;
}

// The decode-once branch of launch_o (the small-M kernel aside).
inline bool a8_takes_decode_once(const GemmI8Args& p) {
    return p.w8 && a8_decode_once(p.M, p.N, p.K) && p.group_size % 64 == 0 && p.ldx % 16 == 0 &&
           (uintptr_t)p.xq % 16 == 0 && (uintptr_t)p.w8 % 16 == 0;
}

template <int BITS, bool CB, typename TSrel>
hipError_t launch_o(const GemmI8Args& p, hipStream_t st) {
    if (p.y_dtype != DT_F32 && p.y_dtype != DT_F16 && p.y_dtype != DT_BF16) return hipErrorInvalidValue;
    if (p.lora.t && !gemm_i8_fuses_lora(p)) return hipErrorInvalidValue;  // only the DMA GEMM adds LoRA
    if (a8_smallm_ok(p)) {
        if (p.res.r) return hipErrorInvalidValue;  // the caller checks gemm_i8_fuses_residual first
        const dim3 grid((unsigned)((p.N + 15) / 16)), block(512);
        if (p.M <= 16) hipLaunchKernelGGL((a8_smallm_kernel<BITS, CB, TSrel, 1>), grid, block, 0, st, p);
        else hipLaunchKernelGGL((a8_smallm_kernel<BITS, CB, TSrel, 2>), grid, block, 0, st, p);
        return hipGetLastError();
    }
    if (a8_takes_decode_once(p)) {
        const int64_t segs = p.N * (p.K / 64);
        if (4 * segs + 256 > (int64_t)UINT32_MAX) return hipErrorInvalidValue;  // the grid kernel's 32-bit indices
        if (!p.w8_ready) {
            hipLaunchKernelGGL((a8_grid_kernel<BITS, CB, TSrel>), dim3((unsigned)((4 * segs + 255) / 256)), dim3(256), 0,
                               st, p, p.w8);
            hipError_t err = hipGetLastError();
            if (err != hipSuccess) return err;
        }
        auto tiles = [&](int bm, int bn) { return ((p.M + bm - 1) / bm) * ((p.N + bn - 1) / bn); };
        // LoRA term in the epilogue by up dtype (none: -1)
        const int ldu = !p.lora.t ? -1 : p.lora.up_dt;
        auto go = [&]<int BMV, int BNV>() {
            const dim3 grid((unsigned)tiles(BMV, BNV));
            switch (ldu) {
                case -1: hipLaunchKernelGGL((gemm_i8dma_kernel<BMV, BNV, 128, 2, false>), grid, dim3(512), 0, st, p, p.w8); break;
                case DT_BF16: hipLaunchKernelGGL((gemm_i8dma_kernel<BMV, BNV, 128, 2, false, DT_BF16>), grid, dim3(512), 0, st, p, p.w8); break;
                case DT_F16: hipLaunchKernelGGL((gemm_i8dma_kernel<BMV, BNV, 128, 2, false, DT_F16>), grid, dim3(512), 0, st, p, p.w8); break;
                case DT_F32: hipLaunchKernelGGL((gemm_i8dma_kernel<BMV, BNV, 128, 2, false, DT_F32>), grid, dim3(512), 0, st, p, p.w8); break;
            }
        };
        if (ldu != -1 && ldu != DT_BF16 && ldu != DT_F16 && ldu != DT_F32) return hipErrorInvalidValue;
        const int64_t m1 = ldu == -1 && tiles(256, 256) >= 192 ? tail_split_rows(p.M, p.N) : 0;
        if (m1) {  // whole rounds of 256 x 256 tiles, then the rest as one round of 128 x 256 tiles
            GemmI8Args top = p, rest = p;
            top.M = m1;
            rest.M = p.M - m1;
            rest.xq = p.xq + m1 * p.ldx;
            rest.sx = p.sx + m1;
            rest.y = (uint8_t*)p.y + m1 * p.ldy * dt_bytes(p.y_dtype);
            if (p.res.r) rest.res.r = (const uint8_t*)p.res.r + m1 * p.res.ldr * dt_bytes(p.res.r_dt);
            auto tiles_of = [](const GemmI8Args& g, int bm) { return ((g.M + bm - 1) / bm) * ((g.N + 255) / 256); };
            hipLaunchKernelGGL((gemm_i8dma_kernel<256, 256, 128, 2, false>), dim3((unsigned)tiles_of(top, 256)), dim3(512), 0,
                               st, top, top.w8);
            const hipError_t err = hipGetLastError();
            if (err != hipSuccess) return err;
            hipLaunchKernelGGL((gemm_i8dma_kernel<128, 256, 128, 2, false>), dim3((unsigned)tiles_of(rest, 128)), dim3(512),
                               0, st, rest, rest.w8);
            return hipGetLastError();
        }
        if (tiles(256, 256) >= 192)
            go.template operator()<256, 256>();
        // 128 x 160 tiles (2 x 5 waves, no LoRA term) when they make one round of at least 3/4 of
        // the 256 CUs and 256 x 256 tiles would not fill the GPU (M1024 N5120: 256 of them)
        else if (ldu == -1 && tiles(128, 160) >= 192 && tiles(128, 160) <= 256) {
            const dim3 grid((unsigned)tiles(128, 160));
            hipLaunchKernelGGL((gemm_i8dma_kernel<128, 160, 128, 2, false, -1, 2, 5>), grid,
                               dim3(i8dma_threads<2, 5>()), 0, st, p, p.w8);
        }
        // 128 x 256 also when it fits one round on the 256 CUs and 128 x 128 would not: one round of
        // the larger tile beats 1.25 rounds of the smaller (M1024 K13824 N5120: 150.6 vs 157.1 us)
        else if (tiles(128, 256) >= 192 || (tiles(128, 256) <= 256 && tiles(128, 128) > 256))
            go.template operator()<128, 256>();
        else if (tiles(128, 128) >= 128)
            go.template operator()<128, 128>();
        else  // grids of fewer than 128 tiles of 128 x 128 (a few hundred rows): twice the workgroups
            go.template operator()<128, 64>();
        return hipGetLastError();
    }
    // large tiles when the grid still fills the GPU and one scale covers each row's k-tile
    const int64_t big_tiles = ((p.N + 255) / 256) * ((p.M + 255) / 256);
    if (p.group_size % 64 == 0 && p.K % BKA == 0 && p.ldq % 16 == 0 && big_tiles >= 192) {
        dim3 grid((unsigned)big_tiles), block(512);
        if (p.group_size >= 128)  // one scale per k-tile row: the decoding thread pair shares its table
            hipLaunchKernelGGL((gemm_a8_kernel<BITS, CB, TSrel, true>), grid, block, 0, st, p);
        else
            hipLaunchKernelGGL((gemm_a8_kernel<BITS, CB, TSrel, false>), grid, block, 0, st, p);
        return hipGetLastError();
    }
    if (p.res.r) return hipErrorInvalidValue;  // the caller checks gemm_i8_fuses_residual first
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

template <int BITS, bool CB>
hipError_t launch_grid(const GemmI8Args& p, hipStream_t st) {
    const int64_t segs = p.N * (p.K / 64);
    if (4 * segs + 256 > (int64_t)UINT32_MAX) return hipErrorInvalidValue;  // the kernel's 32-bit indices
    const dim3 grid((unsigned)((4 * segs + 255) / 256));
    switch (p.s_rel_dtype) {
        case DT_E4M3: hipLaunchKernelGGL((a8_grid_kernel<BITS, CB, uint8_t>), grid, dim3(256), 0, st, p, p.w8); break;
        case DT_F16: hipLaunchKernelGGL((a8_grid_kernel<BITS, CB, f16>), grid, dim3(256), 0, st, p, p.w8); break;
        case DT_BF16: hipLaunchKernelGGL((a8_grid_kernel<BITS, CB, bf16_t>), grid, dim3(256), 0, st, p, p.w8); break;
        case DT_F32: hipLaunchKernelGGL((a8_grid_kernel<BITS, CB, float>), grid, dim3(256), 0, st, p, p.w8); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace

// The conditions under which launch_o takes the decode-once DMA GEMM, and the LoRA operands it reads
// with 16-byte loads.
bool gemm_i8_fuses_lora(const GemmI8Args& p) {
    const bool dma = p.w8 && a8_decode_once(p.M, p.N, p.K) && p.group_size % 64 == 0 && p.ldx % 16 == 0 &&
                     (uintptr_t)p.xq % 16 == 0 && (uintptr_t)p.w8 % 16 == 0 && !a8_smallm_ok(p);
    const LoraTile& L = p.lora;
    const int es = L.up_dt == DT_F32 ? 4 : 2;
    return dma && L.t && L.up && L.R >= 8 && L.R % 8 == 0 && L.R <= 2 * i8dma_lora_rank(L.up_dt) &&
           (uintptr_t)L.t % 16 == 0 && (uintptr_t)L.up % 16 == 0 &&
           (L.ld_up * es) % 16 == 0 && (L.up_dt == DT_BF16 || L.up_dt == DT_F16 || L.up_dt == DT_F32);
}

// The large-tile kernels launch_o takes (the decode-once DMA GEMM, the fused-decode 256 x 256
// GEMM) apply p.res in their staged epilogue; the small-M and 128 x 128 kernels do not.
bool gemm_i8_fuses_residual(const GemmI8Args& p) {
    if (a8_smallm_ok(p)) return false;
    if (p.w8 && a8_decode_once(p.M, p.N, p.K) && p.group_size % 64 == 0 && p.ldx % 16 == 0 &&
        (uintptr_t)p.xq % 16 == 0 && (uintptr_t)p.w8 % 16 == 0)
        return true;
    const int64_t big_tiles = ((p.N + 255) / 256) * ((p.M + 255) / 256);
    return p.group_size % 64 == 0 && p.K % BKA == 0 && p.ldq % 16 == 0 && big_tiles >= 192;
}

bool a8_grid_supported(const GemmI8Args& p) {
    return (p.bits == 4 || (p.bits == 6 && !p.codebook)) && p.K % 64 == 0 && p.group_size % 64 == 0 &&
           p.ldq % 16 == 0 && (uintptr_t)p.q % 16 == 0 && (uintptr_t)p.w8 % 16 == 0;
}

hipError_t run_a8_grid(const GemmI8Args& p, hipStream_t st) {
    if (p.N == 0 || p.K == 0) return hipSuccess;
    if (!a8_grid_supported(p)) return hipErrorInvalidValue;
    if (p.bits == 4) return p.codebook ? launch_grid<4, true>(p, st) : launch_grid<4, false>(p, st);
    return launch_grid<6, false>(p, st);
}

bool a8_prepass_supported(const PrologueArgs& a, const GemmI8Args& p) {
    if (p.M < A8_PREPASS_ROWS) return false;
    if (a.mode != PROLOGUE_A8 || (a.x_dtype != DT_F16 && a.x_dtype != DT_BF16) || (a.G != 128 && a.G != 256)) return false;
    if (a.M != p.M || a.M < 1 || a.K != p.K || a.K > PROLOGUE_ROW_MAX || a.qo != p.xq || a.so != p.sx || a.ldo != p.ldx ||
        a.xr)
        return false;
    int nt = 0, slots = 0;
    prologue_shape(a.K, nt, slots);
    if (slots > 2) return false;
    if (p.y_dtype != DT_F32 && p.y_dtype != DT_F16 && p.y_dtype != DT_BF16) return false;
    if (p.s_rel_dtype != DT_E4M3 && p.s_rel_dtype != DT_F16 && p.s_rel_dtype != DT_BF16 && p.s_rel_dtype != DT_F32)
        return false;
    if (p.K % 64 || !a8_grid_supported(p) || a8_smallm_ok(p) || !a8_takes_decode_once(p)) return false;
    const int64_t threads = 4 * p.N * (p.K / 64);
    return threads + nt <= (int64_t)UINT32_MAX && p.M + (threads + nt - 1) / nt <= INT32_MAX;
}

hipError_t run_a8_prepass(const PrologueArgs& a, const GemmI8Args& p, hipStream_t st) {
    if (!a8_prepass_supported(a, p)) return hipErrorInvalidValue;
    int nt = 0, slots = 0;
    prologue_shape(a.K, nt, slots);
    const int64_t blocks = p.M + (4 * p.N * (p.K / 64) + nt - 1) / nt;
    const A8PrepassArgs pa{a.x, a.ldx, (a.K % 16 == 0) && (a.ldx % 16 == 0) && (a.ldo % 16 == 0) && ((uintptr_t)a.x % 64 == 0),
                           a.qo, a.so};
    auto go = [&](auto kern) {
        hipLaunchKernelGGL(kern, dim3((unsigned)blocks), dim3((unsigned)nt), 0, st, pa, p);
        return hipGetLastError();
    };
    auto by_bits = [&]<typename TIn, int G, int SL>() {
        return p.bits == 4 ? go(a8_prepass_kernel<TIn, G, SL, 4>) : go(a8_prepass_kernel<TIn, G, SL, 6>);
    };
    auto by_slots = [&]<typename TIn, int G>() {
        return slots <= 1 ? by_bits.template operator()<TIn, G, 1>() : by_bits.template operator()<TIn, G, 2>();
    };
    auto by_group = [&]<typename TIn>() {
        return a.G == 128 ? by_slots.template operator()<TIn, 128>() : by_slots.template operator()<TIn, 256>();
    };
    return a.x_dtype == DT_F16 ? by_group.template operator()<f16>() : by_group.template operator()<bf16_t>();
}

hipError_t run_gemm_i8(const GemmI8Args& p, hipStream_t st) {
    if (p.M == 0 || p.N == 0) return hipSuccess;
    if (p.K % 64 != 0) return hipErrorInvalidValue;
    if (p.bits == 4) return p.codebook ? launch_s<4, true>(p, st) : launch_s<4, false>(p, st);
    if (p.bits == 6) return launch_s<6, false>(p, st);
    return hipErrorInvalidValue;
}

}  // namespace qlin
