// Weight-only linear for large M on the fp16 MFMA (v_mfma_f32_16x16x32_f16), fp32 accumulate.
//
// Tile 128 (M) x 128 (N) x 64 (K), 256 threads = 4 waves in a 2x2 grid, each wave 64x64 (4x4
// MFMA tiles).  Activations arrive as the prologue's range-normalized fp16 rows (x * 2^-E[m]).
// The packed weight tile is decoded in the load stage, straight into the fp16 B tile in LDS:
//   INT8: w = q exactly (|q| <= 128 is exact in fp16); the per-channel scale joins the epilogue.
//   GGUF: w = fp16(value * 2^-e[n]) with value the exact fp32 decode and e[n] the row exponent of
//         max|w[n,:]| (so |w| < 1 and the fp16 GEMM cannot overflow for K <= 65504).
// Epilogue: y = acc * 2^E[m] * (scale[n] | 2^e[n]) + bias[n], cast to the output dtype.
// Global->LDS is double-buffered through registers: the next tile's loads are issued before the
// current tile's MFMAs.
#include <type_traits>
#include <utility>

#include "qlin_internal.h"
#include "lora_frag.h"
#include "gguf_exact.h"

namespace qlin {
namespace {

constexpr int BM = 128, BN = 128, BK = 64, PADK = 8, LDK = BK + PADK;  // LDS row: 72 halves

struct TileRegs {
    u32x4 a[4];   // 32 fp16 of one A row half
    u32x4 b[4];   // 32 fp16 of one B row half (already decoded)
};

__device__ __forceinline__ uint32_t pack2(f16 lo, f16 hi) {
    return (uint32_t)__builtin_bit_cast(uint16_t, lo) | ((uint32_t)__builtin_bit_cast(uint16_t, hi) << 16);
}

// 4 int8 (one dword) -> 4 exact fp16 (two dwords)
__device__ __forceinline__ void i8x4_to_f16(uint32_t w, uint32_t& lo, uint32_t& hi) {
    const uint32_t u = w ^ 0x80808080u;  // q + 128 as unsigned bytes
    const f16x2 off = {(f16)-1152.0f, (f16)-1152.0f};
    lo = __builtin_bit_cast(uint32_t, __builtin_bit_cast(f16x2, __builtin_amdgcn_perm(0x64646464u, u, 0x04010400u)) + off);
    hi = __builtin_bit_cast(uint32_t, __builtin_bit_cast(f16x2, __builtin_amdgcn_perm(0x64646464u, u, 0x04030402u)) + off);
}

// A: row r = tid/2 of the tile, 32 halves from column 32*(tid%2).
__device__ __forceinline__ void load_a(const f16* __restrict__ x, int64_t ldx, int64_t M, int64_t K, int64_t m0,
                                       int64_t k0, int tid, bool vec_ok, TileRegs& R) {
    const int r = tid >> 1, h = tid & 1;
    const int64_t m = m0 + r, k = k0 + 32 * h;
    if (m < M && vec_ok && k + 32 <= K) {
        const u32x4* p = reinterpret_cast<const u32x4*>(x + m * ldx + k);
#pragma unroll
        for (int i = 0; i < 4; ++i) R.a[i] = p[i];
    } else {
        uint32_t w[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            f16 lo = (f16)0.0f, hi = (f16)0.0f;
            if (m < M && k + 2 * i < K) lo = x[m * ldx + k + 2 * i];
            if (m < M && k + 2 * i + 1 < K) hi = x[m * ldx + k + 2 * i + 1];
            w[i] = pack2(lo, hi);
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) R.a[i] = u32x4{w[4 * i], w[4 * i + 1], w[4 * i + 2], w[4 * i + 3]};
    }
}

// INT8 weight tile: row n = tid/2, 32 int8 from column 32*(tid%2) -> 32 exact fp16.
__device__ __forceinline__ void load_b_int8(const int8_t* __restrict__ w, int64_t ldw, int64_t N, int64_t K,
                                            int64_t n0, int64_t k0, int tid, bool vec_ok, TileRegs& R) {
    const int r = tid >> 1, h = tid & 1;
    const int64_t n = n0 + r, k = k0 + 32 * h;
    uint32_t ww[8];
    if (n < N && vec_ok && k + 32 <= K) {
        const u32x4* p = reinterpret_cast<const u32x4*>(w + n * ldw + k);
        const u32x4 a = p[0], b = p[1];
        ww[0] = a.x; ww[1] = a.y; ww[2] = a.z; ww[3] = a.w; ww[4] = b.x; ww[5] = b.y; ww[6] = b.z; ww[7] = b.w;
    } else {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            uint32_t v = 0;
#pragma unroll
            for (int t = 0; t < 4; ++t)
                if (n < N && k + 4 * i + t < K) v |= (uint32_t)(uint8_t)w[n * ldw + k + 4 * i + t] << (8 * t);
            ww[i] = v;
        }
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        uint32_t p[4];
        i8x4_to_f16(ww[2 * i], p[0], p[1]);
        i8x4_to_f16(ww[2 * i + 1], p[2], p[3]);
        R.b[i] = u32x4{p[0], p[1], p[2], p[3]};
    }
}

// Decoded fp16 weight tile (WO_F16): row n = tid/2, 32 halves from column 32*(tid%2), loaded as
// stored (K % 32 == 0, 16-byte aligned rows).  Rows past N re-read row N - 1 (their outputs are
// never stored); the half past K (K % 64 == 32) is zero, as in the decoding load.
__device__ __forceinline__ void load_b_f16(const f16* __restrict__ w, int64_t ldw, int64_t N, int64_t K, int64_t n0,
                                           int64_t k0, int tid, TileRegs& R) {
    const int r = tid >> 1, h = tid & 1;
    const int64_t n = min(n0 + r, N - 1), k = k0 + 32 * h;
    const bool in = k < K;
    const u32x4* p = reinterpret_cast<const u32x4*>(w + n * ldw + (in ? k : 0));
    const u32x4 z = {0u, 0u, 0u, 0u};
#pragma unroll
    for (int i = 0; i < 4; ++i) R.b[i] = in ? p[i] : z;
}

// GGUF weight tile: row n = tid/2, 32 values from column 32*(tid%2): exact fp32 decode, scaled by
// 2^-e[n], rounded once to fp16.  Requires K % 32 == 0 and rows made of whole blocks.
template <int T>
__device__ __forceinline__ void load_b_gguf(const uint8_t* __restrict__ w, int64_t N, int64_t K,
                                            const int32_t* __restrict__ wexp, int64_t n0, int64_t k0, int tid,
                                            TileRegs& R) {
    constexpr int QK = gguf::Info<T>::QK, TS = gguf::Info<T>::TS;
    const int r = tid >> 1, h = tid & 1;
    const int64_t n = n0 + r, k = k0 + 32 * h;
    if (n < N && k < K) {
        const int64_t row_bytes = (K / QK) * TS;
        const int64_t blk = k / QK;
        const int j0 = (int)(k - blk * QK);
        const uint8_t* b = w + n * row_bytes + blk * TS;
        const int e = wexp[n];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            float v[8];
            gguf::decode8<T>(b, j0 + 8 * i, v);
            uint32_t p[4];
#pragma unroll
            for (int j = 0; j < 4; ++j)
                p[j] = pack2((f16)__builtin_ldexpf(v[2 * j], -e), (f16)__builtin_ldexpf(v[2 * j + 1], -e));
            R.b[i] = u32x4{p[0], p[1], p[2], p[3]};
        }
    } else {
#pragma unroll
        for (int i = 0; i < 4; ++i) R.b[i] = u32x4{0u, 0u, 0u, 0u};
    }
}

__device__ __forceinline__ void store_tile(f16* As, f16* Bs, int tid, const TileRegs& R) {
    const int r = tid >> 1, h = tid & 1;
    u32x4* pa = reinterpret_cast<u32x4*>(As + r * LDK + 32 * h);
    u32x4* pb = reinterpret_cast<u32x4*>(Bs + r * LDK + 32 * h);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        pa[i] = R.a[i];
        pb[i] = R.b[i];
    }
}

template <int WK, int GT>
__global__ __launch_bounds__(256) void gemm_f16_kernel(GemmF16Args a) {
    __shared__ __attribute__((aligned(16))) f16 smem[2][2][BM * LDK];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int64_t n0 = (int64_t)blockIdx.x * BN, m0 = (int64_t)blockIdx.y * BM;
    const f16* x = a.x;
    const bool a_vec = (a.ldx % 8 == 0) && ((uintptr_t)x % 16 == 0);
    const bool b_vec = (a.ldw % 16 == 0) && ((uintptr_t)a.w % 16 == 0);
    const int ktiles = (int)((a.K + BK - 1) / BK);

    f32x4 acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

    TileRegs R;
    auto fetch = [&](int kt) {
        const int64_t k0 = (int64_t)kt * BK;
        load_a(x, a.ldx, a.M, a.K, m0, k0, tid, a_vec, R);
        if constexpr (WK == WO_INT8) load_b_int8((const int8_t*)a.w, a.ldw, a.N, a.K, n0, k0, tid, b_vec, R);
        else if constexpr (WK == WO_F16) load_b_f16((const f16*)a.w, a.ldw, a.N, a.K, n0, k0, tid, R);
        else load_b_gguf<GT>((const uint8_t*)a.w, a.N, a.K, a.wexp, n0, k0, tid, R);
    };

    fetch(0);
    store_tile(smem[0][0], smem[0][1], tid, R);
    __syncthreads();
    const int r16 = lane & 15, g = lane >> 4;
    for (int kt = 0; kt < ktiles; ++kt) {
        const int buf = kt & 1;
        fetch(min(kt + 1, ktiles - 1));  // unconditional (see below); past the end: re-reads the last tile
        __builtin_amdgcn_sched_barrier(0);  // the loads go out before the MFMAs
        const f16* As = smem[buf][0];
        const f16* Bs = smem[buf][1];
#pragma unroll
        for (int kk = 0; kk < BK / 32; ++kk) {
            f16x8 af[4], bf[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                af[i] = *reinterpret_cast<const f16x8*>(As + (wm * 64 + i * 16 + r16) * LDK + kk * 32 + 8 * g);
                bf[i] = *reinterpret_cast<const f16x8*>(Bs + (wn * 64 + i * 16 + r16) * LDK + kk * 32 + 8 * g);
            }
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af[i], bf[j], acc[i][j], 0, 0, 0);
        }
        // unconditional: a conditional use lets the compiler sink the loads past the MFMAs; the
        // last iteration writes the unread buffer
        __builtin_amdgcn_sched_barrier(0);
        store_tile(smem[buf ^ 1][0], smem[buf ^ 1][1], tid, R);
        __syncthreads();
    }

    // Epilogue.  acc[i][j][v] = D[m = wm*64 + 16i + 4g + v][n = wn*64 + 16j + r16].  Its operands
    // (row and weight exponents, scales, bias) are loaded before the first store: a load between
    // stores would wait for the stores before it.
    int xev[4][4], cev[4];
    uint32_t csb[4], bvb[4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int v = 0; v < 4; ++v) xev[i][v] = a.xexp ? a.xexp[min(m0 + wm * 64 + 16 * i + 4 * g + v, a.M - 1)] : 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int64_t n = min(n0 + wn * 64 + 16 * j + r16, a.N - 1);
        if constexpr (WK == WO_INT8) {
            csb[j] = load_bits_rt(a.scale, a.scale_dtype, n * a.scale_stride);
            cev[j] = 0;
        } else {
            csb[j] = 0u;
            cev[j] = a.wexp[n];
        }
        bvb[j] = a.bias ? load_bits_rt(a.bias, a.bias_dtype, n) : 0u;
    }
    // every output in place first, then (per output dtype) its stored bits in a register of its
    // own and the stores: rewriting the data register of a store in flight would wait for it
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        float cs = 1.0f;
        if constexpr (WK == WO_INT8) cs = bits_to_f32_rt(csb[j], a.scale_dtype);
        const float bv = a.bias ? bits_to_f32_rt(bvb[j], a.bias_dtype) : 0.0f;
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                float val = __builtin_ldexpf(acc[i][j][v], xev[i][v] + cev[j]);
                if constexpr (WK == WO_INT8) val *= cs;
                val += bv;
                acc[i][j][v] = val;
            }
    }
    auto at = [&](int i, int j, int v, int64_t& idx) {
        const int64_t m = m0 + wm * 64 + 16 * i + 4 * g + v, n = n0 + wn * 64 + 16 * j + r16;
        idx = m * a.ldy + n;
        return m < a.M && n < a.N;
    };
    if (a.y_dtype == DT_F32) {
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int v = 0; v < 4; ++v) {
                    int64_t idx;
                    if (at(i, j, v, idx)) reinterpret_cast<float*>(a.y)[idx] = acc[i][j][v];
                }
    } else {
        uint32_t hb[4][4][4];
        const bool h16 = a.y_dtype == DT_F16;
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int v = 0; v < 4; ++v)
                    hb[i][j][v] = h16 ? (uint32_t)__builtin_bit_cast(uint16_t, (f16)acc[i][j][v])
                                      : (uint32_t)f32_to_bf16_bits(acc[i][j][v]);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int v = 0; v < 4; ++v) {
                    int64_t idx;
                    if (at(i, j, v, idx)) reinterpret_cast<uint16_t*>(a.y)[idx] = (uint16_t)hb[i][j][v];
                }
    }
}


// ------------------------------------------------------------------------------------------------
// INT8 weight-only kernel: 512 threads = 8 waves (4 M x 2 N), tile BM x BN x 64 with BM, BN in
// {64, 128, 256} chosen by shape (256 x 256: LDS double buffer of 2 x 72 KiB).  Two waves per SIMD, so one wave's MFMAs cover
// the other's memory waits.  The int8 tile is converted exactly in the load stage with byte
// permutes: fp16 bits 0x6400 | (q + 128) = 1024 + q + 128, minus 1152, two values per packed add.
// The next k-tile's loads are issued before the current tile's MFMAs and staged after them.
// ------------------------------------------------------------------------------------------------
constexpr int WBK = 64, WLDK = WBK + 8;  // k-tile and LDS row stride (halves)

// Tile order for an 8-XCD part (block b runs on XCD b % 8): each XCD takes a contiguous run of the
// tile sequence, which walks groups of 4 M-tiles across all N-tiles, so tiles resident at the same
// time on one XCD share activation and weight panels in its L2.
__device__ __forceinline__ void xcd_tile_f16(int b, int nblocks, int n_m, int n_n, int& mt, int& nt) {
    constexpr int XCD = 8, GROUP_M = 4;
    const int per = nblocks / XCD;  // the last nblocks % 8 blocks keep the plain order
    const int t = b < XCD * per ? (b % XCD) * per + b / XCD : b;
    const int group = t / (GROUP_M * n_n);
    const int first_m = group * GROUP_M;
    const int gm = min(n_m - first_m, GROUP_M);
    mt = first_m + (t % (GROUP_M * n_n)) % gm;
    nt = (t % (GROUP_M * n_n)) / gm;
}


// DEEP: two register sets, so each k-tile's loads are issued two k-tiles before they are staged
// (requires an even number of k-tiles); otherwise one.
template <int BMT, int BNT, bool DEEP>
__global__ __launch_bounds__(512) void gemm_wo_i8_kernel(GemmF16Args a) {
    constexpr int NT = 512;
    constexpr int WM = BMT / 4, WN = BNT / 2;
    // 32 x 32 x 16 MFMA sub-tiles where the wave tile allows (about 1.6x the throughput of the
    // 16 x 16 x 32 form here), else 16 x 16 x 32
    constexpr bool MF32 = WM % 32 == 0 && WN % 32 == 0;
    constexpr int SUB = MF32 ? 32 : 16, TI = WM / SUB, TJ = WN / SUB;
    constexpr int UA = WBK / 8;                 // 16-byte activation units per row and k-tile
    constexpr int NA = BMT * UA / NT;           // ... per thread
    constexpr int TPR = NT / BNT;               // threads per weight row
    constexpr int VPT = WBK / TPR;              // weight values (bytes) per thread and k-tile
    static_assert(NA >= 1 && TI >= 1 && TJ >= 1 && VPT % 8 == 0, "tile shape");
    // one LDS block: double-buffered operands in the loop, then the output staging of the epilogue
    __shared__ __attribute__((aligned(16))) f16 smem[2 * (BMT + BNT) * WLDK];
    f16 (*As)[BMT * WLDK] = reinterpret_cast<f16 (*)[BMT * WLDK]>(smem);
    f16 (*Bs)[BNT * WLDK] = reinterpret_cast<f16 (*)[BNT * WLDK]>(smem + 2 * BMT * WLDK);
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int r16 = lane & 15, g = lane >> 4, r32 = lane & 31, h32 = lane >> 5;
    int mt, nt;
    xcd_tile_f16(blockIdx.x, (int)gridDim.x, (int)((a.M + BMT - 1) / BMT), (int)((a.N + BNT - 1) / BNT), mt, nt);
    const int64_t n0 = (int64_t)nt * BNT, m0 = (int64_t)mt * BMT;
    const int ktiles = (int)(a.K / WBK);

    // rows past M or N re-read the last row (never stored); pointers fixed along K
    const f16* arow[NA];
#pragma unroll
    for (int i = 0; i < NA; ++i) {
        const int u = tid + NT * i;
        arow[i] = a.x + min(m0 + u / UA, a.M - 1) * a.ldx + 8 * (u % UA);
    }
    const int br = tid / TPR, bh = tid % TPR;  // weight row br, values VPT*bh .. of a k-tile
    const int8_t* wrow = (const int8_t*)a.w + min(n0 + br, a.N - 1) * a.ldw + VPT * bh;

    struct Regs {
        u32x4 a[NA];
        uint32_t b[VPT / 4];
    };
    auto fetch = [&](int kt, Regs& R) {
        const int k0 = min(kt, ktiles - 1) * WBK;  // past the end: re-reads the last tile
#pragma unroll
        for (int i = 0; i < NA; ++i) R.a[i] = *reinterpret_cast<const u32x4*>(arow[i] + k0);
        if constexpr (VPT >= 16) {
#pragma unroll
            for (int h = 0; h < VPT / 16; ++h) {
                const u32x4 v = *reinterpret_cast<const u32x4*>(wrow + k0 + 16 * h);
                R.b[4 * h] = v.x; R.b[4 * h + 1] = v.y; R.b[4 * h + 2] = v.z; R.b[4 * h + 3] = v.w;
            }
        } else {
            const u32x2 v = *reinterpret_cast<const u32x2*>(wrow + k0);
            R.b[0] = v.x; R.b[1] = v.y;
        }
    };
    auto stage = [&](int buf, const Regs& R) {
#pragma unroll
        for (int i = 0; i < NA; ++i) {
            const int u = tid + NT * i;
            *reinterpret_cast<u32x4*>(&As[buf][(u / UA) * WLDK + 8 * (u % UA)]) = R.a[i];
        }
        u32x4* pb = reinterpret_cast<u32x4*>(&Bs[buf][br * WLDK + VPT * bh]);
#pragma unroll
        for (int h = 0; h < VPT / 8; ++h) {
            uint32_t o[4];
            i8x4_to_f16(R.b[2 * h], o[0], o[1]);
            i8x4_to_f16(R.b[2 * h + 1], o[2], o[3]);
            pb[h] = u32x4{o[0], o[1], o[2], o[3]};
        }
    };

    typedef typename std::conditional<MF32, f32x16, f32x4>::type Acc;
    Acc acc[TI][TJ];
#pragma unroll
    for (int i = 0; i < TI; ++i)
#pragma unroll
        for (int j = 0; j < TJ; ++j)
#pragma unroll
            for (int r = 0; r < (MF32 ? 16 : 4); ++r) acc[i][j][r] = 0.f;
    auto compute = [&](int buf) {
        if constexpr (MF32) {
            // lane l holds row (column) l % 32 and the 8 consecutive k 8 (l / 32) .. + 7 of a
            // 16-value step, in both operands alike
            const f16* as = &As[buf][(wm * WM + r32) * WLDK + 8 * h32];
            const f16* bs = &Bs[buf][(wn * WN + r32) * WLDK + 8 * h32];
#pragma unroll
            for (int kk = 0; kk < WBK / 16; ++kk) {
                f16x8 bf[TJ];
#pragma unroll
                for (int j = 0; j < TJ; ++j) bf[j] = *reinterpret_cast<const f16x8*>(bs + 32 * j * WLDK + 16 * kk);
#pragma unroll
                for (int i = 0; i < TI; ++i) {
                    const f16x8 af = *reinterpret_cast<const f16x8*>(as + 32 * i * WLDK + 16 * kk);
#pragma unroll
                    for (int j = 0; j < TJ; ++j)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af, bf[j], acc[i][j], 0, 0, 0);
                }
            }
        } else {
            const f16* as = &As[buf][(wm * WM + r16) * WLDK + 8 * g];
            const f16* bs = &Bs[buf][(wn * WN + r16) * WLDK + 8 * g];
#pragma unroll
            for (int kk = 0; kk < WBK / 32; ++kk) {
                f16x8 bf[TJ];
#pragma unroll
                for (int j = 0; j < TJ; ++j) bf[j] = *reinterpret_cast<const f16x8*>(bs + 16 * j * WLDK + 32 * kk);
#pragma unroll
                for (int i = 0; i < TI; ++i) {
                    const f16x8 af = *reinterpret_cast<const f16x8*>(as + 16 * i * WLDK + 32 * kk);
#pragma unroll
                    for (int j = 0; j < TJ; ++j)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(af, bf[j], acc[i][j], 0, 0, 0);
                }
            }
        }
    };
    // Each step: loads for a later tile go out first (sched_barrier), then this tile's MFMAs, then
    // (after another sched_barrier: staging waits for loads) the next tile is staged.  Every load
    // is used unconditionally: a conditional use lets the compiler sink it past the MFMAs.
    Regs R0, R1;
    fetch(0, R0);
    stage(0, R0);
    if constexpr (DEEP) {
        fetch(1, R1);
        __syncthreads();
        for (int kt = 0; kt < ktiles; kt += 2) {
            fetch(kt + 2, R0);
            __builtin_amdgcn_sched_barrier(0);
            compute(0);
            __builtin_amdgcn_sched_barrier(0);
            stage(1, R1);
            __syncthreads();
            fetch(kt + 3, R1);
            __builtin_amdgcn_sched_barrier(0);
            compute(1);
            __builtin_amdgcn_sched_barrier(0);
            stage(0, R0);
            __syncthreads();
        }
    } else {
        __syncthreads();
        for (int kt = 0; kt < ktiles; ++kt) {
            const int buf = kt & 1;
            fetch(kt + 1, R0);
            __builtin_amdgcn_sched_barrier(0);
            compute(buf);
            __builtin_amdgcn_sched_barrier(0);
            stage(buf ^ 1, R0);
            __syncthreads();
        }
    }

    // Epilogue: y = ldexp(acc, xexp[m]) * scale[n] + bias[n].  The fp32 tile goes through LDS in
    // passes of RP rows (row stride BNT + 8 words), then every thread writes 8 consecutive outputs of
    // a row with 16-byte stores.  32 x 32 sub-tiles: lane l, register r holds row 8 (r / 4) +
    // 4 (l / 32) + r % 4, column l % 32; 16 x 16: row 4 (l / 16) + r, column l % 16.
    // Every operand of the epilogue is requested before the first store (the tile's row exponents
    // go to LDS): a global load between the stores would wait for the stores before it.  Each pass
    // computes all of a thread's outputs before its stores; the passes synchronize LDS only.
    constexpr int ORW = BNT + 8, ERB = BMT * 4;
    constexpr int CPR = BNT / 8;                 // 8-column chunks per row
    constexpr int RP = (BMT * CPR / NT <= 4 && BMT * ORW * 4 + ERB <= (int)sizeof(smem)) ? BMT
                       : (BMT / 2 * CPR / NT <= 4 && BMT / 2 * ORW * 4 + ERB <= (int)sizeof(smem)) ? BMT / 2 : BMT / 4;
    static_assert(RP * ORW * 4 + ERB <= (int)sizeof(smem) && RP % WM == 0, "output staging must fit");
    static_assert(NT % CPR == 0 && (RP * CPR) % NT == 0, "chunks must split evenly");
    constexpr int Q = RP * CPR / NT;             // chunks per thread and pass
    float* ot = reinterpret_cast<float*>(smem);
    int* erow = reinterpret_cast<int*>(reinterpret_cast<uint8_t*>(smem) + sizeof(smem) - ERB);
    const int cc = tid % CPR;                    // this thread's chunk (the same in every pass)
    const int64_t nc = n0 + 8 * cc;
    const int ncount = (int)max<int64_t>(0, min<int64_t>(8, a.N - nc));
    const int xer = a.xexp ? a.xexp[min(m0 + min(tid, BMT - 1), (int64_t)a.M - 1)] : 0;
    uint32_t csb[8], bvb[8], rsb[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        const int64_t n = min(nc + e, a.N - 1);
        csb[e] = load_bits_rt(a.scale, a.scale_dtype, n * a.scale_stride);
        bvb[e] = a.bias ? load_bits_rt(a.bias, a.bias_dtype, n) : 0u;
    }
    residual_scale_bits8(a.res, nc, a.N, rsb);
    float cs[8], bv[8], rsv[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        cs[e] = bits_to_f32_rt(csb[e], a.scale_dtype);
        bv[e] = a.bias ? bits_to_f32_rt(bvb[e], a.bias_dtype) : 0.0f;
    }
    residual_scales8(a.res, rsb, rsv);
    const bool vec = (a.ldy % 8 == 0) && ((uintptr_t)a.y % 16 == 0);
#pragma unroll
    for (int pass = 0; pass < BMT / RP; ++pass) {
        lds_barrier();  // the operand buffers (or the previous pass) are no longer read
        if (pass == 0 && tid < BMT) erow[tid] = xer;
        if ((wm * WM) / RP == pass) {
            const int rw = wm * WM - pass * RP;  // this wave's first row in the staging block
#pragma unroll
            for (int i = 0; i < TI; ++i)
#pragma unroll
                for (int j = 0; j < TJ; ++j)
#pragma unroll
                    for (int r = 0; r < (MF32 ? 16 : 4); ++r) {
                        const int row = MF32 ? rw + 32 * i + 8 * (r / 4) + 4 * h32 + r % 4 : rw + 16 * i + 4 * g + r;
                        const int col = MF32 ? wn * WN + 32 * j + r32 : wn * WN + 16 * j + r16;
                        ot[row * ORW + col] = acc[i][j][r];
                    }
        }
        lds_barrier();
        float v[Q][8];
#pragma unroll
        for (int q = 0; q < Q; ++q) {
            const int row = tid / CPR + (NT / CPR) * q;
            const f32x4 v0 = *reinterpret_cast<const f32x4*>(ot + row * ORW + 8 * cc);
            const f32x4 v1 = *reinterpret_cast<const f32x4*>(ot + row * ORW + 8 * cc + 4);
            const int e2 = erow[pass * RP + row];
#pragma unroll
            for (int e = 0; e < 8; ++e) v[q][e] = __builtin_ldexpf(e < 4 ? v0[e] : v1[e - 4], e2) * cs[e] + bv[e];
        }
        int64_t mq[Q];
#pragma unroll
        for (int q = 0; q < Q; ++q) mq[q] = m0 + pass * RP + tid / CPR + (NT / CPR) * q;
        if (a.res.r) residual_apply8<Q>(a.res, mq, nc, a.M, a.N, rsv, v);
#pragma unroll
        for (int q = 0; q < Q; ++q) {
            const int64_t m = mq[q];
            if (m < a.M && ncount > 0) store8_rt(a.y, a.y_dtype, m * a.ldy + nc, v[q], ncount, vec);
        }
    }
}

// INT8 weight-only GEMM with both operands moved by LDS DMA: y = epilogue(x[M, K] . w[N, K]^T), x the
// normalized fp16 activations, w the int8 weights as stored (no widening before LDS, so a 64-value
// k-tile brings in 32 KB of activations and 16 KB of weights).  Tile BMT x 256, 8 waves 2 (M) x
// 4 (N), v_mfma_f32_32x32x16_f16, STAGES k-tiles in flight.
//
// k order inside a 64-value k-tile: MFMA step s = 2p + e (p, e in {0, 1}) gives the lanes of half
// h (lane / 32) the 8 values k = 32p + 16h + 8e .. + 7 in both operands, so one 16-byte read of a
// weight row (chunk 2p + h, 16 int8) feeds steps 2p and 2p + 1.  The int8 values become exact fp16
// in registers after the read.  LDS rows: activations 128 bytes (8 chunks, chunk c of row r stored
// at c ^ (r / 2) % 8), weights 64 bytes (4 chunks, at c ^ (r / 4) % 4): the 16 rows a 16-lane group
// reads land in 16 distinct bank groups.
// LDU >= 0: the LoRA term of a.lora (up of dtype LDU) joins the epilogue: the accumulators become
// their fp32 base values ldexp(acc, E) * scale + bias, then base + lora_scale * t up^T with t and up
// staged through LDS (lora_tile_epilogue), the order of the separate LoRA kernel; the staged values
// are final, so the output is rounded once.
// Largest LoRA rank the 256 x 256, 3-stage kernel stages in its LDS at once (the row exponents
// aside); twice that is added in two passes.
constexpr int wo_dma_lora_rank(int du) {
    constexpr int lds = 3 * (256 * 64 * 2 + 256 * 64) - 256 * 4;
    return du == DT_F32 ? lora_max_rank<DT_F32, 256, 256>(lds) : lora_max_rank<DT_BF16, 256, 256>(lds);
}

template <int BMT, int STAGES, int LDU = -1>
__global__ __launch_bounds__(512) void gemm_wo_dma_kernel(GemmF16Args a) {
    constexpr int NT = 512, BNT = 256, KT = 64;
    // waves 2 (M) x 4 (N): each converted weight fragment feeds TI = 4 activation sub-tiles
    constexpr int WM = BMT / 2, WN = BNT / 4, TI = WM / 32, TJ = WN / 32;
    constexpr int ASZ = BMT * KT * 2, BSZ = BNT * KT;   // bytes per stage
    constexpr int NA = ASZ / 16 / NT, NB = BSZ / 16 / NT;
    static_assert(TI >= 1 && NA * 16 * NT == ASZ && NB * 16 * NT == BSZ, "tile shape");
    __shared__ __attribute__((aligned(16))) uint8_t smem[STAGES * (ASZ + BSZ)];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave & 1, wn = wave >> 1, r32 = lane & 31, h = lane >> 5;
    int mt, nt;
    xcd_tile_f16(blockIdx.x, (int)gridDim.x, (int)((a.M + BMT - 1) / BMT), (int)((a.N + BNT - 1) / BNT), mt, nt);
    const int64_t n0 = (int64_t)nt * BNT, m0 = (int64_t)mt * BMT;
    const int ktiles = (int)(a.K / KT);

    // DMA instruction i of wave w fills physical chunk u = NT i + 64 w + lane of a stage: activation
    // row u / 8, weight row u / 4.  The logical chunk it holds is the same for every i.
    const int ca = (lane % 8) ^ ((4 * wave + lane / 16) % 8);
    const int cb = (lane % 4) ^ (lane / 16);
    const f16* asrc[NA];
    const int8_t* bsrc[NB];
#pragma unroll
    for (int i = 0; i < NA; ++i)
        asrc[i] = a.x + min(m0 + (NT * i + 64 * wave + lane) / 8, a.M - 1) * a.ldx + 8 * ca;
#pragma unroll
    for (int i = 0; i < NB; ++i)
        bsrc[i] = (const int8_t*)a.w + min(n0 + (NT * i + 64 * wave + lane) / 4, a.N - 1) * a.ldw + 16 * cb;
    auto dma = [&](int kt, int buf) {
        const int k0 = min(kt, ktiles - 1) * KT;  // past the end: re-reads the last tile
        uint8_t* st = smem + buf * (ASZ + BSZ);
#pragma unroll
        for (int i = 0; i < NA; ++i) lds_dma16(asrc[i] + k0, st + 16 * (NT * i + 64 * wave));
#pragma unroll
        for (int i = 0; i < NB; ++i) lds_dma16(bsrc[i] + k0, st + ASZ + 16 * (NT * i + 64 * wave));
    };

    f32x16 acc[TI][TJ];
#pragma unroll
    for (int i = 0; i < TI; ++i)
#pragma unroll
        for (int j = 0; j < TJ; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;
    // this lane's rows: activation rows wm WM + 32 i + r32 (swizzle (row / 2) % 8 = (r32 / 2) % 8
    // since WM and 32 are multiples of 16), weight rows wn WN + 32 j + r32 (swizzle (r32 / 4) % 4)
    const int swa = (r32 / 2) % 8, swb = (r32 / 4) % 4;
    auto mfmas = [&](int buf) {
        const uint8_t* as = smem + buf * (ASZ + BSZ) + (wm * WM + r32) * (KT * 2);
        const uint8_t* bs = smem + buf * (ASZ + BSZ) + ASZ + (wn * WN + r32) * KT;
#pragma unroll
        for (int pp = 0; pp < 2; ++pp) {
            f16x8 bf[2][TJ];
#pragma unroll
            for (int j = 0; j < TJ; ++j) {
                const u32x4 q = *reinterpret_cast<const u32x4*>(bs + 32 * j * KT + 16 * ((2 * pp + h) ^ swb));
                uint32_t o[8];
                i8x4_to_f16(q.x, o[0], o[1]);
                i8x4_to_f16(q.y, o[2], o[3]);
                i8x4_to_f16(q.z, o[4], o[5]);
                i8x4_to_f16(q.w, o[6], o[7]);
                bf[0][j] = __builtin_bit_cast(f16x8, u32x4{o[0], o[1], o[2], o[3]});
                bf[1][j] = __builtin_bit_cast(f16x8, u32x4{o[4], o[5], o[6], o[7]});
            }
#pragma unroll
            for (int e = 0; e < 2; ++e) {
                const int c = 16 * ((4 * pp + 2 * h + e) ^ swa);
#pragma unroll
                for (int i = 0; i < TI; ++i) {
                    const f16x8 af = *reinterpret_cast<const f16x8*>(as + 32 * i * (KT * 2) + c);
#pragma unroll
                    for (int j = 0; j < TJ; ++j)
                        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af, bf[e][j], acc[i][j], 0, 0, 0);
                }
            }
        }
    };

    // Barrier without a memory fence: the DMA data a wave needs is covered by its wait_vmcnt, and
    // the loop writes LDS only by DMA; the fragment reads of a buffer complete before the barrier
    // after which the next DMA may overwrite it.
    constexpr int ND = NA + NB;
#pragma unroll
    for (int st = 0; st < STAGES - 1; ++st) dma(st, st);
    wait_vmcnt<(STAGES - 2) * ND>();
    __builtin_amdgcn_s_barrier();
    // unrolled by STAGES: every stage buffer index is a constant (1-2% faster on the A8 configs)
    for (int k0 = 0; k0 < ktiles; k0 += STAGES) {
#pragma unroll
        for (int s = 0; s < STAGES; ++s) {
            const int kt = k0 + s;
            if (kt >= ktiles) break;
            dma(kt + STAGES - 1, (s + STAGES - 1) % STAGES);
            __builtin_amdgcn_sched_barrier(0);
            mfmas(s);
            wait_lgkmcnt0();
            wait_vmcnt<(STAGES - 2) * ND>();  // tile kt + 1 has landed
            __builtin_amdgcn_s_barrier();
        }
    }
    wait_vmcnt<0>();

    // Epilogue: y = ldexp(acc, xexp[m]) * scale[n] + bias[n], staged through LDS in passes of RP
    // rows (row stride BNT + 8 words); every thread writes 8 consecutive outputs with 16-byte stores.
    // Lane l, register r of a 32 x 32 sub-tile holds row 8 (r / 4) + 4 (l / 32) + r % 4, column l % 32.
    // Every operand of the epilogue is requested before the first store (the tile's row exponents
    // go to LDS): a global load between the stores would wait for the stores before it (one counter
    // counts both), a memory round trip per stored row.  Each pass computes all of a thread's
    // outputs before its stores, the passes synchronize LDS only.
    constexpr int ORW = BNT + 8, ERB = BMT * 4, CPR = BNT / 8;
    constexpr int RP = (BMT * CPR / NT <= 4 && BMT * ORW * 4 + ERB <= (int)sizeof(smem)) ? BMT
                       : (BMT / 2 * CPR / NT <= 4 && BMT / 2 * ORW * 4 + ERB <= (int)sizeof(smem)) ? BMT / 2 : BMT / 4;
    static_assert(RP * ORW * 4 + ERB <= (int)sizeof(smem) && RP % 32 == 0, "output staging must fit");
    static_assert(NT % CPR == 0 && (RP * CPR) % NT == 0, "chunks must split evenly");
    constexpr int Q = RP * CPR / NT;  // chunks per thread and pass
    float* ot = reinterpret_cast<float*>(smem);
    int* erow = reinterpret_cast<int*>(smem + sizeof(smem) - ERB);
    const int cc = tid % CPR;
    const int64_t nc = n0 + 8 * cc;
    const int ncount = (int)max<int64_t>(0, min<int64_t>(8, a.N - nc));
    // row exponent of thread tid (threads past the tile re-read its last row; tid < BMT stores it)
    const int xer = a.xexp ? a.xexp[min(m0 + min(tid, BMT - 1), (int64_t)a.M - 1)] : 0;
    // the store loop's scales and bias as raw bits (with a LoRA term the staged values are final)
    constexpr int CB8 = LDU >= 0 ? 1 : 8;
    uint32_t csb[CB8], bvb[CB8];
    if constexpr (LDU < 0) {
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const int64_t n = min(nc + e, a.N - 1);
            csb[e] = load_bits_rt(a.scale, a.scale_dtype, n * a.scale_stride);
            bvb[e] = a.bias ? load_bits_rt(a.bias, a.bias_dtype, n) : 0u;
        }
    }
    uint32_t rsb[8];
    residual_scale_bits8(a.res, nc, a.N, rsb);
    const bool vec = (a.ldy % 8 == 0) && ((uintptr_t)a.y % 16 == 0);
    if constexpr (LDU >= 0) {
        constexpr int RC = lora_max_rank<LDU, BMT, BNT>((int)sizeof(smem) - BMT * 4);
        static_assert(RC == wo_dma_lora_rank(LDU), "the host's rank limit must match");
        uint32_t csj[TJ], bvj[TJ];
#pragma unroll
        for (int j = 0; j < TJ; ++j) {
            const int64_t n = min(n0 + wn * WN + 32 * j + r32, a.N - 1);
            csj[j] = load_bits_rt(a.scale, a.scale_dtype, n * a.scale_stride);
            bvj[j] = a.bias ? load_bits_rt(a.bias, a.bias_dtype, n) : 0u;
        }
        lds_barrier();  // every wave is past the main loop: the operand buffers are free
        if (tid < BMT) erow[tid] = xer;
        lds_barrier();
#pragma unroll
        for (int j = 0; j < TJ; ++j) {
            const float csn = bits_to_f32_rt(csj[j], a.scale_dtype);
            const float bvn = a.bias ? bits_to_f32_rt(bvj[j], a.bias_dtype) : 0.0f;
#pragma unroll
            for (int i = 0; i < TI; ++i)
#pragma unroll
                for (int r = 0; r < 16; ++r)
                    acc[i][j][r] = __builtin_ldexpf(acc[i][j][r], erow[wm * WM + 32 * i + 8 * (r / 4) + 4 * h + r % 4]) * csn + bvn;
        }
        lora_tile_epilogue_ranks<LDU, BMT, BNT, RC, NT, TI, TJ>(a.lora, smem, m0, n0, a.M, a.N, wm * WM, wn * WN, tid, lane, acc);
    }
    float cs[CB8], bv[CB8], rsv[8];
    residual_scales8(a.res, rsb, rsv);
    if constexpr (LDU < 0) {
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            cs[e] = bits_to_f32_rt(csb[e], a.scale_dtype);
            bv[e] = a.bias ? bits_to_f32_rt(bvb[e], a.bias_dtype) : 0.0f;
        }
    }
#pragma unroll
    for (int pass = 0; pass < BMT / RP; ++pass) {
        lds_barrier();  // the operand buffers (or the previous pass) are no longer read
        if constexpr (LDU < 0)
            if (pass == 0 && tid < BMT) erow[tid] = xer;
        // the wave's 32-row sub-tiles that fall in this pass
#pragma unroll
        for (int i = 0; i < TI; ++i)
            if ((wm * WM + 32 * i) / RP == pass) {
                const int rw = wm * WM + 32 * i - pass * RP;
#pragma unroll
                for (int j = 0; j < TJ; ++j)
#pragma unroll
                    for (int r = 0; r < 16; ++r)
                        ot[(rw + 8 * (r / 4) + 4 * h + r % 4) * ORW + wn * WN + 32 * j + r32] = acc[i][j][r];
            }
        lds_barrier();
        float v[Q][8];
#pragma unroll
        for (int q = 0; q < Q; ++q) {
            const int row = tid / CPR + (NT / CPR) * q;
            const f32x4 v0 = *reinterpret_cast<const f32x4*>(ot + row * ORW + 8 * cc);
            const f32x4 v1 = *reinterpret_cast<const f32x4*>(ot + row * ORW + 8 * cc + 4);
            if constexpr (LDU >= 0) {  // staged final values
#pragma unroll
                for (int e = 0; e < 8; ++e) v[q][e] = e < 4 ? v0[e] : v1[e - 4];
            } else {
                const int e2 = erow[pass * RP + row];
#pragma unroll
                for (int e = 0; e < 8; ++e) v[q][e] = __builtin_ldexpf(e < 4 ? v0[e] : v1[e - 4], e2) * cs[e] + bv[e];
            }
        }
        int64_t mq[Q];
#pragma unroll
        for (int q = 0; q < Q; ++q) mq[q] = m0 + pass * RP + tid / CPR + (NT / CPR) * q;
        if (a.res.r) residual_apply8<Q>(a.res, mq, nc, a.M, a.N, rsv, v);
#pragma unroll
        for (int q = 0; q < Q; ++q) {
            const int64_t m = mq[q];
            if (m < a.M && ncount > 0) store8_rt(a.y, a.y_dtype, m * a.ldy + nc, v[q], ncount, vec);
        }
    }
}

// Wait until at most (STAGES - 2) stages of this wave's DMAs are outstanding, for a wave that
// issues `nd` DMAs per stage (wave-uniform, 1..8).
template <int STAGES>
__device__ __forceinline__ void wait_stages(int nd) {
    switch (nd) {
        case 1: wait_vmcnt<(STAGES - 2) * 1>(); break;
        case 2: wait_vmcnt<(STAGES - 2) * 2>(); break;
        case 3: wait_vmcnt<(STAGES - 2) * 3>(); break;
        case 4: wait_vmcnt<(STAGES - 2) * 4>(); break;
        case 5: wait_vmcnt<(STAGES - 2) * 5>(); break;
        case 6: wait_vmcnt<(STAGES - 2) * 6>(); break;
        case 7: wait_vmcnt<(STAGES - 2) * 7>(); break;
        default: wait_vmcnt<(STAGES - 2) * 8>(); break;
    }
}

// INT8 weight-only GEMM for grids too small for 256 x 256 tiles (a few hundred activation rows):
// BMT x BNT output tiles of 32 x 32 MFMA sub-tiles.  Each wave owns one 32-column sub-tile for all
// BMT rows on one of KH parts of every k-tile, so each weight chunk is converted to fp16 once per
// workgroup and feeds BMT / 32 MFMAs; the KH partial sums are added through LDS at the end, always
// in the same order.  Both operands arrive by LDS DMA through a ring of STAGES k-tiles of KT
// values.  One DMA instruction moves whole runs of KT bytes (weights) or 2 KT bytes (activations)
// of a few rows, so each weight row is read in long contiguous runs rather than 64-byte pieces of
// thousands of rows at once.
// LDS rows hold CH = row bytes / 16 chunks; logical chunk c of row r sits at c ^ sw(r) with
// sw(r) = (r / (16 / CH)) % CH for CH < 16 and r % 16 otherwise, so the 16 rows one 16-lane group
// reads at one logical chunk land in 16 distinct 16-byte bank groups.  k order: 32-value step s of
// a k-tile, MFMA e of lane half h takes k = 32 s + 16 h + 8 e .. + 7 in both operands, so one
// 16-byte weight read (logical chunk 2 s + h) feeds both MFMAs of the step; the activation chunk
// is 4 s + 2 h + e.  W16: the weights are fp16 (a decoded GGUF tensor, y = ldexp(acc, xexp[m] +
// wexp[n]) + bias[n]), laid out in LDS like the activations, chunk 4 s + 2 h + e.
template <int BMT, int BNT, int KT>
constexpr int wo_dmas_kparts() {
    return (8 / (BNT / 32)) < (KT / 32) ? (8 / (BNT / 32)) : (KT / 32);
}
template <int BMT, int BNT, int KT>
constexpr int wo_dmas_waves() {
    return (BNT / 32) * wo_dmas_kparts<BMT, BNT, KT>();
}

template <int CH>
__device__ __forceinline__ int lds_swz(int r) {
    if constexpr (CH < 16) return (r / (16 / CH)) % CH;
    else return r % 16;
}

template <int BMT, int BNT, int KT, int STAGES, bool W16 = false>
__global__ __launch_bounds__((64 * wo_dmas_waves<BMT, BNT, KT>())) void gemm_wo_dmas_kernel(GemmF16Args a) {
    constexpr int TM = BMT / 32, TN = BNT / 32;
    constexpr int KH = wo_dmas_kparts<BMT, BNT, KT>();
    constexpr int NW = TN * KH;
    constexpr int SPW = KT / 32 / KH;                          // 32-value k steps per wave per k-tile
    constexpr int ES = W16 ? 2 : 1;                           // bytes per weight
    constexpr int CA = KT / 8, CB = KT * ES / 16;             // 16-byte chunks per LDS row
    constexpr int ASZ = BMT * KT * 2, BSZ = BNT * KT * ES;     // bytes per stage
    constexpr int WA = BMT * CA / 64, WB = BNT * CB / 64;     // wave-wide DMA instructions per stage
    constexpr int NA = (WA + NW - 1) / NW, NB = (WB + NW - 1) / NW;
    static_assert(BMT % 32 == 0 && BNT % 32 == 0 && NW <= 8 && STAGES >= 3, "tile shape");
    static_assert(KT % 64 == 0 && (KT / 32) % KH == 0, "k parts");
    static_assert((BMT * CA) % 64 == 0 && (BNT * CB) % 64 == 0, "whole DMA instructions");
    static_assert(NA + NB <= 8, "DMAs per wave");
    __shared__ __attribute__((aligned(16))) uint8_t smem[STAGES * (ASZ + BSZ)];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int r32 = lane & 31, h = lane >> 5;
    const int tn = wave % TN, kh = wave / TN;
    int mt, nt;
    xcd_tile_f16(blockIdx.x, (int)gridDim.x, (int)((a.M + BMT - 1) / BMT), (int)((a.N + BNT - 1) / BNT), mt, nt);
    const int64_t n0 = (int64_t)nt * BNT, m0 = (int64_t)mt * BMT;
    const int ktiles = (int)(a.K / KT);

    // DMA instruction j (0 <= j < WA for activations, 0 <= j < WB for weights) is issued by wave
    // j % NW and fills physical chunks u = 64 j + lane of its operand's stage: row u / CH, position
    // u % CH, holding logical chunk (u % CH) ^ sw(row).  Rows past M or N re-read the last row
    // (never stored).
    const f16* asrc[NA];
    const uint8_t* bsrc[NB];
    int na = 0, nb = 0;
#pragma unroll
    for (int i = 0; i < NA; ++i) {
        const int j = wave + NW * i, u = 64 * j + lane, row = u / CA;
        asrc[i] = a.x + min(m0 + row, a.M - 1) * a.ldx + 8 * ((u % CA) ^ lds_swz<CA>(row));
        na += j < WA;
    }
#pragma unroll
    for (int i = 0; i < NB; ++i) {
        const int j = wave + NW * i, u = 64 * j + lane, row = u / CB;
        bsrc[i] = (const uint8_t*)a.w + min(n0 + row, a.N - 1) * a.ldw * ES + 16 * ((u % CB) ^ lds_swz<CB>(row));
        nb += j < WB;
    }
    const int nd = na + nb;
    auto dma = [&](int kt, int buf) {
        const int64_t k0 = (int64_t)min(kt, ktiles - 1) * KT;  // past the end: re-reads the last tile
        uint8_t* st = smem + buf * (ASZ + BSZ);
#pragma unroll
        for (int i = 0; i < NA; ++i)
            if (i < na) lds_dma16(asrc[i] + k0, st + 16 * 64 * (wave + NW * i));
#pragma unroll
        for (int i = 0; i < NB; ++i)
            if (i < nb) lds_dma16(bsrc[i] + k0 * ES, st + ASZ + 16 * 64 * (wave + NW * i));
    };

    f32x16 acc[TM];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[i][r] = 0.f;
    const int rb = 32 * tn + r32, swb = lds_swz<CB>(rb);
    int swa[TM];
#pragma unroll
    for (int i = 0; i < TM; ++i) swa[i] = lds_swz<CA>(32 * i + r32);
    auto mfmas = [&](int buf) {
        const uint8_t* as = smem + buf * (ASZ + BSZ) + r32 * (KT * 2);
        const uint8_t* bs = smem + buf * (ASZ + BSZ) + ASZ + rb * (KT * ES);
        // every fragment of the k-tile is read before the first MFMA
        u32x4 q[SPW];
        f16x8 bw[W16 ? SPW : 1][2];
        f16x8 av[SPW][TM][2];
#pragma unroll
        for (int j = 0; j < SPW; ++j) {
            const int s = kh * SPW + j;
            if constexpr (W16) {
#pragma unroll
                for (int e = 0; e < 2; ++e)
                    bw[j][e] = *reinterpret_cast<const f16x8*>(bs + 16 * ((4 * s + 2 * h + e) ^ swb));
            } else {
                q[j] = *reinterpret_cast<const u32x4*>(bs + 16 * ((2 * s + h) ^ swb));
            }
#pragma unroll
            for (int i = 0; i < TM; ++i)
#pragma unroll
                for (int e = 0; e < 2; ++e)
                    av[j][i][e] = *reinterpret_cast<const f16x8*>(as + 32 * i * (KT * 2) +
                                                                  16 * ((4 * s + 2 * h + e) ^ swa[i]));
        }
#pragma unroll
        for (int j = 0; j < SPW; ++j) {
            f16x8 b0, b1;
            if constexpr (W16) {
                b0 = bw[j][0];
                b1 = bw[j][1];
            } else {
                uint32_t o[8];
                i8x4_to_f16(q[j].x, o[0], o[1]);
                i8x4_to_f16(q[j].y, o[2], o[3]);
                i8x4_to_f16(q[j].z, o[4], o[5]);
                i8x4_to_f16(q[j].w, o[6], o[7]);
                b0 = __builtin_bit_cast(f16x8, u32x4{o[0], o[1], o[2], o[3]});
                b1 = __builtin_bit_cast(f16x8, u32x4{o[4], o[5], o[6], o[7]});
            }
#pragma unroll
            for (int i = 0; i < TM; ++i) acc[i] = __builtin_amdgcn_mfma_f32_32x32x16_f16(av[j][i][0], b0, acc[i], 0, 0, 0);
#pragma unroll
            for (int i = 0; i < TM; ++i) acc[i] = __builtin_amdgcn_mfma_f32_32x32x16_f16(av[j][i][1], b1, acc[i], 0, 0, 0);
        }
    };

    // Barrier without a memory fence: each wave's wait covers its own DMAs, the loop writes LDS only
    // by DMA, and the fragment reads of a buffer complete before the barrier after which the next
    // DMA may overwrite it.
#pragma unroll
    for (int st = 0; st < STAGES - 1; ++st) dma(st, st);
    wait_stages<STAGES>(nd);
    __builtin_amdgcn_s_barrier();
    // unrolled by STAGES: every stage buffer index is a constant (1-2% faster on the A8 configs)
    for (int k0 = 0; k0 < ktiles; k0 += STAGES) {
#pragma unroll
        for (int s = 0; s < STAGES; ++s) {
            const int kt = k0 + s;
            if (kt >= ktiles) break;
            dma(kt + STAGES - 1, (s + STAGES - 1) % STAGES);
            __builtin_amdgcn_sched_barrier(0);
            mfmas(s);
            wait_lgkmcnt0();
            wait_stages<STAGES>(nd);  // tile kt + 1 has landed
            __builtin_amdgcn_s_barrier();
        }
    }
    wait_vmcnt<0>();
    __syncthreads();

    // Epilogue: the sub-tiles go to LDS as fp32 (row stride BNT + 4 words), k part 0 first, then
    // parts 1 .. KH - 1 added in order.  Lane l, register r of a 32 x 32 sub-tile holds row
    // 8 (r / 4) + 4 (l / 32) + r % 4, column l % 32.  Then y = ldexp(acc, xexp[m]) * scale[n] +
    // bias[n], 8 consecutive outputs per thread with 16-byte stores.  The scales, bias and row
    // exponents are requested before the parts are added (their round trip overlaps the LDS passes,
    // and no global load sits between the stores); the passes synchronize LDS only.
    constexpr int ORW = BNT + 4;
    static_assert(BMT * ORW * 4 <= (int)sizeof(smem), "output staging must fit");
    constexpr int NT = 64 * NW, CPR = BNT / 8, Q = (BMT * CPR + NT - 1) / NT;
    float* ot = reinterpret_cast<float*>(smem);
    float* op = ot + 4 * h * ORW + 32 * tn + r32;
    int xeq[Q];
    uint32_t csb[Q][8], bvb[Q][8], rsb[Q][8];
#pragma unroll
    for (int q = 0; q < Q; ++q) {
        const int c = min(tid + NT * q, BMT * CPR - 1), row = c / CPR, cq = c % CPR;
        xeq[q] = a.xexp ? a.xexp[min(m0 + row, (int64_t)a.M - 1)] : 0;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const int64_t n = min(n0 + 8 * cq + e, a.N - 1);
            if constexpr (W16) csb[q][e] = (uint32_t)a.wexp[n];  // the weight row's exponent
            else csb[q][e] = load_bits_rt(a.scale, a.scale_dtype, n * a.scale_stride);
            bvb[q][e] = a.bias ? load_bits_rt(a.bias, a.bias_dtype, n) : 0u;
        }
        residual_scale_bits8(a.res, n0 + 8 * cq, a.N, rsb[q]);
    }
#pragma unroll
    for (int part = 0; part < KH; ++part) {
        if (kh == part) {
#pragma unroll
            for (int i = 0; i < TM; ++i)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    float* d = op + (32 * i + 8 * (r / 4) + r % 4) * ORW;
                    *d = part == 0 ? acc[i][r] : *d + acc[i][r];
                }
        }
        lds_barrier();
    }
    const bool vec = (a.ldy % 8 == 0) && ((uintptr_t)a.y % 16 == 0);
    float v[Q][8];
#pragma unroll
    for (int q = 0; q < Q; ++q) {
        const int c = min(tid + NT * q, BMT * CPR - 1), row = c / CPR, cq = c % CPR;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const float bv = a.bias ? bits_to_f32_rt(bvb[q][e], a.bias_dtype) : 0.0f;
            if constexpr (W16) {
                v[q][e] = __builtin_ldexpf(ot[row * ORW + 8 * cq + e], xeq[q] + (int)csb[q][e]) + bv;
            } else {
                const float cs = bits_to_f32_rt(csb[q][e], a.scale_dtype);
                v[q][e] = __builtin_ldexpf(ot[row * ORW + 8 * cq + e], xeq[q]) * cs + bv;
            }
        }
    }
    if (a.res.r) {
        int64_t mq[Q], ncq[Q];
        float rsq[Q][8];
#pragma unroll
        for (int q = 0; q < Q; ++q) {
            const int c = min(tid + NT * q, BMT * CPR - 1);
            mq[q] = m0 + c / CPR;
            ncq[q] = n0 + 8 * (c % CPR);
            residual_scales8(a.res, rsb[q], rsq[q]);
        }
        residual_apply8<Q>(a.res, mq, ncq, a.M, a.N, rsq, v);
    }
#pragma unroll
    for (int q = 0; q < Q; ++q) {
        const int c = tid + NT * q, row = c / CPR, cq = c % CPR;
        const int64_t m = m0 + row, nc = n0 + 8 * cq;
        if (c < BMT * CPR && m < a.M && nc < a.N)
            store8_rt(a.y, a.y_dtype, m * a.ldy + nc, v[q], (int)min<int64_t>(8, a.N - nc), vec);
    }
}

template <int WK, int GT>
hipError_t launch1(const GemmF16Args& a, hipStream_t st) {
    if (a.y_dtype != DT_F32 && a.y_dtype != DT_F16 && a.y_dtype != DT_BF16) return hipErrorInvalidValue;
    if constexpr (WK == WO_INT8) {
        // the largest tile whose grid still fills the GPU (about 160 workgroups or more), when the
        // operands allow 16-byte loads
        const bool vec = a.K % WBK == 0 && a.ldx % 8 == 0 && (uintptr_t)a.x % 16 == 0 && a.ldw % 16 == 0 &&
                         (uintptr_t)a.w % 16 == 0;
        auto tiles = [&](int bm, int bn) { return ((a.M + bm - 1) / bm) * ((a.N + bn - 1) / bn); };
        if (vec && tiles(256, 256) >= 160) {
            const dim3 grid((unsigned)tiles(256, 256));
            const int64_t m1 = a.lora.t ? 0 : tail_split_rows(a.M, a.N);
            if (m1) {  // whole rounds of 256 x 256 tiles, then the rest as one round of 128 x 256 tiles
                GemmF16Args top = a, rest = a;
                top.M = m1;
                rest.M = a.M - m1;
                rest.x = a.x + m1 * a.ldx;
                if (a.xexp) rest.xexp = a.xexp + m1;
                rest.y = (uint8_t*)a.y + m1 * a.ldy * dt_bytes(a.y_dtype);
                if (a.res.r) rest.res.r = (const uint8_t*)a.res.r + m1 * a.res.ldr * dt_bytes(a.res.r_dt);
                auto tiles_of = [](const GemmF16Args& g, int bm) { return ((g.M + bm - 1) / bm) * ((g.N + 255) / 256); };
                hipLaunchKernelGGL((gemm_wo_dma_kernel<256, 3>), dim3((unsigned)tiles_of(top, 256)), dim3(512), 0, st, top);
                const hipError_t err = hipGetLastError();
                if (err != hipSuccess) return err;
                hipLaunchKernelGGL((gemm_wo_dma_kernel<128, 3>), dim3((unsigned)tiles_of(rest, 128)), dim3(512), 0, st, rest);
                return hipGetLastError();
            }
            if (!a.lora.t) hipLaunchKernelGGL((gemm_wo_dma_kernel<256, 3>), grid, dim3(512), 0, st, a);
            else if (a.lora.up_dt == DT_BF16) hipLaunchKernelGGL((gemm_wo_dma_kernel<256, 3, DT_BF16>), grid, dim3(512), 0, st, a);
            else if (a.lora.up_dt == DT_F16) hipLaunchKernelGGL((gemm_wo_dma_kernel<256, 3, DT_F16>), grid, dim3(512), 0, st, a);
            else if (a.lora.up_dt == DT_F32) hipLaunchKernelGGL((gemm_wo_dma_kernel<256, 3, DT_F32>), grid, dim3(512), 0, st, a);
            else return hipErrorInvalidValue;
            return hipGetLastError();
        }
        if (a.lora.t) return hipErrorInvalidValue;  // only the 256 x 256 DMA kernel adds a LoRA term
        // grids of fewer than 160 tiles of 128 x 128: small tiles through a DMA ring, the one of
        // 64 x 128, 64 x 64, 32 x 128, 32 x 64 with the most workgroups that still run in one round
        // on the 256 CUs; the widest k-tile K allows (256 values per weight row per stage measured
        // 20% faster than 64 at M = 256, K = N = 3072)
        if (vec && tiles(128, 128) < 160) {
            int bm = 32, bn = 64, best = 0;
            for (auto [m_, n_] : {std::pair{64, 128}, {64, 64}, {32, 128}, {32, 64}}) {
                const int64_t t = tiles(m_, n_);
                if (t <= 256 && t > best) { best = (int)t; bm = m_; bn = n_; }
            }
            int kt = a.K % 256 == 0 ? 256 : a.K % 128 == 0 ? 128 : 64;
            if (bm == 64 && bn == 128 && kt == 256) kt = 128;  // 64 KB per stage would leave two stages
            const dim3 grid((unsigned)tiles(bm, bn));
#define QLIN_WOS(BMV, BNV, KTV, STV)                                                                            \
    if (bm == BMV && bn == BNV && kt == KTV) {                                                                  \
        hipLaunchKernelGGL((gemm_wo_dmas_kernel<BMV, BNV, KTV, STV>), grid, dim3(64 * wo_dmas_waves<BMV, BNV, KTV>()), 0, st, a); \
        return hipGetLastError();                                                                               \
    }
            QLIN_WOS(64, 128, 128, 4) QLIN_WOS(64, 128, 64, 8)
            QLIN_WOS(64, 64, 256, 3) QLIN_WOS(64, 64, 128, 4) QLIN_WOS(64, 64, 64, 8)
            QLIN_WOS(32, 128, 256, 3) QLIN_WOS(32, 128, 128, 6) QLIN_WOS(32, 128, 64, 8)
            QLIN_WOS(32, 64, 256, 4) QLIN_WOS(32, 64, 128, 8) QLIN_WOS(32, 64, 64, 8)
#undef QLIN_WOS
        }
        if (vec) {
        // two-deep prefetch for the smaller tiles (at 256 x 256 it spills and measured slower)
        const bool deep = (a.K / WBK) % 2 == 0;
#define QLIN_WO(BMV, BNV)                                                                                       \
    if (tiles(BMV, BNV) >= 160 || (BMV == 64 && BNV == 64)) {                                                  \
        if (deep && BMV * BNV < 256 * 256)                                                                      \
            hipLaunchKernelGGL((gemm_wo_i8_kernel<BMV, BNV, true>), dim3((unsigned)tiles(BMV, BNV)), dim3(512), 0, st, a); \
        else                                                                                                    \
            hipLaunchKernelGGL((gemm_wo_i8_kernel<BMV, BNV, false>), dim3((unsigned)tiles(BMV, BNV)), dim3(512), 0, st, a); \
        return hipGetLastError();                                                                               \
    }
            QLIN_WO(256, 256)
            QLIN_WO(128, 256)
            QLIN_WO(128, 128)
            QLIN_WO(64, 128)
            QLIN_WO(64, 64)
#undef QLIN_WO
        }
    }
    if constexpr (WK == WO_F16) {
        // decoded fp16 weights: the DMA-ring kernel with the largest tile whose grid still fills the
        // GPU in one round (256 workgroups), or 128 x 128 past that
        const bool vec = a.K % 64 == 0 && a.ldx % 8 == 0 && (uintptr_t)a.x % 16 == 0 && a.ldw % 8 == 0 &&
                         (uintptr_t)a.w % 16 == 0;
        if (vec) {
            auto tiles = [&](int bm, int bn) { return ((a.M + bm - 1) / bm) * ((a.N + bn - 1) / bn); };
            int bm = 128, bn = 128;
            if (tiles(128, 128) < 256) {
                int64_t best = 0;
                for (auto [m_, n_] : {std::pair{64, 128}, {64, 64}, {32, 128}, {32, 64}}) {
                    const int64_t t = tiles(m_, n_);
                    if (t <= 256 && t > best) { best = t; bm = m_; bn = n_; }
                }
            }
            const int kt = a.K % 128 == 0 && bm < 128 ? 128 : 64;
            const dim3 grid((unsigned)tiles(bm, bn));
#define QLIN_WOS16(BMV, BNV, KTV, STV)                                                                          \
    if (bm == BMV && bn == BNV && kt == KTV) {                                                                  \
        hipLaunchKernelGGL((gemm_wo_dmas_kernel<BMV, BNV, KTV, STV, true>), grid,                               \
                           dim3(64 * wo_dmas_waves<BMV, BNV, KTV>()), 0, st, a);                                \
        return hipGetLastError();                                                                               \
    }
            QLIN_WOS16(128, 128, 64, 4)
            QLIN_WOS16(64, 128, 128, 3) QLIN_WOS16(64, 128, 64, 6)
            QLIN_WOS16(64, 64, 128, 4) QLIN_WOS16(64, 64, 64, 8)
            QLIN_WOS16(32, 128, 128, 3) QLIN_WOS16(32, 128, 64, 6)
            QLIN_WOS16(32, 64, 128, 6) QLIN_WOS16(32, 64, 64, 8)
#undef QLIN_WOS16
        }
    }
    if (a.res.r) return hipErrorInvalidValue;  // the caller checks gemm_f16_fuses_residual first
    dim3 grid((unsigned)((a.N + BN - 1) / BN), (unsigned)((a.M + BM - 1) / BM)), block(256);
    hipLaunchKernelGGL((gemm_f16_kernel<WK, GT>), grid, block, 0, st, a);
    return hipGetLastError();
}

template <int T>
__global__ __launch_bounds__(256) void gguf_row_exp_kernel(const uint8_t* __restrict__ w, int64_t K,
                                                            int32_t* __restrict__ e) {
    constexpr int QK = gguf::Info<T>::QK, TS = gguf::Info<T>::TS;
    __shared__ float red[4];
    const int64_t n = blockIdx.x;
    const int64_t row_bytes = (K / QK) * TS;
    const uint8_t* row = w + n * row_bytes;
    float amax = 0.0f;
    for (int64_t j = (int64_t)threadIdx.x * 8; j < K; j += 256 * 8) {
        const int64_t blk = j / QK;
        float v[8];
        gguf::decode8<T>(row + blk * TS, (int)(j - blk * QK), v);
#pragma unroll
        for (int t = 0; t < 8; ++t) amax = fmaxf(amax, fabsf(v[t]));
    }
    amax = wave_max(amax);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = amax;
    __syncthreads();
    if (threadIdx.x == 0) e[n] = frexp_exp(fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3])));
}

}  // namespace

// The operand conditions under which launch1 takes the 256 x 256 DMA kernel, and the LoRA operands it
// reads with 16-byte loads.
bool gemm_f16_fuses_lora(const GemmF16Args& a) {
    if (a.wkind != WO_INT8 || a.M <= 0 || a.N <= 0) return false;
    const bool vec = a.K % WBK == 0 && a.ldx % 8 == 0 && (uintptr_t)a.x % 16 == 0 && a.ldw % 16 == 0 &&
                     (uintptr_t)a.w % 16 == 0;
    const int64_t tiles = ((a.M + 255) / 256) * ((a.N + 255) / 256);
    const LoraTile& L = a.lora;
    const int es = L.up_dt == DT_F32 ? 4 : 2;
    return vec && tiles >= 160 && L.t && L.up && L.R >= 8 && L.R % 8 == 0 && L.R <= 2 * wo_dma_lora_rank(L.up_dt) &&
           (uintptr_t)L.t % 16 == 0 &&
           (uintptr_t)L.up % 16 == 0 && (L.ld_up * es) % 16 == 0 &&
           (L.up_dt == DT_BF16 || L.up_dt == DT_F16 || L.up_dt == DT_F32);
}

// launch1 ends in a kernel with the staged 8-output epilogue (which applies a.res) whenever the
// operands allow its 16-byte loads: the INT8 DMA / register-staged kernels and the DMA-ring kernel
// on decoded fp16 weights; the generic 128 x 128 kernel (GGUF tiles decoded as loaded, unaligned
// operands) does not take a residual.
bool gemm_f16_fuses_residual(const GemmF16Args& a) {
    if (a.wkind == WO_INT8)
        return a.K % WBK == 0 && a.ldx % 8 == 0 && (uintptr_t)a.x % 16 == 0 && a.ldw % 16 == 0 && (uintptr_t)a.w % 16 == 0;
    if (a.wkind == WO_F16)
        return a.K % 64 == 0 && a.ldx % 8 == 0 && (uintptr_t)a.x % 16 == 0 && a.ldw % 8 == 0 && (uintptr_t)a.w % 16 == 0;
    return false;
}

hipError_t run_gemm_f16(const GemmF16Args& a, hipStream_t st) {
    if (a.M == 0 || a.N == 0) return hipSuccess;
    if (a.wkind == WO_INT8) return launch1<WO_INT8, 0>(a, st);
    if (a.wkind == WO_F16) {
        if (a.K % 32 || a.ldw % 8 || (uintptr_t)a.w % 16) return hipErrorInvalidValue;
        return launch1<WO_F16, 0>(a, st);
    }
    hipError_t err = hipErrorInvalidValue;
    bool ok = gguf::dispatch_type(a.gguf_type, [&]<int T>() { err = launch1<WO_GGUF, T>(a, st); });
    return ok ? err : hipErrorInvalidValue;
}

// One workgroup per weight row n: the row's exponent e[n] (of its largest |w|, as
// gguf_row_exp_kernel computes it) and the row stored as fp16(w 2^-e[n]), 8 values per 16-byte
// store.  CPT > 0: the packed row is first copied to LDS in dwords (the decode's byte reads then
// hit LDS, not the texture path), and each thread decodes its CPT chunks of 8 values (chunk c at
// 8 (tid + 256 c)) once and keeps them in registers (K <= 2048 CPT); CPT = 0: any K, the row
// decoded twice from global memory (the second time from cache).
template <int T, int CPT>
__global__ __launch_bounds__(256) void gguf_decode_f16_kernel(const uint8_t* __restrict__ w, int64_t row_bytes,
                                                              int64_t K, int32_t* __restrict__ wexp,
                                                              f16* __restrict__ out) {
    constexpr int QK = gguf::Info<T>::QK, TS = gguf::Info<T>::TS;
    constexpr int RW = CPT > 0 ? (CPT * 2048 / QK * TS + 3) / 4 : 1;  // dwords of the longest row
    __shared__ float red[4];
    __shared__ uint32_t rs[RW];
    const int64_t n = blockIdx.x;
    const uint8_t* row = w + n * row_bytes;
    if constexpr (CPT > 0) {
        if ((((uintptr_t)w | (uintptr_t)row_bytes) & 3) == 0) {
            const uint32_t* r4 = reinterpret_cast<const uint32_t*>(row);
            for (int i = threadIdx.x; i < row_bytes / 4; i += 256) rs[i] = r4[i];
        } else {
            for (int i = threadIdx.x; i < row_bytes; i += 256) reinterpret_cast<uint8_t*>(rs)[i] = row[i];
        }
        __syncthreads();
        row = reinterpret_cast<const uint8_t*>(rs);
    }
    f16* orow = out + n * K;
    auto decode = [&](int64_t j, float* v) {
        const int64_t blk = j / QK;
        gguf::decode8<T>(row + blk * TS, (int)(j - blk * QK), v);
    };
    auto store = [&](int64_t j, const float* v, int e) {
        uint32_t p[4];
#pragma unroll
        for (int t = 0; t < 4; ++t)
            p[t] = pack2((f16)__builtin_ldexpf(v[2 * t], -e), (f16)__builtin_ldexpf(v[2 * t + 1], -e));
        *reinterpret_cast<u32x4*>(orow + j) = u32x4{p[0], p[1], p[2], p[3]};
    };
    float amax = 0.0f;
    float v[CPT > 0 ? CPT : 1][8];
    if constexpr (CPT > 0) {
#pragma unroll
        for (int c = 0; c < CPT; ++c) {
            const int64_t j = ((int64_t)threadIdx.x + 256 * c) * 8;
            if (j < K) decode(j, v[c]);
            else
#pragma unroll
                for (int t = 0; t < 8; ++t) v[c][t] = 0.0f;
#pragma unroll
            for (int t = 0; t < 8; ++t) amax = fmaxf(amax, fabsf(v[c][t]));
        }
    } else {
        for (int64_t j = (int64_t)threadIdx.x * 8; j < K; j += 256 * 8) {
            decode(j, v[0]);
#pragma unroll
            for (int t = 0; t < 8; ++t) amax = fmaxf(amax, fabsf(v[0][t]));
        }
    }
    amax = wave_max(amax);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = amax;
    __syncthreads();
    const int e = frexp_exp(fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3])));
    if (threadIdx.x == 0) wexp[n] = e;
    if constexpr (CPT > 0) {
#pragma unroll
        for (int c = 0; c < CPT; ++c) {
            const int64_t j = ((int64_t)threadIdx.x + 256 * c) * 8;
            if (j < K) store(j, v[c], e);
        }
    } else {
        for (int64_t j = (int64_t)threadIdx.x * 8; j < K; j += 256 * 8) {
            decode(j, v[0]);
            store(j, v[0], e);
        }
    }
}

hipError_t run_gguf_decode_f16(int type, const uint8_t* w, int64_t row_bytes, int64_t N, int64_t K, int32_t* e,
                               f16* out, hipStream_t st) {
    if (N == 0 || K == 0) return hipSuccess;
    if (K % 32 || (uintptr_t)out % 16) return hipErrorInvalidValue;
    hipError_t err = hipErrorInvalidValue;
    const int64_t cpt = (K + 2047) / 2048;
    bool ok = gguf::dispatch_type(type, [&]<int T>() {
        const dim3 grid((unsigned)N), block(256);
        if (cpt <= 1) hipLaunchKernelGGL((gguf_decode_f16_kernel<T, 1>), grid, block, 0, st, w, row_bytes, K, e, out);
        else if (cpt <= 2) hipLaunchKernelGGL((gguf_decode_f16_kernel<T, 2>), grid, block, 0, st, w, row_bytes, K, e, out);
        else if (cpt <= 4) hipLaunchKernelGGL((gguf_decode_f16_kernel<T, 4>), grid, block, 0, st, w, row_bytes, K, e, out);
        else hipLaunchKernelGGL((gguf_decode_f16_kernel<T, 0>), grid, block, 0, st, w, row_bytes, K, e, out);
        err = hipGetLastError();
    });
    return ok ? err : hipErrorInvalidValue;
}

hipError_t run_gguf_row_exp(int type, const uint8_t* w, int64_t N, int64_t K, int32_t* e, hipStream_t st) {
    if (N == 0) return hipSuccess;
    hipError_t err = hipErrorInvalidValue;
    bool ok = gguf::dispatch_type(type, [&]<int T>() {
        hipLaunchKernelGGL((gguf_row_exp_kernel<T>), dim3((unsigned)N), dim3(256), 0, st, w, K, e);
        err = hipGetLastError();
    });
    return ok ? err : hipErrorInvalidValue;
}

}  // namespace qlin
