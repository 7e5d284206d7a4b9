// Unmerged LoRA on a finished linear: y[m, n] <- y[m, n] + scale * sum_r t[m, r] up[n, r], with
// t = x down^T (roblennon/mac-kernels-public: the lora_down / lora_up / lora_scale keywords of the
// quantized linears, bench/bench_lora_sidepath_kernel.py:80, semantics
// docs/upstream/comfy-kitchen-mps-backend.md:54-57; the activation is the caller's x, before any
// ConvRot rotation).
//
// Both products run on v_mfma_f32_32x32x16_bf16 with every operand that is not already bf16 split
// into bf16 parts hi = bf16(v), lo = bf16(v - hi).  bf16 x bf16 products are exact in fp32 and bf16
// has fp32's exponent range, so there is no overflow or normalization; hi + lo carries 16
// significand bits (the lo x lo product, ~2^-16 of a term, is dropped).  t is kept in fp32.
//
//   lora_down_kernel: one workgroup per 32 rows x 64 ranks (32 when R <= 32) of t and K split, 4
//     waves on contiguous K quarters, added through LDS in a fixed order (the result does not
//     depend on timing).  Fragments come straight from global memory, 8 steps of loads in flight.
//   The K range is split S ways over workgroups (S fp32 partials of t) when the row tiles alone
//     would leave CUs idle; lora_sum_kernel adds the partials in split order.
//   lora_up_kernel: 128 x 128 output tiles, 4 waves of 64 x 64, the rank in chunks of 64 staged
//     in LDS; the tile is staged through LDS, then each output is read, increased by scale * acc
//     in fp32 and rounded once to y's dtype, 8 outputs per thread.  When the base linear left its
//     output in an fp32 buffer (`base`), that is read instead of y, so a 16-bit y is rounded once.
#include "lora_frag.h"

namespace qlin {

namespace {

// 16-value steps whose loads are in flight together: 8 x (1 + NH) 16-byte pieces for 16-bit
// operands at NH = 1, fewer with two rank halves or an fp32 operand (8 registers per piece)
template <int DX, int DD, int NH>
constexpr int lora_pf() { return (DX == DT_F32 || DD == DT_F32 ? 4 : 8) / NH; }

// t_s[m, r] = sum over split s's k of x[m, k] down[r, k] (fp32 partial s of [S][M][R]) for 32 rows
// and 32 NH ranks per workgroup: 4 waves, each a contiguous quarter of the split's 16-value steps
// for all of the tile's ranks, the quarters added through LDS in order.  Lane l holds row (rank)
// l % 32 and the 8 k values 8 (l / 32) .. + 7 of a step in both operands, so the 4 loads of 4
// consecutive steps cover 128 contiguous bytes of each row.  x is read once when R <= 32 NH.
template <int DX, int DD, bool VEC, int NH>
__global__ __launch_bounds__(256) void lora_down_kernel(LoraArgs a) {
    constexpr int PF = lora_pf<DX, DD, NH>(), RW = 32 * NH + 1;
    __shared__ float red[4][32 * RW];
    const int tid = threadIdx.x, lane = tid & 63, kq = tid >> 6;
    const int r32 = lane & 31, h = lane >> 5;
    const int64_t m0 = (int64_t)blockIdx.y * 32, q0 = (int64_t)blockIdx.x * 32 * NH;
    const int64_t xm = min(m0 + r32, a.M - 1);  // rows past the end repeat
    int64_t dr[NH];
#pragma unroll
    for (int i = 0; i < NH; ++i) dr[i] = min(q0 + 32 * i + r32, a.R - 1);
    f32x16 acc[NH];
#pragma unroll
    for (int i = 0; i < NH; ++i)
#pragma unroll
        for (int e = 0; e < 16; ++e) acc[i][e] = 0.f;
    // this wave's steps [w0, w1): quarter kq of split blockIdx.z's steps
    const int64_t steps = (a.K + 15) / 16, sp = blockIdx.z;
    const int64_t st0 = steps * sp / a.S, st1 = steps * (sp + 1) / a.S;
    const int64_t w0 = st0 + (st1 - st0) * kq / 4, w1 = st0 + (st1 - st0) * (kq + 1) / 4;
    // every lane of a wave runs the same trip count; steps past the quarter (or K) count zero
    for (int64_t s0 = w0; s0 < w1; s0 += PF) {
        Raw8<DX> xr[PF];
        Raw8<DD> dv[PF][NH];
        if (VEC && s0 + PF <= w1 && 16 * (s0 + PF) <= a.K) {
            // the whole batch is inside the quarter and K (uniform over the wave): one base
            // pointer per operand row and constant offsets, no clamping
            const int64_t k = 16 * s0 + 8 * h;
#pragma unroll
            for (int j = 0; j < PF; ++j) {
                xr[j] = raw_load<DX, true>(a.x, a.ldx, xm, k + 16 * j, k + 16 * j + 8);
#pragma unroll
                for (int i = 0; i < NH; ++i) dv[j][i] = raw_load<DD, true>(a.down, a.ld_down, dr[i], k + 16 * j, k + 16 * j + 8);
            }
        } else {
#pragma unroll
            for (int j = 0; j < PF; ++j) {
                const int64_t k = 16 * (s0 + j) + 8 * h;
                xr[j] = raw_load<DX, VEC>(a.x, a.ldx, xm, k, a.K);
#pragma unroll
                for (int i = 0; i < NH; ++i) dv[j][i] = raw_load<DD, VEC>(a.down, a.ld_down, dr[i], k, a.K);
            }
        }
        __builtin_amdgcn_sched_barrier(0);  // every load of the batch goes out before the first MFMA
#pragma unroll
        for (int j = 0; j < PF; ++j) {
            const Raw8<DX> xz = zero_unless(xr[j], s0 + j < w1 && 16 * (s0 + j) + 8 * h < a.K);
#pragma unroll
            for (int i = 0; i < NH; ++i) mfma_raw<DX, DD>(xz, dv[j][i], acc[i]);
        }
    }
    // C layout: lane l, register e holds row 8 (e / 4) + 4 (l / 32) + e % 4, column l % 32
#pragma unroll
    for (int i = 0; i < NH; ++i)
#pragma unroll
        for (int e = 0; e < 16; ++e) red[kq][(8 * (e / 4) + 4 * h + e % 4) * RW + 32 * i + r32] = acc[i][e];
    __syncthreads();
    for (int e = tid; e < 32 * 32 * NH; e += 256) {
        const int row = e / (32 * NH), col = e % (32 * NH);
        const int64_t m = m0 + row, q = q0 + col;
        if (m >= a.M || q >= a.R) continue;
        const int o = row * RW + col;
        a.t[(sp * a.M + m) * a.R + q] = ((red[0][o] + red[1][o]) + red[2][o]) + red[3][o];
    }
}

// The same partials for ranks up to 128 with both operands staged in LDS: one workgroup per 32 rows
// and all ranks (R <= 32 NH, NH in {1, 2, 4}) over split blockIdx.z's k-tiles of LD_KT values.  The
// tiles arrive by LDS DMA through a ring of LD_STAGES, every row as whole 16-byte chunks (64 lanes of
// an instruction cover 1 KiB of consecutive row bytes: a few cache lines, against 32 rows touched by
// each fragment load of lora_down_kernel), chunk c of row r stored at c ^ (r % chunks per row) so
// the 32 rows of a fragment read spread over the banks.  Wave w takes rank block w % NH and k part
// w / NH of each tile's 16-value steps; the 4 / NH parts are added through LDS in order at the end.
// Rows past M repeat row M - 1 and ranks past R repeat rank R - 1; neither is stored.
constexpr int LD_KT = 64;
template <int DX, int DD, int NH>
constexpr int lora_lds_stages() {
    constexpr int bytes = 32 * LD_KT * (DX == DT_F32 ? 4 : 2) + 32 * NH * LD_KT * (DD == DT_F32 ? 4 : 2);
    return bytes <= 24 * 1024 ? 4 : 3;
}
template <int DX, int DD, int NH>
__global__ __launch_bounds__(256) void lora_down_lds_kernel(LoraArgs a) {
    constexpr int EX = DX == DT_F32 ? 4 : 2, ED = DD == DT_F32 ? 4 : 2;
    constexpr int CX = LD_KT * EX / 16, CD = LD_KT * ED / 16;           // 16-byte chunks per row
    constexpr int XSZ = 32 * LD_KT * EX, DSZ = 32 * NH * LD_KT * ED;     // bytes per stage
    constexpr int NXI = XSZ / 1024, NDI = DSZ / 1024;                    // 1 KiB DMA instructions per stage
    constexpr int NI = (NXI + NDI) / 4, KQ = 4 / NH, SPP = LD_KT / 16 / KQ;
    constexpr int STAGES = lora_lds_stages<DX, DD, NH>();
    static_assert((NXI + NDI) % 4 == 0 && NI <= 16 && (STAGES - 2) * NI < 64, "DMA rounds");
    static_assert(KQ * NH == 4 && SPP >= 1, "wave split");
    constexpr int RW = 33;                                               // reduction row stride (floats)
    static_assert(KQ * NH * 32 * RW * 4 <= STAGES * (XSZ + DSZ), "reduction buffer must fit");
    __shared__ __attribute__((aligned(16))) uint8_t smem[STAGES * (XSZ + DSZ)];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int r32 = lane & 31, h = lane >> 5, rb = wave % NH, kq = wave / NH;
    const int64_t m0 = (int64_t)blockIdx.y * 32, sp = blockIdx.z;
    const int64_t tiles = a.K / LD_KT, t0 = tiles * sp / a.S, t1 = tiles * (sp + 1) / a.S;
    // DMA instruction i of this wave is instruction g = wave + 4 i of the stage: x (g < NXI) or down
    const uint8_t* src[NI];
    int dst[NI];
#pragma unroll
    for (int i = 0; i < NI; ++i) {
        const int g = wave + 4 * i;
        if (g < NXI) {
            const int u = 64 * g + lane, row = u / CX, c = (u % CX) ^ (row % CX);
            src[i] = reinterpret_cast<const uint8_t*>(a.x) + (min(m0 + row, a.M - 1) * a.ldx) * EX + 16 * c;
            dst[i] = 1024 * g;
        } else {
            const int u = 64 * (g - NXI) + lane, row = u / CD, c = (u % CD) ^ (row % CD);
            src[i] = reinterpret_cast<const uint8_t*>(a.down) + (min<int64_t>(row, a.R - 1) * a.ld_down) * ED + 16 * c;
            dst[i] = XSZ + 1024 * (g - NXI);
        }
    }
    auto dma = [&](int64_t kt, int buf) {
        const int64_t k0 = min(kt, t1 - 1) * LD_KT;  // past the split: re-reads its last tile
#pragma unroll
        for (int i = 0; i < NI; ++i) lds_dma16(src[i] + k0 * (dst[i] < XSZ ? EX : ED), smem + buf * (XSZ + DSZ) + dst[i]);
    };
    f32x16 acc;
#pragma unroll
    for (int e = 0; e < 16; ++e) acc[e] = 0.f;
    // fragment of step s: row r32 (x) or 32 rb + r32 (down), values 16 s + 8 h .. + 7
    auto frag_x = [&](const uint8_t* st, int s) {
        Raw8<DX> r;
        const uint8_t* row = st + r32 * (LD_KT * EX);
        if constexpr (DX == DT_F32) {
            r.v[0] = *reinterpret_cast<const u32x4*>(row + 16 * ((4 * s + 2 * h) ^ (r32 % CX)));
            r.v[1] = *reinterpret_cast<const u32x4*>(row + 16 * ((4 * s + 2 * h + 1) ^ (r32 % CX)));
        } else {
            r.v[0] = *reinterpret_cast<const u32x4*>(row + 16 * ((2 * s + h) ^ (r32 % CX)));
        }
        return r;
    };
    auto frag_d = [&](const uint8_t* st, int s) {
        Raw8<DD> r;
        const int rr = 32 * rb + r32;
        const uint8_t* row = st + XSZ + rr * (LD_KT * ED);
        if constexpr (DD == DT_F32) {
            r.v[0] = *reinterpret_cast<const u32x4*>(row + 16 * ((4 * s + 2 * h) ^ (rr % CD)));
            r.v[1] = *reinterpret_cast<const u32x4*>(row + 16 * ((4 * s + 2 * h + 1) ^ (rr % CD)));
        } else {
            r.v[0] = *reinterpret_cast<const u32x4*>(row + 16 * ((2 * s + h) ^ (rr % CD)));
        }
        return r;
    };
    // Barrier without a memory fence: each wave's wait covers its own DMAs, the loop writes LDS only
    // by DMA, and the fragment reads of a buffer complete before the barrier after which it is refilled.
#pragma unroll
    for (int s = 0; s < STAGES - 1; ++s) dma(t0 + s, s);
    wait_vmcnt<(STAGES - 2) * NI>();
    __builtin_amdgcn_s_barrier();
    for (int64_t kt = t0; kt < t1; ++kt) {
        dma(kt + STAGES - 1, (int)((kt - t0 + STAGES - 1) % STAGES));
        __builtin_amdgcn_sched_barrier(0);
        const uint8_t* st = smem + ((kt - t0) % STAGES) * (XSZ + DSZ);
        Raw8<DX> xr[SPP];
        Raw8<DD> dr[SPP];
#pragma unroll
        for (int j = 0; j < SPP; ++j) {
            xr[j] = frag_x(st, kq * SPP + j);
            dr[j] = frag_d(st, kq * SPP + j);
        }
#pragma unroll
        for (int j = 0; j < SPP; ++j) mfma_raw<DX, DD>(xr[j], dr[j], acc);
        wait_lgkmcnt0();
        wait_vmcnt<(STAGES - 2) * NI>();
        __builtin_amdgcn_s_barrier();
    }
    wait_vmcnt<0>();
    __syncthreads();
    // C layout: lane l, register e holds row 8 (e / 4) + 4 (l / 32) + e % 4, rank 32 rb + l % 32
    float* red = reinterpret_cast<float*>(smem);
    if constexpr (KQ > 1) {
#pragma unroll
        for (int e = 0; e < 16; ++e) red[((kq * NH + rb) * 32 + 8 * (e / 4) + 4 * h + e % 4) * RW + r32] = acc[e];
        __syncthreads();
        if (kq == 0) {
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                float v = acc[e];
#pragma unroll
                for (int q = 1; q < KQ; ++q) v += red[((q * NH + rb) * 32 + 8 * (e / 4) + 4 * h + e % 4) * RW + r32];
                acc[e] = v;
            }
        }
    }
    if (kq == 0) {
        const int64_t q = 32 * rb + r32;
#pragma unroll
        for (int e = 0; e < 16; ++e) {
            const int64_t m = m0 + 8 * (e / 4) + 4 * h + e % 4;
            if (m < a.M && q < a.R) a.t[(sp * a.M + m) * a.R + q] = acc[e];
        }
    }
}

// t[i] = sum over s, in split order, of partial s (for S > 1), written after the partials.
// Partials go in groups of 8 whose loads are all issued before the first add (a group past S
// re-reads partial S - 1 and drops it), so the latency is paid once per 8 partials.
__global__ __launch_bounds__(256) void lora_sum_kernel(const float* __restrict__ part, int S, int64_t n,
                                                       float* __restrict__ t) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= n) return;
    float v = 0.f;
    for (int s0 = 0; s0 < S; s0 += 8) {
        float p[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) p[j] = part[min(s0 + j, S - 1) * n + i];
#pragma unroll
        for (int j = 0; j < 8; ++j) v = s0 + j == 0 ? p[j] : (s0 + j < S ? v + p[j] : v);
    }
    t[i] = v;
}

// y[m, n] = dtype(float(y[m, n]) + scale * sum_r t[m, r] up[n, r]) for a 128 x 128 tile: 4 waves of
// 64 x 64 (2 x 2 MFMA sub-tiles), the rank in chunks of 64.  Each chunk of t (fp32 [M][R]) is staged
// in LDS for the tile's 128 rows; up fragments come from global memory.
// The output tile is staged through the same LDS in two 64-row halves, so y is read and written 8
// outputs per thread.
constexpr int UP_T = 128, UP_RC = 64;
template <int DU, bool VEC>
__global__ __launch_bounds__(256) void lora_up_kernel(LoraArgs a) {
    // one buffer: the t chunk during the rank loop, then 64-row halves of the output tile
    constexpr int TSW = UP_RC + 4, OTW = UP_T + 4;
    constexpr int SZ = UP_T * TSW > 64 * OTW ? UP_T * TSW : 64 * OTW;
    __shared__ __attribute__((aligned(16))) float smem[SZ];
    float* ts = smem;
    float* ot = smem;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int r32 = lane & 31, h = lane >> 5, wm = wave >> 1, wn = wave & 1;
    const int64_t mt = (int64_t)blockIdx.y * UP_T, nt = (int64_t)blockIdx.x * UP_T;
    f32x16 acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;
    int64_t un[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) un[j] = min(nt + 64 * wn + 32 * j + r32, a.N - 1);
    // the tile's y (8 outputs per thread and chunk, rows clamped) is requested first, so its
    // memory round trip overlaps the rank loop; 16-bit outputs only (f32 y takes the plain path)
    const bool vec = a.ldy % 8 == 0 && (uintptr_t)a.y % 16 == 0;
    constexpr int YC = UP_T * UP_T / 8 / 256;  // output chunks per thread
    const bool ypre = vec && a.y_dt != DT_F32 && a.N % 8 == 0 && !a.base;
    const bool bvec = a.base && a.ldb % 4 == 0 && (uintptr_t)a.base % 16 == 0;
    u32x4 yv[YC];
    if (ypre) {
#pragma unroll
        for (int j = 0; j < YC; ++j) {
            const int c = tid + 256 * j, row = c / (UP_T / 8), col = 8 * (c % (UP_T / 8));
            const int64_t m = min(mt + row, a.M - 1), n = min(nt + col, a.N - 8);
            yv[j] = *reinterpret_cast<const u32x4*>(reinterpret_cast<const uint16_t*>(a.y) + m * a.ldy + n);
        }
    }
    for (int64_t rc = 0; rc < a.R; rc += UP_RC) {
        __syncthreads();  // the previous chunk's t is no longer read
        if (a.R % 4 == 0) {
            // 16-byte pieces: piece e = row e / 16, ranks 4 (e % 16) .. + 3, loaded from a clamped
            // rank (all before any store), pieces past R zeroed
            constexpr int PPT = UP_T * UP_RC / 4 / 256;  // pieces per thread
            f32x4 pv[PPT];
#pragma unroll
            for (int i = 0; i < PPT; ++i) {
                const int e = tid + 256 * i, row = e / (UP_RC / 4);
                const int64_t m = min(mt + row, a.M - 1), r = min(rc + 4 * (e % (UP_RC / 4)), a.R - 4);
                pv[i] = *reinterpret_cast<const f32x4*>(a.t + m * a.R + r);
            }
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int i = 0; i < PPT; ++i) {
                const int e = tid + 256 * i, row = e / (UP_RC / 4), c = 4 * (e % (UP_RC / 4));
                *reinterpret_cast<f32x4*>(ts + row * TSW + c) = rc + c < a.R ? pv[i] : f32x4{0.f, 0.f, 0.f, 0.f};
            }
        } else {
            for (int e = tid; e < UP_T * UP_RC; e += 256) {
                const int row = e / UP_RC, c = e % UP_RC;
                const int64_t m = min(mt + row, a.M - 1), r = rc + c;
                ts[row * TSW + c] = r < a.R ? a.t[m * a.R + r] : 0.f;
            }
        }
        __syncthreads();
        // 4 rank steps of 16 per chunk; up loads of the chunk go out first
        Raw8<DU> ur[4][2];
#pragma unroll
        for (int q = 0; q < 4; ++q)
#pragma unroll
            for (int j = 0; j < 2; ++j) ur[q][j] = raw_load<DU, VEC>(a.up, a.ld_up, un[j], rc + 16 * q + 8 * h, a.R);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const bool in = rc + 16 * q + 8 * h < a.R;
#pragma unroll
            for (int i = 0; i < 2; ++i) {
                const float* tp = ts + (64 * wm + 32 * i + r32) * TSW + 16 * q + 8 * h;
                float tv[8];
#pragma unroll
                for (int e = 0; e < 8; ++e) tv[e] = in ? tp[e] : 0.f;  // zero past R (LDS holds zeros too)
                bf16x8 th, tl;
                split8(tv, th, tl);
#pragma unroll
                for (int j = 0; j < 2; ++j) {
                    bf16x8 uh, ul;
                    if constexpr (DU == DT_BF16) {
                        uh = __builtin_bit_cast(bf16x8, ur[q][j].v[0]);
                    } else {
                        float uv[8];
                        raw_to_f32(ur[q][j], uv);
                        split8(uv, uh, ul);
                    }
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(th, uh, acc[i][j], 0, 0, 0);
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(tl, uh, acc[i][j], 0, 0, 0);
                    if constexpr (DU != DT_BF16) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(th, ul, acc[i][j], 0, 0, 0);
                }
            }
        }
    }
    // C layout: lane l, register e holds row 8 (e / 4) + 4 (l / 32) + e % 4, column l % 32.  Two
    // passes: the waves of row half `pass` stage their 64 rows, then every thread updates y.  A
    // pass requests all of its base (or y) values before its first store -- a load between stores
    // would wait for the stores before it -- and its barriers order LDS only.
    constexpr int CPT = 64 * UP_T / 8 / 256;  // 8-output chunks per thread and pass
    for (int pass = 0; pass < 2; ++pass) {
    float v[CPT][8];
#pragma unroll
    for (int j = 0; j < CPT; ++j) {
        const int c = tid + 256 * j, row = c / (UP_T / 8), col = 8 * (c % (UP_T / 8));
        const int64_t m = min(mt + 64 * pass + row, a.M - 1), n = nt + col;  // rows past M re-read M - 1
        const int cnt = (int)max<int64_t>(0, min<int64_t>(8, a.N - n));
        if (a.base) {  // the base output in fp32: one rounding of base + side into y
            if (bvec && cnt == 8) {
                raw_to_f32(raw_load<DT_F32, true>(a.base, a.ldb, m, n, a.N), v[j]);
            } else {
#pragma unroll
                for (int e = 0; e < 8; ++e) v[j][e] = e < cnt ? a.base[m * a.ldb + n + e] : 0.0f;
            }
        } else if (ypre) {
            const u32x4 q = yv[pass * (YC / 2) + j];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                v[j][2 * e] = bits_to_f32_rt(q[e] & 0xFFFFu, a.y_dt);
                v[j][2 * e + 1] = bits_to_f32_rt(q[e] >> 16, a.y_dt);
            }
        } else if (vec && cnt == 8) {
            if (a.y_dt == DT_F32) {
                raw_to_f32(raw_load<DT_F32, true>(a.y, a.ldy, m, n, a.N), v[j]);
            } else if (a.y_dt == DT_F16) {
                raw_to_f32(raw_load<DT_F16, true>(a.y, a.ldy, m, n, a.N), v[j]);
            } else {
                raw_to_f32(raw_load<DT_BF16, true>(a.y, a.ldy, m, n, a.N), v[j]);
            }
        } else {
#pragma unroll
            for (int e = 0; e < 8; ++e) v[j][e] = e < cnt ? load_rt(a.y, a.y_dt, m * a.ldy + n + e) : 0.0f;
        }
    }
    lds_barrier();  // t (or the previous half) is no longer read
    if (wm == pass) {
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int j = 0; j < 2; ++j)
#pragma unroll
                for (int e = 0; e < 16; ++e)
                    ot[(32 * i + 8 * (e / 4) + 4 * h + e % 4) * OTW + 64 * wn + 32 * j + r32] = acc[i][j][e];
    }
    lds_barrier();
#pragma unroll
    for (int j = 0; j < CPT; ++j) {
        const int c = tid + 256 * j, row = c / (UP_T / 8), col = 8 * (c % (UP_T / 8));
#pragma unroll
        for (int e = 0; e < 8; ++e) v[j][e] = v[j][e] + a.scale * ot[row * OTW + col + e];
    }
#pragma unroll
    for (int j = 0; j < CPT; ++j) {
        const int c = tid + 256 * j, row = c / (UP_T / 8), col = 8 * (c % (UP_T / 8));
        const int64_t m = mt + 64 * pass + row, n = nt + col;
        if (m >= a.M || n >= a.N) continue;
        store8_rt(a.y, a.y_dt, m * a.ldy + n, v[j], (int)min<int64_t>(8, a.N - n), vec);
    }
    }
}

}  // namespace

hipError_t run_lora_t(const LoraArgs& a, hipStream_t st, const float** t_final) {
    if (a.R < 1 || !a.t) return hipErrorInvalidValue;
    if (a.S < 1 || a.S > LORA_MAX_SPLITS) return hipErrorInvalidValue;
    const int nh = a.R <= 32 ? 1 : 2;  // rank halves per workgroup
    const dim3 dgrid((unsigned)((a.R + 32 * nh - 1) / (32 * nh)), (unsigned)((a.M + 31) / 32), (unsigned)a.S);
    bool ok = false;
    const bool vd = a.vec_x && a.vec_down;
    // ranks to 128 with rows of whole 64-value tiles: the LDS-staged kernel, every rank in one workgroup
    const bool lds = vd && a.R <= 128 && a.K % LD_KT == 0 && a.K / LD_KT >= a.S;
    const int nl = a.R <= 32 ? 1 : a.R <= 64 ? 2 : 4;
    const dim3 lgrid(1u, (unsigned)((a.M + 31) / 32), (unsigned)a.S);
    auto down = [&]<int DX, int DD>() {
        if (a.x_dt == DX && a.down_dt == DD) {
            if (lds && nl == 1) hipLaunchKernelGGL((lora_down_lds_kernel<DX, DD, 1>), lgrid, dim3(256), 0, st, a);
            else if (lds && nl == 2) hipLaunchKernelGGL((lora_down_lds_kernel<DX, DD, 2>), lgrid, dim3(256), 0, st, a);
            else if (lds) hipLaunchKernelGGL((lora_down_lds_kernel<DX, DD, 4>), lgrid, dim3(256), 0, st, a);
            else if (vd && nh == 1) hipLaunchKernelGGL((lora_down_kernel<DX, DD, true, 1>), dgrid, dim3(256), 0, st, a);
            else if (vd) hipLaunchKernelGGL((lora_down_kernel<DX, DD, true, 2>), dgrid, dim3(256), 0, st, a);
            else if (nh == 1) hipLaunchKernelGGL((lora_down_kernel<DX, DD, false, 1>), dgrid, dim3(256), 0, st, a);
            else hipLaunchKernelGGL((lora_down_kernel<DX, DD, false, 2>), dgrid, dim3(256), 0, st, a);
            ok = true;
        }
    };
    auto by_down = [&]<int DX>() {
        down.template operator()<DX, DT_F32>();
        down.template operator()<DX, DT_F16>();
        down.template operator()<DX, DT_BF16>();
    };
    by_down.template operator()<DT_F32>();
    by_down.template operator()<DT_F16>();
    by_down.template operator()<DT_BF16>();
    if (!ok) return hipErrorInvalidValue;
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    const float* fin = a.t;  // one t: the partials' sum when K was split
    if (a.S > 1) {
        const int64_t n = a.M * a.R;
        float* sum = a.t + (int64_t)a.S * n;
        hipLaunchKernelGGL(lora_sum_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, a.t, a.S, n, sum);
        if ((e = hipGetLastError()) != hipSuccess) return e;
        fin = sum;
    }
    if (t_final) *t_final = fin;
    return hipSuccess;
}

hipError_t run_lora(const LoraArgs& a, hipStream_t st) {
    if (a.M == 0 || a.N == 0) return hipSuccess;
    LoraArgs u = a;  // the up kernel reads the final t
    const float* tf = nullptr;
    hipError_t e = run_lora_t(a, st, &tf);
    if (e != hipSuccess) return e;
    u.t = const_cast<float*>(tf);
    const bool vu = a.vec_up;
    const dim3 ugrid((unsigned)((a.N + UP_T - 1) / UP_T), (unsigned)((a.M + UP_T - 1) / UP_T));
#define QLIN_LORA_UP(DU)                                                                              \
    if (vu) hipLaunchKernelGGL((lora_up_kernel<DU, true>), ugrid, dim3(256), 0, st, u);               \
    else hipLaunchKernelGGL((lora_up_kernel<DU, false>), ugrid, dim3(256), 0, st, u);
    switch (a.up_dt) {
        case DT_F32: QLIN_LORA_UP(DT_F32) break;
        case DT_F16: QLIN_LORA_UP(DT_F16) break;
        case DT_BF16: QLIN_LORA_UP(DT_BF16) break;
        default: return hipErrorInvalidValue;
    }
#undef QLIN_LORA_UP
    return hipGetLastError();
}

// Splits so that the 32-row tiles make about 512 workgroups (2 per CU), at least 256 k-values each,
// at most LORA_MAX_SPLITS: a few rows (a decode step) still spread their K over the GPU.
int lora_splits(int64_t M, int64_t K, int64_t R) {
    (void)R;
    const int64_t tiles = (M + 31) / 32;
    int64_t s = (512 + tiles - 1) / std::max<int64_t>(tiles, 1);
    s = std::min<int64_t>(s, std::max<int64_t>(K / 256, 1));
    return (int)std::max<int64_t>(1, std::min<int64_t>(s, LORA_MAX_SPLITS));
}

}  // namespace qlin
