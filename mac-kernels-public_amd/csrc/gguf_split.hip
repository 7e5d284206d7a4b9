// GGUF linear from a few dozen to a few hundred activation rows, with the weight decoded in the
// load stage, the activations shared in LDS and K split across workgroups where the grid is short.
//
// A kernel that keeps all of K inside one workgroup of 16 weight rows makes every CU stream all
// of x: M x K x 2 bytes (512 KiB at M = 64, K = 4096) against 36 KiB of weights, through loads
// that each touch 16 rows.  Here:
//   * a workgroup owns 128 weight rows (8 waves x 16), all M rows (MT m-tiles of 16) and one of S
//     K ranges; grid = ceil(N / 128) x S, S chosen so the grid covers the GPU about once.  At
//     K = N = 4096 (S = 8) a CU reads 64 KiB of x and 72 KiB of Q4_K weights;
//   * per stage (SV values) the activation slice is loaded once, 16 bytes per lane with 512 or
//     1024 contiguous bytes per row, into LDS (rows padded by 16 bytes so the fragment reads are
//     conflict-free), and all eight waves read their MFMA A fragments from there;
//   * the eight waves form four pairs; a pair owns 32 weight rows (two 16-row n-tiles), stages them
//     through LDS and splits each stage's K range in halves, one per wave.  A wave folds the block
//     scales into its fp16 B operand (w * 2^k rounded to fp16, k per weight row and K half) instead
//     of applying them per block to the MFMA results (measured at K = N = 4096 against that exact
//     form: 3-7% faster at 64 rows, 5-27% at 256, Q6_K 6% at 5-16 rows; relative Frobenius error
//     2-4e-4 of a float64 product).  Each B fragment feeds the MT m-tiles; the two halves'
//     accumulators are added through LDS at the end;
//   * the next stage's activations and weights are in flight while a stage is computed;
//   * above 64 rows the grid's z dimension holds m-tiles of 64 rows, each decoding the weight
//     again (measured at K = N = 4096: 2x faster than decoding the weight once to fp16 and running
//     the fp16-weight GEMM at 65-128 rows, 1.15-1.3x at 512, slower from ~1024 rows);
//   * S > 1: each workgroup stores its fp32 partial tile to the workspace ([S][M][N]) and a second
//     kernel adds the S partials in split order (the result does not depend on timing) and applies
//     the epilogue; S = 1: the epilogue runs in place.  The epilogue is y = ldexp(acc, xexp[m]) +
//     bias[n], then, with a residual, y = r[m, n] + rs[n] * y (one fma), rounded once to y's type.
#include "gguf_mfma_decode.h"
#include "lora_frag.h"

namespace qlin {

namespace {

using namespace gguf_mfma;

constexpr int SP_WAVES = 8;
constexpr int SP_THREADS = SP_WAVES * 64;
constexpr int SP_ROWS = 16 * SP_WAVES;  // weight rows per workgroup
constexpr int SP_TARGET_BLOCKS = 256;   // one workgroup per CU
constexpr int SP_MAX_SPLITS = 8;        // partial tiles added by the reduction kernel

template <int T, int MT, bool W32, bool LD>
__global__ __launch_bounds__(SP_THREADS) void gguf_split_kernel(
    const f16* __restrict__ x, int64_t ldx, int M, const int32_t* __restrict__ xexp,
    const uint8_t* __restrict__ w, int64_t row_bytes, int N, int K, int S,
    const void* __restrict__ bias, int bias_dt, void* __restrict__ y, int y_dt, int64_t ldy,
    float* __restrict__ part, ResidualTile res, LoraDownRows dn) {
    using F = SM<T>;
    constexpr int QK = F::QK, TS = F::TS, UNIT = F::UNIT, VPL = UNIT / 4, SBLK = F::SBLK;
    constexpr int SV = SBLK * QK;                    // values per stage
    constexpr int RSB = SBLK * TS;                   // stage bytes per weight row
    // LDS weight row stride: padded for over-reads, and an odd number of 16-byte units so that
    // the 16 rows a decode read touches fall in different banks
    constexpr int RS0 = ((RSB + 15) / 16) * 16 + 16;
    constexpr int RS = (RS0 / 16) % 2 ? RS0 : RS0 + 16;
    static_assert(RSB % 4 == 0 && RSB >= 16, "stage rows must be whole dwords");
    constexpr int UPR = (RSB + 15) / 16;             // 16-byte weight units per row (last one overlaps)
    constexpr int HALF = 16 * UPR;                   // weight units each wave of a pair loads per stage
    constexpr int NPF = (HALF + 63) / 64;            // weight units per lane
    constexpr int UPS = SV / UNIT;                   // scale units per stage
    constexpr int UH = UPS / 2;                      // scale units per K half
    constexpr int UPB = QK / UNIT;                   // scale units per block
    static_assert(UPS % 2 == 0 && (UPB % UH == 0 || UH % UPB == 0), "K halves must align with blocks");
    constexpr int XR = MT * (W32 ? 32 : 16);         // activation rows held (rows past M repeat row M - 1)
    constexpr int XRS = SV * 2 + 16;                 // LDS activation row stride (bytes)
    constexpr int CPR = SV / 8;                      // 16-byte activation chunks per row
    constexpr int XPT = XR * CPR / SP_THREADS;       // activation chunks per thread and stage
    static_assert(XR * CPR % SP_THREADS == 0, "activation stage must split evenly over the threads");
    typedef typename FragT<VPL>::type V;
    typedef uint32_t LU __attribute__((ext_vector_type(4), aligned(4)));

    __shared__ __attribute__((aligned(16))) uint8_t xs[XR * XRS];
    __shared__ __attribute__((aligned(16))) uint8_t wsm[SP_ROWS * RS];
    // LD: this workgroup's LoRA down rows for the stage (NR <= 2 rows of SV values, f32 at most)
    constexpr int DSM = LD ? 2 * SV * 4 : 16;
    __shared__ __attribute__((aligned(16))) uint8_t dsm[DSM];

    // Waves 0..3 and 4..7 cover the first and second half of every stage's units; wave w % 4 of
    // each half owns weight rows 32 (w % 4) .. + 31 of the tile (two n-tiles), so every activation
    // fragment read from LDS feeds two MFMAs.
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int np = wave & 3, kh = wave >> 2;
    const int n0 = blockIdx.x * SP_ROWS + np * 32;  // this wave pair's first weight row
    const int nl = lane & 15, g = lane >> 4;
    const int split = blockIdx.y;
    // m-tile blockIdx.z holds activation rows m0 .. m0 + XR - 1; from here on M counts its rows
    const int m0 = blockIdx.z * XR, Mall = M;
    x += (int64_t)m0 * ldx;
    if (xexp) xexp += m0;
    M = min(XR, Mall - m0);
    const int stages = K / SV;
    const int st0 = (int)((int64_t)stages * split / S), st1 = (int)((int64_t)stages * (split + 1) / S);
    const int last = st1 - 1;  // the host keeps S <= stages, so every split has a stage
    uint8_t* my = wsm + np * 32 * RS;
    const int ilim = (MT == 1 && M < 4) ? M : 4;

    // No load below branches on the lane: activation rows past M re-read row M - 1, weight rows
    // past N re-read row N - 1 (their results are never stored), and each wave's last weight unit
    // is re-read by the lanes past it.
    // Stages held in registers ahead of LDS.  One: the next stage's loads go out as soon as the
    // current one is committed to LDS, before its math.  Two (both of a workgroup's usual stages
    // requested before the first wait) held 40 more registers and spilled Q8_0's 272-byte stage
    // rows; one measured faster at K = N = 4096 (same process): Q8_0 M64 15.7 -> 13.6 us, the
    // 4.5-bit formats at M64 4-5% and at M17 3-6%, within 2% either way at M256.
    constexpr int PF = 1;
    u32x4 xq[PF][XPT];
    auto issue_x = [&](int st, u32x4* dst) {
        const int64_t k = (int64_t)min(st, last) * SV;
#pragma unroll
        for (int j = 0; j < XPT; ++j) {
            const int c = tid + SP_THREADS * j, r = c / CPR, cc = c % CPR;
            dst[j] = *reinterpret_cast<const u32x4*>(x + (int64_t)min(r, M - 1) * ldx + k + 8 * cc);
        }
    };
    auto commit_x = [&](const u32x4* src) {
#pragma unroll
        for (int j = 0; j < XPT; ++j) {
            const int c = tid + SP_THREADS * j, r = c / CPR, cc = c % CPR;
            *reinterpret_cast<u32x4*>(xs + r * XRS + 16 * cc) = src[j];
        }
    };
    // The pair's 32 x UPR load units: the K-half-0 wave takes the first half, the other the rest.
    auto unit_of = [&](int i) { return kh * HALF + min(lane + 64 * i, HALF - 1); };
    LU pf[PF][NPF];
    auto issue_w = [&](int st, LU* dst) {
        st = min(st, last);
#pragma unroll
        for (int i = 0; i < NPF; ++i) {
            const int u = unit_of(i), r = u / UPR;
            const int off = min((u - r * UPR) * 16, RSB - 16);
            dst[i] = *reinterpret_cast<const LU*>(w + (int64_t)min(n0 + r, N - 1) * row_bytes + (int64_t)st * RSB + off);
        }
    };
    // Unconditional: lanes past the last unit re-write its bytes (issue_w loaded that same unit).
    auto commit_w = [&](const LU* src) {
#pragma unroll
        for (int i = 0; i < NPF; ++i) {
            const int u = unit_of(i), r = u / UPR;
            const int off = min((u - r * UPR) * 16, RSB - 16);
            *reinterpret_cast<LU*>(my + r * RS + off) = src[i];
        }
    };
    // LD: the stage's slice of this workgroup's down rows, 16 bytes per thread (NR * SV * es bytes,
    // at most SP_THREADS pieces); row j is rank blockIdx.x + gridDim.x * j (past R: rank R - 1, never
    // stored).
    const int des = LD && dn.dt == DT_F32 ? 4 : 2;
    const int dpieces = LD ? dn.NR * SV * des / 16 : 0;
    u32x4 dq[PF];
    auto issue_d = [&](int st, u32x4& dst) {
        if constexpr (LD) {
            if (tid < dpieces) {
                const int j = tid * 16 / (SV * des), o = tid * 16 - j * SV * des;
                const int64_t r = min((int)blockIdx.x + (int)gridDim.x * j, dn.R - 1);
                dst = *reinterpret_cast<const u32x4*>(reinterpret_cast<const uint8_t*>(dn.down) +
                                                      (r * dn.ld + (int64_t)min(st, last) * SV) * des + o);
            }
        }
    };
    auto commit_d = [&](const u32x4& src) {
        if constexpr (LD) {
            if (tid < dpieces) *reinterpret_cast<u32x4*>(dsm + tid * 16) = src;
        }
    };
    // LD: thread (pair p = tid / TPP, part kc = tid % TPP) sums x[m] . down[j] over values
    // kc * KCN .. + KCN - 1 of each stage, m = p % XR, j = p / XR; the TPP parts meet by xor
    // shuffles at the end (fixed order).
    const int tpp = LD ? SP_THREADS / (XR * max(dn.NR, 1)) : 1, kcn = SV / tpp;
    const int dkc = tid % tpp, dp = tid / tpp, dm = dp % XR, dj = dp / XR;
    float tacc = 0.f;
    auto down_dot = [&]() {
        if constexpr (LD) {
            const uint8_t* xp = xs + dm * XRS + 2 * dkc * kcn;
            const uint8_t* dq8 = dsm + ((int64_t)dj * SV + dkc * kcn) * des;
            for (int i = 0; i < kcn; i += 8) {
                const f16x8 xv = *reinterpret_cast<const f16x8*>(xp + 2 * i);
                float dv[8];
                if (dn.dt == DT_F32) {
                    const f32x4 a = *reinterpret_cast<const f32x4*>(dq8 + 4 * i);
                    const f32x4 b = *reinterpret_cast<const f32x4*>(dq8 + 4 * i + 16);
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        dv[e] = a[e];
                        dv[4 + e] = b[e];
                    }
                } else {
                    const u32x4 a = *reinterpret_cast<const u32x4*>(dq8 + 2 * i);
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        dv[2 * e] = bits_to_f32_rt(a[e] & 0xFFFFu, dn.dt);
                        dv[2 * e + 1] = bits_to_f32_rt(a[e] >> 16, dn.dt);
                    }
                }
#pragma unroll
                for (int e = 0; e < 8; ++e) tacc = __builtin_fmaf((float)xv[e], dv[e], tacc);
            }
        }
    };

    f32x4 acc[2][MT];
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int i = 0; i < MT; ++i) acc[t][i] = f32x4{0.f, 0.f, 0.f, 0.f};
    const uint8_t* srow[2] = {my + nl * RS, my + (16 + nl) * RS};
    const uint8_t* xrow = xs + nl * XRS + 2 * VPL * g;  // A fragment: row mt * 16 + nl, values VPL*g.. of a unit

    // This wave's half of a stage (units H * UH .. H * UH + UH - 1) on 16 x 16 tiles, in the folded
    // form described at the 32 x 32 path below: lane (nl, g) holds weight row nl of n-tile t in its
    // B operand and column nl of n-tile t in its accumulators, so one power of two per (lane, t).
    auto compute = [&]<int H>() {
        constexpr int U0 = H * UH, B0 = U0 * UNIT / QK, B1 = ((U0 + UH) * UNIT - 1) / QK;
        int e[2];
        float f[2];
        f32x4 c[2][MT];
#pragma unroll
        for (int t = 0; t < 2; ++t) {
            float bnd = 0.f;
#pragma unroll
            for (int blk = B0; blk <= B1; ++blk) bnd = fmaxf(bnd, F::bound(srow[t], blk * TS));
            e[t] = __builtin_amdgcn_frexp_expf(bnd);
            f[t] = __builtin_ldexpf(1.0f, 15 - e[t]);
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) c[t][mt] = f32x4{0.f, 0.f, 0.f, 0.f};
        }
#pragma unroll
        for (int uu = 0; uu < UH; ++uu) {
            const int u = U0 + uu, blk = u * UNIT / QK, v0 = (u * UNIT) % QK + VPL * g;
            V bf[2];
#pragma unroll
            for (int t = 0; t < 2; ++t) bf[t] = F::getf(srow[t], blk * TS, v0, f[t]);
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) {
                const V af = *reinterpret_cast<const V*>(xrow + mt * 16 * XRS + 2 * UNIT * u);
#pragma unroll
                for (int t = 0; t < 2; ++t) c[t][mt] = mfma16<VPL>(af, bf[t], c[t][mt]);
            }
        }
#pragma unroll
        for (int t = 0; t < 2; ++t) {
            const float inv = __builtin_ldexpf(1.0f, e[t] - 15);
#pragma unroll
            for (int mt = 0; mt < MT; ++mt)
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    if (i < ilim) acc[t][mt][i] = __builtin_fmaf(c[t][mt][i], inv, acc[t][mt][i]);
        }
    };

    // 32 x 32 tiles (W32, more than 16 activation rows): the pair's 32 weight rows form one n-tile
    // and each m-tile holds 32 activation rows.  Lane (r32, h) decodes weight row r32 and reads
    // activation row r32 of each m-tile; a 16-value MFMA step of unit u takes values u * UNIT +
    // 16 s + 8 h .. + 7 of the stage in both operands.  Output register r of m-tile mt is row
    // mt * 32 + 8 (r / 4) + 4 h + r % 4, column r32 of the n-tile.
    const int r32 = lane & 31, h32 = lane >> 5;
    f32x16 acc32[W32 ? MT : 1];
#pragma unroll
    for (int i = 0; i < (W32 ? MT : 1); ++i)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc32[i][r] = 0.f;
    const uint8_t* srow32 = my + r32 * RS;
    const uint8_t* xrow32 = xs + r32 * XRS + 16 * h32;
    // The B operand in the folded form: w * f rounded to fp16, f = 2^(15 - e) with |w| < 2^e over
    // this wave's half of the stage for weight row r32 (both lanes of the row derive the same e),
    // so that one MFMA chain runs over the whole half and the result is scaled back once.  Per
    // 16-value step this replaces a block-scale multiply of every accumulator (and, with block
    // minima, a second MFMA against the minima) by 4 packed fp16 multiplies of the operand.
    auto bfragf = [&](int blk, int v0, float f) {
        if constexpr (VPL == 8) {
            return F::getf(srow32, blk * TS, v0, f);
        } else {
            const f16x4 lo = F::getf(srow32, blk * TS, v0, f), hi = F::getf(srow32, blk * TS, v0 + 4, f);
            return f16x8{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
        }
    };
    auto mfma32 = [](f16x8 a, f16x8 b, f32x16 c) { return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0); };
    constexpr int STEPS = UNIT / 16;
    auto compute32 = [&]<int H>() {
        constexpr int U0 = H * UH, B0 = U0 * UNIT / QK, B1 = ((U0 + UH) * UNIT - 1) / QK;
        float bnd = 0.f;
#pragma unroll
        for (int blk = B0; blk <= B1; ++blk) bnd = fmaxf(bnd, F::bound(srow32, blk * TS));
        const int e = __builtin_amdgcn_frexp_expf(bnd);  // bnd < 2^e
        const float f = __builtin_ldexpf(1.0f, 15 - e);
        f32x16 c[MT];
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
            for (int r = 0; r < 16; ++r) c[mt][r] = 0.f;
#pragma unroll
        for (int uu = 0; uu < UH; ++uu) {
            const int u = U0 + uu, blk = u * UNIT / QK;
#pragma unroll
            for (int s = 0; s < STEPS; ++s) {
                const f16x8 bf = bfragf(blk, (u * UNIT) % QK + 16 * s + 8 * h32, f);
#pragma unroll
                for (int mt = 0; mt < MT; ++mt) {
                    const f16x8 af = *reinterpret_cast<const f16x8*>(xrow32 + mt * 32 * XRS + 2 * (u * UNIT + 16 * s));
                    c[mt] = mfma32(af, bf, c[mt]);
                }
            }
        }
        const float inv = __builtin_ldexpf(1.0f, e - 15);
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
            for (int r = 0; r < 16; ++r) acc32[mt][r] = __builtin_fmaf(c[mt][r], inv, acc32[mt][r]);
    };

#pragma unroll
    for (int j = 0; j < PF; ++j) {
        issue_x(st0 + j, xq[j]);
        issue_w(st0 + j, pf[j]);
        issue_d(st0 + j, dq[j]);
    }
    for (int c0 = st0; c0 < st1; c0 += PF)
#pragma unroll
    for (int jp = 0; jp < PF; ++jp) {
        const int st = c0 + jp;
        if (st >= st1) break;
        lds_barrier();  // every wave is done with the previous stage's LDS
        commit_x(xq[jp]);
        commit_w(pf[jp]);
        commit_d(dq[jp]);
        if (st + PF < st1) {  // refill the freed registers with the stage PF ahead (uniform branch)
            issue_x(st + PF, xq[jp]);
            issue_w(st + PF, pf[jp]);
            issue_d(st + PF, dq[jp]);
        }
        __builtin_amdgcn_sched_barrier(0);  // the next stages' loads stay ahead of this stage's math
        lds_barrier();  // this stage is in LDS
        if constexpr (W32) {
            if (kh == 0) compute32.template operator()<0>();
            else compute32.template operator()<1>();
        } else {
            if (kh == 0) compute.template operator()<0>();
            else compute.template operator()<1>();
        }
        down_dot();
    }
    if constexpr (LD) {
        for (int o = tpp / 2; o >= 1; o /= 2) tacc += __shfl_xor(tacc, o, 64);
        const int r = (int)blockIdx.x + (int)gridDim.x * dj;
        if (dkc == 0 && dm < M && r < dn.R) dn.tpart[((int64_t)split * Mall + m0 + dm) * dn.R + r] = tacc;
    }

    // The two K halves meet in LDS (reusing the activation buffer) in a fixed order, and the
    // [XR x 128] tile leaves with every output row as 512 contiguous bytes.  Lane (nl, g),
    // register i of n-tile t, m-tile mt holds row mt * 16 + 4 * g + i, column 32 np + 16 t + nl.
    constexpr int ORS = SP_ROWS * 4 + 16;  // LDS output row stride (bytes)
    static_assert(ORS <= XRS, "the output tile must fit in the activation buffer");
    auto out_at = [&](int t, int mt, int i) {
        return reinterpret_cast<float*>(xs + (mt * 16 + 4 * g + i) * ORS + 4 * (np * 32 + 16 * t + nl));
    };
    auto out32 = [&](int mt, int r) {
        return reinterpret_cast<float*>(xs + (mt * 32 + 8 * (r / 4) + 4 * h32 + r % 4) * ORS + 4 * (np * 32 + r32));
    };
    lds_barrier();  // every wave is done with the last stage's activations
    if (kh == 1) {
        if constexpr (W32) {
#pragma unroll
            for (int mt = 0; mt < MT; ++mt)
#pragma unroll
                for (int r = 0; r < 16; ++r) *out32(mt, r) = acc32[mt][r];
        } else {
#pragma unroll
            for (int t = 0; t < 2; ++t)
#pragma unroll
                for (int mt = 0; mt < MT; ++mt)
#pragma unroll
                    for (int i = 0; i < 4; ++i) *out_at(t, mt, i) = acc[t][mt][i];
        }
    }
    lds_barrier();
    if (kh == 0) {
        if constexpr (W32) {
#pragma unroll
            for (int mt = 0; mt < MT; ++mt)
#pragma unroll
                for (int r = 0; r < 16; ++r) *out32(mt, r) = acc32[mt][r] + *out32(mt, r);
        } else {
#pragma unroll
            for (int t = 0; t < 2; ++t)
#pragma unroll
                for (int mt = 0; mt < MT; ++mt)
#pragma unroll
                    for (int i = 0; i < 4; ++i) *out_at(t, mt, i) = acc[t][mt][i] + *out_at(t, mt, i);
        }
    }
    lds_barrier();
    const int nt0 = blockIdx.x * SP_ROWS;
    if (part) {
        // Partials: 16-byte non-temporal stores (streamed to memory rather than kept in L2, where
        // the end of the kernel would have to write the tiles back); a row's N % 4 tail goes element
        // by element.
#pragma unroll
        for (int j = 0; j < XR * (SP_ROWS / 4) / SP_THREADS; ++j) {
            const int c = tid + SP_THREADS * j, r = c / (SP_ROWS / 4), n = nt0 + 4 * (c % (SP_ROWS / 4));
            if (r >= M || n >= N) continue;
            const f32x4 v = *reinterpret_cast<const f32x4*>(xs + r * ORS + 16 * (c % (SP_ROWS / 4)));
            float* d = part + ((int64_t)split * Mall + m0 + r) * N + n;
            if (N % 4 == 0) {
                __builtin_nontemporal_store(v, reinterpret_cast<f32x4*>(d));
            } else {
                for (int q = 0; q < 4 && n + q < N; ++q) __builtin_nontemporal_store(v[q], d + q);
            }
        }
        return;
    }
    const bool vec = ldy % 4 == 0 && (uintptr_t)y % (y_dt == 0 ? 16 : 8) == 0;
#pragma unroll
    for (int j = 0; j < XR * (SP_ROWS / 4) / SP_THREADS; ++j) {
        const int c = tid + SP_THREADS * j, r = c / (SP_ROWS / 4), n = nt0 + 4 * (c % (SP_ROWS / 4));
        if (r >= M || n >= N) continue;
        const f32x4 v = *reinterpret_cast<const f32x4*>(xs + r * ORS + 16 * (c % (SP_ROWS / 4)));
        const int e = xexp ? xexp[r] : 0;
        float o[4];
#pragma unroll
        for (int q = 0; q < 4; ++q)
            o[q] = __builtin_ldexpf(v[q], e) + (bias ? load_rt(bias, bias_dt, min(n + q, N - 1)) : 0.0f);
        if (res.r) residual_apply4(res, m0 + r, n, N, o);
        store4_rt(y, y_dt, (int64_t)(m0 + r) * ldy + n, o, min(4, N - n), vec);
    }
}

// y[m][n] = ldexp(sum over s in order of part[s][m][n], xexp[m]) + bias[n]; four columns per thread,
// all S partial loads in flight at once.
template <int S>
__global__ __launch_bounds__(256) void gguf_split_reduce_kernel(
    const float* __restrict__ part, int M, int N, const int32_t* __restrict__ xexp,
    const void* __restrict__ bias, int bias_dt, void* __restrict__ y, int y_dt, int64_t ldy, int xcd_blocks,
    ResidualTile res) {
    int m, n;
    if (xcd_blocks) {
        // The split kernel's workgroup (x, s) is dispatched to XCD (s * blocks + x) % 8 = x % 8 when
        // the row-block count is a multiple of 8: every partial of row block x was written through
        // that XCD's L2.  Workgroup b reduces only row blocks x = b % 8 (mod 8), 4 outputs a thread.
        const int xcd = blockIdx.x & 7, j = blockIdx.x >> 3;
        const int64_t per = (int64_t)(xcd_blocks / 8) * SP_ROWS * M;  // outputs of this XCD's row blocks
        const int64_t idx = (int64_t)j * 1024 + 4 * threadIdx.x;
        if (idx >= per) return;
        const int q = (int)(idx / ((int64_t)SP_ROWS * M)), rem = (int)(idx % ((int64_t)SP_ROWS * M));
        m = rem / SP_ROWS;
        n = (xcd + 8 * q) * SP_ROWS + rem % SP_ROWS;
    } else {
        const int nq = (N + 3) / 4;
        const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
        if (t >= (int64_t)M * nq) return;
        m = (int)(t / nq);
        n = (int)(t % nq) * 4;
    }
    const int64_t mn = (int64_t)M * N;
    const float* p = part + (int64_t)m * N + n;
    const int e = xexp ? xexp[m] : 0;
    f32x4 s;
    if (N % 4 == 0) {
        f32x4 v[S];
#pragma unroll
        for (int k = 0; k < S; ++k) v[k] = *reinterpret_cast<const f32x4*>(p + k * mn);
        s = v[0];
#pragma unroll
        for (int k = 1; k < S; ++k) s += v[k];
    } else {
        for (int q = 0; q < 4; ++q) {
            float v[S];
#pragma unroll
            for (int k = 0; k < S; ++k) v[k] = n + q < N ? p[q + k * mn] : 0.0f;
            s[q] = v[0];
#pragma unroll
            for (int k = 1; k < S; ++k) s[q] += v[k];
        }
    }
    float o[4];
#pragma unroll
    for (int q = 0; q < 4; ++q)
        o[q] = __builtin_ldexpf(s[q], e) + (bias ? load_rt(bias, bias_dt, min(n + q, N - 1)) : 0.0f);
    if (res.r) residual_apply4(res, m, n, N, o);
    // one 8-byte (f16, bf16) or 16-byte (f32) store per thread where rows allow it
    const bool vec = ldy % 4 == 0 && (uintptr_t)y % (y_dt == 0 ? 16 : 8) == 0;
    store4_rt(y, y_dt, (int64_t)m * ldy + n, o, min(4, N - n), vec);
}

// The reduction with an unmerged LoRA term (S > 1): one workgroup of 4 waves per 32 x 128 output
// tile, each wave a 32 x 32 sub-tile in the MFMA C layout (lane l, register r: row 8 (r / 4) +
// 4 (l / 32) + r % 4, column l % 32).  The S partials are added in split order and the base
// ldexp(sum, xexp[m]) + bias[n] formed as in gguf_split_reduce_kernel; lora_tile_epilogue_ranks then
// adds lora_scale * t up^T to those fp32 values (bf16 MFMAs on exact hi / lo parts, ranks up to
// 2 x 64), and the tile leaves through LDS as 8-output row pieces, rounded once.  Workgroup b takes
// row block b % blocks, so with a multiple of 8 row blocks it runs on the XCD that wrote that
// block's partials.  Measured at K = N = 4096 (Q4_K, rank 16-128, same process): 0.1-1.9 us per
// call faster than 64 x 128 tiles of 8 waves (half the workgroups, each reading twice the partials
// of y and of t), which were 1.3 us faster than 32 x 64 tiles at M = 64.
constexpr int SPL_BM = 32, SPL_BN = SP_ROWS, SPL_NT = 256, SPL_LDS = 48 * 1024;
template <int DU, int S>
__global__ __launch_bounds__(SPL_NT) void gguf_split_lora_reduce_kernel(
    const float* __restrict__ part, int M, int N, const int32_t* __restrict__ xexp, const void* __restrict__ bias,
    int bias_dt, void* __restrict__ y, int y_dt, int64_t ldy, LoraTile L) {
    constexpr int BNT = SPL_BN, NT = SPL_NT, ORW = BNT + 4;
    constexpr int RC = lora_max_rank<DU, SPL_BM, BNT>(SPL_LDS);
    static_assert(RC == 64, "one pass of 64 ranks fits (two passes to 128)");
    static_assert(SPL_BM * ORW * 4 <= SPL_LDS, "output staging must fit");
    __shared__ __attribute__((aligned(16))) uint8_t lds[SPL_LDS];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int r32 = lane & 31, h = lane >> 5, wi = wave >> 2, wj = wave & 3;
    const int blocks = (N + BNT - 1) / BNT;
    const int64_t n0 = (int64_t)(blockIdx.x % blocks) * BNT, m0 = (int64_t)(blockIdx.x / blocks) * SPL_BM;
    const int64_t n = min(n0 + 32 * wj + r32, (int64_t)N - 1), mn = (int64_t)M * N;
    // every partial of the sub-tile is requested before the first add; rows past M re-read row M - 1
    f32x16 v[S];
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        const int64_t m = min(m0 + 32 * wi + 8 * (r / 4) + 4 * h + r % 4, (int64_t)M - 1);
#pragma unroll
        for (int s = 0; s < S; ++s) v[s][r] = part[s * mn + m * N + n];
    }
    const float bvn = bias ? load_rt(bias, bias_dt, n) : 0.0f;
    f32x16 acc[1][1];
#pragma unroll
    for (int r = 0; r < 16; ++r) {
        float sum = v[0][r];
#pragma unroll
        for (int s = 1; s < S; ++s) sum += v[s][r];
        const int64_t m = min(m0 + 32 * wi + 8 * (r / 4) + 4 * h + r % 4, (int64_t)M - 1);
        acc[0][0][r] = __builtin_ldexpf(sum, xexp ? xexp[m] : 0) + bvn;
    }
    lora_tile_epilogue_ranks<DU, SPL_BM, BNT, RC, NT, 1, 1, true>(L, lds, m0, n0, M, N, 32 * wi, 32 * wj, tid, lane, acc);
    float* ot = reinterpret_cast<float*>(lds);
#pragma unroll
    for (int r = 0; r < 16; ++r) ot[(32 * wi + 8 * (r / 4) + 4 * h + r % 4) * ORW + 32 * wj + r32] = acc[0][0][r];
    __syncthreads();
    const bool vec = ldy % 8 == 0 && (uintptr_t)y % 16 == 0;
#pragma unroll
    for (int q = 0; q < SPL_BM * BNT / 8 / NT; ++q) {
        const int c = tid + NT * q, row = c / (BNT / 8), col = 8 * (c % (BNT / 8));
        const int64_t m = m0 + row, nc = n0 + col;
        if (m >= M || nc >= N) continue;
        float o[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) o[e] = ot[row * ORW + col + e];
        store8_rt(y, y_dt, m * ldy + nc, o, (int)min<int64_t>(8, N - nc), vec);
    }
}

template <int T>
constexpr int stage_values() { return SM<T>::SBLK * SM<T>::QK; }

template <int T>
hipError_t launch_t(const GgufSplitArgs& a, hipStream_t st) {
    // above 64 rows: m-tiles of 64 rows (32 x 32 MFMA tiles) along the grid's z
    dim3 grid((unsigned)((a.N + SP_ROWS - 1) / SP_ROWS), (unsigned)a.S, (unsigned)((a.M + 63) / 64)), block(SP_THREADS);
    float* part = a.S > 1 ? a.part : nullptr;
#define QLIN_SP_LAUNCH(MTV, W32V, LDV)                                                                          \
    hipLaunchKernelGGL((gguf_split_kernel<T, MTV, W32V, LDV>), grid, block, 0, st, a.x, a.ldx, a.M, a.xexp, a.w, \
                       a.row_bytes, a.N, a.K, a.S, a.bias, a.bias_dtype, a.y, a.y_dtype, a.ldy, part, a.res, a.down)
    // 16-row m-tiles up to 16 rows, then 32 x 32 tiles (the 32 x 32 x 16 MFMA moves about 1.7x the
    // values per cycle of the 16 x 16 x 32 form)
    const bool ld = a.down.down != nullptr;
    if (ld && (a.M <= 16 || a.S < 2 || !a.down.tpart || a.down.NR < 1 || a.down.NR > 2 ||
               (int64_t)grid.x * a.down.NR < a.down.R))
        return hipErrorInvalidValue;
    if (a.M <= 16) QLIN_SP_LAUNCH(1, false, false);
    else if (a.M <= 32) {
        if (ld) QLIN_SP_LAUNCH(1, true, true);
        else QLIN_SP_LAUNCH(1, true, false);
    } else {
        if (ld) QLIN_SP_LAUNCH(2, true, true);
        else QLIN_SP_LAUNCH(2, true, false);
    }
#undef QLIN_SP_LAUNCH
    hipError_t err = hipGetLastError();
    if (err != hipSuccess || a.S == 1) return err;
    if (a.lora.t) {
        const dim3 lgrid((unsigned)(((a.N + SPL_BN - 1) / SPL_BN) * ((a.M + SPL_BM - 1) / SPL_BM)));
#define QLIN_SPL_REDUCE(DU, SV)                                                                                      \
    hipLaunchKernelGGL((gguf_split_lora_reduce_kernel<DU, SV>), lgrid, dim3(SPL_NT), 0, st, a.part, a.M, a.N,       \
                       a.xexp, a.bias, a.bias_dtype, a.y, a.y_dtype, a.ldy, a.lora)
#define QLIN_SPL_S(DU)                      \
    switch (a.S) {                          \
        case 2: QLIN_SPL_REDUCE(DU, 2); break; \
        case 3: QLIN_SPL_REDUCE(DU, 3); break; \
        case 4: QLIN_SPL_REDUCE(DU, 4); break; \
        case 5: QLIN_SPL_REDUCE(DU, 5); break; \
        case 6: QLIN_SPL_REDUCE(DU, 6); break; \
        case 7: QLIN_SPL_REDUCE(DU, 7); break; \
        case 8: QLIN_SPL_REDUCE(DU, 8); break; \
        default: return hipErrorInvalidValue; \
    }
        if (a.lora.up_dt == DT_F32) QLIN_SPL_S(DT_F32)
        else if (a.lora.up_dt == DT_F16) QLIN_SPL_S(DT_F16)
        else QLIN_SPL_S(DT_BF16)
#undef QLIN_SPL_S
#undef QLIN_SPL_REDUCE
        return hipGetLastError();
    }
    // row blocks in multiples of 8 (N a multiple of 1024): reduce each block on the XCD that wrote it
    const int blocks = (int)((a.N + SP_ROWS - 1) / SP_ROWS);
    const int xcd_blocks = (a.N % SP_ROWS == 0 && blocks % 8 == 0) ? blocks : 0;
    const int64_t threads = (int64_t)a.M * ((a.N + 3) / 4);
    const dim3 rgrid(xcd_blocks ? (unsigned)(8 * (((int64_t)(blocks / 8) * SP_ROWS * a.M + 1023) / 1024))
                                : (unsigned)((threads + 255) / 256));
#define QLIN_SP_REDUCE(SV)                                                                                    \
    hipLaunchKernelGGL(gguf_split_reduce_kernel<SV>, rgrid, dim3(256), 0, st, a.part, a.M, a.N, a.xexp, a.bias, \
                       a.bias_dtype, a.y, a.y_dtype, a.ldy, xcd_blocks, a.res)
    switch (a.S) {
        case 2: QLIN_SP_REDUCE(2); break;
        case 3: QLIN_SP_REDUCE(3); break;
        case 4: QLIN_SP_REDUCE(4); break;
        case 5: QLIN_SP_REDUCE(5); break;
        case 6: QLIN_SP_REDUCE(6); break;
        case 7: QLIN_SP_REDUCE(7); break;
        case 8: QLIN_SP_REDUCE(8); break;
        default: return hipErrorInvalidValue;
    }
#undef QLIN_SP_REDUCE
    return hipGetLastError();
}

}  // namespace

int gguf_split_parts(int type, int64_t M, int64_t N, int64_t K, int64_t row_bytes, int min_parts) {
    if (M < 1 || N < 1) return 0;
    int parts = 0;
    gguf::dispatch_type(type, [&]<int T>() {
        constexpr int SV = stage_values<T>(), RSB = SM<T>::SBLK * SM<T>::TS;
        if (K % SV || RSB % 4 || row_bytes % 4) return;
        const int64_t stages = K / SV, tiles = (N + SP_ROWS - 1) / SP_ROWS * ((M + 63) / 64);
        // from 3/4 of the target on, one split: the partials and the reduction cost more than the
        // idle quarter (K = N = 4096, M = 384, 192 tiles: 2 splits 42-58 us, one split ~37-52)
        const int64_t s = tiles * 4 >= SP_TARGET_BLOCKS * 3 ? 1 : (SP_TARGET_BLOCKS + tiles - 1) / tiles;
        parts = (int)std::max<int64_t>(1, std::min<int64_t>(std::min<int64_t>(std::max<int64_t>(s, min_parts), stages),
                                                           SP_MAX_SPLITS));
    });
    return parts;
}

int gguf_split_down_ranks(const GgufSplitArgs& a, int R, int down_dt, int64_t ld_down, const void* down) {
    // measured at K = N = 4096 (Q4_K, 4 calls per graph, against the separate down kernel): 2.5-4 us
    // faster at 24-128 rows with 1 or 2 ranks per column and 4 or more splits; 1.5-4.7 us slower
    // with 4 ranks per column (rank 128), and with 2 splits (256 rows and more: 6-43 us)
    if (a.M <= 16 || a.S < 4 || !down || R < 1) return 0;
    if (down_dt != DT_F32 && down_dt != DT_F16 && down_dt != DT_BF16) return 0;
    const int es = down_dt == DT_F32 ? 4 : 2;
    if ((uintptr_t)down % 16 || (ld_down * es) % 16) return 0;
    const int64_t blocks = (a.N + SP_ROWS - 1) / SP_ROWS, nr = (R + blocks - 1) / blocks;
    return nr <= 1 ? 1 : nr <= 2 ? 2 : 0;
}

bool gguf_split_fuses_lora(const GgufSplitArgs& a) {
    const LoraTile& L = a.lora;
    const int es = L.up_dt == DT_F32 ? 4 : 2;
    return a.M > 16 && a.S > 1 && !a.res.r && L.up && L.R >= 8 && L.R % 8 == 0 && L.R <= 128 &&
           (uintptr_t)L.up % 16 == 0 && (L.ld_up * es) % 16 == 0 &&
           (L.up_dt == DT_BF16 || L.up_dt == DT_F16 || L.up_dt == DT_F32);
}

hipError_t run_gguf_split(const GgufSplitArgs& a, hipStream_t st) {
    if (a.y_dtype != DT_F32 && a.y_dtype != DT_F16 && a.y_dtype != DT_BF16) return hipErrorInvalidValue;
    if (a.lora.t && (!gguf_split_fuses_lora(a) || (uintptr_t)a.lora.t % 16)) return hipErrorInvalidValue;
    if (a.S < 1 || a.S > SP_MAX_SPLITS || (a.S > 1 && !a.part) || (a.ldx % 8) || ((uintptr_t)a.x % 16)) return hipErrorInvalidValue;
    hipError_t err = hipErrorInvalidValue;
    bool ok = gguf::dispatch_type(a.type, [&]<int T>() {
        if ((a.K % stage_values<T>()) || a.S > a.K / stage_values<T>()) return;
        err = launch_t<T>(a, st);
    });
    return ok ? err : hipErrorInvalidValue;
}

}  // namespace qlin
