// GGUF linear for small M (1..64 activation rows): the weight-streaming (HBM-bound) regime.
//
// Grid: one workgroup of W waves (8, or 16 up to 16 activation rows when K has a stage for each
// wave) per 16 weight rows n; the K range is split across the waves in stages (256 values, or 512
// for the 210/110-byte K-quant blocks), and the partial sums are reduced through LDS at the end.  Each wave keeps one or two stages of weight loads in
// flight (16-, 8- or 4-byte units as the block size allows) and, separately, the activation
// fragments of the next D scale units; no load sits behind a lane-dependent branch, so the
// memory latencies overlap instead of adding up.  Per stage a wave copies its weight registers
// into its own LDS region and refills them with the stage PF ahead.  From there every lane decodes the MFMA B operand for
// (row n = lane % 16, k slice lane / 16) as EXACT small integers in fp16 -- nibbles become
// 1024 + q through v_perm_b32 with 0x64 exponent bytes -- and runs v_mfma_f32_16x16x{32,16}_f16
// against the fp16 activations.  Scales stay in fp32:
//   * per-block formats (Q4_0, Q4_1, Q5_0, Q5_1, Q8_0, IQ4_NL) and Q6_K / IQ4_XS (whose scaled
//     codes exceed fp16's exact-integer range): y += a_unit * C (+ b_unit * sum x),
//   * K-quants with small sub-scales (Q2_K, Q3_K, Q4_K, Q5_K): the 6-bit (4-bit) sub-scale is
//     folded into the operand exactly (|sc * q| <= 1953, computed by one fp16 FMA), the sub-block
//     minimum rides in a second MFMA, both accumulate over the 256-value block inside the MFMA
//     accumulators, and the fp16 block scales d, dmin are applied once per block.
// No fp16 weight rounding and no range normalization: every product is formed in fp32.
#include <type_traits>

#include "gguf_mfma_decode.h"

namespace qlin {

namespace {

using namespace gguf_mfma;

// Waves per workgroup.  The grid has one workgroup per 16 weight rows (256 at N = 4096), so a CU
// holds one: 16 waves (4 per SIMD) hide the weight and activation latencies of a K = 4096 call
// better than 8 (each wave then owns one stage; 13-18% faster at M = 8 and 16).
constexpr int SM_WAVES = 8;
constexpr int SM_WAVES_WIDE = 16;

// Formats that fit the 128 registers of 16 waves without spilling: 256-value stages, and no
// per-unit offset term (Q4_1, Q5_1 carry a second MFMA and its sums).
template <int T>
constexpr bool wide_ok() {
    using F = SM<T>;
    return F::SBLK * F::QK == 256 && !(F::KIND == 0 && F::MIN);
}

constexpr int pow2_floor(int v) { return v >= 2 ? 2 * pow2_floor(v / 2) : 1; }

// --------------------------------------------------------------------------------------------
template <int T, int MT, int W>
__global__ __launch_bounds__(64 * W) void gguf_smallm_kernel(
    const f16* __restrict__ x, int64_t ldx, int M, const int32_t* __restrict__ xexp,
    const uint8_t* __restrict__ w, int64_t row_bytes, int N, int K,
    const void* __restrict__ bias, int bias_dt, void* __restrict__ y, int y_dt, int64_t ldy,
    const void* __restrict__ wscale, int wscale_dt, int64_t wscale_stride) {
    using F = SM<T>;
    constexpr int QK = F::QK, TS = F::TS, UNIT = F::UNIT, VPL = UNIT / 4, SBLK = F::SBLK;
    constexpr int SV = SBLK * QK;                    // values per stage
    constexpr int RSB = SBLK * TS;                   // stage bytes per row
    // LDS row stride: padded for over-reads, and an odd number of 16-byte units so that the 16
    // rows a fragment read touches fall in different banks
    constexpr int RS0 = ((RSB + 15) / 16) * 16 + 16;
    constexpr int RS = (RS0 / 16) % 2 ? RS0 : RS0 + 16;
    static_assert(RSB % 4 == 0 && RSB >= 16, "stage rows must be whole dwords");
    // 16-byte load units (dword alignment suffices); a row's last unit ends at the row's last
    // byte and may overlap the one before it
    constexpr int UPR = (RSB + 15) / 16;             // load units per row
    constexpr int UNITS = 16 * UPR;                  // load units per stage
    constexpr int NPF = (UNITS + 63) / 64;           // load units per lane per stage
    // stages held in registers: two when a stage is small, else one (two stages in flight at
    // MT >= 3 measured slower: the activation stream already fills the memory pipeline); one with
    // 16 waves, where a wave usually owns a single stage
    constexpr int PF = W == SM_WAVES_WIDE ? 1 : (NPF <= 12 && MT <= 2) ? 2 : 1;
    constexpr int UPS = SV / UNIT;                   // scale units per stage
    constexpr int UPB = QK / UNIT;                   // scale units per block
    // activation fragments in flight: D units ahead of the MFMAs (at most 64 VGPRs of them)
    constexpr int XV = MT * VPL / 2;
    constexpr int D = (UPS * XV <= 64) ? UPS : pow2_floor(64 / XV);
    static_assert(D >= 1 && UPS % D == 0, "x prefetch depth must divide the stage");
    typedef typename FragT<VPL>::type V;
    typedef uint32_t LU __attribute__((ext_vector_type(4), aligned(4)));

    constexpr int STAGE_BYTES = W * 16 * RS;
    constexpr int RED_BYTES = W * MT * 4 * 64 * 4;
    __shared__ __attribute__((aligned(16))) uint8_t smem[STAGE_BYTES > RED_BYTES ? STAGE_BYTES : RED_BYTES];
    float (*red)[MT][4][64] = reinterpret_cast<float (*)[MT][4][64]>(smem);

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int n0 = blockIdx.x * 16;
    const int nl = lane & 15, g = lane >> 4;
    const int stages = K / SV;
    const int st0 = (stages * wave) / W, st1 = (stages * (wave + 1)) / W;
    uint8_t* my = smem + wave * 16 * RS;
    // rows of the 4 outputs this lane holds per m-tile: 4*g + i; skip FMAs for rows past M when M <= 4
    const int ilim = (MT == 1 && M < 4) ? M : 4;
    // the epilogue's operands for this thread's outputs e = tid + 64 W j (row exponent, weight scale
    // and bias as raw bits), requested now so that the epilogue needs no memory round trip; the
    // 16-wave variant (128 registers) loads them at the end instead
    constexpr int EPT = (MT * 256 + 64 * W - 1) / (64 * W);
    constexpr bool EPRE = W != SM_WAVES_WIDE;
    int exe[EPT];
    uint32_t ews[EPT], ebv[EPT];
#pragma unroll
    for (int j = 0; j < (EPRE ? EPT : 0); ++j) {
        const int e = min(tid + 64 * W * j, MT * 256 - 1);
        const int em = min((e >> 8) * 16 + 4 * ((e & 63) >> 4) + ((e & 255) >> 6), M - 1);
        const int en = min(n0 + (e & 15), N - 1);
        exe[j] = xexp ? xexp[em] : 0;
        ews[j] = wscale ? load_bits_rt(wscale, wscale_dt, en * wscale_stride) : 0u;
        ebv[j] = bias ? load_bits_rt(bias, bias_dt, en) : 0u;
    }

    // No load below branches on the lane: activation rows past M re-read row M - 1 and weight rows
    // past N re-read row N - 1 (their results are never stored).  With 8 waves, stages past this
    // wave's range re-read its last stage (never committed); with 16 (one stage per wave at
    // K = 4096) such refills are skipped instead, by a branch uniform across the wave: the
    // re-reads only delayed the final barrier, which waits for every load in flight.
    constexpr bool SKIP = W == SM_WAVES_WIDE;
    const f16* xrow[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) xrow[mt] = x + (int64_t)min(mt * 16 + nl, M - 1) * ldx + VPL * g;
    const int last = st1 - 1;

    f32x4 acc[MT];
#pragma unroll
    for (int i = 0; i < MT; ++i) acc[i] = f32x4{0.f, 0.f, 0.f, 0.f};

    LU pf[PF][NPF];
    auto issue = [&](int st, LU* buf) {
        st = min(st, last);
#pragma unroll
        for (int i = 0; i < NPF; ++i) {
            const int u = (UNITS % 64 == 0) ? lane + 64 * i : min(lane + 64 * i, UNITS - 1);
            const int r = u / UPR;
            const int off = min((u - r * UPR) * 16, RSB - 16);
            buf[i] = *reinterpret_cast<const LU*>(w + (int64_t)min(n0 + r, N - 1) * row_bytes + (int64_t)st * RSB + off);
        }
    };
    // Unconditional: lanes past the last unit re-write its bytes (issue() loaded that same unit
    // for them).  A guarded store would let the compiler sink the guarded lanes' load into the
    // guard, behind a wait for every load in flight.
    auto commit = [&](const LU* buf) {
#pragma unroll
        for (int i = 0; i < NPF; ++i) {
            const int u = (UNITS % 64 == 0) ? lane + 64 * i : min(lane + 64 * i, UNITS - 1);
            const int r = u / UPR;
            const int off = min((u - r * UPR) * 16, RSB - 16);
            *reinterpret_cast<LU*>(my + r * RS + off) = buf[i];
        }
    };
    V xr[D][MT];
    auto load_xu = [&](int st, int u, V* dst) {
        const int64_t k = (int64_t)min(st, last) * SV + u * UNIT;
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) dst[mt] = *reinterpret_cast<const V*>(xrow[mt] + k);
    };

    V ones;
#pragma unroll
    for (int i = 0; i < VPL; ++i) ones[i] = (f16)1.0f;

    if (st0 < st1) {
        // first stage's weights, its first D activation units, then the other prefetched stages
        issue(st0, pf[0]);
#pragma unroll
        for (int d = 0; d < D; ++d) load_xu(st0, d, xr[d]);
#pragma unroll
        for (int j = 1; j < PF; ++j) issue(st0 + j, pf[j]);

        for (int c0 = st0; c0 < st1; c0 += PF) {
#pragma unroll
            for (int j = 0; j < PF; ++j) {
                const int st = c0 + j;
                if (st >= st1) break;
                __builtin_amdgcn_wave_barrier();
                __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
                commit(pf[j]);
                __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
                __builtin_amdgcn_wave_barrier();
                __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
                if (!SKIP || st + PF < st1) issue(st + PF, pf[j]);  // refill with the stage PF ahead
                const uint8_t* srow = my + nl * RS;
                // unit u's activations sit in xr[u % D]; once used, the slot takes unit u + D
                auto next_x = [&](int u) {
                    if (u + D < UPS) load_xu(st, u + D, xr[u % D]);
                    else if (!SKIP || st + 1 < st1) load_xu(st + 1, u + D - UPS, xr[u % D]);
                };
                if constexpr (F::KIND == 0) {
#pragma unroll
                    for (int u = 0; u < UPS; ++u) {
                        const int blk = (u * UNIT) / QK;
                        const int v0 = (u * UNIT) % QK + VPL * g;
                        float a, b;
                        const V bf = F::get(srow, blk * TS, v0, a, b);
#pragma unroll
                        for (int mt = 0; mt < MT; ++mt) {
                            const V af = xr[u % D][mt];
                            const f32x4 c = mfma16<VPL>(af, bf, f32x4{0.f, 0.f, 0.f, 0.f});
                            if constexpr (F::MIN) {
                                const f32x4 c1 = mfma16<VPL>(af, ones, f32x4{0.f, 0.f, 0.f, 0.f});
#pragma unroll
                                for (int i = 0; i < 4; ++i)
                                    if (i < ilim) acc[mt][i] += a * c[i] + b * c1[i];
                            } else {
#pragma unroll
                                for (int i = 0; i < 4; ++i)
                                    if (i < ilim) acc[mt][i] += a * c[i];
                            }
                        }
                        next_x(u);
                    }
                } else {
#pragma unroll
                    for (int blk = 0; blk < SBLK; ++blk) {
                        f32x4 c1[MT], c2[MT];
#pragma unroll
                        for (int mt = 0; mt < MT; ++mt) {
                            c1[mt] = f32x4{0.f, 0.f, 0.f, 0.f};
                            c2[mt] = f32x4{0.f, 0.f, 0.f, 0.f};
                        }
#pragma unroll
                        for (int ub = 0; ub < UPB; ++ub) {
                            const int u = blk * UPB + ub;
                            const int v0 = ub * UNIT + VPL * g;
                            f16 mv;
                            const V bf = F::get(srow, blk * TS, v0, mv);
                            V bm;
#pragma unroll
                            for (int i = 0; i < VPL; ++i) bm[i] = mv;
#pragma unroll
                            for (int mt = 0; mt < MT; ++mt) {
                                const V af = xr[u % D][mt];
                                c1[mt] = mfma16<VPL>(af, bf, c1[mt]);
                                if constexpr (F::MIN) c2[mt] = mfma16<VPL>(af, bm, c2[mt]);
                            }
                            next_x(u);
                        }
                        float d, dmin;
                        F::block(srow, blk * TS, d, dmin);
#pragma unroll
                        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
                            for (int i = 0; i < 4; ++i)
                                if (i < ilim) {
                                    acc[mt][i] += d * c1[mt][i];
                                    if constexpr (F::MIN) acc[mt][i] -= dmin * c2[mt][i];
                                }
                    }
                }
            }
        }
    }

    __syncthreads();  // stage buffers are reused for the cross-wave reduction
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int i = 0; i < 4; ++i) red[wave][mt][i][lane] = acc[mt][i];
    __syncthreads();
    // 16 x 16 outputs per m-tile; thread e handles element (i = e/64, source lane = e%64).
#pragma unroll
    for (int j = 0; j < EPT; ++j) {
        const int e = tid + 64 * W * j;
        const int mt = e >> 8, rem = e & 255, i = rem >> 6, sl = rem & 63;
        const int m = mt * 16 + 4 * (sl >> 4) + i;
        const int n = n0 + (sl & 15);
        if (e < MT * 256 && m < M && n < N) {
            float sum = 0.0f;
#pragma unroll
            for (int wv = 0; wv < W; ++wv) sum += red[wv][mt][i][sl];
            if constexpr (!EPRE) {
                exe[j] = xexp ? xexp[m] : 0;
                ews[j] = wscale ? load_bits_rt(wscale, wscale_dt, (int64_t)n * wscale_stride) : 0u;
                ebv[j] = bias ? load_bits_rt(bias, bias_dt, n) : 0u;
            }
            float v = xexp ? __builtin_ldexpf(sum, exe[j]) : sum;
            if (wscale) v *= bits_to_f32_rt(ews[j], wscale_dt);
            if (bias) v += bits_to_f32_rt(ebv[j], bias_dt);
            store_rt(y, y_dt, (int64_t)m * ldy + n, v);
        }
    }
}

template <int T>
hipError_t launch_t(const GgufSmallMArgs& a, hipStream_t st) {
    dim3 grid((unsigned)((a.N + 15) / 16));
    if constexpr (wide_ok<T>()) {
        if (a.M <= 16 && a.K / (SM<T>::SBLK * SM<T>::QK) >= SM_WAVES_WIDE) {
            hipLaunchKernelGGL((gguf_smallm_kernel<T, 1, SM_WAVES_WIDE>), grid, dim3(64 * SM_WAVES_WIDE), 0, st,
                               a.x, a.ldx, a.M, a.xexp, a.w, a.row_bytes, a.N, a.K, a.bias, a.bias_dtype, a.y,
                               a.y_dtype, a.ldy, a.wscale, a.wscale_dtype, a.wscale_stride);
            return hipGetLastError();
        }
    }
    const dim3 block(64 * SM_WAVES);
#define QLIN_SM_LAUNCH(MTV)                                                                               \
    hipLaunchKernelGGL((gguf_smallm_kernel<T, MTV, SM_WAVES>), grid, block, 0, st, a.x, a.ldx, a.M, a.xexp, a.w, \
                       a.row_bytes, a.N, a.K, a.bias, a.bias_dtype, a.y, a.y_dtype, a.ldy, a.wscale,         \
                       a.wscale_dtype, a.wscale_stride)
    switch ((a.M + 15) / 16) {
        case 1: QLIN_SM_LAUNCH(1); break;
        case 2: QLIN_SM_LAUNCH(2); break;
        case 3: QLIN_SM_LAUNCH(3); break;
        case 4: QLIN_SM_LAUNCH(4); break;
        default: return hipErrorInvalidValue;
    }
#undef QLIN_SM_LAUNCH
    return hipGetLastError();
}

}  // namespace

bool gguf_smallm_supported(int type, int64_t M, int64_t K, int64_t row_bytes) {
    if (M < 1 || M > 64) return false;
    bool ok = false;
    gguf::dispatch_type(type, [&]<int T>() {
        constexpr int SV = SM<T>::SBLK * SM<T>::QK, RSB = SM<T>::SBLK * SM<T>::TS;
        ok = (K % SV == 0) && (RSB % 4 == 0) && (row_bytes % 4 == 0);
    });
    return ok;
}

bool int8_smallm_supported(int64_t M, int64_t K, int64_t ldw, const void* w) {
    constexpr int SV = SM<INT8_ROWS>::SBLK * SM<INT8_ROWS>::QK;
    return M >= 1 && M <= 64 && K % SV == 0 && ldw % 4 == 0 && (uintptr_t)w % 4 == 0;
}

hipError_t run_int8_smallm(const GgufSmallMArgs& a, hipStream_t st) {
    if (a.y_dtype != DT_F32 && a.y_dtype != DT_F16 && a.y_dtype != DT_BF16) return hipErrorInvalidValue;
    if (!int8_smallm_supported(a.M, a.K, a.row_bytes, a.w) || !a.wscale) return hipErrorInvalidValue;
    return launch_t<INT8_ROWS>(a, st);
}

hipError_t run_gguf_smallm(const GgufSmallMArgs& a, hipStream_t st) {
    if (a.y_dtype != DT_F32 && a.y_dtype != DT_F16 && a.y_dtype != DT_BF16) return hipErrorInvalidValue;
    hipError_t err = hipErrorInvalidValue;
    bool ok = gguf::dispatch_type(a.type, [&]<int T>() { err = launch_t<T>(a, st); });
    return ok ? err : hipErrorInvalidValue;
}

}  // namespace qlin
