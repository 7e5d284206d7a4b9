// GGUF linear for small M (1..64 activation rows): the weight-streaming (HBM-bound) regime.
//
// Grid: one 512-thread workgroup (8 waves) per 16 weight rows n; the K range is split across
// the 8 waves in stages of 256 values, and the partial sums are reduced through LDS at the end.
// Per stage a wave copies the 16 rows' packed blocks for those 256 values into its own LDS
// region with coalesced dword loads (prefetching the next stage into registers while it
// computes), then for every scale group (unit) decodes exact small-integer codes for the MFMA B
// operand (lane = row n, lane/16 = k slice), multiplies with the fp16 activations on
// v_mfma_f32_16x16x{32,16}_f16 and applies the unit's fp32 scale and offset to the 4 outputs it
// holds:  y[m,n] += a[n,u] * sum_k x[m,k] q[n,k] + b[n,u] * sum_k x[m,k].
// Accumulation is fp32 throughout; no fp16 weight rounding and no range normalization are needed.
#include "qlin_internal.h"
#include "gguf_codes.h"

namespace qlin {

namespace {

constexpr int SM_WAVES = 8;
constexpr int SM_THREADS = SM_WAVES * 64;

template <int VPL> struct FragT;
template <> struct FragT<8> { typedef f16x8 type; };
template <> struct FragT<4> { typedef f16x4 type; };

template <int VPL>
__device__ __forceinline__ f32x4 mfma16(typename FragT<VPL>::type a, typename FragT<VPL>::type b) {
    f32x4 z = {0.f, 0.f, 0.f, 0.f};
    if constexpr (VPL == 8) return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, z, 0, 0, 0);
    else return __builtin_amdgcn_mfma_f32_16x16x16f16(a, b, z, 0, 0, 0);
}

template <int VPL>
__device__ __forceinline__ typename FragT<VPL>::type load_x(const f16* __restrict__ x, int64_t ldx, int m, int M,
                                                            int64_t k) {
    typedef typename FragT<VPL>::type V;
    if (m >= M) return V{};
    return *reinterpret_cast<const V*>(x + (int64_t)m * ldx + k);
}

template <int T, int MT, typename TOut, typename TBias>
__global__ __launch_bounds__(SM_THREADS) void gguf_smallm_kernel(
    const f16* __restrict__ x, int64_t ldx, int M, const int32_t* __restrict__ xexp,
    const uint8_t* __restrict__ w, int64_t row_bytes, int N, int K,
    const TBias* __restrict__ bias, TOut* __restrict__ y, int64_t ldy) {
    using C = gguf::Codes<T>;
    constexpr int QK = C::QK, TS = C::TS, UNIT = C::UNIT, VPL = UNIT / 4;
    constexpr int SBLK = 256 / QK;                 // blocks per row per stage
    constexpr int RSB = SBLK * TS;                 // stage bytes per row
    constexpr int RS = ((RSB + 15) / 16) * 16 + 16; // LDS row stride (padded for over-reads)
    constexpr int WORDS = 16 * RSB / 4;            // dwords per stage (RSB is even; x16 rows)
    static_assert((16 * RSB) % 4 == 0, "stage must be whole dwords");
    constexpr int NPF = (WORDS + 63) / 64;          // prefetch dwords per lane
    constexpr int UPS = 256 / UNIT;                 // units per stage
    typedef typename FragT<VPL>::type V;

    constexpr int STAGE_BYTES = SM_WAVES * 16 * RS;
    constexpr int RED_BYTES = SM_WAVES * MT * 4 * 64 * 4;
    __shared__ __attribute__((aligned(16))) uint8_t smem[STAGE_BYTES > RED_BYTES ? STAGE_BYTES : RED_BYTES];
    float (*red)[MT][4][64] = reinterpret_cast<float (*)[MT][4][64]>(smem);

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int n0 = blockIdx.x * 16;
    const int nl = lane & 15, g = lane >> 4;
    const int stages = K / 256;
    const int st0 = (stages * wave) / SM_WAVES, st1 = (stages * (wave + 1)) / SM_WAVES;
    uint8_t* my = smem + wave * 16 * RS;

    f32x4 acc[MT];
#pragma unroll
    for (int i = 0; i < MT; ++i) acc[i] = f32x4{0.f, 0.f, 0.f, 0.f};

    // dword u of the stage: row r = u / (RSB/4) when RSB % 4 == 0; RSB may be 2 mod 4 (Q6_K
    // with one block), so the copy runs over 16-bit halves in that case.
    uint32_t pf[NPF];
    auto issue = [&](int st) {
        if constexpr (RSB % 4 == 0) {
#pragma unroll
            for (int i = 0; i < NPF; ++i) {
                const int u = lane + 64 * i;
                uint32_t v = 0;
                if (u < WORDS) {
                    const int r = u / (RSB / 4);
                    const int off = (u - r * (RSB / 4)) * 4;
                    if (n0 + r < N)
                        v = *reinterpret_cast<const uint32_t*>(w + (int64_t)(n0 + r) * row_bytes +
                                                               (int64_t)st * RSB + off);
                }
                pf[i] = v;
            }
        } else {
#pragma unroll
            for (int i = 0; i < NPF; ++i) {
                uint32_t v = 0;
#pragma unroll
                for (int hh = 0; hh < 2; ++hh) {
                    const int u = 2 * (lane + 64 * i) + hh;  // 16-bit unit index
                    if (u < 2 * WORDS) {
                        const int r = u / (RSB / 2);
                        const int off = (u - r * (RSB / 2)) * 2;
                        if (n0 + r < N) {
                            const uint16_t h = *reinterpret_cast<const uint16_t*>(
                                w + (int64_t)(n0 + r) * row_bytes + (int64_t)st * RSB + off);
                            v |= (uint32_t)h << (16 * hh);
                        }
                    }
                }
                pf[i] = v;
            }
        }
    };
    auto commit = [&]() {
        if constexpr (RSB % 4 == 0) {
#pragma unroll
            for (int i = 0; i < NPF; ++i) {
                const int u = lane + 64 * i;
                if (u < WORDS) {
                    const int r = u / (RSB / 4);
                    const int off = (u - r * (RSB / 4)) * 4;
                    *reinterpret_cast<uint32_t*>(my + r * RS + off) = pf[i];
                }
            }
        } else {
#pragma unroll
            for (int i = 0; i < NPF; ++i) {
#pragma unroll
                for (int hh = 0; hh < 2; ++hh) {
                    const int u = 2 * (lane + 64 * i) + hh;
                    if (u < 2 * WORDS) {
                        const int r = u / (RSB / 2);
                        const int off = (u - r * (RSB / 2)) * 2;
                        *reinterpret_cast<uint16_t*>(my + r * RS + off) = (uint16_t)(pf[i] >> (16 * hh));
                    }
                }
            }
        }
    };

    V ones;
#pragma unroll
    for (int i = 0; i < VPL; ++i) ones[i] = (f16)1.0f;

    if (st0 < st1) issue(st0);
    for (int st = st0; st < st1; ++st) {
        __builtin_amdgcn_wave_barrier();
        commit();
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        if (st + 1 < st1) issue(st + 1);
        const uint8_t* srow = my + nl * RS;
        const int64_t kst = (int64_t)st * 256;
#pragma unroll
        for (int u = 0; u < UPS; ++u) {
            const int blk = (u * UNIT) / QK;
            const int v0 = (u * UNIT) % QK + VPL * g;
            int q[VPL];
            float a, b;
            C::get(srow, blk * TS, v0, q, a, b);
            V bf;
#pragma unroll
            for (int i = 0; i < VPL; ++i) bf[i] = (f16)(float)q[i];
            const int64_t k = kst + u * UNIT + VPL * g;
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) {
                const V af = load_x<VPL>(x, ldx, mt * 16 + nl, M, k);
                const f32x4 c = mfma16<VPL>(af, bf);
                if constexpr (C::MIN) {
                    const f32x4 c1 = mfma16<VPL>(af, ones);
#pragma unroll
                    for (int i = 0; i < 4; ++i) acc[mt][i] += a * c[i] + b * c1[i];
                } else {
#pragma unroll
                    for (int i = 0; i < 4; ++i) acc[mt][i] += a * c[i];
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
    for (int e = tid; e < MT * 256; e += SM_THREADS) {
        const int mt = e >> 8, rem = e & 255, i = rem >> 6, sl = rem & 63;
        float sum = 0.0f;
#pragma unroll
        for (int wv = 0; wv < SM_WAVES; ++wv) sum += red[wv][mt][i][sl];
        const int m = mt * 16 + 4 * (sl >> 4) + i;
        const int n = n0 + (sl & 15);
        if (m < M && n < N) {
            float v = xexp ? __builtin_ldexpf(sum, xexp[m]) : sum;
            if (bias) v += load_f(bias + n);
            store_out(y + (int64_t)m * ldy + n, v);
        }
    }
}

template <int T, typename TOut, typename TBias>
hipError_t launch_t(const GgufSmallMArgs& a, hipStream_t st) {
    dim3 grid((unsigned)((a.N + 15) / 16)), block(SM_THREADS);
    const int mt = (a.M + 15) / 16;
#define QLIN_SM_LAUNCH(MTV)                                                                          \
    hipLaunchKernelGGL((gguf_smallm_kernel<T, MTV, TOut, TBias>), grid, block, 0, st, a.x, a.ldx, a.M, \
                       a.xexp, a.w, a.row_bytes, a.N, a.K, (const TBias*)a.bias, (TOut*)a.y, a.ldy)
    switch (mt) {
        case 1: QLIN_SM_LAUNCH(1); break;
        case 2: QLIN_SM_LAUNCH(2); break;
        case 3: QLIN_SM_LAUNCH(3); break;
        case 4: QLIN_SM_LAUNCH(4); break;
        default: return hipErrorInvalidValue;
    }
#undef QLIN_SM_LAUNCH
    return hipGetLastError();
}

template <typename TOut, typename TBias>
hipError_t launch_bias(const GgufSmallMArgs& a, hipStream_t st) {
    hipError_t err = hipErrorInvalidValue;
    bool ok = gguf::dispatch_type(a.type, [&]<int T>() { err = launch_t<T, TOut, TBias>(a, st); });
    return ok ? err : hipErrorInvalidValue;
}

template <typename TOut>
hipError_t launch_out(const GgufSmallMArgs& a, hipStream_t st) {
    switch (a.bias_dtype) {
        case DT_F32: return launch_bias<TOut, float>(a, st);
        case DT_F16: return launch_bias<TOut, f16>(a, st);
        case DT_BF16: return launch_bias<TOut, bf16_t>(a, st);
        default: return launch_bias<TOut, float>(a, st);  // bias == nullptr
    }
}

}  // namespace

bool gguf_smallm_supported(int type, int64_t M, int64_t K, int64_t row_bytes) {
    int qk, ts;
    if (!gguf::type_info(type, qk, ts)) return false;
    if (M < 1 || M > 64 || K % 256 != 0) return false;
    const int rsb = (256 / qk) * ts;
    if (rsb % 2) return false;
    // dword copies need every stage start 4-aligned; half-word copies 2-aligned.
    if (rsb % 4 == 0) return row_bytes % 4 == 0;
    return row_bytes % 2 == 0;
}

hipError_t run_gguf_smallm(const GgufSmallMArgs& a, hipStream_t st) {
    switch (a.y_dtype) {
        case DT_F32: return launch_out<float>(a, st);
        case DT_F16: return launch_out<f16>(a, st);
        case DT_BF16: return launch_out<bf16_t>(a, st);
    }
    return hipErrorInvalidValue;
}

}  // namespace qlin
