// Standalone decodes of the packed formats (bit-exact with the reference's fp32 decode).
//   GGUF:  flat element e -> block e/QK, eight values per thread (gguf_exact.h), so rows that
//          straddle blocks are handled (roblennon/mac-kernels-public
//          docs/research/2026-10-03-gguf-on-metal.md:38).
//   INT8:  out[n,k] = f32(q[n,k]) * scale[n]  (modal/weight_error_app.py:122-123).
//   W4A8:  w8 = clamp(rne(level * f32(s_rel)), -127, 127), out = w8 or f32(w8) * s_channel[n]
//          (modal/weight_error_app.py:326-338).
// Contraction stays off in this file: each multiply and add rounds separately, as in the
// reference's numpy / torch decoders.
#pragma clang fp contract(off)
#include "qlin_internal.h"
#include "gguf_exact.h"

namespace qlin {
namespace {

// One rounding of the exact fp32 value to the output type (software round-to-nearest-even).
__device__ __forceinline__ void store_exact(float* p, float v) { *p = v; }
__device__ __forceinline__ void store_exact(f16* p, float v) {
    *reinterpret_cast<uint16_t*>(p) = f32_to_f16_bits_rne(v);
}
__device__ __forceinline__ void store_exact(bf16_t* p, float v) { p->bits = f32_to_bf16_bits(v); }

template <int T, typename TOut>
__global__ __launch_bounds__(256) void dequant_gguf_kernel(const uint8_t* __restrict__ w, int64_t total,
                                                            TOut* __restrict__ out) {
    constexpr int QK = gguf::Info<T>::QK, TS = gguf::Info<T>::TS;
    const int64_t e0 = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * 8;
    if (e0 >= total) return;
    const int64_t blk = e0 / QK;
    const int j = (int)(e0 - blk * QK);
    float v[8];
    gguf::decode8<T>(w + blk * TS, j, v);
    if (e0 + 8 <= total) {
        if constexpr (sizeof(TOut) == 4) {
            f32x4* p = reinterpret_cast<f32x4*>(out + e0);
            p[0] = f32x4{v[0], v[1], v[2], v[3]};
            p[1] = f32x4{v[4], v[5], v[6], v[7]};
        } else {
#pragma unroll
            for (int t = 0; t < 8; ++t) store_exact(out + e0 + t, v[t]);
        }
    } else {
        for (int t = 0; t < 8 && e0 + t < total; ++t) store_exact(out + e0 + t, v[t]);
    }
}

template <typename TS_>
__device__ __forceinline__ float scale_at(const TS_* s, int64_t i) { return load_f(s + i); }

template <typename TScale>
__global__ __launch_bounds__(256) void dequant_int8_kernel(const int8_t* __restrict__ q, int64_t N, int64_t K,
                                                            int64_t ldq, const TScale* __restrict__ scale,
                                                            int64_t scale_stride, float* __restrict__ out) {
    const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t kq = (K + 3) / 4;
    if (idx >= N * kq) return;
    const int64_t n = idx / kq, k0 = (idx - n * kq) * 4;
    const float s = scale_at(scale, n * scale_stride);
    for (int t = 0; t < 4 && k0 + t < K; ++t) out[n * K + k0 + t] = (float)q[n * ldq + k0 + t] * s;
}

template <typename TSrel, typename TOut>
__global__ __launch_bounds__(256) void dequant_w4a8_kernel(const uint8_t* __restrict__ q, int64_t N, int64_t K,
                                                            int64_t ldq, int bits, int gs,
                                                            const TSrel* __restrict__ s_rel, int64_t ld_srel,
                                                            const float* __restrict__ s_ch,
                                                            const float* __restrict__ codebook,
                                                            TOut* __restrict__ out) {
    const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= N * K) return;
    const int64_t n = idx / K, k = idx - n * K;
    const uint8_t* row = q + n * ldq;
    int code = (row[k >> 1] >> (4 * (k & 1))) & 0xF;
    if (bits == 6) code |= ((row[K / 2 + (k >> 2)] >> (2 * (k & 3))) & 3) << 4;
    const float level = codebook ? codebook[code] : (float)(code - (1 << (bits - 1)));
    float sr;
    if constexpr (sizeof(TSrel) == 1) sr = e4m3_to_f32(((const uint8_t*)s_rel)[n * ld_srel + k / gs]);
    else sr = load_f(s_rel + n * ld_srel + k / gs);
    float t = __builtin_rintf(level * sr);
    t = fminf(fmaxf(t, -127.0f), 127.0f);
    if constexpr (sizeof(TOut) == 1) out[idx] = (int8_t)(int)t;
    else out[idx] = t * s_ch[n];
}

}  // namespace

hipError_t run_dequant_gguf(int type, const uint8_t* w, int64_t total, void* out, int out_dtype, hipStream_t st) {
    if (total == 0) return hipSuccess;
    const int64_t threads = (total + 7) / 8;
    dim3 grid((unsigned)((threads + 255) / 256)), block(256);
    hipError_t err = hipErrorInvalidValue;
    bool ok = gguf::dispatch_type(type, [&]<int T>() {
        switch (out_dtype) {
            case DT_F32: hipLaunchKernelGGL((dequant_gguf_kernel<T, float>), grid, block, 0, st, w, total, (float*)out); break;
            case DT_F16: hipLaunchKernelGGL((dequant_gguf_kernel<T, f16>), grid, block, 0, st, w, total, (f16*)out); break;
            case DT_BF16: hipLaunchKernelGGL((dequant_gguf_kernel<T, bf16_t>), grid, block, 0, st, w, total, (bf16_t*)out); break;
            default: return;
        }
        err = hipGetLastError();
    });
    return ok ? err : hipErrorInvalidValue;
}

hipError_t run_dequant_int8(const int8_t* q, int64_t N, int64_t K, int64_t ldq, const void* scale, int scale_dtype,
                            int64_t scale_stride, float* out, hipStream_t st) {
    const int64_t threads = N * ((K + 3) / 4);
    if (threads == 0) return hipSuccess;
    dim3 grid((unsigned)((threads + 255) / 256)), block(256);
    if (scale_dtype == DT_F32)
        hipLaunchKernelGGL((dequant_int8_kernel<float>), grid, block, 0, st, q, N, K, ldq, (const float*)scale, scale_stride, out);
    else if (scale_dtype == DT_F16)
        hipLaunchKernelGGL((dequant_int8_kernel<f16>), grid, block, 0, st, q, N, K, ldq, (const f16*)scale, scale_stride, out);
    else if (scale_dtype == DT_BF16)
        hipLaunchKernelGGL((dequant_int8_kernel<bf16_t>), grid, block, 0, st, q, N, K, ldq, (const bf16_t*)scale, scale_stride, out);
    else
        return hipErrorInvalidValue;
    return hipGetLastError();
}

hipError_t run_dequant_w4a8(const uint8_t* q, int64_t N, int64_t K, int64_t ldq, int bits, int gs, const void* s_rel,
                            int s_rel_dtype, int64_t ld_srel, const float* s_ch, const float* codebook, void* out,
                            int out_dtype, hipStream_t st) {
    const int64_t threads = N * K;
    if (threads == 0) return hipSuccess;
    dim3 grid((unsigned)((threads + 255) / 256)), block(256);
    auto go = [&](auto srel_tag, auto out_tag) {
        using TSr = decltype(srel_tag);
        using TO = decltype(out_tag);
        hipLaunchKernelGGL((dequant_w4a8_kernel<TSr, TO>), grid, block, 0, st, q, N, K, ldq, bits, gs, (const TSr*)s_rel,
                           ld_srel, s_ch, codebook, (TO*)out);
    };
    auto go_out = [&](auto srel_tag) {
        if (out_dtype == DT_I8) go(srel_tag, int8_t{});
        else go(srel_tag, float{});
    };
    if (out_dtype != DT_I8 && out_dtype != DT_F32) return hipErrorInvalidValue;
    switch (s_rel_dtype) {
        case DT_E4M3: go_out(uint8_t{}); break;
        case DT_F16: go_out(f16{}); break;
        case DT_F32: go_out(float{}); break;
        case DT_BF16: go_out(bf16_t{}); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace qlin
