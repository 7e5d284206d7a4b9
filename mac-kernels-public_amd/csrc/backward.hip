// Input gradient of the frozen-weight packed linears (roblennon/mac-kernels-public:
// int8_linear_grad_input, bench/bench_int8_backward.py:15, 52; the backward of
// int8_linear_trainable / w4a8_linear_trainable, train/train_lora.py:187-188, 210, 221).
//
// The weight in the original basis is W[n, :] = s[n] q[n, :] H (q the stored int8 codes or the
// W4A8 int8 grid, s the per-row scale, H the block Hadamard of the ConvRot group, H = H^T = H^-1),
// so  dx = dy W = ((dy diag(s)) q) H.
//   bwd_rows_kernel: a[m, n] = fp16((dy[m, n] s[n]) 2^-E[m]), E[m] the exponent of the row's
//     max |dy s| (one rounding, no overflow or underflow of the row's large values), rows
//     zero-padded to a multiple of 64;
//   bwd_gemm_kernel: c = a q over n with fp16 MFMA (the int8 codes are exact fp16), one
//     workgroup per 64 rows x 256 columns of dx; the weight tile is read row by row (k
//     contiguous) and written to LDS transposed, k-major, so that every MFMA fragment is one
//     16-byte LDS read; the epilogue scales rows by 2^E[m], applies H to each 16-lane run of
//     the row and rounds once to dx's dtype.
#include "qlin_internal.h"
#include "hadamard.h"

namespace qlin {

namespace {

constexpr int BW_BM = 64, BW_BK = 256, BW_BN = 32;
constexpr int BW_LS = BW_BN + 8;  // LDS row stride in halves: 80 bytes, conflict-free fragment reads
constexpr int BW_OW = BW_BK + BW_BK / 4;  // epilogue row stride in floats: 4 pad floats per 16

// a[m, :] = fp16(dy[m, :] * s * 2^-E[m]), zero past N up to lda; e[m] = E[m].
template <typename T>
__global__ __launch_bounds__(256) void bwd_rows_kernel(const T* __restrict__ dy, int64_t ldd, int64_t N,
                                                       const void* __restrict__ s, int s_dt, int64_t s_stride,
                                                       f16* __restrict__ a, int64_t lda, int32_t* __restrict__ e) {
    __shared__ float red[4];
    const int64_t m = blockIdx.x;
    const int tid = threadIdx.x;
    const T* row = dy + m * ldd;
    float amax = 0.f;
    for (int64_t n = tid; n < N; n += 256) {
        const float v = dtype_traits<T>::to_f32(row[n]) * load_rt(s, s_dt, n * s_stride);
        amax = fmaxf(amax, fabsf(v));
    }
    amax = wave_max(amax);
    if ((tid & 63) == 0) red[tid >> 6] = amax;
    __syncthreads();
    amax = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    const int E = frexp_exp(amax);
    f16* out = a + m * lda;
    for (int64_t n = tid; n < lda; n += 256) {
        const float v = n < N ? dtype_traits<T>::to_f32(row[n]) * load_rt(s, s_dt, n * s_stride) : 0.f;
        out[n] = (f16)__builtin_ldexpf(v, -E);
    }
    if (tid == 0) e[m] = E;
}

// 8 rows x 4 columns of int8 (one dword per row) -> per column, the 8 rows as exact fp16 (16 bytes).
__device__ __forceinline__ void transpose8x4(const uint32_t* r, u32x4* col) {
    uint32_t c[2][4];
#pragma unroll
    for (int g = 0; g < 2; ++g) {
        const uint32_t* q = r + 4 * g;
        // 4 x 4 byte transpose: t0 = [q00 q10 q01 q11], t1 = [q02 q12 q03 q13], t2, t3 likewise for rows 2, 3
        const uint32_t t0 = __builtin_amdgcn_perm(q[1], q[0], 0x05010400u);
        const uint32_t t1 = __builtin_amdgcn_perm(q[1], q[0], 0x07030602u);
        const uint32_t t2 = __builtin_amdgcn_perm(q[3], q[2], 0x05010400u);
        const uint32_t t3 = __builtin_amdgcn_perm(q[3], q[2], 0x07030602u);
        c[g][0] = __builtin_amdgcn_perm(t2, t0, 0x05040100u);
        c[g][1] = __builtin_amdgcn_perm(t2, t0, 0x07060302u);
        c[g][2] = __builtin_amdgcn_perm(t3, t1, 0x05040100u);
        c[g][3] = __builtin_amdgcn_perm(t3, t1, 0x07060302u);
    }
    const f16x2 off = {(f16)-1152.0f, (f16)-1152.0f};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        uint32_t h[4];
#pragma unroll
        for (int g = 0; g < 2; ++g) {
            // fp16 bits 0x6400 | (q + 128) = 1152 + q, minus 1152: exact
            const uint32_t u = c[g][j] ^ 0x80808080u;
            h[2 * g] = __builtin_bit_cast(uint32_t, __builtin_bit_cast(f16x2, __builtin_amdgcn_perm(0x64646464u, u, 0x04010400u)) + off);
            h[2 * g + 1] = __builtin_bit_cast(uint32_t, __builtin_bit_cast(f16x2, __builtin_amdgcn_perm(0x64646464u, u, 0x04030402u)) + off);
        }
        col[j] = u32x4{h[0], h[1], h[2], h[3]};
    }
}

struct BwdRegs {
    u32x4 a;        // 8 halves of one row of the a tile
    uint32_t b[8];  // 4 int8 of each of 8 weight rows
};

// dx tile: rows m0 .. m0 + 63, columns k0 .. k0 + 255.  4 waves; wave w owns columns 64 w .. + 63
// of the tile (2 x 2 sub-tiles of 32 x 32).  Stage = 32 values of n: a tile [64][32] fp16 and
// weight tile [32][256] int8, the latter stored in LDS as [256][32] fp16.  Two LDS buffers, and
// each stage's global loads are issued two stages ahead of its use.
template <int G>
__global__ __launch_bounds__(256) void bwd_gemm_kernel(BwdGemmArgs p) {
    __shared__ __attribute__((aligned(16))) f16 smem[2 * (BW_BM + BW_BK) * BW_LS];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int r32 = lane & 31, h = lane >> 5;
    const int64_t m0 = (int64_t)blockIdx.y * BW_BM, k0 = (int64_t)blockIdx.x * BW_BK;
    // global load assignment: a row tid / 4, 8 halves at 8 (tid % 4); weight rows 8 no .. 8 no + 7
    // (no = lane % 4) and columns 4 kq .. 4 kq + 3 (kq = 16 wave + lane / 4)
    const f16* ap = p.a + min(m0 + tid / 4, p.M - 1) * p.lda + 8 * (tid & 3);
    const int no = lane & 3, kq = 16 * wave + (lane >> 2);
    const int8_t* bp = p.b + min(k0 + 4 * kq, p.K - 4);
    const int nst = (int)(p.lda / BW_BN);  // lda is N rounded up to 64; a is zero past N
    const int8_t* bq = bp + (int64_t)(8 * no) * p.ldb;  // this lane's first weight row of a stage
    auto load = [&](int s, BwdRegs& r) {
        r.a = *reinterpret_cast<const u32x4*>(ap + (int64_t)BW_BN * s);
        if ((int64_t)BW_BN * (s + 1) <= p.N) {
            // whole stage inside N (uniform): one base pointer, rows at constant multiples of ldb
            const int8_t* b0 = bq + (int64_t)BW_BN * s * p.ldb;
#pragma unroll
            for (int i = 0; i < 8; ++i) r.b[i] = *reinterpret_cast<const uint32_t*>(b0 + i * p.ldb);
        } else {
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const int64_t n = min((int64_t)BW_BN * s + 8 * no + i, p.N - 1);  // rows past N meet a = 0
                r.b[i] = *reinterpret_cast<const uint32_t*>(bp + n * p.ldb);
            }
        }
    };
    auto store = [&](const BwdRegs& r, int buf) {
        f16* As = smem + buf * (BW_BM + BW_BK) * BW_LS;
        f16* Bs = As + BW_BM * BW_LS;
        *reinterpret_cast<u32x4*>(As + (tid >> 2) * BW_LS + 8 * (tid & 3)) = r.a;
        u32x4 col[4];
        transpose8x4(r.b, col);
#pragma unroll
        for (int c = 0; c < 4; ++c) *reinterpret_cast<u32x4*>(Bs + (4 * kq + c) * BW_LS + 8 * no) = col[c];
    };
    f32x16 acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;
    auto compute = [&](int buf) {
        const f16* As = smem + buf * (BW_BM + BW_BK) * BW_LS;
        const f16* Bs = As + BW_BM * BW_LS;
#pragma unroll
        for (int st = 0; st < BW_BN / 16; ++st) {
            f16x8 af[2], bf[2];
#pragma unroll
            for (int i = 0; i < 2; ++i) af[i] = *reinterpret_cast<const f16x8*>(As + (32 * i + r32) * BW_LS + 16 * st + 8 * h);
#pragma unroll
            for (int j = 0; j < 2; ++j)
                bf[j] = *reinterpret_cast<const f16x8*>(Bs + (64 * wave + 32 * j + r32) * BW_LS + 16 * st + 8 * h);
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[i], bf[j], acc[i][j], 0, 0, 0);
        }
    };
    // stage s lives in register set s % 2 and LDS buffer s % 2; nst is even (lda is a multiple of
    // 64), so every iteration runs two whole stages.  Loads past the last stage re-read stage
    // nst - 1 (in bounds) and are never computed.
    BwdRegs r0, r1;
    load(0, r0);
    load(1, r1);
    store(r0, 0);
    __syncthreads();
    for (int s = 0; s < nst; s += 2) {
        load(min(s + 2, nst - 1), r0);
        compute(0);
        store(r1, 1);
        __syncthreads();
        load(min(s + 3, nst - 1), r1);
        compute(1);
        store(r0, 0);
        __syncthreads();
    }
    // epilogue, two passes of 32 rows through LDS (the pipeline buffers are no longer read):
    // element (row, c) at row * BW_OW + c + 4 (c / 16)
    float* ot = reinterpret_cast<float*>(smem);
    const bool vec = (p.ldo % 8 == 0) && ((uintptr_t)p.out % 16 == 0);
#pragma unroll
    for (int pass = 0; pass < 2; ++pass) {  // unrolled: acc[pass] must stay in registers
        if (pass) __syncthreads();
        // C layout: lane l, register e holds row 8 (e / 4) + 4 (l / 32) + e % 4, column l % 32
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const int row = 8 * (e / 4) + 4 * h + e % 4, c = 64 * wave + 32 * j + r32;
                ot[row * BW_OW + c + 4 * (c >> 4)] = acc[pass][j][e];
            }
        __syncthreads();
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
            const int row = 8 * wave + 4 * hh + (lane >> 4), run = lane & 15;
            const float* src = ot + row * BW_OW + 20 * run;
            float v[16];
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const f32x4 t = *reinterpret_cast<const f32x4*>(src + 4 * q);
                v[4 * q] = t.x; v[4 * q + 1] = t.y; v[4 * q + 2] = t.z; v[4 * q + 3] = t.w;
            }
            const int64_t m = m0 + 32 * pass + row, k = k0 + 16 * run;
            const int E = p.e[min(m, p.M - 1)];
            if constexpr (G > 0) {
                hadamard16<G>(v, lane);
                const float nrm = hadamard_norm<G>();
#pragma unroll
                for (int i = 0; i < 16; ++i) v[i] *= nrm;
            }
#pragma unroll
            for (int i = 0; i < 16; ++i) v[i] = __builtin_ldexpf(v[i], E);
            if (m < p.M && k < p.K) {
                store8_rt(p.out, p.out_dt, m * p.ldo + k, v, 8, vec);
                store8_rt(p.out, p.out_dt, m * p.ldo + k + 8, v + 8, 8, vec);
            }
        }
    }
}

}  // namespace

hipError_t run_bwd_rows(const void* dy, int dy_dt, int64_t ldd, int64_t M, int64_t N, const void* s, int s_dt,
                        int64_t s_stride, f16* a, int64_t lda, int32_t* e, hipStream_t st) {
    if (M == 0) return hipSuccess;
    if (lda < N || lda % (2 * BW_BN)) return hipErrorInvalidValue;
    const dim3 grid((unsigned)M), block(256);
    switch (dy_dt) {
        case DT_F32: hipLaunchKernelGGL((bwd_rows_kernel<float>), grid, block, 0, st, (const float*)dy, ldd, N, s, s_dt, s_stride, a, lda, e); break;
        case DT_F16: hipLaunchKernelGGL((bwd_rows_kernel<f16>), grid, block, 0, st, (const f16*)dy, ldd, N, s, s_dt, s_stride, a, lda, e); break;
        case DT_BF16: hipLaunchKernelGGL((bwd_rows_kernel<bf16_t>), grid, block, 0, st, (const bf16_t*)dy, ldd, N, s, s_dt, s_stride, a, lda, e); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t run_bwd_gemm(const BwdGemmArgs& p, hipStream_t st) {
    if (p.M == 0 || p.K == 0) return hipSuccess;
    // the kernel's loads assume: K a multiple of 16 (4-byte weight loads from clamped columns),
    // 4-byte aligned weight rows, lda a multiple of 64 covering N, N >= 1
    if (p.K % 16 || p.ldb % 4 || (uintptr_t)p.b % 4 || p.lda % (2 * BW_BN) || p.lda < p.N || p.N < 1 ||
        (uintptr_t)p.a % 16)
        return hipErrorInvalidValue;
    const dim3 grid((unsigned)((p.K + BW_BK - 1) / BW_BK), (unsigned)((p.M + BW_BM - 1) / BW_BM));
    bool ok = false;
    auto go = [&]<int G>() {
        hipLaunchKernelGGL((bwd_gemm_kernel<G>), grid, dim3(256), 0, st, p);
        ok = true;
    };
    if (!dispatch_group(p.G, go) || !ok) return hipErrorInvalidValue;
    return hipGetLastError();
}

}  // namespace qlin
