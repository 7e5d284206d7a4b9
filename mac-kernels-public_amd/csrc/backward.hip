// Input gradient of the frozen-weight packed linears (roblennon/mac-kernels-public:
// int8_linear_grad_input, bench/bench_int8_backward.py:15, 52; the backward of
// int8_linear_trainable / w4a8_linear_trainable, train/train_lora.py:187-188, 210, 221).
//
// The weight in the original basis is W[n, :] = s[n] q[n, :] H (q the stored int8 codes or the
// W4A8 int8 grid, s the per-row scale, H the block Hadamard of the ConvRot group, H = H^T = H^-1),
// so  dx = dy W = ((dy diag(s)) q) H.
//   bwd_rows_kernel: a[m, n] = fp16((dy[m, n] s[n]) 2^-E[m]), E[m] the exponent of the row's
//     max |dy s| (one rounding, no overflow or underflow of the row's large values), rows
//     zero-padded to a multiple of 128;
//   bwd_gemm_kernel: c = a q over n with fp16 MFMA (the int8 codes are exact fp16), one
//     workgroup per 128 rows x 256 columns of dx; the weight tile goes to LDS as stored (rows
//     of n, k contiguous) and each MFMA fragment (8 consecutive n of one column) is one
//     transposing 8-byte LDS read, widened in registers; the epilogue scales rows by 2^E[m],
//     applies H to each 16-lane run of the row and rounds once to dx's dtype.
#include "qlin_internal.h"
#include "hadamard.h"

namespace qlin {

namespace {

constexpr int BW_BM = 128, BW_BK = 256, BW_BN = 64;
constexpr int BW_RING = 2;  // register sets: a stage's loads are issued two stages before its use
constexpr int BW_LS = BW_BN + 8;  // a tile LDS row stride in halves: 80 bytes, conflict-free fragment reads
// weight tile in LDS as stored, [64 n][256 k] int8, row r's 16-byte chunk c at chunk c ^ 2 (r % 8):
// the 16-byte writes of a row and the transposing fragment reads (8 rows x 2 chunk halves per
// 16 lanes, even and odd chunks in the two groups of a 32-lane half) fall on distinct banks
constexpr int BW_LB = BW_BK;
constexpr int BW_BUF = BW_BM * BW_LS * 2 + BW_BN * BW_LB;  // bytes per pipeline buffer
__device__ __forceinline__ int bw_chunk(int row, int c) { return c ^ (2 * (row & 7)); }
constexpr int BW_OW = BW_BK + BW_BK / 4;  // epilogue row stride in floats: 4 pad floats per 16

// a[m, :] = fp16(dy[m, :] * s * 2^-E[m]), zero past N up to lda; e[m] = E[m].  8 consecutive
// values per thread and step, 16-byte loads and stores when the rows allow.
template <typename T>
__device__ __forceinline__ void load8_row(const T* row, int64_t n, int64_t N, bool vec, float* v) {
    if (vec && n + 8 <= N) {
        if constexpr (sizeof(T) == 2) {
            const u32x4 w = *reinterpret_cast<const u32x4*>(row + n);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                T lo, hi;
                const uint16_t l16 = (uint16_t)(w[i] & 0xFFFFu), h16 = (uint16_t)(w[i] >> 16);
                __builtin_memcpy(&lo, &l16, 2);
                __builtin_memcpy(&hi, &h16, 2);
                v[2 * i] = dtype_traits<T>::to_f32(lo);
                v[2 * i + 1] = dtype_traits<T>::to_f32(hi);
            }
        } else {
            const f32x4 a = *reinterpret_cast<const f32x4*>(row + n), b = *reinterpret_cast<const f32x4*>(row + n + 4);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                v[i] = a[i];
                v[4 + i] = b[i];
            }
        }
    } else {
#pragma unroll
        for (int i = 0; i < 8; ++i) v[i] = n + i < N ? dtype_traits<T>::to_f32(row[n + i]) : 0.f;
    }
}

// 8 scale values from n (stride 0: one value for every row of the weight)
template <typename TS>
__device__ __forceinline__ void load8_scale(const TS* s, int64_t n, int64_t N, int64_t stride, float* v) {
    if (stride == 0) {
        const float c = dtype_traits<TS>::to_f32(s[0]);
#pragma unroll
        for (int i = 0; i < 8; ++i) v[i] = c;
    } else if (sizeof(TS) == 4 && n + 8 <= N && (uintptr_t)(s + n) % 16 == 0) {
        const f32x4 a = *reinterpret_cast<const f32x4*>(s + n), b = *reinterpret_cast<const f32x4*>(s + n + 4);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            v[i] = a[i];
            v[4 + i] = b[i];
        }
    } else {
#pragma unroll
        for (int i = 0; i < 8; ++i) v[i] = n + i < N ? dtype_traits<TS>::to_f32(s[n + i]) : 0.f;
    }
}

template <typename T, typename TS>
__global__ __launch_bounds__(256) void bwd_rows_kernel(const T* __restrict__ dy, int64_t ldd, int64_t N,
                                                       const TS* __restrict__ s, int64_t s_stride,
                                                       f16* __restrict__ a, int64_t lda, int32_t* __restrict__ e) {
    __shared__ float red[4];
    const int64_t m = blockIdx.x;
    const int tid = threadIdx.x;
    const T* row = dy + m * ldd;
    const bool vec = ldd % 8 == 0 && (uintptr_t)dy % 16 == 0;
    float amax = 0.f;
    for (int64_t n = 8 * tid; n < N; n += 2048) {
        float v[8], sv[8];
        load8_row(row, n, N, vec, v);
        load8_scale(s, n, N, s_stride, sv);
#pragma unroll
        for (int i = 0; i < 8; ++i) amax = fmaxf(amax, fabsf(v[i] * sv[i]));  // zeros past N
    }
    amax = wave_max(amax);
    if ((tid & 63) == 0) red[tid >> 6] = amax;
    __syncthreads();
    amax = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    const int E = frexp_exp(amax);
    f16* out = a + m * lda;
    for (int64_t n = 8 * tid; n < lda; n += 2048) {  // lda is a multiple of 128: whole 8-value pieces
        float v[8], sv[8];
        load8_row(row, n, N, vec, v);
        load8_scale(s, n, N, s_stride, sv);
        f16x8 hv;
#pragma unroll
        for (int i = 0; i < 8; ++i) hv[i] = (f16)__builtin_ldexpf(v[i] * sv[i], -E);  // 0 past N
        *reinterpret_cast<f16x8*>(out + n) = hv;
    }
    if (tid == 0) e[m] = E;
}

// 8 int8 (two dwords, in order) -> 8 exact fp16: bits 0x6400 | (q + 128) = 1152 + q, minus 1152.
__device__ __forceinline__ f16x8 i8x8_to_f16(uint32_t w0, uint32_t w1) {
    const f16x2 off = {(f16)-1152.0f, (f16)-1152.0f};
    const uint32_t u0 = w0 ^ 0x80808080u, u1 = w1 ^ 0x80808080u;
    const f16x2 h0 = __builtin_bit_cast(f16x2, __builtin_amdgcn_perm(0x64646464u, u0, 0x04010400u)) + off;
    const f16x2 h1 = __builtin_bit_cast(f16x2, __builtin_amdgcn_perm(0x64646464u, u0, 0x04030402u)) + off;
    const f16x2 h2 = __builtin_bit_cast(f16x2, __builtin_amdgcn_perm(0x64646464u, u1, 0x04010400u)) + off;
    const f16x2 h3 = __builtin_bit_cast(f16x2, __builtin_amdgcn_perm(0x64646464u, u1, 0x04030402u)) + off;
    return f16x8{h0[0], h0[1], h1[0], h1[1], h2[0], h2[1], h3[0], h3[1]};
}

struct BwdRegs {
    u32x4 a[2];  // 16 halves of one row of the a tile
    u32x4 b[2];  // 16 int8 of each of two weight rows
};

typedef int v2i __attribute__((ext_vector_type(2)));

// dx tile: rows m0 .. m0 + 127, columns k0 .. k0 + 255.  8 waves: wave w owns rows 64 (w / 4) ..
// + 63 and columns 64 (w % 4) .. + 63 of the tile (2 x 2 sub-tiles of 32 x 32).  Stage = 64 values
// of n: a tile [128][64] fp16 and weight tile [64][256] int8, the latter stored in LDS as read and
// transposed by the fragment reads, then widened to fp16.  Two LDS buffers and two
// register sets: each stage's global loads are issued two stages before it is computed.  WPE = 4
// caps the registers at 128 so that two workgroups share a CU (grids beyond one round).  Measured
// at M = 1056: a three-set ring, buffer loads with scalar row offsets and LDS DMA of both tiles in
// three stages were slower.
// The tile size sets the operand bytes per MFMA: at 128 x 256 a 64-value stage brings 32 KB for
// 4.2 MFLOP.
template <int G, int WPE>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(WPE, 8))) void bwd_gemm_kernel(BwdGemmArgs p) {
    constexpr int SMEM = 2 * BW_BUF > 32 * BW_OW * 4 ? 2 * BW_BUF : 32 * BW_OW * 4;
    __shared__ __attribute__((aligned(16))) uint8_t smem[SMEM];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int r32 = lane & 31, h = lane >> 5, wm = wave >> 2, wk = wave & 3;
    const int64_t m0 = (int64_t)blockIdx.y * BW_BM, k0 = (int64_t)blockIdx.x * BW_BK;
    // global load assignment: a row tid / 4, 16 halves at 16 (tid % 4); weight rows tid / 16 and
    // 32 + tid / 16 of the stage, 16 bytes at column 16 (tid % 16) of the tile
    const f16* ap = p.a + min(m0 + tid / 4, p.M - 1) * p.lda + 16 * (tid & 3);
    const int brow = tid >> 4, bc = tid & 15;
    const int8_t* bp = p.b + min(k0 + 16 * bc, p.K - 16);  // columns past K re-read (never stored)
    const int nst = (int)(p.lda / BW_BN);  // lda is N rounded up to 128; a is zero past N
    auto load = [&](int s, BwdRegs& r) {
        const u32x4* pa = reinterpret_cast<const u32x4*>(ap + (int64_t)BW_BN * s);
        r.a[0] = pa[0];
        r.a[1] = pa[1];
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int64_t n = min((int64_t)BW_BN * s + 32 * i + brow, p.N - 1);  // rows past N meet a = 0
            r.b[i] = *reinterpret_cast<const u32x4*>(bp + n * p.ldb);
        }
    };
    auto store = [&](const BwdRegs& r, int buf) {
        f16* As = reinterpret_cast<f16*>(smem + buf * BW_BUF);
        uint8_t* Bs = smem + buf * BW_BUF + BW_BM * BW_LS * 2;
        f16* ad = As + (tid >> 2) * BW_LS + 16 * (tid & 3);
        *reinterpret_cast<u32x4*>(ad) = r.a[0];
        *reinterpret_cast<u32x4*>(ad + 8) = r.a[1];
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int row = 32 * i + brow;
            *reinterpret_cast<u32x4*>(Bs + row * BW_LB + 16 * bw_chunk(row, bc)) = r.b[i];
        }
    };
    // transposing fragment reads: in each 16-lane group, lane i names row nb + i / 2 at column
    // kc + 8 (i % 2) and receives column kc + i of rows nb .. nb + 7 (ds_read_b64_tr_b8)
    const int gi = lane & 15, g = lane >> 4;
    f32x16 acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;
    auto compute = [&](int buf) {
        const f16* As = reinterpret_cast<const f16*>(smem + buf * BW_BUF);
        const uint8_t* Bs = smem + buf * BW_BUF + BW_BM * BW_LS * 2;
#pragma unroll
        for (int st = 0; st < BW_BN / 16; ++st) {
            f16x8 af[2], bf[2];
#pragma unroll
            for (int i = 0; i < 2; ++i)
                af[i] = *reinterpret_cast<const f16x8*>(As + (64 * wm + 32 * i + r32) * BW_LS + 16 * st + 8 * h);
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const int row = 16 * st + 8 * (g >> 1) + (gi >> 1), kc = 64 * wk + 32 * j + 16 * (g & 1);
                const uint8_t* src = Bs + row * BW_LB + 16 * bw_chunk(row, kc >> 4) + 8 * (gi & 1);
                const v2i w = __builtin_amdgcn_ds_read_tr8_b64_v2i32((__attribute__((address_space(3))) v2i*)src);
                bf[j] = i8x8_to_f16((uint32_t)w.x, (uint32_t)w.y);
            }
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(af[i], bf[j], acc[i][j], 0, 0, 0);
        }
    };
    // stage s lives in register set s % 2 and LDS buffer s % 2.  Loads past the last stage re-read
    // stage nst - 1 (in bounds) and are never computed.
    BwdRegs r0, r1;
    load(0, r0);
    load(1, r1);
    store(r0, 0);
    __syncthreads();
    const int last = nst - 1;
    for (int s = 0; s < nst; s += BW_RING) {
        load(min(s + 2, last), r0);
        compute(0);
        store(r1, 1);
        __syncthreads();
        load(min(s + 3, last), r1);
        compute(1);
        store(r0, 0);
        __syncthreads();
    }
    // epilogue, four passes of 32 rows through LDS (the pipeline buffers are no longer read):
    // element (row, c) at row * BW_OW + c + 4 (c / 16)
    float* ot = reinterpret_cast<float*>(smem);
    const bool vec = (p.ldo % 8 == 0) && ((uintptr_t)p.out % 16 == 0);
#pragma unroll
    for (int pass = 0; pass < 4; ++pass) {  // unrolled: acc[pass % 2] must stay in registers
        if (pass) __syncthreads();
        // C layout: lane l, register e holds row 8 (e / 4) + 4 (l / 32) + e % 4, column l % 32
        if (wm == pass / 2) {
#pragma unroll
            for (int j = 0; j < 2; ++j)
#pragma unroll
                for (int e = 0; e < 16; ++e) {
                    const int row = 8 * (e / 4) + 4 * h + e % 4, c = 64 * wk + 32 * j + r32;
                    ot[row * BW_OW + c + 4 * (c >> 4)] = acc[pass % 2][j][e];
                }
        }
        __syncthreads();
        const int row = 4 * wave + (lane >> 4), run = lane & 15;
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

}  // namespace

hipError_t run_bwd_rows(const void* dy, int dy_dt, int64_t ldd, int64_t M, int64_t N, const void* s, int s_dt,
                        int64_t s_stride, f16* a, int64_t lda, int32_t* e, hipStream_t st) {
    if (M == 0) return hipSuccess;
    if (lda < N || lda % (BW_RING * BW_BN)) return hipErrorInvalidValue;
    bool ok = false;
    auto go = [&](auto dy_tag, auto s_tag) {
        using T = decltype(dy_tag);
        using TS = decltype(s_tag);
        hipLaunchKernelGGL((bwd_rows_kernel<T, TS>), dim3((unsigned)M), dim3(256), 0, st, (const T*)dy, ldd, N,
                           (const TS*)s, s_stride, a, lda, e);
        ok = true;
    };
    auto by_s = [&](auto dy_tag) {
        if (s_dt == DT_F32) go(dy_tag, float{});
        else if (s_dt == DT_F16) go(dy_tag, f16{});
        else if (s_dt == DT_BF16) go(dy_tag, bf16_t{});
    };
    if (dy_dt == DT_F32) by_s(float{});
    else if (dy_dt == DT_F16) by_s(f16{});
    else if (dy_dt == DT_BF16) by_s(bf16_t{});
    if (!ok) return hipErrorInvalidValue;
    return hipGetLastError();
}

hipError_t run_bwd_gemm(const BwdGemmArgs& p, hipStream_t st) {
    if (p.M == 0 || p.K == 0) return hipSuccess;
    // the kernel's loads assume: K a multiple of 16 (4-byte weight loads from clamped columns),
    // 16-byte aligned weight rows, lda a multiple of 128 covering N, N >= 1
    if (p.K % 16 || p.ldb % 16 || (uintptr_t)p.b % 16 || p.lda % (BW_RING * BW_BN) || p.lda < p.N || p.N < 1 ||
        (uintptr_t)p.a % 16)
        return hipErrorInvalidValue;
    const dim3 grid((unsigned)((p.K + BW_BK - 1) / BW_BK), (unsigned)((p.M + BW_BM - 1) / BW_BM));
    bool ok = false;
    // grids of more than one workgroup per CU: 128 registers (4 waves per SIMD, a few spilled), two
    // workgroups per CU (mlp.down-sized grids: 300 against 319 us); one round: the unconstrained
    // kernel (148 against 154 us)
    const bool two = (int64_t)grid.x * grid.y > 256;
    auto go = [&]<int G>() {
        if (two) hipLaunchKernelGGL((bwd_gemm_kernel<G, 4>), grid, dim3(512), 0, st, p);
        else hipLaunchKernelGGL((bwd_gemm_kernel<G, 1>), grid, dim3(512), 0, st, p);
        ok = true;
    };
    if (!dispatch_group(p.G, go) || !ok) return hipErrorInvalidValue;
    return hipGetLastError();
}

}  // namespace qlin
