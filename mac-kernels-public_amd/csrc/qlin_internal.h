// Internal launcher interfaces between the kernel translation units and the C ABI (capi.cpp).
#pragma once
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "qlin_device.h"

namespace qlin {

enum { DT_F32 = 0, DT_F16 = 1, DT_BF16 = 2, DT_I8 = 3, DT_U8 = 4, DT_I32 = 5, DT_E4M3 = 6, DT_NONE = -1 };
enum { PROLOGUE_WO = 0, PROLOGUE_A8 = 1, PROLOGUE_ROT_F32 = 2 };

// ---- activation prologue (prologue.hip) ----
struct PrologueArgs {
    int mode = PROLOGUE_WO;
    int x_dtype = DT_F16;
    const void* x = nullptr;
    int64_t ldx = 0;
    int64_t M = 0;
    int K = 0;
    int G = 0;                 // rotation group, 0 = none
    f16* xo = nullptr;         // WO: normalized fp16 rows
    int64_t ldo = 0;           // row stride of every output (elements)
    int32_t* eo = nullptr;     // WO: row exponents
    int8_t* qo = nullptr;      // A8: int8 rows
    float* so = nullptr;       // A8: fp32 scales
    void* xr = nullptr;        // A8: optional rotated copy in x's dtype
    float* fo = nullptr;       // ROT_F32: rotated fp32 rows
};
hipError_t run_prologue(const PrologueArgs& a, hipStream_t st);

// ---- GGUF small-M linear (gguf_smallm.hip) ----
struct GgufSmallMArgs {
    int type = 0;
    const f16* x = nullptr;
    int64_t ldx = 0;
    int M = 0;
    const int32_t* xexp = nullptr;  // per-row exponent to restore (nullptr = 0)
    const uint8_t* w = nullptr;
    int64_t row_bytes = 0;
    int N = 0, K = 0;
    const void* bias = nullptr;
    int bias_dtype = DT_NONE;
    void* y = nullptr;
    int y_dtype = DT_F16;
    int64_t ldy = 0;
    const void* wscale = nullptr;   // INT8 rows: per-row weight scale (nullptr for GGUF)
    int wscale_dtype = DT_F32;
    int64_t wscale_stride = 1;
};
bool gguf_smallm_supported(int type, int64_t M, int64_t K, int64_t row_bytes);
hipError_t run_gguf_smallm(const GgufSmallMArgs& a, hipStream_t st);

// ---- GGUF linear with activations shared in LDS and K split across workgroups (gguf_split.hip) ----
// Residual operand of a GEMM epilogue: y = dtype(r[m, n] + rs[n] * base[m, n]) with base the
// epilogue's fp32 value (bias and any LoRA term added), one fma and one rounding -- the arithmetic
// of the separate residual kernel (run_residual), so both give the same bits.  r == nullptr: none.
struct ResidualTile {
    const void* r = nullptr;     // [M, N], row stride ldr (elements)
    int r_dt = DT_F16;
    int64_t ldr = 0;
    const void* rs = nullptr;    // [N], or nullptr for 1
    int rs_dt = DT_F16;
};

// LoRA term added by a GEMM epilogue to its own output tile: y = dtype(base + scale * t up^T), t the
// fp32 low-rank activation [M, R] (row stride R), up [N, R] (f32 / f16 / bf16, row stride ld_up).
// t == nullptr: no LoRA term.  With t_parts > 1, t holds that many K-split partials t_s [M, R]
// (t_stride floats apart), added in split order when the tile loads them; with t_exp, row m of
// the sum is scaled by 2^t_exp[m] (the row exponent of normalized activations).
struct LoraTile {
    const float* t = nullptr;
    const void* up = nullptr;
    int up_dt = DT_BF16;
    int64_t ld_up = 0;
    int64_t R = 0;
    float scale = 1.0f;
    int64_t ld_t = 0;                // row stride of t (0: R)
    int t_parts = 1;
    int64_t t_stride = 0;
    const int32_t* t_exp = nullptr;
};

// The LoRA down product computed by the GGUF split kernel from the activation slices it already
// holds in LDS: t_s[m, r] = sum over split s's K range of x[m, k] down[r, k], fp32 partials
// [S][M][R] (row stride R).  Workgroup column b (of ceil(N / 128)) takes ranks b, b + blocks, ...:
// NR of them (1 or 2).  down: f32 / f16 / bf16 rows of 16-byte aligned 8-value pieces.
struct LoraDownRows {
    const void* down = nullptr;      // [R, K], row stride ld (elements); nullptr: no down product
    int dt = DT_BF16;
    int64_t ld = 0;
    int R = 0;
    int NR = 0;
    float* tpart = nullptr;
};

struct GgufSplitArgs {
    int type = 0;
    const f16* x = nullptr;          // fp16 activations, 16-byte aligned, ldx % 8 == 0
    int64_t ldx = 0;
    int M = 0;
    const int32_t* xexp = nullptr;   // per-row exponent to restore (nullptr = 0)
    const uint8_t* w = nullptr;
    int64_t row_bytes = 0;
    int N = 0, K = 0;
    int S = 1;                       // K splits (gguf_split_parts)
    float* part = nullptr;           // S > 1: fp32 partials [S][M][N]
    ResidualTile res;                // y = r + rs * (linear + bias), in the kernel that writes y
    LoraTile lora;                   // + scale * t up^T in the reduction (gguf_split_fuses_lora)
    LoraDownRows down;               // t's partials from the split kernel (gguf_split_down_ranks)
    const void* bias = nullptr;
    int bias_dtype = DT_NONE;
    void* y = nullptr;
    int y_dtype = DT_F16;
    int64_t ldy = 0;
};
// Number of K splits this path uses for the shape, 0 when it does not take it.
int gguf_split_parts(int type, int64_t M, int64_t N, int64_t K, int64_t row_bytes, int min_parts = 1);
// The reduction carries a LoRA term (lora.t, 16-byte aligned): more than 16 rows (32 x 32 tiles),
// S > 1, no residual, rank a multiple of 8 up to 128, 16-byte aligned up rows.
bool gguf_split_fuses_lora(const GgufSplitArgs& a);
// Ranks per workgroup column (1 or 2) with which the split kernel itself computes t's partials for
// a LoRA call of rank R (a.down), 0 when it does not: fewer than 17 rows, fewer than 4 K splits,
// more than 2 ranks per column, a down factor without 16-byte aligned 8-value pieces.
int gguf_split_down_ranks(const GgufSplitArgs& a, int R, int down_dt, int64_t ld_down, const void* down);
hipError_t run_gguf_split(const GgufSplitArgs& a, hipStream_t st);

// ---- GGUF single-row linear (gguf_gemv.hip) ----
// INT8 weight rows as a "format" of the small-M MFMA kernel (not a ggml type id): 32-value units
// of raw int8 codes, the per-row scale applied in the epilogue.
constexpr int INT8_ROWS = 1000;
// Longest contraction of the A8 linear and activation quantizer: the int32 sums stay exact while
// K * 128 * 127 < 2^31 (K < 132104).
constexpr int QLIN_MAX_K = 131072;
// Longest contraction of the weight-only linears (INT8, GGUF) and the rotating dequantizers: the
// fp16 MFMAs accumulate in fp32 over normalized operands (|x'| <= 1), so range is not the limit
// (the fp16 GEMM of a dequantizing backend overflows past 65504 terms; this one does not), and the
// row prologue takes rows of any length in 32768-value chunks.  The bound keeps every index and
// workspace size well inside 32-bit element counts per row.
constexpr int QLIN_MAX_K_WO = 1 << 20;
bool int8_smallm_supported(int64_t M, int64_t K, int64_t ldw, const void* w);
hipError_t run_int8_smallm(const GgufSmallMArgs& a, hipStream_t st);

// INT8 weight-only linear for one or two activation rows (int8_gemv.hip): normalized fp16 x, int8 w.
struct Int8GemvArgs {
    const f16* x = nullptr;          // the prologue's normalized fp16 rows (xraw == nullptr)
    int64_t ldx = 0;                 // row stride of x, or of xraw
    const int32_t* xexp = nullptr;
    const void* xraw = nullptr;      // raw fp16 / bf16 rows, rotated and normalized in the kernel
    int x_dtype = DT_F16;            // dtype of xraw
    int G = 0;                       // ConvRot group applied to xraw
    const int8_t* w = nullptr;
    int64_t ldw = 0;
    int64_t M = 0, N = 0, K = 0;
    const void* scale = nullptr;
    int scale_dtype = DT_F32;
    int64_t scale_stride = 1;
    const void* bias = nullptr;
    int bias_dtype = DT_NONE;
    void* y = nullptr;
    int y_dtype = DT_F16;
    int64_t ldy = 0;
};
bool int8_gemv_supported(const Int8GemvArgs& a);

hipError_t run_int8_gemv(const Int8GemvArgs& a, hipStream_t st);

struct GgufGemvArgs {
    int type = 0;
    const f16* x = nullptr;          // one fp16 activation row (16-byte aligned)
    const int32_t* xexp = nullptr;   // its exponent to restore (nullptr = 0)
    const uint8_t* w = nullptr;
    int64_t row_bytes = 0;
    int N = 0, K = 0;
    const void* bias = nullptr;
    int bias_dtype = DT_NONE;
    void* y = nullptr;
    int y_dtype = DT_F16;
};
bool gguf_gemv_supported(int type, int64_t M, int64_t K, int64_t row_bytes, const void* w, const void* x);
hipError_t run_gguf_gemv(const GgufGemvArgs& a, hipStream_t st);

// ---- weight-only fp16 MFMA tile GEMM (gemm_f16.hip) ----
enum { WO_INT8 = 0, WO_GGUF = 1, WO_F16 = 2 };  // WO_F16: fp16 weights w[n] 2^-e[n] (a decoded GGUF tensor)
// Residual scales of the 8 columns nc .. nc + 7 (1 where rs is absent), as raw bits to convert at use.
__device__ __forceinline__ void residual_scale_bits8(const ResidualTile& R, int64_t nc, int64_t N, uint32_t (&b)[8]) {
#pragma unroll
    for (int e = 0; e < 8; ++e) b[e] = (R.r && R.rs) ? load_bits_rt(R.rs, R.rs_dt, min<int64_t>(nc + e, N - 1)) : 0u;
}
__device__ __forceinline__ void residual_scales8(const ResidualTile& R, const uint32_t (&b)[8], float (&s)[8]) {
#pragma unroll
    for (int e = 0; e < 8; ++e) s[e] = R.rs ? bits_to_f32_rt(b[e], R.rs_dt) : 1.0f;
}
// v[q][e] = fma(rs[q][e], v[q][e], r[m[q], nc[q] + e]) for Q staged pieces of 8 outputs: every
// residual value is requested before the first one is used (the caller's stores follow).  Rows
// past M and columns past N read the last valid ones (their outputs are not stored).
template <int Q>
__device__ __forceinline__ void residual_apply8(const ResidualTile& R, const int64_t (&m)[Q], const int64_t (&nc)[Q],
                                                int64_t M, int64_t N, const float (&rsv)[Q][8], float (&v)[Q][8]) {
    uint32_t raw[Q][8];
    const bool f32 = R.r_dt == DT_F32;
    const bool aligned = R.ldr % 8 == 0 && (uintptr_t)R.r % 16 == 0;
#pragma unroll
    for (int q = 0; q < Q; ++q) {
        const int64_t row = min<int64_t>(m[q], M - 1) * R.ldr;
        if (aligned && nc[q] + 8 <= N) {
            if (f32) {
                const u32x4* p = reinterpret_cast<const u32x4*>(reinterpret_cast<const float*>(R.r) + row + nc[q]);
                const u32x4 a = p[0], b = p[1];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    raw[q][e] = a[e];
                    raw[q][e + 4] = b[e];
                }
            } else {
                const u32x4 a = *reinterpret_cast<const u32x4*>(reinterpret_cast<const uint16_t*>(R.r) + row + nc[q]);
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    raw[q][2 * e] = a[e] & 0xFFFFu;
                    raw[q][2 * e + 1] = a[e] >> 16;
                }
            }
        } else {
#pragma unroll
            for (int e = 0; e < 8; ++e)
                raw[q][e] = load_bits_rt(R.r, R.r_dt, row + min<int64_t>(min<int64_t>(nc[q], N - 1) + e, N - 1));
        }
    }
#pragma unroll
    for (int q = 0; q < Q; ++q)
#pragma unroll
        for (int e = 0; e < 8; ++e) v[q][e] = __builtin_fmaf(rsv[q][e], v[q][e], bits_to_f32_rt(raw[q][e], R.r_dt));
}
// o[q] = fma(rs[n + q], o[q], r[m, n + q]) for the 4 outputs n .. n + 3 of row m (columns past N
// read column N - 1; their outputs are not stored): the four residual values are requested first.
__device__ __forceinline__ void residual_apply4(const ResidualTile& R, int64_t m, int64_t n, int64_t N, float (&o)[4]) {
    float r[4], s[4];
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const int64_t c = min<int64_t>(n + q, N - 1);
        r[q] = load_rt(R.r, R.r_dt, m * R.ldr + c);
        s[q] = R.rs ? load_rt(R.rs, R.rs_dt, c) : 1.0f;
    }
#pragma unroll
    for (int q = 0; q < 4; ++q) o[q] = __builtin_fmaf(s[q], o[q], r[q]);
}
// The same for Q rows that share the columns nc .. nc + 7 and their scales.
template <int Q>
__device__ __forceinline__ void residual_apply8(const ResidualTile& R, const int64_t (&m)[Q], int64_t nc, int64_t M,
                                                int64_t N, const float (&rs)[8], float (&v)[Q][8]) {
    int64_t ncq[Q];
    float rsq[Q][8];
#pragma unroll
    for (int q = 0; q < Q; ++q) {
        ncq[q] = nc;
#pragma unroll
        for (int e = 0; e < 8; ++e) rsq[q][e] = rs[e];
    }
    residual_apply8<Q>(R, m, ncq, M, N, rsq, v);
}

// Bytes per element of an output, residual or activation dtype (f32, f16, bf16).
inline int dt_bytes(int dt) { return dt == DT_F32 ? 4 : 2; }

// A grid of 256 x 256 output tiles on the 256 CUs whose last round leaves most CUs idle: the rows
// returned (a multiple of 256) keep those tiles in whole rounds, the rest take one round of 128 x
// 256 tiles in a second launch (about 0.6 of a 256 x 256 tile's time each); 0 when that does not
// save a third of a round.
inline int64_t tail_split_rows(int64_t M, int64_t N) {
    const int64_t nt = (N + 255) / 256, tiles = (M + 255) / 256 * nt, rounds = (tiles + 255) / 256;
    if (tiles <= 256) return 0;
    const int64_t mt1 = (rounds - 1) * 256 / nt, m1 = 256 * mt1, rest = M - m1;
    if (mt1 < 1 || rest <= 0 || (rest + 127) / 128 * nt > 256) return 0;
    const double split = (double)((mt1 * nt + 255) / 256) + 0.6;
    return split <= (double)rounds - 0.33 ? m1 : 0;
}

struct GemmF16Args {
    int wkind = WO_INT8;
    int gguf_type = 0;
    const f16* x = nullptr;          // normalized fp16 activations [M, K]
    int64_t ldx = 0;
    const int32_t* xexp = nullptr;   // per-row exponents of x (nullptr = 0)
    int64_t M = 0, N = 0, K = 0;
    const void* w = nullptr;         // int8 [N, K] (ldw elements) or GGUF bytes
    int64_t ldw = 0;
    const void* scale = nullptr;     // INT8: per-row scale (f32 or f16), scale_stride 0 = scalar
    int scale_dtype = DT_F32;
    int64_t scale_stride = 1;
    const int32_t* wexp = nullptr;   // GGUF: per-row weight exponent
    const void* bias = nullptr;
    int bias_dtype = DT_NONE;
    void* y = nullptr;
    int y_dtype = DT_F16;
    int64_t ldy = 0;
    LoraTile lora;                   // INT8, 256 x 256 DMA tiles only (gemm_f16_fuses_lora)
    ResidualTile res;                // the staged-epilogue kernels only (gemm_f16_fuses_residual)
};
hipError_t run_gemm_f16(const GemmF16Args& a, hipStream_t st);
// The GGUF weight's row exponents e[n] (as run_gguf_row_exp) and the weight decoded once as
// fp16(w[n][k] 2^-e[n]) into out [N][K] (row stride K), with the GEMM load stage's arithmetic:
// exact fp32 decode, scaling by 2^-e[n], one rounding.
hipError_t run_gguf_decode_f16(int type, const uint8_t* w, int64_t row_bytes, int64_t N, int64_t K, int32_t* e,
                               f16* out, hipStream_t st);
// Whether run_gemm_f16 takes a kernel that adds a.lora in its epilogue for these operands.
bool gemm_f16_fuses_lora(const GemmF16Args& a);
// Whether run_gemm_f16 takes a kernel that applies a.res in its epilogue for these operands.
bool gemm_f16_fuses_residual(const GemmF16Args& a);

// GGUF per-row weight exponent: e[n] = exponent bounding max |w[n, :]| (gemm_f16.hip).
hipError_t run_gguf_row_exp(int type, const uint8_t* w, int64_t N, int64_t K, int32_t* e, hipStream_t st);

// ---- A8 int8 MFMA tile GEMM for AsymW4A8Int8 weights (gemm_i8.hip) ----
struct GemmI8Args {
    const int8_t* xq = nullptr;      // int8 activations [M, K]
    int64_t ldx = 0;
    const float* sx = nullptr;       // per-row activation scale
    int64_t M = 0, N = 0, K = 0;
    const uint8_t* q = nullptr;      // packed codes [N, K*bits/8]
    int64_t ldq = 0;                 // bytes per row
    int bits = 4;
    int group_size = 16;
    const void* s_rel = nullptr;     // [N, K/gs]
    int s_rel_dtype = DT_E4M3;
    int64_t ld_srel = 0;
    const float* s_ch = nullptr;     // [N]
    const float* codebook = nullptr; // [16] or nullptr
    const void* bias = nullptr;
    int bias_dtype = DT_NONE;
    void* y = nullptr;
    int y_dtype = DT_F16;
    int64_t ldy = 0;
    int8_t* w8 = nullptr;            // workspace for the decoded int8 grid [N, K] (decode-once path)
    bool w8_ready = false;           // w8 already holds the grid (run_a8_prepass decoded it)
    LoraTile lora;                   // decode-once DMA GEMM only (gemm_i8_fuses_lora)
    ResidualTile res;                // the large-tile kernels only (gemm_i8_fuses_residual)
};
// Whether run_gemm_i8 takes a kernel that adds p.lora in its epilogue for these operands.
bool gemm_i8_fuses_lora(const GemmI8Args& p);
// Whether run_gemm_i8 takes a kernel that applies p.res in its epilogue for these operands.
bool gemm_i8_fuses_residual(const GemmI8Args& p);
// A8 calls that decode the weight grid once into the workspace (N * K bytes) and run the int8 DMA
// GEMM on it: from 512 activation rows (two or more 256-row tiles would each decode the weight in
// the fused-decode kernel: W6A8 K5120 M512 N27648 138 vs 167 us, M960 N13824 110 vs 160 us), and
// above the small-M kernel's 32 rows wherever the grid has too few 256 x 256 tiles for the
// fused-decode kernel (the 128 x 128 kernel that decodes every tile it loads then leaves most CUs
// idle: W4A8 M256 K = N = 4096 42.5 vs 103.7 us).  One 256-row tile over a wide grid stays fused
// (W4A8 M256 K4096 N49152: 86 vs 151 us).
inline bool a8_decode_once(int64_t M, int64_t N, int64_t K) {
    if (K % 128) return false;
    return M >= 512 || (M > 32 && ((M + 255) / 256) * ((N + 255) / 256) < 192);
}
// The int8 weight grid alone into p.w8 ([N][K], row stride K), one thread per 64-code segment:
// group_size a multiple of 64, 16-byte aligned code rows.
bool a8_grid_supported(const GemmI8Args& p);
hipError_t run_a8_grid(const GemmI8Args& p, hipStream_t st);
// The A8 prologue a (into p.xq, p.sx) and the weight-grid decode into p.w8 in one launch, for calls
// of at least A8_PREPASS_ROWS rows that run_gemm_i8 serves with the decode-once GEMM: 16-bit
// activations, rotation group 128 or 256, rows of at most 32768 values.  After it, run_gemm_i8 with
// p.w8_ready skips the decode.
constexpr int64_t A8_PREPASS_ROWS = 2048;
bool a8_prepass_supported(const PrologueArgs& a, const GemmI8Args& p);
hipError_t run_a8_prepass(const PrologueArgs& a, const GemmI8Args& p, hipStream_t st);

// Unmerged LoRA: y += scale * (x down^T) up^T after the base linear (lora.hip).
struct LoraArgs {
    const void* x = nullptr;     // [M, K] f32/f16/bf16, unit column stride
    int x_dt = DT_F16;
    int64_t ldx = 0;
    const void* down = nullptr;  // [R, K]
    int down_dt = DT_BF16;
    int64_t ld_down = 0;
    const void* up = nullptr;    // [N, R]
    int up_dt = DT_BF16;
    int64_t ld_up = 0;
    bool vec_x = false, vec_down = false, vec_up = false;  // 16-byte loads of 8 values allowed
    float scale = 1.0f;
    int64_t M = 0, N = 0, K = 0, R = 0;
    float* t = nullptr;          // workspace: x down^T as S fp32 partials [S][M][R] (K split S ways)
    int S = 1;
    void* y = nullptr;           // [M, N] f32/f16/bf16, read and rewritten
    int y_dt = DT_F16;
    int64_t ldy = 0;
    const float* base = nullptr; // optional fp32 [M, N] base output: y = dtype(base + side) instead
    int64_t ldb = 0;
};
hipError_t run_lora(const LoraArgs& a, hipStream_t st);
// t = x down^T alone (the K-split partials and their sum); *t_final receives the [M, R] result.
hipError_t run_lora_t(const LoraArgs& a, hipStream_t st, const float** t_final);

// Residual epilogue (epilogue.hip): y = dtype(res + rscale[n] * base), base fp32 [M, N].
struct ResidualArgs {
    const float* base = nullptr;
    int64_t ldb = 0;
    const void* res = nullptr;
    int res_dt = DT_F32;
    int64_t ldr = 0;
    const void* rscale = nullptr;   // [N] or nullptr (1)
    int rscale_dt = DT_F32;
    void* y = nullptr;
    int y_dt = DT_F16;
    int64_t ldy = 0;
    int64_t M = 0, N = 0;
};
hipError_t run_residual(const ResidualArgs& a, hipStream_t st);

// ---- frozen-weight input gradient (backward.hip) ----
struct BwdGemmArgs {
    const f16* a = nullptr;      // [M][lda] normalized dy * s, zero past N (lda = N rounded up to 128)
    int64_t lda = 0;
    const int32_t* e = nullptr;  // [M] row exponents
    const int8_t* b = nullptr;   // [N][ldb] int8 weight codes (rotated basis)
    int64_t ldb = 0;
    int64_t M = 0, N = 0, K = 0;
    int G = 0;                   // ConvRot group applied to the output rows (0 = none)
    void* out = nullptr;         // dx [M][ldo]
    int out_dt = DT_F16;
    int64_t ldo = 0;
};
hipError_t run_bwd_rows(const void* dy, int dy_dt, int64_t ldd, int64_t M, int64_t N, const void* s, int s_dt,
                        int64_t s_stride, f16* a, int64_t lda, int32_t* e, hipStream_t st);
hipError_t run_bwd_gemm(const BwdGemmArgs& p, hipStream_t st);
// K splits of the LoRA down-projection for this shape (the workspace holds that many partials).
constexpr int LORA_MAX_SPLITS = 32;
int lora_splits(int64_t M, int64_t K, int64_t R);
hipError_t run_gemm_i8(const GemmI8Args& a, hipStream_t st);

// ---- standalone decodes (dequant.hip) ----
hipError_t run_dequant_gguf(int type, const uint8_t* w, int64_t total, void* out, int out_dtype, hipStream_t st);
hipError_t run_dequant_int8(const int8_t* q, int64_t N, int64_t K, int64_t ldq, const void* scale, int scale_dtype,
                            int64_t scale_stride, float* out, hipStream_t st);
hipError_t run_dequant_w4a8(const uint8_t* q, int64_t N, int64_t K, int64_t ldq, int bits, int gs, const void* s_rel,
                            int s_rel_dtype, int64_t ld_srel, const float* s_ch, const float* codebook, void* out,
                            int out_dtype, hipStream_t st);

}  // namespace qlin
