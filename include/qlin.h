/*
 * qlin -- quantized-linear engine for AMD MI355X (gfx950).  C ABI.
 *
 * Every entry point is extern "C", takes plain pointers/sizes (qlin_tensor descriptors) and a
 * HIP stream, launches asynchronously on that stream and never allocates device memory: the
 * caller passes a workspace sized by qlin_workspace_size().  The caller owns every buffer.
 * Inputs are read-only; packed weights are never copied or rewritten.
 *
 * Return codes: QLIN_OK on success; QLIN_EUNSUPPORTED when the call is well-formed but outside
 * what the kernels implement (the caller falls back, as the reference's registry does with
 * NoCapableBackendError); QLIN_EINVAL for malformed arguments; QLIN_EHIP for a HIP runtime
 * error; QLIN_EWORKSPACE when the workspace is too small.  qlin_last_error() returns a message
 * for the calling thread's most recent failure.
 *
 * Each entry point cites the reference interface it replaces (roblennon/mac-kernels-public);
 * the reference's own implementations live in un-vendored comfy-kitchen forks, so the cited
 * lines are its call sites, which pin names, argument order and semantics.
 */
#ifndef QLIN_H
#define QLIN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum {
    QLIN_OK = 0,
    QLIN_EUNSUPPORTED = 1,
    QLIN_EINVAL = 2,
    QLIN_EHIP = 3,
    QLIN_EWORKSPACE = 4,
} qlin_status;

typedef enum {
    QLIN_DT_F32 = 0,
    QLIN_DT_F16 = 1,
    QLIN_DT_BF16 = 2,
    QLIN_DT_I8 = 3,
    QLIN_DT_U8 = 4,
    QLIN_DT_I32 = 5,
    QLIN_DT_E4M3 = 6,
} qlin_dtype;

/* Strided tensor view.  shape/stride are in elements; unused dims are ignored. */
typedef struct {
    void* data;
    int32_t dtype;   /* qlin_dtype */
    int32_t ndim;    /* 1..4 */
    int64_t shape[4];
    int64_t stride[4];
} qlin_tensor;

/* Operation ids for qlin_workspace_size(). */
typedef enum {
    QLIN_OP_INT8_LINEAR = 0,
    QLIN_OP_W4A8_LINEAR = 1,
    QLIN_OP_GGUF_LINEAR = 2,
    QLIN_OP_LORA = 3,   /* qlin_lora_apply: param = the LoRA rank R */
    QLIN_OP_INT8_GRAD_INPUT = 4,  /* qlin_int8_linear_grad_input: M rows of dy, N outputs, K inputs */
    QLIN_OP_W4A8_GRAD_INPUT = 5,  /* qlin_w4a8_linear_grad_input (holds the decoded int8 grid, N*K bytes) */
    QLIN_OP_INT8_LINEAR_LORA = 6, /* qlin_int8_linear_lora: param = the LoRA rank R */
    QLIN_OP_W4A8_LINEAR_LORA = 7, /* qlin_w4a8_linear_lora: param = the LoRA rank R | group_size << 16 */
    QLIN_OP_INT8_LINEAR_RESIDUAL = 8,  /* qlin_int8_linear_residual: param as QLIN_OP_INT8_LINEAR */
    QLIN_OP_W4A8_LINEAR_RESIDUAL = 9,  /* qlin_w4a8_linear_residual: param as QLIN_OP_W4A8_LINEAR */
    QLIN_OP_GGUF_LINEAR_RESIDUAL = 10, /* qlin_gguf_linear_residual: param = the ggml type */
    QLIN_OP_GGUF_LINEAR_LORA = 11,     /* qlin_gguf_linear_lora: param = the ggml type | R << 8 */
} qlin_op;

/* ggml type ids accepted by the GGUF entry points (enum ggml_type). */
enum {
    QLIN_GGML_Q4_0 = 2, QLIN_GGML_Q4_1 = 3, QLIN_GGML_Q5_0 = 6, QLIN_GGML_Q5_1 = 7,
    QLIN_GGML_Q8_0 = 8, QLIN_GGML_Q2_K = 10, QLIN_GGML_Q3_K = 11, QLIN_GGML_Q4_K = 12,
    QLIN_GGML_Q5_K = 13, QLIN_GGML_Q6_K = 14, QLIN_GGML_IQ4_NL = 20, QLIN_GGML_IQ4_XS = 23,
};

int qlin_version(void);
const char* qlin_status_string(qlin_status s);
const char* qlin_last_error(void);

/* Bytes of device workspace an op needs for activations of M rows against an [N, K] weight.
 * `param` is the ConvRot group size (INT8), bits | group_size << 8 (W4A8: bits 4 or 6) or the ggml
 * type (GGUF).  The W4A8 group size decides whether the call decodes the int8 weight grid once into
 * the workspace (N*K bytes; group sizes that are multiples of 64); without it (param = bits) the
 * grid is counted whenever the shape alone would take that path.  `x_dtype` is the activation's
 * qlin_dtype. */
size_t qlin_workspace_size(int op, int64_t M, int64_t N, int64_t K, int param, int x_dtype);

/* Capability probe: QLIN_OK if the op would accept these shapes/parameters, else
 * QLIN_EUNSUPPORTED (message in qlin_last_error()).  Launches nothing. */
qlin_status qlin_query(int op, int64_t M, int64_t N, int64_t K, int param, int x_dtype, int out_dtype);

/* y[M,N] = rot(x)[M,K] @ (q[N,K] * scale[N])^T + bias, weight-only INT8 with optional ConvRot.
 * x: f16/bf16/f32 [M,K] (rows contiguous); q: i8 [N,K] contiguous; scale: f32/f16 [N] or [N,1]
 * or a single element; bias: optional (NULL) f32/f16/bf16 [N]; y: f16/bf16/f32 [M,N].
 * convrot_groupsize: 0 for no rotation, else a Hadamard size (power of 4, or 2*4^p), <= 256.
 * Replaces comfy_kitchen.int8_linear(x, qdata, scale, bias, out_dtype, convrot=...,
 * convrot_groupsize=...)  (bench/bench_ck01_int8.py:57; bench/bench_lora_sidepath_kernel.py:77). */
qlin_status qlin_int8_linear(const qlin_tensor* x, const qlin_tensor* qdata, const qlin_tensor* scale,
                             const qlin_tensor* bias, qlin_tensor* y, int convrot_groupsize,
                             void* workspace, size_t workspace_bytes, void* stream);

/* A8 linear over AsymW4A8Int8 packed weights: per-token int8 activation quantization
 * (quantize_int8_rowwise after the ConvRot rotation), int8 x int8 -> int32 MFMA on the int8
 * weight grid w8 = clamp(rne(level * s_rel), -127, 127), epilogue fp32(acc) * sx[m] * s_channel[n]
 * + bias.  qdata: i8/u8 [N, K*bits/8] (4-bit plane, then for 6 bits the 2-bit plane);
 * s_rel: e4m3/f16/f32 [N, K/group_size]; s_channel: f32 [N]; codebook: optional f32 [16] (4-bit
 * only; NULL = uniform levels code - 2^(bits-1)).
 * Replaces comfy_kitchen ...w4a8_int8.w4a8_int8_linear(x, qdata, s_rel, s_channel, codebook,
 * correction, bias, group_size, convrot_groupsize, out_dtype)  (bench/bench_w4a8_linear.py:82-83;
 * bench/bench_lora_fused_rank.py:42-44); `correction` (asymmetric variant) is not accepted. */
qlin_status qlin_w4a8_linear(const qlin_tensor* x, const qlin_tensor* qdata, const qlin_tensor* s_rel,
                             const qlin_tensor* s_channel, const qlin_tensor* codebook, const qlin_tensor* bias,
                             qlin_tensor* y, int bits, int group_size, int convrot_groupsize,
                             void* workspace, size_t workspace_bytes, void* stream);

/* y[M,N] = x[M,K] @ W^T + bias, W decoded from GGUF blocks of `ggml_type` laid out as
 * consecutive blocks over the row-major [N,K] elements (the GGUF tensor bytes, N*K/qk*ts long).
 * Replaces comfy_kitchen.gguf_linear(x, weight, qtype, shape, bias, out_dtype)
 * (docs/research/2026-10-03-gguf-on-metal.md:85; bench/bench_gguf_linear.py:120).
 * Above 64 rows the size qlin_workspace_size reports includes an fp16 copy of the decoded weight,
 * at most 256 MiB of it (min(N, 256 MiB / (2K)) rows): the call decodes W once, in chunks of
 * weight rows that fit the workspace (multiples of 128 rows), and runs the GEMM on each chunk.  A
 * workspace without room for 128 decoded rows still works (the GEMM then decodes every weight tile
 * it loads, much slower); all meet the same accuracy bar, with different fp32 summation orders. */
qlin_status qlin_gguf_linear(const qlin_tensor* x, const void* weight, int ggml_type, int64_t N, int64_t K,
                             const qlin_tensor* bias, qlin_tensor* y,
                             void* workspace, size_t workspace_bytes, void* stream);

/* qlin_int8_linear / qlin_w4a8_linear with unmerged LoRA fused into the linear: t = x @ lora_down^T
 * (fp32, in the workspace), then the large-M GEMM adds lora_scale * t @ lora_up^T to its own output
 * tile in fp32 after the bias and rounds once into y.  Same operand rules as the plain linears and
 * qlin_lora_apply (lora_down [R, K], lora_up [N, R], f32/f16/bf16; x is the caller's activation,
 * before any ConvRot rotation).  The kernels that carry the term are the 256 x 256 INT8 GEMM (M > 16,
 * grids of 160 tiles or more, 16-byte aligned operands) and the A8 decode-once GEMM (M >= 512, or M > 32 on grids of fewer than 192 tiles of 256 x 256), for a
 * rank that is a multiple of 8, at most 128 (at most 64 for fp32 lora_up in the A8 GEMM; ranks
 * above 64, or 32, in two passes over the tile), with 16-byte aligned lora_up rows; other calls return
 * QLIN_EUNSUPPORTED before launching anything, and the caller runs the plain linear and
 * qlin_lora_apply_base instead.  Workspace: qlin_workspace_size(QLIN_OP_INT8_LINEAR_LORA or
 * QLIN_OP_W4A8_LINEAR_LORA, M, N, K, R, x_dtype).
 * Replaces the lora_down / lora_up / lora_scale keywords of comfy_kitchen int8_linear and
 * w4a8_int8_linear (bench/bench_lora_sidepath_kernel.py:77-80; bench/bench_lora_fused_rank.py:39-44;
 * semantics docs/upstream/comfy-kitchen-mps-backend.md:54-57). */
qlin_status qlin_int8_linear_lora(const qlin_tensor* x, const qlin_tensor* qdata, const qlin_tensor* scale,
                                  const qlin_tensor* bias, qlin_tensor* y, int convrot_groupsize,
                                  const qlin_tensor* lora_down, const qlin_tensor* lora_up, float lora_scale,
                                  void* workspace, size_t workspace_bytes, void* stream);
qlin_status qlin_w4a8_linear_lora(const qlin_tensor* x, const qlin_tensor* qdata, const qlin_tensor* s_rel,
                                  const qlin_tensor* s_channel, const qlin_tensor* codebook, const qlin_tensor* bias,
                                  qlin_tensor* y, int bits, int group_size, int convrot_groupsize,
                                  const qlin_tensor* lora_down, const qlin_tensor* lora_up, float lora_scale,
                                  void* workspace, size_t workspace_bytes, void* stream);

/* qlin_gguf_linear with unmerged LoRA in the epilogue: t = x @ lora_down^T (fp32, in the workspace;
 * formed by the split kernel itself from the activation slices it stages when K is split 4 or more
 * ways and each column of its grid needs at most 2 ranks, else by a separate down kernel first),
 * then the K-split reduction of the split kernel adds lora_scale * t @ lora_up^T to each output tile
 * in fp32 after the bias and rounds once into y.  Taken from 17 rows to the split kernel's limit
 * (512 rows) where K holds at least two of its stages (the call then splits
 * K at least in two), for a rank that is a multiple of 8 up to 128 with 16-byte aligned lora_up rows;
 * other calls return QLIN_EUNSUPPORTED before launching anything, and the caller runs the plain
 * linear and qlin_lora_apply_base.  Workspace: qlin_workspace_size(QLIN_OP_GGUF_LINEAR_LORA, M, N, K,
 * ggml_type | R << 8, x_dtype).  Replaces the lora_down / lora_up / lora_scale keywords of
 * comfy_kitchen gguf_linear (tests/test_gguf_node.py:110-174; the GGUF LoRA in the epilogue,
 * docs/research/2026-10-03-gguf-on-metal.md:97, 107). */
qlin_status qlin_gguf_linear_lora(const qlin_tensor* x, const void* weight, int ggml_type, int64_t N, int64_t K,
                                  const qlin_tensor* bias, qlin_tensor* y, const qlin_tensor* lora_down,
                                  const qlin_tensor* lora_up, float lora_scale, void* workspace,
                                  size_t workspace_bytes, void* stream);

/* Bytes of the fixed per-GPU scratch behind qlin_gguf_linear_noalloc. */
#define QLIN_NOALLOC_SCRATCH_BYTES (16u << 20)

/* qlin_gguf_linear without a workspace argument and without allocating: the same kernels, with
 * their workspace (normalized activations, row exponents, K-split partials) in a fixed
 * QLIN_NOALLOC_SCRATCH_BYTES array per GPU, held until the process ends.  For callers that cannot
 * call hipMalloc or take a caller-sized buffer: code under HIP graph capture, tight serving loops,
 * harnesses that forbid allocation.  A call whose workspace (qlin_workspace_size(QLIN_OP_GGUF_LINEAR,
 * ...), less the decoded weight copy above 64 rows) exceeds the scratch returns QLIN_EWORKSPACE
 * before launching anything (every M <= 64 at N, K <= 8192 fits); the decoded copy is used when
 * the rest of the scratch holds it.  Nothing in the scratch needs to start at zero.  All calls on one GPU share
 * its scratch: calls that overlap in time on that GPU (concurrent streams, or threads) race.
 * No counterpart in the reference; otherwise identical to qlin_gguf_linear (results bit-identical
 * whenever the scratch left over holds the decoded weight copy that qlin_gguf_linear's workspace
 * holds: always up to 64 rows; above, when N*K*2 bytes fit beside the rest). */
qlin_status qlin_gguf_linear_noalloc(const qlin_tensor* x, const void* weight, int ggml_type, int64_t N,
                                     int64_t K, const qlin_tensor* bias, qlin_tensor* y, void* stream);

/* Unmerged LoRA on a finished linear output: y[m,n] = dtype(y[m,n] + lora_scale * sum_r t[m,r] *
 * lora_up[n,r]) with t = x @ lora_down^T kept in fp32 in the workspace (up to 8 K-split partials of
 * M*R*4 bytes and their sum: qlin_workspace_size(QLIN_OP_LORA, M, N, K, R, x_dtype)).  x is the caller's activation (before
 * any ConvRot rotation); x [M,K], lora_down [R,K], lora_up [N,R], y [M,N]: f32/f16/bf16, unit
 * column stride.  Factors enter as hi + lo bf16 parts (16 significand bits; bf16 MFMA, the lo*lo
 * term dropped) with fp32's exponent range; sums are fp32.
 * Replaces the lora_down / lora_up / lora_scale keywords of comfy_kitchen's int8_linear,
 * w4a8_int8_linear and gguf_linear (bench/bench_lora_sidepath_kernel.py:80;
 * bench/bench_lora_fused_rank.py:36; docs/upstream/comfy-kitchen-mps-backend.md:54-57): the
 * caller runs the base linear, then this call on the same stream. */
qlin_status qlin_lora_apply(const qlin_tensor* x, const qlin_tensor* lora_down, const qlin_tensor* lora_up,
                            float lora_scale, qlin_tensor* y, void* workspace, size_t workspace_bytes,
                            void* stream);

/* qlin_lora_apply with the base linear's output read from `base` (f32 [M,N], unit column stride)
 * instead of y: y[m,n] = dtype(base[m,n] + lora_scale * sum_r t[m,r] * lora_up[n,r]).  A caller with
 * a 16-bit y runs the base linear into an fp32 buffer and passes it here, so the base and LoRA
 * terms are added in fp32 and rounded once (the reference adds them in one fp32 sum and rounds
 * once, docs/upstream/comfy-kitchen-mps-backend.md:54-56): a LoRA that cancels the weight gives
 * exactly 0, and a base beyond the 16-bit range that the LoRA term brings back stays finite. */
qlin_status qlin_lora_apply_base(const qlin_tensor* x, const qlin_tensor* lora_down, const qlin_tensor* lora_up,
                                 float lora_scale, const qlin_tensor* base, qlin_tensor* y, void* workspace,
                                 size_t workspace_bytes, void* stream);

/* Residual epilogue of a linear: y[m,n] = dtype(residual[m,n] + residual_scale[n] * base[m,n]) with
 * base the linear's output (bias, and any LoRA term, already added) in an f32 [M,N] buffer; one
 * rounding into y (f32/f16/bf16).  residual: f32/f16/bf16 [M,N]; residual_scale: optional (NULL = 1)
 * f32/f16/bf16 [N].  All views need a unit column stride.
 * Replaces the residual / residual_scale of comfy's linear_input_act on the INT8 kernel
 * (tests/test_lora_sidepath.py:363-386; tests/test_krea_adapter.py:234-236), whose fused epilogue
 * adds "bias and residual in eager's order" (docs/upstream/comfy-kitchen-mps-backend.md:52). */
qlin_status qlin_residual_epilogue(const qlin_tensor* base, const qlin_tensor* residual,
                                   const qlin_tensor* residual_scale, qlin_tensor* y, void* stream);

/* The three linears with a residual in their epilogue: y[m,n] = dtype(residual[m,n] +
 * residual_scale[n] * (linear + bias)[m,n]), each output rounded once -- the arithmetic of
 * qlin_residual_epilogue over the linear's f32 output, to the bit.  The large-M kernels (the INT8
 * GEMMs above 16 rows with 16-byte aligned operands; the A8 decode-once and 256 x 256 fused-decode
 * GEMMs; the GGUF GEMM over the decoded weight above 64 rows) apply it in their epilogue with no
 * f32 [M,N] buffer and no second launch; other calls write the linear in f32 to the end of the
 * workspace and run the residual epilogue after it.  residual: f32/f16/bf16 [M,N] with a unit
 * column stride; residual_scale: optional (NULL = 1) f32/f16/bf16 [N].  Workspace:
 * qlin_workspace_size(QLIN_OP_*_LINEAR_RESIDUAL, M, N, K, param, x_dtype).  The residual keyword has
 * no LoRA form here: with LoRA factors, run qlin_*_linear into an f32 base, qlin_lora_apply_base and
 * qlin_residual_epilogue.
 * Replace the residual / residual_scale of the reference's fused epilogue (see qlin_residual_epilogue). */
qlin_status qlin_int8_linear_residual(const qlin_tensor* x, const qlin_tensor* qdata, const qlin_tensor* scale,
                                      const qlin_tensor* bias, const qlin_tensor* residual,
                                      const qlin_tensor* residual_scale, qlin_tensor* y, int convrot_groupsize,
                                      void* workspace, size_t workspace_bytes, void* stream);
qlin_status qlin_w4a8_linear_residual(const qlin_tensor* x, const qlin_tensor* qdata, const qlin_tensor* s_rel,
                                      const qlin_tensor* s_channel, const qlin_tensor* codebook, const qlin_tensor* bias,
                                      const qlin_tensor* residual, const qlin_tensor* residual_scale, qlin_tensor* y,
                                      int bits, int group_size, int convrot_groupsize, void* workspace,
                                      size_t workspace_bytes, void* stream);
qlin_status qlin_gguf_linear_residual(const qlin_tensor* x, const void* weight, int ggml_type, int64_t N, int64_t K,
                                      const qlin_tensor* bias, const qlin_tensor* residual,
                                      const qlin_tensor* residual_scale, qlin_tensor* y, void* workspace,
                                      size_t workspace_bytes, void* stream);

/* Input gradient of the frozen INT8 linear: dx [M,K] = dy [M,N] @ W with W = rotate(q * scale) the
 * weight in the original basis (convrot_groupsize 0 = no rotation), i.e. dx = ((dy * scale) @ q) H.
 * dy * scale is normalized per row by a power of two and rounded once to fp16; the product runs on
 * fp16 MFMA with exact int8 operands and fp32 accumulation; dx is rounded once to its dtype
 * (f32/f16/bf16).  K must be a multiple of 16 and of the group; N >= 1.  No gradient for the codes,
 * scale or bias.  Workspace: qlin_workspace_size(QLIN_OP_INT8_GRAD_INPUT, M, N, K, 0, dy_dtype).
 * Replaces comfy_kitchen int8_linear_grad_input(dy, qdata, scale, convrot, convrot_groupsize,
 * out_dtype) (bench/bench_int8_backward.py:15, 52) and the backward of int8_linear_trainable
 * (train/train_lora.py:187-188, 210). */
qlin_status qlin_int8_linear_grad_input(const qlin_tensor* dy, const qlin_tensor* qdata, const qlin_tensor* scale,
                                        int convrot_groupsize, qlin_tensor* dx, void* workspace,
                                        size_t workspace_bytes, void* stream);

/* Input gradient of the frozen W4A8 / W6A8 linear: dx = dy @ W with W = rotate(s_channel * grid) the
 * dequantized weight (grid = the int8 grid of the codes, as qlin_dequantize_w4a8 with an int8
 * output); same arithmetic as qlin_int8_linear_grad_input.  Replaces the backward of comfy_kitchen
 * w4a8_linear_trainable (train/train_lora.py:221-223; tests/test_training_packed.py:33-36). */
qlin_status qlin_w4a8_linear_grad_input(const qlin_tensor* dy, const qlin_tensor* qdata, const qlin_tensor* s_rel,
                                        const qlin_tensor* s_channel, const qlin_tensor* codebook, qlin_tensor* dx,
                                        int bits, int group_size, int convrot_groupsize, void* workspace,
                                        size_t workspace_bytes, void* stream);

/* Decode GGUF blocks to a dense [N,K] f32 (bit-exact with gguf-py 0.19.0's fp32 decode), or
 * f16/bf16 (that value rounded once, to nearest even).  Rows may straddle blocks (flat index).
 * Replaces comfy_kitchen dequantize_gguf (docs/research/2026-10-03-gguf-on-metal.md:85, 100). */
qlin_status qlin_dequantize_gguf(const void* weight, int ggml_type, int64_t N, int64_t K, qlin_tensor* out,
                                 void* stream);

/* Decode INT8 codes: out[n,k] = f32(q[n,k]) * scale[n] (rotated basis, bit-exact), then when
 * convrot_groupsize > 0 rotate back to the original basis per group.
 * Replaces dequantize_int8 / dequantize_int8_convrot_weight (modal/weight_error_app.py:122-127;
 * bench/bench_ck01_int8.py:49). */
qlin_status qlin_dequantize_int8(const qlin_tensor* qdata, const qlin_tensor* scale, qlin_tensor* out,
                                 int convrot_groupsize, void* stream);

/* Decode AsymW4A8Int8 storage: int8 grid w8 (when out is i8) or f32 w8*s_channel, rotated back
 * per group when convrot_groupsize > 0 (f32 only).
 * Replaces dequantize_w4a8_int8_weight (modal/weight_error_app.py:326-339;
 * tests/test_training_packed.py:25-26). */
qlin_status qlin_dequantize_w4a8(const qlin_tensor* qdata, const qlin_tensor* s_rel, const qlin_tensor* s_channel,
                                 const qlin_tensor* codebook, qlin_tensor* out, int bits, int group_size,
                                 int convrot_groupsize, void* stream);

/* Per-token activation quantization: q[m,:], scale[m] = quantize_int8_rowwise(rot(x[m,:])) with
 * the arithmetic done in x's dtype as the reference does (modal/weight_error_app.py:109-115).
 * x: f16/bf16/f32 [M,K]; q: i8 [M,K]; scale: f32 [M]; convrot_groupsize 0 = no rotation.
 * xrot (optional, may be NULL): receives the rotated activation in x's dtype. */
qlin_status qlin_quantize_act_int8(const qlin_tensor* x, qlin_tensor* q, qlin_tensor* scale,
                                   int convrot_groupsize, qlin_tensor* xrot, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* QLIN_H */
