// C ABI of libqlin (include/qlin.h): argument validation, workspace layout and dispatch.
// Host code only; kernels live in the other translation units.
#include <algorithm>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <string>

#include "qlin.h"
#include "hadamard.h"
#include "gguf_exact.h"
#include "qlin_internal.h"

using namespace qlin;

// Workspace of qlin_gguf_linear_noalloc: one copy per GPU, loaded with the code object and held
// until the process ends.  Host code never passes `scratch` itself to a kernel or a copy (on the
// host it names a shadow variable, not device memory); it uses the device address that
// hipGetSymbolAddress returns for the current device (scratch_for_stream below).
static __device__ __align__(256) uint8_t scratch[QLIN_NOALLOC_SCRATCH_BYTES];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices];

// The device address of `scratch` on the GPU that runs `stream` (the current device for the null
// stream), looked up once per device with that device current.
qlin_status scratch_for_stream(hipStream_t stream, void*& ptr);

thread_local std::string g_err;

qlin_status fail(qlin_status s, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_err = buf;
    return s;
}

qlin_status hip_status(hipError_t e, const char* what) {
    if (e == hipSuccess) return QLIN_OK;
    return fail(QLIN_EHIP, "%s: %s", what, hipGetErrorString(e));
}

constexpr size_t kAlign = 256;
size_t align_up(size_t v) { return (v + kAlign - 1) / kAlign * kAlign; }

bool valid_group(int g) {
    return g == 0 || g == 4 || g == 8 || g == 16 || g == 32 || g == 64 || g == 128 || g == 256;
}

struct Mat {
    void* data;
    int dtype;
    int64_t rows, cols, ld;
};

// A 2-D matrix view with unit column stride; a 1-D tensor is one row.
qlin_status as_matrix(const qlin_tensor* t, const char* name, Mat& m) {
    if (!t || !t->data) return fail(QLIN_EINVAL, "%s is missing", name);
    if (t->ndim == 1) {
        if (t->shape[0] > 1 && t->stride[0] != 1) return fail(QLIN_EUNSUPPORTED, "%s must be contiguous", name);
        m = {t->data, t->dtype, 1, t->shape[0], t->shape[0]};
        return QLIN_OK;
    }
    if (t->ndim != 2) return fail(QLIN_EUNSUPPORTED, "%s must be 1-D or 2-D (flatten leading dims)", name);
    if (t->shape[1] > 1 && t->stride[1] != 1) return fail(QLIN_EUNSUPPORTED, "%s needs unit column stride", name);
    int64_t ld = t->shape[0] > 1 ? t->stride[0] : t->shape[1];
    if (ld < t->shape[1]) return fail(QLIN_EINVAL, "%s row stride %lld < cols %lld", name, (long long)ld,
                                      (long long)t->shape[1]);
    m = {t->data, t->dtype, t->shape[0], t->shape[1], ld};
    return QLIN_OK;
}

int64_t numel(const qlin_tensor* t) {
    int64_t n = 1;
    for (int i = 0; i < t->ndim; ++i) n *= t->shape[i];
    return n;
}

// A vector of n elements (any of [n], [n,1], [1,n]); returns its element stride.
qlin_status as_vector(const qlin_tensor* t, const char* name, int64_t n, bool allow_scalar, int64_t& stride) {
    if (!t || !t->data) return fail(QLIN_EINVAL, "%s is missing", name);
    int64_t cnt = numel(t);
    if (allow_scalar && cnt == 1) {
        stride = 0;
        return QLIN_OK;
    }
    if (cnt != n) return fail(QLIN_EINVAL, "%s has %lld elements, expected %lld", name, (long long)cnt, (long long)n);
    stride = 1;
    for (int i = 0; i < t->ndim; ++i)
        if (t->shape[i] == n) stride = t->stride[i];
    if (n > 1 && stride != 1) return fail(QLIN_EUNSUPPORTED, "%s must be contiguous", name);
    return QLIN_OK;
}

bool is_float(int dt) { return dt == QLIN_DT_F32 || dt == QLIN_DT_F16 || dt == QLIN_DT_BF16; }

qlin_status check_bias(const qlin_tensor* bias, int64_t N, int& bias_dtype) {
    bias_dtype = DT_NONE;
    if (!bias || !bias->data) return QLIN_OK;
    int64_t st;
    qlin_status s = as_vector(bias, "bias", N, false, st);
    if (s) return s;
    if (!is_float(bias->dtype)) return fail(QLIN_EUNSUPPORTED, "bias dtype %d unsupported", bias->dtype);
    bias_dtype = bias->dtype;
    return QLIN_OK;
}

qlin_status check_xy(const qlin_tensor* x, qlin_tensor* y, int64_t N, int64_t K, Mat& X, Mat& Y) {
    qlin_status s = as_matrix(x, "x", X);
    if (s) return s;
    if (!is_float(X.dtype)) return fail(QLIN_EUNSUPPORTED, "x dtype %d unsupported", X.dtype);
    if (X.cols != K) return fail(QLIN_EINVAL, "x has K=%lld, weight has K=%lld", (long long)X.cols, (long long)K);
    s = as_matrix(y, "y", Y);
    if (s) return s;
    if (!is_float(Y.dtype)) return fail(QLIN_EUNSUPPORTED, "y dtype %d unsupported", Y.dtype);
    if (Y.rows != X.rows || Y.cols != N)
        return fail(QLIN_EINVAL, "y must be [%lld, %lld]", (long long)X.rows, (long long)N);
    return QLIN_OK;
}

// Internal status of an impl asked for a residual its kernel does not apply (nothing launched); never
// returned through the C ABI (the public codes are 0 .. 4).
constexpr qlin_status QLIN_NOT_FUSED = (qlin_status)7;
static_assert(QLIN_NOT_FUSED != QLIN_OK && QLIN_NOT_FUSED > QLIN_EWORKSPACE, "internal status");

// Workspace carve-out (256-byte aligned pieces).
struct Carver {
    uint8_t* base;
    size_t cap, used = 0;
    void* take(size_t bytes) {
        void* p = base ? base + used : nullptr;
        used += align_up(bytes);
        return p;
    }
};

size_t ws_int8(int64_t M, int64_t K) { return align_up((size_t)(M * K * 2)) + align_up((size_t)M * 4); }
// GGUF paths by activation rows: one row -> the VALU GEMV; up to GGUF_SMALLM_MAX_M rows -> the
// MFMA kernels that stream the weights once (the split kernel, K split across workgroups, from
// gguf_split_min_m rows on); up to gguf_fused_max_m rows -> the split kernel's 64-row m-tiles;
// more (or K not a whole number of its stages) -> the weight decoded once + the fp16 GEMM.
constexpr int64_t GGUF_SMALLM_MAX_M = 64;
// Largest M of the INT8 weight-streaming kernels (the GEMV for one or two rows, then small-M MFMA).
constexpr int64_t INT8_SMALLM_MAX_M = 16;
// Measured at K = N = 4096: the split kernel costs ~10 us at any M (two launches, partials) and
// wins from M = 17 on, except Q6_K, whose 16-value units make the per-wave K-split kernel slower
// (same process: split 10.6 us against 10.9 / 12.1 / 14.1 us at M = 3 / 4 / 8; at M = 2 10.0
// against 10.6).
int64_t gguf_split_min_m(int type) { return type == gguf::Q6_K ? 3 : 17; }
// Largest M of the split kernel, whose 64-row m-tiles decode the weight in the load stage (above
// it: the weight decoded once to fp16, then the fp16-weight GEMM).  Measured at K = N = 4096: the
// split kernel is 2x faster at 65-128 rows and 1.1-1.3x at 512 rows (one round of 256 workgroups;
// Q2_K, Q3_K, Q6_K 1.13-1.28x at 512 with the block scales folded into the operand), slower from
// 640 rows on (a second round) for every format.
int64_t gguf_fused_max_m(int) { return 512; }

// K splits of the shared-activation kernel for this call, 0 when another kernel takes it.
int gguf_split_for(int type, int64_t M, int64_t N, int64_t K) {
    int qk, ts;
    if (M < gguf_split_min_m(type) || M > gguf_fused_max_m(type) || !gguf::type_info(type, qk, ts) || K % qk) return 0;
    return gguf_split_parts(type, M, N, K, (K / qk) * ts);
}

// K splits of a GGUF call with a LoRA term: the split kernel's count, at least two (its reduction
// carries the term); 0 when the call cannot take it (16 rows or fewer, past the split kernel's rows,
// K of a single stage).
int gguf_lora_splits(int type, int64_t M, int64_t N, int64_t K) {
    int qk, ts;
    if (M <= 16 || M > gguf_fused_max_m(type) || !gguf::type_info(type, qk, ts) || K % qk) return 0;
    const int S = gguf_split_parts(type, M, N, K, (K / qk) * ts, 2);
    return S >= 2 ? S : 0;
}

size_t ws_gguf(int64_t M, int64_t N, int64_t K, int type) {
    const int S = gguf_split_for(type, M, N, K);
    return align_up((size_t)(M * K * 2)) + align_up((size_t)M * 4) + align_up((size_t)N * 4) +
           (S > 1 ? align_up((size_t)S * M * N * 4) : 0);
}
// Where the split kernel does not take a call above GGUF_SMALLM_MAX_M rows, the tiled GEMM reads
// the weight once per 128-row tile: decoding it once into the workspace (fp16, N x K) and loading
// it as stored beats decoding every tile in that GEMM (Q4_K, K = N = 4096, M = 512: 200 us).  The copy is made in chunks of weight rows
// of at most GGUF_DECODE_BYTES_MAX (the decode of chunk c + 1 follows the GEMM over chunk c on
// the stream), so a large tensor such as a 128256 x 4096 output head needs 256 MiB of workspace,
// not its whole 1 GiB fp16 copy.  The call takes this path when the workspace beyond ws_gguf
// holds at least one chunk of GGUF_DECODE_CHUNK_ROWS rows (or all N); the size query asks for
// min(N, the rows of GGUF_DECODE_BYTES_MAX) rows.
constexpr int64_t GGUF_DECODE_BYTES_MAX = 256ll << 20;
constexpr int64_t GGUF_DECODE_CHUNK_ROWS = 128;  // the GEMM's tile height along N
// Rows of one decoded chunk that `bytes` of workspace hold (a multiple of the chunk unit, or N),
// 0 when not even one unit fits.
int64_t gguf_decode_rows(int64_t N, int64_t K, int64_t bytes) {
    const int64_t fit = std::min<int64_t>(bytes, GGUF_DECODE_BYTES_MAX) / (K * 2);
    if (fit >= N) return N;
    return fit / GGUF_DECODE_CHUNK_ROWS * GGUF_DECODE_CHUNK_ROWS;
}
size_t ws_gguf_decoded(int64_t M, int64_t N, int64_t K, int type) {
    if (M <= GGUF_SMALLM_MAX_M || N <= 0 || K <= 0 || gguf_split_for(type, M, N, K) > 0) return 0;
    const int64_t rows = std::max<int64_t>(gguf_decode_rows(N, K, GGUF_DECODE_BYTES_MAX),
                                           std::min<int64_t>(N, GGUF_DECODE_CHUNK_ROWS));
    return align_up((size_t)(rows * K * 2));
}
// input gradient: normalized dy rows (N rounded up to 128) + row exponents (+ the W4A8 int8 grid)
size_t ws_grad(int64_t M, int64_t N, int64_t K, bool grid) {
    const int64_t lda = (N + 127) / 128 * 128;
    return align_up((size_t)(M * lda * 2)) + align_up((size_t)M * 4) + (grid ? align_up((size_t)(N * K)) : 0);
}

// A8 workspace: int8 activations and their scales, plus the decoded int8 grid (N * K bytes) where
// the call decodes the weight once (a8_decode_once, and a group size that is a multiple of 64;
// group_size 0 = not known, the grid is counted whenever the shape alone would take that path).
bool a8_grid_in_workspace(int64_t M, int64_t N, int64_t K, int group_size) {
    return a8_decode_once(M, N, K) && group_size % 64 == 0;
}
size_t ws_w4a8(int64_t M, int64_t N, int64_t K, int group_size) {
    return align_up((size_t)(M * K)) + align_up((size_t)M * 4) +
           (a8_grid_in_workspace(M, N, K, group_size) ? align_up((size_t)(N * K)) : 0);
}

// LoRA's low-rank activation t = x down^T: S fp32 K-split partials and their sum, or one [M, R].
size_t ws_lora(int64_t M, int64_t K, int64_t R) {
    const int S = lora_splits(M, K, R);
    return align_up((size_t)(S > 1 ? S + 1 : 1) * M * (size_t)(R > 0 ? R : 0) * 4);
}
// A GGUF call's t: ws_lora for the separate down kernel, or the split kernel's own S partials.
size_t ws_gguf_lora_t(int64_t M, int64_t K, int64_t R, int S) {
    return std::max(ws_lora(M, K, R), align_up((size_t)std::max(S, 1) * M * (size_t)(R > 0 ? R : 0) * 4));
}

// LoRA operands of a fused linear call (qlin_int8_linear_lora, qlin_w4a8_linear_lora).
struct LoraIn {
    const qlin_tensor* down;
    const qlin_tensor* up;
    float scale;
};

// down [R, K] and up [N, R], float dtypes, unit column stride.
qlin_status lora_operands(const LoraIn& L, int64_t N, int64_t K, Mat& D, Mat& U) {
    qlin_status s;
    if ((s = as_matrix(L.down, "lora_down", D)) || (s = as_matrix(L.up, "lora_up", U))) return s;
    if (!is_float(D.dtype) || !is_float(U.dtype)) return fail(QLIN_EUNSUPPORTED, "lora operands must be f32/f16/bf16");
    if (D.rows < 1) return fail(QLIN_EINVAL, "lora rank must be positive");
    if (D.cols != K) return fail(QLIN_EINVAL, "lora_down is [%lld, %lld], x has K=%lld", (long long)D.rows,
                                 (long long)D.cols, (long long)K);
    if (U.rows != N || U.cols != D.rows)
        return fail(QLIN_EINVAL, "lora_up must be [%lld, %lld]", (long long)N, (long long)D.rows);
    return QLIN_OK;
}

bool vec8(const Mat& A) {  // 16-byte loads of 8 values along the rows
    const int es = A.dtype == QLIN_DT_F32 ? 4 : 2;
    return A.cols >= 8 && A.cols % 8 == 0 && (A.ld * es) % 16 == 0 && (uintptr_t)A.data % 16 == 0;
}

// Arguments of the t = x down^T kernels writing into `t` (S partials, then their sum).
LoraArgs lora_down_args(const Mat& X, const Mat& D, float* t) {
    LoraArgs a;
    a.x = X.data; a.x_dt = X.dtype; a.ldx = X.ld; a.vec_x = vec8(X);
    a.down = D.data; a.down_dt = D.dtype; a.ld_down = D.ld; a.vec_down = vec8(D);
    a.M = X.rows; a.K = X.cols; a.R = D.rows;
    a.t = t;
    a.S = lora_splits(X.rows, X.cols, D.rows);
    return a;
}

// The final t of lora_down_args(X, D, t): the sum after the S partials when K is split.
float* lora_t_final(float* t, int64_t M, int64_t K, int64_t R) {
    const int S = lora_splits(M, K, R);
    return S > 1 ? t + (int64_t)S * M * R : t;
}

// Runs the weight-only prologue unless x is already usable as the fp16 MFMA operand (fp16, no
// rotation, aligned rows), in which case x itself is used and no exponents are needed.
qlin_status wo_activations(const Mat& X, int G, Carver& ws, hipStream_t st, const f16*& xo, int64_t& ldx,
                           const int32_t*& eo) {
    if (G == 0 && X.dtype == QLIN_DT_F16 && X.ld % 8 == 0 && (uintptr_t)X.data % 16 == 0) {
        xo = (const f16*)X.data;
        ldx = X.ld;
        eo = nullptr;
        (void)ws.take((size_t)(X.rows * X.cols * 2));
        (void)ws.take((size_t)X.rows * 4);
        return QLIN_OK;
    }
    PrologueArgs p;
    p.mode = PROLOGUE_WO;
    p.x_dtype = X.dtype;
    p.x = X.data;
    p.ldx = X.ld;
    p.M = X.rows;
    p.K = (int)X.cols;
    p.G = G;
    p.xo = (f16*)ws.take((size_t)(X.rows * X.cols * 2));
    p.ldo = X.cols;
    p.eo = (int32_t*)ws.take((size_t)X.rows * 4);
    xo = p.xo;
    ldx = X.cols;
    eo = p.eo;
    return hip_status(run_prologue(p, st), "prologue");
}

qlin_status scratch_for_stream(hipStream_t stream, void*& ptr) {
    int cur = 0, dev = 0;
    hipError_t e = hipGetDevice(&cur);
    if (e != hipSuccess) return hip_status(e, "hipGetDevice");
    dev = cur;
    if (stream && (e = hipStreamGetDevice(stream, &dev)) != hipSuccess) return hip_status(e, "hipStreamGetDevice");
    if (dev < 0 || dev >= kMaxDevices) return fail(QLIN_EUNSUPPORTED, "device %d is beyond the %d supported", dev, kMaxDevices);
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        if (dev != cur && (e = hipSetDevice(dev)) != hipSuccess) return hip_status(e, "hipSetDevice");
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (dev != cur) (void)hipSetDevice(cur);
        if (e != hipSuccess) return hip_status(e, "hipGetSymbolAddress(scratch)");
        if (!p) return fail(QLIN_EHIP, "hipGetSymbolAddress(scratch) returned no address");
        g_scratch_ptr[dev] = p;
    }
    ptr = g_scratch_ptr[dev];
    return QLIN_OK;
}

}  // namespace

extern "C" {

int qlin_version(void) { return 1; }

const char* qlin_status_string(qlin_status s) {
    switch (s) {
        case QLIN_OK: return "ok";
        case QLIN_EUNSUPPORTED: return "unsupported";
        case QLIN_EINVAL: return "invalid argument";
        case QLIN_EHIP: return "HIP error";
        case QLIN_EWORKSPACE: return "workspace too small";
    }
    return "unknown";
}

const char* qlin_last_error(void) { return g_err.c_str(); }

size_t qlin_workspace_size(int op, int64_t M, int64_t N, int64_t K, int param, int x_dtype) {
    (void)param;
    (void)x_dtype;
    switch (op) {
        case QLIN_OP_INT8_LINEAR: return ws_int8(M, K);
        case QLIN_OP_W4A8_LINEAR: return ws_w4a8(M, N, K, param >> 8);  // param: bits | group_size << 8
        case QLIN_OP_GGUF_LINEAR: return ws_gguf(M, N, K, param) + ws_gguf_decoded(M, N, K, param);
        case QLIN_OP_INT8_GRAD_INPUT: return ws_grad(M, N, K, false);
        case QLIN_OP_W4A8_GRAD_INPUT: return ws_grad(M, N, K, true);
        case QLIN_OP_INT8_LINEAR_LORA: return ws_int8(M, K) + ws_lora(M, K, param);
        case QLIN_OP_W4A8_LINEAR_LORA:  // param: R | group_size << 16
            return ws_w4a8(M, N, K, param >> 16) + ws_lora(M, K, param & 0xFFFF);
        case QLIN_OP_GGUF_LINEAR_LORA: {  // param: ggml type | R << 8
            const int S = gguf_lora_splits(param & 0xFF, M, N, K);
            return align_up((size_t)(M * K * 2)) + align_up((size_t)M * 4) + align_up((size_t)N * 4) +
                   align_up((size_t)std::max(S, 1) * M * N * 4) + ws_gguf_lora_t(M, K, param >> 8, S);
        }
        // the residual variants: the linear's workspace, then room for its fp32 output when the
        // call's kernel does not apply the residual itself
        case QLIN_OP_INT8_LINEAR_RESIDUAL: return ws_int8(M, K) + align_up((size_t)(M * N * 4)) + 256;
        case QLIN_OP_W4A8_LINEAR_RESIDUAL:
            return ws_w4a8(M, N, K, param >> 8) + align_up((size_t)(M * N * 4)) + 256;
        case QLIN_OP_GGUF_LINEAR_RESIDUAL:
            return ws_gguf(M, N, K, param) + ws_gguf_decoded(M, N, K, param) + align_up((size_t)(M * N * 4)) + 256;
        case QLIN_OP_LORA: {  // the split partials, then their sum
            const int S = lora_splits(M, K, param);
            return align_up((size_t)(S > 1 ? S + 1 : 1) * M * (size_t)(param > 0 ? param : 0) * 4);
        }
    }
    return 0;
}

qlin_status qlin_query(int op, int64_t M, int64_t N, int64_t K, int param, int x_dtype, int out_dtype) {
    if (M < 0 || N < 0 || K < 0) return fail(QLIN_EINVAL, "negative shape");
    if (!is_float(x_dtype) || !is_float(out_dtype)) return fail(QLIN_EUNSUPPORTED, "dtype unsupported");
    switch (op) {
        case QLIN_OP_INT8_LINEAR:
            if (!valid_group(param)) return fail(QLIN_EUNSUPPORTED, "ConvRot group %d unsupported", param);
            if (param && K % param) return fail(QLIN_EUNSUPPORTED, "K %% group != 0");
            if (K > QLIN_MAX_K_WO) return fail(QLIN_EUNSUPPORTED, "K > %d", QLIN_MAX_K_WO);
            return QLIN_OK;
        case QLIN_OP_W4A8_LINEAR:
            if (param != 4 && param != 6) return fail(QLIN_EUNSUPPORTED, "bits %d unsupported", param);
            if (K % 64) return fail(QLIN_EUNSUPPORTED, "K %% 64 != 0");
            if (K > QLIN_MAX_K) return fail(QLIN_EUNSUPPORTED, "K > %d", QLIN_MAX_K);
            return QLIN_OK;
        case QLIN_OP_GGUF_LINEAR: {
            int qk, ts;
            if (!gguf::type_info(param, qk, ts)) return fail(QLIN_EUNSUPPORTED, "ggml type %d unsupported", param);
            if (K % qk) return fail(QLIN_EUNSUPPORTED, "K %% block != 0 (rows straddle blocks)");
            if (K % 32) return fail(QLIN_EUNSUPPORTED, "K %% 32 != 0");
            if (K > QLIN_MAX_K_WO) return fail(QLIN_EUNSUPPORTED, "K > %d", QLIN_MAX_K_WO);
            return QLIN_OK;
        }
    }
    return fail(QLIN_EUNSUPPORTED, "unknown op %d", op);
}

// dx = ((dy diag(s)) b) H on the GPU: the row prologue, then the gradient GEMM.
static qlin_status grad_input(const Mat& DY, const Mat& DX, const int8_t* b, int64_t ldb, int64_t N, int64_t K,
                              const void* sc, int sc_dt, int64_t sst, int G, Carver& ws, hipStream_t st) {
    const int64_t M = DY.rows, lda = (N + 127) / 128 * 128;
    f16* a = (f16*)ws.take((size_t)(M * lda * 2));
    int32_t* e = (int32_t*)ws.take((size_t)M * 4);
    qlin_status s;
    if ((s = hip_status(run_bwd_rows(DY.data, DY.dtype, DY.ld, M, N, sc, sc_dt, sst, a, lda, e, st), "gradient rows")))
        return s;
    BwdGemmArgs p;
    p.a = a; p.lda = lda; p.e = e; p.b = b; p.ldb = ldb; p.M = M; p.N = N; p.K = K; p.G = G;
    p.out = DX.data; p.out_dt = DX.dtype; p.ldo = DX.ld;
    return hip_status(run_bwd_gemm(p, st), "gradient gemm");
}

static qlin_status grad_shapes(int64_t N, int64_t K, int G) {
    if (N < 1) return fail(QLIN_EUNSUPPORTED, "N = 0 (the gradient is zero)");
    if (K % 16) return fail(QLIN_EUNSUPPORTED, "K %% 16 != 0");
    if (!valid_group(G)) return fail(QLIN_EUNSUPPORTED, "ConvRot group %d unsupported", G);
    if (G && K % G) return fail(QLIN_EINVAL, "K %% ConvRot group != 0");
    return QLIN_OK;
}

qlin_status qlin_int8_linear_grad_input(const qlin_tensor* dy, const qlin_tensor* qdata, const qlin_tensor* scale,
                                        int convrot_groupsize, qlin_tensor* dx, void* workspace,
                                        size_t workspace_bytes, void* stream) {
    Mat Q, DY, DX;
    qlin_status s = as_matrix(qdata, "qdata", Q);
    if (s) return s;
    if (Q.dtype != QLIN_DT_I8) return fail(QLIN_EUNSUPPORTED, "qdata must be int8");
    const int64_t N = Q.rows, K = Q.cols;
    // dy [M, N] in, dx [M, K] out
    if ((s = check_xy(dy, dx, K, N, DY, DX))) return s;
    if ((s = grad_shapes(N, K, convrot_groupsize))) return s;
    if (Q.ld % 16 || (uintptr_t)Q.data % 16) return fail(QLIN_EUNSUPPORTED, "qdata rows must be 16-byte aligned");
    int64_t sst;
    if ((s = as_vector(scale, "scale", N, true, sst))) return s;
    if (!is_float(scale->dtype)) return fail(QLIN_EUNSUPPORTED, "scale dtype %d unsupported", scale->dtype);
    const int64_t M = DY.rows;
    if (workspace_bytes < ws_grad(M, N, K, false))
        return fail(QLIN_EWORKSPACE, "workspace %zu < %zu", workspace_bytes, ws_grad(M, N, K, false));
    if (M == 0) return QLIN_OK;
    Carver ws{(uint8_t*)workspace, workspace_bytes};
    return grad_input(DY, DX, (const int8_t*)Q.data, Q.ld, N, K, scale->data, scale->dtype, sst, convrot_groupsize, ws,
                      (hipStream_t)stream);
}

qlin_status qlin_w4a8_linear_grad_input(const qlin_tensor* dy, const qlin_tensor* qdata, const qlin_tensor* s_rel,
                                        const qlin_tensor* s_channel, const qlin_tensor* codebook, qlin_tensor* dx,
                                        int bits, int group_size, int convrot_groupsize, void* workspace,
                                        size_t workspace_bytes, void* stream) {
    if (bits != 4 && bits != 6) return fail(QLIN_EUNSUPPORTED, "bits=%d unsupported (4 or 6)", bits);
    Mat Q, DY, DX, SR;
    qlin_status s = as_matrix(qdata, "qdata", Q);
    if (s) return s;
    if (Q.dtype != QLIN_DT_I8 && Q.dtype != QLIN_DT_U8) return fail(QLIN_EUNSUPPORTED, "qdata must be int8/uint8");
    if ((Q.cols * 8) % bits) return fail(QLIN_EINVAL, "qdata columns do not hold whole codes");
    const int64_t N = Q.rows, K = Q.cols * 8 / bits;
    if ((s = check_xy(dy, dx, K, N, DY, DX))) return s;
    if ((s = grad_shapes(N, K, convrot_groupsize))) return s;
    if (group_size <= 0 || K % group_size) return fail(QLIN_EINVAL, "group_size does not divide K");
    if ((s = as_matrix(s_rel, "s_rel", SR))) return s;
    if (SR.rows != N || SR.cols != K / group_size)
        return fail(QLIN_EINVAL, "s_rel must be [%lld, %lld]", (long long)N, (long long)(K / group_size));
    if (SR.dtype != QLIN_DT_E4M3 && SR.dtype != QLIN_DT_F16 && SR.dtype != QLIN_DT_BF16 && SR.dtype != QLIN_DT_F32 &&
        SR.dtype != QLIN_DT_U8)
        return fail(QLIN_EUNSUPPORTED, "s_rel dtype %d unsupported", SR.dtype);
    int64_t sst;
    if ((s = as_vector(s_channel, "s_channel", N, false, sst))) return s;
    if (s_channel->dtype != QLIN_DT_F32) return fail(QLIN_EUNSUPPORTED, "s_channel must be float32");
    const float* cb = nullptr;
    if (codebook && codebook->data) {
        if (bits != 4) return fail(QLIN_EUNSUPPORTED, "a codebook is only defined for 4-bit codes");
        int64_t cst;
        if ((s = as_vector(codebook, "codebook", 16, false, cst))) return s;
        if (codebook->dtype != QLIN_DT_F32 || cst != 1) return fail(QLIN_EUNSUPPORTED, "codebook must be contiguous float32");
        cb = (const float*)codebook->data;
    }
    const int64_t M = DY.rows;
    if (workspace_bytes < ws_grad(M, N, K, true))
        return fail(QLIN_EWORKSPACE, "workspace %zu < %zu", workspace_bytes, ws_grad(M, N, K, true));
    if (M == 0) return QLIN_OK;
    hipStream_t st = (hipStream_t)stream;
    Carver ws{(uint8_t*)workspace, workspace_bytes};
    int8_t* grid = (int8_t*)ws.take((size_t)(N * K));
    const int srdt = (SR.dtype == QLIN_DT_U8) ? DT_E4M3 : SR.dtype;
    GemmI8Args g;  // the forward's grid decode (four threads per 64 codes) when its layout allows
    g.N = N; g.K = K; g.q = (const uint8_t*)Q.data; g.ldq = Q.ld; g.bits = bits; g.group_size = group_size;
    g.s_rel = SR.data; g.s_rel_dtype = srdt; g.ld_srel = SR.ld; g.s_ch = (const float*)s_channel->data;
    g.codebook = cb; g.w8 = grid;
    if (a8_grid_supported(g)) {
        if ((s = hip_status(run_a8_grid(g, st), "w4a8 grid"))) return s;
    } else if ((s = hip_status(run_dequant_w4a8((const uint8_t*)Q.data, N, K, Q.ld, bits, group_size, SR.data, srdt,
                                                SR.ld, (const float*)s_channel->data, cb, grid, DT_I8, st),
                               "w4a8 grid"))) {
        return s;
    }
    return grad_input(DY, DX, grid, K, N, K, s_channel->data, DT_F32, sst, convrot_groupsize, ws, st);
}

// y = dtype((base or y) + lora_scale * (x down^T) up^T); base, when given, is an fp32 [M, N] view.
static qlin_status lora_impl(const qlin_tensor* x, const qlin_tensor* lora_down, const qlin_tensor* lora_up,
                             float lora_scale, const qlin_tensor* base, qlin_tensor* y, void* workspace,
                             size_t workspace_bytes, void* stream) {
    Mat X, D, U, Y, B{};
    qlin_status s;
    if ((s = as_matrix(x, "x", X)) || (s = as_matrix(lora_down, "lora_down", D)) ||
        (s = as_matrix(lora_up, "lora_up", U)) || (s = as_matrix(y, "y", Y)))
        return s;
    if (!is_float(X.dtype) || !is_float(D.dtype) || !is_float(U.dtype) || !is_float(Y.dtype))
        return fail(QLIN_EUNSUPPORTED, "lora operands must be f32/f16/bf16");
    const int64_t M = X.rows, K = X.cols, R = D.rows, N = U.rows;
    if (D.cols != K) return fail(QLIN_EINVAL, "lora_down is [%lld, %lld], x has K=%lld", (long long)R,
                                 (long long)D.cols, (long long)K);
    if (U.cols != R) return fail(QLIN_EINVAL, "lora_up has rank %lld, lora_down %lld", (long long)U.cols, (long long)R);
    if (Y.rows != M || Y.cols != N) return fail(QLIN_EINVAL, "y must be [%lld, %lld]", (long long)M, (long long)N);
    if (R < 1) return fail(QLIN_EINVAL, "lora rank must be positive");
    if (base) {
        if ((s = as_matrix(base, "base", B))) return s;
        if (B.dtype != QLIN_DT_F32 || B.rows != M || B.cols != N)
            return fail(QLIN_EINVAL, "base must be a float32 [%lld, %lld]", (long long)M, (long long)N);
    }
    const int S = lora_splits(M, K, R);
    const size_t need = align_up((size_t)(S > 1 ? S + 1 : 1) * M * (size_t)R * 4);
    if (workspace_bytes < need) return fail(QLIN_EWORKSPACE, "workspace %zu < %zu", workspace_bytes, need);
    if (M == 0 || N == 0) return QLIN_OK;
    auto vec = [](const Mat& A) {
        const int es = A.dtype == QLIN_DT_F32 ? 4 : 2;
        return A.cols >= 8 && A.cols % 8 == 0 && (A.ld * es) % 16 == 0 && (uintptr_t)A.data % 16 == 0;
    };
    LoraArgs a;
    a.x = X.data; a.x_dt = X.dtype; a.ldx = X.ld; a.vec_x = vec(X);
    a.down = D.data; a.down_dt = D.dtype; a.ld_down = D.ld; a.vec_down = vec(D);
    a.up = U.data; a.up_dt = U.dtype; a.ld_up = U.ld; a.vec_up = vec(U);
    a.scale = lora_scale;
    a.M = M; a.N = N; a.K = K; a.R = R;
    a.t = (float*)workspace;
    a.S = S;
    a.y = Y.data; a.y_dt = Y.dtype; a.ldy = Y.ld;
    a.base = base ? (const float*)B.data : nullptr; a.ldb = base ? B.ld : 0;
    return hip_status(run_lora(a, (hipStream_t)stream), "lora");
}

qlin_status qlin_lora_apply(const qlin_tensor* x, const qlin_tensor* lora_down, const qlin_tensor* lora_up,
                            float lora_scale, qlin_tensor* y, void* workspace, size_t workspace_bytes, void* stream) {
    return lora_impl(x, lora_down, lora_up, lora_scale, nullptr, y, workspace, workspace_bytes, stream);
}

qlin_status qlin_lora_apply_base(const qlin_tensor* x, const qlin_tensor* lora_down, const qlin_tensor* lora_up,
                                 float lora_scale, const qlin_tensor* base, qlin_tensor* y, void* workspace,
                                 size_t workspace_bytes, void* stream) {
    if (!base || !base->data) return fail(QLIN_EINVAL, "base is missing");
    return lora_impl(x, lora_down, lora_up, lora_scale, base, y, workspace, workspace_bytes, stream);
}

qlin_status qlin_residual_epilogue(const qlin_tensor* base, const qlin_tensor* residual,
                                   const qlin_tensor* residual_scale, qlin_tensor* y, void* stream) {
    Mat B, R, Y;
    qlin_status s;
    if ((s = as_matrix(base, "base", B)) || (s = as_matrix(residual, "residual", R)) || (s = as_matrix(y, "y", Y)))
        return s;
    if (B.dtype != QLIN_DT_F32) return fail(QLIN_EUNSUPPORTED, "base must be float32");
    if (!is_float(R.dtype) || !is_float(Y.dtype)) return fail(QLIN_EUNSUPPORTED, "residual and y must be f32/f16/bf16");
    if (R.rows != B.rows || R.cols != B.cols || Y.rows != B.rows || Y.cols != B.cols)
        return fail(QLIN_EINVAL, "base, residual and y must all be [%lld, %lld]", (long long)B.rows, (long long)B.cols);
    ResidualArgs a;
    if (residual_scale && residual_scale->data) {
        int64_t rst;
        if ((s = as_vector(residual_scale, "residual_scale", B.cols, true, rst))) return s;
        if (!is_float(residual_scale->dtype)) return fail(QLIN_EUNSUPPORTED, "residual_scale must be f32/f16/bf16");
        if (rst == 0 && B.cols > 1) return fail(QLIN_EUNSUPPORTED, "residual_scale must have N elements");
        a.rscale = residual_scale->data;
        a.rscale_dt = residual_scale->dtype;
    }
    a.base = (const float*)B.data; a.ldb = B.ld;
    a.res = R.data; a.res_dt = R.dtype; a.ldr = R.ld;
    a.y = Y.data; a.y_dt = Y.dtype; a.ldy = Y.ld;
    a.M = B.rows; a.N = B.cols;
    return hip_status(run_residual(a, (hipStream_t)stream), "residual epilogue");
}

// The INT8 weight-only linear; with L, the LoRA term joins the epilogue of the large-M DMA GEMM
// (QLIN_EUNSUPPORTED, before anything is launched, when another kernel would take the call).
// R: a residual the GEMM epilogue applies; when the call would take another kernel the impl returns
// QLIN_NOT_FUSED before launching anything (linear_with_residual then adds it in a second kernel).
static qlin_status int8_linear_impl(const qlin_tensor* x, const qlin_tensor* qdata, const qlin_tensor* scale,
                                    const qlin_tensor* bias, qlin_tensor* y, int convrot_groupsize, const LoraIn* L,
                                    void* workspace, size_t workspace_bytes, void* stream,
                                    const ResidualTile* R = nullptr) {
    Mat Q, X, Y;
    qlin_status s = as_matrix(qdata, "qdata", Q);
    if (s) return s;
    if (Q.dtype != QLIN_DT_I8) return fail(QLIN_EUNSUPPORTED, "qdata must be int8");
    const int64_t N = Q.rows, K = Q.cols;
    if ((s = check_xy(x, y, N, K, X, Y))) return s;
    if (!valid_group(convrot_groupsize)) return fail(QLIN_EUNSUPPORTED, "ConvRot group %d unsupported", convrot_groupsize);
    if (convrot_groupsize && K % convrot_groupsize)
        return fail(QLIN_EINVAL, "K=%lld is not a multiple of the ConvRot group %d", (long long)K, convrot_groupsize);
    if (K > QLIN_MAX_K_WO) return fail(QLIN_EUNSUPPORTED, "K > %d", QLIN_MAX_K_WO);
    int64_t sst;
    if ((s = as_vector(scale, "scale", N, true, sst))) return s;
    if (!is_float(scale->dtype)) return fail(QLIN_EUNSUPPORTED, "scale dtype %d unsupported", scale->dtype);
    int bdt;
    if ((s = check_bias(bias, N, bdt))) return s;
    Mat D{}, U{};
    if (L && (s = lora_operands(*L, N, K, D, U))) return s;
    const int64_t M = X.rows;
    const size_t need = ws_int8(M, K) + (L ? ws_lora(M, K, D.rows) : 0);
    if (workspace_bytes < need) return fail(QLIN_EWORKSPACE, "workspace %zu < %zu", workspace_bytes, need);
    if (M == 0 || N == 0) return QLIN_OK;
    hipStream_t st = (hipStream_t)stream;
    Carver ws{(uint8_t*)workspace, workspace_bytes};
    if (R) {
        // only the large-M GEMM applies a residual: its operands as run_gemm_f16 will see them
        if (L || M <= INT8_SMALLM_MAX_M) return QLIN_NOT_FUSED;
        GemmF16Args p;
        p.wkind = WO_INT8;
        p.K = K; p.w = Q.data; p.ldw = Q.ld;
        const bool direct = convrot_groupsize == 0 && X.dtype == QLIN_DT_F16 && X.ld % 8 == 0 && (uintptr_t)X.data % 16 == 0;
        p.x = direct ? (const f16*)X.data : (const f16*)ws.base; p.ldx = direct ? X.ld : K;
        if (!gemm_f16_fuses_residual(p)) return QLIN_NOT_FUSED;
    }
    if (L) {
        // the GEMM's operands are known before anything is launched: the activations are x itself
        // or the prologue's rows at the start of the workspace, t follows
        const bool direct = convrot_groupsize == 0 && X.dtype == QLIN_DT_F16 && X.ld % 8 == 0 && (uintptr_t)X.data % 16 == 0;
        Carver lay = ws;
        const f16* xo = (const f16*)lay.take((size_t)(M * K * 2));
        (void)lay.take((size_t)M * 4);
        float* t = (float*)lay.take(ws_lora(M, K, D.rows));
        GemmF16Args a;
        a.wkind = WO_INT8;
        a.x = direct ? (const f16*)X.data : xo; a.ldx = direct ? X.ld : K;
        a.M = M; a.N = N; a.K = K;
        a.w = Q.data; a.ldw = Q.ld;
        a.scale = scale->data; a.scale_dtype = scale->dtype; a.scale_stride = sst;
        a.bias = bias ? bias->data : nullptr; a.bias_dtype = bdt;
        a.y = Y.data; a.y_dtype = Y.dtype; a.ldy = Y.ld;
        a.lora.t = lora_t_final(t, M, K, D.rows); a.lora.up = U.data; a.lora.up_dt = U.dtype; a.lora.ld_up = U.ld;
        a.lora.R = D.rows; a.lora.scale = L->scale;
        if (M <= INT8_SMALLM_MAX_M || !gemm_f16_fuses_lora(a))
            return fail(QLIN_EUNSUPPORTED, "the LoRA term is fused only into the large-M GEMM (rank a multiple of 8, "
                                           "16-byte aligned lora_up rows)");
        const float* tf = nullptr;
        if ((s = hip_status(run_lora_t(lora_down_args(X, D, t), st, &tf), "lora down"))) return s;
        if ((s = wo_activations(X, convrot_groupsize, ws, st, a.x, a.ldx, a.xexp))) return s;
        return hip_status(run_gemm_f16(a, st), "int8 gemm with LoRA");
    }
    // weight streaming for few rows: the VALU GEMV (one or two rows), then the small-M MFMA kernel.
    // With a rotation, the GEMV rotates and normalizes fp16 / bf16 rows itself (no prologue launch).
    if (M <= 2 && convrot_groupsize) {
        Int8GemvArgs g;
        g.xraw = X.data; g.x_dtype = X.dtype; g.ldx = X.ld; g.G = convrot_groupsize;
        g.w = (const int8_t*)Q.data; g.ldw = Q.ld;
        g.M = M; g.N = N; g.K = K;
        g.scale = scale->data; g.scale_dtype = scale->dtype; g.scale_stride = sst;
        g.bias = bias ? bias->data : nullptr; g.bias_dtype = bdt;
        g.y = Y.data; g.y_dtype = Y.dtype; g.ldy = Y.ld;
        if (int8_gemv_supported(g)) return hip_status(run_int8_gemv(g, st), "int8 gemv");
    }
    GemmF16Args a;
    if ((s = wo_activations(X, convrot_groupsize, ws, st, a.x, a.ldx, a.xexp))) return s;
    if (M <= 2) {
        Int8GemvArgs g;
        g.x = a.x; g.ldx = a.ldx; g.xexp = a.xexp;
        g.w = (const int8_t*)Q.data; g.ldw = Q.ld;
        g.M = M; g.N = N; g.K = K;
        g.scale = scale->data; g.scale_dtype = scale->dtype; g.scale_stride = sst;
        g.bias = bias ? bias->data : nullptr; g.bias_dtype = bdt;
        g.y = Y.data; g.y_dtype = Y.dtype; g.ldy = Y.ld;
        if (int8_gemv_supported(g)) return hip_status(run_int8_gemv(g, st), "int8 gemv");
    }
    if (M <= INT8_SMALLM_MAX_M && int8_smallm_supported(M, K, Q.ld, Q.data)) {
        GgufSmallMArgs g;
        g.type = INT8_ROWS;
        g.x = a.x; g.ldx = a.ldx; g.M = (int)M; g.xexp = a.xexp;
        g.w = (const uint8_t*)Q.data; g.row_bytes = Q.ld; g.N = (int)N; g.K = (int)K;
        g.bias = bias ? bias->data : nullptr; g.bias_dtype = bdt;
        g.y = Y.data; g.y_dtype = Y.dtype; g.ldy = Y.ld;
        g.wscale = scale->data; g.wscale_dtype = scale->dtype; g.wscale_stride = sst;
        return hip_status(run_int8_smallm(g, st), "int8 small-M");
    }
    a.wkind = WO_INT8;
    a.M = M; a.N = N; a.K = K;
    a.w = Q.data; a.ldw = Q.ld;
    a.scale = scale->data; a.scale_dtype = scale->dtype; a.scale_stride = sst;
    a.bias = bias ? bias->data : nullptr; a.bias_dtype = bdt;
    a.y = Y.data; a.y_dtype = Y.dtype; a.ldy = Y.ld;
    if (R) a.res = *R;
    return hip_status(run_gemm_f16(a, st), "int8 gemm");
}

// y = dtype(residual + residual_scale * linear): `run(yo, R, ws, bytes)` runs the linear into yo,
// applying R in its GEMM epilogue; when it returns QLIN_NOT_FUSED (another kernel takes the call,
// nothing launched), the linear goes to an fp32 [M, N] buffer at the end of the workspace and the
// residual kernel adds it with the same fma and rounding.
extern "C++" template <class Run>
static qlin_status linear_with_residual(const qlin_tensor* y, const qlin_tensor* residual,
                                        const qlin_tensor* residual_scale, void* workspace, size_t workspace_bytes,
                                        void* stream, Run run) {
    Mat Y, Rm;
    qlin_status s;
    if ((s = as_matrix(y, "y", Y)) || (s = as_matrix(residual, "residual", Rm))) return s;
    if (!is_float(Rm.dtype)) return fail(QLIN_EUNSUPPORTED, "residual must be f32/f16/bf16");
    if (Rm.rows != Y.rows || Rm.cols != Y.cols)
        return fail(QLIN_EINVAL, "residual must be [%lld, %lld]", (long long)Y.rows, (long long)Y.cols);
    ResidualTile R;
    R.r = Rm.data; R.r_dt = Rm.dtype; R.ldr = Rm.ld;
    if (residual_scale && residual_scale->data) {
        int64_t rst;
        if ((s = as_vector(residual_scale, "residual_scale", Y.cols, false, rst))) return s;
        if (!is_float(residual_scale->dtype)) return fail(QLIN_EUNSUPPORTED, "residual_scale must be f32/f16/bf16");
        R.rs = residual_scale->data;
        R.rs_dt = residual_scale->dtype;
    }
    const size_t bb = align_up((size_t)(Y.rows * Y.cols * 4));
    if (workspace_bytes < bb + 256) return fail(QLIN_EWORKSPACE, "workspace %zu < %zu", workspace_bytes, bb + 256);
    if ((s = run(const_cast<qlin_tensor*>(y), &R, workspace, workspace_bytes - bb - 256)) != QLIN_NOT_FUSED) return s;
    uintptr_t b = (uintptr_t)workspace + workspace_bytes - bb;
    b &= ~(uintptr_t)255;
    qlin_tensor yb{};
    yb.data = (void*)b; yb.dtype = QLIN_DT_F32; yb.ndim = 2;
    yb.shape[0] = Y.rows; yb.shape[1] = Y.cols; yb.stride[0] = Y.cols; yb.stride[1] = 1;
    if ((s = run(&yb, nullptr, workspace, b - (uintptr_t)workspace))) return s;
    if (Y.rows == 0 || Y.cols == 0) return QLIN_OK;
    ResidualArgs a;
    a.base = (const float*)yb.data; a.ldb = Y.cols;
    a.res = Rm.data; a.res_dt = Rm.dtype; a.ldr = Rm.ld;
    a.rscale = R.rs; a.rscale_dt = R.rs_dt;
    a.y = Y.data; a.y_dt = Y.dtype; a.ldy = Y.ld;
    a.M = Y.rows; a.N = Y.cols;
    return hip_status(run_residual(a, (hipStream_t)stream), "residual epilogue");
}

qlin_status qlin_int8_linear_residual(const qlin_tensor* x, const qlin_tensor* qdata, const qlin_tensor* scale,
                                      const qlin_tensor* bias, const qlin_tensor* residual,
                                      const qlin_tensor* residual_scale, qlin_tensor* y, int convrot_groupsize,
                                      void* workspace, size_t workspace_bytes, void* stream) {
    return linear_with_residual(y, residual, residual_scale, workspace, workspace_bytes, stream,
                                [&](qlin_tensor* yo, const ResidualTile* R, void* w, size_t wb) {
                                    return int8_linear_impl(x, qdata, scale, bias, yo, convrot_groupsize, nullptr, w, wb,
                                                            stream, R);
                                });
}

qlin_status qlin_int8_linear(const qlin_tensor* x, const qlin_tensor* qdata, const qlin_tensor* scale,
                             const qlin_tensor* bias, qlin_tensor* y, int convrot_groupsize, void* workspace,
                             size_t workspace_bytes, void* stream) {
    return int8_linear_impl(x, qdata, scale, bias, y, convrot_groupsize, nullptr, workspace, workspace_bytes, stream);
}

qlin_status qlin_int8_linear_lora(const qlin_tensor* x, const qlin_tensor* qdata, const qlin_tensor* scale,
                                  const qlin_tensor* bias, qlin_tensor* y, int convrot_groupsize,
                                  const qlin_tensor* lora_down, const qlin_tensor* lora_up, float lora_scale,
                                  void* workspace, size_t workspace_bytes, void* stream) {
    const LoraIn L{lora_down, lora_up, lora_scale};
    return int8_linear_impl(x, qdata, scale, bias, y, convrot_groupsize, &L, workspace, workspace_bytes, stream);
}

// The GGUF linear over a given workspace (the caller's, or the no-allocation entry point's scratch).
static qlin_status gguf_linear_impl(const qlin_tensor* x, const void* weight, int ggml_type, int64_t N, int64_t K,
                                    const qlin_tensor* bias, qlin_tensor* y, void* workspace, size_t workspace_bytes,
                                    void* stream, const ResidualTile* R = nullptr) {
    int qk, ts;
    if (!gguf::type_info(ggml_type, qk, ts)) return fail(QLIN_EUNSUPPORTED, "ggml type %d unsupported", ggml_type);
    if (!weight) return fail(QLIN_EINVAL, "weight is missing");
    if (K % qk) return fail(QLIN_EUNSUPPORTED, "K=%lld is not a whole number of %d-value blocks", (long long)K, qk);
    if (K % 32) return fail(QLIN_EUNSUPPORTED, "K %% 32 != 0");
    if (K > QLIN_MAX_K_WO) return fail(QLIN_EUNSUPPORTED, "K > %d", QLIN_MAX_K_WO);
    Mat X, Y;
    qlin_status s = check_xy(x, y, N, K, X, Y);
    if (s) return s;
    int bdt;
    if ((s = check_bias(bias, N, bdt))) return s;
    const int64_t M = X.rows;
    if (workspace_bytes < ws_gguf(M, N, K, ggml_type))
        return fail(QLIN_EWORKSPACE, "workspace %zu < %zu", workspace_bytes, ws_gguf(M, N, K, ggml_type));
    if (M == 0 || N == 0) return QLIN_OK;
    const int64_t row_bytes = (K / qk) * ts;
    hipStream_t st = (hipStream_t)stream;
    Carver ws{(uint8_t*)workspace, workspace_bytes};
    const bool aligned = ((uintptr_t)weight % 4) == 0;
    // a residual rides in the epilogue of the split kernel (or its reduction) and of the GEMM over
    // the decoded fp16 weight (with room for the decoded rows); the GEMV and the small-M kernel
    // return QLIN_NOT_FUSED before any launch
    const int S = aligned ? gguf_split_for(ggml_type, M, N, K) : 0;
    if (R && S == 0 &&
        (M <= GGUF_SMALLM_MAX_M || K % 64 || (uintptr_t)workspace % 16 ||
         gguf_decode_rows(N, K, (int64_t)workspace_bytes - (int64_t)ws_gguf(M, N, K, ggml_type)) <= 0))
        return QLIN_NOT_FUSED;
    if (M == 1 && aligned) {
        const f16* xo;
        int64_t ldx;
        const int32_t* eo;
        Carver probe = ws;
        // the activation row must be fp16 and 16-byte aligned: use x itself or the prologue's row
        if ((s = wo_activations(X, 0, probe, st, xo, ldx, eo))) return s;
        if (gguf_gemv_supported(ggml_type, 1, K, row_bytes, weight, xo)) {
            GgufGemvArgs g;
            g.type = ggml_type; g.x = xo; g.xexp = eo; g.w = (const uint8_t*)weight; g.row_bytes = row_bytes;
            g.N = (int)N; g.K = (int)K;
            g.bias = bias ? bias->data : nullptr; g.bias_dtype = bdt;
            g.y = Y.data; g.y_dtype = Y.dtype;
            return hip_status(run_gguf_gemv(g, st), "gguf gemv");
        }
    }
    if (S > 0) {
        GgufSplitArgs a;
        a.type = ggml_type;
        if ((s = wo_activations(X, 0, ws, st, a.x, a.ldx, a.xexp))) return s;
        a.M = (int)M; a.N = (int)N; a.K = (int)K; a.S = S;
        a.part = S > 1 ? (float*)ws.take((size_t)S * M * N * 4) : nullptr;
        a.w = (const uint8_t*)weight; a.row_bytes = row_bytes;
        a.bias = bias ? bias->data : nullptr; a.bias_dtype = bdt;
        a.y = Y.data; a.y_dtype = Y.dtype; a.ldy = Y.ld;
        if (R) a.res = *R;
        return hip_status(run_gguf_split(a, st), "gguf split-K");
    }
    if (aligned && M <= GGUF_SMALLM_MAX_M && gguf_smallm_supported(ggml_type, M, K, row_bytes)) {
        GgufSmallMArgs a;
        a.type = ggml_type;
        int64_t ldx;
        if ((s = wo_activations(X, 0, ws, st, a.x, ldx, a.xexp))) return s;
        a.ldx = ldx;
        a.M = (int)M; a.N = (int)N; a.K = (int)K;
        a.w = (const uint8_t*)weight; a.row_bytes = row_bytes;
        a.bias = bias ? bias->data : nullptr; a.bias_dtype = bdt;
        a.y = Y.data; a.y_dtype = Y.dtype; a.ldy = Y.ld;
        return hip_status(run_gguf_smallm(a, st), "gguf small-M");
    }
    GemmF16Args a;
    if ((s = wo_activations(X, 0, ws, st, a.x, a.ldx, a.xexp))) return s;
    int32_t* wexp = (int32_t*)ws.take((size_t)N * 4);
    a.gguf_type = ggml_type;
    a.M = M; a.N = N; a.K = K;
    a.wexp = wexp;
    if (const int64_t rows = M > GGUF_SMALLM_MAX_M ? gguf_decode_rows(N, K, (int64_t)(workspace_bytes - ws.used)) : 0;
        rows > 0) {
        f16* w16 = (f16*)ws.take((size_t)(rows * K * 2));
        a.wkind = WO_F16;
        a.w = w16; a.ldw = K;
        a.bias_dtype = bdt;
        a.y_dtype = Y.dtype; a.ldy = Y.ld;
        const size_t ysz = Y.dtype == QLIN_DT_F32 ? 4 : 2, bsz = bdt == QLIN_DT_F32 ? 4 : 2;
        for (int64_t n0 = 0; n0 < N; n0 += rows) {
            const int64_t nc = std::min(rows, N - n0);
            if ((s = hip_status(run_gguf_decode_f16(ggml_type, (const uint8_t*)weight + n0 * row_bytes, row_bytes, nc, K,
                                                    wexp + n0, w16, st),
                                "gguf decode")))
                return s;
            a.N = nc;
            a.wexp = wexp + n0;
            a.bias = bias ? (const uint8_t*)bias->data + n0 * bsz : nullptr;
            a.y = (uint8_t*)Y.data + n0 * ysz;
            if (R) {
                a.res = *R;
                a.res.r = (const uint8_t*)R->r + n0 * (R->r_dt == QLIN_DT_F32 ? 4 : 2);
                if (R->rs) a.res.rs = (const uint8_t*)R->rs + n0 * (R->rs_dt == QLIN_DT_F32 ? 4 : 2);
            }
            if ((s = hip_status(run_gemm_f16(a, st), "gguf gemm"))) return s;
        }
        return QLIN_OK;
    } else {
        if ((s = hip_status(run_gguf_row_exp(ggml_type, (const uint8_t*)weight, N, K, wexp, st), "gguf row exponents")))
            return s;
        a.wkind = WO_GGUF;
        a.w = weight; a.ldw = row_bytes;
    }
    a.bias = bias ? bias->data : nullptr; a.bias_dtype = bdt;
    a.y = Y.data; a.y_dtype = Y.dtype; a.ldy = Y.ld;
    return hip_status(run_gemm_f16(a, st), "gguf gemm");
}

qlin_status qlin_gguf_linear(const qlin_tensor* x, const void* weight, int ggml_type, int64_t N, int64_t K,
                             const qlin_tensor* bias, qlin_tensor* y, void* workspace, size_t workspace_bytes,
                             void* stream) {
    return gguf_linear_impl(x, weight, ggml_type, N, K, bias, y, workspace, workspace_bytes, stream);
}

qlin_status qlin_gguf_linear_lora(const qlin_tensor* x, const void* weight, int ggml_type, int64_t N, int64_t K,
                                  const qlin_tensor* bias, qlin_tensor* y, const qlin_tensor* lora_down,
                                  const qlin_tensor* lora_up, float lora_scale, void* workspace,
                                  size_t workspace_bytes, void* stream) {
    int qk, ts;
    if (!gguf::type_info(ggml_type, qk, ts)) return fail(QLIN_EUNSUPPORTED, "ggml type %d unsupported", ggml_type);
    if (!weight) return fail(QLIN_EINVAL, "weight is missing");
    if (K % qk) return fail(QLIN_EUNSUPPORTED, "K=%lld is not a whole number of %d-value blocks", (long long)K, qk);
    if (K > QLIN_MAX_K_WO) return fail(QLIN_EUNSUPPORTED, "K > %d", QLIN_MAX_K_WO);
    Mat X, Y, D, U;
    qlin_status s = check_xy(x, y, N, K, X, Y);
    if (s) return s;
    int bdt;
    if ((s = check_bias(bias, N, bdt))) return s;
    const LoraIn L{lora_down, lora_up, lora_scale};
    if ((s = lora_operands(L, N, K, D, U))) return s;
    const int64_t M = X.rows, R = D.rows;
    const int S = ((uintptr_t)weight % 4) == 0 ? gguf_lora_splits(ggml_type, M, N, K) : 0;
    GgufSplitArgs a;
    a.type = ggml_type;
    a.M = (int)M; a.N = (int)N; a.K = (int)K; a.S = S;
    a.w = (const uint8_t*)weight; a.row_bytes = (K / qk) * ts;
    a.bias = bias ? bias->data : nullptr; a.bias_dtype = bdt;
    a.y = Y.data; a.y_dtype = Y.dtype; a.ldy = Y.ld;
    a.lora.up = U.data; a.lora.up_dt = U.dtype; a.lora.ld_up = U.ld; a.lora.R = R; a.lora.scale = lora_scale;
    if (S < 2 || !gguf_split_fuses_lora(a) || (uintptr_t)workspace % 16)
        return fail(QLIN_EUNSUPPORTED, "the GGUF LoRA term is fused only into the split kernel's reduction (17 to 512 "
                                       "rows, K of two stages or more, a 4-byte aligned weight), "
                                       "for a rank that is a multiple of 8 up to 128 with 16-byte aligned lora_up rows");
    const size_t need = align_up((size_t)(M * K * 2)) + align_up((size_t)M * 4) + align_up((size_t)N * 4) +
                        align_up((size_t)S * M * N * 4) + ws_gguf_lora_t(M, K, R, S);
    if (workspace_bytes < need) return fail(QLIN_EWORKSPACE, "workspace %zu < %zu", workspace_bytes, need);
    if (M == 0 || N == 0) return QLIN_OK;
    hipStream_t st = (hipStream_t)stream;
    Carver ws{(uint8_t*)workspace, workspace_bytes};
    float* t = (float*)ws.take(ws_gguf_lora_t(M, K, R, S));
    // t = x down^T: by the split kernel itself from the activation slices it stages (its S partials,
    // added and scaled by the row exponents in the reduction), or by the separate down kernel first
    const int NR = gguf_split_down_ranks(a, (int)R, D.dtype, D.ld, D.data);
    if (!NR) {
        const float* tf = nullptr;
        if ((s = hip_status(run_lora_t(lora_down_args(X, D, t), st, &tf), "lora down"))) return s;
        a.lora.t = tf;
    }
    if ((s = wo_activations(X, 0, ws, st, a.x, a.ldx, a.xexp))) return s;
    if (NR) {
        a.down.down = D.data; a.down.dt = D.dtype; a.down.ld = D.ld; a.down.R = (int)R; a.down.NR = NR;
        a.down.tpart = t;
        a.lora.t = t; a.lora.t_parts = S; a.lora.t_stride = M * R; a.lora.t_exp = a.xexp;
    }
    a.part = (float*)ws.take((size_t)S * M * N * 4);
    return hip_status(run_gguf_split(a, st), "gguf split-K with LoRA");
}

qlin_status qlin_gguf_linear_residual(const qlin_tensor* x, const void* weight, int ggml_type, int64_t N, int64_t K,
                                      const qlin_tensor* bias, const qlin_tensor* residual,
                                      const qlin_tensor* residual_scale, qlin_tensor* y, void* workspace,
                                      size_t workspace_bytes, void* stream) {
    return linear_with_residual(y, residual, residual_scale, workspace, workspace_bytes, stream,
                                [&](qlin_tensor* yo, const ResidualTile* R, void* w, size_t wb) {
                                    return gguf_linear_impl(x, weight, ggml_type, N, K, bias, yo, w, wb, stream, R);
                                });
}

qlin_status qlin_gguf_linear_noalloc(const qlin_tensor* x, const void* weight, int ggml_type, int64_t N, int64_t K,
                                     const qlin_tensor* bias, qlin_tensor* y, void* stream) {
    int qk, ts;
    if (!gguf::type_info(ggml_type, qk, ts)) return fail(QLIN_EUNSUPPORTED, "ggml type %d unsupported", ggml_type);
    Mat X;
    qlin_status s = as_matrix(x, "x", X);
    if (s) return s;
    if (N < 0 || K < 0) return fail(QLIN_EINVAL, "negative shape");
    const size_t need = ws_gguf(X.rows, N, K, ggml_type);
    if (need > QLIN_NOALLOC_SCRATCH_BYTES)
        return fail(QLIN_EWORKSPACE,
                    "qlin_gguf_linear_noalloc: this call needs %zu bytes of scratch, more than its fixed %zu; "
                    "use qlin_gguf_linear with a workspace",
                    need, (size_t)QLIN_NOALLOC_SCRATCH_BYTES);
    void* ws = nullptr;
    if ((s = scratch_for_stream((hipStream_t)stream, ws))) return s;
    return gguf_linear_impl(x, weight, ggml_type, N, K, bias, y, ws, QLIN_NOALLOC_SCRATCH_BYTES, stream);
}

// The A8 linear; with L, the LoRA term joins the epilogue of the decode-once DMA GEMM
// (QLIN_EUNSUPPORTED, before anything is launched, when another kernel would take the call).
static qlin_status w4a8_linear_impl(const qlin_tensor* x, const qlin_tensor* qdata, const qlin_tensor* s_rel,
                                    const qlin_tensor* s_channel, const qlin_tensor* codebook, const qlin_tensor* bias,
                                    qlin_tensor* y, int bits, int group_size, int convrot_groupsize, const LoraIn* L,
                                    void* workspace, size_t workspace_bytes, void* stream,
                                    const ResidualTile* R = nullptr) {
    if (bits != 4 && bits != 6) return fail(QLIN_EUNSUPPORTED, "bits=%d unsupported (4 or 6)", bits);
    Mat Q, X, Y, SR;
    qlin_status s = as_matrix(qdata, "qdata", Q);
    if (s) return s;
    if (Q.dtype != QLIN_DT_I8 && Q.dtype != QLIN_DT_U8) return fail(QLIN_EUNSUPPORTED, "qdata must be int8/uint8");
    if ((Q.cols * 8) % bits) return fail(QLIN_EINVAL, "qdata columns do not hold whole codes");
    const int64_t N = Q.rows, K = Q.cols * 8 / bits;
    if ((s = check_xy(x, y, N, K, X, Y))) return s;
    if (group_size <= 0 || group_size % 8 || K % group_size)
        return fail(QLIN_EUNSUPPORTED, "group_size %d unsupported for K=%lld", group_size, (long long)K);
    if (K % 64) return fail(QLIN_EUNSUPPORTED, "K %% 64 != 0");
    if (K > QLIN_MAX_K) return fail(QLIN_EUNSUPPORTED, "K > %d", QLIN_MAX_K);
    if (Q.ld % 16 || (uintptr_t)Q.data % 16) return fail(QLIN_EUNSUPPORTED, "qdata rows must be 16-byte aligned");
    if (!valid_group(convrot_groupsize)) return fail(QLIN_EUNSUPPORTED, "ConvRot group %d unsupported", convrot_groupsize);
    if (convrot_groupsize && K % convrot_groupsize) return fail(QLIN_EINVAL, "K %% ConvRot group != 0");
    if ((s = as_matrix(s_rel, "s_rel", SR))) return s;
    if (SR.rows != N || SR.cols != K / group_size)
        return fail(QLIN_EINVAL, "s_rel must be [%lld, %lld]", (long long)N, (long long)(K / group_size));
    if (SR.dtype != QLIN_DT_E4M3 && SR.dtype != QLIN_DT_F16 && SR.dtype != QLIN_DT_BF16 && SR.dtype != QLIN_DT_F32 &&
        SR.dtype != QLIN_DT_U8)
        return fail(QLIN_EUNSUPPORTED, "s_rel dtype %d unsupported", SR.dtype);
    int64_t sst;
    if ((s = as_vector(s_channel, "s_channel", N, false, sst))) return s;
    if (s_channel->dtype != QLIN_DT_F32) return fail(QLIN_EUNSUPPORTED, "s_channel must be float32");
    const float* cb = nullptr;
    if (codebook && codebook->data) {
        if (bits != 4) return fail(QLIN_EUNSUPPORTED, "a codebook is only defined for 4-bit codes");
        int64_t cst;
        if ((s = as_vector(codebook, "codebook", 16, false, cst))) return s;
        if (codebook->dtype != QLIN_DT_F32) return fail(QLIN_EUNSUPPORTED, "codebook must be float32");
        cb = (const float*)codebook->data;
    }
    int bdt;
    if ((s = check_bias(bias, N, bdt))) return s;
    Mat D{}, U{};
    if (L && (s = lora_operands(*L, N, K, D, U))) return s;
    const int64_t M = X.rows;
    const size_t need = ws_w4a8(M, N, K, group_size) + (L ? ws_lora(M, K, D.rows) : 0);
    if (workspace_bytes < need) return fail(QLIN_EWORKSPACE, "workspace %zu < %zu", workspace_bytes, need);
    if (M == 0 || N == 0) return QLIN_OK;
    hipStream_t st = (hipStream_t)stream;
    Carver ws{(uint8_t*)workspace, workspace_bytes};
    // workspace: int8 activations, their scales, the decoded weight grid (a8_grid_in_workspace), then
    // LoRA's t
    int8_t* qo = (int8_t*)ws.take((size_t)(M * K));
    float* so = (float*)ws.take((size_t)M * 4);
    GemmI8Args g;
    g.xq = qo; g.ldx = K; g.sx = so;
    g.M = M; g.N = N; g.K = K;
    g.q = (const uint8_t*)Q.data; g.ldq = Q.ld; g.bits = bits; g.group_size = group_size;
    g.s_rel = SR.data; g.s_rel_dtype = (SR.dtype == QLIN_DT_U8) ? DT_E4M3 : SR.dtype; g.ld_srel = SR.ld;
    g.s_ch = (const float*)s_channel->data; g.codebook = cb;
    g.bias = bias ? bias->data : nullptr; g.bias_dtype = bdt;
    g.y = Y.data; g.y_dtype = Y.dtype; g.ldy = Y.ld;
    if (a8_grid_in_workspace(M, N, K, group_size)) g.w8 = (int8_t*)ws.take((size_t)(N * K));
    if (R) {  // only the large-tile GEMMs apply a residual in their epilogue
        if (L || !gemm_i8_fuses_residual(g)) return QLIN_NOT_FUSED;
        g.res = *R;
    }
    float* t = nullptr;
    if (L) {
        t = (float*)ws.take(ws_lora(M, K, D.rows));
        g.lora.t = lora_t_final(t, M, K, D.rows); g.lora.up = U.data; g.lora.up_dt = U.dtype; g.lora.ld_up = U.ld;
        g.lora.R = D.rows; g.lora.scale = L->scale;
        if (!gemm_i8_fuses_lora(g))
            return fail(QLIN_EUNSUPPORTED, "the LoRA term is fused only into the A8 GEMM that runs after the weight grid is decoded "
                                           "once (from 512 rows, or above 32 rows on grids of fewer than 192 tiles of 256 x "
                                           "256; a group size that is a multiple of 64), for a rank that is a multiple of 8 "
                                           "with 16-byte aligned lora_up rows");
        const float* tf = nullptr;
        if ((s = hip_status(run_lora_t(lora_down_args(X, D, t), st, &tf), "lora down"))) return s;
    }
    PrologueArgs p;
    p.mode = PROLOGUE_A8;
    p.x_dtype = X.dtype;
    p.x = X.data;
    p.ldx = X.ld;
    p.M = M;
    p.K = (int)K;
    p.G = convrot_groupsize;
    p.qo = qo;
    p.ldo = K;
    p.so = so;
    if (a8_prepass_supported(p, g)) {  // the prologue and the grid decode in one launch
        if ((s = hip_status(run_a8_prepass(p, g, st), "A8 prologue and grid decode"))) return s;
        g.w8_ready = true;
    } else if ((s = hip_status(run_prologue(p, st), "A8 prologue"))) {
        return s;
    }
    return hip_status(run_gemm_i8(g, st), L ? "A8 gemm with LoRA" : "A8 gemm");
}

qlin_status qlin_w4a8_linear(const qlin_tensor* x, const qlin_tensor* qdata, const qlin_tensor* s_rel,
                             const qlin_tensor* s_channel, const qlin_tensor* codebook, const qlin_tensor* bias,
                             qlin_tensor* y, int bits, int group_size, int convrot_groupsize, void* workspace,
                             size_t workspace_bytes, void* stream) {
    return w4a8_linear_impl(x, qdata, s_rel, s_channel, codebook, bias, y, bits, group_size, convrot_groupsize, nullptr,
                            workspace, workspace_bytes, stream);
}

qlin_status qlin_w4a8_linear_residual(const qlin_tensor* x, const qlin_tensor* qdata, const qlin_tensor* s_rel,
                                      const qlin_tensor* s_channel, const qlin_tensor* codebook, const qlin_tensor* bias,
                                      const qlin_tensor* residual, const qlin_tensor* residual_scale, qlin_tensor* y,
                                      int bits, int group_size, int convrot_groupsize, void* workspace,
                                      size_t workspace_bytes, void* stream) {
    return linear_with_residual(y, residual, residual_scale, workspace, workspace_bytes, stream,
                                [&](qlin_tensor* yo, const ResidualTile* R, void* w, size_t wb) {
                                    return w4a8_linear_impl(x, qdata, s_rel, s_channel, codebook, bias, yo, bits,
                                                            group_size, convrot_groupsize, nullptr, w, wb, stream, R);
                                });
}

qlin_status qlin_w4a8_linear_lora(const qlin_tensor* x, const qlin_tensor* qdata, const qlin_tensor* s_rel,
                                  const qlin_tensor* s_channel, const qlin_tensor* codebook, const qlin_tensor* bias,
                                  qlin_tensor* y, int bits, int group_size, int convrot_groupsize,
                                  const qlin_tensor* lora_down, const qlin_tensor* lora_up, float lora_scale,
                                  void* workspace, size_t workspace_bytes, void* stream) {
    const LoraIn L{lora_down, lora_up, lora_scale};
    return w4a8_linear_impl(x, qdata, s_rel, s_channel, codebook, bias, y, bits, group_size, convrot_groupsize, &L,
                            workspace, workspace_bytes, stream);
}

qlin_status qlin_dequantize_gguf(const void* weight, int ggml_type, int64_t N, int64_t K, qlin_tensor* out,
                                 void* stream) {
    int qk, ts;
    if (!gguf::type_info(ggml_type, qk, ts)) return fail(QLIN_EUNSUPPORTED, "ggml type %d unsupported", ggml_type);
    if (!weight) return fail(QLIN_EINVAL, "weight is missing");
    if ((N * K) % qk) return fail(QLIN_EINVAL, "N*K is not a whole number of blocks");
    if (!out || !out->data || !is_float(out->dtype)) return fail(QLIN_EINVAL, "out must be a float tensor");
    if (numel(out) != N * K) return fail(QLIN_EINVAL, "out must hold N*K elements");
    for (int i = out->ndim - 1, expect = 1; i >= 0; --i) {
        if (out->shape[i] > 1 && out->stride[i] != expect) return fail(QLIN_EUNSUPPORTED, "out must be contiguous");
        expect *= (int)out->shape[i];
    }
    if (out->dtype == QLIN_DT_F32 && (uintptr_t)out->data % 16) return fail(QLIN_EUNSUPPORTED, "out must be 16-byte aligned");
    return hip_status(run_dequant_gguf(ggml_type, (const uint8_t*)weight, N * K, out->data, out->dtype,
                                       (hipStream_t)stream), "gguf dequantize");
}

qlin_status qlin_dequantize_int8(const qlin_tensor* qdata, const qlin_tensor* scale, qlin_tensor* out,
                                 int convrot_groupsize, void* stream) {
    Mat Q, O;
    qlin_status s = as_matrix(qdata, "qdata", Q);
    if (s) return s;
    if (Q.dtype != QLIN_DT_I8) return fail(QLIN_EUNSUPPORTED, "qdata must be int8");
    if ((s = as_matrix(out, "out", O))) return s;
    if (O.dtype != QLIN_DT_F32 || O.rows != Q.rows || O.cols != Q.cols || O.ld != O.cols)
        return fail(QLIN_EINVAL, "out must be a contiguous float32 [N, K]");
    int64_t sst;
    if ((s = as_vector(scale, "scale", Q.rows, true, sst))) return s;
    if (!is_float(scale->dtype)) return fail(QLIN_EUNSUPPORTED, "scale dtype unsupported");
    if (!valid_group(convrot_groupsize) || (convrot_groupsize && Q.cols % convrot_groupsize))
        return fail(QLIN_EUNSUPPORTED, "ConvRot group %d unsupported for K=%lld", convrot_groupsize, (long long)Q.cols);
    hipStream_t st = (hipStream_t)stream;
    if ((s = hip_status(run_dequant_int8((const int8_t*)Q.data, Q.rows, Q.cols, Q.ld, scale->data, scale->dtype, sst,
                                         (float*)O.data, st), "int8 dequantize")))
        return s;
    if (convrot_groupsize) {
        if (Q.cols > QLIN_MAX_K_WO) return fail(QLIN_EUNSUPPORTED, "K > %d", QLIN_MAX_K_WO);
        PrologueArgs p;
        p.mode = PROLOGUE_ROT_F32; p.x_dtype = DT_F32; p.x = O.data; p.ldx = O.cols;
        p.M = O.rows; p.K = (int)O.cols; p.G = convrot_groupsize; p.fo = (float*)O.data; p.ldo = O.cols;
        return hip_status(run_prologue(p, st), "rotation");
    }
    return QLIN_OK;
}

qlin_status qlin_dequantize_w4a8(const qlin_tensor* qdata, const qlin_tensor* s_rel, const qlin_tensor* s_channel,
                                 const qlin_tensor* codebook, qlin_tensor* out, int bits, int group_size,
                                 int convrot_groupsize, void* stream) {
    if (bits != 4 && bits != 6) return fail(QLIN_EUNSUPPORTED, "bits=%d unsupported", bits);
    Mat Q, SR, O;
    qlin_status s = as_matrix(qdata, "qdata", Q);
    if (s) return s;
    if (Q.dtype != QLIN_DT_I8 && Q.dtype != QLIN_DT_U8) return fail(QLIN_EUNSUPPORTED, "qdata must be int8/uint8");
    if ((Q.cols * 8) % bits) return fail(QLIN_EINVAL, "qdata columns do not hold whole codes");
    const int64_t N = Q.rows, K = Q.cols * 8 / bits;
    if (group_size <= 0 || K % group_size) return fail(QLIN_EINVAL, "group_size does not divide K");
    if ((s = as_matrix(s_rel, "s_rel", SR))) return s;
    if (SR.rows != N || SR.cols != K / group_size) return fail(QLIN_EINVAL, "s_rel shape mismatch");
    if (SR.dtype != QLIN_DT_E4M3 && SR.dtype != QLIN_DT_F16 && SR.dtype != QLIN_DT_BF16 && SR.dtype != QLIN_DT_F32 &&
        SR.dtype != QLIN_DT_U8)
        return fail(QLIN_EUNSUPPORTED, "s_rel dtype %d unsupported", SR.dtype);
    if ((s = as_matrix(out, "out", O))) return s;
    if (O.rows != N || O.cols != K || O.ld != K) return fail(QLIN_EINVAL, "out must be a contiguous [N, K]");
    if (O.dtype != QLIN_DT_I8 && O.dtype != QLIN_DT_F32) return fail(QLIN_EUNSUPPORTED, "out must be int8 or float32");
    if (O.dtype == QLIN_DT_I8 && convrot_groupsize) return fail(QLIN_EINVAL, "the int8 grid has no original-basis form");
    int64_t sst;
    if ((s = as_vector(s_channel, "s_channel", N, false, sst))) return s;
    if (s_channel->dtype != QLIN_DT_F32) return fail(QLIN_EUNSUPPORTED, "s_channel must be float32");
    const float* cb = nullptr;
    if (codebook && codebook->data) {
        // 6-bit codes reach 63: a 16-entry table is only defined for 4-bit codes
        if (bits != 4) return fail(QLIN_EUNSUPPORTED, "a codebook is only defined for 4-bit codes");
        int64_t cst;
        if ((s = as_vector(codebook, "codebook", 16, false, cst))) return s;
        if (codebook->dtype != QLIN_DT_F32) return fail(QLIN_EUNSUPPORTED, "codebook must be float32");
        cb = (const float*)codebook->data;
    }
    if (!valid_group(convrot_groupsize) || (convrot_groupsize && K % convrot_groupsize))
        return fail(QLIN_EUNSUPPORTED, "ConvRot group %d unsupported", convrot_groupsize);
    if (N == 0 || K == 0) return QLIN_OK;
    hipStream_t st = (hipStream_t)stream;
    const int srdt = (SR.dtype == QLIN_DT_U8) ? DT_E4M3 : SR.dtype;
    if (O.dtype == QLIN_DT_I8) {  // the forward's grid decode (four threads per 64 codes) when its layout allows
        GemmI8Args g;
        g.N = N; g.K = K; g.q = (const uint8_t*)Q.data; g.ldq = Q.ld; g.bits = bits; g.group_size = group_size;
        g.s_rel = SR.data; g.s_rel_dtype = srdt; g.ld_srel = SR.ld; g.s_ch = (const float*)s_channel->data;
        g.codebook = cb; g.w8 = (int8_t*)O.data;
        if (a8_grid_supported(g)) return hip_status(run_a8_grid(g, st), "w4a8 grid");
    }
    if ((s = hip_status(run_dequant_w4a8((const uint8_t*)Q.data, N, K, Q.ld, bits, group_size, SR.data, srdt, SR.ld,
                                         (const float*)s_channel->data, cb, O.data, O.dtype, st), "w4a8 dequantize")))
        return s;
    if (convrot_groupsize) {
        if (K > QLIN_MAX_K_WO) return fail(QLIN_EUNSUPPORTED, "K > %d", QLIN_MAX_K_WO);
        PrologueArgs p;
        p.mode = PROLOGUE_ROT_F32; p.x_dtype = DT_F32; p.x = O.data; p.ldx = K;
        p.M = N; p.K = (int)K; p.G = convrot_groupsize; p.fo = (float*)O.data; p.ldo = K;
        return hip_status(run_prologue(p, st), "rotation");
    }
    return QLIN_OK;
}

qlin_status qlin_quantize_act_int8(const qlin_tensor* x, qlin_tensor* q, qlin_tensor* scale, int convrot_groupsize,
                                   qlin_tensor* xrot, void* stream) {
    Mat X, Qm;
    qlin_status s = as_matrix(x, "x", X);
    if (s) return s;
    if (!is_float(X.dtype)) return fail(QLIN_EUNSUPPORTED, "x dtype unsupported");
    if ((s = as_matrix(q, "q", Qm))) return s;
    if (Qm.dtype != QLIN_DT_I8 || Qm.rows != X.rows || Qm.cols != X.cols || Qm.ld != X.cols)
        return fail(QLIN_EINVAL, "q must be a contiguous int8 [M, K]");
    int64_t sst;
    if ((s = as_vector(scale, "scale", X.rows, false, sst))) return s;
    if (scale->dtype != QLIN_DT_F32) return fail(QLIN_EINVAL, "scale must be float32");
    if (!valid_group(convrot_groupsize) || (convrot_groupsize && X.cols % convrot_groupsize))
        return fail(QLIN_EUNSUPPORTED, "ConvRot group %d unsupported", convrot_groupsize);
    if (X.cols > QLIN_MAX_K) return fail(QLIN_EUNSUPPORTED, "K > %d", QLIN_MAX_K);
    void* xr = nullptr;
    if (xrot && xrot->data) {
        Mat XR;
        if ((s = as_matrix(xrot, "xrot", XR))) return s;
        if (XR.dtype != X.dtype || XR.rows != X.rows || XR.cols != X.cols || XR.ld != X.cols)
            return fail(QLIN_EINVAL, "xrot must be a contiguous [M, K] in x's dtype");
        xr = XR.data;
    }
    PrologueArgs p;
    p.mode = PROLOGUE_A8; p.x_dtype = X.dtype; p.x = X.data; p.ldx = X.ld; p.M = X.rows; p.K = (int)X.cols;
    p.G = convrot_groupsize; p.qo = (int8_t*)Qm.data; p.ldo = X.cols; p.so = (float*)scale->data; p.xr = xr;
    return hip_status(run_prologue(p, (hipStream_t)stream), "activation quantization");
}

}  // extern "C"
