// Eager entry points for PyTorch: the plain linears (no LoRA, no residual) called straight from
// Python with torch tensors.  Each builds the qlin_tensor descriptors, takes the output and the
// workspace from torch's allocator and calls the C ABI (include/qlin.h) on the current stream,
// so an eager call costs one Python -> C++ crossing instead of the descriptor packing and ctypes
// marshalling of qlin/_lib.py.  The argument rules and declines are those of qlin/ops.py, which
// runs every other call (LoRA, residual) through ctypes.
//
// Errors leave as QlinStatusError("<status>:<message>"); qlin/ops.py turns a status into
// NoCapableBackendError (QLIN_EUNSUPPORTED), ValueError (QLIN_EINVAL, QLIN_EWORKSPACE) or
// QlinError, exactly as for its ctypes calls.
#include <torch/extension.h>
#include <c10/hip/HIPStream.h>

#include <string>
#include <unordered_map>
#include <vector>

#include "qlin.h"

namespace {

struct StatusError : std::exception {
    std::string what_;
    StatusError(int status, const std::string& msg) : what_(std::to_string(status) + ":" + msg) {}
    const char* what() const noexcept override { return what_.c_str(); }
};

[[noreturn]] void fail(int status, const std::string& msg) { throw StatusError(status, msg); }

void check(qlin_status st) {
    if (st != QLIN_OK) fail(st, qlin_last_error());
}

int dtype_of(at::ScalarType t) {
    switch (t) {
        case at::kFloat: return QLIN_DT_F32;
        case at::kHalf: return QLIN_DT_F16;
        case at::kBFloat16: return QLIN_DT_BF16;
        case at::kChar: return QLIN_DT_I8;
        case at::kByte: return QLIN_DT_U8;
        case at::kInt: return QLIN_DT_I32;
        case at::kFloat8_e4m3fn: return QLIN_DT_E4M3;
        default: return -1;
    }
}

bool is_float(at::ScalarType t) { return t == at::kFloat || t == at::kHalf || t == at::kBFloat16; }

// A descriptor of t; dtype -1 keeps t's own.
qlin_tensor desc(const at::Tensor& t, int dtype = -1) {
    qlin_tensor d{};
    d.data = t.data_ptr();
    d.dtype = dtype >= 0 ? dtype : dtype_of(t.scalar_type());
    const int64_t nd = t.dim();
    if (nd == 0) {
        d.ndim = 1;
        d.shape[0] = 1;
        d.stride[0] = 1;
        return d;
    }
    if (nd > 4) fail(QLIN_EINVAL, "at most 4 dims");
    d.ndim = (int32_t)nd;
    for (int64_t i = 0; i < nd; ++i) {
        d.shape[i] = t.size(i);
        d.stride[i] = t.stride(i);
    }
    return d;
}

const qlin_tensor* opt(const c10::optional<at::Tensor>& t, qlin_tensor& d) {
    if (!t.has_value()) return nullptr;
    d = desc(*t);
    return &d;
}

void on_device(const char* op, const at::Tensor& t, int& dev) {
    if (!t.is_cuda())
        fail(QLIN_EUNSUPPORTED, std::string("tensor on ") + t.device().str() + ", the kernels need a ROCm device");
    const int d = t.get_device();
    if (dev < 0) dev = d;
    else if (d != dev)
        fail(QLIN_EINVAL, std::string(op) + ": tensors on different devices (cuda:" + std::to_string(dev) + ", cuda:" +
                              std::to_string(d) + ")");
}

// x as a 2-D operand [M, K] the kernels take: unit column stride, rows at least K apart, 16-byte
// aligned start (a copy otherwise); `lead` gets the leading shape.
at::Tensor as_2d(const at::Tensor& x, int64_t k, std::vector<int64_t>& lead) {
    if (x.dim() < 1 || x.size(-1) != k)
        fail(QLIN_EINVAL, "x has " + std::to_string(x.dim() ? x.size(-1) : 0) + " input features, the weight has " +
                              std::to_string(k));
    lead.assign(x.sizes().begin(), x.sizes().end() - 1);
    at::Tensor x2 = x.dim() == 2 ? x : x.reshape({-1, k});
    if (x2.size(0) > 1 && (x2.stride(1) != 1 || x2.stride(0) < k)) x2 = x2.contiguous();
    if (reinterpret_cast<uintptr_t>(x2.data_ptr()) % 16) x2 = x2.clone(at::MemoryFormat::Contiguous);
    return x2;
}

at::Tensor output(const at::Tensor& x2, int64_t n, const c10::optional<at::ScalarType>& out_dtype) {
    const at::ScalarType dt = out_dtype.value_or(x2.scalar_type());
    if (!is_float(dt)) fail(QLIN_EUNSUPPORTED, "out_dtype unsupported");
    return at::empty({x2.size(0), n}, x2.options().dtype(dt));
}

at::Tensor shaped(const at::Tensor& y, std::vector<int64_t>& lead, int64_t n) {
    if (lead.size() == 1) return y;
    lead.push_back(n);
    return y.view(lead);
}

c10::optional<at::Tensor> bias_1d(const c10::optional<at::Tensor>& bias, int64_t n) {
    if (!bias.has_value()) return bias;
    const at::Tensor& b = *bias;
    if (b.numel() != n)
        fail(QLIN_EINVAL, "bias has " + std::to_string(b.numel()) + " elements, expected " + std::to_string(n));
    if (b.dim() == 1 && b.is_contiguous()) return bias;
    return b.reshape({n}).contiguous();
}

// One workspace per (device, stream), grown on demand: calls on one stream run in order, so they
// can share it.  During HIP-graph capture every call takes its own buffer from the graph's pool
// (a cached buffer could be replaced after the capture while the graph still uses it).
struct WsKey {
    int dev;
    hipStream_t stream;
    bool operator==(const WsKey& o) const { return dev == o.dev && stream == o.stream; }
};
struct WsHash {
    size_t operator()(const WsKey& k) const { return std::hash<void*>()(k.stream) ^ (size_t)k.dev; }
};
std::unordered_map<WsKey, at::Tensor, WsHash>& ws_cache() {
    static std::unordered_map<WsKey, at::Tensor, WsHash> cache;
    return cache;
}

at::Tensor workspace_for(size_t nbytes, const at::Tensor& like, hipStream_t stream) {
    nbytes = nbytes ? nbytes : 1;
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(stream, &cap) != hipSuccess) fail(QLIN_EHIP, "hipStreamIsCapturing failed");
    const auto opts = like.options().dtype(at::kByte);
    if (cap != hipStreamCaptureStatusNone) return at::empty({(int64_t)nbytes}, opts);
    const WsKey key{(int)like.get_device(), stream};
    auto& cache = ws_cache();
    auto it = cache.find(key);
    if (it == cache.end() || (size_t)it->second.numel() < nbytes) {
        at::Tensor w = at::empty({(int64_t)std::max<size_t>(nbytes, 1u << 20)}, opts);
        cache[key] = w;
        return w;
    }
    return it->second;
}

hipStream_t current_stream(const at::Tensor& t) { return c10::hip::getCurrentHIPStream(t.get_device()).stream(); }

// (qk, block bytes) per ggml type id, given once by the Python package (its GGUF_TYPES table).
std::unordered_map<int64_t, std::pair<int64_t, int64_t>>& gguf_table() {
    static std::unordered_map<int64_t, std::pair<int64_t, int64_t>> t;
    return t;
}

void set_gguf_types(const std::unordered_map<int64_t, std::pair<int64_t, int64_t>>& types) { gguf_table() = types; }

at::Tensor gguf_linear(const at::Tensor& x, const at::Tensor& weight, int64_t tid, int64_t n, int64_t k,
                       const c10::optional<at::Tensor>& bias, const c10::optional<at::ScalarType>& out_dtype) {
    int dev = -1;
    on_device("gguf_linear", x, dev);
    on_device("gguf_linear", weight, dev);
    if (bias.has_value()) on_device("gguf_linear", *bias, dev);
    const auto it = gguf_table().find(tid);
    if (it == gguf_table().end()) fail(QLIN_EUNSUPPORTED, "ggml type " + std::to_string(tid) + " unsupported");
    if (weight.scalar_type() != at::kByte) fail(QLIN_EUNSUPPORTED, "weight must be the uint8 block bytes");
    if (!weight.is_contiguous()) fail(QLIN_EUNSUPPORTED, "weight bytes must be contiguous");
    const int64_t qk = it->second.first, ts = it->second.second;
    if (k % qk || weight.numel() != n * (k / qk) * ts)
        fail(QLIN_EINVAL, "weight has " + std::to_string(weight.numel()) + " bytes, expected " +
                              std::to_string(n * (k / qk) * ts) + " for (" + std::to_string(n) + ", " + std::to_string(k) +
                              ")");
    if (!is_float(x.scalar_type())) fail(QLIN_EUNSUPPORTED, "x dtype unsupported");
    std::vector<int64_t> lead;
    const at::Tensor x2 = as_2d(x, k, lead);
    at::Tensor y = output(x2, n, out_dtype);
    if (x2.size(0) == 0 || n == 0) return shaped(y, lead, n);
    const auto b = bias_1d(bias, n);
    const hipStream_t st = current_stream(x2);
    const at::Tensor ws = workspace_for(
        qlin_workspace_size(QLIN_OP_GGUF_LINEAR, x2.size(0), n, k, (int)tid, dtype_of(x2.scalar_type())), x2, st);
    qlin_tensor dx = desc(x2), dy = desc(y), db;
    check(qlin_gguf_linear(&dx, weight.data_ptr(), (int)tid, n, k, opt(b, db), &dy, ws.data_ptr(), (size_t)ws.numel(), st));
    return shaped(y, lead, n);
}

at::Tensor int8_linear(const at::Tensor& x, const at::Tensor& qdata, const at::Tensor& scale,
                       const c10::optional<at::Tensor>& bias, const c10::optional<at::ScalarType>& out_dtype,
                       int64_t convrot_groupsize) {
    int dev = -1;
    on_device("int8_linear", x, dev);
    on_device("int8_linear", qdata, dev);
    on_device("int8_linear", scale, dev);
    if (bias.has_value()) on_device("int8_linear", *bias, dev);
    if (qdata.scalar_type() != at::kChar || qdata.dim() != 2) fail(QLIN_EUNSUPPORTED, "qdata must be a 2-D int8 tensor");
    if (!is_float(x.scalar_type())) fail(QLIN_EUNSUPPORTED, "x dtype unsupported");
    const int64_t n = qdata.size(0), k = qdata.size(1);
    std::vector<int64_t> lead;
    const at::Tensor x2 = as_2d(x, k, lead);
    at::Tensor y = output(x2, n, out_dtype);
    if (x2.size(0) == 0 || n == 0) return shaped(y, lead, n);
    const at::Tensor s = (scale.dim() == 1 || (scale.numel() != 1 && scale.numel() != n)) ? scale : scale.reshape({-1});
    const auto b = bias_1d(bias, n);
    const hipStream_t st = current_stream(x2);
    const at::Tensor ws = workspace_for(qlin_workspace_size(QLIN_OP_INT8_LINEAR, x2.size(0), n, k, (int)convrot_groupsize,
                                                            dtype_of(x2.scalar_type())),
                                        x2, st);
    qlin_tensor dx = desc(x2), dq = desc(qdata), ds = desc(s), dy = desc(y), db;
    check(qlin_int8_linear(&dx, &dq, &ds, opt(b, db), &dy, (int)convrot_groupsize, ws.data_ptr(), (size_t)ws.numel(), st));
    return shaped(y, lead, n);
}

at::Tensor f32_1d(const at::Tensor& t) {
    if (t.dim() == 1 && t.scalar_type() == at::kFloat && t.is_contiguous()) return t;
    return t.reshape({-1}).to(at::kFloat).contiguous();
}

at::Tensor w4a8_int8_linear(const at::Tensor& x, const at::Tensor& qdata, const at::Tensor& s_rel,
                            const at::Tensor& s_channel, const c10::optional<at::Tensor>& codebook,
                            const c10::optional<at::Tensor>& bias, int64_t group_size, int64_t convrot_groupsize,
                            const c10::optional<at::ScalarType>& out_dtype) {
    int dev = -1;
    for (const at::Tensor* t : {&x, &qdata, &s_rel, &s_channel}) on_device("w4a8_int8_linear", *t, dev);
    if (codebook.has_value()) on_device("w4a8_int8_linear", *codebook, dev);
    if (bias.has_value()) on_device("w4a8_int8_linear", *bias, dev);
    if (!is_float(x.scalar_type())) fail(QLIN_EUNSUPPORTED, "x dtype unsupported");
    if (qdata.dim() != 2 || s_rel.dim() != 2) fail(QLIN_EINVAL, "qdata and s_rel must be 2-D");
    const int64_t k = s_rel.size(1) * group_size;
    const int64_t bits = k ? (qdata.size(1) * 8) / k : 0;
    if ((bits != 4 && bits != 6) || qdata.size(1) * 8 != bits * k)
        fail(QLIN_EINVAL, "qdata [" + std::to_string(qdata.size(0)) + ", " + std::to_string(qdata.size(1)) +
                              "] does not hold 4- or 6-bit codes for K=" + std::to_string(k));
    const int64_t n = qdata.size(0);
    int srdt;
    switch (s_rel.scalar_type()) {
        case at::kFloat8_e4m3fn: srdt = QLIN_DT_E4M3; break;
        case at::kHalf: case at::kBFloat16: case at::kFloat: srdt = dtype_of(s_rel.scalar_type()); break;
        default: fail(QLIN_EUNSUPPORTED, "s_rel dtype unsupported");
    }
    std::vector<int64_t> lead;
    const at::Tensor x2 = as_2d(x, k, lead);
    at::Tensor y = output(x2, n, out_dtype);
    if (x2.size(0) == 0 || n == 0) return shaped(y, lead, n);
    const at::Tensor q = (qdata.scalar_type() == at::kChar || qdata.scalar_type() == at::kByte) ? qdata : qdata.view(at::kChar);
    c10::optional<at::Tensor> cb;
    if (codebook.has_value()) cb = f32_1d(*codebook);
    const at::Tensor sch = f32_1d(s_channel);
    const auto b = bias_1d(bias, n);
    const hipStream_t st = current_stream(x2);
    const at::Tensor ws = workspace_for(qlin_workspace_size(QLIN_OP_W4A8_LINEAR, x2.size(0), n, k,
                                                            (int)(bits | group_size << 8), dtype_of(x2.scalar_type())),
                                        x2, st);
    qlin_tensor dx = desc(x2), dq = desc(q), dsr = desc(s_rel, srdt), dsc = desc(sch), dy = desc(y), dcb, db;
    check(qlin_w4a8_linear(&dx, &dq, &dsr, &dsc, opt(cb, dcb), opt(b, db), &dy, (int)bits, (int)group_size,
                           (int)convrot_groupsize, ws.data_ptr(), (size_t)ws.numel(), st));
    return shaped(y, lead, n);
}

// The cached workspace for (device of `like`, current stream), at least nbytes (for the ctypes
// calls of qlin/ops.py, so that both routes share one buffer per stream).
at::Tensor workspace(int64_t nbytes, const at::Tensor& like) {
    return workspace_for((size_t)std::max<int64_t>(nbytes, 1), like, current_stream(like));
}

void release_workspaces() { ws_cache().clear(); }

}  // namespace

PYBIND11_MODULE(TORCH_EXTENSION_NAME, m) {
    static pybind11::exception<StatusError> status_error(m, "QlinStatusError", PyExc_RuntimeError);
    pybind11::register_exception_translator([](std::exception_ptr p) {
        try {
            if (p) std::rethrow_exception(p);
        } catch (const StatusError& e) {
            status_error(e.what());
        }
    });
    m.def("set_gguf_types", &set_gguf_types);
    m.def("gguf_linear", &gguf_linear);
    m.def("int8_linear", &int8_linear);
    m.def("w4a8_int8_linear", &w4a8_int8_linear);
    m.def("workspace", &workspace);
    m.def("release_workspaces", &release_workspaces);
}
