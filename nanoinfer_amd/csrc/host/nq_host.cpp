// C++ host API over libnq_hip.so: reference-shaped tensors, weights and the
// backend factory (declared in nq_host.hpp).
#include "nq_host.hpp"

#include <hip/hip_runtime_api.h>

#include <algorithm>
#include <cstring>
#include <stdexcept>
#include <string>
#include <unordered_map>

#include "../../../include/nq.h"

namespace ni {
namespace hip {

namespace {

thread_local void* g_stream = nullptr;

void require(bool cond, const char* msg) {
    if (!cond) throw std::invalid_argument(msg);
}

void hip_check(hipError_t e, const char* what) {
    if (e != hipSuccess) throw std::runtime_error(std::string(what) + ": " + hipGetErrorString(e));
}

// A non-OK status becomes the exception the reference throws at that point.
void nq_check(nq_status st) {
    if (st == NQ_OK) return;
    const std::string msg = std::string(nq_status_name(st)) + ": " + nq_last_error();
    if (st == NQ_HIP_ERROR || st == NQ_IO_ERROR) throw std::runtime_error(msg);
    throw std::invalid_argument(msg);
}

std::shared_ptr<void> device_alloc(size_t bytes) {
    void* p = nullptr;
    if (bytes > 0) hip_check(hipMalloc(&p, bytes), "hipMalloc");
    return std::shared_ptr<void>(p, [](void* q) {
        if (q) (void)hipFree(q);
    });
}

nq_dtype abi_dtype(DType d) {
    require(d == DType::F32 || d == DType::F16, "activation dtype must be F32 or F16");
    return d == DType::F32 ? NQ_F32 : NQ_F16;
}

// Grow-only device workspace per (thread, device) for the W8A8 and split-K
// weight-only entry points.
struct Workspace {
    std::shared_ptr<void> buf;
    size_t bytes = 0;
};
thread_local std::unordered_map<int, Workspace> g_ws;

void* workspace(size_t bytes) {
    int dev = 0;
    hip_check(hipGetDevice(&dev), "hipGetDevice");
    Workspace& w = g_ws[dev];
    if (w.bytes < bytes) {
        // The old buffer may still be read by queued work on this stream.
        hip_check(hipStreamSynchronize(static_cast<hipStream_t>(g_stream)), "hipStreamSynchronize");
        w.buf = device_alloc(bytes);
        w.bytes = bytes;
    }
    return w.buf.get();
}

void check_device_2d(const Tensor& t, const char* msg) {
    require(t.on_device() && t.ndim() == 2, msg);
}

}  // namespace

const char* format_name(Format f) {
    switch (f) {
        case Format::F32: return "f32";
        case Format::F16: return "f16";
        case Format::BF16: return "bf16";
        case Format::Q8: return "q8";
        case Format::Q4: return "q4";
        case Format::Q4G: return "q4g";
        case Format::W8A8: return "w8a8";
    }
    return "?";
}

QuantMode quant_mode(const std::string& s) {
    if (s == "fp32" || s == "none") return QuantMode::None;
    if (s == "q8") return QuantMode::Q8;
    if (s == "q4") return QuantMode::Q4;
    if (s == "q4g") return QuantMode::Q4G;
    if (s == "w8a8") return QuantMode::W8A8;
    throw std::invalid_argument("unknown quant mode '" + s + "' (fp32|q8|q4|q4g|w8a8)");
}

size_t dtype_bytes(DType d) {
    switch (d) {
        case DType::F32: return 4;
        case DType::F16: return 2;
        case DType::I8: return 1;
        case DType::U8: return 1;
        case DType::I32: return 4;
    }
    return 4;
}

void set_stream(void* s) { g_stream = s; }
void* current_stream() { return g_stream; }

static int64_t product(const std::vector<int64_t>& shape) {
    int64_t n = 1;
    for (int64_t d : shape) {
        require(d >= 0, "negative tensor dimension");
        n *= d;
    }
    return n;
}

Tensor::Tensor(std::vector<int64_t> shape) : shape_(std::move(shape)) {
    numel_ = product(shape_);
    host_.assign(static_cast<size_t>(numel_), 0.0f);
}

Tensor::Tensor(std::vector<int64_t> shape, DType dtype, Device device)
    : shape_(std::move(shape)), dtype_(dtype), device_(device) {
    numel_ = product(shape_);
    if (device_ == Device::CPU) {
        require(dtype_ == DType::F32, "host tensors are fp32");
        host_.assign(static_cast<size_t>(numel_), 0.0f);
    } else {
        dev_ = device_alloc(nbytes());
    }
}

Tensor Tensor::rows(int64_t begin, int64_t count) const {
    require(on_device() && ndim() >= 1 && begin >= 0 && count >= 0 && begin + count <= size(0),
            "Tensor::rows: a row range of a device tensor");
    Tensor t;
    t.shape_ = shape_;
    t.shape_[0] = count;
    t.numel_ = product(t.shape_);
    t.dtype_ = dtype_;
    t.device_ = device_;
    const size_t row_bytes = size(0) ? nbytes() / static_cast<size_t>(size(0)) : 0;
    t.dev_ = std::shared_ptr<void>(dev_, static_cast<char*>(dev_.get()) + static_cast<size_t>(begin) * row_bytes);
    return t;
}

HipPolicy& hip_policy() {
    static HipPolicy p;
    return p;
}

Tensor to_device(const Tensor& host, DType dtype) {
    require(!host.on_device(), "to_device expects a host tensor");
    Tensor d(host.shape(), dtype, Device::HIP);
    hipStream_t s = static_cast<hipStream_t>(g_stream);
    if (d.numel() == 0) return d;
    if (dtype == DType::F32) {
        hip_check(hipMemcpyAsync(d.device_ptr(), host.data(), d.nbytes(), hipMemcpyHostToDevice, s), "H2D");
    } else if (dtype == DType::F16) {
        std::vector<_Float16> h(static_cast<size_t>(host.numel()));
        for (size_t i = 0; i < h.size(); ++i) h[i] = static_cast<_Float16>(host[static_cast<int64_t>(i)]);
        hip_check(hipMemcpyAsync(d.device_ptr(), h.data(), d.nbytes(), hipMemcpyHostToDevice, s), "H2D");
    } else {
        throw std::invalid_argument("to_device: only F32 / F16 from host fp32");
    }
    hip_check(hipStreamSynchronize(s), "hipStreamSynchronize");  // the staging buffer dies here
    return d;
}

Tensor to_host(const Tensor& dev) {
    require(dev.on_device(), "to_host expects a device tensor");
    Tensor h(dev.shape());
    hipStream_t s = static_cast<hipStream_t>(g_stream);
    hip_check(hipStreamSynchronize(s), "hipStreamSynchronize");
    if (dev.numel() == 0) return h;
    const size_t n = static_cast<size_t>(dev.numel());
    switch (dev.dtype()) {
        case DType::F32:
            hip_check(hipMemcpy(h.data(), dev.device_ptr(), dev.nbytes(), hipMemcpyDeviceToHost), "D2H");
            break;
        case DType::F16: {
            std::vector<_Float16> t(n);
            hip_check(hipMemcpy(t.data(), dev.device_ptr(), dev.nbytes(), hipMemcpyDeviceToHost), "D2H");
            for (size_t i = 0; i < n; ++i) h.data()[i] = static_cast<float>(t[i]);
            break;
        }
        case DType::I8: {
            std::vector<int8_t> t(n);
            hip_check(hipMemcpy(t.data(), dev.device_ptr(), n, hipMemcpyDeviceToHost), "D2H");
            for (size_t i = 0; i < n; ++i) h.data()[i] = static_cast<float>(t[i]);
            break;
        }
        case DType::U8: {
            std::vector<uint8_t> t(n);
            hip_check(hipMemcpy(t.data(), dev.device_ptr(), n, hipMemcpyDeviceToHost), "D2H");
            for (size_t i = 0; i < n; ++i) h.data()[i] = static_cast<float>(t[i]);
            break;
        }
        case DType::I32: {
            std::vector<int32_t> t(n);
            hip_check(hipMemcpy(t.data(), dev.device_ptr(), dev.nbytes(), hipMemcpyDeviceToHost), "D2H");
            for (size_t i = 0; i < n; ++i) h.data()[i] = static_cast<float>(t[i]);
            break;
        }
    }
    return h;
}

// Weights arrive as host fp32 (the reference's load path) or device fp32.
static Tensor device_f32(const Tensor& w) {
    if (w.on_device()) {
        require(w.dtype() == DType::F32, "weights must be fp32");
        return w;
    }
    return to_device(w, DType::F32);
}

QTensor quantize_q8(const Tensor& w) {
    require(w.ndim() == 2, "quantize_q8 expects a 2-D [out, in] weight");
    const Tensor wd = device_f32(w);
    QTensor t;
    t.out = w.size(0);
    t.in = w.size(1);
    t.q = Tensor({t.out, t.in}, DType::I8, Device::HIP);
    t.scale = Tensor({t.out}, DType::F32, Device::HIP);
    nq_check(nq_quantize_q8(static_cast<const float*>(wd.device_ptr()), t.out, t.in,
                            static_cast<int8_t*>(t.q.device_ptr()), static_cast<float*>(t.scale.device_ptr()),
                            g_stream));
    if (!w.on_device()) hip_check(hipStreamSynchronize(static_cast<hipStream_t>(g_stream)), "sync");
    return t;
}

Q4GTensor quantize_q4g(const Tensor& w, int64_t group, DType scale_dtype) {
    require(w.ndim() == 2, "quantize_q4g expects a 2-D [out, in] weight");
    require(group > 0, "quantize_q4g: group must be positive");
    const Tensor wd = device_f32(w);
    Q4GTensor t;
    t.out = w.size(0);
    t.in = w.size(1);
    t.group = group;
    t.q = Tensor({t.out, (t.in + 1) / 2}, DType::U8, Device::HIP);
    t.scale = Tensor({t.out, (t.in + group - 1) / group}, scale_dtype, Device::HIP);
    nq_check(nq_quantize_q4g(static_cast<const float*>(wd.device_ptr()), t.out, t.in, group,
                             static_cast<uint8_t*>(t.q.device_ptr()), t.scale.device_ptr(),
                             abi_dtype(scale_dtype), g_stream));
    if (!w.on_device()) hip_check(hipStreamSynchronize(static_cast<hipStream_t>(g_stream)), "sync");
    return t;
}

Q4GTensor quantize_q4(const Tensor& w) {
    require(w.ndim() == 2, "quantize_q4 expects a 2-D [out, in] weight");
    return quantize_q4g(w, std::max<int64_t>(1, w.size(1)));
}

static const float* bias_ptr(const Tensor* bias, int64_t out, const char* who) {
    if (!bias) return nullptr;
    require(bias->on_device() && bias->dtype() == DType::F32, who);
    require(bias->numel() == out, "bias must match out-features");
    return static_cast<const float*>(bias->device_ptr());
}

namespace {
Tensor linear_q8_path(const Tensor& x, const QTensor& w, const Tensor* bias, DType out_dtype, int path) {
    check_device_2d(x, "linear_q8 expects 2-D device x");
    require(x.size(1) == w.in, "linear_q8: x cols must match weight in-features");
    const float* b = bias_ptr(bias, w.out, "linear_q8: bias must be a device fp32 tensor");
    Tensor y({x.size(0), w.out}, out_dtype, Device::HIP);
    const size_t need = nq_linear_wq_workspace_size(x.size(0), w.out, w.in);
    void* ws = need ? workspace(need) : nullptr;
    nq_check(nq_linear_q8_ex(x.device_ptr(), abi_dtype(x.dtype()), static_cast<const int8_t*>(w.q.device_ptr()),
                             static_cast<const float*>(w.scale.device_ptr()), b, y.device_ptr(),
                             abi_dtype(out_dtype), x.size(0), w.out, w.in, ws, need, path, g_stream));
    return y;
}
}  // namespace

Tensor linear_q8(const Tensor& x, const QTensor& w, const Tensor* bias, DType out_dtype) {
    return linear_q8_path(x, w, bias, out_dtype, NQ_PATH_AUTO);
}

Tensor linear_w8a8(const Tensor& x, const QTensor& w, const Tensor* bias, DType out_dtype) {
    check_device_2d(x, "linear_w8a8 expects 2-D device x");
    require(x.size(1) == w.in, "linear_w8a8: x cols must match weight in-features");
    const float* b = bias_ptr(bias, w.out, "linear_w8a8: bias must be a device fp32 tensor");
    Tensor y({x.size(0), w.out}, out_dtype, Device::HIP);
    const size_t need = nq_linear_w8a8_workspace_size(x.size(0), w.out, w.in);
    void* ws = need ? workspace(need) : nullptr;
    nq_check(nq_linear_w8a8(x.device_ptr(), abi_dtype(x.dtype()), static_cast<const int8_t*>(w.q.device_ptr()),
                            static_cast<const float*>(w.scale.device_ptr()), b, y.device_ptr(),
                            abi_dtype(out_dtype), x.size(0), w.out, w.in, ws, need, NQ_PATH_AUTO, g_stream));
    return y;
}

Tensor linear_q4g(const Tensor& x, const Q4GTensor& w, const Tensor* bias, DType out_dtype) {
    check_device_2d(x, "linear_q4g expects 2-D device x");
    require(x.size(1) == w.in, "linear_q4g: x cols must match weight in-features");
    const float* b = bias_ptr(bias, w.out, "linear_q4g: bias must be a device fp32 tensor");
    Tensor y({x.size(0), w.out}, out_dtype, Device::HIP);
    const size_t need = nq_linear_wq_workspace_size(x.size(0), w.out, w.in);
    void* ws = need ? workspace(need) : nullptr;
    nq_check(nq_linear_q4g_ws(x.device_ptr(), abi_dtype(x.dtype()), static_cast<const uint8_t*>(w.q.device_ptr()),
                              w.scale.device_ptr(), abi_dtype(w.scale.dtype()), w.group, b, y.device_ptr(),
                              abi_dtype(out_dtype), x.size(0), w.out, w.in, ws, need, g_stream));
    return y;
}

Tensor linear_q8(const Tensor& x, const QTensor& w, const Tensor* bias) { return linear_q8(x, w, bias, x.dtype()); }
Tensor linear_w8a8(const Tensor& x, const QTensor& w, const Tensor* bias) { return linear_w8a8(x, w, bias, x.dtype()); }
Tensor linear_q4g(const Tensor& x, const Q4GTensor& w, const Tensor* bias) { return linear_q4g(x, w, bias, x.dtype()); }

Tensor embedding_q8(const QTensor& table, const std::vector<int64_t>& ids) {
    Tensor out({static_cast<int64_t>(ids.size()), table.in}, DType::F32, Device::HIP);
    nq_check(nq_embedding_q8(static_cast<const int8_t*>(table.q.device_ptr()),
                             static_cast<const float*>(table.scale.device_ptr()), table.out, table.in, ids.data(),
                             static_cast<int64_t>(ids.size()), out.device_ptr(), NQ_F32, g_stream));
    return out;
}

Tensor Weight::gather(const std::vector<int64_t>&) const {
    throw std::runtime_error("Weight::gather: this weight is not an embedding table");  // quant.cpp:473-475
}

namespace {

int64_t q_bytes(const Tensor& q, const Tensor& scale) {
    return static_cast<int64_t>(q.nbytes() + scale.nbytes());
}

class HipQ8Weight : public Weight {
protected:
    QTensor t_;

public:
    explicit HipQ8Weight(QTensor t) : t_(std::move(t)) {}
    Tensor linear(const Tensor& x, const Tensor* bias) const override { return linear_q8(x, t_, bias); }
    Format format() const override { return Format::Q8; }
    int64_t bytes() const override { return q_bytes(t_.q, t_.scale); }
    int64_t fp32_bytes() const override { return t_.out * t_.in * 4; }
};

class HipW8A8Weight : public HipQ8Weight {
public:
    using HipQ8Weight::HipQ8Weight;
    Tensor linear(const Tensor& x, const Tensor* bias) const override { return linear_w8a8(x, t_, bias); }
    Format format() const override { return Format::W8A8; }
};

// The int8 embedding / LM head (CudaEmbedQ8Weight, cuda_quant.cu:350-379):
// linear() follows hip_policy() as the reference's follows cuda_policy().
class HipEmbedQ8Weight : public HipQ8Weight {
public:
    using HipQ8Weight::HipQ8Weight;
    Tensor linear(const Tensor& x, const Tensor* bias) const override {
        const HipPolicy& pol = hip_policy();
        if (pol.use_w8a8_lmhead && x.ndim() == 2 && x.size(0) > kGemvMaxM) return linear_w8a8(x, t_, bias);
        return linear_q8_path(x, t_, bias, x.dtype(), pol.force_tiled_q8 ? NQ_PATH_MFMA : NQ_PATH_AUTO);
    }
    Tensor gather(const std::vector<int64_t>& ids) const override { return embedding_q8(t_, ids); }
    const QTensor& codes() const { return t_; }
};

class HipQ4GWeight : public Weight {
    Q4GTensor t_;
    Format fmt_;

public:
    HipQ4GWeight(Q4GTensor t, Format f) : t_(std::move(t)), fmt_(f) {}
    Tensor linear(const Tensor& x, const Tensor* bias) const override { return linear_q4g(x, t_, bias); }
    Format format() const override { return fmt_; }
    int64_t bytes() const override { return q_bytes(t_.q, t_.scale); }
    int64_t fp32_bytes() const override { return t_.out * t_.in * 4; }
};

}  // namespace

std::unique_ptr<Weight> make_quantized(const Tensor& w, QuantMode mode) {
    switch (mode) {
        case QuantMode::Q8: return std::make_unique<HipQ8Weight>(quantize_q8(w));
        case QuantMode::Q4: return std::make_unique<HipQ4GWeight>(quantize_q4(w), Format::Q4);
        case QuantMode::Q4G: return std::make_unique<HipQ4GWeight>(quantize_q4g(w, 32), Format::Q4G);
        case QuantMode::W8A8: return std::make_unique<HipW8A8Weight>(quantize_q8(w));
        case QuantMode::None: return nullptr;
    }
    return nullptr;
}

std::unique_ptr<Weight> make_q8_embed(const Tensor& w) { return std::make_unique<HipEmbedQ8Weight>(quantize_q8(w)); }

Tensor load_bin(const std::string& path) {
    int32_t dt = 0, nd = 0;
    int64_t shape[8] = {};
    nq_check(nq_nit_info(path.c_str(), &dt, &nd, shape, 8));
    Tensor t(std::vector<int64_t>(shape, shape + nd), DType::F32, Device::HIP);
    nq_check(nq_nit_load_f32(path.c_str(), static_cast<float*>(t.device_ptr()), t.numel(), g_stream));
    return t;
}

std::unique_ptr<Weight> load_quantized(const std::string& path, QuantMode mode) {
    int32_t dt = 0, nd = 0;
    int64_t shape[8] = {};
    nq_check(nq_nit_info(path.c_str(), &dt, &nd, shape, 8));
    require(nd == 2, "load_quantized expects a 2-D [out, in] weight file");
    const int64_t out = shape[0], in = shape[1];
    if (mode == QuantMode::None) return nullptr;
    if (mode == QuantMode::Q8 || mode == QuantMode::W8A8) {
        QTensor t;
        t.out = out;
        t.in = in;
        t.q = Tensor({out, in}, DType::I8, Device::HIP);
        t.scale = Tensor({out}, DType::F32, Device::HIP);
        nq_check(nq_nit_load_q8(path.c_str(), static_cast<int8_t*>(t.q.device_ptr()),
                                static_cast<float*>(t.scale.device_ptr()), out, in, g_stream));
        if (mode == QuantMode::Q8) return std::make_unique<HipQ8Weight>(std::move(t));
        return std::make_unique<HipW8A8Weight>(std::move(t));
    }
    const int64_t group = mode == QuantMode::Q4 ? std::max<int64_t>(1, in) : 32;
    Q4GTensor t;
    t.out = out;
    t.in = in;
    t.group = group;
    t.q = Tensor({out, (in + 1) / 2}, DType::U8, Device::HIP);
    t.scale = Tensor({out, (in + group - 1) / group}, DType::F32, Device::HIP);
    nq_check(nq_nit_load_q4g(path.c_str(), static_cast<uint8_t*>(t.q.device_ptr()), t.scale.device_ptr(), NQ_F32,
                             group, out, in, g_stream));
    return std::make_unique<HipQ4GWeight>(std::move(t), mode == QuantMode::Q4 ? Format::Q4 : Format::Q4G);
}

std::vector<int64_t> lm_head_argmax(const Tensor& x, const QTensor& head, const Tensor* bias) {
    check_device_2d(x, "lm_head_argmax expects a device [m, in] activation");
    require(x.size(1) == head.in, "lm_head_argmax: x cols must match weight in-features");
    const int64_t m = x.size(0);
    Tensor ids64({2 * m}, DType::I32, Device::HIP);  // int64 ids, held as pairs of int32
    const size_t wsb = nq_lm_head_argmax_q8_workspace_size(m, head.out, head.in);
    Tensor ws({static_cast<int64_t>((wsb + 3) / 4 + 64)}, DType::I32, Device::HIP);
    nq_check(nq_lm_head_argmax_q8(x.device_ptr(), x.dtype() == DType::F16 ? NQ_F16 : NQ_F32,
                                  static_cast<const int8_t*>(head.q.device_ptr()),
                                  static_cast<const float*>(head.scale.device_ptr()),
                                  bias ? static_cast<const float*>(bias->device_ptr()) : nullptr,
                                  static_cast<int64_t*>(ids64.device_ptr()), m, head.out, head.in,
                                  ws.device_ptr(), ws.nbytes(), g_stream));
    std::vector<int64_t> out(static_cast<size_t>(m));
    hip_check(hipMemcpyAsync(out.data(), ids64.device_ptr(), out.size() * sizeof(int64_t), hipMemcpyDeviceToHost,
                             static_cast<hipStream_t>(g_stream)),
              "hipMemcpyAsync");
    hip_check(hipStreamSynchronize(static_cast<hipStream_t>(g_stream)), "hipStreamSynchronize");
    return out;
}

std::vector<int64_t> lm_head_argmax(const Tensor& x, const Weight& head, const Tensor* bias) {
    const auto* e = dynamic_cast<const HipEmbedQ8Weight*>(&head);
    require(e != nullptr, "lm_head_argmax: the head must be an int8 embedding weight (make_q8_embed)");
    return lm_head_argmax(x, e->codes(), bias);
}

std::unique_ptr<Weight> HipBackend::make_quant_weight(const Tensor& host, QuantMode mode) const {
    return make_quantized(host, mode);
}

std::unique_ptr<Weight> HipBackend::make_embed_weight(const Tensor& host) const { return make_q8_embed(host); }

}  // namespace hip
}  // namespace ni
