// C++ host API of the MI355X quantized-weight path: the reference's nicore quant
// interface (cpp/src/quant.hpp:32-141, cpp/src/backend.hpp:104-114) restated over
// libnq_hip.so's C ABI, in namespace ni::hip (the reference's names, one level
// down, so both can link into one program).
//
// Same names, argument meaning and error behaviour as the reference:
//   quantize_q8 / quantize_q4g / quantize_q4      (quant.hpp:57, :97, :114)
//   linear_q8 / linear_w8a8 / linear_q4g          (quant.hpp:64, :80, :116)
//   embedding_q8                                  (quant.hpp:72)
//   Weight, make_quantized, make_q8_embed         (quant.hpp:120-141)
//   HipBackend::make_quant_weight / make_embed_weight (backend.hpp:109-114)
//   load_bin (serialize.hpp:32), argmax of the LM head (sampling.cpp:14-20)
// Shape and argument errors throw std::invalid_argument, device errors throw
// std::runtime_error (quant.cpp:23-25, cuda_internal.cuh:24).
//
// Tensors live on the host (fp32, as the reference's Tensor) or on the GPU
// (fp32 / fp16 / int8 / uint8 / int32 device buffers). Quantized weights are
// always device-resident: unlike the reference CUDA backend, which uploads only
// W8A8 and leaves Q8/Q4/Q4G on the host (cuda_quant.cu:390-395), every mode here
// quantizes on the GPU and runs its linear there. Device ops are enqueued on the
// calling thread's current stream and return without synchronizing; to_host()
// synchronizes that stream.
#pragma once

#include <cstdint>
#include <memory>
#include <string>
#include <utility>
#include <vector>

namespace ni {
namespace hip {

enum class QuantMode { None, Q8, Q4, Q4G, W8A8 };       // quant.hpp:32
enum class Format { F32, F16, BF16, Q8, Q4, Q4G, W8A8 };  // quant.hpp:41
enum class DType { F32, F16, I8, U8, I32 };
enum class Device { CPU, HIP };

const char* format_name(Format f);     // quant.cpp:447-458
QuantMode quant_mode(const std::string& name);  // nicpp.cpp:51-59
size_t dtype_bytes(DType d);

// The calling thread's stream for every device op (nullptr = the null stream).
void set_stream(void* hip_stream);
void* current_stream();

// A row-major tensor: a host fp32 vector, or a device buffer of `dtype`.
class Tensor {
public:
    Tensor() = default;
    explicit Tensor(std::vector<int64_t> shape);                    // host fp32, zero-filled
    Tensor(std::vector<int64_t> shape, DType dtype, Device device);  // device: uninitialised

    const std::vector<int64_t>& shape() const { return shape_; }
    int64_t ndim() const { return static_cast<int64_t>(shape_.size()); }
    int64_t size(int64_t d) const { return shape_.at(static_cast<size_t>(d)); }
    int64_t numel() const { return numel_; }
    DType dtype() const { return dtype_; }
    Device device() const { return device_; }
    bool on_device() const { return device_ == Device::HIP; }

    float* data() { return host_.data(); }               // host fp32 only
    const float* data() const { return host_.data(); }
    float& operator[](int64_t i) { return host_[static_cast<size_t>(i)]; }
    float operator[](int64_t i) const { return host_[static_cast<size_t>(i)]; }

    void* device_ptr() const { return dev_.get(); }     // device only
    // Rows [begin, begin + count) of a device tensor as a tensor sharing its
    // buffer (the first dimension narrowed).
    Tensor rows(int64_t begin, int64_t count) const;
    size_t nbytes() const { return static_cast<size_t>(numel_) * dtype_bytes(dtype_); }

private:
    std::vector<int64_t> shape_;
    int64_t numel_ = 0;
    DType dtype_ = DType::F32;
    Device device_ = Device::CPU;
    std::vector<float> host_;
    std::shared_ptr<void> dev_;
};

Tensor to_device(const Tensor& host, DType dtype = DType::F32);  // fp32 host -> device (fp32 / fp16)
Tensor to_host(const Tensor& dev);                               // device -> host fp32 (synchronizes)

// An int8-quantized [out, in] weight on the device (quant.hpp:49-54).
struct QTensor {
    Tensor q;      // I8 [out, in]
    Tensor scale;  // F32 [out]
    int64_t out = 0, in = 0;
};

// Group-wise int4 [out, in] on the device (quant.hpp:105-111); scale is fp32
// (the reference layout) or fp16 (storage variant), [out, ceil(in / group)].
struct Q4GTensor {
    Tensor q;      // U8 [out, ceil(in / 2)]
    Tensor scale;  // F32 or F16 [out, ceil(in / group)]
    int64_t out = 0, in = 0, group = 0;
};

QTensor quantize_q8(const Tensor& w);
Q4GTensor quantize_q4g(const Tensor& w, int64_t group = 32, DType scale_dtype = DType::F32);
Q4GTensor quantize_q4(const Tensor& w);  // group == in (quant.cpp:212-233)

// x: device [m, in] (fp32 or fp16); returns device [m, out] of out_dtype
// (default: x's dtype). bias: device fp32 [out] or nullptr.
Tensor linear_q8(const Tensor& x, const QTensor& w, const Tensor* bias = nullptr);
Tensor linear_w8a8(const Tensor& x, const QTensor& w, const Tensor* bias = nullptr);
Tensor linear_q4g(const Tensor& x, const Q4GTensor& w, const Tensor* bias = nullptr);
Tensor linear_q8(const Tensor& x, const QTensor& w, const Tensor* bias, DType out_dtype);
Tensor linear_w8a8(const Tensor& x, const QTensor& w, const Tensor* bias, DType out_dtype);
Tensor linear_q4g(const Tensor& x, const Q4GTensor& w, const Tensor* bias, DType out_dtype);
Tensor embedding_q8(const QTensor& table, const std::vector<int64_t>& ids);

// Kernel selection of the int8 embedding / LM-head weight: the two fields of the
// reference's CudaPolicy (cuda_backend.hpp:43-89) that reach the quantized path.
// use_w8a8_lmhead: its linear at m > kGemvMaxM (prefill) runs as W8A8 on the same
// int8 codes (cuda_quant.cu:362-372); opt-in, since the activation quant can flip
// a close greedy token. force_tiled_q8: its weight-only linear runs the MFMA GEMM
// at any m (cuda_quant.cu:308), for A/B runs. Process-wide and mutable, as
// cuda_policy(); not to be flipped while another thread runs a linear.
struct HipPolicy {
    bool use_w8a8_lmhead = false;
    bool force_tiled_q8 = false;
};
HipPolicy& hip_policy();
constexpr int64_t kGemvMaxM = 8;  // the decode GEMVs' activation batch

// Polymorphic device weight (quant.hpp:120-133).
class Weight {
public:
    virtual ~Weight() = default;
    virtual Tensor linear(const Tensor& x, const Tensor* bias) const = 0;
    virtual Tensor gather(const std::vector<int64_t>& ids) const;  // throws unless an embedding
    virtual Format format() const = 0;
    virtual int64_t bytes() const = 0;
    virtual int64_t fp32_bytes() const = 0;
};

std::unique_ptr<Weight> make_quantized(const Tensor& w, QuantMode mode);  // nullptr for None
std::unique_ptr<Weight> make_q8_embed(const Tensor& w);

// Weight files (serialize.hpp:1-35): load_bin's NIT0/NIT1 tensor onto the device
// as fp32, and a quantized weight read and quantized on the device (the file's
// payload never exists as an fp32 host tensor). File errors throw
// std::runtime_error, as load_bin does.
Tensor load_bin(const std::string& path);
std::unique_ptr<Weight> load_quantized(const std::string& path, QuantMode mode);  // nullptr for None

// Greedy next-token ids for each row of x: the argmax of linear_q8(x, head, bias)
// with the reference's first-index / NaN rules (sampling.cpp:14-20), computed
// without writing the logits. Synchronizes the stream.
std::vector<int64_t> lm_head_argmax(const Tensor& x, const QTensor& head, const Tensor* bias = nullptr);
// The same for an int8 embedding Weight (make_q8_embed);
// std::invalid_argument for any other weight.
std::vector<int64_t> lm_head_argmax(const Tensor& x, const Weight& head, const Tensor* bias = nullptr);

// The backend factory seam (backend.hpp:109-114): host fp32 weights in,
// device-resident quantized weights out.
class HipBackend {
public:
    std::unique_ptr<Weight> make_quant_weight(const Tensor& host, QuantMode mode) const;
    std::unique_ptr<Weight> make_embed_weight(const Tensor& host) const;
    const char* name() const { return "hip"; }
};

// Model dimensions from the exporter's config.txt (config.hpp:18-60, the
// key/value format of config.cpp:8-80). The architecture fields this path does
// not implement (qk_norm, MoE, sliding window, gelu, rope scaling, muP
// multipliers) are accepted only at their identity values; otherwise
// load_config throws std::runtime_error.
struct Config {
    int64_t vocab_size = 0;
    int64_t hidden_size = 0;
    int64_t intermediate_size = 0;
    int64_t num_layers = 0;
    int64_t num_attention_heads = 0;
    int64_t num_kv_heads = 0;
    int64_t head_dim = 0;
    int64_t max_position_embeddings = 0;
    float rms_norm_eps = 1e-6f;
    float rope_theta = 10000.0f;
    int64_t tie_word_embeddings = 0;
    int64_t eos_token_id = -1;
    int64_t qkv_bias = 1;
    int64_t n_rep() const { return num_attention_heads / num_kv_heads; }
};
Config load_config(const std::string& path);

// The decoder on the GPU (model.hpp:22-131): config.txt + every <name>.bin
// (NIT0 / NIT1) from weights_dir; the projections are device Weights of `mode`
// (make_quantized), the embedding and LM head the int8 embed Weight
// (make_q8_embed, the reference's quantize_embed). forward() recomputes the
// whole sequence (model.cpp:166-193 without a KV cache) and returns the fp32
// logits [seq, vocab] on the host. Only Device::HIP and a quant mode are
// accepted (std::invalid_argument otherwise).
class Model {
public:
    explicit Model(const std::string& weights_dir, QuantMode mode = QuantMode::W8A8, Device device = Device::HIP);
    Tensor forward(const std::vector<int64_t>& ids) const;
    // The greedy next token after ids (sampling.cpp:95 on forward's last row),
    // with the argmax fused into the LM-head GEMV of the last position: no
    // logits are written or copied to the host.
    int64_t next_token(const std::vector<int64_t>& ids) const;
    const Config& config() const { return cfg_; }
    Device device() const { return Device::HIP; }
    // {actual weight bytes, bytes if everything were fp32} (model.cpp:298-322).
    std::pair<int64_t, int64_t> weight_bytes() const;

private:
    Tensor hidden(const std::vector<int64_t>& ids) const;  // final-normed [seq, hidden], device fp32
    const Weight& head() const { return lm_head_ ? *lm_head_ : *embed_; }  // model.cpp:290-296
    struct Layer {
        std::unique_ptr<Weight> qkv, o, gate_up, down;  // q|k|v and gate|up fused by output rows
        Tensor qkv_bias, in_norm, post_norm;             // device fp32
    };
    Config cfg_;
    std::vector<Layer> layers_;
    Tensor final_norm_, cos_, sin_;
    std::unique_ptr<Weight> embed_, lm_head_;  // lm_head_ only for an untied checkpoint
};

}  // namespace hip
}  // namespace ni
