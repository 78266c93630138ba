// The decoder caller of the quantized projections on the GPU: the reference's
// Model (cpp/src/model.hpp:22-131, model.cpp:40-193) for the Qwen2-style
// architecture, loading config.txt + every <name>.bin from a weights directory
// and running forward() with every projection a device Weight built by
// make_quantized (the HipBackend factory), the int8 embedding / LM head built
// by make_q8_embed, and the fp32 ops in between on the device (rmsnorm, RoPE,
// causal GQA attention, silu * mul: nq_rmsnorm_f32, nq_rope_qkv,
// nq_attention_causal_f32, nq_silu_mul_f32).
//
// Projections that share an input are stored concatenated by output rows
// (q|k|v, gate|up): quantization is per row (per row and group for Q4G), so
// the codes and scales equal those of the separate weights, and each pair of
// projections is one linear.
#include <hip/hip_runtime_api.h>

#include <cmath>
#include <cstring>
#include <filesystem>
#include <fstream>
#include <stdexcept>
#include <string>
#include <unordered_map>

#include "../../../include/nq.h"
#include "nq_host.hpp"

namespace fs = std::filesystem;

namespace ni {
namespace hip {

namespace {

void hip_ok(hipError_t e, const char* what) {
    if (e != hipSuccess) throw std::runtime_error(std::string(what) + ": " + hipGetErrorString(e));
}

void nq_ok(nq_status st) {
    if (st == NQ_OK) return;
    const std::string msg = std::string(nq_status_name(st)) + ": " + nq_last_error();
    if (st == NQ_HIP_ERROR || st == NQ_IO_ERROR) throw std::runtime_error(msg);
    throw std::invalid_argument(msg);
}

hipStream_t stream() { return static_cast<hipStream_t>(current_stream()); }

float* fp(const Tensor& t) { return static_cast<float*>(t.device_ptr()); }

// Rows of device fp32 tensors stacked into one [sum(rows), cols] (or 1-D) tensor.
Tensor concat_rows(const std::vector<const Tensor*>& parts) {
    int64_t rows = 0;
    const int64_t cols = parts[0]->ndim() == 2 ? parts[0]->size(1) : 1;
    for (const Tensor* p : parts) {
        if (!p->on_device() || p->dtype() != DType::F32 || (p->ndim() == 2 ? p->size(1) : 1) != cols)
            throw std::runtime_error("Model: fused projections need fp32 weights of one width");
        rows += p->ndim() == 2 ? p->size(0) : p->numel();
    }
    Tensor out(parts[0]->ndim() == 2 ? std::vector<int64_t>{rows, cols} : std::vector<int64_t>{rows}, DType::F32,
               Device::HIP);
    size_t off = 0;
    for (const Tensor* p : parts) {
        hip_ok(hipMemcpyAsync(static_cast<char*>(out.device_ptr()) + off, p->device_ptr(), p->nbytes(),
                              hipMemcpyDeviceToDevice, stream()),
               "hipMemcpyAsync");
        off += p->nbytes();
    }
    return out;
}

}  // namespace

Config load_config(const std::string& path) {
    std::ifstream f(path);
    if (!f) throw std::runtime_error("load_config: cannot open " + path);
    Config c;
    std::string key;
    // Architecture fields this path does not implement: accepted only at their
    // identity values (the Qwen2.5 defaults of config.hpp:37-60).
    int64_t qk_norm = 0, n_experts = 0, sliding_window = 0;
    std::string act_fn = "silu", rope_scaling = "none";
    float mults[4] = {1.0f, 1.0f, 1.0f, 1.0f};
    while (f >> key) {
        if (key == "vocab_size") f >> c.vocab_size;
        else if (key == "hidden_size") f >> c.hidden_size;
        else if (key == "intermediate_size") f >> c.intermediate_size;
        else if (key == "num_layers") f >> c.num_layers;
        else if (key == "num_attention_heads") f >> c.num_attention_heads;
        else if (key == "num_kv_heads") f >> c.num_kv_heads;
        else if (key == "head_dim") f >> c.head_dim;
        else if (key == "max_position_embeddings") f >> c.max_position_embeddings;
        else if (key == "rms_norm_eps") f >> c.rms_norm_eps;
        else if (key == "rope_theta") f >> c.rope_theta;
        else if (key == "tie_word_embeddings") f >> c.tie_word_embeddings;
        else if (key == "eos_token_id") f >> c.eos_token_id;
        else if (key == "qkv_bias") f >> c.qkv_bias;
        else if (key == "qk_norm") f >> qk_norm;
        else if (key == "act_fn") f >> act_fn;
        else if (key == "rope_scaling") f >> rope_scaling;
        else if (key == "embedding_multiplier") f >> mults[0];
        else if (key == "attention_multiplier") f >> mults[1];
        else if (key == "residual_multiplier") f >> mults[2];
        else if (key == "logits_scaling") f >> mults[3];
        else if (key == "n_experts") f >> n_experts;
        else if (key == "sliding_window") f >> sliding_window;
        else {
            std::string ignored;
            f >> ignored;  // unknown key: skip its value (config.cpp:58)
        }
    }
    auto need = [](int64_t v, const char* name) {
        if (v <= 0) throw std::runtime_error("load_config: missing or invalid '" + std::string(name) + "'");
    };
    need(c.vocab_size, "vocab_size");
    need(c.hidden_size, "hidden_size");
    need(c.intermediate_size, "intermediate_size");
    need(c.num_layers, "num_layers");
    need(c.num_attention_heads, "num_attention_heads");
    need(c.num_kv_heads, "num_kv_heads");
    need(c.head_dim, "head_dim");
    need(c.max_position_embeddings, "max_position_embeddings");
    if (c.num_attention_heads % c.num_kv_heads != 0)
        throw std::runtime_error("load_config: num_attention_heads must be divisible by num_kv_heads");
    if (qk_norm || n_experts || sliding_window || act_fn != "silu" || rope_scaling != "none" || mults[0] != 1.0f ||
        mults[1] != 1.0f || mults[2] != 1.0f || mults[3] != 1.0f)
        throw std::runtime_error(
            "load_config: the hip model implements the Qwen2 architecture (no qk_norm, MoE, sliding window, "
            "gelu, rope scaling or muP multipliers)");
    return c;
}

Model::Model(const std::string& weights_dir, QuantMode mode, Device device) {
    if (device != Device::HIP) throw std::invalid_argument("Model: this build runs on the GPU only (device 'hip')");
    if (mode == QuantMode::None)
        throw std::invalid_argument("Model: the hip model runs quantized projections (mode q8, q4, q4g or w8a8)");
    cfg_ = load_config(weights_dir + "/config.txt");
    std::unordered_map<std::string, Tensor> w;
    for (const auto& entry : fs::directory_iterator(weights_dir)) {
        const fs::path& p = entry.path();
        if (p.extension() == ".bin") w.emplace(p.stem().string(), load_bin(p.string()));  // model.cpp:50-57
    }
    if (w.empty()) throw std::runtime_error("Model: no .bin weights in " + weights_dir);
    auto take = [&w](const std::string& name) -> Tensor {
        auto it = w.find(name);
        if (it == w.end()) throw std::runtime_error("Model: missing weight " + name);
        Tensor t = it->second;
        w.erase(it);
        return t;
    };
    const int64_t H = cfg_.hidden_size, I = cfg_.intermediate_size, d = cfg_.head_dim;
    const int64_t qo = cfg_.num_attention_heads * d, kvo = cfg_.num_kv_heads * d;
    auto check2d = [](const Tensor& t, int64_t r, int64_t c, const std::string& name) {
        if (t.ndim() != 2 || t.size(0) != r || t.size(1) != c)
            throw std::runtime_error("Model: " + name + " has the wrong shape");
    };
    for (int64_t li = 0; li < cfg_.num_layers; ++li) {
        const std::string L = "layers." + std::to_string(li) + ".";
        Layer ly;
        Tensor q = take(L + "self_attn.q_proj.weight"), k = take(L + "self_attn.k_proj.weight"),
               v = take(L + "self_attn.v_proj.weight");
        check2d(q, qo, H, "q_proj");
        check2d(k, kvo, H, "k_proj");
        check2d(v, kvo, H, "v_proj");
        ly.qkv = make_quantized(concat_rows({&q, &k, &v}), mode);
        if (cfg_.qkv_bias) {
            Tensor qb = take(L + "self_attn.q_proj.bias"), kb = take(L + "self_attn.k_proj.bias"),
                   vb = take(L + "self_attn.v_proj.bias");
            ly.qkv_bias = concat_rows({&qb, &kb, &vb});
        }
        Tensor o = take(L + "self_attn.o_proj.weight");
        check2d(o, H, qo, "o_proj");
        ly.o = make_quantized(o, mode);
        Tensor g = take(L + "mlp.gate_proj.weight"), u = take(L + "mlp.up_proj.weight");
        check2d(g, I, H, "gate_proj");
        check2d(u, I, H, "up_proj");
        ly.gate_up = make_quantized(concat_rows({&g, &u}), mode);
        Tensor dn = take(L + "mlp.down_proj.weight");
        check2d(dn, H, I, "down_proj");
        ly.down = make_quantized(dn, mode);
        ly.in_norm = take(L + "input_layernorm.weight");
        ly.post_norm = take(L + "post_attention_layernorm.weight");
        layers_.push_back(std::move(ly));
    }
    final_norm_ = take("norm.weight");
    // The int8 embedding / tied LM head (the reference's quantize_embed, model.cpp:137-145):
    // this path has no dense GEMM, so the hip model always takes it.
    Tensor emb = take("embed_tokens.weight");
    check2d(emb, cfg_.vocab_size, H, "embed_tokens");
    embed_ = make_q8_embed(emb);
    // An untied checkpoint's own head; without lm_head.weight the head stays the
    // embedding, as the reference's Model leaves lm_head_ null (model.cpp:187, 290-296).
    if (!cfg_.tie_word_embeddings) {
        auto it = w.find("lm_head.weight");
        if (it != w.end()) {
            check2d(it->second, cfg_.vocab_size, H, "lm_head");
            lm_head_ = make_q8_embed(it->second);
            w.erase(it);
        }
    }
    // RoPE tables (ops.cpp:120-142): inv_freq and angles in double, rounded to float.
    const int64_t P = cfg_.max_position_embeddings, half = d / 2;
    Tensor cs({P, d}), sn({P, d});
    for (int64_t p = 0; p < P; ++p)
        for (int64_t i = 0; i < half; ++i) {
            const double inv = 1.0 / std::pow(double(cfg_.rope_theta), double(2 * i) / double(d));
            const double ang = double(p) * inv;
            cs[p * d + i] = cs[p * d + i + half] = static_cast<float>(std::cos(ang));
            sn[p * d + i] = sn[p * d + i + half] = static_cast<float>(std::sin(ang));
        }
    cos_ = to_device(cs);
    sin_ = to_device(sn);
    hip_ok(hipStreamSynchronize(stream()), "hipStreamSynchronize");
}

Tensor Model::hidden(const std::vector<int64_t>& ids) const {
    const int64_t s = static_cast<int64_t>(ids.size());
    if (s == 0) throw std::invalid_argument("Model::forward: empty ids");
    if (s > cfg_.max_position_embeddings)
        throw std::invalid_argument("Model::forward: sequence longer than max_position_embeddings");
    const int64_t H = cfg_.hidden_size, I = cfg_.intermediate_size, d = cfg_.head_dim;
    const int64_t nh = cfg_.num_attention_heads, nkv = cfg_.num_kv_heads, qkvw = (nh + 2 * nkv) * d;
    const float eps = cfg_.rms_norm_eps;
    Tensor x = embed_->gather(ids);  // ids are range-checked by the gather (invalid_argument)
    Tensor h({s, H}, DType::F32, Device::HIP);
    Tensor q({nh, s, d}, DType::F32, Device::HIP), k({nkv, s, d}, DType::F32, Device::HIP),
        v({nkv, s, d}, DType::F32, Device::HIP), a({s, nh * d}, DType::F32, Device::HIP),
        act({s, I}, DType::F32, Device::HIP);
    Tensor pending;  // the previous layer's MLP output, added by the next norm
    void* st = current_stream();
    for (const Layer& ly : layers_) {
        // x += pending (model.cpp:190); h = rmsnorm(x) (model.cpp:166)
        nq_ok(nq_rmsnorm_f32(fp(x), pending.numel() ? fp(pending) : nullptr, fp(x), fp(ly.in_norm), eps, s, H,
                             fp(h), st));
        const Tensor qkv = ly.qkv->linear(h, ly.qkv_bias.numel() ? &ly.qkv_bias : nullptr);
        nq_ok(nq_rope_qkv(qkv.device_ptr(), NQ_F32, s, qkvw, nh, nkv, d, fp(cos_), fp(sin_), fp(q), fp(k), fp(v),
                          st));
        nq_ok(nq_attention_causal_f32(fp(q), fp(k), fp(v), nh, nkv, s, d, fp(a), st));
        const Tensor o = ly.o->linear(a, nullptr);
        // x += o (model.cpp:178); h = rmsnorm(x) (model.cpp:181)
        nq_ok(nq_rmsnorm_f32(fp(x), fp(o), fp(x), fp(ly.post_norm), eps, s, H, fp(h), st));
        const Tensor gu = ly.gate_up->linear(h, nullptr);
        nq_ok(nq_silu_mul_f32(fp(gu), fp(gu) + I, 2 * I, s, I, fp(act), st));  // ops.cpp:86-100
        pending = ly.down->linear(act, nullptr);
    }
    nq_ok(nq_rmsnorm_f32(fp(x), fp(pending), fp(x), fp(final_norm_), eps, s, H, fp(h), st));
    return h;
}

Tensor Model::forward(const std::vector<int64_t>& ids) const { return to_host(head().linear(hidden(ids), nullptr)); }

int64_t Model::next_token(const std::vector<int64_t>& ids) const {
    const Tensor h = hidden(ids);
    return lm_head_argmax(h.rows(h.size(0) - 1, 1), head())[0];
}

std::pair<int64_t, int64_t> Model::weight_bytes() const {
    int64_t actual = 0, fp32 = 0;
    auto raw = [&](const Tensor& t) {
        actual += t.numel() * 4;
        fp32 += t.numel() * 4;
    };
    auto wt = [&](const Weight& w) {
        actual += w.bytes();
        fp32 += w.fp32_bytes();
    };
    for (const Layer& ly : layers_) {
        wt(*ly.qkv);
        wt(*ly.o);
        wt(*ly.gate_up);
        wt(*ly.down);
        raw(ly.in_norm);
        raw(ly.post_norm);
        raw(ly.qkv_bias);
    }
    raw(final_norm_);
    wt(*embed_);
    if (lm_head_) wt(*lm_head_);
    return {actual, fp32};
}

}  // namespace hip
}  // namespace ni
