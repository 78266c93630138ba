// pybind11 module `nicpp` for the MI355X quant path: the reference's QuantMode /
// quant_mode surface (cpp/bindings/nicpp.cpp:51-76) plus the device weight
// factory (backend.hpp:109-114) with device "hip". Host arrays cross the
// boundary as numpy fp32; device work releases the GIL, as the reference's
// forward does (nicpp.cpp:221-233). Errors: std::invalid_argument -> ValueError,
// std::runtime_error -> RuntimeError (pybind11's standard translation).
#include <pybind11/numpy.h>
#include <pybind11/pybind11.h>
#include <pybind11/stl.h>

#include <cstring>
#include <memory>
#include <stdexcept>
#include <string>

#include "nq_host.hpp"

namespace py = pybind11;
using namespace ni::hip;

namespace {

Tensor host_from_numpy(const py::array_t<float, py::array::c_style | py::array::forcecast>& a) {
    std::vector<int64_t> shape(a.shape(), a.shape() + a.ndim());
    Tensor t(shape);
    if (t.numel()) std::memcpy(t.data(), a.data(), sizeof(float) * static_cast<size_t>(t.numel()));
    return t;
}

py::array_t<float> numpy_from_host(const Tensor& t) {
    std::vector<py::ssize_t> shape(t.shape().begin(), t.shape().end());
    py::array_t<float> out(shape);
    if (t.numel()) std::memcpy(out.mutable_data(), t.data(), sizeof(float) * static_cast<size_t>(t.numel()));
    return out;
}

DType dtype_from_string(const std::string& s) {
    if (s == "f32" || s == "fp32" || s == "float32") return DType::F32;
    if (s == "f16" || s == "fp16" || s == "float16") return DType::F16;
    throw std::invalid_argument("unknown activation dtype '" + s + "' (f32|f16)");
}

// A device weight held by Python.
struct PyWeight {
    std::shared_ptr<Weight> w;

    py::array_t<float> linear(const py::array_t<float, py::array::c_style | py::array::forcecast>& x,
                              py::object bias, const std::string& dtype) const {
        const DType dt = dtype_from_string(dtype);
        Tensor xh = host_from_numpy(x);
        if (xh.ndim() != 2) throw std::invalid_argument("linear expects 2-D x");
        Tensor bh;
        bool has_bias = !bias.is_none();
        if (has_bias) bh = host_from_numpy(bias.cast<py::array_t<float, py::array::c_style | py::array::forcecast>>());
        Tensor yh;
        {
            py::gil_scoped_release release;
            const Tensor xd = to_device(xh, dt);
            Tensor bd;
            if (has_bias) bd = to_device(bh, DType::F32);
            yh = to_host(w->linear(xd, has_bias ? &bd : nullptr));
        }
        return numpy_from_host(yh);
    }

    py::array_t<float> gather(const std::vector<int64_t>& ids) const {
        Tensor h;
        {
            py::gil_scoped_release release;
            h = to_host(w->gather(ids));
        }
        return numpy_from_host(h);
    }
};

struct PyBackend {
    std::string device;
    HipBackend impl;

    explicit PyBackend(const std::string& dev) : device(dev) {
        if (dev != "hip") throw std::invalid_argument("device must be 'hip' (the CPU path is the reference's own)");
    }
    py::object make_quant_weight(const py::array_t<float, py::array::c_style | py::array::forcecast>& w,
                                 QuantMode mode) const {
        Tensor h = host_from_numpy(w);
        std::unique_ptr<Weight> q;
        {
            py::gil_scoped_release release;
            q = impl.make_quant_weight(h, mode);
        }
        if (!q) return py::none();
        return py::cast(PyWeight{std::shared_ptr<Weight>(std::move(q))});
    }
    // A weight straight from a NIT0/NIT1 file (load_bin + make_quant_weight), quantized on the device.
    py::object load_quant_weight(const std::string& path, QuantMode mode) const {
        std::unique_ptr<Weight> q;
        {
            py::gil_scoped_release release;
            q = load_quantized(path, mode);
        }
        if (!q) return py::none();
        return py::cast(PyWeight{std::shared_ptr<Weight>(std::move(q))});
    }
    PyWeight make_embed_weight(const py::array_t<float, py::array::c_style | py::array::forcecast>& w) const {
        Tensor h = host_from_numpy(w);
        std::unique_ptr<Weight> q;
        {
            py::gil_scoped_release release;
            q = impl.make_embed_weight(h);
        }
        return PyWeight{std::shared_ptr<Weight>(std::move(q))};
    }
};

}  // namespace

PYBIND11_MODULE(nicpp, m) {
    m.doc() = "MI355X quantized-weight path: QuantMode, device weight factory (device='hip').";

    py::enum_<QuantMode>(m, "QuantMode", "Weight quantization mode.")
        .value("NONE", QuantMode::None, "fp32 (no quantization)")
        .value("Q8", QuantMode::Q8, "per-channel int8")
        .value("Q4", QuantMode::Q4, "per-channel int4")
        .value("Q4G", QuantMode::Q4G, "group-wise int4 (32-blocks)")
        .value("W8A8", QuantMode::W8A8, "int8 weight x int8 activation");
    m.def("quant_mode", &quant_mode, py::arg("name"), "Parse 'fp32'|'q8'|'q4'|'q4g'|'w8a8' into a QuantMode.");

    py::enum_<Format>(m, "Format")
        .value("F32", Format::F32)
        .value("F16", Format::F16)
        .value("BF16", Format::BF16)
        .value("Q8", Format::Q8)
        .value("Q4", Format::Q4)
        .value("Q4G", Format::Q4G)
        .value("W8A8", Format::W8A8);
    m.def("format_name", &format_name);

    py::class_<PyWeight>(m, "Weight")
        .def("linear", &PyWeight::linear, py::arg("x"), py::arg("bias") = py::none(), py::arg("dtype") = "f32",
             "y = x @ dequant(w)^T + bias on the GPU; x host fp32 [m, in] (sent as dtype), returns host fp32.")
        .def("gather", &PyWeight::gather, py::arg("ids"))
        .def("format", [](const PyWeight& p) { return p.w->format(); })
        .def("bytes", [](const PyWeight& p) { return p.w->bytes(); })
        .def("fp32_bytes", [](const PyWeight& p) { return p.w->fp32_bytes(); });

    py::class_<PyBackend>(m, "Backend")
        .def(py::init<const std::string&>(), py::arg("device") = "hip")
        .def_readonly("device", &PyBackend::device)
        .def("make_quant_weight", &PyBackend::make_quant_weight, py::arg("w"), py::arg("mode"))
        .def("make_embed_weight", &PyBackend::make_embed_weight, py::arg("w"))
        .def("load_quant_weight", &PyBackend::load_quant_weight, py::arg("path"), py::arg("mode"));

    m.def("make_backend", [](const std::string& device) { return PyBackend(device); }, py::arg("device") = "hip");

    // The process-wide kernel-selection policy of the int8 embedding / LM head
    // (the reference's cuda_policy() fields use_w8a8_lmhead and force_tiled_q8,
    // cuda_backend.hpp:43-89).
    m.def("set_policy", [](bool use_w8a8_lmhead, bool force_tiled_q8) {
              hip_policy().use_w8a8_lmhead = use_w8a8_lmhead;
              hip_policy().force_tiled_q8 = force_tiled_q8;
          }, py::arg("use_w8a8_lmhead") = false, py::arg("force_tiled_q8") = false);
    m.def("policy", []() {
        py::dict d;
        d["use_w8a8_lmhead"] = hip_policy().use_w8a8_lmhead;
        d["force_tiled_q8"] = hip_policy().force_tiled_q8;
        return d;
    });

    py::class_<Config>(m, "Config", "Model dimensions read from config.txt.")
        .def_readonly("vocab_size", &Config::vocab_size)
        .def_readonly("hidden_size", &Config::hidden_size)
        .def_readonly("intermediate_size", &Config::intermediate_size)
        .def_readonly("num_layers", &Config::num_layers)
        .def_readonly("num_attention_heads", &Config::num_attention_heads)
        .def_readonly("num_kv_heads", &Config::num_kv_heads)
        .def_readonly("head_dim", &Config::head_dim)
        .def_readonly("max_position_embeddings", &Config::max_position_embeddings)
        .def_readonly("rms_norm_eps", &Config::rms_norm_eps)
        .def_readonly("rope_theta", &Config::rope_theta)
        .def_readonly("tie_word_embeddings", &Config::tie_word_embeddings)
        .def_readonly("eos_token_id", &Config::eos_token_id)
        .def_readonly("qkv_bias", &Config::qkv_bias)
        .def_property_readonly("n_rep", &Config::n_rep);

    // The reference's Model binding (nicpp.cpp:207-233, 317): the same
    // constructor arguments, forward with the GIL released, config and
    // weight_bytes. device must be "hip" and mode a quant mode.
    py::class_<Model>(m, "Model")
        .def(py::init([](const std::string& weights_dir, QuantMode mode, const std::string& device) {
                 if (device != "hip")
                     throw std::invalid_argument("device must be 'hip' (the CPU path is the reference's own)");
                 std::unique_ptr<Model> mdl;
                 {
                     py::gil_scoped_release release;
                     mdl = std::make_unique<Model>(weights_dir, mode, Device::HIP);
                 }
                 return mdl;
             }),
             py::arg("weights_dir"), py::arg("mode") = QuantMode::W8A8, py::arg("device") = "hip",
             "Load config.txt + every <name>.bin (NIT0 / NIT1) from weights_dir; the projections are "
             "quantized on the GPU in `mode`, the embedding / LM head to int8.")
        .def_property_readonly("config", [](const Model& self) { return self.config(); })
        .def(
            "forward",
            [](const Model& self, const std::vector<int64_t>& ids, py::object cache) {
                if (!cache.is_none())
                    throw std::invalid_argument("forward: the hip model recomputes the sequence (no KV cache)");
                Tensor logits;
                {
                    py::gil_scoped_release release;
                    logits = self.forward(ids);
                }
                return numpy_from_host(logits);
            },
            py::arg("ids"), py::arg("cache") = py::none(), "Token ids -> logits [seq, vocab] (numpy fp32).")
        .def(
            "generate",
            [](const Model& self, const std::vector<int64_t>& prompt, int max_tokens, int64_t eos_id) {
                if (prompt.empty()) throw std::invalid_argument("generate: empty prompt");
                std::vector<int64_t> ids = prompt, out;
                {
                    py::gil_scoped_release release;
                    for (int t = 0; t < max_tokens; ++t) {
                        // the argmax fused into the last position's LM-head GEMV
                        const int64_t nxt = self.next_token(ids);
                        out.push_back(nxt);
                        if (nxt == eos_id) break;
                        ids.push_back(nxt);
                    }
                }
                return out;
            },
            py::arg("prompt"), py::arg("max_tokens") = 20, py::arg("eos_id") = -1,
            "Greedy continuation of prompt by full recompute; returns the new ids. Each pick is the "
            "LM-head GEMV with the argmax fused in (no logits leave the GPU).")
        .def("next_token", [](const Model& self, const std::vector<int64_t>& ids) {
                 py::gil_scoped_release release;
                 return self.next_token(ids);
             }, py::arg("ids"), "The greedy next token after ids (argmax of forward(ids)[-1]).")
        .def("weight_bytes", &Model::weight_bytes, "(actual_bytes, fp32_bytes) of the weights.");
}
