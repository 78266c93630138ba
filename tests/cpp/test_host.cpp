// GPU test of the C++ host API (nanoinfer_amd/csrc/host/nq_host.hpp), in the
// style of the reference's dependency-free C++ tests (cpp/tests/test_util.hpp:
// CHECK / CHECK_CLOSE, non-zero exit on failure). The cases follow
// cpp/tests/test_quant.cpp, run through the device weights: known answers,
// linear == dequantized matmul, factory routing and formats, error behaviour.
#include <cmath>
#include <cstdio>
#include <cstring>
#include <random>
#include <stdexcept>
#include <vector>

#include "../../nanoinfer_amd/csrc/host/nq_host.hpp"

using namespace ni::hip;

static int g_failures = 0;
#define CHECK(cond)                                                     \
    do {                                                                \
        if (!(cond)) {                                                  \
            std::printf("FAIL %s:%d  %s\n", __FILE__, __LINE__, #cond); \
            ++g_failures;                                               \
        }                                                               \
    } while (0)
#define CHECK_CLOSE(a, b, tol)                                                                        \
    do {                                                                                              \
        const double _d = std::fabs(double(a) - double(b));                                           \
        if (!(_d <= (tol))) {                                                                         \
            std::printf("FAIL %s:%d  |%g - %g| = %g > %g\n", __FILE__, __LINE__, double(a), double(b), \
                        _d, double(tol));                                                             \
            ++g_failures;                                                                             \
        }                                                                                             \
    } while (0)

static Tensor make(std::vector<int64_t> shape, std::vector<float> vals) {
    Tensor t(std::move(shape));
    for (int64_t i = 0; i < t.numel(); ++i) t[i] = vals[static_cast<size_t>(i)];
    return t;
}

static Tensor randn(std::vector<int64_t> shape, std::mt19937_64& rng, float sd = 1.0f) {
    std::normal_distribution<float> nd(0.0f, sd);
    Tensor t(std::move(shape));
    for (int64_t i = 0; i < t.numel(); ++i) t[i] = nd(rng);
    return t;
}

// y = x @ deq^T + b in double, deq [out, in] host.
static std::vector<double> ref_linear(const Tensor& x, const Tensor& deq, const Tensor* b) {
    const int64_t m = x.shape()[0], k = x.shape()[1], n = deq.shape()[0];
    std::vector<double> y(static_cast<size_t>(m * n));
    for (int64_t i = 0; i < m; ++i)
        for (int64_t o = 0; o < n; ++o) {
            double s = b ? (*b)[o] : 0.0;
            for (int64_t j = 0; j < k; ++j) s += double(x[i * k + j]) * deq[o * k + j];
            y[static_cast<size_t>(i * n + o)] = s;
        }
    return y;
}

static Tensor dequant_q8(const QTensor& q) {
    Tensor codes = to_host(q.q), sc = to_host(q.scale), d({q.out, q.in});
    for (int64_t o = 0; o < q.out; ++o)
        for (int64_t j = 0; j < q.in; ++j) d[o * q.in + j] = codes[o * q.in + j] * sc[o];
    return d;
}

int main() {
    // quantize_q8 known answers (test_quant.cpp:24-34)
    {
        QTensor q = quantize_q8(make({2, 3}, {1, 2, 4, -8, 0, 8}));
        Tensor codes = to_host(q.q), sc = to_host(q.scale);
        CHECK(q.out == 2 && q.in == 3);
        CHECK_CLOSE(sc[0], 4.0 / 127.0, 1e-9);
        CHECK_CLOSE(sc[1], 8.0 / 127.0, 1e-9);
        CHECK(codes[2] == 127 && codes[3] == -127 && codes[4] == 0);
    }
    // all-zero row (test_quant.cpp:87-96)
    {
        QTensor q = quantize_q8(make({2, 2}, {0, 0, 3, -3}));
        Tensor codes = to_host(q.q), sc = to_host(q.scale);
        CHECK(sc[0] == 0.0f && codes[0] == 0 && codes[1] == 0);
    }
    // linear_q8 / linear_w8a8 / linear_q4g == dequantized matmul (test_quant.cpp:51-116, :263-280)
    {
        std::mt19937_64 rng(1);
        Tensor x = randn({3, 64}, rng), w = randn({5, 64}, rng), b = randn({5}, rng);
        Tensor xd = to_device(x), bd = to_device(b);
        QTensor q = quantize_q8(w);
        Tensor deq = dequant_q8(q);
        std::vector<double> ref = ref_linear(x, deq, &b);
        Tensor y = to_host(linear_q8(xd, q, &bd));
        for (int64_t i = 0; i < y.numel(); ++i) CHECK_CLOSE(y[i], ref[static_cast<size_t>(i)], 1e-4);
        // W8A8: the activation quant is quantize_q8 applied to x
        Tensor xdeq = dequant_q8(quantize_q8(x));
        std::vector<double> ref8 = ref_linear(xdeq, deq, &b);
        Tensor y8 = to_host(linear_w8a8(xd, q, &bd));
        for (int64_t i = 0; i < y8.numel(); ++i) CHECK_CLOSE(y8[i], ref8[static_cast<size_t>(i)], 1e-3);
        // fp16 activations and outputs
        Tensor yh = to_host(linear_q8(to_device(x, DType::F16), q, &bd, DType::F16));
        for (int64_t i = 0; i < yh.numel(); ++i) CHECK_CLOSE(yh[i], ref[static_cast<size_t>(i)], 2e-2);
    }
    {
        std::mt19937_64 rng(6);
        for (int64_t m : {3, 16}) {
            Tensor x = randn({m, 256}, rng), w = randn({5, 256}, rng), b = randn({5}, rng);
            Q4GTensor q = quantize_q4g(w, 32);
            Tensor codes = to_host(q.q), sc = to_host(q.scale), deq({5, 256});
            for (int64_t o = 0; o < 5; ++o)
                for (int64_t j = 0; j < 256; ++j) {
                    const int byte = static_cast<int>(codes[o * 128 + j / 2]);
                    const int nib = (j & 1) ? (byte >> 4) : (byte & 15);
                    deq[o * 256 + j] = float(nib - 8) * sc[o * 8 + j / 32];
                }
            Tensor bd = to_device(b);
            std::vector<double> ref = ref_linear(x, deq, &b);
            Tensor y = to_host(linear_q4g(to_device(x), q, &bd));
            for (int64_t i = 0; i < y.numel(); ++i) CHECK_CLOSE(y[i], ref[static_cast<size_t>(i)], 1e-4);
        }
    }
    // Q4 byte layout (test_quant.cpp:199-211)
    {
        Q4GTensor q = quantize_q4(make({1, 2}, {7, -7}));
        Tensor codes = to_host(q.q), sc = to_host(q.scale);
        CHECK(q.q.numel() == 1 && codes[0] == 0x1F && sc[0] == 1.0f);
    }
    // factory routing, formats, bytes (test_quant.cpp:145-157, :345-381)
    {
        std::mt19937_64 rng(12);
        Tensor x = randn({2, 64}, rng), w = randn({4, 64}, rng);
        HipBackend be;
        auto w8 = be.make_quant_weight(w, QuantMode::W8A8);
        auto q8 = be.make_quant_weight(w, QuantMode::Q8);
        auto q4 = be.make_quant_weight(w, QuantMode::Q4);
        auto q4g = be.make_quant_weight(w, QuantMode::Q4G);
        CHECK(be.make_quant_weight(w, QuantMode::None) == nullptr);
        CHECK(w8->format() == Format::W8A8 && q8->format() == Format::Q8);
        CHECK(q4->format() == Format::Q4 && q4g->format() == Format::Q4G);
        CHECK(w8->bytes() == q8->bytes() && w8->bytes() == 4 * 64 + 4 * 4);
        CHECK(q4g->bytes() < q4g->fp32_bytes());
        CHECK(std::strcmp(format_name(q4g->format()), "q4g") == 0);
        Tensor xd = to_device(x);
        Tensor a = to_host(w8->linear(xd, nullptr)), b = to_host(linear_w8a8(xd, quantize_q8(w)));
        for (int64_t i = 0; i < a.numel(); ++i) CHECK(a[i] == b[i]);
        bool threw = false;
        try { q8->gather({0}); } catch (const std::runtime_error&) { threw = true; }
        CHECK(threw);
        auto emb = be.make_embed_weight(w);
        Tensor g = to_host(emb->gather({3, 0, 3}));
        Tensor deq = dequant_q8(quantize_q8(w));
        for (int64_t c = 0; c < 64; ++c) CHECK(g[c] == deq[3 * 64 + c] && g[64 + c] == deq[c]);
        CHECK(emb->format() == Format::Q8);
    }
    // error behaviour (quant.cpp:23-25, :297; test_quant.cpp:332-343, :403-411)
    {
        bool threw = false;
        try { quantize_q4g(make({2, 8}, std::vector<float>(16, 1.0f)), 0); } catch (const std::invalid_argument&) { threw = true; }
        CHECK(threw);
        threw = false;
        QTensor q = quantize_q8(make({3, 4}, {0, 1, 2, 3, 4, 5, 6, 7, 8, 9, 10, 11}));
        try { embedding_q8(q, {3}); } catch (const std::invalid_argument&) { threw = true; }
        CHECK(threw);
        threw = false;
        try { linear_q8(to_device(make({1, 5}, {1, 2, 3, 4, 5})), q); } catch (const std::invalid_argument&) { threw = true; }
        CHECK(threw);
        threw = false;
        try { quant_mode("int3"); } catch (const std::invalid_argument&) { threw = true; }
        CHECK(threw && quant_mode("w8a8") == QuantMode::W8A8);
    }
    // weight files (serialize.cpp:11-72, test_io.cpp:68-84) and the greedy LM head (sampling.cpp:14-20)
    {
        const char* path = "test_host_nit1.bin";
        {
            std::FILE* f = std::fopen(path, "wb");
            const int32_t hdr[4] = {1, 2, 4, 64};  // NIT1, bf16 payload, [4, 64]
            std::fwrite("NIT1", 1, 4, f);
            std::fwrite(hdr, 4, 4, f);
            for (int i = 0; i < 4 * 64; ++i) {
                const float v = (i % 64 == 7 + 11 * (i / 64)) ? 2.5f : 0.0625f * static_cast<float>((i * 7) % 5 - 2);
                uint32_t bits;
                std::memcpy(&bits, &v, 4);
                const uint16_t top = static_cast<uint16_t>(bits >> 16);  // the values are exact in bf16
                std::fwrite(&top, 2, 1, f);
            }
            std::fclose(f);
        }
        Tensor dev = load_bin(path);
        Tensor host = to_host(dev);
        CHECK(host.ndim() == 2 && host.size(0) == 4 && host.size(1) == 64 && host[7] == 2.5f && host[2] == 0.125f && host[3] == -0.0625f);
        auto w8 = load_quantized(path, QuantMode::W8A8);
        auto ref = make_quantized(host, QuantMode::W8A8);
        Tensor x = to_device(make({2, 64}, std::vector<float>(128, 1.0f)));
        Tensor a = to_host(w8->linear(x, nullptr)), b = to_host(ref->linear(x, nullptr));
        for (int64_t i = 0; i < a.numel(); ++i) CHECK(a[i] == b[i]);
        CHECK(load_quantized(path, QuantMode::Q4G)->format() == Format::Q4G);
        // rows 0..3 carry a 2.5 spike at columns 7, 18, 29, 40: x = e_29 picks row 2
        std::vector<float> e(64, 0.0f);
        e[29] = 1.0f;
        const std::vector<int64_t> ids = lm_head_argmax(to_device(make({1, 64}, e)), quantize_q8(host));
        CHECK(ids.size() == 1 && ids[0] == 2);
        bool threw = false;
        try { load_bin("missing_weight_file.bin"); } catch (const std::runtime_error&) { threw = true; }
        CHECK(threw);
        std::remove(path);
    }
    std::printf(g_failures ? "test_host: %d failures\n" : "test_host: ok\n", g_failures);
    return g_failures ? 1 : 0;
}
