// C-ABI shim over the reference's own CPU quant path — TEST INFRASTRUCTURE ONLY.
//
// Compiled (by oracle/Makefile) together with the reference sources where they
// lie: /root/reference/cpp/src/{quant,tensor,ops}.cpp. The output goes to
// oracle/_ref/libnqref.so (git-ignored). It exists so that the C oracle can be
// checked against the real reference, so that tests/golden/gen_golden.py can
// write fixtures, and so that bench.py can time the reference's own AVX2+OpenMP
// path as the CPU baseline. The shim copies plain arrays into ni::Tensor /
// QTensor / Q4GTensor, calls the reference function, and copies the result out.
// Each nqr_* function has the same signature as its nqo_* twin in nq_oracle.h.
#include <cstdint>
#include <cstring>
#include <exception>
#include <vector>

#include "ops.hpp"
#include "parallel.hpp"
#include "quant.hpp"
#include "simd.hpp"
#include "tensor.hpp"

#if defined(_OPENMP)
#include <omp.h>
#endif

using ni::Tensor;

namespace {
Tensor host2d(const float* p, int64_t r, int64_t c) {
    Tensor t({r, c});
    if (r * c) std::memcpy(t.data(), p, sizeof(float) * size_t(r * c));
    return t;
}
Tensor host1d(const float* p, int64_t n) {
    Tensor t({n});
    if (n) std::memcpy(t.data(), p, sizeof(float) * size_t(n));
    return t;
}
void out2d(const Tensor& t, float* y) {
    if (t.numel()) std::memcpy(y, t.data(), sizeof(float) * size_t(t.numel()));
}
ni::QTensor qt(const int8_t* q, const float* s, int64_t out, int64_t in) {
    ni::QTensor t;
    t.out = out;
    t.in = in;
    t.q.assign(q, q + out * in);
    t.scale.assign(s, s + out);
    return t;
}
ni::Q4GTensor q4gt(const uint8_t* q, const float* s, int64_t out, int64_t in, int64_t g) {
    ni::Q4GTensor t;
    t.out = out;
    t.in = in;
    t.group = g;
    t.q.assign(q, q + out * ((in + 1) / 2));
    t.scale.assign(s, s + out * ((in + g - 1) / g));
    return t;
}
}  // namespace

#define NQR_TRY(body)                       \
    try {                                   \
        body;                               \
        return 0;                           \
    } catch (const std::exception&) {       \
        return -1;                          \
    }

extern "C" {

int nqr_max_threads(void) { return ni::max_threads(); }
void nqr_set_threads(int n) {
#if defined(_OPENMP)
    if (n > 0) omp_set_num_threads(n);
#else
    (void)n;
#endif
}
const char* nqr_simd_target(void) { return ni::simd::target(); }

int nqr_quantize_q8(const float* w, int64_t out, int64_t in, int8_t* q, float* scale) {
    NQR_TRY({
        ni::QTensor t = ni::quantize_q8(host2d(w, out, in));
        std::memcpy(q, t.q.data(), t.q.size());
        std::memcpy(scale, t.scale.data(), t.scale.size() * sizeof(float));
    })
}

int nqr_dequantize_q8(const int8_t* q, const float* s, int64_t out, int64_t in, float* w) {
    NQR_TRY(out2d(ni::dequantize_q8(qt(q, s, out, in)), w))
}

int nqr_embedding_q8(const int8_t* q, const float* s, int64_t vocab, int64_t hidden,
                     const int64_t* ids, int64_t n, float* out) {
    NQR_TRY(out2d(ni::embedding_q8(qt(q, s, vocab, hidden), std::vector<int64_t>(ids, ids + n)), out))
}

int nqr_linear_q8(const float* x, int64_t m, const int8_t* q, const float* s, int64_t out,
                  int64_t in, const float* bias, float* y) {
    NQR_TRY({
        Tensor b = bias ? host1d(bias, out) : Tensor();
        out2d(ni::linear_q8(host2d(x, m, in), qt(q, s, out, in), bias ? &b : nullptr), y);
    })
}

int nqr_linear_w8a8(const float* x, int64_t m, const int8_t* q, const float* s, int64_t out,
                    int64_t in, const float* bias, float* y) {
    NQR_TRY({
        Tensor b = bias ? host1d(bias, out) : Tensor();
        out2d(ni::linear_w8a8(host2d(x, m, in), qt(q, s, out, in), bias ? &b : nullptr), y);
    })
}

// The reference exposes no int32 accumulator; simd::dot_qq is the exact integer
// core linear_w8a8 calls (quant.cpp:205), so the shim evaluates it directly.
int nqr_w8a8_acc(const int8_t* xq, int64_t m, const int8_t* wq, int64_t out, int64_t in,
                 int32_t* acc) {
    for (int64_t i = 0; i < m; ++i)
        for (int64_t o = 0; o < out; ++o) acc[i * out + o] = ni::simd::dot_qq(xq + i * in, wq + o * in, in);
    return 0;
}

int nqr_quantize_q4g(const float* w, int64_t out, int64_t in, int64_t group, uint8_t* q,
                     float* scale) {
    NQR_TRY({
        ni::Q4GTensor t = ni::quantize_q4g(host2d(w, out, in), group);
        std::memcpy(q, t.q.data(), t.q.size());
        std::memcpy(scale, t.scale.data(), t.scale.size() * sizeof(float));
    })
}

int nqr_dequantize_q4g(const uint8_t* q, const float* s, int64_t out, int64_t in, int64_t group,
                       float* w) {
    NQR_TRY(out2d(ni::dequantize_q4g(q4gt(q, s, out, in, group)), w))
}

int nqr_linear_q4g(const float* x, int64_t m, const uint8_t* q, const float* s, int64_t out,
                   int64_t in, int64_t group, const float* bias, float* y) {
    NQR_TRY({
        Tensor b = bias ? host1d(bias, out) : Tensor();
        out2d(ni::linear_q4g(host2d(x, m, in), q4gt(q, s, out, in, group), bias ? &b : nullptr), y);
    })
}

int nqr_quantize_q4(const float* w, int64_t out, int64_t in, uint8_t* q, float* scale) {
    NQR_TRY({
        ni::Q4Tensor t = ni::quantize_q4(host2d(w, out, in));
        std::memcpy(q, t.q.data(), t.q.size());
        std::memcpy(scale, t.scale.data(), t.scale.size() * sizeof(float));
    })
}

int nqr_linear_q4(const float* x, int64_t m, const uint8_t* q, const float* s, int64_t out,
                  int64_t in, const float* bias, float* y) {
    NQR_TRY({
        ni::Q4Tensor t;
        t.out = out;
        t.in = in;
        t.q.assign(q, q + out * ((in + 1) / 2));
        t.scale.assign(s, s + out);
        Tensor b = bias ? host1d(bias, out) : Tensor();
        out2d(ni::linear_q4(host2d(x, m, in), t, bias ? &b : nullptr), y);
    })
}

void nqr_unpack_q4(const uint8_t* packed, int8_t* out, int64_t n) { ni::simd::unpack_q4(packed, out, n); }

int nqr_linear_f32(const float* x, int64_t m, const float* w, int64_t out, int64_t in,
                   const float* bias, float* y) {
    NQR_TRY({
        Tensor b = bias ? host1d(bias, out) : Tensor();
        out2d(ni::linear(host2d(x, m, in), host2d(w, out, in), bias ? &b : nullptr), y);
    })
}

// ---- ops.cpp functions the greedy-token reference decoder restates ---------
// (tests/model_ref.py): rmsnorm ops.cpp:272-290, build_rope_cache / apply_rope
// :120-166, attention :206-270, silu :86-92. Exported so that fixtures written
// from the reference's own build pin those numpy restatements.
static Tensor host3d(const float* p, int64_t a, int64_t b, int64_t c) {
    Tensor t({a, b, c});
    if (a * b * c) std::memcpy(t.data(), p, sizeof(float) * size_t(a * b * c));
    return t;
}

int nqr_rmsnorm(const float* x, int64_t rows, int64_t d, const float* w, float eps, float* y) {
    NQR_TRY(out2d(ni::rmsnorm(host2d(x, rows, d), host1d(w, d), eps), y))
}

int nqr_rope_cache(int64_t seq, int64_t head_dim, float theta, float* cos, float* sin) {
    NQR_TRY({
        ni::RopeCache c = ni::build_rope_cache(seq, head_dim, theta);
        out2d(c.cos, cos);
        out2d(c.sin, sin);
    })
}

int nqr_apply_rope(const float* x, int64_t heads, int64_t seq, int64_t dim, const float* cos,
                   const float* sin, int64_t table_len, int64_t pos_offset, float* y) {
    NQR_TRY(out2d(ni::apply_rope(host3d(x, heads, seq, dim), host2d(cos, table_len, dim),
                                 host2d(sin, table_len, dim), pos_offset),
                  y))
}

int nqr_attention(const float* q, const float* k, const float* v, int64_t heads, int64_t sq,
                  int64_t sk, int64_t dim, int causal, int64_t query_offset, float* y) {
    NQR_TRY(out2d(ni::attention(host3d(q, heads, sq, dim), host3d(k, heads, sk, dim),
                                host3d(v, heads, sk, dim), causal != 0, query_offset),
                  y))
}

int nqr_silu(const float* x, int64_t n, float* y) { NQR_TRY(out2d(ni::silu(host1d(x, n)), y)) }

}  // extern "C"
