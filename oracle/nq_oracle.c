/* CPU oracle for the quantized-weight matrix path — TEST INFRASTRUCTURE ONLY.
 *
 * Restates the reference CPU quant path in plain C so the GPU kernels have a
 * checker on the GPU box, where the reference sources do not exist. Each
 * function cites the reference file:line it follows. Only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg load this library.
 *
 * Numerics that must match the reference exactly:
 *   - absmax uses the std::max(a, b) = (a < b) ? b : a comparison, so a NaN
 *     element never becomes the absmax (quant.cpp:100);
 *   - scale = absmax / qmax in fp32; code = nearbyint(w / scale) under the
 *     default (ties-to-even) rounding mode, clamped to +-qmax, NaN -> 0,
 *     scale <= 0 -> 0 (quant.cpp:31-38);
 *   - float-activation dots accumulate in double (simd.hpp:56-152), the int8
 *     dot in int32 (simd.hpp:160-197);
 *   - the epilogues are written with fma() where the reference's
 *     `a * b + c` expression is contracted by its -O3 -mfma build.
 * Output channels are split across OpenMP threads exactly like the reference
 * (parallel.hpp:42, kParallelMinRows = 64); one thread owns each output's whole
 * reduction, so results do not depend on the thread count.
 */
#include "nq_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

#if defined(_OPENMP)
#include <omp.h>
#endif

#define NQO_PARALLEL_MIN_ROWS 64 /* parallel.hpp:42 */

static const float kQ8Max = 127.0f; /* quant.cpp:14 */
static const float kQ4Max = 7.0f;   /* quant.cpp:15 */

int nqo_max_threads(void) {
#if defined(_OPENMP)
    return omp_get_max_threads();
#else
    return 1;
#endif
}

void nqo_set_threads(int n) {
#if defined(_OPENMP)
    if (n > 0) omp_set_num_threads(n);
#else
    (void)n;
#endif
}

/* quant.cpp:31-38 */
float nqo_round_clamp(float w, float scale, float qmax) {
    if (scale <= 0.0f) return 0.0f;
    float r = nearbyintf(w / scale);
    if (r > qmax) r = qmax;
    if (r < -qmax) r = -qmax;
    if (isnan(r)) return 0.0f;
    return r;
}

/* std::max(absmax, |v|) as quant.cpp:100 evaluates it. */
static inline float absmax_step(float absmax, float v) {
    const float a = fabsf(v);
    return (absmax < a) ? a : absmax;
}

static inline int64_t q4_row_bytes(int64_t in) { return (in + 1) / 2; } /* quant.cpp:40 */
static inline int64_t n_blocks(int64_t in, int64_t g) { return (in + g - 1) / g; } /* :60 */

/* quant.cpp:43-47 */
static inline int q4_code(const uint8_t* row, int64_t j) {
    const uint8_t byte = row[j / 2];
    const uint8_t nib = (j & 1) ? (uint8_t)(byte >> 4) : (uint8_t)(byte & 0x0F);
    return (int)nib - 8;
}

/* quant.cpp:71-75 */
static inline void pack_nibble(uint8_t* row, int64_t j, int code) {
    const uint8_t nib = (uint8_t)(code + 8);
    if (j & 1) row[j / 2] |= (uint8_t)(nib << 4);
    else row[j / 2] |= nib;
}

/* quant.cpp:88-108 */
int nqo_quantize_q8(const float* w, int64_t out, int64_t in, int8_t* q, float* scale) {
    if (out < 0 || in < 0) return -1;
    for (int64_t o = 0; o < out; ++o) {
        const float* wr = w + o * in;
        float absmax = 0.0f;
        for (int64_t j = 0; j < in; ++j) absmax = absmax_step(absmax, wr[j]);
        const float s = absmax / kQ8Max;
        scale[o] = s;
        for (int64_t j = 0; j < in; ++j) q[o * in + j] = (int8_t)nqo_round_clamp(wr[j], s, kQ8Max);
    }
    return 0;
}

/* quant.cpp:110-119 */
int nqo_dequantize_q8(const int8_t* q, const float* scale, int64_t out, int64_t in, float* w) {
    if (out < 0 || in < 0) return -1;
    for (int64_t o = 0; o < out; ++o)
        for (int64_t j = 0; j < in; ++j) w[o * in + j] = (float)q[o * in + j] * scale[o];
    return 0;
}

/* quant.cpp:121-134 */
int nqo_embedding_q8(const int8_t* q, const float* scale, int64_t vocab, int64_t hidden,
                     const int64_t* ids, int64_t n, float* out) {
    for (int64_t r = 0; r < n; ++r)
        if (ids[r] < 0 || ids[r] >= vocab) return -1;
    for (int64_t r = 0; r < n; ++r) {
        const int64_t id = ids[r];
        const float s = scale[id];
        for (int64_t c = 0; c < hidden; ++c) out[r * hidden + c] = (float)q[id * hidden + c] * s;
    }
    return 0;
}

/* simd.hpp:107-152: sum x[i]*q[i] in double (each product is exact). */
static inline double dot_qf32(const float* x, const int8_t* q, int64_t n) {
    double t = 0.0;
    for (int64_t i = 0; i < n; ++i) t += (double)x[i] * (double)q[i];
    return t;
}

/* simd.hpp:160-197 */
static inline int32_t dot_qq(const int8_t* a, const int8_t* b, int64_t n) {
    int32_t t = 0;
    for (int64_t i = 0; i < n; ++i) t += (int32_t)a[i] * (int32_t)b[i];
    return t;
}

/* simd.hpp:59-102 */
static inline double dot_f32(const float* a, const float* b, int64_t n) {
    double t = 0.0;
    for (int64_t i = 0; i < n; ++i) t += (double)a[i] * (double)b[i];
    return t;
}

/* quant.cpp:136-163 */
int nqo_linear_q8(const float* x, int64_t m, const int8_t* q, const float* scale, int64_t out,
                  int64_t in, const float* bias, float* y) {
    if (m < 0 || out < 0 || in < 0) return -1;
#if defined(_OPENMP)
#pragma omp parallel for schedule(static) if (out >= NQO_PARALLEL_MIN_ROWS)
#endif
    for (int64_t o = 0; o < out; ++o) {
        const int8_t* qr = q + o * in;
        const double s = (double)scale[o];
        const double b = bias ? (double)bias[o] : 0.0;
        for (int64_t i = 0; i < m; ++i) y[i * out + o] = (float)fma(dot_qf32(x + i * in, qr, in), s, b);
    }
    return 0;
}

/* quant.cpp:179-193 */
int nqo_act_quant(const float* x, int64_t m, int64_t k, int8_t* xq, float* a_scale) {
    return nqo_quantize_q8(x, m, k, xq, a_scale);
}

/* quant.cpp:195-208, integer core only. */
int nqo_w8a8_acc(const int8_t* xq, int64_t m, const int8_t* wq, int64_t out, int64_t in,
                 int32_t* acc) {
    if (m < 0 || out < 0 || in < 0) return -1;
#if defined(_OPENMP)
#pragma omp parallel for schedule(static) if (out >= NQO_PARALLEL_MIN_ROWS)
#endif
    for (int64_t o = 0; o < out; ++o)
        for (int64_t i = 0; i < m; ++i) acc[i * out + o] = dot_qq(xq + i * in, wq + o * in, in);
    return 0;
}

/* quant.cpp:165-210 */
int nqo_linear_w8a8(const float* x, int64_t m, const int8_t* wq, const float* w_scale,
                    int64_t out, int64_t in, const float* bias, float* y) {
    if (m < 0 || out < 0 || in < 0) return -1;
    int8_t* xq = (int8_t*)malloc((size_t)(m * in > 0 ? m * in : 1));
    float* as = (float*)malloc((size_t)(m > 0 ? m : 1) * sizeof(float));
    if (!xq || !as) {
        free(xq);
        free(as);
        return -1;
    }
    nqo_act_quant(x, m, in, xq, as);
#if defined(_OPENMP)
#pragma omp parallel for schedule(static) if (out >= NQO_PARALLEL_MIN_ROWS)
#endif
    for (int64_t o = 0; o < out; ++o) {
        const int8_t* qr = wq + o * in;
        const double ws = (double)w_scale[o];
        const double b = bias ? (double)bias[o] : 0.0;
        for (int64_t i = 0; i < m; ++i) {
            const double acc = (double)dot_qq(xq + i * in, qr, in);
            y[i * out + o] = (float)fma(acc * (double)as[i], ws, b);
        }
    }
    free(xq);
    free(as);
    return 0;
}

/* quant.cpp:295-321 */
int nqo_quantize_q4g(const float* w, int64_t out, int64_t in, int64_t group, uint8_t* q,
                     float* scale) {
    if (group <= 0 || out < 0 || in < 0) return -1;
    const int64_t rb = q4_row_bytes(in), blocks = n_blocks(in, group);
    memset(q, 0, (size_t)(out * rb));
    for (int64_t o = 0; o < out; ++o) {
        uint8_t* row = q + o * rb;
        const float* wr = w + o * in;
        for (int64_t b = 0; b < blocks; ++b) {
            const int64_t j0 = b * group, j1 = (j0 + group < in) ? j0 + group : in;
            float absmax = 0.0f;
            for (int64_t j = j0; j < j1; ++j) absmax = absmax_step(absmax, wr[j]);
            const float s = absmax / kQ4Max;
            scale[o * blocks + b] = s;
            for (int64_t j = j0; j < j1; ++j) pack_nibble(row, j, (int)nqo_round_clamp(wr[j], s, kQ4Max));
        }
    }
    return 0;
}

/* quant.cpp:323-335 */
int nqo_dequantize_q4g(const uint8_t* q, const float* scale, int64_t out, int64_t in,
                       int64_t group, float* w) {
    if (group <= 0 || out < 0 || in < 0) return -1;
    const int64_t rb = q4_row_bytes(in), blocks = n_blocks(in, group);
    for (int64_t o = 0; o < out; ++o)
        for (int64_t j = 0; j < in; ++j)
            w[o * in + j] = (float)q4_code(q + o * rb, j) * scale[o * blocks + j / group];
    return 0;
}

/* quant.cpp:337-389 */
int nqo_linear_q4g(const float* x, int64_t m, const uint8_t* q, const float* scale, int64_t out,
                   int64_t in, int64_t group, const float* bias, float* y) {
    if (group <= 0 || m < 0 || out < 0 || in < 0) return -1;
    const int64_t rb = q4_row_bytes(in), blocks = n_blocks(in, group);
#if defined(_OPENMP)
#pragma omp parallel for schedule(static) if (out >= NQO_PARALLEL_MIN_ROWS)
#endif
    for (int64_t o = 0; o < out; ++o) {
        const uint8_t* row = q + o * rb;
        const float* srow = scale + o * blocks;
        const double bias_o = bias ? (double)bias[o] : 0.0;
        for (int64_t i = 0; i < m; ++i) {
            const float* xr = x + i * in;
            double acc = 0.0;
            for (int64_t bk = 0; bk < blocks; ++bk) {
                const int64_t j0 = bk * group, j1 = (j0 + group < in) ? j0 + group : in;
                double bsum = 0.0;
                for (int64_t j = j0; j < j1; ++j) bsum += (double)xr[j] * (double)q4_code(row, j);
                acc = fma(bsum, (double)srow[bk], acc);
            }
            y[i * out + o] = (float)(acc + bias_o);
        }
    }
    return 0;
}

/* quant.cpp:212-233: per-row int4 == Q4G with one block per row. */
int nqo_quantize_q4(const float* w, int64_t out, int64_t in, uint8_t* q, float* scale) {
    return nqo_quantize_q4g(w, out, in, in > 0 ? in : 1, q, scale);
}

/* quant.cpp:247-293: acc = sum x*code (double), y = acc*scale + b. */
int nqo_linear_q4(const float* x, int64_t m, const uint8_t* q, const float* scale, int64_t out,
                  int64_t in, const float* bias, float* y) {
    if (m < 0 || out < 0 || in < 0) return -1;
    const int64_t rb = q4_row_bytes(in);
#if defined(_OPENMP)
#pragma omp parallel for schedule(static) if (out >= NQO_PARALLEL_MIN_ROWS)
#endif
    for (int64_t o = 0; o < out; ++o) {
        const uint8_t* row = q + o * rb;
        const double s = (double)scale[o];
        const double b = bias ? (double)bias[o] : 0.0;
        for (int64_t i = 0; i < m; ++i) {
            const float* xr = x + i * in;
            double acc = 0.0;
            for (int64_t j = 0; j < in; ++j) acc += (double)xr[j] * (double)q4_code(row, j);
            y[i * out + o] = (float)fma(acc, s, b);
        }
    }
    return 0;
}

/* simd.hpp:206-238 */
void nqo_unpack_q4(const uint8_t* packed, int8_t* out, int64_t n) {
    for (int64_t j = 0; j < n; ++j) out[j] = (int8_t)q4_code(packed, j);
}

/* ops.cpp:42-69 */
int nqo_linear_f32(const float* x, int64_t m, const float* w, int64_t out, int64_t in,
                   const float* bias, float* y) {
    if (m < 0 || out < 0 || in < 0) return -1;
#if defined(_OPENMP)
#pragma omp parallel for schedule(static) if (out >= NQO_PARALLEL_MIN_ROWS)
#endif
    for (int64_t o = 0; o < out; ++o) {
        const double b = bias ? (double)bias[o] : 0.0;
        for (int64_t i = 0; i < m; ++i) y[i * out + o] = (float)(dot_f32(x + i * in, w + o * in, in) + b);
    }
    return 0;
}
