/* CPU oracle for the quantized-weight matrix path — TEST INFRASTRUCTURE ONLY.
 *
 * A plain-C restatement of the reference CPU quant path
 * (cpp/src/quant.cpp, cpp/src/simd.hpp, cpp/src/ops.cpp:42-69). Only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it, and only
 * as the checker / the timed CPU baseline. The product path (libnq_hip.so)
 * never links or calls it.
 *
 * Layout conventions (identical to the reference, quant.hpp:48-111):
 *   weights [out, in] row-major, K (= in) contiguous;
 *   Q8:  int8 codes [out*in] + fp32 scale [out];
 *   Q4G: packed nibbles [out*ceil(in/2)] (even column -> low nibble, stored
 *        code+8) + fp32 scale [out*ceil(in/group)].
 *
 * Return codes: 0 = ok, -1 = invalid argument (the reference throws
 * std::invalid_argument in the same places).
 */
#ifndef NQ_ORACLE_H
#define NQ_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* quant.cpp:31-38 */
float nqo_round_clamp(float w, float scale, float qmax);

/* quant.cpp:88-108 (per-row absmax/127, round half-even, clamp, NaN->0). */
int nqo_quantize_q8(const float* w, int64_t out, int64_t in, int8_t* q, float* scale);
/* quant.cpp:110-119 */
int nqo_dequantize_q8(const int8_t* q, const float* scale, int64_t out, int64_t in, float* w);
/* quant.cpp:121-134; returns -1 on an out-of-range id (reference throws). */
int nqo_embedding_q8(const int8_t* q, const float* scale, int64_t vocab, int64_t hidden,
                     const int64_t* ids, int64_t n, float* out);
/* quant.cpp:136-163 with simd.hpp:107-152 (double accumulation). */
int nqo_linear_q8(const float* x, int64_t m, const int8_t* q, const float* scale, int64_t out,
                  int64_t in, const float* bias, float* y);
/* Activation half of quant.cpp:179-193 (identical to nqo_quantize_q8 applied to x). */
int nqo_act_quant(const float* x, int64_t m, int64_t k, int8_t* xq, float* a_scale);
/* Integer core of quant.cpp:195-208 with simd.hpp:160-197: acc[i,o] = sum_j xq[i,j]*wq[o,j]. */
int nqo_w8a8_acc(const int8_t* xq, int64_t m, const int8_t* wq, int64_t out, int64_t in,
                 int32_t* acc);
/* quant.cpp:165-210 (act quant, int32 dot, double epilogue). */
int nqo_linear_w8a8(const float* x, int64_t m, const int8_t* wq, const float* w_scale,
                    int64_t out, int64_t in, const float* bias, float* y);
/* quant.cpp:295-321. q must hold out*ceil(in/2) bytes; it is zero-filled here. */
int nqo_quantize_q4g(const float* w, int64_t out, int64_t in, int64_t group, uint8_t* q,
                     float* scale);
/* quant.cpp:323-335 */
int nqo_dequantize_q4g(const uint8_t* q, const float* scale, int64_t out, int64_t in,
                       int64_t group, float* w);
/* quant.cpp:337-389 (per-block double partial sum times block scale). */
int nqo_linear_q4g(const float* x, int64_t m, const uint8_t* q, const float* scale, int64_t out,
                   int64_t in, int64_t group, const float* bias, float* y);
/* quant.cpp:212-233 / 247-293: per-row int4 is Q4G with group == in. */
int nqo_quantize_q4(const float* w, int64_t out, int64_t in, uint8_t* q, float* scale);
int nqo_linear_q4(const float* x, int64_t m, const uint8_t* q, const float* scale, int64_t out,
                  int64_t in, const float* bias, float* y);
/* simd.hpp:206-238: n packed int4 codes -> int8 codes (nibble - 8). */
void nqo_unpack_q4(const uint8_t* packed, int8_t* out, int64_t n);
/* ops.cpp:42-69: dense fp32 linear, double accumulation (the tests' dequant reference). */
int nqo_linear_f32(const float* x, int64_t m, const float* w, int64_t out, int64_t in,
                   const float* bias, float* y);
/* Threads the OpenMP loops may use (1 without OpenMP). */
int nqo_max_threads(void);
void nqo_set_threads(int n);

#ifdef __cplusplus
}
#endif

#endif /* NQ_ORACLE_H */
