/* nq.h — C ABI of libnq_hip.so, the MI355X (gfx950) quantized-weight matrix path.
 *
 * Every entry point takes device pointers, plain sizes and a HIP stream
 * (hipStream_t passed as void*; NULL = the null stream), enqueues its kernels on
 * that stream and returns without synchronizing. No entry point allocates
 * device memory: scratch space, where a path needs it, is a caller-owned
 * workspace whose size the matching *_workspace_size() call returns.
 *
 * Layouts follow the reference (cpp/src/quant.hpp:48-111):
 *   weights        [n, k] row-major, k contiguous (n = out-features, k = in);
 *   Q8 / W8A8      int8 codes [n*k] + fp32 per-row scale [n];
 *   Q4G            packed nibbles [n*ceil(k/2)] (column 2i -> low nibble of byte
 *                  i, stored as code+8) + one scale per (row, group)
 *                  [n*ceil(k/group)], fp32 (reference) or fp16 (storage variant);
 *   activations    x [m, k] row-major, fp32 or fp16; y [m, n] fp32 or fp16;
 *   bias           fp32 [n] or NULL.
 *
 * Errors: a non-NQ_OK status leaves the stream untouched (validation happens
 * before any launch) except NQ_HIP_ERROR, which reports a failed launch.
 * nq_last_error() returns the calling thread's message for its last failure —
 * the text the reference puts in its std::invalid_argument / runtime_error.
 */
#ifndef NQ_H
#define NQ_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum nq_status {
    NQ_OK = 0,
    NQ_BAD_SHAPE = 1, /* dims negative / inconsistent / beyond the 32-bit index range */
    NQ_BAD_ALIGN = 2, /* a pointer is not aligned to its element size */
    NQ_HIP_ERROR = 3, /* a HIP runtime call or kernel launch failed */
    NQ_BAD_ARG = 4,   /* null pointer, unknown enum, too-small workspace, bad id */
    NQ_IO_ERROR = 5,  /* a weight file cannot be read or is malformed (load_bin's errors) */
} nq_status;

typedef enum nq_dtype { NQ_F32 = 0, NQ_F16 = 1 } nq_dtype;

/* Kernel selection for the W8A8 linears. AUTO: m <= 4 (m <= 8 when k >= 4096 or n >= 8192)
 * -> workgroup-per-rows GEMV (v_dot4_i32_i8), larger m -> int8 MFMA GEMM; nq_linear_w8a8 runs
 * m = 1 as one GEMV launch with the act quant fused in, and with AUTO tries the one-launch
 * decode kernel (m * k <= 4096, or m <= 4 and m * k <= 8192) and the decode kernel over the act quant's codes
 * (m <= 16 with n and k <= 2048; m <= 8 with k <= 1024 and n <= 5120; m = 5..8 with k >= 8192 and
 * n <= 2048; m <= 32 with n <= 1536 and m <= 64 with n <= 512, both with k <= 2048) before
 * the rest. The forced values exist for A/B
 * tests, like the reference's CudaPolicy::force_tiled_w8a8
 * (cuda_backend.hpp:43-89). GENERIC is the scalar bounds-checked kernel. */
typedef enum nq_path { NQ_PATH_AUTO = 0, NQ_PATH_GEMV = 1, NQ_PATH_MFMA = 2, NQ_PATH_GENERIC = 3 } nq_path;

/* Library identification and error text. */
const char* nq_version(void);
const char* nq_status_name(int status);
const char* nq_last_error(void);

/* ---- quantize / pack (device side) ------------------------------------------
 * nq_quantize_q8 replaces the host quantize_q8 (quant.cpp:88-108) that
 * make_cuda_w8a8 / make_cuda_q8_embed run before upload (cuda_quant.cu:345-388):
 * scale[o] = max_j|w[o,j]| / 127 (fp32), q = round-half-even(w / scale)
 * clamped to +-127, NaN -> 0, all-zero row -> scale 0. Bit-exact with the
 * reference. w: fp32 [out, in]. */
nq_status nq_quantize_q8(const float* w, int64_t out, int64_t in, int8_t* q, float* scale,
                         void* stream);

/* Replaces quantize_q4g (quant.cpp:295-321): per (row, group) scale = absmax/7
 * computed in fp32, codes in [-7,7] from that fp32 scale, packed code+8 with the
 * even column in the low nibble. scale_dtype NQ_F16 stores the fp32 scale rounded
 * to fp16 (round-to-nearest-even); the codes are unchanged. q and scale are fully
 * written (no pre-zeroing needed). */
nq_status nq_quantize_q4g(const float* w, int64_t out, int64_t in, int64_t group, uint8_t* q,
                          void* scale, nq_dtype scale_dtype, void* stream);

/* Replace the reference's dequantize_q8 (quant.cpp:110-119) and dequantize_q4g
 * (quant.cpp:323-335), test helpers there: w[o,j] = float(q[o,j]) * scale[o] and
 * w[o,j] = float(nib(o,j) - 8) * scale[o, j / group], one fp32 multiply per
 * element (fp16 scales widened exactly first). w: [out, in] fp32 (the reference's
 * output) or fp16 (that value rounded). Bit-exact with the reference for fp32. */
nq_status nq_dequantize_q8(const int8_t* q, const float* scale, int64_t out, int64_t in, void* w,
                           nq_dtype w_dtype, void* stream);
nq_status nq_dequantize_q4g(const uint8_t* q, const void* scale, nq_dtype scale_dtype, int64_t group,
                            int64_t out, int64_t in, void* w, nq_dtype w_dtype, void* stream);

/* Replaces activation_quant_kernel (cuda_quant.cu:38-58) / the act-quant loop of
 * linear_w8a8 (quant.cpp:179-193): per-row a_scale = absmax/127 and int8 codes,
 * computed on the fp32 value of x (fp16 x is widened exactly first). */
nq_status nq_act_quant_i8(const void* x, nq_dtype x_dtype, int64_t m, int64_t k, int8_t* xq,
                          float* a_scale, void* stream);

/* ---- activation quant fused into its producer ------------------------------------
 * The act-quant of linear_w8a8 (quant.cpp:179-193) applied to the output of the
 * op that produces the activation, without writing that output: the W8A8 GEMM
 * (nq_gemm_w8a8) then consumes xq / a_scale. No reference counterpart as one
 * call: the reference runs rmsnorm (ops.cpp:272-290) or silu + mul
 * (ops.cpp:86-100) and then linear_w8a8 on the materialised tensor
 * (model.cpp:176-190). rmsnorm: y = x * (1/sqrt(mean(x^2) + eps)) * w, w fp32 [k];
 * silu_mul: y = gate / (1 + exp(-gate)) * up, gate and up rows at stride ld. */
/* The act quant of a head-major attention output x [heads, s, head_dim]: row p
 * of the result is row p of the [s, heads * head_dim] matrix its transpose
 * gives (the o_proj input, model.cpp:175-178), without materialising it. Same
 * codes and scales as nq_act_quant_i8 on that matrix. head_dim % 8 == 0,
 * heads * head_dim <= 16384, x 16-byte aligned. */
nq_status nq_act_quant_i8_heads(const void* x, nq_dtype x_dtype, int64_t heads, int64_t s, int64_t head_dim,
                                int8_t* xq, float* a_scale, void* stream);
nq_status nq_rmsnorm_quant_i8(const void* x, nq_dtype x_dtype, const float* w, float eps, int64_t m,
                              int64_t k, int8_t* xq, float* a_scale, void* stream);
/* The residual add before a norm fused in as well: h = x + r (stored to h as the
 * tensor add would, fp32 sum rounded once to the dtype; h may be x), then the
 * rmsnorm + act quant of nq_rmsnorm_quant_i8 on h (model.cpp:175-186: x += attn
 * / mlp output, then the next pre-norm). */
nq_status nq_add_rmsnorm_quant_i8(const void* x, const void* r, nq_dtype dtype, const float* w, float eps,
                                  int64_t m, int64_t k, void* h, int8_t* xq, float* a_scale, void* stream);
nq_status nq_silu_mul_quant_i8(const void* gate, const void* up, nq_dtype dtype, int64_t m, int64_t k,
                               int64_t ld, int8_t* xq, float* a_scale, void* stream);

/* ---- weight-only linears ------------------------------------------------------
 * Replaces cuda_linear_q8 (cuda/cuda.hpp:53, cuda_quant.cu:300-322) and the CPU
 * linear_q8 (quant.cpp:136-163): y[i,o] = (sum_j x[i,j]*q[o,j]) * w_scale[o] + b[o],
 * fp32 accumulation. */
nq_status nq_linear_q8(const void* x, nq_dtype x_dtype, const int8_t* q, const float* w_scale,
                       const float* bias, void* y, nq_dtype y_dtype, int64_t m, int64_t n,
                       int64_t k, void* stream);

/* The same linears with a caller workspace: batched activations whose weight
 * has too few rows to fill the GPU (small n, long k: m = 64, n = 1536, k = 8960)
 * split K into ranges whose fp32 partial sums (one [m, n] plane per range) the
 * workspace holds, then sum the planes in range order (deterministic). The
 * split changes the fp32 summation order, not the arithmetic: the results
 * agree with nq_linear_q8 / nq_linear_q4g to rounding. workspace: >=
 * nq_linear_wq_workspace_size(m, n, k) bytes (0: the shape does not split, and
 * NULL is accepted), 256-byte aligned. No counterpart in the reference, whose
 * cuda_linear_q8 (cuda_quant.cu:300-322) takes no workspace. */
size_t nq_linear_wq_workspace_size(int64_t m, int64_t n, int64_t k);
nq_status nq_linear_q8_ws(const void* x, nq_dtype x_dtype, const int8_t* q, const float* w_scale,
                          const float* bias, void* y, nq_dtype y_dtype, int64_t m, int64_t n, int64_t k,
                          void* workspace, size_t workspace_bytes, void* stream);

/* ---- decoder-caller support (outside the quantized matrix path) ----------------
 * RoPE of the q and k heads of a fused q|k|v output (ops.cpp:120-166: half-split
 * tables, x*cos + rotate_half(x)*sin in fp32) written head-major q [heads, s, d],
 * k [kv, s, d], with v copied to [kv, s, d]: the layout the attention takes.
 * qkv [s, ld] (ld >= (heads + 2 kv) d), cos/sin fp32 [>= s, d]. */
nq_status nq_rope_qkv(const void* qkv, nq_dtype dtype, int64_t s, int64_t ld, int64_t heads, int64_t kv_heads,
                      int64_t head_dim, const float* cos, const float* sin, void* q, void* k, void* v,
                      void* stream);

/* fp32 ops the C++ decoder caller runs between its quantized projections, with
 * the reference's arithmetic (ops.cpp): rmsnorm (ops.cpp:272-290; the sum of
 * squares in double) on rows x [m, k], optionally after the residual add
 * h = x + r (stored to h, which may be x; r == NULL skips it); silu(gate) * up
 * (ops.cpp:86-100) on rows at stride ld; causal GQA attention (ops.cpp:206-270,
 * repeat_kv :190-204) of head-major q [heads, s, d], k / v [kv_heads, s, d]
 * into token-major out [s, heads * d], s <= 16384. */
nq_status nq_rmsnorm_f32(const float* x, const float* r, float* h, const float* w, float eps, int64_t m, int64_t k,
                         float* y, void* stream);
nq_status nq_silu_mul_f32(const float* gate, const float* up, int64_t ld, int64_t m, int64_t k, float* y,
                          void* stream);
nq_status nq_attention_causal_f32(const float* q, const float* k, const float* v, int64_t heads, int64_t kv_heads,
                                  int64_t s, int64_t head_dim, float* out, void* stream);

/* ---- weight files: quantize on load -------------------------------------------
 * NIT0 / NIT1 files (serialize.hpp:1-23; load_bin serialize.cpp:11-72): the same
 * header checks as load_bin (bad magic, unknown dtype, negative ndim or dim,
 * short payload, trailing bytes -> NQ_IO_ERROR; at most 8 dims). The payload is
 * uploaded in row chunks of at most 64 MiB (a bf16 payload at 2 bytes per
 * element and inflated on the device by bits << 16, exact as in load_bin) and
 * quantized there by nq_quantize_q8 / nq_quantize_q4g, so the codes and scales
 * equal quantize_q8 / quantize_q4g of load_bin's fp32 tensor bit for bit. The
 * calls return after the stream has drained (they allocate and free pinned
 * host and device staging). */
nq_status nq_nit_info(const char* path, int32_t* dtype, int32_t* ndim, int64_t* shape, int32_t max_dims);
nq_status nq_nit_load_f32(const char* path, float* dst, int64_t numel, void* stream);
nq_status nq_nit_load_q8(const char* path, int8_t* q, float* scale, int64_t out, int64_t in, void* stream);
nq_status nq_nit_load_q4g(const char* path, uint8_t* q, void* scale, nq_dtype scale_dtype, int64_t group,
                          int64_t out, int64_t in, void* stream);

/* LM head with the greedy pick fused in: ids[i] = argmax_o y[i,o] of the
 * nq_linear_q8 fp32 logits, with the reference's tie and NaN rules (argmax,
 * sampling.cpp:14-20: first index of the maximum under a strict >, and 0 when
 * logit 0 is NaN). Replaces the decode step's cuda_linear_q8 on the int8 embed /
 * lm_head weight followed by the host argmax (cuda_quant.cu:357-379 ->
 * sampling.cpp:95) without writing the vocabulary-sized logits: every GEMV
 * workgroup reduces its rows to one (value, index) partial. The logits are
 * the q8 GEMV's fp32 values, bit for bit nq_linear_q8's output for m <= 8 (same
 * kernel and row grouping); larger m runs the GEMV in slices of 8 rows (as
 * nq_linear_q8 does where its MFMA GEMM does not apply). Shapes outside the GEMV's fast path (k %
 * 16 != 0, k > 16384, misaligned operands) compute the logits into the
 * workspace first. ids: int64 [m], 8-byte aligned. workspace (its first 256 bytes hold
 * the final reduction's per-row key and ticket): >=
 * nq_lm_head_argmax_q8_workspace_size(m, n, k) bytes, 256-byte aligned. */
size_t nq_lm_head_argmax_q8_workspace_size(int64_t m, int64_t n, int64_t k);
nq_status nq_lm_head_argmax_q8(const void* x, nq_dtype x_dtype, const int8_t* q, const float* w_scale,
                               const float* bias, int64_t* ids, int64_t m, int64_t n, int64_t k,
                               void* workspace, size_t workspace_bytes, void* stream);

/* Replaces linear_q4g (quant.cpp:337-389; the reference has no GPU int4 kernel):
 * y[i,o] = sum_blocks scale[o,blk] * (sum_{j in blk} x[i,j]*(nib-8)) + b[o]. */
nq_status nq_linear_q4g(const void* x, nq_dtype x_dtype, const uint8_t* q, const void* scale,
                        nq_dtype scale_dtype, int64_t group, const float* bias, void* y,
                        nq_dtype y_dtype, int64_t m, int64_t n, int64_t k, void* stream);
/* nq_linear_q4g with the split-K workspace of nq_linear_q8_ws (same size rule). */
nq_status nq_linear_q4g_ws(const void* x, nq_dtype x_dtype, const uint8_t* q, const void* scale,
                           nq_dtype scale_dtype, int64_t group, const float* bias, void* y,
                           nq_dtype y_dtype, int64_t m, int64_t n, int64_t k, void* workspace,
                           size_t workspace_bytes, void* stream);
/* The weight-only linears with a kernel choice per call (the nq_path values), the
 * per-call form of the reference's global CudaPolicy::force_tiled_q8
 * (cuda_backend.hpp:57-59, read at cuda_quant.cu:308), which forces the tiled
 * int8 GEMM at decode m for A/B runs. AUTO is nq_linear_q8_ws / nq_linear_q4g_ws;
 * GEMV runs the decode GEMV in slices of 8 activation rows at any m; MFMA runs the
 * fp16 MFMA GEMM at any m (NQ_BAD_ARG when k % 32 != 0, a Q4G group is not 32 *
 * 2^j, or x / q are not 16-byte aligned); GENERIC the bounds-checked scalar
 * kernel. Every path computes the same sums in fp32; they agree to rounding.
 * Same workspace rule as nq_linear_q8_ws. */
nq_status nq_linear_q8_ex(const void* x, nq_dtype x_dtype, const int8_t* q, const float* w_scale,
                          const float* bias, void* y, nq_dtype y_dtype, int64_t m, int64_t n, int64_t k,
                          void* workspace, size_t workspace_bytes, int path, void* stream);
nq_status nq_linear_q4g_ex(const void* x, nq_dtype x_dtype, const uint8_t* q, const void* scale,
                           nq_dtype scale_dtype, int64_t group, const float* bias, void* y,
                           nq_dtype y_dtype, int64_t m, int64_t n, int64_t k, void* workspace,
                           size_t workspace_bytes, int path, void* stream);

/* ---- W8A8 ------------------------------------------------------------------------
 * Replaces cuda_linear_w8a8 (cuda/cuda.hpp:41, cuda_quant.cu:250-284) and the CPU
 * linear_w8a8 (quant.cpp:165-210): dynamic per-row int8 activation quant, exact
 * int32 accumulation, y = float(acc) * a_scale[i] * w_scale[o] + b[o].
 * workspace: >= nq_linear_w8a8_workspace_size(m, n, k) bytes, 256-byte aligned;
 * the reference allocated xq/a_scale per call (cuda_quant.cu:253-258). */
size_t nq_linear_w8a8_workspace_size(int64_t m, int64_t n, int64_t k);
nq_status nq_linear_w8a8(const void* x, nq_dtype x_dtype, const int8_t* wq, const float* w_scale,
                         const float* bias, void* y, nq_dtype y_dtype, int64_t m, int64_t n,
                         int64_t k, void* workspace, size_t workspace_bytes, int path,
                         void* stream);

/* The same linear on activations that are already quantized (xq, a_scale from
 * nq_act_quant_i8) — the GEMM half of cuda_linear_w8a8 (cuda_quant.cu:260-283).
 * workspace: >= nq_gemm_w8a8_workspace_size(m, n, k) bytes (split-K partials). */
size_t nq_gemm_w8a8_workspace_size(int64_t m, int64_t n, int64_t k);
nq_status nq_gemm_w8a8(const int8_t* xq, const float* a_scale, const int8_t* wq,
                       const float* w_scale, const float* bias, void* y, nq_dtype y_dtype,
                       int64_t m, int64_t n, int64_t k, void* workspace, size_t workspace_bytes,
                       int path, void* stream);

/* No counterpart in the reference. nq_linear_w8a8 for callers that cannot
 * allocate (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc): the same kernels and results, with the workspace taken
 * from a static device array of nq_linear_w8a8_noalloc_max_scratch() bytes
 * (32 MiB) that each GPU holds for the life of the process. A shape whose
 * nq_linear_w8a8_workspace_size() exceeds it returns NQ_BAD_SHAPE before
 * anything is enqueued. The call allocates nothing. Every call on one GPU uses
 * that GPU's array: calls that overlap on one GPU (other streams, other host
 * threads) race. */
size_t nq_linear_w8a8_noalloc_max_scratch(void);
nq_status nq_linear_w8a8_noalloc(const void* x, nq_dtype x_dtype, const int8_t* wq, const float* w_scale,
                                 const float* bias, void* y, nq_dtype y_dtype, int64_t m, int64_t n, int64_t k,
                                 int path, void* stream);

/* Debug/parity entry: the exact int32 accumulators acc[i,o] = sum_j xq[i,j]*wq[o,j]
 * of the chosen path (the integer core of simd::dot_qq, simd.hpp:160-197, which
 * the reference never exposes). Same workspace rule as nq_gemm_w8a8. */
nq_status nq_w8a8_acc_i32(const int8_t* xq, const int8_t* wq, int32_t* acc, int64_t m, int64_t n,
                          int64_t k, void* workspace, size_t workspace_bytes, int path,
                          void* stream);

/* ---- int8 embedding gather --------------------------------------------------------
 * Replaces cuda_embedding_q8 (cuda/cuda.hpp:46, cuda_quant.cu:286-298) and
 * embedding_q8 (quant.cpp:121-134): out[r,c] = codes[ids[r],c] * scale[ids[r]].
 * ids is a HOST array, as in the reference; an id outside [0, vocab) returns
 * NQ_BAD_ARG before anything is enqueued. */
nq_status nq_embedding_q8(const int8_t* codes, const float* scale, int64_t vocab, int64_t hidden,
                          const int64_t* ids, int64_t n, void* out, nq_dtype out_dtype,
                          void* stream);

#ifdef __cplusplus
}
#endif

#endif /* NQ_H */
