// Decoder-caller support (not part of the quantized matrix path): RoPE on the
// q and k heads of a fused q|k|v projection output, written head-major for the
// attention kernel, with v copied to the same layout. One launch replaces the
// split / transpose / rotate-half / multiply-add chain of tensor ops that
// ops.cpp:120-166 (rope tables, apply_rope) becomes in the caller.
//   qkv  [s, ld] rows: q heads (heads*d) | k heads (kv*d) | v heads (kv*d)
//   cos, sin fp32 [>= s, d] (the half-split tables, cat([c, c]))
//   q [heads, s, d], k [kv, s, d], v [kv, s, d]
// out[j] = x[j] * cos[p, j] + rot[j] * sin[p, j], rot = cat(-x[d/2:], x[:d/2]),
// in fp32 with one rounding to the output type.
#include <hip/hip_runtime.h>

#include "nq_device.hpp"
#include "nq_internal.hpp"

namespace nq {
namespace {

template <typename T>
__global__ __launch_bounds__(256) void rope_qkv_kernel(const T* __restrict__ qkv, int s, int64_t ld, int heads, int kv,
                                                       int d, const float* __restrict__ cs, const float* __restrict__ sn,
                                                       T* __restrict__ q, T* __restrict__ k, T* __restrict__ v) {
    // one thread per (head, position, j < d/2); heads are q | k | v in order
    const int half = d >> 1;
    const int64_t total = static_cast<int64_t>(heads + 2 * kv) * s * half;
    const int64_t t = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (t >= total) return;
    const int j = static_cast<int>(t % half);
    const int64_t hp = t / half;
    const int p = static_cast<int>(hp % s), h = static_cast<int>(hp / s);
    const T* src = qkv + static_cast<int64_t>(p) * ld + static_cast<int64_t>(h) * d;
    const float x0 = to_f32(src[j]), x1 = to_f32(src[j + half]);
    T* dst;
    if (h < heads) dst = q + (static_cast<int64_t>(h) * s + p) * d;
    else if (h < heads + kv) dst = k + (static_cast<int64_t>(h - heads) * s + p) * d;
    else {
        dst = v + (static_cast<int64_t>(h - heads - kv) * s + p) * d;
        dst[j] = src[j];
        dst[j + half] = src[j + half];
        return;
    }
    const float* c = cs + static_cast<int64_t>(p) * d;
    const float* n = sn + static_cast<int64_t>(p) * d;
    dst[j] = from_f32<T>(x0 * c[j] - x1 * n[j]);
    dst[j + half] = from_f32<T>(x1 * c[j + half] + x0 * n[j + half]);
}

}  // namespace
}  // namespace nq

using namespace nq;

extern "C" nq_status nq_rope_qkv(const void* qkv, nq_dtype dtype, int64_t s, int64_t ld, int64_t heads,
                                 int64_t kv_heads, int64_t head_dim, const float* cos, const float* sin, void* q,
                                 void* k, void* v, void* stream) {
    NQ_REQUIRE(dtype_ok(dtype), NQ_BAD_ARG, "rope_qkv: unknown dtype");
    NQ_REQUIRE(s >= 0 && heads >= 0 && kv_heads >= 0 && head_dim >= 0 && head_dim % 2 == 0 &&
                   ld >= (heads + 2 * kv_heads) * head_dim && s <= kMaxIndex && ld <= kMaxIndex &&
                   (heads + 2 * kv_heads) * s * (head_dim / 2) <= kMaxIndex * 64,
               NQ_BAD_SHAPE, "rope_qkv: bad shape s=%lld ld=%lld heads=%lld kv=%lld d=%lld", (long long)s,
               (long long)ld, (long long)heads, (long long)kv_heads, (long long)head_dim);
    const int64_t total = (heads + 2 * kv_heads) * s * (head_dim / 2);
    if (total == 0) return NQ_OK;
    NQ_REQUIRE(qkv && cos && sin && q && (kv_heads == 0 || (k && v)), NQ_BAD_ARG, "rope_qkv: null pointer");
    const size_t es = dtype_size(dtype);
    NQ_REQUIRE(aligned(qkv, es) && aligned(q, es) && aligned(k, es) && aligned(v, es) && aligned(cos, 4) &&
                   aligned(sin, 4),
               NQ_BAD_ALIGN, "rope_qkv: misaligned pointer");
    hipStream_t st = as_stream(stream);
    const unsigned grid = static_cast<unsigned>((total + 255) / 256);
    const int si = static_cast<int>(s), h = static_cast<int>(heads), kv = static_cast<int>(kv_heads),
              d = static_cast<int>(head_dim);
    if (dtype == NQ_F32)
        rope_qkv_kernel<float><<<grid, 256, 0, st>>>(static_cast<const float*>(qkv), si, ld, h, kv, d, cos, sin,
                                                     static_cast<float*>(q), static_cast<float*>(k), static_cast<float*>(v));
    else
        rope_qkv_kernel<_Float16><<<grid, 256, 0, st>>>(static_cast<const _Float16*>(qkv), si, ld, h, kv, d, cos, sin,
                                                        static_cast<_Float16*>(q), static_cast<_Float16*>(k),
                                                        static_cast<_Float16*>(v));
    return launch_status("rope_qkv");
}
