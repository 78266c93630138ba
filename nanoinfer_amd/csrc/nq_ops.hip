// Decoder-caller support outside the quantized matrix path: the fp32 ops the
// C++ Model runs between its quantized projections, with the reference's
// arithmetic (cpp/src/ops.cpp), so the device forward tracks the reference's
// CPU forward closely:
//   rmsnorm    ops.cpp:272-290  sum of squares in double, scale = 1/sqrt(float(ss/d) + eps), x * scale * w
//   silu, mul  ops.cpp:86-100   v / (1 + exp(-v)), then the product in float
//   attention  ops.cpp:206-270  causal, scores float(dot) * scale with the dot in double,
//                               float exp, double denominator, double sums of double(e) * inv * v
// These are correctness-first kernels for the caller (one workgroup per row or
// per (query, head)), not tuned hot-path kernels.
#include <hip/hip_runtime.h>

#include "nq_device.hpp"
#include "nq_internal.hpp"

namespace nq {
namespace {

constexpr int kOpsThreads = 256;

// Sum of a double over the workgroup, a fixed-order tree in LDS.
__device__ double block_sum_f64(double v, double* red) {
    const int tid = threadIdx.x;
    red[tid] = v;
    __syncthreads();
    for (int s = kOpsThreads / 2; s > 0; s >>= 1) {
        if (tid < s) red[tid] += red[tid + s];
        __syncthreads();
    }
    const double r = red[0];
    __syncthreads();
    return r;
}

__device__ float block_max_f32(float v, float* red) {
    const int tid = threadIdx.x;
    red[tid] = v;
    __syncthreads();
    for (int s = kOpsThreads / 2; s > 0; s >>= 1) {
        if (tid < s) red[tid] = red[tid + s] > red[tid] ? red[tid + s] : red[tid];
        __syncthreads();
    }
    const float r = red[0];
    __syncthreads();
    return r;
}

// One workgroup per row. With r: h = x + r is stored (the residual add that
// precedes the norm; h may be x) and the norm runs on h.
__global__ __launch_bounds__(kOpsThreads) void rmsnorm_f32_kernel(const float* x, const float* r, float* h,
                                                                  const float* __restrict__ w, float eps, int k,
                                                                  float* y) {
    __shared__ double red[kOpsThreads];
    const size_t off = static_cast<size_t>(blockIdx.x) * k;
    double ss = 0.0;
    for (int c = threadIdx.x; c < k; c += kOpsThreads) {
        float v = x[off + c];
        if (r) {
            v = v + r[off + c];
            h[off + c] = v;
        }
        ss += static_cast<double>(v) * static_cast<double>(v);
    }
    ss = block_sum_f64(ss, red);
    const float scale = __fdiv_rn(1.0f, __fsqrt_rn(static_cast<float>(ss / k) + eps));
    const float* src = r ? h : x;
    for (int c = threadIdx.x; c < k; c += kOpsThreads) y[off + c] = src[off + c] * scale * w[c];
}

__global__ __launch_bounds__(kOpsThreads) void silu_mul_f32_kernel(const float* __restrict__ g,
                                                                   const float* __restrict__ u, int64_t ld, int k,
                                                                   float* __restrict__ y) {
    const size_t in = static_cast<size_t>(blockIdx.x) * ld, out = static_cast<size_t>(blockIdx.x) * k;
    for (int c = threadIdx.x; c < k; c += kOpsThreads) {
        const float v = g[in + c];
        y[out + c] = __fdiv_rn(v, 1.0f + expf(-v)) * u[in + c];
    }
}

// One workgroup per (query i, head h): q [H, s, d], k / v [KV, s, d] head-major,
// out [s, H * d] token-major (the o_proj input). Scores of keys 0..i live in LDS.
__global__ __launch_bounds__(kOpsThreads) void attention_causal_f32_kernel(const float* __restrict__ q,
                                                                           const float* __restrict__ kk,
                                                                           const float* __restrict__ v, int heads,
                                                                           int n_rep, int s, int d,
                                                                           float* __restrict__ out) {
    extern __shared__ float sc[];
    __shared__ double red[kOpsThreads];
    __shared__ float redf[kOpsThreads];
    const int i = blockIdx.x, hh = blockIdx.y, kvh = hh / n_rep, tid = threadIdx.x;
    const float* qi = q + (static_cast<size_t>(hh) * s + i) * d;
    const float* kh = kk + static_cast<size_t>(kvh) * s * d;
    const float* vh = v + static_cast<size_t>(kvh) * s * d;
    const float scale = __fdiv_rn(1.0f, __fsqrt_rn(static_cast<float>(d)));
    float mx = -__builtin_inff();
    for (int j = tid; j <= i; j += kOpsThreads) {
        double dot = 0.0;
        for (int c = 0; c < d; ++c) dot = __builtin_fma(static_cast<double>(qi[c]), static_cast<double>(kh[static_cast<size_t>(j) * d + c]), dot);
        const float sj = static_cast<float>(dot) * scale;
        sc[j] = sj;
        mx = sj > mx ? sj : mx;
    }
    mx = block_max_f32(mx, redf);
    double den = 0.0;
    for (int j = tid; j <= i; j += kOpsThreads) {
        const float e = expf(sc[j] - mx);
        sc[j] = e;
        den += e;
    }
    den = block_sum_f64(den, red);
    const double inv = static_cast<double>(static_cast<float>(1.0 / den));
    for (int c = tid; c < d; c += kOpsThreads) {
        double acc = 0.0;
        for (int j = 0; j <= i; ++j) acc += static_cast<double>(sc[j]) * inv * static_cast<double>(vh[static_cast<size_t>(j) * d + c]);
        out[static_cast<size_t>(i) * heads * d + static_cast<size_t>(hh) * d + c] = static_cast<float>(acc);
    }
}

}  // namespace
}  // namespace nq

using namespace nq;

extern "C" nq_status nq_rmsnorm_f32(const float* x, const float* r, float* h, const float* w, float eps, int64_t m,
                                    int64_t k, float* y, void* stream) {
    NQ_REQUIRE(m >= 0 && k >= 0 && m <= kMaxIndex && k <= kMaxIndex, NQ_BAD_SHAPE, "rmsnorm_f32: bad shape");
    if (m == 0 || k == 0) return NQ_OK;
    NQ_REQUIRE(x && w && y && (!r || h), NQ_BAD_ARG, "rmsnorm_f32: null pointer");
    NQ_REQUIRE(aligned(x, 4) && aligned(w, 4) && aligned(y, 4) && aligned(r, 4) && aligned(h, 4), NQ_BAD_ALIGN,
               "rmsnorm_f32: misaligned pointer");
    rmsnorm_f32_kernel<<<static_cast<unsigned>(m), kOpsThreads, 0, as_stream(stream)>>>(x, r, h, w, eps,
                                                                                         static_cast<int>(k), y);
    return launch_status("rmsnorm_f32_kernel");
}

extern "C" nq_status nq_silu_mul_f32(const float* gate, const float* up, int64_t ld, int64_t m, int64_t k, float* y,
                                     void* stream) {
    NQ_REQUIRE(m >= 0 && k >= 0 && ld >= k && m <= kMaxIndex && k <= kMaxIndex, NQ_BAD_SHAPE,
               "silu_mul_f32: bad shape");
    if (m == 0 || k == 0) return NQ_OK;
    NQ_REQUIRE(gate && up && y, NQ_BAD_ARG, "silu_mul_f32: null pointer");
    silu_mul_f32_kernel<<<static_cast<unsigned>(m), kOpsThreads, 0, as_stream(stream)>>>(gate, up, ld,
                                                                                          static_cast<int>(k), y);
    return launch_status("silu_mul_f32_kernel");
}

extern "C" nq_status nq_attention_causal_f32(const float* q, const float* k, const float* v, int64_t heads,
                                             int64_t kv_heads, int64_t s, int64_t head_dim, float* out,
                                             void* stream) {
    NQ_REQUIRE(heads > 0 && kv_heads > 0 && heads % kv_heads == 0 && s >= 0 && head_dim > 0 && s <= 16384 &&
                   heads <= 65535 && head_dim <= 1024,
               NQ_BAD_SHAPE, "attention_causal_f32: bad shape (heads %% kv_heads == 0, s <= 16384)");
    if (s == 0) return NQ_OK;
    NQ_REQUIRE(q && k && v && out, NQ_BAD_ARG, "attention_causal_f32: null pointer");
    const size_t lds = static_cast<size_t>(s) * sizeof(float);
    if (nq_status st = set_dynamic_lds(reinterpret_cast<const void*>(attention_causal_f32_kernel), lds,
                                       "attention_causal_f32"))
        return st;
    const dim3 grid(static_cast<unsigned>(s), static_cast<unsigned>(heads));
    attention_causal_f32_kernel<<<grid, kOpsThreads, lds, as_stream(stream)>>>(
        q, k, v, static_cast<int>(heads), static_cast<int>(heads / kv_heads), static_cast<int>(s),
        static_cast<int>(head_dim), out);
    return launch_status("attention_causal_f32_kernel");
}
