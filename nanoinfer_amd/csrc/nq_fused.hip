// Activation quantization fused into its producers: rmsnorm -> int8 and
// silu(gate) * up -> int8. Each workgroup owns one row, keeps the produced fp32
// values in registers, reduces their absmax across the workgroup and writes the
// int8 codes and the row scale exactly as the activation quant of linear_w8a8
// does (quant.cpp:179-193: a_scale = absmax / 127, round half to even, clamp),
// so the W8A8 GEMM can consume them directly (nq_gemm_w8a8). The producer math
// follows the reference ops: rmsnorm ops.cpp:272-290 (x * (1 / sqrt(mean(x^2) +
// eps)) * w; the sum of squares is fp32 here, fp64 in the reference), silu
// ops.cpp:86-93 (v / (1 + exp(-v))) and mul ops.cpp:95-100.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <type_traits>

#include "nq_device.hpp"
#include "nq_internal.hpp"

namespace nq {
namespace {

// silu(g) = g / (1 + exp(-g)) from the hardware exp2 and reciprocal (about 1 ulp
// each): the vector kernels are VALU-bound, and the libm-accurate expf plus an
// IEEE divide cost ~25 instructions per element. Limits match the formula:
// g -> -inf gives -0 (NaN at -inf, as -inf / inf), +inf gives +inf, NaN stays NaN.
__device__ __forceinline__ float silu_f32(float g) {
    const float e = __builtin_amdgcn_exp2f(g * -1.44269504088896341f);
    return g * __builtin_amdgcn_rcpf(1.0f + e);
}

// Workgroup-wide reduction of one float through LDS (wave reduction first).
template <int NT, bool MAX>
__device__ __forceinline__ float block_reduce(float v, float* red) {
    v = MAX ? wave_absmax(v) : wave_sum_f32(v);
    const int tid = threadIdx.x;
    __syncthreads();  // red may still be read from a previous reduction
    if ((tid & 63) == 0) red[tid >> 6] = v;
    __syncthreads();
    float r = red[0];
#pragma unroll
    for (int w = 1; w < NT / 64; ++w) r = MAX ? absmax_step(r, red[w]) : r + red[w];
    return r;
}

// Quantizes the CPT x 8 fp32 values a thread holds (vector e = tid + c*NT of
// the row) with the row's absmax, and stores them as 8-byte code vectors.
template <int CPT, int NT>
__device__ __forceinline__ void quantize_store(const float (&v)[CPT][8], int steps, float am, float* red,
                                               int8_t* qr, float* a_scale_row) {
    const float absmax = block_reduce<NT, true>(am, red);
    const float sc = absmax / 127.0f;
    if (threadIdx.x == 0) *a_scale_row = sc;
    const RowQuantizer rq(sc);
    typedef int v2i __attribute__((ext_vector_type(2)));
#pragma unroll
    for (int c = 0; c < CPT; ++c) {
        const int e = threadIdx.x + c * NT;
        if (e < steps) {
            int lo = 0, hi = 0;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                lo |= (static_cast<int>(rq.code(v[c][j], 127.0f)) & 0xFF) << (8 * j);
                hi |= (static_cast<int>(rq.code(v[c][j + 4], 127.0f)) & 0xFF) << (8 * j);
            }
            reinterpret_cast<v2i*>(qr)[e] = v2i{lo, hi};
        }
    }
}

template <typename XT>
struct Vec8;
template <>
struct Vec8<float> {
    f4 a, b;
    __device__ __forceinline__ void load(const float* p) {
        a = reinterpret_cast<const f4*>(p)[0];
        b = reinterpret_cast<const f4*>(p)[1];
    }
    __device__ __forceinline__ float at(int j) const { return j < 4 ? a[j] : b[j - 4]; }
    // this = u + v, element-wise in fp32 (the sum a tensor add would store)
    __device__ __forceinline__ void set_sum(const Vec8& u, const Vec8& v) {
        a = u.a + v.a;
        b = u.b + v.b;
    }
    __device__ __forceinline__ void store(float* p) const {
        reinterpret_cast<f4*>(p)[0] = a;
        reinterpret_cast<f4*>(p)[1] = b;
    }
};
template <>
struct Vec8<_Float16> {
    typedef _Float16 h8 __attribute__((ext_vector_type(8)));
    h8 a;
    __device__ __forceinline__ void load(const _Float16* p) { a = *reinterpret_cast<const h8*>(p); }
    __device__ __forceinline__ float at(int j) const { return static_cast<float>(a[j]); }
    // fp32 sum rounded once to fp16, as an fp16 tensor add stores it
    __device__ __forceinline__ void set_sum(const Vec8& u, const Vec8& v) {
#pragma unroll
        for (int j = 0; j < 8; ++j) a[j] = from_f32<_Float16>(u.at(j) + v.at(j));
    }
    __device__ __forceinline__ void store(_Float16* p) const { *reinterpret_cast<h8*>(p) = a; }
};

// rmsnorm + quant: x row [k] (k % 8 == 0, 16-byte aligned rows), w fp32 [k].
// ADD: the row is first h = x + r (the residual add that precedes the norm),
// stored to h as a tensor add would, and the norm runs on h.
template <typename XT, int CPT, int NT, bool ADD = false>
// x and r are not __restrict__: the in-place add passes h == x.
__global__ __launch_bounds__(NT) void rmsnorm_quant_kernel(const XT* x, const float* __restrict__ w,
                                                           float eps, int k, int8_t* __restrict__ xq,
                                                           float* __restrict__ a_scale, const XT* r = nullptr,
                                                           XT* h = nullptr) {
    __shared__ float red[NT / 64];
    const int row = blockIdx.x, tid = threadIdx.x, steps = k >> 3;
    const XT* xr = x + static_cast<size_t>(row) * k;
    Vec8<XT> xv[CPT];
    f4 wv[CPT][2];
#pragma unroll
    for (int c = 0; c < CPT; ++c) {
        const int e = min(tid + c * NT, steps - 1);  // unconditional: all loads in flight together
        xv[c].load(xr + 8 * e);
        wv[c][0] = reinterpret_cast<const f4*>(w + 8 * e)[0];
        wv[c][1] = reinterpret_cast<const f4*>(w + 8 * e)[1];
    }
    if constexpr (ADD) {
        const XT* rr = r + static_cast<size_t>(row) * k;
        Vec8<XT> rv[CPT];
#pragma unroll
        for (int c = 0; c < CPT; ++c) rv[c].load(rr + 8 * min(tid + c * NT, steps - 1));
#pragma unroll
        for (int c = 0; c < CPT; ++c) {
            xv[c].set_sum(xv[c], rv[c]);
            // h may alias x: every element is read above before this thread writes it
            if (tid + c * NT < steps) xv[c].store(h + static_cast<size_t>(row) * k + 8 * (tid + c * NT));
        }
    }
    __builtin_amdgcn_sched_barrier(0);  // every load issued before the math (the scheduler interleaved them)
    float ss = 0.0f;
#pragma unroll
    for (int c = 0; c < CPT; ++c) {
        float p = 0.0f;
#pragma unroll
        for (int j = 0; j < 8; ++j) p = __builtin_fmaf(xv[c].at(j), xv[c].at(j), p);
        ss += tid + c * NT < steps ? p : 0.0f;
    }
    ss = block_reduce<NT, false>(ss, red);
    const float scale = 1.0f / __builtin_sqrtf(ss / static_cast<float>(k) + eps);
    float v[CPT][8];
    float am = 0.0f;
#pragma unroll
    for (int c = 0; c < CPT; ++c) {
        float a = 0.0f;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            v[c][j] = xv[c].at(j) * scale * (j < 4 ? wv[c][0][j] : wv[c][1][j - 4]);
            a = absmax_step(a, v[c][j]);
        }
        am = tid + c * NT < steps ? absmax_step(am, a) : am;
    }
    quantize_store<CPT, NT>(v, steps, am, red, xq + static_cast<size_t>(row) * k, a_scale + row);
}

// silu(gate) * up + quant: gate / up rows [k] at row stride ld elements.
template <typename XT, int CPT, int NT>
__global__ __launch_bounds__(NT) void silu_mul_quant_kernel(const XT* __restrict__ gate, const XT* __restrict__ up,
                                                            int64_t ld, int k, int8_t* __restrict__ xq,
                                                            float* __restrict__ a_scale) {
    __shared__ float red[NT / 64];
    const int row = blockIdx.x, tid = threadIdx.x, steps = k >> 3;
    const XT* gr = gate + static_cast<size_t>(row) * ld;
    const XT* ur = up + static_cast<size_t>(row) * ld;
    Vec8<XT> gv[CPT], uv[CPT];
#pragma unroll
    for (int c = 0; c < CPT; ++c) {
        const int e = min(tid + c * NT, steps - 1);
        gv[c].load(gr + 8 * e);
        uv[c].load(ur + 8 * e);
    }
    __builtin_amdgcn_sched_barrier(0);  // every load issued before the math (the scheduler interleaved them)
    float v[CPT][8];
    float am = 0.0f;
#pragma unroll
    for (int c = 0; c < CPT; ++c) {
        float a = 0.0f;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const float g = gv[c].at(j);
            v[c][j] = silu_f32(g) * uv[c].at(j);
            a = absmax_step(a, v[c][j]);
        }
        am = tid + c * NT < steps ? absmax_step(am, a) : am;
    }
    quantize_store<CPT, NT>(v, steps, am, red, xq + static_cast<size_t>(row) * k, a_scale + row);
}

// Rows too long or not vector-aligned for the kernels above: one workgroup per
// row, strided scalar loops; the produced values are recomputed in the quantize
// pass instead of being held in registers.
template <typename XT, bool RMS>
__global__ __launch_bounds__(256) void fused_quant_generic_kernel(const XT* __restrict__ a, const XT* __restrict__ b,
                                                                  const float* __restrict__ w, float eps, int64_t ld,
                                                                  int k, int8_t* __restrict__ xq,
                                                                  float* __restrict__ a_scale) {
    __shared__ float red[4];
    const int row = blockIdx.x, tid = threadIdx.x;
    const XT* ar = a + static_cast<size_t>(row) * ld;
    const XT* br = RMS ? nullptr : b + static_cast<size_t>(row) * ld;
    float scale = 1.0f;
    if constexpr (RMS) {
        float ss = 0.0f;
        for (int j = tid; j < k; j += 256) ss = __builtin_fmaf(to_f32(ar[j]), to_f32(ar[j]), ss);
        ss = block_reduce<256, false>(ss, red);
        scale = 1.0f / __builtin_sqrtf(ss / static_cast<float>(k) + eps);
    }
    auto value = [&](int j) {
        if constexpr (RMS) {
            return to_f32(ar[j]) * scale * w[j];
        } else {
            const float g = to_f32(ar[j]);
            return silu_f32(g) * to_f32(br[j]);
        }
    };
    float am = 0.0f;
    for (int j = tid; j < k; j += 256) am = absmax_step(am, value(j));
    const float absmax = block_reduce<256, true>(am, red);
    const float sc = absmax / 127.0f;
    if (tid == 0) a_scale[row] = sc;
    const RowQuantizer rq(sc);
    int8_t* qr = xq + static_cast<size_t>(row) * k;
    for (int j = tid; j < k; j += 256) qr[j] = static_cast<int8_t>(rq.code(value(j), 127.0f));
}

// Launch shape: 256 threads up to 2048 elements per row, else 1024 threads with
// up to 4 vectors of 8 elements each (k <= 32768); with m >= 256 and k > 8192,
// 512 threads.
template <typename Fn>
void by_shape(int64_t m, int64_t k, Fn&& fn) {
    // With m >= 256 rows, 256 threads per row up to 2048 vectors (k <= 16384):
    // several vectors per thread keep more loads in flight and let 4-6 rows
    // share a CU, where a 1024-thread row with one vector per thread ran at
    // two thirds of the rate. Fewer rows cannot fill the GPU that way and take
    // 1024 threads per row (shorter per-row latency).
    const int64_t steps = k / 8;
    using I = std::integral_constant<int, 256>;
    const int64_t per = m >= 256 ? (steps + 255) / 256 : (steps <= 256 ? 1 : 0);
    // Past 1024 vectors per row (k > 8192), 512 threads with 3-4 vectors each
    // (silu*up quant, k = 8960: m = 512 7.9 -> 7.0 us, m = 2048 19.6 -> 18.9).
    if (per >= 5 && per <= 8) {
        if ((steps + 511) / 512 == 3) return fn(std::integral_constant<int, 3>{}, std::integral_constant<int, 512>{});
        return fn(std::integral_constant<int, 4>{}, std::integral_constant<int, 512>{});
    }
    switch (per) {
        case 0: break;
        case 1: return fn(std::integral_constant<int, 1>{}, I{});
        case 2: return fn(std::integral_constant<int, 2>{}, I{});
        case 3: return fn(std::integral_constant<int, 3>{}, I{});
        case 4: return fn(std::integral_constant<int, 4>{}, I{});  // 5..8 took the 512-thread rows above
        default: break;
    }
    switch ((steps + 1023) / 1024) {
        case 1: return fn(std::integral_constant<int, 1>{}, std::integral_constant<int, 1024>{});
        case 2: return fn(std::integral_constant<int, 2>{}, std::integral_constant<int, 1024>{});
        case 3: return fn(std::integral_constant<int, 3>{}, std::integral_constant<int, 1024>{});
        default: return fn(std::integral_constant<int, 4>{}, std::integral_constant<int, 1024>{});
    }
}

nq_status check_fused(int64_t m, int64_t k, const void* xq, const float* a_scale, nq_dtype dt, const char* who) {
    NQ_REQUIRE(m >= 0 && k >= 0 && m <= kMaxIndex && k <= kMaxIndex, NQ_BAD_SHAPE, "%s: bad shape m=%lld k=%lld",
               who, (long long)m, (long long)k);
    NQ_REQUIRE(dtype_ok(dt), NQ_BAD_ARG, "%s: unknown dtype %d", who, int(dt));
    NQ_REQUIRE(m == 0 || (a_scale && (k == 0 || xq)), NQ_BAD_ARG, "%s: null pointer", who);
    NQ_REQUIRE(aligned(a_scale, 4), NQ_BAD_ALIGN, "%s: misaligned a_scale", who);
    return NQ_OK;
}

}  // namespace
}  // namespace nq

using namespace nq;

extern "C" nq_status nq_rmsnorm_quant_i8(const void* x, nq_dtype x_dtype, const float* w, float eps, int64_t m,
                                         int64_t k, int8_t* xq, float* a_scale, void* stream) {
    if (nq_status st = check_fused(m, k, xq, a_scale, x_dtype, "rmsnorm_quant_i8")) return st;
    if (m == 0) return NQ_OK;
    NQ_REQUIRE(k > 0, NQ_BAD_SHAPE, "rmsnorm_quant_i8: k must be positive");
    NQ_REQUIRE(x && w, NQ_BAD_ARG, "rmsnorm_quant_i8: null pointer");
    NQ_REQUIRE(aligned(x, dtype_size(x_dtype)) && aligned(w, 4), NQ_BAD_ALIGN, "rmsnorm_quant_i8: misaligned pointer");
    hipStream_t s = as_stream(stream);
    const unsigned grid = static_cast<unsigned>(m);
    const int ki = static_cast<int>(k);
    const bool vec = k % 8 == 0 && k <= 32768 && aligned(x, 16) && aligned(w, 16) && aligned(xq, 8);
    auto go = [&](auto* xp) {
        using XT = std::remove_const_t<std::remove_pointer_t<decltype(xp)>>;
        if (vec)
            by_shape(m, k, [&](auto cpt, auto nt) {
                rmsnorm_quant_kernel<XT, decltype(cpt)::value, decltype(nt)::value>
                    <<<grid, decltype(nt)::value, 0, s>>>(xp, w, eps, ki, xq, a_scale);
            });
        else
            fused_quant_generic_kernel<XT, true><<<grid, 256, 0, s>>>(xp, nullptr, w, eps, k, ki, xq, a_scale);
    };
    if (x_dtype == NQ_F32) go(static_cast<const float*>(x));
    else go(static_cast<const _Float16*>(x));
    return launch_status("rmsnorm_quant_i8");
}

__global__ void add_rows_kernel(const float* x, const float* r, float* h, int64_t n) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i < n) h[i] = x[i] + r[i];
}
__global__ void add_rows_kernel(const _Float16* x, const _Float16* r, _Float16* h, int64_t n) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i < n) h[i] = from_f32<_Float16>(static_cast<float>(x[i]) + static_cast<float>(r[i]));
}

extern "C" nq_status nq_add_rmsnorm_quant_i8(const void* x, const void* r, nq_dtype dtype, const float* w, float eps,
                                             int64_t m, int64_t k, void* h, int8_t* xq, float* a_scale,
                                             void* stream) {
    if (nq_status st = check_fused(m, k, xq, a_scale, dtype, "add_rmsnorm_quant_i8")) return st;
    if (m == 0) return NQ_OK;
    NQ_REQUIRE(k > 0, NQ_BAD_SHAPE, "add_rmsnorm_quant_i8: k must be positive");
    NQ_REQUIRE(x && r && h && w, NQ_BAD_ARG, "add_rmsnorm_quant_i8: null pointer");
    const size_t es = dtype_size(dtype);
    NQ_REQUIRE(aligned(x, es) && aligned(r, es) && aligned(h, es) && aligned(w, 4), NQ_BAD_ALIGN,
               "add_rmsnorm_quant_i8: misaligned pointer");
    hipStream_t s = as_stream(stream);
    const unsigned grid = static_cast<unsigned>(m);
    const int ki = static_cast<int>(k);
    const bool vec = k % 8 == 0 && k <= 32768 && aligned(x, 16) && aligned(r, 16) && aligned(h, 16) &&
                     aligned(w, 16) && aligned(xq, 8);
    auto go = [&](auto* xp, auto* rp, auto* hp) {
        using XT = std::remove_const_t<std::remove_pointer_t<decltype(xp)>>;
        if (vec) {
            by_shape(m, k, [&](auto cpt, auto nt) {
                rmsnorm_quant_kernel<XT, decltype(cpt)::value, decltype(nt)::value, true>
                    <<<grid, decltype(nt)::value, 0, s>>>(xp, w, eps, ki, xq, a_scale, rp, hp);
            });
        } else {
            const int64_t n = m * k;
            add_rows_kernel<<<static_cast<unsigned>((n + 255) / 256), 256, 0, s>>>(xp, rp, hp, n);
            fused_quant_generic_kernel<XT, true><<<grid, 256, 0, s>>>(hp, nullptr, w, eps, k, ki, xq, a_scale);
        }
    };
    if (dtype == NQ_F32)
        go(static_cast<const float*>(x), static_cast<const float*>(r), static_cast<float*>(h));
    else
        go(static_cast<const _Float16*>(x), static_cast<const _Float16*>(r), static_cast<_Float16*>(h));
    return launch_status("add_rmsnorm_quant_i8");
}

extern "C" nq_status nq_silu_mul_quant_i8(const void* gate, const void* up, nq_dtype dtype, int64_t m, int64_t k,
                                          int64_t ld, int8_t* xq, float* a_scale, void* stream) {
    if (nq_status st = check_fused(m, k, xq, a_scale, dtype, "silu_mul_quant_i8")) return st;
    if (m == 0) return NQ_OK;
    NQ_REQUIRE(k > 0 && ld >= k, NQ_BAD_SHAPE, "silu_mul_quant_i8: need 0 < k <= ld");
    NQ_REQUIRE(gate && up, NQ_BAD_ARG, "silu_mul_quant_i8: null pointer");
    const size_t es = dtype_size(dtype);
    NQ_REQUIRE(aligned(gate, es) && aligned(up, es), NQ_BAD_ALIGN, "silu_mul_quant_i8: misaligned pointer");
    hipStream_t s = as_stream(stream);
    const unsigned grid = static_cast<unsigned>(m);
    const int ki = static_cast<int>(k);
    const bool vec = k % 8 == 0 && k <= 32768 && (ld * es) % 16 == 0 && aligned(gate, 16) && aligned(up, 16) &&
                     aligned(xq, 8);
    auto go = [&](auto* gp, auto* upp) {
        using XT = std::remove_const_t<std::remove_pointer_t<decltype(gp)>>;
        if (vec)
            by_shape(m, k, [&](auto cpt, auto nt) {
                silu_mul_quant_kernel<XT, decltype(cpt)::value, decltype(nt)::value>
                    <<<grid, decltype(nt)::value, 0, s>>>(gp, upp, ld, ki, xq, a_scale);
            });
        else
            fused_quant_generic_kernel<XT, false><<<grid, 256, 0, s>>>(gp, upp, nullptr, 0.0f, ld, ki, xq, a_scale);
    };
    if (dtype == NQ_F32) go(static_cast<const float*>(gate), static_cast<const float*>(up));
    else go(static_cast<const _Float16*>(gate), static_cast<const _Float16*>(up));
    return launch_status("silu_mul_quant_i8");
}
