// Quantize / pack kernels: per-row int8 (weights and dynamic activations) and
// group-wise int4 nibble packing. All are bit-exact with the reference
// quantizers (quant.cpp:88-108, :179-193, :295-321): the same fp32 absmax and
// divide, round-half-even and clamp; max is order-free so the parallel absmax
// equals the serial scan.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <type_traits>

#include "nq_device.hpp"
#include "nq_internal.hpp"

namespace nq {
namespace {

constexpr int kRowThreads = 256;

// One workgroup per row: absmax over the row (block reduction through LDS),
// scale = absmax / 127, then each thread quantizes its strided elements.
// Used for weights (quantize_q8) and activations (W8A8 act quant).
template <typename XT>
__global__ __launch_bounds__(kRowThreads) void quantize_rows_i8_kernel(
    const XT* __restrict__ x, int8_t* __restrict__ q, float* __restrict__ scale, int k) {
    __shared__ float red[kRowThreads / kWave];
    const int row = blockIdx.x;
    const XT* xr = x + static_cast<size_t>(row) * k;
    int8_t* qr = q + static_cast<size_t>(row) * k;
    const int tid = threadIdx.x;

    float am = 0.0f;
    for (int j = tid; j < k; j += kRowThreads) am = absmax_step(am, to_f32(xr[j]));
    am = wave_absmax(am);
    if ((tid & (kWave - 1)) == 0) red[tid / kWave] = am;
    __syncthreads();
    float absmax = red[0];
#pragma unroll
    for (int w = 1; w < kRowThreads / kWave; ++w) absmax = absmax_step(absmax, red[w]);
    const float s = absmax / 127.0f;
    if (tid == 0) scale[row] = s;
    const RowQuantizer rq(s);
    for (int j = tid; j < k; j += kRowThreads) qr[j] = static_cast<int8_t>(rq.code(to_f32(xr[j]), 127.0f));
}

template <typename ST>
__device__ __forceinline__ void store_scale(ST* p, float s);
template <>
__device__ __forceinline__ void store_scale<float>(float* p, float s) { *p = s; }
template <>
__device__ __forceinline__ void store_scale<_Float16>(_Float16* p, float s) {
    *p = static_cast<_Float16>(s);
}

// Even group: one thread per (row, block). A block starts on an even column, so
// the bytes it packs belong to it alone; a trailing odd column fills only the
// low nibble (quant.cpp:71-75), exactly as the zero-initialised reference buffer.
template <typename ST>
__global__ void quantize_q4g_even_kernel(const float* __restrict__ w, uint8_t* __restrict__ q,
                                         ST* __restrict__ scale, int out, int in, int group,
                                         int blocks) {
    const int64_t t = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (t >= static_cast<int64_t>(out) * blocks) return;
    const int o = static_cast<int>(t / blocks), b = static_cast<int>(t % blocks);
    const float* wr = w + static_cast<size_t>(o) * in;
    uint8_t* row = q + static_cast<size_t>(o) * ((in + 1) / 2);
    const int j0 = b * group, j1 = min(j0 + group, in);
    float am = 0.0f;
    for (int j = j0; j < j1; ++j) am = absmax_step(am, wr[j]);
    const float s = am / 7.0f;
    store_scale(scale + t, s);
    const RowQuantizer rq(s);
    for (int j = j0; j < j1; j += 2) {
        const int lo = static_cast<int>(rq.code(wr[j], 7.0f)) + 8;
        const int hi = (j + 1 < j1) ? static_cast<int>(rq.code(wr[j + 1], 7.0f)) + 8 : 0;
        row[j / 2] = static_cast<uint8_t>(lo | (hi << 4));
    }
}

// Vector path (group = 8 G with G a power of two <= 64, in % 8 == 0): lane t
// owns 8 consecutive columns (two 16-byte loads) of a row whose chunks are
// padded to a multiple of G, so the G lanes of one block are an aligned run of
// a wave; the block absmax is a G-lane shuffle reduction (order-free), and the
// lane writes its 4 packed bytes with one 32-bit store. Lanes past the row's
// end (a partial last block) contribute 0 to the absmax and store nothing.
template <typename ST, int G>
__global__ __launch_bounds__(256) void quantize_q4g_vec_kernel(const float* __restrict__ w, uint32_t* __restrict__ q,
                                                               ST* __restrict__ scale, int out, int in, int blocks,
                                                               int cpr) {
    const int64_t t = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    const bool live = t < static_cast<int64_t>(out) * cpr;
    const int o = live ? static_cast<int>(t / cpr) : 0, cc = live ? static_cast<int>(t % cpr) : 0;
    const bool act = live && cc * 8 < in;
    const f4* src = reinterpret_cast<const f4*>(w + static_cast<size_t>(o) * in + (act ? cc * 8 : 0));
    const f4 a = src[0], b = src[1];
    const float v[8] = {a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
    float am = 0.0f;
#pragma unroll
    for (int j = 0; j < 8; ++j) am = absmax_step(am, v[j]);
    am = act ? am : 0.0f;
    am = group_absmax<G>(am, static_cast<int>(threadIdx.x & 63));
    const float s = am / 7.0f;
    if (!act) return;
    if (cc % G == 0) store_scale(scale + static_cast<size_t>(o) * blocks + cc / G, s);
    const RowQuantizer rq(s);
    uint32_t word = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const uint32_t lo = static_cast<uint32_t>(static_cast<int>(rq.code(v[2 * j], 7.0f)) + 8);
        const uint32_t hi = static_cast<uint32_t>(static_cast<int>(rq.code(v[2 * j + 1], 7.0f)) + 8);
        word |= (lo | (hi << 4)) << (8 * j);
    }
    q[static_cast<size_t>(o) * (in / 8) + cc] = word;
}

// Odd group: one thread per packed byte; each of its two columns recomputes its
// block's absmax (blocks can straddle bytes). The thread owning a block's first
// column writes that block's scale.
template <typename ST>
__global__ void quantize_q4g_odd_kernel(const float* __restrict__ w, uint8_t* __restrict__ q,
                                        ST* __restrict__ scale, int out, int in, int group,
                                        int blocks) {
    const int rb = (in + 1) / 2;
    const int64_t t = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (t >= static_cast<int64_t>(out) * rb) return;
    const int o = static_cast<int>(t / rb), byte = static_cast<int>(t % rb);
    const float* wr = w + static_cast<size_t>(o) * in;
    int nib[2] = {0, 0};
    for (int h = 0; h < 2; ++h) {
        const int j = 2 * byte + h;
        if (j >= in) break;
        const int b = j / group, j0 = b * group, j1 = min(j0 + group, in);
        float am = 0.0f;
        for (int jj = j0; jj < j1; ++jj) am = absmax_step(am, wr[jj]);
        const float s = am / 7.0f;
        if (j == j0) store_scale(scale + static_cast<size_t>(o) * blocks + b, s);
        nib[h] = static_cast<int>(round_clamp(wr[j], s, 7.0f)) + 8;
    }
    q[static_cast<size_t>(o) * rb + byte] = static_cast<uint8_t>(nib[0] | (nib[1] << 4));
}

// ---- activation quant (vectorized) ------------------------------
// One workgroup per row, 8 elements per 16-byte step held in registers between
// the absmax pass and the quantize pass (x is read once).
// HEADS: x is head-major [k / hd, m, hd] (an attention output) and row `row`
// is the concatenation of its heads' row-`row` segments, i.e. the rows of the
// [m, k] matrix its transpose would produce (hd = 8 * epr elements per head).
template <typename XT, int CPT, int NT, bool HEADS = false>
__global__ __launch_bounds__(NT) void act_quant_vec_kernel(const XT* __restrict__ x, int8_t* __restrict__ xq,
                                                           float* __restrict__ a_scale, int m, int k, int epr = 0) {
    __shared__ float red[NT / 64];
    const int tid = threadIdx.x;
    typedef XT v8 __attribute__((ext_vector_type(8)));
    const int row = blockIdx.x, steps = k >> 3;
    const v8* xr = reinterpret_cast<const v8*>(x + static_cast<size_t>(row) * (HEADS ? 8 * epr : k));
    v8 v[CPT];
    float am = 0.0f;
    // Loads are unconditional (indices past the row re-read its last vector and
    // are left out of the absmax), so all CPT of them are in flight together.
#pragma unroll
    for (int c = 0; c < CPT; ++c) {
        const int e = min(tid + c * NT, steps - 1);
        if constexpr (HEADS)
            v[c] = xr[static_cast<size_t>(e / epr) * m * epr + e % epr];
        else
            v[c] = xr[e];
    }
    __builtin_amdgcn_sched_barrier(0);  // keep every load ahead of the absmax math
#pragma unroll
    for (int c = 0; c < CPT; ++c) {
        float a = 0.0f;
#pragma unroll
        for (int j = 0; j < 8; ++j) a = absmax_step(a, to_f32(v[c][j]));
        am = tid + c * NT < steps ? absmax_step(am, a) : am;
    }
    am = wave_absmax(am);
    if ((tid & 63) == 0) red[tid >> 6] = am;
    __syncthreads();
    float a = red[0];
#pragma unroll
    for (int w = 1; w < NT / 64; ++w) a = absmax_step(a, red[w]);
    const float sc = a / 127.0f;
    if (tid == 0) a_scale[row] = sc;
    const RowQuantizer rq(sc);
    typedef int v2i __attribute__((ext_vector_type(2)));
    v2i* qr = reinterpret_cast<v2i*>(xq + static_cast<size_t>(row) * k);
#pragma unroll
    for (int c = 0; c < CPT; ++c) {
        const int e = tid + c * NT;
        if (e < steps) {
            int lo = 0, hi = 0;
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                lo |= (static_cast<int>(rq.code(to_f32(v[c][j]), 127.0f)) & 0xFF) << (8 * j);
                hi |= (static_cast<int>(rq.code(to_f32(v[c][j + 4]), 127.0f)) & 0xFF) << (8 * j);
            }
            qr[e] = v2i{lo, hi};
        }
    }
}

nq_status check_rows(int64_t rows, int64_t cols, const char* who) {
    NQ_REQUIRE(rows >= 0 && cols >= 0, NQ_BAD_SHAPE, "%s: negative shape [%lld, %lld]", who,
               (long long)rows, (long long)cols);
    NQ_REQUIRE(rows <= kMaxIndex && cols <= kMaxIndex && rows * cols <= (int64_t(1) << 40),
               NQ_BAD_SHAPE, "%s: shape [%lld, %lld] exceeds the supported range", who,
               (long long)rows, (long long)cols);
    return NQ_OK;
}

}  // namespace

// Activation quant: the vectorized kernel when k fits it, else the scalar row kernel.
nq_status act_quant(const void* x, nq_dtype xdt, int64_t m, int64_t k, int8_t* xq, float* as,
                    hipStream_t s) {
    // One workgroup per row: for m >= 256, 256 threads with up to 8 vectors of
    // 8 elements each (k <= 16384; several vectors per thread keep more loads
    // in flight and let several rows share a CU), else 1024 threads with up to 8.
    const bool vec = k > 0 && k % 8 == 0 && k <= 8 * 1024 * 8 && aligned(x, 16) && aligned(xq, 8);
    if (vec) {
        const unsigned grid = static_cast<unsigned>(m);
        const int64_t steps = k / 8;
        const int mi = static_cast<int>(m), ki = static_cast<int>(k);
        auto go = [&](auto* xp) {
            using XT = std::remove_const_t<std::remove_pointer_t<decltype(xp)>>;
            // Few rows (m < 256) cannot fill the GPU with 256-thread rows: their
            // per-row latency rules, so they take 1024 threads (the k = 8960 act
            // quant at m = 16: 256 threads 8.0 us, 1024 threads 6.0 us; at m = 2048
            // the opposite, 31 vs 41 us).
            const int64_t per = m >= 256 ? (steps + 255) / 256 : (steps <= 256 ? 1 : 0);
            // Past 1024 vectors per row, 512 threads with 3-4 vectors each (k =
            // 8960 fp16: m = 512 7.1 -> 5.6 us, m = 2048 15.3 -> 14.0 us).
            if (per >= 5 && per <= 8) {
                if ((steps + 511) / 512 == 3)
                    act_quant_vec_kernel<XT, 3, 512><<<grid, 512, 0, s>>>(xp, xq, as, mi, ki);
                else
                    act_quant_vec_kernel<XT, 4, 512><<<grid, 512, 0, s>>>(xp, xq, as, mi, ki);
                return;
            }
            switch (per) {
                case 0: break;
                case 1: act_quant_vec_kernel<XT, 1, 256><<<grid, 256, 0, s>>>(xp, xq, as, mi, ki); return;
                case 2: act_quant_vec_kernel<XT, 2, 256><<<grid, 256, 0, s>>>(xp, xq, as, mi, ki); return;
                case 3: act_quant_vec_kernel<XT, 3, 256><<<grid, 256, 0, s>>>(xp, xq, as, mi, ki); return;
                case 4: act_quant_vec_kernel<XT, 4, 256><<<grid, 256, 0, s>>>(xp, xq, as, mi, ki); return;
                default: break;  // 5..8 took the 512-thread rows above; more: 1024 threads
            }
            switch ((steps + 1023) / 1024) {
                case 1: act_quant_vec_kernel<XT, 1, 1024><<<grid, 1024, 0, s>>>(xp, xq, as, mi, ki); break;
                case 2: act_quant_vec_kernel<XT, 2, 1024><<<grid, 1024, 0, s>>>(xp, xq, as, mi, ki); break;
                case 3: act_quant_vec_kernel<XT, 3, 1024><<<grid, 1024, 0, s>>>(xp, xq, as, mi, ki); break;
                case 4: act_quant_vec_kernel<XT, 4, 1024><<<grid, 1024, 0, s>>>(xp, xq, as, mi, ki); break;
                default: act_quant_vec_kernel<XT, 8, 1024><<<grid, 1024, 0, s>>>(xp, xq, as, mi, ki); break;
            }
        };
        if (xdt == NQ_F32) go(static_cast<const float*>(x));
        else go(static_cast<const _Float16*>(x));
        return launch_status("act_quant_vec_kernel");
    }
    const unsigned grid = static_cast<unsigned>(m);
    if (xdt == NQ_F32)
        quantize_rows_i8_kernel<float><<<grid, kRowThreads, 0, s>>>(static_cast<const float*>(x), xq, as, static_cast<int>(k));
    else
        quantize_rows_i8_kernel<_Float16><<<grid, kRowThreads, 0, s>>>(static_cast<const _Float16*>(x), xq, as, static_cast<int>(k));
    return launch_status("quantize_rows_i8_kernel");
}
}  // namespace nq

using namespace nq;

extern "C" nq_status nq_quantize_q8(const float* w, int64_t out, int64_t in, int8_t* q,
                                    float* scale, void* stream) {
    if (nq_status st = check_rows(out, in, "nq_quantize_q8")) return st;
    if (out == 0) return NQ_OK;
    NQ_REQUIRE(scale && (in == 0 || (w && q)), NQ_BAD_ARG, "nq_quantize_q8: null pointer");
    NQ_REQUIRE(aligned(w, 4) && aligned(scale, 4), NQ_BAD_ALIGN, "nq_quantize_q8: misaligned fp32");
    // The weight quantizer is the activation quantizer's arithmetic
    // (quant.cpp:88-108 and :179-193 both take absmax / 127 and round_clamp).
    return act_quant(w, NQ_F32, out, in, q, scale, as_stream(stream));
}

extern "C" nq_status nq_act_quant_i8_heads(const void* x, nq_dtype x_dtype, int64_t heads, int64_t s,
                                           int64_t head_dim, int8_t* xq, float* a_scale, void* stream) {
    NQ_REQUIRE(heads >= 0 && s >= 0 && head_dim >= 0 && s <= kMaxIndex, NQ_BAD_SHAPE,
               "nq_act_quant_i8_heads: negative shape");
    NQ_REQUIRE(dtype_ok(x_dtype), NQ_BAD_ARG, "nq_act_quant_i8_heads: unknown x dtype %d", int(x_dtype));
    const int64_t k = heads * head_dim;
    NQ_REQUIRE(head_dim % 8 == 0 && k <= 16384 && (heads * s * head_dim) <= (int64_t(1) << 40), NQ_BAD_SHAPE,
               "nq_act_quant_i8_heads: needs head_dim %% 8 == 0 and heads * head_dim <= 16384");
    if (s == 0) return NQ_OK;
    NQ_REQUIRE(a_scale && (k == 0 || (x && xq)), NQ_BAD_ARG, "nq_act_quant_i8_heads: null pointer");
    NQ_REQUIRE(aligned(x, 16) && aligned(xq, 8) && aligned(a_scale, 4), NQ_BAD_ALIGN,
               "nq_act_quant_i8_heads: x must be 16-byte aligned, xq 8-byte aligned");
    if (k == 0) return act_quant(x, x_dtype, s, 0, xq, a_scale, as_stream(stream));
    hipStream_t st = as_stream(stream);
    const unsigned grid = static_cast<unsigned>(s);
    const int mi = static_cast<int>(s), ki = static_cast<int>(k), epr = static_cast<int>(head_dim / 8);
    const int64_t steps = k / 8;
    auto go = [&](auto* xp) {
        using XT = std::remove_const_t<std::remove_pointer_t<decltype(xp)>>;
        switch ((steps + 255) / 256) {
            case 1: act_quant_vec_kernel<XT, 1, 256, true><<<grid, 256, 0, st>>>(xp, xq, a_scale, mi, ki, epr); break;
            case 2: act_quant_vec_kernel<XT, 2, 256, true><<<grid, 256, 0, st>>>(xp, xq, a_scale, mi, ki, epr); break;
            case 3: act_quant_vec_kernel<XT, 3, 256, true><<<grid, 256, 0, st>>>(xp, xq, a_scale, mi, ki, epr); break;
            case 4: act_quant_vec_kernel<XT, 4, 256, true><<<grid, 256, 0, st>>>(xp, xq, a_scale, mi, ki, epr); break;
            default: act_quant_vec_kernel<XT, 8, 256, true><<<grid, 256, 0, st>>>(xp, xq, a_scale, mi, ki, epr); break;
        }
    };
    if (x_dtype == NQ_F32) go(static_cast<const float*>(x));
    else go(static_cast<const _Float16*>(x));
    return launch_status("act_quant_i8_heads");
}

extern "C" nq_status nq_act_quant_i8(const void* x, nq_dtype x_dtype, int64_t m, int64_t k,
                                     int8_t* xq, float* a_scale, void* stream) {
    if (nq_status st = check_rows(m, k, "nq_act_quant_i8")) return st;
    NQ_REQUIRE(dtype_ok(x_dtype), NQ_BAD_ARG, "nq_act_quant_i8: unknown x dtype %d", int(x_dtype));
    if (m == 0) return NQ_OK;
    NQ_REQUIRE(a_scale && (k == 0 || (x && xq)), NQ_BAD_ARG, "nq_act_quant_i8: null pointer");
    NQ_REQUIRE(aligned(x, dtype_size(x_dtype)) && aligned(a_scale, 4), NQ_BAD_ALIGN,
               "nq_act_quant_i8: misaligned pointer");
    return act_quant(x, x_dtype, m, k, xq, a_scale, as_stream(stream));
}

extern "C" nq_status nq_quantize_q4g(const float* w, int64_t out, int64_t in, int64_t group,
                                     uint8_t* q, void* scale, nq_dtype scale_dtype,
                                     void* stream) {
    if (nq_status st = check_rows(out, in, "nq_quantize_q4g")) return st;
    NQ_REQUIRE(group > 0, NQ_BAD_SHAPE, "quantize_q4g: group must be positive");
    NQ_REQUIRE(group <= kMaxIndex, NQ_BAD_SHAPE, "quantize_q4g: group too large");
    NQ_REQUIRE(dtype_ok(scale_dtype), NQ_BAD_ARG, "nq_quantize_q4g: unknown scale dtype");
    if (out == 0 || in == 0) return NQ_OK;
    NQ_REQUIRE(w && q && scale, NQ_BAD_ARG, "nq_quantize_q4g: null pointer");
    NQ_REQUIRE(aligned(w, 4) && aligned(scale, dtype_size(scale_dtype)), NQ_BAD_ALIGN,
               "nq_quantize_q4g: misaligned pointer");
    const int o = static_cast<int>(out), k = static_cast<int>(in), g = static_cast<int>(group);
    const int blocks = static_cast<int>((in + group - 1) / group);
    const int threads = 256;
    hipStream_t s = as_stream(stream);
    const int gl = g / 8;  // lanes per block on the vector path
    if (g % 8 == 0 && gl <= 64 && (gl & (gl - 1)) == 0 && k % 8 == 0 && aligned(w, 16) && aligned(q, 4)) {
        const int cpr = ((k / 8 + gl - 1) / gl) * gl;
        const unsigned grid = static_cast<unsigned>((out * cpr + 255) / 256);
        auto go = [&](auto gtag, auto* sp) {
            constexpr int G = decltype(gtag)::value;
            using ST = std::remove_pointer_t<decltype(sp)>;
            quantize_q4g_vec_kernel<ST, G><<<grid, 256, 0, s>>>(w, reinterpret_cast<uint32_t*>(q), sp, o, k, blocks, cpr);
        };
        auto with_g = [&](auto* sp) {
            switch (gl) {
                case 1: go(std::integral_constant<int, 1>{}, sp); break;
                case 2: go(std::integral_constant<int, 2>{}, sp); break;
                case 4: go(std::integral_constant<int, 4>{}, sp); break;
                case 8: go(std::integral_constant<int, 8>{}, sp); break;
                case 16: go(std::integral_constant<int, 16>{}, sp); break;
                case 32: go(std::integral_constant<int, 32>{}, sp); break;
                default: go(std::integral_constant<int, 64>{}, sp); break;
            }
        };
        if (scale_dtype == NQ_F32) with_g(static_cast<float*>(scale));
        else with_g(static_cast<_Float16*>(scale));
    } else if (g % 2 == 0) {
        const int64_t total = out * blocks;
        const unsigned grid = static_cast<unsigned>((total + threads - 1) / threads);
        if (scale_dtype == NQ_F32)
            quantize_q4g_even_kernel<float><<<grid, threads, 0, s>>>(w, q, static_cast<float*>(scale), o, k, g, blocks);
        else
            quantize_q4g_even_kernel<_Float16><<<grid, threads, 0, s>>>(w, q, static_cast<_Float16*>(scale), o, k, g, blocks);
    } else {
        const int64_t total = out * ((in + 1) / 2);
        const unsigned grid = static_cast<unsigned>((total + threads - 1) / threads);
        if (scale_dtype == NQ_F32)
            quantize_q4g_odd_kernel<float><<<grid, threads, 0, s>>>(w, q, static_cast<float*>(scale), o, k, g, blocks);
        else
            quantize_q4g_odd_kernel<_Float16><<<grid, threads, 0, s>>>(w, q, static_cast<_Float16*>(scale), o, k, g, blocks);
    }
    return launch_status("quantize_q4g_kernel");
}
