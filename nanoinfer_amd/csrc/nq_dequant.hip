// Weight dequantize on the device: the inverse of the two quantizers, one
// multiply per element exactly as the reference's test helpers compute it.
//   dequantize_q8  (quant.cpp:110-119):  w[o,j] = float(q[o,j]) * scale[o]
//   dequantize_q4g (quant.cpp:323-335):  w[o,j] = float(nib(o,j) - 8) * scale[o, j / group]
// Both are HBM-bound element maps (read 1 or 1/2 byte of codes, write 4 or 2
// bytes per element). A thread owns 8 consecutive elements of one row when the
// row length is a multiple of 8 (one 8-byte / 4-byte code load, two 16-byte fp32
// stores or one 16-byte fp16 store); other shapes take the per-element kernel.
#include <hip/hip_runtime.h>

#include "nq_device.hpp"
#include "nq_internal.hpp"

namespace nq {
namespace {

constexpr int kThreads = 256;

template <typename OT>
__device__ __forceinline__ void store8(OT* dst, const float (&v)[8]);
template <>
__device__ __forceinline__ void store8<float>(float* dst, const float (&v)[8]) {
    reinterpret_cast<f4*>(dst)[0] = f4{v[0], v[1], v[2], v[3]};
    reinterpret_cast<f4*>(dst)[1] = f4{v[4], v[5], v[6], v[7]};
}
template <>
__device__ __forceinline__ void store8<_Float16>(_Float16* dst, const float (&v)[8]) {
    typedef _Float16 h8 __attribute__((ext_vector_type(8)));
    h8 o;
#pragma unroll
    for (int i = 0; i < 8; ++i) o[i] = from_f32<_Float16>(v[i]);
    *reinterpret_cast<h8*>(dst) = o;
}

// q8, in % 8 == 0: chunk c covers elements 8c .. 8c+7 of the flattened [out, in].
template <typename OT>
__global__ __launch_bounds__(kThreads) void dequant_q8_vec_kernel(const int8_t* __restrict__ q,
                                                                  const float* __restrict__ scale,
                                                                  int64_t chunks, int chunks_per_row,
                                                                  OT* __restrict__ w) {
    const int64_t c = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
    if (c >= chunks) return;
    const float s = scale[c / chunks_per_row];
    const uint2 b = reinterpret_cast<const uint2*>(q)[c];
    float v[8];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        v[i] = static_cast<float>(static_cast<int8_t>(b.x >> (8 * i))) * s;
        v[4 + i] = static_cast<float>(static_cast<int8_t>(b.y >> (8 * i))) * s;
    }
    store8<OT>(w + c * 8, v);
}

template <typename OT>
__global__ __launch_bounds__(kThreads) void dequant_q8_any_kernel(const int8_t* __restrict__ q,
                                                                  const float* __restrict__ scale,
                                                                  int64_t total, int64_t in,
                                                                  OT* __restrict__ w) {
    const int64_t e = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
    if (e >= total) return;
    w[e] = from_f32<OT>(static_cast<float>(q[e]) * scale[e / in]);
}

template <typename ST>
__device__ __forceinline__ float load_scale(const ST* s, int64_t i) { return to_f32(s[i]); }

// q4g, in % 8 == 0: a row is in / 2 bytes, so chunk c (8 elements) is the
// 4-byte word c of the packed codes; element 2i is the low nibble of byte i.
template <typename ST, typename OT>
__global__ __launch_bounds__(kThreads) void dequant_q4g_vec_kernel(const uint8_t* __restrict__ q,
                                                                   const ST* __restrict__ scale,
                                                                   int64_t chunks, int chunks_per_row,
                                                                   int blocks, int group,
                                                                   OT* __restrict__ w) {
    const int64_t c = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
    if (c >= chunks) return;
    const int64_t row = c / chunks_per_row;
    const int j0 = static_cast<int>(c - row * chunks_per_row) * 8;
    const uint32_t b = reinterpret_cast<const uint32_t*>(q)[c];
    const ST* srow = scale + row * blocks;
    float v[8];
    // The 8 columns span at most a few groups; look each scale up once per group run.
    int blk = j0 / group;
    int64_t next = static_cast<int64_t>(blk + 1) * group;
    float s = load_scale(srow, blk);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        if (j0 + i >= next) {
            blk = (j0 + i) / group;
            next = static_cast<int64_t>(blk + 1) * group;
            s = load_scale(srow, blk);
        }
        const int nib = static_cast<int>((b >> (4 * i)) & 0xF);
        v[i] = static_cast<float>(nib - 8) * s;
    }
    store8<OT>(w + c * 8, v);
}

template <typename ST, typename OT>
__global__ __launch_bounds__(kThreads) void dequant_q4g_any_kernel(const uint8_t* __restrict__ q,
                                                                   const ST* __restrict__ scale,
                                                                   int64_t total, int64_t in, int64_t row_bytes,
                                                                   int64_t blocks, int64_t group,
                                                                   OT* __restrict__ w) {
    const int64_t e = static_cast<int64_t>(blockIdx.x) * kThreads + threadIdx.x;
    if (e >= total) return;
    const int64_t o = e / in, j = e - o * in;
    const uint8_t byte = q[o * row_bytes + (j >> 1)];
    const int nib = (j & 1) ? (byte >> 4) : (byte & 0xF);
    w[e] = from_f32<OT>(static_cast<float>(nib - 8) * load_scale(scale, o * blocks + j / group));
}

inline unsigned grid_for(int64_t items) { return static_cast<unsigned>((items + kThreads - 1) / kThreads); }

}  // namespace
}  // namespace nq

using namespace nq;

extern "C" nq_status nq_dequantize_q8(const int8_t* q, const float* scale, int64_t out, int64_t in, void* w,
                                      nq_dtype w_dtype, void* stream) {
    NQ_REQUIRE(out >= 0 && in >= 0, NQ_BAD_SHAPE, "dequantize_q8: negative shape");
    NQ_REQUIRE(out <= kMaxIndex && in <= kMaxIndex && out * in <= (kMaxIndex + 1) * 4, NQ_BAD_SHAPE, "dequantize_q8: shape too large");
    NQ_REQUIRE(dtype_ok(w_dtype), NQ_BAD_ARG, "dequantize_q8: unknown output dtype");
    if (out == 0 || in == 0) return NQ_OK;
    NQ_REQUIRE(q && scale && w, NQ_BAD_ARG, "dequantize_q8: null pointer");
    NQ_REQUIRE(aligned(scale, 4) && aligned(w, dtype_size(w_dtype)), NQ_BAD_ALIGN,
               "dequantize_q8: misaligned pointer");
    hipStream_t s = as_stream(stream);
    const int64_t total = out * in;
    const bool vec = in % 8 == 0 && aligned(q, 8) && aligned(w, 16);
    if (vec) {
        const int64_t chunks = total / 8;
        const int cpr = static_cast<int>(in / 8);
        if (w_dtype == NQ_F32)
            dequant_q8_vec_kernel<float><<<grid_for(chunks), kThreads, 0, s>>>(q, scale, chunks, cpr,
                                                                               static_cast<float*>(w));
        else
            dequant_q8_vec_kernel<_Float16><<<grid_for(chunks), kThreads, 0, s>>>(q, scale, chunks, cpr,
                                                                                  static_cast<_Float16*>(w));
    } else if (w_dtype == NQ_F32) {
        dequant_q8_any_kernel<float><<<grid_for(total), kThreads, 0, s>>>(q, scale, total, in, static_cast<float*>(w));
    } else {
        dequant_q8_any_kernel<_Float16><<<grid_for(total), kThreads, 0, s>>>(q, scale, total, in,
                                                                             static_cast<_Float16*>(w));
    }
    return launch_status("dequantize_q8");
}

namespace {
template <typename ST, typename OT>
void launch_q4g(const uint8_t* q, const void* scale, int64_t out, int64_t in, int64_t group, void* w, bool vec,
                hipStream_t s) {
    const int64_t total = out * in, blocks = (in + group - 1) / group;
    const ST* sc = static_cast<const ST*>(scale);
    OT* dst = static_cast<OT*>(w);
    if (vec) {
        const int64_t chunks = total / 8;
        dequant_q4g_vec_kernel<ST, OT><<<grid_for(chunks), kThreads, 0, s>>>(
            q, sc, chunks, static_cast<int>(in / 8), static_cast<int>(blocks), static_cast<int>(group), dst);
    } else {
        dequant_q4g_any_kernel<ST, OT><<<grid_for(total), kThreads, 0, s>>>(q, sc, total, in, (in + 1) / 2, blocks,
                                                                            group, dst);
    }
}
}  // namespace

extern "C" nq_status nq_dequantize_q4g(const uint8_t* q, const void* scale, nq_dtype scale_dtype, int64_t group,
                                       int64_t out, int64_t in, void* w, nq_dtype w_dtype, void* stream) {
    NQ_REQUIRE(out >= 0 && in >= 0, NQ_BAD_SHAPE, "dequantize_q4g: negative shape");
    NQ_REQUIRE(group > 0, NQ_BAD_SHAPE, "dequantize_q4g: group must be positive");
    NQ_REQUIRE(out <= kMaxIndex && in <= kMaxIndex && out * in <= (kMaxIndex + 1) * 4, NQ_BAD_SHAPE, "dequantize_q4g: shape too large");
    NQ_REQUIRE(dtype_ok(w_dtype) && dtype_ok(scale_dtype), NQ_BAD_ARG, "dequantize_q4g: unknown dtype");
    if (out == 0 || in == 0) return NQ_OK;
    NQ_REQUIRE(q && scale && w, NQ_BAD_ARG, "dequantize_q4g: null pointer");
    NQ_REQUIRE(aligned(scale, dtype_size(scale_dtype)) && aligned(w, dtype_size(w_dtype)), NQ_BAD_ALIGN,
               "dequantize_q4g: misaligned pointer");
    const bool vec = in % 8 == 0 && aligned(q, 4) && aligned(w, 16) && group <= kMaxIndex;
    hipStream_t s = as_stream(stream);
    if (scale_dtype == NQ_F32) {
        if (w_dtype == NQ_F32) launch_q4g<float, float>(q, scale, out, in, group, w, vec, s);
        else launch_q4g<float, _Float16>(q, scale, out, in, group, w, vec, s);
    } else {
        if (w_dtype == NQ_F32) launch_q4g<_Float16, float>(q, scale, out, in, group, w, vec, s);
        else launch_q4g<_Float16, _Float16>(q, scale, out, in, group, w, vec, s);
    }
    return launch_status("dequantize_q4g");
}
