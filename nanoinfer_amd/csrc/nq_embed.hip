// Int8 embedding gather: out[r, c] = codes[ids[r], c] * scale[ids[r]]
// (quant.cpp:121-134, cuda_quant.cu:240-247). The ids arrive as a host array,
// as in the reference; they are range-checked on the host and passed to the
// kernel by value in batches, so the call needs no device allocation or copy.
#include <hip/hip_runtime.h>

#include "nq_device.hpp"
#include "nq_internal.hpp"

namespace nq {
namespace {

constexpr int kIdsPerLaunch = 256;

struct IdBatch {
    int64_t id[kIdsPerLaunch];
};

// One workgroup per gathered row; 16 codes per thread-step when the row is
// 16-byte aligned, scalar otherwise. The multiply is one fp32 product, the same
// single rounding as the reference.
template <typename OT>
__global__ void embedding_q8_kernel(const int8_t* __restrict__ codes, const float* __restrict__ scale,
                                    IdBatch ids, int hidden, OT* __restrict__ out) {
    const int r = blockIdx.x;
    const int64_t id = ids.id[r];
    const int8_t* src = codes + static_cast<size_t>(id) * hidden;
    const float s = scale[id];
    OT* dst = out + static_cast<size_t>(r) * hidden;
    for (int c = threadIdx.x; c < hidden; c += blockDim.x)
        dst[c] = from_f32<OT>(static_cast<float>(src[c]) * s);
}

}  // namespace
}  // namespace nq

using namespace nq;

extern "C" nq_status nq_embedding_q8(const int8_t* codes, const float* scale, int64_t vocab,
                                     int64_t hidden, const int64_t* ids, int64_t n, void* out,
                                     nq_dtype out_dtype, void* stream) {
    NQ_REQUIRE(vocab >= 0 && hidden >= 0 && n >= 0, NQ_BAD_SHAPE, "embedding_q8: negative shape");
    NQ_REQUIRE(hidden <= kMaxIndex && vocab <= kMaxIndex, NQ_BAD_SHAPE, "embedding_q8: shape too large");
    NQ_REQUIRE(dtype_ok(out_dtype), NQ_BAD_ARG, "embedding_q8: unknown out dtype");
    if (n == 0) return NQ_OK;
    NQ_REQUIRE(ids, NQ_BAD_ARG, "embedding_q8: null ids");
    for (int64_t r = 0; r < n; ++r)
        NQ_REQUIRE(ids[r] >= 0 && ids[r] < vocab, NQ_BAD_ARG, "embedding_q8: id out of range");
    if (hidden == 0) return NQ_OK;
    NQ_REQUIRE(codes && scale && out, NQ_BAD_ARG, "embedding_q8: null pointer");
    NQ_REQUIRE(aligned(scale, 4) && aligned(out, dtype_size(out_dtype)), NQ_BAD_ALIGN,
               "embedding_q8: misaligned pointer");
    hipStream_t s = as_stream(stream);
    const int h = static_cast<int>(hidden);
    const int threads = hidden >= 256 ? 256 : 64;
    for (int64_t r0 = 0; r0 < n; r0 += kIdsPerLaunch) {
        const int cnt = static_cast<int>(n - r0 < kIdsPerLaunch ? n - r0 : kIdsPerLaunch);
        IdBatch b{};
        for (int i = 0; i < cnt; ++i) b.id[i] = ids[r0 + i];
        const size_t off = static_cast<size_t>(r0) * hidden;
        if (out_dtype == NQ_F32)
            embedding_q8_kernel<float><<<cnt, threads, 0, s>>>(codes, scale, b, h, static_cast<float*>(out) + off);
        else
            embedding_q8_kernel<_Float16><<<cnt, threads, 0, s>>>(codes, scale, b, h, static_cast<_Float16*>(out) + off);
        if (nq_status st = launch_status("embedding_q8_kernel")) return st;
    }
    return NQ_OK;
}
