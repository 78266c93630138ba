// Measurement helper, not part of the quantized path: a streaming read of a
// device buffer, so the benchmark can time the floor a decode GEMV of the same
// bytes argues from (one pass over the bytes, 16-byte non-temporal loads as the
// GEMVs issue them, nothing written but one word that the data never selects).
#include <hip/hip_runtime.h>

#include "nq_device.hpp"
#include "nq_internal.hpp"

namespace nq {
namespace {

constexpr int kReadThreads = 256, kReadUnroll = 4;

// Workgroup g reads chunks [g * 1024, g * 1024 + 1024) of 16 bytes: each lane
// issues its 4 loads back to back (chunk index clamped, never predicated, so
// all four are in flight together) and folds them with XOR.
__global__ __launch_bounds__(kReadThreads) void read_probe_kernel(const v4i* __restrict__ p, int64_t chunks,
                                                                  int* __restrict__ sink) {
    const int64_t base = static_cast<int64_t>(blockIdx.x) * kReadThreads * kReadUnroll + threadIdx.x;
    v4i v[kReadUnroll];
#pragma unroll
    for (int u = 0; u < kReadUnroll; ++u) {
        const int64_t c = base + u * kReadThreads;
        v[u] = __builtin_nontemporal_load(p + (c < chunks ? c : chunks - 1));
    }
    int acc = 0;
#pragma unroll
    for (int u = 0; u < kReadUnroll; ++u) acc ^= v[u][0] ^ v[u][1] ^ v[u][2] ^ v[u][3];
    if (acc == 0x5EED1E55 && threadIdx.x == 0) sink[blockIdx.x & 63] = acc;
}

}  // namespace
}  // namespace nq

using namespace nq;

extern "C" nq_status nq_probe_read(const void* p, size_t bytes, int* sink, void* stream) {
    NQ_REQUIRE(p && sink, NQ_BAD_ARG, "probe_read: null pointer");
    NQ_REQUIRE(aligned(p, 16) && bytes % 16 == 0, NQ_BAD_ALIGN, "probe_read: 16-byte aligned whole chunks required");
    if (bytes == 0) return NQ_OK;
    const int64_t chunks = static_cast<int64_t>(bytes / 16);
    const int64_t per = kReadThreads * kReadUnroll;
    read_probe_kernel<<<static_cast<unsigned>((chunks + per - 1) / per), kReadThreads, 0, as_stream(stream)>>>(
        static_cast<const v4i*>(p), chunks, sink);
    return launch_status("read_probe_kernel");
}
