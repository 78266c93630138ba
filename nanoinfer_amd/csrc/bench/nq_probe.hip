// Measurement helper for bench.py, built into libnq_bench.so (not the product
// library): a streaming read of a device buffer, the floor a decode GEMV of the
// same bytes argues from. One pass over the bytes with 16-byte non-temporal
// loads, as the GEMVs issue them; optionally `out_bytes` written at the end (one
// 16-byte store per lane of the first out_bytes / 16 lanes of the grid), the
// shape of a GEMV's y store. Nothing else is written but one word that the
// data never selects.
#include <hip/hip_runtime.h>

#include <cstdint>

#include "../../../include/nq_bench.h"

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));

// Workgroup g reads chunks [g * T * U, (g + 1) * T * U) of 16 bytes: each lane
// issues its U loads back to back (chunk index clamped, never predicated, so
// all U are in flight together) and folds them with XOR.
template <int T, int U>
__global__ __launch_bounds__(T) void read_probe_kernel(const v4i* __restrict__ p, int64_t chunks,
                                                       v4i* __restrict__ out, int64_t out_chunks,
                                                       int* __restrict__ sink) {
    const int64_t base = static_cast<int64_t>(blockIdx.x) * T * U + threadIdx.x;
    v4i v[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const int64_t c = base + u * T;
        v[u] = __builtin_nontemporal_load(p + (c < chunks ? c : chunks - 1));
    }
    int acc = 0;
#pragma unroll
    for (int u = 0; u < U; ++u) acc ^= v[u][0] ^ v[u][1] ^ v[u][2] ^ v[u][3];
    const int64_t lane = static_cast<int64_t>(blockIdx.x) * T + threadIdx.x;
    if (lane < out_chunks) out[lane] = v4i{acc, acc, acc, acc};
    if (acc == 0x5EED1E55 && threadIdx.x == 0) sink[blockIdx.x & 63] = acc;
}

template <int T, int U>
int launch(const void* p, int64_t chunks, void* out, int64_t out_chunks, int* sink, hipStream_t s) {
    const int64_t per = static_cast<int64_t>(T) * U;
    read_probe_kernel<T, U><<<static_cast<unsigned>((chunks + per - 1) / per), T, 0, s>>>(
        static_cast<const v4i*>(p), chunks, static_cast<v4i*>(out), out_chunks, sink);
    return hipGetLastError() == hipSuccess ? 0 : 3;
}

}  // namespace

extern "C" int nq_probe_read_cfg(const void* p, size_t bytes, int threads, int loads_per_lane, void* out,
                                 size_t out_bytes, int* sink, void* stream) {
    if (!p || !sink || (out_bytes && !out)) return 4;
    if (reinterpret_cast<uintptr_t>(p) % 16 || bytes % 16 || reinterpret_cast<uintptr_t>(out) % 16 ||
        out_bytes % 16)
        return 2;
    if (bytes == 0) return 0;
    const int64_t chunks = static_cast<int64_t>(bytes / 16), oc = static_cast<int64_t>(out_bytes / 16);
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    switch (threads * 100 + loads_per_lane) {
        case 25601: return launch<256, 1>(p, chunks, out, oc, sink, s);
        case 25602: return launch<256, 2>(p, chunks, out, oc, sink, s);
        case 25604: return launch<256, 4>(p, chunks, out, oc, sink, s);
        case 25608: return launch<256, 8>(p, chunks, out, oc, sink, s);
        case 51201: return launch<512, 1>(p, chunks, out, oc, sink, s);
        case 51202: return launch<512, 2>(p, chunks, out, oc, sink, s);
        case 51204: return launch<512, 4>(p, chunks, out, oc, sink, s);
        case 51208: return launch<512, 8>(p, chunks, out, oc, sink, s);
        case 102401: return launch<1024, 1>(p, chunks, out, oc, sink, s);
        case 102402: return launch<1024, 2>(p, chunks, out, oc, sink, s);
        case 102404: return launch<1024, 4>(p, chunks, out, oc, sink, s);
        default: return 4;
    }
}

extern "C" int nq_probe_read(const void* p, size_t bytes, int* sink, void* stream) {
    return nq_probe_read_cfg(p, bytes, 256, 4, nullptr, 0, sink, stream);
}
