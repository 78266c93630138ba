// Weight files in the reference's NIT0 / NIT1 format, read and quantized on the
// device (serialize.hpp:1-23, load_bin serialize.cpp:11-72):
//   "NIT0" | int32 ndim | int32 shape[ndim] | fp32 payload
//   "NIT1" | int32 dtype (0 fp32, 1 bf16) | int32 ndim | int32 shape[ndim] | payload
// little-endian, row-major. The header checks are load_bin's (bad magic, unknown
// dtype, negative ndim or dim, short payload, trailing bytes), each an
// NQ_IO_ERROR with the same reason in its message.
//
// The reference inflates a bf16 payload to fp32 on the host (bits << 16, exact)
// and quantizes there (quant.cpp:88-108, :295-321) before uploading codes
// (cuda_quant.cu:345-388). Here the raw payload goes to the device in row
// chunks (bf16 at half the bytes), a kernel inflates bf16 exactly the same way,
// and the device quantizers (nq_quantize_q8 / nq_quantize_q4g, bit-exact with
// the reference) write the codes and scales straight into the caller's
// buffers. Chunks of at most 64 MiB of payload keep host and device staging
// bounded for vocabulary-sized matrices; two pinned host buffers let the file
// read of one chunk overlap the upload and quantization of the previous one.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cerrno>
#include <cstring>

#include "nq_internal.hpp"

namespace nq {
namespace {

__global__ void bf16_to_f32_kernel(const uint16_t* __restrict__ in, float* __restrict__ out, int64_t n) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i < n) out[i] = __builtin_bit_cast(float, static_cast<uint32_t>(in[i]) << 16);
}

struct NitFile {
    FILE* f = nullptr;
    int32_t dtype = 0;  // 0 fp32, 1 bf16
    int32_t ndim = 0;
    int64_t shape[8] = {};
    int64_t numel = 1;
    ~NitFile() {
        if (f) std::fclose(f);
    }
    size_t esz() const { return dtype == 1 ? 2 : 4; }
};

// Opens and validates a NIT file; on success the stream sits at the payload.
nq_status nit_open(const char* path, NitFile& n) {
    NQ_REQUIRE(path, NQ_BAD_ARG, "nit: null path");
    n.f = std::fopen(path, "rb");
    NQ_REQUIRE(n.f, NQ_IO_ERROR, "nit: cannot open %s (%s)", path, std::strerror(errno));
    char magic[4];
    NQ_REQUIRE(std::fread(magic, 1, 4, n.f) == 4, NQ_IO_ERROR, "nit: bad magic in %s", path);
    const bool v1 = std::memcmp(magic, "NIT1", 4) == 0;
    NQ_REQUIRE(v1 || std::memcmp(magic, "NIT0", 4) == 0, NQ_IO_ERROR, "nit: bad magic in %s", path);
    if (v1) {
        NQ_REQUIRE(std::fread(&n.dtype, 4, 1, n.f) == 1, NQ_IO_ERROR, "nit: short read in %s", path);
        NQ_REQUIRE(n.dtype == 0 || n.dtype == 1, NQ_IO_ERROR, "nit: unknown dtype %d in %s", n.dtype, path);
    }
    NQ_REQUIRE(std::fread(&n.ndim, 4, 1, n.f) == 1, NQ_IO_ERROR, "nit: short read in %s", path);
    NQ_REQUIRE(n.ndim >= 0, NQ_IO_ERROR, "nit: negative ndim in %s", path);
    NQ_REQUIRE(n.ndim <= 8, NQ_IO_ERROR, "nit: %d dims in %s (at most 8 supported)", n.ndim, path);
    for (int i = 0; i < n.ndim; ++i) {
        int32_t d = 0;
        NQ_REQUIRE(std::fread(&d, 4, 1, n.f) == 1, NQ_IO_ERROR, "nit: short read in %s", path);
        NQ_REQUIRE(d >= 0, NQ_IO_ERROR, "nit: negative shape dim in %s", path);
        NQ_REQUIRE(d == 0 || n.numel <= (int64_t(1) << 40) / d, NQ_IO_ERROR, "nit: shape too large in %s", path);
        n.shape[i] = d;
        n.numel *= d;
    }
    const long start = std::ftell(n.f);
    NQ_REQUIRE(start >= 0 && std::fseek(n.f, 0, SEEK_END) == 0, NQ_IO_ERROR, "nit: cannot seek in %s", path);
    const long end = std::ftell(n.f);
    const int64_t need = n.numel * static_cast<int64_t>(n.esz());
    NQ_REQUIRE(end - start >= need, NQ_IO_ERROR, "nit: short read in %s", path);
    NQ_REQUIRE(end - start == need, NQ_IO_ERROR, "nit: trailing bytes (shape/data mismatch) in %s", path);
    NQ_REQUIRE(std::fseek(n.f, start, SEEK_SET) == 0, NQ_IO_ERROR, "nit: cannot seek in %s", path);
    return NQ_OK;
}

// Streams the payload (`total` elements) to the device as fp32 in chunks of at
// most `chunk` elements and calls consume(dev_f32, first, count) on the stream
// for each chunk.
template <typename Fn>
nq_status nit_stream(NitFile& n, const char* path, int64_t total, int64_t chunk, hipStream_t s, Fn&& consume) {
    if (total == 0) return NQ_OK;
    const size_t esz = n.esz();
    const size_t chunk_elems = static_cast<size_t>(std::min(total, chunk));
    void* host[2] = {nullptr, nullptr};
    hipEvent_t done[2] = {nullptr, nullptr};
    void* dev_raw = nullptr;
    float* dev_f32 = nullptr;
    nq_status st = NQ_OK;
    auto hip_ok = [&](hipError_t e, const char* what) {
        if (e == hipSuccess) return true;
        st = fail(NQ_HIP_ERROR, "nit: %s: %s", what, hipGetErrorString(e));
        return false;
    };
    bool ok = hip_ok(hipHostMalloc(&host[0], chunk_elems * esz, hipHostMallocDefault), "hipHostMalloc") &&
              hip_ok(hipHostMalloc(&host[1], chunk_elems * esz, hipHostMallocDefault), "hipHostMalloc") &&
              hip_ok(hipEventCreateWithFlags(&done[0], hipEventDisableTiming), "hipEventCreate") &&
              hip_ok(hipEventCreateWithFlags(&done[1], hipEventDisableTiming), "hipEventCreate") &&
              hip_ok(hipMalloc(reinterpret_cast<void**>(&dev_f32), chunk_elems * 4), "hipMalloc");
    if (ok && esz == 2) ok = hip_ok(hipMalloc(&dev_raw, chunk_elems * 2), "hipMalloc");
    for (int64_t e0 = 0, c = 0; ok && e0 < total; e0 += chunk, ++c) {
        const size_t ne = static_cast<size_t>(std::min(chunk, total - e0));
        const int b = static_cast<int>(c & 1);
        // the upload that last read this pinned buffer has finished
        if (c >= 2 && !hip_ok(hipEventSynchronize(done[b]), "hipEventSynchronize")) break;
        if (std::fread(host[b], esz, ne, n.f) != ne) {
            st = fail(NQ_IO_ERROR, "nit: short read in %s", path);
            break;
        }
        void* dst = esz == 2 ? dev_raw : static_cast<void*>(dev_f32);
        if (!hip_ok(hipMemcpyAsync(dst, host[b], ne * esz, hipMemcpyHostToDevice, s), "hipMemcpyAsync") ||
            !hip_ok(hipEventRecord(done[b], s), "hipEventRecord"))
            break;
        if (esz == 2) {
            const unsigned grid = static_cast<unsigned>((ne + 255) / 256);
            bf16_to_f32_kernel<<<grid, 256, 0, s>>>(static_cast<const uint16_t*>(dev_raw), dev_f32,
                                                   static_cast<int64_t>(ne));
            if ((st = launch_status("nit bf16 inflate")) != NQ_OK) break;
        }
        if ((st = consume(static_cast<const float*>(dev_f32), e0, static_cast<int64_t>(ne))) != NQ_OK) break;
    }
    // The staging buffers are released only after the stream has drained.
    const hipError_t sync = hipStreamSynchronize(s);
    if (st == NQ_OK && sync != hipSuccess) st = fail(NQ_HIP_ERROR, "nit: hipStreamSynchronize: %s", hipGetErrorString(sync));
    for (int i = 0; i < 2; ++i) {
        if (host[i]) (void)hipHostFree(host[i]);
        if (done[i]) (void)hipEventDestroy(done[i]);
    }
    if (dev_raw) (void)hipFree(dev_raw);
    if (dev_f32) (void)hipFree(dev_f32);
    return st;
}

constexpr int64_t kChunkBytes = int64_t(64) << 20;

// Whole rows per chunk, a multiple of 16 rows (keeps sub-buffer offsets of the
// codes and scales as aligned as their bases).
int64_t row_chunk(int64_t rows, int64_t cols, size_t esz) {
    const int64_t r = std::max<int64_t>(16, kChunkBytes / std::max<int64_t>(1, cols * static_cast<int64_t>(esz)) / 16 * 16);
    return std::min(rows, r) * cols;
}

nq_status nit_expect_2d(const NitFile& n, const char* path, int64_t out, int64_t in) {
    NQ_REQUIRE(n.ndim == 2 && n.shape[0] == out && n.shape[1] == in, NQ_BAD_SHAPE,
               "nit: %s holds a %d-d tensor, expected [%lld, %lld]", path, n.ndim, (long long)out, (long long)in);
    return NQ_OK;
}

}  // namespace
}  // namespace nq

using namespace nq;

extern "C" nq_status nq_nit_info(const char* path, int32_t* dtype, int32_t* ndim, int64_t* shape, int32_t max_dims) {
    NitFile n;
    if (nq_status st = nit_open(path, n)) return st;
    NQ_REQUIRE(n.ndim <= max_dims, NQ_BAD_ARG, "nit_info: %s has %d dims, room for %d", path, n.ndim, max_dims);
    if (dtype) *dtype = n.dtype;
    if (ndim) *ndim = n.ndim;
    for (int i = 0; i < n.ndim; ++i)
        if (shape) shape[i] = n.shape[i];
    return NQ_OK;
}

extern "C" nq_status nq_nit_load_f32(const char* path, float* dst, int64_t numel, void* stream) {
    NitFile n;
    if (nq_status st = nit_open(path, n)) return st;
    NQ_REQUIRE(n.numel == numel, NQ_BAD_SHAPE, "nit_load_f32: %s holds %lld elements, expected %lld", path,
               (long long)n.numel, (long long)numel);
    NQ_REQUIRE(numel == 0 || dst, NQ_BAD_ARG, "nit_load_f32: null destination");
    NQ_REQUIRE(aligned(dst, 4), NQ_BAD_ALIGN, "nit_load_f32: misaligned destination");
    hipStream_t s = as_stream(stream);
    return nit_stream(n, path, numel, kChunkBytes / 4, s, [&](const float* src, int64_t e0, int64_t ne) -> nq_status {
        const hipError_t e = hipMemcpyAsync(dst + e0, src, static_cast<size_t>(ne) * 4, hipMemcpyDeviceToDevice, s);
        return e == hipSuccess ? NQ_OK : fail(NQ_HIP_ERROR, "nit_load_f32: hipMemcpyAsync: %s", hipGetErrorString(e));
    });
}

extern "C" nq_status nq_nit_load_q8(const char* path, int8_t* q, float* scale, int64_t out, int64_t in,
                                    void* stream) {
    NitFile n;
    if (nq_status st = nit_open(path, n)) return st;
    if (nq_status st = nit_expect_2d(n, path, out, in)) return st;
    hipStream_t s = as_stream(stream);
    if (out == 0 || in == 0) return nq_quantize_q8(nullptr, out, in, q, scale, stream);
    return nit_stream(n, path, out * in, row_chunk(out, in, n.esz()), s,
                      [&](const float* src, int64_t e0, int64_t ne) -> nq_status {
                          const int64_t r0 = e0 / in;
                          return nq_quantize_q8(src, ne / in, in, q + r0 * in, scale + r0, stream);
                      });
}

extern "C" nq_status nq_nit_load_q4g(const char* path, uint8_t* q, void* scale, nq_dtype scale_dtype, int64_t group,
                                     int64_t out, int64_t in, void* stream) {
    NitFile n;
    if (nq_status st = nit_open(path, n)) return st;
    if (nq_status st = nit_expect_2d(n, path, out, in)) return st;
    NQ_REQUIRE(group > 0, NQ_BAD_ARG, "nit_load_q4g: group must be positive");
    NQ_REQUIRE(dtype_ok(scale_dtype), NQ_BAD_ARG, "nit_load_q4g: unknown scale dtype");
    hipStream_t s = as_stream(stream);
    if (out == 0 || in == 0) return nq_quantize_q4g(nullptr, out, in, group, q, scale, scale_dtype, stream);
    const int64_t qrow = (in + 1) / 2, srow = (in + group - 1) / group;
    return nit_stream(n, path, out * in, row_chunk(out, in, n.esz()), s,
                      [&](const float* src, int64_t e0, int64_t ne) -> nq_status {
                          const int64_t r0 = e0 / in;
                          char* sp = static_cast<char*>(scale) + static_cast<size_t>(r0 * srow) * dtype_size(scale_dtype);
                          return nq_quantize_q4g(src, ne / in, in, group, q + r0 * qrow, sp, scale_dtype, stream);
                      });
}
