// Weight-only Q8 / Q4G linears for batched activations (m > 8) on the fp16
// matrix cores: the reference runs these as fp32 dot products per output
// (quant.cpp:136-163, :337-389; its CUDA tiled Q8 kernel cuda_quant.cu:165-204
// is the m > 16 counterpart). Codes are converted to fp16 exactly in registers
// and multiplied with fp16 activations by v_mfma_f32_16x16x32_f16 (fp32
// accumulation); fp32 activations are split into an fp16 high part and an fp16
// remainder, two MFMAs, so they keep ~22 bits.
//
// Operands: A = activations (16 rows of m), B = weights (16 rows of n), so a
// lane's four results share one weight row (n = lane % 16) and that row's scale.
// One MFMA covers one 32-column chunk of K: lane quarter q supplies columns
// 8q..8q+7 of it. For Q4G every chunk lies in one group (group % 32 == 0), so
// the MFMA starts from zero and the group scale is applied to its fp32 result
// before accumulation, as the reference scales each block sum (quant.cpp:378-
// 386). For Q8 the row scale is applied once in the epilogue (quant.cpp:155-161).
// Inside a lane's 8 columns the pairs are ordered (c, c+4): the int4 nibble
// trick produces them that way (cf. the decode GEMV) and the activations are
// permuted to match; the sum over a chunk is order-independent.
//
// Waves interleave chunks of K with a 4-deep prefetch ring of raw buffer loads
// (out-of-range rows and chunks read zeros); the per-wave partial tiles are
// reduced through LDS in wave order, so results are deterministic.
#include <hip/hip_runtime.h>

#include <type_traits>

#include "nq_device.hpp"
#include "nq_internal.hpp"

namespace nq {
namespace {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
constexpr int kWqRing = 4, kOob = 0x7FFFFFF0;
// Waves per workgroup: 16 for one 16-row tile of x (more loads in flight per
// CU), 8 for larger tiles (their prefetch ring needs up to 256 VGPRs).
template <int TM>
constexpr int wq_waves() { return TM == 1 ? 16 : 8; }

// Activation fragment of one chunk: 8 values of one row, as fp16 pairs (c, c+4).
template <typename XT>
struct XFrag;
template <>
struct XFrag<_Float16> {
    v4i raw;  // 8 halves
    __device__ __forceinline__ void load(__amdgpu_buffer_rsrc_t rs, int off) {
        raw = __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(rs, off, 0, 0));
    }
    __device__ __forceinline__ void operands(h8& hi, h8& lo) const {
        const h8 v = __builtin_bit_cast(h8, raw);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            hi[2 * j] = v[j];
            hi[2 * j + 1] = v[j + 4];
        }
        lo = h8{};
    }
};
template <>
struct XFrag<float> {
    v4i a, b;  // 8 floats
    __device__ __forceinline__ void load(__amdgpu_buffer_rsrc_t rs, int off) {
        a = __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(rs, off, 0, 0));
        b = __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(rs, off == kOob ? kOob : off + 16, 0, 0));
    }
    __device__ __forceinline__ void operands(h8& hi, h8& lo) const {
        const f4 fa = __builtin_bit_cast(f4, a), fb = __builtin_bit_cast(f4, b);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const float v0 = fa[j], v1 = fb[j];  // columns j and j + 4
            const _Float16 h0 = static_cast<_Float16>(v0), h1 = static_cast<_Float16>(v1);
            hi[2 * j] = h0;
            hi[2 * j + 1] = h1;
            lo[2 * j] = static_cast<_Float16>(v0 - static_cast<float>(h0));
            lo[2 * j + 1] = static_cast<_Float16>(v1 - static_cast<float>(h1));
        }
    }
};

// Weight fragment of one chunk: 8 codes of one row as fp16 pairs (c, c+4).
template <bool Q4>
struct WFrag;
template <>
struct WFrag<true> {  // 8 nibbles = one dword, nibble e = column e
    int w;
    __device__ __forceinline__ void load(__amdgpu_buffer_rsrc_t rs, int off) {
        w = __builtin_amdgcn_raw_buffer_load_b32(rs, off, 0, 0);
    }
    __device__ __forceinline__ h8 codes() const {
        const h2 off = {static_cast<_Float16>(-1032.0f), static_cast<_Float16>(-1032.0f)};
        const unsigned u = static_cast<unsigned>(w);
        h8 r;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const h2 p = __builtin_bit_cast(h2, ((u >> (4 * j)) & 0x000F000Fu) | 0x64006400u) + off;
            r[2 * j] = p[0];
            r[2 * j + 1] = p[1];
        }
        return r;
    }
};
template <>
struct WFrag<false> {  // 8 int8 codes = two dwords, byte t of dword d = column 4d + t
    int w0, w1;
    __device__ __forceinline__ void load(__amdgpu_buffer_rsrc_t rs, int off) {
        typedef int v2i __attribute__((ext_vector_type(2)));
        const v2i v = __builtin_bit_cast(v2i, __builtin_amdgcn_raw_buffer_load_b64(rs, off, 0, 0));
        w0 = v[0];
        w1 = v[1];
    }
    __device__ __forceinline__ h8 codes() const {
        // (byte t of w0, byte t of w1) into the low bytes of two halves; XOR with
        // 0x6480 gives the fp16 value 1024 + (code + 128) exactly; -1152 -> code.
        const h2 off = {static_cast<_Float16>(-1152.0f), static_cast<_Float16>(-1152.0f)};
        h8 r;
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            const unsigned sel = 0x0C000C00u | static_cast<unsigned>(t) | (static_cast<unsigned>(4 + t) << 16);
            const unsigned b = __builtin_amdgcn_perm(static_cast<unsigned>(w1), static_cast<unsigned>(w0), sel);
            const h2 p = __builtin_bit_cast(h2, b ^ 0x64806480u) + off;
            r[2 * t] = p[0];
            r[2 * t + 1] = p[1];
        }
        return r;
    }
};

template <bool Q4, int TM, int TN, typename XT, typename YT, typename ST>
__global__ __launch_bounds__(wq_waves<TM>() * 64) void gemm_wq_kernel(
    const XT* __restrict__ x, const uint8_t* __restrict__ wq, const ST* __restrict__ scale,
    const float* __restrict__ bias, YT* __restrict__ y, int m, int n, int k, int group) {
    constexpr int kWqWaves = wq_waves<TM>();
    __shared__ f4 part[kWqWaves][TM][TN][64];
    // group / 32 is a power of two (checked on the host): chunk c uses group c >> gsh.
    const int gsh = Q4 ? __builtin_ctz(static_cast<unsigned>(group >> 5)) : 0;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int r = lane & 15, q = lane >> 4;
    const int n0 = blockIdx.x * (16 * TN);
    // gridDim.y blocks of 64 activation rows
    x += static_cast<size_t>(blockIdx.y) * 64 * k;
    y += static_cast<size_t>(blockIdx.y) * 64 * n;
    m = min(64, m - static_cast<int>(blockIdx.y) * 64);
    const int chunks = k >> 5;
    const int rowb = Q4 ? (k >> 1) : k;  // weight bytes per row
    const int groups = Q4 ? k / group : 1;
    const __amdgpu_buffer_rsrc_t xrs = __builtin_amdgcn_make_buffer_rsrc(const_cast<XT*>(x), 0, m * k * static_cast<int>(sizeof(XT)), 0x00020000);
    const __amdgpu_buffer_rsrc_t wrs = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(wq), 0, n * rowb, 0x00020000);

    const __amdgpu_buffer_rsrc_t srs = __builtin_amdgcn_make_buffer_rsrc(const_cast<ST*>(scale), 0, n * groups * static_cast<int>(sizeof(ST)), 0x00020000);
    int xo[TM], wo[TN], so[TN];
#pragma unroll
    for (int i = 0; i < TM; ++i) {
        const int row = i * 16 + r;
        xo[i] = row < m ? (row * k + 8 * q) * static_cast<int>(sizeof(XT)) : kOob;
    }
#pragma unroll
    for (int j = 0; j < TN; ++j) {
        const int row = n0 + j * 16 + r;
        wo[j] = row < n ? row * rowb + (Q4 ? 4 * q : 8 * q) : kOob;
        so[j] = row < n ? row * groups * static_cast<int>(sizeof(ST)) : kOob;
    }

    // Wave w takes chunks w, w + W, ...; steps = its count.
    const int steps = wave < chunks ? (chunks - wave + kWqWaves - 1) / kWqWaves : 0;
    struct Stage {
        XFrag<XT> xf[TM];
        WFrag<Q4> wf[TN];
        float s[TN];
    };
    auto load = [&](int t, Stage& st) {
        const int c = wave + t * kWqWaves;
        const bool in = t < steps;
#pragma unroll
        for (int i = 0; i < TM; ++i)
            st.xf[i].load(xrs, in && xo[i] != kOob ? xo[i] + c * 32 * static_cast<int>(sizeof(XT)) : kOob);
#pragma unroll
        for (int j = 0; j < TN; ++j) {
            st.wf[j].load(wrs, in && wo[j] != kOob ? wo[j] + c * (Q4 ? 16 : 32) : kOob);
            if constexpr (Q4) {
                const int o = in && so[j] != kOob ? so[j] + (c >> gsh) * static_cast<int>(sizeof(ST)) : kOob;
                if constexpr (sizeof(ST) == 4)
                    st.s[j] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(srs, o, 0, 0));
                else
                    st.s[j] = static_cast<float>(__builtin_bit_cast(_Float16, __builtin_amdgcn_raw_buffer_load_b16(srs, o, 0, 0)));
            }
        }
    };
    f4 acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = f4{0, 0, 0, 0};
    auto compute = [&](const Stage& st) {
        h8 b[TN];
#pragma unroll
        for (int j = 0; j < TN; ++j) b[j] = st.wf[j].codes();
#pragma unroll
        for (int i = 0; i < TM; ++i) {
            h8 hi, lo;
            st.xf[i].operands(hi, lo);
#pragma unroll
            for (int j = 0; j < TN; ++j) {
                if constexpr (Q4) {
                    f4 d = __builtin_amdgcn_mfma_f32_16x16x32_f16(hi, b[j], f4{0, 0, 0, 0}, 0, 0, 0);
                    if constexpr (sizeof(XT) == 4) d = __builtin_amdgcn_mfma_f32_16x16x32_f16(lo, b[j], d, 0, 0, 0);
#pragma unroll
                    for (int v = 0; v < 4; ++v) acc[i][j][v] = __builtin_fmaf(d[v], st.s[j], acc[i][j][v]);
                } else {
                    acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(hi, b[j], acc[i][j], 0, 0, 0);
                    if constexpr (sizeof(XT) == 4) acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(lo, b[j], acc[i][j], 0, 0, 0);
                }
            }
        }
    };
    Stage ring[kWqRing];
#pragma unroll
    for (int p = 0; p < kWqRing; ++p) load(p, ring[p]);
    auto step = [&](int t, auto phase) {
        constexpr int P = decltype(phase)::value;
        compute(ring[P]);
        load(t + kWqRing, ring[P]);
    };
    int t = 0;
    for (; t + kWqRing <= steps; t += kWqRing) {
        step(t, std::integral_constant<int, 0>{});
        step(t + 1, std::integral_constant<int, 1>{});
        step(t + 2, std::integral_constant<int, 2>{});
        step(t + 3, std::integral_constant<int, 3>{});
    }
    if (t < steps) step(t, std::integral_constant<int, 0>{});
    if (t + 1 < steps) step(t + 1, std::integral_constant<int, 1>{});
    if (t + 2 < steps) step(t + 2, std::integral_constant<int, 2>{});

    // Deterministic cross-wave sum: partial tiles to LDS, added in wave order.
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) part[wave][i][j][lane] = acc[i][j];
    __syncthreads();
    for (int e = tid; e < TM * TN * 64 * 4; e += kWqWaves * 64) {
        const int v = e & 3, l = (e >> 2) & 63, ij = e >> 8, i = ij / TN, j = ij % TN;
        const int mm = i * 16 + 4 * (l >> 4) + v, nn = n0 + j * 16 + (l & 15);
        if (mm >= m || nn >= n) continue;
        float s = 0.0f;
        for (int w = 0; w < kWqWaves; ++w) s += part[w][i][j][l][v];
        if constexpr (!Q4) s *= to_f32(scale[nn]);
        y[static_cast<size_t>(mm) * n + nn] = from_f32<YT>(s + (bias ? bias[nn] : 0.0f));
    }
}

template <bool Q4, typename XT, typename YT, typename ST>
nq_status launch_wq(const XT* x, const uint8_t* w, const ST* sc, const float* b, YT* y, int m, int n, int k,
                    int g, hipStream_t s) {
    // 16 weight rows per workgroup, 32 for tall weights at m <= 32 (the LDS
    // tile of per-wave partials stays within 32 KB); 64-row blocks of x over
    // gridDim.y.
    const unsigned mblocks = static_cast<unsigned>((m + 63) / 64);
    auto go = [&](auto tmtag, auto tntag) {
        constexpr int TM = decltype(tmtag)::value, TN = decltype(tntag)::value;
        const dim3 grid(static_cast<unsigned>((n + 16 * TN - 1) / (16 * TN)), mblocks);
        gemm_wq_kernel<Q4, TM, TN, XT, YT, ST><<<grid, wq_waves<TM>() * 64, 0, s>>>(x, w, sc, b, y, m, n, k, g);
    };
    auto with_tn = [&](auto tmtag) {
        if constexpr (decltype(tmtag)::value <= 2) {
            if (n > 4096) return go(tmtag, std::integral_constant<int, 2>{});
        }
        go(tmtag, std::integral_constant<int, 1>{});
    };
    switch (m > 64 ? 4 : (m + 15) / 16) {
        case 1: with_tn(std::integral_constant<int, 1>{}); break;
        case 2: with_tn(std::integral_constant<int, 2>{}); break;
        case 3: with_tn(std::integral_constant<int, 3>{}); break;
        default: with_tn(std::integral_constant<int, 4>{}); break;
    }
    return launch_status("gemm_wq_kernel");
}

}  // namespace

// Whether the MFMA path takes this call (the caller runs GEMV slices otherwise):
// whole 32-column chunks, groups of a power-of-two number of chunks, 16-byte aligned operands and
// 32-bit buffer offsets.
bool wq_gemm_ok(bool q4, const void* x, size_t x_elem, const void* w, int64_t m, int64_t n, int64_t k,
                int64_t group) {
    const int64_t rowb = q4 ? k / 2 : k;
    // Shape rule (measured): the GEMM runs one workgroup per 16 (or 32) weight
    // rows, each reading all of x, so below 4096 rows it fills under 256 CUs; a
    // GEMV slice of 8 rows plus a remainder slice is then faster up to m = 15.
    if (m <= 8 || (m < 16 && n < 4096)) return false;
    return k > 0 && k % 32 == 0 && (!q4 || (group % 32 == 0 && ((group / 32) & (group / 32 - 1)) == 0)) && aligned(x, 16) && aligned(w, 16) &&
           m <= (int64_t(65535) * 64) && std::min<int64_t>(m, 64) * k * static_cast<int64_t>(x_elem) < (int64_t(1) << 31) - 64 &&
           n * rowb < (int64_t(1) << 31) - 64;
}

// All m rows in one launch: 64-row blocks of x over gridDim.y (each block
// streams the weight once).
template <bool Q4, typename XT, typename YT, typename ST>
nq_status wq_gemm(const XT* x, const uint8_t* w, const ST* sc, const float* b, YT* y, int64_t m, int64_t n,
                  int64_t k, int64_t group, hipStream_t s) {
    return launch_wq<Q4>(x, w, sc, b, y, static_cast<int>(m), static_cast<int>(n), static_cast<int>(k),
                         static_cast<int>(group), s);
}

#define NQ_WQ_INST(Q4, XT, YT, ST)                                                                          \
    template nq_status wq_gemm<Q4, XT, YT, ST>(const XT*, const uint8_t*, const ST*, const float*, YT*, \
                                               int64_t, int64_t, int64_t, int64_t, hipStream_t);
NQ_WQ_INST(false, float, float, float)
NQ_WQ_INST(false, float, _Float16, float)
NQ_WQ_INST(false, _Float16, float, float)
NQ_WQ_INST(false, _Float16, _Float16, float)
NQ_WQ_INST(true, float, float, float)
NQ_WQ_INST(true, float, _Float16, float)
NQ_WQ_INST(true, _Float16, float, float)
NQ_WQ_INST(true, _Float16, _Float16, float)
NQ_WQ_INST(true, float, float, _Float16)
NQ_WQ_INST(true, float, _Float16, _Float16)
NQ_WQ_INST(true, _Float16, float, _Float16)
NQ_WQ_INST(true, _Float16, _Float16, _Float16)
#undef NQ_WQ_INST

}  // namespace nq
