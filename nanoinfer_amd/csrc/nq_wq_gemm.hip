// Weight-only Q8 / Q4G linears for batched activations (m > 8) on the fp16
// matrix cores: the reference runs these as fp32 dot products per output
// (quant.cpp:136-163, :337-389; its CUDA tiled Q8 kernel cuda_quant.cu:165-204
// is the m > 16 counterpart). Codes are converted to fp16 exactly in registers
// and multiplied with fp16 activations by v_mfma_f32_16x16x32_f16 (fp32
// accumulation). fp32 activations take the bf16 matrix cores instead: each value
// is split exactly into three bf16 parts (the top 8 significant bits by
// truncation, the next 8 the same way, and the remainder, which has at most 8
// bits left), the codes become bf16 exactly, and three
// v_mfma_f32_16x16x32_bf16 multiply them. bf16 has fp32's exponent range, so
// every finite fp32 activation with |x| >= 2^-110 (all three parts normal) is
// represented exactly and each product is exact in fp32: no overflow above
// 65504 and no precision lost to fp16 subnormals.
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

#include <iterator>
#include <type_traits>

#include "nq_device.hpp"
#include "nq_internal.hpp"

namespace nq {
namespace {

typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef __bf16 b8 __attribute__((ext_vector_type(8)));

__device__ __forceinline__ unsigned f32_bits(float f) { return __builtin_bit_cast(unsigned, f); }
// Eight fp32 values whose low 16 bits are zero (each exactly a bf16) as eight bf16.
__device__ __forceinline__ b8 pack_bf16(const float (&f)[8]) {
    v4i r;
#pragma unroll
    for (int i = 0; i < 4; ++i) r[i] = static_cast<int>(__builtin_amdgcn_perm(f32_bits(f[2 * i + 1]), f32_bits(f[2 * i]), 0x07060302u));
    return __builtin_bit_cast(b8, r);
}
constexpr int kWqRing = 4, kOob = 0x7FFFFFF0;

template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}
// Waves per workgroup: 16 for one 16-row tile of x (more loads in flight per
// CU), 8 for larger tiles (their prefetch ring needs up to 256 VGPRs).
template <int TM>
constexpr int wq_waves() { return TM == 1 ? 16 : 8; }

// Activation fragment of one chunk: 8 values of one row.
template <typename XT>
struct XFrag;
template <>
struct XFrag<_Float16> {
    v4i raw;  // 8 halves
    __device__ __forceinline__ void load(__amdgpu_buffer_rsrc_t rs, int off) {
        raw = __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(rs, off, 0, 0));
    }
    // The 8 halves in the order WFrag<Q4>::codes() gives the weight codes:
    // column order for int8, pairs (c, c+4) for int4 (the nibble trick's order).
    template <bool Q4>
    __device__ __forceinline__ h8 operands() const {
        if constexpr (!Q4) return __builtin_bit_cast(h8, raw);
        const h8 v = __builtin_bit_cast(h8, raw);
        h8 hi;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            hi[2 * j] = v[j];
            hi[2 * j + 1] = v[j + 4];
        }
        return hi;
    }
};
template <>
struct XFrag<float> {
    v4i a, b;  // 8 floats
    __device__ __forceinline__ void load(__amdgpu_buffer_rsrc_t rs, int off) {
        a = __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(rs, off, 0, 0));
        b = __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(rs, off == kOob ? kOob : off + 16, 0, 0));
    }
    // Exact split v = hi + mid + lo of the 8 values in column order: hi and mid
    // truncate to 8 significant bits, so v - hi and (v - hi) - mid are exact and
    // the remainder fits a bf16. A non-finite v keeps its value in hi and zero
    // in the other parts (inf - inf would make them NaN).
    __device__ __forceinline__ void split3(b8& hi, b8& mid, b8& lo) const {
        const f4 fa = __builtin_bit_cast(f4, a), fb = __builtin_bit_cast(f4, b);
        float h[8], md[8], l[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const float v = e < 4 ? fa[e] : fb[e - 4];
            h[e] = __builtin_bit_cast(float, f32_bits(v) & 0xFFFF0000u);
            float r1 = v - h[e];
            r1 = r1 == r1 ? r1 : 0.0f;
            md[e] = __builtin_bit_cast(float, f32_bits(r1) & 0xFFFF0000u);
            l[e] = r1 - md[e];
        }
        hi = pack_bf16(h);
        mid = pack_bf16(md);
        lo = pack_bf16(l);
    }
};

// Weight fragment of one chunk: 8 codes of one row as fp16 (int4: pairs
// (c, c+4); int8: column order).
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
            // one v_and_or_b32 (mask in an SGPR, magic in a VGPR) per pair
            unsigned b;
            asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(b) : "v"(u >> (4 * j)), "s"(0x000F000Fu), "v"(0x64006400u));
            const h2 p = __builtin_bit_cast(h2, b) + off;
            r[2 * j] = p[0];
            r[2 * j + 1] = p[1];
        }
        return r;
    }
    // The 8 codes in column order as bf16 (nib - 8 is exact).
    __device__ __forceinline__ b8 codes_bf16() const {
        const unsigned u = static_cast<unsigned>(w);
        float f[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) f[e] = static_cast<float>((u >> (4 * e)) & 0xFu) - 8.0f;
        return pack_bf16(f);
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
        // Columns (2t, 2t + 1) into the low bytes of two halves (bytes 2t, 2t + 1
        // of the pair w1:w0); XOR with 0x6480 gives the fp16 value 1024 + (code +
        // 128) exactly; -1152 -> code. Column order, so the activation fragment
        // needs no permutation.
        const h2 off = {static_cast<_Float16>(-1152.0f), static_cast<_Float16>(-1152.0f)};
        h8 r;
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            const unsigned sel = 0x0C000C00u | static_cast<unsigned>(2 * t) | (static_cast<unsigned>(2 * t + 1) << 16);
            const unsigned b = __builtin_amdgcn_perm(static_cast<unsigned>(w1), static_cast<unsigned>(w0), sel);
            const h2 p = __builtin_bit_cast(h2, b ^ 0x64806480u) + off;
            r[2 * t] = p[0];
            r[2 * t + 1] = p[1];
        }
        return r;
    }
    // The 8 codes in column order as bf16: byte + 128 as a float, minus 128 (exact).
    __device__ __forceinline__ b8 codes_bf16() const {
        const unsigned u0 = static_cast<unsigned>(w0) ^ 0x80808080u, u1 = static_cast<unsigned>(w1) ^ 0x80808080u;
        float f[8];
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            f[t] = static_cast<float>((u0 >> (8 * t)) & 0xFFu) - 128.0f;
            f[4 + t] = static_cast<float>((u1 >> (8 * t)) & 0xFFu) - 128.0f;
        }
        return pack_bf16(f);
    }
};

template <bool Q4, int TM, int TN, typename XT, typename YT, typename ST, bool SPLIT = false>
__global__ __launch_bounds__(wq_waves<TM>() * 64) void gemm_wq_kernel(
    const XT* __restrict__ x, const uint8_t* __restrict__ wq, const ST* __restrict__ scale,
    const float* __restrict__ bias, YT* __restrict__ y, int m, int n, int k, int group, float* __restrict__ planes,
    int split_chunks) {
    constexpr int kWqWaves = wq_waves<TM>();
    __shared__ f4 part[kWqWaves][TM][TN][64];
    // group / 32 is a power of two (checked on the host): chunk c uses group c >> gsh.
    const int gsh = Q4 ? __builtin_ctz(static_cast<unsigned>(group >> 5)) : 0;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int r = lane & 15, q = lane >> 4;
    const int n0 = blockIdx.x * (16 * TN);
    const int m_all = m;
    // gridDim.y blocks of 64 activation rows
    x += static_cast<size_t>(blockIdx.y) * 64 * k;
    y += static_cast<size_t>(blockIdx.y) * 64 * n;
    m = min(64, m - static_cast<int>(blockIdx.y) * 64);
    // SPLIT: gridDim.z ranges of split_chunks chunks of K (the unsplit kernel is
    // compiled without the range arithmetic)
    const int c_begin = SPLIT ? static_cast<int>(blockIdx.z) * split_chunks : 0;
    const int chunks = SPLIT ? min(k >> 5, c_begin + split_chunks) - c_begin : k >> 5;
    const int rowb = Q4 ? (k >> 1) : k;  // weight bytes per row
    const int groups = Q4 ? (k + group - 1) / group : 1;  // scales per row: ceil, a short last group
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

    // Wave w takes chunks c_begin + w, + W, ...; steps = its count.
    const int steps = wave < chunks ? (chunks - wave + kWqWaves - 1) / kWqWaves : 0;
    struct Stage {
        XFrag<XT> xf[TM];
        WFrag<Q4> wf[TN];
        float s[TN];
    };
    auto load = [&](int t, Stage& st) {
        const int c = c_begin + wave + t * kWqWaves;
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
        if constexpr (sizeof(XT) == 4) {  // fp32 x: three bf16 MFMAs per chunk
            b8 b[TN];
#pragma unroll
            for (int j = 0; j < TN; ++j) b[j] = st.wf[j].codes_bf16();
#pragma unroll
            for (int i = 0; i < TM; ++i) {
                b8 hi, mid, lo;
                st.xf[i].split3(hi, mid, lo);
#pragma unroll
                for (int j = 0; j < TN; ++j) {
                    const f4 c0 = Q4 ? f4{0, 0, 0, 0} : acc[i][j];
                    f4 d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(hi, b[j], c0, 0, 0, 0);
                    d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(mid, b[j], d, 0, 0, 0);
                    d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(lo, b[j], d, 0, 0, 0);
                    if constexpr (Q4) {
#pragma unroll
                        for (int v = 0; v < 4; ++v) acc[i][j][v] = __builtin_fmaf(d[v], st.s[j], acc[i][j][v]);
                    } else {
                        acc[i][j] = d;
                    }
                }
            }
        } else {
            h8 b[TN];
#pragma unroll
            for (int j = 0; j < TN; ++j) b[j] = st.wf[j].codes();
#pragma unroll
            for (int i = 0; i < TM; ++i) {
                const h8 hi = st.xf[i].template operands<Q4>();
#pragma unroll
                for (int j = 0; j < TN; ++j) {
                    if constexpr (Q4) {
                        const f4 d = __builtin_amdgcn_mfma_f32_16x16x32_f16(hi, b[j], f4{0, 0, 0, 0}, 0, 0, 0);
#pragma unroll
                        for (int v = 0; v < 4; ++v) acc[i][j][v] = __builtin_fmaf(d[v], st.s[j], acc[i][j][v]);
                    } else {
                        acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(hi, b[j], acc[i][j], 0, 0, 0);
                    }
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
        if constexpr (SPLIT) {  // this range's raw sum (Q8 before its row scale)
            planes[(static_cast<size_t>(blockIdx.z) * m_all + blockIdx.y * 64 + mm) * n + nn] = s;
            continue;
        }
        if constexpr (!Q4) s *= to_f32(scale[nn]);
        y[static_cast<size_t>(mm) * n + nn] = from_f32<YT>(s + (bias ? bias[nn] : 0.0f));
    }
}

// Sums the split-K planes part[splits][m][n] (splits <= kWqMaxSplits) in plane
// order, then the Q8 row scale and the bias, as the unsplit epilogue applies
// them. One output per thread with all its plane loads issued before the first
// add (one latency, not one per plane); four outputs per thread in 16-byte loads
// measured slower (n = 2048, k = 8192, m = 64: 15.5 vs 12.8 us for the split
// linear), a quarter of the threads each waiting on larger requests.
constexpr int kWqMaxSplits = 16;
template <bool Q4, typename YT, typename ST>
__global__ __launch_bounds__(256) void wq_reduce_kernel(const float* __restrict__ part, int splits,
                                                        const ST* __restrict__ scale, const float* __restrict__ bias,
                                                        YT* __restrict__ y, int m, int n) {
    const size_t mn = static_cast<size_t>(m) * n;
    const size_t i = static_cast<size_t>(blockIdx.x) * 256 + threadIdx.x;
    if (i >= mn) return;
    float a[kWqMaxSplits];
#pragma unroll
    for (int sp = 0; sp < kWqMaxSplits; ++sp)
        if (sp < splits) a[sp] = part[sp * mn + i];
    float t = a[0];
#pragma unroll
    for (int sp = 1; sp < kWqMaxSplits; ++sp)
        if (sp < splits) t += a[sp];
    const int c = static_cast<int>(i % n);
    if constexpr (!Q4) t *= to_f32(scale[c]);
    y[i] = from_f32<YT>(t + (bias ? bias[c] : 0.0f));
}

template <bool Q4, typename YT, typename ST>
nq_status launch_wq_reduce(const float* planes, int splits, const ST* sc, const float* b, YT* y, int m, int n,
                           hipStream_t s) {
    const size_t mn = static_cast<size_t>(m) * n;
    wq_reduce_kernel<Q4><<<static_cast<unsigned>((mn + 255) / 256), 256, 0, s>>>(planes, splits, sc, b, y, m, n);
    return launch_status("wq_reduce_kernel");
}

// Launch plan of the 16-row kernel: tm 16-row tiles of x (1..4), tn 16-row
// tiles of the weight (1, 2), K in `splits` ranges of `per` chunks.
struct WqRowPlan {
    int tm, tn, splits, per;
};

template <bool Q4, typename XT, typename YT, typename ST>
nq_status launch_wq(const XT* x, const uint8_t* w, const ST* sc, const float* b, YT* y, int m, int n, int k,
                    int g, WqRowPlan p, float* planes, hipStream_t s) {
    // 16 weight rows per workgroup, 32 for tall weights at m <= 32 (the LDS
    // tile of per-wave partials stays within 32 KB); 64-row blocks of x over
    // gridDim.y; K ranges over gridDim.z when planes are given.
    if (!planes || p.splits <= 1) {
        planes = nullptr;
        p.splits = 1;
        p.per = k / 32;
    }
    const unsigned mblocks = static_cast<unsigned>((m + 63) / 64);
    auto go = [&](auto tmtag, auto tntag) {
        constexpr int TM = decltype(tmtag)::value, TN = decltype(tntag)::value;
        const dim3 grid(static_cast<unsigned>((n + 16 * TN - 1) / (16 * TN)), mblocks, static_cast<unsigned>(p.splits));
        if (planes)
            gemm_wq_kernel<Q4, TM, TN, XT, YT, ST, true><<<grid, wq_waves<TM>() * 64, 0, s>>>(x, w, sc, b, y, m, n, k,
                                                                                             g, planes, p.per);
        else
            gemm_wq_kernel<Q4, TM, TN, XT, YT, ST><<<grid, wq_waves<TM>() * 64, 0, s>>>(x, w, sc, b, y, m, n, k, g,
                                                                                       nullptr, p.per);
    };
    auto with_tn = [&](auto tmtag) {
        if constexpr (decltype(tmtag)::value <= 2) {
            if (p.tn == 2) return go(tmtag, std::integral_constant<int, 2>{});
        }
        go(tmtag, std::integral_constant<int, 1>{});
    };
    switch (p.tm) {
        case 1: with_tn(std::integral_constant<int, 1>{}); break;
        case 2: with_tn(std::integral_constant<int, 2>{}); break;
        case 3: with_tn(std::integral_constant<int, 3>{}); break;
        default: with_tn(std::integral_constant<int, 4>{}); break;
    }
    if (nq_status st = launch_status("gemm_wq_kernel")) return st;
    return planes ? launch_wq_reduce<Q4>(planes, p.splits, sc, b, y, m, n, s) : NQ_OK;
}

// ---- wide tiles for fp16 activations -----------------------------------------------------
// One (16*WM*FM) x (16*WN*FN) output tile per workgroup, WM x WN waves (4 x 2,
// 4 x 3, 4 x 4, or 2 x 6 for 256-row Q8 tiles), each (16*FM) x (16*FN)
// outputs, as in the wide W8A8 kernel: K advances in slabs
// of SK columns (64 or 128) that LDS-DMA (buffer_load ... lds) writes into a
// ring of as many slots as fit in 160 KB; the request for slab kt + D - 1 goes
// out after the barrier that frees its slot. A slab holds the activation tile
// (fp16 rows of 2*SK bytes), the weight codes (SK or SK/2 bytes per row) and,
// for Q4G, the tile's group scales of the slab. 256-row tiles take 64-column
// slabs (three fit: 256 x 288 in one round beat two rounds of 128 x 288 with
// 128-column slabs); smaller tiles take 128-column slabs. Each lane loads the
// chunk an XOR swizzle puts in its LDS slot (16-byte chunk c of a row of C
// chunks at slot c ^ ((r >> log2(16 / C)) & (C - 1))), so the 16 rows of a
// fragment read hit distinct banks. Codes become fp16 exactly in registers
// after the LDS read (the WFrag conversions above); A = activations, B =
// weights, so a lane's four results share one weight row. Q8: one MFMA chain
// over K, row scale in the epilogue. Q4G: an MFMA chain over each group's
// chunks (at most one slab), scaled by the group scale into the fp32 accumulator.
template <int C>
__device__ __forceinline__ int wq_swz(int r) {  // slot XOR of row r, C 16-byte chunks per row
    constexpr int S = C >= 16 ? 0 : C == 8 ? 1 : C == 4 ? 2 : 3;
    return (r >> S) & (C - 1);
}

template <bool Q4, int SK, int FM, int FN, int GSH, typename YT, typename ST, typename XT = _Float16, int WN = 2,
          int WM = 4, int DMAX = 8>
struct WqWideShape {
    static constexpr int kNW = WM * WN;  // waves: WM along m, WN along n
    static constexpr int kBM = WM * 16 * FM, kBN = WN * 16 * FN, kT = SK / 32;  // MFMA K steps per slab
    static constexpr int kXRow = static_cast<int>(sizeof(XT)) * SK, kWRow = Q4 ? SK / 2 : SK;  // bytes per row and slab
    static constexpr int kXC = kXRow / 16, kWC = kWRow / 16;         // 16-byte chunks per row
    // Scales per weight row and slab (Q4G): groups of 32 << GSH columns, one per
    // slab when a group covers the slab (GSH = kGBig stands for all such groups).
    static constexpr int kGBig = SK == 128 ? 2 : 1;
    static constexpr int kSPer = Q4 ? (GSH >= kGBig ? 1 : kT >> GSH) : 0;
    static constexpr int kSRow = kSPer * static_cast<int>(sizeof(ST));
    static constexpr int kCPG = GSH >= kGBig ? kT : 1 << GSH;  // MFMA steps per scaled chain
    static constexpr int kXB = kBM * kXRow / 1024, kWB = kBN * kWRow / 1024;  // 1 KB requests
    static constexpr int kNB = kXB + kWB, kQ = (kNB + kNW - 1) / kNW;
    // 256-byte scale requests; the last may run past the tile's rows into the
    // region's padding.
    static constexpr int kNS = (kBN * kSRow + 255) / 256, kQS = (kNS + kNW - 1) / kNW;
    static constexpr int kXOff = 0, kWOff = kBM * kXRow, kSOff = kWOff + kBN * kWRow;
    static constexpr int kSlab = kSOff + kNS * 256;
    // fp16 epilogue: the tile's weight scales (Q8) and bias in LDS, DMA'd at the
    // start, after the ring and the staging rows.
    static constexpr int kEpsN = (kBN + 63) / 64 * 64;
    static constexpr int kEpsBytes = sizeof(YT) == 2 ? 2 * kEpsN * 4 : 0;
    // Ring slots: with the default depth, where three or more fit in half the
    // LDS, as many as let two workgroups share a CU (n = 8960, k = 1536, m = 64:
    // Q4G 17.1 -> 15.5 us; n = 4864, k = 896, m = 128 Q8 10.6 -> 9.5); otherwise
    // as many as 160 KB holds beside the sink, at most DMAX.
    static constexpr int kDTwo = (80 * 1024 - 1024 - kEpsBytes) / kSlab;
    static constexpr int kD = DMAX == 8 && kDTwo >= 3 ? std::min(8, kDTwo)
                                                      : std::min(DMAX, (160 * 1024 - 1024 - kEpsBytes) / kSlab);
    static constexpr int kSink = kD * kSlab;
    // fp16 staging rows padded by 16 bytes (an odd multiple of 16: the rows a
    // store instruction touches fall on distinct banks).
    static constexpr int kStg = kBN * 2 + 16;
    static constexpr size_t kStage = size_t(kBM) * kStg;
    static constexpr size_t kEps = (std::max<size_t>(size_t(kSink) + 1024, sizeof(YT) == 2 ? kStage : 0) + 15) / 16 * 16;
    static constexpr size_t kLds = kEps + kEpsBytes;
    static_assert(kLds <= 160 * 1024, "LDS");
    static_assert(kD >= 2, "two slabs must fit");
    static_assert(kQ + kQS <= 63, "vmcnt range");
    static_assert(!Q4 || kSRow % 4 == 0, "scale rows are whole dwords");
};

template <bool Q4, int SK, int FM, int FN, int GSH, typename YT, typename ST, typename XT, int WN, int WM, int DMAX>
__global__ __launch_bounds__(WM * WN * 64) void gemm_wq_wide_kernel(
    const XT* __restrict__ x, const uint8_t* __restrict__ wq, const ST* __restrict__ scale,
    const float* __restrict__ bias, YT* __restrict__ y, int m, int n, int k, int tiles_m, int tiles_n,
    int gsh_rt, float* __restrict__ planes, int split_slabs) {
    using S = WqWideShape<Q4, SK, FM, FN, GSH, YT, ST, XT, WN, WM, DMAX>;
    constexpr int NW = S::kNW;
    constexpr bool F32X = sizeof(XT) == 4;  // fp32 activations: three bf16 parts, three bf16 MFMAs
    constexpr int BM = S::kBM, BN = S::kBN, D = S::kD, Q = S::kQ, QS = S::kQS, XB = S::kXB, NB = S::kNB;
    constexpr int T = S::kT, XROW = S::kXRow, WROW = S::kWRow, XC = S::kXC, WC = S::kWC;
    // group = 32 << gsh columns; GSH = kGBig stands for every group of at
    // least one slab (one scale per slab), its shift given at run time.
    const int gsh = GSH >= S::kGBig ? gsh_rt : GSH;
    extern __shared__ __attribute__((aligned(16))) int8_t lds[];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave / WN, wn = wave % WN;
    const int total = tiles_m * tiles_n;
    const int per = (total + 7) / 8, xcd = blockIdx.x % 8, idx = blockIdx.x / 8;
    const int full = total - 8 * (per - 1);
    const int lin = xcd < full ? xcd * per + idx : full * per + (xcd - full) * (per - 1) + idx;
    const int m0 = (lin % tiles_m) * BM, n0 = (lin / tiles_m) * BN;

    const int wrow_bytes = Q4 ? k / 2 : k;
    const int groups = Q4 ? (k + (32 << gsh) - 1) >> (5 + gsh) : 1;  // ceil: a short last group
    const __amdgpu_buffer_rsrc_t xrs = __builtin_amdgcn_make_buffer_rsrc(const_cast<XT*>(x), 0, m * k * static_cast<int>(sizeof(XT)), 0x00020000);
    const __amdgpu_buffer_rsrc_t wrs = __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(wq), 0, n * wrow_bytes, 0x00020000);
    const __amdgpu_buffer_rsrc_t srs = __builtin_amdgcn_make_buffer_rsrc(const_cast<ST*>(scale), 0, Q4 ? n * groups * static_cast<int>(sizeof(ST)) : 0, 0x00020000);
    // 1 KB request q of wave w = block b = q * 8 + w: blocks [0, XB) hold
    // 1024 / XROW activation rows each, [XB, NB) 1024 / WROW weight rows, the
    // rest spares (they read zeros into the sink).
    int voff[Q], loff[Q];
#pragma unroll
    for (int q = 0; q < Q; ++q) {
        const int b = q * NW + wave;
        const bool real = b < NB;
        if (b < XB) {
            const int r = b * (1024 / XROW) + lane / XC, c = (lane % XC) ^ wq_swz<XC>(r);
            voff[q] = m0 + r < m ? (m0 + r) * k * static_cast<int>(sizeof(XT)) + c * 16 : kOob;
        } else {
            const int r = (b - XB) * (1024 / WROW) + lane / WC, c = (lane % WC) ^ wq_swz<WC>(r);
            voff[q] = real && n0 + r < n ? (n0 + r) * wrow_bytes + c * 16 : kOob;
        }
        loff[q] = real ? b * 1024 : S::kSink;
    }
    // 256-byte scale request q of wave w = block b: kSRow / 4 lanes per weight row.
    int soffv[QS > 0 ? QS : 1], sloff[QS > 0 ? QS : 1];
#pragma unroll
    for (int q = 0; q < QS; ++q) {
        const int b = q * NW + wave;
        constexpr int LPR = S::kSRow / 4 > 0 ? S::kSRow / 4 : 1;
        const int r = b * (64 / LPR) + lane / LPR;
        soffv[q] = b < S::kNS && n0 + r < n ? (n0 + r) * groups * static_cast<int>(sizeof(ST)) + (lane % LPR) * 4 : kOob;
        sloff[q] = b < S::kNS ? S::kSOff + b * 256 : S::kSink;
    }
    // gridDim.y ranges of split_slabs slabs of K (one range without a split)
    // Only the two-slot ring (DMAX < 8) runs split K; the other instantiations
    // are compiled without the range arithmetic.
    constexpr bool kSplit = DMAX < 8;
    const int kb = kSplit ? static_cast<int>(blockIdx.y) * split_slabs : 0;
    const int nk = kSplit ? min(k / SK, kb + split_slabs) - kb : k / SK;
    const unsigned lds_base = static_cast<unsigned>(reinterpret_cast<uintptr_t>(lds));
    auto issue = [&](int sl) {
        const unsigned slot = static_cast<unsigned>(sl % D) * S::kSlab;
        const bool in = sl < nk;
        const int xo = in ? (kb + sl) * XROW : kOob, wo = in ? (kb + sl) * WROW : kOob;
#pragma unroll
        for (int q = 0; q < Q; ++q) {
            const int b = q * NW + wave;
            const unsigned dst = lds_base + (b < NB ? slot : 0u) + static_cast<unsigned>(loff[q]);
            if (b < XB)
                asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, %3 offen lds"
                             ::"s"(dst), "v"(voff[q]), "s"(xrs), "s"(xo) : "memory");
            else
                asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, %3 offen lds"
                             ::"s"(dst), "v"(voff[q]), "s"(wrs), "s"(wo) : "memory");
        }
        if constexpr (Q4) {
            // the slab's first group (its groups are consecutive in the row)
            const int so = in ? (((kb + sl) * T) >> gsh) * static_cast<int>(sizeof(ST)) : kOob;
#pragma unroll
            for (int q = 0; q < QS; ++q) {
                const int b = q * NW + wave;
                const unsigned dst = lds_base + (b < S::kNS ? slot : 0u) + static_cast<unsigned>(sloff[q]);
                asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dword %1, %2, %3 offen lds"
                             ::"s"(dst), "v"(soffv[q]), "s"(srs), "s"(so) : "memory");
            }
        }
    };

    f4 acc[FN][FM];
#pragma unroll
    for (int i = 0; i < FN; ++i)
#pragma unroll
        for (int j = 0; j < FM; ++j) acc[i][j] = f4{0, 0, 0, 0};
    const int fr = lane & 15, fq = lane >> 4;
    int fxo[FM], fwr[FN];
#pragma unroll
    for (int j = 0; j < FM; ++j) fxo[j] = wm * 16 * FM + j * 16 + fr;
#pragma unroll
    for (int i = 0; i < FN; ++i) fwr[i] = wn * 16 * FN + i * 16 + fr;

    if constexpr (sizeof(YT) == 2) {
        // Epilogue operands by dword DMA, ahead of the ring (the slab waits cover
        // them): request e < NC is 64 weight scales (Q8; Q4G reads ones), the
        // rest 64 bias values; past n or without bias the loads read zeros.
        constexpr int NC = S::kEpsN / 64;
        const __amdgpu_buffer_rsrc_t wsr = __builtin_amdgcn_make_buffer_rsrc(const_cast<ST*>(scale), 0, Q4 ? 0 : n * 4, 0x00020000);
        const __amdgpu_buffer_rsrc_t brs = __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(bias ? bias : reinterpret_cast<const float*>(scale)), 0, bias ? n * 4 : 0, 0x00020000);
        for (int e = wave; e < 2 * NC; e += NW) {
            const unsigned dst = lds_base + static_cast<unsigned>(S::kEps) + static_cast<unsigned>(e * 256);
            const int vo = (n0 + (e % NC) * 64 + lane) * 4;
            if (e < NC)
                asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dword %1, %2, 0 offen lds" ::"s"(dst), "v"(vo), "s"(wsr) : "memory");
            else
                asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dword %1, %2, 0 offen lds" ::"s"(dst), "v"(vo), "s"(brs) : "memory");
        }
    }
    // Fragment addresses: a 16-row step moves a row's chunk swizzle by a
    // multiple of its chunk count (16 / C rows share one XOR value and C <= 16),
    // so every fragment of a wave shares the swizzle of its first row and the
    // fragments differ by constant offsets (immediate LDS offsets).
    static_assert(XC <= 16 && WC <= 16, "swizzle shared by the fragments");
    const int xr0 = fxo[0], wr0 = fwr[0];
    const int xsw = wq_swz<XC>(xr0), wsw = wq_swz<WC>(wr0);
    const int xlane = S::kXOff + xr0 * XROW, wlane = S::kWOff + wr0 * WROW, slane = S::kSOff + wr0 * S::kSRow;
#pragma unroll
    for (int sl = 0; sl < D - 1; ++sl) issue(sl);
    unsigned slot_off = 0;  // (kt % D) * kSlab, kept as a plain rotating offset
    for (int kt = 0; kt < nk; ++kt) {
        wait_vmcnt<(Q + (Q4 ? QS : 0)) * (D - 2)>();
        __builtin_amdgcn_s_barrier();
        issue(kt + D - 1);
        const int8_t* base = lds + slot_off;
        slot_off = slot_off + S::kSlab == static_cast<unsigned>(D * S::kSlab) ? 0u : slot_off + S::kSlab;
        f4 part[FN][FM];
#pragma unroll
        for (int t = 0; t < T; ++t) {
            // fp16 x: one fp16 MFMA per fragment pair; fp32 x: three bf16 ones.
            using XOp = std::conditional_t<F32X, b8, h8>;
            XOp xa[FM], xm[FM], xl[FM], wb[FN];
            if constexpr (F32X) {  // 8 floats = chunks 8t + 2 fq and the next
                const int c = t * 8 + fq * 2;
                const int8_t* pa = base + xlane + ((c ^ xsw) << 4);
                const int8_t* pb = base + xlane + (((c + 1) ^ xsw) << 4);
#pragma unroll
                for (int j = 0; j < FM; ++j) {
                    XFrag<float> f;
                    f.a = *reinterpret_cast<const v4i*>(pa + j * 16 * XROW);
                    f.b = *reinterpret_cast<const v4i*>(pb + j * 16 * XROW);
                    f.split3(xa[j], xm[j], xl[j]);
                }
            } else {  // 8 halves = chunk 4t + fq
                const int8_t* pa = base + xlane + (((t * 4 + fq) ^ xsw) << 4);
#pragma unroll
                for (int j = 0; j < FM; ++j) {
                    XFrag<_Float16> f;
                    f.raw = *reinterpret_cast<const v4i*>(pa + j * 16 * XROW);
                    xa[j] = f.template operands<Q4>();
                }
            }
            if constexpr (Q4) {  // 8 codes = one dword: chunk t, dword fq
                const int8_t* pw = base + wlane + ((t ^ wsw) << 4) + fq * 4;
#pragma unroll
                for (int i = 0; i < FN; ++i) {
                    WFrag<true> f;
                    f.w = *reinterpret_cast<const int*>(pw + i * 16 * WROW);
                    if constexpr (F32X) wb[i] = f.codes_bf16();
                    else wb[i] = f.codes();
                }
            } else {  // 8 codes = two dwords: chunk 2t + fq / 2, half fq % 2
                typedef int v2i __attribute__((ext_vector_type(2)));
                const int8_t* pw = base + wlane + (((t * 2 + (fq >> 1)) ^ wsw) << 4) + (fq & 1) * 8;
#pragma unroll
                for (int i = 0; i < FN; ++i) {
                    const v2i v = *reinterpret_cast<const v2i*>(pw + i * 16 * WROW);
                    WFrag<false> f;
                    f.w0 = v[0];
                    f.w1 = v[1];
                    if constexpr (F32X) wb[i] = f.codes_bf16();
                    else wb[i] = f.codes();
                }
            }
            auto mma = [&](const XOp& a, const XOp& b, const f4& c) {
                if constexpr (F32X) return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
                else return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
            };
            // Q4G: the group's last step scales each fragment's partial into the
            // accumulator, one fragment behind its MFMAs so the adds do not wait
            // on the MFMA they follow.
            const bool scale_now = Q4 && t % S::kCPG == S::kCPG - 1;
            float sc[Q4 ? FN : 1];
            if constexpr (Q4) {
                if (scale_now) {
                    const int gi = GSH >= S::kGBig ? 0 : t >> GSH;  // group within the slab
                    const int8_t* ps = base + slane + gi * static_cast<int>(sizeof(ST));
#pragma unroll
                    for (int i = 0; i < FN; ++i) {
                        if constexpr (sizeof(ST) == 4) sc[i] = *reinterpret_cast<const float*>(ps + i * 16 * S::kSRow);
                        else sc[i] = static_cast<float>(*reinterpret_cast<const _Float16*>(ps + i * 16 * S::kSRow));
                    }
                }
            }
            auto scale_into = [&](int i, int j) {
#pragma unroll
                for (int v = 0; v < 4; ++v) acc[i][j][v] = __builtin_fmaf(part[i][j][v], sc[i], acc[i][j][v]);
            };
#pragma unroll
            for (int i = 0; i < FN; ++i)
#pragma unroll
                for (int j = 0; j < FM; ++j) {
                    f4& d = Q4 ? part[i][j] : acc[i][j];
                    const f4 c0 = Q4 && t % S::kCPG == 0 ? f4{0, 0, 0, 0} : d;
                    d = mma(xa[j], wb[i], c0);
                    if constexpr (F32X) {
                        d = mma(xm[j], wb[i], d);
                        d = mma(xl[j], wb[i], d);
                    }
                    if constexpr (Q4) {
                        if (scale_now && (i > 0 || j > 0)) scale_into(j > 0 ? i : i - 1, j > 0 ? j - 1 : FM - 1);
                    }
                }
            if constexpr (Q4) {
                if (scale_now) scale_into(FN - 1, FM - 1);
                __builtin_amdgcn_sched_barrier(0);  // keep the next step's reads below (registers)
            }
        }
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // this slab's reads are done
    }
    wait_vmcnt<0>();

    // Lane l holds, for fragment (i, j), rows m0 + wm*16*FM + j*16 + 4*(l/16) + v
    // of column n0 + wn*16*FN + i*16 + l%16.
    if constexpr (kSplit) {  // this range's raw sums (Q8 before its row scale) into plane blockIdx.y
        float* pl = planes + static_cast<size_t>(blockIdx.y) * m * n;
#pragma unroll
        for (int i = 0; i < FN; ++i) {
            const int col = n0 + fwr[i];
            if (col >= n) continue;
#pragma unroll
            for (int j = 0; j < FM; ++j)
#pragma unroll
                for (int v = 0; v < 4; ++v) {
                    const int row = m0 + fxo[j] - fr + 4 * fq + v;
                    if (row < m) pl[static_cast<size_t>(row) * n + col] = acc[i][j][v];
                }
        }
        return;
    }
    if constexpr (sizeof(YT) == 2) {
        if ((n & 7) == 0) {
            __syncthreads();  // every wave is done with the ring
#pragma unroll
            for (int i = 0; i < FN; ++i) {
                const int cl = fwr[i];
                const float* eps = reinterpret_cast<const float*>(lds + S::kEps);
                const float ws = Q4 ? 1.0f : eps[cl];
                const float b = eps[S::kEpsN + cl];
#pragma unroll
                for (int j = 0; j < FM; ++j)
#pragma unroll
                    for (int v = 0; v < 4; ++v) {
                        const int rl = fxo[j] - fr + 4 * fq + v;
                        const float val = Q4 ? acc[i][j][v] + b : acc[i][j][v] * ws + b;
                        *reinterpret_cast<_Float16*>(lds + rl * S::kStg + cl * 2) = static_cast<_Float16>(val);
                    }
            }
            __syncthreads();
            constexpr int CPR = BN / 8;
            for (int c = tid; c < BM * CPR; c += NW * 64) {
                const int rl = c / CPR, cc = c % CPR;
                const int row = m0 + rl, col = n0 + cc * 8;
                if (row < m && col < n)
                    __builtin_nontemporal_store(*reinterpret_cast<const v4i*>(lds + rl * S::kStg + cc * 16),
                                                reinterpret_cast<v4i*>(y + static_cast<size_t>(row) * n + col));
            }
            return;
        }
    }
#pragma unroll
    for (int i = 0; i < FN; ++i) {
        const int col = n0 + fwr[i];
        if (col >= n) continue;
        const float ws = Q4 ? 1.0f : to_f32(scale[col]);
        const float b = bias ? bias[col] : 0.0f;
#pragma unroll
        for (int j = 0; j < FM; ++j)
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const int row = m0 + fxo[j] - fr + 4 * fq + v;
                if (row < m) {
                    const float val = Q4 ? acc[i][j][v] + b : acc[i][j][v] * ws + b;
                    y[static_cast<size_t>(row) * n + col] = from_f32<YT>(val);
                }
            }
    }
}

template <bool Q4, int SK, int FM, int FN, int GSH, typename YT, typename ST, typename XT, int WN, int WM = 4,
          int DMAX = 8>
nq_status launch_wq_wide(const XT* x, const uint8_t* w, const ST* sc, const float* b, YT* y, int m, int n,
                         int k, int gsh, float* planes, int splits, int split_slabs, hipStream_t s) {
    using S = WqWideShape<Q4, SK, FM, FN, GSH, YT, ST, XT, WN, WM, DMAX>;
    auto* fn = gemm_wq_wide_kernel<Q4, SK, FM, FN, GSH, YT, ST, XT, WN, WM, DMAX>;
    if (nq_status st = set_dynamic_lds(reinterpret_cast<const void*>(fn), S::kLds, "gemm_wq_wide")) return st;
    const int tm = (m + S::kBM - 1) / S::kBM, tn = (n + S::kBN - 1) / S::kBN;
    fn<<<dim3(tm * tn, splits), S::kNW * 64, S::kLds, s>>>(x, w, sc, b, y, m, n, k, tm, tn, gsh, planes, split_slabs);
    return launch_status("gemm_wq_wide_kernel");
}

// Tiles of the wide path: (64 * fm) x (32 * fn) with sk-column slabs, by
// falling area. 256-row tiles need 64-column slabs. The plan takes the least
// rounds x (area + 21504), rounds = ceil(tiles / 256): a round of tiles took
// about 14 us + 0.65 us per 1024 outputs of the tile at k = 1536 (m = 512, n =
// 8960: 256 x 128 tiles 34.3 us, 128 x 256 39.0, 128 x 288 44.3, 256 x 256
// 55.6, 256 x 288 61.2; m = 2048: 256 x 288 in one round 67.0 us, 128 x 288 in
// two 91.9, 256 x 128 in three 100).
struct WqTile {
    int fm, fn, sk;
    bool shallow = false;  // a two-slot ring (fm = 1, fn = 2 or 4): more workgroups per CU
};
constexpr WqTile kWqTiles[] = {{4, 9, 64}, {4, 8, 64}, {2, 9, 128}, {4, 4, 64}, {2, 8, 128},
                               {2, 4, 128}, {1, 8, 128}, {1, 4, 128}, {1, 2, 128}};
// fp32 activations take twice the LDS per row: 64-column slabs and at most 128-row tiles.
constexpr WqTile kWqTilesF32[] = {{2, 9, 64}, {2, 8, 64}, {2, 4, 64}, {1, 8, 64}, {1, 4, 64}, {1, 2, 64}};
struct WqPlan {
    WqTile tile;
    int64_t tiles;
};
WqPlan plan_wq_wide(int64_t m, int64_t n, bool sk64_ok, bool f32x) {
    int64_t best_cost = 0;
    WqPlan p{{0, 0, 0}, 0};
    const WqTile* tiles = f32x ? kWqTilesF32 : kWqTiles;
    const int count = f32x ? static_cast<int>(std::size(kWqTilesF32)) : static_cast<int>(std::size(kWqTiles));
    for (int ti = 0; ti < count; ++ti) {
        const WqTile& t = tiles[ti];
        if (t.sk == 64 && !sk64_ok) continue;
        const int64_t c = ((m + 64 * t.fm - 1) / (64 * t.fm)) * ((n + 32 * t.fn - 1) / (32 * t.fn));
        const int64_t cost = ((c + 255) / 256) * ((64 * t.fm) * (32 * t.fn) + 21504);
        if (best_cost == 0 || cost < best_cost) {
            best_cost = cost;
            p = {t, c};
        }
    }
    return p;
}
// 64-column slabs: Q8, or Q4G in groups of 32 (a scaled chain per MFMA step;
// longer chains kept the 256-row tiles' partial sums live and spilled).
template <bool Q4, typename ST>
bool wq_sk64_ok(int64_t group) {
    return !Q4 || group == 32;
}

template <bool Q4, typename XT, typename YT, typename ST>
nq_status wq_wide_tiles(const XT* x, const uint8_t* w, const ST* sc, const float* b, YT* y, int m, int n, int k,
                        int group, WqTile pick, float* planes, int splits, int split_slabs, hipStream_t s) {
    constexpr bool F32X = sizeof(XT) == 4;
    const int gsh = Q4 ? __builtin_ctz(static_cast<unsigned>(group >> 5)) : 0;
    // Q8 tile widths that split in three (four) 16-column multiples run 12 (16)
    // waves, as in the W8A8 wide kernel (m = 2048: 74.3 -> 71.7 us); Q4G keeps 8
    // waves (its group-scaled partial sums do not fit 170 registers: 106.9 vs
    // 128.9 us; with the scaling one fragment behind its MFMAs 12 waves fit but
    // ran 99.5 vs 91.1).
    using std::integral_constant;
    // One wave layout and fragment shape: the group-size dispatch of Q4G.
    auto launch_g = [&](auto skt, auto fmt, auto fnt, auto wnt, auto wmt, auto dt) -> nq_status {
        constexpr int SK = decltype(skt)::value, FM = decltype(fmt)::value, FN = decltype(fnt)::value;
        constexpr int WN = decltype(wnt)::value, WM = decltype(wmt)::value, DM = decltype(dt)::value;
        constexpr int BIG = SK == 128 ? 2 : 1;  // one scale per slab from this shift on
        if constexpr (!Q4) {
            return launch_wq_wide<false, SK, FM, FN, 0, YT, ST, XT, WN, WM, DM>(x, w, sc, b, y, m, n, k, 0, planes, splits, split_slabs, s);
        } else {
            if (gsh == 0) return launch_wq_wide<true, SK, FM, FN, 0, YT, ST, XT, WN, WM, DM>(x, w, sc, b, y, m, n, k, 0, planes, splits, split_slabs, s);
            if constexpr (SK == 64) {  // excluded by wq_sk64_ok
                return fail(NQ_BAD_ARG, "gemm_wq_wide: 64-column slabs take groups of 32 only (got %d)", group);
            } else {
                if (gsh == 1) return launch_wq_wide<true, SK, FM, FN, 1, YT, ST, XT, WN, WM, DM>(x, w, sc, b, y, m, n, k, 1, planes, splits, split_slabs, s);
                if constexpr (sizeof(ST) == 2) {  // excluded by wq_wide_ok
                    return fail(NQ_BAD_ARG, "gemm_wq_wide: fp16 scales in groups of %d are not supported", group);
                } else {
                    return launch_wq_wide<true, SK, FM, FN, BIG, YT, ST, XT, WN, WM, DM>(x, w, sc, b, y, m, n, k, gsh, planes, splits, split_slabs, s);
                }
            }
        }
    };
    auto with_g = [&](auto skt, auto fmt, auto fnt) -> nq_status {
        constexpr int SK = decltype(skt)::value, FM = decltype(fmt)::value, FN2 = decltype(fnt)::value;
        constexpr int WN = Q4 ? 2 : FN2 % 3 == 0 ? 3 : FN2 % 4 == 0 ? 4 : 2, FN = FN2 * 2 / WN;
        using D8 = integral_constant<int, 8>;
        if constexpr (FM == 1 && (FN2 == 2 || FN2 == 4)) {
            if (pick.shallow)  // two ring slots: two or three workgroups per CU
                return launch_g(skt, fmt, integral_constant<int, FN>{}, integral_constant<int, WN>{},
                                integral_constant<int, 4>{}, integral_constant<int, 2>{});
        }
        if constexpr (!Q4 && !F32X && FM == 4 && FN2 % 3 == 0) {
            // 256-row Q8 tiles as 2 x 6 waves of (128 x 16 * FN2 / 3): each
            // weight fragment is converted to fp16 by two waves instead of four
            // (the conversion is a third of the MFMA time; m = 2048: 66.1 -> 63.7 us).
            return launch_g(skt, integral_constant<int, 8>{}, integral_constant<int, FN2 / 3>{},
                            integral_constant<int, 6>{}, integral_constant<int, 2>{}, D8{});
        } else {
            return launch_g(skt, fmt, integral_constant<int, FN>{}, integral_constant<int, WN>{},
                            integral_constant<int, 4>{}, D8{});
        }
    };
    using I64 = integral_constant<int, 64>;
    using I128 = integral_constant<int, 128>;
    if constexpr (F32X) {
        switch (pick.fm * 100 + pick.fn) {
            case 209: return with_g(I64{}, integral_constant<int, 2>{}, integral_constant<int, 9>{});
            case 208: return with_g(I64{}, integral_constant<int, 2>{}, integral_constant<int, 8>{});
            case 204: return with_g(I64{}, integral_constant<int, 2>{}, integral_constant<int, 4>{});
            case 108: return with_g(I64{}, integral_constant<int, 1>{}, integral_constant<int, 8>{});
            case 104: return with_g(I64{}, integral_constant<int, 1>{}, integral_constant<int, 4>{});
            default: return with_g(I64{}, integral_constant<int, 1>{}, integral_constant<int, 2>{});
        }
    } else {
        switch (pick.fm * 100 + pick.fn) {
            case 409: return with_g(I64{}, integral_constant<int, 4>{}, integral_constant<int, 9>{});
            case 408: return with_g(I64{}, integral_constant<int, 4>{}, integral_constant<int, 8>{});
            case 404: return with_g(I64{}, integral_constant<int, 4>{}, integral_constant<int, 4>{});
            case 209: return with_g(I128{}, integral_constant<int, 2>{}, integral_constant<int, 9>{});
            case 208: return with_g(I128{}, integral_constant<int, 2>{}, integral_constant<int, 8>{});
            case 204: return with_g(I128{}, integral_constant<int, 2>{}, integral_constant<int, 4>{});
            case 108: return with_g(I128{}, integral_constant<int, 1>{}, integral_constant<int, 8>{});
            case 104: return with_g(I128{}, integral_constant<int, 1>{}, integral_constant<int, 4>{});
            default: return with_g(I128{}, integral_constant<int, 1>{}, integral_constant<int, 2>{});
        }
    }
}

template <bool Q4, typename XT, typename YT, typename ST>
nq_status wq_wide(const XT* x, const uint8_t* w, const ST* sc, const float* b, YT* y, int m, int n, int k,
                  int group, WqTile pick, float* planes, int splits, int split_slabs, hipStream_t s) {
    if (!planes || splits <= 1 || !pick.shallow) {  // one range over all of K (split K runs shallow tiles)
        planes = nullptr;
        splits = 1;
        split_slabs = k / pick.sk;
        pick.shallow = false;
    }
    if (nq_status st = wq_wide_tiles<Q4>(x, w, sc, b, y, m, n, k, group, pick, splits > 1 ? planes : nullptr, splits,
                                         split_slabs, s))
        return st;
    return splits > 1 ? launch_wq_reduce<Q4>(planes, splits, sc, b, y, m, n, s) : NQ_OK;
}

// The wide path's contract: k % 128 == 0, 32-bit offsets, for Q4G fp16 scales
// groups of 32 or 64 columns (a slab's scales are whole dwords), fp32 scales
// any power-of-two multiple of 32; fp32 activations (split into an fp16 high
// part and an fp16 remainder after the LDS read, two MFMAs) take 64-column
// slabs, so Q4G only in groups of 32 there. It runs from
// m = 32 when its tiles number at least 128, and for every m > 128; otherwise
// the 16-row kernel, which streams the weight once per 64 rows of x, is faster
// (measured, k = 1536: m = 64, n = 8960 Q8 23.9 -> 12.0 us, Q4G 29.8 -> 15.0;
// m = 128 38.4 -> 17.9; m = 64, n = 1536 (24 tiles) 9.2 vs 11.8; long K with
// few tiles, m = 64, n = 1536, k = 8960: 40.4 vs 53.6).
template <bool Q4, typename XT, typename ST>
bool wq_wide_contract(int64_t m, int64_t n, int64_t k, int64_t group) {
    constexpr bool F32X = sizeof(XT) == 4;
    if (F32X && !wq_sk64_ok<Q4, ST>(group)) return false;
    if (k % 128 != 0 || m * k * static_cast<int64_t>(sizeof(XT)) >= (int64_t(1) << 31) - 64) return false;
    if (!Q4) return n * k < (int64_t(1) << 31) - 64;
    if (sizeof(ST) == 2 && group != 32 && group != 64) return false;
    return n * (k / 2) < (int64_t(1) << 31) - 64 && n * ((k + group - 1) / group) * int64_t(sizeof(ST)) < (int64_t(1) << 31) - 64;
}
template <bool Q4, typename XT, typename ST>
bool wq_wide_ok(int64_t m, int64_t n, int64_t k, int64_t group) {
    if (m < 32 || (m <= 128 && plan_wq_wide(m, n, wq_sk64_ok<Q4, ST>(group), sizeof(XT) == 4).tiles < 128)) return false;
    return wq_wide_contract<Q4, XT, ST>(m, n, k, group);
}

// Split-K, when the caller gives a workspace for the fp32 partial planes. A
// weight with few rows leaves most CUs idle, each workgroup walking all of K,
// so long K splits into up to kWqMaxSplits ranges summed by wq_reduce_kernel
// (a second launch and the planes' traffic). Wide split (k >= 2048, 16 <= m <=
// 128, fp32 x from m = 32): 64 x 64 tiles (64 x 128 above m = 64) with a
// two-slot LDS ring, so two or three workgroups share a CU (with the deep ring
// of the unsplit tiles, one workgroup of 8 waves per CU left the SIMDs waiting:
// n = 1536, k = 8960, m = 64 18.5 -> 15.5 us), about kWqWideSplitWgs workgroups
// of at least kWqMinSlabs slabs. It runs ahead of the unsplit wide tiles
// whenever it splits. Measured (us, unsplit -> split, fp16 / fp32 x): n = 1536,
// k = 8960: m = 16 20.6 -> 13.2, m = 64 43.4 -> 15.6 / 80.3 -> 25.0, m = 128
// 42.9 -> 21.1; n = 896, k = 4864, m = 64 25.1 -> 10.2; n = 8960, k = 4096, m =
// 16 27.3 -> 19.0, m = 64 28.5 -> 22.4; n = 4096, k = 4096, m = 128 28.4 ->
// 26.1 (m = 16 11.8 -> 12.7: the one loss kept; fp32 x at m = 16 lost 16.5 ->
// 23.1, the split kernel converting all 64 tile rows, hence m >= 32 there).
// From k = 2048 (was 4096), found on Qwen2.5-7B shapes (k = 3584, fp16 x, q4g /
// q8): m = 64, n = 4608 42.4 -> 16.6 / 36.0 -> 15.1; m = 64, n = 3584 23.0 ->
// 15.4; m = 32 22.5 -> 14.1; m = 16 19.0 -> 12.9; m = 128 30.0 -> 25.2; m = 64,
// n = 1536, k = 2048 14.7 -> 10.2. From k = 1024 lost at m = 16..32 and n = 8960
// (k = 1536, m = 16: 7.2 -> 9.3; m = 64, n = 8960: 15.4 -> 16.5).
// Otherwise the 16-row kernel splits when its unsplit grid is under 256
// workgroups and k >= 4096 (or at most 32 workgroups at m > 32 or fp32 x), to
// about kWqRowSplitWgs workgroups with at least two chunks per wave (n = 256,
// k = 1536, m = 64: 10.6 -> 8.7). Short K with a hundred or more workgroups
// stays whole (n = 1536, k = 1536, m = 64 split: 10.7 -> 11.6).
constexpr int kWqRowSplitWgs = 1024, kWqWideSplitWgs = 768, kWqMinSlabs = 4;
struct WqRoute {
    bool wide;
    WqTile tile;         // wide
    int splits, per;     // K ranges and slabs (wide) or chunks (16-row) per range
    WqRowPlan row;       // 16-row
};
WqRoute plan_wq_route(int64_t m, int64_t n, int64_t k, bool wide_ok, bool wide_contract, bool sk64_ok, bool f32x,
                      bool allow_split, bool q4) {
    WqRoute r{};
    // Past m = 128 the split tiles take over where the unsplit plan leaves under
    // 128 tiles (under 256 on K >= 8192) and the split tiles alone number under
    // 256 (us, fp16 x, Q8 / Q4G, unsplit -> split: m = 192, n = 1536, k = 8960
    // 51.1 -> 24.2 / 67.2 -> 24.5; m = 512, n = 896, k = 4864 29.9 -> 21.5 / 38.4
    // -> 23.3; m = 256, n = 2048, k = 8192 48.2 -> 33.9 / 61.9 -> 34.6; m = 512,
    // n = 1536, k = 8960 53.7 -> 44.8 / 67.5 -> 47.8; m = 1024 83.1 -> 76.6 /
    // 104.6 -> 80.8; fp32 x, m = 256: 150.4 -> 58.9 / 169.3 -> 56.3; m = 192, n =
    // 896, k = 4864 83.3 -> 25.8 / 93.5 -> 25.6). Not where the split tiles fill
    // the part already (m = 2048, n = 1536, k = 8960: 101.2 against 128.4) nor on
    // k = 4096 with 128 or more tiles (m = 192, n = 4096: no gain). From m = 65 the
    // split needs fewer than 256 split tiles: on wider weights the unsplit wide
    // tiles win (Q8 / Q4G, m = 128, k = 4096: n = 28672 85.8 -> 54.6 / 91.7 ->
    // 71.0; n = 17920, k = 2048 37.1 -> 25.1 / 39.3 -> 36.6; m = 100, n = 28672
    // 84.8 -> 57.0 / 87.2 -> 67.0; n = 37888, k = 3584 95.6 -> 69.4 / 99.3 ->
    // 101.7); at m <= 64 the split keeps them (m = 16, n = 28672, k = 4096, Q4G:
    // 47.5 against 80.7).
    const bool big_split = m > 128 && plan_wq_wide(m, n, sk64_ok, f32x).tiles < (k >= 8192 ? 256 : 128);
    if (allow_split && wide_contract && m >= (f32x ? 32 : q4 || k >= 8192 ? 5 : 9) && (m <= 128 || big_split) && k >= 2048) {
        WqTile t{1, m <= 64 ? 2 : 4, f32x ? 64 : 128};
        t.shallow = true;
        const int64_t tiles = ((m + 63) / 64) * ((n + 32 * t.fn - 1) / (32 * t.fn)), nk = k / t.sk;
        const int64_t sp = std::min<int64_t>({kWqMaxSplits, (kWqWideSplitWgs + tiles - 1) / tiles, nk / kWqMinSlabs});
        if (sp >= 2 && (m <= 64 || tiles < 256)) {
            const int64_t per = (nk + sp - 1) / sp;
            r.wide = true;
            r.tile = t;
            r.per = static_cast<int>(per);
            r.splits = static_cast<int>((nk + per - 1) / per);
            return r;
        }
    }
    if (wide_ok) {
        r.wide = true;
        r.tile = plan_wq_wide(m, n, sk64_ok, f32x).tile;
        r.splits = 1;
        r.per = static_cast<int>(k / r.tile.sk);
        return r;
    }
    WqRowPlan& p = r.row;
    p.tm = m > 64 ? 4 : static_cast<int>((m + 15) / 16);
    p.tn = p.tm <= 2 && n > 4096 ? 2 : 1;
    const int64_t chunks = k / 32, waves = p.tm == 1 ? 16 : 8;
    const int64_t wgs = (n + 16 * p.tn - 1) / (16 * p.tn) * ((m + 63) / 64);
    int64_t sp = 1;
    if (allow_split && wgs < 256 && (k >= 4096 || (wgs <= 32 && (m > 32 || f32x))))
        sp = std::max<int64_t>(1, std::min<int64_t>({(kWqRowSplitWgs + wgs - 1) / wgs, kWqMaxSplits, chunks / (2 * waves)}));
    p.per = static_cast<int>((chunks + sp - 1) / sp);
    p.splits = static_cast<int>((chunks + p.per - 1) / p.per);
    r.splits = p.splits;
    r.per = p.per;
    return r;
}
size_t wq_route_bytes(const WqRoute& r, int64_t m, int64_t n) {
    return r.splits > 1 ? round_up(static_cast<size_t>(r.splits) * static_cast<size_t>(m) * static_cast<size_t>(n) * 4, 256) : 0;
}
// m = 9..15 runs the GEMM from 1536 weight rows or on k <= 1024 (us, GEMV slices
// -> GEMM, m = 9 / 15, fp16 x: n = 3584, k = 3584 Q8 14.2 / 19.2 -> 8.9 / 10.0,
// Q4G 16.5 / 24.8 -> 11.6 / 12.4; n = k = 1536 Q8 7.2 / 8.5 -> 5.4 / 5.9; n = k =
// 896 Q4G 6.7 / 8.1 -> 4.9 / 5.1; fp32 x, n = 1536, k = 8960 Q8 19.5 / 28.2 -> 15.9
// / 17.7, Q4G 29.0 / 43.6 -> 18.7 / 20.6), and on narrower weights when a
// workspace lets fp16 activations take the split wide tiles: k >= 4096 and at
// least 6 Mi codes. GEMV slices stay on the rest (n = 896, k = 4864, fp16 x Q8
// 9.1 against 10.6, fp32 x 9.2 against 14.6; n = 256, k = 1536 5.7 against 6.5).
// int4 codes with fp16 x at m = 5..8 on a workspace: the split wide tiles (the
// GEMV re-reads the activation rows per two weight rows, and the unsplit GEMM
// converts and scales the codes per 64-row tile). us, GEMV -> split GEMM, m = 8:
// n = 28672, k = 4096 75.2 -> 50.7; n = 37888, k = 3584 86.5 -> 50.2; n = 4096,
// k = 14336 41.8 -> 27.0; n = 3584, k = 18944 45.6 -> 29.1; n = 8960, k = 3072
// 24.1 -> 18.6; n = 6144, k = 4096 19.9 -> 15.1; n = 4608, k = 3584 15.1 -> 12.7;
// n = 2048, k = 8192 12.9 -> 12.0. Kept on the GEMV: weights under 14 Mi codes
// (n = 1536, k = 8960 12.6 against 13.5; n = 2048, k = 4096 8.5 against 9.7;
// n = 3072, k = 4096 even), k < 3072 (n = 6144, k = 2048 10.9 against 12.1) and
// LM heads (n = 65536 even, n = 128256 280 against 296). Since the K-split tile
// GEMV (4096 <= k <= 18432, or from 3072 on 8192 rows) these tiles keep the rest of
// k < 4096 and k > 18432 (the tile GEMV, m =
// 8: n = 28672, k = 4096 49.0 -> 41.6; n = 4096, k = 14336 26.5 -> 24.5; n =
// 6144, k = 4096 15.7 -> 13.4; n = 37888, k = 3584 50.5 vs 51.9; n = 3584, k =
// 18944 stays 29.3 against 42.9).
bool wq_q4_batch5_shape(int64_t m, int64_t n, int64_t k) {
    return m >= 5 && m <= 8 && ((k >= 3072 && k < 4096 && n < 8192) || k > 18432) && k % 128 == 0 && n >= 2048 && n < 65536 &&
           n * k >= (int64_t(14) << 20);
}
// int8 codes with fp16 x at m = 5..8 on long K (k >= 8192) from 2048 rows: the
// split wide tiles too (us, m = 8, GEMV or unsplit GEMM -> split: n = 3584, k =
// 18944 39.0 -> 28.6; n = 2048, k = 16384 23.0 -> 15.6; n = 2048, k = 8192 13.5
// -> 10.8; n = 4096, k = 14336 25.0 -> 24.2; n = 1536, k = 8960 kept, 11.7
// against 12.2; shorter K kept, n = 3584, k = 3584 9.8 against 11.0).
// Since the K-split int8 tile GEMV (3072 <= k <= 9216, 12 Mi codes) these tiles
// and the unsplit GEMM above keep only k > 9216 and k < 4096 there (m = 8, us: n = 2048, k =
// 8192 10.8 -> 9.7; n = 8960, k = 5120 29.0 -> 20.7; n = 4096, k = 14336 stays,
// 24 against 38).
bool wq_q8_batch5_shape(int64_t m, int64_t n, int64_t k) {
    return m >= 5 && m <= 8 && k > 9216 && k % 128 == 0 && n >= 2048;
}
bool wq_gemm_shape_ok(int64_t m, int64_t n, int64_t k, size_t x_elem, bool ws) {
    return m > 8 && (m >= 16 || n >= 1536 || k <= 1024 ||
                     (ws && x_elem == 2 && k >= 4096 && k % 128 == 0 && n * k >= (int64_t(6) << 20)));
}
}  // namespace

// Whether the MFMA path takes this call (the caller runs GEMV slices otherwise):
// whole 32-column chunks, groups of a power-of-two number of chunks, 16-byte aligned operands and
// 32-bit buffer offsets.
// forced: the caller asked for this path (NQ_PATH_MFMA); only the operand contract applies.
bool wq_gemm_ok(bool q4, const void* x, size_t x_elem, const void* w, int64_t m, int64_t n, int64_t k,
                int64_t group, bool ws, bool forced) {
    const int64_t rowb = q4 ? k / 2 : k;
    // Shape rule (measured, wq_gemm_shape_ok): up to m = 15 a narrow weight with
    // long rows keeps GEMV slices of 8 rows plus a remainder slice.
    // int8 codes with fp16 x at m = 5..8 on large weights: the GEMV's per-row
    // FMAs make it VALU-bound there (m = 8, fp16 x, us, GEMV -> GEMM: n = 28672,
    // k = 4096 69.3 -> 46.0; n = 128256, k = 4096 279.5 -> 174.2; n = 4096, k =
    // 14336 37.8 -> 25.8; n = 17920, k = 1536 19.0 -> 14.8; n = 4096, k = 4096
    // 13.3 -> 10.4; m = 5, n = 28672 60.2 -> 43.6; smaller weights keep the GEMV:
    // n = 1536, k = 8960 11.7 -> 16.8). int4 codes with fp16 x: the split wide
    // tiles on wq_q4_batch5_shape when a workspace is given (the unsplit GEMM
    // gains nothing there).
    // fp32 x at m = 5..8 (int8 and int4 codes): the GEMM from n, k >= 4096 and on
    // the long K of the chunk-striding GEMVs (int8 k > 9216; int4 k > 18432 from
    // n = 3072), whose slices re-read 8 fp32 activation rows per workgroup (m = 8,
    // us, GEMV -> GEMM, int8 / int4: n = 4096, k = 14336 113.1 -> 35.5 / 119.6 ->
    // 44.7; n = 3584, k = 18944 128.8 -> 44.9 / 126.3 -> 56.9; n = 6144, k = 4096
    // 19.5 -> 17.4 / 29.4 -> 24.2; int8 n = 2048, k = 10240 37.0 -> 26.8; n = 1536,
    // k = 8960 keeps the GEMV: 14.6 against 22.9; int4 n = 1536, k = 9728 22.8
    // against 30.7). int4 codes with fp32 x on k <= 18432 now take the fp32 tile
    // GEMV instead (n = 8960, k = 5120 52.9 -> 45.6; n = 14336, k = 4096 46.2 ->
    // 45.0; n = 4096, k = 4096 16.8 -> 15.8).
    const bool batch5 = m >= 5 && m <= 8 &&
                        ((!q4 && x_elem == 2 && n >= 4096 && n * k >= (int64_t(16) << 20) && (k < 4096 || k > 9216)) ||
                         (q4 && x_elem == 2 && ws && group <= 64 && wq_q4_batch5_shape(m, n, k)) ||
                         (!q4 && x_elem == 2 && ws && wq_q8_batch5_shape(m, n, k)) ||
                         (x_elem == 4 && ((!q4 && n >= 4096 && k >= 4096) || (!q4 && k > 9216) ||
                                          (q4 && k > 18432 && n >= 3072))));
    if (!forced && !batch5 && !wq_gemm_shape_ok(m, n, k, x_elem, ws)) return false;
    return m > 0 && k > 0 && k % 32 == 0 && (!q4 || (group % 32 == 0 && ((group / 32) & (group / 32 - 1)) == 0)) && aligned(x, 16) && aligned(w, 16) &&
           m <= (int64_t(65535) * 64) && std::min<int64_t>(m, 64) * k * static_cast<int64_t>(x_elem) < (int64_t(1) << 31) - 64 &&
           n * rowb < (int64_t(1) << 31) - 64;
}

// All m rows in one launch: 64-row blocks of x over gridDim.y (each block
// streams the weight once).
template <bool Q4, typename XT, typename YT, typename ST>
nq_status wq_gemm(const XT* x, const uint8_t* w, const ST* sc, const float* b, YT* y, int64_t m, int64_t n,
                  int64_t k, int64_t group, void* workspace, size_t workspace_bytes, hipStream_t s) {
    const bool sk64 = wq_sk64_ok<Q4, ST>(group), f32x = sizeof(XT) == 4;
    const bool wide_ok = wq_wide_ok<Q4, XT, ST>(m, n, k, group), contract = wq_wide_contract<Q4, XT, ST>(m, n, k, group);
    WqRoute r = plan_wq_route(m, n, k, wide_ok, contract, sk64, f32x, workspace != nullptr, Q4);
    if (r.splits > 1 && workspace_bytes < wq_route_bytes(r, m, n))
        r = plan_wq_route(m, n, k, wide_ok, contract, sk64, f32x, false, Q4);
    float* planes = r.splits > 1 ? static_cast<float*>(workspace) : nullptr;
    const int mi = static_cast<int>(m), ni = static_cast<int>(n), ki = static_cast<int>(k), gi = static_cast<int>(group);
    if (r.wide) return wq_wide<Q4>(x, w, sc, b, y, mi, ni, ki, gi, r.tile, planes, r.splits, r.per, s);
    return launch_wq<Q4>(x, w, sc, b, y, mi, ni, ki, gi, r.row, planes, s);
}

// Workspace the split-K planes take at this shape (0: no split): the most any
// activation dtype or group size can plan, so one size serves every call.
size_t wq_workspace_bytes(int64_t m, int64_t n, int64_t k) {
    if (m <= 0 || n <= 0 || k <= 0 || !(wq_gemm_shape_ok(m, n, k, 2, true) || wq_q4_batch5_shape(m, n, k) ||
                                                   wq_q8_batch5_shape(m, n, k))) return 0;
    size_t most = 0;
    for (int f32x = 0; f32x < 2; ++f32x)
        for (int contract = 0; contract < 2; ++contract)
            for (int q4 = 0; q4 < 2; ++q4)
                most = std::max(most, wq_route_bytes(plan_wq_route(m, n, k, false, contract, true, f32x, true, q4), m, n));
    return most;
}

#define NQ_WQ_INST(Q4, XT, YT, ST)                                                                          \
    template nq_status wq_gemm<Q4, XT, YT, ST>(const XT*, const uint8_t*, const ST*, const float*, YT*, \
                                               int64_t, int64_t, int64_t, int64_t, void*, size_t, hipStream_t);
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
