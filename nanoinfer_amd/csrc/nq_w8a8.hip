// W8A8 GEMM on the gfx950 int8 matrix cores, plus the W8A8 entry points.
//
// xq [m, k] int8 (per-row dynamic quant) x wq [n, k] int8 (per-row weight
// quant) -> exact int32 accumulators -> y = float(acc)*a_scale*w_scale + b.
// Both operands are K-contiguous, which is exactly the per-lane layout of
// v_mfma_i32_16x16x64_i8: lane l supplies 16 consecutive K bytes of A row
// (l % 16) and of B column (l % 16) for K slice (l / 16); the 16x16 int32
// result lands as rows 4*(l/16)+v, column l%16, v = 0..3.
//
// Tiles: a workgroup of 4 waves owns a BM x BN output tile; its A/B K-slabs
// (64 bytes deep) are staged through LDS with a 16-byte row pad (80-byte row
// stride) so the ds_read_b128 operand fetches of the 16 rows of an MFMA tile
// spread over the banks. The next slab's global loads are issued before the
// current slab's MFMAs. Skinny m (batched decode, 16..64 rows) uses split-K:
// each K range adds its int32 partial tile into a zeroed workspace with
// atomic adds (integer addition is exact and order-free, so the result is
// bit-identical to a single pass), then a finalize pass applies the epilogue.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <type_traits>

#include "nq_device.hpp"
#include "nq_internal.hpp"

namespace nq {

nq_status gemv_w8a8_launch(const int8_t* xq, const float* as, const int8_t* w, const float* ws,
                           const float* bias, void* y, nq_dtype ydt, int32_t* acc_out, int64_t m,
                           int64_t n, int64_t k, bool generic, hipStream_t s);

namespace {

constexpr int kBK = 64;         // K bytes per MFMA step / LDS slab
constexpr int kLdsRow = kBK + 16;  // padded LDS row stride (bytes)
constexpr int kGemmThreads = 256;

enum class Out { Y, ACC, ATOMIC };

template <int BM, int BN, int WAVES_M, int WAVES_N, Out OUT, typename YT>
__global__ __launch_bounds__(kGemmThreads) void gemm_w8a8_mfma_kernel(
    const int8_t* __restrict__ xq, const float* __restrict__ as, const int8_t* __restrict__ wq,
    const float* __restrict__ ws, const float* __restrict__ bias, YT* __restrict__ y,
    int32_t* __restrict__ acc_out, int m, int n, int k, int k_split) {
    static_assert(WAVES_M * WAVES_N == 4, "4 waves per workgroup");
    constexpr int WM = BM / WAVES_M, WN = BN / WAVES_N;
    constexpr int TM = WM / 16, TN = WN / 16;
    static_assert(TM >= 1 && TN >= 1 && WM % 16 == 0 && WN % 16 == 0, "wave tile");
    constexpr int A_CHUNKS = BM * kBK / 16, B_CHUNKS = BN * kBK / 16;
    constexpr int A_PER = (A_CHUNKS + kGemmThreads - 1) / kGemmThreads;
    constexpr int B_PER = (B_CHUNKS + kGemmThreads - 1) / kGemmThreads;

    __shared__ __attribute__((aligned(16))) int8_t As[BM * kLdsRow];
    __shared__ __attribute__((aligned(16))) int8_t Bs[BN * kLdsRow];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave / WAVES_N, wn = wave % WAVES_N;
    const int m0 = blockIdx.y * BM, n0 = blockIdx.x * BN;
    const int kb = blockIdx.z * k_split;
    const int ke = min(k, kb + k_split);

    v4i ra[A_PER], rb[B_PER];
    auto load_slab = [&](int k0) {
#pragma unroll
        for (int i = 0; i < A_PER; ++i) {
            const int c = tid + i * kGemmThreads;
            const int row = c >> 2, kc = (c & 3) * 16;
            const bool ok = (A_CHUNKS % kGemmThreads == 0 || c < A_CHUNKS) && m0 + row < m && k0 + kc < ke;
            ra[i] = ok ? *reinterpret_cast<const v4i*>(xq + static_cast<size_t>(m0 + row) * k + k0 + kc)
                       : v4i{0, 0, 0, 0};
        }
#pragma unroll
        for (int i = 0; i < B_PER; ++i) {
            const int c = tid + i * kGemmThreads;
            const int row = c >> 2, kc = (c & 3) * 16;
            const bool ok = (B_CHUNKS % kGemmThreads == 0 || c < B_CHUNKS) && n0 + row < n && k0 + kc < ke;
            rb[i] = ok ? *reinterpret_cast<const v4i*>(wq + static_cast<size_t>(n0 + row) * k + k0 + kc)
                       : v4i{0, 0, 0, 0};
        }
    };
    auto store_slab = [&]() {
#pragma unroll
        for (int i = 0; i < A_PER; ++i) {
            const int c = tid + i * kGemmThreads;
            if (A_CHUNKS % kGemmThreads == 0 || c < A_CHUNKS)
                *reinterpret_cast<v4i*>(As + (c >> 2) * kLdsRow + (c & 3) * 16) = ra[i];
        }
#pragma unroll
        for (int i = 0; i < B_PER; ++i) {
            const int c = tid + i * kGemmThreads;
            if (B_CHUNKS % kGemmThreads == 0 || c < B_CHUNKS)
                *reinterpret_cast<v4i*>(Bs + (c >> 2) * kLdsRow + (c & 3) * 16) = rb[i];
        }
    };

    v4i acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = v4i{0, 0, 0, 0};

    const int frag_row = lane & 15, frag_k = (lane >> 4) * 16;
    if (kb < ke) load_slab(kb);
    for (int k0 = kb; k0 < ke; k0 += kBK) {
        store_slab();
        __syncthreads();
        if (k0 + kBK < ke) load_slab(k0 + kBK);
        v4i fa[TM], fb[TN];
#pragma unroll
        for (int i = 0; i < TM; ++i)
            fa[i] = *reinterpret_cast<const v4i*>(As + (wm * WM + i * 16 + frag_row) * kLdsRow + frag_k);
#pragma unroll
        for (int j = 0; j < TN; ++j)
            fb[j] = *reinterpret_cast<const v4i*>(Bs + (wn * WN + j * 16 + frag_row) * kLdsRow + frag_k);
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int j = 0; j < TN; ++j)
                acc[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(fa[i], fb[j], acc[i][j], 0, 0, 0);
        __syncthreads();
    }

#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) {
            const int col = n0 + wn * WN + j * 16 + (lane & 15);
            if (col >= n) continue;
            const float wsc = (OUT == Out::Y) ? ws[col] : 0.0f;
            const float b = (OUT == Out::Y && bias) ? bias[col] : 0.0f;
#pragma unroll
            for (int v = 0; v < 4; ++v) {
                const int row = m0 + wm * WM + i * 16 + (lane >> 4) * 4 + v;
                if (row >= m) continue;
                const size_t o = static_cast<size_t>(row) * n + col;
                if constexpr (OUT == Out::ATOMIC) {
                    atomicAdd(acc_out + o, acc[i][j][v]);
                } else if constexpr (OUT == Out::ACC) {
                    acc_out[o] = acc[i][j][v];
                } else {
                    y[o] = from_f32<YT>(w8a8_epilogue(acc[i][j][v], as[row], wsc, b));
                }
            }
        }
}

__global__ void fill_i32_kernel(int32_t* __restrict__ p, int64_t count) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i < count) p[i] = 0;
}

// ---- skinny W8A8 GEMM (3 <= m <= 64): batched decode ------------------------------------
// A workgroup owns TN 16-column MFMA tiles of weight rows and all m activation
// rows (TM 16-row tiles) over one K range; its waves take interleaved 64-byte K
// steps of that range, with operands loaded straight from global memory in the
// MFMA lane layout (weights streamed once, non-temporal; the small xq stays in
// L2) and three steps in flight per wave. The per-wave int32 partial tiles are
// added into one LDS tile with ds_add (exact, order-free). A single K range
// applies the epilogue directly. With several K ranges (very long K only) each
// range atomically adds its tile into a zeroed int32 accumulator and a separate
// finalize launch applies the epilogue: on this multi-XCD part, finishing inside
// the kernel would need agent-scope L2 writeback/invalidate fences, which cost
// far more than the extra launch.
template <int TM, int TN, Out OUT, typename YT>
__global__ __launch_bounds__(1024) void gemm_w8a8_skinny_kernel(
    const int8_t* __restrict__ xq, const float* __restrict__ as, const int8_t* __restrict__ wq,
    const float* __restrict__ ws, const float* __restrict__ bias, YT* __restrict__ y,
    int32_t* __restrict__ acc_out, int m, int n, int k, int k_split) {
    constexpr int PD = 3;  // steps in flight per wave
    __shared__ int tile[TM][TN][4][64];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, nthr = blockDim.x;
    const int nw = nthr >> 6;
    const int n0 = blockIdx.x * (TN * 16);
    const bool split = gridDim.y > 1;
    const int kb = blockIdx.y * k_split, ke = min(k, kb + k_split);
    const int fr = lane & 15, fk = (lane >> 4) * 16;
    for (int q = tid; q < TM * TN * 256; q += nthr) (&tile[0][0][0][0])[q] = 0;

    v4i acc[TM][TN];
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j) acc[i][j] = v4i{0, 0, 0, 0};

    auto load = [&](int k0, v4i (&a)[TM], v4i (&b)[TN]) {
        const bool kin = k0 + fk < ke;
#pragma unroll
        for (int i = 0; i < TM; ++i) {
            const int row = i * 16 + fr;
            a[i] = (kin && row < m) ? *reinterpret_cast<const v4i*>(xq + static_cast<size_t>(row) * k + k0 + fk)
                                    : v4i{0, 0, 0, 0};
        }
#pragma unroll
        for (int j = 0; j < TN; ++j) {
            const int col = n0 + j * 16 + fr;
            b[j] = (kin && col < n)
                       ? __builtin_nontemporal_load(reinterpret_cast<const v4i*>(wq + static_cast<size_t>(col) * k + k0 + fk))
                       : v4i{0, 0, 0, 0};
        }
    };
    const int kstep = nw * kBK;
    const int k0 = kb + wave * kBK;
    v4i a[PD][TM], b[PD][TN];
#pragma unroll
    for (int p = 0; p < PD; ++p) load(k0 + p * kstep, a[p], b[p]);
    for (int base = 0;; base += PD) {
        bool done = false;
#pragma unroll
        for (int p = 0; p < PD; ++p) {
            const int kc = k0 + (base + p) * kstep;
            if (kc >= ke) {
                done = true;
                break;
            }
#pragma unroll
            for (int i = 0; i < TM; ++i)
#pragma unroll
                for (int j = 0; j < TN; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a[p][i], b[p][j], acc[i][j], 0, 0, 0);
            load(kc + PD * kstep, a[p], b[p]);
        }
        if (done) break;
    }
    __syncthreads();  // tile zeroed
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
#pragma unroll
            for (int v = 0; v < 4; ++v) atomicAdd(&tile[i][j][v][lane], acc[i][j][v]);
    __syncthreads();
    for (int q = tid; q < TM * TN * 256; q += nthr) {
        const int l = q & 63, v = (q >> 6) & 3, j = (q >> 8) % TN, i = (q >> 8) / TN;
        const int row = i * 16 + (l >> 4) * 4 + v, col = n0 + j * 16 + (l & 15);
        if (row >= m || col >= n) continue;
        const int sum = tile[i][j][v][l];
        const size_t o = static_cast<size_t>(row) * n + col;
        if (split) {
            atomicAdd(acc_out + o, sum);
        } else if constexpr (OUT == Out::ACC) {
            acc_out[o] = sum;
        } else {
            const float bb = bias ? bias[col] : 0.0f;
            y[o] = from_f32<YT>(w8a8_epilogue(sum, as[row], ws[col], bb));
        }
    }
}

template <typename YT>
__global__ void w8a8_finalize_kernel(const int32_t* __restrict__ acc, const float* __restrict__ as,
                                     const float* __restrict__ ws, const float* __restrict__ bias,
                                     YT* __restrict__ y, int m, int n) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= static_cast<int64_t>(m) * n) return;
    const int row = static_cast<int>(i / n), col = static_cast<int>(i % n);
    const float b = bias ? bias[col] : 0.0f;
    y[i] = from_f32<YT>(w8a8_epilogue(acc[i], as[row], ws[col], b));
}

// ---- plans --------------------------------------------------------------------------
constexpr int kTargetBlocks = 1024;  // ~4 workgroups per CU on 256 CUs
constexpr int kSkinnyMaxM = 64;

// Large m: 128x128 tiles, K split (atomic int32 accumulation) only when the
// tile count alone cannot fill the chip.
struct BigPlan {
    int splits, k_split;
};
BigPlan plan_big(int64_t m, int64_t n, int64_t k) {
    const int64_t tiles = ((m + 127) / 128) * ((n + 127) / 128);
    const int64_t kslabs = (k + kBK - 1) / kBK;
    int64_t splits = 1;
    if (tiles < kTargetBlocks / 4) splits = std::min<int64_t>((kTargetBlocks / 4 + tiles - 1) / tiles, std::max<int64_t>(1, kslabs / 4));
    const int64_t per = (kslabs + splits - 1) / splits;
    BigPlan p;
    p.k_split = static_cast<int>(std::max<int64_t>(1, per) * kBK);
    p.splits = static_cast<int>(std::max<int64_t>(1, (k + p.k_split - 1) / p.k_split));
    return p;
}

// Skinny m: 32 columns per workgroup when that still gives >= 128 workgroups,
// else 16; waves for about three K steps each (4..16). K is split across
// workgroups only when one range would leave a wave more than 6 steps.
struct SkinnyPlan {
    int tm, tn, ntiles, splits, k_split, waves;
    size_t acc_bytes;
};
SkinnyPlan plan_skinny(int64_t m, int64_t n, int64_t k) {
    SkinnyPlan p{};
    p.tm = static_cast<int>((m + 15) / 16);
    p.tn = (n + 31) / 32 >= 128 ? 2 : 1;
    p.ntiles = static_cast<int>((n + 16 * p.tn - 1) / (16 * p.tn));
    const int64_t kslabs = (k + kBK - 1) / kBK;
    const int64_t splits = std::max<int64_t>(1, (kslabs + 16 * 6 - 1) / (16 * 6));
    const int64_t per = (kslabs + splits - 1) / splits;
    p.k_split = static_cast<int>(per * kBK);
    p.splits = static_cast<int>((k + p.k_split - 1) / p.k_split);
    p.waves = static_cast<int>(std::min<int64_t>(16, std::max<int64_t>(4, (per + 2) / 3)));
    if (p.splits > 1) p.acc_bytes = round_up(static_cast<size_t>(m * n) * 4, 256);
    return p;
}

size_t gemm_ws_bytes(int64_t m, int64_t n, int64_t k) {
    if (m <= 0 || n <= 0 || k <= 0) return 0;
    if (m <= kSkinnyMaxM) {
        return plan_skinny(m, n, k).acc_bytes;
    }
    const BigPlan p = plan_big(m, n, k);
    return p.splits > 1 ? round_up(static_cast<size_t>(m * n) * 4, 256) : 0;
}

// Skinny launch. zeroed: a split plan's accumulator was already cleared by
// this call's activation-quant kernel; else it is cleared here.
nq_status gemm_skinny(const int8_t* xq, const float* as, const int8_t* wq, const float* ws,
                      const float* bias, void* y, nq_dtype ydt, int32_t* acc_out, int64_t m,
                      int64_t n, int64_t k, void* workspace, size_t ws_bytes, bool zeroed,
                      hipStream_t s) {
    const SkinnyPlan p = plan_skinny(m, n, k);
    int32_t* accum = acc_out;
    if (p.splits > 1) {
        if (!acc_out) {
            NQ_REQUIRE(workspace && ws_bytes >= p.acc_bytes, NQ_BAD_ARG,
                       "w8a8 gemm: workspace of %zu bytes required, %zu given", p.acc_bytes, ws_bytes);
            NQ_REQUIRE(aligned(workspace, 256), NQ_BAD_ALIGN, "w8a8 gemm: workspace must be 256-byte aligned");
            accum = static_cast<int32_t*>(workspace);
        }
        if (!zeroed || acc_out) {
            fill_i32_kernel<<<static_cast<unsigned>((m * n + 255) / 256), 256, 0, s>>>(accum, m * n);
            if (nq_status st = launch_status("fill_i32_kernel")) return st;
        }
    }
    const dim3 grid(static_cast<unsigned>(p.ntiles), static_cast<unsigned>(p.splits));
    const int threads = p.waves * 64;
    const int mi = static_cast<int>(m), ni = static_cast<int>(n), ki = static_cast<int>(k);
    auto go = [&](auto tmtag, auto tntag) {
        constexpr int TM = decltype(tmtag)::value, TN = decltype(tntag)::value;
        if (acc_out || p.splits > 1)
            gemm_w8a8_skinny_kernel<TM, TN, Out::ACC, float><<<grid, threads, 0, s>>>(xq, as, wq, ws, bias, nullptr, accum, mi, ni, ki, p.k_split);
        else if (ydt == NQ_F32)
            gemm_w8a8_skinny_kernel<TM, TN, Out::Y, float><<<grid, threads, 0, s>>>(xq, as, wq, ws, bias, static_cast<float*>(y), nullptr, mi, ni, ki, p.k_split);
        else
            gemm_w8a8_skinny_kernel<TM, TN, Out::Y, _Float16><<<grid, threads, 0, s>>>(xq, as, wq, ws, bias, static_cast<_Float16*>(y), nullptr, mi, ni, ki, p.k_split);
    };
    auto with_tn = [&](auto tmtag) {
        if (p.tn == 1) go(tmtag, std::integral_constant<int, 1>{});
        else go(tmtag, std::integral_constant<int, 2>{});
    };
    switch (p.tm) {
        case 1: with_tn(std::integral_constant<int, 1>{}); break;
        case 2: with_tn(std::integral_constant<int, 2>{}); break;
        case 3: with_tn(std::integral_constant<int, 3>{}); break;
        default: with_tn(std::integral_constant<int, 4>{}); break;
    }
    if (nq_status st = launch_status("gemm_w8a8_skinny_kernel")) return st;
    if (p.splits > 1 && !acc_out) {
        const unsigned g = static_cast<unsigned>((m * n + 255) / 256);
        if (ydt == NQ_F32)
            w8a8_finalize_kernel<float><<<g, 256, 0, s>>>(accum, as, ws, bias, static_cast<float*>(y), mi, ni);
        else
            w8a8_finalize_kernel<_Float16><<<g, 256, 0, s>>>(accum, as, ws, bias, static_cast<_Float16*>(y), mi, ni);
        return launch_status("w8a8_finalize_kernel");
    }
    return NQ_OK;
}

// Big-m launch (128x128 tiles).
nq_status gemm_big(const int8_t* xq, const float* as, const int8_t* wq, const float* ws,
                   const float* bias, void* y, nq_dtype ydt, int32_t* acc_out, int64_t m, int64_t n,
                   int64_t k, void* workspace, size_t ws_bytes, hipStream_t s) {
    const BigPlan p = plan_big(m, n, k);
    const int mi = static_cast<int>(m), ni = static_cast<int>(n), ki = static_cast<int>(k);
    dim3 grid(static_cast<unsigned>((n + 127) / 128), static_cast<unsigned>((m + 127) / 128),
              static_cast<unsigned>(p.splits));
    if (p.splits == 1) {
        if (acc_out)
            gemm_w8a8_mfma_kernel<128, 128, 2, 2, Out::ACC, float><<<grid, kGemmThreads, 0, s>>>(xq, as, wq, ws, bias, nullptr, acc_out, mi, ni, ki, p.k_split);
        else if (ydt == NQ_F32)
            gemm_w8a8_mfma_kernel<128, 128, 2, 2, Out::Y, float><<<grid, kGemmThreads, 0, s>>>(xq, as, wq, ws, bias, static_cast<float*>(y), nullptr, mi, ni, ki, p.k_split);
        else
            gemm_w8a8_mfma_kernel<128, 128, 2, 2, Out::Y, _Float16><<<grid, kGemmThreads, 0, s>>>(xq, as, wq, ws, bias, static_cast<_Float16*>(y), nullptr, mi, ni, ki, p.k_split);
        return launch_status("gemm_w8a8_mfma_kernel");
    }
    const size_t need = round_up(static_cast<size_t>(m * n) * 4, 256);
    int32_t* acc = acc_out;
    if (!acc) {
        NQ_REQUIRE(workspace && ws_bytes >= need, NQ_BAD_ARG,
                   "w8a8 gemm: workspace of %zu bytes required, %zu given", need, ws_bytes);
        NQ_REQUIRE(aligned(workspace, 4), NQ_BAD_ALIGN, "w8a8 gemm: misaligned workspace");
        acc = static_cast<int32_t*>(workspace);
    }
    const int64_t count = m * n;
    fill_i32_kernel<<<static_cast<unsigned>((count + 255) / 256), 256, 0, s>>>(acc, count);
    gemm_w8a8_mfma_kernel<128, 128, 2, 2, Out::ATOMIC, float><<<grid, kGemmThreads, 0, s>>>(xq, as, wq, ws, bias, nullptr, acc, mi, ni, ki, p.k_split);
    if (nq_status st = launch_status("gemm_w8a8_mfma_kernel(split)")) return st;
    if (!acc_out) {
        const unsigned g = static_cast<unsigned>((count + 255) / 256);
        if (ydt == NQ_F32)
            w8a8_finalize_kernel<float><<<g, 256, 0, s>>>(acc, as, ws, bias, static_cast<float*>(y), mi, ni);
        else
            w8a8_finalize_kernel<_Float16><<<g, 256, 0, s>>>(acc, as, ws, bias, static_cast<_Float16*>(y), mi, ni);
    }
    return launch_status("w8a8_finalize_kernel");
}

nq_status check_w8a8(int64_t m, int64_t n, int64_t k, int path, const char* who) {
    NQ_REQUIRE(m >= 0 && n >= 0 && k >= 0, NQ_BAD_SHAPE, "%s: negative shape", who);
    NQ_REQUIRE(m <= kMaxIndex && n <= kMaxIndex && k <= kMaxIndex && m * k <= (int64_t(1) << 40) &&
                   n * k <= (int64_t(1) << 40) && m * n <= (int64_t(1) << 40),
               NQ_BAD_SHAPE, "%s: shape m=%lld n=%lld k=%lld exceeds the supported range", who,
               (long long)m, (long long)n, (long long)k);
    // |acc| <= k * 127^2 must stay below 2^31 for the int32 core to be exact.
    NQ_REQUIRE(k <= 133152, NQ_BAD_SHAPE, "%s: k=%lld overflows the int32 accumulator", who, (long long)k);
    NQ_REQUIRE(path >= NQ_PATH_AUTO && path <= NQ_PATH_GENERIC, NQ_BAD_ARG, "%s: unknown path %d", who, path);
    return NQ_OK;
}

bool mfma_ok(const int8_t* xq, const int8_t* wq, int64_t k) {
    return k > 0 && k % 16 == 0 && aligned(xq, 16) && aligned(wq, 16);
}

// AUTO: the v_dot4 GEMV only at m <= 2 (its per-row dot work grows with m while
// one 16x16x64 MFMA covers 16 activation rows), the MFMA kernels above.
int resolve_path(int path, int64_t m) {
    return path == NQ_PATH_AUTO ? (m <= 2 ? NQ_PATH_GEMV : NQ_PATH_MFMA) : path;
}

// Runs the chosen path on pre-quantized activations.
nq_status run_gemm(const int8_t* xq, const float* as, const int8_t* wq, const float* ws,
                   const float* bias, void* y, nq_dtype ydt, int32_t* acc_out, int64_t m,
                   int64_t n, int64_t k, void* workspace, size_t ws_bytes, int path, bool zeroed,
                   hipStream_t s) {
    int p = resolve_path(path, m);
    if (p == NQ_PATH_MFMA && !mfma_ok(xq, wq, k)) p = NQ_PATH_GENERIC;
    if (p == NQ_PATH_MFMA) {
        if (m <= kSkinnyMaxM)
            return gemm_skinny(xq, as, wq, ws, bias, y, ydt, acc_out, m, n, k, workspace, ws_bytes, zeroed, s);
        return gemm_big(xq, as, wq, ws, bias, y, ydt, acc_out, m, n, k, workspace, ws_bytes, s);
    }
    if (p == NQ_PATH_GEMV && m > 8) {
        // The GEMV holds at most 8 activation rows; larger m runs in slices of 8.
        for (int64_t r0 = 0; r0 < m; r0 += 8) {
            const int64_t mm = std::min<int64_t>(8, m - r0);
            char* yp = y ? static_cast<char*>(y) + static_cast<size_t>(r0 * n) * dtype_size(ydt) : nullptr;
            if (nq_status st = gemv_w8a8_launch(xq + r0 * k, as ? as + r0 : nullptr, wq, ws, bias, yp, ydt,
                                                acc_out ? acc_out + r0 * n : nullptr, mm, n, k, false, s))
                return st;
        }
        return NQ_OK;
    }
    return gemv_w8a8_launch(xq, as, wq, ws, bias, y, ydt, acc_out, m, n, k, p == NQ_PATH_GENERIC, s);
}

}  // namespace
}  // namespace nq

using namespace nq;

namespace nq {
nq_status act_quant(const void* x, nq_dtype xdt, int64_t m, int64_t k, int8_t* xq, float* as,
                    void* zero, size_t zero_bytes, hipStream_t s);
bool gemv_w8a8_fused_launch(const void* x, nq_dtype xdt, const int8_t* w, const float* ws,
                            const float* bias, void* y, nq_dtype ydt, int64_t m, int64_t n,
                            int64_t k, hipStream_t s, nq_status* st);

}  // namespace nq

extern "C" size_t nq_gemm_w8a8_workspace_size(int64_t m, int64_t n, int64_t k) {
    return gemm_ws_bytes(m, n, k);
}

extern "C" size_t nq_linear_w8a8_workspace_size(int64_t m, int64_t n, int64_t k) {
    if (m <= 0) return 0;
    return round_up(static_cast<size_t>(m * k), 256) + round_up(static_cast<size_t>(m) * 4, 256) +
           gemm_ws_bytes(m, n, k);
}

extern "C" nq_status nq_gemm_w8a8(const int8_t* xq, const float* a_scale, const int8_t* wq,
                                  const float* w_scale, const float* bias, void* y,
                                  nq_dtype y_dtype, int64_t m, int64_t n, int64_t k,
                                  void* workspace, size_t workspace_bytes, int path,
                                  void* stream) {
    if (nq_status st = check_w8a8(m, n, k, path, "gemm_w8a8")) return st;
    NQ_REQUIRE(dtype_ok(y_dtype), NQ_BAD_ARG, "gemm_w8a8: unknown y dtype");
    if (m == 0 || n == 0) return NQ_OK;
    NQ_REQUIRE(y && a_scale && w_scale && (k == 0 || (xq && wq)), NQ_BAD_ARG, "gemm_w8a8: null pointer");
    NQ_REQUIRE(aligned(y, dtype_size(y_dtype)) && aligned(a_scale, 4) && aligned(w_scale, 4) &&
                   aligned(bias, 4),
               NQ_BAD_ALIGN, "gemm_w8a8: misaligned pointer");
    return run_gemm(xq, a_scale, wq, w_scale, bias, y, y_dtype, nullptr, m, n, k, workspace,
                    workspace_bytes, path, false, as_stream(stream));
}

extern "C" nq_status nq_w8a8_acc_i32(const int8_t* xq, const int8_t* wq, int32_t* acc, int64_t m,
                                     int64_t n, int64_t k, void* workspace, size_t workspace_bytes,
                                     int path, void* stream) {
    if (nq_status st = check_w8a8(m, n, k, path, "w8a8_acc_i32")) return st;
    if (m == 0 || n == 0) return NQ_OK;
    NQ_REQUIRE(acc && (k == 0 || (xq && wq)), NQ_BAD_ARG, "w8a8_acc_i32: null pointer");
    NQ_REQUIRE(aligned(acc, 4), NQ_BAD_ALIGN, "w8a8_acc_i32: misaligned acc");
    return run_gemm(xq, nullptr, wq, nullptr, nullptr, nullptr, NQ_F32, acc, m, n, k, workspace,
                    workspace_bytes, path, false, as_stream(stream));
}

extern "C" nq_status nq_linear_w8a8(const void* x, nq_dtype x_dtype, const int8_t* wq,
                                    const float* w_scale, const float* bias, void* y,
                                    nq_dtype y_dtype, int64_t m, int64_t n, int64_t k,
                                    void* workspace, size_t workspace_bytes, int path,
                                    void* stream) {
    if (nq_status st = check_w8a8(m, n, k, path, "linear_w8a8")) return st;
    NQ_REQUIRE(dtype_ok(x_dtype) && dtype_ok(y_dtype), NQ_BAD_ARG, "linear_w8a8: unknown dtype");
    if (m == 0 || n == 0) return NQ_OK;
    NQ_REQUIRE(y && w_scale && (k == 0 || (x && wq)), NQ_BAD_ARG, "linear_w8a8: null pointer");
    NQ_REQUIRE(aligned(x, dtype_size(x_dtype)) && aligned(y, dtype_size(y_dtype)) &&
                   aligned(w_scale, 4) && aligned(bias, 4),
               NQ_BAD_ALIGN, "linear_w8a8: misaligned pointer");
    const size_t need = nq_linear_w8a8_workspace_size(m, n, k);
    NQ_REQUIRE(workspace && workspace_bytes >= need, NQ_BAD_ARG,
               "linear_w8a8: workspace of %zu bytes required, %zu given", need, workspace_bytes);
    NQ_REQUIRE(aligned(workspace, 256), NQ_BAD_ALIGN, "linear_w8a8: workspace must be 256-byte aligned");
    hipStream_t s = as_stream(stream);
    const int p = resolve_path(path, m);
    if (p == NQ_PATH_GEMV) {
        nq_status st = NQ_OK;
        if (gemv_w8a8_fused_launch(x, x_dtype, wq, w_scale, bias, y, y_dtype, m, n, k, s, &st)) return st;
    }
    char* base = static_cast<char*>(workspace);
    int8_t* xq = reinterpret_cast<int8_t*>(base);
    float* as = reinterpret_cast<float*>(base + round_up(static_cast<size_t>(m * k), 256));
    char* rest = reinterpret_cast<char*>(as) + round_up(static_cast<size_t>(m) * 4, 256);
    const size_t rest_bytes = workspace_bytes - static_cast<size_t>(rest - base);
    // A split skinny plan needs its accumulator cleared: the activation-quant
    // launch does it with extra workgroups.
    void* zero = nullptr;
    size_t zero_bytes = 0;
    if (p == NQ_PATH_MFMA && m <= kSkinnyMaxM && mfma_ok(xq, wq, k)) {
        const SkinnyPlan sp = plan_skinny(m, n, k);
        if (sp.splits > 1) {
            zero = rest;
            zero_bytes = sp.acc_bytes;
        }
    }
    if (nq_status st = act_quant(x, x_dtype, m, k, xq, as, zero, zero_bytes, s)) return st;
    return run_gemm(xq, as, wq, w_scale, bias, y, y_dtype, nullptr, m, n, k, rest, rest_bytes, p,
                    zero_bytes > 0, s);
}
