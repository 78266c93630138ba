// Decode GEMVs (m <= 8): weight-only int8, group-wise int4, and W8A8.
//
// Mapping (all three kernels): one workgroup owns R output rows and the whole
// K extent of those rows. K is cut into 16-byte chunks (16 int8 codes, or 32
// packed int4 codes); thread t of the workgroup owns chunk t of every one of
// the R rows, so each lane issues R independent global_load_dwordx4 up front
// (coalesced: the 64 lanes of a wave read 1 KiB contiguous per row) and reuses
// the activation chunk it loads for all R rows. Per-lane partials are reduced
// across the wave with DPP and the gfx950 row swaps, across waves through LDS in a fixed
// order (deterministic), then scaled once per row at the store — the reference
// "accumulate then scale" order (quant.cpp:155-161, cuda_quant.cu:217-235).
//
// Shapes outside the fast path (k not a multiple of the chunk, misaligned
// pointers, k beyond the chunk budget of one workgroup) run a generic
// bounds-checked wave-per-row kernel with the same arithmetic.
#include <hip/hip_runtime.h>

#include <type_traits>

#include "nq_device.hpp"
#include "nq_internal.hpp"

namespace nq {
bool wq_gemm_ok(bool q4, const void* x, size_t x_elem, const void* w, int64_t m, int64_t n, int64_t k,
                int64_t group, bool ws, bool forced = false);
template <bool Q4, typename XT, typename YT, typename ST>
nq_status wq_gemm(const XT* x, const uint8_t* w, const ST* sc, const float* b, YT* y, int64_t m, int64_t n,
                  int64_t k, int64_t group, void* workspace, size_t workspace_bytes, hipStream_t s);
size_t wq_workspace_bytes(int64_t m, int64_t n, int64_t k);

namespace {

constexpr int kMaxGemvWaves = 9;          // 576 lanes: int8 k <= 9216, int4 k <= 18432
constexpr int kMaxGemvThreads = kMaxGemvWaves * kWave;
// The long-K kernels' workgroups (several chunks per lane): int8 weight-only
// 256 lanes; int4 and W8A8 512 (m = 1, us, 256 -> 512 lanes: int4 n = 3584, k =
// 18944 11.5 -> 10.7, n = 4096, k = 28672 16.6 -> 15.8; W8A8 n = 3584, k = 18944
// 18.6 -> 18.0; int8 lost: n = 4096, k = 14336 12.8 -> 13.1, m = 4 3-7%).
constexpr int kLongKThreads = 256, kLongKThreadsWide = 512;

// Rows per workgroup as a function of the activation-row count: more rows =
// more reuse of each loaded activation chunk, fewer = more workgroups.
template <int M>
constexpr int rows_for() {
    return M <= 2 ? 4 : 2;
}

// W8A8 GEMV: every workgroup reads all M activation rows of its K range, so
// R >= M rows per workgroup keeps those reads at or below the weight bytes.
template <int M>
constexpr int w8a8_rows_for() {
    return M <= 4 ? 4 : M;
}

// Wave-reduces the R x M accumulators and leaves the wave totals in
// red[wave][r * M + i] (one exchange network for all of them).
// BPERM: exchanges through ds_bpermute instead of DPP / row swaps (see
// wave_reduce_stage_bperm), for the kernels whose all-VALU reduction spilled.
template <int R, int M, bool BPERM = false, typename T>
__device__ __forceinline__ T wave_reduce_rows(T (&acc)[R][M], int lane) {
    constexpr int NV = R * M;
    if constexpr (NV == 1) {
        if constexpr (std::is_floating_point_v<T>) return wave_sum_f32(acc[0][0]);
        else return wave_sum_i32(acc[0][0]);
    } else {
        T v[NV];
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
            for (int i = 0; i < M; ++i) v[r * M + i] = acc[r][i];
        if constexpr (BPERM) wave_reduce_stage_bperm<NV, 32>(v, lane);
        else wave_reduce_multi<NV>(v, lane);
        return v[0];
    }
}
// The wave's total of value j = r * M + i is in lane j * (64 / (R * M)).
template <int R, int M, bool BPERM = false, typename T>
__device__ __forceinline__ void reduce_to_lds(T (&acc)[R][M], T* red, int wave, int lane) {
    constexpr int NV = R * M, G = 64 / NV;
    const T v = wave_reduce_rows<R, M, BPERM>(acc, lane);
    if (lane % G == 0) red[wave * NV + lane / G] = v;
}

// ---- activation chunk loaders ------------------------------------------------------
// One lane's 16-element activation chunk as raw vector registers. Every load in
// the kernels below is unconditional (lanes past the last chunk re-read chunk 0,
// activation rows past m re-read row m - 1, and their partial sums are dropped
// by a select), so the compiler issues all weight, scale and activation loads of
// a lane back to back and the lane waits for memory once.
template <typename XT>
struct XChunk;
template <>
struct XChunk<float> {
    f4 v[4];
    __device__ __forceinline__ void load(const float* p) {
        const f4* q = reinterpret_cast<const f4*>(p);
#pragma unroll
        for (int i = 0; i < 4; ++i) v[i] = q[i];
    }
    __device__ __forceinline__ float at(int e) const { return v[e >> 2][e & 3]; }
};
template <>
struct XChunk<_Float16> {
    typedef _Float16 h8 __attribute__((ext_vector_type(8)));
    h8 v[2];
    __device__ __forceinline__ void load(const _Float16* p) {
        const h8* q = reinterpret_cast<const h8*>(p);
        v[0] = q[0];
        v[1] = q[1];
    }
    __device__ __forceinline__ float at(int e) const { return static_cast<float>(v[e >> 3][e & 7]); }
};

// Greedy-argmax partial of a run of logits: the best (value, index) by
// "greater value, then smaller index" over the non-NaN values, i.e. the
// reference's left-to-right scan with a strict > (sampling.cpp:14-20); i ==
// INT_MAX when the run holds no non-NaN value. i == -1 flags that logit 0 is
// NaN, which makes that scan return 0 whatever follows.
struct ArgPart {
    float v;
    int i;
};
constexpr int kArgNone = 0x7FFFFFFF;
// Per activation row of the fused LM head: the running best as one 64-bit key
// (order-preserving bits of the value above, 0xFFFFFFFF - index below, so the
// larger key is the larger value and, on ties, the smaller index; all ones:
// logit 0 is NaN; 0: no candidate) and the count of final workgroups done. The
// GEMV zeroes both; the final kernel's device-scope atomics update them.
struct ArgCtl {
    unsigned long long key;
    unsigned ticket, pad;
};
constexpr int kArgCtlBytes = 256;  // 8 rows, at the start of the fused path's workspace
__device__ __forceinline__ bool arg_better(float v, int i, float bv, int bi) {
    return v > bv || (v == bv && i < bi);
}

// Row group of this workgroup. Workgroup ids are dealt round-robin over the 8
// XCDs; numbering the groups so that XCD x takes a contiguous run of them keeps
// each output line written by one XCD (its L2 holds whole dirty lines instead
// of eight partial copies that meet at write-back): int4 GEMV at k = 8960,
// n = 1536 4.65 -> 4.56 us. Block 0 keeps group 0.
__device__ __forceinline__ int xcd_row_group() {
    const int g = gridDim.x, per = (g + 7) / 8, xcd = blockIdx.x % 8, idx = blockIdx.x / 8;
    const int full = g - 8 * (per - 1);  // XCDs [0, full) take `per` groups, the rest per - 1
    return xcd < full ? xcd * per + idx : full * per + (xcd - full) * (per - 1) + idx;
}

// ---- weight-only int8 ------------------------------------------------------------
// AM: instead of storing y, reduce this workgroup's R logits of each activation
// row to an ArgPart (part[i * gridDim.x + blockIdx.x]); the logits are the same
// fp32 values the plain kernel would store, so argmax(fused) == argmax(y).
// XS > 1: XS workgroups per row group, each taking M of the activation rows
// (neighbouring indices of xcd_row_group, so the XS readers of a weight row
// group run together on one XCD and share its L2).
// MAXT: the launch bound (576 threads, or 1024 for one fp16 row on 9216 < k <= 12288).
template <int R, int M, typename XT, typename YT, bool AM = false, int XS = 1, int MAXT = kMaxGemvThreads>
__global__ __launch_bounds__(MAXT) void gemv_q8_kernel(
    const XT* __restrict__ x, const int8_t* __restrict__ w, const float* __restrict__ ws,
    const float* __restrict__ bias, YT* __restrict__ y, int m, int n, int k, ArgPart* __restrict__ part,
    ArgCtl* __restrict__ ctl) {
    static_assert(XS == 1 || !AM, "activation slices write y");
    __shared__ float red[(MAXT / kWave) * R * M];
    const int tid = threadIdx.x, wave = tid >> 6, nw = block_threads() >> 6;
    const int chunks = k >> 4;
    const bool act = tid < chunks;
    int rg = xcd_row_group();
    if constexpr (XS > 1) {
        const int sl = rg % XS;  // rows [sl * M, sl * M + M) of x and y; m > (XS - 1) * M
        rg /= XS;
        x += static_cast<size_t>(sl) * M * k;
        y += static_cast<size_t>(sl) * M * n;
        m -= sl * M;
    }
    const int row0 = rg * R;

    const int c = act ? tid : 0;
    // One or two activation rows: their chunks are requested first and the
    // weight rows after them in order, so each row's dot starts when its own
    // load lands (as the int4 GEMV).
    constexpr bool kXFirst = M <= 2;
    XChunk<XT> xc[M];
    if constexpr (kXFirst) {
#pragma unroll
        for (int i = 0; i < M; ++i) xc[i].load(x + static_cast<size_t>(min(i, m - 1)) * k + c * 16);
        __builtin_amdgcn_sched_barrier(0);
    }
    v4i wv[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const int row = min(row0 + r, n - 1);
        wv[r] = __builtin_nontemporal_load(reinterpret_cast<const v4i*>(w + static_cast<size_t>(row) * k + c * 16));
        if constexpr (kXFirst) __builtin_amdgcn_sched_barrier(0);
    }
    if constexpr (!kXFirst) {
#pragma unroll
        for (int i = 0; i < M; ++i) xc[i].load(x + static_cast<size_t>(min(i, m - 1)) * k + c * 16);
    }
    // The weight scale of the row this lane may store, requested behind the
    // weights instead of after the reduction, where the load of a cold scale
    // line would add its latency to every workgroup's end (n = 4864, k = 896,
    // fp32 x: 3.39 -> 3.28 us; k = 1536, n = 8960 fp16 5.06 -> 4.92).
    constexpr int G1 = 64 / (R * M);
    const int er = (!AM && nw == 1) ? (tid & 63) / G1 / M : tid / M;
    const float ws_early = ws[min(row0 + min(er, R - 1), n - 1)];

    float acc[R][M];
#pragma unroll
    for (int i = 0; i < M; ++i) {
#pragma unroll
        for (int r = 0; r < R; ++r) {
            float p = 0.0f;
#pragma unroll
            for (int d = 0; d < 4; ++d) {
                const int wd = wv[r][d];
                p = __builtin_fmaf(xc[i].at(4 * d + 0), sbyte_f32<0>(wd), p);
                p = __builtin_fmaf(xc[i].at(4 * d + 1), sbyte_f32<1>(wd), p);
                p = __builtin_fmaf(xc[i].at(4 * d + 2), sbyte_f32<2>(wd), p);
                p = __builtin_fmaf(xc[i].at(4 * d + 3), sbyte_f32<3>(wd), p);
            }
            acc[r][i] = act ? p : 0.0f;
        }
    }
    if (!AM && nw == 1) {
        // One wave (k <= 1024): its lanes hold the row totals after the exchange;
        // no LDS round trip and no barrier.
        constexpr int G = 64 / (R * M);
        const float v = wave_reduce_rows<R, M>(acc, tid);
        if (tid % G == 0) {
            const int j = tid / G, r = j / M, i = j % M, row = row0 + r;
            if (row < n && i < m) {
                const float b = bias ? bias[row] : 0.0f;
                y[static_cast<size_t>(i) * n + row] = from_f32<YT>(__builtin_fmaf(v, ws_early, b));
            }
        }
        return;
    }
    reduce_to_lds<R, M>(acc, red, wave, tid & 63);
    __syncthreads();
    if constexpr (AM) {
        __shared__ float logit[R * M];
        if (tid < R * M) {
            const int r = tid / M, i = tid % M, row = row0 + r;
            if (row < n && i < m) {
                float s = 0.0f;
                for (int wv_i = 0; wv_i < nw; ++wv_i) s += red[(wv_i * R + r) * M + i];
                const float b = bias ? bias[row] : 0.0f;
                logit[r * M + i] = __builtin_fmaf(s, ws_early, b);
            }
        }
        __syncthreads();
        if (tid < M && tid < m) {
            float bv = -__builtin_inff();
            int bi = kArgNone;
            for (int r = 0; r < R && row0 + r < n; ++r) {
                const float v = logit[r * M + tid];
                if (row0 + r == 0 && v != v) {
                    bi = -1;
                    break;
                }
                if (arg_better(v, row0 + r, bv, bi)) {
                    bv = v;
                    bi = row0 + r;
                }
            }
            part[static_cast<size_t>(tid) * gridDim.x + blockIdx.x] = ArgPart{bv, bi};
            if (blockIdx.x == 0) ctl[tid] = ArgCtl{0, 0, 0};  // read by the next launch only
        }
        return;
    }
    if (tid < R * M) {
        const int r = tid / M, i = tid % M, row = row0 + r;
        if (row < n && i < m) {
            float s = 0.0f;
            for (int wv_i = 0; wv_i < nw; ++wv_i) s += red[(wv_i * R + r) * M + i];
            const float b = bias ? bias[row] : 0.0f;
            y[static_cast<size_t>(i) * n + row] = from_f32<YT>(__builtin_fmaf(s, ws_early, b));
        }
    }
}

// Rows of 1024 < k <= 2048 in one wave: two 16-byte chunks per lane (lane l and
// l + 64), no cross-wave reduction; the lanes holding the row totals after the
// exchange store them.
template <int R, int M, typename XT, typename YT>
__global__ __launch_bounds__(kWave) void gemv_q8_short_kernel(
    const XT* __restrict__ x, const int8_t* __restrict__ w, const float* __restrict__ ws,
    const float* __restrict__ bias, YT* __restrict__ y, int m, int n, int k) {
    constexpr int T = 2;
    const int lane = threadIdx.x;
    const int chunks = k >> 4;
    const int row0 = xcd_row_group() * R;
    bool act[T];
    int c[T];
#pragma unroll
    for (int t = 0; t < T; ++t) {
        act[t] = lane + kWave * t < chunks;
        c[t] = act[t] ? lane + kWave * t : 0;
    }
    XChunk<XT> xc[T][M];
#pragma unroll
    for (int t = 0; t < T; ++t)
#pragma unroll
        for (int i = 0; i < M; ++i) xc[t][i].load(x + static_cast<size_t>(min(i, m - 1)) * k + c[t] * 16);
    __builtin_amdgcn_sched_barrier(0);
    v4i wv[R][T];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const int row = min(row0 + r, n - 1);
#pragma unroll
        for (int t = 0; t < T; ++t)
            wv[r][t] = __builtin_nontemporal_load(reinterpret_cast<const v4i*>(w + static_cast<size_t>(row) * k + c[t] * 16));
        __builtin_amdgcn_sched_barrier(0);
    }
    constexpr int G = 64 / (R * M);
    const float ws_early = ws[min(row0 + min(lane / G / M, R - 1), n - 1)];
    float acc[R][M];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int i = 0; i < M; ++i) acc[r][i] = 0.0f;
#pragma unroll
    for (int t = 0; t < T; ++t)
#pragma unroll
        for (int i = 0; i < M; ++i)
#pragma unroll
            for (int r = 0; r < R; ++r) {
                float p = 0.0f;
#pragma unroll
                for (int d = 0; d < 4; ++d) {
                    const int wd = wv[r][t][d];
                    p = __builtin_fmaf(xc[t][i].at(4 * d + 0), sbyte_f32<0>(wd), p);
                    p = __builtin_fmaf(xc[t][i].at(4 * d + 1), sbyte_f32<1>(wd), p);
                    p = __builtin_fmaf(xc[t][i].at(4 * d + 2), sbyte_f32<2>(wd), p);
                    p = __builtin_fmaf(xc[t][i].at(4 * d + 3), sbyte_f32<3>(wd), p);
                }
                acc[r][i] += act[t] ? p : 0.0f;
            }
    const float v = wave_reduce_rows<R, M, (R * M >= 16)>(acc, lane);
    if (lane % G == 0) {
        const int j = lane / G, r = j / M, i = j % M, row = row0 + r;
        if (row < n && i < m) {
            const float b = bias ? bias[row] : 0.0f;
            y[static_cast<size_t>(i) * n + row] = from_f32<YT>(__builtin_fmaf(v, ws_early, b));
        }
    }
}

// int8 codes to fp16 pairs: byte b becomes the half 0x6400 | (b ^ 0x80), i.e.
// 1024 + (b + 128), and subtracting 1152 leaves b exactly. Pair j of a dword
// holds codes 2j and 2j + 1 (the activation's natural pair order).
__device__ __forceinline__ void q8_pairs(unsigned wd, h2& p0, h2& p1) {
    const h2 off = {static_cast<_Float16>(-1152.0f), static_cast<_Float16>(-1152.0f)};
    const unsigned wx = wd ^ 0x80808080u;
    p0 = __builtin_bit_cast(h2, __builtin_amdgcn_perm(0x64646464u, wx, 0x04010400u)) + off;
    p1 = __builtin_bit_cast(h2, __builtin_amdgcn_perm(0x64646464u, wx, 0x04030402u)) + off;
}
// Batches of 3..8 fp16 activation rows of int8 weights: the int4 tile kernel's
// layout with 16-byte chunks (wave w takes chunks w * 64 + lane, + 64 S, ...);
// each lane turns its 16 codes of a row into fp16 pairs once and runs one
// v_dot2 step per pair and activation row (exact products), the row scale after
// the sums.
template <int R, int M, typename YT>
__global__ __launch_bounds__(512) void gemv_q8_tile_kernel(
    const _Float16* __restrict__ x, const int8_t* __restrict__ w, const float* __restrict__ ws,
    const float* __restrict__ bias, YT* __restrict__ y, int m, int n, int k) {
    constexpr int NV = R * M, G = 64 / NV;
    __shared__ float red[8][NV];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, nw = block_threads() >> 6;
    const int chunks = k >> 4;
    const int row0 = xcd_row_group() * R;
    float acc[R][M];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int i = 0; i < M; ++i) acc[r][i] = 0.0f;
#pragma unroll 1
    for (int c0 = wave * kWave; c0 < chunks; c0 += kWave * nw) {
        const int c = c0 + lane;
        const bool act = c < chunks;
        const int cc = act ? c : 0;
        XChunk<_Float16> xc[M];
#pragma unroll
        for (int i = 0; i < M; ++i) xc[i].load(x + static_cast<size_t>(min(i, m - 1)) * k + cc * 16);
        v4i wv[R];
#pragma unroll
        for (int r = 0; r < R; ++r)
            wv[r] = __builtin_nontemporal_load(
                reinterpret_cast<const v4i*>(w + static_cast<size_t>(min(row0 + r, n - 1)) * k + cc * 16));
#pragma unroll
        for (int r = 0; r < R; ++r) {
            h2 cp[8];
#pragma unroll
            for (int d = 0; d < 4; ++d) q8_pairs(static_cast<unsigned>(wv[r][d]), cp[2 * d], cp[2 * d + 1]);
#pragma unroll
            for (int i = 0; i < M; ++i) {
                const h2* xp = reinterpret_cast<const h2*>(&xc[i].v[0]);
                float p = 0.0f;
#pragma unroll
                for (int j = 0; j < 8; ++j) p = __builtin_amdgcn_fdot2(cp[j], xp[j], p, false);
                acc[r][i] += act ? p : 0.0f;
            }
        }
    }
    const float v = wave_reduce_rows<R, M, true>(acc, lane);
    if (lane % G == 0) red[wave][lane / G] = v;
    __syncthreads();
    if (tid < NV) {
        const int r = tid / M, i = tid % M, row = row0 + r;
        if (row < n && i < m) {
            float t = 0.0f;
            for (int q = 0; q < nw; ++q) t += red[q][tid];
            y[static_cast<size_t>(i) * n + row] = from_f32<YT>(__builtin_fmaf(t, ws[row], bias ? bias[row] : 0.0f));
        }
    }
}

// ---- group-wise int4 ------------------------------------------------------------------
// Exact int4 x fp16 dot over one 16-byte chunk (32 codes) with packed fp16 math.
// Nibble e of dword d is column 8d+e. Masking a dword with 0x000F000F keeps
// columns 8d and 8d+4 in the low 4 bits of its two halves; OR 0x6400 makes each
// half the fp16 value 1024 + nibble (exact) and adding -1032 gives the code
// nibble - 8 exactly. Masking with 0x00F000F0 instead keeps columns 8d+1 and
// 8d+5 as 1024 + 16 * nibble (still exact: the fp16 spacing at 1024..2047 is 1),
// and adding -1152 gives 16 * code, so no shift is needed for odd nibbles; the
// dword shifted right by 8 serves columns 8d+2/8d+6 and 8d+3/8d+7 the same way.
// Each v_dot2_f32_f16 multiplies two (code, x) pairs with exact products and
// accumulates in fp32, the 16x-scaled pairs into their own sum, rescaled by the
// exact 1/16 at the end. xp[4d + j] holds the pair (x[8d+j], x[8d+j+4]).
__device__ __forceinline__ h2 q4_pair(unsigned w, unsigned mask) {
    unsigned b;
    // v_and_or_b32 with the mask in an SGPR: one instruction for (w & mask) | 0x64006400.
    asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(b) : "v"(w), "s"(mask), "v"(0x64006400u));
    return __builtin_bit_cast(h2, b);
}
__device__ __forceinline__ float dot32_q4_f16(v4i wv, const h2 (&xp)[16]) {
    const h2 off1 = {static_cast<_Float16>(-1032.0f), static_cast<_Float16>(-1032.0f)};
    const h2 off16 = {static_cast<_Float16>(-1152.0f), static_cast<_Float16>(-1152.0f)};
    float p1 = 0.0f, p16 = 0.0f;
#pragma unroll
    for (int d = 0; d < 4; ++d) {
        const unsigned w = static_cast<unsigned>(wv[d]);
        const unsigned u = w >> 8;
        p1 = __builtin_amdgcn_fdot2(q4_pair(w, 0x000F000Fu) + off1, xp[4 * d + 0], p1, false);
        p16 = __builtin_amdgcn_fdot2(q4_pair(w, 0x00F000F0u) + off16, xp[4 * d + 1], p16, false);
        p1 = __builtin_amdgcn_fdot2(q4_pair(u, 0x000F000Fu) + off1, xp[4 * d + 2], p1, false);
        p16 = __builtin_amdgcn_fdot2(q4_pair(u, 0x00F000F0u) + off16, xp[4 * d + 3], p16, false);
    }
    return __builtin_fmaf(p16, 0.0625f, p1);
}

// dot32_q4_f16 with the 0x64006400 magic in a caller-held VGPR: in a loop the
// asm operand would otherwise be rematerialized, and hoisted, once per use.
__device__ __forceinline__ float dot32_q4_f16m(v4i wv, const h2 (&xp)[16], unsigned magic) {
    const h2 off1 = {static_cast<_Float16>(-1032.0f), static_cast<_Float16>(-1032.0f)};
    const h2 off16 = {static_cast<_Float16>(-1152.0f), static_cast<_Float16>(-1152.0f)};
    auto pair = [&](unsigned w, unsigned mask) {
        unsigned b;
        asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(b) : "v"(w), "s"(mask), "v"(magic));
        return __builtin_bit_cast(h2, b);
    };
    float p1 = 0.0f, p16 = 0.0f;
#pragma unroll
    for (int d = 0; d < 4; ++d) {
        const unsigned w = static_cast<unsigned>(wv[d]);
        const unsigned u = w >> 8;
        p1 = __builtin_amdgcn_fdot2(pair(w, 0x000F000Fu) + off1, xp[4 * d + 0], p1, false);
        p16 = __builtin_amdgcn_fdot2(pair(w, 0x00F000F0u) + off16, xp[4 * d + 1], p16, false);
        p1 = __builtin_amdgcn_fdot2(pair(u, 0x000F000Fu) + off1, xp[4 * d + 2], p1, false);
        p16 = __builtin_amdgcn_fdot2(pair(u, 0x00F000F0u) + off16, xp[4 * d + 3], p16, false);
    }
    return __builtin_fmaf(p16, 0.0625f, p1);
}

// The same chunk dot in fp32 for fp32 activations.
__device__ __forceinline__ float dot32_q4_f32(v4i wv, const float (&xf)[32]) {
    float p = 0.0f;
#pragma unroll
    for (int d = 0; d < 4; ++d) {
        const unsigned wd = static_cast<unsigned>(wv[d]);
#pragma unroll
        for (int e = 0; e < 8; ++e)
            p = __builtin_fmaf(xf[8 * d + e], static_cast<float>(static_cast<int>((wd >> (4 * e)) & 15u) - 8), p);
    }
    return p;
}

// XS: workgroups per row group over slices of M activation rows (as gemv_q8_kernel).
template <int R, int M, typename XT, typename YT, typename ST, int LB = kMaxGemvThreads, int XS = 1>
__global__ __launch_bounds__(LB) void gemv_q4g_kernel(
    const XT* __restrict__ x, const uint8_t* __restrict__ w, const ST* __restrict__ scale,
    const float* __restrict__ bias, YT* __restrict__ y, int m, int n, int k, int group) {
    __shared__ float red[kMaxGemvWaves * R * M];
    const int tid = threadIdx.x, wave = tid >> 6, nw = block_threads() >> 6;
    const int chunks = k >> 5;  // 32 codes per 16-byte chunk
    const int rb = k >> 1;
    const bool act = tid < chunks;
    int rg = xcd_row_group();
    if constexpr (XS > 1) {
        const int sl = rg % XS;  // rows [sl * M, sl * M + M) of x and y; m > (XS - 1) * M
        rg /= XS;
        x += static_cast<size_t>(sl) * M * k;
        y += static_cast<size_t>(sl) * M * n;
        m -= sl * M;
    }
    const int row0 = rg * R;

    const int c = act ? tid : 0;
    v4i wv[R];
    ST sraw[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const int row = min(row0 + r, n - 1);
        wv[r] = __builtin_nontemporal_load(reinterpret_cast<const v4i*>(w + static_cast<size_t>(row) * rb + c * 16));
    }
    const unsigned ug = static_cast<unsigned>(group);
    const unsigned blocks = ug == 32 ? static_cast<unsigned>(chunks) : (static_cast<unsigned>(k) + ug - 1) / ug;  // ceil: a short last group
    const unsigned blk = ug == 32 ? static_cast<unsigned>(c) : static_cast<unsigned>(c * 32) / ug;
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const int row = min(row0 + r, n - 1);
        sraw[r] = scale[static_cast<size_t>(row) * blocks + blk];
    }
    // Activation chunks of all M rows are loaded up front while they fit in 64
    // VGPRs (fp16 m <= 4, fp32 m <= 2); larger batches load one row at a time.
    constexpr bool kAllX = M * 32 * sizeof(XT) <= 256;
    auto load_x = [&](int i, XChunk<XT>& lo, XChunk<XT>& hi) {
        const XT* xp = x + static_cast<size_t>(min(i, m - 1)) * k + c * 32;
        lo.load(xp);
        hi.load(xp + 16);
    };
    XChunk<XT> xlo[kAllX ? M : 1], xhi[kAllX ? M : 1];
    if constexpr (kAllX) {
#pragma unroll
        for (int i = 0; i < M; ++i) load_x(i, xlo[i], xhi[i]);
    }

    float acc[R][M];
#pragma unroll
    for (int i = 0; i < M; ++i) {
        XChunk<XT> lo, hi;
        if constexpr (kAllX) {
            lo = xlo[i];
            hi = xhi[i];
        } else {
            load_x(i, lo, hi);
        }
        if constexpr (sizeof(XT) == 2) {
            const typename XChunk<XT>::h8 q[4] = {lo.v[0], lo.v[1], hi.v[0], hi.v[1]};
            h2 pairs[16];
#pragma unroll
            for (int d = 0; d < 4; ++d)
#pragma unroll
                for (int j = 0; j < 4; ++j) pairs[4 * d + j] = h2{q[d][j], q[d][j + 4]};
#pragma unroll
            for (int r = 0; r < R; ++r) acc[r][i] = dot32_q4_f16(wv[r], pairs) * to_f32(sraw[r]);
        } else {
            float xf[32];
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                xf[e] = lo.at(e);
                xf[16 + e] = hi.at(e);
            }
#pragma unroll
            for (int r = 0; r < R; ++r) acc[r][i] = dot32_q4_f32(wv[r], xf) * to_f32(sraw[r]);
        }
#pragma unroll
        for (int r = 0; r < R; ++r) acc[r][i] = act ? acc[r][i] : 0.0f;
    }
    // int4 batches of 8 rows (and 4 fp16 rows) spilled with the all-VALU
    // exchanges (m = 8, k = 8960, n = 1536: 96 -> 12 us with ds_bpermute)
    constexpr bool kBperm = R * M >= 16 || (M == 4 && sizeof(XT) == 2);
    // One wave (k <= 2048): write from the lanes holding the totals. Not for
    // 2 rows x 4 fp32 activation rows, where it raised the spills from 4 to 6, nor
    // for one fp16 activation row: the untaken branch cost the k = 8960 kernel
    // 4.61 -> 4.76 us in code generation, against 3.14 -> 3.09 at k = 1536.
    constexpr bool kLaneOut = !(R == 2 && M == 4 && sizeof(XT) == 4) && !(M == 1 && sizeof(XT) == 2);
    if (kLaneOut && nw == 1) {
        constexpr int G = 64 / (R * M);
        const float v = wave_reduce_rows<R, M, kBperm>(acc, tid);
        if (tid % G == 0) {
            const int j = tid / G, r = j / M, i = j % M, row = row0 + r;
            if (row < n && i < m) y[static_cast<size_t>(i) * n + row] = from_f32<YT>(v + (bias ? bias[row] : 0.0f));
        }
        return;
    }
    reduce_to_lds<R, M, kBperm>(acc, red, wave, tid & 63);
    __syncthreads();
    if (tid < R * M) {
        const int r = tid / M, i = tid % M, row = row0 + r;
        if (row < n && i < m) {
            float s = 0.0f;
            for (int wv_i = 0; wv_i < nw; ++wv_i) s += red[(wv_i * R + r) * M + i];
            const float b = bias ? bias[row] : 0.0f;
            y[static_cast<size_t>(i) * n + row] = from_f32<YT>(s + b);
        }
    }
}

// Exact int4 x fp16 dot over half a chunk (8 bytes, 16 codes), as dot32_q4_f16.
__device__ __forceinline__ float dot16_q4_f16(unsigned w0, unsigned w1, const h2 (&xp)[8]) {
    const h2 off1 = {static_cast<_Float16>(-1032.0f), static_cast<_Float16>(-1032.0f)};
    const h2 off16 = {static_cast<_Float16>(-1152.0f), static_cast<_Float16>(-1152.0f)};
    float p1 = 0.0f, p16 = 0.0f;
#pragma unroll
    for (int d = 0; d < 2; ++d) {
        const unsigned w = d ? w1 : w0;
        const unsigned u = w >> 8;
        p1 = __builtin_amdgcn_fdot2(q4_pair(w, 0x000F000Fu) + off1, xp[4 * d + 0], p1, false);
        p16 = __builtin_amdgcn_fdot2(q4_pair(w, 0x00F000F0u) + off16, xp[4 * d + 1], p16, false);
        p1 = __builtin_amdgcn_fdot2(q4_pair(u, 0x000F000Fu) + off1, xp[4 * d + 2], p1, false);
        p16 = __builtin_amdgcn_fdot2(q4_pair(u, 0x00F000F0u) + off16, xp[4 * d + 3], p16, false);
    }
    return __builtin_fmaf(p16, 0.0625f, p1);
}
// One fp16 activation row, half a chunk per lane: lane t takes K columns
// 16t .. 16t + 15 (8 bytes of codes, 32 bytes of x) of each of the R rows, so a
// workgroup has twice the waves of gemv_q4g_kernel, each lane one 8-byte load
// per row. group is a multiple of 32, so a half chunk has one scale.
// The activation chunk is requested first and each row's scale and codes after
// it, so a row's dot starts when its own load lands (the in-order load counter
// would otherwise hold every row until the last load); R = 3 or 6 rows per
// workgroup cut the activation re-reads, which every workgroup takes from L2
// (n = 1536, k = 8960: 2 rows with x last 4.49-4.64 us, 3 rows x first
// 4.32-4.35; n = 8960, k = 5120: 9.03 -> 7.26 with 6 rows).
// MAXT: the launch bound (576 threads, or 1024 for 9216 < k <= 16384).
template <int R, typename YT, typename ST, int MAXT = kMaxGemvThreads>
__global__ __launch_bounds__(MAXT) void gemv_q4g_x1h_half_kernel(
    const _Float16* __restrict__ x, const uint8_t* __restrict__ w, const ST* __restrict__ scale,
    const float* __restrict__ bias, YT* __restrict__ y, int n, int k, int group) {
    constexpr int RP = R <= 1 ? 1 : R <= 2 ? 2 : R <= 4 ? 4 : 8;  // reduced values, a power of two
    __shared__ float red[(MAXT / kWave) * R];
    const int tid = threadIdx.x, wave = tid >> 6, nw = block_threads() >> 6;
    const int halves = k >> 4, rb = k >> 1;
    const int row0 = xcd_row_group() * R;
    const bool act = tid < halves;
    const int hc = act ? tid : 0;  // half chunk: K columns 16 hc .. 16 hc + 15
    XChunk<_Float16> xc;
    xc.load(x + hc * 16);
    __builtin_amdgcn_sched_barrier(0);  // the activation request goes out first
    typedef int v2i_t __attribute__((ext_vector_type(2)));
    const unsigned ug = static_cast<unsigned>(group);
    const unsigned blocks = (static_cast<unsigned>(k) + ug - 1) / ug;  // ceil: a short last group
    const unsigned blk = static_cast<unsigned>(hc * 16) / ug;
    v2i_t wv[R];
    ST sraw[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const size_t row = static_cast<size_t>(min(row0 + r, n - 1));
        sraw[r] = scale[row * blocks + blk];
        wv[r] = __builtin_nontemporal_load(reinterpret_cast<const v2i_t*>(w + row * rb + hc * 8));
        __builtin_amdgcn_sched_barrier(0);  // rows in order: row r's dot waits only for rows <= r
    }
    h2 pairs[8];
#pragma unroll
    for (int d = 0; d < 2; ++d)
#pragma unroll
        for (int j = 0; j < 4; ++j) pairs[4 * d + j] = h2{xc.v[d][j], xc.v[d][j + 4]};
    float acc[RP][1];
#pragma unroll
    for (int r = 0; r < RP; ++r) {
        if (r < R) {
            const float p = dot16_q4_f16(static_cast<unsigned>(wv[r][0]), static_cast<unsigned>(wv[r][1]), pairs) *
                            to_f32(sraw[r]);
            acc[r][0] = act ? p : 0.0f;
        } else {
            acc[r][0] = 0.0f;
        }
    }
    constexpr int G = 64 / RP;
    const float v = wave_reduce_rows<RP, 1>(acc, tid & 63);
    if ((tid & 63) % G == 0 && (tid & 63) / G < R) red[wave * R + (tid & 63) / G] = v;
    __syncthreads();
    if (tid < R) {
        const int row = row0 + tid;
        if (row < n) {
            float s = 0.0f;
            for (int q = 0; q < nw; ++q) s += red[q * R + tid];
            y[row] = from_f32<YT>(s + (bias ? bias[row] : 0.0f));
        }
    }
}

// Exact int4 x fp32 dot over half a chunk (16 codes), as dot32_q4_f32.
__device__ __forceinline__ float dot16_q4_f32(unsigned w0, unsigned w1, const XChunk<float>& xc) {
    float p = 0.0f;
#pragma unroll
    for (int d = 0; d < 2; ++d) {
        const unsigned wd = d ? w1 : w0;
#pragma unroll
        for (int e = 0; e < 8; ++e)
            p = __builtin_fmaf(xc.at(8 * d + e), static_cast<float>(static_cast<int>((wd >> (4 * e)) & 15u) - 8), p);
    }
    return p;
}
// Short rows (k <= 1024, or 2048 with T = 2), one wave per workgroup: half a chunk per lane (8
// bytes of codes, 16 codes) as the one-row kernel above, so a row of k = 896
// occupies 56 lanes instead of 28 and each lane's activation vectors (16
// elements per activation row) serve R rows of 16 codes, the int8 GEMV's ratio
// at half its code bytes. The lanes holding the row totals after the exchange
// store them (no LDS, no barrier). T = 2: two half chunks per lane (lane l and
// l + 64), k <= 2048.
template <int R, int M, typename XT, typename YT, typename ST, int T = 1>
__global__ __launch_bounds__(kWave) void gemv_q4g_short_kernel(
    const XT* __restrict__ x, const uint8_t* __restrict__ w, const ST* __restrict__ scale,
    const float* __restrict__ bias, YT* __restrict__ y, int m, int n, int k, int group) {
    const int lane = threadIdx.x;
    const int halves = k >> 4, rb = k >> 1;
    const int row0 = xcd_row_group() * R;
    bool act[T];
    int hc[T];  // half chunk of pass t: K columns 16 hc .. 16 hc + 15
#pragma unroll
    for (int t = 0; t < T; ++t) {
        act[t] = lane + kWave * t < halves;
        hc[t] = act[t] ? lane + kWave * t : 0;
    }
    XChunk<XT> xc[T][M];
#pragma unroll
    for (int t = 0; t < T; ++t)
#pragma unroll
        for (int i = 0; i < M; ++i) xc[t][i].load(x + static_cast<size_t>(min(i, m - 1)) * k + hc[t] * 16);
    __builtin_amdgcn_sched_barrier(0);  // the activation requests go out first
    typedef int v2i_t __attribute__((ext_vector_type(2)));
    const unsigned ug = static_cast<unsigned>(group);
    const unsigned blocks = (static_cast<unsigned>(k) + ug - 1) / ug;
    v2i_t wv[R][T];
    ST sraw[R][T];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const size_t row = static_cast<size_t>(min(row0 + r, n - 1));
#pragma unroll
        for (int t = 0; t < T; ++t) {
            sraw[r][t] = scale[row * blocks + static_cast<unsigned>(hc[t] * 16) / ug];
            wv[r][t] = __builtin_nontemporal_load(reinterpret_cast<const v2i_t*>(w + row * rb + hc[t] * 8));
        }
        __builtin_amdgcn_sched_barrier(0);  // rows in order: row r's dot waits only for rows <= r
    }
    float acc[R][M];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int i = 0; i < M; ++i) acc[r][i] = 0.0f;
#pragma unroll
    for (int t = 0; t < T; ++t) {
#pragma unroll
        for (int i = 0; i < M; ++i) {
            float p[R];
            if constexpr (sizeof(XT) == 2) {
                h2 pairs[8];
#pragma unroll
                for (int d = 0; d < 2; ++d)
#pragma unroll
                    for (int j = 0; j < 4; ++j) pairs[4 * d + j] = h2{xc[t][i].v[d][j], xc[t][i].v[d][j + 4]};
#pragma unroll
                for (int r = 0; r < R; ++r)
                    p[r] = dot16_q4_f16(static_cast<unsigned>(wv[r][t][0]), static_cast<unsigned>(wv[r][t][1]), pairs) *
                           to_f32(sraw[r][t]);
            } else {
#pragma unroll
                for (int r = 0; r < R; ++r)
                    p[r] = dot16_q4_f32(static_cast<unsigned>(wv[r][t][0]), static_cast<unsigned>(wv[r][t][1]),
                                        xc[t][i]) *
                           to_f32(sraw[r][t]);
            }
#pragma unroll
            for (int r = 0; r < R; ++r) acc[r][i] += act[t] ? p[r] : 0.0f;
        }
    }
    constexpr int G = 64 / (R * M);
    const float v = wave_reduce_rows<R, M, (R * M >= 16)>(acc, lane);
    if (lane % G == 0) {
        const int j = lane / G, r = j / M, i = j % M, row = row0 + r;
        if (row < n && i < m) y[static_cast<size_t>(i) * n + row] = from_f32<YT>(v + (bias ? bias[row] : 0.0f));
    }
}

// Batches of 3..8 fp16 activation rows: a workgroup of S waves owns R weight
// rows and splits K between its waves (wave w takes half chunks w * 64 + lane,
// then + 64 S, ...). Each lane converts its 16 codes of a weight row to fp16
// pairs once and reuses them for all M activation rows (exact products via
// v_dot2_f32_f16, as dot16_q4_f16), so per 8 bytes of codes it does M dot
// steps instead of re-reading the codes per activation row; the R x M partial
// sums are exchanged within the wave, then summed over the S waves in LDS.
template <int R, int M, typename YT, typename ST>
__global__ __launch_bounds__(512) void gemv_q4g_tile_kernel(
    const _Float16* __restrict__ x, const uint8_t* __restrict__ w, const ST* __restrict__ scale,
    const float* __restrict__ bias, YT* __restrict__ y, int m, int n, int k, int group) {
    constexpr int NV = R * M, G = 64 / NV;
    __shared__ float red[8][NV];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, nw = block_threads() >> 6;
    const int halves = k >> 4, rb = k >> 1;
    const int row0 = xcd_row_group() * R;
    const unsigned ug = static_cast<unsigned>(group);
    const unsigned blocks = (static_cast<unsigned>(k) + ug - 1) / ug;
    const h2 off1 = {static_cast<_Float16>(-1032.0f), static_cast<_Float16>(-1032.0f)};
    typedef int v2i_t __attribute__((ext_vector_type(2)));
    float acc[R][M];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int i = 0; i < M; ++i) acc[r][i] = 0.0f;
#pragma unroll 1
    for (int h0 = wave * kWave; h0 < halves; h0 += kWave * nw) {
        const int h = h0 + lane;
        const bool act = h < halves;
        const int hc = act ? h : 0;
        XChunk<_Float16> xc[M];
#pragma unroll
        for (int i = 0; i < M; ++i) xc[i].load(x + static_cast<size_t>(min(i, m - 1)) * k + hc * 16);
        v2i_t wv[R];
        ST sr[R];
        const unsigned blk = static_cast<unsigned>(hc * 16) / ug;
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const size_t row = static_cast<size_t>(min(row0 + r, n - 1));
            sr[r] = scale[row * blocks + blk];
            wv[r] = __builtin_nontemporal_load(reinterpret_cast<const v2i_t*>(w + row * rb + hc * 8));
        }
        h2 xp[M][8];
#pragma unroll
        for (int i = 0; i < M; ++i)
#pragma unroll
            for (int d = 0; d < 2; ++d)
#pragma unroll
                for (int j = 0; j < 4; ++j) xp[i][4 * d + j] = h2{xc[i].v[d][j], xc[i].v[d][j + 4]};
#pragma unroll
        for (int r = 0; r < R; ++r) {
            h2 cp[8];
            // every nibble shifted down to bits 0..3 of its half (one shift per two
            // pairs, shared by the M activation rows) so one accumulator takes all
            // 16 exact products (against separate x1 / x16 sums combined per
            // activation row: m = 4, n = 28672, k = 4096 34.4 -> 28.2 us; 2-4% on
            // the other long-K shapes)
#pragma unroll
            for (int d = 0; d < 2; ++d) {
                const unsigned wd = static_cast<unsigned>(wv[r][d]), u = wd >> 8;
                cp[4 * d + 0] = q4_pair(wd, 0x000F000Fu) + off1;
                cp[4 * d + 1] = q4_pair(wd >> 4, 0x000F000Fu) + off1;
                cp[4 * d + 2] = q4_pair(u, 0x000F000Fu) + off1;
                cp[4 * d + 3] = q4_pair(u >> 4, 0x000F000Fu) + off1;
            }
            const float s = act ? to_f32(sr[r]) : 0.0f;
#pragma unroll
            for (int i = 0; i < M; ++i) {
                float p = 0.0f;
#pragma unroll
                for (int j = 0; j < 8; ++j) p = __builtin_amdgcn_fdot2(cp[j], xp[i][j], p, false);
                acc[r][i] = __builtin_fmaf(p, s, acc[r][i]);
            }
        }
    }
    const float v = wave_reduce_rows<R, M, true>(acc, lane);
    if (lane % G == 0) red[wave][lane / G] = v;
    __syncthreads();
    if (tid < NV) {
        const int r = tid / M, i = tid % M, row = row0 + r;
        if (row < n && i < m) {
            float t = 0.0f;
            for (int q = 0; q < nw; ++q) t += red[q][tid];
            y[static_cast<size_t>(i) * n + row] = from_f32<YT>(t + (bias ? bias[row] : 0.0f));
        }
    }
}

// fp32 activation rows: the tile kernels' layout with fp32 FMAs (the codes of a
// row converted to float once per lane and reused over the M activation rows).
// Q4: 16-code half chunks (group scale per half chunk, as the fp16 form); else
// int8 16-byte chunks, the row scale after the sums.
template <bool Q4, int R, int M, typename YT, typename ST>
__global__ __launch_bounds__(512) void gemv_tile_f32_kernel(
    const float* __restrict__ x, const uint8_t* __restrict__ w, const ST* __restrict__ scale,
    const float* __restrict__ bias, YT* __restrict__ y, int m, int n, int k, int group) {
    constexpr int NV = R * M, G = 64 / NV;
    __shared__ float red[8][NV];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, nw = block_threads() >> 6;
    const int units = k >> 4;  // 16 codes per lane and step
    const int rb = Q4 ? (k >> 1) : k;
    const int row0 = xcd_row_group() * R;
    const unsigned ug = static_cast<unsigned>(group);
    const unsigned blocks = Q4 ? (static_cast<unsigned>(k) + ug - 1) / ug : 1;
    typedef int v2i_t __attribute__((ext_vector_type(2)));
    float acc[R][M];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int i = 0; i < M; ++i) acc[r][i] = 0.0f;
#pragma unroll 1
    for (int u0 = wave * kWave; u0 < units; u0 += kWave * nw) {
        const int u = u0 + lane;
        const bool act = u < units;
        const int uc = act ? u : 0;
        XChunk<float> xc[M];
#pragma unroll
        for (int i = 0; i < M; ++i) xc[i].load(x + static_cast<size_t>(min(i, m - 1)) * k + uc * 16);
        unsigned wd[R][Q4 ? 2 : 4];
        float sr[R];
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const size_t row = static_cast<size_t>(min(row0 + r, n - 1));
            if constexpr (Q4) {
                sr[r] = to_f32(scale[row * blocks + static_cast<unsigned>(uc * 16) / ug]);
                const v2i_t v = __builtin_nontemporal_load(reinterpret_cast<const v2i_t*>(w + row * rb + uc * 8));
                wd[r][0] = static_cast<unsigned>(v[0]);
                wd[r][1] = static_cast<unsigned>(v[1]);
            } else {
                const v4i v = __builtin_nontemporal_load(reinterpret_cast<const v4i*>(w + row * rb + uc * 16));
#pragma unroll
                for (int d = 0; d < 4; ++d) wd[r][d] = static_cast<unsigned>(v[d]);
            }
        }
#pragma unroll
        for (int r = 0; r < R; ++r) {
            float cf[16];
            if constexpr (Q4) {
#pragma unroll
                for (int d = 0; d < 2; ++d)
#pragma unroll
                    for (int e = 0; e < 8; ++e)
                        cf[8 * d + e] = static_cast<float>(static_cast<int>((wd[r][d] >> (4 * e)) & 15u) - 8);
            } else {
#pragma unroll
                for (int d = 0; d < 4; ++d) {
                    const int v = static_cast<int>(wd[r][d]);
                    cf[4 * d + 0] = sbyte_f32<0>(v);
                    cf[4 * d + 1] = sbyte_f32<1>(v);
                    cf[4 * d + 2] = sbyte_f32<2>(v);
                    cf[4 * d + 3] = sbyte_f32<3>(v);
                }
            }
            const float s = Q4 ? (act ? sr[r] : 0.0f) : 1.0f;
#pragma unroll
            for (int i = 0; i < M; ++i) {
                float p = 0.0f;
#pragma unroll
                for (int e = 0; e < 16; ++e) p = __builtin_fmaf(xc[i].at(e), cf[e], p);
                if constexpr (Q4) acc[r][i] = __builtin_fmaf(p, s, acc[r][i]);
                else acc[r][i] += act ? p : 0.0f;
            }
        }
    }
    const float v = wave_reduce_rows<R, M, true>(acc, lane);
    if (lane % G == 0) red[wave][lane / G] = v;
    __syncthreads();
    if (tid < NV) {
        const int r = tid / M, i = tid % M, row = row0 + r;
        if (row < n && i < m) {
            float t = 0.0f;
            for (int q = 0; q < nw; ++q) t += red[q][tid];
            const float b = bias ? bias[row] : 0.0f;
            if constexpr (Q4) y[static_cast<size_t>(i) * n + row] = from_f32<YT>(t + b);
            else y[static_cast<size_t>(i) * n + row] = from_f32<YT>(__builtin_fmaf(t, to_f32(scale[row]), b));
        }
    }
}

// ---- W8A8 (int8 x int8 -> int32) ------------------------------------------------------
// ACC_OUT: write the raw int32 accumulators instead of the scaled output.
template <int R, int M, typename YT, bool ACC_OUT>
__global__ __launch_bounds__(kMaxGemvThreads) void gemv_w8a8_kernel(
    const int8_t* __restrict__ xq, const float* __restrict__ as, const int8_t* __restrict__ w,
    const float* __restrict__ ws, const float* __restrict__ bias, YT* __restrict__ y,
    int32_t* __restrict__ acc_out, int m, int n, int k) {
    __shared__ int red[kMaxGemvWaves * R * M];
    const int tid = threadIdx.x, wave = tid >> 6, nw = block_threads() >> 6;
    const int chunks = k >> 4;
    const bool act = tid < chunks;
    const int row0 = xcd_row_group() * R;

    const int c = act ? tid : 0;
    v4i wv[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const int row = min(row0 + r, n - 1);
        wv[r] = __builtin_nontemporal_load(reinterpret_cast<const v4i*>(w + static_cast<size_t>(row) * k + c * 16));
    }
    v4i xv[M];
#pragma unroll
    for (int i = 0; i < M; ++i) xv[i] = *reinterpret_cast<const v4i*>(xq + static_cast<size_t>(min(i, m - 1)) * k + c * 16);
    const float ws_early = ACC_OUT ? 0.0f : ws[min(row0 + min(tid / M, R - 1), n - 1)];  // as gemv_q8_kernel
    int acc[R][M];
#pragma unroll
    for (int i = 0; i < M; ++i) {
#pragma unroll
        for (int r = 0; r < R; ++r) {
            int p = 0;
#pragma unroll
            for (int d = 0; d < 4; ++d) p = __builtin_amdgcn_sdot4(xv[i][d], wv[r][d], p, false);
            acc[r][i] = act ? p : 0;
        }
    }
    reduce_to_lds<R, M>(acc, red, wave, tid & 63);
    __syncthreads();
    if (tid < R * M) {
        const int r = tid / M, i = tid % M, row = row0 + r;
        if (row < n && i < m) {
            int s = 0;
            for (int wv_i = 0; wv_i < nw; ++wv_i) s += red[(wv_i * R + r) * M + i];
            if constexpr (ACC_OUT) {
                acc_out[static_cast<size_t>(i) * n + row] = s;
            } else {
                const float b = bias ? bias[row] : 0.0f;
                y[static_cast<size_t>(i) * n + row] = from_f32<YT>(w8a8_epilogue(s, as[i], ws_early, b));
            }
        }
    }
}

// ---- W8A8 decode with the activation quant fused in -----------------------------------
// The workgroup already spans the whole K of its rows, so it holds every element
// of the (at most 8) activation rows: it reduces each row's absmax across its
// waves, derives a_scale = absmax / 127 exactly as the activation-quant kernel
// does, quantizes its own 16-element chunk in registers and runs the same
// v_dot4_i32_i8 core. Identical int32 accumulators and epilogue, one launch.
// W1: one wave (k <= 1024): the wave's butterfly absmax is the row's in every
// lane (no LDS round trip or barrier), and the lanes holding the row totals
// store them.
template <int R, int M, typename XT, typename YT, bool W1 = false>
__global__ __launch_bounds__(kMaxGemvThreads) void gemv_w8a8_fused_kernel(
    const XT* __restrict__ x, const int8_t* __restrict__ w, const float* __restrict__ ws,
    const float* __restrict__ bias, YT* __restrict__ y, int m, int n, int k) {
    __shared__ float amax_red[kMaxGemvWaves * M];
    __shared__ int red[kMaxGemvWaves * R * M];
    const int tid = threadIdx.x, wave = tid >> 6, nw = block_threads() >> 6;
    const int chunks = k >> 4;
    const bool act = tid < chunks;
    const int row0 = xcd_row_group() * R;

    const int c = act ? tid : 0;
    // The activation loads go out first: the absmax below waits on them, and the
    // in-order load counter would otherwise make it wait for the weight rows too,
    // putting the absmax, the barrier and the quantize after the weights' HBM
    // latency instead of under it.
    XChunk<XT> xc[M];
#pragma unroll
    for (int i = 0; i < M; ++i) xc[i].load(x + static_cast<size_t>(min(i, m - 1)) * k + c * 16);
    __builtin_amdgcn_sched_barrier(0);
    v4i wv[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const int row = min(row0 + r, n - 1);
        wv[r] = __builtin_nontemporal_load(reinterpret_cast<const v4i*>(w + static_cast<size_t>(row) * k + c * 16));
    }
    constexpr int G1 = 64 / (R * M);  // the storing lanes' rows, as gemv_q8_kernel
    const float ws_early = ws[min(row0 + min(W1 ? (tid & 63) / G1 / M : tid / M, R - 1), n - 1)];
    float am[M];
#pragma unroll
    for (int i = 0; i < M; ++i) {
        float a = 0.0f;
#pragma unroll
        for (int e = 0; e < 16; ++e) a = absmax_step(a, xc[i].at(e));
        am[i] = act ? a : 0.0f;
    }
    float as[M];
    if constexpr (W1) {
#pragma unroll
        for (int i = 0; i < M; ++i) as[i] = wave_absmax(am[i]) / 127.0f;  // am >= 0: as the fold below
    } else {
#pragma unroll
        for (int i = 0; i < M; ++i) {
            const float a = wave_absmax(am[i]);
            if ((tid & 63) == 0) amax_red[wave * M + i] = a;
        }
        __syncthreads();
#pragma unroll
        for (int i = 0; i < M; ++i) {
            float a = 0.0f;
            for (int v = 0; v < nw; ++v) a = absmax_step(a, amax_red[v * M + i]);
            as[i] = a / 127.0f;
        }
    }

    int acc[R][M];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int i = 0; i < M; ++i) acc[r][i] = 0;
#pragma unroll
    for (int i = 0; i < M; ++i) {
        {
            const RowQuantizer rq(as[i]);
            int qd[4];
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                float v[8];
#pragma unroll
                for (int e = 0; e < 8; ++e) v[e] = xc[i].at(8 * h + e);
                rq.pack8(v, qd[2 * h], qd[2 * h + 1]);
            }
#pragma unroll
            for (int r = 0; r < R; ++r)
#pragma unroll
                for (int d = 0; d < 4; ++d) acc[r][i] = __builtin_amdgcn_sdot4(qd[d], wv[r][d], acc[r][i], false);
#pragma unroll
            for (int r = 0; r < R; ++r) acc[r][i] = act ? acc[r][i] : 0;
        }
    }
    if constexpr (W1) {
        constexpr int G = 64 / (R * M);
        const int v = wave_reduce_rows<R, M>(acc, tid);
        if (tid % G == 0) {
            const int j = tid / G, r = j / M, i = j % M, row = row0 + r;
            if (row < n && i < m) {
                const float b = bias ? bias[row] : 0.0f;
                y[static_cast<size_t>(i) * n + row] = from_f32<YT>(w8a8_epilogue(v, as[i], ws_early, b));
            }
        }
        return;
    }
    reduce_to_lds<R, M>(acc, red, wave, tid & 63);
    __syncthreads();
    if (tid < R * M) {
        const int r = tid / M, i = tid % M, row = row0 + r;
        if (row < n && i < m) {
            int s = 0;
            for (int v = 0; v < nw; ++v) s += red[(v * R + r) * M + i];
            const float b = bias ? bias[row] : 0.0f;
            y[static_cast<size_t>(i) * n + row] = from_f32<YT>(w8a8_epilogue(s, as[i], ws_early, b));
        }
    }
}

// ---- W8A8 decode in one launch: act quant into LDS, then the weight stream ---------------
// For m <= 8 activation rows. Workgroups of 16 waves, at most one per CU: the
// workgroup quantizes all m rows into LDS (every workgroup does; the m * k
// activations are L2-resident and small next to the weights), with the same
// absmax, divide and rounding as nq_act_quant_i8 (RowQuantizer), so codes and
// scales are identical. Each wave takes groups of R weight rows (group g =
// blockIdx.x + gridDim.x * (wave + 16 * i)); with short K its first group's
// weight loads go out before the quantization, so HBM latency overlaps it. Lane l owns 16-byte
// chunk positions l, l + 64, ... of the rows, reads the m code chunks of each
// position from LDS once (shared by the R rows) and accumulates exact int32
// sums with v_dot4_i32_i8; with short K the next group's loads are issued
// before the current group's math. The int32 sums are order independent and
// the epilogue is w8a8_epilogue: outputs equal the GEMV and MFMA paths bit for bit.
constexpr int kDecThreads = 1024;
constexpr int kDecMaxCodes = 128 * 1024;  // m * k bytes of codes in LDS

template <typename XT>
struct Vec8x;
template <>
struct Vec8x<_Float16> {
    typedef _Float16 h8 __attribute__((ext_vector_type(8)));
    h8 v;
    __device__ __forceinline__ void load(const _Float16* p) { v = *reinterpret_cast<const h8*>(p); }
    __device__ __forceinline__ float at(int j) const { return static_cast<float>(v[j]); }
};
template <>
struct Vec8x<float> {
    f4 a, b;
    __device__ __forceinline__ void load(const float* p) {
        a = reinterpret_cast<const f4*>(p)[0];
        b = reinterpret_cast<const f4*>(p)[1];
    }
    __device__ __forceinline__ float at(int j) const { return j < 4 ? a[j] : b[j - 4]; }
};

// PRE: x holds codes already (int8 [m, k] from nq_act_quant_i8, scales in
// pre_scale); phase 1 then only copies them into LDS.
// S > 1 (codes only): the waves of a workgroup form groups of S, and the S
// waves of a group share its weight rows, each taking M / S activation rows
// (narrow weights with many rows: more waves stream, each with a short chain).
template <int M, int R, int T, typename XT, typename YT, bool PRE = false, int S = 1>
__global__ __launch_bounds__(kDecThreads) void w8a8_decode_kernel(const XT* __restrict__ x,
                                                                  const int8_t* __restrict__ w,
                                                                  const float* __restrict__ ws,
                                                                  const float* __restrict__ bias,
                                                                  YT* __restrict__ y, int m, int n, int k,
                                                                  const float* __restrict__ pre_scale = nullptr) {
    extern __shared__ __attribute__((aligned(16))) int8_t xq[];  // [M][k] codes
    __shared__ float amax_red[kDecThreads / 64][M];
    __shared__ float a_scale[M];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int cpr = k >> 4;  // 16-byte code chunks per row
    const int vpr = k >> 3;  // 8-element activation vectors per row

    static_assert(S == 1 || (PRE && M % S == 0 && (kDecThreads / 64) % S == 0), "row slices");
    constexpr int MS = M / S;  // activation rows per wave
    const int i0 = (wave % S) * MS;

    // This wave's first group of weights, requested before anything else.
    const int groups = (n + R - 1) / R;
    const int wstride = gridDim.x * (kDecThreads / 64 / S);
    int g = blockIdx.x + gridDim.x * (wave / S);
    const v4i* wv = reinterpret_cast<const v4i*>(w);
    constexpr bool DB = T <= 2;
    v4i cur[T][R], nxt[DB ? T : 1][DB ? R : 1];
    auto load = [&](int grp, auto& buf) {
        const int r0 = min(grp, groups - 1) * R;
#pragma unroll
        for (int t = 0; t < T; ++t) {
            const int c = min(lane + 64 * t, cpr - 1);
#pragma unroll
            for (int r = 0; r < R; ++r)
                buf[t][r] = __builtin_nontemporal_load(wv + static_cast<size_t>(min(r0 + r, n - 1)) * cpr + c);
        }
    };
    // The activations are requested before that first group: phase 1 waits on
    // them, and the in-order load counter would otherwise hold it until the
    // weights had arrived too (long K: the weights are not held across phase 1,
    // whose activation vectors need the registers).
    if constexpr (PRE) {
        // Phase 1 for pre-quantized codes: 16-byte copies into LDS (rows past m zero).
        const int8_t* xc = reinterpret_cast<const int8_t*>(x);
        constexpr int UC = (M * T * 64 + kDecThreads - 1) / kDecThreads;  // M * cpr <= M * 64 T chunks
        v4i cv[UC];
#pragma unroll
        for (int u = 0; u < UC; ++u) {
            const int v = tid + kDecThreads * u, i = v / cpr;
            cv[u] = v < M * cpr && i < m ? *reinterpret_cast<const v4i*>(xc + static_cast<size_t>(i) * k + 16 * (v - i * cpr))
                                         : v4i{0, 0, 0, 0};
        }
        __builtin_amdgcn_sched_barrier(0);
        if constexpr (DB)
            if (g < groups) load(g, cur);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int u = 0; u < UC; ++u) {
            const int v = tid + kDecThreads * u;
            if (v < M * cpr) reinterpret_cast<v4i*>(xq)[v] = cv[u];
        }
        if (tid < M) a_scale[tid] = tid < m ? pre_scale[tid] : 0.0f;
        __syncthreads();
    } else {
    // Phase 1: each thread's activation vectors (v = tid + 1024 u) in registers,
    // per-row absmax, the row scales, then the codes into LDS.
    const int nv = M * vpr;
    constexpr int U = (M * T + 7) / 8;  // k <= 1024 T, so M * k / 8 <= 1024 U vectors
    Vec8x<XT> xv[U];
    float am[M];
#pragma unroll
    for (int i = 0; i < M; ++i) am[i] = 0.0f;
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const int v = min(tid + kDecThreads * u, nv - 1), i = v / vpr;
        xv[u].load(x + static_cast<size_t>(min(i, m - 1)) * k + 8 * (v - i * vpr));
    }
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (DB)
        if (g < groups) load(g, cur);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const int v = tid + kDecThreads * u;
        if (v < nv) {
            const int i = v / vpr;
            float a = 0.0f;
#pragma unroll
            for (int j = 0; j < 8; ++j) a = absmax_step(a, xv[u].at(j));
#pragma unroll
            for (int r = 0; r < M; ++r) am[r] = (r == i) ? absmax_step(am[r], a) : am[r];
        }
    }
#pragma unroll
    for (int i = 0; i < M; ++i) {
        const float a = wave_absmax(am[i]);
        if (lane == 0) amax_red[wave][i] = a;
    }
    __syncthreads();
    if (tid < M) {
        float a = 0.0f;
        for (int w2 = 0; w2 < kDecThreads / 64; ++w2) a = absmax_step(a, amax_red[w2][tid]);
        a_scale[tid] = a / 127.0f;
    }
    __syncthreads();
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const int v = tid + kDecThreads * u;
        if (v < nv) {
            const int i = v / vpr;
            int lo = 0, hi = 0;
            if (i < m) {
                const RowQuantizer rq(a_scale[i]);
                float vv[8];
#pragma unroll
                for (int j = 0; j < 8; ++j) vv[j] = xv[u].at(j);
                rq.pack8(vv, lo, hi);
            }
            typedef int v2i __attribute__((ext_vector_type(2)));
            reinterpret_cast<v2i*>(xq)[v] = v2i{lo, hi};  // rows past m hold zero codes
        }
    }
    __syncthreads();
    }

    // Phase 2: groups of R weight rows; T passes of 64 chunk positions.
    constexpr int G = 64 / (R * MS);
    for (; g < groups; g += wstride) {
        // The storing lane's weight scale, requested ahead of the next group's
        // weights so that waiting for it does not wait for them.
        const float wsv = ws[min(g * R + lane / G / MS, n - 1)];
        // The next group only where there is one: a clamped re-load of the last
        // group by every wave without a second group hammered one L2 channel.
        if constexpr (DB) {
            if (g + wstride < groups) load(g + wstride, nxt);
        }
        else load(g, cur);
        int acc[R * MS];
#pragma unroll
        for (int j = 0; j < R * MS; ++j) acc[j] = 0;
#pragma unroll
        for (int t = 0; t < T; ++t) {
            const int c = lane + 64 * t;
            if (c < cpr) {
#pragma unroll
                for (int i = 0; i < MS; ++i) {
                    const v4i a = reinterpret_cast<const v4i*>(xq)[(i0 + i) * cpr + c];
#pragma unroll
                    for (int r = 0; r < R; ++r)
#pragma unroll
                        for (int d = 0; d < 4; ++d)
                            acc[r * MS + i] = __builtin_amdgcn_sdot4(a[d], cur[t][r][d], acc[r * MS + i], false);
                }
            }
        }
        wave_reduce_multi<R * MS>(acc, lane);
        const int idx = lane / G, r = idx / MS, i = i0 + idx % MS, row = g * R + r;
        if (lane % G == 0 && row < n && i < m) {
            const float b = bias ? bias[row] : 0.0f;
            y[static_cast<size_t>(i) * n + row] = from_f32<YT>(w8a8_epilogue(acc[0], a_scale[i], wsv, b));
        }
        if constexpr (DB) {
#pragma unroll
            for (int t = 0; t < T; ++t)
#pragma unroll
                for (int r = 0; r < R; ++r) cur[t][r] = nxt[t][r];
        }
    }
}

// ---- long K: several 16-byte chunks per lane --------------------------------------------
// The kernels above give each lane one 16-byte weight chunk of a row, so a
// 576-lane workgroup covers int8 k <= 9216 and int4 k <= 18432. Longer rows
// (Llama-3-8B's down projection, k = 14336; Qwen2.5-7B's, k = 18944) take these:
// 256 (int8) or 512 (int4, W8A8) lanes stride K one chunk at a time, R weight
// rows per workgroup (their R loads in flight per lane, several workgroups per
// CU), the same per-chunk dot products as the one-chunk kernels and the same
// cross-wave reduction.

template <int R, int M, typename XT, typename YT>
__global__ __launch_bounds__(kLongKThreads) void gemv_q8_longk_kernel(
    const XT* __restrict__ x, const int8_t* __restrict__ w, const float* __restrict__ ws,
    const float* __restrict__ bias, YT* __restrict__ y, int m, int n, int k) {
    __shared__ float red[(kLongKThreads / kWave) * R * M];
    const int tid = threadIdx.x, wave = tid >> 6;
    const int chunks = k >> 4, row0 = xcd_row_group() * R;
    const float ws_early = ws[min(row0 + min(tid / M, R - 1), n - 1)];  // the storing lane's row scale, early
    float acc[R][M];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int i = 0; i < M; ++i) acc[r][i] = 0.0f;
#pragma unroll 1
    for (int c = tid; c < chunks; c += kLongKThreads) {
        v4i wv[R];
#pragma unroll
        for (int r = 0; r < R; ++r)
            wv[r] = __builtin_nontemporal_load(
                reinterpret_cast<const v4i*>(w + static_cast<size_t>(min(row0 + r, n - 1)) * k + c * 16));
#pragma unroll
        for (int i = 0; i < M; ++i) {
            XChunk<XT> xc;
            xc.load(x + static_cast<size_t>(min(i, m - 1)) * k + c * 16);
#pragma unroll
            for (int r = 0; r < R; ++r) {
                float p = acc[r][i];
#pragma unroll
                for (int d = 0; d < 4; ++d) {
                    const int wd = wv[r][d];
                    p = __builtin_fmaf(xc.at(4 * d + 0), sbyte_f32<0>(wd), p);
                    p = __builtin_fmaf(xc.at(4 * d + 1), sbyte_f32<1>(wd), p);
                    p = __builtin_fmaf(xc.at(4 * d + 2), sbyte_f32<2>(wd), p);
                    p = __builtin_fmaf(xc.at(4 * d + 3), sbyte_f32<3>(wd), p);
                }
                acc[r][i] = p;
            }
        }
    }
    reduce_to_lds<R, M, (R * M >= 16)>(acc, red, wave, tid & 63);
    __syncthreads();
    if (tid < R * M) {
        const int r = tid / M, i = tid % M, row = row0 + r;
        if (row < n && i < m) {
            float s = 0.0f;
#pragma unroll
            for (int q = 0; q < kLongKThreads / kWave; ++q) s += red[(q * R + r) * M + i];
            const float b = bias ? bias[row] : 0.0f;
            y[static_cast<size_t>(i) * n + row] = from_f32<YT>(__builtin_fmaf(s, ws_early, b));
        }
    }
}

// group: a multiple of 32 (each chunk's 32 codes share one scale).
template <int R, int M, typename XT, typename YT, typename ST>
__global__ __launch_bounds__(kLongKThreadsWide) void gemv_q4g_longk_kernel(
    const XT* __restrict__ x, const uint8_t* __restrict__ w, const ST* __restrict__ scale,
    const float* __restrict__ bias, YT* __restrict__ y, int m, int n, int k, int group) {
    __shared__ float red[(kLongKThreadsWide / kWave) * R * M];
    const int tid = threadIdx.x, wave = tid >> 6;
    const int chunks = k >> 5, rb = k >> 1, row0 = xcd_row_group() * R;
    const int blocks = (k + group - 1) / group;
    unsigned magic = 0x64006400u;
    asm volatile("" : "+v"(magic));  // one VGPR for every nibble pair below
    float acc[R][M];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int i = 0; i < M; ++i) acc[r][i] = 0.0f;
#pragma unroll 1
    for (int c = tid; c < chunks; c += kLongKThreadsWide) {
        v4i wv[R];
        float sc[R];
        const int blk = (c * 32) / group;
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const size_t row = static_cast<size_t>(min(row0 + r, n - 1));
            wv[r] = __builtin_nontemporal_load(reinterpret_cast<const v4i*>(w + row * rb + c * 16));
            sc[r] = to_f32(scale[row * blocks + blk]);
        }
#pragma unroll
        for (int i = 0; i < M; ++i) {
            const XT* xp = x + static_cast<size_t>(min(i, m - 1)) * k + c * 32;
            XChunk<XT> lo, hi;
            lo.load(xp);
            hi.load(xp + 16);
            // the codes as seen by this activation row: without the opaque copy
            // the compiler converts every code once for all M rows and keeps the
            // converted values live
            v4i wq[R];
#pragma unroll
            for (int r = 0; r < R; ++r) {
                wq[r] = wv[r];
                if constexpr (M > 1) asm volatile("" : "+v"(wq[r]));
            }
            if constexpr (sizeof(XT) == 2) {
                const typename XChunk<XT>::h8 q[4] = {lo.v[0], lo.v[1], hi.v[0], hi.v[1]};
                h2 pairs[16];
#pragma unroll
                for (int e = 0; e < 4; ++e)
#pragma unroll
                    for (int j = 0; j < 4; ++j) pairs[4 * e + j] = h2{q[e][j], q[e][j + 4]};
#pragma unroll
                for (int r = 0; r < R; ++r) acc[r][i] = __builtin_fmaf(dot32_q4_f16m(wq[r], pairs, magic), sc[r], acc[r][i]);
            } else {
                float xf[32];
#pragma unroll
                for (int e = 0; e < 16; ++e) {
                    xf[e] = lo.at(e);
                    xf[16 + e] = hi.at(e);
                }
#pragma unroll
                for (int r = 0; r < R; ++r) acc[r][i] = __builtin_fmaf(dot32_q4_f32(wq[r], xf), sc[r], acc[r][i]);
            }
        }
    }
    reduce_to_lds<R, M, (R * M >= 16)>(acc, red, wave, tid & 63);
    __syncthreads();
    if (tid < R * M) {
        const int r = tid / M, i = tid % M, row = row0 + r;
        if (row < n && i < m) {
            float s = 0.0f;
#pragma unroll
            for (int q = 0; q < kLongKThreadsWide / kWave; ++q) s += red[(q * R + r) * M + i];
            y[static_cast<size_t>(i) * n + row] = from_f32<YT>(s + (bias ? bias[row] : 0.0f));
        }
    }
}

// int8 activation codes: exact int32 sums (equal to every other W8A8 path).
template <int R, int M, typename YT, bool ACC_OUT>
__global__ __launch_bounds__(kLongKThreadsWide) void gemv_w8a8_longk_kernel(
    const int8_t* __restrict__ xq, const float* __restrict__ as, const int8_t* __restrict__ w,
    const float* __restrict__ ws, const float* __restrict__ bias, YT* __restrict__ y,
    int32_t* __restrict__ acc_out, int m, int n, int k) {
    __shared__ int red[(kLongKThreadsWide / kWave) * R * M];
    const int tid = threadIdx.x, wave = tid >> 6;
    const int chunks = k >> 4, row0 = xcd_row_group() * R;
    const float ws_early = ACC_OUT ? 0.0f : ws[min(row0 + min(tid / M, R - 1), n - 1)];  // the storing lane's
    int acc[R][M];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int i = 0; i < M; ++i) acc[r][i] = 0;
#pragma unroll 1
    for (int c = tid; c < chunks; c += kLongKThreadsWide) {
        v4i wv[R], xv[M];
#pragma unroll
        for (int r = 0; r < R; ++r)
            wv[r] = __builtin_nontemporal_load(
                reinterpret_cast<const v4i*>(w + static_cast<size_t>(min(row0 + r, n - 1)) * k + c * 16));
#pragma unroll
        for (int i = 0; i < M; ++i)
            xv[i] = *reinterpret_cast<const v4i*>(xq + static_cast<size_t>(min(i, m - 1)) * k + c * 16);
#pragma unroll
        for (int i = 0; i < M; ++i)
#pragma unroll
            for (int r = 0; r < R; ++r) {
                int p = acc[r][i];
#pragma unroll
                for (int d = 0; d < 4; ++d) p = __builtin_amdgcn_sdot4(xv[i][d], wv[r][d], p, false);
                acc[r][i] = p;
            }
    }
    reduce_to_lds<R, M, (R * M >= 16)>(acc, red, wave, tid & 63);
    __syncthreads();
    if (tid < R * M) {
        const int r = tid / M, i = tid % M, row = row0 + r;
        if (row < n && i < m) {
            int s = 0;
#pragma unroll
            for (int q = 0; q < kLongKThreadsWide / kWave; ++q) s += red[(q * R + r) * M + i];
            if constexpr (ACC_OUT) {
                acc_out[static_cast<size_t>(i) * n + row] = s;
            } else {
                const float b = bias ? bias[row] : 0.0f;
                y[static_cast<size_t>(i) * n + row] = from_f32<YT>(w8a8_epilogue(s, as[i], ws_early, b));
            }
        }
    }
}

// ---- generic bounds-checked kernels (any k, any alignment) -----------------------------
// One wave per output row; lanes stride K one element at a time; rows of x loop.
template <typename XT, typename YT>
__global__ void gemv_q8_generic_kernel(const XT* __restrict__ x, const int8_t* __restrict__ w,
                                       const float* __restrict__ ws, const float* __restrict__ bias,
                                       YT* __restrict__ y, int m, int n, int k) {
    const int row = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (row >= n) return;
    const int8_t* wr = w + static_cast<size_t>(row) * k;
    const float b = bias ? bias[row] : 0.0f;
    for (int i = 0; i < m; ++i) {
        const XT* xr = x + static_cast<size_t>(i) * k;
        float p = 0.0f;
        for (int j = lane; j < k; j += kWave) p = __builtin_fmaf(to_f32(xr[j]), static_cast<float>(wr[j]), p);
        p = wave_sum_f32(p);
        if (lane == 0) y[static_cast<size_t>(i) * n + row] = from_f32<YT>(__builtin_fmaf(p, ws[row], b));
    }
}

template <typename XT, typename YT, typename ST>
__global__ void gemv_q4g_generic_kernel(const XT* __restrict__ x, const uint8_t* __restrict__ w,
                                        const ST* __restrict__ scale, const float* __restrict__ bias,
                                        YT* __restrict__ y, int m, int n, int k, int group) {
    const int row = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (row >= n) return;
    const int rb = (k + 1) / 2, blocks = (k + group - 1) / group;
    const uint8_t* wr = w + static_cast<size_t>(row) * rb;
    const ST* sr = scale + static_cast<size_t>(row) * blocks;
    const float b = bias ? bias[row] : 0.0f;
    for (int i = 0; i < m; ++i) {
        const XT* xr = x + static_cast<size_t>(i) * k;
        float acc = 0.0f;
        // Lanes take whole blocks so each block's partial sum is scaled once.
        for (int blk = lane; blk < blocks; blk += kWave) {
            const int j0 = blk * group, j1 = min(j0 + group, k);
            float p = 0.0f;
            for (int j = j0; j < j1; ++j) {
                const int nib = (j & 1) ? (wr[j >> 1] >> 4) : (wr[j >> 1] & 15);
                p = __builtin_fmaf(to_f32(xr[j]), static_cast<float>(nib - 8), p);
            }
            acc = __builtin_fmaf(p, to_f32(sr[blk]), acc);
        }
        acc = wave_sum_f32(acc);
        if (lane == 0) y[static_cast<size_t>(i) * n + row] = from_f32<YT>(acc + b);
    }
}

template <typename YT, bool ACC_OUT>
__global__ void gemv_w8a8_generic_kernel(const int8_t* __restrict__ xq, const float* __restrict__ as,
                                         const int8_t* __restrict__ w, const float* __restrict__ ws,
                                         const float* __restrict__ bias, YT* __restrict__ y,
                                         int32_t* __restrict__ acc_out, int m, int n, int k) {
    const int row = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6);
    const int lane = threadIdx.x & 63;
    if (row >= n) return;
    const int8_t* wr = w + static_cast<size_t>(row) * k;
    for (int i = 0; i < m; ++i) {
        const int8_t* xr = xq + static_cast<size_t>(i) * k;
        int p = 0;
        for (int j = lane; j < k; j += kWave) p += static_cast<int>(xr[j]) * static_cast<int>(wr[j]);
        p = wave_sum_i32(p);
        if (lane == 0) {
            if constexpr (ACC_OUT) {
                acc_out[static_cast<size_t>(i) * n + row] = p;
            } else {
                const float b = bias ? bias[row] : 0.0f;
                y[static_cast<size_t>(i) * n + row] = from_f32<YT>(w8a8_epilogue(p, as[i], ws[row], b));
            }
        }
    }
}

// ---- greedy argmax over logits ---------------------------------------------------------
// Wave then workgroup reduction of (value, index) pairs by arg_better; the
// order is a total one on distinct indices, so the result does not depend on
// the reduction tree.
template <int O>
__device__ __forceinline__ void arg_step(float& bv, int& bi, int lane) {
    const float ov = xchg<O>(bv, lane);
    const int oi = xchg<O>(bi, lane);
    if (arg_better(ov, oi, bv, bi)) {
        bv = ov;
        bi = oi;
    }
}
template <int NT>
__device__ __forceinline__ void arg_reduce_block(float& bv, int& bi, float* sv, int* si) {
    const int tid = threadIdx.x;
    arg_step<32>(bv, bi, tid & 63);
    arg_step<16>(bv, bi, tid & 63);
    arg_step<8>(bv, bi, tid & 63);
    arg_step<4>(bv, bi, tid & 63);
    arg_step<2>(bv, bi, tid & 63);
    arg_step<1>(bv, bi, tid & 63);
    if ((tid & 63) == 0) {
        sv[tid >> 6] = bv;
        si[tid >> 6] = bi;
    }
    __syncthreads();
    bv = sv[0];
    bi = si[0];
#pragma unroll
    for (int w = 1; w < NT / 64; ++w)
        if (arg_better(sv[w], si[w], bv, bi)) {
            bv = sv[w];
            bi = si[w];
        }
}

// Partials of fp32 logits [m, n]: workgroup (j, i) scans elements
// [j * seg, (j + 1) * seg) of row i.
__global__ __launch_bounds__(256) void argmax_logits_kernel(const float* __restrict__ logits, int n, int seg,
                                                            ArgPart* __restrict__ part) {
    __shared__ float sv[4];
    __shared__ int si[4];
    const int i = blockIdx.y, j = blockIdx.x, tid = threadIdx.x;
    const float* row = logits + static_cast<size_t>(i) * n;
    const int beg = j * seg, end = min(n, beg + seg);
    float bv = -__builtin_inff();
    int bi = kArgNone;
    for (int e = beg + tid; e < end; e += 256) {
        const float v = row[e];
        if (arg_better(v, e, bv, bi)) {
            bv = v;
            bi = e;
        }
    }
    arg_reduce_block<256>(bv, bi, sv, si);
    if (tid == 0) {
        if (j == 0 && row[0] != row[0]) bi = -1;
        part[static_cast<size_t>(i) * gridDim.x + j] = ArgPart{bv, bi};
    }
}

// Final pass: row i's nparts partials -> ids[i] (0 when logit 0 is NaN). Each
// thread issues 8 independent loads before comparing (a load-compare chain
// waited one memory latency per partial: 18992 partials took ~20 us).
__global__ __launch_bounds__(1024) void argmax_final_kernel(const ArgPart* __restrict__ part, int nparts,
                                                            int64_t* __restrict__ ids) {
    constexpr int U = 8;
    __shared__ float sv[16];
    __shared__ int si[16];
    const int i = blockIdx.x, tid = threadIdx.x;
    const ArgPart* p = part + static_cast<size_t>(i) * nparts;
    float bv = -__builtin_inff();
    int bi = kArgNone;
    for (int base = tid; base < nparts; base += 1024 * U) {
        ArgPart q[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int j = base + u * 1024;
            q[u] = p[min(j, nparts - 1)];
            if (j >= nparts) q[u].i = kArgNone;
        }
#pragma unroll
        for (int u = 0; u < U; ++u)
            if (q[u].i >= 0 && arg_better(q[u].v, q[u].i, bv, bi)) {
                bv = q[u].v;
                bi = q[u].i;
            }
    }
    arg_reduce_block<1024>(bv, bi, sv, si);
    if (tid == 0) ids[i] = (p[0].i == -1 || bi == kArgNone) ? 0 : bi;
}

// Fused path's final reduction: gridDim.x workgroups per activation row
// (blockIdx.y), each reducing T * U partials with all its loads in flight, then
// one 64-bit agent-scope atomic max of its key and a ticket; the workgroup
// that takes the last ticket reads the key and writes the id. Ordering: each
// workgroup's key max is sequenced before its ticket increment, which is a
// release; the last ticket's increment is also an acquire, so every key max
// happens before its load of the key (release sequence on the ticket). Same
// result as argmax_final_kernel: the reference scan's first maximal index, 0
// when logit 0 is NaN or nothing qualifies.
__device__ __forceinline__ unsigned arg_order_bits(float v) {
    const unsigned u = __builtin_bit_cast(unsigned, v);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
template <int T, int U>
__global__ __launch_bounds__(T) void argmax_final_multi_kernel(const ArgPart* __restrict__ part, int nparts,
                                                                ArgCtl* __restrict__ ctl, int64_t* __restrict__ ids) {
    __shared__ float sv[16];
    __shared__ int si[16];
    const int i = blockIdx.y, tid = threadIdx.x;
    const ArgPart* p = part + static_cast<size_t>(i) * nparts;
    const int base = blockIdx.x * T * U + tid;
    ArgPart q[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const int j = base + u * T;
        q[u] = p[min(j, nparts - 1)];
        if (j >= nparts) q[u].i = kArgNone;
    }
    float bv = -__builtin_inff();
    int bi = kArgNone;
#pragma unroll
    for (int u = 0; u < U; ++u)
        if (q[u].i >= 0 && arg_better(q[u].v, q[u].i, bv, bi)) {
            bv = q[u].v;
            bi = q[u].i;
        }
    arg_reduce_block<T>(bv, bi, sv, si);
    if (tid == 0) {
        unsigned long long key = 0;
        if (blockIdx.x == 0 && p[0].i == -1) key = ~0ull;
        else if (bi != kArgNone) key = (static_cast<unsigned long long>(arg_order_bits(bv)) << 32) | (0xFFFFFFFFu - static_cast<unsigned>(bi));
        __hip_atomic_fetch_max(&ctl[i].key, key, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const unsigned t = __hip_atomic_fetch_add(&ctl[i].ticket, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
        if (t == gridDim.x - 1) {
            const unsigned long long f = __hip_atomic_load(&ctl[i].key, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            ids[i] = (f == ~0ull || f == 0) ? 0 : static_cast<int64_t>(0xFFFFFFFFu - static_cast<unsigned>(f & 0xFFFFFFFFu));
        }
    }
}
constexpr int kArgFinalT = 256, kArgFinalU = 8;

// ---- host dispatch ----------------------------------------------------------------------
inline int m_bucket(int64_t m) { return m <= 1 ? 1 : m <= 2 ? 2 : m <= 4 ? 4 : 8; }

// Rows per workgroup of the q8 GEMV. Very tall weights (an LM head) have
// workgroups to spare: 8 rows per workgroup halves the activation re-reads
// (measured 38.5 -> 36 us at n = 151936, k = 1536; 4 rows stay best at n = 4864).
//
// fp32 activations at m = 5..8: each workgroup reads all m rows of x (16 bytes
// of codes per lane meet 8 x 64 bytes of x), so the x re-reads rather than the
// weight bound the 2-row grid; 4 or 8 rows per workgroup cut them (measured, us,
// 2 -> 4 -> 8 rows, m = 8: n = 1536, k = 8960 24.1 -> 19.8 -> 15.6; n = 8960, k =
// 1536 20.2 -> 14.7 -> 13.4; n = 4864, k = 896 7.38 -> 6.35 -> 6.55; n = 896, k =
// 4864 8.42 -> 7.61 -> 9.38; n = k = 1536 5.52 -> 5.65 -> 6.15); at m = 3..4 4
// rows (2 -> 4: 15.8 -> 11.0, 11.1 -> 8.4, 5.07 -> 4.43, 6.26 -> 4.94; n = k =
// 1536 4.18 -> 4.30). fp16 x keeps 2 (its x chunks are half the bytes; 4 rows
// measured slower on four of the five shapes).
template <int M, typename XT>
int q8_rows(int n, int k) {
    if (M <= 2 && n >= 32768) return 8;
    if (M == 4 && sizeof(XT) == 4) return static_cast<int64_t>(n) * k >= (int64_t(3) << 20) ? 4 : 2;
    if (M == 8 && sizeof(XT) == 4) {
        const int64_t nk = static_cast<int64_t>(n) * k;
        return nk >= (int64_t(8) << 20) ? 8 : nk >= (int64_t(3) << 20) ? 4 : 2;
    }
    return rows_for<M>();
}

template <int M, bool AM = false, typename XT, typename YT>
void launch_q8(const XT* x, const int8_t* w, const float* ws, const float* b, YT* y, int m, int n,
               int k, hipStream_t s, ArgPart* part = nullptr, ArgCtl* ctl = nullptr) {
    const int chunks = k >> 4;
    const int threads = ((chunks + kWave - 1) / kWave) * kWave;
    constexpr int R = rows_for<M>();
    const int rows = q8_rows<M, XT>(n, k);
    // fp16 activation rows 3..8 on 3072 <= k <= 9216 (4096 at m = 5..8, where the
    // MFMA GEMM keeps k = 3584: n = 37888 46.4 against 49.3) and at least 12 Mi
    // codes: the K-split tile kernel, 8 weight rows per workgroup from k = 8192 (and at m =
    // 3..4 from 12288 rows), else 4. us, old -> new: m = 4, n = 8960, k = 5120
    // 19.0 -> 14.1; n = 4096, k = 4096 8.8 -> 7.1; n = 28672 34.9 -> 28.1; n =
    // 1536, k = 8960 8.9 -> 7.7; m = 8 (from the MFMA GEMM where it took these):
    // n = 8960, k = 5120 29.0 -> 20.7; n = 14336, k = 4096 25.3 -> 22.9; n =
    // 1536, k = 8960 12.4 -> 10.1. Smaller weights (n = 1536, k = 4096 5.0 ->
    // 5.3) and short K (k = 2048 4.0 -> 4.7) lost, k = 14336 even (m = 3..4).
    // fp32 activations, m = 3..4, int8 codes on weights of 8192 rows or more: the
    // fp32 tile kernel (us: n = 8960, k = 5120 25.5 -> 20.3; n = 14336, k = 4096
    // 27.9 -> 24.9; narrower weights lost, n = 1536, k = 8960 11.0 -> 12.6).
    if constexpr (!AM && sizeof(XT) == 4 && M == 4) {
        if (k >= 3072 && k <= 9216 && n >= 8192) {
            const int groups = (n + 3) / 4;
            int S = (2048 + groups - 1) / groups;
            S = S < 1 ? 1 : S > 8 ? 8 : S;
            gemv_tile_f32_kernel<false, 4, 4, YT, float><<<groups, 64 * S, 0, s>>>(
                x, reinterpret_cast<const uint8_t*>(w), ws, b, y, m, n, k, 0);
            return;
        }
    }
    // m = 2 on the same shapes: 4 weight rows from 4096 rows, 8 on fewer rows
    // from k = 8192 (us, old -> new: n = 8960, k = 5120 13.6 -> 11.0; n = 28672, k
    // = 4096 28.4 -> 22.3; n = 2048, k = 8192 6.8 -> 6.2; n = 1536, k = 8960 6.5 ->
    // 6.4; 4 rows there lost, 7.0).
    if constexpr (!AM && sizeof(XT) == 2 && M == 2) {
        if (k >= 3072 && k <= 9216 && static_cast<int64_t>(n) * k >= (int64_t(12) << 20) && (n >= 4096 || k >= 8192)) {
            const bool r8 = n < 4096;
            const int RT = r8 ? 8 : 4, groups = (n + RT - 1) / RT;
            int S = (2048 + groups - 1) / groups;
            S = S < 1 ? 1 : S > 8 ? 8 : S;
            if (r8)
                gemv_q8_tile_kernel<8, 2, YT><<<groups, 64 * S, 0, s>>>(x, w, ws, b, y, m, n, k);
            else
                gemv_q8_tile_kernel<4, 2, YT><<<groups, 64 * S, 0, s>>>(x, w, ws, b, y, m, n, k);
            return;
        }
    }
    if constexpr (!AM && sizeof(XT) == 2 && (M == 4 || M == 8)) {
        if (k >= (M == 8 ? 4096 : 3072) && k <= 9216 && static_cast<int64_t>(n) * k >= (int64_t(12) << 20)) {
            const bool r8 = k >= 8192 || (M == 4 && n >= 12288);
            const int RT = r8 ? 8 : 4, groups = (n + RT - 1) / RT;
            int S = (2048 + groups - 1) / groups;
            S = S < 1 ? 1 : S > 8 ? 8 : S;
            if (r8)
                gemv_q8_tile_kernel<8, M, YT><<<groups, 64 * S, 0, s>>>(x, w, ws, b, y, m, n, k);
            else
                gemv_q8_tile_kernel<4, M, YT><<<groups, 64 * S, 0, s>>>(x, w, ws, b, y, m, n, k);
            return;
        }
    }
    // 1024 < k <= 2048 in one wave, two chunks per lane, 2 weight rows: one
    // activation row on up to 6144 weight rows with fp16 x (us: n = k = 1536 3.23
    // -> 3.02; n = 6144, k = 2048 4.64 -> 4.42) or 2048 with fp32 x (3.26 -> 3.09;
    // n = 6144 lost 4.66 -> 4.99), and fp16 m = 3..4 from 6144 rows (n = 6144, k =
    // 2048 6.94 -> 6.31; n = 17920, k = 1536 11.8 -> 11.5; narrower even or worse).
    if constexpr (!AM && (M == 1 || (M == 4 && sizeof(XT) == 2))) {
        const bool take = M == 4 ? n >= 6144 : n <= (sizeof(XT) == 2 ? 6144 : 2048);
        if (k > 1024 && k <= 2048 && take) {
            gemv_q8_short_kernel<2, M, XT, YT><<<(n + 1) / 2, kWave, 0, s>>>(x, w, ws, b, y, m, n, k);
            return;
        }
    }
    // m = 2: a workgroup per activation row, the pair on one XCD (n = 1536, k =
    // 8960 fp16 x 7.47 -> 5.88 us, fp32 x 7.71 -> 6.71; n = 4864, k = 896 fp16
    // 3.96 -> 3.58; n = k = 1536 3.87 -> 3.41), except tall short-K weights (n =
    // 8960, k = 1536 lost 6.04 -> 6.48).
    if constexpr (M == 2 && !AM) {
        if (m > 1 && rows == R && (n < 8192 || k >= 4096)) {
            gemv_q8_kernel<R, 1, XT, YT, false, 2><<<(n + R - 1) / R * 2, threads, 0, s>>>(x, w, ws, b, y, m, n, k,
                                                                                           part, ctl);
            return;
        }
    }
    // fp32 activations at m = 5..8: two workgroups per row group, 4 activation
    // rows each (half the x registers and twice the workgroups; the pair shares
    // the weight rows through its XCD's L2), 8 weight rows where q8_rows picks 8
    // on short K, else 4; long K with at least 256 groups of 8 keeps the single
    // 8 x 8 workgroup (us, m = 8, old -> new: n = 1536, k = 8960 15.41 -> 14.05;
    // n = 8960, k = 1536 13.75 -> 12.20; n = 4864, k = 896 6.20 -> 5.41; n = k =
    // 1536 5.55 -> 4.49; n = 256, k = 1536 3.99 -> 3.64; n = 2048, k = 8192 stays
    // 13.74, against 14.55 / 16.35 with the pairs).
    // fp16 activations the same way on short K (m = 8: n = 8960, k = 1536 11.28 ->
    // 10.83; n = 4864, k = 896, m = 6 5.23 -> 5.05; n = 1536, k = 8960 lost 11.40 ->
    // 12.50).
    // fp16 activations at m = 3..4 on wide weights: 4 weight rows per workgroup
    // (half the activation re-reads; us, 2 -> 4 rows, m = 4: n = 28672, k = 4096
    // 40.0 -> 32.6; n = 6144, k = 4096 11.4 -> 10.6; n = 17920, k = 1536 even;
    // narrower or longer-K weights lost: n = 1536, k = 8960 7.9 -> 9.7; n = 4608,
    // k = 3584 8.6 -> 8.8).
    if constexpr (M == 4 && !AM && sizeof(XT) == 2) {
        if (n >= 6144 && k <= 8192) {
            gemv_q8_kernel<4, 4, XT, YT><<<(n + 3) / 4, threads, 0, s>>>(x, w, ws, b, y, m, n, k, part, ctl);
            return;
        }
    }
    if constexpr (M == 8 && !AM && sizeof(XT) == 2) {
        if (k < 4096) {
            gemv_q8_kernel<4, 4, XT, YT, false, 2><<<(n + 3) / 4 * 2, threads, 0, s>>>(x, w, ws, b, y, m, n, k,
                                                                                       part, ctl);
            return;
        }
    }
    if constexpr (M == 8 && !AM && sizeof(XT) == 4) {  // m = 5..8 (the M = 8 bucket)
        const bool long_k = k >= 4096;
        if (long_k && rows == 8 && n >= 8 * 256) {
            gemv_q8_kernel<8, 8, XT, YT><<<(n + 7) / 8, threads, 0, s>>>(x, w, ws, b, y, m, n, k, part, ctl);
        } else if (!long_k && rows == 8) {
            gemv_q8_kernel<8, 4, XT, YT, false, 2><<<(n + 7) / 8 * 2, threads, 0, s>>>(x, w, ws, b, y, m, n, k,
                                                                                       part, ctl);
        } else {
            gemv_q8_kernel<4, 4, XT, YT, false, 2><<<(n + 3) / 4 * 2, threads, 0, s>>>(x, w, ws, b, y, m, n, k,
                                                                                       part, ctl);
        }
        return;
    }
    if constexpr (!(M == 8 && !AM && sizeof(XT) == 4)) {
        if constexpr (M <= 2 || (M == 8 && sizeof(XT) == 4)) {  // the other row counts q8_rows picks
            if (rows == 8 && R != 8) {
                gemv_q8_kernel<8, M, XT, YT, AM><<<(n + 7) / 8, threads, 0, s>>>(x, w, ws, b, y, m, n, k, part, ctl);
                return;
            }
        }
        if constexpr (M >= 4 && sizeof(XT) == 4) {
            if (rows == 4) {
                gemv_q8_kernel<4, M, XT, YT, AM><<<(n + 3) / 4, threads, 0, s>>>(x, w, ws, b, y, m, n, k, part, ctl);
                return;
            }
        }
        gemv_q8_kernel<R, M, XT, YT, AM><<<(n + R - 1) / R, threads, 0, s>>>(x, w, ws, b, y, m, n, k, part, ctl);
    }
}

template <typename XT, typename YT>
void dispatch_q8(const XT* x, const int8_t* w, const float* ws, const float* b, YT* y, int m, int n,
                 int k, hipStream_t s) {
    switch (m_bucket(m)) {
        case 1: launch_q8<1>(x, w, ws, b, y, m, n, k, s); break;
        case 2: launch_q8<2>(x, w, ws, b, y, m, n, k, s); break;
        case 4: launch_q8<4>(x, w, ws, b, y, m, n, k, s); break;
        default: launch_q8<8>(x, w, ws, b, y, m, n, k, s); break;
    }
}

template <int M, typename XT, typename YT, typename ST>
void launch_q4g(const XT* x, const uint8_t* w, const ST* sc, const float* b, YT* y, int m, int n,
                int k, int g, hipStream_t s) {
    // Two rows per workgroup: the workgroup's 5..9 waves split K, which spreads
    // the unpack math over many SIMDs, and each activation chunk serves two rows
    // (measured at k = 8960, n = 1536: 1 row 4.83 us, 2 rows 4.46, 3 rows (512
    // workgroups, two per CU) 4.51, 4 rows 4.82, 6 rows 5.21, 8 rows 4.98).
    // fp32 activations at m = 2..8: 4 rows, so each 128-byte activation chunk
    // serves twice the codes (with 2 rows the x re-reads bound the kernel); the
    // 320-thread launch bound (k <= 10240) leaves 256 VGPRs per lane, where the
    // 576-thread bound spilled 7-22 of them (m = 8, n = 1536, k = 8960: 30.2 ->
    // 23.2 us; n = 8960, k = 1536 33.3 -> 20.1; m = 4, n = 1536, k = 8960 19.0 ->
    // 15.0; m = 2: 11.7 -> 10.6, n = 8960, k = 1536 10.4 -> 8.0). fp16
    // activations measured slower with 4 rows (12.5 -> 19.6), m = 1 about even.
    constexpr int R = 2;
    const int chunks = k >> 5;
    const int threads = ((chunks + kWave - 1) / kWave) * kWave;
    // fp16 activation rows 3..8 on long K (k >= 4096, or 3072 from 8192 rows: at k
    // = 3584 it lost on n = 3584, m = 8 12.8 -> 13.9, and won on n = 37888, m = 4
    // 44.9 -> 40.3, m = 8 54.4 -> 52.9; n = 8960, k = 3072, m = 8 18.5 -> 14.8): the
    // K-split tile kernel, 4 weight rows per workgroup (8 at m = 5..8 on fewer
    // than 4096 rows). us, old -> new: m = 4, n = 8960, k = 5120 21.6 -> 17.2; n =
    // 1536, k = 8960 9.7 -> 8.9; m = 8, n = 1536, k = 8960 12.8 -> 11.7 (4 rows
    // 14.1); n = 4096, k = 4096 13.2 -> 9.9; n = 6144 20.3 -> 13.3; m = 4, n = 4096,
    // k = 14336 25.9 -> 19.6. It lost at m = 4, k = 3584 (8.7 -> 9.2), on short K
    // (k = 1536: 3.8 -> 5.1) and on narrow weights (n = 896, k = 4864: m = 4 4.9
    // -> 5.3, m = 8 7.9 -> 9.4).
    // fp32 activations, m = 2..8, int4 codes on long K: the fp32 tile kernel, 4
    // weight rows (us, old -> new: m = 4, n = 14336, k = 4096 34.6 -> 22.7; n =
    // 4096, k = 4096 13.0 -> 9.8; n = 1536, k = 8960 15.5 -> 12.6; m = 8, n =
    // 8960, k = 5120 52.9 -> 45.6 (from the MFMA GEMM); n = 2048, k = 8192 21.3 ->
    // 16.5; m = 2, n = 14336, k = 4096 21.7 -> 16.4; m = 2 lost on fewer than 2048
    // rows, n = 1536, k = 8960 8.5 -> 9.2).
    if constexpr (sizeof(XT) == 4 && (M == 2 || M == 4 || M == 8)) {
        if (k >= 3072 && k <= 18432 && n >= (M == 2 ? 2048 : 1024)) {
            const int groups = (n + 3) / 4;
            int S = (2048 + groups - 1) / groups;
            S = S < 1 ? 1 : S > 8 ? 8 : S;
            gemv_tile_f32_kernel<true, 4, M, YT, ST><<<groups, 64 * S, 0, s>>>(x, w, sc, b, y, m, n, k, g);
            return;
        }
    }
    // m = 2 the same way from k = 4096 on 2048 rows or more (us, old -> new: n =
    // 4096, k = 14336 16.4 -> 12.9; n = 28672, k = 4096 21.7 -> 19.1; n = 2048, k
    // = 8192 6.45 -> 5.81; n = 1536, k = 8960 lost 6.1 -> 6.5).
    if constexpr (sizeof(XT) == 2 && M == 2) {
        if ((k >= 4096 || (k >= 3072 && n >= 8192)) && k <= 18432 && n >= 2048) {
            const int groups = (n + 3) / 4;
            int S = (2048 + groups - 1) / groups;
            S = S < 1 ? 1 : S > 8 ? 8 : S;
            gemv_q4g_tile_kernel<4, 2, YT, ST><<<groups, 64 * S, 0, s>>>(x, w, sc, b, y, m, n, k, g);
            return;
        }
    }
    if constexpr (sizeof(XT) == 2 && (M == 4 || M == 8)) {
        if ((k >= 4096 || (k >= 3072 && n >= 8192)) && k <= 18432 && n >= 1024) {
            const bool r8 = M == 8 && n < 4096;
            const int RT = r8 ? 8 : 4, groups = (n + RT - 1) / RT;
            int S = (2048 + groups - 1) / groups;
            S = S < 1 ? 1 : S > 8 ? 8 : S;
            if constexpr (M == 8) {
                if (r8) {
                    gemv_q4g_tile_kernel<8, 8, YT, ST><<<groups, 64 * S, 0, s>>>(x, w, sc, b, y, m, n, k, g);
                    return;
                }
            }
            gemv_q4g_tile_kernel<4, M, YT, ST><<<groups, 64 * S, 0, s>>>(x, w, sc, b, y, m, n, k, g);
            return;
        }
    }
    // Short rows: half a chunk per lane in one wave, 2 weight rows per workgroup,
    // 4 on tall weights (us, old -> new, m = 1 / 2 / 4 / 8, fp16 x: n = 4864, k =
    // 896 3.66 -> 3.30 / 4.52 -> 3.79 / 5.87 -> 4.75 / 8.78 -> 7.50; n = 9728
    // 4.39 -> 3.79 (4 rows) / 5.69 -> 4.67 / 8.03 -> 6.18 / 13.9 -> 10.1; fp32
    // x: n = 4864 4.63 -> 3.56 / 5.53 -> 3.97 / 6.99 -> 4.87 / 9.87 -> 7.68; n =
    // 9728 5.94 -> 4.22 / 7.12 -> 4.83 / 10.6 -> 6.42 / 17.1 -> 12.2). The
    // one-chunk kernel left half of each wave idle there (28 of 64 lanes at k =
    // 896) and re-read 32 activation elements per 16 bytes of codes. m = 5..8
    // takes 4 rows with fp32 x or from 8192 rows (fp32 x, n = 4864, k = 896 8.2
    // -> 6.8; n = 9728 12.4 -> 10.4; fp16 x n = 9728 7.7 -> 7.3; fp16 x on fewer
    // rows even).
    if (k <= 1024) {
        constexpr bool f32x = sizeof(XT) == 4;
        const bool four = M == 8 ? f32x || n >= 8192
                          : M == 1 ? n >= 8192
                          : M == 2 ? n >= (f32x ? 4096 : 8192)
                                   : f32x && n >= 4096;
        if (four) {
            if constexpr (M != 4 || f32x)
                gemv_q4g_short_kernel<4, M, XT, YT, ST><<<(n + 3) / 4, kWave, 0, s>>>(x, w, sc, b, y, m, n, k, g);
        } else {
            if constexpr (M != 8 || !f32x)  // (always four rows there)
                gemv_q4g_short_kernel<2, M, XT, YT, ST><<<(n + 1) / 2, kWave, 0, s>>>(x, w, sc, b, y, m, n, k, g);
        }
        return;
    }
    // k <= 2048: two half chunks per lane (us, old -> new: fp16 x, m = 4, n =
    // 17920, k = 1536 12.4 -> 11.5; m = 8 22.9 -> 17.9; n = 6144, k = 2048 11.2
    // -> 8.4; m = 2 5.02 -> 4.71; fp32 x, m = 1, n = 6144 5.78 -> 4.77, with 4
    // rows n = 17920 8.54 -> 7.92; m = 2, n = k = 1536 4.39 -> 3.71; m = 4 4.86 ->
    // 4.40). Left out where it lost: one fp16 row on tall weights (n = 8960
    // 4.58 -> 4.81), fp16 m = 2 and fp32 m = 4 from 8192 rows (8.34 -> 8.46, 11.8
    // -> 12.1) and fp32 m = 5..8, whose 16 activation chunks per lane spill (19.7
    // -> 26.7).
    if (k <= 2048) {
        constexpr bool f32x = sizeof(XT) == 4;
        if constexpr (M == 1 && f32x) {
            if (n >= 8192)
                gemv_q4g_short_kernel<4, 1, XT, YT, ST, 2><<<(n + 3) / 4, kWave, 0, s>>>(x, w, sc, b, y, m, n, k, g);
            else
                gemv_q4g_short_kernel<2, 1, XT, YT, ST, 2><<<(n + 1) / 2, kWave, 0, s>>>(x, w, sc, b, y, m, n, k, g);
            return;
        } else if constexpr ((M == 2 || M == 4) || (M == 8 && !f32x)) {
            const bool two = M == 8 || (M == 2 ? (f32x || n < 8192) : (!f32x || n < 8192));
            if (two) {
                gemv_q4g_short_kernel<2, M, XT, YT, ST, 2><<<(n + 1) / 2, kWave, 0, s>>>(x, w, sc, b, y, m, n, k, g);
                return;
            }
        }
    }
    // One fp16 activation row on long K: half a chunk per lane, twice the waves
    // (k = 8960, n = 1536: 4.67-4.69 -> 4.52-4.55 us with 2 rows; one row 5.85,
    // 2 or 3 whole chunks per lane 5.6-5.8), 3 rows per workgroup with the
    // activation loaded first, 6 for tall weights (n = 8960, k = 5120: whole
    // chunks with 2 / 4 / 6 rows 8.0 / 7.6 / 8.3 us, half chunks with 6 rows 7.3).
    if constexpr (M == 1 && sizeof(XT) == 2) {
        const int th = ((2 * chunks + kWave - 1) / kWave) * kWave;
        // From k = 2048 on tall weights (6 rows; us: n = 14336, k = 4096 9.2 -> 8.75;
        // n = 6144 5.6 -> 5.3; n = 4608, k = 3584 4.8 -> 4.57; n = 4096 and 28672
        // even), from k = 5120 below 4096 rows (n = 3584, k = 3584 lost 4.33 -> 4.6).
        if ((chunks >= 160 || (chunks >= 64 && n >= 4096)) && th <= kMaxGemvThreads) {
            if (n >= 4096)
                gemv_q4g_x1h_half_kernel<6, YT, ST><<<(n + 5) / 6, th, 0, s>>>(x, w, sc, b, y, n, k, g);
            else
                gemv_q4g_x1h_half_kernel<3, YT, ST><<<(n + 2) / 3, th, 0, s>>>(x, w, sc, b, y, n, k, g);
            return;
        }
        // 9216 < k <= 16384: the same half chunks with up to 16 waves, against one
        // whole chunk per lane over 2 rows (us: n = 4096, k = 14336 10.6 -> 9.6; n
        // = 4096, k = 11008 9.1 -> 7.9; n = 5120, k = 13824 12.3 -> 11.5; n = 2048,
        // k = 12288 6.2 -> 6.0; n = 8192, k = 14336 18.2 -> 16.4-16.8 with 6 rows;
        // n = 14336, k = 12288 24.2 -> 20.3-22.9; 4 rows on n >= 8192 17.0 / 21.9-22.8,
        // 2 rows lost everywhere).
        if (th > kMaxGemvThreads && th <= 1024) {
            if (n >= 8192)
                gemv_q4g_x1h_half_kernel<6, YT, ST, 1024><<<(n + 5) / 6, th, 0, s>>>(x, w, sc, b, y, n, k, g);
            else if (n >= 4096)
                gemv_q4g_x1h_half_kernel<4, YT, ST, 1024><<<(n + 3) / 4, th, 0, s>>>(x, w, sc, b, y, n, k, g);
            else
                gemv_q4g_x1h_half_kernel<3, YT, ST, 1024><<<(n + 2) / 3, th, 0, s>>>(x, w, sc, b, y, n, k, g);
            return;
        }
    }
    // Pairs of workgroups per row group over halves of the activation rows (as
    // the q8 GEMV; us, m = 8 / 4, old -> pairs): m = 3..4 always (n = 1536, k =
    // 8960 fp16 10.48 -> 9.31, fp32 15.17 -> 14.96; n = 4864, k = 896 fp16 m = 3
    // 6.59 -> 5.42); m = 5..8 fp32 x from k = 1024 (k = 8960 23.6 -> 21.6, n =
    // 8960, k = 1536 20.1 -> 19.0; n = 4864, k = 896 lost 9.74 -> 10.56), fp16 x
    // on short K (n = 8960, k = 1536 13.0 -> 12.5; k = 8960 lost 12.0 -> 17.9).
    // m = 2: fp32 x on long K (n = 1536, k = 8960: 10.83 -> 8.30; fp16 x and
    // short K lost 2-4%).
    // (m = 2 with fp16 x never pairs; the M = 4 bucket, m = 3..4, always does)
    constexpr bool kPairs = (M == 2 && sizeof(XT) == 4) || M == 4 || M == 8;
    if constexpr (kPairs) {
        constexpr int MH = M / 2;
        const bool pairs = M == 2   ? k >= 4096
                           : M == 4 ? true
                                    : sizeof(XT) == 4 ? k >= 1024 : k < 4096;
        if (pairs) {
            if constexpr (sizeof(XT) == 4) {
                if (threads <= 320 && n >= 1024) {
                    gemv_q4g_kernel<4, MH, XT, YT, ST, 320, 2><<<(n + 3) / 4 * 2, threads, 0, s>>>(x, w, sc, b, y, m, n,
                                                                                                 k, g);
                    return;
                }
                // Past k = 10240 the same 4 rows on the 576-thread bound for up to two
                // activation rows per workgroup (143 VGPRs, no spills; us, 2 -> 4 rows:
                // m = 2, n = 4096, k = 14336 36.4 -> 26.1; m = 4 64.2 -> 44.6; n = 8192,
                // k = 11008 103.7 -> 75.4; n = 1536, k = 12288 23.3 -> 16.9).
                if constexpr (MH == 1) {  // (m = 3..4 there: the fp32 tile kernel above)
                    if (threads > 320 && n >= 1024) {
                        gemv_q4g_kernel<4, MH, XT, YT, ST, kMaxGemvThreads, 2><<<(n + 3) / 4 * 2, threads, 0, s>>>(
                            x, w, sc, b, y, m, n, k, g);
                        return;
                    }
                }
            } else {
                // m = 3..4 on wide, short-K weights: 4 weight rows per workgroup pair
                // (us, m = 4: n = 28672, k = 4096 38.0 -> 35.0; n = 17920, k = 1536
                // 13.5 -> 12.6; n = 3584, k = 3584 7.8 -> 7.5; lost on n = 1536, k =
                // 8960 9.7 -> 11.3 and n = 4096, k = 14336 26.7 -> 29.1).
                if constexpr (M == 4) {
                    if (n >= 3584 && k <= 4096) {
                        gemv_q4g_kernel<4, MH, XT, YT, ST, kMaxGemvThreads, 2><<<(n + 3) / 4 * 2, threads, 0, s>>>(
                            x, w, sc, b, y, m, n, k, g);
                        return;
                    }
                }
                gemv_q4g_kernel<R, MH, XT, YT, ST, kMaxGemvThreads, 2><<<(n + R - 1) / R * 2, threads, 0, s>>>(
                    x, w, sc, b, y, m, n, k, g);
                return;
            }
        }
    }
    if constexpr (M == 4 && sizeof(XT) == 2) {
        return;  // the pairs above took every m = 3..4 launch
    } else {
        if constexpr (M == 2 && sizeof(XT) == 4) {  // (M = 4 and 8 pair on this condition above)
            if (threads <= 320 && n >= 1024) {  // 256+ workgroups (n = 256, m = 5: 5.66 -> 6.76 us with 4 rows)
                gemv_q4g_kernel<4, M, XT, YT, ST, 320><<<(n + 3) / 4, threads, 0, s>>>(x, w, sc, b, y, m, n, k, g);
                return;
            }
        }
        if constexpr (M == 1) {
            // Tall weights: more rows per workgroup, fewer re-reads of the
            // activation chunk (every workgroup reads all of x, as many bytes as
            // two rows of codes at k = 4096): fp16 x, us, 2 / 4 / 8 rows: n =
            // 128256, k = 4096 64.5 / 54.5 / 52.7; n = 152064, k = 3584 66.2 /
            // 58.2 / 54.7; n = 37888, k = 3584 18.1 / 16.0 / 16.6; n = 28672 14.8 /
            // 13.7 / 14.4; n = 6144 5.7 / 6.0 / 6.6 (fewer workgroups lose below).
            // fp32 x (128 bytes of x per 16 bytes of codes): 4 rows from 4096 rows or
            // k = 4096, 8 from 24576 rows (us, 2 -> 4 rows: n = 4096, k = 14336 22.8 ->
            // 14.8; n = 17920, k = 1536 11.0 -> 8.6; n = 6144, k = 4096 9.5 -> 8.4; n =
            // 1536, k = 8960 7.5 -> 7.3; n = 28672, k = 4096 23.3 -> 20.6 with 8 rows;
            // n = k = 1536 lost 3.5 -> 3.8).
            if constexpr (sizeof(XT) == 4) {
                if (n >= 24576) {
                    gemv_q4g_kernel<8, 1, XT, YT, ST><<<(n + 7) / 8, threads, 0, s>>>(x, w, sc, b, y, m, n, k, g);
                    return;
                }
                if (n >= 4096 || k >= 4096) {
                    gemv_q4g_kernel<4, 1, XT, YT, ST><<<(n + 3) / 4, threads, 0, s>>>(x, w, sc, b, y, m, n, k, g);
                    return;
                }
            }
            if (n >= 65536) {
                gemv_q4g_kernel<8, 1, XT, YT, ST><<<(n + 7) / 8, threads, 0, s>>>(x, w, sc, b, y, m, n, k, g);
                return;
            }
            if (n >= 24576) {
                gemv_q4g_kernel<4, 1, XT, YT, ST><<<(n + 3) / 4, threads, 0, s>>>(x, w, sc, b, y, m, n, k, g);
                return;
            }
        }
        gemv_q4g_kernel<R, M, XT, YT, ST><<<(n + R - 1) / R, threads, 0, s>>>(x, w, sc, b, y, m, n, k, g);
    }
}

template <typename XT, typename YT, typename ST>
void dispatch_q4g(const XT* x, const uint8_t* w, const ST* sc, const float* b, YT* y, int m, int n,
                  int k, int g, hipStream_t s) {
    switch (m_bucket(m)) {
        case 1: launch_q4g<1>(x, w, sc, b, y, m, n, k, g, s); break;
        case 2: launch_q4g<2>(x, w, sc, b, y, m, n, k, g, s); break;
        case 4: launch_q4g<4>(x, w, sc, b, y, m, n, k, g, s); break;
        default: launch_q4g<8>(x, w, sc, b, y, m, n, k, g, s); break;
    }
}

// Long-K launches (one m bucket of up to 8 activation rows each): 4 weight rows
// per workgroup for up to four activation rows, 2 for more (m = 3..4 with 2 rows
// re-read the activation twice as often: n = 8192, k = 28672 int8 86.5 -> 64.8
// us with 4 rows; n = 4096, k = 14336 int8 22.9 -> 19.8, W8A8 20.6 -> 17.6; n =
// 4096, k = 28672 int4 40.5 -> 37.8); one activation row
// on 8192 weight rows or more takes 8 (half the activation re-reads: n = 8192,
// k = 28672 int8 42.8 -> 39.9 us, int4 27.5 -> 26.2; n = 14336, k = 10240 27.5 ->
// 26.1; n = 1536, k = 20480 lost 10.5 -> 11.3).
template <typename XT, typename YT>
void dispatch_q8_longk(const XT* x, const int8_t* w, const float* ws, const float* b, YT* y, int m, int n, int k,
                       hipStream_t s) {
    auto go = [&](auto mt) {
        constexpr int M = decltype(mt)::value, R = M <= 4 ? 4 : 2;
        gemv_q8_longk_kernel<R, M, XT, YT><<<(n + R - 1) / R, kLongKThreads, 0, s>>>(x, w, ws, b, y, m, n, k);
    };
    // One fp16 row up to k = 12288: one 16-byte chunk per lane over up to 16 waves,
    // 4 rows per workgroup (us, long-K kernel -> this: n = 4096, k = 11008 11.9 ->
    // 10.0; n = 2048, k = 12288 8.0 -> 6.8; n = 1536, k = 10240 6.8 -> 5.9; n =
    // 14336, k = 12288 29.8 -> 28.2; k = 14336 and fp32 x lost: 12.2 -> 12.6, 14.1 ->
    // 14.7).
    if constexpr (sizeof(XT) == 2) {
        if (m == 1 && k <= 12288) {
            const int th = ((k / 16 + kWave - 1) / kWave) * kWave;
            gemv_q8_kernel<4, 1, XT, YT, false, 1, 1024><<<(n + 3) / 4, th, 0, s>>>(x, w, ws, b, y, m, n, k, nullptr,
                                                                                    nullptr);
            return;
        }
    }
    if (m == 1 && n >= 8192) {
        gemv_q8_longk_kernel<8, 1, XT, YT><<<(n + 7) / 8, kLongKThreads, 0, s>>>(x, w, ws, b, y, m, n, k);
        return;
    }
    switch (m_bucket(m)) {
        case 1: go(std::integral_constant<int, 1>{}); break;
        case 2: go(std::integral_constant<int, 2>{}); break;
        case 4: go(std::integral_constant<int, 4>{}); break;
        default: go(std::integral_constant<int, 8>{}); break;
    }
}
template <typename XT, typename YT, typename ST>
void dispatch_q4g_longk(const XT* x, const uint8_t* w, const ST* sc, const float* b, YT* y, int m, int n, int k,
                        int group, hipStream_t s) {
    auto go = [&](auto mt) {
        constexpr int M = decltype(mt)::value, R = M <= 4 ? 4 : 2;
        gemv_q4g_longk_kernel<R, M, XT, YT, ST><<<(n + R - 1) / R, kLongKThreadsWide, 0, s>>>(x, w, sc, b, y, m, n, k,
                                                                                          group);
    };
    if (m == 1 && n >= 8192) {
        gemv_q4g_longk_kernel<8, 1, XT, YT, ST><<<(n + 7) / 8, kLongKThreadsWide, 0, s>>>(x, w, sc, b, y, m, n, k, group);
        return;
    }
    switch (m_bucket(m)) {
        case 1: go(std::integral_constant<int, 1>{}); break;
        case 2: go(std::integral_constant<int, 2>{}); break;
        case 4: go(std::integral_constant<int, 4>{}); break;
        default: go(std::integral_constant<int, 8>{}); break;
    }
}

nq_status check_linear(const void* x, const void* w, const void* y, int64_t m, int64_t n,
                       int64_t k, const char* who) {
    NQ_REQUIRE(m >= 0 && n >= 0 && k >= 0, NQ_BAD_SHAPE, "%s: negative shape", who);
    NQ_REQUIRE(m <= kMaxIndex && n <= kMaxIndex && k <= kMaxIndex && m * k <= (int64_t(1) << 40) &&
                   n * k <= (int64_t(1) << 40) && m * n <= (int64_t(1) << 40),
               NQ_BAD_SHAPE, "%s: shape m=%lld n=%lld k=%lld exceeds the supported range", who,
               (long long)m, (long long)n, (long long)k);
    if (m == 0 || n == 0) return NQ_OK;
    NQ_REQUIRE(y && (k == 0 || (x && w)), NQ_BAD_ARG, "%s: null pointer", who);
    return NQ_OK;
}

}  // namespace

// Exposed to the W8A8 entry points (nq_w8a8.hip).
nq_status gemv_w8a8_launch(const int8_t* xq, const float* as, const int8_t* w, const float* ws,
                           const float* bias, void* y, nq_dtype ydt, int32_t* acc_out, int64_t m,
                           int64_t n, int64_t k, bool generic, hipStream_t s) {
    const int mi = static_cast<int>(m), ni = static_cast<int>(n), ki = static_cast<int>(k);
    const bool fast = !generic && k > 0 && k % 16 == 0 && k / 16 <= kMaxGemvThreads && m <= 8 &&
                      aligned(xq, 16) && aligned(w, 16);
    const bool long_k = !generic && k % 16 == 0 && k / 16 > kMaxGemvThreads && m <= 8 && aligned(xq, 16) &&
                        aligned(w, 16);
    if (long_k) {
        auto go = [&](auto mt) {
            constexpr int M = decltype(mt)::value, R = M <= 4 ? 4 : 2;
            const unsigned grid = static_cast<unsigned>((n + R - 1) / R);
            if (acc_out)
                gemv_w8a8_longk_kernel<R, M, float, true><<<grid, kLongKThreadsWide, 0, s>>>(xq, as, w, ws, bias, nullptr,
                                                                                         acc_out, mi, ni, ki);
            else if (ydt == NQ_F32)
                gemv_w8a8_longk_kernel<R, M, float, false><<<grid, kLongKThreadsWide, 0, s>>>(
                    xq, as, w, ws, bias, static_cast<float*>(y), nullptr, mi, ni, ki);
            else
                gemv_w8a8_longk_kernel<R, M, _Float16, false><<<grid, kLongKThreadsWide, 0, s>>>(
                    xq, as, w, ws, bias, static_cast<_Float16*>(y), nullptr, mi, ni, ki);
        };
        switch (m_bucket(m)) {
            case 1: go(std::integral_constant<int, 1>{}); break;
            case 2: go(std::integral_constant<int, 2>{}); break;
            case 4: go(std::integral_constant<int, 4>{}); break;
            default: go(std::integral_constant<int, 8>{}); break;
        }
        return launch_status("gemv_w8a8_longk_kernel");
    }
    if (!fast) {
        const int wpb = 4;
        const unsigned grid = static_cast<unsigned>((n + wpb - 1) / wpb);
        if (acc_out)
            gemv_w8a8_generic_kernel<float, true><<<grid, wpb * kWave, 0, s>>>(xq, as, w, ws, bias, nullptr, acc_out, mi, ni, ki);
        else if (ydt == NQ_F32)
            gemv_w8a8_generic_kernel<float, false><<<grid, wpb * kWave, 0, s>>>(xq, as, w, ws, bias, static_cast<float*>(y), nullptr, mi, ni, ki);
        else
            gemv_w8a8_generic_kernel<_Float16, false><<<grid, wpb * kWave, 0, s>>>(xq, as, w, ws, bias, static_cast<_Float16*>(y), nullptr, mi, ni, ki);
        return launch_status("gemv_w8a8_generic_kernel");
    }
    const int threads = ((ki / 16 + kWave - 1) / kWave) * kWave;
    auto go = [&](auto mtag) {
        constexpr int M = decltype(mtag)::value;
        constexpr int R = w8a8_rows_for<M>();
        const unsigned grid = static_cast<unsigned>((n + R - 1) / R);
        if (acc_out)
            gemv_w8a8_kernel<R, M, float, true><<<grid, threads, 0, s>>>(xq, as, w, ws, bias, nullptr, acc_out, mi, ni, ki);
        else if (ydt == NQ_F32)
            gemv_w8a8_kernel<R, M, float, false><<<grid, threads, 0, s>>>(xq, as, w, ws, bias, static_cast<float*>(y), nullptr, mi, ni, ki);
        else
            gemv_w8a8_kernel<R, M, _Float16, false><<<grid, threads, 0, s>>>(xq, as, w, ws, bias, static_cast<_Float16*>(y), nullptr, mi, ni, ki);
    };
    switch (m_bucket(m)) {
        case 1: go(std::integral_constant<int, 1>{}); break;
        case 2: go(std::integral_constant<int, 2>{}); break;
        case 4: go(std::integral_constant<int, 4>{}); break;
        default: go(std::integral_constant<int, 8>{}); break;
    }
    return launch_status("gemv_w8a8_kernel");
}

namespace {
// W8A8 batches (m <= 8) over the activation codes: the tile layout with
// v_dot4_i32_i8 on 16-byte chunks of weight and activation codes (exact int32
// sums, so the results equal every other W8A8 path bit for bit); a workgroup of
// S waves owns R weight rows and splits K between its waves.
template <int R, int M, typename YT>
__global__ __launch_bounds__(512) void gemv_w8a8_tile_kernel(
    const int8_t* __restrict__ xq, const float* __restrict__ as, const int8_t* __restrict__ w,
    const float* __restrict__ ws, const float* __restrict__ bias, YT* __restrict__ y, int m, int n, int k) {
    constexpr int NV = R * M, G = 64 / NV;
    __shared__ int red[8][NV];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, nw = block_threads() >> 6;
    const int chunks = k >> 4;
    const int row0 = xcd_row_group() * R;
    int acc[R][M];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int i = 0; i < M; ++i) acc[r][i] = 0;
#pragma unroll 1
    for (int c0 = wave * kWave; c0 < chunks; c0 += kWave * nw) {
        const int c = c0 + lane;
        const bool act = c < chunks;
        const int cc = act ? c : 0;
        v4i xv[M];
#pragma unroll
        for (int i = 0; i < M; ++i) xv[i] = *reinterpret_cast<const v4i*>(xq + static_cast<size_t>(min(i, m - 1)) * k + cc * 16);
        v4i wv[R];
#pragma unroll
        for (int r = 0; r < R; ++r)
            wv[r] = __builtin_nontemporal_load(
                reinterpret_cast<const v4i*>(w + static_cast<size_t>(min(row0 + r, n - 1)) * k + cc * 16));
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
            for (int i = 0; i < M; ++i) {
                int p = 0;
#pragma unroll
                for (int d = 0; d < 4; ++d) p = __builtin_amdgcn_sdot4(xv[i][d], wv[r][d], p, false);
                acc[r][i] += act ? p : 0;
            }
    }
    const int v = wave_reduce_rows<R, M, true>(acc, lane);
    if (lane % G == 0) red[wave][lane / G] = v;
    __syncthreads();
    if (tid < NV) {
        const int r = tid / M, i = tid % M, row = row0 + r;
        if (row < n && i < m) {
            int t = 0;
            for (int q = 0; q < nw; ++q) t += red[q][tid];
            const float b = bias ? bias[row] : 0.0f;
            y[static_cast<size_t>(i) * n + row] = from_f32<YT>(w8a8_epilogue(t, as[i], ws[row], b));
        }
    }
}
}  // namespace

// Host launch of the W8A8 tile kernel over pre-quantized codes (m <= 8, k % 16
// == 0, 16-byte aligned codes); returns false (nothing launched) outside that.
bool w8a8_tile_launch(const int8_t* xq, const float* as, const int8_t* w, const float* ws, const float* bias,
                      void* y, nq_dtype ydt, int64_t m, int64_t n, int64_t k, hipStream_t s, nq_status* st) {
    if (!(m >= 1 && m <= 8 && k > 0 && k % 16 == 0 && aligned(w, 16) && aligned(xq, 16) && n <= kMaxIndex))
        return false;
    const int mi = static_cast<int>(m), ni = static_cast<int>(n), ki = static_cast<int>(k);
    auto go = [&](auto mtag, auto* yp) {
        constexpr int M = decltype(mtag)::value;
        constexpr int R = 4;
        const int groups = (ni + R - 1) / R;
        int S = (2048 + groups - 1) / groups;
        S = S < 1 ? 1 : S > 8 ? 8 : S;
        gemv_w8a8_tile_kernel<R, M><<<groups, 64 * S, 0, s>>>(xq, as, w, ws, bias, yp, mi, ni, ki);
    };
    auto with_y = [&](auto mtag) {
        if (ydt == NQ_F32) go(mtag, static_cast<float*>(y));
        else go(mtag, static_cast<_Float16*>(y));
    };
    with_y(std::integral_constant<int, 8>{});
    *st = launch_status("gemv_w8a8_tile_kernel");
    return true;
}

// The decode kernel for m <= 8 (see w8a8_decode_kernel): with pre_scale ==
// nullptr it quantizes x itself (one launch), else x is the int8 codes of
// nq_act_quant_i8 and pre_scale their row scales (then also m <= 32, as one
// batch of 16 or 32). Returns false (nothing launched) outside its contract:
// k % 16 == 0, k <= 9216, the padded m * k codes within 128 KB of LDS, 16-byte
// aligned x and w.
bool w8a8_decode_launch(const void* x, nq_dtype xdt, const int8_t* w, const float* ws, const float* bias,
                        void* y, nq_dtype ydt, int64_t m, int64_t n, int64_t k, hipStream_t s, nq_status* st,
                        const float* pre_scale) {
    // 9..64 rows: pre-quantized codes only, as one batch of 16, 32 or 64 (32 and
    // 64 for k <= 2048)
    const int mb = m > 32 ? 64 : m > 16 ? 32 : m > 8 ? 16 : m_bucket(m);
    if (!(m >= 1 && m <= (pre_scale ? 64 : 8) && k > 0 && k % 16 == 0 && (k + 1023) / 1024 <= 9 &&
          (mb <= 16 || k <= 2048) &&
          static_cast<int64_t>(mb) * k <= kDecMaxCodes &&
          aligned(w, 16) && aligned(x, 16) && n <= kMaxIndex))
        return false;
    const int mi = static_cast<int>(m), ni = static_cast<int>(n), ki = static_cast<int>(k);
    const int T = (ki / 16 + 63) / 64;
    // The forms nq_linear_w8a8 reaches (the others are not compiled): in-kernel
    // quant at m = 2..4 with k <= 4096 and m = 5..8 with k <= 1024 (m = 1 takes
    // the fused-quant GEMV); over codes at m = 5..8 with k <= 2048 or k >= 8192,
    // and m = 9..64 with k <= 2048.
    const int tb = T <= 2 ? 2 : T <= 4 ? 4 : 9;
    if (!(pre_scale ? (mb == 8 ? tb != 4 : mb >= 16 && tb == 2) : (mb == 2 || mb == 4) ? tb <= 4 : mb == 8 && tb == 2))
        return false;
    const size_t lds = static_cast<size_t>(mb) * ki;
    int dev = 0, cus = 256;
    if (hipGetDevice(&dev) == hipSuccess) (void)hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
    *st = NQ_OK;
    auto go = [&](auto mtag, auto rtag, auto ttag, auto* xp, auto* yp) {
        constexpr int M = decltype(mtag)::value, R = decltype(rtag)::value, TT = decltype(ttag)::value;
        // Waves that share a row group, each with M / S activation rows: 8 rows per
        // wave from 16 (n = 256, k = 1536: m = 16 6.64 -> 6.25 us, m = 64 10.76 ->
        // 7.46); 4 at m = 8 with single-row groups (k/v 6.07 -> 5.91; with 2-row
        // groups, n = 4864, k = 896, it lost 7.07 -> 7.24) and on long K (n = 1536,
        // k = 8960: 11.25 -> 11.07 with the act quant; 2 rows per wave 11.85).
        constexpr int S = M >= 16 ? M / 8 : M == 8 && (R == 1 || TT > 2) ? 2 : 1;
        using XT = std::remove_const_t<std::remove_pointer_t<decltype(xp)>>;
        using YT = std::remove_pointer_t<decltype(yp)>;
        const int groups = (ni + R - 1) / R;
        const unsigned grid = static_cast<unsigned>(std::max(1, std::min(cus, groups)));
        constexpr bool kPre = M == 8 ? TT != 4 : M >= 16 && TT == 2;
        constexpr bool kFused = (M == 2 || M == 4) ? TT <= 4 : M == 8 && TT == 2;
        if (pre_scale) {
            if constexpr (kPre) {
                auto* fn = w8a8_decode_kernel<M, R, TT, int8_t, YT, true, S>;
                if ((*st = set_dynamic_lds(reinterpret_cast<const void*>(fn), lds, "w8a8_decode"))) return;
                fn<<<grid, kDecThreads, lds, s>>>(static_cast<const int8_t*>(x), w, ws, bias, yp, mi, ni, ki, pre_scale);
            }
        } else if constexpr (kFused) {
            auto* fn = w8a8_decode_kernel<M, R, TT, XT, YT>;
            if ((*st = set_dynamic_lds(reinterpret_cast<const void*>(fn), lds, "w8a8_decode"))) return;
            fn<<<grid, kDecThreads, lds, s>>>(xp, w, ws, bias, yp, mi, ni, ki, nullptr);
        }
    };
    // Passes padded up to 2, 4 or 9 (a masked extra pass re-loads the last
    // chunk). R rows per group: the m code chunks read from LDS per pass serve R
    // rows; long K keeps R <= 2 for registers, and short-K weights with fewer
    // rows than 16 per CU take single-row groups, so that most of a CU's 16 waves
    // stream (m = 8, n = k = 1536 with codes: 7.06 -> 6.49 us; n = 2048: 7.22 ->
    // 6.61; from 4 per CU; 48 per CU lost at n = 4864 and 8960).
    const bool few = n < 16 * static_cast<int64_t>(cus);
    auto with_t = [&](auto mtag, auto* xp, auto* yp) {
        constexpr int M = decltype(mtag)::value;
        // short K: 2 rows from m = 2 (m = 8 over codes, n = 4864, k = 896: 7.59
        // -> 7.19 us with 2 rows against 4; 1 row at m = 2..4 lost 0.2-0.5 us)
        constexpr int RS = M == 1 || M >= 32 ? 1 : 2;
        constexpr int RL = M == 16 ? 1 : RS < 2 ? RS : 2;                // long K
        using One = std::integral_constant<int, 1>;
        if constexpr (M >= 16) {  // k <= 2048 (T = 2); one row per group (n <= 2048 is "few" at m <= 16)
            go(mtag, One{}, std::integral_constant<int, 2>{}, xp, yp);
        } else if (T <= 2) {
            if (few) go(mtag, One{}, std::integral_constant<int, 2>{}, xp, yp);
            else go(mtag, std::integral_constant<int, RS>{}, std::integral_constant<int, 2>{}, xp, yp);
        } else if (T <= 4) {
            go(mtag, std::integral_constant<int, RL>{}, std::integral_constant<int, 4>{}, xp, yp);
        } else {
            go(mtag, std::integral_constant<int, RL>{}, std::integral_constant<int, 9>{}, xp, yp);
        }
    };
    auto with_m = [&](auto* xp, auto* yp) {
        switch (mb) {
            case 2: with_t(std::integral_constant<int, 2>{}, xp, yp); break;
            case 4: with_t(std::integral_constant<int, 4>{}, xp, yp); break;
            case 8: with_t(std::integral_constant<int, 8>{}, xp, yp); break;
            case 16: with_t(std::integral_constant<int, 16>{}, xp, yp); break;
            case 32: with_t(std::integral_constant<int, 32>{}, xp, yp); break;
            default: with_t(std::integral_constant<int, 64>{}, xp, yp); break;
        }
    };
    auto with_y = [&](auto* xp) {
        if (ydt == NQ_F32) with_m(xp, static_cast<float*>(y));
        else with_m(xp, static_cast<_Float16*>(y));
    };
    // (with pre_scale the activation type only picks an instantiation; x is int8)
    if (xdt == NQ_F32 && !pre_scale) with_y(static_cast<const float*>(x));
    else with_y(static_cast<const _Float16*>(x));
    if (*st == NQ_OK) *st = launch_status("w8a8_decode_kernel");
    return true;
}

// Fused act-quant + GEMV for m = 1 (every workgroup quantizes all m rows: at
// m = 2 and long K the separate act quant plus the GEMV measured faster, k =
// 8960, n = 1536: 10.9 vs 8.7 us; k = 4864, n = 896: 7.4 vs 6.6). Returns
// false (nothing launched) when the shape is outside its fast path; the caller
// then quantizes and runs the GEMV.
bool gemv_w8a8_fused_launch(const void* x, nq_dtype xdt, const int8_t* w, const float* ws,
                            const float* bias, void* y, nq_dtype ydt, int64_t m, int64_t n,
                            int64_t k, hipStream_t s, nq_status* st) {
    if (!(m == 1 && k > 0 && k % 16 == 0 && k / 16 <= kMaxGemvThreads && aligned(w, 16) && aligned(x, 16)))
        return false;
    const int mi = static_cast<int>(m), ni = static_cast<int>(n), ki = static_cast<int>(k);
    const int threads = ((ki / 16 + kWave - 1) / kWave) * kWave;
    // 8 weight rows per workgroup from 2048 rows or k = 4096 (every workgroup
    // quantizes the whole activation row, so more rows share that work; us, 4 ->
    // 8 rows: n = 1536, k = 8960 7.86 -> 6.43; n = 17920, k = 1536 8.04 -> 7.29;
    // n = 4096, k = 4096 6.65 -> 5.96; n = 4864, k = 896 3.61 -> 3.12; the LM
    // head, n = 151936, 50.6 -> 38.0; n = 256 lost 3.04 -> 4.01 and n = k = 1536
    // was even; 16 rows no better than 8), else 4.
    const bool big = n >= 2048 || k >= 4096;
    auto go = [&](auto mtag, auto* xp, auto* yp) {
        constexpr int M = decltype(mtag)::value;
        using XT = std::remove_const_t<std::remove_pointer_t<decltype(xp)>>;
        using YT = std::remove_pointer_t<decltype(yp)>;
        auto run = [&](auto rtag) {
            constexpr int R = decltype(rtag)::value;
            const unsigned grid = static_cast<unsigned>((n + R - 1) / R);
            if (threads == kWave)
                gemv_w8a8_fused_kernel<R, M, XT, YT, true><<<grid, threads, 0, s>>>(xp, w, ws, bias, yp, mi, ni, ki);
            else
                gemv_w8a8_fused_kernel<R, M, XT, YT><<<grid, threads, 0, s>>>(xp, w, ws, bias, yp, mi, ni, ki);
        };
        if (big) run(std::integral_constant<int, 8>{});
        else run(std::integral_constant<int, rows_for<M>()>{});
    };
    auto with_y = [&](auto* xp) {
        if (ydt == NQ_F32) go(std::integral_constant<int, 1>{}, xp, static_cast<float*>(y));
        else go(std::integral_constant<int, 1>{}, xp, static_cast<_Float16*>(y));
    };
    if (xdt == NQ_F32) with_y(static_cast<const float*>(x));
    else with_y(static_cast<const _Float16*>(x));
    *st = launch_status("gemv_w8a8_fused_kernel");
    return true;
}

namespace {
// A workspace passed to the *_ws linears must hold the split-K planes the
// shape plans (NULL / 0 bytes only where it plans none).
nq_status check_wq_workspace(const void* ws, size_t bytes, int64_t m, int64_t n, int64_t k, const char* who) {
    const size_t need = m > 0 && n > 0 ? wq_workspace_bytes(m, n, k) : 0;
    NQ_REQUIRE(bytes >= need && (need == 0 || ws), NQ_BAD_ARG, "%s: workspace of %zu bytes, %zu needed", who, bytes, need);
    NQ_REQUIRE(aligned(ws, 256), NQ_BAD_ALIGN, "%s: workspace must be 256-byte aligned", who);
    return NQ_OK;
}

// path: NQ_PATH_AUTO (the shape rules below), NQ_PATH_GEMV (GEMV slices of 8
// rows at any m), NQ_PATH_MFMA (the fp16 MFMA GEMM at any m; NQ_BAD_ARG where
// its operand contract does not hold), NQ_PATH_GENERIC (the bounds-checked
// wave-per-row kernel).
nq_status linear_q8_impl(const void* x, nq_dtype x_dtype, const int8_t* q, const float* w_scale, const float* bias,
                         void* y, nq_dtype y_dtype, int64_t m, int64_t n, int64_t k, void* ws, size_t ws_bytes,
                         void* stream, int path = NQ_PATH_AUTO) {
    NQ_REQUIRE(dtype_ok(x_dtype) && dtype_ok(y_dtype), NQ_BAD_ARG, "linear_q8: unknown dtype");
    NQ_REQUIRE(path >= NQ_PATH_AUTO && path <= NQ_PATH_GENERIC, NQ_BAD_ARG, "linear_q8: unknown path %d", path);
    if (m == 0 || n == 0) return NQ_OK;
    NQ_REQUIRE(w_scale, NQ_BAD_ARG, "linear_q8: null w_scale");
    NQ_REQUIRE(aligned(x, dtype_size(x_dtype)) && aligned(y, dtype_size(y_dtype)) &&
                   aligned(w_scale, 4) && aligned(bias, 4),
               NQ_BAD_ALIGN, "linear_q8: misaligned pointer");
    hipStream_t s = as_stream(stream);
    const int ni = static_cast<int>(n), ki = static_cast<int>(k);
    // Batched activations: the fp16 MFMA GEMM when the shape rule in wq_gemm_ok
    // picks it, else GEMV slices of 8 rows.
    const bool mfma = path == NQ_PATH_MFMA;
    NQ_REQUIRE(!mfma || wq_gemm_ok(false, x, dtype_size(x_dtype), q, m, n, k, 32, ws != nullptr, true), NQ_BAD_ARG,
               "linear_q8: the MFMA path needs k %% 32 == 0 and 16-byte aligned x and q (m=%lld n=%lld k=%lld)",
               (long long)m, (long long)n, (long long)k);
    if (mfma || (path == NQ_PATH_AUTO && wq_gemm_ok(false, x, dtype_size(x_dtype), q, m, n, k, 32, ws != nullptr))) {
        const uint8_t* w = reinterpret_cast<const uint8_t*>(q);
        if (x_dtype == NQ_F32 && y_dtype == NQ_F32)
            return wq_gemm<false>(static_cast<const float*>(x), w, w_scale, bias, static_cast<float*>(y), m, n, k, 32, ws, ws_bytes, s);
        if (x_dtype == NQ_F32)
            return wq_gemm<false>(static_cast<const float*>(x), w, w_scale, bias, static_cast<_Float16*>(y), m, n, k, 32, ws, ws_bytes, s);
        if (y_dtype == NQ_F32)
            return wq_gemm<false>(static_cast<const _Float16*>(x), w, w_scale, bias, static_cast<float*>(y), m, n, k, 32, ws, ws_bytes, s);
        return wq_gemm<false>(static_cast<const _Float16*>(x), w, w_scale, bias, static_cast<_Float16*>(y), m, n, k, 32, ws, ws_bytes, s);
    }
    const bool fast = path != NQ_PATH_GENERIC && k % 16 == 0 && k > 0 && k / 16 <= kMaxGemvThreads &&
                      aligned(q, 16) && aligned(x, 16);
    const bool long_k = path != NQ_PATH_GENERIC && k % 16 == 0 && k / 16 > kMaxGemvThreads && aligned(q, 16) &&
                        aligned(x, 16);
    // Otherwise x rows beyond 8 run in slices of 8 (each slice re-streams the weight).
    for (int64_t r0 = 0; r0 < m; r0 += 8) {
        const int mi = static_cast<int>(m - r0 < 8 ? m - r0 : 8);
        const size_t xo = static_cast<size_t>(r0) * k, yo = static_cast<size_t>(r0) * n;
        if (long_k) {
            if (x_dtype == NQ_F32 && y_dtype == NQ_F32)
                dispatch_q8_longk(static_cast<const float*>(x) + xo, q, w_scale, bias, static_cast<float*>(y) + yo, mi, ni, ki, s);
            else if (x_dtype == NQ_F32)
                dispatch_q8_longk(static_cast<const float*>(x) + xo, q, w_scale, bias, static_cast<_Float16*>(y) + yo, mi, ni, ki, s);
            else if (y_dtype == NQ_F32)
                dispatch_q8_longk(static_cast<const _Float16*>(x) + xo, q, w_scale, bias, static_cast<float*>(y) + yo, mi, ni, ki, s);
            else
                dispatch_q8_longk(static_cast<const _Float16*>(x) + xo, q, w_scale, bias, static_cast<_Float16*>(y) + yo, mi, ni, ki, s);
        } else if (fast) {
            if (x_dtype == NQ_F32 && y_dtype == NQ_F32)
                dispatch_q8(static_cast<const float*>(x) + xo, q, w_scale, bias, static_cast<float*>(y) + yo, mi, ni, ki, s);
            else if (x_dtype == NQ_F32)
                dispatch_q8(static_cast<const float*>(x) + xo, q, w_scale, bias, static_cast<_Float16*>(y) + yo, mi, ni, ki, s);
            else if (y_dtype == NQ_F32)
                dispatch_q8(static_cast<const _Float16*>(x) + xo, q, w_scale, bias, static_cast<float*>(y) + yo, mi, ni, ki, s);
            else
                dispatch_q8(static_cast<const _Float16*>(x) + xo, q, w_scale, bias, static_cast<_Float16*>(y) + yo, mi, ni, ki, s);
        } else {
            const unsigned grid = static_cast<unsigned>((n + 3) / 4);
            if (x_dtype == NQ_F32 && y_dtype == NQ_F32)
                gemv_q8_generic_kernel<<<grid, 256, 0, s>>>(static_cast<const float*>(x) + xo, q, w_scale, bias, static_cast<float*>(y) + yo, mi, ni, ki);
            else if (x_dtype == NQ_F32)
                gemv_q8_generic_kernel<<<grid, 256, 0, s>>>(static_cast<const float*>(x) + xo, q, w_scale, bias, static_cast<_Float16*>(y) + yo, mi, ni, ki);
            else if (y_dtype == NQ_F32)
                gemv_q8_generic_kernel<<<grid, 256, 0, s>>>(static_cast<const _Float16*>(x) + xo, q, w_scale, bias, static_cast<float*>(y) + yo, mi, ni, ki);
            else
                gemv_q8_generic_kernel<<<grid, 256, 0, s>>>(static_cast<const _Float16*>(x) + xo, q, w_scale, bias, static_cast<_Float16*>(y) + yo, mi, ni, ki);
        }
        if (nq_status st = launch_status("gemv_q8_kernel")) return st;
    }
    return NQ_OK;
}

nq_status linear_q4g_impl(const void* x, nq_dtype x_dtype, const uint8_t* q, const void* scale,
                          nq_dtype scale_dtype, int64_t group, const float* bias, void* y, nq_dtype y_dtype,
                          int64_t m, int64_t n, int64_t k, void* ws, size_t ws_bytes, void* stream,
                          int path = NQ_PATH_AUTO) {
    NQ_REQUIRE(group > 0 && group <= kMaxIndex, NQ_BAD_SHAPE, "linear_q4g: group must be positive");
    NQ_REQUIRE(path >= NQ_PATH_AUTO && path <= NQ_PATH_GENERIC, NQ_BAD_ARG, "linear_q4g: unknown path %d", path);
    NQ_REQUIRE(dtype_ok(x_dtype) && dtype_ok(y_dtype) && dtype_ok(scale_dtype), NQ_BAD_ARG,
               "linear_q4g: unknown dtype");
    if (m == 0 || n == 0) return NQ_OK;
    NQ_REQUIRE(k == 0 || scale, NQ_BAD_ARG, "linear_q4g: null scale");
    NQ_REQUIRE(aligned(x, dtype_size(x_dtype)) && aligned(y, dtype_size(y_dtype)) &&
                   aligned(scale, dtype_size(scale_dtype)) && aligned(bias, 4),
               NQ_BAD_ALIGN, "linear_q4g: misaligned pointer");
    hipStream_t s = as_stream(stream);
    const int ni = static_cast<int>(n), ki = static_cast<int>(k), gi = static_cast<int>(group);
    // Batched activations: the fp16 MFMA GEMM when the shape rule in wq_gemm_ok
    // picks it, else GEMV slices of 8 rows.
    const bool mfma = path == NQ_PATH_MFMA;
    NQ_REQUIRE(!mfma || wq_gemm_ok(true, x, dtype_size(x_dtype), q, m, n, k, group, ws != nullptr, true), NQ_BAD_ARG,
               "linear_q4g: the MFMA path needs k %% 32 == 0, group = 32 * 2^j and 16-byte aligned x and q "
               "(m=%lld n=%lld k=%lld group=%lld)", (long long)m, (long long)n, (long long)k, (long long)group);
    if (mfma || (path == NQ_PATH_AUTO && wq_gemm_ok(true, x, dtype_size(x_dtype), q, m, n, k, group, ws != nullptr))) {
        auto go = [&](auto* xp, auto* yp) {
            if (scale_dtype == NQ_F32)
                return wq_gemm<true>(xp, q, static_cast<const float*>(scale), bias, yp, m, n, k, group, ws, ws_bytes, s);
            return wq_gemm<true>(xp, q, static_cast<const _Float16*>(scale), bias, yp, m, n, k, group, ws, ws_bytes, s);
        };
        auto with_y = [&](auto* xp) {
            if (y_dtype == NQ_F32) return go(xp, static_cast<float*>(y));
            return go(xp, static_cast<_Float16*>(y));
        };
        if (x_dtype == NQ_F32) return with_y(static_cast<const float*>(x));
        return with_y(static_cast<const _Float16*>(x));
    }
    const bool fast = path != NQ_PATH_GENERIC && k % 32 == 0 && k > 0 && group % 32 == 0 &&
                      k / 32 <= kMaxGemvThreads && aligned(q, 16) && aligned(x, 16);
    const bool long_k = path != NQ_PATH_GENERIC && k % 32 == 0 && group % 32 == 0 && k / 32 > kMaxGemvThreads &&
                        aligned(q, 16) && aligned(x, 16);
    for (int64_t r0 = 0; r0 < m; r0 += 8) {
        const int mi = static_cast<int>(m - r0 < 8 ? m - r0 : 8);
        const size_t xo = static_cast<size_t>(r0) * k, yo = static_cast<size_t>(r0) * n;
        auto run = [&](auto* xp, auto* yp, auto* sp) {
            if (long_k)
                dispatch_q4g_longk(xp + xo, q, sp, bias, yp + yo, mi, ni, ki, gi, s);
            else if (fast)
                dispatch_q4g(xp + xo, q, sp, bias, yp + yo, mi, ni, ki, gi, s);
            else
                gemv_q4g_generic_kernel<<<static_cast<unsigned>((n + 3) / 4), 256, 0, s>>>(
                    xp + xo, q, sp, bias, yp + yo, mi, ni, ki, gi);
        };
        auto with_scale = [&](auto* xp, auto* yp) {
            if (scale_dtype == NQ_F32) run(xp, yp, static_cast<const float*>(scale));
            else run(xp, yp, static_cast<const _Float16*>(scale));
        };
        auto with_y = [&](auto* xp) {
            if (y_dtype == NQ_F32) with_scale(xp, static_cast<float*>(y));
            else with_scale(xp, static_cast<_Float16*>(y));
        };
        if (x_dtype == NQ_F32) with_y(static_cast<const float*>(x));
        else with_y(static_cast<const _Float16*>(x));
        if (nq_status st = launch_status("gemv_q4g_kernel")) return st;
    }
    return NQ_OK;
}
}  // namespace
}  // namespace nq

using namespace nq;

extern "C" nq_status nq_linear_q8(const void* x, nq_dtype x_dtype, const int8_t* q, const float* w_scale,
                                  const float* bias, void* y, nq_dtype y_dtype, int64_t m, int64_t n, int64_t k,
                                  void* stream) {
    if (nq_status st = check_linear(x, q, y, m, n, k, "linear_q8")) return st;
    return linear_q8_impl(x, x_dtype, q, w_scale, bias, y, y_dtype, m, n, k, nullptr, 0, stream);
}

extern "C" nq_status nq_linear_q4g(const void* x, nq_dtype x_dtype, const uint8_t* q, const void* scale,
                                   nq_dtype scale_dtype, int64_t group, const float* bias, void* y,
                                   nq_dtype y_dtype, int64_t m, int64_t n, int64_t k, void* stream) {
    if (nq_status st = check_linear(x, q, y, m, n, k, "linear_q4g")) return st;
    return linear_q4g_impl(x, x_dtype, q, scale, scale_dtype, group, bias, y, y_dtype, m, n, k, nullptr, 0, stream);
}

extern "C" size_t nq_linear_wq_workspace_size(int64_t m, int64_t n, int64_t k) {
    return m > 0 && n > 0 && k > 0 && k <= kMaxIndex && n <= kMaxIndex ? wq_workspace_bytes(m, n, k) : 0;
}

extern "C" nq_status nq_linear_q8_ws(const void* x, nq_dtype x_dtype, const int8_t* q, const float* w_scale,
                                     const float* bias, void* y, nq_dtype y_dtype, int64_t m, int64_t n, int64_t k,
                                     void* workspace, size_t workspace_bytes, void* stream) {
    if (nq_status st = check_linear(x, q, y, m, n, k, "linear_q8_ws")) return st;
    if (nq_status st = check_wq_workspace(workspace, workspace_bytes, m, n, k, "linear_q8_ws")) return st;
    return linear_q8_impl(x, x_dtype, q, w_scale, bias, y, y_dtype, m, n, k, workspace, workspace_bytes, stream);
}

extern "C" nq_status nq_linear_q4g_ws(const void* x, nq_dtype x_dtype, const uint8_t* q, const void* scale,
                                      nq_dtype scale_dtype, int64_t group, const float* bias, void* y,
                                      nq_dtype y_dtype, int64_t m, int64_t n, int64_t k, void* workspace,
                                      size_t workspace_bytes, void* stream) {
    if (nq_status st = check_linear(x, q, y, m, n, k, "linear_q4g_ws")) return st;
    if (nq_status st = check_wq_workspace(workspace, workspace_bytes, m, n, k, "linear_q4g_ws")) return st;
    return linear_q4g_impl(x, x_dtype, q, scale, scale_dtype, group, bias, y, y_dtype, m, n, k, workspace,
                           workspace_bytes, stream);
}

extern "C" nq_status nq_linear_q8_ex(const void* x, nq_dtype x_dtype, const int8_t* q, const float* w_scale,
                                     const float* bias, void* y, nq_dtype y_dtype, int64_t m, int64_t n, int64_t k,
                                     void* workspace, size_t workspace_bytes, int path, void* stream) {
    if (nq_status st = check_linear(x, q, y, m, n, k, "linear_q8_ex")) return st;
    if (nq_status st = check_wq_workspace(workspace, workspace_bytes, m, n, k, "linear_q8_ex")) return st;
    return linear_q8_impl(x, x_dtype, q, w_scale, bias, y, y_dtype, m, n, k, workspace, workspace_bytes, stream,
                          path);
}

extern "C" nq_status nq_linear_q4g_ex(const void* x, nq_dtype x_dtype, const uint8_t* q, const void* scale,
                                      nq_dtype scale_dtype, int64_t group, const float* bias, void* y,
                                      nq_dtype y_dtype, int64_t m, int64_t n, int64_t k, void* workspace,
                                      size_t workspace_bytes, int path, void* stream) {
    if (nq_status st = check_linear(x, q, y, m, n, k, "linear_q4g_ex")) return st;
    if (nq_status st = check_wq_workspace(workspace, workspace_bytes, m, n, k, "linear_q4g_ex")) return st;
    return linear_q4g_impl(x, x_dtype, q, scale, scale_dtype, group, bias, y, y_dtype, m, n, k, workspace,
                           workspace_bytes, stream, path);
}

// ---- LM head with fused greedy argmax ----------------------------------------------------
namespace nq {
namespace {
constexpr int kArgSeg = 4096;  // logits per partial on the unfused path
// Fused path: the q8 GEMV's fast kernel (k % 16 == 0, k / 16 within one
// workgroup, 16-byte aligned operands) writes one partial per workgroup.
bool lm_head_fused_ok(const void* x, const int8_t* q, int64_t k) {
    return k > 0 && k % 16 == 0 && k / 16 <= kMaxGemvThreads && aligned(q, 16) && aligned(x, 16);
}
size_t lm_head_ws(int64_t m, int64_t n, int64_t k, bool fused) {
    // one partial per workgroup of at least 2 rows (rows_for), per activation row of a slice
    if (fused) return kArgCtlBytes + round_up(static_cast<size_t>(std::min<int64_t>(m, 8)) * ((n + 1) / 2) * sizeof(ArgPart), 256);
    return round_up(static_cast<size_t>(m) * n * 4, 256) +
           round_up(static_cast<size_t>(m) * ((n + kArgSeg - 1) / kArgSeg) * sizeof(ArgPart), 256);
}
}  // namespace
}  // namespace nq

extern "C" size_t nq_lm_head_argmax_q8_workspace_size(int64_t m, int64_t n, int64_t k) {
    if (m <= 0 || n <= 0 || k < 0) return 0;
    return std::max(lm_head_ws(m, n, k, true), lm_head_ws(m, n, k, false));
}

extern "C" nq_status nq_lm_head_argmax_q8(const void* x, nq_dtype x_dtype, const int8_t* q, const float* w_scale,
                                          const float* bias, int64_t* ids, int64_t m, int64_t n, int64_t k,
                                          void* workspace, size_t workspace_bytes, void* stream) {
    NQ_REQUIRE(m >= 0 && n >= 0 && k >= 0 && m <= kMaxIndex && n < kArgNone && k <= kMaxIndex, NQ_BAD_SHAPE,
               "lm_head_argmax_q8: bad shape m=%lld n=%lld k=%lld", (long long)m, (long long)n, (long long)k);
    NQ_REQUIRE(dtype_ok(x_dtype), NQ_BAD_ARG, "lm_head_argmax_q8: unknown dtype");
    if (m == 0) return NQ_OK;
    NQ_REQUIRE(n > 0, NQ_BAD_SHAPE, "lm_head_argmax_q8: empty vocabulary");
    NQ_REQUIRE(ids && w_scale && (k == 0 || (x && q)), NQ_BAD_ARG, "lm_head_argmax_q8: null pointer");
    NQ_REQUIRE(aligned(ids, 8) && aligned(w_scale, 4) && aligned(bias, 4) && aligned(x, dtype_size(x_dtype)),
               NQ_BAD_ALIGN, "lm_head_argmax_q8: misaligned pointer");
    const bool fused = lm_head_fused_ok(x, q, k);
    const size_t need = lm_head_ws(m, n, k, fused);
    NQ_REQUIRE(workspace && workspace_bytes >= need, NQ_BAD_ARG,
               "lm_head_argmax_q8: workspace of %zu bytes required, %zu given", need, workspace_bytes);
    NQ_REQUIRE(aligned(workspace, 256), NQ_BAD_ALIGN, "lm_head_argmax_q8: workspace must be 256-byte aligned");
    hipStream_t s = as_stream(stream);
    const int ni = static_cast<int>(n), ki = static_cast<int>(k);
    if (!fused) {
        // Logits through nq_linear_q8 (fp32), then a two-pass argmax over them.
        float* logits = static_cast<float*>(workspace);
        ArgPart* part = reinterpret_cast<ArgPart*>(static_cast<char*>(workspace) + round_up(static_cast<size_t>(m) * n * 4, 256));
        if (nq_status st = nq_linear_q8(x, x_dtype, q, w_scale, bias, logits, NQ_F32, m, n, k, stream)) return st;
        const int nseg = (ni + kArgSeg - 1) / kArgSeg;
        argmax_logits_kernel<<<dim3(static_cast<unsigned>(nseg), static_cast<unsigned>(m)), 256, 0, s>>>(logits, ni, kArgSeg, part);
        argmax_final_kernel<<<static_cast<unsigned>(m), 1024, 0, s>>>(part, nseg, ids);
        return launch_status("lm_head_argmax_q8");
    }
    ArgCtl* ctl = static_cast<ArgCtl*>(workspace);
    ArgPart* part = reinterpret_cast<ArgPart*>(static_cast<char*>(workspace) + kArgCtlBytes);
    // Activation rows in slices of 8 (the GEMV's batch), each with the kernel
    // and row grouping nq_linear_q8 uses for that slice, so the fused logits
    // equal nq_linear_q8's fp32 output bit for bit.
    for (int64_t r0 = 0; r0 < m; r0 += 8) {
        const int mi = static_cast<int>(std::min<int64_t>(8, m - r0));
        int nwg = 0;
        auto go = [&](auto* xp) {
            using XT = std::remove_const_t<std::remove_pointer_t<decltype(xp)>>;
            const XT* xs = xp + static_cast<size_t>(r0) * k;
            float* none = nullptr;
            switch (m_bucket(mi)) {
                case 1: nwg = (ni + q8_rows<1, XT>(ni, ki) - 1) / q8_rows<1, XT>(ni, ki); launch_q8<1, true>(xs, q, w_scale, bias, none, mi, ni, ki, s, part, ctl); break;
                case 2: nwg = (ni + q8_rows<2, XT>(ni, ki) - 1) / q8_rows<2, XT>(ni, ki); launch_q8<2, true>(xs, q, w_scale, bias, none, mi, ni, ki, s, part, ctl); break;
                case 4: nwg = (ni + q8_rows<4, XT>(ni, ki) - 1) / q8_rows<4, XT>(ni, ki); launch_q8<4, true>(xs, q, w_scale, bias, none, mi, ni, ki, s, part, ctl); break;
                default: nwg = (ni + q8_rows<8, XT>(ni, ki) - 1) / q8_rows<8, XT>(ni, ki); launch_q8<8, true>(xs, q, w_scale, bias, none, mi, ni, ki, s, part, ctl); break;
            }
        };
        if (x_dtype == NQ_F32) go(static_cast<const float*>(x));
        else go(static_cast<const _Float16*>(x));
        const unsigned nfin = static_cast<unsigned>((nwg + kArgFinalT * kArgFinalU - 1) / (kArgFinalT * kArgFinalU));
        argmax_final_multi_kernel<kArgFinalT, kArgFinalU><<<dim3(nfin, static_cast<unsigned>(mi)), kArgFinalT, 0, s>>>(
            part, nwg, ctl, ids + r0);
        if (nq_status st = launch_status("lm_head_argmax_q8")) return st;
    }
    return NQ_OK;
}
