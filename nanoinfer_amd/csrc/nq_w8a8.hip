// W8A8 GEMM on the gfx950 int8 matrix cores, plus the W8A8 entry points.
//
// xq [m, k] int8 (per-row dynamic quant) x wq [n, k] int8 (per-row weight
// quant) -> exact int32 accumulators -> y = float(acc)*a_scale*w_scale + b.
// Both operands are K-contiguous, which is exactly the per-lane layout of
// v_mfma_i32_16x16x64_i8: lane l supplies 16 consecutive K bytes of A row
// (l % 16) and of B column (l % 16) for K slice (l / 16); the 16x16 int32
// result lands as rows 4*(l/16)+v, column l%16, v = 0..3.
//
// Two MFMA kernels: a skinny one for batched decode (m <= 64: operands
// loaded straight into the MFMA lane layout, K steps interleaved over waves);
// and the wide-tile kernel (rounds of up to 256 tiles of 64 x 32 .. 256 x 320,
// LDS-DMA ring of 128-byte K slabs), which takes the shapes with m > 64 and
// decode batches with tall weights. When a launch would have too few
// workgroups, they split K: each K range writes its int32 partial tile to its
// own workspace plane and a reduction launch sums the planes in a fixed order
// (integer addition is exact, so the result is bit-identical to a single pass)
// and applies the epilogue.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <mutex>
#include <type_traits>

#include "nq_device.hpp"
#include "nq_internal.hpp"

namespace nq {

nq_status gemv_w8a8_launch(const int8_t* xq, const float* as, const int8_t* w, const float* ws,
                           const float* bias, void* y, nq_dtype ydt, int32_t* acc_out, int64_t m,
                           int64_t n, int64_t k, bool generic, hipStream_t s);

namespace {

constexpr int kBK = 64;         // K bytes per MFMA step / LDS slab

enum class Out { Y, ACC, PARTIAL };

template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// ---- wide-tile W8A8 GEMM: one (64*WM) x (32*FN) tile per CU ------------------------------
// For shapes whose 256 x 256..320 (or 128 x 256..320) tiles number at most one
// per CU (m = 2048, n = 8960: 8 x 32 tiles of 256 x 288; m = 512, n = 17920:
// 4 x 63 tiles of 128 x 288), a single round of tiles beats two rounds of
// smaller tiles: every output tile costs one pass over its A rows and B rows,
// and a second round would leave most CUs idle. WM x 2 waves (WM = 4 or 2), each
// 64 x 16*FN outputs (4 x FN fragments, 4*FN int32 accumulator registers). K
// advances in 128-byte slabs (two MFMA K steps) through an LDS ring of as many
// slots D as fit (2 for 256 x 288 tiles, 3 for 128 x 288, up to 8 for small
// tiles) filled by LDS-DMA; the request for slab kt + D - 1 goes out right after the
// barrier that frees its slot. A 1 KB DMA request covers 8 rows x 128 bytes,
// i.e. whole 128-byte cache lines: with 64-byte slabs (16 rows x 64 bytes per
// request, a 4-slot ring) every request touched twice as many lines and the
// loads of the same tile took longer even with more slabs in flight. Chunk c
// of row r sits in slot c ^ ((r >> 1) & 7) of its 128-byte LDS row, so the
// 16 rows of a fragment read hit distinct banks. All fragment reads of a K
// step are issued before its first MFMA (a scheduling barrier keeps the
// compiler from sinking them next to their uses, which left LDS latency
// exposed). The block of DMA requests does not split evenly over the waves;
// the spare requests read zeros into a 1 KB sink so every wave counts the same
// number per slab. When k % 128 == 64 the last slab's upper half reads zeros.
// fp16 results go through LDS in two halves of the tile's rows and leave as
// 16-byte row chunks with non-temporal stores (a one-round grid writes its
// whole output at the end, which no later work overlaps).
template <int WM, int FN, int FM, int WN = 2>
struct WideShape {
    static constexpr int kWM = WM, kWN = WN, kWaves = WM * WN, kRow = 128;
    static constexpr int kBM = kWM * FM * 16, kBN = kWN * FN * 16;
    static constexpr int kXB = kBM / 8, kNB = kXB + kBN / 8, kQ = (kNB + kWaves - 1) / kWaves;
    static constexpr int kSlab = (kBM + kBN) * kRow;
    // Ring slots: when three or more fit in half the LDS, as many as let two
    // workgroups share a CU (64 x 64 tiles: 4, 64 x 128: 3; with 8 or 6 slots one
    // workgroup per CU left its 8 waves waiting on memory: config 4 q|k|v 8.09 ->
    // 7.23 us, o 7.93 -> 7.13, m = 64 gate/up 11.5 -> 10.8, m = 128 n = 8960 13.0
    // -> 12.6; 3 slots of 64 x 64 (three workgroups) lost: down 23.5 -> 28.0);
    // otherwise as many as 160 KB holds beside the sink (at most 8).
    static constexpr int kEpsBytes = (kBM + 2 * ((kBN + 63) / 64) * 64) * 4;
    static constexpr int kDTwo = (80 * 1024 - 1024 - kEpsBytes) / kSlab;
    static constexpr int kD = kDTwo >= 3 ? std::min(8, kDTwo) : std::min(8, (160 * 1024 - 1024 - kEpsBytes) / kSlab);
    static_assert(kD >= 2, "two slabs must fit");
    static constexpr int kSink = kD * kSlab;  // 1 KB
    // fp16 staging rows of the epilogue: 16 bytes of padding make the stride an
    // odd multiple of 16, so the 16 rows of a fragment store hit distinct banks
    // (an unpadded 576-byte stride put 4 rows on each bank group).
    static constexpr int kStg = kBN * 2 + 16;
    // The tile's activation row scales, weight scales and bias (fp16 epilogue
    // only): fetched into LDS at the start, after the ring and the staging rows;
    // loaded in the epilogue instead, their latency sat between the last MFMA
    // and the first store (config 5a 34.2 -> 31.7 us).
    static constexpr size_t kEps = (std::max<size_t>(size_t(kSink) + 1024, size_t(kBM / 2) * kStg) + 15) / 16 * 16;
    static constexpr int kEpsReq = (kBM + 63) / 64 + 2 * ((kBN + 63) / 64);
    static constexpr size_t kLds = kEps + kEpsBytes;
    static_assert(kLds <= 160 * 1024, "LDS");
};

template <int WM, int FN, int FM, Out OUT, typename YT, int WN = 2>
__global__ __launch_bounds__(WM * WN * 64) void gemm_w8a8_wide_kernel(
    const int8_t* __restrict__ xq, const float* __restrict__ as, const int8_t* __restrict__ wq,
    const float* __restrict__ ws, const float* __restrict__ bias, YT* __restrict__ y,
    int32_t* __restrict__ acc_out, int m, int n, int k, int tiles_m, int tiles_n, int k_slabs) {
    using S = WideShape<WM, FN, FM, WN>;
    constexpr int NW = S::kWaves, Q = S::kQ, XB = S::kXB, NB = S::kNB, BM = S::kBM, BN = S::kBN, D = S::kD;
    extern __shared__ __attribute__((aligned(16))) int8_t lds[];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave / S::kWN, wn = wave % S::kWN;
    // Workgroup ids are dealt round-robin over the 8 XCDs: XCD x takes a
    // contiguous range of tiles (row tile fastest), so its tiles share A row
    // blocks and B column blocks in its L2.
    const int total = tiles_m * tiles_n;
    const int per = (total + 7) / 8, xcd = blockIdx.x % 8, idx = blockIdx.x / 8;
    const int full = total - 8 * (per - 1);  // XCDs [0, full) own `per` tiles, the rest per - 1
    const int lin = xcd < full ? xcd * per + idx : full * per + (xcd - full) * (per - 1) + idx;
    const int m0 = (lin % tiles_m) * BM, n0 = (lin / tiles_m) * BN;

    const __amdgpu_buffer_rsrc_t xrs = __builtin_amdgcn_make_buffer_rsrc(const_cast<int8_t*>(xq), 0, m * k, 0x00020000);
    const __amdgpu_buffer_rsrc_t wrs = __builtin_amdgcn_make_buffer_rsrc(const_cast<int8_t*>(wq), 0, n * k, 0x00020000);
    constexpr int kOob = 0x7FFFFFF0;
    // Request q of wave w moves 1 KB block b = q * NW + w of the slab: blocks
    // [0, XB) are 8 activation rows each, [XB, NB) 8 weight rows, the rest
    // spares. Lane i writes LDS bytes 16i..16i+15 of the block (row i/8,
    // slot i%8) and loads the chunk the swizzle puts there. vtail: the same
    // offsets with the upper half of the row (chunks 4..7) out of range.
    int voff[Q], vtail[Q], loff[Q];
#pragma unroll
    for (int q = 0; q < Q; ++q) {
        const int b = q * NW + wave;
        const bool real = b < NB, isx = b < XB;
        const int r = (isx ? b : b - XB) * 8 + (lane >> 3);
        const int c = (lane & 7) ^ ((r >> 1) & 7);
        const int grow = (isx ? m0 : n0) + r;
        voff[q] = real && grow < (isx ? m : n) ? grow * k + c * 16 : kOob;
        vtail[q] = c < 4 ? voff[q] : kOob;
        loff[q] = real ? b * 1024 : S::kSink;
    }
    // This workgroup's K range: slabs [s0, s1) (all of K unless the launch
    // splits K over gridDim.y; OUT == PARTIAL then stores the range's int32
    // tile into plane blockIdx.y).
    const int nslab = (k + S::kRow - 1) / S::kRow;
    const bool half_tail = (k % S::kRow) != 0;  // k % 64 == 0 by contract
    const int s0 = blockIdx.y * k_slabs, s1 = min(nslab, s0 + k_slabs), nk = s1 - s0;
    const unsigned lds_base = static_cast<unsigned>(reinterpret_cast<uintptr_t>(lds));
    auto issue = [&](int sl) {  // sl counts from s0
        const unsigned slot = static_cast<unsigned>(sl % D) * S::kSlab;
        const int g = s0 + sl;
        const int soff = g < s1 ? g * S::kRow : kOob;
        const bool tail = half_tail && g == nslab - 1;
#pragma unroll
        for (int q = 0; q < Q; ++q) {
            const int b = q * NW + wave;  // wave-uniform
            const unsigned dst = lds_base + (b < NB ? slot : 0u) + static_cast<unsigned>(loff[q]);
            const int vo = tail ? vtail[q] : voff[q];
            if (b < XB)
                asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, %3 offen lds"
                             ::"s"(dst), "v"(vo), "s"(xrs), "s"(soff) : "memory");
            else
                asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, %3 offen lds"
                             ::"s"(dst), "v"(vo), "s"(wrs), "s"(soff) : "memory");
        }
    };

    v4i acc[FN][FM];  // [n fragment][m fragment]
#pragma unroll
    for (int i = 0; i < FN; ++i)
#pragma unroll
        for (int j = 0; j < FM; ++j) acc[i][j] = v4i{0, 0, 0, 0};
    const int fr = lane & 15, fc = lane >> 4;
    // Fragment byte offsets of MFMA K step t (0, 1) within a slab.
    auto swz128 = [](int r, int c) { return r * S::kRow + ((c ^ ((r >> 1) & 7)) << 4); };
    int fxo[2][FM], fwo[2][FN];
#pragma unroll
    for (int t = 0; t < 2; ++t) {
#pragma unroll
        for (int j = 0; j < FM; ++j) fxo[t][j] = swz128(wm * FM * 16 + j * 16 + fr, t * 4 + fc);
#pragma unroll
        for (int i = 0; i < FN; ++i) fwo[t][i] = swz128(BM + wn * FN * 16 + i * 16 + fr, t * 4 + fc);
    }

    constexpr bool kStaged = OUT == Out::Y && sizeof(YT) == 2;
    if constexpr (kStaged) {
        // Epilogue operands into LDS by dword DMA: request e of the tile is
        // 64 values of as (rows m0..), ws (columns n0..) or bias; past m / n
        // (or without bias) the loads read zeros. Issued before the ring, so
        // the slab waits below also cover them.
        constexpr int NA = (BM + 63) / 64, NC = (BN + 63) / 64;
        const __amdgpu_buffer_rsrc_t ars = __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(as), 0, m * 4, 0x00020000);
        const __amdgpu_buffer_rsrc_t wsr = __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(ws), 0, n * 4, 0x00020000);
        const __amdgpu_buffer_rsrc_t brs = __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(bias ? bias : ws), 0, bias ? n * 4 : 0, 0x00020000);
        for (int e = wave; e < S::kEpsReq; e += NW) {
            const unsigned dst = lds_base + static_cast<unsigned>(S::kEps) + static_cast<unsigned>(e < NA ? e * 256 : BM * 4 + (e - NA) * 256);
            if (e < NA) {
                const int vo = (m0 + e * 64 + lane) * 4;
                asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dword %1, %2, 0 offen lds" ::"s"(dst), "v"(vo), "s"(ars) : "memory");
            } else if (e < NA + NC) {
                const int vo = (n0 + (e - NA) * 64 + lane) * 4;
                asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dword %1, %2, 0 offen lds" ::"s"(dst), "v"(vo), "s"(wsr) : "memory");
            } else {
                const int vo = (n0 + (e - NA - NC) * 64 + lane) * 4;
                asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dword %1, %2, 0 offen lds" ::"s"(dst), "v"(vo), "s"(brs) : "memory");
            }
        }
    }
#pragma unroll
    for (int sl = 0; sl < D - 1; ++sl) issue(sl);
    for (int kt = 0; kt < nk; ++kt) {
        wait_vmcnt<Q * (D - 2)>();  // own requests of slab kt landed
        __builtin_amdgcn_s_barrier();  // everyone's landed; slot of slab kt - 1 is free
        issue(kt + D - 1);
        const int8_t* base = lds + (kt % D) * S::kSlab;
#pragma unroll
        for (int t = 0; t < 2; ++t) {
            v4i fx[FM], fw[FN];
#pragma unroll
            for (int j = 0; j < FM; ++j) fx[j] = *reinterpret_cast<const v4i*>(base + fxo[t][j]);
#pragma unroll
            for (int i = 0; i < FN; ++i) fw[i] = *reinterpret_cast<const v4i*>(base + fwo[t][i]);
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int i = 0; i < FN; ++i)
#pragma unroll
                for (int j = 0; j < FM; ++j) acc[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(fw[i], fx[j], acc[i][j], 0, 0, 0);
        }
        // this slab's fragment reads are done before the next barrier frees its slot
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    }
    wait_vmcnt<0>();  // the ring's tail requests (zero reads) have retired

    // Lane l holds, for fragment (i, j), output row m0 + wm*FM*16 + j*16 + (l % 16)
    // and columns n0 + wn*16*FN + i*16 + 4*(l / 16) + (0..3).
    const int row_in = fr, col_in = fc * 4;
    if constexpr (OUT == Out::PARTIAL) acc_out += static_cast<size_t>(blockIdx.y) * m * n;
    if constexpr (OUT == Out::Y && sizeof(YT) == 2) {
        if ((n & 7) == 0) {
            typedef _Float16 h4 __attribute__((ext_vector_type(4)));
            constexpr int CPR = BN / 8;  // 16-byte chunks per tile row
            constexpr int HW = WM / 2, HR = BM / 2;  // wave rows and tile rows per half
#pragma unroll
            for (int half = 0; half < 2; ++half) {
                __syncthreads();  // the ring (first half) or the staging rows (second) are free
                if (wm / HW == half) {
#pragma unroll
                    for (int j = 0; j < FM; ++j) {
                        const int rl = (wm % HW) * FM * 16 + j * 16 + row_in;  // row within the half
                        const float* eps = reinterpret_cast<const float*>(lds + S::kEps);
                        const float a_s = eps[half * HR + rl];
#pragma unroll
                        for (int i = 0; i < FN; ++i) {
                            const int cl = wn * FN * 16 + i * 16 + col_in;
                            const f4 w4 = *reinterpret_cast<const f4*>(eps + BM + cl);
                            const f4 b4 = *reinterpret_cast<const f4*>(eps + BM + ((BN + 63) / 64) * 64 + cl);
                            h4 r;
#pragma unroll
                            for (int v = 0; v < 4; ++v) r[v] = from_f32<_Float16>(w8a8_epilogue(acc[i][j][v], a_s, w4[v], b4[v]));
                            *reinterpret_cast<h4*>(lds + rl * S::kStg + cl * 2) = r;
                        }
                    }
                }
                __syncthreads();
                for (int c = tid; c < HR * CPR; c += NW * 64) {
                    const int rl = c / CPR, cc = c % CPR;
                    const int row = m0 + half * HR + rl, col = n0 + cc * 8;
                    if (row < m && col < n)
                        __builtin_nontemporal_store(*reinterpret_cast<const v4i*>(lds + rl * S::kStg + cc * 16),
                                                    reinterpret_cast<v4i*>(y + static_cast<size_t>(row) * n + col));
                }
            }
            return;
        }
    }
#pragma unroll
    for (int j = 0; j < FM; ++j) {
        const int row = m0 + wm * FM * 16 + j * 16 + row_in;
        if (row >= m) continue;
        const float a_s = OUT == Out::Y ? as[row] : 0.0f;
#pragma unroll
        for (int i = 0; i < FN; ++i) {
            const int col = n0 + wn * FN * 16 + i * 16 + col_in;
            const size_t o = static_cast<size_t>(row) * n + col;
            if (col + 3 < n && (n & 3) == 0) {
                if constexpr (OUT != Out::Y) {
                    *reinterpret_cast<v4i*>(acc_out + o) = acc[i][j];
                } else {
                    const f4 w4 = *reinterpret_cast<const f4*>(ws + col);
                    const f4 b4 = bias ? *reinterpret_cast<const f4*>(bias + col) : f4{0, 0, 0, 0};
                    if constexpr (sizeof(YT) == 4) {
                        f4 r;
#pragma unroll
                        for (int v = 0; v < 4; ++v) r[v] = w8a8_epilogue(acc[i][j][v], a_s, w4[v], b4[v]);
                        *reinterpret_cast<f4*>(y + o) = r;
                    } else {
                        typedef _Float16 h4 __attribute__((ext_vector_type(4)));
                        h4 r;
#pragma unroll
                        for (int v = 0; v < 4; ++v) r[v] = from_f32<YT>(w8a8_epilogue(acc[i][j][v], a_s, w4[v], b4[v]));
                        *reinterpret_cast<h4*>(y + o) = r;
                    }
                }
            } else {
#pragma unroll
                for (int v = 0; v < 4; ++v) {
                    if (col + v >= n) break;
                    if constexpr (OUT != Out::Y) acc_out[o + v] = acc[i][j][v];
                    else y[o + v] = from_f32<YT>(w8a8_epilogue(acc[i][j][v], a_s, ws[col + v], bias ? bias[col + v] : 0.0f));
                }
            }
        }
    }
}

// ---- skinny W8A8 GEMM (3 <= m <= 64): batched decode ------------------------------------
// A workgroup owns TN 16-column MFMA tiles of weight rows and all m activation
// rows (TM 16-row tiles) over one K range; its waves take interleaved 64-byte K
// steps of that range, with operands loaded straight from global memory in the
// MFMA lane layout (weights streamed once, non-temporal; the small xq stays in
// L2) and three steps in flight per wave. The per-wave int32 partial tiles are
// added into one LDS tile with ds_add (exact, order-free). A single K range
// applies the epilogue directly. With several K ranges (very long K only) each
// range stores its tile into its own int32 workspace plane and a reduction
// launch applies the epilogue: on this multi-XCD part, finishing inside the
// kernel would need agent-scope L2 writeback/invalidate fences, and
// device-scope atomics into one plane, both measured far slower.
template <int TM, int TN, Out OUT, typename YT>
__global__ __launch_bounds__(1024) void gemm_w8a8_skinny_kernel(
    const int8_t* __restrict__ xq, const float* __restrict__ as, const int8_t* __restrict__ wq,
    const float* __restrict__ ws, const float* __restrict__ bias, YT* __restrict__ y,
    int32_t* __restrict__ acc_out, int m_total, int n, int k, int k_split) {
    constexpr int PD = 3;  // steps in flight per wave
    __shared__ int tile[TM][TN][4][64];
    // gridDim.z blocks of 64 activation rows (m > 64 in one launch); split
    // planes keep the full [m_total, n] layout.
    const size_t row_base = static_cast<size_t>(blockIdx.z) * 64;
    const int m = min(64, m_total - static_cast<int>(row_base));
    xq += row_base * k;
    if (as) as += row_base;
    const size_t out_base = row_base * n;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, nthr = block_threads();
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

    // Raw buffer loads: rows past m / n, and K positions past this range, get an
    // offset beyond the buffer so the hardware returns zeros. No load sits
    // behind a branch, so the three steps of the ring really are in flight
    // together (a predicated load makes the compiler wait for every
    // outstanding load before each MFMA).
    const __amdgpu_buffer_rsrc_t xrs = __builtin_amdgcn_make_buffer_rsrc(const_cast<int8_t*>(xq), 0, m * k, 0x00020000);
    const __amdgpu_buffer_rsrc_t wrs = __builtin_amdgcn_make_buffer_rsrc(const_cast<int8_t*>(wq), 0, n * k, 0x00020000);
    constexpr int kOob = 0x7FFFFFF0;
    int xo[TM], wo[TN];
#pragma unroll
    for (int i = 0; i < TM; ++i) xo[i] = i * 16 + fr < m ? (i * 16 + fr) * k + fk : kOob;
#pragma unroll
    for (int j = 0; j < TN; ++j) wo[j] = n0 + j * 16 + fr < n ? (n0 + j * 16 + fr) * k + fk : kOob;

    // The range has S 64-byte steps; wave w takes steps w, w + nw, ... (its
    // count: steps). Each workgroup starts at its own rotation of the range, so
    // the hundreds of workgroups reading the same activation rows at once spread
    // over different L2 lines instead of queueing on the same ones.
    const int S = (ke - kb + kBK - 1) / kBK;
    const int steps = wave < S ? (S - wave + nw - 1) / nw : 0;
    const int rot = S > 0 ? static_cast<int>((blockIdx.x * 5u) % static_cast<unsigned>(S)) : 0;
    auto load = [&](int t, v4i (&a)[TM], v4i (&b)[TN]) {
        // Steps past the wave's last one (the ring's tail prefetch) and rows
        // past m / n read as zeros without touching memory (the offset stays
        // kOob: no arithmetic on it, so no signed overflow).
        const int st = wave + t * nw;
        int sr = st + rot;
        sr = sr >= S ? sr - S : sr;
        const int kc = kb + sr * kBK;
        const bool kin = st < S && kc + fk < ke;
#pragma unroll
        for (int i = 0; i < TM; ++i)
            a[i] = __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(xrs, kin && xo[i] != kOob ? xo[i] + kc : kOob, 0, 0));
#pragma unroll
        for (int j = 0; j < TN; ++j)
            b[j] = __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(wrs, kin && wo[j] != kOob ? wo[j] + kc : kOob, 0, 0));
    };
    v4i a[PD][TM], b[PD][TN];
#pragma unroll
    for (int p = 0; p < PD; ++p) load(p, a[p], b[p]);
    auto step = [&](int t, auto phase) {
        constexpr int P = decltype(phase)::value;
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
            for (int j = 0; j < TN; ++j)
                acc[i][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a[P][i], b[P][j], acc[i][j], 0, 0, 0);
        load(t + PD, a[P], b[P]);
    };
    int t = 0;
    for (; t + PD <= steps; t += PD) {
        step(t, std::integral_constant<int, 0>{});
        step(t + 1, std::integral_constant<int, 1>{});
        step(t + 2, std::integral_constant<int, 2>{});
    }
    if (t < steps) step(t, std::integral_constant<int, 0>{});
    if (t + 1 < steps) step(t + 1, std::integral_constant<int, 1>{});
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
        const size_t o = out_base + static_cast<size_t>(row) * n + col;
        if (split) {
            acc_out[static_cast<size_t>(blockIdx.y) * m_total * n + o] = sum;  // this range's plane
        } else if constexpr (OUT == Out::ACC) {
            acc_out[o] = sum;
        } else {
            const float bb = bias ? bias[col] : 0.0f;
            y[o] = from_f32<YT>(w8a8_epilogue(sum, as[row], ws[col], bb));
        }
    }
}

// Sums the split-K partial planes [splits][m][n] in plane order (int32: exact)
// into the int32 accumulators (TO_ACC) or through the epilogue into y.
template <typename YT, bool TO_ACC>
__global__ void w8a8_reduce_kernel(const int32_t* __restrict__ parts, int splits, const float* __restrict__ as,
                                   const float* __restrict__ ws, const float* __restrict__ bias,
                                   YT* __restrict__ y, int32_t* __restrict__ acc, int m, int n) {
    const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    const int64_t mn = static_cast<int64_t>(m) * n;
    if (i >= mn) return;
    // Eight plane loads in flight per step rather than one per add (int32 sums
    // are exact in any order).
    int sum = 0;
    for (int s0 = 0; s0 < splits; s0 += 8) {
        int v[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) v[u] = s0 + u < splits ? parts[(s0 + u) * mn + i] : 0;
#pragma unroll
        for (int u = 0; u < 8; ++u) sum += v[u];
    }
    if constexpr (TO_ACC) {
        acc[i] = sum;
    } else {
        const int row = static_cast<int>(i / n), col = static_cast<int>(i % n);
        y[i] = from_f32<YT>(w8a8_epilogue(sum, as[row], ws[col], bias ? bias[col] : 0.0f));
    }
}

// ---- plans --------------------------------------------------------------------------
constexpr int kTargetBlocks = 1024;  // ~4 workgroups per CU on 256 CUs
constexpr int kSkinnyMaxM = 64;

// Skinny m: 32 columns per workgroup when that still gives >= 128 workgroups,
// else 16; waves for about three K steps each (4..16). K is split across
// workgroups only when one range would leave a wave more than 6 steps.
struct SkinnyPlan {
    int tm, tn, ntiles, splits, k_split, waves;
    size_t acc_bytes;
};
SkinnyPlan plan_skinny(int64_t m, int64_t n, int64_t k) {
    SkinnyPlan p{};
    p.tm = static_cast<int>((std::min<int64_t>(m, kSkinnyMaxM) + 15) / 16);
    p.tn = (n + 31) / 32 >= 128 ? 2 : 1;
    p.ntiles = static_cast<int>((n + 16 * p.tn - 1) / (16 * p.tn));
    const int64_t kslabs = (k + kBK - 1) / kBK;
    const int64_t splits = std::max<int64_t>(1, (kslabs + 16 * 6 - 1) / (16 * 6));
    const int64_t per = (kslabs + splits - 1) / splits;
    p.k_split = static_cast<int>(per * kBK);
    p.splits = static_cast<int>((k + p.k_split - 1) / p.k_split);
    p.waves = static_cast<int>(std::min<int64_t>(16, std::max<int64_t>(4, (per + 2) / 3)));
    if (p.splits > 1) p.acc_bytes = round_up(static_cast<size_t>(p.splits) * static_cast<size_t>(m * n) * 4, 256);
    return p;
}

// Sums split-K partial planes [splits][m][n] into acc_out, or through the
// epilogue into y.
nq_status reduce_partials(const int32_t* parts, int splits, const float* as, const float* ws, const float* bias,
                          void* y, nq_dtype ydt, int32_t* acc_out, int m, int n, hipStream_t s) {
    const unsigned g = static_cast<unsigned>((static_cast<int64_t>(m) * n + 255) / 256);
    if (acc_out)
        w8a8_reduce_kernel<float, true><<<g, 256, 0, s>>>(parts, splits, as, ws, bias, nullptr, acc_out, m, n);
    else if (ydt == NQ_F32)
        w8a8_reduce_kernel<float, false><<<g, 256, 0, s>>>(parts, splits, as, ws, bias, static_cast<float*>(y), nullptr, m, n);
    else
        w8a8_reduce_kernel<_Float16, false><<<g, 256, 0, s>>>(parts, splits, as, ws, bias, static_cast<_Float16*>(y), nullptr, m, n);
    return launch_status("w8a8_reduce_kernel");
}

// Skinny launch. A split plan stores one int32 partial plane per K range in
// the workspace and a reduction launch sums them (into acc_out, or through the
// epilogue into y).
nq_status gemm_skinny(const int8_t* xq, const float* as, const int8_t* wq, const float* ws,
                      const float* bias, void* y, nq_dtype ydt, int32_t* acc_out, int64_t m,
                      int64_t n, int64_t k, void* workspace, size_t ws_bytes, hipStream_t s) {
    const SkinnyPlan p = plan_skinny(m, n, k);
    int32_t* parts = nullptr;
    if (p.splits > 1) {
        NQ_REQUIRE(workspace && ws_bytes >= p.acc_bytes, NQ_BAD_ARG,
                   "w8a8 gemm: workspace of %zu bytes required, %zu given", p.acc_bytes, ws_bytes);
        NQ_REQUIRE(aligned(workspace, 256), NQ_BAD_ALIGN, "w8a8 gemm: workspace must be 256-byte aligned");
        parts = static_cast<int32_t*>(workspace);
    }
    const dim3 grid(static_cast<unsigned>(p.ntiles), static_cast<unsigned>(p.splits),
                    static_cast<unsigned>((m + kSkinnyMaxM - 1) / kSkinnyMaxM));
    const int threads = p.waves * 64;
    const int mi = static_cast<int>(m), ni = static_cast<int>(n), ki = static_cast<int>(k);
    auto go = [&](auto tmtag, auto tntag) {
        constexpr int TM = decltype(tmtag)::value, TN = decltype(tntag)::value;
        if (p.splits > 1)
            gemm_w8a8_skinny_kernel<TM, TN, Out::ACC, float><<<grid, threads, 0, s>>>(xq, as, wq, ws, bias, nullptr, parts, mi, ni, ki, p.k_split);
        else if (acc_out)
            gemm_w8a8_skinny_kernel<TM, TN, Out::ACC, float><<<grid, threads, 0, s>>>(xq, as, wq, ws, bias, nullptr, acc_out, mi, ni, ki, p.k_split);
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
    if (p.splits == 1) return NQ_OK;
    return reduce_partials(parts, p.splits, as, ws, bias, y, ydt, acc_out, mi, ni, s);
}

// Big-m plan. The wide-tile kernel takes every shape except few tiles with a
// long K. Among the tile shapes below it picks the least modeled time
// rounds x (3.5 + 1.32 (BM + BN) / 100 + 3.24 BM BN / 10^4) us (k = 1536),
// rounds = ceil(tiles / 256) (one tile per CU per round; a half-empty last
// round costs a full one): a least-squares fit to 50 measured shape x tile
// points (within 20%) that picks the measured best tile, or one within 3%, on
// all of them. Examples: m = 512, n = 8960: 256 x 128 tiles 19.7 us, 64 x 96
// in three rounds 25.2, 256 x 288 31.9; m = 768: 256 x 128 19.9, 64 x 64 44.2;
// m = 512, n = 2048: 64 x 64 7.7, 64 x 128 9.9, 128 x 128 12.4; m = 4096, n =
// 8960: 256 x 288 in two rounds 77.1, 256 x 256 (560 tiles) 94.2; m = 8192, n =
// 1536: 256 x 256 32.2 vs 256 x 288 34.9 (the same 192 tiles, less padding). When the chosen round has fewer than 128
// tiles and K is long, plan_prefill splits K over 64 x 64 tiles instead: each
// range stores its int32 partial tile into its own workspace plane and a
// reduction launch sums the planes and applies the epilogue (device-scope
// atomics into one plane measured several times slower).
struct WideTile {
    int fm, fn;  // tile = (64 * fm) x (32 * fn), 8 waves of (16 * fm) x (16 * fn)
};
// By falling area; of two equal areas the 64-row-per-wave tile comes first
// (m = 1024, n = 8192, k = 4096: 256 x 128 44.0 us, 128 x 256 44.6).
constexpr WideTile kWideTiles[] = {{4, 10}, {4, 9}, {4, 8}, {2, 10}, {2, 9}, {4, 4}, {2, 8},
                                   {2, 4}, {2, 2}, {1, 4}, {1, 3}, {1, 2}};
struct PrefillPlan {
    int wide_fm, wide_fn;  // tile = (64 * wide_fm) x (32 * wide_fn)
    int tiles, splits, k_slabs;  // k_slabs: 128-byte slabs per K range when split
    size_t acc_bytes;            // partial planes of a split plan
};
// m > 64: the wide tile the cost model picks (one round of tiles, at most one per
// CU, or several rounds of the largest tile); when it leaves fewer than 128
// tiles and K is long (>= 64 slabs of 64 bytes), 64 x 64 tiles with K in S =
// min(6, 256 / tiles) ranges, so that one round of about 170..256 workgroups
// shares the work (each range's int32 tile into its own plane, then the
// reduction launch). Measured against the 128 x 128-tile split-K kernel this
// replaced (us, S in brackets): m = 128, n = 1536, k = 8960 21.1 -> 13.0 [4]; n =
// 896, k = 4864 20.2 -> 9.6 [6]; n = 2048, k = 8192 18.8 -> 11.5 [4]; n = 1536,
// k = 4096 18.7 -> 9.9 [4]; m = 192: 20.5 -> 14.5 [3], 20.0 -> 10.0 [6], 19.5 ->
// 15.1 [2], 18.9 -> 11.0 [3]; m = 256: 21.2 -> 17.0 [2], 20.4 -> 10.7 [4], 19.8 ->
// 12.2 [2]; m = 384, n = 896, k = 4864 21.0 -> 11.7 [3]. On K >= 8192 128 tiles
// split too (m = 128, n = 4096, k = 14336: 36.3 -> 26.4 us in two ranges; k =
// 4096 lost, 12.8 -> 13.3).
PrefillPlan plan_prefill(int64_t m, int64_t n, int64_t k) {
    PrefillPlan p{};
    const int nk = std::max(1, static_cast<int>(k / kBK));  // also sized for shapes outside the contract
    int64_t best_cost = 0, best_tiles = 0;
    for (const WideTile& t : kWideTiles) {
        const int64_t c = ((m + 64 * t.fm - 1) / (64 * t.fm)) * ((n + 32 * t.fn - 1) / (32 * t.fn));
        const int64_t bm = 64 * t.fm, bn = 32 * t.fn;
        const int64_t cost = ((c + 255) / 256) * (35000 + 132 * (bm + bn) + 324 * bm * bn / 100);
        if (best_cost == 0 || cost < best_cost) {
            best_cost = cost;
            best_tiles = c;
            p.wide_fm = t.fm;
            p.wide_fn = t.fn;
        }
    }
    p.tiles = static_cast<int>(best_tiles);
    p.splits = 1;
    if (best_tiles >= (k >= 8192 ? 256 : 128) || nk < 64) return p;
    const int64_t t64 = ((m + 63) / 64) * ((n + 63) / 64);
    const int nsl = static_cast<int>((k + 127) / 128);
    const int64_t sp = std::min<int64_t>({6, 256 / std::max<int64_t>(1, t64),
                                          (int64_t(64) << 20) / std::max<int64_t>(1, m * n * 4)});  // <= 64 MiB of planes
    if (sp < 2) return p;
    p.wide_fm = 1;
    p.wide_fn = 2;
    p.tiles = static_cast<int>(t64);
    p.k_slabs = static_cast<int>((nsl + sp - 1) / sp);
    p.splits = (nsl + p.k_slabs - 1) / p.k_slabs;
    if (p.splits > 1) p.acc_bytes = round_up(static_cast<size_t>(p.splits) * static_cast<size_t>(m * n) * 4, 256);
    return p;
}

template <int WM, int FN, int FM, Out OUT, typename YT, int WN = 2>
nq_status launch_wide(const int8_t* xq, const float* as, const int8_t* wq, const float* ws, const float* bias,
                      YT* y, int32_t* acc_out, int m, int n, int k, hipStream_t s, int splits = 1,
                      int k_slabs = 1 << 30) {
    using S = WideShape<WM, FN, FM, WN>;
    auto* fn = gemm_w8a8_wide_kernel<WM, FN, FM, OUT, YT, WN>;
    if (nq_status st = set_dynamic_lds(reinterpret_cast<const void*>(fn), S::kLds, "gemm_w8a8_wide")) return st;
    const int tm = (m + S::kBM - 1) / S::kBM, tn = (n + S::kBN - 1) / S::kBN;
    const dim3 grid(static_cast<unsigned>(tm * tn), static_cast<unsigned>(splits));
    fn<<<grid, S::kWaves * 64, S::kLds, s>>>(xq, as, wq, ws, bias, y, acc_out, m, n, k, tm, tn, k_slabs);
    return launch_status("gemm_w8a8_wide_kernel");
}

// One round of wide-kernel tiles of (64 * fm) x (32 * fn).
// With splits > 1 each K range of k_slabs 128-byte slabs stores its int32
// partial tile into plane i of `parts` and a reduction launch applies the epilogue.
nq_status launch_wide_tile(int fm, int fn, const int8_t* xq, const float* as, const int8_t* wq, const float* ws,
                           const float* bias, void* y, nq_dtype ydt, int32_t* acc_out, int mi, int ni, int ki,
                           hipStream_t s, int splits = 1, int k_slabs = 1 << 30, int32_t* parts = nullptr) {
    // More waves along n where the tile width allows: widths that split in three
    // 16-column multiples run 12 waves (4 x 3), in four 16 waves (4 x 4), else 8
    // (4 x 2). Three or four waves per SIMD hide more of the LDS latency (config
    // 5a, 256 x 288: 64 x 96 per wave 34.8 us vs 64 x 144 37.5; m = 8192, n =
    // 1536, 256 x 256: 16 waves 27.1 us vs 8 waves 32.2; m = 512, n = 8960,
    // 128 x 256: 16.8 vs 19.5).
    auto wide = [&](auto fmtag, auto fntag) -> nq_status {
        constexpr int FM = decltype(fmtag)::value, FN2 = decltype(fntag)::value;
        constexpr int WN = FN2 % 3 == 0 ? 3 : FN2 % 4 == 0 ? 4 : 2, FN = FN2 * 2 / WN;  // 16-column fragments per wave
        if (splits > 1) {
            // Split K runs the 64 x 32 tiles (plan_small_wide: when they number at
            // most 128; wider tiles are chosen only past 256 of them) and the 64 x 64
            // tiles (plan_prefill: long K with fewer than 128 tiles).
            if constexpr (FM == 1 && FN2 <= 2) {
                const nq_status st = launch_wide<4, FN, FM, Out::PARTIAL, float, WN>(xq, as, wq, ws, bias, nullptr,
                                                                                     parts, mi, ni, ki, s, splits,
                                                                                     k_slabs);
                if (st != NQ_OK) return st;
                return reduce_partials(parts, splits, as, ws, bias, y, ydt, acc_out, mi, ni, s);
            } else {
                return fail(NQ_BAD_ARG, "w8a8 gemm: split K on a %d x %d tile", 64 * FM, 32 * FN2);
            }
        }
        if (acc_out)
            return launch_wide<4, FN, FM, Out::ACC, float, WN>(xq, as, wq, ws, bias, nullptr, acc_out, mi, ni, ki, s);
        if (ydt == NQ_F32)
            return launch_wide<4, FN, FM, Out::Y, float, WN>(xq, as, wq, ws, bias, static_cast<float*>(y), nullptr,
                                                             mi, ni, ki, s);
        return launch_wide<4, FN, FM, Out::Y, _Float16, WN>(xq, as, wq, ws, bias, static_cast<_Float16*>(y),
                                                            nullptr, mi, ni, ki, s);
    };
    using std::integral_constant;
    switch (fm * 100 + fn) {
        case 409: return wide(integral_constant<int, 4>{}, integral_constant<int, 9>{});
        case 408: return wide(integral_constant<int, 4>{}, integral_constant<int, 8>{});
        case 410: return wide(integral_constant<int, 4>{}, integral_constant<int, 10>{});
        case 404: return wide(integral_constant<int, 4>{}, integral_constant<int, 4>{});
        case 209: return wide(integral_constant<int, 2>{}, integral_constant<int, 9>{});
        case 208: return wide(integral_constant<int, 2>{}, integral_constant<int, 8>{});
        case 210: return wide(integral_constant<int, 2>{}, integral_constant<int, 10>{});
        case 204: return wide(integral_constant<int, 2>{}, integral_constant<int, 4>{});
        case 202: return wide(integral_constant<int, 2>{}, integral_constant<int, 2>{});
        case 104: return wide(integral_constant<int, 1>{}, integral_constant<int, 4>{});
        case 103: return wide(integral_constant<int, 1>{}, integral_constant<int, 3>{});
        case 102: return wide(integral_constant<int, 1>{}, integral_constant<int, 2>{});
        case 101: return wide(integral_constant<int, 1>{}, integral_constant<int, 1>{});
        default: return fail(NQ_BAD_ARG, "w8a8 gemm: no wide tile %d x %d", 64 * fm, 32 * fn);
    }
}

nq_status gemm_big(const int8_t* xq, const float* as, const int8_t* wq, const float* ws,
                   const float* bias, void* y, nq_dtype ydt, int32_t* acc_out, int64_t m, int64_t n,
                   int64_t k, void* workspace, size_t ws_bytes, hipStream_t s) {
    const int mi = static_cast<int>(m), ni = static_cast<int>(n), ki = static_cast<int>(k);
    const PrefillPlan p = plan_prefill(m, n, k);
    if (p.splits == 1) return launch_wide_tile(p.wide_fm, p.wide_fn, xq, as, wq, ws, bias, y, ydt, acc_out, mi, ni, ki, s);
    NQ_REQUIRE(workspace && ws_bytes >= p.acc_bytes, NQ_BAD_ARG,
               "w8a8 gemm: workspace of %zu bytes required, %zu given", p.acc_bytes, ws_bytes);
    NQ_REQUIRE(aligned(workspace, 256), NQ_BAD_ALIGN, "w8a8 gemm: workspace must be 256-byte aligned");
    return launch_wide_tile(p.wide_fm, p.wide_fn, xq, as, wq, ws, bias, y, ydt, acc_out, mi, ni, ki, s, p.splits,
                            p.k_slabs, static_cast<int32_t*>(workspace));
}

// The wide kernel's contract: whole 64-byte K slabs and 32-bit
// buffer offsets.
bool prefill_ok(int64_t m, int64_t n, int64_t k) {
    return k % kBK == 0 && m * k < (int64_t(1) << 31) - 64 && n * k < (int64_t(1) << 31) - 64;
}

// Decode batches (m <= 64): one round of 64 x (32 * fn) wide tiles (rows past
// m read zeros without touching memory) when the tiles, times the K ranges,
// number at least 128; otherwise (fn = 0) the skinny kernel. Short K (<= 4096)
// runs unsplit: k = 1536, n = 8960: m = 16 8.6 -> 7.2 us, m = 32 11.1 -> 7.4,
// m = 64 15.7 -> 8.4 against the skinny kernel. Longer K splits into up to 8
// ranges of at least 8 slabs for m > 16 (k = 8960, n = 1536: m = 32 12.9 ->
// 10.7 us, m = 64 17.1 -> 11.2 in five ranges; at m <= 16 the skinny kernel's
// own split is as fast).
struct SmallWidePlan {
    int fn, splits, k_slabs;
    size_t acc_bytes;
};
SmallWidePlan plan_small_wide(int64_t m, int64_t n, int64_t k, bool rounds = true) {
    SmallWidePlan p{};
    if (m > kSkinnyMaxM || m <= 0 || n <= 0 || k <= 0 || !prefill_ok(m, n, k)) return p;
    int64_t best = 0;
    int fn = 0;
    for (int f = 4; f >= 1; --f) {
        const int64_t c = (n + 32 * f - 1) / (32 * f);
        if (c <= 256 && c > best) {
            best = c;
            fn = f;
        }
    }
    // Tall weights: 64 x 128 tiles in more than one round, against the skinny
    // kernel's 16- or 32-column workgroups (m = 64, k = 3584, n = 37888: 84.3 ->
    // 42.9 us; n = 128256, k = 4096: 273.9 -> 119.5; m = 24: 174.2 -> 113.9;
    // m = 20, n = 60000, k = 2048: 54.5 -> 29.0). The GEMV / MFMA choice at m <= 8
    // keeps the one-round test (m = 5, n = 40000, k = 3072 lost 32.0 -> 35.2).
    if (best == 0 && rounds && k <= 4096) {
        fn = 4;
        best = (n + 127) / 128;
    }
    if (best == 0) return p;
    const int nslab = static_cast<int>((k + 127) / 128);
    int splits = 1;
    if (k > 4096) {
        if (m <= 16) return p;
        splits = static_cast<int>(std::min<int64_t>({8, 256 / best, nslab / 8}));
        splits = std::max(1, splits);
    }
    if (best * splits < 128) return p;
    p.fn = fn;
    p.k_slabs = (nslab + splits - 1) / splits;
    p.splits = (nslab + p.k_slabs - 1) / p.k_slabs;
    if (p.splits > 1) p.acc_bytes = round_up(static_cast<size_t>(p.splits) * static_cast<size_t>(m * n) * 4, 256);
    return p;
}

// Workspace of the MFMA GEMM for this shape: the int32 partial planes of the
// plan run_gemm picks (the small-m wide tiles or the skinny plan for m <= 64,
// the wide-tile plan for m > 64, the skinny 64-row blocks for shapes outside
// the wide kernel's contract); zero when the plan does not split K.
// One skinny launch covers all m rows (64-row blocks over gridDim.z) when its
// split planes stay within 64 MiB.
bool skinny_one_launch(int64_t m, int64_t n, int64_t k) {
    return (m + kSkinnyMaxM - 1) / kSkinnyMaxM <= 65535 && plan_skinny(m, n, k).acc_bytes <= (size_t(64) << 20);
}

size_t gemm_ws_bytes(int64_t m, int64_t n, int64_t k) {
    if (m <= 0 || n <= 0 || k <= 0) return 0;
    if (m <= kSkinnyMaxM) {
        const SmallWidePlan sw = plan_small_wide(m, n, k);
        return sw.fn ? sw.acc_bytes : plan_skinny(m, n, k).acc_bytes;
    }
    if (prefill_ok(m, n, k)) return plan_prefill(m, n, k).acc_bytes;
    return skinny_one_launch(m, n, k) ? plan_skinny(m, n, k).acc_bytes : plan_skinny(kSkinnyMaxM, n, k).acc_bytes;
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

// The skinny kernel's contract: 32-bit buffer offsets (k % 16 == 0 is mfma_ok's).
bool skinny_ok(int64_t m, int64_t n, int64_t k) {
    return std::min<int64_t>(m, kSkinnyMaxM) * k < (int64_t(1) << 31) - 64 && n * k < (int64_t(1) << 31) - 64;
}

// AUTO: the v_dot4 GEMV up to m = 4, and up to m = 8 for long K (where the
// skinny MFMA plan splits K and pays for a reduction launch) or tall weights
// that the small-m wide tiles do not take (m = 8, n = 8960, k = 1536: GEMV
// 10.25 us, skinny MFMA 10.83, wide tiles 7.1); the
// GEMV's per-row dot work grows with m while one 16x16x64 MFMA covers 16
// activation rows, so the MFMA kernels take larger m. Measured on the decode
// shapes k = 1536 / 8960, n = 256 .. 8960.
int resolve_path(int path, int64_t m, int64_t n, int64_t k) {
    if (path != NQ_PATH_AUTO) return path;
    return (m <= 4 || (m <= 8 && (k >= 4096 || (n >= 8192 && !plan_small_wide(m, n, k, false).fn)))) ? NQ_PATH_GEMV
                                                                                          : NQ_PATH_MFMA;
}

// Runs the chosen path on pre-quantized activations.
nq_status run_gemm(const int8_t* xq, const float* as, const int8_t* wq, const float* ws,
                   const float* bias, void* y, nq_dtype ydt, int32_t* acc_out, int64_t m,
                   int64_t n, int64_t k, void* workspace, size_t ws_bytes, int path, hipStream_t s) {
    int p = resolve_path(path, m, n, k);
    if (p == NQ_PATH_MFMA && !mfma_ok(xq, wq, k)) p = NQ_PATH_GENERIC;
    // Weights past 2^31 bytes exceed the MFMA kernels' 32-bit buffer offsets;
    // the v_dot4 GEMV (64-bit addressing) takes them, in slices of 8 rows.
    if (p == NQ_PATH_MFMA && !skinny_ok(m, n, k)) p = NQ_PATH_GEMV;
    if (p == NQ_PATH_MFMA) {
        const SmallWidePlan sw = plan_small_wide(m, n, k);
        if (sw.fn) {
            int32_t* parts = nullptr;
            if (sw.splits > 1) {
                NQ_REQUIRE(workspace && ws_bytes >= sw.acc_bytes, NQ_BAD_ARG,
                           "w8a8 gemm: workspace of %zu bytes required, %zu given", sw.acc_bytes, ws_bytes);
                NQ_REQUIRE(aligned(workspace, 256), NQ_BAD_ALIGN, "w8a8 gemm: workspace must be 256-byte aligned");
                parts = static_cast<int32_t*>(workspace);
            }
            return launch_wide_tile(1, sw.fn, xq, as, wq, ws, bias, y, ydt, acc_out, static_cast<int>(m),
                                    static_cast<int>(n), static_cast<int>(k), s, sw.splits, sw.k_slabs, parts);
        }
        if (m <= kSkinnyMaxM)
            return gemm_skinny(xq, as, wq, ws, bias, y, ydt, acc_out, m, n, k, workspace, ws_bytes, s);
        // (The skinny kernel over 64-row blocks in one launch was measured on the
        // m = 512 decoder shapes too: qkv 12.9 -> 20.7 us, down 29.6 -> 78 us
        // against the tiled plans, so it only takes what the wide kernel cannot.)
        if (prefill_ok(m, n, k))
            return gemm_big(xq, as, wq, ws, bias, y, ydt, acc_out, m, n, k, workspace, ws_bytes, s);
        if (skinny_one_launch(m, n, k))
            return gemm_skinny(xq, as, wq, ws, bias, y, ydt, acc_out, m, n, k, workspace, ws_bytes, s);
        // Otherwise the skinny kernel on 64-row blocks, one launch each (each
        // block re-streams the weight).
        for (int64_t r0 = 0; r0 < m; r0 += kSkinnyMaxM) {
            const int64_t mm = std::min<int64_t>(kSkinnyMaxM, m - r0);
            char* yp = y ? static_cast<char*>(y) + static_cast<size_t>(r0 * n) * dtype_size(ydt) : nullptr;
            if (nq_status st = gemm_skinny(xq + r0 * k, as ? as + r0 : nullptr, wq, ws, bias, yp, ydt,
                                           acc_out ? acc_out + r0 * n : nullptr, mm, n, k, workspace, ws_bytes, s))
                return st;
        }
        return NQ_OK;
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
// m * k up to which a decode batch quantizes its activations inside the GEMV
// kernel (each workgroup quantizes them again, so long rows pay more in VALU
// than the separate launch costs).
constexpr int64_t kDecodeFuseMax = 4096;
// Shapes on which the decode kernel over pre-quantized codes beat the GEMV /
// MFMA paths (m = 8: k/v 7.45 -> 6.37 us, q/o 7.46 -> 7.07; m = 16: k/v 7.77 ->
// 6.86, q/o 7.81 -> 7.49); wide weights (n = 8960) stay on those (m = 8: 10.3 vs
// 10.3; m = 16: 12.4 vs 10.3), and so do long-K ones (k = 8960) at m = 9..16
// (15.9 vs 14.6).
constexpr int64_t kDecodePreMaxN = 2048, kDecodePreMaxK = 2048;
// Up to 8 rows, a weight of short rows (k <= 1024) also takes it to 5120 rows
// (m = 8, n = 4864, k = 896: 8.23 -> 7.54 us; n = 8960 stays: 9.82 vs 10.29).
constexpr int64_t kDecodePreShortK = 1024, kDecodePreShortMaxN = 5120;
// 5 to 8 rows on long K up to 2048 rows (n = 1536, k = 8960: m = 8 11.25 -> 11.07
// us, m = 6 11.09 -> 10.89; k = 4096, n = 2048 lost 8.19 -> 8.31).
constexpr int64_t kDecodePreLongK = 8192;
// 17 to 64 rows as one batch of 32 or 64, 8 rows per wave, on narrow weights
// (k = 1536: n = 256, m = 32 8.75 -> 6.68 us, m = 64 10.76 -> 7.46; n = 512, m =
// 64 10.50 -> 8.29; n = 1536, m = 32 8.86 -> 8.35, m = 64 10.76 vs 11.49 stays).
constexpr int64_t kDecodePre32MaxN = 1536, kDecodePre64MaxN = 512;
nq_status act_quant(const void* x, nq_dtype xdt, int64_t m, int64_t k, int8_t* xq, float* as, hipStream_t s);
bool w8a8_tile_launch(const int8_t* xq, const float* as, const int8_t* w, const float* ws, const float* bias,
                      void* y, nq_dtype ydt, int64_t m, int64_t n, int64_t k, hipStream_t s, nq_status* st);
bool gemv_w8a8_fused_launch(const void* x, nq_dtype xdt, const int8_t* w, const float* ws,
                            const float* bias, void* y, nq_dtype ydt, int64_t m, int64_t n,
                            int64_t k, hipStream_t s, nq_status* st);
bool w8a8_decode_launch(const void* x, nq_dtype xdt, const int8_t* w, const float* ws, const float* bias,
                        void* y, nq_dtype ydt, int64_t m, int64_t n, int64_t k, hipStream_t s, nq_status* st,
                        const float* pre_scale);

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
                    workspace_bytes, path, as_stream(stream));
}

extern "C" nq_status nq_w8a8_acc_i32(const int8_t* xq, const int8_t* wq, int32_t* acc, int64_t m,
                                     int64_t n, int64_t k, void* workspace, size_t workspace_bytes,
                                     int path, void* stream) {
    if (nq_status st = check_w8a8(m, n, k, path, "w8a8_acc_i32")) return st;
    if (m == 0 || n == 0) return NQ_OK;
    NQ_REQUIRE(acc && (k == 0 || (xq && wq)), NQ_BAD_ARG, "w8a8_acc_i32: null pointer");
    NQ_REQUIRE(aligned(acc, 4), NQ_BAD_ALIGN, "w8a8_acc_i32: misaligned acc");
    return run_gemm(xq, nullptr, wq, nullptr, nullptr, nullptr, NQ_F32, acc, m, n, k, workspace,
                    workspace_bytes, path, as_stream(stream));
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
    const int p = resolve_path(path, m, n, k);
    // Decode batches (AUTO): for m <= 8 the activation quant inside the decode
    // kernel while the rows are short (every workgroup quantizes all m rows, a
    // VALU cost that grows with m * k); else, up to m = 16, one act-quant launch
    // and the decode kernel on its codes where the weight is small.
    // One activation row takes the fused-quant GEMV first, whatever k: its
    // workgroups stream their rows once and quantize one short row (m = 1: n = k =
    // 1536 5.29 -> 3.41 us, n = 256 4.30 -> 3.11, n = 4864, k = 896 5.44 -> 4.72
    // against the decode kernel; m = 2..4 measured even and keep it).
    const bool decode = path == NQ_PATH_AUTO && m <= 8;
    const bool decode16 = path == NQ_PATH_AUTO && m <= 16;
    if (p == NQ_PATH_GEMV) {
        nq_status st = NQ_OK;
        if (gemv_w8a8_fused_launch(x, x_dtype, wq, w_scale, bias, y, y_dtype, m, n, k, s, &st)) return st;
    }
    // Up to 4 rows the in-kernel quant stays cheap to 8192 codes (m = 4, n = k =
    // 1536: 6.75 -> 6.06 us; m = 3: 6.65 -> 5.69; n = 256: 6.23 -> 5.17); at 8
    // rows and k = 1536 it lost (7.0 -> 8.1), which the 4096 limit keeps out, and
    // so did fp32 activations on a tall weight (m = 4, n = 8960: 7.84 -> 8.45).
    if (decode && (m * k <= kDecodeFuseMax ||
                   (m <= 4 && m * k <= 2 * kDecodeFuseMax && (x_dtype == NQ_F16 || n <= 4096)))) {
        nq_status st = NQ_OK;
        if (w8a8_decode_launch(x, x_dtype, wq, w_scale, bias, y, y_dtype, m, n, k, s, &st, nullptr)) return st;
    }
    char* base = static_cast<char*>(workspace);
    int8_t* xq = reinterpret_cast<int8_t*>(base);
    float* as = reinterpret_cast<float*>(base + round_up(static_cast<size_t>(m * k), 256));
    char* rest = reinterpret_cast<char*>(as) + round_up(static_cast<size_t>(m) * 4, 256);
    const size_t rest_bytes = workspace_bytes - static_cast<size_t>(rest - base);
    if (nq_status st = act_quant(x, x_dtype, m, k, xq, as, s)) return st;
    // 5..8 rows on large weights with long rows or many of them: the K-split tile
    // GEMV over the codes, 4 weight rows per workgroup (us, m = 8: n = 4096, k =
    // 14336 26.4 -> 21.1; n = 4608, k = 3584 14.1 -> 11.6; n = 28672, k = 4096
    // 32.6 -> 31.2; the Qwen2.5-1.5B shapes and n = k = 4096 lost, 10.2 -> 10.6,
    // and so did m = 9..16 and narrow weights, config 3's down projection n = 1536,
    // k = 8960 11.1 -> 11.6; LM heads keep the MFMA tiles, 111.8 against 114.3).
    if (path == NQ_PATH_AUTO && m >= 5 && m <= 8 && n * k >= (int64_t(12) << 20) && k >= 3072 &&
        ((k >= 8192 && n >= 2048) || n >= 4608) && n < 65536) {
        nq_status st = NQ_OK;
        if (w8a8_tile_launch(xq, as, wq, w_scale, bias, y, y_dtype, m, n, k, s, &st)) return st;
    }
    if (decode16 && ((n <= kDecodePreMaxN && k <= kDecodePreMaxK) ||
                     (m <= 8 && k <= kDecodePreShortK && n <= kDecodePreShortMaxN) ||
                     (m > 4 && m <= 8 && k >= kDecodePreLongK && n <= kDecodePreMaxN)) ||
        (path == NQ_PATH_AUTO && m > 16 && k <= kDecodePreMaxK &&
         ((m <= 32 && n <= kDecodePre32MaxN) || (m <= 64 && n <= kDecodePre64MaxN)))) {
        nq_status st = NQ_OK;
        if (w8a8_decode_launch(xq, NQ_F16, wq, w_scale, bias, y, y_dtype, m, n, k, s, &st, as)) return st;
    }
    return run_gemm(xq, as, wq, w_scale, bias, y, y_dtype, nullptr, m, n, k, rest, rest_bytes, p, s);
}

// ---- the allocation-free W8A8 linear -------------------------------------------------------
// nq_linear_w8a8 with its workspace in a static device array instead of a
// caller buffer, for callers that cannot allocate (graph capture, serving
// loops). Each GPU holds its own copy of `scratch` for the life of the
// process; its address is looked up once per device with hipGetSymbolAddress
// (host code never passes the array's name itself). The workspace holds the
// activation codes, the row scales and the split-K partial planes, each fully
// written before it is read, so it needs no clearing between calls. Calls that
// overlap on one GPU share the array and race.
namespace nq {
namespace {
constexpr size_t kScratchBytes = size_t(32) << 20;
constexpr int kScratchDevices = 64;
static __device__ __align__(256) unsigned char scratch[kScratchBytes];

struct ScratchSlot {
    std::once_flag once;
    void* ptr = nullptr;
    hipError_t err = hipSuccess;
};
ScratchSlot g_scratch[kScratchDevices];

// The device address of this device's `scratch` (nullptr + message on failure).
nq_status scratch_for_current_device(void** out) {
    int dev = 0;
    NQ_REQUIRE(hipGetDevice(&dev) == hipSuccess, NQ_HIP_ERROR, "linear_w8a8_noalloc: hipGetDevice failed");
    NQ_REQUIRE(dev >= 0 && dev < kScratchDevices, NQ_HIP_ERROR, "linear_w8a8_noalloc: device %d beyond %d", dev,
               kScratchDevices);
    ScratchSlot& sl = g_scratch[dev];
    std::call_once(sl.once, [&sl] {
        void* p = nullptr;
        sl.err = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        sl.ptr = sl.err == hipSuccess ? p : nullptr;
    });
    NQ_REQUIRE(sl.err == hipSuccess && sl.ptr, NQ_HIP_ERROR, "linear_w8a8_noalloc: hipGetSymbolAddress failed (%s)",
               hipGetErrorString(sl.err));
    *out = sl.ptr;
    return NQ_OK;
}
}  // namespace
}  // namespace nq

extern "C" size_t nq_linear_w8a8_noalloc_max_scratch(void) { return nq::kScratchBytes; }

extern "C" nq_status nq_linear_w8a8_noalloc(const void* x, nq_dtype x_dtype, const int8_t* wq,
                                            const float* w_scale, const float* bias, void* y, nq_dtype y_dtype,
                                            int64_t m, int64_t n, int64_t k, int path, void* stream) {
    if (nq_status st = check_w8a8(m, n, k, path, "linear_w8a8_noalloc")) return st;
    if (m == 0 || n == 0) return nq_linear_w8a8(x, x_dtype, wq, w_scale, bias, y, y_dtype, m, n, k, nullptr, 0,
                                                path, stream);
    const size_t need = nq_linear_w8a8_workspace_size(m, n, k);
    NQ_REQUIRE(need <= kScratchBytes, NQ_BAD_SHAPE,
               "linear_w8a8_noalloc: m=%lld n=%lld k=%lld needs %zu bytes of scratch, the static buffer holds %zu",
               (long long)m, (long long)n, (long long)k, need, kScratchBytes);
    void* ws = nullptr;
    if (nq_status st = scratch_for_current_device(&ws)) return st;
    return nq_linear_w8a8(x, x_dtype, wq, w_scale, bias, y, y_dtype, m, n, k, ws, kScratchBytes, path, stream);
}
