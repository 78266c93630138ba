// Device-side helpers shared by the gfx950 kernels: vector types, wave64
// reductions, fp16 conversion, and the bit-exact quantizer rounding.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace nq {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef float f4 __attribute__((ext_vector_type(4)));

constexpr int kWave = 64;

// Element load/store for the two activation dtypes (x / y are fp32 or fp16).
__device__ __forceinline__ float to_f32(float v) { return v; }
__device__ __forceinline__ float to_f32(_Float16 v) { return static_cast<float>(v); }
template <typename T>
__device__ __forceinline__ T from_f32(float v);
template <>
__device__ __forceinline__ float from_f32<float>(float v) { return v; }
// The fp16 store rounds the finished fp32 value (round-to-nearest-even): the
// empty asm keeps the compiler from folding the producing fma/mul into a
// mixed-precision v_fma_mix* that would round the exact result to fp16 once,
// so an fp16 output is always the fp32 output rounded, bit for bit.
template <>
__device__ __forceinline__ _Float16 from_f32<_Float16>(float v) {
    asm volatile("" : "+v"(v));
    return static_cast<_Float16>(v);
}

// Quantizer rounding, bit-exact with the reference round_clamp (quant.cpp:31-38):
// IEEE fp32 divide (hipcc keeps fp32 division correctly rounded), rint =
// round-half-even, clamp with ordered compares so a NaN survives to the isnan
// test and becomes 0, scale <= 0 -> 0.
__device__ __forceinline__ float round_clamp(float w, float scale, float qmax) {
    if (scale <= 0.0f) return 0.0f;
    float r = __builtin_rintf(w / scale);
    if (r > qmax) r = qmax;
    if (r < -qmax) r = -qmax;
    if (r != r) return 0.0f;
    return r;
}

// The same rounding for a whole row that shares one scale, without a divide per
// element in the common case. a = w * rcp(s) differs from the exact quotient
// w / s by < 2^-21 relative (v_rcp_f32 is 1 ulp, the product adds half an ulp),
// and for codes of one row |w / s| <= 127 * (1 + 2^-23), so with |a| < 128 the
// error |a - w / s| is below 3e-5. When a is farther than 2e-4 from every
// half-integer, the correctly rounded quotient lies in the same rounding
// interval and rint(a) == rint(w / s); the rest (near-ties, NaN/Inf, |a| >= 128,
// scales outside [2^-100, 2^100] where rcp could flush) take the exact divide of
// round_clamp. The narrow band keeps that divergent slow path rare (~2.5% of
// wave-wide element slots for uniformly spread fractions).
struct RowQuantizer {
    float s, inv;
    bool fast;
    __device__ __forceinline__ explicit RowQuantizer(float scale) : s(scale) {
        fast = scale >= 0x1p-100f && scale <= 0x1p100f;
        inv = fast ? __builtin_amdgcn_rcpf(scale) : 0.0f;
    }
    __device__ __forceinline__ float code(float w, float qmax) const {
        if (fast) {
            const float a = w * inv;
            const float t = __builtin_rintf(a);
            if (__builtin_fabsf(a - t) < 0.4998f && __builtin_fabsf(a) < 128.0f)
                return __builtin_fminf(__builtin_fmaxf(t, -qmax), qmax);
        }
        return round_clamp(w, s, qmax);
    }
    // code() of N values with one branch for all of them: the reciprocal path
    // for each, and round_clamp for all N when any falls in the rounding band
    // (or the scale is outside the fast range). The fast path is only kept where
    // it equals round_clamp, so the codes are code()'s, element for element.
    // The W8A8 decode kernels' quantize runs this way (m = 1, n = k = 1536: 5.04
    // -> 4.63 us; n = 896, k = 4864: 4.44 -> 4.14); the row-per-workgroup act
    // quant measured slower with it (m = 8, k = 8960: 3.92 -> 4.27) and keeps code().
    template <int N>
    __device__ __forceinline__ void codes(const float (&w)[N], float qmax, float (&out)[N]) const {
        bool ok = fast;
#pragma unroll
        for (int e = 0; e < N; ++e) {
            const float a = w[e] * inv;
            const float t = __builtin_rintf(a);
            ok = ok && __builtin_fabsf(a - t) < 0.4998f && __builtin_fabsf(a) < 128.0f;
            out[e] = __builtin_fminf(__builtin_fmaxf(t, -qmax), qmax);
        }
        if (!ok) {
#pragma unroll
            for (int e = 0; e < N; ++e) out[e] = round_clamp(w[e], s, qmax);
        }
    }
    // Eight int8 codes packed little-endian into two dwords (column order).
    __device__ __forceinline__ void pack8(const float (&w)[8], int& lo, int& hi) const {
        float c[8];
        codes<8>(w, 127.0f, c);
        lo = hi = 0;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            lo |= (static_cast<int>(c[j]) & 0xFF) << (8 * j);
            hi |= (static_cast<int>(c[j + 4]) & 0xFF) << (8 * j);
        }
    }
};

// Threads per workgroup, read at kernel start. blockDim.x comes from the second
// 64-byte line of the kernel arguments; left to itself the compiler loads it where
// it is first used, which in the GEMVs is after the workgroup barrier, so a cold
// scalar miss sat on the critical path of every workgroup (int4 GEMV, n = 24,
// k = 8960: 3.59 -> 3.42 us; within noise at the bench shapes, where other
// workgroups have the line in L2 by then). The empty asm makes the value, and its
// load, due at the point of the call, beside the other argument loads.
__device__ __forceinline__ int block_threads() {
    const int t = blockDim.x;
    asm volatile("" ::"s"(t));
    return t;
}

// std::max(absmax, |v|) exactly as quant.cpp:100 evaluates it: a NaN |v| leaves
// absmax unchanged.
__device__ __forceinline__ float absmax_step(float absmax, float v) {
    const float a = __builtin_fabsf(v);
    return (absmax < a) ? a : absmax;
}

// DPP lane moves inside a 16-lane row. Controls: quad_perm xor1 = 0xB1,
// quad_perm xor2 = 0x4E, row_half_mirror = 0x141, row_mirror = 0x140.
template <int CTRL>
__device__ __forceinline__ int dpp(int v) {
    return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xF, 0xF, true);
}

// Cross-row exchanges without the LDS unit (gfx950 v_permlane{16,32}_swap):
// swap_sum16(a, b) returns, in every lane, its own row pair's combination: in
// rows 0 and 2 (lane bit 4 clear) a + (the partner row's a), in rows 1 and 3
// b + (the partner row's b)... precisely: the instruction swaps the odd rows of
// a with the even rows of b, so r[0] + r[1] is a_even + a_odd' in even rows and
// b_even' + b_odd in odd rows, where ' marks the partner lane (lane ^ 16).
// With a == b this is the pair sum v_even + v_odd, bit-identical in both lanes.
// swap_sum32 is the same for lane ^ 32 (lower and upper half of the wave).
//
// row_swap returns the two swapped registers as (first, second). Each element
// of the builtin's vector result is copied into a named unsigned before any
// other use: read as __builtin_bit_cast(T, r[1]), this toolchain's front end
// extracted element 0 for both (r[0] + r[1] became 2 * r[0]).
struct SwapPair {
    unsigned first, second;
};
template <int O>
__device__ __forceinline__ SwapPair row_swap(unsigned a, unsigned b) {
    static_assert(O == 16 || O == 32, "row swaps");
    if constexpr (O == 16) {
        const auto r = __builtin_amdgcn_permlane16_swap(a, b, false, false);
        const unsigned r0 = r[0], r1 = r[1];
        return SwapPair{r0, r1};
    } else {
        const auto r = __builtin_amdgcn_permlane32_swap(a, b, false, false);
        const unsigned r0 = r[0], r1 = r[1];
        return SwapPair{r0, r1};
    }
}
template <int O, typename T>
__device__ __forceinline__ T swap_sum(T a, T b) {
    const SwapPair r = row_swap<O>(__builtin_bit_cast(unsigned, a), __builtin_bit_cast(unsigned, b));
    return __builtin_bit_cast(T, r.first) + __builtin_bit_cast(T, r.second);
}
template <typename T>
__device__ __forceinline__ T swap_sum16(T a, T b) { return swap_sum<16>(a, b); }
template <typename T>
__device__ __forceinline__ T swap_sum32(T a, T b) { return swap_sum<32>(a, b); }
// The partner of a lane in the other row half (lane ^ 16) or wave half (lane ^ 32).
template <int O>
__device__ __forceinline__ unsigned swap_partner(unsigned v, int lane) {
    const SwapPair r = row_swap<O>(v, v);
    return (lane & O) ? r.first : r.second;
}

// Full wave64 sum, result in every lane, all VALU (no LDS round trips): DPP
// inside each 16-lane row, then the two row swaps. Each step adds two values
// that are identical across the lanes that combine them, so every lane ends
// with the same bits. Integer adds are exact; the float variant fixes one order.
__device__ __forceinline__ int wave_sum_i32(int v) {
    v += dpp<0xB1>(v);
    v += dpp<0x4E>(v);
    v += dpp<0x141>(v);
    v += dpp<0x140>(v);
    v = swap_sum16(v, v);
    return swap_sum32(v, v);
}

__device__ __forceinline__ float wave_sum_f32(float v) {
    v += __int_as_float(dpp<0xB1>(__float_as_int(v)));
    v += __int_as_float(dpp<0x4E>(__float_as_int(v)));
    v += __int_as_float(dpp<0x141>(__float_as_int(v)));
    v += __int_as_float(dpp<0x140>(__float_as_int(v)));
    v = swap_sum16(v, v);
    return swap_sum32(v, v);
}

// absmax reduction over the wave (max is order-free, so this equals the serial
// std::max scan bit for bit; NaN never wins, as in absmax_step). The running
// values are never NaN, so combining them is symmetric.
__device__ __forceinline__ float wave_absmax(float v) {
    v = absmax_step(v, __int_as_float(dpp<0xB1>(__float_as_int(v))));
    v = absmax_step(v, __int_as_float(dpp<0x4E>(__float_as_int(v))));
    v = absmax_step(v, __int_as_float(dpp<0x141>(__float_as_int(v))));
    v = absmax_step(v, __int_as_float(dpp<0x140>(__float_as_int(v))));
    v = absmax_step(v, __uint_as_float(swap_partner<16>(__float_as_uint(v), __lane_id())));
    v = absmax_step(v, __uint_as_float(swap_partner<32>(__float_as_uint(v), __lane_id())));
    return v;
}

// The exchange partner of stage O of wave_reduce_multi: a lane that shares
// every lane bit above O and differs in bit O (quad_perm for 1 and 2, the
// 8- and 16-lane mirrors for 4 and 8, the row swaps for 16 and 32).
template <int O, typename T>
__device__ __forceinline__ T xchg(T v, int lane) {
    const int b = __builtin_bit_cast(int, v);
    int r;
    if constexpr (O == 1) r = dpp<0xB1>(b);
    else if constexpr (O == 2) r = dpp<0x4E>(b);
    else if constexpr (O == 4) r = dpp<0x141>(b);
    else if constexpr (O == 8) r = dpp<0x140>(b);
    else r = static_cast<int>(swap_partner<O>(static_cast<unsigned>(b), lane));
    return __builtin_bit_cast(T, r);
}

// Sums NV per-lane values (NV a power of two <= 64) over the wave with NV - 1
// exchanges plus log2(64 / NV) more: each exchange stage halves the values a
// lane keeps (the half selected by its lane bit) and adds the partner's copy.
// On return v[0] of lane l is the wave total of value index l / (64 / NV),
// identical in the 64 / NV lanes of that group. Fixed order, deterministic.
// All exchanges are VALU (DPP and the gfx950 row swaps): no LDS round trips on
// the tail of the kernels that end with this reduction.
template <int CNT, int O, int NV, typename T>
__device__ __forceinline__ void wave_reduce_stage(T (&v)[NV], int lane) {
    if constexpr (O >= 1) {
        if constexpr (CNT > 1) {
            constexpr int half = CNT / 2;
            if constexpr (O >= 16) {
                // one swap moves both halves: even side keeps v[j], odd side v[j + half]
#pragma unroll
                for (int j = 0; j < half; ++j)
                    v[j] = O == 16 ? swap_sum16(v[j], v[j + half]) : swap_sum32(v[j], v[j + half]);
            } else {
                const bool hi = (lane & O) != 0;
#pragma unroll
                for (int j = 0; j < half; ++j) {
                    const T keep = hi ? v[j + half] : v[j];
                    const T send = hi ? v[j] : v[j + half];
                    v[j] = keep + xchg<O>(send, lane);
                }
            }
            wave_reduce_stage<half, O / 2>(v, lane);
        } else {
            if constexpr (O >= 16) v[0] = O == 16 ? swap_sum16(v[0], v[0]) : swap_sum32(v[0], v[0]);
            else v[0] += xchg<O>(v[0], lane);
            wave_reduce_stage<1, O / 2>(v, lane);
        }
    }
}

// absmax over aligned groups of G lanes (G a power of two <= 64), result in
// every lane of the group: the stage-O partners stay inside the group.
template <int G, int O = 1>
__device__ __forceinline__ float group_absmax(float am, int lane) {
    if constexpr (O < G) {
        am = absmax_step(am, xchg<O>(am, lane));
        return group_absmax<G, 2 * O>(am, lane);
    } else {
        return am;
    }
}

// The same reduction with ds_bpermute (__shfl_xor) exchanges at every stage:
// for many values (NV >= 8) the all-VALU exchanges above left the compiler
// free to interleave all stages with the producing math, which spilled up to
// 150 VGPRs in the int4 GEMV at m = 8; the LDS-routed exchanges keep the
// stages in order at the cost of an LDS round trip each.
template <int CNT, int O, int NV, typename T>
__device__ __forceinline__ void wave_reduce_stage_bperm(T (&v)[NV], int lane) {
    if constexpr (O >= 1) {
        if constexpr (CNT > 1) {
            constexpr int half = CNT / 2;
            const bool hi = (lane & O) != 0;
#pragma unroll
            for (int j = 0; j < half; ++j) {
                const T keep = hi ? v[j + half] : v[j];
                const T send = hi ? v[j] : v[j + half];
                v[j] = keep + __shfl_xor(send, O);
            }
            wave_reduce_stage_bperm<half, O / 2>(v, lane);
        } else {
            v[0] += __shfl_xor(v[0], O);
            wave_reduce_stage_bperm<1, O / 2>(v, lane);
        }
    }
}

template <int NV, typename T>
__device__ __forceinline__ T wave_reduce_multi(T (&v)[NV], int lane) {
    static_assert(NV >= 1 && NV <= 64 && (NV & (NV - 1)) == 0, "power of two");
    wave_reduce_stage<NV, 32>(v, lane);
    return v[0];
}

// Signed byte i of a dword as float.
template <int I>
__device__ __forceinline__ float sbyte_f32(int d) {
    return static_cast<float>((d << (24 - 8 * I)) >> 24);
}

// The W8A8 epilogue, shared by the GEMV and the MFMA GEMM so both produce the
// same bits from the same int32: float(acc) * a_scale * w_scale + bias
// (the reference GPU store, cuda_quant.cu:112 / :156).
__device__ __forceinline__ float w8a8_epilogue(int acc, float as, float ws, float b) {
    return __builtin_fmaf(static_cast<float>(acc) * as, ws, b);
}

}  // namespace nq
