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
};

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

// Full wave64 sum, result in every lane. The in-row steps use DPP; the two
// cross-row steps use ds_swizzle-free bpermutes. Integer adds are exact, so the
// int32 variant is order-independent; the float variant fixes one order.
__device__ __forceinline__ int wave_sum_i32(int v) {
    v += dpp<0xB1>(v);
    v += dpp<0x4E>(v);
    v += dpp<0x141>(v);
    v += dpp<0x140>(v);
    v += __shfl_xor(v, 16);
    v += __shfl_xor(v, 32);
    return v;
}

__device__ __forceinline__ float wave_sum_f32(float v) {
    v += __int_as_float(dpp<0xB1>(__float_as_int(v)));
    v += __int_as_float(dpp<0x4E>(__float_as_int(v)));
    v += __int_as_float(dpp<0x141>(__float_as_int(v)));
    v += __int_as_float(dpp<0x140>(__float_as_int(v)));
    v += __shfl_xor(v, 16);
    v += __shfl_xor(v, 32);
    return v;
}

// absmax reduction over the wave (max is order-free, so this equals the serial
// std::max scan bit for bit; NaN never wins, as in absmax_step).
__device__ __forceinline__ float wave_absmax(float v) {
    v = absmax_step(v, __int_as_float(dpp<0xB1>(__float_as_int(v))));
    v = absmax_step(v, __int_as_float(dpp<0x4E>(__float_as_int(v))));
    v = absmax_step(v, __int_as_float(dpp<0x141>(__float_as_int(v))));
    v = absmax_step(v, __int_as_float(dpp<0x140>(__float_as_int(v))));
    v = absmax_step(v, __shfl_xor(v, 16));
    v = absmax_step(v, __shfl_xor(v, 32));
    return v;
}

// Sums NV per-lane values (NV a power of two <= 64) over the wave with NV - 1
// exchanges plus log2(64 / NV) more: each exchange stage halves the values a
// lane keeps (the half selected by its lane bit) and adds the partner's copy.
// On return v[0] of lane l is the wave total of value index l / (64 / NV),
// identical in the 64 / NV lanes of that group. Fixed order, deterministic.
template <int CNT, int O, int NV, typename T>
__device__ __forceinline__ void wave_reduce_stage(T (&v)[NV], int lane) {
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
            wave_reduce_stage<half, O / 2>(v, lane);
        } else {
            v[0] += __shfl_xor(v[0], O);
            wave_reduce_stage<1, O / 2>(v, lane);
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
