// Shared device helpers for the gdn2 HIP kernels (gfx950 / CDNA4, wave64).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

#include "../../include/gdn2_hip.h"

namespace gdn2 {

constexpr int kWave = 64;

// bf16 is handled as raw 16-bit patterns so that the kernels depend on no
// vendor half/bf16 class: widening is a shift, narrowing is round-to-nearest-
// even on the float bits (NaN kept quiet).
struct bf16_t {
    uint16_t bits;
};
struct f16_t {
    _Float16 v;
};

__device__ __forceinline__ float bf16_bits_to_f32(uint16_t b)
{
    return __uint_as_float(static_cast<uint32_t>(b) << 16);
}

// Round-to-nearest-even narrowing; gfx950 does it in hardware (v_cvt_pk_bf16_f32).
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f)
{
    return __builtin_bit_cast(uint16_t, static_cast<__bf16>(f));
}

__device__ __forceinline__ uint32_t f32x2_to_bf16x2_bits(float lo, float hi)
{
    typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
    const bf16x2_t v = {static_cast<__bf16>(lo), static_cast<__bf16>(hi)};
    return __builtin_bit_cast(uint32_t, v);
}

template <typename T>
struct io;

template <>
struct io<float> {
    static __device__ __forceinline__ float ld(const float *p, int64_t i) { return p[i]; }
    static __device__ __forceinline__ void st(float *p, int64_t i, float x) { p[i] = x; }
};

template <>
struct io<bf16_t> {
    static __device__ __forceinline__ float ld(const bf16_t *p, int64_t i)
    {
        return bf16_bits_to_f32(p[i].bits);
    }
    static __device__ __forceinline__ void st(bf16_t *p, int64_t i, float x)
    {
        p[i].bits = f32_to_bf16_bits(x);
    }
};

template <>
struct io<f16_t> {
    static __device__ __forceinline__ float ld(const f16_t *p, int64_t i)
    {
        return static_cast<float>(p[i].v);
    }
    static __device__ __forceinline__ void st(f16_t *p, int64_t i, float x)
    {
        p[i].v = static_cast<_Float16>(x);
    }
};

__device__ __forceinline__ float wave_sum(float x)
{
#pragma unroll
    for (int off = kWave / 2; off > 0; off >>= 1) x += __shfl_xor(x, off, kWave);
    return x;
}

// torch.nn.functional.softplus with its default threshold of 20, from the
// hardware exp2 / log2 instead of the library expf / log1pf (which cost about
// as much as the rest of the prologue):  max(x, 0) + log1p(e^-|x|), with
// log1p(u) = u ln(w) / (w - 1) for w = 1 + u (Kahan's correction of the
// rounding of w; u itself when w rounds to 1): a few ulp in fp32.
__device__ __forceinline__ float softplus_f(float x)
{
    constexpr float kLog2eF = 1.4426950408889634f, kLn2F = 0.6931471805599453f;
    const float u = __builtin_amdgcn_exp2f(-fabsf(x) * kLog2eF);  // e^-|x| in (0, 1]
    const float w = 1.0f + u;
    const float l1p = w == 1.0f ? u : u * (__builtin_amdgcn_logf(w) * kLn2F) * __builtin_amdgcn_rcpf(w - 1.0f);
    const float r = fmaxf(x, 0.0f) + l1p;
    return x > 20.0f ? x : r;
}

// torch.sigmoid in fp32 (GDN2_FLAG_SIGMOID_BW): 1 / (1 + e^-x) with the
// hardware reciprocal (1 ulp), 0 for x -> -inf.
__device__ __forceinline__ float sigmoid_f(float x) { return __builtin_amdgcn_rcpf(1.0f + __expf(-x)); }

// x * sigmoid(x) with the hardware reciprocal (1 ulp in fp32) instead of an
// IEEE divide, for the module's SiLUs whose results are rounded to the input
// dtype right after (the short convolution, the output gate).
__device__ __forceinline__ float silu_f32(float x) { return x * __builtin_amdgcn_rcpf(1.0f + __expf(-x)); }

// x rounded to T (nearest even) and back to fp32: the rounding of a torch op
// computed in T.
template <typename T>
__device__ __forceinline__ float round_to(float x)
{
    if constexpr (std::is_same<T, bf16_t>::value)
        return bf16_bits_to_f32(f32_to_bf16_bits(x));
    else if constexpr (std::is_same<T, f16_t>::value)
        return static_cast<float>(static_cast<_Float16>(x));
    else
        return x;
}

// Decay activation applied in-kernel when GDN2_FLAG_GATE_IN_KERNEL is set:
//   g = -exp(A_log[h]) * softplus(g_raw + dt_bias[h, d])         (default)
//   g = lower_bound * sigmoid(exp(A_log[h]) * (g_raw + dt_bias))  (lower-bound form)
__device__ __forceinline__ float gate_activation(float graw, float a_log, float dt_bias,
                                                 int use_lower_bound, float lower_bound)
{
    const float x = graw + dt_bias;
    const float a = expf(a_log);
    if (use_lower_bound) return lower_bound * sigmoid_f(a * x);
    return -a * softplus_f(x);
}

}  // namespace gdn2
