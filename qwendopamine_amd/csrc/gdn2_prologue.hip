// Prologue and epilogue of the gdn2 mixer module (gfx950), both HBM-bound
// elementwise passes:
//
//  * short_conv_kernel -- ShortConvolution.forward (reference
//    models/gdn2/gdn2.py:395-430): causal depthwise conv1d of width W over
//    the token axis, plus bias and SiLU, for up to three tensors (q, k, v)
//    in one launch, with the reference's conv-cache semantics.
//  * gated_rmsnorm_kernel -- RMSNormGated.forward (gdn2.py:433-452):
//    x * rsqrt(mean(x^2) + eps) * weight * silu(z) over the last axis.
//
// Both follow the reference's rounding: it computes in the input dtype, so
// every torch op's result is rounded to that dtype (the conv output before
// the SiLU; x^2, the mean, mean + eps, the rsqrt, and each product of the
// norm), while each op itself runs in fp32 as torch's kernels do.

#include "gdn2_common.h"
#include "gdn2_internal.h"

namespace gdn2 {

namespace {

template <typename T>
__device__ __forceinline__ float round_to(float x);
template <>
__device__ __forceinline__ float round_to<float>(float x)
{
    return x;
}
template <>
__device__ __forceinline__ float round_to<bf16_t>(float x)
{
    return bf16_bits_to_f32(f32_to_bf16_bits(x));
}
template <>
__device__ __forceinline__ float round_to<f16_t>(float x)
{
    return static_cast<float>(static_cast<_Float16>(x));
}

__device__ __forceinline__ float silu_f32(float x) { return x / (1.0f + expf(-x)); }

// One thread per (tensor, batch row, channel d, tile of TT tokens).  The
// thread keeps the last W inputs of its channel in registers, so each input
// is read once (plus W-1 tokens of history at the tile start); a wave covers
// 64 consecutive channels, so every access is a coalesced row segment.
template <typename T, int W>
__global__ __launch_bounds__(256) void short_conv_kernel(ConvParams p, int TT)
{
    const ConvTensor ct = p.t[blockIdx.z];
    const int D = ct.D;
    const int d = blockIdx.x * 256 + static_cast<int>(threadIdx.x);
    if (d >= D) return;  // no barriers below
    const int tiles = (p.T + TT - 1) / TT;
    const int b = blockIdx.y / tiles, tile = blockIdx.y % tiles;
    const int t0 = tile * TT, t1 = t0 + TT < p.T ? t0 + TT : p.T;
    const T *x = static_cast<const T *>(ct.x);
    T *y = static_cast<T *>(ct.y);
    const int64_t row0 = static_cast<int64_t>(b) * p.T;

    float wt[W];
#pragma unroll
    for (int j = 0; j < W; ++j) wt[j] = io<T>::ld(static_cast<const T *>(ct.w), static_cast<int64_t>(d) * W + j);
    const float bias = ct.bias ? io<T>::ld(static_cast<const T *>(ct.bias), d) : 0.0f;

    // hist[j] = input of token t - (W-1) + j; tokens before 0 come from the
    // cache on a single-token call (gdn2.py:409-412), else zero padding.
    float hist[W];
#pragma unroll
    for (int j = 0; j < W - 1; ++j) {
        const int tt = t0 - (W - 1) + j;
        float v = 0.0f;
        if (tt >= 0)
            v = io<T>::ld(x, (row0 + tt) * D + d);
        else if (p.T == 1 && ct.cache_in)
            v = io<T>::ld(static_cast<const T *>(ct.cache_in),
                          (static_cast<int64_t>(b) * D + d) * (W - 1) + (W - 1 + tt));
        hist[j] = v;
    }
    for (int t = t0; t < t1; ++t) {
        hist[W - 1] = io<T>::ld(x, (row0 + t) * D + d);
        float acc = 0.0f;
#pragma unroll
        for (int j = 0; j < W; ++j) acc = fmaf(wt[j], hist[j], acc);
        float out = round_to<T>(acc + bias);
        if (p.silu) out = round_to<T>(silu_f32(out));
        io<T>::st(y, (row0 + t) * D + d, out);
#pragma unroll
        for (int j = 0; j < W - 1; ++j) hist[j] = hist[j + 1];
    }
    // New cache: the last ncache inputs (gdn2.py:412-418), written by the
    // tile that holds the last token; hist[0..W-2] are tokens T-W+1..T-1.
    if (ct.cache_out && t1 == p.T) {
        T *co = static_cast<T *>(ct.cache_out);
        for (int c = 0; c < p.ncache; ++c) {
            float v = 0.0f;
#pragma unroll
            for (int j = 0; j < W - 1; ++j)
                if (j == W - 1 - p.ncache + c) v = hist[j];
            io<T>::st(co, (static_cast<int64_t>(b) * D + d) * p.ncache + c, v);
        }
    }
}

// One wave per row of N = 64 * EPL elements at most; four rows per workgroup.
template <typename T, int EPL>
__global__ __launch_bounds__(256) void gated_rmsnorm_kernel(NormParams p)
{
    const int lane = threadIdx.x & 63;
    const int64_t row = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
    if (row >= p.rows) return;  // whole waves leave; no barriers below
    const int N = p.N;
    const T *x = static_cast<const T *>(p.x) + row * N;
    const T *z = static_cast<const T *>(p.z) + row * N;
    float xv[EPL], sq = 0.0f;
#pragma unroll
    for (int e = 0; e < EPL; ++e) {
        const int c = lane + 64 * e;
        xv[e] = c < N ? io<T>::ld(x, c) : 0.0f;
        sq += round_to<T>(xv[e] * xv[e]);
    }
    const float var = round_to<T>(wave_sum(sq) / static_cast<float>(N));
    const float inv = round_to<T>(rsqrtf(round_to<T>(var + p.eps)));
#pragma unroll
    for (int e = 0; e < EPL; ++e) {
        const int c = lane + 64 * e;
        if (c >= N) continue;
        const float wgt = p.w_f32 ? static_cast<const float *>(p.weight)[c]
                                  : io<T>::ld(static_cast<const T *>(p.weight), c);
        const float a = round_to<T>(xv[e] * inv);
        const float gz = round_to<T>(silu_f32(io<T>::ld(z, c)));
        if (p.w_f32) {
            // An fp32 weight promotes the rest of the expression to fp32.
            static_cast<float *>(p.out)[row * N + c] = a * wgt * gz;
        } else {
            io<T>::st(static_cast<T *>(p.out), row * N + c, round_to<T>(round_to<T>(a * wgt) * gz));
        }
    }
}

template <typename T, int W>
hipError_t conv_w(const ConvParams &p, int maxD, int ntensors, hipStream_t s)
{
    const int TT = 64;
    const int tiles = (p.T + TT - 1) / TT;
    hipLaunchKernelGGL((short_conv_kernel<T, W>), dim3((maxD + 255) / 256, p.B * tiles, ntensors),
                       dim3(256), 0, s, p, TT);
    return hipGetLastError();
}

template <typename T>
hipError_t conv_t(const ConvParams &p, int maxD, int ntensors, hipStream_t s)
{
    switch (p.W) {
    case 1: return conv_w<T, 1>(p, maxD, ntensors, s);
    case 2: return conv_w<T, 2>(p, maxD, ntensors, s);
    case 3: return conv_w<T, 3>(p, maxD, ntensors, s);
    case 4: return conv_w<T, 4>(p, maxD, ntensors, s);
    case 5: return conv_w<T, 5>(p, maxD, ntensors, s);
    case 6: return conv_w<T, 6>(p, maxD, ntensors, s);
    case 7: return conv_w<T, 7>(p, maxD, ntensors, s);
    default: return conv_w<T, 8>(p, maxD, ntensors, s);
    }
}

template <typename T>
hipError_t norm_t(const NormParams &p, hipStream_t s)
{
    const dim3 grid(static_cast<unsigned>((p.rows + 3) / 4));
    if (p.N <= 64) hipLaunchKernelGGL((gated_rmsnorm_kernel<T, 1>), grid, dim3(256), 0, s, p);
    else if (p.N <= 128) hipLaunchKernelGGL((gated_rmsnorm_kernel<T, 2>), grid, dim3(256), 0, s, p);
    else if (p.N <= 256) hipLaunchKernelGGL((gated_rmsnorm_kernel<T, 4>), grid, dim3(256), 0, s, p);
    else hipLaunchKernelGGL((gated_rmsnorm_kernel<T, 8>), grid, dim3(256), 0, s, p);
    return hipGetLastError();
}

}  // namespace

hipError_t launch_short_conv(const ConvParams &p, int io_dtype, int maxD, int ntensors,
                             hipStream_t stream)
{
    switch (io_dtype) {
    case GDN2_DTYPE_F32: return conv_t<float>(p, maxD, ntensors, stream);
    case GDN2_DTYPE_BF16: return conv_t<bf16_t>(p, maxD, ntensors, stream);
    default: return conv_t<f16_t>(p, maxD, ntensors, stream);
    }
}

hipError_t launch_gated_rmsnorm(const NormParams &p, int io_dtype, hipStream_t stream)
{
    switch (io_dtype) {
    case GDN2_DTYPE_F32: return norm_t<float>(p, stream);
    case GDN2_DTYPE_BF16: return norm_t<bf16_t>(p, stream);
    default: return norm_t<f16_t>(p, stream);
    }
}

}  // namespace gdn2
