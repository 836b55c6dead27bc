// Backward of the gdn2 mixer's prologue and epilogue (gfx950), for training:
//
//  * short_conv_bwd_kernel -- the gradient of ShortConvolution.forward
//    (reference models/gdn2/gdn2.py:395-430) on a prefill call (no cache):
//    y = silu(round(b + sum_j w_j x_{t-W+1+j})).  Recomputes the rounded
//    pre-activation, dpre = round(dy * silu'(pre)) as torch's SiLU backward
//    does, dx_t = sum_j w_j dpre_{t+W-1-j}, and per-tile partial sums of
//    dw_j = sum_t dpre_t x_{t-W+1+j} and db = sum_t dpre_t.
//  * gated_rmsnorm_bwd_kernel -- the gradient of RMSNormGated.forward
//    (gdn2.py:433-452): with r = rsqrt(mean(x^2) + eps), xn = x r, s = silu(z),
//      dx = r (g - xn mean(g xn)),  g = dy w s
//      dz = dy xn w silu'(z),       dw = sum over rows of dy xn s
//    in fp32, with per-workgroup partial sums of dw.
//  * partial_reduce_kernel -- sums the partials over tiles / waves in a fixed
//    order (deterministic) and writes the weight-shaped gradients.
//
// All three are HBM-bound elementwise / reduction passes.

#include <type_traits>

#include "gdn2_common.h"
#include "gdn2_internal.h"

namespace gdn2 {

namespace {

// silu'(x) = sigmoid(x) (1 + x (1 - sigmoid(x))), torch's formula.
__device__ __forceinline__ float silu_grad(float x)
{
    const float s = 1.0f / (1.0f + expf(-x));
    return s * (1.0f + x * (1.0f - s));
}

// One thread per (batch row, channel d, tile of TT tokens); a wave covers 64
// consecutive channels, so every row access is a coalesced segment.  The
// thread holds inputs t0-W+1 .. t0+TT+W-2 and upstream gradients
// t0 .. t0+TT+W-2 of its channel.
template <typename T, int W, int TT>
__global__ __launch_bounds__(256) void short_conv_bwd_kernel(ConvBwdParams p)
{
    constexpr int NX = TT + 2 * (W - 1), NG = TT + W - 1;
    const int d = blockIdx.x * 256 + static_cast<int>(threadIdx.x);
    if (d >= p.D) return;  // no barriers below
    const int tiles = (p.T + TT - 1) / TT;
    const int b = blockIdx.y / tiles, tile = blockIdx.y % tiles;
    const int t0 = tile * TT;
    const T *x = static_cast<const T *>(p.x);
    const T *dy = static_cast<const T *>(p.dy);
    const int64_t row0 = static_cast<int64_t>(b) * p.T;

    // Every request first, from clamped (valid) rows; rows outside the
    // sequence are zeroed below.
    float xin[NX], gin[NG];
#pragma unroll
    for (int r = 0; r < NX; ++r) {
        const int tt = t0 - (W - 1) + r;
        const int tc = tt < 0 ? 0 : (tt < p.T ? tt : p.T - 1);
        xin[r] = io<T>::ld(x, (row0 + tc) * p.ldx + d);
    }
#pragma unroll
    for (int r = 0; r < NG; ++r) {
        const int tt = t0 + r;
        const int tc = tt < p.T ? tt : p.T - 1;
        gin[r] = io<T>::ld(dy, (row0 + tc) * p.D + d);
    }
    float wt[W];
#pragma unroll
    for (int j = 0; j < W; ++j) wt[j] = io<T>::ld(static_cast<const T *>(p.w), static_cast<int64_t>(d) * W + j);
    const float bias = p.bias ? io<T>::ld(static_cast<const T *>(p.bias), d) : 0.0f;
#pragma unroll
    for (int r = 0; r < NX; ++r) {
        const int tt = t0 - (W - 1) + r;
        if (tt < 0 || tt >= p.T) xin[r] = 0.0f;
    }
    // dpre for tokens t0 .. t0+NG-1 (zero past the sequence end).
    float dpre[NG];
#pragma unroll
    for (int r = 0; r < NG; ++r) {
        float acc = 0.0f;
#pragma unroll
        for (int j = 0; j < W; ++j) acc = fmaf(wt[j], xin[r + j], acc);
        const float pre = round_to<T>(acc + bias);  // the forward's rounded conv output
        const float g = p.silu ? round_to<T>(gin[r] * silu_grad(pre)) : gin[r];
        dpre[r] = t0 + r < p.T ? g : 0.0f;
    }
    float dw[W], db = 0.0f;
#pragma unroll
    for (int j = 0; j < W; ++j) dw[j] = 0.0f;
    T *dx = static_cast<T *>(p.dx);
#pragma unroll
    for (int i = 0; i < TT; ++i) {
        const int t = t0 + i;
        if (t >= p.T) break;
        float acc = 0.0f;
#pragma unroll
        for (int j = 0; j < W; ++j) acc = fmaf(wt[j], dpre[i + W - 1 - j], acc);
        io<T>::st(dx, (row0 + t) * p.D + d, acc);
#pragma unroll
        for (int j = 0; j < W; ++j) dw[j] = fmaf(dpre[i], xin[i + j], dw[j]);
        db += dpre[i];
    }
    // Partials [tile][W + 1][D]: channel-contiguous for coalesced writes.
    float *part = p.part + static_cast<int64_t>(blockIdx.y) * (W + 1) * p.D;
#pragma unroll
    for (int j = 0; j < W; ++j) part[static_cast<int64_t>(j) * p.D + d] = dw[j];
    part[static_cast<int64_t>(W) * p.D + d] = db;
}

// A grid of workgroups walking the rows: wave w of workgroup b handles rows
// (4 (4 b + w) + j) + k * 16 * gridDim.x, j < 4 (four rows' requests in
// flight per iteration); lane l holds columns l, l + 64, ... (up to 4).  The
// four waves' partial sums of dw are combined in LDS in a fixed order and
// written as the workgroup's partial row part[b][N].
template <typename T, typename TW, int MAXC>
__global__ __launch_bounds__(256) void gated_rmsnorm_bwd_kernel(NormBwdParams p)
{
    constexpr int RPI = 4;
    __shared__ float s_acc[4][256];
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int N = p.N;
    const T *x = static_cast<const T *>(p.x);
    const T *z = static_cast<const T *>(p.z);
    const T *dy = static_cast<const T *>(p.dy);
    T *dx = static_cast<T *>(p.dx);
    T *dz = static_cast<T *>(p.dz);
    float wv_[MAXC], acc[MAXC];
#pragma unroll
    for (int i = 0; i < MAXC; ++i) {
        const int c = lane + 64 * i;
        wv_[i] = c < N ? io<TW>::ld(static_cast<const TW *>(p.weight), c) : 0.0f;
        acc[i] = 0.0f;
    }
    const int64_t stride = static_cast<int64_t>(gridDim.x) * 16;
    for (int64_t base = (static_cast<int64_t>(blockIdx.x) * 4 + wv) * RPI; base < p.rows; base += stride) {
        float xv[RPI][MAXC], zv[RPI][MAXC], gv[RPI][MAXC];
#pragma unroll
        for (int j = 0; j < RPI; ++j) {
            const int64_t row = base + j < p.rows ? base + j : p.rows - 1;  // valid address
#pragma unroll
            for (int i = 0; i < MAXC; ++i) {
                const int c = lane + 64 * i;
                const int64_t off = row * N + (c < N ? c : N - 1);
                xv[j][i] = io<T>::ld(x, off);
                zv[j][i] = io<T>::ld(z, off);
                gv[j][i] = io<T>::ld(dy, off);
            }
        }
#pragma unroll
        for (int j = 0; j < RPI; ++j) {
            const int64_t row = base + j;
            const bool live = row < p.rows;
            float sq = 0.0f;
#pragma unroll
            for (int i = 0; i < MAXC; ++i) {
                if (lane + 64 * i >= N || !live) xv[j][i] = zv[j][i] = gv[j][i] = 0.0f;
                sq = fmaf(xv[j][i], xv[j][i], sq);
            }
            sq = wave_sum(sq);
            const float r = rsqrtf(sq / static_cast<float>(N) + p.eps);
            float xn[MAXC], g[MAXC], dot = 0.0f;
#pragma unroll
            for (int i = 0; i < MAXC; ++i) {
                xn[i] = xv[j][i] * r;
                const float sg = 1.0f / (1.0f + expf(-zv[j][i]));
                const float sz = zv[j][i] * sg;
                g[i] = gv[j][i] * wv_[i] * sz;
                dot = fmaf(g[i], xn[i], dot);
                // dz = dy xn w silu'(z); dw += dy xn s
                const float dzv = gv[j][i] * xn[i] * wv_[i] * (sg * (1.0f + zv[j][i] * (1.0f - sg)));
                const int c = lane + 64 * i;
                if (live && c < N) io<T>::st(dz, row * N + c, dzv);
                acc[i] = fmaf(gv[j][i], xn[i] * sz, acc[i]);
            }
            dot = wave_sum(dot) / static_cast<float>(N);
#pragma unroll
            for (int i = 0; i < MAXC; ++i) {
                const int c = lane + 64 * i;
                if (live && c < N) io<T>::st(dx, row * N + c, r * (g[i] - xn[i] * dot));
            }
        }
    }
#pragma unroll
    for (int i = 0; i < MAXC; ++i) s_acc[wv][lane + 64 * i] = acc[i];
#pragma unroll
    for (int i = MAXC; i < 4; ++i) s_acc[wv][lane + 64 * i] = 0.0f;
    __syncthreads();
    for (int c = threadIdx.x; c < N; c += 256)
        p.part[static_cast<int64_t>(blockIdx.x) * N + c] = (s_acc[0][c] + s_acc[1][c]) + (s_acc[2][c] + s_acc[3][c]);
}

// out[e] = sum over k < nparts of part[k * E + e], e < E, in a fixed order
// (deterministic): workgroup b takes 64 consecutive e, its four waves the
// parts k = w mod 4 with four accumulators each, combined in LDS.  Written in
// TO.  With W > 0, elements e = j * D + d of [W + 1][D] partials go to a
// [D][W] weight (j < W) and a [D] bias (j == W).
template <typename TO>
__global__ __launch_bounds__(256) void partial_reduce_kernel(const float *part, int64_t nparts, int64_t E,
                                                             void *out, void *out_bias, int D, int W)
{
    __shared__ float s_sum[4][64];
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int64_t e = static_cast<int64_t>(blockIdx.x) * 64 + lane;
    const int64_t ec = e < E ? e : E - 1;
    float a[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    int64_t k = wv;
    for (; k + 12 < nparts; k += 16) {
#pragma unroll
        for (int u = 0; u < 4; ++u) a[u] += part[(k + 4 * u) * E + ec];
    }
    for (; k < nparts; k += 4) a[0] += part[k * E + ec];
    s_sum[wv][lane] = (a[0] + a[1]) + (a[2] + a[3]);
    __syncthreads();
    if (wv != 0 || e >= E) return;
    const float s = (s_sum[0][lane] + s_sum[1][lane]) + (s_sum[2][lane] + s_sum[3][lane]);
    if (W == 0) {
        io<TO>::st(static_cast<TO *>(out), e, s);
        return;
    }
    const int j = static_cast<int>(e / D), d = static_cast<int>(e % D);
    if (j < W)
        io<TO>::st(static_cast<TO *>(out), static_cast<int64_t>(d) * W + j, s);
    else if (out_bias)
        io<TO>::st(static_cast<TO *>(out_bias), d, s);
}

template <typename T, int W>
hipError_t conv_bwd_w(const ConvBwdParams &p, hipStream_t s)
{
    constexpr int TT = 32;
    const int tiles = (p.T + TT - 1) / TT;
    hipLaunchKernelGGL((short_conv_bwd_kernel<T, W, TT>), dim3((p.D + 255) / 256, p.B * tiles), dim3(256), 0, s,
                       p);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    const int64_t E = static_cast<int64_t>(W + 1) * p.D;
    hipLaunchKernelGGL((partial_reduce_kernel<T>), dim3(static_cast<unsigned>((E + 63) / 64)), dim3(256), 0, s,
                       p.part, static_cast<int64_t>(p.B) * tiles, E, p.dw, p.dbias, p.D, W);
    return hipGetLastError();
}

template <typename T>
hipError_t conv_bwd_t(const ConvBwdParams &p, hipStream_t s)
{
    switch (p.W) {
    case 1: return conv_bwd_w<T, 1>(p, s);
    case 2: return conv_bwd_w<T, 2>(p, s);
    case 3: return conv_bwd_w<T, 3>(p, s);
    case 4: return conv_bwd_w<T, 4>(p, s);
    case 5: return conv_bwd_w<T, 5>(p, s);
    case 6: return conv_bwd_w<T, 6>(p, s);
    case 7: return conv_bwd_w<T, 7>(p, s);
    default: return conv_bwd_w<T, 8>(p, s);
    }
}

template <typename T, typename TW>
hipError_t norm_bwd_t(const NormBwdParams &p, hipStream_t s)
{
    const int blocks = static_cast<int>(norm_bwd_blocks(p.rows));
    // Columns per lane: N <= 64, 128 or 256.
    if (p.N <= 64)
        hipLaunchKernelGGL((gated_rmsnorm_bwd_kernel<T, TW, 1>), dim3(blocks), dim3(256), 0, s, p);
    else if (p.N <= 128)
        hipLaunchKernelGGL((gated_rmsnorm_bwd_kernel<T, TW, 2>), dim3(blocks), dim3(256), 0, s, p);
    else
        hipLaunchKernelGGL((gated_rmsnorm_bwd_kernel<T, TW, 4>), dim3(blocks), dim3(256), 0, s, p);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL((partial_reduce_kernel<TW>), dim3((p.N + 63) / 64), dim3(256), 0, s, p.part,
                       static_cast<int64_t>(blocks), static_cast<int64_t>(p.N), p.dweight, nullptr, p.N, 0);
    return hipGetLastError();
}

}  // namespace

int64_t conv_bwd_partial_floats(int B, int T, int D, int W)
{
    return static_cast<int64_t>(B) * ((T + 31) / 32) * (W + 1) * D;
}

int64_t norm_bwd_blocks(int64_t rows)
{
    // At least 16 rows (four per wave) per workgroup, at most 1024 workgroups
    // (four per CU): one partial row per workgroup.
    const int64_t b = (rows + 15) / 16;
    return b < 1 ? 1 : (b > 1024 ? 1024 : b);
}

hipError_t launch_short_conv_bwd(const ConvBwdParams &p, int io_dtype, hipStream_t stream)
{
    if (p.B == 0 || p.T == 0 || p.D == 0) return hipSuccess;
    switch (io_dtype) {
    case GDN2_DTYPE_F32: return conv_bwd_t<float>(p, stream);
    case GDN2_DTYPE_BF16: return conv_bwd_t<bf16_t>(p, stream);
    default: return conv_bwd_t<f16_t>(p, stream);
    }
}

hipError_t launch_gated_rmsnorm_bwd(const NormBwdParams &p, int io_dtype, hipStream_t stream)
{
    if (p.rows == 0) return hipSuccess;
    if (p.w_f32) {
        switch (io_dtype) {
        case GDN2_DTYPE_F32: return norm_bwd_t<float, float>(p, stream);
        case GDN2_DTYPE_BF16: return norm_bwd_t<bf16_t, float>(p, stream);
        default: return norm_bwd_t<f16_t, float>(p, stream);
        }
    }
    switch (io_dtype) {
    case GDN2_DTYPE_F32: return norm_bwd_t<float, float>(p, stream);
    case GDN2_DTYPE_BF16: return norm_bwd_t<bf16_t, bf16_t>(p, stream);
    default: return norm_bwd_t<f16_t, f16_t>(p, stream);
    }
}

}  // namespace gdn2
