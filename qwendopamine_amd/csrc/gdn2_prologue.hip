// Prologue and epilogue of the gdn2 mixer module (gfx950), both HBM-bound
// elementwise passes:
//
//  * short_conv_kernel -- ShortConvolution.forward (reference
//    models/gdn2/gdn2.py:395-430): causal depthwise conv1d of width W over
//    the token axis, plus bias and SiLU, for up to three tensors (q, k, v)
//    in one launch, with the reference's conv-cache semantics.
//  * gated_rmsnorm_kernel -- RMSNormGated.forward (gdn2.py:433-452):
//    x * rsqrt(mean(x^2) + eps) * weight * silu(z) over the last axis;
//    without z (GATE false) the same pass is RMSNorm.forward
//    (models/normalization.py:40-51), weight * (x * rsqrt(mean(x^2) + eps)).
//
// Both follow the reference's rounding: it computes in the input dtype, so
// every torch op's result is rounded to that dtype (the conv output before
// the SiLU; x^2, the mean, mean + eps, the rsqrt, and each product of the
// norm), while each op itself runs in fp32 as torch's kernels do.

#include <type_traits>

#include "gdn2_common.h"
#include "gdn2_internal.h"

namespace gdn2 {

namespace {

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
            v = io<T>::ld(x, (row0 + tt) * ct.ldx + d);
        else if (p.T == 1 && ct.cache_in)
            v = io<T>::ld(static_cast<const T *>(ct.cache_in),
                          (static_cast<int64_t>(b) * D + d) * (W - 1) + (W - 1 + tt));
        hist[j] = v;
    }
    for (int t = t0; t < t1; ++t) {
        hist[W - 1] = io<T>::ld(x, (row0 + t) * ct.ldx + d);
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
template <typename T, int EPL, bool GATE>
__global__ __launch_bounds__(256) void gated_rmsnorm_kernel(NormParams p)
{
    const int lane = threadIdx.x & 63;
    const int64_t row = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
    if (row >= p.rows) return;  // whole waves leave; no barriers below
    const int N = p.N;
    const T *x = static_cast<const T *>(p.x) + row * N;
    const T *z = GATE ? static_cast<const T *>(p.z) + row * N : nullptr;
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
        if (p.w_f32) {
            // An fp32 weight promotes the rest of the expression to fp32.
            static_cast<float *>(p.out)[row * N + c] =
                GATE ? a * wgt * round_to<T>(silu_f32(io<T>::ld(z, c))) : a * wgt;
        } else {
            const float aw = round_to<T>(a * wgt);
            io<T>::st(static_cast<T *>(p.out), row * N + c,
                      GATE ? round_to<T>(aw * round_to<T>(silu_f32(io<T>::ld(z, c)))) : aw);
        }
    }
}

// 16 bytes of T as floats and back (vector memory accesses of 8 bf16/fp16 or
// 4 fp32 values).
template <typename T>
struct Vec16 {
    static constexpr int N = 16 / static_cast<int>(sizeof(T));
    static __device__ __forceinline__ void load(const T *p, float (&v)[N])
    {
        const uint4 u = *reinterpret_cast<const uint4 *>(p);
        const unsigned w[4] = {u.x, u.y, u.z, u.w};
        if constexpr (sizeof(T) == 4) {
#pragma unroll
            for (int i = 0; i < 4; ++i) v[i] = __uint_as_float(w[i]);
        } else {
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const uint16_t b = static_cast<uint16_t>((i & 1) ? (w[i >> 1] >> 16) : (w[i >> 1] & 0xffffu));
                if constexpr (std::is_same<T, bf16_t>::value)
                    v[i] = bf16_bits_to_f32(b);
                else
                    v[i] = static_cast<float>(__builtin_bit_cast(_Float16, b));
            }
        }
    }
    static __device__ __forceinline__ void store(T *p, const float (&v)[N])
    {
        unsigned w[4];
        if constexpr (sizeof(T) == 4) {
#pragma unroll
            for (int i = 0; i < 4; ++i) w[i] = __float_as_uint(v[i]);
        } else {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                uint16_t lo, hi;
                if constexpr (std::is_same<T, bf16_t>::value) {
                    lo = f32_to_bf16_bits(v[2 * i]);
                    hi = f32_to_bf16_bits(v[2 * i + 1]);
                } else {
                    lo = __builtin_bit_cast(uint16_t, static_cast<_Float16>(v[2 * i]));
                    hi = __builtin_bit_cast(uint16_t, static_cast<_Float16>(v[2 * i + 1]));
                }
                w[i] = static_cast<unsigned>(lo) | (static_cast<unsigned>(hi) << 16);
            }
        }
        *reinterpret_cast<uint4 *>(p) = make_uint4(w[0], w[1], w[2], w[3]);
    }
};

// Vectorised short convolution: one thread per (16-byte group of CPT
// channels, tile of TT tokens), one wave per workgroup.  All of a tile's
// input rows are requested before any is used, so a wave keeps TT + W - 1
// 16-byte loads in flight; each access is a contiguous 1 KB row segment.
template <typename T, int W, int TT>
__global__ __launch_bounds__(64) void short_conv_vec_kernel(ConvParams p)
{
    using VT = Vec16<T>;
    constexpr int CPT = VT::N;
    const ConvTensor ct = p.t[blockIdx.z];
    const int D = ct.D, G = D / CPT;
    const int g = blockIdx.x * 64 + static_cast<int>(threadIdx.x);
    if (g >= G) return;  // no barriers below
    const int tiles = (p.T + TT - 1) / TT;
    const int b = blockIdx.y / tiles, tile = blockIdx.y % tiles;
    const int t0 = tile * TT;
    const int d0 = g * CPT;
    const T *x = static_cast<const T *>(ct.x);
    T *y = static_cast<T *>(ct.y);
    const int64_t row0 = static_cast<int64_t>(b) * p.T;

    // Rows t0-W+1 .. t0+TT-1 (clamped to valid rows; rows outside the
    // sequence are replaced by history or zeros below).
    float xin[W - 1 + TT][CPT];
#pragma unroll
    for (int r = 0; r < W - 1 + TT; ++r) {
        const int tt = t0 - (W - 1) + r;
        const int tc = tt < 0 ? 0 : (tt < p.T ? tt : p.T - 1);
        VT::load(x + (row0 + tc) * ct.ldx + d0, xin[r]);
    }
    // The group's weights [CPT][W] are W contiguous 16-byte pieces.
    float wflat[W][CPT], wt[W][CPT], bias[CPT];
#pragma unroll
    for (int q = 0; q < W; ++q)
        VT::load(static_cast<const T *>(ct.w) + static_cast<int64_t>(d0) * W + q * CPT, wflat[q]);
#pragma unroll
    for (int c = 0; c < CPT; ++c)
#pragma unroll
        for (int j = 0; j < W; ++j) wt[j][c] = wflat[(c * W + j) / CPT][(c * W + j) % CPT];
    if (ct.bias) {
        VT::load(static_cast<const T *>(ct.bias) + d0, bias);
    } else {
#pragma unroll
        for (int c = 0; c < CPT; ++c) bias[c] = 0.0f;
    }
#pragma unroll
    for (int r = 0; r < W - 1; ++r) {
        const int tt = t0 - (W - 1) + r;
        if (tt < 0) {
#pragma unroll
            for (int c = 0; c < CPT; ++c)
                xin[r][c] = (p.T == 1 && ct.cache_in)
                                ? io<T>::ld(static_cast<const T *>(ct.cache_in),
                                            (static_cast<int64_t>(b) * D + d0 + c) * (W - 1) + (W - 1 + tt))
                                : 0.0f;
        }
    }
#pragma unroll
    for (int i = 0; i < TT; ++i) {
        const int t = t0 + i;
        if (t >= p.T) break;
        float out[CPT];
#pragma unroll
        for (int c = 0; c < CPT; ++c) {
            float acc = 0.0f;
#pragma unroll
            for (int j = 0; j < W; ++j) acc = fmaf(wt[j][c], xin[i + j][c], acc);
            out[c] = round_to<T>(acc + bias[c]);
            if (p.silu) out[c] = round_to<T>(silu_f32(out[c]));
        }
        VT::store(y + (row0 + t) * D + d0, out);
    }
    if (ct.cache_out && t0 + TT >= p.T) {
        // The last W-1 inputs are rows (p.T - t0) .. (p.T - t0 + W - 2) of xin.
        T *co = static_cast<T *>(ct.cache_out);
        const int last = p.T - t0;  // index in xin of token p.T - (W - 1) ... shifted by W-1
#pragma unroll
        for (int r = 0; r < W - 1 + TT; ++r) {
            const int k = r - last;  // position within the last W-1 inputs
            const int c0 = k - (W - 1 - p.ncache);
            if (k >= 0 && k < W - 1 && c0 >= 0) {
#pragma unroll
                for (int c = 0; c < CPT; ++c)
                    io<T>::st(co, (static_cast<int64_t>(b) * D + d0 + c) * p.ncache + c0, xin[r][c]);
            }
        }
    }
}

// Vectorised gated RMS norm: LPR lanes per row, VPL 16-byte pieces (EPV
// values each) per lane, so a row of N = VPL * LPR * EPV values moves as
// VPL passes of LPR contiguous 16-byte pieces and is reduced by
// xor-shuffles inside its lane group.  Each thread takes RPT rows (RPB rows
// apart) and requests all of them before computing.  GATE false: no z, the
// plain RMSNorm.
template <typename T, int LPR, int RPT, int VPL, bool GATE, bool ADD = false>
__global__ __launch_bounds__(256) void gated_rmsnorm_vec_kernel(NormParams p)
{
    static_assert(!(ADD && GATE), "the residual add precedes the plain norm");
    using VT = Vec16<T>;
    constexpr int EPV = VT::N, RPB = 256 / LPR, EPL = VPL * EPV, PS = LPR * EPV;
    const int N = VPL * PS;
    const int sub = threadIdx.x % LPR;
    int64_t off[RPT];
    bool live[RPT];
    float xv[RPT][EPL], zv[RPT][GATE ? EPL : 1];
#pragma unroll
    for (int r = 0; r < RPT; ++r) {
        int64_t row = (static_cast<int64_t>(blockIdx.x) * RPT + r) * RPB + threadIdx.x / LPR;
        live[r] = row < p.rows;
        if (!live[r]) row = p.rows - 1;  // stay in bounds; keep the shuffles uniform
        off[r] = row * N + sub * EPV;
#pragma unroll
        for (int v = 0; v < VPL; ++v) {
            float t[EPV];
            VT::load(static_cast<const T *>(p.x) + off[r] + v * PS, t);
#pragma unroll
            for (int e = 0; e < EPV; ++e) xv[r][v * EPV + e] = t[e];
            if constexpr (ADD) {
                // The residual sum in the io dtype, as torch's x + h.
                VT::load(static_cast<const T *>(p.res) + off[r] + v * PS, t);
#pragma unroll
                for (int e = 0; e < EPV; ++e) xv[r][v * EPV + e] = round_to<T>(xv[r][v * EPV + e] + t[e]);
            }
            if constexpr (GATE) {
                VT::load(static_cast<const T *>(p.z) + off[r] + v * PS, t);
#pragma unroll
                for (int e = 0; e < EPV; ++e) zv[r][v * EPV + e] = t[e];
            }
        }
    }
    float wgt[EPL];
#pragma unroll
    for (int e = 0; e < EPL; ++e) {
        const int c = (e / EPV) * PS + sub * EPV + e % EPV;
        wgt[e] = p.w_f32 ? static_cast<const float *>(p.weight)[c]
                         : io<T>::ld(static_cast<const T *>(p.weight), c);
    }
#pragma unroll
    for (int r = 0; r < RPT; ++r) {
        float sq = 0.0f;
#pragma unroll
        for (int e = 0; e < EPL; ++e) sq += round_to<T>(xv[r][e] * xv[r][e]);
#pragma unroll
        for (int o = 1; o < LPR; o <<= 1) sq += __shfl_xor(sq, o, 64);
        const float var = round_to<T>(sq / static_cast<float>(N));
        const float inv = round_to<T>(rsqrtf(round_to<T>(var + p.eps)));
        float out[EPL];
#pragma unroll
        for (int e = 0; e < EPL; ++e) {
            const float a = round_to<T>(xv[r][e] * inv);
            if constexpr (GATE) {
                const float gz = round_to<T>(silu_f32(zv[r][e]));
                out[e] = p.w_f32 ? a * wgt[e] * gz : round_to<T>(round_to<T>(a * wgt[e]) * gz);
            } else {
                out[e] = p.w_f32 ? a * wgt[e] : round_to<T>(a * wgt[e]);
            }
        }
        if (!live[r]) continue;
        if constexpr (ADD) {
#pragma unroll
            for (int v = 0; v < VPL; ++v) {
                float t[EPV];
#pragma unroll
                for (int e = 0; e < EPV; ++e) t[e] = xv[r][v * EPV + e];
                VT::store(static_cast<T *>(p.sum_out) + off[r] + v * PS, t);
            }
        }
#pragma unroll
        for (int v = 0; v < VPL; ++v) {
            if (p.w_f32) {
                float *o = static_cast<float *>(p.out) + off[r] + v * PS;
#pragma unroll
                for (int e = 0; e < EPV; e += 4)
                    *reinterpret_cast<float4 *>(o + e) =
                        make_float4(out[v * EPV + e], out[v * EPV + e + 1], out[v * EPV + e + 2],
                                    out[v * EPV + e + 3]);
            } else {
                float t[EPV];
#pragma unroll
                for (int e = 0; e < EPV; ++e) t[e] = out[v * EPV + e];
                VT::store(static_cast<T *>(p.out) + off[r] + v * PS, t);
            }
        }
    }
}

template <typename T, int W>
hipError_t conv_w(const ConvParams &p, int maxD, int ntensors, bool vec, hipStream_t s)
{
    if (vec) {
        constexpr int TT = 8, CPT = Vec16<T>::N;
        const int tiles = (p.T + TT - 1) / TT;
        const int groups = maxD / CPT;
        hipLaunchKernelGGL((short_conv_vec_kernel<T, W, TT>), dim3((groups + 63) / 64, p.B * tiles, ntensors),
                           dim3(64), 0, s, p);
        return hipGetLastError();
    }
    const int TT = 64;
    const int tiles = (p.T + TT - 1) / TT;
    hipLaunchKernelGGL((short_conv_kernel<T, W>), dim3((maxD + 255) / 256, p.B * tiles, ntensors),
                       dim3(256), 0, s, p, TT);
    return hipGetLastError();
}

template <typename T>
hipError_t conv_t(const ConvParams &p, int maxD, int ntensors, hipStream_t s)
{
    // 16-byte channel groups when every tensor's rows allow them.
    constexpr int CPT = Vec16<T>::N;
    bool vec = true;
    for (int i = 0; i < ntensors; ++i) {
        const ConvTensor &c = p.t[i];
        vec = vec && c.D % CPT == 0 && c.ldx % CPT == 0 &&
              ((reinterpret_cast<uintptr_t>(c.x) | reinterpret_cast<uintptr_t>(c.y) |
                reinterpret_cast<uintptr_t>(c.w) | reinterpret_cast<uintptr_t>(c.bias)) & 15) == 0;
    }
    switch (p.W) {
    case 1: return conv_w<T, 1>(p, maxD, ntensors, vec, s);
    case 2: return conv_w<T, 2>(p, maxD, ntensors, vec, s);
    case 3: return conv_w<T, 3>(p, maxD, ntensors, vec, s);
    case 4: return conv_w<T, 4>(p, maxD, ntensors, vec, s);
    case 5: return conv_w<T, 5>(p, maxD, ntensors, vec, s);
    case 6: return conv_w<T, 6>(p, maxD, ntensors, vec, s);
    case 7: return conv_w<T, 7>(p, maxD, ntensors, vec, s);
    default: return conv_w<T, 8>(p, maxD, ntensors, vec, s);
    }
}

template <typename T, int LPR, int VPL, bool GATE>
hipError_t norm_vec(const NormParams &p, hipStream_t s)
{
    constexpr int RPT = 1, RPB = 256 / LPR;
    const dim3 grid(static_cast<unsigned>((p.rows + RPB * RPT - 1) / (RPB * RPT)));
    if constexpr (!GATE) {
        if (p.res) {
            hipLaunchKernelGGL((gated_rmsnorm_vec_kernel<T, LPR, RPT, VPL, false, true>), grid, dim3(256), 0, s, p);
            return hipGetLastError();
        }
    }
    hipLaunchKernelGGL((gated_rmsnorm_vec_kernel<T, LPR, RPT, VPL, GATE>), grid, dim3(256), 0, s, p);
    return hipGetLastError();
}

template <typename T, bool GATE>
hipError_t norm_g(const NormParams &p, hipStream_t s)
{
    // Rows of N = VPL * LPR * (16 bytes of T), LPR a power of two <= 64,
    // VPL in {1, 2, 4}, 16-byte aligned.
    constexpr int EPV = Vec16<T>::N;
    const bool aligned = ((reinterpret_cast<uintptr_t>(p.x) | reinterpret_cast<uintptr_t>(p.z) |
                           reinterpret_cast<uintptr_t>(p.out) | reinterpret_cast<uintptr_t>(p.res) |
                           reinterpret_cast<uintptr_t>(p.sum_out)) & 15) == 0;
    if (aligned && p.N % EPV == 0) {
        switch (p.N / EPV) {
        case 4: return norm_vec<T, 4, 1, GATE>(p, s);
        case 8: return norm_vec<T, 8, 1, GATE>(p, s);
        case 16: return norm_vec<T, 16, 1, GATE>(p, s);
        case 32: return norm_vec<T, 32, 1, GATE>(p, s);
        case 64: return norm_vec<T, 64, 1, GATE>(p, s);
        case 128: return norm_vec<T, 64, 2, GATE>(p, s);
        case 256: return norm_vec<T, 64, 4, GATE>(p, s);
        default: break;
        }
    }
    if (p.res) return hipErrorInvalidValue;  // the residual add has the vectorised path only (checked by the caller)
    const dim3 grid(static_cast<unsigned>((p.rows + 3) / 4));
    if (p.N <= 64) hipLaunchKernelGGL((gated_rmsnorm_kernel<T, 1, GATE>), grid, dim3(256), 0, s, p);
    else if (p.N <= 128) hipLaunchKernelGGL((gated_rmsnorm_kernel<T, 2, GATE>), grid, dim3(256), 0, s, p);
    else if (p.N <= 256) hipLaunchKernelGGL((gated_rmsnorm_kernel<T, 4, GATE>), grid, dim3(256), 0, s, p);
    else if (p.N <= 512) hipLaunchKernelGGL((gated_rmsnorm_kernel<T, 8, GATE>), grid, dim3(256), 0, s, p);
    else if (p.N <= 1024) hipLaunchKernelGGL((gated_rmsnorm_kernel<T, 16, GATE>), grid, dim3(256), 0, s, p);
    else hipLaunchKernelGGL((gated_rmsnorm_kernel<T, 32, GATE>), grid, dim3(256), 0, s, p);
    return hipGetLastError();
}

template <typename T>
hipError_t norm_t(const NormParams &p, hipStream_t s)
{
    return p.z ? norm_g<T, true>(p, s) : norm_g<T, false>(p, s);
}

// SwiGLU product: one thread per 16-byte piece of the output; a and b are the
// two column halves of the fused w1 / w2 projection's rows.
template <typename T>
__global__ __launch_bounds__(256) void silu_mul_kernel(SiluMulParams p)
{
    using VT = Vec16<T>;
    constexpr int EPV = VT::N;
    const int PPR = p.H / EPV;
    const int64_t idx = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    if (idx >= p.rows * PPR) return;
    const int64_t row = idx / PPR;
    const int c = static_cast<int>(idx - row * PPR) * EPV;
    const T *ab = static_cast<const T *>(p.ab) + row * p.ld + c;
    float a[EPV], b[EPV], o[EPV];
    VT::load(ab, a);
    VT::load(ab + p.H, b);
#pragma unroll
    for (int e = 0; e < EPV; ++e) {
        // torch's silu in float: x / (1 + exp(-x)) with an accurate exp and an IEEE divide.
        const float s = a[e] / (1.0f + expf(-a[e]));
        o[e] = round_to<T>(round_to<T>(s) * b[e]);
    }
    VT::store(static_cast<T *>(p.out) + row * p.H + c, o);
}

template <typename T>
hipError_t silu_mul_t(const SiluMulParams &p, hipStream_t s)
{
    const int64_t n = p.rows * (p.H / Vec16<T>::N);
    hipLaunchKernelGGL((silu_mul_kernel<T>), dim3(static_cast<unsigned>((n + 255) / 256)), dim3(256), 0, s, p);
    return hipGetLastError();
}

}  // namespace

hipError_t launch_silu_mul(const SiluMulParams &p, int io_dtype, hipStream_t stream)
{
    switch (io_dtype) {
    case GDN2_DTYPE_F32: return silu_mul_t<float>(p, stream);
    case GDN2_DTYPE_BF16: return silu_mul_t<bf16_t>(p, stream);
    default: return silu_mul_t<f16_t>(p, stream);
    }
}

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
