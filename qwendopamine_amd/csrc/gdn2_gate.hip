// The decay gate activation and its VJP for the training path (gfx950).
//
// Forward (reference kda_gate_fwd, gdn2_ops/chunk_kda.py:3223-3251, kernel
// :3089-3148): per element of g [tokens, H, K]
//   x = g + dt_bias[h, c]
//   y = -exp(A_log[h]) * softplus(x)                     (default)
//   y = lower_bound * sigmoid(exp(A_log[h]) * x)         (GDN2_FLAG_LOWER_BOUND)
// in fp32, the same formula the chunk and token-serial kernels apply under
// GDN2_FLAG_GATE_IN_KERNEL (gate_activation in gdn2_common.h).
//
// Backward (reference kda_gate_bwd, chunk_kda.py:3254-3292, kernel
// :3151-3220): given dy = dL/dy,
//   dg       = dy * dy/dx       (-a sigmoid(x), or lower_bound a s (1 - s))
//   dA_log   = sum over tokens and channels of dy * dy/dA_log
//              (y itself, or dg * x for the bounded form)
//   ddt_bias = sum over tokens of dg
// One workgroup per (64-token block, head) writes its partial sums of dA_log
// and ddt_bias to a workspace; a second kernel adds the blocks in order, so
// the result does not depend on scheduling.
#include <hip/hip_runtime.h>

#include "gdn2_chunk.h"
#include "gdn2_internal.h"

namespace gdn2 {

namespace {

constexpr int kGateBT = 64;  // tokens per backward workgroup

struct GateParams {
    const void *g;
    const float *A_log, *dt_bias;
    float lower_bound;
    int use_lb;
    float *y;         // forward output (fp32)
    const float *dy;  // backward input (fp32)
    void *dg;         // backward output (g's dtype)
    float *part_a;    // [nblk, H] partial dA_log
    float *part_b;    // [nblk, H, K] partial ddt_bias (null without dt_bias)
    int64_t tokens;
    int H, K, vec_ok;
};

// Channels 4q .. 4q+3 of row (token, h): one thread; K <= 256 (64 quads).
template <typename TG>
__global__ __launch_bounds__(256) void gate_fwd_kernel(GateParams p)
{
    const int64_t rows = p.tokens * p.H;
    const int quads = (p.K + 3) / 4;
    const int64_t idx = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    const int64_t row = idx / quads;
    if (row >= rows) return;
    const int c0 = 4 * static_cast<int>(idx - row * quads);
    const int h = static_cast<int>(row % p.H);
    const int64_t off = row * p.K;
    float x[4], db[4] = {0.f, 0.f, 0.f, 0.f};
    load4(static_cast<const TG *>(p.g), off, c0, p.K, true, p.vec_ok, x);
    if (p.dt_bias) load4(p.dt_bias, static_cast<int64_t>(h) * p.K, c0, p.K, true, p.vec_ok, db);
    const float a_log = p.A_log[h];
    float y[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) y[i] = gate_activation(x[i], a_log, db[i], p.use_lb, p.lower_bound);
    store4(p.y, off, c0, p.K, y);
}

// Workgroup (token block tb, head h): thread (r, q) takes channels 4q..4q+3
// of tokens tb * 64 + r, r + 4, ...; per-channel sums over its tokens, then
// over the four token lanes in LDS.
template <typename TG>
__global__ __launch_bounds__(256) void gate_bwd_kernel(GateParams p)
{
    __shared__ float s_b[4][256];
    __shared__ float s_a[4];
    const int tb = blockIdx.x / p.H, h = blockIdx.x % p.H;
    const int q = threadIdx.x & 63, r = threadIdx.x >> 6;
    const int c0 = 4 * q;
    const bool live = c0 < p.K;
    const float a = expf(p.A_log[h]);
    float db[4] = {0.f, 0.f, 0.f, 0.f};
    if (p.dt_bias && live) load4(p.dt_bias, static_cast<int64_t>(h) * p.K, c0, p.K, true, p.vec_ok, db);
    float sb[4] = {0.f, 0.f, 0.f, 0.f}, sa = 0.f;
    const int64_t t_end = p.tokens < static_cast<int64_t>(tb + 1) * kGateBT ? p.tokens
                                                                           : static_cast<int64_t>(tb + 1) * kGateBT;
    for (int64_t t = static_cast<int64_t>(tb) * kGateBT + r; t < t_end; t += 4) {
        if (!live) break;
        const int64_t off = (t * p.H + h) * p.K;
        float x[4], dy[4], dg[4];
        load4(static_cast<const TG *>(p.g), off, c0, p.K, true, p.vec_ok, x);
        load4(p.dy, off, c0, p.K, true, p.vec_ok, dy);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float xi = x[i] + db[i];
            if (p.use_lb) {
                const float s = sigmoid_f(a * xi);
                dg[i] = dy[i] * (p.lower_bound * s * (1.0f - s)) * a;
                sa = fmaf(dg[i], xi, sa);
            } else {
                dg[i] = -a * dy[i] * sigmoid_f(xi);
                sa = fmaf(dy[i], -a * softplus_f(xi), sa);
            }
            sb[i] += dg[i];
        }
        store4(static_cast<TG *>(p.dg), off, c0, p.K, dg);  // rounded to g's dtype
    }
    // Channels beyond K were never loaded (zero sums).
    sa = wave_sum(sa);
    if ((threadIdx.x & 63) == 0) s_a[r] = sa;
#pragma unroll
    for (int i = 0; i < 4; ++i) s_b[r][c0 + i] = sb[i];  // c0 + 3 <= 255
    __syncthreads();
    const int64_t blk = tb;
    if (threadIdx.x == 0) p.part_a[blk * p.H + h] = (s_a[0] + s_a[1]) + (s_a[2] + s_a[3]);
    if (p.part_b) {
        for (int c = threadIdx.x; c < p.K; c += 256)
            p.part_b[(blk * p.H + h) * p.K + c] = (s_b[0][c] + s_b[1][c]) + (s_b[2][c] + s_b[3][c]);
    }
}

// dA_log[h] and ddt_bias[h, c]: the blocks' partial sums added in block order.
__global__ __launch_bounds__(256) void gate_bwd_sum_kernel(GateParams p, int nblk, float *dA_log, float *ddt_bias)
{
    const int64_t idx = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    const int64_t nb = static_cast<int64_t>(p.H) * p.K;
    if (idx < p.H) {
        float s = 0.f;
        for (int b = 0; b < nblk; ++b) s += p.part_a[static_cast<int64_t>(b) * p.H + idx];
        dA_log[idx] = s;
    }
    if (ddt_bias && idx < nb) {
        float s = 0.f;
        for (int b = 0; b < nblk; ++b) s += p.part_b[static_cast<int64_t>(b) * nb + idx];
        ddt_bias[idx] = s;
    }
}

int64_t gate_blocks(int64_t tokens) { return (tokens + kGateBT - 1) / kGateBT; }

}  // namespace

size_t gate_bwd_workspace_bytes(int64_t tokens, int H, int K, bool has_bias)
{
    const int64_t nblk = gate_blocks(tokens);
    const int64_t a = round_up(nblk * H * 4, 256);
    return static_cast<size_t>(a + (has_bias ? round_up(nblk * H * static_cast<int64_t>(K) * 4, 256) : 0));
}

int launch_gate_fwd(const void *g, int g_dtype, const float *A_log, const float *dt_bias, float lower_bound,
                    unsigned flags, float *y, int64_t tokens, int H, int K, hipStream_t stream)
{
    GateParams p{};
    p.g = g;
    p.A_log = A_log;
    p.dt_bias = dt_bias;
    p.lower_bound = lower_bound;
    p.use_lb = (flags & GDN2_FLAG_LOWER_BOUND) != 0;
    p.y = y;
    p.tokens = tokens;
    p.H = H;
    p.K = K;
    p.vec_ok = (K % 4) == 0;
    const int64_t threads = tokens * H * ((K + 3) / 4);
    if (threads == 0) return GDN2_OK;
    const dim3 grid(static_cast<unsigned>((threads + 255) / 256));
    switch (g_dtype) {
    case GDN2_DTYPE_F32: hipLaunchKernelGGL(gate_fwd_kernel<float>, grid, dim3(256), 0, stream, p); break;
    case GDN2_DTYPE_BF16: hipLaunchKernelGGL(gate_fwd_kernel<bf16_t>, grid, dim3(256), 0, stream, p); break;
    default: hipLaunchKernelGGL(gate_fwd_kernel<f16_t>, grid, dim3(256), 0, stream, p); break;
    }
    return hipGetLastError() == hipSuccess ? GDN2_OK : GDN2_ERR_LAUNCH;
}

int launch_gate_bwd(const void *g, int g_dtype, const float *A_log, const float *dt_bias, float lower_bound,
                    unsigned flags, const float *dy, void *dg, float *dA_log, float *ddt_bias, int64_t tokens,
                    int H, int K, void *workspace, hipStream_t stream)
{
    GateParams p{};
    p.g = g;
    p.A_log = A_log;
    p.dt_bias = dt_bias;
    p.lower_bound = lower_bound;
    p.use_lb = (flags & GDN2_FLAG_LOWER_BOUND) != 0;
    p.dy = dy;
    p.dg = dg;
    p.tokens = tokens;
    p.H = H;
    p.K = K;
    p.vec_ok = (K % 4) == 0;
    const int64_t nblk = gate_blocks(tokens);
    p.part_a = static_cast<float *>(workspace);
    p.part_b = dt_bias ? reinterpret_cast<float *>(static_cast<unsigned char *>(workspace) +
                                                   round_up(nblk * H * 4, 256))
                       : nullptr;
    if (nblk > 0) {
        const dim3 grid(static_cast<unsigned>(nblk * H));
        switch (g_dtype) {
        case GDN2_DTYPE_F32: hipLaunchKernelGGL(gate_bwd_kernel<float>, grid, dim3(256), 0, stream, p); break;
        case GDN2_DTYPE_BF16: hipLaunchKernelGGL(gate_bwd_kernel<bf16_t>, grid, dim3(256), 0, stream, p); break;
        default: hipLaunchKernelGGL(gate_bwd_kernel<f16_t>, grid, dim3(256), 0, stream, p); break;
        }
        if (hipGetLastError() != hipSuccess) return GDN2_ERR_LAUNCH;
    }
    const int64_t n = static_cast<int64_t>(H) * K;
    hipLaunchKernelGGL(gate_bwd_sum_kernel, dim3(static_cast<unsigned>((n + 255) / 256)), dim3(256), 0, stream, p,
                       static_cast<int>(nblk), dA_log, dt_bias ? ddt_bias : nullptr);
    return hipGetLastError() == hipSuccess ? GDN2_OK : GDN2_ERR_LAUNCH;
}

}  // namespace gdn2
