// extern "C" entry points of libgdn2_hip.so: argument validation and dispatch.
// Declarations and the reference interfaces they replace: include/gdn2_hip.h.

#include "gdn2_chunk.h"
#include "gdn2_common.h"
#include "gdn2_internal.h"

using namespace gdn2;

static bool valid_dtype(int d)
{
    return d == GDN2_DTYPE_F32 || d == GDN2_DTYPE_BF16 || d == GDN2_DTYPE_F16;
}

static int check_chunk_args(int io_dtype, int g_dtype, const int64_t *cu_seqlens,
                            const int64_t *cu_seqlens_host, int num_seqs, int B, int T, int H,
                            int K, int V, unsigned flags, const float *A_log)
{
    if (!valid_dtype(io_dtype) || !valid_dtype(g_dtype)) return GDN2_ERR_INVALID;
    if (B < 0 || T < 0 || H <= 0 || K <= 0 || V <= 0) return GDN2_ERR_INVALID;
    if (flags & ~(GDN2_FLAG_L2NORM_QK | GDN2_FLAG_GATE_IN_KERNEL | GDN2_FLAG_LOWER_BOUND |
                  GDN2_FLAG_SAVE_FOR_BWD | GDN2_FLAG_TRANSPOSE_STATE | GDN2_FLAG_SIGMOID_BW))
        return GDN2_ERR_INVALID;
    if ((flags & GDN2_FLAG_LOWER_BOUND) && !(flags & GDN2_FLAG_GATE_IN_KERNEL))
        return GDN2_ERR_INVALID;
    if ((flags & GDN2_FLAG_GATE_IN_KERNEL) && !A_log) return GDN2_ERR_INVALID;
    // Gate logits are an inference option: the backward reads b and w as given.
    if ((flags & GDN2_FLAG_SIGMOID_BW) && (flags & GDN2_FLAG_SAVE_FOR_BWD)) return GDN2_ERR_INVALID;
    if ((cu_seqlens == nullptr) != (cu_seqlens_host == nullptr)) return GDN2_ERR_INVALID;
    if (cu_seqlens && (B != 1 || num_seqs < 0)) return GDN2_ERR_INVALID;
    if (cu_seqlens_host) {
        if (cu_seqlens_host[0] != 0 || cu_seqlens_host[num_seqs] != T) return GDN2_ERR_INVALID;
        for (int i = 0; i < num_seqs; ++i)
            if (cu_seqlens_host[i + 1] < cu_seqlens_host[i]) return GDN2_ERR_INVALID;
    }
    return GDN2_OK;
}

static void fill_chunk_args(ChunkFwdArgs &a, const void *q, const void *k, const void *v,
                            const void *g, const void *b, const void *w, void *o,
                            const float *h0, float *ht, const float *A_log, const float *dt_bias,
                            float lower_bound, const int64_t *cu_seqlens, const int64_t *cu_host,
                            int num_seqs, int B, int T, int H, int K, int V, float scale,
                            unsigned flags, void *workspace, size_t workspace_bytes)
{
    a.q = q; a.k = k; a.v = v; a.g = g; a.b = b; a.w = w; a.o = o;
    a.h0 = h0;
    a.ht = ht;
    a.A_log = A_log;
    a.dt_bias = dt_bias;
    a.lower_bound = lower_bound;
    a.cu_seqlens = cu_seqlens;
    a.cu_host = cu_host;
    a.num_seqs = cu_seqlens ? num_seqs : B;
    a.B = B; a.T = T; a.H = H; a.K = K; a.V = V;
    a.scale = scale;
    a.flags = flags;
    a.workspace = workspace;
    a.workspace_bytes = workspace_bytes;
    a.stages = 3;
}

extern "C" {

int gdn2_abi_version(void) { return GDN2_ABI_VERSION; }

const char *gdn2_status_string(int status)
{
    switch (status) {
    case GDN2_OK: return "ok";
    case GDN2_ERR_INVALID: return "invalid argument";
    case GDN2_ERR_UNSUPPORTED: return "unsupported shape, dtype or option";
    case GDN2_ERR_LAUNCH: return "kernel launch failed";
    case GDN2_ERR_WORKSPACE: return "workspace missing or too small";
    case GDN2_ERR_SCRATCH:
        return "the shape needs more than the static scratch array of gdn2_chunk_fwd_static "
               "holds (GDN2_STATIC_SCRATCH_BYTES = 72 MiB); use gdn2_chunk_fwd with a workspace";
    default: return "unknown status";
    }
}

int gdn2_recurrent_fwd_ex(const void *q, const void *k, const void *v, const void *g,
                          const void *b, const void *w, int io_dtype, int g_dtype, void *o,
                          const float *initial_state, int64_t initial_state_rows,
                          int64_t initial_state_row_stride, float *final_state,
                          int64_t final_state_rows, int64_t final_state_row_stride,
                          const float *A_log, const float *dt_bias, float lower_bound,
                          const int64_t *cu_seqlens, int num_seqs,
                          const void *ssm_state_indices, int indices_dtype,
                          int64_t indices_numel, int64_t indices_seq_stride,
                          const void *num_accepted_tokens, int accepted_dtype, int B, int T,
                          int H, int HV, int K, int V, float scale, unsigned flags,
                          void *stream)
{
    if (!valid_dtype(io_dtype) || !valid_dtype(g_dtype)) return GDN2_ERR_INVALID;
    if (B < 0 || T < 0 || H <= 0 || HV <= 0 || K <= 0 || V <= 0) return GDN2_ERR_INVALID;
    if (HV % H != 0) return GDN2_ERR_INVALID;
    if (flags & ~(GDN2_FLAG_L2NORM_QK | GDN2_FLAG_GATE_IN_KERNEL | GDN2_FLAG_LOWER_BOUND |
                  GDN2_FLAG_TRANSPOSE_STATE | GDN2_FLAG_INPLACE_FINAL_STATE | GDN2_FLAG_SIGMOID_BW))
        return GDN2_ERR_INVALID;
    if ((flags & GDN2_FLAG_LOWER_BOUND) && !(flags & GDN2_FLAG_GATE_IN_KERNEL))
        return GDN2_ERR_INVALID;
    if ((flags & GDN2_FLAG_GATE_IN_KERNEL) && !A_log) return GDN2_ERR_INVALID;
    if (K > 256 || (V % 4) != 0) return GDN2_ERR_UNSUPPORTED;
    if ((flags & GDN2_FLAG_TRANSPOSE_STATE) && (K % 4) != 0) return GDN2_ERR_UNSUPPORTED;
    int N = B;
    if (cu_seqlens) {
        if (B != 1 || num_seqs < 0) return GDN2_ERR_INVALID;
        N = num_seqs;
    }
    const int64_t ntok = static_cast<int64_t>(B) * T;
    if (ntok > 0 && (!q || !k || !v || !g || !b || !w || !o)) return GDN2_ERR_INVALID;
    // State rows: 16-byte aligned, non-overlapping heads.
    const int64_t slab = static_cast<int64_t>(HV) * K * V;
    const bool pooled = ssm_state_indices != nullptr;
    if (initial_state) {
        if (initial_state_row_stride < slab || (initial_state_row_stride % 4) != 0 ||
            initial_state_rows < 0 || (reinterpret_cast<uintptr_t>(initial_state) & 15) != 0)
            return GDN2_ERR_INVALID;
        if (!pooled && initial_state_rows < N) return GDN2_ERR_INVALID;
    }
    if (final_state) {
        if (final_state_row_stride < slab || (final_state_row_stride % 4) != 0 ||
            final_state_rows < 0 || (reinterpret_cast<uintptr_t>(final_state) & 15) != 0)
            return GDN2_ERR_INVALID;
        if (!pooled && final_state_rows < N) return GDN2_ERR_INVALID;
    }
    if (pooled) {
        if (indices_dtype != GDN2_DTYPE_I32 && indices_dtype != GDN2_DTYPE_I64) return GDN2_ERR_INVALID;
        if (indices_numel < 0 || indices_seq_stride < 0) return GDN2_ERR_INVALID;
        if (num_accepted_tokens && accepted_dtype != GDN2_DTYPE_I32 &&
            accepted_dtype != GDN2_DTYPE_I64)
            return GDN2_ERR_INVALID;
    }
    if (N == 0) return GDN2_OK;
    if (static_cast<int64_t>(N) * HV > 2147483647LL) return GDN2_ERR_UNSUPPORTED;

    RecurrentParams p;
    p.q = q; p.k = k; p.v = v; p.g = g; p.b = b; p.w = w; p.o = o;
    p.h0 = initial_state;
    p.ht = final_state;
    p.A_log = A_log;
    p.dt_bias = dt_bias;
    p.lower_bound = lower_bound;
    p.cu_seqlens = cu_seqlens;
    p.T = T; p.H = H; p.HV = HV; p.K = K; p.V = V;
    p.scale = scale;
    p.flags = flags;
    p.h0_rows = initial_state ? initial_state_rows : 0;
    p.h0_stride = initial_state_row_stride;
    p.ht_rows = final_state ? final_state_rows : 0;
    p.ht_stride = final_state_row_stride;
    p.state_indices = ssm_state_indices;
    p.accepted = pooled ? num_accepted_tokens : nullptr;
    p.idx_numel = pooled ? indices_numel : 0;
    p.idx_seq_stride = pooled ? indices_seq_stride : 0;
    p.idx_i64 = indices_dtype == GDN2_DTYPE_I64;
    p.acc_i64 = accepted_dtype == GDN2_DTYPE_I64;
    const hipError_t err =
        launch_recurrent_fwd(p, io_dtype, g_dtype, N, static_cast<hipStream_t>(stream));
    return err == hipSuccess ? GDN2_OK : GDN2_ERR_LAUNCH;
}

int gdn2_recurrent_fwd(const void *q, const void *k, const void *v, const void *g,
                       const void *b, const void *w, int io_dtype, int g_dtype, void *o,
                       const float *initial_state, float *final_state, const float *A_log,
                       const float *dt_bias, float lower_bound, const int64_t *cu_seqlens,
                       int num_seqs, int B, int T, int H, int HV, int K, int V, float scale,
                       unsigned flags, void *stream)
{
    if (flags & (GDN2_FLAG_TRANSPOSE_STATE | GDN2_FLAG_INPLACE_FINAL_STATE)) return GDN2_ERR_INVALID;
    const int64_t rows = cu_seqlens ? num_seqs : B;
    const int64_t slab = static_cast<int64_t>(HV) * K * V;
    return gdn2_recurrent_fwd_ex(q, k, v, g, b, w, io_dtype, g_dtype, o, initial_state, rows,
                                 slab, final_state, rows, slab, A_log, dt_bias, lower_bound,
                                 cu_seqlens, num_seqs, nullptr, GDN2_DTYPE_I64, 0, 0, nullptr,
                                 GDN2_DTYPE_I64, B, T, H, HV, K, V, scale, flags, stream);
}

int gdn2_short_conv_fwd(int ntensors, const void *const *x, const void *const *weight,
                        const void *const *bias, const void *const *cache_in,
                        void *const *cache_out, void *const *y, const int *dims, int io_dtype,
                        int B, int T, int W, int silu, void *stream)
{
    return gdn2_short_conv_fwd_ex(ntensors, x, nullptr, weight, bias, cache_in, cache_out, y, dims,
                                  io_dtype, B, T, W, silu, stream);
}

int gdn2_short_conv_fwd_ex(int ntensors, const void *const *x, const int64_t *x_row_stride,
                           const void *const *weight, const void *const *bias,
                           const void *const *cache_in, void *const *cache_out, void *const *y,
                           const int *dims, int io_dtype, int B, int T, int W, int silu, void *stream)
{
    if (!valid_dtype(io_dtype)) return GDN2_ERR_INVALID;
    if (ntensors < 1 || ntensors > 3 || !x || !weight || !y || !dims) return GDN2_ERR_INVALID;
    if (B < 0 || T < 0 || W < 1) return GDN2_ERR_INVALID;
    if (W > 8) return GDN2_ERR_UNSUPPORTED;
    ConvParams p;
    p.B = B; p.T = T; p.W = W;
    p.ncache = T == 1 ? W - 1 : (T < W - 1 ? T : W - 1);
    p.silu = silu != 0;
    int maxD = 0;
    for (int i = 0; i < 3; ++i) {
        const int j = i < ntensors ? i : 0;
        ConvTensor &c = p.t[i];
        c.D = dims[j];
        if (c.D <= 0) return GDN2_ERR_INVALID;
        c.ldx = x_row_stride ? x_row_stride[j] : c.D;
        if (c.ldx < c.D) return GDN2_ERR_INVALID;
        if (B * static_cast<int64_t>(T) > 0 && (!x[j] || !weight[j] || !y[j])) return GDN2_ERR_INVALID;
        c.x = x[j]; c.w = weight[j]; c.y = y[j];
        c.bias = bias ? bias[j] : nullptr;
        c.cache_in = cache_in ? cache_in[j] : nullptr;
        c.cache_out = cache_out ? cache_out[j] : nullptr;
        if (i < ntensors && c.D > maxD) maxD = c.D;
    }
    if (B == 0 || T == 0) return GDN2_OK;
    const hipError_t err = launch_short_conv(p, io_dtype, maxD, ntensors, static_cast<hipStream_t>(stream));
    return err == hipSuccess ? GDN2_OK : GDN2_ERR_LAUNCH;
}

int gdn2_gated_rmsnorm_fwd(const void *x, const void *z, const void *weight, int weight_dtype,
                           void *out, int io_dtype, int64_t rows, int N, float eps, void *stream)
{
    if (!valid_dtype(io_dtype) || !valid_dtype(weight_dtype)) return GDN2_ERR_INVALID;
    if (weight_dtype != io_dtype && weight_dtype != GDN2_DTYPE_F32) return GDN2_ERR_INVALID;
    if (rows < 0 || N <= 0) return GDN2_ERR_INVALID;
    if (N > 2048) return GDN2_ERR_UNSUPPORTED;
    if (rows == 0) return GDN2_OK;
    if (!x || !weight || !out) return GDN2_ERR_INVALID;  // z may be NULL: no gate
    if ((rows + 3) / 4 > 2147483647LL) return GDN2_ERR_UNSUPPORTED;
    NormParams p;
    p.x = x; p.z = z; p.weight = weight; p.out = out;
    p.rows = rows; p.N = N; p.eps = eps;
    p.w_f32 = weight_dtype == GDN2_DTYPE_F32 && io_dtype != GDN2_DTYPE_F32;
    const hipError_t err = launch_gated_rmsnorm(p, io_dtype, static_cast<hipStream_t>(stream));
    return err == hipSuccess ? GDN2_OK : GDN2_ERR_LAUNCH;
}

int gdn2_add_rms_norm_fwd(const void *x, const void *residual, void *sum_out, const void *weight,
                          int weight_dtype, void *out, int io_dtype, int64_t rows, int N, float eps,
                          void *stream)
{
    if (!valid_dtype(io_dtype) || !valid_dtype(weight_dtype)) return GDN2_ERR_INVALID;
    if (weight_dtype != io_dtype && weight_dtype != GDN2_DTYPE_F32) return GDN2_ERR_INVALID;
    if (rows < 0 || N <= 0) return GDN2_ERR_INVALID;
    if (rows == 0) return GDN2_OK;
    if (!x || !residual || !sum_out || !weight || !out) return GDN2_ERR_INVALID;
    // One vectorised pass: rows of 4..256 16-byte pieces (a power of two), 16-byte aligned.
    const int epv = io_dtype == GDN2_DTYPE_F32 ? 4 : 8;
    const int pieces = N / epv;
    const uintptr_t addr = reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(residual) |
                           reinterpret_cast<uintptr_t>(sum_out) | reinterpret_cast<uintptr_t>(out);
    if (N % epv != 0 || pieces < 4 || pieces > 256 || (pieces & (pieces - 1)) != 0 || (addr & 15) != 0)
        return GDN2_ERR_UNSUPPORTED;
    if (rows > 2147483647LL) return GDN2_ERR_UNSUPPORTED;
    NormParams p;
    p.x = x; p.z = nullptr; p.weight = weight; p.out = out;
    p.rows = rows; p.N = N; p.eps = eps;
    p.w_f32 = weight_dtype == GDN2_DTYPE_F32 && io_dtype != GDN2_DTYPE_F32;
    p.res = residual; p.sum_out = sum_out;
    const hipError_t err = launch_gated_rmsnorm(p, io_dtype, static_cast<hipStream_t>(stream));
    return err == hipSuccess ? GDN2_OK : GDN2_ERR_LAUNCH;
}

int gdn2_silu_mul_fwd(const void *ab, int64_t ab_row_stride, void *out, int io_dtype, int64_t rows,
                      int H, void *stream)
{
    if (!valid_dtype(io_dtype) || rows < 0 || H <= 0) return GDN2_ERR_INVALID;
    if (rows == 0) return GDN2_OK;
    if (!ab || !out || ab_row_stride < 2LL * H) return GDN2_ERR_INVALID;
    const int epv = io_dtype == GDN2_DTYPE_F32 ? 4 : 8;
    if (H % epv != 0 || ab_row_stride % epv != 0 ||
        ((reinterpret_cast<uintptr_t>(ab) | reinterpret_cast<uintptr_t>(out)) & 15) != 0)
        return GDN2_ERR_UNSUPPORTED;
    if ((rows * (H / epv) + 255) / 256 > 2147483647LL) return GDN2_ERR_UNSUPPORTED;
    SiluMulParams p;
    p.ab = ab; p.out = out; p.rows = rows; p.ld = ab_row_stride; p.H = H;
    const hipError_t err = launch_silu_mul(p, io_dtype, static_cast<hipStream_t>(stream));
    return err == hipSuccess ? GDN2_OK : GDN2_ERR_LAUNCH;
}

int gdn2_skinny_linear(const void *x, int64_t x_row_stride, const void *weight, int64_t weight_row_stride,
                       const void *bias, void *y, int64_t y_row_stride, int io_dtype, int M, int N, int K,
                       void *stream)
{
    if (!valid_dtype(io_dtype) || M < 0 || N < 0 || K < 0) return GDN2_ERR_INVALID;
    if (M == 0 || N == 0) return GDN2_OK;
    if (!x || !weight || !y || x_row_stride < K || weight_row_stride < K || y_row_stride < N) return GDN2_ERR_INVALID;
    if (!skinny_linear_supported(io_dtype, M, K)) return GDN2_ERR_UNSUPPORTED;
    if (((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(weight)) & 15) != 0 ||
        x_row_stride % 8 != 0 || weight_row_stride % 8 != 0)
        return GDN2_ERR_UNSUPPORTED;
    if (N > 2147483647 - 8) return GDN2_ERR_UNSUPPORTED;
    SkinnyParams p;
    p.x = x; p.w = weight; p.bias = bias; p.y = y;
    p.ldx = x_row_stride; p.ldw = weight_row_stride; p.ldy = y_row_stride;
    p.M = M; p.N = N; p.K = K;
    const hipError_t err = launch_skinny_linear(p, io_dtype, static_cast<hipStream_t>(stream));
    return err == hipSuccess ? GDN2_OK : GDN2_ERR_LAUNCH;
}

static int skinny_addnorm_impl(const void *x, int64_t x_row_stride, const void *residual,
                               int64_t residual_row_stride, void *sum_out, int64_t sum_row_stride,
                               const void *norm_weight, float eps, const void *weight, int64_t weight_row_stride,
                               const void *bias, void *y, int64_t y_row_stride, int io_dtype, int M, int N, int K,
                               int glu, void *stream)
{
    if (!valid_dtype(io_dtype) || M < 0 || N < 0 || K < 0) return GDN2_ERR_INVALID;
    if (M == 0 || N == 0) return GDN2_OK;
    if (glu && N % 2 != 0) return GDN2_ERR_INVALID;
    if (!x || !residual || !sum_out || !norm_weight || !weight || !y || x_row_stride < K ||
        residual_row_stride < K || sum_row_stride < K || weight_row_stride < K || y_row_stride < (glu ? N / 2 : N))
        return GDN2_ERR_INVALID;
    if (!skinny_linear_supported(io_dtype, M, K) || M > 4 || K > 2048) return GDN2_ERR_UNSUPPORTED;
    if (((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(residual) |
          reinterpret_cast<uintptr_t>(sum_out) | reinterpret_cast<uintptr_t>(weight) |
          reinterpret_cast<uintptr_t>(norm_weight)) & 15) != 0 ||
        x_row_stride % 8 != 0 || residual_row_stride % 8 != 0 || sum_row_stride % 8 != 0 || weight_row_stride % 8 != 0)
        return GDN2_ERR_UNSUPPORTED;
    if (N > 2147483647 - 8) return GDN2_ERR_UNSUPPORTED;
    SkinnyParams p;
    p.x = x; p.w = weight; p.bias = bias; p.y = y;
    p.ldx = x_row_stride; p.ldw = weight_row_stride; p.ldy = y_row_stride;
    p.M = M; p.N = N; p.K = K;
    p.norm = 1; p.res = residual; p.nw = norm_weight; p.sum_out = sum_out;
    p.ldres = residual_row_stride; p.ldsum = sum_row_stride; p.eps = eps;
    p.glu_out = glu;
    const hipError_t err = launch_skinny_linear(p, io_dtype, static_cast<hipStream_t>(stream));
    return err == hipSuccess ? GDN2_OK : GDN2_ERR_LAUNCH;
}

int gdn2_skinny_linear_addnorm(const void *x, int64_t x_row_stride, const void *residual,
                               int64_t residual_row_stride, void *sum_out, int64_t sum_row_stride,
                               const void *norm_weight, float eps, const void *weight, int64_t weight_row_stride,
                               const void *bias, void *y, int64_t y_row_stride, int io_dtype, int M, int N, int K,
                               void *stream)
{
    return skinny_addnorm_impl(x, x_row_stride, residual, residual_row_stride, sum_out, sum_row_stride, norm_weight,
                               eps, weight, weight_row_stride, bias, y, y_row_stride, io_dtype, M, N, K, 0, stream);
}

int gdn2_skinny_linear_addnorm_swiglu(const void *x, int64_t x_row_stride, const void *residual,
                                      int64_t residual_row_stride, void *sum_out, int64_t sum_row_stride,
                                      const void *norm_weight, float eps, const void *weight,
                                      int64_t weight_row_stride, const void *bias, void *y, int64_t y_row_stride,
                                      int io_dtype, int M, int N, int K, void *stream)
{
    return skinny_addnorm_impl(x, x_row_stride, residual, residual_row_stride, sum_out, sum_row_stride, norm_weight,
                               eps, weight, weight_row_stride, bias, y, y_row_stride, io_dtype, M, N, K, 1, stream);
}

int gdn2_small_linear_pair(const void *x0, int64_t x0_row_stride, const void *weight0, const void *bias0, void *y0,
                           int64_t y0_row_stride, int N0, const void *x1, int64_t x1_row_stride,
                           const void *weight1, const void *bias1, void *y1, int64_t y1_row_stride, int N1,
                           int io_dtype, int M, int K, void *stream)
{
    if (!valid_dtype(io_dtype) || M < 0 || K < 1 || N0 < 0 || N1 < 0) return GDN2_ERR_INVALID;
    if (M == 0 || (N0 == 0 && N1 == 0)) return GDN2_OK;
    if (!small_linear_supported(io_dtype, M, K)) return GDN2_ERR_UNSUPPORTED;
    SmallLinearParams p;
    p.M = M; p.K = K;
    int n = 0;
    const void *xs[2] = {x0, x1}, *ws[2] = {weight0, weight1}, *bs[2] = {bias0, bias1};
    void *ys[2] = {y0, y1};
    const int64_t lx[2] = {x0_row_stride, x1_row_stride}, ly[2] = {y0_row_stride, y1_row_stride};
    const int Ns[2] = {N0, N1};
    for (int i = 0; i < 2; ++i) {
        if (Ns[i] == 0) continue;
        if (!xs[i] || !ws[i] || !ys[i] || lx[i] < K || ly[i] < Ns[i]) return GDN2_ERR_INVALID;
        if (((reinterpret_cast<uintptr_t>(xs[i]) | reinterpret_cast<uintptr_t>(ws[i])) & 15) != 0 || lx[i] % 8 != 0)
            return GDN2_ERR_UNSUPPORTED;
        SmallLinearProblem &q = p.prob[n++];
        q.x = xs[i]; q.w = ws[i]; q.bias = bs[i]; q.y = ys[i]; q.ldx = lx[i]; q.ldy = ly[i]; q.N = Ns[i];
    }
    const hipError_t err = launch_small_linear(p, n, io_dtype, static_cast<hipStream_t>(stream));
    return err == hipSuccess ? GDN2_OK : GDN2_ERR_LAUNCH;
}

size_t gdn2_argmax_rows_workspace_size(int64_t rows, int64_t n, int io_dtype)
{
    if (!valid_dtype(io_dtype) || rows < 1 || n < 1 || rows > 65535) return 0;
    const int s = argmax_splits(n, io_dtype);
    return s > 1 ? static_cast<size_t>(rows) * s * (sizeof(int64_t) + sizeof(float)) : 0;
}

int gdn2_argmax_rows(const void *x, int64_t x_row_stride, int io_dtype, int64_t rows, int64_t n, int64_t *out,
                     int64_t out_stride, void *workspace, size_t workspace_bytes, void *stream)
{
    if (!valid_dtype(io_dtype) || rows < 0 || n < 1) return GDN2_ERR_INVALID;
    if (rows == 0) return GDN2_OK;
    if (!x || !out || x_row_stride < n || out_stride < 1) return GDN2_ERR_INVALID;
    const int es = io_dtype == GDN2_DTYPE_F32 ? 4 : 2;
    if ((reinterpret_cast<uintptr_t>(x) & 15) != 0 || (x_row_stride * es) % 16 != 0) return GDN2_ERR_UNSUPPORTED;
    if (rows > 2147483647LL) return GDN2_ERR_UNSUPPORTED;
    ArgmaxParams p;
    p.x = x; p.ld = x_row_stride; p.rows = rows; p.n = n; p.out = out; p.out_stride = out_stride;
    p.splits = 1; p.pps = 0; p.part_v = nullptr; p.part_i = nullptr;
    const size_t need = gdn2_argmax_rows_workspace_size(rows, n, io_dtype);
    if (workspace && need > 0) {
        if (workspace_bytes < need || (reinterpret_cast<uintptr_t>(workspace) & 7) != 0) return GDN2_ERR_WORKSPACE;
        p.splits = argmax_splits(n, io_dtype);
        const int64_t pieces = n / (io_dtype == GDN2_DTYPE_F32 ? 4 : 8);
        p.pps = (pieces + p.splits - 1) / p.splits;
        p.part_i = static_cast<int64_t *>(workspace);
        p.part_v = reinterpret_cast<float *>(p.part_i + rows * p.splits);
    }
    const hipError_t err = launch_argmax_rows(p, io_dtype, static_cast<hipStream_t>(stream));
    return err == hipSuccess ? GDN2_OK : GDN2_ERR_LAUNCH;
}

size_t gdn2_attn_decode_workspace_size(int B, int G, int qpk, int D, int64_t max_len)
{
    if (B < 0 || G < 0 || qpk < 1 || D < 1 || max_len < 1) return 0;
    return attn_decode_workspace_floats(B, G, qpk, D, max_len) * sizeof(float);
}

int gdn2_attn_decode(const void *qkv, const float *cos, const float *sin, int rope_pairs, int64_t rope_row_stride,
                     const int64_t *pos, void *k_cache, void *v_cache, void *out, int io_dtype, int B, int G,
                     int qpk, int D, int64_t max_len, float scale, void *workspace, size_t workspace_bytes,
                     void *stream)
{
    if (!valid_dtype(io_dtype) || B < 0 || G < 0 || qpk < 1 || D < 1 || max_len < 1) return GDN2_ERR_INVALID;
    if (B == 0 || G == 0) return GDN2_OK;
    if (!qkv || !pos || !k_cache || !v_cache || !out) return GDN2_ERR_INVALID;
    if (rope_pairs < 0 || 2 * rope_pairs > D) return GDN2_ERR_INVALID;
    if (rope_pairs > 0 && (!cos || !sin)) return GDN2_ERR_INVALID;
    if (rope_row_stride < 0 || (rope_row_stride > 0 && rope_row_stride < rope_pairs)) return GDN2_ERR_INVALID;
    if (!attn_decode_supported(io_dtype, qpk, D)) return GDN2_ERR_UNSUPPORTED;
    if ((reinterpret_cast<uintptr_t>(k_cache) | reinterpret_cast<uintptr_t>(v_cache)) & 15) return GDN2_ERR_UNSUPPORTED;
    if (static_cast<int64_t>(B) * G > 2147483647LL || max_len > 2147483647LL) return GDN2_ERR_UNSUPPORTED;
    AttnDecodeParams p;
    p.qkv = qkv; p.cos = cos; p.sin = sin;
    p.rope_pairs = rope_pairs;
    p.rope_stride = rope_row_stride;
    p.pos = pos; p.k_cache = k_cache; p.v_cache = v_cache; p.out = out;
    p.max_len = max_len; p.B = B; p.G = G; p.qpk = qpk; p.D = D; p.scale = scale;
    p.splits = attn_decode_splits(max_len);
    p.part = static_cast<float *>(workspace);
    if (p.splits > 1 && (!workspace || workspace_bytes < gdn2_attn_decode_workspace_size(B, G, qpk, D, max_len)))
        return GDN2_ERR_WORKSPACE;
    const hipError_t err = launch_attn_decode(p, io_dtype, static_cast<hipStream_t>(stream));
    return err == hipSuccess ? GDN2_OK : GDN2_ERR_LAUNCH;
}

size_t gdn2_gate_bwd_workspace_size(int64_t tokens, int H, int K, int has_dt_bias)
{
    if (tokens < 0 || H <= 0 || K <= 0 || K > 256) return 0;
    return gate_bwd_workspace_bytes(tokens, H, K, has_dt_bias != 0);
}

static int check_gate_args(const void *g_raw, int g_dtype, const float *A_log, unsigned flags, int64_t tokens,
                           int H, int K)
{
    if (!valid_dtype(g_dtype) || tokens < 0 || H <= 0 || K <= 0) return GDN2_ERR_INVALID;
    if (flags & ~GDN2_FLAG_LOWER_BOUND) return GDN2_ERR_INVALID;
    if (K > 256) return GDN2_ERR_UNSUPPORTED;
    if (!A_log || (tokens > 0 && !g_raw)) return GDN2_ERR_INVALID;
    return GDN2_OK;
}

int gdn2_gate_fwd(const void *g_raw, int g_dtype, const float *A_log, const float *dt_bias, float lower_bound,
                  unsigned flags, float *y, int64_t tokens, int H, int K, void *stream)
{
    const int st = check_gate_args(g_raw, g_dtype, A_log, flags, tokens, H, K);
    if (st != GDN2_OK) return st;
    if (tokens > 0 && !y) return GDN2_ERR_INVALID;
    return launch_gate_fwd(g_raw, g_dtype, A_log, dt_bias, lower_bound, flags, y, tokens, H, K,
                           static_cast<hipStream_t>(stream));
}

int gdn2_gate_bwd(const void *g_raw, int g_dtype, const float *A_log, const float *dt_bias, float lower_bound,
                  unsigned flags, const float *dy, void *dg_raw, float *dA_log, float *ddt_bias, int64_t tokens,
                  int H, int K, void *workspace, size_t workspace_bytes, void *stream)
{
    const int st = check_gate_args(g_raw, g_dtype, A_log, flags, tokens, H, K);
    if (st != GDN2_OK) return st;
    if ((tokens > 0 && (!dy || !dg_raw)) || !dA_log || (dt_bias != nullptr) != (ddt_bias != nullptr))
        return GDN2_ERR_INVALID;
    if (!workspace || workspace_bytes < gate_bwd_workspace_bytes(tokens, H, K, dt_bias != nullptr))
        return GDN2_ERR_WORKSPACE;
    return launch_gate_bwd(g_raw, g_dtype, A_log, dt_bias, lower_bound, flags, dy, dg_raw, dA_log, ddt_bias,
                           tokens, H, K, workspace, static_cast<hipStream_t>(stream));
}

size_t gdn2_short_conv_bwd_workspace_size(int B, int T, int D, int conv_width)
{
    if (B < 0 || T < 0 || D < 0 || conv_width < 1 || conv_width > 8) return 0;
    return static_cast<size_t>(conv_bwd_partial_floats(B, T, D, conv_width)) * sizeof(float);
}

int gdn2_short_conv_bwd(const void *x, int64_t x_row_stride, const void *weight, const void *bias,
                        const void *dy, void *dx, void *dweight, void *dbias, int io_dtype, int B,
                        int T, int D, int conv_width, int silu, void *workspace,
                        size_t workspace_bytes, void *stream)
{
    if (!valid_dtype(io_dtype) || B < 0 || T < 0 || D < 0) return GDN2_ERR_INVALID;
    if (conv_width < 1 || conv_width > 8) return GDN2_ERR_UNSUPPORTED;
    if (static_cast<int64_t>(B) * T * D == 0) return GDN2_OK;
    if (!x || !weight || !dy || !dx || !dweight || (dbias && !bias) || x_row_stride < D)
        return GDN2_ERR_INVALID;
    if (static_cast<int64_t>(B) * ((T + 31) / 32) > 65535) return GDN2_ERR_UNSUPPORTED;  // grid.y
    if (!workspace || workspace_bytes < gdn2_short_conv_bwd_workspace_size(B, T, D, conv_width))
        return GDN2_ERR_WORKSPACE;
    ConvBwdParams p;
    p.x = x; p.w = weight; p.bias = bias; p.dy = dy; p.dx = dx; p.dw = dweight; p.dbias = dbias;
    p.part = static_cast<float *>(workspace);
    p.B = B; p.T = T; p.D = D; p.W = conv_width; p.ldx = x_row_stride; p.silu = silu != 0;
    const hipError_t err = launch_short_conv_bwd(p, io_dtype, static_cast<hipStream_t>(stream));
    return err == hipSuccess ? GDN2_OK : GDN2_ERR_LAUNCH;
}

size_t gdn2_gated_rmsnorm_bwd_workspace_size(int64_t rows, int N)
{
    if (rows < 0 || N <= 0 || N > 256) return 0;
    return static_cast<size_t>(norm_bwd_blocks(rows) * N) * sizeof(float);
}

int gdn2_gated_rmsnorm_bwd(const void *x, const void *z, const void *weight, int weight_dtype,
                           const void *dy, void *dx, void *dz, void *dweight, int io_dtype,
                           int64_t rows, int N, float eps, void *workspace, size_t workspace_bytes,
                           void *stream)
{
    if (!valid_dtype(io_dtype) || !valid_dtype(weight_dtype)) return GDN2_ERR_INVALID;
    if (weight_dtype != io_dtype && weight_dtype != GDN2_DTYPE_F32) return GDN2_ERR_INVALID;
    if (rows < 0 || N <= 0) return GDN2_ERR_INVALID;
    if (N > 256) return GDN2_ERR_UNSUPPORTED;
    if (rows == 0) return GDN2_OK;
    if (!x || !z || !weight || !dy || !dx || !dz || !dweight) return GDN2_ERR_INVALID;
    if (!workspace || workspace_bytes < gdn2_gated_rmsnorm_bwd_workspace_size(rows, N))
        return GDN2_ERR_WORKSPACE;
    NormBwdParams p;
    p.x = x; p.z = z; p.weight = weight; p.dy = dy; p.dx = dx; p.dz = dz; p.dweight = dweight;
    p.part = static_cast<float *>(workspace);
    p.rows = rows; p.N = N; p.eps = eps;
    p.w_f32 = weight_dtype == GDN2_DTYPE_F32;
    const hipError_t err = launch_gated_rmsnorm_bwd(p, io_dtype, static_cast<hipStream_t>(stream));
    return err == hipSuccess ? GDN2_OK : GDN2_ERR_LAUNCH;
}

int gdn2_decode_fused(const void *const raw_qkv[3], const int64_t ld_qkv[3], const void *g,
                      int64_t ldg, int g_dtype, const void *b, int64_t ldb, const void *w,
                      int64_t ldw, const void *const conv_weight[3], const void *const conv_bias[3],
                      int conv_width, const void *const conv_cache_in[3],
                      void *const conv_cache_out[3], const float *initial_state,
                      int64_t initial_state_row_stride, float *final_state,
                      int64_t final_state_row_stride, const float *A_log, const float *dt_bias,
                      float lower_bound, const void *gate, int64_t ld_gate,
                      const void *norm_weight, int norm_weight_dtype, float eps, void *o,
                      int io_dtype, int N, int H, int K, int V, float scale, unsigned flags,
                      void *stream)
{
    if (!valid_dtype(io_dtype) || !valid_dtype(g_dtype)) return GDN2_ERR_INVALID;
    if (g_dtype != GDN2_DTYPE_F32 && g_dtype != io_dtype) return GDN2_ERR_UNSUPPORTED;
    if (N < 0 || H <= 0 || K <= 0 || V <= 0) return GDN2_ERR_INVALID;
    if (K != V || (K != 64 && K != 128) || conv_width != 4) return GDN2_ERR_UNSUPPORTED;
    if (flags & ~(GDN2_FLAG_L2NORM_QK | GDN2_FLAG_GATE_IN_KERNEL | GDN2_FLAG_LOWER_BOUND |
                  GDN2_FLAG_SIGMOID_BW))
        return GDN2_ERR_INVALID;
    if ((flags & GDN2_FLAG_LOWER_BOUND) && !(flags & GDN2_FLAG_GATE_IN_KERNEL)) return GDN2_ERR_INVALID;
    if ((flags & GDN2_FLAG_GATE_IN_KERNEL) && !A_log) return GDN2_ERR_INVALID;
    if (static_cast<int64_t>(N) * H > 2147483647LL) return GDN2_ERR_UNSUPPORTED;
    if (N == 0) return GDN2_OK;
    if (!raw_qkv || !ld_qkv || !conv_weight || !g || !b || !w || !o) return GDN2_ERR_INVALID;
    const int64_t HD = static_cast<int64_t>(H) * K;
    DecodeFusedParams p;
    for (int t = 0; t < 3; ++t) {
        if (!raw_qkv[t] || !conv_weight[t] || ld_qkv[t] < HD) return GDN2_ERR_INVALID;
        p.x[t] = raw_qkv[t];
        p.ldx[t] = ld_qkv[t];
        p.cw[t] = conv_weight[t];
        p.cb[t] = conv_bias ? conv_bias[t] : nullptr;
        p.cin[t] = conv_cache_in ? conv_cache_in[t] : nullptr;
        p.cout[t] = conv_cache_out ? conv_cache_out[t] : nullptr;
    }
    if (ldg < HD || ldb < HD || ldw < HD) return GDN2_ERR_INVALID;
    if (gate && (ld_gate < HD || !norm_weight)) return GDN2_ERR_INVALID;
    if (norm_weight && norm_weight_dtype != GDN2_DTYPE_F32 && norm_weight_dtype != io_dtype)
        return GDN2_ERR_INVALID;
    const int64_t slab = HD * V;
    for (const void *st : {static_cast<const void *>(initial_state), static_cast<const void *>(final_state)})
        if (st && (reinterpret_cast<uintptr_t>(st) % 16)) return GDN2_ERR_INVALID;
    if (initial_state && (initial_state_row_stride < slab || initial_state_row_stride % 4))
        return GDN2_ERR_INVALID;
    if (final_state && (final_state_row_stride < slab || final_state_row_stride % 4))
        return GDN2_ERR_INVALID;
    p.g = g; p.b = b; p.w = w;
    p.ldg = ldg; p.ldb = ldb; p.ldw = ldw;
    p.h0 = initial_state;
    p.ht = final_state;
    p.h0_stride = initial_state_row_stride;
    p.ht_stride = final_state_row_stride;
    p.A_log = A_log;
    p.dt_bias = dt_bias;
    p.lower_bound = lower_bound;
    p.z = gate;
    p.ldz = ld_gate;
    p.nw = norm_weight;
    p.nw_f32 = norm_weight && norm_weight_dtype == GDN2_DTYPE_F32 && io_dtype != GDN2_DTYPE_F32;
    p.eps = eps;
    p.o = o;
    p.N = N; p.H = H; p.D = K;
    p.scale = scale;
    p.flags = flags;
    const hipError_t err = launch_decode_fused(p, io_dtype, g_dtype, static_cast<hipStream_t>(stream));
    return err == hipSuccess ? GDN2_OK : GDN2_ERR_LAUNCH;
}

size_t gdn2_chunk_fwd_workspace_size(int B, int T, int H, int K, int V, int io_dtype,
                                     const int64_t *cu_seqlens_host, int num_seqs)
{
    if (B < 0 || T < 0 || H <= 0 || K <= 0 || V <= 0 || !valid_dtype(io_dtype)) return 0;
    return chunk_fwd_workspace_bytes(B, T, H, K, V, io_dtype, cu_seqlens_host, num_seqs);
}

int gdn2_chunk_fwd(const void *q, const void *k, const void *v, const void *g, const void *b,
                   const void *w, int io_dtype, int g_dtype, void *o,
                   const float *initial_state, float *final_state, const float *A_log,
                   const float *dt_bias, float lower_bound, const int64_t *cu_seqlens,
                   const int64_t *cu_seqlens_host, int num_seqs, int B, int T, int H, int K,
                   int V, float scale, unsigned flags, void *workspace,
                   size_t workspace_bytes, void *stream)
{
    ChunkFwdArgs a;
    const int st = check_chunk_args(io_dtype, g_dtype, cu_seqlens, cu_seqlens_host, num_seqs, B,
                                    T, H, K, V, flags, A_log);
    if (st != GDN2_OK) return st;
    if (static_cast<int64_t>(B) * T > 0 && (!q || !k || !v || !g || !b || !w || !o))
        return GDN2_ERR_INVALID;
    fill_chunk_args(a, q, k, v, g, b, w, o, initial_state, final_state, A_log, dt_bias,
                    lower_bound, cu_seqlens, cu_seqlens_host, num_seqs, B, T, H, K, V, scale,
                    flags, workspace, workspace_bytes);
    a.stages = 3;
    return launch_chunk_fwd(a, io_dtype, g_dtype, static_cast<hipStream_t>(stream));
}

int gdn2_chunk_fwd_gated_norm(const void *q, const void *k, const void *v, const void *g,
                              const void *b, const void *w, int io_dtype, int g_dtype, void *o,
                              const void *gate, int64_t ld_gate, const void *norm_weight, float eps,
                              const float *initial_state, float *final_state, const float *A_log,
                              const float *dt_bias, float lower_bound, const int64_t *cu_seqlens,
                              const int64_t *cu_seqlens_host, int num_seqs, int B, int T, int H,
                              int K, int V, float scale, unsigned flags, void *workspace,
                              size_t workspace_bytes, void *stream)
{
    ChunkFwdArgs a;
    const int st = check_chunk_args(io_dtype, g_dtype, cu_seqlens, cu_seqlens_host, num_seqs, B,
                                    T, H, K, V, flags, A_log);
    if (st != GDN2_OK) return st;
    if (flags & GDN2_FLAG_SAVE_FOR_BWD) return GDN2_ERR_INVALID;  // an inference epilogue
    if (io_dtype != GDN2_DTYPE_BF16 || (V != 16 && V != 32 && V != 64)) return GDN2_ERR_UNSUPPORTED;
    if (static_cast<int64_t>(B) * T > 0 &&
        (!q || !k || !v || !g || !b || !w || !o || !gate || !norm_weight))
        return GDN2_ERR_INVALID;
    // 8-byte gate and output accesses: 4-value groups of every row.
    if (ld_gate < static_cast<int64_t>(H) * V || (ld_gate % 4) != 0 ||
        (reinterpret_cast<uintptr_t>(gate) % 8) != 0 || (reinterpret_cast<uintptr_t>(o) % 8) != 0)
        return GDN2_ERR_INVALID;
    fill_chunk_args(a, q, k, v, g, b, w, o, initial_state, final_state, A_log, dt_bias,
                    lower_bound, cu_seqlens, cu_seqlens_host, num_seqs, B, T, H, K, V, scale,
                    flags, workspace, workspace_bytes);
    a.stages = 3;
    a.z = gate;
    a.ldz = ld_gate;
    a.nw = norm_weight;
    a.eps = eps;
    return launch_chunk_fwd(a, io_dtype, g_dtype, static_cast<hipStream_t>(stream));
}

int gdn2_chunk_fwd_conv(const void *q, int64_t ld_q, const void *k, int64_t ld_k, const void *v, int64_t ld_v,
                        const void *conv_q, const void *conv_k, const void *conv_v, int conv_width,
                        int conv_silu, const void *g, const void *b, const void *w, int io_dtype,
                        int g_dtype, void *o, const void *gate, int64_t ld_gate,
                        const void *norm_weight, float eps, const float *initial_state,
                        float *final_state, const float *A_log, const float *dt_bias, float lower_bound,
                        const int64_t *cu_seqlens, const int64_t *cu_seqlens_host, int num_seqs, int B,
                        int T, int H, int K, int V, float scale, unsigned flags, void *workspace,
                        size_t workspace_bytes, void *stream)
{
    ChunkFwdArgs a;
    const int st = check_chunk_args(io_dtype, g_dtype, cu_seqlens, cu_seqlens_host, num_seqs, B,
                                    T, H, K, V, flags, A_log);
    if (st != GDN2_OK) return st;
    if (flags & GDN2_FLAG_SAVE_FOR_BWD) return GDN2_ERR_INVALID;  // an inference prologue
    if (conv_width != 4 || (conv_silu != 0 && conv_silu != 1)) return GDN2_ERR_UNSUPPORTED;
    if (io_dtype != GDN2_DTYPE_BF16 || (K != 32 && K != 64 && K != 128) || V % 16 != 0)
        return GDN2_ERR_UNSUPPORTED;
    if (gate && V != 16 && V != 32 && V != 64) return GDN2_ERR_UNSUPPORTED;
    if (static_cast<int64_t>(B) * T > 0 &&
        (!q || !k || !v || !g || !b || !w || !o || !conv_q || !conv_k || !conv_v || (gate && !norm_weight)))
        return GDN2_ERR_INVALID;
    // 16-byte row pieces of q, k, v, w and the taps.
    auto a16 = [](const void *x) { return (reinterpret_cast<uintptr_t>(x) % 16) == 0; };
    if (ld_q < static_cast<int64_t>(H) * K || ld_k < static_cast<int64_t>(H) * K ||
        ld_v < static_cast<int64_t>(H) * V || ld_q % 8 || ld_k % 8 || ld_v % 8 || !a16(q) || !a16(k) ||
        !a16(v) || !a16(w) || !a16(b) || !a16(g) || !a16(conv_q) || !a16(conv_k) || !a16(conv_v))
        return GDN2_ERR_INVALID;
    if (gate && (ld_gate < static_cast<int64_t>(H) * V || (ld_gate % 4) != 0 ||
                 (reinterpret_cast<uintptr_t>(gate) % 8) != 0 || (reinterpret_cast<uintptr_t>(o) % 8) != 0))
        return GDN2_ERR_INVALID;
    fill_chunk_args(a, q, k, v, g, b, w, o, initial_state, final_state, A_log, dt_bias,
                    lower_bound, cu_seqlens, cu_seqlens_host, num_seqs, B, T, H, K, V, scale,
                    flags, workspace, workspace_bytes);
    a.stages = 3;
    a.conv_w[0] = conv_q;
    a.conv_w[1] = conv_k;
    a.conv_w[2] = conv_v;
    a.ldq = ld_q;
    a.ldk = ld_k;
    a.ldv = ld_v;
    a.conv_silu = conv_silu;
    if (gate) {
        a.z = gate;
        a.ldz = ld_gate;
        a.nw = norm_weight;
        a.eps = eps;
    }
    return launch_chunk_fwd(a, io_dtype, g_dtype, static_cast<hipStream_t>(stream));
}

int gdn2_chunk_fwd_prep(const void *q, const void *k, const void *g, const void *b,
                        int io_dtype, int g_dtype, const float *A_log, const float *dt_bias,
                        float lower_bound, const int64_t *cu_seqlens,
                        const int64_t *cu_seqlens_host, int num_seqs, int B, int T, int H,
                        int K, int V, float scale, unsigned flags, void *workspace,
                        size_t workspace_bytes, void *stream)
{
    ChunkFwdArgs a;
    const int st = check_chunk_args(io_dtype, g_dtype, cu_seqlens, cu_seqlens_host, num_seqs, B,
                                    T, H, K, V, flags, A_log);
    if (st != GDN2_OK) return st;
    // The separate scan entry point has no flags, so w could not be activated there.
    if (flags & GDN2_FLAG_SIGMOID_BW) return GDN2_ERR_INVALID;
    if (static_cast<int64_t>(B) * T > 0 && (!q || !k || !g || !b)) return GDN2_ERR_INVALID;
    fill_chunk_args(a, q, k, nullptr, g, b, nullptr, nullptr, nullptr, nullptr, A_log, dt_bias,
                    lower_bound, cu_seqlens, cu_seqlens_host, num_seqs, B, T, H, K, V, scale,
                    flags, workspace, workspace_bytes);
    a.stages = 1;
    return launch_chunk_fwd(a, io_dtype, g_dtype, static_cast<hipStream_t>(stream));
}

int gdn2_chunk_fwd_scan(const void *v, const void *w, int io_dtype, void *o,
                        const float *initial_state, float *final_state,
                        const int64_t *cu_seqlens, const int64_t *cu_seqlens_host, int num_seqs,
                        int B, int T, int H, int K, int V, void *workspace,
                        size_t workspace_bytes, void *stream)
{
    ChunkFwdArgs a;
    const int st = check_chunk_args(io_dtype, GDN2_DTYPE_F32, cu_seqlens, cu_seqlens_host,
                                    num_seqs, B, T, H, K, V, 0u, nullptr);
    if (st != GDN2_OK) return st;
    if (static_cast<int64_t>(B) * T > 0 && (!v || !w || !o)) return GDN2_ERR_INVALID;
    fill_chunk_args(a, nullptr, nullptr, v, nullptr, nullptr, w, o, initial_state, final_state,
                    nullptr, nullptr, 0.f, cu_seqlens, cu_seqlens_host, num_seqs, B, T, H, K, V,
                    1.f, 0u, workspace, workspace_bytes);
    a.stages = 2;
    return launch_chunk_fwd(a, io_dtype, GDN2_DTYPE_F32, static_cast<hipStream_t>(stream));
}

size_t gdn2_chunk_train_workspace_size(int B, int T, int H, int K, int V, int io_dtype,
                                       const int64_t *cu_seqlens_host, int num_seqs)
{
    if (B < 0 || T < 0 || H <= 0 || K <= 0 || V <= 0 || !valid_dtype(io_dtype)) return 0;
    return chunk_train_workspace_bytes(B, T, H, K, V, io_dtype, cu_seqlens_host, num_seqs);
}

int gdn2_chunk_states(const void *saved, size_t saved_bytes, int io_dtype, void *out, int transpose,
                      const int64_t *cu_seqlens_host, int num_seqs, int B, int T, int H, int K,
                      int V, void *stream)
{
    if (!valid_dtype(io_dtype) || B < 0 || T < 0 || H <= 0 || K <= 0 || V <= 0) return GDN2_ERR_INVALID;
    if (cu_seqlens_host && (B != 1 || num_seqs < 0)) return GDN2_ERR_INVALID;
    const bool wide = chunk_wide(K, io_dtype);
    if (!wide && !chunk_k_supported(K, io_dtype)) return GDN2_ERR_UNSUPPORTED;
    const int64_t nc = count_chunks(B, T, cu_seqlens_host, num_seqs);
    if (nc == 0) return GDN2_OK;
    if (!saved || !out) return GDN2_ERR_INVALID;
    if (wide) {
        if (saved_bytes < wide_train_workspace_bytes(B, T, H, K, V, cu_seqlens_host, num_seqs))
            return GDN2_ERR_WORKSPACE;
        const hipError_t err = launch_chunk_states_wide(saved, out, transpose != 0, nc, H, K, V,
                                                        static_cast<hipStream_t>(stream));
        return err == hipSuccess ? GDN2_OK : GDN2_ERR_LAUNCH;
    }
    const TrainLayout tl = train_layout(nc, H, K, V, io_dtype);
    if (saved_bytes < static_cast<size_t>(tl.total)) return GDN2_ERR_WORKSPACE;
    const hipError_t err = launch_chunk_states(static_cast<const unsigned char *>(saved) + tl.hs, io_dtype, out,
                                               transpose != 0, nc, H, K, V, static_cast<hipStream_t>(stream));
    return err == hipSuccess ? GDN2_OK : GDN2_ERR_LAUNCH;
}

size_t gdn2_chunk_bwd_workspace_size(int B, int T, int H, int K, int V, int io_dtype,
                                     const int64_t *cu_seqlens_host, int num_seqs)
{
    if (B < 0 || T < 0 || H <= 0 || K <= 0 || V <= 0 || !valid_dtype(io_dtype)) return 0;
    return chunk_bwd_workspace_bytes(B, T, H, K, V, io_dtype, cu_seqlens_host, num_seqs);
}

int gdn2_chunk_bwd(const void *q, const void *k, const void *v, const void *g, const void *b,
                   const void *w, int io_dtype, int g_dtype, const void *dout,
                   const float *dht, void *dq, void *dk, void *dv, void *dg, void *db, void *dw,
                   float *dh0, const int64_t *cu_seqlens, const int64_t *cu_seqlens_host,
                   int num_seqs, int B, int T, int H, int K, int V, float scale,
                   unsigned flags, const void *saved, size_t saved_bytes, void *workspace,
                   size_t workspace_bytes, void *stream)
{
    const int st = check_chunk_args(io_dtype, g_dtype, cu_seqlens, cu_seqlens_host, num_seqs, B,
                                    T, H, K, V, flags & ~GDN2_FLAG_SAVE_FOR_BWD, nullptr);
    if (st != GDN2_OK) return st;
    if (flags & (GDN2_FLAG_GATE_IN_KERNEL | GDN2_FLAG_LOWER_BOUND)) return GDN2_ERR_UNSUPPORTED;
    if (static_cast<int64_t>(B) * T > 0 &&
        (!q || !k || !v || !g || !b || !w || !dout || !dq || !dk || !dv || !dg || !db || !dw))
        return GDN2_ERR_INVALID;
    ChunkBwdArgs a;
    a.q = q; a.k = k; a.v = v; a.g = g; a.b = b; a.w = w; a.dout = dout;
    a.dht = dht;
    a.dq = dq; a.dk = dk; a.dv = dv; a.dg = dg; a.db = db; a.dw = dw;
    a.dh0 = dh0;
    a.cu_seqlens = cu_seqlens;
    a.cu_host = cu_seqlens_host;
    a.num_seqs = cu_seqlens ? num_seqs : B;
    a.B = B; a.T = T; a.H = H; a.K = K; a.V = V;
    a.scale = scale;
    a.flags = flags;
    a.saved = saved;
    a.saved_bytes = saved_bytes;
    a.workspace = workspace;
    a.workspace_bytes = workspace_bytes;
    return launch_chunk_bwd(a, io_dtype, g_dtype, static_cast<hipStream_t>(stream));
}

}  // extern "C"
