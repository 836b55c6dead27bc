// Internal host-side interfaces between the C ABI (gdn2_api.hip) and the
// kernel translation units.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include <atomic>

namespace gdn2 {

// Workgroups of `kern` (at `threads` per workgroup) that the current device
// holds at once: occupancy per CU x CUs, looked up once per device and kept in
// `cache` (one per kernel instantiation, zero = not yet known).  The entries
// are atomics, so host threads that launch together for the first time may
// both compute the value and store the same result.
template <typename Kern>
hipError_t resident_slots(Kern kern, int threads, std::atomic<int> (&cache)[64], int *slots)
{
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    int n = dev < 64 ? cache[dev].load(std::memory_order_relaxed) : 0;
    if (n == 0) {
        int cus = 0, per_cu = 0;
        e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev);
        if (e != hipSuccess) return e;
        e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kern, threads, 0);
        if (e != hipSuccess) return e;
        n = (cus > 0 ? cus : 1) * (per_cu > 0 ? per_cu : 1);
        if (dev < 64) cache[dev].store(n, std::memory_order_relaxed);
    }
    *slots = n;
    return hipSuccess;
}

struct RecurrentParams {
    const void *q, *k, *v, *g, *b, *w;
    void *o;
    const float *h0;
    float *ht;
    const float *A_log;
    const float *dt_bias;
    float lower_bound;
    const int64_t *cu_seqlens;
    int T, H, HV, K, V;
    float scale;
    unsigned flags;
    // State rows: row r of a state array starts at base + r * stride (floats);
    // row indices outside [0, rows) are padding (read as zero, not stored).
    int64_t h0_rows, h0_stride, ht_rows, ht_stride;
    // Continuous batching / speculative decoding (fused_recurrent_gdn2.py:215-224,
    // 311-326): sequence n, position t uses slot state_indices[n * idx_seq_stride + t].
    const void *state_indices;  // NULL = no state pool
    const void *accepted;       // num_accepted_tokens, NULL = not speculative
    int64_t idx_numel, idx_seq_stride;
    int idx_i64, acc_i64;
};

hipError_t launch_recurrent_fwd(const RecurrentParams &p, int io_dtype, int g_dtype, int N,
                                hipStream_t stream);

// Fused module decode step (one token per sequence, HV == H, K == V == D):
// short convolution of the raw q / k / v projections with the conv caches,
// gate and b / w activations, the recurrence, and the gated RMS norm of the
// output.  Row n of a [N, C] input is at base + n * ld (unit channel stride).
struct DecodeFusedParams {
    const void *x[3];     // raw q, k, v projection rows: channel h * D + c of head h
    int64_t ldx[3];
    const void *cw[3];    // conv weights [H * D, W]
    const void *cb[3];    // conv biases [H * D] or NULL
    const void *cin[3];   // conv caches [N, H * D, W - 1] or NULL (zero history)
    void *cout[3];        // new conv caches (may equal cin) or NULL
    const void *g, *b, *w;
    int64_t ldg, ldb, ldw;
    const float *h0;      // [N, H, D, D] rows h0_stride apart, or NULL
    float *ht;            // may equal h0 (in place), or NULL
    int64_t h0_stride, ht_stride;
    const float *A_log, *dt_bias;
    float lower_bound;
    const void *z;        // output gate rows [N, H * D] (NULL: no gate)
    int64_t ldz;
    const void *nw;       // norm weight [D] (NULL: no norm, o as computed)
    int nw_f32;           // norm weight (and output) float32 while the io dtype is 16-bit
    float eps;
    void *o;              // [N, H, D]
    int N, H, D;
    float scale;
    unsigned flags;
};

hipError_t launch_decode_fused(const DecodeFusedParams &p, int io_dtype, int g_dtype,
                               hipStream_t stream);

struct ChunkFwdArgs {
    const void *q, *k, *v, *g, *b, *w;
    void *o;
    const float *h0;
    float *ht;
    const float *A_log;
    const float *dt_bias;
    float lower_bound;
    const int64_t *cu_seqlens;
    const int64_t *cu_host;
    int num_seqs;
    int B, T, H, K, V;
    float scale;
    unsigned flags;
    void *workspace;
    size_t workspace_bytes;
    int stages;  // bit 0: prep, bit 1: scan
    // Gated output norm fused into the scan (null z: none).
    const void *z = nullptr;
    int64_t ldz = 0;
    const void *nw = nullptr;
    float eps = 0.f;
    // Short convolutions of q, k, v fused into the kernels (null taps: none);
    // q, k, v are then the raw projections with these token row strides.
    const void *conv_w[3] = {nullptr, nullptr, nullptr};
    int64_t ldq = 0, ldk = 0, ldv = 0;
    int conv_silu = 0;
};

size_t chunk_fwd_workspace_bytes(int B, int T, int H, int K, int V, int io_dtype,
                                 const int64_t *cu_host, int num_seqs);
int launch_chunk_fwd(const ChunkFwdArgs &a, int io_dtype, int g_dtype, hipStream_t stream);

struct ChunkBwdArgs {
    const void *q, *k, *v, *g, *b, *w, *dout;
    const float *dht;
    void *dq, *dk, *dv, *dg, *db, *dw;
    float *dh0;
    const int64_t *cu_seqlens;
    const int64_t *cu_host;
    int num_seqs;
    int B, T, H, K, V;
    float scale;
    unsigned flags;
    const void *saved;  // training workspace of the forward
    size_t saved_bytes;
    void *workspace;    // backward scratch
    size_t workspace_bytes;
};

size_t chunk_train_workspace_bytes(int B, int T, int H, int K, int V, int io_dtype,
                                   const int64_t *cu_host, int num_seqs);
size_t chunk_bwd_workspace_bytes(int B, int T, int H, int K, int V, int io_dtype,
                                 const int64_t *cu_host, int num_seqs);
int launch_chunk_bwd(const ChunkBwdArgs &a, int io_dtype, int g_dtype, hipStream_t stream);

// Decay gate activation and its VJP (gdn2_gate.hip).
size_t gate_bwd_workspace_bytes(int64_t tokens, int H, int K, bool has_bias);
int launch_gate_fwd(const void *g, int g_dtype, const float *A_log, const float *dt_bias, float lower_bound,
                    unsigned flags, float *y, int64_t tokens, int H, int K, hipStream_t stream);
int launch_gate_bwd(const void *g, int g_dtype, const float *A_log, const float *dt_bias, float lower_bound,
                    unsigned flags, const float *dy, void *dg, float *dA_log, float *ddt_bias, int64_t tokens,
                    int H, int K, void *workspace, hipStream_t stream);

// Float32 chunk op with 128 < d_k <= 256 (gdn2_chunk_wide.hip): token-serial
// kernels with chunk start states kept for the backward, for the key widths
// whose fp32 chunk workspace does not fit the MFMA kernels' LDS.
bool chunk_wide(int K, int io_dtype);
size_t wide_train_workspace_bytes(int B, int T, int H, int K, int V, const int64_t *cu_host, int num_seqs);
size_t wide_bwd_workspace_bytes(int B, int T, int H, int K, int V, const int64_t *cu_host, int num_seqs);
int launch_chunk_fwd_wide(const ChunkFwdArgs &a, int g_dtype, hipStream_t stream);
int launch_chunk_bwd_wide(const ChunkBwdArgs &a, int g_dtype, hipStream_t stream);
hipError_t launch_chunk_states_wide(const void *hs, void *out, bool transpose, int64_t nc, int H, int K, int V,
                                    hipStream_t stream);

// Chunk start states saved by a training forward -> [nc, H, K, V] (or
// [nc, H, V, K]) in io_dtype.
hipError_t launch_chunk_states(const void *hs, int io_dtype, void *out, bool transpose, int64_t nc,
                               int H, int K, int V, hipStream_t stream);

// Short convolution (prologue): up to three tensors per launch.
struct ConvTensor {
    const void *x;          // [B, T, D]: row (b, t) at x + (b * T + t) * ldx
    const void *w;          // [D, W]
    const void *bias;       // [D] or NULL
    const void *cache_in;   // [B, D, W-1] or NULL (read on single-token calls)
    void *cache_out;        // [B, D, ncache] or NULL
    void *y;                // [B, T, D]
    int D;
    int64_t ldx;            // input row stride in elements (>= D)
};

struct ConvParams {
    ConvTensor t[3];
    int B, T, W, ncache;
    int silu;
};

hipError_t launch_short_conv(const ConvParams &p, int io_dtype, int maxD, int ntensors,
                             hipStream_t stream);

// Gated RMS norm (epilogue).
struct NormParams {
    const void *x, *z, *weight;
    void *out;
    int64_t rows;
    int N;
    int w_f32;  // weight (and output) in float32 while x, z are 16-bit
    float eps;
    // Residual add before a plain norm (z null): x <- round(x + res), written
    // to sum_out, then normalised.  Null: none.
    const void *res = nullptr;
    void *sum_out = nullptr;
};

hipError_t launch_gated_rmsnorm(const NormParams &p, int io_dtype, hipStream_t stream);

// The SwiGLU product of the decoder hosts: out[r, c] = round(round(silu(a)) * b)
// with a = ab[r, c], b = ab[r, H + c] (row stride ld), out [rows, H].
struct SiluMulParams {
    const void *ab;
    void *out;
    int64_t rows, ld;
    int H;
};
hipError_t launch_silu_mul(const SiluMulParams &p, int io_dtype, hipStream_t stream);

// Few-row linear layer: y[m, n] = x[m, :] . W[n, :] (+ bias[n]) for M <= 8
// rows, K a multiple of 512 (K / 512 in {1, 2, 4, 6, 8}), 16-bit io.
struct SkinnyParams {
    const void *x, *w, *bias;
    void *y;
    int64_t ldx, ldw, ldy;  // row strides in elements
    int M, N, K;
    // norm: the product's input is RMSNorm(x + res) with weight nw (io dtype)
    // and eps, as gdn2_add_rms_norm_fwd computes it; workgroup 0 writes the
    // sums x + res to sum_out.  M <= 4, K in {512, 1024, 2048}.
    int norm = 0;
    const void *res = nullptr, *nw = nullptr;
    void *sum_out = nullptr;
    int64_t ldres = 0, ldsum = 0;
    float eps = 0.f;
    // glu_out: y[m, c] = round(round(silu(a)) * b) for a = row c and b = row
    // c + N / 2 of the product (N even; y has N / 2 columns): SwiGLU's product
    // as the epilogue of the fused w1 / w2 projection.  K <= 2048.
    int glu_out = 0;
};
bool skinny_linear_supported(int io_dtype, int M, int K);
hipError_t launch_skinny_linear(const SkinnyParams &p, int io_dtype, hipStream_t stream);

// Few-row linear layers with a small inner dimension (K in {32, 64, 128, 256}),
// up to two independent problems of the same M and K per launch.
struct SmallLinearProblem {
    const void *x, *w, *bias;  // x rows ldx apart; W [N, K] contiguous; bias [N] or null
    void *y;                   // rows ldy apart
    int64_t ldx, ldy;
    int N;
};
struct SmallLinearParams {
    SmallLinearProblem prob[2];
    int M, K;
};
bool small_linear_supported(int io_dtype, int M, int K);
hipError_t launch_small_linear(const SmallLinearParams &p, int nprob, int io_dtype, hipStream_t stream);

// Single-token attention of the decoder host's attention layers: RoPE of q and
// k, the KV-cache store at position *pos, softmax attention over positions
// 0 .. *pos.  qkv [B, G, qpk + 2, D] (qpk q heads, k, v per KV group), caches
// [B, G, max_len, D], out [B, G * qpk, D]; cos / sin the token's fp32
// rotation row of rope_pairs values.
struct AttnDecodeParams {
    const void *qkv;
    const float *cos, *sin;
    int rope_pairs;
    int64_t rope_stride;  // 0: cos / sin are the token's row; else rows of tables indexed by *pos
    const int64_t *pos;
    void *k_cache, *v_cache, *out;
    int64_t max_len;
    int B, G, qpk, D;
    float scale;
    // Positions split over `splits` workgroups per KV group; with more than
    // one, their partial states go to part (attn_decode_workspace_floats) and
    // a second kernel merges them.
    int splits;
    float *part;
};
bool attn_decode_supported(int io_dtype, int qpk, int D);
int attn_decode_splits(int64_t max_len);
size_t attn_decode_workspace_floats(int B, int G, int qpk, int D, int64_t max_len);

// Row-wise argmax: out[r * out_stride] = first index of the maximum of row r
// (rows ld elements apart, n values; NaN is the maximum).
struct ArgmaxParams {
    const void *x;
    int64_t ld, rows, n, out_stride;
    int64_t *out;
    // Split form: each row's pieces over `splits` workgroups of pps pieces,
    // whose (value, index) candidates part_v / part_i [rows][splits] a second
    // kernel merges.
    int splits;
    int64_t pps;
    float *part_v;
    int64_t *part_i;
};
// Workgroups per row of the split form (1: the single-workgroup kernel).
int argmax_splits(int64_t n, int io_dtype);
hipError_t launch_argmax_rows(const ArgmaxParams &p, int io_dtype, hipStream_t stream);
hipError_t launch_attn_decode(const AttnDecodeParams &p, int io_dtype, hipStream_t stream);

// Backward of the short convolution on a prefill call (no cache).
struct ConvBwdParams {
    const void *x;      // [B, T, D] input rows: row (b, t) at x + (b * T + t) * ldx
    const void *w;      // [D, W]
    const void *bias;   // [D] or NULL
    const void *dy;     // [B, T, D] gradient of the output, contiguous
    void *dx;           // [B, T, D], contiguous
    void *dw;           // [D, W]
    void *dbias;        // [D] or NULL
    float *part;        // conv_bwd_partial_floats(B, T, D, W) floats of scratch
    int B, T, D, W;
    int64_t ldx;
    int silu;
};
int64_t conv_bwd_partial_floats(int B, int T, int D, int W);
hipError_t launch_short_conv_bwd(const ConvBwdParams &p, int io_dtype, hipStream_t stream);

// Backward of the gated RMS norm (rows of N <= 256 values).
struct NormBwdParams {
    const void *x, *z, *weight, *dy;
    void *dx, *dz, *dweight;
    float *part;        // norm_bwd_blocks(rows) * N floats of scratch
    int64_t rows;
    int N;
    int w_f32;          // weight (and its gradient) in float32
    float eps;
};
int64_t norm_bwd_blocks(int64_t rows);
hipError_t launch_gated_rmsnorm_bwd(const NormBwdParams &p, int io_dtype, hipStream_t stream);

}  // namespace gdn2
