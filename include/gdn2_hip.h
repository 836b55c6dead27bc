/*
 * gdn2_hip.h -- C ABI of libgdn2_hip.so, the MI355X (gfx950) execution backend
 * of the gdn2 (GatedDeltaNet2) token mixer.
 *
 * Every entry point takes raw device pointers, plain integer sizes and a HIP
 * stream passed as `void *` (a hipStream_t; NULL = the default stream), and
 * returns a gdn2_status code.  No torch or HIP types appear in the signatures,
 * so ctypes / cgo / JNI can bind them directly.
 *
 * Tensor layouts (all contiguous, innermost dimension last):
 *   q, k        [B, T, H,  K]     io_dtype
 *   v, w, o     [B, T, HV, V]     io_dtype
 *   g, b        [B, T, HV, K]     g in g_dtype, b in io_dtype
 *   states      [N, HV, K, V]     float32 (V fastest), N = B, or the number of
 *                                 packed sequences when cu_seqlens is given
 * HV must be a multiple of H (grouped value heads); the chunk entry points
 * require HV == H, as the reference chunk op does.
 *
 * Calls are asynchronous on `stream`.  Argument errors are reported before
 * anything is launched; GDN2_ERR_LAUNCH reports a failed kernel launch.
 */
#ifndef GDN2_HIP_H
#define GDN2_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define GDN2_ABI_VERSION 2

enum gdn2_dtype {
    GDN2_DTYPE_F32 = 0,
    GDN2_DTYPE_BF16 = 1,
    GDN2_DTYPE_F16 = 2,
    GDN2_DTYPE_I32 = 3, /* index tensors only (ssm_state_indices, ...) */
    GDN2_DTYPE_I64 = 4,
};

enum gdn2_status {
    GDN2_OK = 0,
    GDN2_ERR_INVALID = -1,     /* bad pointer, shape or flag combination   */
    GDN2_ERR_UNSUPPORTED = -2, /* valid request this build does not handle */
    GDN2_ERR_LAUNCH = -3,      /* the HIP runtime rejected a launch        */
    GDN2_ERR_WORKSPACE = -4,   /* workspace missing or too small           */
    GDN2_ERR_SCRATCH = -5,     /* gdn2_chunk_fwd_static: the shape needs    *
                                * more than GDN2_STATIC_SCRATCH_BYTES       */
};

/* Flags (bitwise or). */
#define GDN2_FLAG_L2NORM_QK 1u      /* q, k <- x / max(||x||, 1e-6) in-kernel  */
#define GDN2_FLAG_GATE_IN_KERNEL 2u /* g is the raw gate pre-activation        */
#define GDN2_FLAG_LOWER_BOUND 4u    /* with GATE_IN_KERNEL: bounded sigmoid    */
#define GDN2_FLAG_SAVE_FOR_BWD 8u   /* gdn2_chunk_fwd: keep what the backward   *
                                     * needs in a training-size workspace       */
#define GDN2_FLAG_TRANSPOSE_STATE 16u     /* recurrent and chunk calls: states  *
                                           * are [.., V, K] (K fastest)         */
#define GDN2_FLAG_INPLACE_FINAL_STATE 32u /* gdn2_recurrent_fwd_ex with state  *
                                           * indices: per-token states go to    *
                                           * the indexed slots, not token rows  */
#define GDN2_FLAG_SIGMOID_BW 64u /* recurrent calls and gdn2_chunk_fwd (not    *
                                  * with SAVE_FOR_BWD, not gdn2_chunk_fwd_prep): *
                                  * b and w hold the pre-activation logits; the  *
                                  * kernels use sigmoid(b), sigmoid(w) in fp32   *
                                  * (the module's b_proj / w_proj activations,   *
                                  * gdn2.py:864-865)                             */

int gdn2_abi_version(void);
const char *gdn2_status_string(int status);

/*
 * Token-serial forward: decode steps and short prefills.
 * Replaces fused_recurrent_gdn2 / fused_recurrent_gdn2_fwd
 * (reference src/qwendopamine/models/gdn2/gdn2_ops/fused_recurrent_gdn2.py:461-555
 * and :344-458), whose arithmetic is torch_recurrent_gdn2 (gdn2.py:100-184).
 *
 *   initial_state  NULL = zero state.
 *   final_state    NULL = not stored; may equal initial_state (in-place update,
 *                  the reference's inplace_final_state).
 *   A_log [HV], dt_bias [HV*K]  used only with GDN2_FLAG_GATE_IN_KERNEL
 *                  (dt_bias may be NULL); lower_bound only with LOWER_BOUND.
 *   cu_seqlens     NULL, or num_seqs+1 int64 offsets into T (then B == 1).
 */
int gdn2_recurrent_fwd(const void *q, const void *k, const void *v, const void *g,
                       const void *b, const void *w, int io_dtype, int g_dtype, void *o,
                       const float *initial_state, float *final_state, const float *A_log,
                       const float *dt_bias, float lower_bound, const int64_t *cu_seqlens,
                       int num_seqs, int B, int T, int H, int HV, int K, int V, float scale,
                       unsigned flags, void *stream);

/*
 * Token-serial forward with the serving options of fused_recurrent_gdn2_fwd
 * (reference gdn2_ops/fused_recurrent_gdn2.py:344-458, kernel :129-341):
 * a state pool addressed through ssm_state_indices (continuous batching),
 * num_accepted_tokens (speculative decoding) and the transposed state layout.
 * gdn2_recurrent_fwd is this call with rows = N, row strides = HV*K*V and no
 * indices.
 *
 *   initial_state / final_state   float32 arrays of *_rows rows, row r of a
 *       state at base + r*row_stride (elements; row_stride >= HV*K*V and a
 *       multiple of 4), each row [HV, K, V] ([HV, V, K] with
 *       GDN2_FLAG_TRANSPOSE_STATE, which then needs K % 4 == 0).
 *   ssm_state_indices  NULL, or indices_numel int32/int64 (indices_dtype =
 *       GDN2_DTYPE_I32/I64) slot numbers; sequence n, position t reads entry
 *       n*indices_seq_stride + t (the reference's addressing, :215-224, 312-320).
 *       With indices, sequence n starts from initial_state row
 *       idx[n*stride + i0] (i0 = num_accepted_tokens[n] - 1, else 0), and the
 *       state after each of its tokens t is stored
 *         - to final_state row idx[n*stride + t] with GDN2_FLAG_INPLACE_FINAL_STATE,
 *         - else to final_state row bos + t (the token's packed position).
 *       Without indices the final state of sequence n goes to row n.
 *       An index entry outside [0, indices_numel) or a slot outside
 *       [0, rows) is a padded entry: that state is read as zero / not
 *       stored (the reference does not guard these accesses).
 *   num_accepted_tokens  NULL, or N int32/int64 counts (accepted_dtype);
 *       used only with ssm_state_indices.
 */
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
                          void *stream);

/*
 * Short convolution of the mixer's prologue.  Replaces ShortConvolution.forward
 * (reference src/qwendopamine/models/gdn2/gdn2.py:395-430) for up to three
 * tensors (q, k, v) in one launch: for tensor i,
 *   y_i[b, t, d] = act(bias_i[d] + sum_j weight_i[d, j] * x_i[b, t - W + 1 + j, d])
 * with act = SiLU when `silu` is set; x_i, y_i [B, T, D_i] and weight_i
 * [D_i, W] (the Conv1d weight [D, 1, W]), bias_i [D_i] or NULL, all io_dtype.
 * Tokens before 0 are zero, or, on a single-token call (T == 1), the cache
 * cache_in_i [B, D_i, W-1] (may be NULL).  cache_out_i (may be NULL) receives
 * the last min(T, W-1) inputs as [B, D_i, min(T, W-1)] (W-1 columns when
 * T == 1), as the reference's new conv state.  Like the reference, the
 * convolution runs over the packed token axis (no cu_seqlens).
 * 1 <= ntensors <= 3, 1 <= W <= 8.
 */
int gdn2_short_conv_fwd(int ntensors, const void *const *x, const void *const *weight,
                        const void *const *bias, const void *const *cache_in,
                        void *const *cache_out, void *const *y, const int *dims, int io_dtype,
                        int B, int T, int W, int silu, void *stream);

/*
 * gdn2_short_conv_fwd with strided input rows: row (b, t) of x_i starts at
 * x_i + (b*T + t) * x_row_stride[i] elements (x_row_stride[i] >= D_i; NULL =
 * contiguous rows).  It lets q, k and v be column ranges of one fused input
 * projection's output, as the module's inference path produces them, with no
 * copies.  Same reference function as gdn2_short_conv_fwd (gdn2.py:395-430).
 */
int gdn2_short_conv_fwd_ex(int ntensors, const void *const *x, const int64_t *x_row_stride,
                           const void *const *weight, const void *const *bias,
                           const void *const *cache_in, void *const *cache_out, void *const *y,
                           const int *dims, int io_dtype, int B, int T, int W, int silu,
                           void *stream);

/*
 * Gated RMS norm of the mixer's epilogue.  Replaces RMSNormGated.forward
 * (reference gdn2.py:433-452): for each of `rows` rows of N values,
 *   out = x * rsqrt(mean(x^2) + eps) * weight * silu(z)
 * with the reference's rounding to io_dtype after every op.  weight [N] is
 * io_dtype, or float32 (weight_dtype = GDN2_DTYPE_F32), in which case torch's
 * promotion makes the last two products and `out` float32.
 * z = NULL drops the gate: out = weight * (x * rsqrt(mean(x^2) + eps)), the
 * plain RMSNorm.forward of the decoder hosts (reference
 * models/normalization.py:40-51), with the same rounding.  N <= 2048.
 */
int gdn2_gated_rmsnorm_fwd(const void *x, const void *z, const void *weight, int weight_dtype,
                           void *out, int io_dtype, int64_t rows, int N, float eps, void *stream);

/*
 * Residual add and the next pre-norm of a decoder block in one pass:
 *   sum_out = x + residual                  (rounded to io_dtype, torch's add)
 *   out     = gdn2_gated_rmsnorm_fwd(sum_out, z = NULL, weight)
 * Replaces `x = x + h` followed by `norm_2(x)` inside Block.forward, and the
 * last block's `x + h` followed by the model's final norm (reference
 * src/qwendopamine/models/gdn2_gpt/model.py:240-248 and the ln_f call of
 * GDN2GPT.forward), with RMSNorm.forward's rounding (reference
 * models/normalization.py:40-51): both outputs equal the two separate ops bit
 * for bit.  Rows of N values with N / (16 bytes of io_dtype) a power of two in
 * [4, 256] and 16-byte aligned x, residual, sum_out, out; other shapes return
 * GDN2_ERR_UNSUPPORTED (the caller keeps the two ops).
 */
int gdn2_add_rms_norm_fwd(const void *x, const void *residual, void *sum_out, const void *weight,
                          int weight_dtype, void *out, int io_dtype, int64_t rows, int N, float eps,
                          void *stream);

/*
 * SwiGLU's gated product (reference src/qwendopamine/models/gdn2_gpt/model.py:74-77,
 * `F.silu(x1) * x2`) on the output of one fused w1 / w2 projection:
 *   out[r, c] = round(round(silu(ab[r, c])) * ab[r, H + c])
 * with row r of ab at ab + r * ab_row_stride (>= 2H) and out [rows, H]
 * contiguous, rounded to io_dtype after each op as torch is.  H and the row
 * stride multiples of 16 bytes of io_dtype, 16-byte aligned pointers.
 */
int gdn2_silu_mul_fwd(const void *ab, int64_t ab_row_stride, void *out, int io_dtype, int64_t rows,
                      int H, void *stream);

/*
 * The decoder hosts' linear layers on a decode step's few rows:
 *   y[m, n] = sum_k x[m, k] * weight[n, k] (+ bias[n]),   m < M <= 8
 * with fp32 accumulation and one rounding to io_dtype (bf16 or fp16), as
 * torch's F.linear; the summation order differs from torch's GEMM, so the
 * results agree to rounding.  Replaces the nn.Linear / F.linear calls of one
 * decode step: SwiGLU's w1 / w2 / w3 (reference
 * src/qwendopamine/models/gdn2_gpt/model.py:74-78), the attention and gdn2
 * projections and the LM head (model.py GDN2GPT.forward; gdn2.py's q / k / v /
 * gate projections and o_proj).  Rows of x, weight and y are
 * x_row_stride / weight_row_stride / y_row_stride elements apart (unit column
 * stride).  K / 512 in {1, 2, 4, 6, 8} (M <= 4 beyond K = 2048), x and weight
 * 16-byte aligned with row
 * strides multiples of 8 elements; other shapes return GDN2_ERR_UNSUPPORTED
 * (the caller keeps torch's GEMM).
 */
int gdn2_skinny_linear(const void *x, int64_t x_row_stride, const void *weight, int64_t weight_row_stride,
                       const void *bias, void *y, int64_t y_row_stride, int io_dtype, int M, int N, int K,
                       void *stream);

/*
 * A decoder block's residual add and pre-norm feeding a few-row linear layer,
 * in one launch:
 *   sum_out = x + residual                      (written once)
 *   y       = gdn2_skinny_linear(RMSNorm(sum_out; norm_weight, eps), weight, bias)
 * with the normalised rows formed while the product stages its input, with
 * gdn2_add_rms_norm_fwd's roundings and summation order: equal bit for bit to
 * gdn2_add_rms_norm_fwd followed by gdn2_skinny_linear.  Replaces
 * `x = x + h; mlp(norm_2(x))`'s first GEMM in Block.forward (reference
 * src/qwendopamine/models/gdn2_gpt/model.py:240-248, models/normalization.py:40-51).
 * M <= 4, K in {512, 1024, 2048}, norm_weight in io_dtype; 16-byte aligned
 * x, residual, sum_out, weight with row strides multiples of 8 elements;
 * else GDN2_ERR_UNSUPPORTED.
 */
int gdn2_skinny_linear_addnorm(const void *x, int64_t x_row_stride, const void *residual,
                               int64_t residual_row_stride, void *sum_out, int64_t sum_row_stride,
                               const void *norm_weight, float eps, const void *weight, int64_t weight_row_stride,
                               const void *bias, void *y, int64_t y_row_stride, int io_dtype, int M, int N, int K,
                               void *stream);

/*
 * gdn2_skinny_linear_addnorm whose output is SwiGLU's gated product: with
 * weight the stacked [w1; w2] (N rows, N even), y[m, c] =
 * round(round(silu(a)) * b) for a = p[m, c], b = p[m, c + N / 2] of the
 * product p (each rounded to io_dtype first), y [M, N / 2]: bit for bit
 * gdn2_skinny_linear_addnorm followed by gdn2_silu_mul_fwd, in one launch (a
 * wave holds rows c and c + N / 2).  Replaces `F.silu(w1(n)) * w2(n)` with
 * n = norm_2(x + h) (reference src/qwendopamine/models/gdn2_gpt/model.py:74-78,
 * :240-248) on a decode step's rows.  Same limits as
 * gdn2_skinny_linear_addnorm.
 */
int gdn2_skinny_linear_addnorm_swiglu(const void *x, int64_t x_row_stride, const void *residual,
                                      int64_t residual_row_stride, void *sum_out, int64_t sum_row_stride,
                                      const void *norm_weight, float eps, const void *weight,
                                      int64_t weight_row_stride, const void *bias, void *y, int64_t y_row_stride,
                                      int io_dtype, int M, int N, int K, void *stream);

/*
 * Two few-row linear layers with a small inner dimension in one launch:
 *   y_i[m, n] = sum_k x_i[m, k] * weight_i[n, k] (+ bias_i[n]),  i = 0, 1
 * for the module's second-stage gate projections of a decode step (reference
 * gdn2.py:591-594 and :615-618: f_proj[1] Linear(head_v_dim, key_dim) and
 * g_proj[1] Linear(head_v_dim, value_dim, bias)), which share M and K.
 * Weights [N_i, K] contiguous; x_i rows x_i_row_stride elements apart (a
 * multiple of 8, x_i 16-byte aligned); fp32 sums rounded once.  N_i = 0 skips
 * a problem.  bf16 / fp16, K in {32, 64, 128, 256}, M <= min(8, K / 8); else
 * GDN2_ERR_UNSUPPORTED.
 */
int gdn2_small_linear_pair(const void *x0, int64_t x0_row_stride, const void *weight0, const void *bias0, void *y0,
                           int64_t y0_row_stride, int N0, const void *x1, int64_t x1_row_stride,
                           const void *weight1, const void *bias1, void *y1, int64_t y1_row_stride, int N1,
                           int io_dtype, int M, int K, void *stream);

/*
 * One decode step of the hybrid host's attention layers (one token per
 * sequence), in one launch: RoPE of the token's q heads and k (interleaved
 * pairs, fp32, rounded to io_dtype), the store of k and v into the caches at
 * position *pos, and softmax attention of each q head over cache positions
 * 0 .. *pos of its KV group.  Replaces the single-token path of
 * CausalSelfAttention.forward (reference
 * src/qwendopamine/models/gdn2_gpt/model.py:89-173: apply_rope :40-61, the KV
 * cache update and the masked scaled_dot_product_attention).
 *   qkv      [B, G, qpk + 2, D] io_dtype: per KV group, qpk q heads, k, v
 *            (the fused attn projection's layout)
 *   cos, sin fp32 rotation of the token (rope_pairs values; channels from
 *            2 * rope_pairs on are not rotated); with rope_row_stride > 0
 *            they are instead whole tables of at least max_len rows,
 *            rope_row_stride floats apart, and the kernel reads row *pos
 *            (so the host needs no per-step selection of the row)
 *   pos      device int64: the token's position (one for all sequences)
 *   k_cache, v_cache  [B, G, max_len, D] io_dtype, updated at pos
 *   out      [B, G * qpk, D] io_dtype
 * Scores and probabilities are fp32 (the output is rounded once); the host's
 * torch path rounds the scores and probabilities to io_dtype, so the two agree
 * to that rounding.  A position outside [0, max_len) leaves the caches alone
 * and writes zeros.  bf16 / fp16, D in {64, 128}, qpk in {1, 2, 4}; else
 * GDN2_ERR_UNSUPPORTED.  Caches longer than 1024 positions are split over
 * several workgroups per KV group, whose partial softmax states are merged by
 * a second kernel: workspace of gdn2_attn_decode_workspace_size() bytes
 * (0 for caches of up to 1024 positions, where workspace may be NULL).
 */
size_t gdn2_attn_decode_workspace_size(int B, int G, int qpk, int D, int64_t max_len);
int gdn2_attn_decode(const void *qkv, const float *cos, const float *sin, int rope_pairs, int64_t rope_row_stride,
                     const int64_t *pos, void *k_cache, void *v_cache, void *out, int io_dtype, int B, int G,
                     int qpk, int D, int64_t max_len, float scale, void *workspace, size_t workspace_bytes,
                     void *stream);

/*
 * Greedy decoding's argmax over the LM head's logits (the logits of reference
 * src/qwendopamine/models/gdn2_gpt/model.py:304-380, GPT.forward; the
 * reference has no decoding loop, the hybrid host's greedy decoder calls this
 * in place of torch.argmax and keeps its semantics): out[r * out_stride] = the first index of the
 * maximum of row r, NaN counting as the maximum.  x rows x_row_stride
 * elements apart (16-byte aligned), n values each, io_dtype f32 / bf16 / fp16.
 * With a workspace of gdn2_argmax_rows_workspace_size() bytes (8-byte
 * aligned; 0 for rows of up to 1024 16-byte pieces) each row is split over
 * several workgroups and a second launch merges their candidates; with
 * workspace NULL one workgroup scans each row (one launch).
 */
size_t gdn2_argmax_rows_workspace_size(int64_t rows, int64_t n, int io_dtype);
int gdn2_argmax_rows(const void *x, int64_t x_row_stride, int io_dtype, int64_t rows, int64_t n, int64_t *out,
                     int64_t out_stride, void *workspace, size_t workspace_bytes, void *stream);

/*
 * The in-kernel decay gate as a separate differentiable step, for training
 * calls of the chunk op with use_gate_in_kernel (reference kda_gate_fwd and
 * kda_gate_bwd, src/qwendopamine/models/gdn2/gdn2_ops/chunk_kda.py:3223-3292,
 * kernels :3089-3220).  g_raw [tokens, H, K] in g_dtype (f32 / bf16 / fp16),
 * A_log [H] and dt_bias [H*K] (or NULL) float32, K <= 256:
 *   y = -exp(A_log[h]) * softplus(g_raw + dt_bias[h, c]), or with
 *   GDN2_FLAG_LOWER_BOUND y = lower_bound * sigmoid(exp(A_log[h]) * (g_raw + dt_bias)),
 * the formula of GDN2_FLAG_GATE_IN_KERNEL.  gdn2_gate_fwd writes y (float32);
 * gdn2_gate_bwd takes dy (float32) and writes dg_raw (g_dtype), dA_log [H] and
 * ddt_bias [H*K] (float32; NULL with dt_bias NULL), the two sums over tokens
 * taken per 64-token block and then added in block order (deterministic).
 * workspace: at least gdn2_gate_bwd_workspace_size() bytes.
 */
size_t gdn2_gate_bwd_workspace_size(int64_t tokens, int H, int K, int has_dt_bias);
int gdn2_gate_fwd(const void *g_raw, int g_dtype, const float *A_log, const float *dt_bias,
                  float lower_bound, unsigned flags, float *y, int64_t tokens, int H, int K,
                  void *stream);
int gdn2_gate_bwd(const void *g_raw, int g_dtype, const float *A_log, const float *dt_bias,
                  float lower_bound, unsigned flags, const float *dy, void *dg_raw, float *dA_log,
                  float *ddt_bias, int64_t tokens, int H, int K, void *workspace,
                  size_t workspace_bytes, void *stream);

/*
 * Backward of the short convolution on a prefill call (no cache), for training
 * without torch's conv: the gradient of ShortConvolution.forward (reference
 * gdn2.py:395-430, whose backward torch's autograd runs through F.conv1d and
 * F.silu), y = silu(round(bias + conv(x))).  Recomputes the rounded
 * pre-activation, then dpre = round(dy * silu'(pre)) (torch's SiLU backward),
 *   dx[t] = sum_j w[j] dpre[t + W-1-j],
 *   dweight[d, j] = sum_{b,t} dpre[t] x[t-W+1+j],  dbias[d] = sum_{b,t} dpre[t]
 * with fp32 accumulation, deterministic (per-tile partials summed in a fixed
 * order).  x rows [B*T, x_row_stride >= D]; dy, dx contiguous [B, T, D];
 * weight / dweight [D, W]; bias / dbias [D] or NULL; silu: apply the SiLU.
 * workspace: at least gdn2_short_conv_bwd_workspace_size() bytes.
 */
size_t gdn2_short_conv_bwd_workspace_size(int B, int T, int D, int conv_width);
int gdn2_short_conv_bwd(const void *x, int64_t x_row_stride, const void *weight, const void *bias,
                        const void *dy, void *dx, void *dweight, void *dbias, int io_dtype, int B,
                        int T, int D, int conv_width, int silu, void *workspace,
                        size_t workspace_bytes, void *stream);

/*
 * Backward of the gated RMS norm (reference RMSNormGated.forward, gdn2.py:433-452,
 * whose backward torch's autograd runs through its five ops): for `rows` rows of
 * N <= 256 values, with r = rsqrt(mean(x^2) + eps), xn = x r, s = silu(z),
 *   dx = r (g - xn mean(g xn)),  g = dy weight s;   dz = dy xn weight silu'(z);
 *   dweight = sum over rows of dy xn s
 * in fp32 (deterministic partial sums).  weight / dweight in io_dtype or float32.
 * workspace: at least gdn2_gated_rmsnorm_bwd_workspace_size() bytes.
 */
size_t gdn2_gated_rmsnorm_bwd_workspace_size(int64_t rows, int N);
int gdn2_gated_rmsnorm_bwd(const void *x, const void *z, const void *weight, int weight_dtype,
                           const void *dy, void *dx, void *dz, void *dweight, int io_dtype,
                           int64_t rows, int N, float eps, void *workspace, size_t workspace_bytes,
                           void *stream);

/*
 * Fused module decode step: one token per sequence through the whole mixer
 * core, with no HBM round trip of q, k, v or o in between.  Replaces, for the
 * decode call of GatedDeltaNet2.forward, the chain
 *   ShortConvolution of q, k, v with the conv caches   (reference gdn2.py:395-430)
 *   -> gate and b / w activations                      (gdn2.py:840-866)
 *   -> fused_recurrent_gdn2 (T = 1, in-place state)    (gdn2_ops/fused_recurrent_gdn2.py:461-555)
 *   -> RMSNormGated of the output with its gate        (gdn2.py:433-452)
 * for num_v_heads == num_heads and K == V in {64, 128}.
 *
 *   raw_qkv[t] + n * ld_qkv[t]     row n of the raw q / k / v projections (before
 *                                  the convolution), channel h * K + c of head h
 *   g, b, w (+ n * ld)             decay (raw with GDN2_FLAG_GATE_IN_KERNEL), erase and
 *                                  write gates (logits with GDN2_FLAG_SIGMOID_BW),
 *                                  rows [H * K]
 *   conv_weight[t] [H*K, W], conv_bias[t] [H*K] or NULL, W = conv_width = 4
 *   conv_cache_in[t]  [N, H*K, W-1] or NULL (zero history); conv_cache_out[t]
 *                     receives the last W-1 inputs, may equal conv_cache_in[t]
 *   initial_state / final_state    [N, H, K, V] float32 rows at the given row
 *                     strides (elements), may be the same array (in place); the
 *                     initial state may be NULL (zero)
 *   gate + n * ld_gate  the output gate g_proj(x) [H * V] (NULL: no gate)
 *   norm_weight [V] in io_dtype or float32 (NULL: o is returned un-normalised)
 *   o  [N, H, V] in io_dtype, float32 when norm_weight is float32 and io_dtype
 *      is not (torch's promotion)
 * Flags: GDN2_FLAG_L2NORM_QK, GATE_IN_KERNEL, LOWER_BOUND, SIGMOID_BW.
 */
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
                      void *stream);

/*
 * Bytes of device workspace gdn2_chunk_fwd needs for this shape.
 */
size_t gdn2_chunk_fwd_workspace_size(int B, int T, int H, int K, int V, int io_dtype,
                                     const int64_t *cu_seqlens_host, int num_seqs);

/*
 * Chunkwise-parallel (C = 64) forward: prefill and training forward.
 * Replaces chunk_gdn2 / chunk_gdn2_fwd
 * (reference src/qwendopamine/models/gdn2/gdn2_ops/chunk_gdn2.py:1268-1434 and
 * :1165-1264).  Same arguments as gdn2_recurrent_fwd with HV == H, plus a
 * device workspace of at least gdn2_chunk_fwd_workspace_size() bytes.
 * cu_seqlens_host mirrors cu_seqlens on the host (the reference's
 * cu_seqlens_cpu); both NULL or both given.
 * d_k <= 256 in every io dtype.  float32 inputs with 128 < d_k <= 256 (and
 * d_v <= 256) run the recurrence token by token with the chunk start states
 * kept for the backward; they need no workspace outside training.
 */
int gdn2_chunk_fwd(const void *q, const void *k, const void *v, const void *g, const void *b,
                   const void *w, int io_dtype, int g_dtype, void *o,
                   const float *initial_state, float *final_state, const float *A_log,
                   const float *dt_bias, float lower_bound, const int64_t *cu_seqlens,
                   const int64_t *cu_seqlens_host, int num_seqs, int B, int T, int H, int K,
                   int V, float scale, unsigned flags, void *workspace,
                   size_t workspace_bytes, void *stream);

/*
 * gdn2_chunk_fwd with the module's gated output norm applied in the scan's
 * output stage: o = RMSNormGated(chunk output, gate) in io_dtype, the output
 * never leaving the chip unnormalised.  Replaces chunk_gdn2 followed by
 * RMSNormGated.forward (reference gdn2_ops/chunk_gdn2.py:1268-1434 and
 * src/qwendopamine/models/gdn2/gdn2.py:433-452, as GatedDeltaNet2.forward calls
 * them at gdn2.py:875-927), with the norm's roundings of gdn2_gated_rmsnorm_fwd:
 * the result equals gdn2_chunk_fwd followed by gdn2_gated_rmsnorm_fwd bit for bit.
 *   gate         [total tokens, ld_gate] rows in io_dtype; head h reads columns
 *                h*V .. h*V+V-1 (a column range of a wider tensor is allowed)
 *   norm_weight  [V] in io_dtype
 * Inference only (GDN2_FLAG_SAVE_FOR_BWD is rejected); bf16 io and V in
 * {16, 32, 64} (one workgroup owns a whole value row), otherwise
 * GDN2_ERR_UNSUPPORTED.  ld_gate a multiple of 4, gate and o 8-byte aligned.
 */
int gdn2_chunk_fwd_gated_norm(const void *q, const void *k, const void *v, const void *g,
                              const void *b, const void *w, int io_dtype, int g_dtype, void *o,
                              const void *gate, int64_t ld_gate, const void *norm_weight, float eps,
                              const float *initial_state, float *final_state, const float *A_log,
                              const float *dt_bias, float lower_bound, const int64_t *cu_seqlens,
                              const int64_t *cu_seqlens_host, int num_seqs, int B, int T, int H,
                              int K, int V, float scale, unsigned flags, void *workspace,
                              size_t workspace_bytes, void *stream);

/*
 * gdn2_chunk_fwd on the raw q, k, v projections, with the module's three
 * short convolutions (causal depthwise conv1d of width 4, no bias, optional
 * SiLU) applied inside the chunk kernels: prep convolves q and k as it lands
 * their rows, the scan's copy waves convolve v as they form w * v.  Replaces
 * ShortConvolution.forward for q, k, v followed by chunk_gdn2 (reference
 * src/qwendopamine/models/gdn2/gdn2.py:395-430 and
 * gdn2_ops/chunk_gdn2.py:1268-1434, as GatedDeltaNet2.forward calls them at
 * gdn2.py:815-833 and 875-927), prefill without a conv cache: rows before a
 * sequence's first token read as zero (per cu_seqlens sequence).  Every
 * convolution output is rounded to io_dtype before and after the SiLU, as in
 * gdn2_short_conv_fwd, so without cu_seqlens the result equals
 * gdn2_short_conv_fwd followed by gdn2_chunk_fwd bit for bit.
 *   q, k, v        raw rows with token strides ld_q, ld_k, ld_v (elements,
 *                  multiples of 8); head h reads columns h*K.. (h*V.. for v)
 *   conv_q/k/v     [H*K or H*V][4] taps in io_dtype (the conv1d weights)
 *   gate           optional: non-NULL applies the gated output norm as
 *                  gdn2_chunk_fwd_gated_norm does (then V in {16, 32, 64})
 * The new conv caches (the last three raw rows) are not written: they are
 * slices of q, k, v.  Inference only; bf16 io, K in {32, 64, 128}, V a
 * multiple of 16 split into whole value slices, conv_width 4, otherwise
 * GDN2_ERR_UNSUPPORTED.  q, k, v, g, b, w and the taps 16-byte aligned.
 */
int gdn2_chunk_fwd_conv(const void *q, int64_t ld_q, const void *k, int64_t ld_k, const void *v,
                        int64_t ld_v, const void *conv_q, const void *conv_k, const void *conv_v,
                        int conv_width, int conv_silu, const void *g, const void *b, const void *w,
                        int io_dtype, int g_dtype, void *o, const void *gate, int64_t ld_gate,
                        const void *norm_weight, float eps, const float *initial_state,
                        float *final_state, const float *A_log, const float *dt_bias,
                        float lower_bound, const int64_t *cu_seqlens,
                        const int64_t *cu_seqlens_host, int num_seqs, int B, int T, int H, int K,
                        int V, float scale, unsigned flags, void *workspace,
                        size_t workspace_bytes, void *stream);

/*
 * The two stages of gdn2_chunk_fwd, for callers that schedule or time them
 * separately.  Calling prep then scan on the same workspace equals
 * gdn2_chunk_fwd.
 *
 * Stage 1 -- per-chunk K-side work, all chunks in parallel (in-kernel L2 norm,
 * scale and gate; in-chunk cumulative decay; decayed q.k^T and (b*k).k^T
 * products; the triangular inverse of the WY/UT transform).  Replaces
 * chunk_gdn2_fwd_intra + recompute_w_u_fwd_gdn2 (reference
 * gdn2_ops/chunk_gdn2.py:1010-1162).  Reads q, k, g, b; writes the workspace.
 */
int gdn2_chunk_fwd_prep(const void *q, const void *k, const void *g, const void *b,
                        int io_dtype, int g_dtype, const float *A_log, const float *dt_bias,
                        float lower_bound, const int64_t *cu_seqlens,
                        const int64_t *cu_seqlens_host, int num_seqs, int B, int T, int H,
                        int K, int V, float scale, unsigned flags, void *workspace,
                        size_t workspace_bytes, void *stream);

/*
 * Stage 2 -- the sequential inter-chunk state scan and the outputs.  Replaces
 * chunk_gated_delta_rule_fwd_h (reference gdn2_ops/chunk_kda.py:2217-2294) and
 * the output stage chunk_gla_fwd_o_gk (called at chunk_gdn2.py:1243-1255).
 * Reads v, w, the initial state and the workspace; writes o and the final
 * state.
 */
int gdn2_chunk_fwd_scan(const void *v, const void *w, int io_dtype, void *o,
                        const float *initial_state, float *final_state,
                        const int64_t *cu_seqlens, const int64_t *cu_seqlens_host, int num_seqs,
                        int B, int T, int H, int K, int V, void *workspace,
                        size_t workspace_bytes, void *stream);

/*
 * Bytes of the training workspace: gdn2_chunk_fwd with GDN2_FLAG_SAVE_FOR_BWD
 * writes, next to its per-chunk blobs, the chunk start states and chunk
 * values U (fp32 precision) that gdn2_chunk_bwd reads back (the tensors the
 * reference forward saves for backward, chunk_gdn2.py:2424-2447).
 * The same buffer is then passed unchanged to gdn2_chunk_bwd.
 */
size_t gdn2_chunk_train_workspace_size(int B, int T, int H, int K, int V, int io_dtype,
                                       const int64_t *cu_seqlens_host, int num_seqs);

/*
 * The per-chunk start states of a gdn2_chunk_fwd call made with
 * GDN2_FLAG_SAVE_FOR_BWD, read from its training workspace `saved`: writes
 * out [nc, H, K, V] (transpose = 0) or [nc, H, V, K] (transpose != 0) in
 * io_dtype, nc = total chunks of 64 tokens (sequence-major, as the
 * reference's chunk indices).  Replaces the `h` that chunk_gdn2 returns with
 * return_intermediate_states (reference gdn2_ops/chunk_gdn2.py:1257-1263,
 * 1415-1421; h from chunk_gated_delta_rule_fwd_h in the inputs' dtype,
 * chunk_kda.py:2263).
 */
int gdn2_chunk_states(const void *saved, size_t saved_bytes, int io_dtype, void *out, int transpose,
                      const int64_t *cu_seqlens_host, int num_seqs, int B, int T, int H, int K,
                      int V, void *stream);

/*
 * Bytes of device scratch gdn2_chunk_bwd needs for this shape.
 */
size_t gdn2_chunk_bwd_workspace_size(int B, int T, int H, int K, int V, int io_dtype,
                                     const int64_t *cu_seqlens_host, int num_seqs);

/*
 * Chunkwise backward.  Replaces chunk_gdn2_bwd and the gradient mapping of
 * ChunkGDN2Function.backward (reference gdn2_ops/chunk_gdn2.py:2170-2325 and
 * :2480-2547): given do [B,T,H,V] (io_dtype) and optionally dht [N,H,K,V]
 * (float32, gradient of the final state), writes
 *   dq, dk, db [B,T,H,K] (io_dtype), dg [B,T,H,K] (g_dtype),
 *   dv, dw [B,T,H,V] (io_dtype), and dh0 [N,H,K,V] (float32, may be NULL),
 * the gradients with respect to the raw inputs of the forward (through the
 * in-kernel L2 norm when GDN2_FLAG_L2NORM_QK is set, and the scale).
 * q, k, v, g, b, w, scale, flags and cu_seqlens must be those of the forward
 * call, and `saved` the training workspace it filled.  The in-kernel gate
 * (GDN2_FLAG_GATE_IN_KERNEL) is not differentiated here: callers that need
 * gradients apply the gate before the op (GDN2_ERR_UNSUPPORTED otherwise).
 */
int gdn2_chunk_bwd(const void *q, const void *k, const void *v, const void *g, const void *b,
                   const void *w, int io_dtype, int g_dtype, const void *dout,
                   const float *dht, void *dq, void *dk, void *dv, void *dg, void *db, void *dw,
                   float *dh0, const int64_t *cu_seqlens, const int64_t *cu_seqlens_host,
                   int num_seqs, int B, int T, int H, int K, int V, float scale,
                   unsigned flags, const void *saved, size_t saved_bytes, void *workspace,
                   size_t workspace_bytes, void *stream);

/*
 * gdn2_chunk_fwd without a workspace argument: allocates nothing.
 * This entry point has no counterpart in the reference.  It is for callers that
 * cannot allocate device memory: code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc.  Arguments and results are those of
 * gdn2_chunk_fwd (inference only: GDN2_FLAG_SAVE_FOR_BWD is rejected); the
 * per-chunk blobs live in a static device array of GDN2_STATIC_SCRATCH_BYTES
 * (72 MiB) on each GPU the library runs on, held until the process ends.
 * A shape whose gdn2_chunk_fwd_workspace_size() exceeds that returns
 * GDN2_ERR_SCRATCH before anything is launched (72 MiB holds 1143 (chunk, head)
 * blobs at d_k = 128 in bf16 / fp16, e.g. 4096 tokens x 16 heads).
 * `stream` must belong to the current device.  Every call on one GPU shares
 * that GPU's array: calls that overlap on one GPU (two streams or two host
 * threads) race.
 */
#define GDN2_STATIC_SCRATCH_BYTES 75497472
int gdn2_chunk_fwd_static(const void *q, const void *k, const void *v, const void *g,
                          const void *b, const void *w, int io_dtype, int g_dtype, void *o,
                          const float *initial_state, float *final_state, const float *A_log,
                          const float *dt_bias, float lower_bound, const int64_t *cu_seqlens,
                          const int64_t *cu_seqlens_host, int num_seqs, int B, int T, int H,
                          int K, int V, float scale, unsigned flags, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* GDN2_HIP_H */
