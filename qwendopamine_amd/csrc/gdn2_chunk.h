// Definitions shared by the chunkwise forward and backward kernels (gfx950).
//
// Chunk geometry: C = 64 tokens per chunk, 16-token sub-blocks, chunks of
// all sequences numbered consecutively (gc), one workspace blob per
// (chunk, head) written by the forward prep kernel.  The blob layout, the
// chunk location helpers and the in-block decay scans live here so that the
// backward kernels read exactly what the forward wrote.
#pragma once

#include <type_traits>

#include "gdn2_mfma.h"

namespace gdn2 {

// Native 16-byte vector: loads and stores of it stay single instructions and
// arrays of it stay in registers (struct copies of uint4 lower to memcpy).
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

constexpr int kChunk = 64;
constexpr float kLog2e = 1.4426950408889634f;
// Largest in-block decay span (log2 units, ~ e^80) for which the factored
// diagonal block keeps every factor inside the normal fp32/bf16 range.
constexpr float kDiagSpanLimit2 = 115.0f;

struct ChunkParams {
    const void *q, *k, *v, *g, *b, *w;
    void *o;
    const float *h0;
    float *ht;
    const float *A_log;
    const float *dt_bias;
    float lower_bound;
    const int64_t *cu_seqlens;
    int num_seqs, T, H, K, V;
    int nt;  // chunks per sequence without cu_seqlens
    float scale;
    unsigned flags;
    int vec_ok;  // K % 4 == 0: 4-wide input loads
    void *ws;    // per-chunk blobs (prep writes, scan reads)
    // Training mode (both null otherwise): the scan also writes, per chunk,
    // its start state (hs) and its U (us), in K16 A-order blocks of width
    // VP = V rounded up to 16.
    void *hs, *us;
    int VP;
    // Gated output norm in the scan (inference, BV == V): gate rows z (token
    // row stride ldz, head h at column h * V), weight nw [V], eps.  z == null
    // leaves the outputs unnormalised.
    const void *z;
    int64_t ldz;
    const void *nw;
    float eps;
    // Short convolutions in the kernels (inference, conv_w[0] != null): q, k
    // and v are the raw projections (token row strides ldq, ldk, ldv; head h
    // at column h * K or h * V), conv_w[i] the [H * K or H * V][4] taps of
    // q, k, v in the input dtype, conv_silu the SiLU after each; rows before
    // a sequence's first token read as zero.
    const void *conv_w[3];
    int64_t ldq, ldk, ldv;
    int conv_silu;
};

// Per (chunk, head) blob, in storage elements.
template <PrecKind PK, int KP>
struct Blob {
    using st = typename Prec<PK>::st;
    static constexpr int64_t X = 0;                 // [64][64]   (I + L)^{-1}
    static constexpr int64_t WN = 4096;             // [64][KP]   -W
    static constexpr int64_t QB = 4096 + 64 * KP;   // [64][KP]   Qbar
    static constexpr int64_t AQ = 4096 + 128 * KP;  // [64][64]   Aqk
    static constexpr int64_t KT = 8192 + 128 * KP;  // [KP][64]   Ktilde^T
    static constexpr int64_t GL = 8192 + 192 * KP;  // KP floats  exp(G_last)
    static constexpr int64_t SIZE = GL + KP * 4 / static_cast<int64_t>(sizeof(st));
    static constexpr int64_t BYTES = SIZE * static_cast<int64_t>(sizeof(st));
    static_assert(BYTES % 16 == 0, "blob must be a whole number of 16-byte units");
};

template <class PP>
__device__ __forceinline__ void locate_chunk(const PP &p, int gc, int &n, int &j,
                                             int64_t &bos, int64_t &len)
{
    if (!p.cu_seqlens) {
        n = gc / p.nt;
        j = gc % p.nt;
        bos = static_cast<int64_t>(n) * p.T;
        len = p.T;
        return;
    }
    int acc = 0;
    n = 0;
    j = 0;
    bos = 0;
    len = 0;
    for (int s = 0; s < p.num_seqs; ++s) {
        const int64_t b0 = p.cu_seqlens[s], e0 = p.cu_seqlens[s + 1];
        const int c = static_cast<int>((e0 - b0 + kChunk - 1) / kChunk);
        if (gc < acc + c) {
            n = s;
            j = gc - acc;
            bos = b0;
            len = e0 - b0;
            return;
        }
        acc += c;
    }
}

template <class PP>
__device__ __forceinline__ int seq_chunk_base(const PP &p, int n, int64_t &bos,
                                              int64_t &len)
{
    if (!p.cu_seqlens) {
        bos = static_cast<int64_t>(n) * p.T;
        len = p.T;
        return n * p.nt;
    }
    int acc = 0;
    for (int s = 0; s < n; ++s)
        acc += static_cast<int>((p.cu_seqlens[s + 1] - p.cu_seqlens[s] + kChunk - 1) / kChunk);
    bos = p.cu_seqlens[n];
    len = p.cu_seqlens[n + 1] - bos;
    return acc;
}

// 4 consecutive channels c0..c0+3 of one row, zero outside [0, K) or when !ok.
template <typename T>
__device__ __forceinline__ void load4(const T *base, int64_t off, int c0, int K, bool ok, int vec_ok,
                                      float (&x)[4])
{
    if (ok && vec_ok && c0 + 4 <= K) {
        if constexpr (std::is_same<T, float>::value) {
            const float4 a = *reinterpret_cast<const float4 *>(base + off + c0);
            x[0] = a.x; x[1] = a.y; x[2] = a.z; x[3] = a.w;
        } else if constexpr (std::is_same<T, bf16_t>::value) {
            const uint2 u = *reinterpret_cast<const uint2 *>(base + off + c0);
            x[0] = __uint_as_float(u.x << 16);
            x[1] = __uint_as_float(u.x & 0xffff0000u);
            x[2] = __uint_as_float(u.y << 16);
            x[3] = __uint_as_float(u.y & 0xffff0000u);
        } else {
#pragma unroll
            for (int i = 0; i < 4; ++i) x[i] = io<T>::ld(base, off + c0 + i);
        }
        return;
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) x[i] = (ok && c0 + i < K) ? io<T>::ld(base, off + c0 + i) : 0.0f;
}

// Store 4 consecutive values x[0..3] at base[off + c0 ..]: one vector store
// when all four are in [0, n) and the address is aligned, else element-wise.
template <typename T>
__device__ __forceinline__ void store4(T *base, int64_t off, int c0, int n, const float (&x)[4])
{
    T *p = base + off + c0;
    if (c0 + 4 <= n && (reinterpret_cast<uintptr_t>(p) & (4 * sizeof(T) - 1)) == 0) {
        if constexpr (std::is_same<T, float>::value) {
            *reinterpret_cast<float4 *>(p) = make_float4(x[0], x[1], x[2], x[3]);
        } else if constexpr (std::is_same<T, bf16_t>::value) {
            *reinterpret_cast<uint2 *>(p) = make_uint2(f32x2_to_bf16x2_bits(x[0], x[1]),
                                                       f32x2_to_bf16x2_bits(x[2], x[3]));
        } else {
#pragma unroll
            for (int i = 0; i < 4; ++i) io<T>::st(p, i, x[i]);
        }
        return;
    }
#pragma unroll
    for (int i = 0; i < 4; ++i)
        if (c0 + i < n) io<T>::st(p, i, x[i]);
}

// Element (row k, column v) of the [K, V] state of (sequence n, head h) in a
// [N, H, K, V] array, or [N, H, V, K] with GDN2_FLAG_TRANSPOSE_STATE (the
// reference's transpose_state_layout).
__device__ __forceinline__ int64_t state_index(unsigned flags, int n, int h, int row, int col, int H,
                                               int K, int V)
{
    const int64_t base = static_cast<int64_t>(n) * H + h;
    return (flags & GDN2_FLAG_TRANSPOSE_STATE) ? (base * V + col) * K + row : (base * K + row) * V + col;
}

__device__ __forceinline__ float fexp2(float x) { return __builtin_amdgcn_exp2f(x); }

// Inclusive prefix sum over the 16 lanes of each DPP row (lanes 16r..16r+15),
// Hillis-Steele with row_shr:1,2,4,8; lanes shifted in from outside the row
// read 0 (bound_ctrl), so no masking is needed.
template <int CTRL>
__device__ __forceinline__ float dpp_row_shr(float x)
{
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), CTRL,
                                                                 0xf, 0xf, true));
}

__device__ __forceinline__ float row16_scan(float x)
{
    x += dpp_row_shr<0x111>(x);
    x += dpp_row_shr<0x112>(x);
    x += dpp_row_shr<0x114>(x);
    x += dpp_row_shr<0x118>(x);
    return x;
}

// Padded key width of the chunk kernels (d_k <= 256; 256 only for 16-bit io,
// whose blob still fits the scans' LDS once).
inline int kp_for(int K) { return K <= 32 ? 32 : (K <= 64 ? 64 : (K <= 128 ? 128 : 256)); }
inline bool chunk_k_supported(int K, int io_dtype) { return K <= 128 || (K <= 256 && io_dtype != GDN2_DTYPE_F32); }
inline int bv_for(int V) { return V <= 16 ? 16 : (V <= 32 ? 32 : 64); }

// Value-slice width of the sequential scans: the widest of 64/32/16 columns
// whose (sequence, head, slice) workgroups still cover the 256 CUs, so that
// few long sequences do not leave most of the chip idle.
inline int scan_bv(int num_pairs, int V)
{
    int bv = bv_for(V);
    while (bv > 16 && static_cast<int64_t>(num_pairs) * ((V + bv - 1) / bv) < 256) bv /= 2;
    return bv;
}

inline int64_t count_chunks(int B, int T, const int64_t *cu_host, int num_seqs)
{
    if (!cu_host) return static_cast<int64_t>(B) * ((T + kChunk - 1) / kChunk);
    int64_t c = 0;
    for (int i = 0; i < num_seqs; ++i) c += (cu_host[i + 1] - cu_host[i] + kChunk - 1) / kChunk;
    return c;
}

inline int64_t blob_bytes(int io_dtype, int KP)
{
    const bool f32 = io_dtype == GDN2_DTYPE_F32;
    switch (KP) {
    case 32: return f32 ? Blob<PrecKind::F32, 32>::BYTES : Blob<PrecKind::BF16, 32>::BYTES;
    case 64: return f32 ? Blob<PrecKind::F32, 64>::BYTES : Blob<PrecKind::BF16, 64>::BYTES;
    case 128: return f32 ? Blob<PrecKind::F32, 128>::BYTES : Blob<PrecKind::BF16, 128>::BYTES;
    default: return Blob<PrecKind::BF16, 256>::BYTES;
    }
}

inline int64_t round_up(int64_t x, int64_t a) { return (x + a - 1) / a * a; }

// Training workspace: the forward's blobs followed by what the backward
// re-reads (per-chunk start states and U in the MFMA operand precision),
// each region 256-byte aligned.
struct TrainLayout {
    int64_t blob, hs, us, total;
};

inline TrainLayout train_layout(int64_t nc, int H, int K, int V, int io_dtype)
{
    const int KP = kp_for(K);
    const int64_t VP = round_up(V, 16);
    const int64_t es = io_dtype == GDN2_DTYPE_F32 ? 4 : 2;
    TrainLayout t;
    t.blob = 0;
    t.hs = round_up(nc * H * blob_bytes(io_dtype, KP), 256);
    t.us = t.hs + round_up(nc * H * KP * VP * es, 256);
    t.total = t.us + round_up(nc * H * 64 * VP * es, 256);
    return t;
}

// Wait until at most N vector memory requests of this wave are outstanding
// (gfx9 s_waitcnt: vmcnt in bits 3:0 and 15:14; expcnt and lgkmcnt at their
// no-wait maxima).  Loads complete in issue order, so this waits for every
// request older than the N newest.
template <int N>
__device__ __forceinline__ void wait_vm_newest()
{
    static_assert(N >= 0 && N < 64, "vmcnt is a 6-bit count");
    __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}

// Backward scratch: per-chunk end-state gradients (dhs) and dY = X^T dU (dys).
struct BwdLayout {
    int64_t dhs, dys, total;
};

inline BwdLayout bwd_layout(int64_t nc, int H, int K, int V, int io_dtype)
{
    const int KP = kp_for(K);
    const int64_t VP = round_up(V, 16);
    const int64_t es = io_dtype == GDN2_DTYPE_F32 ? 4 : 2;
    BwdLayout t;
    t.dhs = 0;
    t.dys = round_up(nc * H * KP * VP * es, 256);
    t.total = t.dys + round_up(nc * H * 64 * VP * es, 256);
    return t;
}

}  // namespace gdn2
