// Chunk op for float32 inputs with 128 < d_k <= 256 (gfx950).
//
// At this key width the MFMA chunk kernels' per-(chunk, head) workspace is
// 231 KB in fp32, more than a CU's 160 KB of LDS, so the float32 chunk op
// (reference chunk_gdn2.py:1268-1434, which accepts d_k <= 256 in any dtype,
// :1380-1382) runs the recurrence token by token here, in fp32 throughout:
//
//   P_t = Diag(e^{g_t}) S_{t-1},  r = P_t^T (b_t * k_t),  u = w_t * v_t - r,
//   S_t = P_t + k_t u^T,  o_t = S_t^T q_t           (gdn2.py:156-179)
//
// with q, k L2-normalised (F.normalize, eps 1e-6) and q scaled in-kernel.
//
// Mapping: one workgroup per (sequence, head, slice of up to 128 value
// columns) with one wave per 16 columns (at most 8 waves, so that a wave may
// hold 256 registers; V <= 256 is two slices).  Lane l of a wave holds state
// rows 4l .. 4l+3 of its 16 columns in registers (64 floats), so sums over
// the value columns stay inside a lane and sums over the key rows are one
// butterfly reduction of 16 column partials across the wave (reduce16): every
// lane ends with the total of one column and the totals are broadcast with
// v_readlane.  The waves of a head never exchange data in the forward.
//
// Training: the forward also stores each chunk's start state (every 64
// tokens, [nc, H, K, V] fp32, the "hs" region of the training workspace).
// The backward walks the chunks in reverse: from the chunk's start state it
// recomputes the chunk's decayed states P_t (to a per-(sequence, head)
// scratch) and values u_t (LDS), then runs the reverse recurrence
//
//   dS += q dO^T,  dq = S_t dO,  dk = dS u,  du = dS^T k,  dv = du * w,
//   dw = du * v,  dr = -du,  de = P_t dr,  dP = dS + e dr^T,
//   dg = rowsum(dP * P_t),  dS <- Diag(e^{g_t}) dP
//
// (the VJP of the recurrence above, e = b * k).  The per-row sums of the
// waves are combined through LDS per token (the second slice's sums go to a
// workspace plane); a second kernel adds the slices, applies db = de * k,
// dk += de * b and the L2-norm and scale chain rule per (token, head) row.
#include <hip/hip_runtime.h>

#include "gdn2_chunk.h"
#include "gdn2_internal.h"

namespace gdn2 {

namespace {

constexpr int kCols = 16;     // value columns per wave
constexpr int kMaxWaves = 8;  // value columns per workgroup: 128
constexpr int kSliceCols = kMaxWaves * kCols;
constexpr int kMaxV = 2 * kSliceCols;
constexpr int kMaxK = 256;

struct WideParams {
    const float *q, *k, *v, *g, *b, *w;
    float *o;
    const float *h0;
    float *ht;
    const float *A_log, *dt_bias;
    float lower_bound;
    const int64_t *cu_seqlens;
    int num_seqs, T, H, K, V, nt;
    float scale;
    unsigned flags;
    int vec_ok;
    float *hs;  // chunk start states [nc, H, K, V] or null
    // backward
    const float *dout, *dht;
    float *dq, *dk, *dv, *dg, *db, *dw, *dh0;
    float *pws;   // per (sequence, head, slice): the decayed states of one chunk
    float *part;  // second slice's row sums dq, dk, de, dg: 4 planes of [rows, K]
    int64_t rows; // B * T * H
    int nsl;      // value slices
};

__device__ __forceinline__ float bcast(float x, int src)
{
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(x), src));
}

// x[c] summed over the 64 lanes of the wave, for c = (lane >> 2) & 15: a
// reduce-scatter butterfly (lane bit 5 picks column bit 3, bit 4 bit 2, bit 3
// bit 1, bit 2 bit 0), then the last two lane bits summed.  17 exchanges
// instead of 16 full reductions.
__device__ __forceinline__ float reduce16(const float (&x)[16])
{
    const int lane = threadIdx.x & (kWave - 1);
    float a[8], b[4], c[2];
    const bool h5 = (lane & 32) != 0, h4 = (lane & 16) != 0, h3 = (lane & 8) != 0, h2 = (lane & 4) != 0;
#pragma unroll
    for (int j = 0; j < 8; ++j)
        a[j] = (h5 ? x[8 + j] : x[j]) + __shfl_xor(h5 ? x[j] : x[8 + j], 32, kWave);
#pragma unroll
    for (int j = 0; j < 4; ++j)
        b[j] = (h4 ? a[4 + j] : a[j]) + __shfl_xor(h4 ? a[j] : a[4 + j], 16, kWave);
#pragma unroll
    for (int j = 0; j < 2; ++j)
        c[j] = (h3 ? b[2 + j] : b[j]) + __shfl_xor(h3 ? b[j] : b[2 + j], 8, kWave);
    float d = (h2 ? c[1] : c[0]) + __shfl_xor(h2 ? c[0] : c[1], 4, kWave);
    d += __shfl_xor(d, 2, kWave);
    d += __shfl_xor(d, 1, kWave);
    return d;
}

// The token's normalised rows and gates of this lane's four key rows.
struct TokenRows {
    float q[4], k[4], e[4], a[4];
    float invq, invk;
};

__device__ __forceinline__ void token_rows(const WideParams &p, int h, int64_t tok, int r0, float a_log,
                                           const float (&dtb)[4], bool sig_b, TokenRows &t)
{
    const int64_t rk = (tok * p.H + h) * p.K;
    float qv[4], kv[4], gv[4], bv[4];
    load4(p.q, rk, r0, p.K, true, p.vec_ok, qv);
    load4(p.k, rk, r0, p.K, true, p.vec_ok, kv);
    load4(p.g, rk, r0, p.K, true, p.vec_ok, gv);
    load4(p.b, rk, r0, p.K, true, p.vec_ok, bv);
    float qq = 0.f, kk = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        qq = fmaf(qv[i], qv[i], qq);
        kk = fmaf(kv[i], kv[i], kk);
    }
    qq = wave_sum(qq);
    kk = wave_sum(kk);
    const bool l2 = (p.flags & GDN2_FLAG_L2NORM_QK) != 0;
    const bool gate = (p.flags & GDN2_FLAG_GATE_IN_KERNEL) != 0;
    const int use_lb = (p.flags & GDN2_FLAG_LOWER_BOUND) != 0;
    t.invq = l2 ? 1.0f / fmaxf(sqrtf(qq), 1e-6f) : 1.0f;
    t.invk = l2 ? 1.0f / fmaxf(sqrtf(kk), 1e-6f) : 1.0f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        t.q[i] = qv[i] * t.invq * p.scale;
        t.k[i] = kv[i] * t.invk;
        const float bb = sig_b ? sigmoid_f(bv[i]) : bv[i];
        t.e[i] = bb * t.k[i];
        const float gk = gate ? gate_activation(gv[i], a_log, dtb[i], use_lb, p.lower_bound) : gv[i];
        t.a[i] = expf(gk);
    }
}

__device__ __forceinline__ int64_t hs_row(const WideParams &p, int64_t gc, int h)
{
    return (gc * p.H + h) * static_cast<int64_t>(p.K) * p.V;
}

__global__ __launch_bounds__(512) void wide_fwd_kernel(WideParams p)
{
    const int pair = blockIdx.x / p.nsl, slice = blockIdx.x % p.nsl;
    const int n = pair / p.H, h = pair % p.H;
    const int lane = threadIdx.x & (kWave - 1), wv = threadIdx.x / kWave;
    const int c0 = kSliceCols * slice + kCols * wv, r0 = 4 * lane, myc = (lane >> 2) & 15;
    const int K = p.K, V = p.V;
    int64_t bos, len;
    const int cb = seq_chunk_base(p, n, bos, len);
    const bool sig = (p.flags & GDN2_FLAG_SIGMOID_BW) != 0;
    const bool gate = (p.flags & GDN2_FLAG_GATE_IN_KERNEL) != 0;
    const float a_log = gate ? p.A_log[h] : 0.0f;
    float dtb[4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
        dtb[i] = (gate && p.dt_bias && r0 + i < K) ? p.dt_bias[static_cast<int64_t>(h) * K + r0 + i] : 0.0f;

    float S[4][kCols];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < kCols; ++j)
            S[i][j] = (p.h0 && r0 + i < K && c0 + j < V)
                          ? p.h0[state_index(p.flags, n, h, r0 + i, c0 + j, p.H, K, V)]
                          : 0.0f;

    for (int64_t t = 0; t < len; ++t) {
        if (p.hs && (t % kChunk) == 0) {
            float *dst = p.hs + hs_row(p, cb + t / kChunk, h);
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < kCols; ++j)
                    if (r0 + i < K && c0 + j < V) dst[static_cast<int64_t>(r0 + i) * V + c0 + j] = S[i][j];
        }
        const int64_t tok = bos + t;
        TokenRows tr;
        token_rows(p, h, tok, r0, a_log, dtb, sig, tr);
        const int64_t rv = (tok * p.H + h) * V;
        const bool col_ok = c0 + myc < V;
        const float vme = col_ok ? p.v[rv + c0 + myc] : 0.0f;
        float wme = col_ok ? p.w[rv + c0 + myc] : 0.0f;
        if (sig) wme = sigmoid_f(wme);
        float kq = 0.f;
#pragma unroll
        for (int i = 0; i < 4; ++i) kq = fmaf(tr.k[i], tr.q[i], kq);
        kq = wave_sum(kq);
        float xr[kCols], xo[kCols];
#pragma unroll
        for (int j = 0; j < kCols; ++j) {
            xr[j] = 0.f;
            xo[j] = 0.f;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                S[i][j] *= tr.a[i];
                xr[j] = fmaf(S[i][j], tr.e[i], xr[j]);
                xo[j] = fmaf(S[i][j], tr.q[i], xo[j]);
            }
        }
        const float r = reduce16(xr), po = reduce16(xo);
        const float u = wme * vme - r;  // column myc
        if ((lane & 3) == 0 && col_ok) p.o[rv + c0 + myc] = fmaf(kq, u, po);
#pragma unroll
        for (int j = 0; j < kCols; ++j) {
            const float uj = bcast(u, 4 * j);
#pragma unroll
            for (int i = 0; i < 4; ++i) S[i][j] = fmaf(tr.k[i], uj, S[i][j]);
        }
    }
    if (p.ht) {
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < kCols; ++j)
                if (r0 + i < K && c0 + j < V)
                    p.ht[state_index(p.flags, n, h, r0 + i, c0 + j, p.H, K, V)] = S[i][j];
    }
}

// Decayed-state scratch of one (sequence, head): [64 tokens][W waves][16
// groups of 4 values][64 lanes] float4, so each store / load instruction of a
// wave moves 1 KB of consecutive bytes.
__device__ __forceinline__ float4 *pws_slot(const WideParams &p, int item, int W, int tt, int wv, int grp)
{
    const int64_t base = static_cast<int64_t>(item) * kChunk * W * kCols * 4 * kWave;
    const int lane = threadIdx.x & (kWave - 1);
    return reinterpret_cast<float4 *>(p.pws + base) + ((static_cast<int64_t>(tt) * W + wv) * 16 + grp) * kWave + lane;
}

__global__ __launch_bounds__(512) void wide_bwd_kernel(WideParams p)
{
    __shared__ float sU[kChunk][kSliceCols];      // u of the chunk's tokens
    __shared__ float sPart[kMaxWaves][4][kMaxK];  // one token's per-wave row partials
    __shared__ float sInv[kChunk][2];             // 1 / ||q||, 1 / ||k||

    const int item = blockIdx.x;
    const int pair = item / p.nsl, slice = item % p.nsl;
    const int n = pair / p.H, h = pair % p.H;
    const int W = blockDim.x / kWave;
    const int lane = threadIdx.x & (kWave - 1), wv = threadIdx.x / kWave;
    const int cw = kCols * wv;  // the wave's first column within the slice
    const int c0 = kSliceCols * slice + cw, r0 = 4 * lane, myc = (lane >> 2) & 15;
    const int K = p.K, V = p.V;
    int64_t bos, len;
    const int cb = seq_chunk_base(p, n, bos, len);
    const float dtb[4] = {0.f, 0.f, 0.f, 0.f};

    float dS[4][kCols];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < kCols; ++j)
            dS[i][j] = (p.dht && r0 + i < K && c0 + j < V)
                           ? p.dht[state_index(p.flags, n, h, r0 + i, c0 + j, p.H, K, V)]
                           : 0.0f;

    const int nch = static_cast<int>((len + kChunk - 1) / kChunk);
    for (int jc = nch - 1; jc >= 0; --jc) {
        const int64_t t0 = static_cast<int64_t>(jc) * kChunk;
        const int nt = static_cast<int>(len - t0 < kChunk ? len - t0 : kChunk);
        // Recompute the chunk from its start state: P_t to the scratch, u_t to LDS.
        float S[4][kCols];
        {
            const float *src = p.hs + hs_row(p, cb + jc, h);
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < kCols; ++j)
                    S[i][j] = (r0 + i < K && c0 + j < V) ? src[static_cast<int64_t>(r0 + i) * V + c0 + j] : 0.0f;
        }
        for (int tt = 0; tt < nt; ++tt) {
            const int64_t tok = bos + t0 + tt;
            TokenRows tr;
            token_rows(p, h, tok, r0, 0.0f, dtb, false, tr);
            if (threadIdx.x == 0) {
                sInv[tt][0] = tr.invq;
                sInv[tt][1] = tr.invk;
            }
            const int64_t rv = (tok * p.H + h) * V;
            const bool col_ok = c0 + myc < V;
            const float vme = col_ok ? p.v[rv + c0 + myc] : 0.0f;
            const float wme = col_ok ? p.w[rv + c0 + myc] : 0.0f;
            float xr[kCols];
#pragma unroll
            for (int j = 0; j < kCols; ++j) {
                xr[j] = 0.f;
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    S[i][j] *= tr.a[i];
                    xr[j] = fmaf(S[i][j], tr.e[i], xr[j]);
                }
            }
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int jj = 0; jj < 4; ++jj)
                    *pws_slot(p, item, W, tt, wv, 4 * i + jj) =
                        make_float4(S[i][4 * jj], S[i][4 * jj + 1], S[i][4 * jj + 2], S[i][4 * jj + 3]);
            const float u = wme * vme - reduce16(xr);
            if ((lane & 3) == 0) sU[tt][cw + myc] = u;
#pragma unroll
            for (int j = 0; j < kCols; ++j) {
                const float uj = bcast(u, 4 * j);
#pragma unroll
                for (int i = 0; i < 4; ++i) S[i][j] = fmaf(tr.k[i], uj, S[i][j]);
            }
        }
        __syncthreads();  // sU, sInv of the chunk; the scratch stores precede their loads below
        for (int tt = nt - 1; tt >= 0; --tt) {
            const int64_t tok = bos + t0 + tt;
            const int64_t rk = (tok * p.H + h) * K, rv = (tok * p.H + h) * V;
            float qv[4], kv[4], gv[4], bv[4];
            load4(p.q, rk, r0, K, true, p.vec_ok, qv);
            load4(p.k, rk, r0, K, true, p.vec_ok, kv);
            load4(p.g, rk, r0, K, true, p.vec_ok, gv);
            load4(p.b, rk, r0, K, true, p.vec_ok, bv);
            const float invq = sInv[tt][0], invk = sInv[tt][1];
            float qh[4], kh[4], e[4], a[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                qh[i] = qv[i] * invq * p.scale;
                kh[i] = kv[i] * invk;
                e[i] = bv[i] * kh[i];
                a[i] = expf(gv[i]);
            }
            float dO[kCols], u[kCols];
#pragma unroll
            for (int j = 0; j < kCols; ++j) {
                dO[j] = c0 + j < V ? p.dout[rv + c0 + j] : 0.0f;
                u[j] = sU[tt][cw + j];
            }
            const bool col_ok = c0 + myc < V;
            const float vme = col_ok ? p.v[rv + c0 + myc] : 0.0f;
            const float wme = col_ok ? p.w[rv + c0 + myc] : 0.0f;
            float P[4][kCols];
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int jj = 0; jj < 4; ++jj) {
                    const float4 x = *pws_slot(p, item, W, tt, wv, 4 * i + jj);
                    P[i][4 * jj] = x.x;
                    P[i][4 * jj + 1] = x.y;
                    P[i][4 * jj + 2] = x.z;
                    P[i][4 * jj + 3] = x.w;
                }
            float dqh[4], dkh[4], deh[4], dgh[4], xd[kCols];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                dqh[i] = 0.f;
                dkh[i] = 0.f;
#pragma unroll
                for (int j = 0; j < kCols; ++j) {
                    const float st = fmaf(kh[i], u[j], P[i][j]);
                    dS[i][j] = fmaf(qh[i], dO[j], dS[i][j]);
                    dqh[i] = fmaf(st, dO[j], dqh[i]);
                    dkh[i] = fmaf(dS[i][j], u[j], dkh[i]);
                }
            }
#pragma unroll
            for (int j = 0; j < kCols; ++j) {
                xd[j] = 0.f;
#pragma unroll
                for (int i = 0; i < 4; ++i) xd[j] = fmaf(dS[i][j], kh[i], xd[j]);
            }
            const float du = reduce16(xd);  // column myc
            if ((lane & 3) == 0 && col_ok) {
                p.dv[rv + c0 + myc] = du * wme;
                p.dw[rv + c0 + myc] = du * vme;
            }
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                deh[i] = 0.f;
                dgh[i] = 0.f;
            }
#pragma unroll
            for (int j = 0; j < kCols; ++j) {
                const float dr = -bcast(du, 4 * j);
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    deh[i] = fmaf(P[i][j], dr, deh[i]);
                    const float dp = fmaf(e[i], dr, dS[i][j]);
                    dgh[i] = fmaf(dp, P[i][j], dgh[i]);
                    dS[i][j] = a[i] * dp;
                }
            }
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                sPart[wv][0][r0 + i] = dqh[i];
                sPart[wv][1][r0 + i] = dkh[i];
                sPart[wv][2][r0 + i] = deh[i];
                sPart[wv][3][r0 + i] = dgh[i];
            }
            __syncthreads();
            for (int idx = threadIdx.x; idx < 4 * K; idx += blockDim.x) {
                const int qn = idx / K, r = idx - qn * K;
                float s = 0.f;
                for (int x = 0; x < W; ++x) s += sPart[x][qn][r];
                float *dst = slice ? p.part + qn * p.rows * K
                                   : (qn == 0 ? p.dq : (qn == 1 ? p.dk : (qn == 2 ? p.db : p.dg)));
                dst[rk + r] = s;
            }
            __syncthreads();
        }
    }
    if (p.dh0) {
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < kCols; ++j)
                if (r0 + i < K && c0 + j < V)
                    p.dh0[state_index(p.flags, n, h, r0 + i, c0 + j, p.H, K, V)] = dS[i][j];
    }
}

// Per (token, head) row, from the backward kernel's gradients with respect to
// the normalised q (dq), normalised k (dk, without the erase path) and the
// erase vector e = b * k (db): db = de * k, dk += de * b, then the scale and
// the VJP of x / max(||x||, 1e-6) for q and k.  In place; one wave per row.
__global__ __launch_bounds__(256) void wide_bwd_finish_kernel(WideParams p, int64_t rows)
{
    const int64_t row = static_cast<int64_t>(blockIdx.x) * 4 + threadIdx.x / kWave;
    if (row >= rows) return;
    const int lane = threadIdx.x & (kWave - 1), r0 = 4 * lane, K = p.K;
    const int64_t off = row * K;
    float qv[4], kv[4], bv[4], dq[4], dk[4], de[4];
    load4(p.q, off, r0, K, true, p.vec_ok, qv);
    load4(p.k, off, r0, K, true, p.vec_ok, kv);
    load4(p.b, off, r0, K, true, p.vec_ok, bv);
    load4(p.dq, off, r0, K, true, p.vec_ok, dq);
    load4(p.dk, off, r0, K, true, p.vec_ok, dk);
    load4(p.db, off, r0, K, true, p.vec_ok, de);
    if (p.nsl > 1) {
        // The second value slice's row sums.
        float x[4];
        load4(p.part, off, r0, K, true, p.vec_ok, x);
#pragma unroll
        for (int i = 0; i < 4; ++i) dq[i] += x[i];
        load4(p.part + rows * K, off, r0, K, true, p.vec_ok, x);
#pragma unroll
        for (int i = 0; i < 4; ++i) dk[i] += x[i];
        load4(p.part + 2 * rows * K, off, r0, K, true, p.vec_ok, x);
#pragma unroll
        for (int i = 0; i < 4; ++i) de[i] += x[i];
        float dg[4];
        load4(p.dg, off, r0, K, true, p.vec_ok, dg);
        load4(p.part + 3 * rows * K, off, r0, K, true, p.vec_ok, x);
#pragma unroll
        for (int i = 0; i < 4; ++i) dg[i] += x[i];
        store4(p.dg, off, r0, K, dg);
    }
    const bool l2 = (p.flags & GDN2_FLAG_L2NORM_QK) != 0;
    float qq = 0.f, kk = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        qq = fmaf(qv[i], qv[i], qq);
        kk = fmaf(kv[i], kv[i], kk);
    }
    qq = wave_sum(qq);
    kk = wave_sum(kk);
    const float nq = sqrtf(qq), nk = sqrtf(kk);
    const float invk = l2 ? 1.0f / fmaxf(nk, 1e-6f) : 1.0f;
    float gq[4], gk[4], dbo[4], pq = 0.f, pk = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const float kh = kv[i] * invk;
        dbo[i] = de[i] * kh;
        gq[i] = dq[i] * p.scale;      // gradient of q / max(||q||, eps)
        gk[i] = fmaf(de[i], bv[i], dk[i]);  // gradient of k / max(||k||, eps)
        pq = fmaf(qv[i], gq[i], pq);
        pk = fmaf(kv[i], gk[i], pk);
    }
    float rq[4], rk[4];
    if (l2) {
        pq = wave_sum(pq);
        pk = wave_sum(pk);
        const bool bq = nq > 1e-6f, bk = nk > 1e-6f;
        const float iq = 1.0f / fmaxf(nq, 1e-6f), ik = 1.0f / fmaxf(nk, 1e-6f);
        // y = x / n:  dx = (dy - y (y . dy)) / n for n > eps, dy / eps otherwise.
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            rq[i] = bq ? (gq[i] - qv[i] * iq * (pq * iq)) * iq : gq[i] * 1e6f;
            rk[i] = bk ? (gk[i] - kv[i] * ik * (pk * ik)) * ik : gk[i] * 1e6f;
        }
    } else {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            rq[i] = gq[i];
            rk[i] = gk[i];
        }
    }
    store4(p.dq, off, r0, K, rq);
    store4(p.dk, off, r0, K, rk);
    store4(p.db, off, r0, K, dbo);
}

WideParams wide_params(const void *q, const void *k, const void *v, const void *g, const void *b,
                       const void *w, const int64_t *cu_seqlens, int num_seqs, int T, int H, int K,
                       int V, float scale, unsigned flags)
{
    WideParams p{};
    p.q = static_cast<const float *>(q);
    p.k = static_cast<const float *>(k);
    p.v = static_cast<const float *>(v);
    p.g = static_cast<const float *>(g);
    p.b = static_cast<const float *>(b);
    p.w = static_cast<const float *>(w);
    p.cu_seqlens = cu_seqlens;
    p.num_seqs = num_seqs;
    p.T = T;
    p.H = H;
    p.K = K;
    p.V = V;
    p.nt = (T + kChunk - 1) / kChunk;
    p.scale = scale;
    p.flags = flags;
    p.vec_ok = (K % 4) == 0;
    return p;
}

// Waves per workgroup (every slice gets the first slice's count; columns at
// or beyond V are masked) and value slices.
int waves_for(int V) { return (V < kSliceCols ? V + kCols - 1 : kSliceCols) / kCols; }
int slices_for(int V) { return (V + kSliceCols - 1) / kSliceCols; }

int64_t pws_bytes(int64_t pairs, int V)
{
    return round_up(pairs * slices_for(V) * kChunk * waves_for(V) * kCols * 4 * kWave * 4, 256);
}

}  // namespace

bool chunk_wide(int K, int io_dtype) { return io_dtype == GDN2_DTYPE_F32 && K > 128 && K <= kMaxK; }

size_t wide_train_workspace_bytes(int B, int T, int H, int K, int V, const int64_t *cu_host, int num_seqs)
{
    const int64_t nc = count_chunks(B, T, cu_host, num_seqs);
    return static_cast<size_t>(round_up(nc * H * static_cast<int64_t>(K) * V * 4, 256));
}

size_t wide_bwd_workspace_bytes(int B, int T, int H, int K, int V, const int64_t *cu_host, int num_seqs)
{
    const int64_t nc = count_chunks(B, T, cu_host, num_seqs);
    if (nc == 0) return 0;
    const int64_t pairs = static_cast<int64_t>(cu_host ? num_seqs : B) * H;
    const int64_t rows = static_cast<int64_t>(B) * T * H;
    const int64_t part = slices_for(V) > 1 ? 4 * rows * K * 4 : 0;
    return static_cast<size_t>(pws_bytes(pairs, V) + part);
}

int launch_chunk_fwd_wide(const ChunkFwdArgs &a, int g_dtype, hipStream_t stream)
{
    if (a.V > kMaxV || a.z || a.conv_w[0] || a.stages != 3 || g_dtype != GDN2_DTYPE_F32)
        return GDN2_ERR_UNSUPPORTED;
    const bool train = (a.flags & GDN2_FLAG_SAVE_FOR_BWD) != 0;
    if (train && (!a.workspace ||
                  a.workspace_bytes < wide_train_workspace_bytes(a.B, a.T, a.H, a.K, a.V, a.cu_host, a.num_seqs)))
        return GDN2_ERR_WORKSPACE;
    const int64_t items = static_cast<int64_t>(a.num_seqs) * a.H * slices_for(a.V);
    if (items > 2147483647LL) return GDN2_ERR_UNSUPPORTED;
    if (items == 0) return GDN2_OK;
    WideParams p = wide_params(a.q, a.k, a.v, a.g, a.b, a.w, a.cu_seqlens, a.num_seqs, a.T, a.H, a.K, a.V,
                               a.scale, a.flags);
    p.o = static_cast<float *>(a.o);
    p.h0 = a.h0;
    p.ht = a.ht;
    p.A_log = a.A_log;
    p.dt_bias = a.dt_bias;
    p.lower_bound = a.lower_bound;
    p.hs = train ? static_cast<float *>(a.workspace) : nullptr;
    p.nsl = slices_for(a.V);
    hipLaunchKernelGGL(wide_fwd_kernel, dim3(static_cast<unsigned>(items)), dim3(kWave * waves_for(a.V)), 0,
                       stream, p);
    return hipGetLastError() == hipSuccess ? GDN2_OK : GDN2_ERR_LAUNCH;
}

int launch_chunk_bwd_wide(const ChunkBwdArgs &a, int g_dtype, hipStream_t stream)
{
    if (a.V > kMaxV || g_dtype != GDN2_DTYPE_F32) return GDN2_ERR_UNSUPPORTED;
    const size_t need_saved = wide_train_workspace_bytes(a.B, a.T, a.H, a.K, a.V, a.cu_host, a.num_seqs);
    const size_t need_ws = wide_bwd_workspace_bytes(a.B, a.T, a.H, a.K, a.V, a.cu_host, a.num_seqs);
    if (need_saved > 0 && (!a.saved || a.saved_bytes < need_saved)) return GDN2_ERR_WORKSPACE;
    if (need_ws > 0 && (!a.workspace || a.workspace_bytes < need_ws)) return GDN2_ERR_WORKSPACE;
    const int64_t pairs = static_cast<int64_t>(a.num_seqs) * a.H;
    const int64_t items = pairs * slices_for(a.V);
    if (items > 2147483647LL) return GDN2_ERR_UNSUPPORTED;
    if (items == 0) return GDN2_OK;
    WideParams p = wide_params(a.q, a.k, a.v, a.g, a.b, a.w, a.cu_seqlens, a.num_seqs, a.T, a.H, a.K, a.V,
                               a.scale, a.flags);
    p.hs = const_cast<float *>(static_cast<const float *>(a.saved));
    p.dout = static_cast<const float *>(a.dout);
    p.dht = a.dht;
    p.dq = static_cast<float *>(a.dq);
    p.dk = static_cast<float *>(a.dk);
    p.dv = static_cast<float *>(a.dv);
    p.dg = static_cast<float *>(a.dg);
    p.db = static_cast<float *>(a.db);
    p.dw = static_cast<float *>(a.dw);
    p.dh0 = a.dh0;
    p.nsl = slices_for(a.V);
    p.rows = static_cast<int64_t>(a.B) * a.T * a.H;
    p.pws = static_cast<float *>(a.workspace);
    p.part = p.nsl > 1 ? reinterpret_cast<float *>(static_cast<unsigned char *>(a.workspace) + pws_bytes(pairs, a.V))
                       : nullptr;
    hipLaunchKernelGGL(wide_bwd_kernel, dim3(static_cast<unsigned>(items)), dim3(kWave * waves_for(a.V)), 0,
                       stream, p);
    if (hipGetLastError() != hipSuccess) return GDN2_ERR_LAUNCH;
    if (p.rows > 0) {
        hipLaunchKernelGGL(wide_bwd_finish_kernel, dim3(static_cast<unsigned>((p.rows + 3) / 4)), dim3(256), 0,
                           stream, p, p.rows);
        if (hipGetLastError() != hipSuccess) return GDN2_ERR_LAUNCH;
    }
    return GDN2_OK;
}

namespace {

// Chunk start states of a wide training forward ([nc, H, K, V] fp32) as the
// intermediate states of chunk_gdn2: [nc, H, K, V] or [nc, H, V, K].
__global__ __launch_bounds__(256) void wide_states_kernel(const float *hs, float *out, int trans, int64_t total,
                                                          int K, int V)
{
    const int64_t idx = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    if (idx >= total) return;
    const int64_t kv = static_cast<int64_t>(K) * V;
    const int64_t base = idx / kv * kv, e = idx - base;
    if (!trans) {
        out[idx] = hs[idx];
        return;
    }
    const int v = static_cast<int>(e / K), k = static_cast<int>(e - static_cast<int64_t>(v) * K);
    out[idx] = hs[base + static_cast<int64_t>(k) * V + v];
}

}  // namespace

hipError_t launch_chunk_states_wide(const void *hs, void *out, bool transpose, int64_t nc, int H, int K, int V,
                                    hipStream_t stream)
{
    const int64_t total = nc * H * K * V;
    if (total == 0) return hipSuccess;
    hipLaunchKernelGGL(wide_states_kernel, dim3(static_cast<unsigned>((total + 255) / 256)), dim3(256), 0, stream,
                       static_cast<const float *>(hs), static_cast<float *>(out), int(transpose), total, K, V);
    return hipGetLastError();
}

}  // namespace gdn2
