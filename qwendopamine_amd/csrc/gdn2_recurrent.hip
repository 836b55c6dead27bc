// Token-serial gdn2 forward for decode steps and short prefills (gfx950).
//
// Arithmetic: reference models/gdn2/gdn2.py:156-179 (torch_recurrent_gdn2), per
// token and (sequence, value head):
//     S <- Diag(exp(g)) S ;  r = S^T (b*k) ;  u = w*v - r ;  S <- S + k u^T ;  o = S^T q
// with q, k L2-normalised (F.normalize, eps 1e-6) and q scaled, fused in-kernel.
// Interface: reference fused_recurrent_gdn2.py:344-458 (GVA, varlen, in-place
// final state, optional in-kernel gate activation).
//
// Mapping.  One 256-thread workgroup owns the float32 state slab S[:, c0:c0+VB]
// of one (sequence, value head) -- K rows of VB columns, V contiguous in HBM.
// Thread t holds a float4 of columns 4*(t % TPR) for rows (t / TPR) + i*RG,
// i < NR, in VGPRs for the whole token loop, so a decode step reads and
// writes every state byte exactly once with 16-byte coalesced accesses
// (one wavefront row = 2 x 512 B for VB = 128).  The two K-reductions of a
// token (r = S^T e and the S^T q partial) are summed across the row groups of
// a wave with xor-shuffles and across the 4 waves through 4 KB of LDS.
// The output uses o = (Diag(a)S)^T q + u (k.q), so S is swept once per token.

#include "gdn2_common.h"
#include "gdn2_internal.h"

namespace gdn2 {


template <typename T>
struct vec4io;

template <>
struct vec4io<float> {
    static __device__ __forceinline__ float4 ld(const float *p, int64_t i)
    {
        return *reinterpret_cast<const float4 *>(p + i);
    }
    static __device__ __forceinline__ void st(float *p, int64_t i, float4 x)
    {
        *reinterpret_cast<float4 *>(p + i) = x;
    }
};

template <>
struct vec4io<bf16_t> {
    static __device__ __forceinline__ float4 ld(const bf16_t *p, int64_t i)
    {
        const uint2 u = *reinterpret_cast<const uint2 *>(p + i);
        return make_float4(__uint_as_float(u.x << 16), __uint_as_float(u.x & 0xffff0000u),
                           __uint_as_float(u.y << 16), __uint_as_float(u.y & 0xffff0000u));
    }
    static __device__ __forceinline__ void st(bf16_t *p, int64_t i, float4 x)
    {
        uint2 u;
        u.x = static_cast<uint32_t>(f32_to_bf16_bits(x.x)) |
              (static_cast<uint32_t>(f32_to_bf16_bits(x.y)) << 16);
        u.y = static_cast<uint32_t>(f32_to_bf16_bits(x.z)) |
              (static_cast<uint32_t>(f32_to_bf16_bits(x.w)) << 16);
        *reinterpret_cast<uint2 *>(p + i) = u;
    }
};

template <>
struct vec4io<f16_t> {
    static __device__ __forceinline__ float4 ld(const f16_t *p, int64_t i)
    {
        return make_float4(static_cast<float>(p[i].v), static_cast<float>(p[i + 1].v),
                           static_cast<float>(p[i + 2].v), static_cast<float>(p[i + 3].v));
    }
    static __device__ __forceinline__ void st(f16_t *p, int64_t i, float4 x)
    {
        p[i].v = static_cast<_Float16>(x.x);
        p[i + 1].v = static_cast<_Float16>(x.y);
        p[i + 2].v = static_cast<_Float16>(x.z);
        p[i + 3].v = static_cast<_Float16>(x.w);
    }
};

__device__ __forceinline__ float4 f4_fma(float4 a, float s, float4 c)
{
    return make_float4(fmaf(a.x, s, c.x), fmaf(a.y, s, c.y), fmaf(a.z, s, c.z),
                       fmaf(a.w, s, c.w));
}

__device__ __forceinline__ float4 shfl_xor4(float4 x, int off)
{
    return make_float4(__shfl_xor(x.x, off, kWave), __shfl_xor(x.y, off, kWave),
                       __shfl_xor(x.z, off, kWave), __shfl_xor(x.w, off, kWave));
}

__device__ __forceinline__ int64_t load_index(const void *p, int is64, int64_t i)
{
    return is64 ? static_cast<const int64_t *>(p)[i]
                : static_cast<int64_t>(static_cast<const int32_t *>(p)[i]);
}

// State-pool slot of index entry `pos`, or -1 for a padded entry (entry or
// slot out of range).
__device__ __forceinline__ int64_t pool_slot(const RecurrentParams &p, int64_t pos, int64_t rows)
{
    if (pos < 0 || pos >= p.idx_numel) return -1;
    const int64_t s = load_index(p.state_indices, p.idx_i64, pos);
    return (s >= 0 && s < rows) ? s : -1;
}

// Start of the initial state of (sequence n, value head hv), or NULL (zero
// state).  With a state pool the row is the slot of entry
// n * idx_seq_stride + i0, i0 = num_accepted_tokens[n] - 1 when speculative
// (fused_recurrent_gdn2.py:215-232).
__device__ __forceinline__ const float *initial_row(const RecurrentParams &p, int n, int hv)
{
    if (!p.h0) return nullptr;
    int64_t row = n;
    if (p.state_indices) {
        const int64_t i0 = p.accepted ? load_index(p.accepted, p.acc_i64, n) - 1 : 0;
        row = pool_slot(p, static_cast<int64_t>(n) * p.idx_seq_stride + i0, p.h0_rows);
        if (row < 0) return nullptr;
    }
    return p.h0 + row * p.h0_stride + static_cast<int64_t>(hv) * p.K * p.V;
}

// Where the state after token t (0-based within sequence n, packed position
// tok) is stored, or NULL: with a state pool every token's state goes to the
// slot of entry n * idx_seq_stride + t (in place) or to row tok
// (fused_recurrent_gdn2.py:311-326); otherwise only the last token's state,
// to row n (:328-333).
__device__ __forceinline__ float *store_row(const RecurrentParams &p, int n, int hv, int64_t t,
                                            int64_t tok)
{
    if (!p.ht) return nullptr;
    int64_t row = n;
    if (p.state_indices) {
        row = (p.flags & GDN2_FLAG_INPLACE_FINAL_STATE)
                  ? pool_slot(p, static_cast<int64_t>(n) * p.idx_seq_stride + t, p.ht_rows)
                  : (tok < p.ht_rows ? tok : -1);
        if (row < 0) return nullptr;
    }
    return p.ht + row * p.ht_stride + static_cast<int64_t>(hv) * p.K * p.V;
}

// Transposed state rows ([V, K] per head, element (k, v) at base[v*K + k]).
// The slab (K rows x VB columns) moves through an LDS tile in blocks of KB
// rows: 16-byte accesses run along k in HBM, and the registers keep the
// layout of the [K, V] path (thread (rg, cq) holds row rg + i*RG, columns
// c0 + 4cq .. +3).  Rows >= K and columns >= V read as zero and are not stored.
template <int NR, int TPR>
struct TransposedSlab {
    static constexpr int RG = 256 / TPR, VB = 4 * TPR;
    static constexpr int KB = RG > 32 ? RG : 32;  // rows per block
    static constexpr int BI = KB / RG;            // register rows (i) per block
    static constexpr int LD = KB + 1;             // tile row stride (floats)
    static constexpr int Q = KB / 4;              // float4 per tile row
    static constexpr int PER = VB * Q / 256;      // float4 per thread per block
    static constexpr int TILE_FLOATS = VB * LD;
    static_assert(VB * Q % 256 == 0, "tile must split evenly over 256 threads");

    // Every block's requests leave before the first one is used.  Block b's
    // PER (= BI) raw float4 wait in raw[b0 .. b0 + BI) -- the register rows
    // its transposed values end up in when NR >= BI (NR is then a multiple of
    // BI), a separate BI-entry array otherwise.  Pieces outside the slab read
    // the slab's first element (always valid) and are zeroed when written to
    // the tile.
    static constexpr int RAWN = NR >= BI ? NR : BI;
    static __device__ void load(float4 (&st)[NR], const float *base, int K, int V, int c0,
                                float *tile)
    {
        static_assert(PER == BI, "a block's raw pieces fill exactly its register rows");
        const int tid = threadIdx.x, cq = tid % TPR, rg = tid / TPR;
        float4 rawbuf[NR >= BI ? 1 : RAWN];
        float4 *raw = NR >= BI ? st : rawbuf;
#pragma unroll
        for (int b0 = 0; b0 < NR; b0 += BI) {
            const int k0 = b0 * RG;
#pragma unroll
            for (int j = 0; j < PER; ++j) {
                const int idx = tid + j * 256, vl = idx / Q, kq = idx % Q;
                const int vv = c0 + vl, kk = k0 + 4 * kq;
                const int64_t off = (vv < V && kk < K) ? static_cast<int64_t>(vv) * K + kk : 0;
                raw[b0 + j] = *reinterpret_cast<const float4 *>(base + off);
            }
        }
#pragma unroll
        for (int b0 = 0; b0 < NR; b0 += BI) {
            const int k0 = b0 * RG;
#pragma unroll
            for (int j = 0; j < PER; ++j) {
                const int idx = tid + j * 256, vl = idx / Q, kq = idx % Q;
                const int vv = c0 + vl, kk = k0 + 4 * kq;
                const float4 x = (vv < V && kk < K) ? raw[b0 + j] : make_float4(0.f, 0.f, 0.f, 0.f);
                float *t = tile + vl * LD + 4 * kq;
                t[0] = x.x; t[1] = x.y; t[2] = x.z; t[3] = x.w;
            }
            __syncthreads();
#pragma unroll
            for (int ii = 0; ii < BI; ++ii) {
                if (b0 + ii < NR) {
                    const int rl = rg + ii * RG;
                    const float *t = tile + 4 * cq * LD + rl;
                    st[b0 + ii] = make_float4(t[0], t[LD], t[2 * LD], t[3 * LD]);
                }
            }
            __syncthreads();
        }
    }

    static __device__ void store(const float4 (&st)[NR], float *base, int K, int V, int c0,
                                 float *tile)
    {
        const int tid = threadIdx.x, cq = tid % TPR, rg = tid / TPR;
#pragma unroll
        for (int b0 = 0; b0 < NR; b0 += BI) {
            const int k0 = b0 * RG;
#pragma unroll
            for (int ii = 0; ii < BI; ++ii) {
                if (b0 + ii < NR) {
                    const int rl = rg + ii * RG;
                    float *t = tile + 4 * cq * LD + rl;
                    t[0] = st[b0 + ii].x; t[LD] = st[b0 + ii].y;
                    t[2 * LD] = st[b0 + ii].z; t[3 * LD] = st[b0 + ii].w;
                }
            }
            __syncthreads();
#pragma unroll
            for (int j = 0; j < PER; ++j) {
                const int idx = tid + j * 256, vl = idx / Q, kq = idx % Q;
                const int vv = c0 + vl, kk = k0 + 4 * kq;
                if (vv < V && kk < K) {
                    const float *t = tile + vl * LD + 4 * kq;
                    *reinterpret_cast<float4 *>(base + static_cast<int64_t>(vv) * K + kk) =
                        make_float4(t[0], t[1], t[2], t[3]);
                }
            }
            __syncthreads();
        }
    }
};

// Stores the register slab (columns c0 + 4cq.., rows rg + i*RG) to the state
// row at dst, in [K, V] or transposed [V, K] order.  Called by the whole
// workgroup (the transposed path synchronises).
template <int NR, int TPR>
__device__ __forceinline__ void store_state(const float4 (&st)[NR], float *dst, int K, int V,
                                            int c0, bool trans, float *tile)
{
    if (trans) {
        TransposedSlab<NR, TPR>::store(st, dst, K, V, c0, tile);
        return;
    }
    constexpr int RG = 256 / TPR;
    const int cq = threadIdx.x % TPR, rg = threadIdx.x / TPR, col = c0 + 4 * cq;
    if (col >= V) return;
#pragma unroll
    for (int i = 0; i < NR; ++i) {
        const int r = rg + i * RG;
        if (r < K) *reinterpret_cast<float4 *>(dst + static_cast<int64_t>(r) * V + col) = st[i];
    }
}

// TPR threads cover one state row of VB = 4*TPR columns; RG = 256/TPR row
// groups; each thread keeps NR rows (NR*RG >= K).
template <typename TI, typename TG, int NR, int TPR>
__global__ __launch_bounds__(256) void recurrent_fwd_kernel(RecurrentParams p)
{
    constexpr int RG = 256 / TPR;
    constexpr int VB = 4 * TPR;
    static_assert(TPR <= 32 && (TPR & (TPR - 1)) == 0, "TPR must be a power of two <= 32");

    const int K = p.K, V = p.V;
    const int nh = blockIdx.x;
    const int vs = blockIdx.y;
    const int n = nh / p.HV, hv = nh % p.HV;
    const int h = hv / (p.HV / p.H);

    int64_t bos, len;
    if (p.cu_seqlens) {
        bos = p.cu_seqlens[n];
        len = p.cu_seqlens[n + 1] - bos;
    } else {
        bos = static_cast<int64_t>(n) * p.T;
        len = p.T;
    }

    const int tid = threadIdx.x;
    const int lane = tid & (kWave - 1), wid = tid / kWave;
    const int cq = tid % TPR, rg = tid / TPR;
    const int col = vs * VB + 4 * cq;
    const bool col_ok = col < V;

    __shared__ float s_q[256], s_k[256], s_e[256], s_a[256];
    __shared__ float s_part[4][4];
    __shared__ float4 s_red[4][2][TPR];

    const TI *q = static_cast<const TI *>(p.q);
    const TI *k = static_cast<const TI *>(p.k);
    const TI *v = static_cast<const TI *>(p.v);
    const TI *b = static_cast<const TI *>(p.b);
    const TI *w = static_cast<const TI *>(p.w);
    const TG *g = static_cast<const TG *>(p.g);
    TI *o = static_cast<TI *>(p.o);
    const bool l2 = (p.flags & GDN2_FLAG_L2NORM_QK) != 0;
    const bool gate = (p.flags & GDN2_FLAG_GATE_IN_KERNEL) != 0;
    const int use_lb = (p.flags & GDN2_FLAG_LOWER_BOUND) != 0;
    const bool sig_bw = (p.flags & GDN2_FLAG_SIGMOID_BW) != 0;

    using TS = TransposedSlab<NR, TPR>;
    extern __shared__ float s_tile[];  // TS::TILE_FLOATS floats, transposed layout only
    const bool trans = (p.flags & GDN2_FLAG_TRANSPOSE_STATE) != 0;
    const bool per_token = p.state_indices != nullptr;
    float4 st[NR];
    const float *h0row = initial_row(p, n, hv);
    if (trans && h0row) {
        TS::load(st, h0row, K, V, vs * VB, s_tile);
    } else {
#pragma unroll
        for (int i = 0; i < NR; ++i) {
            const int r = rg + i * RG;
            st[i] = make_float4(0.f, 0.f, 0.f, 0.f);
            if (h0row && col_ok && r < K)
                st[i] = *reinterpret_cast<const float4 *>(h0row + static_cast<int64_t>(r) * V + col);
        }
    }

    // The gate parameters are indexed by key head, as the reference kernel does
    // (fused_recurrent_gdn2.py:259-265); HV == H outside grouped value heads.
    const float a_log = gate ? p.A_log[h] : 0.0f;

    for (int64_t t = 0; t < len; ++t) {
        const int64_t tok = bos + t;
        const int64_t qk_off = (tok * p.H + h) * K;
        const int64_t gb_off = (tok * p.HV + hv) * K;
        const int64_t vw_off = (tok * p.HV + hv) * V;

        float qv = 0.f, kv = 0.f, gv = 0.f, bv = 0.f;
        if (tid < K) {
            qv = io<TI>::ld(q, qk_off + tid);
            kv = io<TI>::ld(k, qk_off + tid);
            gv = io<TG>::ld(g, gb_off + tid);
            bv = io<TI>::ld(b, gb_off + tid);
        }
        float4 vv = make_float4(0.f, 0.f, 0.f, 0.f), ww = vv;
        if (col_ok) {
            vv = vec4io<TI>::ld(v, vw_off + col);
            ww = vec4io<TI>::ld(w, vw_off + col);
        }
        if (sig_bw) {
            bv = sigmoid_f(bv);
            ww = make_float4(sigmoid_f(ww.x), sigmoid_f(ww.y), sigmoid_f(ww.z), sigmoid_f(ww.w));
        }
        float rq = wave_sum(qv * qv), rk = wave_sum(kv * kv), rqk = wave_sum(qv * kv);
        if (lane == 0) {
            s_part[wid][0] = rq;
            s_part[wid][1] = rk;
            s_part[wid][2] = rqk;
        }
        __syncthreads();
        float qq = 0.f, kk = 0.f, qk = 0.f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            qq += s_part[i][0];
            kk += s_part[i][1];
            qk += s_part[i][2];
        }
        const float invq = l2 ? 1.0f / fmaxf(sqrtf(qq), 1e-6f) : 1.0f;
        const float invk = l2 ? 1.0f / fmaxf(sqrtf(kk), 1e-6f) : 1.0f;
        if (tid < K) {
            const float kn = kv * invk;
            s_q[tid] = qv * invq * p.scale;
            s_k[tid] = kn;
            s_e[tid] = bv * kn;
            float gk = gv;
            if (gate) {
                const float db = p.dt_bias ? p.dt_bias[h * K + tid] : 0.0f;
                gk = gate_activation(gv, a_log, db, use_lb, p.lower_bound);
            }
            s_a[tid] = expf(gk);
        }
        const float kq = qk * invq * invk * p.scale;
        __syncthreads();

        float4 pr = make_float4(0.f, 0.f, 0.f, 0.f), po = pr;
#pragma unroll
        for (int i = 0; i < NR; ++i) {
            const int r = rg + i * RG;
            if (r < K) {
                const float a = s_a[r];
                st[i].x *= a;
                st[i].y *= a;
                st[i].z *= a;
                st[i].w *= a;
                pr = f4_fma(st[i], s_e[r], pr);
                po = f4_fma(st[i], s_q[r], po);
            }
        }
#pragma unroll
        for (int off = TPR; off < kWave; off <<= 1) {
            const float4 a = shfl_xor4(pr, off), c = shfl_xor4(po, off);
            pr.x += a.x; pr.y += a.y; pr.z += a.z; pr.w += a.w;
            po.x += c.x; po.y += c.y; po.z += c.z; po.w += c.w;
        }
        if (lane < TPR) {
            s_red[wid][0][cq] = pr;
            s_red[wid][1][cq] = po;
        }
        __syncthreads();
        float4 R = s_red[0][0][cq], PO = s_red[0][1][cq];
#pragma unroll
        for (int i = 1; i < 4; ++i) {
            const float4 a = s_red[i][0][cq], c = s_red[i][1][cq];
            R.x += a.x; R.y += a.y; R.z += a.z; R.w += a.w;
            PO.x += c.x; PO.y += c.y; PO.z += c.z; PO.w += c.w;
        }
        const float4 u = make_float4(ww.x * vv.x - R.x, ww.y * vv.y - R.y, ww.z * vv.z - R.z,
                                     ww.w * vv.w - R.w);
#pragma unroll
        for (int i = 0; i < NR; ++i) {
            const int r = rg + i * RG;
            if (r < K) {
                const float kr = s_k[r];
                st[i].x = fmaf(kr, u.x, st[i].x);
                st[i].y = fmaf(kr, u.y, st[i].y);
                st[i].z = fmaf(kr, u.z, st[i].z);
                st[i].w = fmaf(kr, u.w, st[i].w);
            }
        }
        if (rg == 0 && col_ok) vec4io<TI>::st(o, vw_off + col, f4_fma(u, kq, PO));
        __syncthreads();
        if (per_token) {
            float *dst = store_row(p, n, hv, t, tok);
            if (dst) store_state<NR, TPR>(st, dst, K, V, vs * VB, trans, s_tile);
        }
    }

    if (!per_token) {
        float *dst = store_row(p, n, hv, len - 1, bos + len - 1);
        if (dst) store_state<NR, TPR>(st, dst, K, V, vs * VB, trans, s_tile);
    }
}

// Decode step (T = 1, no cu_seqlens) specialised for d_k = d_v = 128.
// Same arithmetic and thread mapping as recurrent_fwd_kernel, but each
// workgroup walks two consecutive (sequence, value head) slabs and issues the
// second slab's 64 KB of state loads before computing the first, so state
// reads of one slab overlap the state writes of the other.  A decode step is
// one pass over the whole state, so this overlap is what separates it from a
// plain read-then-write of 2 x 64 KB per workgroup.
template <typename TI, typename TG, bool H0>
__global__ __launch_bounds__(256) void decode_step_kernel(RecurrentParams p, int nslabs)
{
    constexpr int KD = 128, VD = 128, TPR = 32, RG = 8, NR = KD / RG, SLABS = 2;
    const int tid = threadIdx.x;
    const int lane = tid & (kWave - 1), wid = tid / kWave;
    const int cq = tid % TPR, rg = tid / TPR;
    const int col = 4 * cq;

    __shared__ float s_q[KD], s_k[KD], s_e[KD], s_a[KD];
    __shared__ float s_part[4][4];
    __shared__ float4 s_red[4][2][TPR];

    const TI *q = static_cast<const TI *>(p.q);
    const TI *k = static_cast<const TI *>(p.k);
    const TI *v = static_cast<const TI *>(p.v);
    const TI *b = static_cast<const TI *>(p.b);
    const TI *w = static_cast<const TI *>(p.w);
    const TG *g = static_cast<const TG *>(p.g);
    TI *o = static_cast<TI *>(p.o);
    const bool l2 = (p.flags & GDN2_FLAG_L2NORM_QK) != 0;
    const bool gate = (p.flags & GDN2_FLAG_GATE_IN_KERNEL) != 0;
    const int use_lb = (p.flags & GDN2_FLAG_LOWER_BOUND) != 0;
    const bool sig_bw = (p.flags & GDN2_FLAG_SIGMOID_BW) != 0;

    // Every request below reads an always-valid address: the token inputs of
    // both slabs first, then both slabs' state.  A slab past the end reads the
    // last slab, and a state row that does not exist (no initial state, or a
    // padded pool entry) reads slab 0 of the state array and is zeroed where it
    // is used.  A load whose result were picked against zero here, or a load
    // inside a per-slab branch, would make the compiler wait for the first
    // slab's state before the second slab's requests leave.
    const int slab0 = blockIdx.x * SLABS;
    float qv[SLABS], kv[SLABS], gv[SLABS], bv[SLABS];
    float4 vv[SLABS], ww[SLABS];
    const int tk = tid & (KD - 1);
#pragma unroll
    for (int s = 0; s < SLABS; ++s) {
        const int slab = slab0 + s < nslabs ? slab0 + s : nslabs - 1;
        const int n = slab / p.HV, hv = slab % p.HV;
        const int h = hv / (p.HV / p.H);
        const int64_t qk_off = (static_cast<int64_t>(n) * p.H + h) * KD;
        qv[s] = io<TI>::ld(q, qk_off + tk);
        kv[s] = io<TI>::ld(k, qk_off + tk);
        gv[s] = io<TG>::ld(g, static_cast<int64_t>(slab) * KD + tk);
        bv[s] = io<TI>::ld(b, static_cast<int64_t>(slab) * KD + tk);
        vv[s] = vec4io<TI>::ld(v, static_cast<int64_t>(slab) * VD + col);
        ww[s] = vec4io<TI>::ld(w, static_cast<int64_t>(slab) * VD + col);
    }
    // Store rows (a state pool reads its index entries here) and the in-kernel
    // gate's parameters, also before any state request.  With an initial
    // state the gate parameters are read unconditionally (from the state
    // array when absent, and then unused).
    float *dst[SLABS];
    float dtb[SLABS], alg[SLABS];
#pragma unroll
    for (int s = 0; s < SLABS; ++s) {
        const int slab = slab0 + s < nslabs ? slab0 + s : nslabs - 1;
        const int n = slab / p.HV, hv = slab % p.HV;
        const int h = hv / (p.HV / p.H);
        dst[s] = store_row(p, n, hv, 0, n);
        dtb[s] = alg[s] = 0.f;
        if constexpr (H0) {
            const float *dsrc = p.dt_bias ? p.dt_bias : p.h0;
            const float *asrc = p.A_log ? p.A_log : p.h0;
            dtb[s] = dsrc[h * KD + tk];
            alg[s] = asrc[h];
        } else if (gate) {
            dtb[s] = p.dt_bias ? p.dt_bias[h * KD + tk] : 0.0f;
            alg[s] = p.A_log[h];
        }
    }
    float4 st[SLABS][NR];
    bool zst[SLABS];
    // H0 (a compile-time choice, so that no branch separates the loads from
    // their use): an initial-state array exists.
    if constexpr (H0) {
        // Both rows first (a state pool reads its index entries here), then
        // both slabs' loads back to back.
        const float *src[SLABS];
#pragma unroll
        for (int s = 0; s < SLABS; ++s) {
            const int slab = slab0 + s < nslabs ? slab0 + s : nslabs - 1;
            const float *row = initial_row(p, slab / p.HV, slab % p.HV);
            zst[s] = row == nullptr;
            src[s] = row ? row : p.h0;
        }
#pragma unroll
        for (int s = 0; s < SLABS; ++s)
#pragma unroll
            for (int i = 0; i < NR; ++i)
                st[s][i] = *reinterpret_cast<const float4 *>(src[s] + (rg + i * RG) * VD + col);
    } else {
#pragma unroll
        for (int s = 0; s < SLABS; ++s) {
            zst[s] = true;
#pragma unroll
            for (int i = 0; i < NR; ++i) st[s][i] = make_float4(0.f, 0.f, 0.f, 0.f);
        }
    }
#pragma unroll
    for (int s = 0; s < SLABS; ++s) {
        const int slab = slab0 + s;
        if (slab >= nslabs) break;
        const int64_t vw_off = static_cast<int64_t>(slab) * VD;

        float qv_ = 0.f, kv_ = 0.f, gv_ = 0.f, bv_ = 0.f;
        if (tid < KD) {
            qv_ = qv[s];
            kv_ = kv[s];
            gv_ = gv[s];
            bv_ = bv[s];
        }
        float4 vv_ = vv[s], ww_ = ww[s];
        if (sig_bw) {
            bv_ = sigmoid_f(bv_);
            ww_ = make_float4(sigmoid_f(ww_.x), sigmoid_f(ww_.y), sigmoid_f(ww_.z), sigmoid_f(ww_.w));
        }
        const float rq = wave_sum(qv_ * qv_), rk = wave_sum(kv_ * kv_), rqk = wave_sum(qv_ * kv_);
        if (lane == 0) {
            s_part[wid][0] = rq;
            s_part[wid][1] = rk;
            s_part[wid][2] = rqk;
        }
        __syncthreads();
        float qq = 0.f, kk = 0.f, qk = 0.f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            qq += s_part[i][0];
            kk += s_part[i][1];
            qk += s_part[i][2];
        }
        const float invq = l2 ? 1.0f / fmaxf(sqrtf(qq), 1e-6f) : 1.0f;
        const float invk = l2 ? 1.0f / fmaxf(sqrtf(kk), 1e-6f) : 1.0f;
        if (tid < KD) {
            const float kn = kv_ * invk;
            s_q[tid] = qv_ * invq * p.scale;
            s_k[tid] = kn;
            s_e[tid] = bv_ * kn;
            float gk = gv_;
            if (gate) {
                const float db = p.dt_bias ? dtb[s] : 0.0f;
                gk = gate_activation(gv_, alg[s], db, use_lb, p.lower_bound);
            }
            s_a[tid] = expf(gk);
        }
        const float kq = qk * invq * invk * p.scale;
        __syncthreads();

        float4 pr = make_float4(0.f, 0.f, 0.f, 0.f), po = pr;
        // Opaque here, so that the zeroing of a missing row is not hoisted up
        // to the loads (where overwriting their registers would wait for them).
        int zs = zst[s] ? 1 : 0;
        asm volatile("" : "+v"(zs));
#pragma unroll
        for (int i = 0; i < NR; ++i) {
            const int r = rg + i * RG;
            if (zs) st[s][i] = make_float4(0.f, 0.f, 0.f, 0.f);
            const float a = s_a[r];
            st[s][i].x *= a;
            st[s][i].y *= a;
            st[s][i].z *= a;
            st[s][i].w *= a;
            pr = f4_fma(st[s][i], s_e[r], pr);
            po = f4_fma(st[s][i], s_q[r], po);
        }
        {
            const float4 a = shfl_xor4(pr, 32), c = shfl_xor4(po, 32);
            pr.x += a.x; pr.y += a.y; pr.z += a.z; pr.w += a.w;
            po.x += c.x; po.y += c.y; po.z += c.z; po.w += c.w;
        }
        if (lane < TPR) {
            s_red[wid][0][cq] = pr;
            s_red[wid][1][cq] = po;
        }
        __syncthreads();
        float4 R = s_red[0][0][cq], PO = s_red[0][1][cq];
#pragma unroll
        for (int i = 1; i < 4; ++i) {
            const float4 a = s_red[i][0][cq], c = s_red[i][1][cq];
            R.x += a.x; R.y += a.y; R.z += a.z; R.w += a.w;
            PO.x += c.x; PO.y += c.y; PO.z += c.z; PO.w += c.w;
        }
        const float4 u = make_float4(ww_.x * vv_.x - R.x, ww_.y * vv_.y - R.y, ww_.z * vv_.z - R.z,
                                     ww_.w * vv_.w - R.w);
        // One token per sequence: its state is the final state (packed position n).
#pragma unroll
        for (int i = 0; i < NR; ++i) {
            const int r = rg + i * RG;
            const float kr = s_k[r];
            st[s][i].x = fmaf(kr, u.x, st[s][i].x);
            st[s][i].y = fmaf(kr, u.y, st[s][i].y);
            st[s][i].z = fmaf(kr, u.z, st[s][i].z);
            st[s][i].w = fmaf(kr, u.w, st[s][i].w);
            if (dst[s]) *reinterpret_cast<float4 *>(dst[s] + r * VD + col) = st[s][i];
        }
        if (rg == 0) vec4io<TI>::st(o, vw_off + col, f4_fma(u, kq, PO));
        __syncthreads();
    }
}

// One step of the half-wave butterfly transpose-reduction over N values per
// lane: lanes with bit N/2 of their half-wave index keep the upper half and
// send the lower one to their partner (lane ^ N/2), the others the opposite;
// after the steps N = 32 .. 2, lane j holds x[j] summed over the 32 lanes.
// Compile-time N keeps every index constant (register arrays indexed at run
// time would be lowered to compare / select chains).
template <int N>
__device__ __forceinline__ void half_wave_butterfly(float (&x)[32], int hl)
{
    constexpr int H2 = N / 2;
    const bool up = (hl & H2) != 0;
#pragma unroll
    for (int t = 0; t < H2; ++t) {
        const float send = up ? x[t] : x[t + H2];
        const float keep = up ? x[t + H2] : x[t];
        x[t] = keep + __shfl_xor(send, H2, kWave);
    }
    if constexpr (N > 2) half_wave_butterfly<H2>(x, hl);
}

// Decode step with [V, K] (transposed) states, K = V = 128: two (sequence,
// value head) slabs per workgroup of 256 threads, requests ordered as in
// decode_step_kernel.  Thread (ck, rv) = (tid % 32, tid / 32) holds key
// columns 4ck..4ck+3 of state rows v = rv + 8i, i < 16, so each half-wave
// reads and writes whole 512-byte rows.  The contractions over K (S^T e and
// S^T q for every v) stay inside the half-wave: a butterfly
// transpose-reduction (exchange half of the remaining values with lane
// ^ 16, 8, 4, 2, 1) leaves lane j of half-wave rv with the complete sum for
// value rv + 8 (j / 2): the e-contraction on even j, the q-contraction on odd j.
template <typename TI, typename TG, bool H0>
__global__ __launch_bounds__(256) void decode_step_t_kernel(RecurrentParams p, int nslabs)
{
    constexpr int KD = 128, VD = 128, NI = 16, SLABS = 2;
    const int tid = threadIdx.x;
    const int lane = tid & (kWave - 1), wid = tid / kWave;
    const int ck = tid & 31, rv = tid >> 5;
    const int kc = 4 * ck;
    const int vsel = rv + 8 * (ck >> 1);  // the value this lane completes

    __shared__ float s_q[KD], s_k[KD], s_e[KD], s_a[KD];
    __shared__ float s_part[4][4];
    __shared__ float s_u[VD];

    const TI *q = static_cast<const TI *>(p.q);
    const TI *k = static_cast<const TI *>(p.k);
    const TI *v = static_cast<const TI *>(p.v);
    const TI *b = static_cast<const TI *>(p.b);
    const TI *w = static_cast<const TI *>(p.w);
    const TG *g = static_cast<const TG *>(p.g);
    TI *o = static_cast<TI *>(p.o);
    const bool l2 = (p.flags & GDN2_FLAG_L2NORM_QK) != 0;
    const bool gate = (p.flags & GDN2_FLAG_GATE_IN_KERNEL) != 0;
    const int use_lb = (p.flags & GDN2_FLAG_LOWER_BOUND) != 0;
    const bool sig_bw = (p.flags & GDN2_FLAG_SIGMOID_BW) != 0;

    // Token inputs, store rows and gate parameters of both slabs, then both
    // slabs' state, all from always-valid addresses (as in decode_step_kernel).
    const int slab0 = blockIdx.x * SLABS;
    float qv[SLABS], kv[SLABS], gv[SLABS], bv[SLABS], vv[SLABS], ww[SLABS];
    const int tk = tid & (KD - 1);
#pragma unroll
    for (int s = 0; s < SLABS; ++s) {
        const int slab = slab0 + s < nslabs ? slab0 + s : nslabs - 1;
        const int n = slab / p.HV, hv = slab % p.HV;
        const int h = hv / (p.HV / p.H);
        const int64_t qk_off = (static_cast<int64_t>(n) * p.H + h) * KD;
        qv[s] = io<TI>::ld(q, qk_off + tk);
        kv[s] = io<TI>::ld(k, qk_off + tk);
        gv[s] = io<TG>::ld(g, static_cast<int64_t>(slab) * KD + tk);
        bv[s] = io<TI>::ld(b, static_cast<int64_t>(slab) * KD + tk);
        vv[s] = io<TI>::ld(v, static_cast<int64_t>(slab) * VD + vsel);
        ww[s] = io<TI>::ld(w, static_cast<int64_t>(slab) * VD + vsel);
    }
    float *dst[SLABS];
    float dtb[SLABS], alg[SLABS];
#pragma unroll
    for (int s = 0; s < SLABS; ++s) {
        const int slab = slab0 + s < nslabs ? slab0 + s : nslabs - 1;
        const int n = slab / p.HV, hv = slab % p.HV;
        const int h = hv / (p.HV / p.H);
        dst[s] = store_row(p, n, hv, 0, n);
        dtb[s] = alg[s] = 0.f;
        if constexpr (H0) {
            const float *dsrc = p.dt_bias ? p.dt_bias : p.h0;
            const float *asrc = p.A_log ? p.A_log : p.h0;
            dtb[s] = dsrc[h * KD + tk];
            alg[s] = asrc[h];
        } else if (gate) {
            dtb[s] = p.dt_bias ? p.dt_bias[h * KD + tk] : 0.0f;
            alg[s] = p.A_log[h];
        }
    }
    float4 st[SLABS][NI];
    bool zst[SLABS];
    if constexpr (H0) {
        const float *src[SLABS];
#pragma unroll
        for (int s = 0; s < SLABS; ++s) {
            const int slab = slab0 + s < nslabs ? slab0 + s : nslabs - 1;
            const float *row = initial_row(p, slab / p.HV, slab % p.HV);
            zst[s] = row == nullptr;
            src[s] = row ? row : p.h0;
        }
#pragma unroll
        for (int s = 0; s < SLABS; ++s)
#pragma unroll
            for (int i = 0; i < NI; ++i)
                st[s][i] = *reinterpret_cast<const float4 *>(src[s] + (rv + 8 * i) * KD + kc);
    } else {
#pragma unroll
        for (int s = 0; s < SLABS; ++s) {
            zst[s] = true;
#pragma unroll
            for (int i = 0; i < NI; ++i) st[s][i] = make_float4(0.f, 0.f, 0.f, 0.f);
        }
    }
#pragma unroll
    for (int s = 0; s < SLABS; ++s) {
        const int slab = slab0 + s;
        if (slab >= nslabs) break;

        float qv_ = 0.f, kv_ = 0.f, gv_ = 0.f, bv_ = 0.f;
        if (tid < KD) {
            qv_ = qv[s];
            kv_ = kv[s];
            gv_ = gv[s];
            bv_ = bv[s];
        }
        float vv_ = vv[s], ww_ = ww[s];
        if (sig_bw) {
            bv_ = sigmoid_f(bv_);
            ww_ = sigmoid_f(ww_);
        }
        const float rq = wave_sum(qv_ * qv_), rk = wave_sum(kv_ * kv_), rqk = wave_sum(qv_ * kv_);
        if (lane == 0) {
            s_part[wid][0] = rq;
            s_part[wid][1] = rk;
            s_part[wid][2] = rqk;
        }
        __syncthreads();
        float qq = 0.f, kk = 0.f, qk = 0.f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            qq += s_part[i][0];
            kk += s_part[i][1];
            qk += s_part[i][2];
        }
        const float invq = l2 ? 1.0f / fmaxf(sqrtf(qq), 1e-6f) : 1.0f;
        const float invk = l2 ? 1.0f / fmaxf(sqrtf(kk), 1e-6f) : 1.0f;
        if (tid < KD) {
            const float kn = kv_ * invk;
            s_q[tid] = qv_ * invq * p.scale;
            s_k[tid] = kn;
            s_e[tid] = bv_ * kn;
            float gk = gv_;
            if (gate) {
                const float db = p.dt_bias ? dtb[s] : 0.0f;
                gk = gate_activation(gv_, alg[s], db, use_lb, p.lower_bound);
            }
            s_a[tid] = expf(gk);
        }
        const float kq = qk * invq * invk * p.scale;
        __syncthreads();

        const float4 a4 = *reinterpret_cast<const float4 *>(&s_a[kc]);
        const float4 e4 = *reinterpret_cast<const float4 *>(&s_e[kc]);
        const float4 q4 = *reinterpret_cast<const float4 *>(&s_q[kc]);
        const float4 k4 = *reinterpret_cast<const float4 *>(&s_k[kc]);
        int zs = zst[s] ? 1 : 0;
        asm volatile("" : "+v"(zs));
        // x[2i] = this lane's part of (S^T e)[rv + 8i], x[2i + 1] of (S^T q)[rv + 8i].
        float x[2 * NI];
#pragma unroll
        for (int i = 0; i < NI; ++i) {
            if (zs) st[s][i] = make_float4(0.f, 0.f, 0.f, 0.f);
            st[s][i].x *= a4.x;
            st[s][i].y *= a4.y;
            st[s][i].z *= a4.z;
            st[s][i].w *= a4.w;
            x[2 * i] = fmaf(st[s][i].w, e4.w, fmaf(st[s][i].z, e4.z, fmaf(st[s][i].y, e4.y, st[s][i].x * e4.x)));
            x[2 * i + 1] =
                fmaf(st[s][i].w, q4.w, fmaf(st[s][i].z, q4.z, fmaf(st[s][i].y, q4.y, st[s][i].x * q4.x)));
        }
        static_assert(2 * NI == 32, "one value per lane of a half-wave");
        half_wave_butterfly<32>(x, ck);
        // Even lanes: u = w v - S^T e for their value; odd lanes: o = S^T q + (k.q) u.
        const float u = ww_ * vv_ - x[0];
        const float u_pair = __shfl_xor(u, 1, kWave);
        if ((ck & 1) == 0) s_u[vsel] = u;
        else io<TI>::st(o, static_cast<int64_t>(slab) * VD + vsel, fmaf(u_pair, kq, x[0]));
        __syncthreads();
#pragma unroll
        for (int i = 0; i < NI; ++i) {
            const float uv = s_u[rv + 8 * i];
            st[s][i] = f4_fma(k4, uv, st[s][i]);
            if (dst[s]) *reinterpret_cast<float4 *>(dst[s] + (rv + 8 * i) * KD + kc) = st[s][i];
        }
        __syncthreads();
    }
}

// Fused module decode step (one token per sequence, HV == H, K == V == D).
// Replaces, for the module's decode call, the chain ShortConvolution x 3
// (reference gdn2.py:395-430) -> gate and b / w activations (gdn2.py:840-866)
// -> fused_recurrent_gdn2 (fused_recurrent_gdn2.py:461-555) -> RMSNormGated
// (gdn2.py:433-452), so that q, k, v and o make no HBM round trip between
// them.  Each step keeps the arithmetic of the separate HIP passes:
//  * the convolution in the op order and roundings of short_conv_vec_kernel
//    (fp32 accumulation, the output rounded to the io dtype before and after
//    the SiLU), the new cache = the last W-1 inputs;
//  * the recurrence as decode_step_kernel computes it (at D = 128 the same
//    thread mapping and summation order);
//  * the output rounded to the io dtype, then the gated norm in the lane
//    layout and op order of gated_rmsnorm_kernel.
// Mapping: D * D / 64 threads per (sequence, head) -- one wave at D = 64, so
// the step needs no block barrier there -- each holding 16 float4 of the
// state; thread c < D owns channel c of the per-channel inputs.
template <typename TI, typename TG, int D, bool H0>
__global__ __launch_bounds__(D * D / 64) void decode_fused_kernel(DecodeFusedParams p)
{
    constexpr int NT = D * D / 64, NW = NT / kWave;
    constexpr int TPR = D / 4, RG = NT / TPR, NR = D / RG, W = 4, EPL = D / kWave;
    static_assert(NR * RG == D && TPR <= kWave && EPL * kWave == D, "decode mapping");
    const int tid = threadIdx.x, lane = tid & (kWave - 1), wid = tid / kWave;
    const int cq = tid % TPR, rg = tid / TPR, col = 4 * cq;
    const int n = blockIdx.x / p.H, h = blockIdx.x % p.H;
    const int64_t HD = static_cast<int64_t>(p.H) * D;

    __shared__ __align__(16) float s_q[D], s_k[D], s_e[D], s_a[D], s_v[D], s_w[D], s_o[D];
    __shared__ float s_part[NW][3];
    __shared__ float4 s_red[NW][2][TPR];

    const bool l2 = (p.flags & GDN2_FLAG_L2NORM_QK) != 0;
    const bool gate = (p.flags & GDN2_FLAG_GATE_IN_KERNEL) != 0;
    const int use_lb = (p.flags & GDN2_FLAG_LOWER_BOUND) != 0;
    const bool sig_bw = (p.flags & GDN2_FLAG_SIGMOID_BW) != 0;

    // Every request first, straight-line: the channel inputs (thread c < D; the
    // others read channel D-1 and discard it), wave 0's output gate and norm
    // weight, then the state.  An absent optional input (conv cache, bias,
    // gate, norm weight, gate parameters) is read from an always-valid address
    // -- the conv weights, HD * W elements -- and zeroed by a uniform factor
    // where it is used: a load behind a branch on the pointer would wait for
    // its data right there, before the next request leaves.
    const bool chan = tid < D;
    const int c = chan ? tid : D - 1;
    const int64_t ch = static_cast<int64_t>(h) * D + c;
    const TI *safe = static_cast<const TI *>(p.cw[0]);
    float xh[3][W], wt[3][W], bias[3], mcache[3], mbias[3];
#pragma unroll
    for (int t = 0; t < 3; ++t) {
        const TI *x = static_cast<const TI *>(p.x[t]);
        const TI *cw = static_cast<const TI *>(p.cw[t]);
        const bool hc = p.cin[t] != nullptr, hb = p.cb[t] != nullptr;
        const TI *ci = hc ? static_cast<const TI *>(p.cin[t]) : safe;
        const TI *cb = hb ? static_cast<const TI *>(p.cb[t]) : safe;
        const int64_t coff = hc ? (n * HD + ch) * (W - 1) : ch;
        mcache[t] = hc ? 1.0f : 0.0f;
        mbias[t] = hb ? 1.0f : 0.0f;
        xh[t][W - 1] = io<TI>::ld(x, n * p.ldx[t] + ch);
#pragma unroll
        for (int j = 0; j < W - 1; ++j) xh[t][j] = io<TI>::ld(ci, coff + (hc ? j : 0));
#pragma unroll
        for (int j = 0; j < W; ++j) wt[t][j] = io<TI>::ld(cw, ch * W + j);
        bias[t] = io<TI>::ld(cb, ch);
    }
    float gv = io<TG>::ld(static_cast<const TG *>(p.g), n * p.ldg + ch);
    float bv = io<TI>::ld(static_cast<const TI *>(p.b), n * p.ldb + ch);
    float wv = io<TI>::ld(static_cast<const TI *>(p.w), n * p.ldw + ch);
    const float *fsafe = reinterpret_cast<const float *>(safe);  // HD * W * sizeof(TI) >= 4 * HD bytes
    const float a_log = (gate ? p.A_log : fsafe)[gate ? h : 0];
    const float dtb = (gate && p.dt_bias ? p.dt_bias : fsafe)[gate && p.dt_bias ? ch : 0];
    const float mdtb = gate && p.dt_bias ? 1.0f : 0.0f;
    const bool hz = p.z != nullptr, hn = p.nw != nullptr;
    const TI *zp = hz ? static_cast<const TI *>(p.z) : safe;
    const TI *nwp = hn && !p.nw_f32 ? static_cast<const TI *>(p.nw) : safe;
    const float *nwf = hn && p.nw_f32 ? static_cast<const float *>(p.nw) : fsafe;
    float zr[EPL], nwr[EPL];
#pragma unroll
    for (int e = 0; e < EPL; ++e) {
        const int cz = lane + kWave * e;
        zr[e] = io<TI>::ld(zp, hz ? n * p.ldz + static_cast<int64_t>(h) * D + cz : cz);
        const float nf = nwf[cz], nt = io<TI>::ld(nwp, cz);
        nwr[e] = p.nw_f32 ? nf : nt;
    }
    float4 st[NR];
    if constexpr (H0) {
        const float *src = p.h0 + n * p.h0_stride + static_cast<int64_t>(h) * D * D;
#pragma unroll
        for (int i = 0; i < NR; ++i) st[i] = *reinterpret_cast<const float4 *>(src + (rg + i * RG) * D + col);
    } else {
#pragma unroll
        for (int i = 0; i < NR; ++i) st[i] = make_float4(0.f, 0.f, 0.f, 0.f);
    }

    // Short convolution + SiLU; the new cache holds the last W-1 inputs (read
    // above by this thread, so an in-place cache update is safe).
    float xc[3];
#pragma unroll
    for (int t = 0; t < 3; ++t) {
#pragma unroll
        for (int j = 0; j < W - 1; ++j) xh[t][j] *= mcache[t];
        float acc = 0.0f;
#pragma unroll
        for (int j = 0; j < W; ++j) acc = fmaf(wt[t][j], xh[t][j], acc);
        xc[t] = round_to<TI>(silu_f32(round_to<TI>(acc + bias[t] * mbias[t])));
        if (chan && p.cout[t]) {
            TI *co = static_cast<TI *>(p.cout[t]);
#pragma unroll
            for (int j = 0; j < W - 1; ++j) io<TI>::st(co, (n * HD + ch) * (W - 1) + j, xh[t][j + 1]);
        }
    }
    if (sig_bw) {
        bv = sigmoid_f(bv);
        wv = sigmoid_f(wv);
    }
    const float gk = gate ? gate_activation(gv, a_log, dtb * mdtb, use_lb, p.lower_bound) : gv;
    const float qx = chan ? xc[0] : 0.0f, kx = chan ? xc[1] : 0.0f;
    float qq = wave_sum(qx * qx), kk = wave_sum(kx * kx), qk = wave_sum(qx * kx);
    if constexpr (NW > 1) {
        if (lane == 0) {
            s_part[wid][0] = qq;
            s_part[wid][1] = kk;
            s_part[wid][2] = qk;
        }
        __syncthreads();
        qq = kk = qk = 0.f;
#pragma unroll
        for (int i = 0; i < NW; ++i) {
            qq += s_part[i][0];
            kk += s_part[i][1];
            qk += s_part[i][2];
        }
    }
    const float invq = l2 ? 1.0f / fmaxf(sqrtf(qq), 1e-6f) : 1.0f;
    const float invk = l2 ? 1.0f / fmaxf(sqrtf(kk), 1e-6f) : 1.0f;
    if (chan) {
        const float kn = kx * invk;
        s_q[c] = qx * invq * p.scale;
        s_k[c] = kn;
        s_e[c] = bv * kn;
        s_a[c] = expf(gk);
        s_v[c] = xc[2];
        s_w[c] = wv;
    }
    const float kq = qk * invq * invk * p.scale;
    __syncthreads();

    float4 pr = make_float4(0.f, 0.f, 0.f, 0.f), po = pr;
#pragma unroll
    for (int i = 0; i < NR; ++i) {
        const int r = rg + i * RG;
        const float a = s_a[r];
        st[i].x *= a;
        st[i].y *= a;
        st[i].z *= a;
        st[i].w *= a;
        pr = f4_fma(st[i], s_e[r], pr);
        po = f4_fma(st[i], s_q[r], po);
    }
#pragma unroll
    for (int off = TPR; off < kWave; off <<= 1) {
        const float4 a = shfl_xor4(pr, off), cc = shfl_xor4(po, off);
        pr.x += a.x; pr.y += a.y; pr.z += a.z; pr.w += a.w;
        po.x += cc.x; po.y += cc.y; po.z += cc.z; po.w += cc.w;
    }
    float4 R = pr, PO = po;
    if constexpr (NW > 1) {
        if (lane < TPR) {
            s_red[wid][0][cq] = pr;
            s_red[wid][1][cq] = po;
        }
        __syncthreads();
        R = s_red[0][0][cq];
        PO = s_red[0][1][cq];
#pragma unroll
        for (int i = 1; i < NW; ++i) {
            const float4 a = s_red[i][0][cq], cc = s_red[i][1][cq];
            R.x += a.x; R.y += a.y; R.z += a.z; R.w += a.w;
            PO.x += cc.x; PO.y += cc.y; PO.z += cc.z; PO.w += cc.w;
        }
    }
    const float4 vv = *reinterpret_cast<const float4 *>(&s_v[col]);
    const float4 ww = *reinterpret_cast<const float4 *>(&s_w[col]);
    const float4 u = make_float4(ww.x * vv.x - R.x, ww.y * vv.y - R.y, ww.z * vv.z - R.z,
                                 ww.w * vv.w - R.w);
    float *dst = p.ht ? p.ht + n * p.ht_stride + static_cast<int64_t>(h) * D * D : nullptr;
#pragma unroll
    for (int i = 0; i < NR; ++i) {
        const int r = rg + i * RG;
        const float kr = s_k[r];
        st[i].x = fmaf(kr, u.x, st[i].x);
        st[i].y = fmaf(kr, u.y, st[i].y);
        st[i].z = fmaf(kr, u.z, st[i].z);
        st[i].w = fmaf(kr, u.w, st[i].w);
        if (dst) *reinterpret_cast<float4 *>(dst + r * D + col) = st[i];
    }
    if (rg == 0) {
        const float4 o4 = f4_fma(u, kq, PO);
        s_o[col] = round_to<TI>(o4.x);
        s_o[col + 1] = round_to<TI>(o4.y);
        s_o[col + 2] = round_to<TI>(o4.z);
        s_o[col + 3] = round_to<TI>(o4.w);
    }
    __syncthreads();
    if (wid != 0) return;  // no barriers below

    // Output: RMSNormGated (gdn2.py:433-452) over the head's D values.
    const int64_t obase = (static_cast<int64_t>(n) * p.H + h) * D;
    float xo[EPL], sq = 0.0f;
#pragma unroll
    for (int e = 0; e < EPL; ++e) {
        xo[e] = s_o[lane + kWave * e];
        sq += round_to<TI>(xo[e] * xo[e]);
    }
    if (!p.nw) {
#pragma unroll
        for (int e = 0; e < EPL; ++e) io<TI>::st(static_cast<TI *>(p.o), obase + lane + kWave * e, xo[e]);
        return;
    }
    const float var = round_to<TI>(wave_sum(sq) / static_cast<float>(D));
    const float inv = round_to<TI>(rsqrtf(round_to<TI>(var + p.eps)));
#pragma unroll
    for (int e = 0; e < EPL; ++e) {
        const int cz = lane + kWave * e;
        const float a = round_to<TI>(xo[e] * inv);
        if (p.nw_f32) {
            // An fp32 weight promotes the rest of the expression to fp32.
            static_cast<float *>(p.o)[obase + cz] = p.z ? a * nwr[e] * round_to<TI>(silu_f32(zr[e])) : a * nwr[e];
        } else {
            const float aw = round_to<TI>(a * nwr[e]);
            io<TI>::st(static_cast<TI *>(p.o), obase + cz,
                       p.z ? round_to<TI>(aw * round_to<TI>(silu_f32(zr[e]))) : aw);
        }
    }
}

template <typename TI, typename TG>
static hipError_t launch_decode_fused_t(const DecodeFusedParams &p, hipStream_t stream)
{
    const dim3 grid(p.N * p.H);
    if (p.D == 64) {
        if (p.h0)
            hipLaunchKernelGGL((decode_fused_kernel<TI, TG, 64, true>), grid, dim3(64), 0, stream, p);
        else
            hipLaunchKernelGGL((decode_fused_kernel<TI, TG, 64, false>), grid, dim3(64), 0, stream, p);
    } else {
        if (p.h0)
            hipLaunchKernelGGL((decode_fused_kernel<TI, TG, 128, true>), grid, dim3(256), 0, stream, p);
        else
            hipLaunchKernelGGL((decode_fused_kernel<TI, TG, 128, false>), grid, dim3(256), 0, stream, p);
    }
    return hipGetLastError();
}

template <typename TI, typename TG, int TPR>
static hipError_t launch_nr(const RecurrentParams &p, int N, hipStream_t stream)
{
    constexpr int RG = 256 / TPR;
    const int need = (p.K + RG - 1) / RG;
    const int nvs = (p.V + 4 * TPR - 1) / (4 * TPR);
    dim3 grid(N * p.HV, nvs);
    // The LDS tile of the transposed state layout (same size for every NR).
    const size_t lds = (p.flags & GDN2_FLAG_TRANSPOSE_STATE)
                           ? TransposedSlab<1, TPR>::TILE_FLOATS * sizeof(float)
                           : 0;
    if (need <= 1)
        hipLaunchKernelGGL((recurrent_fwd_kernel<TI, TG, 1, TPR>), grid, dim3(256), lds, stream, p);
    else if (need <= 2)
        hipLaunchKernelGGL((recurrent_fwd_kernel<TI, TG, 2, TPR>), grid, dim3(256), lds, stream, p);
    else if (need <= 4)
        hipLaunchKernelGGL((recurrent_fwd_kernel<TI, TG, 4, TPR>), grid, dim3(256), lds, stream, p);
    else if (need <= 8)
        hipLaunchKernelGGL((recurrent_fwd_kernel<TI, TG, 8, TPR>), grid, dim3(256), lds, stream, p);
    else if (need <= 16)
        hipLaunchKernelGGL((recurrent_fwd_kernel<TI, TG, 16, TPR>), grid, dim3(256), lds, stream, p);
    else
        hipLaunchKernelGGL((recurrent_fwd_kernel<TI, TG, 32, TPR>), grid, dim3(256), lds, stream, p);
    return hipGetLastError();
}

template <typename TI, typename TG>
static hipError_t launch_tpr(const RecurrentParams &p, int N, hipStream_t stream)
{
    const bool trans = (p.flags & GDN2_FLAG_TRANSPOSE_STATE) != 0;
    if (p.T == 1 && !p.cu_seqlens && p.K == 128 && p.V == 128) {
        const int nslabs = N * p.HV;
        const dim3 grid((nslabs + 1) / 2);
        if (trans && p.h0)
            hipLaunchKernelGGL((decode_step_t_kernel<TI, TG, true>), grid, dim3(256), 0, stream, p, nslabs);
        else if (trans)
            hipLaunchKernelGGL((decode_step_t_kernel<TI, TG, false>), grid, dim3(256), 0, stream, p, nslabs);
        else if (p.h0)
            hipLaunchKernelGGL((decode_step_kernel<TI, TG, true>), grid, dim3(256), 0, stream, p, nslabs);
        else
            hipLaunchKernelGGL((decode_step_kernel<TI, TG, false>), grid, dim3(256), 0, stream, p, nslabs);
        return hipGetLastError();
    }
    // Narrowest row that still covers V with float4 lanes, capped at 128 columns.
    if (p.V <= 16) return launch_nr<TI, TG, 4>(p, N, stream);
    if (p.V <= 32) return launch_nr<TI, TG, 8>(p, N, stream);
    if (p.V <= 64) return launch_nr<TI, TG, 16>(p, N, stream);
    return launch_nr<TI, TG, 32>(p, N, stream);
}

template <typename TI>
static hipError_t launch_g(const RecurrentParams &p, int g_dtype, int N, hipStream_t stream)
{
    switch (g_dtype) {
    case GDN2_DTYPE_F32: return launch_tpr<TI, float>(p, N, stream);
    case GDN2_DTYPE_BF16: return launch_tpr<TI, bf16_t>(p, N, stream);
    default: return launch_tpr<TI, f16_t>(p, N, stream);
    }
}

hipError_t launch_decode_fused(const DecodeFusedParams &p, int io_dtype, int g_dtype,
                               hipStream_t stream)
{
    if (p.N == 0) return hipSuccess;
    switch (io_dtype) {
    case GDN2_DTYPE_F32: return launch_decode_fused_t<float, float>(p, stream);
    case GDN2_DTYPE_BF16:
        return g_dtype == GDN2_DTYPE_F32 ? launch_decode_fused_t<bf16_t, float>(p, stream)
                                         : launch_decode_fused_t<bf16_t, bf16_t>(p, stream);
    default:
        return g_dtype == GDN2_DTYPE_F32 ? launch_decode_fused_t<f16_t, float>(p, stream)
                                         : launch_decode_fused_t<f16_t, f16_t>(p, stream);
    }
}

hipError_t launch_recurrent_fwd(const RecurrentParams &p, int io_dtype, int g_dtype, int N,
                                hipStream_t stream)
{
    switch (io_dtype) {
    case GDN2_DTYPE_F32: return launch_g<float>(p, g_dtype, N, stream);
    case GDN2_DTYPE_BF16: return launch_g<bf16_t>(p, g_dtype, N, stream);
    default: return launch_g<f16_t>(p, g_dtype, N, stream);
    }
}

}  // namespace gdn2
