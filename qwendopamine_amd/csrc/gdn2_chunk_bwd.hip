// Chunkwise gdn2 backward (training), gfx950.
//
// Replaces reference chunk_gdn2_bwd (gdn2_ops/chunk_gdn2.py:2170-2325): the
// dAv (chunk_kda.py:4983-5031), dhu (chunk_kda.py:2297-2374), wy_dqkg
// (chunk_gdn2.py:2023-2096) and intra (chunk_gdn2.py:2099-2167) stages and
// the reverse cumulative sum of dg.  Per chunk, with the forward notation of
// gdn2_chunk_fwd.hip (S0 start state, S1 end state, dS1 its gradient):
//
//   dU  = Aqk^T dO + Kt dS1,   dY = X^T dU          (dv = dY*w, dw = dY*v)
//   dS0 = Qbar^T dO + Diag(exp(G_last)) dS1 + (-W)^T dU
//   dA  = tril(dO U^T),  dL = -strict_tril(dY U^T)
//   dq_r = exp(G_r) (dO S0^T)_r + sum_j dA[r,j] k_j exp(G_r - G_j)
//   de_r = -exp(G_r) (dY S0^T)_r + sum_j dL[r,j] k_j exp(G_r - G_j)
//   dk_j = exp(G_last - G_j) (U dS1^T)_j + sum_r (dA[r,j] q_r + dL[r,j] e_r) exp(G_r - G_j)
//   dG_r = q_r dq_r + e_r de_r - k_r dk_r,   dG_last += rowsum(dS1 * S1)
//   dg   = reverse in-chunk cumulative sum of dG;  e = b*k: db = de*k, dk += de*b
//
// followed by the scale and L2-norm chain rule on dq, dk.
//
// Two kernels, both reading what the training-mode forward left in its
// workspace (per-chunk blobs, start states S0 and U, per-sequence end states):
//  * chunk_bwd_scan_kernel -- one workgroup per (sequence, head, value
//    slice), chunks in reverse order, dS carried in fp32 accumulators.  The
//    copy waves land each forward blob in LDS with every matrix transposed
//    (the backward contracts over the dimension the forward kept), so the
//    compute waves issue the same K16 products as the forward scan.  Writes
//    dv, dw, dh0 and, per chunk, dS1 and dY for the second kernel.
//  * chunk_bwd_kside_kernel -- one workgroup (4 waves, wave R = token block R)
//    per (chunk, head), all chunks in parallel: the V-contractions above on
//    MFMA, the in-chunk pair terms with the forward's factored decays (exact
//    VALU sums on diagonal blocks whose decay span is too wide), the reverse
//    cumsum, and the chain rule to dq, dk, db, dg.

#include <type_traits>

#include "gdn2_chunk.h"
#include "gdn2_internal.h"

namespace gdn2 {

namespace {

struct BwdParams {
    const void *q, *k, *v, *g, *b, *w, *dout;
    const float *dht;
    void *dq, *dk, *dv, *dg, *db, *dw;
    float *dh0;
    const int64_t *cu_seqlens;
    int num_seqs, T, H, K, V, VP, nt;
    float scale;
    unsigned flags;
    int vec_ok;
    const void *blob, *hs, *us;  // training workspace written by the forward
    void *dhs, *dys;                    // backward scratch
};

// Unit j*256 + ct (ct < 256 the copy thread) of a forward blob, 16 bytes,
// landed in LDS with each matrix region transposed: element M[a][b] of a K16
// fragment-native [Mr][Kc] region goes to element M^T[b][a] of the
// fragment-native [Kc][Mr] region at the same base; the exp(G_last) vector
// is copied as is.  Every region boundary is a multiple of 256 units' worth
// of elements, so the region of unit group j is a compile-time constant once
// the caller's loop over j is unrolled.
template <PrecKind PK, int KP>
__device__ __forceinline__ void land_transposed(typename Prec<PK>::st *dst, u32x4 val, int j, int ct)
{
    using BL = Blob<PK, KP>;
    using st = typename Prec<PK>::st;
    constexpr int EPU = 16 / static_cast<int>(sizeof(st));
    static_assert((BL::WN % (EPU * 256)) == 0 && (BL::QB % (EPU * 256)) == 0 &&
                      (BL::AQ % (EPU * 256)) == 0 && (BL::KT % (EPU * 256)) == 0 &&
                      (BL::GL % (EPU * 256)) == 0,
                  "blob regions must align to 256-unit groups");
    const int e0 = EPU * 256 * j;
    const int e = e0 + EPU * ct;
    int base, Mr, Kc;
    if (e0 < BL::WN) {
        base = BL::X; Mr = 64; Kc = 64;
    } else if (e0 < BL::QB) {
        base = BL::WN; Mr = 64; Kc = KP;
    } else if (e0 < BL::AQ) {
        base = BL::QB; Mr = 64; Kc = KP;
    } else if (e0 < BL::KT) {
        base = BL::AQ; Mr = 64; Kc = 64;
    } else if (e0 < BL::GL) {
        base = BL::KT; Mr = KP; Kc = 64;
    } else {
        *reinterpret_cast<u32x4 *>(dst + e) = val;
        return;
    }
    const int loc = e - base, blk = loc >> 8, wi = loc & 255;
    const int nkc = Kc >> 4, nm = Mr >> 4;
    const int mt = blk / nkc, kt = blk - mt * nkc;
    const int L0 = wi >> 2, a0 = L0 & 15, b0 = (L0 >> 4) * 4;
    st *d = dst + base + ((kt * nm + mt) << 8) + 4 * b0 + 64 * (a0 >> 2) + (a0 & 3);
    if constexpr (EPU == 8) {
        // Lanes L0 (row a0) and L0 + 1 (row a0 + 1): the pair (M[a0][b], M[a0+1][b])
        // is contiguous in the transposed block.
        uint32_t *d32 = reinterpret_cast<uint32_t *>(d);
        d32[0] = (val.x & 0xffffu) | (val.z << 16);
        d32[2] = (val.x >> 16) | (val.z & 0xffff0000u);
        d32[4] = (val.y & 0xffffu) | (val.w << 16);
        d32[6] = (val.y >> 16) | (val.w & 0xffff0000u);
    } else {
        // (__uint_as_float takes the component by value; a bit cast of a vector
        // component expression reads the vector's first element instead.)
        d[0] = __uint_as_float(val.x);
        d[4] = __uint_as_float(val.y);
        d[8] = __uint_as_float(val.z);
        d[12] = __uint_as_float(val.w);
    }
}

// ---------------------------------------------------------------------------
// Reverse state scan: one workgroup per (sequence, head, value slice of BV
// columns).  Waves 0..3 compute (wave c owns value columns 16c..16c+15 of
// the slice, dS columns in fp32 accumulators), waves 4..7 land blobs and dO.
// ---------------------------------------------------------------------------
template <PrecKind PK, int KP, int BV, typename TI>
__global__ __launch_bounds__(512) void chunk_bwd_scan_kernel(BwdParams p, int NVB, int NP)
{
    using P = Prec<PK>;
    using st = typename P::st;
    using BL = Blob<PK, KP>;
    using Q = Q4<PK>;
    constexpr bool DB = PK != PrecKind::F32;  // double-buffered blobs (16-bit only)
    constexpr int NBUF = DB ? 2 : 1;
    constexpr int NKT = KP / 16, NKS = KP / 32, NCT = BV / 16;
    constexpr int U16 = static_cast<int>(BL::BYTES / 16);
    constexpr int PF = (U16 + 255) / 256;
    __shared__ __align__(16) st sB[NBUF][BL::SIZE];
    // dO of the chunk as K16 B operands: block (token tile kt, column tile c).
    __shared__ __align__(16) st sD[NBUF][16 * 256];

    // XCD-aware order, as in the forward scan.
    const int Lid = blockIdx.x;
    const int xcd = Lid & 7, rest = Lid >> 3;
    const int vs = rest % NVB, grp = rest / NVB;
    const int pair = 8 * grp + xcd;
    if (pair >= NP) return;
    const int H = p.H, K = p.K, V = p.V, VP = p.VP;
    const int n = pair / H, h = pair % H;

    const int tid = threadIdx.x, wv = tid >> 6, l = tid & 63, m = l & 15, kg = l >> 4;
    const bool copier = wv >= 4;
    const int ctid = tid - 256;
    const bool active = wv < NCT;
    const int col = vs * BV + 16 * wv + m;
    const bool col_ok = active && col < V;
    const int vt = vs * NCT + wv;
    const bool emit = active && 16 * vt < V;
    int64_t bos, len;
    const int gc0 = seq_chunk_base(p, n, bos, len);
    const int nch = static_cast<int>((len + kChunk - 1) / kChunk);

    const TI *vp = static_cast<const TI *>(p.v);
    const TI *wp = static_cast<const TI *>(p.w);
    const TI *dop = static_cast<const TI *>(p.dout);
    TI *dvp = static_cast<TI *>(p.dv);
    TI *dwp = static_cast<TI *>(p.dw);
    const st *wsb = static_cast<const st *>(p.blob);
    auto blob = [&](int gci) {
        return reinterpret_cast<const u32x4 *>(wsb + (static_cast<int64_t>(gci) * H + h) * BL::SIZE);
    };
    auto chunk_rows = [&](int jc, int64_t &t0, int &lc) __attribute__((always_inline)) {
        t0 = bos + static_cast<int64_t>(jc) * kChunk;
        const int64_t rem = len - static_cast<int64_t>(jc) * kChunk;
        lc = rem < kChunk ? static_cast<int>(rem) : kChunk;
    };

    // Copy waves: dO rows of chunk jc for this value slice in the K16
    // B-operand order (zero past the sequence end and past V).
    const int v0 = vs * BV;
    constexpr int EPV = 16 / static_cast<int>(sizeof(TI));
    constexpr int ZT = kChunk * BV / EPV;
    constexpr int NZT = (ZT + 255) / 256;
    const bool dvec = (V % EPV) == 0;
    struct DRaw {
        u32x4 d[NZT];
    };
    auto issue_d = [&](DRaw &r, int jc) __attribute__((always_inline)) {
        int64_t t0;
        int lc;
        chunk_rows(jc, t0, lc);
#pragma unroll
        for (int a = 0; a < NZT; ++a) {
            const int task = ctid + 256 * a;
            const int tok = task / (BV / EPV), c = EPV * (task % (BV / EPV));
            const bool ok = task < ZT && tok < lc && dvec && v0 + c + EPV <= V;
            const int64_t off = ((t0 + tok) * H + h) * V + v0 + c;
            r.d[a] = ok ? *reinterpret_cast<const u32x4 *>(dop + off) : u32x4{0, 0, 0, 0};
        }
    };
    auto land_d = [&](const DRaw &r, int jc, int buf) __attribute__((always_inline)) {
        int64_t t0;
        int lc;
        chunk_rows(jc, t0, lc);
        st *dst = sD[buf];
#pragma unroll
        for (int a = 0; a < NZT; ++a) {
            const int task = ctid + 256 * a;
            if (task >= ZT) continue;
            const int tok = task / (BV / EPV), c = EPV * (task % (BV / EPV));
            const TI *rd = reinterpret_cast<const TI *>(&r.d[a]);
            const bool ok = tok < lc && dvec && v0 + c + EPV <= V;
            const int kt = tok >> 4, kgz = (tok & 15) >> 2, iz = tok & 3;
#pragma unroll
            for (int e = 0; e < EPV; ++e) {
                float x = 0.f;
                if (ok)
                    x = io<TI>::ld(rd, e);
                else if (tok < lc && v0 + c + e < V)
                    x = io<TI>::ld(dop, ((t0 + tok) * H + h) * V + v0 + c + e);
                const int cl = c + e, ct = cl >> 4, nz = cl & 15;
                dst[(kt * 4 + ct) * 256 + (nz + 16 * kgz) * 4 + iz] = P::from_f32(x);
            }
        }
    };

    // Whole blob straight from global memory into LDS buffer 0.
    auto land_all = [&](const u32x4 *src) __attribute__((always_inline)) {
#pragma unroll
        for (int u = 0; u < PF; ++u)
            if (ctid + 256 * u < U16) land_transposed<PK, KP>(sB[0], src[ctid + 256 * u], u, ctid);
    };

    // dS columns of this wave: rows 16kt + 4kg + i, column col; starts at dht.
    f32x4 dS[NKT];
#pragma unroll
    for (int kt = 0; kt < NKT; ++kt) {
        dS[kt] = zero4();
        if (p.dht && col_ok) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int row = 16 * kt + 4 * kg + i;
                if (row < K) dS[kt][i] = p.dht[((static_cast<int64_t>(n) * H + h) * K + row) * V + col];
            }
        }
    }

    // Step s handles chunk nch-1-s.  Barrier schedule as in the forward scan.
    if (copier) {
        DRaw dA, dB;
        if (nch > 0) {
            land_all(blob(gc0 + nch - 1));
            issue_d(dA, nch - 1);
            land_d(dA, nch - 1, 0);
        }
        if constexpr (DB) {
            u32x4 pA[PF], pB[PF];
            auto issue = [&](u32x4 (&dst)[PF], int gci) __attribute__((always_inline)) {
                const u32x4 *src = blob(gci);
#pragma unroll
                for (int u = 0; u < PF; ++u) {
                    const int idx = ctid + 256 * u;
                    dst[u] = src[idx < U16 ? idx : U16 - 1];
                }
            };
            auto land = [&](const u32x4 (&src)[PF], int buf) __attribute__((always_inline)) {
#pragma unroll
                for (int u = 0; u < PF; ++u)
                    if (ctid + 256 * u < U16) land_transposed<PK, KP>(sB[buf], src[u], u, ctid);
            };
            if (nch > 1) {
                issue(pA, gc0 + nch - 2);
                issue_d(dA, nch - 2);
            }
            __syncthreads();
            for (int s = 0; s < nch; s += 2) {
                if (s + 2 < nch) {
                    issue(pB, gc0 + nch - 3 - s);
                    issue_d(dB, nch - 3 - s);
                }
                if (s + 1 < nch) {
                    land_d(dA, nch - 2 - s, 1);
                    land(pA, 1);
                }
                __syncthreads();
                if (s + 1 >= nch) break;
                if (s + 3 < nch) {
                    issue(pA, gc0 + nch - 4 - s);
                    issue_d(dA, nch - 4 - s);
                }
                if (s + 2 < nch) {
                    land_d(dB, nch - 3 - s, 0);
                    land(pB, 0);
                }
                __syncthreads();
            }
        } else {
            __syncthreads();
            for (int s = 0; s < nch; ++s) {
                __syncthreads();
                if (s + 1 < nch) {
                    const int jn = nch - 2 - s;
                    land_all(blob(gc0 + jn));
                    issue_d(dA, jn);
                    land_d(dA, jn, 0);
                    __syncthreads();
                }
            }
        }
    } else {
        const Q ident = identity_q4<PK>(l);
        __syncthreads();
        for (int s = 0; s < nch; ++s) {
            const int buf = DB ? (s & 1) : 0;
            const int jc = nch - 1 - s;
            if (active) {
                const st *Bk = sB[buf];
                int64_t t0;
                int lc;
                chunk_rows(jc, t0, lc);
                const int64_t cb = static_cast<int64_t>(gc0 + jc) * H + h;

                // dS1 of this chunk for the K-side kernel (A-order tiles).
                if (emit) {
                    st *dhb = static_cast<st *>(p.dhs) + cb * (KP * VP);
#pragma unroll
                    for (int kt = 0; kt < NKT; ++kt)
                        st_q4<PK>(dhb + k16_block(kt, vt, VP) + 4 * l,
                                  pack4<PK>(mma1<PK>(zero4(), pack4<PK>(dS[kt]), ident)));
                }

                Q df[4];
#pragma unroll
                for (int kt = 0; kt < 4; ++kt) df[kt] = ld_q4<PK>(sD[buf] + (kt * 4 + wv) * 256 + 4 * l);
                Q sf[NKT];
#pragma unroll
                for (int kt = 0; kt < NKT; ++kt) sf[kt] = pack4<PK>(dS[kt]);

                // dU = Aqk^T dO + Kt dS1 (Aqk^T is block upper triangular).
                Q duf[4];
#pragma unroll
                for (int rt = 0; rt < 4; ++rt) {
                    f32x4 acc = zero4();
#pragma unroll
                    for (int s2 = 0; s2 < 2; ++s2)
                        if (2 * s2 + 1 >= rt)
                            acc = mma2<PK>(acc, ld_q4<PK>(Bk + BL::AQ + k16_block(rt, 2 * s2, 64) + 4 * l),
                                           ld_q4<PK>(Bk + BL::AQ + k16_block(rt, 2 * s2 + 1, 64) + 4 * l),
                                           df[2 * s2], df[2 * s2 + 1]);
#pragma unroll
                    for (int s2 = 0; s2 < NKS; ++s2)
                        acc = mma2<PK>(acc, ld_q4<PK>(Bk + BL::KT + k16_block(rt, 2 * s2, KP) + 4 * l),
                                       ld_q4<PK>(Bk + BL::KT + k16_block(rt, 2 * s2 + 1, KP) + 4 * l),
                                       sf[2 * s2], sf[2 * s2 + 1]);
                    duf[rt] = pack4<PK>(acc);
                }
                // dY = X^T dU; dv = dY * w, dw = dY * v.
                // v and w at this wave's (token, column) positions, for dv, dw.
                float vv[4][4], ww[4][4];
#pragma unroll
                for (int rt = 0; rt < 4; ++rt)
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const int tok = 16 * rt + 4 * kg + i;
                        const bool ok = col_ok && tok < lc;
                        const int64_t off = ((t0 + tok) * H + h) * V + col;
                        vv[rt][i] = ok ? io<TI>::ld(vp, off) : 0.f;
                        ww[rt][i] = ok ? io<TI>::ld(wp, off) : 0.f;
                    }
                st *dyb = static_cast<st *>(p.dys) + cb * (64 * VP);
#pragma unroll
                for (int rt = 0; rt < 4; ++rt) {
                    f32x4 acc = zero4();
#pragma unroll
                    for (int s2 = 0; s2 < 2; ++s2)
                        if (2 * s2 + 1 >= rt)
                            acc = mma2<PK>(acc, ld_q4<PK>(Bk + BL::X + k16_block(rt, 2 * s2, 64) + 4 * l),
                                           ld_q4<PK>(Bk + BL::X + k16_block(rt, 2 * s2 + 1, 64) + 4 * l),
                                           duf[2 * s2], duf[2 * s2 + 1]);
                    if (col_ok) {
#pragma unroll
                        for (int i = 0; i < 4; ++i) {
                            const int tok = 16 * rt + 4 * kg + i;
                            if (tok < lc) {
                                const int64_t off = ((t0 + tok) * H + h) * V + col;
                                io<TI>::st(dvp, off, acc[i] * ww[rt][i]);
                                io<TI>::st(dwp, off, acc[i] * vv[rt][i]);
                            }
                        }
                    }
                    if (emit)
                        st_q4<PK>(dyb + k16_block(rt, vt, VP) + 4 * l,
                                  pack4<PK>(mma1<PK>(zero4(), pack4<PK>(acc), ident)));
                }
                // dS0 = Diag(exp(G_last)) dS1 + Qbar^T dO + (-W)^T dU.
                const float *gl = reinterpret_cast<const float *>(Bk + BL::GL);
#pragma unroll
                for (int kt = 0; kt < NKT; ++kt) {
                    const float4 gv = *reinterpret_cast<const float4 *>(gl + 16 * kt + 4 * kg);
                    dS[kt][0] *= gv.x;
                    dS[kt][1] *= gv.y;
                    dS[kt][2] *= gv.z;
                    dS[kt][3] *= gv.w;
#pragma unroll
                    for (int s2 = 0; s2 < 2; ++s2) {
                        dS[kt] = mma2<PK>(dS[kt], ld_q4<PK>(Bk + BL::QB + k16_block(kt, 2 * s2, 64) + 4 * l),
                                          ld_q4<PK>(Bk + BL::QB + k16_block(kt, 2 * s2 + 1, 64) + 4 * l),
                                          df[2 * s2], df[2 * s2 + 1]);
                        dS[kt] = mma2<PK>(dS[kt], ld_q4<PK>(Bk + BL::WN + k16_block(kt, 2 * s2, 64) + 4 * l),
                                          ld_q4<PK>(Bk + BL::WN + k16_block(kt, 2 * s2 + 1, 64) + 4 * l),
                                          duf[2 * s2], duf[2 * s2 + 1]);
                    }
                }
            }
            __syncthreads();
            if constexpr (!DB) {
                if (s + 1 < nch) __syncthreads();
            }
        }
    }

    if (p.dh0 && col_ok) {
#pragma unroll
        for (int kt = 0; kt < NKT; ++kt)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int row = 16 * kt + 4 * kg + i;
                if (row < K) p.dh0[((static_cast<int64_t>(n) * H + h) * K + row) * V + col] = dS[kt][i];
            }
    }
}


// Decay factor of the (row block Rb, column block Ib) pair at channel c, in
// the factored pair products: 2^(decay strictly between the blocks) below the
// diagonal, 2^(-block span) on it, 0 above it (T = in-block decay totals).
__device__ __forceinline__ float pair_factor(const float (*sT)[128 + 4], int Rb, int Ib, int c)
{
    if (Ib > Rb) return 0.f;
    if (Ib == Rb) return __builtin_amdgcn_exp2f(-sT[Rb][c]);
    float ex = 0.f;
#pragma unroll
    for (int R2 = 1; R2 < 3; ++R2)
        if (R2 > Ib && R2 < Rb) ex += sT[R2][c];
    return __builtin_amdgcn_exp2f(ex);
}

// ---------------------------------------------------------------------------
// K-side gradients: one workgroup (4 waves) per (chunk, head).  Wave R owns
// token rows 16R..16R+15; lane (m, kg) holds row 16R+m, channels
// 16kt + 4kg + i ("A-order", as in the forward prep kernel).
// ---------------------------------------------------------------------------
template <PrecKind PK, int KP, typename TI, typename TG>
__global__ __launch_bounds__(256) void chunk_bwd_kside_kernel(BwdParams p)
{
    using P = Prec<PK>;
    using st = typename P::st;
    using Q = Q4<PK>;
    constexpr int NKT = KP / 16;
    constexpr int NVS = 4;  // value tiles per staged slice (64 columns)
    // dg is a reverse cumulative sum in which the in-chunk pair terms cancel
    // in exact arithmetic; to keep that cancellation accurate, operands that
    // reach dg (chunk states and U from the forward, the factor tiles) carry
    // fp32 precision: for 16-bit MFMA operands as two planes, x = hi + lo.
    constexpr int NPL = PK == PrecKind::F32 ? 1 : 2;
    // Transposed (B-order) factor tiles of every token block, for the pair products.
    __shared__ __align__(16) st sKT[NPL][4][NKT][256];  // k * 2^(T_R - G)       (kend)
    __shared__ __align__(16) st sQT[NPL][4][NKT][256];  // q * 2^G               (qb)
    __shared__ __align__(16) st sET[NPL][4][NKT][256];  // e * 2^G               (eb)
    // dO, U, dY of one 64-column value slice: A-order blocks (token tile, value tile).
    __shared__ __align__(16) st sO[4 * NVS * 256];
    __shared__ __align__(16) st sU[NPL][4 * NVS * 256];
    __shared__ __align__(16) st sY[4 * NVS * 256];
    __shared__ __align__(16) float sT[4][128 + 4];  // in-block decay totals (log2)
    __shared__ __align__(16) float sEr[4][KP];      // 2^(decay before block)
    __shared__ __align__(16) float sEa[4][KP];      // 2^(decay after block)
    __shared__ __align__(16) float sDG[4][KP];      // per-block sums of dG
    __shared__ __align__(16) float sLast[KP];       // exp(G_last) rowsum(dS1 * S0)
    __shared__ __align__(16) float sKK[4][KP];      // per-block sum_j dKt_j * Kt_j

    const int tid = threadIdx.x, R = tid >> 6, l = tid & 63, m = l & 15, kg = l >> 4;
    const int gc = blockIdx.x, h = blockIdx.y;
    const int H = p.H, K = p.K, V = p.V, VP = p.VP;

    int n, jc;
    int64_t bos, len;
    locate_chunk(p, gc, n, jc, bos, len);
    const int nch = static_cast<int>((len + kChunk - 1) / kChunk);
    const int64_t t0 = bos + static_cast<int64_t>(jc) * kChunk;
    const int64_t rem = len - static_cast<int64_t>(jc) * kChunk;
    const int lc = rem < kChunk ? static_cast<int>(rem) : kChunk;
    const int r = 16 * R + m;
    const bool row_ok = r < lc;
    const int64_t roff = ((t0 + r) * H + h) * K;
    const int64_t cb = static_cast<int64_t>(gc) * H + h;

    const TI *q = static_cast<const TI *>(p.q);
    const TI *k = static_cast<const TI *>(p.k);
    const TI *b = static_cast<const TI *>(p.b);
    const TG *g = static_cast<const TG *>(p.g);
    const bool l2 = (p.flags & GDN2_FLAG_L2NORM_QK) != 0;
    const Q ident = identity_q4<PK>(l);

    // Row norms (kept), in-block log2 decay prefix of channel tile kt.
    float invq, invk;
    bool bigq, bigk;  // ||x|| above the F.normalize epsilon
    auto row_tile = [&](int kt, float (&qv)[4], float (&kv)[4], float (&bv)[4], float (&gv)[4])
        __attribute__((always_inline)) {
        const int c0 = 16 * kt + 4 * kg;
        load4<TI>(q, roff, c0, K, row_ok, p.vec_ok, qv);
        load4<TI>(k, roff, c0, K, row_ok, p.vec_ok, kv);
        load4<TI>(b, roff, c0, K, row_ok, p.vec_ok, bv);
        load4<TG>(g, roff, c0, K, row_ok, p.vec_ok, gv);
#pragma unroll
        for (int i = 0; i < 4; ++i) gv[i] = row16_scan(gv[i] * kLog2e);
    };
    {
        float sq = 0.f, sk = 0.f;
#pragma unroll
        for (int kt = 0; kt < NKT; ++kt) {
            float qv[4], kv[4];
            const int c0 = 16 * kt + 4 * kg;
            load4<TI>(q, roff, c0, K, row_ok, p.vec_ok, qv);
            load4<TI>(k, roff, c0, K, row_ok, p.vec_ok, kv);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                sq = fmaf(qv[i], qv[i], sq);
                sk = fmaf(kv[i], kv[i], sk);
            }
        }
        sq += __shfl_xor(sq, 16, 64);
        sq += __shfl_xor(sq, 32, 64);
        sk += __shfl_xor(sk, 16, 64);
        sk += __shfl_xor(sk, 32, 64);
        invq = l2 ? 1.0f / fmaxf(sqrtf(sq), 1e-6f) : 1.0f;
        invk = l2 ? 1.0f / fmaxf(sqrtf(sk), 1e-6f) : 1.0f;
        bigq = sqrtf(sq) > 1e-6f;
        bigk = sqrtf(sk) > 1e-6f;
    }
    const float qmul = invq * p.scale;

    // Block totals and the wide-span flag of this wave's diagonal block.
    bool wide = false;
#pragma unroll
    for (int kt = 0; kt < NKT; ++kt) {
        float qv[4], kv[4], bv[4], gv[4];
        row_tile(kt, qv, kv, bv, gv);
        if (m == 15) {
            *reinterpret_cast<float4 *>(&sT[R][16 * kt + 4 * kg]) = make_float4(gv[0], gv[1], gv[2], gv[3]);
#pragma unroll
            for (int i = 0; i < 4; ++i) wide = wide || (-gv[i] > kDiagSpanLimit2);
        }
    }
    const bool wave_slow = __ballot(wide) != 0;
    __syncthreads();
    for (int e = tid; e < 4 * KP; e += 256) {
        const int Rb = e / KP, c = e % KP;
        float cum = 0.f, after = 0.f;
#pragma unroll
        for (int R2 = 0; R2 < 4; ++R2) {
            if (R2 < Rb) cum += sT[R2][c];
            if (R2 > Rb) after += sT[R2][c];
        }
        sEr[Rb][c] = fexp2(cum);
        sEa[Rb][c] = fexp2(after);
    }
    // Factor tiles, transposed by an identity product.
#pragma unroll
    for (int kt = 0; kt < NKT; ++kt) {
        float qv[4], kv[4], bv[4], gv[4];
        row_tile(kt, qv, kv, bv, gv);
        const float4 tr = *reinterpret_cast<const float4 *>(&sT[R][16 * kt + 4 * kg]);
        const float trv[4] = {tr.x, tr.y, tr.z, tr.w};
        float qb[4], eb[4], ke[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float kn = kv[i] * invk;
            const float e1 = fexp2(gv[i]);
            qb[i] = qv[i] * qmul * e1;
            eb[i] = bv[i] * kn * e1;
            ke[i] = kn * fexp2(trv[i] - gv[i]);
        }
        auto put = [&](st (*dst)[4][NKT][256], const float (&x)[4]) __attribute__((always_inline)) {
            const Q hi = pack4<PK>(x[0], x[1], x[2], x[3]);
            st_q4<PK>(&dst[0][R][kt][4 * l], pack4<PK>(mma1<PK>(zero4(), hi, ident)));
            if constexpr (NPL == 2) {
                float xh[4];
                unpack4<PK>(hi, xh);
                const Q lo = pack4<PK>(x[0] - xh[0], x[1] - xh[1], x[2] - xh[2], x[3] - xh[3]);
                st_q4<PK>(&dst[1][R][kt][4 * l], pack4<PK>(mma1<PK>(zero4(), lo, ident)));
            }
        };
        put(sKT, ke);
        put(sQT, qb);
        put(sET, eb);
    }

    // G_last term, part 1: exp(G_last) rowsum(dS1 * S0).  (With part 2,
    // sum_j dKt_j Kt_j, this is rowsum(dS1 * S1) written through the saved S0
    // and U only, so it stays consistent with the other terms of dg.)  Wave R
    // takes channel tiles R, R+4, ...
    {
        const st *dh = static_cast<const st *>(p.dhs) + cb * (KP * VP);
        const st *s0 = static_cast<const st *>(p.hs) + cb * (NPL * KP * VP);
        for (int dt = R; dt < NKT; dt += 4) {
            float acc = 0.f;
            for (int vt = 0; vt < VP / 16; ++vt) {
                float a[4], c[4];
                unpack4<PK>(ld_q4<PK>(dh + k16_block(dt, vt, VP) + 4 * l), a);
#pragma unroll
                for (int pl = 0; pl < NPL; ++pl) {
                    unpack4<PK>(ld_q4<PK>(s0 + pl * (KP * VP) + k16_block(dt, vt, VP) + 4 * l), c);
#pragma unroll
                    for (int i = 0; i < 4; ++i) acc = fmaf(a[i], c[i], acc);
                }
            }
            acc += __shfl_xor(acc, 16, 64);
            acc += __shfl_xor(acc, 32, 64);
            const int c = 16 * dt + m;
            if (kg == 0) sLast[c] = acc * fexp2(sT[0][c] + sT[1][c] + sT[2][c] + sT[3][c]);
        }
    }

    // V-contractions, one staged 64-column slice at a time:
    //   aT[J] = dAqk^T tile (J, R)    lT[J] = -dL^T tile (J, R)     (J <= R)
    //   aN[I] = dAqk tile (I, R)      lN[I] = -dL tile (I, R)       (I >= R)
    //   cq[dt] = dQbar tile, ce[dt] = -dEbar tile, ck[dt] = dKtilde tile (row data)
    f32x4 aT[4], lT[4], aN[4], lN[4], cq[NKT], ce[NKT], ck[NKT];
#pragma unroll
    for (int J = 0; J < 4; ++J) aT[J] = lT[J] = aN[J] = lN[J] = zero4();
#pragma unroll
    for (int dt = 0; dt < NKT; ++dt) cq[dt] = ce[dt] = ck[dt] = zero4();
    const st *hsb = static_cast<const st *>(p.hs) + cb * (NPL * KP * VP);
    const st *dhb = static_cast<const st *>(p.dhs) + cb * (KP * VP);
    const st *usb = static_cast<const st *>(p.us) + cb * (NPL * 64 * VP);
    const st *dyb = static_cast<const st *>(p.dys) + cb * (64 * VP);
    const TI *dop = static_cast<const TI *>(p.dout);
    const int NVT = VP / 16;
    constexpr int EPU = 16 / static_cast<int>(sizeof(st));
    for (int vt0 = 0; vt0 < NVT; vt0 += NVS) {
        __syncthreads();  // previous slice fully consumed
        // U and dY: contiguous A-order blocks, copied as 16-byte units.
        for (int u = tid; u < 4 * NVS * 256 / EPU; u += 256) {
            const int e = u * EPU, blk = e >> 8, rt = blk / NVS, vl = blk % NVS;
            const bool ok = vt0 + vl < NVT;
            const int64_t src = k16_block(rt, vt0 + vl, VP) + (e & 255);
#pragma unroll
            for (int pl = 0; pl < NPL; ++pl)
                *reinterpret_cast<u32x4 *>(sU[pl] + e) =
                    ok ? *reinterpret_cast<const u32x4 *>(usb + pl * (64 * VP) + src) : u32x4{0, 0, 0, 0};
            *reinterpret_cast<u32x4 *>(sY + e) = ok ? *reinterpret_cast<const u32x4 *>(dyb + src) : u32x4{0, 0, 0, 0};
        }
        // dO: rows of the chunk, 4 consecutive values per A-order group.
        for (int task = tid; task < 64 * NVS * 4; task += 256) {
            const int tok = task / (NVS * 4), grp = task % (NVS * 4);
            const int c = 16 * vt0 + 4 * grp;
            float x[4];
            const int64_t off = ((t0 + tok) * H + h) * static_cast<int64_t>(V);
            const bool ok = tok < lc;
            if (ok && (V % 4) == 0 && c + 4 <= V) {
                load4<TI>(dop, off, c, V, true, 1, x);
            } else {
#pragma unroll
                for (int i = 0; i < 4; ++i) x[i] = (ok && c + i < V) ? io<TI>::ld(dop, off + c + i) : 0.f;
            }
            const int vl = grp >> 2, kgo = grp & 3;
            st_q4<PK>(sO + k16_block(tok >> 4, vl, 16 * NVS) + 4 * ((tok & 15) + 16 * kgo),
                      pack4<PK>(x[0], x[1], x[2], x[3]));
        }
        __syncthreads();
#pragma unroll
        for (int s2 = 0; s2 < NVS / 2; ++s2) {
            const int va = 2 * s2, vb = 2 * s2 + 1;
            const Q oR0 = ld_q4<PK>(sO + k16_block(R, va, 16 * NVS) + 4 * l);
            const Q oR1 = ld_q4<PK>(sO + k16_block(R, vb, 16 * NVS) + 4 * l);
            const Q yR0 = ld_q4<PK>(sY + k16_block(R, va, 16 * NVS) + 4 * l);
            const Q yR1 = ld_q4<PK>(sY + k16_block(R, vb, 16 * NVS) + 4 * l);
            const bool oka = vt0 + va < NVT, okb = vt0 + vb < NVT;
#pragma unroll
            for (int pl = 0; pl < NPL; ++pl) {
                const Q uR0 = ld_q4<PK>(sU[pl] + k16_block(R, va, 16 * NVS) + 4 * l);
                const Q uR1 = ld_q4<PK>(sU[pl] + k16_block(R, vb, 16 * NVS) + 4 * l);
#pragma unroll
                for (int J = 0; J < 4; ++J) {
                    if (J <= R) {
                        const Q u0 = ld_q4<PK>(sU[pl] + k16_block(J, va, 16 * NVS) + 4 * l);
                        const Q u1 = ld_q4<PK>(sU[pl] + k16_block(J, vb, 16 * NVS) + 4 * l);
                        aT[J] = mma2<PK>(aT[J], u0, u1, oR0, oR1);
                        lT[J] = mma2<PK>(lT[J], u0, u1, yR0, yR1);
                    }
                    if (J >= R) {
                        aN[J] = mma2<PK>(aN[J], ld_q4<PK>(sO + k16_block(J, va, 16 * NVS) + 4 * l),
                                         ld_q4<PK>(sO + k16_block(J, vb, 16 * NVS) + 4 * l), uR0, uR1);
                        lN[J] = mma2<PK>(lN[J], ld_q4<PK>(sY + k16_block(J, va, 16 * NVS) + 4 * l),
                                         ld_q4<PK>(sY + k16_block(J, vb, 16 * NVS) + 4 * l), uR0, uR1);
                    }
                }
#pragma unroll
                for (int dt = 0; dt < NKT; ++dt) {
                    const Q z = pack4<PK>(0.f, 0.f, 0.f, 0.f);
                    const st *hp = hsb + pl * (KP * VP);
                    const Q h0 = oka ? ld_q4<PK>(hp + k16_block(dt, vt0 + va, VP) + 4 * l) : z;
                    const Q h1 = okb ? ld_q4<PK>(hp + k16_block(dt, vt0 + vb, VP) + 4 * l) : z;
                    cq[dt] = mma2<PK>(cq[dt], h0, h1, oR0, oR1);
                    ce[dt] = mma2<PK>(ce[dt], h0, h1, yR0, yR1);
                    const Q d0 = oka ? ld_q4<PK>(dhb + k16_block(dt, vt0 + va, VP) + 4 * l) : z;
                    const Q d1 = okb ? ld_q4<PK>(dhb + k16_block(dt, vt0 + vb, VP) + 4 * l) : z;
                    ck[dt] = mma2<PK>(ck[dt], d0, d1, uR0, uR1);
                }
            }
        }
    }

    // Causal masks (and the signs of dL); the diagonal tiles are kept for the
    // exact path.  aT/lT lane values: row 16R+m, column 16J+4kg+i; aN/lN:
    // row 16I+4kg+i, column 16R+m.
    f32x4 dAd = zero4(), dLd = zero4(), dANd = zero4(), dLNd = zero4();
#pragma unroll
    for (int J = 0; J < 4; ++J) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int rT = 16 * R + m, cT = 16 * J + 4 * kg + i;
            aT[J][i] = cT <= rT ? aT[J][i] : 0.f;
            lT[J][i] = cT < rT ? -lT[J][i] : 0.f;
            const int rN = 16 * J + 4 * kg + i, cN = 16 * R + m;
            aN[J][i] = cN <= rN ? aN[J][i] : 0.f;
            lN[J][i] = cN < rN ? -lN[J][i] : 0.f;
        }
        if (J == R) {
            dAd = aT[J];
            dLd = lT[J];
            dANd = aN[J];
            dLNd = lN[J];
        }
    }

    // G_last term, part 2: this block's rows of sum_j dKt_j Kt_j (ck = dKt here).
#pragma unroll
    for (int dt = 0; dt < NKT; ++dt) {
        float qv[4], kv[4], bv[4], gv[4];
        row_tile(dt, qv, kv, bv, gv);
        const float4 tr = *reinterpret_cast<const float4 *>(&sT[R][16 * dt + 4 * kg]);
        const float4 ea = *reinterpret_cast<const float4 *>(&sEa[R][16 * dt + 4 * kg]);
        const float trv[4] = {tr.x, tr.y, tr.z, tr.w}, eav[4] = {ea.x, ea.y, ea.z, ea.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float kt_ = kv[i] * invk * fexp2(trv[i] - gv[i]) * eav[i];
            const float tot = row16_scan(ck[dt][i] * kt_);
            if (m == 15) sKK[R][16 * dt + 4 * kg + i] = tot;
        }
    }

    // Pair products.  The row-data accumulators start from the V-contractions
    // scaled by the decay before / after the block: cq <- Er * dQbar,
    // ce <- Er * dEbar (ce held +dY S0^T, hence the sign), ck <- Ea * dKtilde.
#pragma unroll
    for (int dt = 0; dt < NKT; ++dt) {
        const float4 er = *reinterpret_cast<const float4 *>(&sEr[R][16 * dt + 4 * kg]);
        const float4 ea = *reinterpret_cast<const float4 *>(&sEa[R][16 * dt + 4 * kg]);
        const float erv[4] = {er.x, er.y, er.z, er.w}, eav[4] = {ea.x, ea.y, ea.z, ea.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            cq[dt][i] *= erv[i];
            ce[dt][i] *= -erv[i];
            ck[dt][i] *= eav[i];
        }
    }
    Q baT[4], blT[4], baN[4], blN[4];
#pragma unroll
    for (int J = 0; J < 4; ++J) {
        baT[J] = pack4<PK>(aT[J]);
        blT[J] = pack4<PK>(lT[J]);
        baN[J] = pack4<PK>(aN[J]);
        blN[J] = pack4<PK>(lN[J]);
    }
    // Factor tile (hi + lo planes) times a per-lane decay factor, split again
    // into hi + lo operands.
    struct Q2 {
        Q hi, lo;
    };
    auto scaled = [&](const st (*tile)[4][NKT][256], int blk, int dt, float f) __attribute__((always_inline)) {
        float x[4];
        unpack4<PK>(ld_q4<PK>(&tile[0][blk][dt][4 * l]), x);
        if constexpr (NPL == 2) {
            float y[4];
            unpack4<PK>(ld_q4<PK>(&tile[1][blk][dt][4 * l]), y);
#pragma unroll
            for (int i = 0; i < 4; ++i) x[i] += y[i];
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) x[i] *= f;
        Q2 r;
        r.hi = pack4<PK>(x[0], x[1], x[2], x[3]);
        if constexpr (NPL == 2) {
            float xh[4];
            unpack4<PK>(r.hi, xh);
            r.lo = pack4<PK>(x[0] - xh[0], x[1] - xh[1], x[2] - xh[2], x[3] - xh[3]);
        }
        return r;
    };
    auto mma2x = [&](f32x4 acc, const Q2 &a0, const Q2 &a1, Q b0, Q b1) __attribute__((always_inline)) {
        acc = mma2<PK>(acc, a0.hi, a1.hi, b0, b1);
        if constexpr (NPL == 2) acc = mma2<PK>(acc, a0.lo, a1.lo, b0, b1);
        return acc;
    };
#pragma unroll
    for (int dt = 0; dt < NKT; ++dt) {
        const int c = 16 * dt + m;  // channel of this lane in the transposed tiles
#pragma unroll
        for (int s2 = 0; s2 < 2; ++s2) {
            const int J0 = 2 * s2, J1 = 2 * s2 + 1;
            // Terms of dq, de: column blocks J <= R.
            if (J0 <= R) {
                const float f0 = (J0 == R && wave_slow) ? 0.f : pair_factor(sT, R, J0, c);
                const float f1 = (J1 == R && wave_slow) ? 0.f : pair_factor(sT, R, J1, c);
                const Q2 a0 = scaled(sKT, J0, dt, f0), a1 = scaled(sKT, J1, dt, f1);
                cq[dt] = mma2x(cq[dt], a0, a1, baT[J0], baT[J1]);
                ce[dt] = mma2x(ce[dt], a0, a1, blT[J0], blT[J1]);
            }
            // Terms of dk: row blocks I >= R.
            if (J1 >= R) {
                const float f0 = (J0 == R && wave_slow) ? 0.f : pair_factor(sT, J0, R, c);
                const float f1 = (J1 == R && wave_slow) ? 0.f : pair_factor(sT, J1, R, c);
                ck[dt] = mma2x(ck[dt], scaled(sQT, J0, dt, f0), scaled(sQT, J1, dt, f1), baN[J0], baN[J1]);
                ck[dt] = mma2x(ck[dt], scaled(sET, J0, dt, f0), scaled(sET, J1, dt, f1), blN[J0], blN[J1]);
            }
        }
    }

    // Row data: dq = 2^G cq, de = 2^G ce, dk = 2^(T_R - G) ck, the exact
    // diagonal terms of wide blocks, dG, and its per-block column sums.
    float pq = 0.f, pk = 0.f;  // row sums for the L2-norm chain rule
#pragma unroll
    for (int dt = 0; dt < NKT; ++dt) {
        float qv[4], kv[4], bv[4], gv[4];
        row_tile(dt, qv, kv, bv, gv);
        const float4 tr = *reinterpret_cast<const float4 *>(&sT[R][16 * dt + 4 * kg]);
        const float trv[4] = {tr.x, tr.y, tr.z, tr.w};
        float qn[4], kn[4], en[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            qn[i] = qv[i] * qmul;
            kn[i] = kv[i] * invk;
            en[i] = bv[i] * kn[i];
            cq[dt][i] *= fexp2(gv[i]);
            ce[dt][i] *= fexp2(gv[i]);
            ck[dt][i] *= fexp2(trv[i] - gv[i]);
        }
        if (wave_slow) {
            // Diagonal block summed pair by pair: row m with rows j of this block.
#pragma unroll
            for (int j = 0; j < 16; ++j) {
                const float a = __shfl(dAd[j & 3], m + 16 * (j >> 2), 64);
                const float lv = __shfl(dLd[j & 3], m + 16 * (j >> 2), 64);
                const float aN2 = __shfl(dANd[j & 3], m + 16 * (j >> 2), 64);
                const float lN2 = __shfl(dLNd[j & 3], m + 16 * (j >> 2), 64);
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int src = 16 * kg + j;
                    const float kj = __shfl(kn[i], src, 64), qj = __shfl(qn[i], src, 64);
                    const float ej = __shfl(en[i], src, 64), Gj = __shfl(gv[i], src, 64);
                    const float lo = (j <= m) ? fexp2(gv[i] - Gj) : 0.f;  // row m, column j
                    const float hi = (j >= m) ? fexp2(Gj - gv[i]) : 0.f;  // row j, column m
                    cq[dt][i] = fmaf(a * kj, lo, cq[dt][i]);
                    ce[dt][i] = fmaf(lv * kj, lo, ce[dt][i]);
                    ck[dt][i] = fmaf(aN2 * qj + lN2 * ej, hi, ck[dt][i]);
                }
            }
        }
        float dG[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            dG[i] = qn[i] * cq[dt][i] + en[i] * ce[dt][i] - kn[i] * ck[dt][i];
            // db = de * k; dk += de * b; dq <- scale * dq (w.r.t. the normalised q).
            const float dbv = ce[dt][i] * kn[i];
            ck[dt][i] = fmaf(ce[dt][i], bv[i], ck[dt][i]);
            ce[dt][i] = dbv;
            cq[dt][i] *= p.scale;
            pq = fmaf(qv[i] * invq, cq[dt][i], pq);
            pk = fmaf(kn[i], ck[dt][i], pk);
            // In-block suffix sums of dG (reverse cumsum), block total to LDS.
            const float pre = row16_scan(dG[i]);
            const float tot = __shfl(pre, 16 * kg + 15, 64);
            dG[i] = tot - pre + dG[i];
            if (m == 0) sDG[R][16 * dt + 4 * kg + i] = tot;
        }
        if (row_ok) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int c = 16 * dt + 4 * kg + i;
                if (c < K) io<TI>::st(static_cast<TI *>(p.db), roff + c, ce[dt][i]);
            }
        }
        // ce now carries the in-block suffix sums of dG for the second pass.
        ce[dt][0] = dG[0];
        ce[dt][1] = dG[1];
        ce[dt][2] = dG[2];
        ce[dt][3] = dG[3];
    }
    __syncthreads();
    pq += __shfl_xor(pq, 16, 64);
    pq += __shfl_xor(pq, 32, 64);
    pk += __shfl_xor(pk, 16, 64);
    pk += __shfl_xor(pk, 32, 64);
#pragma unroll
    for (int dt = 0; dt < NKT; ++dt) {
        float qv[4], kv[4];
        const int c0 = 16 * dt + 4 * kg;
        load4<TI>(q, roff, c0, K, row_ok, p.vec_ok, qv);
        load4<TI>(k, roff, c0, K, row_ok, p.vec_ok, kv);
        if (!row_ok) continue;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int c = c0 + i;
            if (c >= K) continue;
            float later = sLast[c] + sKK[0][c] + sKK[1][c] + sKK[2][c] + sKK[3][c];
#pragma unroll
            for (int R2 = 1; R2 < 4; ++R2)
                if (R2 > R) later += sDG[R2][c];
            io<TG>::st(static_cast<TG *>(p.dg), roff + c, ce[dt][i] + later);
            float dq = cq[dt][i], dk = ck[dt][i];
            if (l2) {
                // d/dx of x / max(||x||, eps): (dy - y (y . dy)) / ||x|| above eps, dy / eps below.
                dq = bigq ? (dq - qv[i] * invq * pq) * invq : dq * invq;
                dk = bigk ? (dk - kv[i] * invk * pk) * invk : dk * invk;
            }
            io<TI>::st(static_cast<TI *>(p.dq), roff + c, dq);
            io<TI>::st(static_cast<TI *>(p.dk), roff + c, dk);
        }
    }
}

template <PrecKind PK, int KP, typename TI, typename TG>
hipError_t launch_bwd(const BwdParams &p, int total_chunks, hipStream_t stream)
{
    if (p.num_seqs == 0) return hipSuccess;
    const int NP = p.num_seqs * p.H;
    const int groups = (NP + 7) / 8;
    constexpr int BV = 64;
    const int NVB = (p.V + BV - 1) / BV;
    hipLaunchKernelGGL((chunk_bwd_scan_kernel<PK, KP, BV, TI>), dim3(groups * 8 * NVB), dim3(512), 0,
                       stream, p, NVB, NP);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || total_chunks == 0) return e;
    hipLaunchKernelGGL((chunk_bwd_kside_kernel<PK, KP, TI, TG>), dim3(total_chunks, p.H), dim3(256), 0,
                       stream, p);
    return hipGetLastError();
}

template <PrecKind PK, typename TI, typename TG>
hipError_t launch_bwd_kp(const BwdParams &p, int total_chunks, hipStream_t stream)
{
    switch (kp_for(p.K)) {
    case 32: return launch_bwd<PK, 32, TI, TG>(p, total_chunks, stream);
    case 64: return launch_bwd<PK, 64, TI, TG>(p, total_chunks, stream);
    default: return launch_bwd<PK, 128, TI, TG>(p, total_chunks, stream);
    }
}

}  // namespace

size_t chunk_bwd_workspace_bytes(int B, int T, int H, int K, int V, int io_dtype,
                                 const int64_t *cu_host, int num_seqs)
{
    if (K > 128) return 0;
    const int64_t nc = count_chunks(B, T, cu_host, num_seqs);
    return static_cast<size_t>(bwd_layout(nc, H, K, V, io_dtype).total);
}

size_t chunk_train_workspace_bytes(int B, int T, int H, int K, int V, int io_dtype,
                                   const int64_t *cu_host, int num_seqs)
{
    if (K > 128) return 0;
    const int64_t nc = count_chunks(B, T, cu_host, num_seqs);
    return static_cast<size_t>(train_layout(nc, H, K, V, io_dtype).total);
}

int launch_chunk_bwd(const ChunkBwdArgs &a, int io_dtype, int g_dtype, hipStream_t stream)
{
    if (a.K > 128) return GDN2_ERR_UNSUPPORTED;
    if (g_dtype != GDN2_DTYPE_F32 && g_dtype != io_dtype) return GDN2_ERR_UNSUPPORTED;
    const int64_t nc = count_chunks(a.B, a.T, a.cu_host, a.num_seqs);
    if (nc * a.H > 2147483647LL / 2) return GDN2_ERR_UNSUPPORTED;
    const TrainLayout tl = train_layout(nc, a.H, a.K, a.V, io_dtype);
    const BwdLayout bl = bwd_layout(nc, a.H, a.K, a.V, io_dtype);
    if (nc > 0 && (!a.saved || a.saved_bytes < static_cast<size_t>(tl.total))) return GDN2_ERR_WORKSPACE;
    if (nc > 0 && (!a.workspace || a.workspace_bytes < static_cast<size_t>(bl.total))) return GDN2_ERR_WORKSPACE;

    BwdParams p;
    p.q = a.q; p.k = a.k; p.v = a.v; p.g = a.g; p.b = a.b; p.w = a.w; p.dout = a.dout;
    p.dht = a.dht;
    p.dq = a.dq; p.dk = a.dk; p.dv = a.dv; p.dg = a.dg; p.db = a.db; p.dw = a.dw;
    p.dh0 = a.dh0;
    p.cu_seqlens = a.cu_seqlens;
    p.num_seqs = a.num_seqs;
    p.T = a.T; p.H = a.H; p.K = a.K; p.V = a.V;
    p.VP = static_cast<int>(round_up(a.V, 16));
    p.nt = (a.T + kChunk - 1) / kChunk;
    p.scale = a.scale;
    p.flags = a.flags;
    p.vec_ok = (a.K % 4) == 0;
    const unsigned char *sv = static_cast<const unsigned char *>(a.saved);
    unsigned char *wk = static_cast<unsigned char *>(a.workspace);
    p.blob = sv;
    p.hs = sv ? sv + tl.hs : nullptr;
    p.us = sv ? sv + tl.us : nullptr;
    p.dhs = wk ? wk + bl.dhs : nullptr;
    p.dys = wk ? wk + bl.dys : nullptr;
    const int total = static_cast<int>(nc);

    hipError_t e;
    switch (io_dtype) {
    case GDN2_DTYPE_F32:
        e = launch_bwd_kp<PrecKind::F32, float, float>(p, total, stream);
        break;
    case GDN2_DTYPE_BF16:
        e = g_dtype == GDN2_DTYPE_F32 ? launch_bwd_kp<PrecKind::BF16, bf16_t, float>(p, total, stream)
                                      : launch_bwd_kp<PrecKind::BF16, bf16_t, bf16_t>(p, total, stream);
        break;
    default:
        e = g_dtype == GDN2_DTYPE_F32 ? launch_bwd_kp<PrecKind::BF16, f16_t, float>(p, total, stream)
                                      : launch_bwd_kp<PrecKind::BF16, f16_t, f16_t>(p, total, stream);
        break;
    }
    return e == hipSuccess ? GDN2_OK : GDN2_ERR_LAUNCH;
}

}  // namespace gdn2
