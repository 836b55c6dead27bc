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
//    dh0 and, per chunk, dS1 and dY for the second kernel.
//  * chunk_bwd_kside_kernel -- a persistent grid of 8-wave workgroups (two
//    waves per 16-token block), one (chunk, head) item at a time, all chunks
//    in parallel: dv, dw from dY, the
//    V-contractions above on MFMA over LDS-staged value slices, the in-chunk
//    pair terms with the forward's factored decays (exact VALU sums on
//    diagonal blocks whose decay span is too wide), the reverse cumsum, and
//    the chain rule to dq, dk, db, dg.

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

// LDS layout of the backward scan's transposed blob.  Block b of 256 elements
// (blob offset 256 b) starts at PB * b; with 16-bit storage each 16-lane group
// of a block is followed by 4 elements of padding (PB = 272), so that the 64
// lanes of one landing store (below) reach 64 distinct banks instead of 8.
// Lane l's 4 values of a block are at lane(l).
template <PrecKind PK>
struct TLay {
    static constexpr int GP = sizeof(typename Prec<PK>::st) == 2 ? 4 : 0;  // padding per 16-lane group
    static constexpr int PB = 256 + 4 * GP;
    static __device__ __forceinline__ constexpr int64_t blk(int64_t off) { return (off >> 8) * PB; }
    static __device__ __forceinline__ int lane(int l) { return 4 * l + GP * (l >> 4); }
    template <int KP>
    static constexpr int64_t size()
    {
        return blk(Blob<PK, KP>::GL) + (Blob<PK, KP>::SIZE - Blob<PK, KP>::GL);
    }
};

// Unit j*256 + ct (ct < 256 the copy thread) of a forward blob, 16 bytes,
// landed in LDS with each matrix region transposed: element M[a][b] of a K16
// fragment-native [Mr][Kc] region goes to element M^T[b][a] of the
// fragment-native [Kc][Mr] region at the same base, in the TLay layout; the
// exp(G_last) vector is copied as is.  Every region boundary is a multiple of
// 256 units' worth of elements, so the region of unit group j is a
// compile-time constant once the caller's loop over j is unrolled.
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
        *reinterpret_cast<u32x4 *>(dst + TLay<PK>::blk(BL::GL) + (e - BL::GL)) = val;
        return;
    }
    const int loc = e - base, blk = loc >> 8, wi = loc & 255;
    const int nkc = Kc >> 4, nm = Mr >> 4;
    const int mt = blk / nkc, kt = blk - mt * nkc;
    const int L0 = wi >> 2, a0 = L0 & 15, b0 = (L0 >> 4) * 4;
    // Transposed lane b0 + c + 16 (a0 >> 2), slot a0 & 3.
    st *d = dst + TLay<PK>::blk(base + ((kt * nm + mt) << 8)) + 4 * b0 + (64 + TLay<PK>::GP) * (a0 >> 2) + (a0 & 3);
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
    constexpr bool DB = PK != PrecKind::F32 && KP <= 128;  // double-buffered blobs where two fit
    constexpr int NBUF = DB ? 2 : 1;
    constexpr int NKT = KP / 16, NKS = KP / 32, NCT = BV / 16;
    constexpr int U16 = static_cast<int>(BL::BYTES / 16);
    constexpr int PF = (U16 + 255) / 256;
    using TL = TLay<PK>;
    __shared__ __align__(16) st sB[NBUF][TL::template size<KP>()];
    // dO of the chunk, row-major [token][column of the slice] with a 16-byte
    // skew per row; the compute waves turn each 16-token tile into their K16
    // B operand with one identity product.
    constexpr int LDD = BV + 16 / static_cast<int>(sizeof(st));
    __shared__ __align__(16) st sD[NBUF][64 * LDD];

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

    const TI *dop = static_cast<const TI *>(p.dout);
    const st *wsb = static_cast<const st *>(p.blob);
    auto blob = [&](int gci) {
        return reinterpret_cast<const u32x4 *>(wsb + (static_cast<int64_t>(gci) * H + h) * BL::SIZE);
    };
    auto chunk_rows = [&](int jc, int64_t &t0, int &lc) __attribute__((always_inline)) {
        t0 = bos + static_cast<int64_t>(jc) * kChunk;
        const int64_t rem = len - static_cast<int64_t>(jc) * kChunk;
        lc = rem < kChunk ? static_cast<int>(rem) : kChunk;
    };

    // Copy waves: dO rows of chunk jc for this value slice, row-major in LDS
    // (zero past the sequence end and past V), one 16-byte LDS store per row
    // piece.
    const int v0 = vs * BV;
    constexpr int EPV = 16 / static_cast<int>(sizeof(TI));
    constexpr int ZT = kChunk * BV / EPV;
    constexpr int NZT = (ZT + 255) / 256;
    // Whole 16-byte row pieces for every row of this slice (uniform per workgroup).
    const bool dfast = (V % EPV) == 0 && v0 + BV <= V;
    struct DRaw {
        u32x4 d[NZT];
    };
    // issue_d requests the raw rows, land_d scatters them into LDS, so the two
    // can sit a chunk apart.  On the fast path dead lanes load the chunk's
    // first row piece (always valid) and are zeroed when landed, and land_d
    // touches no global memory: a select on a loaded value, or a load in
    // land_d, would make the request wait for its own data.  Ragged slices
    // load element by element in land_d.
    auto issue_d = [&](auto fastc, DRaw &r, int jc) __attribute__((always_inline)) {
        if constexpr (decltype(fastc)::value) {
            int64_t t0;
            int lc;
            chunk_rows(jc, t0, lc);
#pragma unroll
            for (int a = 0; a < NZT; ++a) {
                const int task = ctid + 256 * a;
                const int tok = task / (BV / EPV), c = EPV * (task % (BV / EPV));
                const bool live = task < ZT && tok < lc;
                const int64_t off = live ? ((t0 + tok) * H + h) * V + v0 + c : (t0 * H + h) * V + v0;
                r.d[a] = *reinterpret_cast<const u32x4 *>(dop + off);
            }
        }
    };
    auto land_d = [&](auto fastc, const DRaw &r, int jc, int buf) __attribute__((always_inline)) {
        int64_t t0;
        int lc;
        chunk_rows(jc, t0, lc);
        st *dst = sD[buf];
        static_assert(EPV * sizeof(st) == 16, "one dO row piece is one 16-byte LDS store");
#pragma unroll
        for (int a = 0; a < NZT; ++a) {
            const int task = ctid + 256 * a;
            if (task >= ZT) continue;
            const int tok = task / (BV / EPV), c = EPV * (task % (BV / EPV));
            const TI *rd = reinterpret_cast<const TI *>(&r.d[a]);
            st zr[EPV];
#pragma unroll
            for (int e = 0; e < EPV; ++e) {
                float x = 0.f;
                if constexpr (decltype(fastc)::value) {
                    x = tok < lc ? io<TI>::ld(rd, e) : 0.f;
                } else {
                    if (tok < lc && v0 + c + e < V) x = io<TI>::ld(dop, ((t0 + tok) * H + h) * V + v0 + c + e);
                }
                zr[e] = P::from_f32(x);
            }
            *reinterpret_cast<u32x4 *>(dst + tok * LDD + c) = __builtin_bit_cast(u32x4, zr);
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
                if (row < K) dS[kt][i] = p.dht[state_index(p.flags, n, h, row, col, H, K, V)];
            }
        }
    }

    // Step s handles chunk nch-1-s.  Barrier schedule as in the forward scan.
    if (copier) {
        // Instantiated for whole-row and for ragged dO slices (uniform per
        // workgroup), so that each loop body is straight-line.
        auto copy_loop = [&](auto fastc) __attribute__((always_inline)) {
            DRaw dA, dB;
            if (nch > 0) {
                land_all(blob(gc0 + nch - 1));
                issue_d(fastc, dA, nch - 1);
                land_d(fastc, dA, nch - 1, 0);
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
                // Step s lands chunk nch-2-s, requested two steps earlier, and
                // reuses its register set for chunk nch-4-s, so every request
                // has two chunk steps of memory latency to hide.  Unrolled by
                // two so that the register sets A / B swap roles at compile time.
                if (nch > 1) {
                    issue(pA, gc0 + nch - 2);
                    issue_d(fastc, dA, nch - 2);
                }
                if (nch > 2) {
                    issue(pB, gc0 + nch - 3);
                    issue_d(fastc, dB, nch - 3);
                }
                __syncthreads();
                for (int s = 0; s < nch; s += 2) {
                    if (s + 1 < nch) {
                        land_d(fastc, dA, nch - 2 - s, 1);
                        land(pA, 1);
                    }
                    if (s + 3 < nch) {
                        issue(pA, gc0 + nch - 4 - s);
                        issue_d(fastc, dA, nch - 4 - s);
                    }
                    __syncthreads();
                    if (s + 1 >= nch) break;
                    if (s + 2 < nch) {
                        land_d(fastc, dB, nch - 3 - s, 0);
                        land(pB, 0);
                    }
                    if (s + 4 < nch) {
                        issue(pB, gc0 + nch - 5 - s);
                        issue_d(fastc, dB, nch - 5 - s);
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
                        issue_d(fastc, dA, jn);
                        land_d(fastc, dA, jn, 0);
                        __syncthreads();
                    }
                }
            }
        };
        if (dfast)
            copy_loop(std::true_type{});
        else
            copy_loop(std::false_type{});
    } else {
        const Q ident = identity_q4<PK>(l);
        const int ll = TL::lane(l);  // this lane's 4 values in a transposed block
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

                // dO read row-major (lane (m, kg): token 16kt+m, columns 4kg..4kg+3
                // of this wave's 16) and transposed by the identity product.
                Q df[4];
#pragma unroll
                for (int kt = 0; kt < 4; ++kt)
                    df[kt] = pack4<PK>(mma1<PK>(zero4(), ld_q4<PK>(sD[buf] + (16 * kt + m) * LDD + 16 * wv + 4 * kg),
                                                ident));
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
                            acc = mma2<PK>(acc, ld_q4<PK>(Bk + TL::blk(BL::AQ + k16_block(rt, 2 * s2, 64)) + ll),
                                           ld_q4<PK>(Bk + TL::blk(BL::AQ + k16_block(rt, 2 * s2 + 1, 64)) + ll),
                                           df[2 * s2], df[2 * s2 + 1]);
#pragma unroll
                    for (int s2 = 0; s2 < NKS; ++s2)
                        acc = mma2<PK>(acc, ld_q4<PK>(Bk + TL::blk(BL::KT + k16_block(rt, 2 * s2, KP)) + ll),
                                       ld_q4<PK>(Bk + TL::blk(BL::KT + k16_block(rt, 2 * s2 + 1, KP)) + ll),
                                       sf[2 * s2], sf[2 * s2 + 1]);
                    duf[rt] = pack4<PK>(acc);
                }
                // dY = X^T dU (dv = dY * w and dw = dY * v are formed by the K-side kernel).
                st *dyb = static_cast<st *>(p.dys) + cb * (64 * VP);
#pragma unroll
                for (int rt = 0; rt < 4; ++rt) {
                    f32x4 acc = zero4();
#pragma unroll
                    for (int s2 = 0; s2 < 2; ++s2)
                        if (2 * s2 + 1 >= rt)
                            acc = mma2<PK>(acc, ld_q4<PK>(Bk + TL::blk(BL::X + k16_block(rt, 2 * s2, 64)) + ll),
                                           ld_q4<PK>(Bk + TL::blk(BL::X + k16_block(rt, 2 * s2 + 1, 64)) + ll),
                                           duf[2 * s2], duf[2 * s2 + 1]);
                    if (emit)
                        st_q4<PK>(dyb + k16_block(rt, vt, VP) + 4 * l,
                                  pack4<PK>(mma1<PK>(zero4(), pack4<PK>(acc), ident)));
                }
                // dS0 = Diag(exp(G_last)) dS1 + Qbar^T dO + (-W)^T dU.
                const float *gl = reinterpret_cast<const float *>(Bk + TL::blk(BL::GL));
#pragma unroll
                for (int kt = 0; kt < NKT; ++kt) {
                    const float4 gv = *reinterpret_cast<const float4 *>(gl + 16 * kt + 4 * kg);
                    dS[kt][0] *= gv.x;
                    dS[kt][1] *= gv.y;
                    dS[kt][2] *= gv.z;
                    dS[kt][3] *= gv.w;
#pragma unroll
                    for (int s2 = 0; s2 < 2; ++s2) {
                        dS[kt] = mma2<PK>(dS[kt], ld_q4<PK>(Bk + TL::blk(BL::QB + k16_block(kt, 2 * s2, 64)) + ll),
                                          ld_q4<PK>(Bk + TL::blk(BL::QB + k16_block(kt, 2 * s2 + 1, 64)) + ll),
                                          df[2 * s2], df[2 * s2 + 1]);
                        dS[kt] = mma2<PK>(dS[kt], ld_q4<PK>(Bk + TL::blk(BL::WN + k16_block(kt, 2 * s2, 64)) + ll),
                                          ld_q4<PK>(Bk + TL::blk(BL::WN + k16_block(kt, 2 * s2 + 1, 64)) + ll),
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
                if (row < K) p.dh0[state_index(p.flags, n, h, row, col, H, K, V)] = dS[kt][i];
            }
    }
}


// Four input values kept in their input format (16-bit inputs: two packed
// registers instead of four), widened to fp32 on use.
template <typename T>
struct Raw4 {
    uint2 u;
    __device__ __forceinline__ void load(const T *p) { u = *reinterpret_cast<const uint2 *>(p); }
    __device__ __forceinline__ void zero() { u = make_uint2(0u, 0u); }
    __device__ __forceinline__ void set(const float (&x)[4])
    {
        u.x = raw16(x[0]) | (raw16(x[1]) << 16);
        u.y = raw16(x[2]) | (raw16(x[3]) << 16);
    }
    __device__ __forceinline__ float operator[](int i) const
    {
        const uint32_t w = (i < 2 ? u.x : u.y) >> (16 * (i & 1));
        return wide16(w & 0xffffu);
    }
    static __device__ __forceinline__ uint32_t raw16(float x)
    {
        if constexpr (std::is_same<T, bf16_t>::value)
            return f32_to_bf16_bits(x);
        else
            return __builtin_bit_cast(uint16_t, static_cast<_Float16>(x));
    }
    static __device__ __forceinline__ float wide16(uint32_t b)
    {
        if constexpr (std::is_same<T, bf16_t>::value)
            return bf16_bits_to_f32(static_cast<uint16_t>(b));
        else
            return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(b)));
    }
};
template <>
struct Raw4<float> {
    float4 f;
    __device__ __forceinline__ void load(const float *p) { f = *reinterpret_cast<const float4 *>(p); }
    __device__ __forceinline__ void zero() { f = make_float4(0.f, 0.f, 0.f, 0.f); }
    __device__ __forceinline__ void set(const float (&x)[4]) { f = make_float4(x[0], x[1], x[2], x[3]); }
    __device__ __forceinline__ float operator[](int i) const
    {
        return i == 0 ? f.x : (i == 1 ? f.y : (i == 2 ? f.z : f.w));
    }
};

// ---------------------------------------------------------------------------
// K-side gradients: a persistent grid of workgroups of 8 waves, each walking
// (chunk, head) items blockIdx.x, blockIdx.x + gridDim.x, ...  Wave
// w = 2R + hh owns token rows 16R..16R+15 (lane (m, kg): row 16R+m) and the
// channel tiles hh*NKH .. hh*NKH+NKH-1 (channels 16dt + 4kg + i, "A-order",
// as in the forward prep kernel).  Both waves of a token block compute the
// block's in-chunk pair tiles (dA, dL over the value dimension), so no wave
// waits on another for them.
// ---------------------------------------------------------------------------
template <PrecKind PK, int KP, typename TI, typename TG>
__global__ __launch_bounds__(512) void chunk_bwd_kside_kernel(BwdParams p, int items)
{
    using P = Prec<PK>;
    using st = typename P::st;
    using Q = Q4<PK>;
    constexpr int NKT = KP / 16;
    constexpr int NKH = NKT / 2;  // channel tiles per wave
    // dg is a reverse cumulative sum in which the in-chunk pair terms cancel
    // in exact arithmetic; to keep that cancellation accurate, the factor
    // tiles of the pair products carry fp32 precision: for 16-bit MFMA
    // operands as two planes, x = hi + lo.
    // At KP = 256 one plane and one value tile per slice: two planes of the three
    // factor tiles alone would take 192 KB of LDS.
    constexpr int NPL = PK == PrecKind::F32 || KP > 128 ? 1 : 2;
    constexpr int NVS = PK == PrecKind::F32 || KP > 128 ? 1 : 2;  // value tiles per staged slice
    constexpr int NLT = (NKT + 7) / 8;  // channel tiles per wave for the G_last rowsum
    constexpr int EPU = 16 / static_cast<int>(sizeof(st));
    constexpr int BLK = 256;
    // Transposed (B-order) factor tiles of every token block, for the pair products.
    __shared__ __align__(16) st sKT[NPL][4][NKT][BLK];  // k * 2^(T_R - G)   (kend)
    __shared__ __align__(16) st sQT[NPL][4][NKT][BLK];  // q * 2^G           (qb)
    __shared__ __align__(16) st sET[NPL][4][NKT][BLK];  // e * 2^G           (eb)
    // One staged value slice (NVS value tiles), A-order blocks.
    constexpr int NB_U = 4 * NVS, NB_Y = 4 * NVS, NB_H = NKT * NVS, NB_D = NKT * NVS;
    constexpr int NB = NB_U + NB_Y + NB_H + NB_D;  // contiguous workspace blocks per slice
    __shared__ __align__(16) st sW[NB * BLK];      // U, dY, h, dh
    __shared__ __align__(16) st sO[4 * NVS * BLK];  // dO
    __shared__ __align__(16) float sT[4][KP];       // in-block decay totals (log2)
    __shared__ __align__(16) float sEr[4][KP];      // 2^(decay before block)
    __shared__ __align__(16) float sEa[4][KP];      // 2^(decay after block)
    __shared__ __align__(16) float sE2[4][KP];      // 2^(T_J): decay across block J
    __shared__ __align__(16) float sE2n[4][KP];     // 2^(-T_J)
    __shared__ __align__(16) float sDG[4][KP];      // per-block sums of dG
    __shared__ __align__(16) float sKK[4][KP];      // per-block sums of dKt * Kt
    __shared__ __align__(16) float sLast[KP];       // exp(G_last) rowsum(dS1 * S0)
    __shared__ float sRow[2][2][64];                // per-half row sums (norms, then L2 dots)
    __shared__ int sWide[4][2];

    const int tid0 = threadIdx.x, wv0 = __builtin_amdgcn_readfirstlane(tid0 >> 6);
    const int H = p.H, K = p.K, V = p.V, VP = p.VP;

    // Rows of an item by direct LDS loads into the factor tiles (16-bit inputs
    // with two factor planes, K == KP): an item's q, k, b, g rows are requested
    // once the previous item's pair products are done, so that it starts on
    // rows already in LDS.  Tensor regions: q -> sKT plane 0, k -> sKT plane 1,
    // b -> sQT plane 0, g -> sET; wave w's part of a region starts at w times its
    // size.  Lane (m, kg) uses row 16R + m, channels 16 (hh NKH + j) + 4 kg + i.
    //  * 16-bit rows: 16-byte piece p = 32 j + 16 h + m holds channels
    //    16 (hh NKH + j) + 8 h .. + 7 of row m at byte 16 p, so lane (m, kg)
    //    reads tile j at 16 (32 j + 16 (kg / 2) + m) + 8 (kg % 2): one 512-byte
    //    run per tile, no bank conflicts.
    //  * fp32 rows: piece 64 j + l (lane l = 16 kg + m) is exactly lane l's tile j.
    // Each request covers 64 consecutive pieces, fetched by 64 lanes from 16
    // rows (64 contiguous bytes of each row).
    constexpr bool PFR = NPL == 2 && sizeof(TI) == 2;
    auto rows_lds = [&](int tensor) __attribute__((always_inline)) {
        return tensor == 0 ? reinterpret_cast<unsigned char *>(&sKT[0][0][0][0])
             : tensor == 1 ? reinterpret_cast<unsigned char *>(&sKT[1][0][0][0])
             : tensor == 2 ? reinterpret_cast<unsigned char *>(&sQT[0][0][0][0])
                           : reinterpret_cast<unsigned char *>(&sET[0][0][0][0]);
    };
    static_assert(!PFR || (8 * NKH * 512 <= static_cast<int>(sizeof(sKT[0])) &&
                           8 * NKH * 256 * static_cast<int>(sizeof(TG)) <= static_cast<int>(sizeof(sET))),
                  "prefetched rows must fit the factor tiles");
    auto dma_rows = [&](int itm, int wvx, int lx) __attribute__((always_inline)) {
        const int gcn = itm / H, hn = itm - gcn * H;
        int nn, jcn;
        int64_t bosn, lenn;
        locate_chunk(p, gcn, nn, jcn, bosn, lenn);
        const int64_t t0n = bosn + static_cast<int64_t>(jcn) * kChunk;
        const int64_t remn = lenn - static_cast<int64_t>(jcn) * kChunk;
        const int lcn = remn < kChunk ? static_cast<int>(remn) : kChunk;
        const int rowi = 16 * (wvx >> 1) + (lx & 15);
        // Rows past the chunk end read its first row (in bounds); they are
        // zeroed where they are used.
        const int64_t row0 = ((t0n + (rowi < lcn ? rowi : 0)) * H + hn) * static_cast<int64_t>(K) +
                             16 * (wvx & 1) * NKH;
        auto go16 = [&](const TI *base, int tensor) __attribute__((always_inline)) {
            unsigned char *dst = rows_lds(tensor) + wvx * (NKH * 512);
#pragma unroll
            for (int t = 0; t < (32 * NKH + 63) / 64; ++t) {
                const int pc = 64 * t + lx;  // piece
                if (pc < 32 * NKH) {
                    const int j = pc >> 5, h = (pc >> 4) & 1;
                    __builtin_amdgcn_global_load_lds(reinterpret_cast<const char *>(base + row0 + 16 * j + 8 * h),
                                                     dst + 1024 * t, 16, 0, 0);
                }
            }
        };
        go16(static_cast<const TI *>(p.q), 0);
        go16(static_cast<const TI *>(p.k), 1);
        go16(static_cast<const TI *>(p.b), 2);
        if constexpr (sizeof(TG) == 4) {
            const TG *gb = static_cast<const TG *>(p.g);
            unsigned char *dst = rows_lds(3) + wvx * (NKH * 1024);
#pragma unroll
            for (int j = 0; j < NKH; ++j)
                __builtin_amdgcn_global_load_lds(reinterpret_cast<const char *>(gb + row0 + 16 * j + 4 * (lx >> 4)),
                                                 dst + 1024 * j, 16, 0, 0);
        } else {
            go16(reinterpret_cast<const TI *>(p.g), 3);
        }
    };
    if (PFR && K == KP && static_cast<int>(blockIdx.x) < items) dma_rows(blockIdx.x, wv0, tid0 & 63);

    for (int item = blockIdx.x; item < items; item += gridDim.x) {
    // The thread and wave indices are made opaque per item so that the
    // compiler does not hoist the many per-lane LDS and global addresses out of
    // the item loop, where they would hold registers through every phase.
    int tid = tid0, wv = wv0;
    asm volatile("" : "+v"(tid));
    asm volatile("" : "+s"(wv));
    const int R = wv >> 1, hh = wv & 1;
    const int l = tid & 63, m = l & 15, kg = l >> 4;
    const int gc = item / H, h = item - (item / H) * H;
    // The rows' direct LDS loads (and, with them, the previous item's
    // gradient stores) are complete before anything of this item, on every
    // path, so that no later barrier has to wait for them.
    if constexpr (PFR) __builtin_amdgcn_s_waitcnt(0);

    int n, jc;
    int64_t bos, len;
    locate_chunk(p, gc, n, jc, bos, len);
    const int64_t t0 = bos + static_cast<int64_t>(jc) * kChunk;
    const int64_t rem = len - static_cast<int64_t>(jc) * kChunk;
    const int lc = rem < kChunk ? static_cast<int>(rem) : kChunk;
    const int r = 16 * R + m;
    const bool row_ok = r < lc;
    const int64_t roff = ((t0 + r) * H + h) * K;
    const int64_t cb = static_cast<int64_t>(gc) * H + h;
    const bool l2 = (p.flags & GDN2_FLAG_L2NORM_QK) != 0;
    const Q ident = identity_q4<PK>(l);

    const st *hsb = static_cast<const st *>(p.hs) + cb * (KP * VP);
    const st *dhb = static_cast<const st *>(p.dhs) + cb * (KP * VP);
    const st *usb = static_cast<const st *>(p.us) + cb * (64 * VP);
    const st *dyb = static_cast<const st *>(p.dys) + cb * (64 * VP);
    const TI *dop = static_cast<const TI *>(p.dout);
    const TI *vp = static_cast<const TI *>(p.v);
    const TI *wp = static_cast<const TI *>(p.w);
    TI *dvp = static_cast<TI *>(p.dv);
    TI *dwp = static_cast<TI *>(p.dw);
    const int NVT = VP / 16;

    // ---- slice staging: workspace blocks as 16-byte units, dO rows as groups of 4 ----
    constexpr int UPB = BLK / EPU;                  // units per block
    constexpr int NUW = NB * UPB;                    // workspace units per slice
    constexpr int NUO = 64 * 4 * NVS;                // dO groups of 4 values per slice
    constexpr int NPRE_W = (NUW + 511) / 512, NPRE_O = (NUO + 511) / 512;
    // Source of workspace unit u of slice vt0 (nullptr past V).
    auto wsrc = [=](int u, int vt0) __attribute__((always_inline)) -> const st * {
        // Selects, not branches or a table: this runs per lane while the
        // slice's requests are being issued.
        const int b = u / UPB, e = (u % UPB) * EPU;
        const bool inU = b < NB_U, inY = b < NB_U + NB_Y, inH = b < NB_U + NB_Y + NB_H;
        const int rb = b - (inU ? 0 : (inY ? NB_U : (inH ? NB_U + NB_Y : NB_U + NB_Y + NB_H)));
        const st *base = inU ? usb : (inY ? dyb : (inH ? hsb : dhb));
        const int rowt = rb / NVS, vl = rb % NVS;
        if (vt0 + vl >= NVT) return nullptr;
        return base + k16_block(rowt, vt0 + vl, VP) + e;
    };
    // Requests never wait on their own data: invalid units and groups read a
    // valid address and are zeroed when landed (validity bits in wok / ook).
    struct Pre {
        u32x4 w[NPRE_W];
        Raw4<TI> o[NPRE_O], v[NPRE_O], w2[NPRE_O];  // dO, and v, w of the same groups for dv and dw
        uint32_t wok, ook;
    };
    auto issue_slice = [&](Pre &pr, int vt0) __attribute__((always_inline)) {
        pr.wok = pr.ook = 0u;
#pragma unroll
        for (int a = 0; a < NPRE_W; ++a) {
            const int u = tid + 512 * a;
            const st *src = u < NUW ? wsrc(u, vt0) : nullptr;
            pr.wok |= (src != nullptr ? 1u : 0u) << a;
            pr.w[a] = *reinterpret_cast<const u32x4 *>(src != nullptr ? src : usb);
        }
#pragma unroll
        for (int a = 0; a < NPRE_O; ++a) {
            const int u = tid + 512 * a;
            const int tok = u / (4 * NVS), c = 16 * vt0 + 4 * (u % (4 * NVS));
            const bool ok = u < NUO && tok < lc && c < V;
            pr.ook |= (ok ? 1u : 0u) << a;
            if ((V % 4) == 0) {
                // Whole groups of 4 (c < V implies c + 4 <= V): row 0 of the
                // chunk, column 0, for invalid groups.
                const int64_t off = ((t0 + (ok ? tok : 0)) * H + h) * static_cast<int64_t>(V) + (ok ? c : 0);
                pr.o[a].load(dop + off);
                pr.v[a].load(vp + off);
                pr.w2[a].load(wp + off);
            } else {
                const int64_t off = ((t0 + tok) * H + h) * static_cast<int64_t>(V);
                float xo[4], xv[4], xw[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const bool oki = ok && c + i < V;
                    xo[i] = oki ? io<TI>::ld(dop, off + c + i) : 0.f;
                    xv[i] = oki ? io<TI>::ld(vp, off + c + i) : 0.f;
                    xw[i] = oki ? io<TI>::ld(wp, off + c + i) : 0.f;
                }
                pr.o[a].set(xo);
                pr.v[a].set(xv);
                pr.w2[a].set(xw);
            }
        }
    };
    auto land_slice = [&](const Pre &pr) __attribute__((always_inline)) {
#pragma unroll
        for (int a = 0; a < NPRE_W; ++a) {
            const int u = tid + 512 * a;
            if (u < NUW)
                *reinterpret_cast<u32x4 *>(sW + u * EPU) = ((pr.wok >> a) & 1u) ? pr.w[a] : u32x4{0, 0, 0, 0};
        }
#pragma unroll
        for (int a = 0; a < NPRE_O; ++a) {
            const int u = tid + 512 * a;
            if (u >= NUO) continue;
            const int tok = u / (4 * NVS), grp = u % (4 * NVS);
            const bool ok = ((pr.ook >> a) & 1u) != 0;
            float x[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) x[i] = ok ? pr.o[a][i] : 0.f;
            st_q4<PK>(sO + k16_block(tok >> 4, grp >> 2, 16 * NVS) + 4 * ((tok & 15) + 16 * (grp & 3)),
                      pack4<PK>(x[0], x[1], x[2], x[3]));
        }
    };
    const st *sUb = sW;
    const st *sYb = sW + NB_U * BLK;
    const st *sHb = sW + (NB_U + NB_Y) * BLK;
    const st *sDb = sW + (NB_U + NB_Y + NB_H) * BLK;
    auto blkU = [=](int rt, int vl) { return sUb + (rt * NVS + vl) * BLK + 4 * l; };
    auto blkY = [=](int rt, int vl) { return sYb + (rt * NVS + vl) * BLK + 4 * l; };
    auto blkH = [=](int dt, int vl) { return sHb + (dt * NVS + vl) * BLK + 4 * l; };
    auto blkD = [=](int dt, int vl) { return sDb + (dt * NVS + vl) * BLK + 4 * l; };
    auto blkO = [=](int rt, int vl) { return sO + (rt * NVS + vl) * BLK + 4 * l; };
    // acc += A . B^T over the staged value tiles (A, B given as tile loaders).
    auto mmav = [&](f32x4 acc, const st *a0, const st *b0) __attribute__((always_inline)) {
        if constexpr (NVS == 2)
            return mma2<PK>(acc, ld_q4<PK>(a0), ld_q4<PK>(a0 + BLK), ld_q4<PK>(b0), ld_q4<PK>(b0 + BLK));
        else
            return mma1<PK>(acc, ld_q4<PK>(a0), ld_q4<PK>(b0));
    };

    Pre pre;

    // ---- rows of this wave: raw q, k, b (input format) and the in-block log2
    // decay prefix G ----
    // (Loaded here for the factor tiles and again after the V-contractions,
    // so that they are not live across them.)
    auto load_rows = [&](Raw4<TI> (&qv)[NKH], Raw4<TI> (&kv)[NKH], Raw4<TI> (&bv)[NKH],
                         float (&gv)[NKH][4], auto between) __attribute__((always_inline)) {
        const TI *q = static_cast<const TI *>(p.q);
        const TI *k = static_cast<const TI *>(p.k);
        const TI *b = static_cast<const TI *>(p.b);
        const TG *g = static_cast<const TG *>(p.g);
        if (K == KP) {
            // Every channel tile is inside K: all loads are requested before any
            // is used (rows past the chunk end read its first row and are zeroed).
            Raw4<TG> rg[NKH];
            if constexpr (PFR) {
                // Requested during the previous item (or before the first),
                // complete since the wait at the top of the item.
                auto rd16 = [&](int tensor, int j) __attribute__((always_inline)) {
                    return *reinterpret_cast<const uint2 *>(rows_lds(tensor) + wv * (NKH * 512) +
                                                            16 * (32 * j + 16 * (kg >> 1) + m) + 8 * (kg & 1));
                };
#pragma unroll
                for (int j = 0; j < NKH; ++j) {
                    qv[j].u = rd16(0, j);
                    kv[j].u = rd16(1, j);
                    bv[j].u = rd16(2, j);
                    if constexpr (sizeof(TG) == 4)
                        rg[j].f = *reinterpret_cast<const float4 *>(rows_lds(3) + wv * (NKH * 1024) + 1024 * j + 16 * l);
                    else
                        rg[j].u = rd16(3, j);
                }
            } else {
                const int64_t off = row_ok ? roff : (t0 * H + h) * static_cast<int64_t>(K);
#pragma unroll
                for (int j = 0; j < NKH; ++j) {
                    const int c0 = 16 * (hh * NKH + j) + 4 * kg;
                    qv[j].load(q + off + c0);
                    kv[j].load(k + off + c0);
                    bv[j].load(b + off + c0);
                    rg[j].load(g + off + c0);
                }
            }
            between();  // more requests, issued before these rows are used
#pragma unroll
            for (int j = 0; j < NKH; ++j) {
                if (!row_ok) {
                    qv[j].zero();
                    kv[j].zero();
                    bv[j].zero();
                }
#pragma unroll
                for (int i = 0; i < 4; ++i) gv[j][i] = row16_scan((row_ok ? rg[j][i] : 0.f) * kLog2e);
            }
            return;
        }
        between();
#pragma unroll
        for (int j = 0; j < NKH; ++j) {
            const int c0 = 16 * (hh * NKH + j) + 4 * kg;
            float x[4];
            load4<TI>(q, roff, c0, K, row_ok, p.vec_ok, x);
            qv[j].set(x);
            load4<TI>(k, roff, c0, K, row_ok, p.vec_ok, x);
            kv[j].set(x);
            load4<TI>(b, roff, c0, K, row_ok, p.vec_ok, x);
            bv[j].set(x);
            load4<TG>(g, roff, c0, K, row_ok, p.vec_ok, gv[j]);
#pragma unroll
            for (int i = 0; i < 4; ++i) gv[j][i] = row16_scan(gv[j][i] * kLog2e);
        }
    };
    // The rows again after the V-contractions, without the gates: their
    // in-block prefix sums G stay in registers from the first load.
    auto reload_qkb = [&](Raw4<TI> (&qv)[NKH], Raw4<TI> (&kv)[NKH], Raw4<TI> (&bv)[NKH]) __attribute__((always_inline)) {
        const TI *q = static_cast<const TI *>(p.q);
        const TI *k = static_cast<const TI *>(p.k);
        const TI *b = static_cast<const TI *>(p.b);
        if (K == KP) {
            const int64_t off = row_ok ? roff : (t0 * H + h) * static_cast<int64_t>(K);
#pragma unroll
            for (int j = 0; j < NKH; ++j) {
                const int c0 = 16 * (hh * NKH + j) + 4 * kg;
                qv[j].load(q + off + c0);
                kv[j].load(k + off + c0);
                bv[j].load(b + off + c0);
            }
#pragma unroll
            for (int j = 0; j < NKH; ++j) {
                if (!row_ok) {
                    qv[j].zero();
                    kv[j].zero();
                    bv[j].zero();
                }
            }
            return;
        }
#pragma unroll
        for (int j = 0; j < NKH; ++j) {
            const int c0 = 16 * (hh * NKH + j) + 4 * kg;
            float x[4];
            load4<TI>(q, roff, c0, K, row_ok, p.vec_ok, x);
            qv[j].set(x);
            load4<TI>(k, roff, c0, K, row_ok, p.vec_ok, x);
            kv[j].set(x);
            load4<TI>(b, roff, c0, K, row_ok, p.vec_ok, x);
            bv[j].set(x);
        }
    };
    float invq, invk, qmul;
    bool bigq, bigk, wave_slow;
    float gv[NKH][4];  // in-block log2 decay prefix G of this wave's rows and channels
    {
    Raw4<TI> qv[NKH], kv[NKH], bv[NKH];
    load_rows(qv, kv, bv, gv, [&]() __attribute__((always_inline)) { issue_slice(pre, 0); });
    {
        float sq = 0.f, sk = 0.f;
        bool wide = false;
#pragma unroll
        for (int j = 0; j < NKH; ++j) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                sq = fmaf(qv[j][i], qv[j][i], sq);
                sk = fmaf(kv[j][i], kv[j][i], sk);
            }
            if (m == 15) {
                *reinterpret_cast<float4 *>(&sT[R][16 * (hh * NKH + j) + 4 * kg]) =
                    make_float4(gv[j][0], gv[j][1], gv[j][2], gv[j][3]);
#pragma unroll
                for (int i = 0; i < 4; ++i) wide = wide || (-gv[j][i] > kDiagSpanLimit2);
            }
        }
        sq += __shfl_xor(sq, 16, 64);
        sq += __shfl_xor(sq, 32, 64);
        sk += __shfl_xor(sk, 16, 64);
        sk += __shfl_xor(sk, 32, 64);
        if (kg == 0) {
            sRow[0][hh][r] = sq;
            sRow[1][hh][r] = sk;
        }
        const bool w_any = __ballot(wide) != 0;
        if (l == 0) sWide[R][hh] = w_any ? 1 : 0;
    }
    __syncthreads();
    const float nq = sqrtf(sRow[0][0][r] + sRow[0][1][r]), nk = sqrtf(sRow[1][0][r] + sRow[1][1][r]);
    invq = l2 ? 1.0f / fmaxf(nq, 1e-6f) : 1.0f;
    invk = l2 ? 1.0f / fmaxf(nk, 1e-6f) : 1.0f;
    bigq = nq > 1e-6f;
    bigk = nk > 1e-6f;
    qmul = invq * p.scale;
    wave_slow = (sWide[R][0] | sWide[R][1]) != 0;
    for (int e = tid; e < 4 * KP; e += 512) {
        const int Rb = e / KP, c = e % KP;
        const float t[4] = {sT[0][c], sT[1][c], sT[2][c], sT[3][c]};
        float cum = 0.f, after = 0.f;
#pragma unroll
        for (int R2 = 0; R2 < 4; ++R2) {
            if (R2 < Rb) cum += t[R2];
            if (R2 > Rb) after += t[R2];
        }
        sEr[Rb][c] = fexp2(cum);
        sEa[Rb][c] = fexp2(after);
        sE2[Rb][c] = fexp2(sT[Rb][c]);
        sE2n[Rb][c] = fexp2(-sT[Rb][c]);
    }
    // Factor tiles of this wave's rows and channels, transposed by an identity product.
#pragma unroll
    for (int j = 0; j < NKH; ++j) {
        const int dt = hh * NKH + j;
        const float4 tr = *reinterpret_cast<const float4 *>(&sT[R][16 * dt + 4 * kg]);
        const float trv[4] = {tr.x, tr.y, tr.z, tr.w};
        float qb[4], eb[4], ke[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float kn = kv[j][i] * invk;
            const float e1 = fexp2(gv[j][i]);
            qb[i] = qv[j][i] * qmul * e1;
            eb[i] = bv[j][i] * kn * e1;
            ke[i] = kn * fexp2(trv[i] - gv[j][i]);
        }
        auto put = [&](st (*dst)[4][NKT][BLK], const float (&x)[4]) __attribute__((always_inline)) {
            const Q hi = pack4<PK>(x[0], x[1], x[2], x[3]);
            st_q4<PK>(&dst[0][R][dt][4 * l], pack4<PK>(mma1<PK>(zero4(), hi, ident)));
            if constexpr (NPL == 2) {
                float xh[4];
                unpack4<PK>(hi, xh);
                const Q lo = pack4<PK>(x[0] - xh[0], x[1] - xh[1], x[2] - xh[2], x[3] - xh[3]);
                st_q4<PK>(&dst[1][R][dt][4 * l], pack4<PK>(mma1<PK>(zero4(), lo, ident)));
            }
        };
        put(sKT, ke);
        put(sQT, qb);
        put(sET, eb);
    }
    }

    // ---- V-contractions over staged slices ----
    //   aT[J] = dAqk^T tile (J, R)    lT[J] = dY U^T tile^T (J, R)    (J <= R)
    //   aN[I] = dAqk tile (I, R)      lN[I] = dY U^T tile (I, R)      (I >= R)
    //   cq[j] = dQbar, ce[j] = dY S0^T, ck[j] = dKtilde (row data, channel tile hh*NKH+j)
    f32x4 aT[4], lT[4], aN[4], lN[4], cq[NKH], ce[NKH], ck[NKH];
#pragma unroll
    for (int J = 0; J < 4; ++J) aT[J] = lT[J] = aN[J] = lN[J] = zero4();
#pragma unroll
    for (int j = 0; j < NKH; ++j) cq[j] = ce[j] = ck[j] = zero4();
    float last_acc[NLT];  // this lane's part of rowsum(dS1 * S0) for channel tiles wv + 8t
#pragma unroll
    for (int t = 0; t < NLT; ++t) last_acc[t] = 0.f;
    for (int vt0 = 0; vt0 < NVT; vt0 += NVS) {
        __syncthreads();  // previous slice fully consumed
        land_slice(pre);
        // dv = dY * w, dw = dY * v for this slice (v, w came with the prefetch).
        Raw4<TI> pv[NPRE_O], pw[NPRE_O];
#pragma unroll
        for (int a = 0; a < NPRE_O; ++a) {
            pv[a] = pre.v[a];
            pw[a] = pre.w2[a];
        }
        __syncthreads();
        if (vt0 + NVS < NVT) issue_slice(pre, vt0 + NVS);
#pragma unroll
        for (int a = 0; a < NPRE_O; ++a) {
            const int u = tid + 512 * a;
            const int tok = u / (4 * NVS), grp = u % (4 * NVS);
            const int c = 16 * vt0 + 4 * grp;
            if (u >= NUO || tok >= lc || c >= V) continue;
            float y[4], xv[4], xw[4];
            unpack4<PK>(ld_q4<PK>(sYb + ((tok >> 4) * NVS + (grp >> 2)) * BLK + 4 * ((tok & 15) + 16 * (grp & 3))), y);
            const int64_t off = ((t0 + tok) * H + h) * static_cast<int64_t>(V);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                xv[i] = y[i] * pw[a][i];
                xw[i] = y[i] * pv[a][i];
            }
            store4<TI>(dvp, off, c, V, xv);
            store4<TI>(dwp, off, c, V, xw);
        }
#pragma unroll
        for (int t = 0; t < NLT; ++t) {
            const int dt = wv + 8 * t;
            if (dt < NKT) {
#pragma unroll
                for (int vl = 0; vl < NVS; ++vl) {
                    float a4[4], c4[4];
                    unpack4<PK>(ld_q4<PK>(blkD(dt, vl)), a4);
                    unpack4<PK>(ld_q4<PK>(blkH(dt, vl)), c4);
#pragma unroll
                    for (int i = 0; i < 4; ++i) last_acc[t] = fmaf(a4[i], c4[i], last_acc[t]);
                }
            }
        }
#pragma unroll
        for (int J = 0; J < 4; ++J) {
            if (J <= R) {
                aT[J] = mmav(aT[J], blkU(J, 0), blkO(R, 0));
                lT[J] = mmav(lT[J], blkU(J, 0), blkY(R, 0));
            }
            if (J >= R) {
                aN[J] = mmav(aN[J], blkO(J, 0), blkU(R, 0));
                lN[J] = mmav(lN[J], blkY(J, 0), blkU(R, 0));
            }
        }
#pragma unroll
        for (int j = 0; j < NKH; ++j) {
            const int dt = hh * NKH + j;
            cq[j] = mmav(cq[j], blkH(dt, 0), blkO(R, 0));
            ce[j] = mmav(ce[j], blkH(dt, 0), blkY(R, 0));
            ck[j] = mmav(ck[j], blkD(dt, 0), blkU(R, 0));
        }
    }

    Raw4<TI> qv[NKH], kv[NKH], bv[NKH];
    reload_qkb(qv, kv, bv);

    // ---- G_last term: part 1 exp(G_last) rowsum(dS1 * S0) (channel tile wv),
    // part 2 this block's sum of dKt * Kt (ck = dKt here).  Together they are
    // rowsum(dS1 * S1) written through the saved S0 and U only. ----
#pragma unroll
    for (int t = 0; t < NLT; ++t) {
        const int dt = wv + 8 * t;
        if (dt < NKT) {
            float acc = last_acc[t];
            acc += __shfl_xor(acc, 16, 64);
            acc += __shfl_xor(acc, 32, 64);
            const int c = 16 * dt + m;
            if (kg == 0) sLast[c] = acc * fexp2(sT[0][c] + sT[1][c] + sT[2][c] + sT[3][c]);
        }
    }
#pragma unroll
    for (int j = 0; j < NKH; ++j) {
        const int dt = hh * NKH + j, c0 = 16 * dt + 4 * kg;
        const float4 tr = *reinterpret_cast<const float4 *>(&sT[R][c0]);
        const float4 ea = *reinterpret_cast<const float4 *>(&sEa[R][c0]);
        const float trv[4] = {tr.x, tr.y, tr.z, tr.w}, eav[4] = {ea.x, ea.y, ea.z, ea.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float kt_ = kv[j][i] * invk * fexp2(trv[i] - gv[j][i]) * eav[i];
            const float tot = row16_scan(ck[j][i] * kt_);
            if (m == 15) sKK[R][c0 + i] = tot;
            ce[j][i] = -ce[j][i];  // dEbar = -dY S0^T
        }
    }

    // ---- causal masks and signs; diagonal tiles kept for the exact path ----
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
    Q baT[4], blT[4], baN[4], blN[4];
#pragma unroll
    for (int J = 0; J < 4; ++J) {
        baT[J] = pack4<PK>(aT[J]);
        blT[J] = pack4<PK>(lT[J]);
        baN[J] = pack4<PK>(aN[J]);
        blN[J] = pack4<PK>(lN[J]);
    }

    // ---- pair products, Horner over blocks.  With P_J the product of block
    // J's factor tiles with the pair tiles, the sums the factored form needs are
    //   dq (and de):  Er dQbar + sum_{J<R} 2^(T_{J+1} + .. + T_{R-1}) P_J + 2^(-T_R) P_R
    //   dk:           Ea dKt   + sum_{I>R} 2^(T_{R+1} + .. + T_{I-1}) P_I + 2^(-T_R) P_R
    // (Er, Ea = decay before / after block R), so the running accumulator is
    // scaled by 2^(T_J) per channel between blocks and the factor tiles are used
    // as stored (hi + lo planes).  The diagonal block is skipped here when its
    // span is too wide for 2^(-T_R) (the exact path below handles it). ----
    auto pmma = [&](f32x4 acc, const st (*tile)[4][NKT][BLK], int blk, int dt, Q bop) __attribute__((always_inline)) {
#pragma unroll
        for (int pl = 0; pl < NPL; ++pl) acc = mma1<PK>(acc, ld_q4<PK>(&tile[pl][blk][dt][4 * l]), bop);
        return acc;
    };
    auto scale_by = [&](f32x4 &acc, const float *tab) __attribute__((always_inline)) {
        const float4 f = *reinterpret_cast<const float4 *>(tab);
        acc[0] *= f.x;
        acc[1] *= f.y;
        acc[2] *= f.z;
        acc[3] *= f.w;
    };
#pragma unroll
    for (int j = 0; j < NKH; ++j) {
        const int dt = hh * NKH + j, c0 = 16 * dt + 4 * kg;
#pragma unroll
        for (int J = 0; J < 3; ++J) {  // dq, de: column blocks J < R
            if (J < R) {
                scale_by(cq[j], &sE2[J][c0]);
                scale_by(ce[j], &sE2[J][c0]);
                cq[j] = pmma(cq[j], sKT, J, dt, baT[J]);
                ce[j] = pmma(ce[j], sKT, J, dt, blT[J]);
            }
        }
#pragma unroll
        for (int I = 3; I > 0; --I) {  // dk: row blocks I > R
            if (I > R) {
                scale_by(ck[j], &sE2[I][c0]);
                ck[j] = pmma(ck[j], sQT, I, dt, baN[I]);
                ck[j] = pmma(ck[j], sET, I, dt, blN[I]);
            }
        }
        if (!wave_slow) {  // diagonal block, factor 2^(-T_R)
            Q dA_R = baT[0], dL_R = blT[0], dN_R = baN[0], dLN_R = blN[0];
#pragma unroll
            for (int J = 1; J < 4; ++J)
                if (J == R) {
                    dA_R = baT[J];
                    dL_R = blT[J];
                    dN_R = baN[J];
                    dLN_R = blN[J];
                }
            f32x4 tq = pmma(zero4(), sKT, R, dt, dA_R);
            f32x4 te = pmma(zero4(), sKT, R, dt, dL_R);
            f32x4 tk = pmma(zero4(), sQT, R, dt, dN_R);
            tk = pmma(tk, sET, R, dt, dLN_R);
            const float4 f = *reinterpret_cast<const float4 *>(&sE2n[R][c0]);
            const float fv[4] = {f.x, f.y, f.z, f.w};
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                cq[j][i] = fmaf(tq[i], fv[i], cq[j][i]);
                ce[j][i] = fmaf(te[i], fv[i], ce[j][i]);
                ck[j][i] = fmaf(tk[i], fv[i], ck[j][i]);
            }
        }
    }

    // ---- row data: dq = 2^G cq, de = 2^G ce, dk = 2^(T_R - G) ck, exact
    // diagonal terms of wide blocks, dG with its in-block suffix sums ----
    float pq = 0.f, pk = 0.f;  // row dots for the L2-norm chain rule
#pragma unroll
    for (int j = 0; j < NKH; ++j) {
        const int dt = hh * NKH + j, c0 = 16 * dt + 4 * kg;
        const float4 tr = *reinterpret_cast<const float4 *>(&sT[R][c0]);
        const float trv[4] = {tr.x, tr.y, tr.z, tr.w};
        float qn[4], kn[4], en[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            qn[i] = qv[j][i] * qmul;
            kn[i] = kv[j][i] * invk;
            en[i] = bv[j][i] * kn[i];
            cq[j][i] *= fexp2(gv[j][i]);
            ce[j][i] *= fexp2(gv[j][i]);
            ck[j][i] *= fexp2(trv[i] - gv[j][i]);
        }
        if (wave_slow) {
#pragma unroll
            for (int jj = 0; jj < 16; ++jj) {
                const int src_l = m + 16 * (jj >> 2);
                const float a = __shfl(dAd[jj & 3], src_l, 64);
                const float lv = __shfl(dLd[jj & 3], src_l, 64);
                const float aN2 = __shfl(dANd[jj & 3], src_l, 64);
                const float lN2 = __shfl(dLNd[jj & 3], src_l, 64);
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int src = 16 * kg + jj;
                    const float kj = __shfl(kn[i], src, 64), qj = __shfl(qn[i], src, 64);
                    const float ej = __shfl(en[i], src, 64), Gj = __shfl(gv[j][i], src, 64);
                    const float lo = (jj <= m) ? fexp2(gv[j][i] - Gj) : 0.f;  // row m, column jj
                    const float hi = (jj >= m) ? fexp2(Gj - gv[j][i]) : 0.f;  // row jj, column m
                    cq[j][i] = fmaf(a * kj, lo, cq[j][i]);
                    ce[j][i] = fmaf(lv * kj, lo, ce[j][i]);
                    ck[j][i] = fmaf(aN2 * qj + lN2 * ej, hi, ck[j][i]);
                }
            }
        }
        float dbv4[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float dG = qn[i] * cq[j][i] + en[i] * ce[j][i] - kn[i] * ck[j][i];
            const float dbv = ce[j][i] * kn[i];
            dbv4[i] = dbv;
            ck[j][i] = fmaf(ce[j][i], bv[j][i], ck[j][i]);  // dk += de * b
            cq[j][i] *= p.scale;                            // w.r.t. the normalised q
            pq = fmaf(qv[j][i] * invq, cq[j][i], pq);
            pk = fmaf(kn[i], ck[j][i], pk);
            const float pre_s = row16_scan(dG);
            const float tot = __shfl(pre_s, 16 * kg + 15, 64);
            if (m == 0) sDG[R][c0 + i] = tot;
            ce[j][i] = tot - pre_s + dG;  // in-block suffix sum of dG
        }
        if (row_ok) store4<TI>(static_cast<TI *>(p.db), roff, c0, K, dbv4);
    }
    pq += __shfl_xor(pq, 16, 64);
    pq += __shfl_xor(pq, 32, 64);
    pk += __shfl_xor(pk, 16, 64);
    pk += __shfl_xor(pk, 32, 64);
    if (kg == 0) {
        sRow[0][hh][r] = pq;
        sRow[1][hh][r] = pk;
    }
    __syncthreads();
    // Every wave's pair products are done: the factor tiles take the next
    // item's rows.
    if (PFR && K == KP && item + static_cast<int>(gridDim.x) < items) dma_rows(item + gridDim.x, wv, l);
    pq = sRow[0][0][r] + sRow[0][1][r];
    pk = sRow[1][0][r] + sRow[1][1][r];
    if (row_ok) {
#pragma unroll
    for (int j = 0; j < NKH; ++j) {
        const int c0 = 16 * (hh * NKH + j) + 4 * kg;
        float dg4[4], dq4[4], dk4[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int c = c0 + i < KP ? c0 + i : KP - 1;
            float later = sLast[c] + sKK[0][c] + sKK[1][c] + sKK[2][c] + sKK[3][c];
#pragma unroll
            for (int R2 = 1; R2 < 4; ++R2)
                if (R2 > R) later += sDG[R2][c];
            dg4[i] = ce[j][i] + later;
            float dq = cq[j][i], dk = ck[j][i];
            if (l2) {
                // d/dx of x / max(||x||, eps): (dy - y (y . dy)) / ||x|| above eps, dy / eps below.
                dq = bigq ? (dq - qv[j][i] * invq * pq) * invq : dq * invq;
                dk = bigk ? (dk - kv[j][i] * invk * pk) * invk : dk * invk;
            }
            dq4[i] = dq;
            dk4[i] = dk;
        }
        store4<TG>(static_cast<TG *>(p.dg), roff, c0, K, dg4);
        store4<TI>(static_cast<TI *>(p.dq), roff, c0, K, dq4);
        store4<TI>(static_cast<TI *>(p.dk), roff, c0, K, dk4);
    }
    }
    // sRow, sT and the block tables are rewritten by the next item.  With the
    // rows' direct LDS loads in flight, the barrier waits only for this
    // wave's LDS accesses (a workgroup fence would also wait for the loads,
    // which the next item's first wait covers).
    if constexpr (PFR)
        asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    else
        __syncthreads();
    }
}

template <PrecKind PK, int KP, typename TI, typename TG>
hipError_t launch_bwd(const BwdParams &p, int total_chunks, hipStream_t stream)
{
    if (p.num_seqs == 0) return hipSuccess;
    const int NP = p.num_seqs * p.H;
    const int groups = (NP + 7) / 8;
    auto go = [&](auto bvtag) {
        constexpr int BV = decltype(bvtag)::value;
        const int NVB = (p.V + BV - 1) / BV;
        hipLaunchKernelGGL((chunk_bwd_scan_kernel<PK, KP, BV, TI>), dim3(groups * 8 * NVB), dim3(512), 0,
                           stream, p, NVB, NP);
    };
    const int bv = scan_bv(NP, p.V);
    if (bv == 16) go(std::integral_constant<int, 16>{});
    else if (bv == 32) go(std::integral_constant<int, 32>{});
    else go(std::integral_constant<int, 64>{});
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || total_chunks == 0) return e;
    // One resident wave of workgroups (occupancy x CUs of the current device,
    // looked up once per device), each walking items (chunk, head) =
    // item / H, item % H with a stride of the grid.
    const auto kern = chunk_bwd_kside_kernel<PK, KP, TI, TG>;
    static std::atomic<int> resident[64];  // per instantiation
    int slots = 0;
    e = resident_slots(kern, 512, resident, &slots);
    if (e != hipSuccess) return e;
    const int64_t items = static_cast<int64_t>(total_chunks) * p.H;
    if (items > (int64_t{1} << 30)) return hipErrorInvalidValue;  // item indices stay in int
    const int grid = static_cast<int>(items < slots ? items : slots);
    hipLaunchKernelGGL(kern, dim3(grid), dim3(512), 0, stream, p, static_cast<int>(items));
    return hipGetLastError();
}

template <PrecKind PK, typename TI, typename TG>
hipError_t launch_bwd_kp(const BwdParams &p, int total_chunks, hipStream_t stream)
{
    switch (kp_for(p.K)) {
    case 32: return launch_bwd<PK, 32, TI, TG>(p, total_chunks, stream);
    case 64: return launch_bwd<PK, 64, TI, TG>(p, total_chunks, stream);
    case 128: return launch_bwd<PK, 128, TI, TG>(p, total_chunks, stream);
    default:
        if constexpr (PK != PrecKind::F32) return launch_bwd<PK, 256, TI, TG>(p, total_chunks, stream);
        return hipErrorInvalidValue;  // not reached: fp32 beyond d_k = 128 is rejected before
    }
}

}  // namespace

size_t chunk_bwd_workspace_bytes(int B, int T, int H, int K, int V, int io_dtype,
                                 const int64_t *cu_host, int num_seqs)
{
    if (chunk_wide(K, io_dtype)) return wide_bwd_workspace_bytes(B, T, H, K, V, cu_host, num_seqs);
    if (!chunk_k_supported(K, io_dtype)) return 0;
    const int64_t nc = count_chunks(B, T, cu_host, num_seqs);
    return static_cast<size_t>(bwd_layout(nc, H, K, V, io_dtype).total);
}

size_t chunk_train_workspace_bytes(int B, int T, int H, int K, int V, int io_dtype,
                                   const int64_t *cu_host, int num_seqs)
{
    if (chunk_wide(K, io_dtype)) return wide_train_workspace_bytes(B, T, H, K, V, cu_host, num_seqs);
    if (!chunk_k_supported(K, io_dtype)) return 0;
    const int64_t nc = count_chunks(B, T, cu_host, num_seqs);
    return static_cast<size_t>(train_layout(nc, H, K, V, io_dtype).total);
}

int launch_chunk_bwd(const ChunkBwdArgs &a, int io_dtype, int g_dtype, hipStream_t stream)
{
    if (chunk_wide(a.K, io_dtype)) return launch_chunk_bwd_wide(a, g_dtype, stream);
    if (!chunk_k_supported(a.K, io_dtype)) return GDN2_ERR_UNSUPPORTED;
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

// Chunk start states of a training forward (K16 A-order tiles of the scan's
// operand precision, the io dtype) rewritten as [nc, H, K, V] or [nc, H, V, K]
// rows: a permutation of elements, one thread per output element so the
// writes are coalesced.  This is the reference's return_intermediate_states
// output (chunk_gdn2.py:1257-1263: h of chunk_gated_delta_rule_fwd_h, in the
// inputs' dtype).
template <typename E>
__global__ __launch_bounds__(256) void chunk_states_kernel(const E *hs, E *out, int trans, int64_t total, int H,
                                                           int K, int V, int KP, int VP)
{
    const int64_t idx = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    if (idx >= total) return;
    const int inner = trans ? K : V, outer = trans ? V : K;
    int64_t r = idx;
    const int a = static_cast<int>(r % inner);
    r /= inner;
    const int b = static_cast<int>(r % outer);
    r /= outer;
    const int hh = static_cast<int>(r % H);
    const int64_t gc = r / H;
    const int k = trans ? a : b, v = trans ? b : a;
    const int kt = k >> 4, m = k & 15, vt = v >> 4, c = v & 15;
    const int64_t src = (gc * H + hh) * static_cast<int64_t>(KP) * VP + k16_block(kt, vt, VP) +
                        4 * (m + 16 * (c >> 2)) + (c & 3);
    out[idx] = hs[src];
}

hipError_t launch_chunk_states(const void *hs, int io_dtype, void *out, bool transpose, int64_t nc,
                               int H, int K, int V, hipStream_t stream)
{
    const int KP = kp_for(K), VP = static_cast<int>(round_up(V, 16));
    const int64_t total = nc * H * K * V;
    const dim3 grid(static_cast<unsigned>((total + 255) / 256));
    if (io_dtype == GDN2_DTYPE_F32)
        hipLaunchKernelGGL((chunk_states_kernel<uint32_t>), grid, dim3(256), 0, stream,
                           static_cast<const uint32_t *>(hs), static_cast<uint32_t *>(out), int(transpose),
                           total, H, K, V, KP, VP);
    else
        hipLaunchKernelGGL((chunk_states_kernel<uint16_t>), grid, dim3(256), 0, stream,
                           static_cast<const uint16_t *>(hs), static_cast<uint16_t *>(out), int(transpose),
                           total, H, K, V, KP, VP);
    return hipGetLastError();
}

}  // namespace gdn2
