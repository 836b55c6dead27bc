// Chunkwise-parallel gdn2 forward (prefill / training forward), gfx950.
//
// Replaces reference chunk_gdn2 / chunk_gdn2_fwd (gdn2_ops/chunk_gdn2.py:1165-1434);
// the arithmetic is that of torch_recurrent_gdn2 (models/gdn2/gdn2.py:100-184)
// regrouped per chunk of C = 64 tokens.  For a chunk with start state S0 and
// in-chunk cumulative log decay G_r = sum_{i<=r} g_i (per key channel), with
// q scaled and normalised, e = b*k, z = w*v:
//
//   Aqk[r,i] = sum_d q_rd k_id exp(G_rd - G_id)      (i <= r)
//   L[r,i]   = sum_d e_rd k_id exp(G_rd - G_id)      (i <  r)
//   X = (I + L)^{-1},  W = X (e*exp(G)),  U = X z - W S0
//   O = (q*exp(G)) S0 + Aqk U,   S1 = Diag(exp(G_last)) S0 + (k*exp(G_last-G))^T U
//
// Only relative decays appear.  The pair products are factored per 16-token
// sub-block R with references that keep every factor in [2^-D, 2^D] (D = the
// sub-block's decay span in log2 units): rows q*2^(G_r - G_start(R)), columns
// k*2^(G_end(I) - G_i) times the decay between the blocks (<= 1), and 2^D on
// the diagonal block.  A diagonal block whose span exceeds kDiagSpanLimit2
// (factors would leave the normal fp32/bf16 range) is formed from four
// products referred to the starts of its 4-token quarters, and the pairs inside
// a quarter whose own span exceeds the limit are summed exactly, pair by pair,
// on the VALU (all 16 columns, in the instantiations whose registers do not
// hold the quarter products).  Decays are handled in log2 units so every
// exponential is one v_exp_f32.
//
// Operands follow the K16 convention of gdn2_mfma.h: accumulators of one
// product are B operands of the next without data movement, and a product
// with the identity transposes a tile in registers.
//
// Two kernels:
//  * chunk_prep_kernel -- a persistent grid of 4-wave workgroups (wave R =
//    16-token block R), each walking (chunk, head) items with the next
//    item's input rows in flight during the current one.  Fused prologue
//    (L2 norm, scale, optional in-kernel gate, in-block prefix sums), Aqk^T and L^T on
//    MFMA, the block-triangular inverse of I + L in fp32, and W^T = Ebar^T X^T.
//    It writes one contiguous "blob" per (chunk, head): X, -W, Qbar, Aqk,
//    Ktilde^T in K16 fragment-native order plus exp(G_last).
//  * chunk_scan_kernel -- one workgroup per (sequence, head, 64-column value
//    slice) walking the chunks in order.  Wave c owns 16 value columns and
//    holds its fp32 state columns S[:, c] as accumulators; with the column
//    split no wave needs another's U or S, so U, O and the state update run
//    from registers.  Each chunk's blob is copied to LDS once per workgroup
//    (double-buffered, the next blob prefetched into registers during the
//    current chunk) and read by all four waves.  Both value slices of a head
//    share an XCD, so the second blob read hits L2.

#include <type_traits>

#include "gdn2_chunk.h"
#include "gdn2_internal.h"

namespace gdn2 {

namespace {

// Four consecutive input values kept as the input dtype's bits (two registers
// for 16-bit inputs, half of what fp32 values take) and widened to fp32 where
// they are used.
template <typename T>
struct Raw4 {
    static constexpr int W = sizeof(T) == 2 ? 2 : 4;
    uint32_t u[W];
    __device__ __forceinline__ void zero()
    {
#pragma unroll
        for (int w = 0; w < W; ++w) u[w] = 0u;
    }
    // p: 4 values, 8-byte (16-bit T) or 16-byte (fp32) aligned.
    __device__ __forceinline__ void load(const T *p)
    {
        if constexpr (W == 2) {
            const uint2 a = *reinterpret_cast<const uint2 *>(p);
            u[0] = a.x;
            u[1] = a.y;
        } else {
            const uint4 a = *reinterpret_cast<const uint4 *>(p);
            u[0] = a.x;
            u[1] = a.y;
            u[2] = a.z;
            u[3] = a.w;
        }
    }
    // Channels c0..c0+3 of the row at element off; zero outside [0, K) or when !ok.
    __device__ __forceinline__ void load_checked(const T *base, int64_t off, int c0, int K, bool ok, int vec_ok)
    {
        if (ok && vec_ok && c0 + 4 <= K) {
            load(base + off + c0);
            return;
        }
        zero();
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            if (!(ok && c0 + i < K)) continue;
            if constexpr (W == 2) {
                const uint32_t bits = reinterpret_cast<const uint16_t *>(base)[off + c0 + i];
                u[i >> 1] |= bits << (16 * (i & 1));
            } else {
                u[i] = reinterpret_cast<const uint32_t *>(base)[off + c0 + i];
            }
        }
    }
    // Four fp32 values into the input dtype's bits (rounded to nearest even).
    __device__ __forceinline__ void set(const float (&x)[4])
    {
        if constexpr (W == 2) {
            uint16_t h[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                if constexpr (std::is_same<T, bf16_t>::value)
                    h[i] = f32_to_bf16_bits(x[i]);
                else
                    h[i] = __builtin_bit_cast(uint16_t, static_cast<_Float16>(x[i]));
            }
            u[0] = h[0] | (static_cast<uint32_t>(h[1]) << 16);
            u[1] = h[2] | (static_cast<uint32_t>(h[3]) << 16);
        } else {
#pragma unroll
            for (int i = 0; i < 4; ++i) u[i] = __float_as_uint(x[i]);
        }
    }
    __device__ __forceinline__ void unpack(float (&x)[4]) const
    {
        if constexpr (std::is_same<T, float>::value) {
#pragma unroll
            for (int i = 0; i < 4; ++i) x[i] = __uint_as_float(u[i]);
        } else if constexpr (std::is_same<T, bf16_t>::value) {
            x[0] = __uint_as_float(u[0] << 16);
            x[1] = __uint_as_float(u[0] & 0xffff0000u);
            x[2] = __uint_as_float(u[1] << 16);
            x[3] = __uint_as_float(u[1] & 0xffff0000u);
        } else {
#pragma unroll
            for (int i = 0; i < 4; ++i)
                x[i] = static_cast<float>(
                    __builtin_bit_cast(_Float16, static_cast<uint16_t>(u[i >> 1] >> (16 * (i & 1)))));
        }
    }
};

// Rows 16R..16R+15 of one [.., K] input (K == KP) for the calling wave:
// 16-byte loads that cover whole rows (lane l: row rr = j*RPI + l/LPR, bytes
// 16*(l%LPR) of it), so every load instruction reads complete 128-byte lines.
template <typename T, int KP>
struct RowLoad {
    static constexpr int RB = KP * static_cast<int>(sizeof(T));  // bytes per row
    static constexpr int RS = RB + 16;                            // LDS row stride (bank skew)
    static constexpr int LPR = RB / 16;                           // lanes per row
    static constexpr int RPI = 64 / LPR;                          // rows per instruction
    static constexpr int NI = 16 / RPI;                           // instructions
    u32x4 v[NI];
    // Rows first..first+15 of the chunk whose row 0 starts at element chunk0;
    // rows at or beyond the chunk length lc read the chunk's row 0 instead
    // (always in bounds) and are zeroed by land(), so no result of a load is
    // selected on before it is needed.
    __device__ __forceinline__ void issue(const T *base, int64_t chunk0, int64_t stride, int first, int lc,
                                          int l)
    {
#pragma unroll
        for (int j = 0; j < NI; ++j) {
            const int row = first + j * RPI + l / LPR;
            const int rc = row < lc ? row : 0;
            const char *src = reinterpret_cast<const char *>(base + chunk0 + rc * stride) + 16 * (l % LPR);
            v[j] = *reinterpret_cast<const u32x4 *>(src);
        }
    }
    __device__ __forceinline__ void clear()
    {
#pragma unroll
        for (int j = 0; j < NI; ++j) v[j] = u32x4{0, 0, 0, 0};
    }
    // Through the wave's LDS scratch into the A-order registers (row m,
    // channels 16kt + 4kg + i); rows rr >= nvalid are zero.
    __device__ __forceinline__ void land(unsigned char *stg, int l, int m, int kg, int nvalid,
                                         float (&out)[KP / 16][4])
    {
#pragma unroll
        for (int j = 0; j < NI; ++j) {
            const int rr = j * RPI + l / LPR;
            *reinterpret_cast<u32x4 *>(stg + rr * RS + 16 * (l % LPR)) =
                rr < nvalid ? v[j] : u32x4{0, 0, 0, 0};
        }
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
        __builtin_amdgcn_wave_barrier();
        const T *row = reinterpret_cast<const T *>(stg + m * RS);
#pragma unroll
        for (int kt = 0; kt < KP / 16; ++kt) {
            float x[4];
            load4<T>(row, 0, 16 * kt + 4 * kg, KP, true, 1, x);
#pragma unroll
            for (int i = 0; i < 4; ++i) out[kt][i] = x[i];
        }
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
        __builtin_amdgcn_wave_barrier();
    }
    // The same, keeping the input dtype's bits.
    __device__ __forceinline__ void land_raw(unsigned char *stg, int l, int m, int kg, int nvalid,
                                             Raw4<T> (&out)[KP / 16])
    {
#pragma unroll
        for (int j = 0; j < NI; ++j) {
            const int rr = j * RPI + l / LPR;
            *reinterpret_cast<u32x4 *>(stg + rr * RS + 16 * (l % LPR)) =
                rr < nvalid ? v[j] : u32x4{0, 0, 0, 0};
        }
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
        __builtin_amdgcn_wave_barrier();
        const T *row = reinterpret_cast<const T *>(stg + m * RS);
#pragma unroll
        for (int kt = 0; kt < KP / 16; ++kt) out[kt].load(row + 16 * kt + 4 * kg);
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
        __builtin_amdgcn_wave_barrier();
    }
};

// Rows first..first+15 as RowLoad, plus the three rows before them (one more
// load instruction, rows first-RPI..first-1 of which the last three are
// used): the window of the causal width-4 convolution.  Rows before lo (the
// sequence start, relative to the chunk) or at / beyond lc read as zero.
template <typename T, int KP>
struct RowLoadConv : RowLoad<T, KP> {
    using Base = RowLoad<T, KP>;
    using Base::LPR;
    using Base::NI;
    using Base::RPI;
    using Base::RS;
    u32x4 hv;
    bool hok;
    __device__ __forceinline__ void issue(const T *base, int64_t chunk0, int64_t stride, int first, int lo, int lc,
                                          int l)
    {
        const int hr = first - RPI + l / LPR;
        hok = hr >= first - 3 && hr >= lo && hr < lc;
        const int rc = hok ? hr : 0;
        hv = *reinterpret_cast<const u32x4 *>(reinterpret_cast<const char *>(base + chunk0 + rc * stride) +
                                              16 * (l % LPR));
        Base::issue(base, chunk0, stride, first, lc, l);
    }
    // Staged as rows first-4..first+15 (LDS rows 0..19); lane (m, kg) then
    // convolves rows m-3..m of channels 16kt + 4kg + i with the taps at
    // `taps` ([KP][4] 16-bit values, this wave's LDS copy):
    //   y = round(sum_j tap[c][j] * x[t-3+j]),  silu: y = round(y * rcp(1 + e^-y))
    // -- the order and roundings of the separate convolution pass.  Rows
    // m >= nvalid are zero.
    __device__ __forceinline__ void land(unsigned char *stg, int l, int m, int kg, int nvalid,
                                         const unsigned char *taps, bool silu, Raw4<T> (&out)[KP / 16])
    {
        static_assert(sizeof(T) == 2, "the fused convolution takes 16-bit inputs");
#pragma unroll
        for (int j = 0; j < NI; ++j) {
            const int rr = j * RPI + l / LPR;
            *reinterpret_cast<u32x4 *>(stg + (4 + rr) * RS + 16 * (l % LPR)) =
                rr < nvalid ? Base::v[j] : u32x4{0, 0, 0, 0};
        }
        const int hs = l / LPR - (RPI - 4);
        if (hs >= 0) *reinterpret_cast<u32x4 *>(stg + hs * RS + 16 * (l % LPR)) = hok ? hv : u32x4{0, 0, 0, 0};
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
        __builtin_amdgcn_wave_barrier();
        auto h2f = [](uint32_t bits) __attribute__((always_inline)) {
            if constexpr (std::is_same<T, bf16_t>::value)
                return __uint_as_float(bits << 16);
            else
                return static_cast<float>(__builtin_bit_cast(_Float16, static_cast<uint16_t>(bits)));
        };
#pragma unroll
        for (int kt = 0; kt < KP / 16; ++kt) {
            const int c0 = 16 * kt + 4 * kg;
            float x[4][4];
#pragma unroll
            for (int jj = 0; jj < 4; ++jj)
                load4<T>(reinterpret_cast<const T *>(stg + (m + 1 + jj) * RS), 0, c0, KP, true, 1, x[jj]);
            const u32x4 ta = *reinterpret_cast<const u32x4 *>(taps + 8 * c0);
            const u32x4 tb = *reinterpret_cast<const u32x4 *>(taps + 8 * c0 + 16);
            const uint32_t tw[8] = {ta[0], ta[1], ta[2], ta[3], tb[0], tb[1], tb[2], tb[3]};
            float y[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                float acc = 0.0f;
#pragma unroll
                for (int jj = 0; jj < 4; ++jj) {
                    const int e = 4 * i + jj;
                    acc = fmaf(h2f(tw[e >> 1] >> (16 * (e & 1)) & 0xffffu), x[jj][i], acc);
                }
                float yi = round_to<T>(acc + 0.0f);
                if (silu) yi = round_to<T>(silu_f32(yi));
                y[i] = m < nvalid ? yi : 0.0f;
            }
            out[kt].set(y);
        }
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
        __builtin_amdgcn_wave_barrier();
    }
};

// One prep work item: chunk gc (global index over all sequences) of head h;
// item = gc * H + h, so neighbouring items read neighbouring rows of the
// [tokens, H, K] inputs and write neighbouring blobs.
struct PrepItem {
    int gc, h, lc;   // lc = tokens in the chunk (<= kChunk)
    int jc;          // chunk index within its sequence
    int64_t t0;      // first token of the chunk
    int64_t chunk0;  // element offset of (token t0, head h, channel 0)
};

__device__ __forceinline__ PrepItem prep_item(const ChunkParams &p, int item)
{
    PrepItem it;
    it.gc = item / p.H;
    it.h = item - it.gc * p.H;
    int n, jc;
    int64_t bos, len;
    locate_chunk(p, it.gc, n, jc, bos, len);
    const int64_t t0 = bos + static_cast<int64_t>(jc) * kChunk;
    const int64_t rem = len - static_cast<int64_t>(jc) * kChunk;
    it.lc = rem < kChunk ? static_cast<int>(rem) : kChunk;
    it.jc = jc;
    it.t0 = t0;
    it.chunk0 = (t0 * p.H + it.h) * static_cast<int64_t>(p.K);
    return it;
}

// ---------------------------------------------------------------------------
// Prep: a persistent grid of workgroups (4 waves each) walking the items
// blockIdx.x, blockIdx.x + gridDim.x, ...  Wave R owns token rows
// 16R..16R+15; lane (m, kg) holds row 16R+m and channels 16kt + 4kg + i.
//
// Sized for three workgroups per CU with 16-bit storage: 52 KB of LDS (the
// block vectors live in the X matrix's space until X is formed, and the
// off-diagonal inverse steps use L's unused upper blocks as scratch) and at
// most 168 registers (q, k, b stay in their 16-bit input form until the
// factors).  fp32 storage at KP = 128 fits one workgroup per CU.
// ---------------------------------------------------------------------------
template <PrecKind PK, int KP, typename TI, typename TG, bool CONV = false>
__global__ __launch_bounds__(256)
__attribute__((amdgpu_waves_per_eu((PK == PrecKind::F32 && KP == 128) || KP > 128 ? 1
                                   : (PK != PrecKind::F32 && KP <= 64 ? 4 : 3)))) void
chunk_prep_kernel(ChunkParams p, int items)
{
    static_assert(!CONV || (sizeof(TI) == 2 && KP <= 128), "the fused convolution takes 16-bit rows, d_k <= 128");
    using P = Prec<PK>;
    using st = typename P::st;
    using BL = Blob<PK, KP>;
    using Q = Q4<PK>;
    constexpr int NKT = KP / 16;
    constexpr int NKS = KP / 32;
    // Row-major [64][KP] keys (storage precision).  The 4-element pad: with 8
    // the pair products' 8-byte row reads counted 1.33 bank-conflict cycles
    // per LDS instruction over the kernel, with 4 (or 12) 0.80.
    constexpr int LDK = KP + 4;
    constexpr int LDF = 64 + 4;  // fp32 [64][64]
    constexpr int SZK = 64 * LDK * static_cast<int>(sizeof(st));
    constexpr int SZ1 = SZK > 64 * LDF * 4 ? SZK : 64 * LDF * 4;
    __shared__ __align__(16) unsigned char smem1[SZ1];  // Kend, then L (fp32)
    __shared__ __align__(16) st sEt[NKT * 4 * 256];     // Ebar^T, K16 blocks (channel, token)
    // sX holds, in turn: waves 0-1's row staging, the block vectors, then X.
    // X keeps only its ten lower 16x16 blocks, (I, J) for J <= I at block
    // I (I + 1) / 2 + J, rows LDB apart: with 16-bit storage at d_k <= 64 this
    // brings the kernel to 40 KB of LDS, four workgroups per CU.
    constexpr int LDB = 16 + 4;
    constexpr int XBS = 16 * LDB;
    constexpr int SZX0 = 10 * XBS > 24 * KP ? 10 * XBS : 24 * KP;
    constexpr int SZX = SZX0 > 8 * (KP * 4 + 16) ? SZX0 : 8 * (KP * 4 + 16);
    __shared__ __align__(16) float sX[SZX];
    __shared__ __align__(16) float sT[4][KP];           // in-block decay totals (log2)
    st *sKend = reinterpret_cast<st *>(smem1);
    float *sL = reinterpret_cast<float *>(smem1);
    // Block vectors, in sX until the inverse writes X there.
    float(*sEr)[KP] = reinterpret_cast<float(*)[KP]>(sX);              // 2^(decay before block)
    float(*sEa)[KP] = reinterpret_cast<float(*)[KP]>(sX + 4 * KP);     // 2^(decay after block)
    float(*sPf)[4][KP] = reinterpret_cast<float(*)[4][KP]>(sX + 8 * KP);  // key scale of block pair (R, I)
    static_assert(24 * KP <= SZX, "block vectors must fit in sX");
    static_assert(sizeof(sX) >= 2 * 16 * (KP * 4 + 16) && sizeof(smem1) >= 2 * 16 * (KP * 4 + 16),
                  "row staging must fit in sX and smem1");

    const int lane = threadIdx.x & 63;
    const int R0 = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);  // wave index, uniform
    const int H = p.H, K = p.K;
    const bool rows_whole = K == KP;  // whole-row 16-byte loads through LDS
    const int64_t stride = static_cast<int64_t>(H) * K;

    const TI *q = static_cast<const TI *>(p.q);
    const TI *k = static_cast<const TI *>(p.k);
    const TI *b = static_cast<const TI *>(p.b);
    const TG *g = static_cast<const TG *>(p.g);

    // Rows staged through a per-wave LDS scratch: sX for waves 0-1, smem1
    // for waves 2-3; both are free from the end of one item (after its last
    // barrier) until the first barrier of the next.
    unsigned char *stg = R0 < 2 ? reinterpret_cast<unsigned char *>(sX) + R0 * (16 * (KP * 4 + 16))
                                : smem1 + (R0 - 2) * (16 * (KP * 4 + 16));
    PrepItem it = prep_item(p, blockIdx.x);

    for (int item = blockIdx.x; item < items; item += gridDim.x) {
        // The lane and wave indices are made opaque per item so that the
        // compiler does not hoist the many per-lane LDS and blob addresses out
        // of the loop, where they would hold registers through every phase.
        int l = lane, R = R0;
        asm volatile("" : "+v"(l));
        asm volatile("" : "+s"(R));
        const int tid = 64 * R + l, m = l & 15, kg = l >> 4;
        const int gc = it.gc, h = it.h, lc = it.lc;
        const int r = 16 * R + m;
        const bool row_ok = r < lc;
        const int64_t roff = it.chunk0 + r * stride;

        Raw4<TI> qr[NKT], kr[NKT], br[NKT];
        float gv[NKT][4];
        if constexpr (CONV) {
            // q and k are the raw projections (K == KP): each wave stages its
            // copy of the head's taps in sEt (unused until the factors) and
            // convolves its rows while landing them.  The taps are requested
            // first, so the wait for them does not cover the rows.
            constexpr int TBY = KP * 8;  // bytes of one tensor's taps [KP][4]
            static_assert(8 * TBY <= static_cast<int>(sizeof(sEt)), "four waves' taps must fit in sEt");
            static_assert(20 * RowLoad<TI, KP>::RS <= 16 * (KP * 4 + 16), "20 staged rows must fit the scratch");
            unsigned char *tq = reinterpret_cast<unsigned char *>(sEt) + R * (2 * TBY);
            unsigned char *tk = tq + TBY;
            const bool tl = 16 * l < TBY;
            const int64_t toff = static_cast<int64_t>(h) * TBY + 16 * (tl ? l : 0);
            const u32x4 wq4 = *reinterpret_cast<const u32x4 *>(static_cast<const unsigned char *>(p.conv_w[0]) + toff);
            const u32x4 wk4 = *reinterpret_cast<const u32x4 *>(static_cast<const unsigned char *>(p.conv_w[1]) + toff);
            RowLoadConv<TI, KP> lq, lk;
            RowLoad<TI, KP> lb;
            RowLoad<TG, KP> lg;
            const int lo = -kChunk * it.jc;
            lq.issue(q, it.t0 * p.ldq + static_cast<int64_t>(h) * KP, p.ldq, 16 * R, lo, lc, l);
            lk.issue(k, it.t0 * p.ldk + static_cast<int64_t>(h) * KP, p.ldk, 16 * R, lo, lc, l);
            lb.issue(b, it.chunk0, stride, 16 * R, lc, l);
            lg.issue(g, it.chunk0, stride, 16 * R, lc, l);
            if (tl) {
                *reinterpret_cast<u32x4 *>(tq + 16 * l) = wq4;
                *reinterpret_cast<u32x4 *>(tk + 16 * l) = wk4;
            }
            const int nvalid = lc - 16 * R;
            const bool silu = p.conv_silu != 0;
            lq.land(stg, l, m, kg, nvalid, tq, silu, qr);
            lk.land(stg, l, m, kg, nvalid, tk, silu, kr);
            lb.land_raw(stg, l, m, kg, nvalid, br);
            lg.land(stg, l, m, kg, nvalid, gv);
        } else if (rows_whole) {
            RowLoad<TI, KP> lq, lk, lb;
            RowLoad<TG, KP> lg;
            lq.issue(q, it.chunk0, stride, 16 * R, lc, l);
            lk.issue(k, it.chunk0, stride, 16 * R, lc, l);
            lb.issue(b, it.chunk0, stride, 16 * R, lc, l);
            lg.issue(g, it.chunk0, stride, 16 * R, lc, l);
            const int nvalid = lc - 16 * R;
            lq.land_raw(stg, l, m, kg, nvalid, qr);
            lk.land_raw(stg, l, m, kg, nvalid, kr);
            lb.land_raw(stg, l, m, kg, nvalid, br);
            lg.land(stg, l, m, kg, nvalid, gv);
        } else {
#pragma unroll
            for (int kt = 0; kt < NKT; ++kt) {
                const int c0 = 16 * kt + 4 * kg;
                qr[kt].load_checked(q, roff, c0, K, row_ok, p.vec_ok);
                kr[kt].load_checked(k, roff, c0, K, row_ok, p.vec_ok);
                br[kt].load_checked(b, roff, c0, K, row_ok, p.vec_ok);
                load4<TG>(g, roff, c0, K, row_ok, p.vec_ok, gv[kt]);
            }
        }
        // b given as logits: activated once here and rounded to the input
        // dtype, as the module's torch sigmoid of b_proj(x) is (gdn2.py:864).
        if (p.flags & GDN2_FLAG_SIGMOID_BW) {
#pragma unroll
            for (int kt = 0; kt < NKT; ++kt) {
                float x[4];
                br[kt].unpack(x);
#pragma unroll
                for (int i = 0; i < 4; ++i) x[i] = sigmoid_f(x[i]);
                br[kt].set(x);
            }
        }

        // Fused prologue: L2 norms (F.normalize semantics) and scale, applied
        // in the factors below; optional gate activation; decay in log2 units.
        float sq = 0.f, sk = 0.f;
#pragma unroll
        for (int kt = 0; kt < NKT; ++kt) {
            float xq[4], xk[4];
            qr[kt].unpack(xq);
            kr[kt].unpack(xk);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                sq = fmaf(xq[i], xq[i], sq);
                sk = fmaf(xk[i], xk[i], sk);
            }
        }
        sq += __shfl_xor(sq, 16, 64);
        sq += __shfl_xor(sq, 32, 64);
        sk += __shfl_xor(sk, 16, 64);
        sk += __shfl_xor(sk, 32, 64);
        const bool l2 = (p.flags & GDN2_FLAG_L2NORM_QK) != 0;
        // 1 / max(||x||, 1e-6) = rsqrt(max(||x||^2, 1e-12)), on the hardware
        // reciprocal square root (1 ulp) instead of an IEEE sqrt and divide.
        const float invq = l2 ? __builtin_amdgcn_rsqf(fmaxf(sq, 1e-12f)) : 1.0f;
        const float invk = l2 ? __builtin_amdgcn_rsqf(fmaxf(sk, 1e-12f)) : 1.0f;
        const float qmul = invq * p.scale;
        // Normalised q (scaled), k and the erase vector e = b * k of tile kt.
        auto qke = [&](int kt, float (&xq)[4], float (&xk)[4], float (&xe)[4]) __attribute__((always_inline)) {
            qr[kt].unpack(xq);
            kr[kt].unpack(xk);
            br[kt].unpack(xe);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                xq[i] *= qmul;
                xk[i] *= invk;
                xe[i] *= xk[i];
            }
        };
        if (p.flags & GDN2_FLAG_GATE_IN_KERNEL) {
            const int use_lb = (p.flags & GDN2_FLAG_LOWER_BOUND) != 0;
            const float a_log = p.A_log[h];
            // dt_bias of this lane's channels, all requested before any is used
            // (a load inside a per-element branch would wait for each one in
            // turn): 4-channel groups when K % 4 == 0, else clamped elements.
            float dbv[NKT][4];
            if (p.dt_bias) {
                const float *db = p.dt_bias + static_cast<int64_t>(h) * K;
#pragma unroll
                for (int kt = 0; kt < NKT; ++kt) {
                    const int c0 = 16 * kt + 4 * kg;
                    if (p.vec_ok) {
                        const float4 d4 = *reinterpret_cast<const float4 *>(db + (c0 < K ? c0 : K - 4));
                        dbv[kt][0] = d4.x;
                        dbv[kt][1] = d4.y;
                        dbv[kt][2] = d4.z;
                        dbv[kt][3] = d4.w;
                    } else {
#pragma unroll
                        for (int i = 0; i < 4; ++i) dbv[kt][i] = db[c0 + i < K ? c0 + i : K - 1];
                    }
                }
            } else {
#pragma unroll
                for (int kt = 0; kt < NKT; ++kt)
#pragma unroll
                    for (int i = 0; i < 4; ++i) dbv[kt][i] = 0.0f;
            }
#pragma unroll
            for (int kt = 0; kt < NKT; ++kt)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int c = 16 * kt + 4 * kg + i;
                    const float act = gate_activation(gv[kt][i], a_log, dbv[kt][i], use_lb, p.lower_bound);
                    gv[kt][i] = (row_ok && c < K) ? act : gv[kt][i];
                }
        }
#pragma unroll
        for (int kt = 0; kt < NKT; ++kt)
#pragma unroll
            for (int i = 0; i < 4; ++i) gv[kt][i] = row16_scan(gv[kt][i] * kLog2e);  // G (log2) from block start
        bool wide = false;
        if (m == 15) {
#pragma unroll
            for (int kt = 0; kt < NKT; ++kt) {
                *reinterpret_cast<float4 *>(&sT[R][16 * kt + 4 * kg]) =
                    make_float4(gv[kt][0], gv[kt][1], gv[kt][2], gv[kt][3]);
#pragma unroll
                for (int i = 0; i < 4; ++i) wide = wide || (-gv[kt][i] > kDiagSpanLimit2);
            }
        }
        // A diagonal block whose decay span (in any channel) is too wide for the
        // factored form is formed below instead of by the block products.
        const bool wave_slow = __ballot(wide) != 0;
        // A wide block is still formed on MFMA (bf16 storage at d_k <= 64 and
        // fp32 storage, where it fits the register budget): four products, each
        // with the factors referred to the decay at the start of one 4-token
        // quarter s, q_r 2^(G_r - G_s) and k_j 2^(G_s - G_j); the lane of row r
        // keeps the product of its quarter.  For a key j before the quarter both
        // factors are <= 1 (one that underflows belongs to a pair whose exact
        // value is below 2^-115 |q||k|).  Pairs inside the quarter are exact as
        // long as its span is <= kDiagSpanLimit2; factors of pairs that the
        // causal mask drops, or of rows of other quarters, are clamped (finite,
        // discarded).  A wave with a wider quarter recomputes the pairs inside
        // the quarters exactly, pair by pair (4 of the 16 columns of a row).
        constexpr bool QPATH = PK == PrecKind::F32 || (KP <= 64 && std::is_same<TI, bf16_t>::value);
        bool qwide = !QPATH;
        if (QPATH && wave_slow) {
#pragma unroll
            for (int kt = 0; kt < NKT; ++kt)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const float prev = __shfl(gv[kt][i], m >= 4 ? l - 4 : l, 64);
                    const float span = m >= 4 ? prev - gv[kt][i] : -gv[kt][i];
                    qwide = qwide || ((m & 3) == 3 && span > kDiagSpanLimit2);
                }
        }
        const bool wave_exact = wave_slow && __ballot(qwide) != 0;
        f32x4 dq = zero4(), dl = zero4();
        // Exact pair sums of row m (this lane's channels, then over the lane
        // groups) for the columns j0 + jj, jj < NJ, with j0 + jj > m dropped;
        // each column sums over (kt, i) in order.
        auto exact_pairs = [&](auto NJc, int j0, float (&cq)[decltype(NJc)::value],
                               float (&cl)[decltype(NJc)::value]) __attribute__((always_inline)) {
            constexpr int NJ = decltype(NJc)::value;
#pragma unroll
            for (int jj = 0; jj < NJ; ++jj) cq[jj] = cl[jj] = 0.f;
#pragma unroll
            for (int kt = 0; kt < NKT; ++kt) {
                float xq[4], xk[4], xe[4];
                qke(kt, xq, xk, xe);
#pragma unroll
                for (int i = 0; i < 4; ++i)
#pragma unroll
                    for (int jj = 0; jj < NJ; ++jj) {
                        const int j = j0 + jj;
                        const float kj = __shfl(xk[i], 16 * kg + j, 64);
                        const float Gj = __shfl(gv[kt][i], 16 * kg + j, 64);
                        const float ex = (j <= m) ? fexp2(gv[kt][i] - Gj) : 0.f;
                        cq[jj] = fmaf(xq[i] * kj, ex, cq[jj]);
                        cl[jj] = fmaf(xe[i] * kj, ex, cl[jj]);
                    }
            }
#pragma unroll
            for (int jj = 0; jj < NJ; ++jj) {
                cq[jj] += __shfl_xor(cq[jj], 16, 64);
                cq[jj] += __shfl_xor(cq[jj], 32, 64);
                cl[jj] += __shfl_xor(cl[jj], 16, 64);
                cl[jj] += __shfl_xor(cl[jj], 32, 64);
            }
        };
        if constexpr (QPATH) {
            if (wave_slow) {
                constexpr float kClamp2 = 120.0f;
#pragma unroll
                for (int s = 0; s < 4; ++s) {
                    // Two key tiles at a time (one 32-wide contraction step), so
                    // that only their factors are live.
                    f32x4 pq = zero4(), pl = zero4();
#pragma unroll
                    for (int s2 = 0; s2 < NKS; ++s2) {
                        Q fa[2], fb[2], fe[2];
#pragma unroll
                        for (int hh = 0; hh < 2; ++hh) {
                            const int kt = 2 * s2 + hh;
                            float xq[4], xk[4], xe[4], a[4], bq[4], be[4];
                            qke(kt, xq, xk, xe);
#pragma unroll
                            for (int i = 0; i < 4; ++i) {
                                const float G = gv[kt][i];
                                const float Gs = s == 0 ? 0.0f : __shfl(G, 16 * kg + 4 * s - 1, 64);
                                const float up = fexp2(fminf(G - Gs, kClamp2));
                                a[i] = xk[i] * fexp2(fminf(Gs - G, kClamp2));
                                bq[i] = xq[i] * up;
                                be[i] = xe[i] * up;
                            }
                            fa[hh] = pack4<PK>(a[0], a[1], a[2], a[3]);
                            fb[hh] = pack4<PK>(bq[0], bq[1], bq[2], bq[3]);
                            fe[hh] = pack4<PK>(be[0], be[1], be[2], be[3]);
                        }
                        pq = mma2<PK>(pq, fa[0], fa[1], fb[0], fb[1]);
                        pl = mma2<PK>(pl, fa[0], fa[1], fe[0], fe[1]);
                    }
                    if ((m >> 2) == s) {
                        dq = pq;
                        dl = pl;
                    }
                }
            }
            if (wave_exact) {
                // Lane (m, kg) of the products holds columns 4 kg .. 4 kg + 3
                // of row m, so the lane with kg = m / 4 holds row m's quarter.
                float cq[4], cl[4];
                exact_pairs(std::integral_constant<int, 4>{}, 4 * (m >> 2), cq, cl);
                if (kg == (m >> 2)) {
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        dq[i] = cq[i];
                        dl[i] = cl[i];
                    }
                }
            }
        } else if (wave_exact) {
            // All 16 columns of row m; lane (m, kg) keeps columns 4 kg .. 4 kg + 3.
            float cq[16], cl[16];
            exact_pairs(std::integral_constant<int, 16>{}, 0, cq, cl);
#pragma unroll
            for (int j = 0; j < 16; ++j)
                if (kg == (j >> 2)) {
                    dq[j & 3] = cq[j];
                    dl[j & 3] = cl[j];
                }
        }
        __syncthreads();

        st *ws = static_cast<st *>(p.ws) + (static_cast<int64_t>(gc) * H + h) * BL::SIZE;
        // Per-channel block vectors.
        for (int e = tid; e < 4 * KP; e += 256) {
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
#pragma unroll
            for (int I = 0; I < 4; ++I) {
                float ex = 0.f;
                if (I == Rb) {
                    ex = -t[Rb];
                } else {
#pragma unroll
                    for (int R2 = 0; R2 < 4; ++R2)
                        if (R2 > I && R2 < Rb) ex += t[R2];
                }
                sPf[Rb][I][c] = I > Rb ? 0.f : fexp2(ex);
            }
            if (Rb == 0) reinterpret_cast<float *>(ws + BL::GL)[c] = fexp2(t[0] + t[1] + t[2] + t[3]);
        }
        __syncthreads();

        // Factors.  Qb / Eb stay in registers as K16 operands of this row block;
        // Qbar goes straight to the blob; Ktilde^T and Ebar^T are transposed by
        // an identity product.
        const Q ident = identity_q4<PK>(l);
        Q fqb[NKT], feb[NKT];
#pragma unroll
        for (int kt = 0; kt < NKT; ++kt) {
            const int c0 = 16 * kt + 4 * kg;
            const float4 er = *reinterpret_cast<const float4 *>(&sEr[R][c0]);
            const float4 ea = *reinterpret_cast<const float4 *>(&sEa[R][c0]);
            const float4 tr = *reinterpret_cast<const float4 *>(&sT[R][c0]);
            const float erv[4] = {er.x, er.y, er.z, er.w};
            const float eav[4] = {ea.x, ea.y, ea.z, ea.w};
            const float trv[4] = {tr.x, tr.y, tr.z, tr.w};
            float xq[4], xk[4], xe[4];
            qke(kt, xq, xk, xe);
            float qb[4], eb[4], ke[4], qbar[4], ebar[4], ktil[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float G = gv[kt][i];
                const float e1 = fexp2(G), e2 = fexp2(trv[i] - G);
                qb[i] = xq[i] * e1;
                eb[i] = xe[i] * e1;
                ke[i] = xk[i] * e2;
                qbar[i] = qb[i] * erv[i];
                ebar[i] = eb[i] * erv[i];
                ktil[i] = ke[i] * eav[i];
            }
            fqb[kt] = pack4<PK>(qb[0], qb[1], qb[2], qb[3]);
            feb[kt] = pack4<PK>(eb[0], eb[1], eb[2], eb[3]);
            st_q4<PK>(ws + BL::QB + k16_block(R, kt, KP) + 4 * l,
                      pack4<PK>(qbar[0], qbar[1], qbar[2], qbar[3]));
            st_q4<PK>(sKend + r * LDK + c0, pack4<PK>(ke[0], ke[1], ke[2], ke[3]));
            const f32x4 dk = mma1<PK>(zero4(), pack4<PK>(ktil[0], ktil[1], ktil[2], ktil[3]), ident);
            st_q4<PK>(ws + BL::KT + k16_block(kt, R, 64) + 4 * l, pack4<PK>(dk));
            const f32x4 de = mma1<PK>(zero4(), pack4<PK>(ebar[0], ebar[1], ebar[2], ebar[3]), ident);
            st_q4<PK>(sEt + k16_block(kt, R, 64) + 4 * l, pack4<PK>(de));
        }
        __syncthreads();

        // Aqk^T(I, R) = Kend_I^T-scaled . Qb_R^T and L^T(I, R) likewise with Eb:
        // A = scaled keys of block I (LDS), B = this block's Qb / Eb (registers).
        // Lane (n, kg) of the result holds Aqk[16R+n][16I+4kg+i], which is the
        // K16 A-operand order of Aqk, so it is stored as is.
        // Instantiated per wave index (a compile-time RR), so that the causal
        // block conditions fold and the block's LDS reads are one straight-line
        // batch instead of a read-wait-use chain behind a branch per block.
        f32x4 aq[4], al[4];
        auto products = [&](auto Rc) __attribute__((always_inline)) {
            constexpr int RR = decltype(Rc)::value;
#pragma unroll
            for (int I = 0; I < 4; ++I) {
                aq[I] = zero4();
                al[I] = zero4();
                if (I <= RR) {
#pragma unroll
                    for (int s = 0; s < NKS; ++s) {
                        Q a[2];
#pragma unroll
                        for (int hh = 0; hh < 2; ++hh) {
                            const int c0 = 32 * s + 16 * hh + 4 * kg;
                            Q raw = ld_q4<PK>(sKend + (16 * I + m) * LDK + c0);
                            if (I != RR - 1) {
                                float x[4];
                                unpack4<PK>(raw, x);
                                const float4 sc = *reinterpret_cast<const float4 *>(&sPf[RR][I][c0]);
                                raw = pack4<PK>(x[0] * sc.x, x[1] * sc.y, x[2] * sc.z, x[3] * sc.w);
                            }
                            a[hh] = raw;
                        }
                        aq[I] = mma2<PK>(aq[I], a[0], a[1], fqb[2 * s], fqb[2 * s + 1]);
                        al[I] = mma2<PK>(al[I], a[0], a[1], feb[2 * s], feb[2 * s + 1]);
                    }
                }
            }
        };
        switch (R) {
        case 0: products(std::integral_constant<int, 0>{}); break;
        case 1: products(std::integral_constant<int, 1>{}); break;
        case 2: products(std::integral_constant<int, 2>{}); break;
        default: products(std::integral_constant<int, 3>{}); break;
        }
        if (wave_slow) {
#pragma unroll
            for (int I = 0; I < 4; ++I)
                if (I == R) {
                    aq[I] = dq;
                    al[I] = dl;
                }
        }
        // Causal masks; Aqk to the blob.
#pragma unroll
        for (int I = 0; I < 4; ++I) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int col = 16 * I + 4 * kg + i, row = 16 * R + m;
                if (!(col <= row)) aq[I][i] = 0.f;
                if (!(col < row)) al[I][i] = 0.f;
            }
            // Blocks (0, 2), (0, 3), (1, 2), (1, 3) lie above the causal diagonal
            // and the inference scan never copies them; the training workspace
            // (p.hs) keeps them, zero, for the backward's transposed landing.
            if (p.hs || !(R < 2 && I >= 2))
                st_q4<PK>(ws + BL::AQ + k16_block(R, I, 64) + 4 * l, pack4<PK>(aq[I]));
        }
        __syncthreads();  // all reads of sKend done; its space becomes L
        // Blocks I <= R only: the upper blocks are never read as L and serve as
        // scratch below.
#pragma unroll
        for (int I = 0; I < 4; ++I)
            if (I <= R)
                *reinterpret_cast<float4 *>(&sL[(16 * R + m) * LDF + 16 * I + 4 * kg]) =
                    make_float4(al[I][0], al[I][1], al[I][2], al[I][3]);
        __syncthreads();

        // X = (I + L)^{-1} in fp32: diagonal 16x16 blocks by forward substitution
        // (lane j = column j); the strictly-upper blocks are zero and not stored.
        auto xblk = [&](int I, int J) __attribute__((always_inline)) { return sX + (I * (I + 1) / 2 + J) * XBS; };
        if (l < 16) {
            const int j = l;
            float x[16];
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                // Four partial sums: the dependent FMA chain of row i is i / 4 long.
                // Row i of the block is read as 16-byte pieces (one LDS request per
                // four values; the products and their order are unchanged).
                float acc[4] = {(i == j) ? 1.f : 0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int q4 = 0; q4 < (i + 3) / 4; ++q4) {
                    const float4 l4 = *reinterpret_cast<const float4 *>(&sL[(16 * R + i) * LDF + 16 * R + 4 * q4]);
                    const float lv[4] = {l4.x, l4.y, l4.z, l4.w};
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        if (4 * q4 + e < i) acc[e] = fmaf(-lv[e], x[4 * q4 + e], acc[e]);
                }
                x[i] = (acc[0] + acc[1]) + (acc[2] + acc[3]);
            }
#pragma unroll
            for (int i = 0; i < 16; ++i) xblk(R, R)[i * LDB + j] = x[i];
        }
        __syncthreads();
        // Off-diagonal blocks, one sub-diagonal at a time:
        //   X_RI = -X_RR * sum_{J=I}^{R-1} L_RJ X_JI.
        // Wave R forms column I = R: besides L and the diagonal blocks it reads
        // only the blocks of its own column from earlier steps, so the steps
        // need a workgroup barrier only at the end (other waves read every
        // column afterwards).
        for (int d = 1; d <= 3; ++d) {
            if (R < 4 - d) {
                const int Rr = R + d, I = R;
                f32x4 t = zero4();
                for (int J = I; J < Rr; ++J)
                    t = mm16_f32(t, sL + (16 * Rr) * LDF + 16 * J, LDF, xblk(J, I), LDB, l);
                // Transposing scratch of wave R (<= 2): L's upper block (0, R + 1).
                float *scr = sL + 16 * (R + 1);
#pragma unroll
                for (int i = 0; i < 4; ++i) scr[(4 * kg + i) * LDF + m] = t[i];
                __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
                __builtin_amdgcn_wave_barrier();
                const f32x4 xr = mm16_f32(zero4(), xblk(Rr, Rr), LDB, scr, LDF, l);
#pragma unroll
                for (int i = 0; i < 4; ++i) xblk(Rr, I)[(4 * kg + i) * LDB + m] = -xr[i];
            }
            if (d < 3) {
                __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
                __builtin_amdgcn_wave_barrier();
            } else {
                __syncthreads();
            }
        }

        // X to the blob (row block R).
        Q xt[4];
#pragma unroll
        for (int J = 0; J < 4; ++J) {
            // Blocks above the diagonal (J > R) are zero: read the diagonal block's
            // address and select zero, so that no branch separates the reads.
            float4 xv = *reinterpret_cast<const float4 *>(xblk(R, J <= R ? J : R) + m * LDB + 4 * kg);
            if (J > R) xv = make_float4(0.f, 0.f, 0.f, 0.f);
            xt[J] = pack4<PK>(xv.x, xv.y, xv.z, xv.w);
            if (p.hs || !(R < 2 && J >= 2))  // as for Aqk above
                st_q4<PK>(ws + BL::X + k16_block(R, J, 64) + 4 * l, xt[J]);
        }
        // W^T(ct, R) = Ebar^T(ct, :) X^T(:, R): B operand X^T(J, R) is row 16R+m of
        // X, i.e. xt[J]; result lane (n, kg) holds W[16R+n][16ct+4kg+i] -- the K16
        // A-operand order of W.  Stored negated.
#pragma unroll
        for (int ct = 0; ct < NKT; ++ct) {
            f32x4 acc = zero4();
#pragma unroll
            for (int s = 0; s < 2; ++s) {
                if (2 * s <= R)
                    acc = mma2<PK>(acc, ld_q4<PK>(sEt + k16_block(ct, 2 * s, 64) + 4 * l),
                                   ld_q4<PK>(sEt + k16_block(ct, 2 * s + 1, 64) + 4 * l), xt[2 * s],
                                   xt[2 * s + 1]);
            }
            st_q4<PK>(ws + BL::WN + k16_block(R, ct, KP) + 4 * l,
                      pack4<PK>(-acc[0], -acc[1], -acc[2], -acc[3]));
        }
        if (item + static_cast<int>(gridDim.x) < items) it = prep_item(p, item + gridDim.x);
        __syncthreads();  // sX / smem1 are read up to here; the next item stages its rows there
    }
}

// Registers of the copy waves' value-row requests for one chunk: NV row
// pieces of v (CONV: the convolution window first) and NW of w.
template <typename Piece, int NV, int NW>
struct ZRows {
    Piece v[NV], w[NW];
};

// Blob units per chunk and lane for the scan's copy waves that also land z rows
// (z) and for those that only copy the blob (b): zl and bl lanes, nc units, one
// lane's z rows costing about zc units, at most maxu units per lane (two
// register sets of them are live).  Chosen so that the busier of the two roles
// has the least work; without blob-only lanes every lane takes an equal share.
struct CopySplit {
    int z, b;
};
constexpr CopySplit copy_split(int nc, int zl, int bl, int zc, int maxu)
{
    const int even = (nc + zl + bl - 1) / (zl + bl);
    if (bl == 0) return CopySplit{even, 0};
    CopySplit best{even, even};
    int best_cost = 1 << 30;
    for (int z = 1; z * zl <= nc && z <= maxu; ++z) {
        const int rem = nc - z * zl;
        const int b = rem > 0 ? (rem + bl - 1) / bl : 1;
        if (b > maxu) continue;
        const int cost = z + zc > b ? z + zc : b;
        if (cost < best_cost) {
            best_cost = cost;
            best = CopySplit{z, b};
        }
    }
    return best;
}

// ---------------------------------------------------------------------------
// Scan: one workgroup per (sequence, head, value slice of BV columns).
// ---------------------------------------------------------------------------
template <PrecKind PK, int KP, int BV, typename TI, bool TRAIN, bool SIGW = false, bool NORM = false,
          bool CONV = false>
__global__ __launch_bounds__(512) void chunk_scan_kernel(ChunkParams p, int NVB, int NP)
{
    static_assert(!CONV || (!TRAIN && sizeof(TI) == 2), "the fused convolution is a 16-bit inference prologue");
    using P = Prec<PK>;
    using st = typename P::st;
    using BL = Blob<PK, KP>;
    using Q = Q4<PK>;
    // Double-buffer the blob where two fit in LDS (16-bit storage, KP <= 128).
    constexpr bool DB = PK != PrecKind::F32 && KP <= 128;
    constexpr int NBUF = DB ? 2 : 1;
    constexpr int NKT = KP / 16, NKS = KP / 32, NCT = BV / 16;
    constexpr int U16 = static_cast<int>(BL::BYTES / 16);
    __shared__ __align__(16) st sB[NBUF][BL::SIZE];
    // z = w * v of the chunk, row-major [token][column of the slice] with a
    // 16-byte skew per row; the compute waves turn each 16-token tile into
    // their K16 B operand with one identity product.
    constexpr int LDZ = BV + 16 / static_cast<int>(sizeof(st));
    __shared__ __align__(16) st sZ[NBUF][64 * LDZ];
    // NORM: per-token sums of squares of each compute wave's 16 output columns,
    // by chunk parity.
    __shared__ float sNP[NORM ? 2 : 1][NORM ? 4 : 1][NORM ? 64 : 1];

    // XCD-aware order: all value slices of a (sequence, head) pair share
    // blockIdx % 8, hence one XCD and one L2.
    const int Lid = blockIdx.x;
    const int xcd = Lid & 7, rest = Lid >> 3;
    const int vs = rest % NVB, grp = rest / NVB;
    const int pair = 8 * grp + xcd;
    if (pair >= NP) return;
    const int H = p.H, K = p.K, V = p.V;
    const int n = pair / H, h = pair % H;

    // The first 8 - NCW waves compute (wave c owns value columns 16c..16c+15
    // of the slice); the last NCW waves only move the per-chunk blobs and z
    // from HBM to LDS.  Every wave that a slice does not need for compute
    // copies (the copies set the pace there): one compute wave and seven copy
    // waves at 16 columns, two and six at 32, four of each at 64 and with the
    // fused norm (whose per-token sums take four compute waves' slots).
    constexpr int NCW = NORM ? 4 : 8 - NCT;
    constexpr int CT = 64 * NCW;  // copy threads
    const int tid = threadIdx.x, wv = tid >> 6, l = tid & 63, m = l & 15, kg = l >> 4;
    const bool copier = wv >= 8 - NCW;
    const int ctid = tid - 64 * (8 - NCW);
    const bool active = wv < NCT;
    const int col = vs * BV + 16 * wv + m;
    const bool col_ok = active && col < V;
    // Training-mode emission: value tile vt of this wave, if inside V.
    const int VP = p.VP, vt = vs * NCT + wv;
    const bool emit = TRAIN && active && 16 * vt < V;
    const Q ident = identity_q4<PK>(l);
    // Outputs leave through transposed tiles when the operand precision is the
    // output dtype (bf16 with bf16 operands, fp32 with fp32 operands).
    constexpr bool OUT_T = (std::is_same<TI, bf16_t>::value && PK == PrecKind::BF16) ||
                           (std::is_same<TI, float>::value && PK == PrecKind::F32);
    static_assert(!NORM || (OUT_T && !TRAIN && !std::is_same<TI, float>::value),
                  "the fused gated norm is a 16-bit inference epilogue");
    // An fp32 accumulator tile (rows 4kg+i, column m) stored transposed, in
    // A-order and the MFMA operand precision (an identity product transposes it).
    auto emit_tile = [&](st *base, int64_t off, f32x4 x) __attribute__((always_inline)) {
        st_q4<PK>(base + off, pack4<PK>(mma1<PK>(zero4(), pack4<PK>(x), ident)));
    };
    int64_t bos, len;
    const int gc0 = seq_chunk_base(p, n, bos, len);
    const int nch = static_cast<int>((len + kChunk - 1) / kChunk);

    const TI *vp = static_cast<const TI *>(p.v);
    const TI *wp = static_cast<const TI *>(p.w);
    TI *op = static_cast<TI *>(p.o);
    // Whole 4-value output pieces when V and the base allow aligned vector stores.
    const bool o_vec = (V % 4) == 0 && (reinterpret_cast<uintptr_t>(op) % (4 * sizeof(TI))) == 0;
    const st *wsb = static_cast<const st *>(p.ws);
    auto blob = [&](int gci) {
        return reinterpret_cast<const u32x4 *>(wsb + (static_cast<int64_t>(gci) * H + h) * BL::SIZE);
    };
    // Blocks (0, 2), (0, 3), (1, 2), (1, 3) of X and of Aqk lie above the causal
    // diagonal and are never read here (the products use blocks (R, J) with
    // J < 2 or J <= R, see pair_off), so the double-buffered per-chunk copies
    // skip them: compact unit c maps to blob unit cmap_unit(c), which steps over
    // the four skipped runs of 2 * BU units.  With c in [b0 + wd u, b0 + wd u +
    // wd) at unrolled step u, each threshold test folds to a constant except in
    // the one step it falls in.
    constexpr int BU = 256 * static_cast<int>(sizeof(st)) / 16;  // units per 16x16 block
    constexpr int AQU = static_cast<int>(BL::AQ * static_cast<int64_t>(sizeof(st)) / 16);
    constexpr int NC = U16 - 8 * BU;
    auto cmap_unit = [](int c, int b0, int wd, int u) __attribute__((always_inline)) {
        auto ge = [&](int t) __attribute__((always_inline)) {
            return t <= b0 + wd * u ? 1 : (t >= b0 + wd * u + wd ? 0 : (c >= t ? 1 : 0));
        };
        return c + 2 * BU * (ge(2 * BU) + ge(4 * BU) + ge(AQU - 2 * BU) + ge(AQU));
    };
    // ASSIST (64-column inference slices, where the four copy waves set the
    // pace and the compute waves wait at the step barrier): each compute lane
    // also copies PFA units of the next chunk, the last NCA compact units,
    // requested before its products and landed after them, ahead of the
    // output stores (so that the wait for them covers no store).
    constexpr bool ASSIST = DB && NCT == 4 && NCW == 4 && !TRAIN && !NORM && !CONV;
    constexpr int PFA = ASSIST ? 4 : 0;
    constexpr int NCA = 256 * PFA;
    constexpr int NCC = NC - NCA;  // compact units the copy waves move
    // Whole blob into LDS, CB requests in flight per copy wave lane at a time
    // (a plain element loop would wait for each load before its store).
    auto copy_blob = [&](int gci, int buf) __attribute__((always_inline)) {
        constexpr int CB = 8;
        const u32x4 *src = blob(gci);
        u32x4 *dst = reinterpret_cast<u32x4 *>(sB[buf]);
        for (int u0 = 0; u0 < U16; u0 += CT * CB) {
            u32x4 t[CB];
#pragma unroll
            for (int c = 0; c < CB; ++c) {
                const int u = u0 + ctid + CT * c;
                t[c] = src[u < U16 ? u : U16 - 1];
            }
#pragma unroll
            for (int c = 0; c < CB; ++c) {
                const int u = u0 + ctid + CT * c;
                if (u < U16) dst[u] = t[c];
            }
        }
    };
    // Copy waves: z = w * v of chunk jc for this value slice, row-major in LDS
    // (zero past the sequence end and past V).  issue_z requests the raw rows
    // (16-byte loads); land_z forms z and stores it with one 16-byte LDS write
    // per row piece, so the two can sit a chunk apart.
    const int v0 = vs * BV;
    constexpr int EPV = 16 / static_cast<int>(sizeof(TI));  // values per 16-byte load
    constexpr int ZT = kChunk * BV / EPV;                    // loads per tensor per chunk
    constexpr int NZT = (ZT + CT - 1) / CT;
    // Whole 16-byte row pieces for every row of this slice (uniform per workgroup).
    const bool zfast = (V % EPV) == 0 && v0 + BV <= V;
    // CONV: lane ctid takes row piece ctid % PPR of NZC consecutive tokens
    // (plus the three rows before them, the convolution window) instead of
    // tokens CT a / PPR apart, so the window rows are shared by its tokens.
    // Slices narrower than 64 use 8-byte pieces (CW = 4 channels), so that
    // more copy lanes share the convolution arithmetic.
    constexpr int CW = BV >= 64 ? EPV : EPV / 2;  // channels per CONV piece
    constexpr int PPR = BV / CW;                  // CONV pieces per token
    constexpr int NZC = (kChunk * PPR + CT - 1) / CT;
    constexpr int NH = 3;                         // window rows before a lane's first token
    using CPiece = std::conditional_t<CW == EPV, u32x4, uint2>;
    using ZRaw = std::conditional_t<CONV, ZRows<CPiece, NZC + NH, NZC>, ZRows<u32x4, NZT, NZT>>;
    auto chunk_rows = [&](int jc, int64_t &t0, int &lc) __attribute__((always_inline)) {
        t0 = bos + static_cast<int64_t>(jc) * kChunk;
        const int64_t rem = len - static_cast<int64_t>(jc) * kChunk;
        lc = rem < kChunk ? static_cast<int>(rem) : kChunk;
    };
    // Slices that do not allow 16-byte loads (ragged V, a slice past V) are
    // assembled element by element here, zero-filled, so that land_z never
    // touches global memory: a load there would make its wait also cover the
    // prefetch of the chunk after.
    using Raw = std::conditional_t<sizeof(TI) == 2, uint16_t, uint32_t>;
    struct RawRow {
        Raw e[EPV];
    };
    // CONV taps of the slice's columns, [column][4] 16-bit values, in LDS:
    // each copy lane stores the taps of its own EPV columns (lanes sharing
    // columns store the same values) and reads back only those, so no
    // barrier is needed.
    const int cz = CW * (ctid % PPR), tz0 = NZC * (ctid / PPR);
    const bool zlane = copier && tz0 < kChunk;
    // Copy lanes with z rows to land (the first ZLANES), and the whole waves
    // holding them (ZL): with seven copy waves some have none, and those take
    // a larger share of the blob instead.
    constexpr int ZLANES = CONV ? PPR * ((kChunk + NZC - 1) / NZC) : (ZT < CT ? ZT : CT);
    constexpr int ZL = (ZLANES + 63) / 64 * 64 < CT ? (ZLANES + 63) / 64 * 64 : CT;
    // WSTAGE (CONV with blob-only copy waves): those waves also request the w
    // rows, activate them (SIGW) and stage them in sW by chunk parity a step
    // before the z lanes form z = v * w, which then read w from LDS.
    constexpr bool WSTAGE = CONV && DB && ZL < CT;
    __shared__ __align__(16) TI sW[WSTAGE ? 2 : 1][WSTAGE ? kChunk * BV : 8];
    __shared__ __align__(16) TI sZT[CONV ? BV * 4 : 8];
    if constexpr (CONV) {
        if (copier) {
            const u32x4 *tp = reinterpret_cast<const u32x4 *>(static_cast<const TI *>(p.conv_w[2]) +
                                                              (static_cast<int64_t>(h) * V + v0 + cz) * 4);
            u32x4 t4[CW / 2];
#pragma unroll
            for (int i = 0; i < CW / 2; ++i) t4[i] = tp[i];
#pragma unroll
            for (int i = 0; i < CW / 2; ++i) reinterpret_cast<u32x4 *>(sZT + 4 * cz)[i] = t4[i];
        }
    }
    // wrows (CONV): this call also requests the lane's w rows (else they are
    // staged in sW by other copy waves).
    auto issue_z = [&](auto fastc, ZRaw &r, int jc, auto wrows) __attribute__((always_inline)) {
        int64_t t0;
        int lc;
        chunk_rows(jc, t0, lc);
        if constexpr (CONV) {
            // Raw v rows (token row stride ldv); window rows before the
            // sequence start and rows of dead lanes load the chunk's first
            // row and are zeroed when landed.
            const int64_t colv = static_cast<int64_t>(h) * V + v0 + cz;
#pragma unroll
            for (int j = 0; j < NZC + NH; ++j) {
                const int tok = tz0 - NH + j;
                const bool ok = zlane && tok < lc && kChunk * jc + tok >= 0;
                r.v[j] = *reinterpret_cast<const CPiece *>(vp + (t0 + (ok ? tok : 0)) * p.ldv + colv);
            }
            if constexpr (decltype(wrows)::value) {
#pragma unroll
                for (int a = 0; a < NZC; ++a) {
                    const int tok = tz0 + a;
                    const bool live = zlane && tok < lc;
                    r.w[a] = *reinterpret_cast<const CPiece *>(wp + ((t0 + (live ? tok : 0)) * H + h) * V + v0 + cz);
                }
            }
        } else if constexpr (decltype(fastc)::value) {
            // Dead lanes load the chunk's first row piece (always valid) and
            // are zeroed when landed: a select on the loaded value here would
            // make the request wait for its own data.
#pragma unroll
            for (int a = 0; a < NZT; ++a) {
                const int task = ctid + CT * a;
                const int tok = task / (BV / EPV), c = EPV * (task % (BV / EPV));
                const bool live = task < ZT && tok < lc;
                const int64_t off = live ? ((t0 + tok) * H + h) * V + v0 + c : (t0 * H + h) * V + v0;
                r.v[a] = *reinterpret_cast<const u32x4 *>(vp + off);
                r.w[a] = *reinterpret_cast<const u32x4 *>(wp + off);
            }
        } else {
#pragma unroll
            for (int a = 0; a < NZT; ++a) {
                const int task = ctid + CT * a;
                const int tok = task / (BV / EPV), c = EPV * (task % (BV / EPV));
                const bool live = task < ZT && tok < lc;
                const int64_t off = ((t0 + tok) * H + h) * V + v0 + c;
                RawRow rv, rw;
#pragma unroll
                for (int e = 0; e < EPV; ++e) {
                    const bool in = live && v0 + c + e < V;
                    rv.e[e] = in ? reinterpret_cast<const Raw *>(vp)[off + e] : Raw(0);
                    rw.e[e] = in ? reinterpret_cast<const Raw *>(wp)[off + e] : Raw(0);
                }
                r.v[a] = __builtin_bit_cast(u32x4, rv);
                r.w[a] = __builtin_bit_cast(u32x4, rw);
            }
        }
    };
    // SIGW (GDN2_FLAG_SIGMOID_BW, inference only): w holds the logits.
    // wlds (CONV): w of chunk jc is read from sW, staged (and activated) by
    // other copy waves, instead of from this lane's registers.
    auto land_z = [&](const ZRaw &r, int jc, int buf, auto wlds) __attribute__((always_inline)) {
        int64_t t0;
        int lc;
        chunk_rows(jc, t0, lc);
        st *dst = sZ[buf];
        static_assert(EPV * sizeof(st) == 16, "one z row piece is one 16-byte LDS store");
        if constexpr (CONV) {
            // v = act(round(sum_j tap[c][j] * v_raw[t-3+j])) in the separate
            // convolution pass's order and roundings, then z = v * w as below.
            if (!zlane) return;
            bool hok[NH];
#pragma unroll
            for (int j = 0; j < NH; ++j) hok[j] = kChunk * jc + tz0 - NH + j >= 0;
            const bool silu = p.conv_silu != 0;
            CPiece wl[NZC];
            if constexpr (decltype(wlds)::value) {
#pragma unroll
                for (int a = 0; a < NZC; ++a)
                    wl[a] = *reinterpret_cast<const CPiece *>(&sW[jc & 1][(tz0 + a) * BV + cz]);
            }
            st zr[NZC][CW];
            // Channel by channel, so that only one column's window is unpacked
            // at a time.
#pragma unroll
            for (int e = 0; e < CW; ++e) {
                const uint2 t2 = reinterpret_cast<const uint2 *>(sZT + 4 * cz)[e];
                const TI *tw = reinterpret_cast<const TI *>(&t2);
                float x[NZC + NH];
#pragma unroll
                for (int j = 0; j < NZC + NH; ++j) {
                    const float xv = io<TI>::ld(reinterpret_cast<const TI *>(&r.v[j]), e);
                    x[j] = (j >= NH || hok[j < NH ? j : 0]) ? xv : 0.f;
                }
#pragma unroll
                for (int a = 0; a < NZC; ++a) {
                    float acc = 0.f;
#pragma unroll
                    for (int jj = 0; jj < 4; ++jj) acc = fmaf(io<TI>::ld(tw, jj), x[a + jj], acc);
                    float vc = round_to<TI>(acc + 0.0f);
                    if (silu) vc = round_to<TI>(silu_f32(vc));
                    float wv_;
                    if constexpr (decltype(wlds)::value) {
                        wv_ = io<TI>::ld(reinterpret_cast<const TI *>(&wl[a]), e);
                    } else {
                        const TI *rw = reinterpret_cast<const TI *>(&r.w[a]);
                        wv_ = SIGW ? round_to<TI>(sigmoid_f(io<TI>::ld(rw, e))) : io<TI>::ld(rw, e);
                    }
                    zr[a][e] = P::from_f32(tz0 + a < lc ? vc * wv_ : 0.f);
                }
            }
#pragma unroll
            for (int a = 0; a < NZC; ++a)
                *reinterpret_cast<CPiece *>(dst + (tz0 + a) * LDZ + cz) = __builtin_bit_cast(CPiece, zr[a]);
            return;
        }
#pragma unroll
        for (int a = 0; a < NZT; ++a) {
            const int task = ctid + CT * a;
            if (task >= ZT) continue;
            const int tok = task / (BV / EPV), c = EPV * (task % (BV / EPV));
            const TI *rv = reinterpret_cast<const TI *>(&r.v[a]);
            const TI *rw = reinterpret_cast<const TI *>(&r.w[a]);
            st zr[EPV];
#pragma unroll
            for (int e = 0; e < EPV; ++e) {
                // Zero past the sequence end (and past V, zero-filled by issue_z);
                // w given as logits is activated here and rounded to the input
                // dtype, as the module's torch sigmoid of w_proj(x) is (gdn2.py:865).
                const float wv_ = SIGW ? round_to<TI>(sigmoid_f(io<TI>::ld(rw, e))) : io<TI>::ld(rw, e);
                const float z = tok < lc ? io<TI>::ld(rv, e) * wv_ : 0.f;
                zr[e] = P::from_f32(z);
            }
            *reinterpret_cast<u32x4 *>(dst + tok * LDZ + c) = __builtin_bit_cast(u32x4, zr);
        }
    };

    // State columns of this wave: S[kt] holds rows 16kt + 4kg + i, column col.
    f32x4 S[NKT];
#pragma unroll
    for (int kt = 0; kt < NKT; ++kt) {
        S[kt] = zero4();
        if (p.h0 && col_ok) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int row = 16 * kt + 4 * kg + i;
                if (row < K) S[kt][i] = p.h0[state_index(p.flags, n, h, row, col, H, K, V)];
            }
        }
    }

    // Copy waves and compute waves run separate loops with the
    // same barrier schedule -- one barrier after the prologue, one per chunk,
    // and in the single-buffer case one more per reload -- so the copy waves'
    // prefetch registers never overlap the compute waves' live ranges.
    if (copier) {
        // The copy loop is instantiated once for 16-byte value rows and once
        // for the element-wise rows of ragged slices (uniform per workgroup),
        // so that each loop body is straight-line and the compiler's
        // load-completion waits stay exact.
        auto copy_loop = [&](auto fastc, auto zrole) __attribute__((always_inline)) {
            // zrole: this wave lands z rows (and its share of the blob); the
            // other copy waves only move blob units.
            constexpr bool ZR = decltype(zrole)::value;
            auto iz = [&](ZRaw &r, int j) __attribute__((always_inline)) {
                if constexpr (ZR) issue_z(fastc, r, j, std::bool_constant<!WSTAGE>{});
            };
            auto lz = [&](const ZRaw &r, int j, int b) __attribute__((always_inline)) {
                if constexpr (ZR) land_z(r, j, b, std::bool_constant<WSTAGE>{});
            };
            ZRaw zA, zB;
            if (nch > 0) {
                copy_blob(gc0, 0);
                issue_z(fastc, zA, 0, std::true_type{});
                land_z(zA, 0, 0, std::false_type{});
            }
            // Lanes without z rows of their own skip land_z; wait for their
            // requests too, so that no request of chunk 0 is left outstanding
            // into the prefetch below.
            wait_vm_newest<0>();
            if constexpr (DB) {
                // Compact units [B0 + WD u, B0 + WD u + WD) at step u of this
                // role's lanes: the z lanes take the first SPL.z steps of ZL
                // units, the blob-only lanes the rest, CT - ZL units a step.
                // A lane's z rows cost about 24 blob units with the convolution
                // (measured with s_memtime stamps in the copy waves: ~1.85 K
                // cycles against ~65 per unit), one without it.
                // At most 20 units per lane, 16 with the convolution at d_k > 64
                // (where the z lanes' window and the staged gate rows also hold
                // registers).
                constexpr CopySplit SPL = copy_split(NCC, ZL, CT - ZL, CONV ? 24 : 1, CONV && KP > 64 ? 16 : 20);
                constexpr int PFC = ZR ? SPL.z : SPL.b;
                constexpr int WD = ZR ? ZL : CT - ZL;
                constexpr int B0 = ZR ? 0 : ZL * SPL.z;
                static_assert(ZL * SPL.z + (CT - ZL) * SPL.b >= NCC, "every blob unit has a copy lane");
                const int rl = ZR ? ctid : ctid - ZL;
                u32x4 pA[PFC], pB[PFC];
                auto issue = [&](u32x4 (&dst)[PFC], int gci) __attribute__((always_inline)) {
                    const u32x4 *src = blob(gci);
#pragma unroll
                    for (int u = 0; u < PFC; ++u) {
                        const int c = B0 + rl + WD * u;
                        dst[u] = src[cmap_unit(c < NCC ? c : NCC - 1, B0, WD, u)];
                    }
                };
                auto land = [&](const u32x4 (&src)[PFC], int buf) __attribute__((always_inline)) {
                    u32x4 *dst = reinterpret_cast<u32x4 *>(sB[buf]);
#pragma unroll
                    for (int u = 0; u < PFC; ++u) {
                        const int c = B0 + rl + WD * u;
                        if (c < NCC) dst[cmap_unit(c, B0, WD, u)] = src[u];
                    }
                };
                // Chunk jc+1 lands in the idle buffer at step jc.  Unrolled by
                // two so that the register sets A / B swap roles at compile time.
                //  * DEEP (training emission, or value slices narrower than 64
                //    so that several workgroups share each blob): chunk jc+1 was
                //    requested two steps earlier and its register set is reused
                //    for chunk jc+3 right after landing, so every request has two
                //    chunk steps of memory latency to hide (training forward at
                //    config 4: 0.69 -> 0.62 ms).
                //  * otherwise chunk jc+2 is requested before chunk jc+1 lands,
                //    one step of latency per request, which measured faster for
                //    64-column slices without emission (0.241 vs 0.251 ms at
                //    config 1).
                //  * CONV at KP = 128 (the v rows' convolution window takes more
                //    registers than the copy waves have left there): one step,
                //    with a single z register set, refilled with chunk jc+2 right
                //    after chunk jc+1 lands from it.
                constexpr bool ONEZ = CONV && KP > 64;
                constexpr bool DEEP = !ONEZ && (TRAIN || BV < 64);
                // Requests are issued unconditionally, past the last chunk for
                // the last chunk again (data unused): with a request skipped on
                // some paths the compiler cannot count the loads issued after
                // the ones being landed and waits for all of them, which makes
                // the prefetch synchronous.
                auto cl = [&](int j) __attribute__((always_inline)) { return j < nch ? j : nch - 1; };
                ZRaw &zC = ONEZ ? zA : zB;  // the set holding chunk jc+2 at the second half
                // WSTAGE, blob-only waves: w rows of chunk j in 16-byte pieces,
                // staged in sW[j & 1] (activated) two half-steps after their
                // request: at step c (landing chunk c+1) the lanes stage chunk
                // c+2, read by the z lanes at step c+1 after a barrier.  The
                // z lanes read sW[(c+1) & 1] at step c, never the buffer that
                // is being staged.
                constexpr bool WB = !ZR && WSTAGE;
                constexpr int WT = kChunk * BV / EPV;
                constexpr int NWT = WB ? (WT + (CT - ZL) - 1) / (CT - ZL) : 1;
                u32x4 wA[NWT], wB[NWT];
                auto issue_w = [&](u32x4 (&d)[NWT], int j) __attribute__((always_inline)) {
                    if constexpr (WB) {
                        int64_t t0;
                        int lc;
                        chunk_rows(j, t0, lc);
#pragma unroll
                        for (int a = 0; a < NWT; ++a) {
                            const int task = rl + (CT - ZL) * a;
                            const int tok = task / (BV / EPV), c = EPV * (task % (BV / EPV));
                            const bool live = task < WT && tok < lc;
                            const int64_t off = live ? ((t0 + tok) * H + h) * V + v0 + c : (t0 * H + h) * V + v0;
                            d[a] = *reinterpret_cast<const u32x4 *>(wp + off);
                        }
                    }
                };
                auto land_w = [&](const u32x4 (&d)[NWT], int j) __attribute__((always_inline)) {
                    if constexpr (WB) {
#pragma unroll
                        for (int a = 0; a < NWT; ++a) {
                            const int task = rl + (CT - ZL) * a;
                            if (task >= WT) continue;
                            const int tok = task / (BV / EPV), c = EPV * (task % (BV / EPV));
                            const TI *x = reinterpret_cast<const TI *>(&d[a]);
                            TI y[EPV];
#pragma unroll
                            for (int e = 0; e < EPV; ++e) {
                                // As the z lanes would: the module's torch sigmoid,
                                // rounded to the input dtype (gdn2.py:865).
                                const float w = io<TI>::ld(x, e);
                                io<TI>::st(y, e, SIGW ? round_to<TI>(sigmoid_f(w)) : w);
                            }
                            *reinterpret_cast<u32x4 *>(&sW[j & 1][tok * BV + c]) = __builtin_bit_cast(u32x4, y);
                        }
                    }
                };
                // Requests of one chunk and role (blob units, z rows or staged w
                // rows), all unconditional for 16-byte rows.  Before a set lands,
                // the only newer requests are the other set's, so an explicit
                // count waits for exactly the set being landed.  It can only add
                // waiting; the compiler's own counts stay exact as long as every
                // path into the loop header has issued the sets in one order.
                constexpr int NREQ = PFC + (!ZR ? (WB ? NWT : 0) : CONV ? NZC + NH + (WSTAGE ? 0 : NZC) : 2 * NZT);
                constexpr bool EXACT = decltype(fastc)::value && (!ONEZ || !ZR);
                // The sets are requested here in the order the loop requests
                // them (the compiler merges the two paths into its header).
                if (nch > 0) {
                    if constexpr (WB) {
                        issue_w(wA, cl(1));
                        land_w(wA, 1);
                    }
                    if constexpr (DEEP) {
                        issue(pA, gc0 + cl(1));
                        iz(zA, cl(1));
                        issue_w(wA, cl(2));
                        issue(pB, gc0 + cl(2));
                        iz(zB, cl(2));
                        issue_w(wB, cl(3));
                    } else {
                        issue_w(wA, cl(2));
                        issue(pA, gc0 + cl(1));
                        iz(zA, cl(1));
                        issue_w(wB, cl(3));
                    }
                }
                __syncthreads();
                // Pairs of chunk steps, then the last step of an odd count, which
                // has nothing left to land: the loop has no exit between its two
                // halves, so every path into its header has issued both sets in
                // the same order and the compiler's load counts stay exact.
                int jc = 0;
                for (; jc + 1 < nch; jc += 2) {
                    if (!DEEP) {
                        issue(pB, gc0 + cl(jc + 2));
                        if (!ONEZ) iz(zB, cl(jc + 2));
                    }
                    if constexpr (EXACT) wait_vm_newest<NREQ>();
                    lz(zA, jc + 1, 1);
                    if (ONEZ) iz(zA, cl(jc + 2));
                    land(pA, 1);
                    land_w(wA, jc + 2);
                    if (DEEP) {
                        issue(pA, gc0 + cl(jc + 3));
                        iz(zA, cl(jc + 3));
                    }
                    issue_w(wA, cl(jc + 4));
                    __syncthreads();
                    if (!DEEP) {
                        issue(pA, gc0 + cl(jc + 3));
                        if (!ONEZ) iz(zA, cl(jc + 3));
                    }
                    if constexpr (EXACT) wait_vm_newest<NREQ>();
                    if (jc + 2 < nch) lz(zC, jc + 2, 0);
                    if (ONEZ) iz(zA, cl(jc + 3));
                    if (jc + 2 < nch) land(pB, 0);
                    land_w(wB, jc + 3);
                    if (DEEP) {
                        issue(pB, gc0 + cl(jc + 4));
                        iz(zB, cl(jc + 4));
                    }
                    issue_w(wB, cl(jc + 5));
                    __syncthreads();
                }
                if (jc < nch) __syncthreads();
            } else {
                __syncthreads();
                for (int jc = 0; jc < nch; ++jc) {
                    __syncthreads();
                    if (jc + 1 < nch) {
                        copy_blob(gc0 + jc + 1, 0);
                        iz(zA, jc + 1);
                        lz(zA, jc + 1, 0);
                        __syncthreads();
                    }
                }
            }
        };
        auto by_role = [&](auto fastc) __attribute__((always_inline)) {
            if constexpr (ZL < CT) {
                if (ctid < ZL)
                    copy_loop(fastc, std::true_type{});
                else
                    copy_loop(fastc, std::false_type{});
            } else {
                copy_loop(fastc, std::true_type{});
            }
        };
        if constexpr (CONV)
            by_role(std::true_type{});  // whole 16-byte row pieces (checked by the host)
        else if (zfast)
            by_role(std::true_type{});
        else
            by_role(std::false_type{});
    } else {
        // NORM (gated output norm, BV == V): chunk jc's rounded, transposed
        // outputs and its gate rows stay in registers until the barrier that
        // ends step jc.  Each compute wave has then written its per-token sums
        // of squares to sNP[jc & 1], and the chunk is normalised and stored at
        // the start of step jc + 1 (the last chunk after the loop).  The sums
        // follow gated_rmsnorm_vec_kernel's order (8 consecutive columns per
        // partial, then a pairwise tree), so the result equals the separate
        // norm pass bit for bit.
        Q otr[4], zq[4];
        float nwv[4] = {0.f, 0.f, 0.f, 0.f};
        const int c0n = 16 * wv + 4 * kg;  // this lane's 4 output columns (BV == V)
        if constexpr (NORM) {
            if (active) {
#pragma unroll
                for (int i = 0; i < 4; ++i) nwv[i] = io<TI>::ld(static_cast<const TI *>(p.nw), c0n + i);
            }
        }
        auto issue_gate = [&](int64_t t0n, int lcn) __attribute__((always_inline)) {
            const TI *zp = static_cast<const TI *>(p.z);
#pragma unroll
            for (int rt = 0; rt < 4; ++rt) {
                const int tok = 16 * rt + m;  // rows past the chunk read its first row (unused)
                const int64_t row = t0n + (tok < lcn ? tok : 0);
                zq[rt] = ld_q4<PK>(reinterpret_cast<const st *>(zp + row * p.ldz + static_cast<int64_t>(h) * V + c0n));
            }
        };
        auto finish_norm = [&](int jn, int64_t t0n, int lcn) __attribute__((always_inline)) {
            const float *P = &sNP[jn & 1][0][0];
#pragma unroll
            for (int rt = 0; rt < 4; ++rt) {
                const int tok = 16 * rt + m;
                float tot;
                if constexpr (NCT >= 4)
                    tot = (P[tok] + P[64 + tok]) + (P[128 + tok] + P[192 + tok]);
                else if constexpr (NCT == 2)
                    tot = P[tok] + P[64 + tok];
                else
                    tot = P[tok];
                const float var = round_to<TI>(tot / static_cast<float>(V));
                const float inv = round_to<TI>(rsqrtf(round_to<TI>(var + p.eps)));
                float x[4], zz[4], out[4];
                unpack4<PK>(otr[rt], x);
                unpack4<PK>(zq[rt], zz);
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const float a = round_to<TI>(x[i] * inv);
                    const float gz = round_to<TI>(silu_f32(zz[i]));
                    out[i] = round_to<TI>(round_to<TI>(a * nwv[i]) * gz);
                }
                if (tok < lcn)
                    st_q4<PK>(reinterpret_cast<st *>(op + ((t0n + tok) * H + h) * V + c0n),
                              pack4<PK>(out[0], out[1], out[2], out[3]));
            }
        };
        __syncthreads();
        for (int jc = 0; jc < nch; ++jc) {
            const int buf = DB ? (jc & 1) : 0;
            if (active) {
            const st *Bk = sB[buf];
            // ASSIST: this lane's units of chunk jc+1 (the last chunk again past
            // the end, data unused), requested before the products so that they
            // hide the latency.
            u32x4 pa[PFA > 0 ? PFA : 1];
            if constexpr (ASSIST) {
                const u32x4 *src = blob(gc0 + (jc + 1 < nch ? jc + 1 : nch - 1));
#pragma unroll
                for (int u = 0; u < PFA; ++u) {
                    const int c = NCC + tid + 256 * u;
                    pa[u] = src[cmap_unit(c < NC ? c : NC - 1, NCC, 256, u)];
                }
            }
            const int64_t t0 = bos + static_cast<int64_t>(jc) * kChunk;
            const int64_t rem = len - static_cast<int64_t>(jc) * kChunk;
            const int lc = rem < kChunk ? static_cast<int>(rem) : kChunk;
            if constexpr (NORM) {
                if (jc > 0) {
                    const int64_t rp = len - static_cast<int64_t>(jc - 1) * kChunk;
                    finish_norm(jc - 1, t0 - kChunk, rp < kChunk ? static_cast<int>(rp) : kChunk);
                }
                issue_gate(t0, lc);
            }

            // Training mode: this chunk's start state, A-order tiles (kt, vt).
            if constexpr (TRAIN) if (emit) {
                st *hsb = static_cast<st *>(p.hs) + (static_cast<int64_t>(gc0 + jc) * H + h) * (KP * VP);
#pragma unroll
                for (int kt = 0; kt < NKT; ++kt) emit_tile(hsb, k16_block(kt, vt, VP) + 4 * l, S[kt]);
            }

            // z = w * v as B operand (contraction over tokens): token tile kt
            // read row-major (lane (m, kg): token 16kt+m, columns 4kg..4kg+3 of
            // this wave's 16) and transposed by the identity product, whose
            // accumulator holds tokens 4kg+i of column m -- the B-operand order.
            Q zf[4];
#pragma unroll
            for (int kt = 0; kt < 4; ++kt)
                zf[kt] = pack4<PK>(mma1<PK>(zero4(), ld_q4<PK>(sZ[buf] + (16 * kt + m) * LDZ + 16 * wv + 4 * kg),
                                            ident));
            Q sf[NKT];
#pragma unroll
            for (int kt = 0; kt < NKT; ++kt) sf[kt] = pack4<PK>(S[kt]);

            // The chunk's products run as 12 steps -- U for token blocks 0-3,
            // O for token blocks 0-3, the state update for pairs of key tiles
            // -- whose LDS A operands are read one step ahead into a second
            // register set (sched_barrier keeps that order), so the MFMAs do
            // not wait on LDS latency.  Outputs and training tiles are stored
            // after the last step.
            f32x4 ua[4], oa[4];
            Q uf[4];
            const float *gl = reinterpret_cast<const float *>(Bk + BL::GL);
            constexpr int NSU = 4, NSO = 4, NSS = (NKT + 1) / 2, NSTEP = NSU + NSO + NSS;
            constexpr int MAXP = 2 + NKS > 4 ? 2 + NKS : 4;  // operand pairs per step
            // Pair j of step st: blob offsets of its two K16 A blocks (or -1).
            auto pair_off = [](int st_, int j, int &o0, int &o1) __attribute__((always_inline)) {
                o0 = o1 = -1;
                if (st_ < NSU + NSO) {
                    const int rt = st_ % 4;
                    const bool isu = st_ < NSU;
                    if (j < NKS) {  // W (U) or Qbar (O) against the state
                        const int base = isu ? BL::WN : BL::QB;
                        o0 = base + k16_block(rt, 2 * j, KP);
                        o1 = base + k16_block(rt, 2 * j + 1, KP);
                    } else if (j - NKS < 2 && 2 * (j - NKS) <= rt) {  // X (U) or Aqk (O), causal
                        const int base = isu ? BL::X : BL::AQ;
                        o0 = base + k16_block(rt, 2 * (j - NKS), 64);
                        o1 = base + k16_block(rt, 2 * (j - NKS) + 1, 64);
                    }
                } else {
                    const int kt = 2 * (st_ - NSU - NSO) + j / 2, sx = j % 2;
                    if (j < 4 && kt < NKT) {
                        o0 = BL::KT + k16_block(kt, 2 * sx, 64);
                        o1 = BL::KT + k16_block(kt, 2 * sx + 1, 64);
                    }
                }
            };
            auto load_step = [&](int st_, Q (&buf)[MAXP][2], float4 (&gb)[2]) __attribute__((always_inline)) {
                if (st_ >= NSU + NSO) {
#pragma unroll
                    for (int hh = 0; hh < 2; ++hh) {
                        const int kt = 2 * (st_ - NSU - NSO) + hh;
                        if (kt < NKT) gb[hh] = *reinterpret_cast<const float4 *>(gl + 16 * kt + 4 * kg);
                    }
                }
#pragma unroll
                for (int j = 0; j < MAXP; ++j) {
                    int o0, o1;
                    pair_off(st_, j, o0, o1);
                    if (o0 >= 0) {
                        buf[j][0] = ld_q4<PK>(Bk + o0 + 4 * l);
                        buf[j][1] = ld_q4<PK>(Bk + o1 + 4 * l);
                    }
                }
            };
            auto run_step = [&](int st_, const Q (&buf)[MAXP][2], const float4 (&gb)[2]) __attribute__((always_inline)) {
                if (st_ < NSU + NSO) {
                    const int rt = st_ % 4;
                    const bool isu = st_ < NSU;
                    f32x4 acc = zero4();
#pragma unroll
                    for (int j = 0; j < MAXP; ++j) {
                        int o0, o1;
                        pair_off(st_, j, o0, o1);
                        if (o0 < 0) continue;
                        if (j < NKS) {
                            acc = mma2<PK>(acc, buf[j][0], buf[j][1], sf[2 * j], sf[2 * j + 1]);
                        } else {
                            const int sx = j - NKS;
                            acc = isu ? mma2<PK>(acc, buf[j][0], buf[j][1], zf[2 * sx], zf[2 * sx + 1])
                                      : mma2<PK>(acc, buf[j][0], buf[j][1], uf[2 * sx], uf[2 * sx + 1]);
                        }
                    }
                    if (isu) {
                        ua[rt] = acc;
                        uf[rt] = pack4<PK>(acc);
                    } else {
                        oa[rt] = acc;
                    }
                } else {
#pragma unroll
                    for (int hh = 0; hh < 2; ++hh) {
                        const int kt = 2 * (st_ - NSU - NSO) + hh;
                        if (kt >= NKT) continue;
                        const float4 gv = gb[hh];
                        S[kt][0] *= gv.x;
                        S[kt][1] *= gv.y;
                        S[kt][2] *= gv.z;
                        S[kt][3] *= gv.w;
                        S[kt] = mma2<PK>(S[kt], buf[2 * hh][0], buf[2 * hh][1], uf[0], uf[1]);
                        S[kt] = mma2<PK>(S[kt], buf[2 * hh + 1][0], buf[2 * hh + 1][1], uf[2], uf[3]);
                    }
                }
            };
            {
                Q bufA[MAXP][2], bufB[MAXP][2];
                float4 gA[2], gB[2];
                load_step(0, bufA, gA);
#pragma unroll
                for (int st_ = 0; st_ < NSTEP; st_ += 2) {
                    if (st_ + 1 < NSTEP) load_step(st_ + 1, bufB, gB);
                    __builtin_amdgcn_sched_barrier(0);
                    run_step(st_, bufA, gA);
                    __builtin_amdgcn_sched_barrier(0);
                    if (st_ + 1 < NSTEP) {
                        if (st_ + 2 < NSTEP) load_step(st_ + 2, bufA, gA);
                        __builtin_amdgcn_sched_barrier(0);
                        run_step(st_ + 1, bufB, gB);
                        __builtin_amdgcn_sched_barrier(0);
                    }
                }
            }
            // ASSIST: land this lane's units of chunk jc+1 before the output
            // stores, so that the wait covers no store.
            if constexpr (ASSIST) {
                if (jc + 1 < nch) {
                    u32x4 *dst = reinterpret_cast<u32x4 *>(sB[buf ^ 1]);
#pragma unroll
                    for (int u = 0; u < PFA; ++u) {
                        const int c = NCC + tid + 256 * u;
                        if (c < NC) dst[cmap_unit(c, NCC, 256, u)] = pa[u];
                    }
                }
            }
            if constexpr (OUT_T) {
                // Each O tile transposed by an identity product (exact: the
                // values are rounded to the output dtype once, by the first
                // pack), so lane (m, kg) holds token 16rt+m, columns 4kg..4kg+3
                // and stores them with one 8-byte (bf16) or 16-byte (fp32)
                // access instead of four 2- or 4-byte ones.
                const int c0 = vs * BV + 16 * wv + 4 * kg;
                const bool vec = o_vec && c0 + 4 <= V;
                // All four transposes are issued before the first store, so that
                // their latencies overlap instead of each one stalling its store.
                Q trs[4];
#pragma unroll
                for (int rt = 0; rt < 4; ++rt) trs[rt] = pack4<PK>(mma1<PK>(zero4(), pack4<PK>(oa[rt]), ident));
#pragma unroll
                for (int rt = 0; rt < 4; ++rt) {
                    const Q tr = trs[rt];
                    if constexpr (NORM) {
                        // Rounded squares summed in order over this lane's 4
                        // columns, continuing the left neighbour's 4 (lanes kg
                        // and kg ^ 1 hold 8 consecutive columns), then the two
                        // 8-column partials of the wave's 16 columns added.
                        otr[rt] = tr;
                        float x[4], r[4];
                        unpack4<PK>(tr, x);
#pragma unroll
                        for (int i = 0; i < 4; ++i) r[i] = round_to<TI>(x[i] * x[i]);
                        const float left = __shfl(((r[0] + r[1]) + r[2]) + r[3], (l + 48) & 63, 64);
                        const float s8 = (kg & 1) ? ((((left + r[0]) + r[1]) + r[2]) + r[3])
                                                  : ((r[0] + r[1]) + r[2]) + r[3];
                        const float pa = __shfl(s8, m + 16, 64), pb = __shfl(s8, m + 48, 64);
                        if (kg == 0) sNP[jc & 1][wv][16 * rt + m] = pa + pb;
                        continue;
                    }
                    const int tok = 16 * rt + m;
                    if (tok >= lc) continue;
                    TI *dst = op + ((t0 + tok) * H + h) * V + c0;
                    if (vec) {
                        st_q4<PK>(reinterpret_cast<st *>(dst), tr);
                    } else {
                        float x[4];
                        unpack4<PK>(tr, x);
#pragma unroll
                        for (int i = 0; i < 4; ++i)
                            if (c0 + i < V) io<TI>::st(dst, i, x[i]);
                    }
                }
            } else if (col_ok) {
#pragma unroll
                for (int rt = 0; rt < 4; ++rt)
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const int tok = 16 * rt + 4 * kg + i;
                        if (tok < lc) io<TI>::st(op, ((t0 + tok) * H + h) * V + col, oa[rt][i]);
                    }
            }
            if constexpr (TRAIN) if (emit) {
                st *usb = static_cast<st *>(p.us) + (static_cast<int64_t>(gc0 + jc) * H + h) * (64 * VP);
#pragma unroll
                for (int rt = 0; rt < 4; ++rt) emit_tile(usb, k16_block(rt, vt, VP) + 4 * l, ua[rt]);
            }
            }
            __syncthreads();
            if constexpr (!DB) {
                if (jc + 1 < nch) __syncthreads();
            }
        }
        if constexpr (NORM) {
            if (active && nch > 0) {
                const int64_t rp = len - static_cast<int64_t>(nch - 1) * kChunk;
                finish_norm(nch - 1, bos + static_cast<int64_t>(nch - 1) * kChunk,
                            rp < kChunk ? static_cast<int>(rp) : kChunk);
            }
        }
    }

    if (p.ht && col_ok) {
#pragma unroll
        for (int kt = 0; kt < NKT; ++kt)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int row = 16 * kt + 4 * kg + i;
                if (row < K) p.ht[state_index(p.flags, n, h, row, col, H, K, V)] = S[kt][i];
            }
    }
}

template <PrecKind PK, int KP, typename TI, typename TG, bool CONV = false>
hipError_t launch_prep(const ChunkParams &p, int total_chunks, hipStream_t stream)
{
    if (total_chunks == 0) return hipSuccess;
    const auto kern = chunk_prep_kernel<PK, KP, TI, TG, CONV>;
    // One resident wave of workgroups (occupancy x CUs of the current device,
    // looked up once per device), each walking items with a stride of the grid.
    static std::atomic<int> resident[64];  // per instantiation
    int slots = 0;
    hipError_t e = resident_slots(kern, 256, resident, &slots);
    if (e != hipSuccess) return e;
    const int64_t items = static_cast<int64_t>(total_chunks) * p.H;
    if (items > (int64_t{1} << 30)) return hipErrorInvalidValue;  // item indices stay in int
    const int grid = static_cast<int>(items < slots ? items : slots);
    hipLaunchKernelGGL(kern, dim3(grid), dim3(256), 0, stream, p, static_cast<int>(items));
    return hipGetLastError();
}

template <PrecKind PK, int KP, typename TI>
hipError_t launch_scan(const ChunkParams &p, int BVsel, hipStream_t stream)
{
    const int NP = p.num_seqs * p.H;
    const int groups = (NP + 7) / 8;
    auto go = [&](auto bvtag) {
        constexpr int BV = decltype(bvtag)::value;
        const int NVB = (p.V + BV - 1) / BV;
        if (p.conv_w[0]) {
            // Fused short convolutions (16-bit inference; the caller checked
            // the shapes), with or without the gated output norm.
            if constexpr (std::is_same<TI, bf16_t>::value && PK == PrecKind::BF16 && KP <= 128) {
                auto conv = [&](auto sigw, auto norm) {
                    hipLaunchKernelGGL((chunk_scan_kernel<PK, KP, BV, TI, false, decltype(sigw)::value,
                                                          decltype(norm)::value, true>),
                                       dim3(groups * 8 * NVB), dim3(512), 0, stream, p, NVB, NP);
                };
                const bool sigw = (p.flags & GDN2_FLAG_SIGMOID_BW) != 0;
                if (p.z) {
                    if (sigw) conv(std::true_type{}, std::true_type{});
                    else conv(std::false_type{}, std::true_type{});
                } else {
                    if (sigw) conv(std::true_type{}, std::false_type{});
                    else conv(std::false_type{}, std::false_type{});
                }
            }
        } else if (p.z) {
            // Gated output norm (bf16 inference; the caller checked BV == V).
            if constexpr (std::is_same<TI, bf16_t>::value && PK == PrecKind::BF16) {
                if (p.flags & GDN2_FLAG_SIGMOID_BW)
                    hipLaunchKernelGGL((chunk_scan_kernel<PK, KP, BV, TI, false, true, true>),
                                       dim3(groups * 8 * NVB), dim3(512), 0, stream, p, NVB, NP);
                else
                    hipLaunchKernelGGL((chunk_scan_kernel<PK, KP, BV, TI, false, false, true>),
                                       dim3(groups * 8 * NVB), dim3(512), 0, stream, p, NVB, NP);
            }
        } else if (p.hs)
            hipLaunchKernelGGL((chunk_scan_kernel<PK, KP, BV, TI, true>), dim3(groups * 8 * NVB),
                               dim3(512), 0, stream, p, NVB, NP);
        else if (p.flags & GDN2_FLAG_SIGMOID_BW)  // never with the training workspace
            hipLaunchKernelGGL((chunk_scan_kernel<PK, KP, BV, TI, false, true>), dim3(groups * 8 * NVB),
                               dim3(512), 0, stream, p, NVB, NP);
        else
            hipLaunchKernelGGL((chunk_scan_kernel<PK, KP, BV, TI, false>), dim3(groups * 8 * NVB),
                               dim3(512), 0, stream, p, NVB, NP);
    };
    if (BVsel == 16) go(std::integral_constant<int, 16>{});
    else if (BVsel == 32) go(std::integral_constant<int, 32>{});
    else go(std::integral_constant<int, 64>{});
    return hipGetLastError();
}

template <PrecKind PK, int KP, typename TI, typename TG>
hipError_t launch_all(const ChunkParams &p, int total_chunks, int stages, hipStream_t stream)
{
    if (stages & 1) {
        hipError_t e = hipErrorInvalidValue;
        if (!p.conv_w[0])
            e = launch_prep<PK, KP, TI, TG>(p, total_chunks, stream);
        else if constexpr (std::is_same<TI, bf16_t>::value && PK == PrecKind::BF16 && KP <= 128)
            e = launch_prep<PK, KP, TI, TG, true>(p, total_chunks, stream);
        if (e != hipSuccess) return e;
    }
    if (!(stages & 2) || p.num_seqs == 0) return hipSuccess;
    // The fused norm needs whole value rows in one workgroup: BV = V.
    return launch_scan<PK, KP, TI>(p, p.z ? bv_for(p.V) : scan_bv(p.num_seqs * p.H, p.V), stream);
}

template <PrecKind PK, typename TI, typename TG>
hipError_t launch_kp(const ChunkParams &p, int total_chunks, int stages, hipStream_t stream)
{
    switch (kp_for(p.K)) {
    case 32: return launch_all<PK, 32, TI, TG>(p, total_chunks, stages, stream);
    case 64: return launch_all<PK, 64, TI, TG>(p, total_chunks, stages, stream);
    case 128: return launch_all<PK, 128, TI, TG>(p, total_chunks, stages, stream);
    default:
        if constexpr (PK != PrecKind::F32) return launch_all<PK, 256, TI, TG>(p, total_chunks, stages, stream);
        return hipErrorInvalidValue;  // not reached: the callers reject fp32 beyond d_k = 128
    }
}

}  // namespace

size_t chunk_fwd_workspace_bytes(int B, int T, int H, int K, int V, int io_dtype,
                                 const int64_t *cu_host, int num_seqs)
{
    (void)V;
    if (chunk_wide(K, io_dtype)) return 0;  // the token-serial path needs no blobs
    if (!chunk_k_supported(K, io_dtype)) return 0;
    const int64_t nc = count_chunks(B, T, cu_host, num_seqs);
    return static_cast<size_t>(nc) * H * static_cast<size_t>(blob_bytes(io_dtype, kp_for(K)));
}

int launch_chunk_fwd(const ChunkFwdArgs &a, int io_dtype, int g_dtype, hipStream_t stream)
{
    if (chunk_wide(a.K, io_dtype)) return launch_chunk_fwd_wide(a, g_dtype, stream);
    if (!chunk_k_supported(a.K, io_dtype)) return GDN2_ERR_UNSUPPORTED;
    if (a.z && (io_dtype != GDN2_DTYPE_BF16 || a.V != bv_for(a.V) || (a.V % 16) != 0 ||
                (a.flags & GDN2_FLAG_SAVE_FOR_BWD)))
        return GDN2_ERR_UNSUPPORTED;
    if (a.conv_w[0]) {
        // Fused convolutions: bf16 rows, K a whole key width (32, 64, 128), V
        // split into whole 16-byte row pieces of whole value slices, forward
        // only.
        const int bv = a.z ? bv_for(a.V) : scan_bv(a.num_seqs * a.H, a.V);
        if (io_dtype != GDN2_DTYPE_BF16 || (a.flags & GDN2_FLAG_SAVE_FOR_BWD) || kp_for(a.K) != a.K ||
            a.K > 128 || a.V % bv != 0 || !a.conv_w[1] || !a.conv_w[2])
            return GDN2_ERR_UNSUPPORTED;
    }
    if (g_dtype != GDN2_DTYPE_F32 && g_dtype != io_dtype) return GDN2_ERR_UNSUPPORTED;
    const int64_t nc = count_chunks(a.B, a.T, a.cu_host, a.num_seqs);
    if (nc * a.H > 2147483647LL / 2) return GDN2_ERR_UNSUPPORTED;
    const bool train = (a.flags & GDN2_FLAG_SAVE_FOR_BWD) != 0;
    const TrainLayout tl = train_layout(nc, a.H, a.K, a.V, io_dtype);
    const size_t need = train ? static_cast<size_t>(tl.total)
                              : chunk_fwd_workspace_bytes(a.B, a.T, a.H, a.K, a.V, io_dtype,
                                                          a.cu_host, a.num_seqs);
    if (need > 0 && (!a.workspace || a.workspace_bytes < need)) return GDN2_ERR_WORKSPACE;

    ChunkParams p;
    p.q = a.q; p.k = a.k; p.v = a.v; p.g = a.g; p.b = a.b; p.w = a.w; p.o = a.o;
    p.h0 = a.h0;
    p.ht = a.ht;
    p.A_log = a.A_log;
    p.dt_bias = a.dt_bias;
    p.lower_bound = a.lower_bound;
    p.cu_seqlens = a.cu_seqlens;
    p.num_seqs = a.num_seqs;
    p.T = a.T; p.H = a.H; p.K = a.K; p.V = a.V;
    p.nt = (a.T + kChunk - 1) / kChunk;
    p.scale = a.scale;
    p.flags = a.flags;
    p.vec_ok = (a.K % 4) == 0;
    p.ws = a.workspace;
    p.VP = static_cast<int>(round_up(a.V, 16));
    p.hs = p.us = nullptr;
    p.z = a.z;
    p.ldz = a.ldz;
    p.nw = a.nw;
    p.eps = a.eps;
    for (int i = 0; i < 3; ++i) p.conv_w[i] = a.conv_w[i];
    p.ldq = a.ldq;
    p.ldk = a.ldk;
    p.ldv = a.ldv;
    p.conv_silu = a.conv_silu;
    if (train) {
        unsigned char *base = static_cast<unsigned char *>(a.workspace);
        p.hs = base + tl.hs;
        p.us = base + tl.us;
    }
    const int total = static_cast<int>(nc);

    hipError_t e;
    switch (io_dtype) {
    case GDN2_DTYPE_F32:
        e = launch_kp<PrecKind::F32, float, float>(p, total, a.stages, stream);
        break;
    case GDN2_DTYPE_BF16:
        e = g_dtype == GDN2_DTYPE_F32 ? launch_kp<PrecKind::BF16, bf16_t, float>(p, total, a.stages, stream)
                                      : launch_kp<PrecKind::BF16, bf16_t, bf16_t>(p, total, a.stages, stream);
        break;
    default:
        // fp16 inputs use bf16 MFMA operands: the factored decay terms reach
        // 2^(+-kDiagSpanLimit2/2), far outside the fp16 exponent range.
        e = g_dtype == GDN2_DTYPE_F32 ? launch_kp<PrecKind::BF16, f16_t, float>(p, total, a.stages, stream)
                                      : launch_kp<PrecKind::BF16, f16_t, f16_t>(p, total, a.stages, stream);
        break;
    }
    return e == hipSuccess ? GDN2_OK : GDN2_ERR_LAUNCH;
}

}  // namespace gdn2
