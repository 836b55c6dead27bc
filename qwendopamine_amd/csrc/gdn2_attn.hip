// Single-token softmax attention of the hybrid decoder host's attention
// layers, gfx950: RoPE of the token's q and k, the KV-cache store at its
// position, and attention over the cache up to that position, in one launch
// per layer (the host's torch path issues about seventeen).
//
// Eight-wave workgroups per (sequence, KV group): one, or for caches longer
// than 1024 positions up to eight, each over its share of the positions, whose
// partial softmax states a second kernel merges.  The token's rotated
// q heads, k and v go to LDS (and k, v to the caches).  Each wave then walks
// the cached positions j = (step * 8 + wave) * PS + slot: the DG lanes of a
// slot each hold 8 channels (one 16-byte piece) of k_j and v_j, requested
// together, and the slot's dot products are completed by xor-shuffles over
// those lanes.  Softmax is online (running maximum, rescaled sums), so the
// cache is read once; the per-slot states are merged across slots by
// shuffles and across waves through LDS.  All sums are fp32; the output is
// rounded once to the io dtype.
#include "gdn2_common.h"
#include "gdn2_internal.h"

namespace gdn2 {
namespace {

constexpr int kAttnWaves = 8;
constexpr float kNegBig = -1.0e30f;  // "no position yet": exp(kNegBig - m) is 0 for any real m


template <typename T>
__device__ __forceinline__ void widen8(uint4 u, float (&f)[8])
{
    const unsigned w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint16_t lo = static_cast<uint16_t>(w[i] & 0xffffu), hi = static_cast<uint16_t>(w[i] >> 16);
        if constexpr (std::is_same<T, bf16_t>::value) {
            f[2 * i] = bf16_bits_to_f32(lo);
            f[2 * i + 1] = bf16_bits_to_f32(hi);
        } else {
            f[2 * i] = static_cast<float>(__builtin_bit_cast(_Float16, lo));
            f[2 * i + 1] = static_cast<float>(__builtin_bit_cast(_Float16, hi));
        }
    }
}

template <typename T, int D, int QPK>
__global__ __launch_bounds__(512) void attn_decode_kernel(AttnDecodeParams p)
{
    // Positions per slot requested at once: as many as the registers allow
    // beside the QPK heads' sums (the cache read is latency-bound at one
    // workgroup per KV group).
    constexpr int kUnroll = QPK <= 2 ? 8 : 4;
    constexpr int DG = D / 8;    // 16-byte channel pieces of a row
    constexpr int PS = 64 / DG;  // position slots per wave
    static_assert(DG * PS == 64, "a wave is PS slots of DG lanes");
    __shared__ __align__(16) float sq[QPK][D];
    __shared__ __align__(16) float skv[2][D];
    __shared__ float sm[kAttnWaves][QPK], sl[kAttnWaves][QPK];
    __shared__ __align__(16) float so[kAttnWaves][QPK][D];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int G = p.G;
    const int b = blockIdx.x / G, g = blockIdx.x - (blockIdx.x / G) * G;
    const int64_t pos = *p.pos;
    const int H = G * QPK;
    T *out = static_cast<T *>(p.out) + (static_cast<int64_t>(b) * H + g * QPK) * D;
    if (pos < 0 || pos >= p.max_len) {
        // Outside the caches: zero output, caches untouched.
        for (int e = tid; e < QPK * D; e += 512) io<T>::st(out, e, 0.0f);
        return;
    }
    const int n = static_cast<int>(pos) + 1;
    // This workgroup's share of the positions: split blockIdx.y of p.splits,
    // in whole steps of the wave layout below.
    const int per_step_all = kAttnWaves * PS;
    const int steps = (n + per_step_all - 1) / per_step_all;
    const int sps = (steps + p.splits - 1) / p.splits;
    const int lo = static_cast<int>(blockIdx.y) * sps * per_step_all;
    const int hi = lo + sps * per_step_all < n ? lo + sps * per_step_all : n;
    const T *x = static_cast<const T *>(p.qkv) + static_cast<int64_t>(b * G + g) * (QPK + 2) * D;
    const int64_t cbase = (static_cast<int64_t>(b) * G + g) * p.max_len * D;
    T *kc = static_cast<T *>(p.k_cache) + cbase;
    T *vc = static_cast<T *>(p.v_cache) + cbase;

    // ---- RoPE of the QPK q heads and k (interleaved pairs, fp32, rounded to
    // the io dtype as the host's torch path), v as is.  The token's rows are
    // requested first, then this workgroup's first batch of cached k, v rows
    // (below), and only then is anything computed: loads complete in order,
    // so the cache rows' latency overlaps the RoPE, the stores and the barrier. ----
    static_assert((QPK + 1) * (D / 2) <= 512 && D <= 512, "one RoPE pair / v channel per thread");
    const bool store = blockIdx.y == 0;  // one split stores the token's k, v
    const int he = tid / (D / 2), ie = tid - (tid / (D / 2)) * (D / 2);
    const bool has_pair = tid < (QPK + 1) * (D / 2), has_v = tid < D;
    float x0 = 0.0f, x1 = 0.0f, cs = 1.0f, sn = 0.0f, xv = 0.0f;
    if (has_pair) {
        x0 = io<T>::ld(x, he * D + 2 * ie);
        x1 = io<T>::ld(x, he * D + 2 * ie + 1);
        if (ie < p.rope_pairs) {
            cs = p.cos[pos * p.rope_stride + ie];
            sn = p.sin[pos * p.rope_stride + ie];
        }
    }
    if (has_v) xv = io<T>::ld(x, (QPK + 1) * D + tid);

    const int slot = lane / DG, dg = lane - (lane / DG) * DG;
    const int per_step = kAttnWaves * PS;
    // kUnroll positions per slot requested at once; positions from pos on read
    // row 0 (always valid) and are skipped or replaced.
    uint4 kr[kUnroll], vr[kUnroll];
    auto request = [&](int j0) __attribute__((always_inline)) {
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) {
            const int j = j0 + u * per_step + wave * PS + slot;
            const int64_t jl = j < pos && j < hi ? j : 0;
            kr[u] = *reinterpret_cast<const uint4 *>(kc + jl * D + dg * 8);
            vr[u] = *reinterpret_cast<const uint4 *>(vc + jl * D + dg * 8);
        }
    };
    request(lo);

    if (has_pair) {
        float y0 = x0, y1 = x1;
        if (ie < p.rope_pairs) {
            y0 = round_to<T>(x0 * cs - x1 * sn);
            y1 = round_to<T>(x0 * sn + x1 * cs);
        }
        if (he < QPK) {
            sq[he][2 * ie] = y0;
            sq[he][2 * ie + 1] = y1;
        } else {
            skv[0][2 * ie] = y0;
            skv[0][2 * ie + 1] = y1;
            if (store) {
                io<T>::st(kc, pos * D + 2 * ie, y0);
                io<T>::st(kc, pos * D + 2 * ie + 1, y1);
            }
        }
    }
    if (has_v) {
        skv[1][tid] = xv;
        if (store) io<T>::st(vc, pos * D + tid, xv);
    }
    __syncthreads();

    // ---- one pass over positions 0 .. pos with online softmax ----
    float qv[QPK][8];
#pragma unroll
    for (int h = 0; h < QPK; ++h)
#pragma unroll
        for (int e = 0; e < 8; ++e) qv[h][e] = sq[h][dg * 8 + e] * p.scale;
    float m[QPK], l[QPK], acc[QPK][8];
#pragma unroll
    for (int h = 0; h < QPK; ++h) {
        m[h] = kNegBig;
        l[h] = 0.0f;
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[h][e] = 0.0f;
    }
    for (int j0 = lo; j0 < hi; j0 += per_step * kUnroll) {
#pragma unroll
        for (int u = 0; u < kUnroll; ++u) {
        const int j = j0 + u * per_step + wave * PS + slot;
        if (j >= hi) continue;  // no shuffles below cross slots, so lanes may drop out per slot
        float kf[8], vf[8];
        if (j == pos) {
            // The token itself: its k, v from LDS (its cache store may still be in flight).
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                kf[e] = skv[0][dg * 8 + e];
                vf[e] = skv[1][dg * 8 + e];
            }
        } else {
            widen8<T>(kr[u], kf);
            widen8<T>(vr[u], vf);
        }
#pragma unroll
        for (int h = 0; h < QPK; ++h) {
            float s = 0.0f;
#pragma unroll
            for (int e = 0; e < 8; ++e) s = fmaf(qv[h][e], kf[e], s);
#pragma unroll
            for (int o = 1; o < DG; o <<= 1) s += __shfl_xor(s, o, 64);  // within the slot's DG lanes
            const float mn = fmaxf(m[h], s);
            const float r = __expf(m[h] - mn), pj = __expf(s - mn);
            l[h] = l[h] * r + pj;
#pragma unroll
            for (int e = 0; e < 8; ++e) acc[h][e] = fmaf(pj, vf[e], acc[h][e] * r);
            m[h] = mn;
        }
        }
        // The next batch (a workgroup's share is one or two batches at up to 1024 positions).
        if (j0 + per_step * kUnroll < hi) request(j0 + per_step * kUnroll);
    }
    // Merge the PS slot states of the wave (lanes with equal dg).
#pragma unroll
    for (int h = 0; h < QPK; ++h) {
#pragma unroll
        for (int o = DG; o < 64; o <<= 1) {
            const float m2 = __shfl_xor(m[h], o, 64), l2 = __shfl_xor(l[h], o, 64);
            const float mn = fmaxf(m[h], m2);
            const float r1 = __expf(m[h] - mn), r2 = __expf(m2 - mn);
            l[h] = l[h] * r1 + l2 * r2;
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const float a2 = __shfl_xor(acc[h][e], o, 64);
                acc[h][e] = acc[h][e] * r1 + a2 * r2;
            }
            m[h] = mn;
        }
        if (slot == 0) {
#pragma unroll
            for (int e = 0; e < 8; ++e) so[wave][h][dg * 8 + e] = acc[h][e];
            if (dg == 0) {
                sm[wave][h] = m[h];
                sl[wave][h] = l[h];
            }
        }
    }
    __syncthreads();
    // Merge the waves; one split normalises and stores, several leave their
    // (max, sum, weighted values) for attn_merge_kernel.
    float *part = p.splits > 1 ? p.part + ((static_cast<int64_t>(blockIdx.x) * p.splits + blockIdx.y) * QPK) * (D + 2)
                               : nullptr;
    for (int e = tid; e < QPK * D; e += 512) {
        const int h = e / D, d = e - h * D;
        float mx = kNegBig;
#pragma unroll
        for (int w = 0; w < kAttnWaves; ++w) mx = fmaxf(mx, sm[w][h]);
        float num = 0.0f, den = 0.0f;
#pragma unroll
        for (int w = 0; w < kAttnWaves; ++w) {
            const float r = __expf(sm[w][h] - mx);
            num = fmaf(so[w][h][d], r, num);
            den = fmaf(sl[w][h], r, den);
        }
        if (p.splits == 1) {
            io<T>::st(out, e, num / den);
        } else {
            part[h * (D + 2) + d] = num;
            if (d == 0) {
                part[h * (D + 2) + D] = mx;
                part[h * (D + 2) + D + 1] = den;
            }
        }
    }
}

// Combines the splits' partial states: thread (row, h, d) of the output.
template <typename T, int D, int QPK>
__global__ __launch_bounds__(256) void attn_merge_kernel(AttnDecodeParams p)
{
    const int64_t e = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    const int64_t total = static_cast<int64_t>(p.B) * p.G * QPK * D;
    if (e >= total) return;
    const int d = static_cast<int>(e % D);
    const int64_t bgh = e / D;                 // (b * G + g) * QPK + h
    const int h = static_cast<int>(bgh % QPK);
    const int64_t bg = bgh / QPK;
    if (*p.pos < 0 || *p.pos >= p.max_len) {
        io<T>::st(static_cast<T *>(p.out), e, 0.0f);
        return;
    }
    const float *part = p.part + (bg * p.splits * QPK + h) * (D + 2);
    const int64_t sstride = static_cast<int64_t>(QPK) * (D + 2);
    float mx = kNegBig;
    for (int s = 0; s < p.splits; ++s) mx = fmaxf(mx, part[s * sstride + D]);
    float num = 0.0f, den = 0.0f;
    for (int s = 0; s < p.splits; ++s) {
        const float r = __expf(part[s * sstride + D] - mx);
        num = fmaf(part[s * sstride + d], r, num);
        den = fmaf(part[s * sstride + D + 1], r, den);
    }
    io<T>::st(static_cast<T *>(p.out), e, num / den);
}

template <typename T, int D, int QPK>
hipError_t attn_q(const AttnDecodeParams &p, hipStream_t s)
{
    hipLaunchKernelGGL((attn_decode_kernel<T, D, QPK>), dim3(static_cast<unsigned>(p.B * p.G), p.splits), dim3(512),
                       0, s, p);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || p.splits == 1) return e;
    const int64_t total = static_cast<int64_t>(p.B) * p.G * QPK * D;
    hipLaunchKernelGGL((attn_merge_kernel<T, D, QPK>), dim3(static_cast<unsigned>((total + 255) / 256)), dim3(256), 0,
                       s, p);
    return hipGetLastError();
}

template <typename T, int D>
hipError_t attn_d(const AttnDecodeParams &p, hipStream_t s)
{
    switch (p.qpk) {
    case 1: return attn_q<T, D, 1>(p, s);
    case 2: return attn_q<T, D, 2>(p, s);
    default: return attn_q<T, D, 4>(p, s);
    }
}

template <typename T>
hipError_t attn_t(const AttnDecodeParams &p, hipStream_t s)
{
    return p.D == 64 ? attn_d<T, 64>(p, s) : attn_d<T, 128>(p, s);
}

// Row-wise argmax (greedy decoding over the LM head's logits): one workgroup of
// 1024 threads per row, each thread scanning 16-byte pieces tid, tid + 1024,
// ..., tid + 1024 (U - 1) with all U of them requested before any is compared
// (U is picked so that one such batch covers a row of the usual vocabulary
// sizes: a row then costs one memory round trip).  The first index of the
// maximum wins, and NaN counts as the maximum (torch's argmax).
template <typename T, int U>
__global__ __launch_bounds__(1024) void argmax_rows_kernel(ArgmaxParams p)
{
    constexpr int EPP = 16 / static_cast<int>(sizeof(T));  // elements per piece
    __shared__ float sv[16];
    __shared__ int64_t si[16];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const T *x = static_cast<const T *>(p.x) + static_cast<int64_t>(blockIdx.x) * p.ld;
    const int64_t pieces = p.n / EPP;
    float best = -INFINITY;
    int64_t bi = p.n;  // "none yet": larger than every index
    // Merge of two candidates: v beats best if larger, or NaN where best is not,
    // or equal / both NaN at a smaller index.
    auto take = [&](float v, int64_t i) __attribute__((always_inline)) {
        const bool vn = v != v, bn = best != best;
        const bool better = (vn && !bn) || (!vn && !bn && v > best) || ((v == best || (vn && bn)) && i < bi);
        if (better) {
            best = v;
            bi = i;
        }
    };
    // A thread's own elements arrive in increasing index order, so there a
    // candidate only has to be strictly larger (or the first NaN, or the first
    // element at all) to win.
    bool have = false;
    auto scan = [&](float v, int64_t i) __attribute__((always_inline)) {
        if (!have || v > best || (v != v && best == best)) {
            best = v;
            bi = i;
        }
        have = true;
    };
    for (int64_t c0 = tid; c0 < pieces; c0 += 1024 * U) {
        uint4 raw[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int64_t c = c0 + 1024 * u;
            raw[u] = *reinterpret_cast<const uint4 *>(x + (c < pieces ? c : c0) * EPP);
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int64_t c = c0 + 1024 * u;
            if (c >= pieces) continue;
            const unsigned w[4] = {raw[u].x, raw[u].y, raw[u].z, raw[u].w};
#pragma unroll
            for (int e = 0; e < EPP; ++e) {
                float v;
                if constexpr (sizeof(T) == 4) {
                    v = __uint_as_float(w[e]);
                } else {
                    const uint16_t h = static_cast<uint16_t>((e & 1) ? (w[e >> 1] >> 16) : (w[e >> 1] & 0xffffu));
                    if constexpr (std::is_same<T, bf16_t>::value)
                        v = bf16_bits_to_f32(h);
                    else
                        v = static_cast<float>(__builtin_bit_cast(_Float16, h));
                }
                scan(v, c * EPP + e);
            }
        }
    }
    // Ragged tail: these indexes exceed every piece's, so the in-order rule holds.
    for (int64_t i = pieces * EPP + tid; i < p.n; i += 1024) scan(io<T>::ld(x, i), i);
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
        const float v2 = __shfl_xor(best, o, 64);
        const int64_t i2 = __shfl_xor(bi, o, 64);
        take(v2, i2);
    }
    if (lane == 0) {
        sv[wave] = best;
        si[wave] = bi;
    }
    __syncthreads();
    if (tid == 0) {
        for (int w2 = 1; w2 < 16; ++w2) take(sv[w2], si[w2]);
        p.out[static_cast<int64_t>(blockIdx.x) * p.out_stride] = bi < p.n ? bi : 0;
    }
}

// Merge rule of two argmax candidates (value, index): larger value, or NaN
// where the other is not, or equal / both NaN at a smaller index.
__device__ __forceinline__ void argmax_take(float &best, int64_t &bi, float v, int64_t i)
{
    const bool vn = v != v, bn = best != best;
    const bool better = (vn && !bn) || (!vn && !bn && v > best) || ((v == best || (vn && bn)) && i < bi);
    if (better) {
        best = v;
        bi = i;
    }
}

// Split form, first pass: workgroup (s, row) scans pieces [s pps, (s + 1) pps)
// of the row (pps = 256 threads x 4 pieces: one batch of requests per
// thread), the last split also the ragged tail, and leaves its candidate.
// A row of 151,936 bf16 logits takes 19 workgroups on 19 CUs instead of one
// CU streaming the whole 304 KB.
template <typename T>
__global__ __launch_bounds__(256) void argmax_part_kernel(ArgmaxParams p)
{
    constexpr int EPP = 16 / static_cast<int>(sizeof(T));
    constexpr int U = 4;
    __shared__ float sv[4];
    __shared__ int64_t si[4];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int64_t row = blockIdx.y;
    const T *x = static_cast<const T *>(p.x) + row * p.ld;
    const int64_t pieces = p.n / EPP;
    const int64_t c_lo = static_cast<int64_t>(blockIdx.x) * p.pps;
    const int64_t c_hi = c_lo + p.pps < pieces ? c_lo + p.pps : pieces;
    float best = -INFINITY;
    int64_t bi = p.n;
    bool have = false;
    auto scan = [&](float v, int64_t i) __attribute__((always_inline)) {
        if (!have || v > best || (v != v && best == best)) {
            best = v;
            bi = i;
        }
        have = true;
    };
    for (int64_t c0 = c_lo + tid; c0 < c_hi; c0 += 256 * U) {
        uint4 raw[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int64_t c = c0 + 256 * u;
            raw[u] = *reinterpret_cast<const uint4 *>(x + (c < c_hi ? c : c0) * EPP);
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int64_t c = c0 + 256 * u;
            if (c >= c_hi) continue;
            const unsigned w[4] = {raw[u].x, raw[u].y, raw[u].z, raw[u].w};
#pragma unroll
            for (int e = 0; e < EPP; ++e) {
                float v;
                if constexpr (sizeof(T) == 4) {
                    v = __uint_as_float(w[e]);
                } else {
                    const uint16_t h = static_cast<uint16_t>((e & 1) ? (w[e >> 1] >> 16) : (w[e >> 1] & 0xffffu));
                    if constexpr (std::is_same<T, bf16_t>::value)
                        v = bf16_bits_to_f32(h);
                    else
                        v = static_cast<float>(__builtin_bit_cast(_Float16, h));
                }
                scan(v, c * EPP + e);
            }
        }
    }
    if (blockIdx.x == gridDim.x - 1)
        for (int64_t i = pieces * EPP + tid; i < p.n; i += 256) scan(io<T>::ld(x, i), i);
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
        const float v2 = __shfl_xor(best, o, 64);
        const int64_t i2 = __shfl_xor(bi, o, 64);
        argmax_take(best, bi, v2, i2);
    }
    if (lane == 0) {
        sv[wave] = best;
        si[wave] = bi;
    }
    __syncthreads();
    if (tid == 0) {
        for (int w2 = 1; w2 < 4; ++w2) argmax_take(best, bi, sv[w2], si[w2]);
        p.part_v[row * p.splits + blockIdx.x] = best;
        p.part_i[row * p.splits + blockIdx.x] = bi;
    }
}

// Split form, second pass: one wave per row merges the splits' candidates.
__global__ __launch_bounds__(64) void argmax_finish_kernel(ArgmaxParams p)
{
    const int lane = threadIdx.x;
    const int64_t row = blockIdx.x;
    float best = -INFINITY;
    int64_t bi = p.n;
    for (int s = lane; s < p.splits; s += 64)
        argmax_take(best, bi, p.part_v[row * p.splits + s], p.part_i[row * p.splits + s]);
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) {
        const float v2 = __shfl_xor(best, o, 64);
        const int64_t i2 = __shfl_xor(bi, o, 64);
        argmax_take(best, bi, v2, i2);
    }
    if (lane == 0) p.out[row * p.out_stride] = bi < p.n ? bi : 0;
}

template <typename T>
void argmax_launch(const ArgmaxParams &p, hipStream_t stream)
{
    if (p.splits > 1) {
        hipLaunchKernelGGL((argmax_part_kernel<T>), dim3(static_cast<unsigned>(p.splits), static_cast<unsigned>(p.rows)),
                           dim3(256), 0, stream, p);
        hipLaunchKernelGGL(argmax_finish_kernel, dim3(static_cast<unsigned>(p.rows)), dim3(64), 0, stream, p);
        return;
    }
    // Pieces in flight per thread: one batch covers a row of up to 1024 * U
    // pieces (U = 20: 163,840 bf16 logits), longer rows loop.
    const dim3 grid(static_cast<unsigned>(p.rows));
    const int64_t per = (p.n / (16 / static_cast<int64_t>(sizeof(T))) + 1023) / 1024;
    if (per <= 4)
        hipLaunchKernelGGL((argmax_rows_kernel<T, 4>), grid, dim3(1024), 0, stream, p);
    else if (per <= 8)
        hipLaunchKernelGGL((argmax_rows_kernel<T, 8>), grid, dim3(1024), 0, stream, p);
    else
        hipLaunchKernelGGL((argmax_rows_kernel<T, 20>), grid, dim3(1024), 0, stream, p);
}

}  // namespace

int argmax_splits(int64_t n, int io_dtype)
{
    const int64_t epp = io_dtype == GDN2_DTYPE_F32 ? 4 : 8;
    const int64_t s = (n / epp + 1023) / 1024;
    return static_cast<int>(s < 1 ? 1 : (s > 4096 ? 4096 : s));
}

hipError_t launch_argmax_rows(const ArgmaxParams &p, int io_dtype, hipStream_t stream)
{
    switch (io_dtype) {
    case GDN2_DTYPE_F32: argmax_launch<float>(p, stream); break;
    case GDN2_DTYPE_BF16: argmax_launch<bf16_t>(p, stream); break;
    default: argmax_launch<f16_t>(p, stream); break;
    }
    return hipGetLastError();
}

int attn_decode_splits(int64_t max_len)
{
    // About 1024 positions per workgroup at a full cache (two batches of
    // requests per wave), at most 8 splits.  At config 3 (cache 2304, 64 KV
    // groups) three splits measured best: decode step 0.870 ms against 0.880 at
    // 512 positions (five splits), 0.883 at 1536 and 0.892 with a single split.
    const int64_t s = (max_len + 1023) / 1024;
    return static_cast<int>(s < 1 ? 1 : (s > 8 ? 8 : s));
}

size_t attn_decode_workspace_floats(int B, int G, int qpk, int D, int64_t max_len)
{
    const int s = attn_decode_splits(max_len);
    return s == 1 ? 0 : static_cast<size_t>(B) * G * s * qpk * (D + 2);
}

bool attn_decode_supported(int io_dtype, int qpk, int D)
{
    return (io_dtype == GDN2_DTYPE_BF16 || io_dtype == GDN2_DTYPE_F16) && (qpk == 1 || qpk == 2 || qpk == 4) &&
           (D == 64 || D == 128);
}

hipError_t launch_attn_decode(const AttnDecodeParams &p, int io_dtype, hipStream_t stream)
{
    return io_dtype == GDN2_DTYPE_BF16 ? attn_t<bf16_t>(p, stream) : attn_t<f16_t>(p, stream);
}

}  // namespace gdn2
