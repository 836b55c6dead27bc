// MFMA operand conventions shared by the gdn2 chunk kernels (gfx950, wave64).
//
// Every contraction is issued as 16x16 output tiles whose contraction axis is
// walked in blocks of 32.  Within a block, lane l = m + 16*kg (m < 16,
// kg < 4) supplies the 8 consecutive contraction indices 32*s + 8*kg + j
// (j < 8) of its row m (A operand) or column m (B operand):
//   * 16-bit precisions issue one v_mfma_f32_16x16x32_{bf16,f16} per block;
//   * fp32 issues eight v_mfma_f32_16x16x4_f32, step j taking element j of
//     every lane (lane group kg then covers index 32*s + 8*kg + j).
// Since A and B always use the same assignment, the order in which the
// hardware sums the contraction index never matters.  The accumulator of a
// 16x16 tile holds D[4*(l/16) + i][l % 16] (i < 4) in lane l.
//
// "Fragment-native" storage (the chunk workspace): a [M][Kc] operand is cut
// into 16 x 32 blocks stored row-block-major; inside a block lane l's eight
// values are contiguous at offset 8*l, so a wave loads one operand block with
// one fully coalesced 16- (or 32-) byte access per lane.
#pragma once

#include "gdn2_common.h"

namespace gdn2 {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

enum class PrecKind { BF16, F16, F32 };

template <PrecKind PK>
struct Prec;

// 16-bit operands: 8 values per lane packed in one uint4.
template <>
struct Prec<PrecKind::BF16> {
    using st = uint16_t;
    struct frag {
        uint4 u;
    };
    static __device__ __forceinline__ st from_f32(float x) { return f32_to_bf16_bits(x); }
    static __device__ __forceinline__ float to_f32(st x) { return bf16_bits_to_f32(x); }
    static __device__ __forceinline__ f32x4 mma(f32x4 acc, frag a, frag b)
    {
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a.u),
                                                       __builtin_bit_cast(bf16x8, b.u), acc, 0,
                                                       0, 0);
    }
};

template <>
struct Prec<PrecKind::F16> {
    using st = uint16_t;
    struct frag {
        uint4 u;
    };
    static __device__ __forceinline__ st from_f32(float x)
    {
        return __builtin_bit_cast(uint16_t, static_cast<_Float16>(x));
    }
    static __device__ __forceinline__ float to_f32(st x)
    {
        return static_cast<float>(__builtin_bit_cast(_Float16, x));
    }
    static __device__ __forceinline__ f32x4 mma(f32x4 acc, frag a, frag b)
    {
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a.u),
                                                      __builtin_bit_cast(f16x8, b.u), acc, 0, 0,
                                                      0);
    }
};

template <>
struct Prec<PrecKind::F32> {
    using st = float;
    struct frag {
        float4 lo, hi;
    };
    static __device__ __forceinline__ st from_f32(float x) { return x; }
    static __device__ __forceinline__ float to_f32(st x) { return x; }
    static __device__ __forceinline__ f32x4 mma(f32x4 acc, frag a, frag b)
    {
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a.lo.x, b.lo.x, acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a.lo.y, b.lo.y, acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a.lo.z, b.lo.z, acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a.lo.w, b.lo.w, acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a.hi.x, b.hi.x, acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a.hi.y, b.hi.y, acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a.hi.z, b.hi.z, acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a.hi.w, b.hi.w, acc, 0, 0, 0);
        return acc;
    }
};

// Load / store the 8 contiguous values of a fragment (address 16-byte aligned
// for 16-bit storage, 32-byte aligned for fp32).
template <PrecKind PK>
__device__ __forceinline__ typename Prec<PK>::frag ld_frag(const typename Prec<PK>::st *p)
{
    typename Prec<PK>::frag f;
    if constexpr (PK == PrecKind::F32) {
        f.lo = reinterpret_cast<const float4 *>(p)[0];
        f.hi = reinterpret_cast<const float4 *>(p)[1];
    } else {
        f.u = *reinterpret_cast<const uint4 *>(p);
    }
    return f;
}

template <PrecKind PK>
__device__ __forceinline__ void st_frag(typename Prec<PK>::st *p, typename Prec<PK>::frag f)
{
    if constexpr (PK == PrecKind::F32) {
        reinterpret_cast<float4 *>(p)[0] = f.lo;
        reinterpret_cast<float4 *>(p)[1] = f.hi;
    } else {
        *reinterpret_cast<uint4 *>(p) = f.u;
    }
}

// Pack / unpack 8 floats.
template <PrecKind PK>
__device__ __forceinline__ typename Prec<PK>::frag pack_frag(const float (&x)[8])
{
    typename Prec<PK>::frag f;
    if constexpr (PK == PrecKind::F32) {
        f.lo = make_float4(x[0], x[1], x[2], x[3]);
        f.hi = make_float4(x[4], x[5], x[6], x[7]);
    } else {
        using P = Prec<PK>;
        f.u.x = static_cast<uint32_t>(P::from_f32(x[0])) | (static_cast<uint32_t>(P::from_f32(x[1])) << 16);
        f.u.y = static_cast<uint32_t>(P::from_f32(x[2])) | (static_cast<uint32_t>(P::from_f32(x[3])) << 16);
        f.u.z = static_cast<uint32_t>(P::from_f32(x[4])) | (static_cast<uint32_t>(P::from_f32(x[5])) << 16);
        f.u.w = static_cast<uint32_t>(P::from_f32(x[6])) | (static_cast<uint32_t>(P::from_f32(x[7])) << 16);
    }
    return f;
}

template <PrecKind PK>
__device__ __forceinline__ void unpack_frag(typename Prec<PK>::frag f, float (&x)[8])
{
    if constexpr (PK == PrecKind::F32) {
        x[0] = f.lo.x; x[1] = f.lo.y; x[2] = f.lo.z; x[3] = f.lo.w;
        x[4] = f.hi.x; x[5] = f.hi.y; x[6] = f.hi.z; x[7] = f.hi.w;
    } else {
        using P = Prec<PK>;
        const uint32_t w[4] = {f.u.x, f.u.y, f.u.z, f.u.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            x[2 * i] = P::to_f32(static_cast<uint16_t>(w[i] & 0xffffu));
            x[2 * i + 1] = P::to_f32(static_cast<uint16_t>(w[i] >> 16));
        }
    }
}

// Element offset of fragment block (mt, kt) of a fragment-native [M][Kc] operand.
__device__ __forceinline__ int64_t fn_block(int mt, int kt, int Kc)
{
    return (static_cast<int64_t>(mt) * (Kc / 32) + kt) * 512;
}

__device__ __forceinline__ f32x4 zero4()
{
    f32x4 z = {0.f, 0.f, 0.f, 0.f};
    return z;
}

// ---------------------------------------------------------------------------
// "K16" convention (second-generation chunk kernels).
//
// A 16x16 operand tile is held as 4 consecutive contraction indices per lane:
// lane l = m + 16*kg holds A[m][4*kg + i] (A operand) or B[4*kg + i][n=m]
// (B operand), i < 4.  This is exactly the layout in which a 16x16 fp32
// accumulator holds D[4*kg + i][n], so an accumulator tile feeds the next
// product as its B operand (contraction over the accumulator's rows) without
// any data movement.  One 16x16x32 MFMA consumes two K16 tiles: lane group kg
// supplies the indices {4kg+i} of the first tile and {16+4kg+i} of the second
// -- any fixed pairing works because A and B use the same one.  fp32 issues
// eight 16x16x4 MFMAs instead, pairing the same indices.
//
// Storage ("K16 fragment-native"): a [M][Kc] operand is cut into 16x16 blocks,
// block (mt, kt) at element offset 256*(mt*(Kc/16) + kt); inside a block lane
// l's 4 values are contiguous at offset 4*l.
// ---------------------------------------------------------------------------

__device__ __forceinline__ int64_t k16_block(int mt, int kt, int Kc)
{
    return (static_cast<int64_t>(mt) * (Kc / 16) + kt) * 256;
}

// 4 values of one lane: 16-bit storage packs them in a uint2, fp32 in a float4.
template <PrecKind PK>
struct Q4;
template <>
struct Q4<PrecKind::BF16> {
    uint2 u;
};
template <>
struct Q4<PrecKind::F16> {
    uint2 u;
};
template <>
struct Q4<PrecKind::F32> {
    float4 f;
};

__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) { return f32x2_to_bf16x2_bits(lo, hi); }

template <PrecKind PK>
__device__ __forceinline__ Q4<PK> pack4(float a, float b, float c, float d)
{
    Q4<PK> r;
    if constexpr (PK == PrecKind::F32) {
        r.f = make_float4(a, b, c, d);
    } else if constexpr (PK == PrecKind::BF16) {
        r.u.x = pack_bf16x2(a, b);
        r.u.y = pack_bf16x2(c, d);
    } else {
        r.u.x = static_cast<uint32_t>(Prec<PK>::from_f32(a)) | (static_cast<uint32_t>(Prec<PK>::from_f32(b)) << 16);
        r.u.y = static_cast<uint32_t>(Prec<PK>::from_f32(c)) | (static_cast<uint32_t>(Prec<PK>::from_f32(d)) << 16);
    }
    return r;
}

template <PrecKind PK>
__device__ __forceinline__ Q4<PK> pack4(f32x4 v)
{
    return pack4<PK>(v[0], v[1], v[2], v[3]);
}

template <PrecKind PK>
__device__ __forceinline__ void unpack4(Q4<PK> q, float (&x)[4])
{
    if constexpr (PK == PrecKind::F32) {
        x[0] = q.f.x; x[1] = q.f.y; x[2] = q.f.z; x[3] = q.f.w;
    } else {
        using P = Prec<PK>;
        x[0] = P::to_f32(static_cast<uint16_t>(q.u.x & 0xffffu));
        x[1] = P::to_f32(static_cast<uint16_t>(q.u.x >> 16));
        x[2] = P::to_f32(static_cast<uint16_t>(q.u.y & 0xffffu));
        x[3] = P::to_f32(static_cast<uint16_t>(q.u.y >> 16));
    }
}

template <PrecKind PK>
__device__ __forceinline__ Q4<PK> ld_q4(const typename Prec<PK>::st *p)
{
    Q4<PK> r;
    if constexpr (PK == PrecKind::F32)
        r.f = *reinterpret_cast<const float4 *>(p);
    else
        r.u = *reinterpret_cast<const uint2 *>(p);
    return r;
}

template <PrecKind PK>
__device__ __forceinline__ void st_q4(typename Prec<PK>::st *p, Q4<PK> v)
{
    if constexpr (PK == PrecKind::F32)
        *reinterpret_cast<float4 *>(p) = v.f;
    else
        *reinterpret_cast<uint2 *>(p) = v.u;
}

// One 16x16x32 step from two K16 tiles of A and two of B.
template <PrecKind PK>
__device__ __forceinline__ f32x4 mma2(f32x4 acc, Q4<PK> a0, Q4<PK> a1, Q4<PK> b0, Q4<PK> b1)
{
    if constexpr (PK == PrecKind::F32) {
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a0.f.x, b0.f.x, acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a0.f.y, b0.f.y, acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a0.f.z, b0.f.z, acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a0.f.w, b0.f.w, acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a1.f.x, b1.f.x, acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a1.f.y, b1.f.y, acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a1.f.z, b1.f.z, acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a1.f.w, b1.f.w, acc, 0, 0, 0);
        return acc;
    } else {
        const uint4 a = make_uint4(a0.u.x, a0.u.y, a1.u.x, a1.u.y);
        const uint4 b = make_uint4(b0.u.x, b0.u.y, b1.u.x, b1.u.y);
        if constexpr (PK == PrecKind::BF16)
            return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                           __builtin_bit_cast(bf16x8, b), acc, 0, 0, 0);
        else
            return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a),
                                                          __builtin_bit_cast(f16x8, b), acc, 0, 0, 0);
    }
}

// One 16x16x16 step from a single K16 tile of A and of B.
template <PrecKind PK>
__device__ __forceinline__ f32x4 mma1(f32x4 acc, Q4<PK> a, Q4<PK> b)
{
    if constexpr (PK == PrecKind::F32) {
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a.f.x, b.f.x, acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a.f.y, b.f.y, acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a.f.z, b.f.z, acc, 0, 0, 0);
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a.f.w, b.f.w, acc, 0, 0, 0);
        return acc;
    } else {
        typedef short s4 __attribute__((ext_vector_type(4)));
        const s4 av = __builtin_bit_cast(s4, a.u);
        const s4 bv = __builtin_bit_cast(s4, b.u);
        if constexpr (PK == PrecKind::BF16)
            return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(av, bv, acc, 0, 0, 0);
        else {
            typedef _Float16 h4 __attribute__((ext_vector_type(4)));
            return __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(h4, a.u),
                                                         __builtin_bit_cast(h4, b.u), acc, 0, 0, 0);
        }
    }
}

// B operand of the 16x16 identity in lane l (rows 4*kg+i, column m).
template <PrecKind PK>
__device__ __forceinline__ Q4<PK> identity_q4(int lane)
{
    const int m = lane & 15, kg = lane >> 4;
    return pack4<PK>(4 * kg == m ? 1.f : 0.f, 4 * kg + 1 == m ? 1.f : 0.f, 4 * kg + 2 == m ? 1.f : 0.f,
                     4 * kg + 3 == m ? 1.f : 0.f);
}

// fp32 16x16 = 16x16 * 16x16 product of row-major LDS matrices (leading
// dimensions lda, ldb), contraction index 4*kk + j for lane group kk, step j.
__device__ __forceinline__ f32x4 mm16_f32(f32x4 acc, const float *A, int lda, const float *B,
                                          int ldb, int lane)
{
    const int m = lane & 15, kk = lane >> 4;
#pragma unroll
    for (int j = 0; j < 4; ++j)
        acc = __builtin_amdgcn_mfma_f32_16x16x4f32(A[m * lda + 4 * kk + j], B[(4 * kk + j) * ldb + m],
                                                   acc, 0, 0, 0);
    return acc;
}

}  // namespace gdn2
