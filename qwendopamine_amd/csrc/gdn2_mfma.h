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
