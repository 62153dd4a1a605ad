// 128-point Sylvester Hadamard butterfly over a 16-lane group (8 elements per lane), shared by the
// Hadamard row transform (hadamard.hip) and the RMSNorm kernels that feed it (rms_norm_kernel.cuh).
// Element 8 * l + j of a block sits in lane l, slot j: index bits 0..2 are in-lane stages, bits 3..6
// lane exchanges at xor 1, 2, 4, 8, taken in that order, each pair (a, b) -> (a + b, a - b) with a the
// lower index, in fp32 -- the order of the reference's warp butterfly (kernels/quant/
// hadamard_inner.cuh:19-46, 127-141), so every caller rounds identically.
#pragma once

#include "common.cuh"

namespace exl3r {

// The value of lane (l ^ M) inside the 16-lane group: quad_perm for xor 1 and 2, ds_swizzle (bit
// mode) for xor 4, a row rotation by 8 for xor 8.
template <int M>
__device__ __forceinline__ float lane_xor(float v)
{
    const int i = __builtin_bit_cast(int, v);
    if constexpr (M == 1) return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, i, DPP_QUAD_XOR1, 0xf, 0xf, false));
    else if constexpr (M == 2) return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, i, DPP_QUAD_XOR2, 0xf, 0xf, false));
    else if constexpr (M == 4) return __builtin_bit_cast(float, __builtin_amdgcn_ds_swizzle(i, 0x101f));
    else return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, i, DPP_ROW_ROR8, 0xf, 0xf, false));
}

// One cross-lane butterfly stage: the lane whose bit M is clear holds a and keeps a + b, its partner
// holds b and keeps a - b.  (Carrying a per-lane sign instead, to make this one fma, does not keep
// the sign of exact zeros: -(x + y) and (-x) + (-y) differ when x + y == 0.)
template <int M>
__device__ __forceinline__ void lane_stage(float (&f)[8], int l16)
{
    #pragma clang fp contract(off)
    const bool upper = (l16 & M) != 0;
    #pragma unroll
    for (int j = 0; j < 8; ++j)
    {
        const float p = lane_xor<M>(f[j]);
        f[j] = upper ? p - f[j] : f[j] + p;
    }
}

// f = r * H128 (block) with r the transform's scale, rounded once after the fp32 butterfly.
__device__ __forceinline__ void butterfly128(float (&f)[8], int l16, float r)
{
    #pragma clang fp contract(off)
    #pragma unroll
    for (int h = 1; h < 8; h <<= 1)
    {
        #pragma unroll
        for (int j = 0; j < 8; ++j)
        {
            if (j & h) continue;
            const float a = f[j], b = f[j | h];
            f[j] = a + b;
            f[j | h] = a - b;
        }
    }
    lane_stage<1>(f, l16);
    lane_stage<2>(f, l16);
    lane_stage<4>(f, l16);
    lane_stage<8>(f, l16);
    #pragma unroll
    for (int j = 0; j < 8; ++j) f[j] = f[j] * r;
}

__device__ __forceinline__ uint32_t hmul2(uint32_t a, uint32_t b)
{
    return __builtin_bit_cast(uint32_t, __builtin_bit_cast(f16x2, a) * __builtin_bit_cast(f16x2, b));
}

// The EXL3 linear's output rotation had_r_128(y, y, None, post) (scale 1) of the 8-element f16 chunk
// at column col of a row, held as lane (col / 8) % 16 of its block's 16-lane group: the fp32
// butterfly, one rounding to f16, then the half post-scale product (post: f16 per column, or null).
__device__ __forceinline__ void output_rotation8(TF16::Vec& v, const void* post, int64_t col)
{
    float f[8];
    unpack8<TF16>(v, f);
    butterfly128(f, (int)((col >> 3) & 15), 0.0883883461356163f);
    v = pack8<TF16>(f);
    if (post)
    {
        const TF16::Vec p = load8<TF16>(post, col);
        #pragma unroll
        for (int q = 0; q < 4; ++q) v.a[q] = hmul2(v.a[q], p.a[q]);
    }
}

}  // namespace exl3r
