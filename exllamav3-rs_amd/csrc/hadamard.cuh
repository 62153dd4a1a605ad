// 128-point Sylvester Hadamard butterfly over a 16-lane group (8 elements per lane), shared by the
// Hadamard row transform (hadamard.hip) and the RMSNorm kernels that feed it (rms_norm_kernel.cuh).
// Element 8 * l + j of a block sits in lane l, slot j: index bits 0..2 are in-lane stages, bits 3..6
// lane exchanges at xor 1, 2, 4, 8, taken in that order, each pair (a, b) -> (a + b, a - b) with a the
// lower index, in fp32 -- the order of the reference's warp butterfly (kernels/quant/
// hadamard_inner.cuh:19-46, 127-141), so every caller rounds identically.
#pragma once

#include <type_traits>

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
// holds b and keeps a - b.  (The exact form, used where the carried-sign form below may not be.)
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

// The same stage with the upper lane's sign carried: every lane keeps v + c * partner (c = -1 in the
// upper lane), one fma whose product is exact, so the upper lane holds fl(b - a) = -fl(a - b).  Two
// partners always carry the same sign (the parity of the lane bits already exchanged), so after the
// four stages lane l holds (-1)^popcount(l) times the reference's value, bit for bit, except that a
// zero may carry either sign; butterfly128 undoes both in its final scale.
template <int M>
__device__ __forceinline__ void lane_stage_carried(float (&f)[8], int l16)
{
    const float c = (l16 & M) != 0 ? -1.0f : 1.0f;
    if constexpr (M == 4)
    {
        #pragma unroll
        for (int j = 0; j < 8; ++j) f[j] = __builtin_fmaf(lane_xor<M>(f[j]), c, f[j]);
    }
    else
    {
        // v_fmac_f32 with the partner read through DPP (hipcc does not fold a DPP move into an fmac).
        // The s_nop covers the two wait states a DPP read needs after a VALU write of the same
        // register; inside the block each source was last written 8 instructions earlier.
#define EXL3R_FMAC_DPP(CTRL)                                                                        \
    asm("s_nop 1\n"                                                                                  \
        "v_fmac_f32_dpp %0, %0, %8 " CTRL " row_mask:0xf bank_mask:0xf\n"                            \
        "v_fmac_f32_dpp %1, %1, %8 " CTRL " row_mask:0xf bank_mask:0xf\n"                            \
        "v_fmac_f32_dpp %2, %2, %8 " CTRL " row_mask:0xf bank_mask:0xf\n"                            \
        "v_fmac_f32_dpp %3, %3, %8 " CTRL " row_mask:0xf bank_mask:0xf\n"                            \
        "v_fmac_f32_dpp %4, %4, %8 " CTRL " row_mask:0xf bank_mask:0xf\n"                            \
        "v_fmac_f32_dpp %5, %5, %8 " CTRL " row_mask:0xf bank_mask:0xf\n"                            \
        "v_fmac_f32_dpp %6, %6, %8 " CTRL " row_mask:0xf bank_mask:0xf\n"                            \
        "v_fmac_f32_dpp %7, %7, %8 " CTRL " row_mask:0xf bank_mask:0xf"                               \
        : "+v"(f[0]), "+v"(f[1]), "+v"(f[2]), "+v"(f[3]), "+v"(f[4]), "+v"(f[5]), "+v"(f[6]), "+v"(f[7]) \
        : "v"(c))
        if constexpr (M == 1) EXL3R_FMAC_DPP("quad_perm:[1,0,3,2]");
        else if constexpr (M == 2) EXL3R_FMAC_DPP("quad_perm:[2,3,0,1]");
        else EXL3R_FMAC_DPP("row_ror:8");
#undef EXL3R_FMAC_DPP
    }
}

// Whether the carried-sign stages may stand in for the exact ones.  In the exact butterfly a result
// is -0 only if every input it depends on is a zero and one of them is -0 (a cancellation of non-zero
// values gives +0, and -0 comes only from (-0) + (-0) or (-0) - (+0)); each of the 128-point
// transform's results depends on all 128 inputs.  So unless some lane holds 8 zero inputs with a -0
// among them (zero_lane16), every zero result is +0, and fma(v, +-r, +0) turns the carried value's
// zero, of either sign, into +0 while it rounds every other product as r * value does (r > 0).
// Otherwise (zero blocks with -0 in them, r <= 0 or NaN) the wave takes the exact stages.
// The test on a lane's 8 f16 inputs as loaded (an f16 zero widens to the fp32 zero of its sign).
__device__ __forceinline__ bool zero_lane16(const TF16::Vec& v)
{
    const uint32_t o = v.a[0] | v.a[1] | v.a[2] | v.a[3];
    return ((o | (o >> 16)) & 0xffffu) == 0x8000u;
}
// Wave-uniform: no lane of the wave raised `zero` (zero_lane16 of any of its blocks) and r > 0.
__device__ __forceinline__ bool carried_ok(bool zero, float r)
{
    return r > 0.0f && __builtin_amdgcn_ballot_w64(zero) == 0;
}

// f = r * H128 (block) with r the transform's scale, rounded once after the fp32 butterfly; CARRIED:
// the carried-sign lane stages (only where carried_ok holds for the wave).  H0 = 2: f already holds the
// first in-lane stage (unpack8_stage1).
template <bool CARRIED, int H0 = 1>
__device__ __forceinline__ void butterfly128_t(float (&f)[8], int l16, float r)
{
    #pragma clang fp contract(off)
    #pragma unroll
    for (int h = H0; h < 8; h <<= 1)
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
    if constexpr (CARRIED)
    {
        lane_stage_carried<1>(f, l16);
        lane_stage_carried<2>(f, l16);
        lane_stage_carried<4>(f, l16);
        lane_stage_carried<8>(f, l16);
        const float sr = (__builtin_popcount(l16 & 15) & 1) ? -r : r;
        // opaque: the fp32 result is what gets rounded to a 16-bit output (an fma feeding the
        // conversion would otherwise become one mixed-precision fma that rounds the exact product).
        #pragma unroll
        for (int j = 0; j < 8; ++j) f[j] = opaque(__builtin_fmaf(f[j], sr, 0.0f));
    }
    else
    {
        lane_stage<1>(f, l16);
        lane_stage<2>(f, l16);
        lane_stage<4>(f, l16);
        lane_stage<8>(f, l16);
        #pragma unroll
        for (int j = 0; j < 8; ++j) f[j] = f[j] * r;
    }
}

// One block per call, exact stages (the callers that rotate one block at a time).
__device__ __forceinline__ void butterfly128(float (&f)[8], int l16, float r) { butterfly128_t<false>(f, l16, r); }

// The butterfly's first in-lane stage (pairs 2i, 2i + 1: the two halves of packed word i) straight from
// an f16 chunk: fl32(a + b) and fl32(a - b) as mixed-precision fmas a * 1 + (+-b), which convert both
// halves exactly and round once, as the fp32 add and subtract of the converted halves do (signed zeros
// included).  One instruction per element instead of a conversion and an add.
__device__ __forceinline__ void unpack8_stage1(const TF16::Vec& v, float (&f)[8])
{
    #pragma unroll
    for (int i = 0; i < 4; ++i)
    {
        const uint32_t w = v.a[i];
        asm("v_fma_mix_f32 %0, %1, 1.0, %1 op_sel:[0,0,1] op_sel_hi:[1,0,1]" : "=v"(f[2 * i]) : "v"(w));
        asm("v_fma_mix_f32 %0, %1, 1.0, -%1 op_sel:[0,0,1] op_sel_hi:[1,0,1]" : "=v"(f[2 * i + 1]) : "v"(w));
    }
}

// f = r * H128 of the f16 chunk v (its lane's share of the block).
template <bool CARRIED>
__device__ __forceinline__ void butterfly128_f16(const TF16::Vec& v, float (&f)[8], int l16, float r)
{
    unpack8_stage1(v, f);
    butterfly128_t<CARRIED, 2>(f, l16, r);
}

// Runs body(std::true_type) where the carried-sign stages are valid for the wave, else
// body(std::false_type): one wave-uniform branch around every butterfly of the body.  ENABLE false
// keeps the exact stages without the test (kernels whose time the butterfly does not set).
template <bool ENABLE, class Body>
__device__ __forceinline__ void with_carried(bool zero, float r, Body&& body)
{
    if constexpr (ENABLE)
    {
        if (carried_ok(zero, r)) body(std::true_type{});
        else body(std::false_type{});
    }
    else
        body(std::false_type{});
}

__device__ __forceinline__ uint32_t hmul2(uint32_t a, uint32_t b)
{
    return __builtin_bit_cast(uint32_t, __builtin_bit_cast(f16x2, a) * __builtin_bit_cast(f16x2, b));
}

// The EXL3 linear's output rotation had_r_128(y, y, None, post) (scale 1) of the 8-element f16 chunk
// at column col of a row, held as lane (col / 8) % 16 of its block's 16-lane group: the fp32
// butterfly, one rounding to f16, then the half post-scale product (post: f16 per column, or null).
template <bool CARRIED = false>
__device__ __forceinline__ void output_rotation8(TF16::Vec& v, const void* post, int64_t col)
{
    float f[8];
    butterfly128_f16<CARRIED>(v, f, (int)((col >> 3) & 15), 0.0883883461356163f);
    v = pack8<TF16>(f);
    if (post)
    {
        const TF16::Vec p = load8<TF16>(post, col);
        #pragma unroll
        for (int q = 0; q < 4; ++q) v.a[q] = hmul2(v.a[q], p.a[q]);
    }
}

}  // namespace exl3r
