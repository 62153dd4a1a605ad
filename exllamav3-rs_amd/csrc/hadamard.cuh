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

// ---------------------------------------------------------------------------------------------
// The 128-point transform on the matrix cores.  H128 is the tensor product of the 2-point transforms
// over the 7 index bits, which can be applied in any grouping: bits {0, 1, 2, 5, 6} are contracted by
// v_mfma_f32_16x16x32_f16 against +-1 f16 operands (the f16 products are exact; the 32-term sums are
// fp32), bits {3, 4} by two carried-sign DPP stages inside each lane quad.  Per 4 blocks (512
// elements) that is 2 MFMAs and 16 DPP fmas per lane, against 24 in-lane and 32 cross-lane
// operations per lane for the butterfly.  The sums are grouped differently from the reference's
// butterfly (kernels/quant/hadamard_inner.cuh:19-46, 127-141), so the fp32 results can differ from it
// by rounding: each is within about 2^-20 * sum|x| of the exact transform, and after the rounding to
// f16 a result equals the butterfly's or is its f16 neighbour, except where the transform cancels to
// below ~2^-17 * r * sum|x| (there both are that close to the exact value).  Zero results are +0.
//
// Lane placement: a wave holds 4 consecutive blocks of one row (64 chunks of 8 elements).  Lane
// l = 16 g + j (j = l & 15, g = l >> 4) holds chunk mfma_chunk(l) = (l & 3) + 4 g + 16 (j >> 2) of the
// span: elements 8 (l & 3) + 32 g + 0..7 of block j >> 2.  Each lane quad reads 64 contiguous bytes of
// 16-bit data and a wave-wide access covers the span's 1 KB.  As MFMA operands, B[k][j] is the data of
// segment j (block j >> 2, index bits 3-4 = j & 3) at k = (index bits 5-6 = g, bits 0-2 = slot), and
// the result rows come back to the lanes that loaded them: D lane l, slot v of MFMA h is index bits
// 0-2 = 4 h + v and bits 5-6 = g, so after the two MFMAs every lane holds its own 8 positions.

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

// Chunk of a 64-chunk span held by lane l (swaps lane bits 2-3 with bits 4-5; its own inverse).
__device__ __forceinline__ int mfma_chunk(int lane) { return (lane & 3) | ((lane >> 2) & 12) | ((lane << 2) & 48); }

// The lane's A operands of the two MFMAs: A_h[i][k] = (-1)^(popcount(go & gk) + popcount((4h + v) & e))
// for row i = 4 go + v (i = lane & 15) and k = 8 gk + e (gk = lane >> 4, slot e).
struct HadMfma
{
    f16x8 a[2];
};

__device__ __forceinline__ HadMfma had_mfma_operands(int lane)
{
    const int go = (lane & 15) >> 2, v = lane & 3, gk = lane >> 4;
    const int pg = __builtin_popcount(go & gk);
    HadMfma H;
    #pragma unroll
    for (int h = 0; h < 2; ++h)
    {
        #pragma unroll
        for (int e = 0; e < 8; ++e)
            H.a[h][e] = ((pg + __builtin_popcount((4 * h + v) & e)) & 1) ? (_Float16)-1.0f : (_Float16)1.0f;
    }
    return H;
}

// The same operands from two words per lane, for kernels short of registers: A_0[e] depends on e only
// through e & 3 (v < 4), so A_0 = {w0, w1, w0, w1} as f16 pairs, and A_1[e] = A_0[e] * (-1)^(e >> 2),
// A_1 = {w0, w1, -w0, -w1}.  had128_mfma_issue_w (below) forms them where the MFMAs are issued.
struct HadMfmaWords
{
    uint32_t w0, w1;
};

__device__ __forceinline__ HadMfmaWords had_mfma_words(int lane)
{
    const HadMfma H = had_mfma_operands(lane);
    return { __builtin_bit_cast(uint32_t, __builtin_shufflevector(H.a[0], H.a[0], 0, 1)),
             __builtin_bit_cast(uint32_t, __builtin_shufflevector(H.a[0], H.a[0], 2, 3)) };
}

// The transform in three steps, so that a caller can issue the MFMAs of several blocks before reading
// any result:
//   had128_mfma_issue: the two MFMAs of the lane's f16 chunk v (must be reached by the whole wave: the
//     MFMA reads every lane; lanes past the data pass zeros and drop the result);
//   mfma_wait: the wait states a VALU read of an MFMA result needs (a 16x16x32 f16 MFMA is 4 passes,
//     under 12 wait states; 16 here), taking the results of the batch as operands so that none of their
//     MFMAs is issued after it; the DPP stages below are inline asm, which the compiler's hazard
//     handling does not see into;
//   had128_mfma_finish: the two carried-sign stages and the scale: f = r * H128 of the block, fp32,
//     before the rounding to the output type.
struct MfmaOut
{
    f32x4 d0, d1;
};

__device__ __forceinline__ MfmaOut had128_mfma_issue(const HadMfma& H, const TF16::Vec& v)
{
    const f16x8 b = __builtin_bit_cast(f16x8, v.a);
    const f32x4 zero = { 0.0f, 0.0f, 0.0f, 0.0f };
    return { __builtin_amdgcn_mfma_f32_16x16x32_f16(H.a[0], b, zero, 0, 0, 0),
             __builtin_amdgcn_mfma_f32_16x16x32_f16(H.a[1], b, zero, 0, 0, 0) };
}

// had128_mfma_issue of one or two chunks from the two words, with one 4-VGPR operand: the MFMAs of A_0
// first, then its upper words negated in place (A_1) for the others.  The empty asm makes the words look
// new at each use, so that the operand is formed here and not kept live between uses.
__device__ __forceinline__ void had128_mfma_issue_w(HadMfmaWords w, const TF16::Vec& v0, MfmaOut& m0)
{
    asm volatile("" : "+v"(w.w0), "+v"(w.w1));
    typedef uint32_t u32x4v __attribute__((ext_vector_type(4)));
    u32x4v a = { w.w0, w.w1, w.w0, w.w1 };
    const f32x4 zero = { 0.0f, 0.0f, 0.0f, 0.0f };
    const f16x8 b0 = __builtin_bit_cast(f16x8, v0.a);
    m0.d0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), b0, zero, 0, 0, 0);
    a.z ^= 0x80008000u;
    a.w ^= 0x80008000u;
    m0.d1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), b0, zero, 0, 0, 0);
}
__device__ __forceinline__ void had128_mfma_issue_w(HadMfmaWords w, const TF16::Vec& v0, const TF16::Vec& v1,
                                                    MfmaOut& m0, MfmaOut& m1)
{
    asm volatile("" : "+v"(w.w0), "+v"(w.w1));
    typedef uint32_t u32x4v __attribute__((ext_vector_type(4)));
    u32x4v a = { w.w0, w.w1, w.w0, w.w1 };
    const f32x4 zero = { 0.0f, 0.0f, 0.0f, 0.0f };
    const f16x8 b0 = __builtin_bit_cast(f16x8, v0.a), b1 = __builtin_bit_cast(f16x8, v1.a);
    m0.d0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), b0, zero, 0, 0, 0);
    m1.d0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), b1, zero, 0, 0, 0);
    a.z ^= 0x80008000u;
    a.w ^= 0x80008000u;
    m0.d1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), b0, zero, 0, 0, 0);
    m1.d1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), b1, zero, 0, 0, 0);
}
template <int N>
__device__ __forceinline__ void had128_mfma_issue_w(HadMfmaWords w, const TF16::Vec (&v)[N], MfmaOut (&m)[N])
{
    asm volatile("" : "+v"(w.w0), "+v"(w.w1));
    typedef uint32_t u32x4v __attribute__((ext_vector_type(4)));
    u32x4v a = { w.w0, w.w1, w.w0, w.w1 };
    const f32x4 zero = { 0.0f, 0.0f, 0.0f, 0.0f };
    #pragma unroll
    for (int n = 0; n < N; ++n)
        m[n].d0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, v[n].a),
                                                        zero, 0, 0, 0);
    a.z ^= 0x80008000u;
    a.w ^= 0x80008000u;
    #pragma unroll
    for (int n = 0; n < N; ++n)
        m[n].d1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, v[n].a),
                                                        zero, 0, 0, 0);
}

__device__ __forceinline__ void mfma_wait(MfmaOut& a)
{
    asm volatile("s_nop 7\ns_nop 7" : "+v"(a.d0), "+v"(a.d1));
}
__device__ __forceinline__ void mfma_wait(MfmaOut& a, MfmaOut& b)
{
    asm volatile("s_nop 7\ns_nop 7" : "+v"(a.d0), "+v"(a.d1), "+v"(b.d0), "+v"(b.d1));
}
__device__ __forceinline__ void mfma_wait(MfmaOut& a, MfmaOut& b, MfmaOut& c, MfmaOut& d)
{
    asm volatile("s_nop 7\ns_nop 7" : "+v"(a.d0), "+v"(a.d1), "+v"(b.d0), "+v"(b.d1), "+v"(c.d0), "+v"(c.d1), "+v"(d.d0),
                 "+v"(d.d1));
}

__device__ __forceinline__ void had128_mfma_finish(const MfmaOut& m, float (&f)[8], int lane, float r)
{
    #pragma unroll
    for (int i = 0; i < 4; ++i)
    {
        f[i] = m.d0[i];
        f[4 + i] = m.d1[i];
    }
    lane_stage_carried<1>(f, lane);
    lane_stage_carried<2>(f, lane);
    // The two carried stages leave (-1)^popcount(lane & 3) times the transform; the scale undoes it.
    const float sr = (__builtin_popcount(lane & 3) & 1) ? -r : r;
    #pragma unroll
    for (int j = 0; j < 8; ++j) f[j] = opaque(__builtin_fmaf(f[j], sr, 0.0f));
}

// f = r * H128 of the lane's f16 chunk v, one block on its own (issue, wait, finish).
__device__ __forceinline__ void had128_mfma(const HadMfma& H, const TF16::Vec& v, float (&f)[8], int lane, float r)
{
    MfmaOut m = had128_mfma_issue(H, v);
    mfma_wait(m);
    had128_mfma_finish(m, f, lane, r);
}

// The f16 post-scale product of an output rotation's chunk (none when post is null).
__device__ __forceinline__ void post_scale8(TF16::Vec& v, const void* post, int64_t col)
{
    if (post)
    {
        const TF16::Vec p = load8<TF16>(post, col);
        #pragma unroll
        for (int q = 0; q < 4; ++q) v.a[q] = hmul2(v.a[q], p.a[q]);
    }
}

// A batch of N (1, 2, 4, 8) transforms' results through one wait.
template <int N>
__device__ __forceinline__ void mfma_wait_all(MfmaOut (&m)[N])
{
    static_assert(N == 1 || N == 2 || N == 4 || N == 8, "batches of 1, 2, 4 or 8");
    if constexpr (N == 1) mfma_wait(m[0]);
    else if constexpr (N == 2) mfma_wait(m[0], m[1]);
    else if constexpr (N == 4) mfma_wait(m[0], m[1], m[2], m[3]);
    else
    {
        mfma_wait(m[0], m[1], m[2], m[3]);
        mfma_wait(m[4], m[5], m[6], m[7]);
    }
}

// The EXL3 linear's output rotation had_r_128(y, y, None, post) (scale 1) of N f16 chunks at columns
// col[n] (mfma_chunk placement), their MFMAs issued together: each transform, one rounding to f16, then
// the half post-scale (post[n] null: none).
template <int N>
__device__ __forceinline__ void output_rotations_mfma(const HadMfma& H, TF16::Vec* v, const void* const* post,
                                                      const int64_t* col, int lane)
{
    MfmaOut m[N];
    #pragma unroll
    for (int n = 0; n < N; ++n) m[n] = had128_mfma_issue(H, v[n]);
    mfma_wait_all(m);
    #pragma unroll
    for (int n = 0; n < N; ++n)
    {
        float f[8];
        had128_mfma_finish(m[n], f, lane, 0.0883883461356163f);
        v[n] = pack8<TF16>(f);
        post_scale8(v[n], post[n], col[n]);
    }
}

}  // namespace exl3r
