// Device-side building blocks shared by the gfx950 row kernels:
//   - dtype tags with 8-element (16-byte per 16-bit tensor) vector load/store and exact
//     conversions (f16/bf16 -> f32 exact, f32 -> f16/bf16 round-to-nearest-even in hardware:
//     v_cvt_f16_f32 and gfx950's v_cvt_pk_bf16_f32);
//   - wave64 reductions built from DPP row ops (quad_perm / row_half_mirror / row_mirror) with
//     one readlane hop across the four 16-lane rows, and a single LDS hop across waves.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace exl3r {

enum : int { DT_F32 = 0, DT_F16 = 1, DT_BF16 = 2, DT_I32 = 3, DT_I64 = 4 };

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
// __builtin_bit_cast(T, vec[i]) of an element of one of these vectors reads element 0 with this
// compiler (the element lvalue is lowered as the vector's own address): every bit_cast here takes a
// value, e.g. (uint32_t)vec[i].

// ---------------------------------------------------------------------------------------------
// dtype tags.  Each tag loads/stores chunks of 8 consecutive elements; F16/BF16 chunks are one
// 16-byte access, F32 chunks two.

struct TNone
{
    static constexpr int code = -1;
    static constexpr int bytes = 0;
    struct Vec {};
};

struct TF32
{
    static constexpr int code = DT_F32;
    static constexpr int bytes = 4;
    struct Vec { u32x4 a, b; };
};
struct TF16
{
    static constexpr int code = DT_F16;
    static constexpr int bytes = 2;
    struct Vec { u32x4 a; };
};
struct TBF16
{
    static constexpr int code = DT_BF16;
    static constexpr int bytes = 2;
    struct Vec { u32x4 a; };
};

__device__ __forceinline__ float f16lo(uint32_t w) { return (float)__builtin_bit_cast(_Float16, (uint16_t)(w & 0xffffu)); }
__device__ __forceinline__ float f16hi(uint32_t w) { return (float)__builtin_bit_cast(_Float16, (uint16_t)(w >> 16)); }
__device__ __forceinline__ float bf16lo(uint32_t w) { return __builtin_bit_cast(float, w << 16); }
__device__ __forceinline__ float bf16hi(uint32_t w) { return __builtin_bit_cast(float, w & 0xffff0000u); }

__device__ __forceinline__ uint32_t pack_f16(float lo, float hi)
{
    f16x2 h = { (_Float16)lo, (_Float16)hi };
    return __builtin_bit_cast(uint32_t, h);
}
__device__ __forceinline__ uint32_t pack_bf16(float lo, float hi)
{
    f32x2 f = { lo, hi };
    bf16x2 h = __builtin_convertvector(f, bf16x2);
    return __builtin_bit_cast(uint32_t, h);
}

// Round an fp32 value to a 16-bit format and back (exact re-expansion).  A scalar
// (_Float16)(a * b) is selected as v_fma_mixlo_f16, which rounds the exact product once instead of
// the fp32 product (a different result when the fp32 product lands on an f16 tie).
// An empty asm statement hides the producing multiply from that pattern (it emits no instruction).
__device__ __forceinline__ float opaque(float v)
{
    asm volatile("" : "+v"(v));
    return v;
}
__device__ __forceinline__ _Float16 to_f16(float v) { return (_Float16)opaque(v); }

// fl32(h * c) for the f16 element h in the low (HI = false) or high half of a packed pair and an fp32 c,
// in one instruction: the mixed-precision fma converts h exactly and adds -0, which leaves every
// product as the fp32 multiply rounds it (x * c + -0 = x * c, signed zeros included).
// The compiler's hazard handling does not see the operands of inline assembly: a c just written by a
// transcendental instruction (v_exp, v_rcp, v_sqrt, ...) needs one wait state before it is read (without
// it the previous value of the register is read), which AFTER_TRANS = true puts in front.
template <bool HI, bool AFTER_TRANS = false>
__device__ __forceinline__ float mul_f16_f32(uint32_t pair, float c)
{
    float r;
    if constexpr (AFTER_TRANS && HI)
        asm("s_nop 0\nv_fma_mix_f32 %0, %1, %2, %3 op_sel:[1,0,0] op_sel_hi:[1,0,0]" : "=v"(r) : "v"(pair), "v"(c), "s"(-0.0f));
    else if constexpr (AFTER_TRANS)
        asm("s_nop 0\nv_fma_mix_f32 %0, %1, %2, %3 op_sel:[0,0,0] op_sel_hi:[1,0,0]" : "=v"(r) : "v"(pair), "v"(c), "s"(-0.0f));
    else if constexpr (HI)
        asm("v_fma_mix_f32 %0, %1, %2, %3 op_sel:[1,0,0] op_sel_hi:[1,0,0]" : "=v"(r) : "v"(pair), "v"(c), "s"(-0.0f));
    else
        asm("v_fma_mix_f32 %0, %1, %2, %3 op_sel:[0,0,0] op_sel_hi:[1,0,0]" : "=v"(r) : "v"(pair), "v"(c), "s"(-0.0f));
    return r;
}
__device__ __forceinline__ float round_f16(float v) { return (float)to_f16(v); }
__device__ __forceinline__ float round_bf16(float v) { return bf16lo(pack_bf16(v, 0.0f)); }

// load8: cached load (weights, embedding tables: reused across rows).  load8s: streaming load with
// the non-temporal hint for operands read exactly once.  store8: every output is written once per
// call, so all stores carry the non-temporal hint.  (Measured on MI355X: a 1 GiB copy reaches
// 6.2 TB/s plain and 6.6 TB/s non-temporal.)
template <class T> __device__ __forceinline__ typename T::Vec load8(const void* base, int64_t elem);
template <class T> __device__ __forceinline__ typename T::Vec load8s(const void* base, int64_t elem);
template <class T> __device__ __forceinline__ void store8(void* base, int64_t elem, const typename T::Vec& v);
template <class T> __device__ __forceinline__ void unpack8(const typename T::Vec& v, float (&f)[8]);
template <class T> __device__ __forceinline__ typename T::Vec pack8(const float (&f)[8]);
template <class T> __device__ __forceinline__ float round_to(float v);

template <> __device__ __forceinline__ TF16::Vec load8<TF16>(const void* base, int64_t e)
{
    return { *(const u32x4*)((const uint16_t*)base + e) };
}
template <> __device__ __forceinline__ TBF16::Vec load8<TBF16>(const void* base, int64_t e)
{
    return { *(const u32x4*)((const uint16_t*)base + e) };
}
template <> __device__ __forceinline__ TF32::Vec load8<TF32>(const void* base, int64_t e)
{
    // Members are assigned one by one: a braced {p[0], p[1]} would be brace-elided into the
    // elements of the first vector member.
    const u32x4* p = (const u32x4*)((const float*)base + e);
    TF32::Vec v;
    v.a = p[0];
    v.b = p[1];
    return v;
}

template <> __device__ __forceinline__ TF16::Vec load8s<TF16>(const void* base, int64_t e)
{
    return { __builtin_nontemporal_load((const u32x4*)((const uint16_t*)base + e)) };
}
template <> __device__ __forceinline__ TBF16::Vec load8s<TBF16>(const void* base, int64_t e)
{
    return { __builtin_nontemporal_load((const u32x4*)((const uint16_t*)base + e)) };
}
template <> __device__ __forceinline__ TF32::Vec load8s<TF32>(const void* base, int64_t e)
{
    const u32x4* p = (const u32x4*)((const float*)base + e);
    TF32::Vec v;
    v.a = __builtin_nontemporal_load(p);
    v.b = __builtin_nontemporal_load(p + 1);
    return v;
}

template <> __device__ __forceinline__ void store8<TF16>(void* base, int64_t e, const TF16::Vec& v)
{
    __builtin_nontemporal_store(v.a, (u32x4*)((uint16_t*)base + e));
}
template <> __device__ __forceinline__ void store8<TBF16>(void* base, int64_t e, const TBF16::Vec& v)
{
    __builtin_nontemporal_store(v.a, (u32x4*)((uint16_t*)base + e));
}
template <> __device__ __forceinline__ void store8<TF32>(void* base, int64_t e, const TF32::Vec& v)
{
    u32x4* p = (u32x4*)((float*)base + e);
    __builtin_nontemporal_store(v.a, p);
    __builtin_nontemporal_store(v.b, p + 1);
}

// Cached stores (no non-temporal hint): the L2 keeps the line, so the halves of a 128-byte line that two
// store instructions write are merged there before the line goes to HBM.
template <class T> __device__ __forceinline__ void store8c(void* base, int64_t elem, const typename T::Vec& v);
template <> __device__ __forceinline__ void store8c<TF16>(void* base, int64_t e, const TF16::Vec& v)
{
    *(u32x4*)((uint16_t*)base + e) = v.a;
}
template <> __device__ __forceinline__ void store8c<TBF16>(void* base, int64_t e, const TBF16::Vec& v)
{
    *(u32x4*)((uint16_t*)base + e) = v.a;
}
template <> __device__ __forceinline__ void store8c<TF32>(void* base, int64_t e, const TF32::Vec& v)
{
    u32x4* p = (u32x4*)((float*)base + e);
    p[0] = v.a;
    p[1] = v.b;
}

// Buffer accesses through a bounded descriptor: a row's base and its length in bytes.  A 16-byte load
// whose offset is at or past the length returns zeros and such a store writes nothing, so lanes and
// rows past the data need neither a branch nor a clamped address.  dword 3 = 0x00020000 (32-bit data
// format, raw addressing) for gfx9 (CDNA) buffer descriptors.  Offsets are 32-bit: rows under 4 GB.
typedef __amdgpu_buffer_rsrc_t brsrc;
constexpr int kBufNT = 2;   // cache policy bits of a non-temporal access (the nt bit)
__device__ __forceinline__ brsrc row_rsrc(const void* base, uint32_t bytes)
{
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, (int)bytes, 0x00020000);
}
__device__ __forceinline__ u32x4 bload16(brsrc r, uint32_t off) { return __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, 0); }
__device__ __forceinline__ u32x4 bload16s(brsrc r, uint32_t off)
{
    return __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, kBufNT);
}
__device__ __forceinline__ void bstore16(brsrc r, uint32_t off, u32x4 v)
{
    __builtin_amdgcn_raw_buffer_store_b128(v, r, off, 0, kBufNT);
}
// A chunk of 8 elements at byte offset off (8 * es bytes: one access, or two for f32).
template <class T> __device__ __forceinline__ typename T::Vec bload8s(brsrc r, uint32_t off)
{
    typename T::Vec v;
    v.a = bload16s(r, off);
    if constexpr (T::bytes == 4) v.b = bload16s(r, off + 16);
    return v;
}

// Split chunks: the 8 elements of a chunk are the quads at e and e + kSplitGap, each one 8-byte (16-bit
// data) or 16-byte (f32) access.  With lane l of a wave taking the quads at 4 l and 256 + 4 l of a
// 512-element span, each wave-wide access of an operand covers one contiguous range: 512 B, or 1 KB for
// f32, where an f32 chunk of 8 contiguous elements is two accesses that each touch every other 16 bytes
// of 2 KB (MI355X, RES_IN f16 x / f32 r / f16 y at [8192, 5120]: 89.3 -> 82 us).
constexpr int kSplitGap = 256;
// First element of chunk c: 8 c, or for split chunks (rows of whole 512-element spans, 64 consecutive
// chunks per wave) the quad at 4 (c % 64) of span c / 64, whose second half is kSplitGap further on.
template <bool SPLIT>
__device__ __forceinline__ int64_t chunk_elem(int64_t c)
{
    if constexpr (SPLIT) return ((c >> 6) << 9) + ((c & 63) << 2);
    else return c * 8;
}

template <class T> __device__ __forceinline__ typename T::Vec load8s_split(const void* base, int64_t e);
template <class T> __device__ __forceinline__ void store8_split(void* base, int64_t e, const typename T::Vec& v);

__device__ __forceinline__ u32x4 load16x2_split(const uint16_t* p)
{
    const u32x2 lo = __builtin_nontemporal_load((const u32x2*)p);
    const u32x2 hi = __builtin_nontemporal_load((const u32x2*)(p + kSplitGap));
    return u32x4{ lo.x, lo.y, hi.x, hi.y };
}
__device__ __forceinline__ void store16x2_split(uint16_t* p, u32x4 v)
{
    __builtin_nontemporal_store(u32x2{ v.x, v.y }, (u32x2*)p);
    __builtin_nontemporal_store(u32x2{ v.z, v.w }, (u32x2*)(p + kSplitGap));
}
template <> __device__ __forceinline__ TF16::Vec load8s_split<TF16>(const void* base, int64_t e)
{
    return { load16x2_split((const uint16_t*)base + e) };
}
template <> __device__ __forceinline__ TBF16::Vec load8s_split<TBF16>(const void* base, int64_t e)
{
    return { load16x2_split((const uint16_t*)base + e) };
}
template <> __device__ __forceinline__ TF32::Vec load8s_split<TF32>(const void* base, int64_t e)
{
    const float* p = (const float*)base + e;
    TF32::Vec v;
    v.a = __builtin_nontemporal_load((const u32x4*)p);
    v.b = __builtin_nontemporal_load((const u32x4*)(p + kSplitGap));
    return v;
}
// Cached form (hot embedding-table rows).
template <class T> __device__ __forceinline__ typename T::Vec load8_split(const void* base, int64_t e);
__device__ __forceinline__ u32x4 load16x2_split_cached(const uint16_t* p)
{
    const u32x2 lo = *(const u32x2*)p, hi = *(const u32x2*)(p + kSplitGap);
    return u32x4{ lo.x, lo.y, hi.x, hi.y };
}
template <> __device__ __forceinline__ TF16::Vec load8_split<TF16>(const void* base, int64_t e)
{
    return { load16x2_split_cached((const uint16_t*)base + e) };
}
template <> __device__ __forceinline__ TBF16::Vec load8_split<TBF16>(const void* base, int64_t e)
{
    return { load16x2_split_cached((const uint16_t*)base + e) };
}
template <> __device__ __forceinline__ TF32::Vec load8_split<TF32>(const void* base, int64_t e)
{
    const float* p = (const float*)base + e;
    TF32::Vec v;
    v.a = *(const u32x4*)p;
    v.b = *(const u32x4*)(p + kSplitGap);
    return v;
}

template <> __device__ __forceinline__ void store8_split<TF16>(void* base, int64_t e, const TF16::Vec& v)
{
    store16x2_split((uint16_t*)base + e, v.a);
}
template <> __device__ __forceinline__ void store8_split<TBF16>(void* base, int64_t e, const TBF16::Vec& v)
{
    store16x2_split((uint16_t*)base + e, v.a);
}
template <> __device__ __forceinline__ void store8_split<TF32>(void* base, int64_t e, const TF32::Vec& v)
{
    float* p = (float*)base + e;
    __builtin_nontemporal_store(v.a, (u32x4*)p);
    __builtin_nontemporal_store(v.b, (u32x4*)(p + kSplitGap));
}

template <> __device__ __forceinline__ void unpack8<TF16>(const TF16::Vec& v, float (&f)[8])
{
    #pragma unroll
    for (int i = 0; i < 4; ++i) { f[2 * i] = f16lo(v.a[i]); f[2 * i + 1] = f16hi(v.a[i]); }
}
template <> __device__ __forceinline__ void unpack8<TBF16>(const TBF16::Vec& v, float (&f)[8])
{
    #pragma unroll
    for (int i = 0; i < 4; ++i) { f[2 * i] = bf16lo(v.a[i]); f[2 * i + 1] = bf16hi(v.a[i]); }
}
// F32 chunks are reinterpreted as whole float vectors before element access: with the packed-fp32
// VALU forms disabled, hipcc (ROCm 7.2) lowers a bit_cast of a single u32x4 element to a broadcast of
// element 0, while a whole-vector bit_cast is lowered correctly.
template <> __device__ __forceinline__ void unpack8<TF32>(const TF32::Vec& v, float (&f)[8])
{
    const f32x4 a = __builtin_bit_cast(f32x4, v.a);
    const f32x4 b = __builtin_bit_cast(f32x4, v.b);
    #pragma unroll
    for (int i = 0; i < 4; ++i) { f[i] = a[i]; f[4 + i] = b[i]; }
}

template <> __device__ __forceinline__ TF16::Vec pack8<TF16>(const float (&f)[8])
{
    TF16::Vec v;
    #pragma unroll
    for (int i = 0; i < 4; ++i) v.a[i] = pack_f16(f[2 * i], f[2 * i + 1]);
    return v;
}
template <> __device__ __forceinline__ TBF16::Vec pack8<TBF16>(const float (&f)[8])
{
    TBF16::Vec v;
    #pragma unroll
    for (int i = 0; i < 4; ++i) v.a[i] = pack_bf16(f[2 * i], f[2 * i + 1]);
    return v;
}
template <> __device__ __forceinline__ TF32::Vec pack8<TF32>(const float (&f)[8])
{
    f32x4 a, b;
    #pragma unroll
    for (int i = 0; i < 4; ++i) { a[i] = f[i]; b[i] = f[4 + i]; }
    TF32::Vec v;
    v.a = __builtin_bit_cast(u32x4, a);
    v.b = __builtin_bit_cast(u32x4, b);
    return v;
}

template <> __device__ __forceinline__ float round_to<TF32>(float v) { return v; }
template <> __device__ __forceinline__ float round_to<TF16>(float v) { return round_f16(v); }
template <> __device__ __forceinline__ float round_to<TBF16>(float v) { return round_bf16(v); }

// Scalar element access (generic fallback kernels).
__device__ __forceinline__ float load1(const void* p, int dt, int64_t i)
{
    if (dt == DT_F16) return (float)((const _Float16*)p)[i];
    if (dt == DT_BF16) return __builtin_bit_cast(float, (uint32_t)((const uint16_t*)p)[i] << 16);
    return ((const float*)p)[i];
}
__device__ __forceinline__ void store1(void* p, int dt, int64_t i, float v)
{
    if (dt == DT_F16) ((_Float16*)p)[i] = to_f16(v);
    else if (dt == DT_BF16) ((uint16_t*)p)[i] = (uint16_t)(pack_bf16(v, 0.0f) & 0xffffu);
    else ((float*)p)[i] = v;
}
__device__ __forceinline__ float round1(float v, int dt)
{
    if (dt == DT_F16) return round_f16(v);
    if (dt == DT_BF16) return round_bf16(v);
    return v;
}

// 8 elements of a runtime-typed vector (norm weights: tiny, L2-resident, uniform branch).
__device__ __forceinline__ void load8_dyn(const void* base, int dt, int64_t e, float (&f)[8])
{
    if (dt == DT_F16) unpack8<TF16>(load8<TF16>(base, e), f);
    else if (dt == DT_BF16) unpack8<TBF16>(load8<TBF16>(base, e), f);
    else unpack8<TF32>(load8<TF32>(base, e), f);
}

// Reciprocal RMS factor from an fp64 sum of squares: the sum is rounded once to fp32, then
// mean = sum / n, and 1 / sqrt(mean + eps) with IEEE-correct fp32 sqrt and division (hipcc's
// default), so the CPU oracle reproduces it bit-for-bit.  (An fp32 sum enters the same way.)
__device__ __forceinline__ float rms_factor(double sum, int n, float eps)
{
    const float mean = (float)sum / (float)n;
    return 1.0f / sqrtf(mean + eps);
}
__device__ __forceinline__ float rms_factor(float sum, int n, float eps)
{
    const float mean = sum / (float)n;
    return 1.0f / sqrtf(mean + eps);
}

// ---------------------------------------------------------------------------------------------
// Activations in fp32, each a product m * sigmoid(z): SiLU m = x, z = x; GELU(tanh) m = x,
// z = 2 sqrt(2/pi) (x + 0.044715 x^3) (0.5 (1 + tanh(u)) = sigmoid(2u), no 1 + tanh cancellation for
// x << 0); SIGMOID m = 1, z = x.  With e^-z = 2^t, sigmoid = 1 / (1 + 2^t): one v_exp_f32 and one
// v_rcp_f32, both within 1 ulp, for any t <= 64 (2^t normal or below 2^-64, where 1 + 2^t == 1; the
// reciprocal's argument in [1, 2^64 + 1], its result normal).  For t > 64 (sigmoid < 2^-64, where
// 1 / (1 + 2^t) == 2^-t to fp32 precision) 2^-t is evaluated as 2^(64 - t) and the 2^-64 is applied
// to the final product, so tail results keep full precision down into the fp32 denormals instead of
// flushing inside v_exp_f32.
enum { ACT_SILU = 0, ACT_GELU = 1, ACT_SIGMOID = 2 };

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kGeluK1 = (float)(-2.0 * 0.79788456080286535588 * 1.4426950408889634074);
constexpr float kGeluK2 = (float)(-2.0 * 0.79788456080286535588 * 0.044715 * 1.4426950408889634074);

// t with e^-z = 2^t.
template <int ACT>
__device__ __forceinline__ float act_t(float x)
{
    if constexpr (ACT == ACT_GELU) return x * fmaf(kGeluK2, x * x, kGeluK1);
    else return x * -kLog2e;
}

// act_f for a t <= 64 or NaN (no tail scaling): the same operations and results as act_f there.
template <int ACT>
__device__ __forceinline__ float act_f_short(float x, float t)
{
    const float s = __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(t));
    return ACT == ACT_SIGMOID ? s : x * s;
}

template <int ACT>
__device__ __forceinline__ float act_f(float x)
{
    const float t = act_t<ACT>(x);   // e^-z = 2^t
    const bool tail = t > 64.0f;
    const float e = __builtin_amdgcn_exp2f(tail ? 64.0f - t : t);   // tail: normal for t <= 190
    const float s = tail ? e : __builtin_amdgcn_rcpf(1.0f + e);
    const float r = ACT == ACT_SIGMOID ? s : x * s;
    return tail ? r * 0x1p-64f : r;
}

// CLAMP_FP16: +-inf -> +-65504, NaN -> 65504, the results of max(-65504, min(v, 65504)) with IEEE
// min / max (which return the non-NaN operand), in one instruction: -med3(-v, -65504, 65504).
// v_med3_f32 returns the min3 of its operands when one is NaN (-65504 here), so NaN maps to +65504;
// -0 and +0 pass through with their signs.  Inline assembly, because the compiler folds the two
// negations away (med3(v, 65504, -65504)), which would map NaN to -65504.
// v must not come straight from a transcendental instruction (see mul_f16_f32: the wait state the
// compiler would put in front of a read of it is not put in front of inline assembly).
__device__ __forceinline__ float nclamp_f16(float v)   // -CLAMP_FP16(v)
{
    float c;
    asm("v_med3_f32 %0, -%1, -%2, %2" : "=v"(c) : "v"(v), "s"(65504.0f));
    return c;
}
__device__ __forceinline__ float clamp_f16(float v) { return -nclamp_f16(v); }

// ---------------------------------------------------------------------------------------------
// Reductions.

template <int CTRL>
__device__ __forceinline__ float dpp(float v)
{
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xf, 0xf, false));
}

constexpr int DPP_QUAD_XOR1 = 0xb1;       // quad_perm [1,0,3,2]
constexpr int DPP_QUAD_XOR2 = 0x4e;       // quad_perm [2,3,0,1]
constexpr int DPP_ROW_HALF_MIRROR = 0x141;
constexpr int DPP_ROW_MIRROR = 0x140;
constexpr int DPP_ROW_ROR8 = 0x128;

// Sum over aligned groups of W lanes (W = 1, 2, 4, ..., 64); every lane of a group gets the sum.
// Must be called with the whole wave active.
template <int W>
__device__ __forceinline__ float group_sum(float v)
{
    if constexpr (W >= 2) v += dpp<DPP_QUAD_XOR1>(v);
    if constexpr (W >= 4) v += dpp<DPP_QUAD_XOR2>(v);
    if constexpr (W >= 8) v += dpp<DPP_ROW_HALF_MIRROR>(v);
    if constexpr (W >= 16) v += dpp<DPP_ROW_MIRROR>(v);
    if constexpr (W >= 32)
        v += __builtin_bit_cast(float, __builtin_amdgcn_ds_swizzle(__builtin_bit_cast(int, v), 0x401f)); // xor 16
    if constexpr (W >= 64)
        v += __shfl_xor(v, 32);
    return v;
}

template <int CTRL>
__device__ __forceinline__ double dpp64(double v)
{
    const uint64_t u = __builtin_bit_cast(uint64_t, v);
    const int lo = __builtin_amdgcn_update_dpp(0, (int)(uint32_t)u, CTRL, 0xf, 0xf, false);
    const int hi = __builtin_amdgcn_update_dpp(0, (int)(uint32_t)(u >> 32), CTRL, 0xf, 0xf, false);
    return __builtin_bit_cast(double, ((uint64_t)(uint32_t)hi << 32) | (uint32_t)lo);
}

// fp64 group sum (as group_sum): used where the statistic must match a double-precision oracle
// bit-for-bit after rounding to fp32.
template <int W>
__device__ __forceinline__ double group_sum64(double v)
{
    if constexpr (W >= 2) v += dpp64<DPP_QUAD_XOR1>(v);
    if constexpr (W >= 4) v += dpp64<DPP_QUAD_XOR2>(v);
    if constexpr (W >= 8) v += dpp64<DPP_ROW_HALF_MIRROR>(v);
    if constexpr (W >= 16) v += dpp64<DPP_ROW_MIRROR>(v);
    if constexpr (W >= 32) v += __shfl_xor(v, 16);
    if constexpr (W >= 64) v += __shfl_xor(v, 32);
    return v;
}

// v(l) + v(l ^ 16) in every lane l: v_permlane16_swap_b32 of v with itself hands both lanes of a pair
// the pair's two values in the same order (the even row's first), so both get the same bits.  Both
// lanes of a pair must be active.
__device__ __forceinline__ float sum_xor16(float v)
{
    const uint32_t u = __builtin_bit_cast(uint32_t, v);
    const auto p = __builtin_amdgcn_permlane16_swap(u, u, false, false);
    return __builtin_bit_cast(float, (uint32_t)p[0]) + __builtin_bit_cast(float, (uint32_t)p[1]);
}
__device__ __forceinline__ double sum_xor16(double v)
{
    const uint64_t u = __builtin_bit_cast(uint64_t, v);
    const uint32_t lo = (uint32_t)u, hi = (uint32_t)(u >> 32);
    const auto pl = __builtin_amdgcn_permlane16_swap(lo, lo, false, false);
    const auto ph = __builtin_amdgcn_permlane16_swap(hi, hi, false, false);
    const double a = __builtin_bit_cast(double, ((uint64_t)(uint32_t)ph[0] << 32) | (uint32_t)pl[0]);
    const double b = __builtin_bit_cast(double, ((uint64_t)(uint32_t)ph[1] << 32) | (uint32_t)pl[1]);
    return a + b;
}

// v(l) + v(l ^ 32) in every lane l, the same bits in both (v_permlane32_swap_b32 of v with itself: the
// lower half's value first).  Both lanes of a pair must be active.
__device__ __forceinline__ double sum_xor32(double v)
{
    const uint64_t u = __builtin_bit_cast(uint64_t, v);
    const uint32_t lo = (uint32_t)u, hi = (uint32_t)(u >> 32);
    const auto pl = __builtin_amdgcn_permlane32_swap(lo, lo, false, false);
    const auto ph = __builtin_amdgcn_permlane32_swap(hi, hi, false, false);
    const double a = __builtin_bit_cast(double, ((uint64_t)(uint32_t)ph[0] << 32) | (uint32_t)pl[0]);
    const double b = __builtin_bit_cast(double, ((uint64_t)(uint32_t)ph[1] << 32) | (uint32_t)pl[1]);
    return a + b;
}

// Full-wave sum, uniform result: row sums by DPP, then the four rows combined through readlane.
__device__ __forceinline__ float wave_sum(float v)
{
    v = group_sum<16>(v);
    int iv = __builtin_bit_cast(int, v);
    float r0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(iv, 0));
    float r1 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(iv, 16));
    float r2 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(iv, 32));
    float r3 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(iv, 48));
    return (r0 + r1) + (r2 + r3);
}

// Workgroup sum (blockDim.x a multiple of 64, at most 1024): one LDS hop across waves.  Every
// thread gets the same value (all waves add the partials in the same order).
__device__ __forceinline__ float block_sum(float v, float* lds16)
{
    v = wave_sum(v);
    const int nw = blockDim.x >> 6;
    if (nw == 1) return v;
    if ((threadIdx.x & 63) == 0) lds16[threadIdx.x >> 6] = v;
    __syncthreads();
    float t = 0.0f;
    for (int i = 0; i < nw; ++i) t += lds16[i];
    return t;
}

// fp64 workgroup sum through LDS (lds must hold one double per wave).
__device__ __forceinline__ double block_sum64(double v, double* lds16)
{
    v = group_sum64<64>(v);
    const int nw = blockDim.x >> 6;
    if (nw == 1) return v;
    if ((threadIdx.x & 63) == 0) lds16[threadIdx.x >> 6] = v;
    __syncthreads();
    double t = 0.0;
    for (int i = 0; i < nw; ++i) t += lds16[i];
    __syncthreads();
    return t;
}

// fp64 workgroup sum with a single barrier, for a workgroup that reduces once: its LDS slots are
// never written again, so no second barrier is needed before the kernel ends.
__device__ __forceinline__ double block_sum64_once(double v, double* lds16)
{
    v = group_sum64<64>(v);
    const int nw = blockDim.x >> 6;
    if (nw == 1) return v;
    if ((threadIdx.x & 63) == 0) lds16[threadIdx.x >> 6] = v;
    __syncthreads();
    double t = 0.0;
    for (int i = 0; i < nw; ++i) t += lds16[i];
    return t;
}

// Workgroup sum with a single barrier (see block_sum64_once), for an fp64 or fp32 partial.
__device__ __forceinline__ double block_sum_once(double v, double* lds16) { return block_sum64_once(v, lds16); }
__device__ __forceinline__ float block_sum_once(float v, float* lds16)
{
    v = group_sum<64>(v);
    const int nw = blockDim.x >> 6;
    if (nw == 1) return v;
    if ((threadIdx.x & 63) == 0) lds16[threadIdx.x >> 6] = v;
    __syncthreads();
    float t = 0.0f;
    for (int i = 0; i < nw; ++i) t += lds16[i];
    return t;
}

// ---------------------------------------------------------------------------------------------
// Host-side runtime dtype -> tag dispatch.

template <class F>
inline bool with_float_type(int dt, F&& f)
{
    switch (dt)
    {
        case DT_F32: f(TF32{}); return true;
        case DT_F16: f(TF16{}); return true;
        case DT_BF16: f(TBF16{}); return true;
        default: return false;
    }
}

}  // namespace exl3r
