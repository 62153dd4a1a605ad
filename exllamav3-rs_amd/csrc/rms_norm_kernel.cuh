// RMSNorm kernel family for gfx950: plain, residual-add-fused (RES_IN) and embedding-gather-fused.
//
// Semantics follow rms_norm_kernel (reference kernels/norm.cu:160-304):
//   f16 x is clamped to +-65504 on read (norm.cu:42-58, 192-196); RES_IN rounds x + r to r's dtype,
//   writes it back to r and normalises the rounded sum (norm.cu:198-223); the sum of squares is an
//   FMA chain (norm.cu:101-108; carried in fp64 here); rmf = rsqrt(sum / dim + eps) * constant_scale
//   (norm.cu:273; IEEE fp32 sqrt and divide here);
//   y = (x * (w + constant_bias)) * rmf in fp32, rounded once (norm.cu:110-124, 232-239, 75-83).
//
// Layout: one row per wave (rows up to 8192 elements) or per workgroup (longer rows).  A row is split
// into chunks of 8 elements; lane t owns chunks t, t + nt, ... (at most MAXV), so every wave-wide
// access is 64 lanes x 16 bytes contiguous.
// The whole row stays in VGPRs between the reduction and the output pass: one HBM read of x (and r),
// one write of y (and r) per row -- the 4-pass minimum for RES_IN, where the reference re-reads r
// at dim > 4096.  The row reduction is a DPP butterfly inside the wave (plus one LDS hop across waves
// for workgroup-per-row).
#pragma once

#include "abi.hpp"
#include "common.cuh"

#include <type_traits>

namespace exl3r {

enum { RMS_PLAIN = 0, RMS_RES_IN = 1, RMS_GATHER = 2 };

struct RmsArgs
{
    const void* x;      // input rows; RMS_GATHER: the embedding table
    int64_t ldx;
    const void* w;      // [dim] weight or nullptr
    int wt;
    void* y;
    int64_t ldy;
    void* r;            // RMS_RES_IN: residual (in/out); RMS_GATHER: optional gathered-row output h
    int64_t ldr;
    const void* ids;    // RMS_GATHER: [rows] token ids (I32 or I64, see idt)
    int idt;
    int64_t vocab;
    int32_t* err;       // RMS_GATHER: device error flag or nullptr
    int64_t rows;
    int dim;
    float eps, cb, cs;
    int xcd;            // XCD-sliced row order (single-pass grids)
};

__device__ __forceinline__ int64_t load_id(const void* ids, int idt, int64_t i)
{
    return idt == DT_I64 ? ((const int64_t*)ids)[i] : (int64_t)((const int32_t*)ids)[i];
}

// Weight chunks are prefetched as one 16-byte access before the row reduction (the whole chunk
// for F16/BF16 weights, the first four floats for F32 weights, whose second half is fetched after
// the reduction), so the L2 fetch overlaps the reduction at 4 VGPRs per chunk.
__device__ __forceinline__ u32x4 prefetch_w8(const void* w, int wt, int64_t e)
{
    return *(const u32x4*)((const char*)w + e * (wt == DT_F32 ? 4 : 2));
}

__device__ __forceinline__ void unpack_w8(u32x4 pre, const void* w, int wt, int64_t e, float (&f)[8])
{
    if (wt == DT_F16) { TF16::Vec v; v.a = pre; unpack8<TF16>(v, f); }
    else if (wt == DT_BF16) { TBF16::Vec v; v.a = pre; unpack8<TBF16>(v, f); }
    else
    {
        TF32::Vec v;
        v.a = pre;
        v.b = *(const u32x4*)((const float*)w + e + 4);
        unpack8<TF32>(v, f);
    }
}

// One row: x (and r) loaded in chunks c = tid, tid + nt, ... (at most MAXV per lane), every load
// issued before any arithmetic; the row is reduced either inside one wave (WAVE: nt == 64, DPP +
// swizzle butterfly, no LDS) or across the workgroup (one LDS hop).
template <class XT, class YT, class RT, int MAXV, int MODE, bool WAVE>
__device__ __forceinline__ void rms_row(const RmsArgs& a, int64_t row, int tid, int nt, double* red)
{
    const int nc = a.dim >> 3;
    const bool has_w = a.w != nullptr;
    const char* xrow;
    bool valid = true;
    if constexpr (MODE == RMS_GATHER)
    {
        int64_t id = load_id(a.ids, a.idt, row);
        valid = id >= 0 && id < a.vocab;
        if (!valid)
        {
            if (tid == 0 && a.err) atomicOr(a.err, 1);
            id = 0;
        }
        xrow = (const char*)a.x + id * a.ldx * XT::bytes;
    }
    else
        xrow = (const char*)a.x + row * a.ldx * XT::bytes;
    char* rrow = (char*)a.r + row * a.ldr * RT::bytes;
    char* yrow = (char*)a.y + row * a.ldy * YT::bytes;

    // Issue every HBM load of the row (x, r) and the weight fetch before any arithmetic.
    typename XT::Vec xv[MAXV];
    [[maybe_unused]] typename RT::Vec rv[MAXV];
    u32x4 wv[MAXV];
    #pragma unroll
    for (int k = 0; k < MAXV; ++k)
    {
        const int c = tid + k * nt;
        if (c < nc)
        {
            if (valid)
            {
                if constexpr (MODE == RMS_GATHER) xv[k] = load8<XT>(xrow, (int64_t)c * 8);   // hot table rows
                else xv[k] = load8s<XT>(xrow, (int64_t)c * 8);
            }
            if constexpr (MODE == RMS_RES_IN) rv[k] = load8s<RT>(rrow, (int64_t)c * 8);
            if (has_w) wv[k] = prefetch_w8(a.w, a.wt, (int64_t)c * 8);
        }
    }

    // Pass 1: residual update and sum of squares.  The row is then cached in its narrowest
    // exact form (x as loaded, or the rounded residual), 4 VGPRs per chunk for 16-bit data,
    // and re-expanded in pass 2.
    using CT = std::conditional_t<MODE == RMS_RES_IN, RT, XT>;
    typename CT::Vec cache[MAXV];
    double ss = 0.0;
    #pragma unroll
    for (int k = 0; k < MAXV; ++k)
    {
        const int c = tid + k * nt;
        if (c < nc)
        {
            float h[8];
            if (valid)
                unpack8<XT>(xv[k], h);
            else
            {
                #pragma unroll
                for (int j = 0; j < 8; ++j) h[j] = 0.0f;
                xv[k] = pack8<XT>(h);
            }
            if constexpr (MODE != RMS_GATHER && XT::code == DT_F16)
            {
                #pragma unroll
                for (int j = 0; j < 8; ++j) h[j] = clamp_f16(h[j]);
            }
            if constexpr (MODE == RMS_RES_IN)
            {
                float rf[8];
                unpack8<RT>(rv[k], rf);
                #pragma unroll
                for (int j = 0; j < 8; ++j) h[j] = h[j] + rf[j];
                cache[k] = pack8<RT>(h);
                store8<RT>(rrow, (int64_t)c * 8, cache[k]);
                unpack8<RT>(cache[k], h);   // the norm sees the rounded residual
            }
            else
                cache[k] = xv[k];
            if constexpr (MODE == RMS_GATHER && RT::code >= 0)
            {
                if (a.r)
                {
                    if constexpr (RT::code == XT::code)
                        store8<XT>(rrow, (int64_t)c * 8, xv[k]);        // bit-exact copy
                    else
                        store8<RT>(rrow, (int64_t)c * 8, pack8<RT>(h)); // exact upcast
                }
            }
            #pragma unroll
            for (int j = 0; j < 8; ++j) ss = fma((double)h[j], (double)h[j], ss);
        }
    }

    // fp64 row sum (exact for 16-bit data), one rounding, IEEE fp32 sqrt and divide.
    if constexpr (WAVE) ss = group_sum64<64>(ss);
    else ss = block_sum64(ss, red);
    const float rmf = rms_factor(ss, a.dim, a.eps) * a.cs;

    // Pass 2: scale, weight, round once, store.
    #pragma unroll
    for (int k = 0; k < MAXV; ++k)
    {
        const int c = tid + k * nt;
        if (c < nc)
        {
            float h[8];
            unpack8<CT>(cache[k], h);
            if constexpr (MODE == RMS_PLAIN && XT::code == DT_F16)
            {
                #pragma unroll
                for (int j = 0; j < 8; ++j) h[j] = clamp_f16(h[j]);
            }
            float o[8];
            if (has_w)
            {
                float wf[8];
                unpack_w8(wv[k], a.w, a.wt, (int64_t)c * 8, wf);
                if (a.cb != 0.0f)
                {
                    #pragma unroll
                    for (int j = 0; j < 8; ++j) wf[j] = wf[j] + a.cb;
                }
                #pragma unroll
                for (int j = 0; j < 8; ++j) o[j] = (h[j] * wf[j]) * rmf;
            }
            else
            {
                #pragma unroll
                for (int j = 0; j < 8; ++j) o[j] = h[j] * rmf;
            }
            store8<YT>(yrow, (int64_t)c * 8, pack8<YT>(o));
        }
    }

}

template <class XT, class YT, class RT, int MAXV, int MODE>
__global__ __launch_bounds__(1024) void k_rms_norm(RmsArgs a)
{
    __shared__ double red[16];
    if (a.xcd && gridDim.x == a.rows)
    {
        rms_row<XT, YT, RT, MAXV, MODE, false>(a, xcd_slice(blockIdx.x, a.rows), threadIdx.x, blockDim.x, red);
        return;
    }
    for (int64_t row = blockIdx.x; row < a.rows; row += gridDim.x)
        rms_row<XT, YT, RT, MAXV, MODE, false>(a, row, threadIdx.x, blockDim.x, red);
}

// Wave-per-row: each wave of a 256-thread workgroup owns one row (dim <= 8192 at MAXV <= 16), so a
// wave keeps up to 16 chunks of x and r (~20 KiB at hidden 5120) in flight and never waits on a
// barrier.
template <class XT, class YT, class RT, int MAXV, int MODE>
__global__ __launch_bounds__(256) void k_rms_norm_wave(RmsArgs a)
{
    const int wpb = blockDim.x >> 6;
    for (int64_t row = (int64_t)blockIdx.x * wpb + (threadIdx.x >> 6); row < a.rows; row += (int64_t)gridDim.x * wpb)
        rms_row<XT, YT, RT, MAXV, MODE, true>(a, row, threadIdx.x & 63, 64, nullptr);
}

// Generic fallback: any dim, any alignment, element-granular, two passes over global memory.
template <int MODE>
__global__ __launch_bounds__(256) void k_rms_norm_generic(RmsArgs a, int xt, int yt, int rt)
{
    __shared__ double red[16];
    const int tid = threadIdx.x;
    for (int64_t row = blockIdx.x; row < a.rows; row += gridDim.x)
    {
        int64_t xoff = row * a.ldx;
        bool valid = true;
        if constexpr (MODE == RMS_GATHER)
        {
            int64_t id = load_id(a.ids, a.idt, row);
            valid = id >= 0 && id < a.vocab;
            if (!valid && tid == 0 && a.err) atomicOr(a.err, 1);
            xoff = valid ? id * a.ldx : 0;
        }
        double ss = 0.0;
        for (int j = tid; j < a.dim; j += blockDim.x)
        {
            float v = valid ? load1(a.x, xt, xoff + j) : 0.0f;
            if (MODE != RMS_GATHER && xt == DT_F16) v = clamp_f16(v);
            if (MODE == RMS_RES_IN)
            {
                v = round1(v + load1(a.r, rt, row * a.ldr + j), rt);
                store1(a.r, rt, row * a.ldr + j, v);
            }
            if (MODE == RMS_GATHER && a.r)
            {
                if (rt == xt && rt != DT_F32 && valid)
                    ((uint16_t*)a.r)[row * a.ldr + j] = ((const uint16_t*)a.x)[xoff + j];
                else
                    store1(a.r, rt, row * a.ldr + j, v);
            }
            ss = fma((double)v, (double)v, ss);
        }
        ss = block_sum64(ss, red);
        const float rmf = rms_factor(ss, a.dim, a.eps) * a.cs;
        for (int j = tid; j < a.dim; j += blockDim.x)
        {
            float v;
            if (MODE == RMS_RES_IN) v = load1(a.r, rt, row * a.ldr + j);
            else
            {
                v = valid ? load1(a.x, xt, xoff + j) : 0.0f;
                if (MODE != RMS_GATHER && xt == DT_F16) v = clamp_f16(v);
            }
            float o;
            if (a.w)
            {
                float wf = load1(a.w, a.wt, j);
                if (a.cb != 0.0f) wf = wf + a.cb;
                o = (v * wf) * rmf;
            }
            else
                o = v * rmf;
            store1(a.y, yt, row * a.ldy + j, o);
        }
        __syncthreads();
    }
}

// ---------------------------------------------------------------------------------------------
// Host-side launch.

// Launch shape.  Rows of up to 8192 elements (1024 chunks) go wave-per-row with MAXV = chunks / 64
// rounded up to a compiled size; longer rows use a workgroup per row (MAXV chunks per thread).
struct RmsShape
{
    bool wave;
    int maxv;
    int threads;
};

inline int rms_wave_maxv(int nc)
{
    static const int opts[8] = { 1, 2, 4, 6, 8, 10, 12, 16 };
    const int need = (nc + 63) / 64;
    for (int m : opts)
        if (m >= need) return m;
    return 0;
}

inline RmsShape rms_shape(int nc, int64_t rows)
{
    auto thr = [&](int m) { int t = (nc + m - 1) / m; return ((t + 63) / 64) * 64; };
    const Tuning& tu = tuning();
    // Wave-per-row measured slower than a workgroup per row on MI355X (C3: 74 vs 64 us, decode rows
    // 6-7 vs 3 us); it is kept as a tuning option.
    if (tu.rms_mode == 2 && rms_wave_maxv(nc) > 0)
        return { true, rms_wave_maxv(nc), 256 };
    if (((tu.rms_maxv >= 1 && tu.rms_maxv <= 5) || tu.rms_maxv == 8) &&
        (tu.rms_threads == 0 || (tu.rms_threads % 64 == 0 && tu.rms_threads <= 1024)))
        return { false, tu.rms_maxv, tu.rms_threads > 0 ? tu.rms_threads : thr(tu.rms_maxv) };
    // MAXV = 8 does not fit the VGPR budget of a 1024-thread bound; it is the last resort.
    static const int opts[3] = { 1, 2, 4 };
    const int target = rows <= 1024 ? 1024 : 384;
    for (int m : opts)
        if (thr(m) <= target) return { false, m, thr(m) };
    if (thr(4) <= 1024) return { false, 4, thr(4) };
    return { false, 8, thr(8) };   // <= 1024 (rms_vec_ok bounds the row at 8192 chunks)
}

template <class XT, class YT, class RT, int MODE>
int launch_rms_vec(RmsArgs a, hipStream_t s)
{
    const RmsShape sh = rms_shape(a.dim / 8, a.rows);
    a.xcd = tuning().xcd;
    if (sh.wave)
    {
        int64_t blocks = (a.rows + 3) / 4;
        const dim3 grid((unsigned)(blocks < kMaxGridX ? blocks : kMaxGridX));
        switch (sh.maxv)
        {
            case 1: k_rms_norm_wave<XT, YT, RT, 1, MODE><<<grid, 256, 0, s>>>(a); break;
            case 2: k_rms_norm_wave<XT, YT, RT, 2, MODE><<<grid, 256, 0, s>>>(a); break;
            case 4: k_rms_norm_wave<XT, YT, RT, 4, MODE><<<grid, 256, 0, s>>>(a); break;
            case 6: k_rms_norm_wave<XT, YT, RT, 6, MODE><<<grid, 256, 0, s>>>(a); break;
            case 8: k_rms_norm_wave<XT, YT, RT, 8, MODE><<<grid, 256, 0, s>>>(a); break;
            case 10: k_rms_norm_wave<XT, YT, RT, 10, MODE><<<grid, 256, 0, s>>>(a); break;
            case 12: k_rms_norm_wave<XT, YT, RT, 12, MODE><<<grid, 256, 0, s>>>(a); break;
            default: k_rms_norm_wave<XT, YT, RT, 16, MODE><<<grid, 256, 0, s>>>(a); break;
        }
        return 0;
    }
    const dim3 grid((unsigned)(a.rows < kMaxGridX ? a.rows : kMaxGridX));
    switch (sh.maxv)
    {
        case 1: k_rms_norm<XT, YT, RT, 1, MODE><<<grid, sh.threads, 0, s>>>(a); break;
        case 2: k_rms_norm<XT, YT, RT, 2, MODE><<<grid, sh.threads, 0, s>>>(a); break;
        case 3: k_rms_norm<XT, YT, RT, 3, MODE><<<grid, sh.threads, 0, s>>>(a); break;
        case 4: k_rms_norm<XT, YT, RT, 4, MODE><<<grid, sh.threads, 0, s>>>(a); break;
        case 5: k_rms_norm<XT, YT, RT, 5, MODE><<<grid, sh.threads, 0, s>>>(a); break;
        default: k_rms_norm<XT, YT, RT, 8, MODE><<<grid, sh.threads, 0, s>>>(a); break;
    }
    return 0;
}

// The vector kernel needs 16-byte aligned rows of whole chunks and a row that fits 1024 x 8 chunks.
inline bool rms_vec_ok(const RmsArgs& a, int xt, int yt, int rt, bool has_r)
{
    if (a.dim % 8 != 0 || a.dim / 8 > 8 * 1024) return false;
    auto ok = [](const void* p, int64_t ld, int dt) {
        return p == nullptr || (aligned16(p) && (ld * dtype_bytes(dt)) % 16 == 0);
    };
    if (!ok(a.x, a.ldx, xt) || !ok(a.y, a.ldy, yt)) return false;
    if (has_r && !ok(a.r, a.ldr, rt)) return false;
    if (a.w && !aligned16(a.w)) return false;
    const RmsShape sh = rms_shape(a.dim / 8, a.rows);
    return sh.wave || ((int64_t)sh.maxv * sh.threads >= a.dim / 8 && sh.threads <= 1024);
}

}  // namespace exl3r
