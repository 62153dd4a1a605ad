// RMSNorm kernel family for gfx950: plain, residual-add-fused (RES_IN) and embedding-gather-fused.
//
// Semantics follow rms_norm_kernel (reference kernels/norm.cu:160-304):
//   f16 x is clamped to +-65504 on read (norm.cu:42-58, 192-196); RES_IN rounds x + r to r's dtype,
//   writes it back to r and normalises the rounded sum (norm.cu:198-223); the sum of squares is an
//   FMA chain (norm.cu:101-108; carried in fp64 here); rmf = rsqrt(sum / dim + eps) * constant_scale
//   (norm.cu:273; IEEE fp32 sqrt and divide here);
//   y = (x * (w + constant_bias)) * rmf in fp32, rounded once (norm.cu:110-124, 232-239, 75-83).
//
// Layout: one row per workgroup (row = row0 + blockIdx.x; the host splits launches beyond the grid
// limit).  A row is split into chunks of 8 elements; thread t owns chunks t, t + nt, ... (at most
// MAXV), so every wave-wide access is 64 lanes x 16 bytes contiguous.
// The whole row stays in VGPRs between the reduction and the output pass: one HBM read of x (and r),
// one write of y (and r) per row -- the 4-pass minimum for RES_IN, where the reference re-reads r
// at dim > 4096.  The row reduction is a DPP butterfly inside each wave and one LDS hop across waves.
#pragma once

#include "abi.hpp"
#include "common.cuh"
#include "hadamard.cuh"

#include <type_traits>

namespace exl3r {

enum { RMS_PLAIN = 0, RMS_RES_IN = 1, RMS_GATHER = 2, RMS_GATED = 3 };

struct RmsArgs
{
    const void* x;      // input rows; RMS_GATHER: the embedding table
    int64_t ldx;
    const void* w;      // [dim] weight or nullptr
    int wt;
    void* y;
    int64_t ldy;
    void* r;            // RMS_RES_IN: residual (in/out); RMS_GATHER: optional gathered-row output h;
                        // RMS_GATED: the gate g (read only)
    int64_t ldr;
    const void* ids;    // RMS_GATHER: [rows] token ids (I32 or I64, see idt)
    int idt;
    int64_t vocab;
    int32_t* err;       // RMS_GATHER: device error flag or nullptr
    int64_t rows;
    int64_t row0;       // first row of this launch (launches of more than kMaxGridX rows are split)
    int dim;
    float eps, cb, cs;
    int gact;           // RMS_GATED: 0 silu, 1 sigmoid
    int gfirst;         // RMS_GATED: gate applied before the norm
    int w_groups;       // RMS_GATED: the weight holds w_groups rows of dim, row r uses r % w_groups
    // Hadamard outputs (HAD_OUT kernels, exl3r_rms_norm_had): output i = had_r_128 of the f16 norm
    // output with pre-scale hpre[i] (f16 [dim] or nullptr), rows at stride ldh, hr = scale / sqrt(128).
    int nh;
    const void* hpre[4];
    void* hout[4];
    int64_t ldh;
    float hr;
    // Row r of the norm takes pre-scale row r % hpre_rows ([hpre_rows, dim], 0 or 1: one row): a
    // projection input made of several norm rows (the head-dim rows of a gated norm) has one scale
    // per column of the whole input row.
    int hpre_rows;
    // HAD_IN kernels: f16 x is first replaced by had_r_128(x) * hxpost (the EXL3 linear's output
    // rotation with its f16 post-scale, or none when null).
    const void* hxpost;
    // Hadamard kernels: the updated residual is written with cached stores (1) instead of non-temporal ones.
    int r_cached;
};

// Hadamard flags of the norm kernels (exl3r_rms_norm_had).
constexpr int HAD_OUT = 1;   // rotated f16 outputs, one per projection
constexpr int HAD_IN = 2;    // x rotated on load
constexpr int HAD_MFMA = 4;  // the transforms on the matrix cores (had128_mfma)

// The matrix-core transforms need chunk mfma_chunk(l) of a wave's 64-chunk span in lane l, while the
// row's loads and stores keep chunk l in lane l (with the permuted placement the norm kernels' f32
// residual and three outputs fetched 1.15x and wrote 1.20x their bytes, against 1.01x and 1.00x with
// the lane-ordered one: a line's halves come from different rows of a store).  A chunk moves between
// the two placements through the lane crossbar (ds_bpermute, no LDS storage; the permutation is its own
// inverse).  Thread counts are multiples of 64, so a wave's chunks c = tid + k * nt are one span of 4
// blocks for every k.
__device__ __forceinline__ TF16::Vec mfma_permute(const TF16::Vec& v, int lane)
{
    const int src = mfma_chunk(lane) << 2;
    TF16::Vec o;
    #pragma unroll
    for (int q = 0; q < 4; ++q) o.a[q] = (uint32_t)__builtin_amdgcn_ds_bpermute(src, (int)v.a[q]);
    return o;
}

// When a row's weight chunks are fetched (a launch-shape choice: the results are the same bits).
//   W_EARLY: with the row's HBM loads, so the L2 fetch overlaps them (latency-bound launches);
//   W_MID:   after pass 1, so the fetch overlaps the row reduction;
//   W_LATE:  chunk by chunk in pass 2, after the reduction.
// Streaming launches fetch it late: the row then holds no weight registers while its HBM loads are in
// flight (MI355X, [8192, 5120]: bf16 residual norm 56.3 us early -> 54.9 late; f16 x / f32 r / f16 y
// 93.6 -> 88.6; plain bf16 norm 31.5 -> 30.7 mid).
enum { W_EARLY = 0, W_MID = 1, W_LATE = 2 };

// RMS_GATED gate activation in fp32.
__device__ __forceinline__ float gate_act(int gact, float g) { return gact ? act_f<ACT_SIGMOID>(g) : act_f<ACT_SILU>(g); }

// Element offset of the weight row a row uses.
template <int MODE>
__device__ __forceinline__ int64_t weight_row(const RmsArgs& a, int64_t row)
{
    // (one weight group, the usual case, skips the per-row 64-bit remainder: a kernel-uniform branch,
    // gated norm [131072, 128] 26.9 -> 25.2 us)
    if constexpr (MODE == RMS_GATED) return a.w_groups == 1 ? 0 : (row % a.w_groups) * a.dim;
    else return 0;
}

// Element offset of the pre-scale row a norm row uses (hpre_rows norm rows form one projection row):
// kernel-uniform branches, a mask for a power-of-two count (heads per projection row), the 64-bit
// remainder otherwise.
__device__ __forceinline__ int64_t pre_row(const RmsArgs& a, int64_t row)
{
    const int pr = a.hpre_rows;
    if (pr <= 1) return 0;
    if ((pr & (pr - 1)) == 0) return (row & (pr - 1)) * a.dim;
    return (row % pr) * a.dim;
}

__device__ __forceinline__ int64_t load_id(const void* ids, int idt, int64_t i)
{
    return idt == DT_I64 ? ((const int64_t*)ids)[i] : (int64_t)((const int32_t*)ids)[i];
}

// A weight chunk is fetched as one 16-byte access at the point the launch's weight mode picks (the
// whole chunk for F16/BF16 weights; for F32 weights the first four floats, the second half being read
// in pass 2), 4 VGPRs per chunk.
// A split chunk (SPLIT) takes its two halves from the quads at e and e + kSplitGap.
template <bool SPLIT = false>
__device__ __forceinline__ u32x4 prefetch_w8(const void* w, int wt, int64_t e)
{
    if constexpr (SPLIT)
    {
        if (wt == DT_F32) return *(const u32x4*)((const float*)w + e);
        const uint16_t* p = (const uint16_t*)w + e;
        const u32x2 lo = *(const u32x2*)p, hi = *(const u32x2*)(p + kSplitGap);
        return u32x4{ lo.x, lo.y, hi.x, hi.y };
    }
    return *(const u32x4*)((const char*)w + e * (wt == DT_F32 ? 4 : 2));
}

template <bool SPLIT = false>
__device__ __forceinline__ void unpack_w8(u32x4 pre, const void* w, int wt, int64_t e, float (&f)[8])
{
    if (wt == DT_F16) { TF16::Vec v; v.a = pre; unpack8<TF16>(v, f); }
    else if (wt == DT_BF16) { TBF16::Vec v; v.a = pre; unpack8<TBF16>(v, f); }
    else
    {
        TF32::Vec v;
        v.a = pre;
        v.b = *(const u32x4*)((const float*)w + e + (SPLIT ? kSplitGap : 4));
        unpack8<TF32>(v, f);
    }
}

// Registers of one row between its loads and its arithmetic.
template <class XT, class RT, int MAXV>
struct RowRegs
{
    typename XT::Vec xv[MAXV];
    typename RT::Vec rv[MAXV];
    u32x4 wv[MAXV];
    bool valid;
};

// Issues every HBM load of one row -- x (and r) in chunks c = tid, tid + nt, ... (at most MAXV per
// lane), plus the weight chunks when load_w -- before any arithmetic.
template <class XT, class RT, int MAXV, int MODE, bool SPLIT = false, int HAD = 0>
__device__ __forceinline__ void rms_load(const RmsArgs& a, int64_t row, int tid, int nt, bool load_w,
                                         RowRegs<XT, RT, MAXV>& L)
{
    const int nc = a.dim >> 3;
    const char* xrow;
    L.valid = true;
    if constexpr (MODE == RMS_GATHER)
    {
        int64_t id = load_id(a.ids, a.idt, row);
        L.valid = id >= 0 && id < a.vocab;
        if (!L.valid)
        {
            if (tid == 0 && a.err) atomicOr(a.err, 1);
            id = 0;
        }
        xrow = (const char*)a.x + id * a.ldx * XT::bytes;
    }
    else
        xrow = (const char*)a.x + row * a.ldx * XT::bytes;
    const char* rrow = (const char*)a.r + row * a.ldr * RT::bytes;
    #pragma unroll
    for (int k = 0; k < MAXV; ++k)
    {
        const int c = tid + k * nt;
        const int64_t e = chunk_elem<SPLIT>(c);
        if constexpr ((HAD & HAD_MFMA) != 0)
        {
            // the transforms read every lane: zeros past the row (one select per word, so that the
            // chunk stays in registers)
            static_assert(MODE != RMS_GATHER, "gathered rows take the butterfly");
            const typename XT::Vec z = load8s<XT>(xrow, c < nc ? e : 0);
            #pragma unroll
            for (int q = 0; q < 4; ++q) L.xv[k].a[q] = c < nc ? z.a[q] : 0u;
            if constexpr (XT::code == DT_F32)
            {
                #pragma unroll
                for (int q = 0; q < 4; ++q) L.xv[k].b[q] = c < nc ? z.b[q] : 0u;
            }
        }
        if (c < nc)
        {
            if ((HAD & HAD_MFMA) == 0 && L.valid)
            {
                if constexpr (SPLIT) L.xv[k] = load8s_split<XT>(xrow, e);
                else if constexpr (MODE == RMS_GATHER) L.xv[k] = load8<XT>(xrow, e);   // hot table rows
                else L.xv[k] = load8s<XT>(xrow, e);
            }
            if constexpr (MODE == RMS_RES_IN || MODE == RMS_GATED)
            {
                if constexpr (SPLIT) L.rv[k] = load8s_split<RT>(rrow, e);
                else L.rv[k] = load8s<RT>(rrow, e);
            }
            if (load_w && a.w) L.wv[k] = prefetch_w8<SPLIT>(a.w, a.wt, weight_row<MODE>(a, row) + e);
        }
    }
}

// Arithmetic and stores of one loaded row; the row sum is reduced across the workgroup (DPP butterfly
// inside each wave, one LDS hop across waves).
// The cached form of a row between the passes: x as loaded, or the rounded residual.
template <class XT, class RT, int MODE>
using RmsCache = std::conditional_t<MODE == RMS_RES_IN, RT, XT>;

// RES_IN stores the updated residual in pass 2, after the reduction, next to y (MI355X, [8192, 5120]:
// f16 x / f32 r / f16 y 93.8 us against 95.9 us storing it in pass 1; bf16 57.1 against 57.3-57.4 us).
template <int MODE, class RT>
constexpr bool kDeferResidual = MODE == RMS_RES_IN;

// Pass 1 of the 8-element chunk at element e of a row: clamp (f16 x), residual update (RES_IN),
// gathered-row copy (GATHER), gate before the norm (GATED), and the chunk's squares added to ss
// (fp64: squares and sums of 16-bit data are exact).  Returns the chunk's cached form.
template <class XT, class RT, int MODE, int HAD = 0, bool SPLIT = false, class ACC = double>
__device__ __forceinline__ typename RmsCache<XT, RT, MODE>::Vec rms_chunk1(const RmsArgs& a, char* rrow, int64_t e,
                                                                          bool valid, typename XT::Vec& xv,
                                                                          const typename RT::Vec& rv, ACC& ss)
{
    // A pass-1 residual store is contiguous: split chunks (two quads 256 apart) must defer it to pass 2,
    // where the split store is used.
    static_assert(!SPLIT || kDeferResidual<MODE, RT> || MODE != RMS_RES_IN, "split chunks store the residual in pass 2");
    using CT = RmsCache<XT, RT, MODE>;
    typename CT::Vec cv;
    float h[8];
    if constexpr ((HAD & HAD_IN) != 0)
    {
        // x = had_r_128(x, post = hxpost) as the projection's own output rotation rounds it: the
        // fp32 butterfly, one rounding to f16, then the half post-scale product.  The chunk's
        // 16-lane group is the 128-element block, as for the outputs.
        static_assert(XT::code == DT_F16 && MODE != RMS_GATHER && MODE != RMS_GATED, "x rotation takes f16 x");
        output_rotation8(xv, a.hxpost, e);
    }
    if (valid)
        unpack8<XT>(xv, h);
    else
    {
        #pragma unroll
        for (int j = 0; j < 8; ++j) h[j] = 0.0f;
        xv = pack8<XT>(h);
    }
    if constexpr (MODE != RMS_GATHER && MODE != RMS_GATED && XT::code == DT_F16)
    {
        #pragma unroll
        for (int j = 0; j < 8; ++j) h[j] = clamp_f16(h[j]);
    }
    if constexpr (MODE == RMS_GATED)
    {
        if (a.gfirst)
        {
            float gf[8];
            unpack8<RT>(rv, gf);
            #pragma unroll
            for (int j = 0; j < 8; ++j) h[j] = h[j] * gate_act(a.gact, gf[j]);
        }
    }
    if constexpr (MODE == RMS_RES_IN)
    {
        float rf[8];
        unpack8<RT>(rv, rf);
        #pragma unroll
        for (int j = 0; j < 8; ++j) h[j] = h[j] + rf[j];
        cv = pack8<RT>(h);
        if constexpr (!kDeferResidual<MODE, RT>) store8<RT>(rrow, e, cv);
        unpack8<RT>(cv, h);   // the norm sees the rounded residual
    }
    else
        cv = xv;
    if constexpr (MODE == RMS_GATHER && RT::code >= 0)
    {
        if (a.r)
        {
            if constexpr (RT::code == XT::code)
                store8<XT>(rrow, e, xv);        // bit-exact copy
            else
                store8<RT>(rrow, e, pack8<RT>(h)); // exact upcast
        }
    }
    #pragma unroll
    for (int j = 0; j < 8; ++j) ss = fma((ACC)h[j], (ACC)h[j], ss);
    return cv;
}

// Pass 2 of the chunk at element e: gate (GATED), weight (row offset wofs), scale, gate after the
// norm (GATED), one rounding: the chunk of y.
template <class XT, class YT, class RT, int MODE, bool SPLIT = false>
__device__ __forceinline__ typename YT::Vec rms_out8(const RmsArgs& a, int64_t e, int64_t wofs,
                                                     const typename RmsCache<XT, RT, MODE>::Vec& cv,
                                                     const typename RT::Vec& rv, u32x4 wv, float rmf)
{
    float h[8];
    unpack8<RmsCache<XT, RT, MODE>>(cv, h);
    if constexpr (MODE == RMS_PLAIN && XT::code == DT_F16)
    {
        #pragma unroll
        for (int j = 0; j < 8; ++j) h[j] = clamp_f16(h[j]);
    }
    float ga[8];
    if constexpr (MODE == RMS_GATED)
    {
        float gf[8];
        unpack8<RT>(rv, gf);
        #pragma unroll
        for (int j = 0; j < 8; ++j)
        {
            ga[j] = gate_act(a.gact, gf[j]);
            if (a.gfirst) h[j] = h[j] * ga[j];
        }
    }
    float o[8];
    if (a.w)
    {
        float wf[8];
        unpack_w8<SPLIT>(wv, a.w, a.wt, wofs + e, wf);
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
    if constexpr (MODE == RMS_GATED)
    {
        if (!a.gfirst)
        {
            #pragma unroll
            for (int j = 0; j < 8; ++j) o[j] = o[j] * ga[j];
        }
    }
    return pack8<YT>(o);
}

// Pass 2 of the chunk at element e: rms_out8, then the stores (y, or the Hadamard outputs by the
// butterfly).
template <class XT, class YT, class RT, int MODE, int HAD, bool SPLIT = false>
__device__ __forceinline__ void rms_chunk2(const RmsArgs& a, int64_t row, char* yrow, int64_t e, int64_t wofs,
                                           const typename RmsCache<XT, RT, MODE>::Vec& cv,
                                           const typename RT::Vec& rv, u32x4 wv, float rmf)
{
    const typename YT::Vec yv = rms_out8<XT, YT, RT, MODE, SPLIT>(a, e, wofs, cv, rv, wv, rmf);
    if constexpr (SPLIT) store8_split<YT>(yrow, e, yv);
    else if constexpr (!(HAD & HAD_OUT)) store8<YT>(yrow, e, yv);
    else
    {
        #pragma clang fp contract(off)
        // The f16 norm output, then each consumer's had_r_128 with its pre-scale.  The chunk's
        // 16-lane group is the block's (lane counts are multiples of 16 and dim % 128 == 0), and
        // l16 is both the lane's place in that group and the chunk's place in the block.
        static_assert(YT::code == DT_F16, "the Hadamard prologue follows an f16 norm output");
        if (a.y) store8<YT>(yrow, e, yv);
        const int l16 = (int)((e >> 3) & 15);
        for (int i = 0; i < a.nh; ++i)
        {
            TF16::Vec v = yv;
            if (a.hpre[i])
            {
                const TF16::Vec p = load8<TF16>(a.hpre[i], pre_row(a, row) + e);
                #pragma unroll
                for (int q = 0; q < 4; ++q) v.a[q] = hmul2(v.a[q], p.a[q]);
            }
            with_carried<true>(zero_lane16(v), a.hr, [&](auto C) {
                float f[8];
                butterfly128_f16<decltype(C)::value>(v, f, l16, a.hr);
                store8<TF16>((char*)a.hout[i] + row * a.ldh * 2, e, pack8<TF16>(f));
            });
        }
    }
}

// ACC: the type of the row's sum of squares -- double (exact for 16-bit data, rounded once to fp32) or
// float (one fp32 FMA chain per lane in chunk order, then the wave butterfly and the cross-wave sum in
// a fixed order: the reference's own precision, norm.cu:101-108, 140-151).
template <class XT, class YT, class RT, int MAXV, int MODE, int HAD, int WM, bool SPLIT = false, class ACC = double>
__device__ __forceinline__ void rms_finish(const RmsArgs& a, int64_t row, int tid, int nt, RowRegs<XT, RT, MAXV>& L,
                                           ACC* red)
{
    const int nc = a.dim >> 3;
    char* rrow = (char*)a.r + row * a.ldr * RT::bytes;
    char* yrow = (char*)a.y + row * a.ldy * YT::bytes;
    constexpr bool MF = (HAD & HAD_MFMA) != 0;
    const int c0 = tid;
    const int lane = tid & 63;
    // chunk held in the matrix-core placement: chunk k of the lane's wave, mfma_chunk(lane) within it
    [[maybe_unused]] const int cp0 = (tid & ~63) | mfma_chunk(lane);
    [[maybe_unused]] HadMfma H;
    if constexpr (MF)
    {
        H = had_mfma_operands(lane);
        if constexpr ((HAD & HAD_IN) != 0)
        {
            // x = the producing projection's output rotation, every lane of the wave taking part
            static_assert(XT::code == DT_F16 && MODE != RMS_GATHER && MODE != RMS_GATED, "x rotation takes f16 x");
            const void* post[MAXV];
            int64_t col[MAXV];
            #pragma unroll
            for (int k = 0; k < MAXV; ++k)
            {
                const int cp = cp0 + k * nt;
                post[k] = cp < nc ? a.hxpost : nullptr;
                col[k] = (int64_t)cp * 8;
                L.xv[k] = mfma_permute(L.xv[k], lane);
            }
            output_rotations_mfma<MAXV>(H, L.xv, post, col, lane);
            #pragma unroll
            for (int k = 0; k < MAXV; ++k) L.xv[k] = mfma_permute(L.xv[k], lane);
        }
    }
    // Pass 1: residual update and sum of squares.  The row is then cached in its narrowest exact
    // form (x as loaded, or the rounded residual), 4 VGPRs per chunk for 16-bit data, and
    // re-expanded in pass 2.
    typename RmsCache<XT, RT, MODE>::Vec cache[MAXV];
    ACC ss = 0;
    #pragma unroll
    for (int k = 0; k < MAXV; ++k)
    {
        const int c = c0 + k * nt;
        if (c < nc)
            cache[k] = rms_chunk1<XT, RT, MODE, MF ? 0 : HAD, SPLIT, ACC>(a, rrow, chunk_elem<SPLIT>(c), L.valid, L.xv[k],
                                                                    L.rv[k], ss);
    }

    const int64_t wofs = weight_row<MODE>(a, row);
    if constexpr (WM == W_MID)
    {
        #pragma unroll
        for (int k = 0; k < MAXV; ++k)
        {
            const int c = c0 + k * nt;
            if (c < nc && a.w) L.wv[k] = prefetch_w8<SPLIT>(a.w, a.wt, wofs + chunk_elem<SPLIT>(c));
        }
    }

    // Row sum (fp64: exact for 16-bit data, then one rounding), IEEE fp32 sqrt and divide.  The
    // workgroup reduces once, so one barrier suffices.
    ss = block_sum_once(ss, red);
    const float rmf = rms_factor(ss, a.dim, a.eps) * a.cs;

    if constexpr (MF)
    {
        // Pass 2 with the matrix-core transforms: the f16 norm output of every live chunk (zeros past the
        // row), then each consumer's had_r_128 with its pre-scale, every lane of the wave taking part.
        static_assert((HAD & HAD_OUT) != 0 && YT::code == DT_F16 && !SPLIT, "the Hadamard outputs follow an f16 norm");
        #pragma unroll
        for (int k = 0; k < MAXV; ++k)
        {
            const int c = c0 + k * nt;
            const int64_t e = (int64_t)c * 8;
            const bool live = c < nc;
            TF16::Vec yv;
            yv.a = u32x4{ 0u, 0u, 0u, 0u };
            if (live)
            {
                if constexpr (WM == W_LATE)
                {
                    if (a.w) L.wv[k] = prefetch_w8(a.w, a.wt, wofs + e);
                }
                if constexpr (kDeferResidual<MODE, RT>)
                {
                    if (a.r_cached) store8c<RT>(rrow, e, cache[k]);
                    else store8<RT>(rrow, e, cache[k]);
                }
                yv = rms_out8<XT, YT, RT, MODE>(a, e, wofs, cache[k], L.rv[k], L.wv[k], rmf);
                if (a.y) store8<YT>(yrow, e, yv);
            }
            // the consumers' transforms of this chunk (at most 4) in the matrix-core placement, their
            // MFMAs issued together, each result moved back to its lane for the store
            const TF16::Vec yp = mfma_permute(yv, lane);
            const int cp = cp0 + k * nt;
            const bool plive = cp < nc;
            const int64_t ep = (int64_t)cp * 8;
            // (in pairs: four results at once would hold 32 more VGPRs and cost a wave per SIMD)
            #pragma unroll
            for (int i0 = 0; i0 < 4; i0 += 2)
            {
                if (i0 >= a.nh) break;
                MfmaOut m[2];
                #pragma unroll
                for (int d = 0; d < 2; ++d)
                {
                    const int i = i0 + d;
                    if (i < a.nh)
                    {
                        TF16::Vec v = yp;
                        if (plive && a.hpre[i])
                        {
                            const TF16::Vec p = load8<TF16>(a.hpre[i], pre_row(a, row) + ep);
                            #pragma unroll
                            for (int q = 0; q < 4; ++q) v.a[q] = hmul2(v.a[q], p.a[q]);
                        }
                        m[d] = had128_mfma_issue(H, v);
                    }
                    else
                        m[d] = MfmaOut{};
                }
                mfma_wait_all(m);
                #pragma unroll
                for (int d = 0; d < 2; ++d)
                {
                    const int i = i0 + d;
                    if (i < a.nh)
                    {
                        float f[8];
                        had128_mfma_finish(m[d], f, lane, a.hr);
                        const TF16::Vec o = mfma_permute(pack8<TF16>(f), lane);
                        if (live) store8<TF16>((char*)a.hout[i] + row * a.ldh * 2, e, o);
                    }
                }
            }
        }
        return;
    }
    // Pass 2: scale, weight, round once, store.
    #pragma unroll
    for (int k = 0; k < MAXV; ++k)
    {
        const int c = tid + k * nt;
        if (c < nc)
        {
            const int64_t e = chunk_elem<SPLIT>(c);
            if constexpr (WM == W_LATE)
            {
                if (a.w) L.wv[k] = prefetch_w8<SPLIT>(a.w, a.wt, wofs + e);
            }
            if constexpr (kDeferResidual<MODE, RT>)
            {
                if constexpr (SPLIT) store8_split<RT>(rrow, e, cache[k]);
                else if constexpr (HAD != 0)
                {
                    if (a.r_cached) store8c<RT>(rrow, e, cache[k]);
                    else store8<RT>(rrow, e, cache[k]);
                }
                else store8<RT>(rrow, e, cache[k]);
            }
            rms_chunk2<XT, YT, RT, MODE, HAD, SPLIT>(a, row, yrow, e, wofs, cache[k], L.rv[k], L.wv[k], rmf);
        }
    }
}

// One row per workgroup: its loads, pass 1, one reduction, pass 2.  (A grid-stride loop over rows, with
// the second barrier it needs before LDS reuse, measured ~1 us slower at [8192, 5120].)
template <class XT, class YT, class RT, int MAXV, int MODE, int HAD = 0, int WM = W_EARLY, bool SPLIT = false,
          class ACC = double>
__global__ __launch_bounds__(1024) void k_rms_norm(RmsArgs a)
{
    static_assert(!SPLIT || (HAD == 0 && (MODE == RMS_PLAIN || MODE == RMS_RES_IN)), "split chunks: plain and residual norms");
    __shared__ ACC red[16];
    const int64_t row = a.row0 + blockIdx.x;
    RowRegs<XT, RT, MAXV> L;
    rms_load<XT, RT, MAXV, MODE, SPLIT, HAD>(a, row, threadIdx.x, blockDim.x, WM == W_EARLY, L);
    rms_finish<XT, YT, RT, MAXV, MODE, HAD, WM, SPLIT, ACC>(a, row, threadIdx.x, blockDim.x, L, red);
}

// Streaming plain / residual norms as a resident grid: workgroup b takes rows b, b + G, b + 2G, ... (G
// workgroups, all resident at once) and issues the loads of its next row before the reduction and
// stores of the current one, so a workgroup's HBM reads stay in flight across its barrier.  The weight
// chunks are fetched once per workgroup.  The two rows in flight alternate between two register sets
// and two LDS reduction slots (a slot is rewritten two rows later, after every wave has passed the
// barrier in between, so one barrier per row suffices).
template <class XT, class YT, class RT, int MAXV, int MODE, class ACC = double>
__global__ __launch_bounds__(1024) void k_rms_norm_pipe(RmsArgs a)
{
    static_assert(MODE == RMS_PLAIN || MODE == RMS_RES_IN, "plain and residual norms");
    __shared__ ACC red[2][16];
    const int tid = threadIdx.x, nt = blockDim.x, nc = a.dim >> 3;
    u32x4 wv[MAXV];
    #pragma unroll
    for (int k = 0; k < MAXV; ++k)
    {
        const int c = tid + k * nt;
        if (c < nc && a.w) wv[k] = prefetch_w8(a.w, a.wt, (int64_t)c * 8);
    }
    const int64_t G = gridDim.x;
    RowRegs<XT, RT, MAXV> A, B;
    int64_t row = blockIdx.x;
    if (row < a.rows) rms_load<XT, RT, MAXV, MODE>(a, row, tid, nt, false, A);
    for (; row < a.rows; row += 2 * G)
    {
        if (row + G < a.rows) rms_load<XT, RT, MAXV, MODE>(a, row + G, tid, nt, false, B);
        #pragma unroll
        for (int k = 0; k < MAXV; ++k) A.wv[k] = wv[k];
        rms_finish<XT, YT, RT, MAXV, MODE, 0, W_EARLY, false, ACC>(a, row, tid, nt, A, red[0]);
        if (row + G >= a.rows) break;
        if (row + 2 * G < a.rows) rms_load<XT, RT, MAXV, MODE>(a, row + 2 * G, tid, nt, false, A);
        #pragma unroll
        for (int k = 0; k < MAXV; ++k) B.wv[k] = wv[k];
        rms_finish<XT, YT, RT, MAXV, MODE, 0, W_EARLY, false, ACC>(a, row + G, tid, nt, B, red[1]);
    }
}

// Short rows (at most 64 chunks of 8): LPR lanes per row (a power of two covering dim / 8), one
// chunk per lane, 256 / LPR rows per workgroup and RPL rows per lane in flight.  The row sum is a
// DPP butterfly inside the LPR-lane group -- no LDS, no barrier -- so a 128-element head row costs
// 16 lanes instead of a workgroup.
// HAD_MFMA (rows of one 128-element block, one f16 output): a wave's 4 rows are one span of
// had128_mfma's placement -- row = lane bits 2-3, chunk = lane bits 0, 1, 4, 5 -- so the row sum runs
// over lanes xor 1, 2, 16 and 32, which groups it as the 16-lane butterfly does (quads, pairs of quads,
// then the two pairs), the same bits.
template <class XT, class YT, class RT, int LPR, int RPL, int MODE, int HAD = 0>
__global__ __launch_bounds__(256) void k_rms_rows(RmsArgs a)
{
    static_assert(MODE != RMS_GATHER, "gathered rows take the workgroup kernel");
    constexpr bool MF = (HAD & HAD_MFMA) != 0;
    static_assert(!MF || (LPR == 16 && (HAD & HAD_OUT) != 0), "matrix-core rows: one block each, an output");
    const int SLOTS = (int)blockDim.x / LPR;   // row slots of the workgroup
    const int l64 = threadIdx.x & 63;
    const int lane = MF ? (l64 & 3) | ((l64 >> 2) & 12) : (int)threadIdx.x % LPR;
    const int slot = MF ? (int)(threadIdx.x >> 6) * 4 + ((l64 >> 2) & 3) : (int)threadIdx.x / LPR;
    const bool lane_ok = lane < (a.dim >> 3);
    const int64_t e = (int64_t)lane * 8;
    [[maybe_unused]] HadMfmaWords hw{};
    if constexpr (MF) hw = had_mfma_words(l64);
    for (int64_t r0 = (int64_t)blockIdx.x * SLOTS * RPL; r0 < a.rows; r0 += (int64_t)gridDim.x * SLOTS * RPL)
    {
        typename XT::Vec xv[RPL];
        typename RT::Vec rv[RPL];
        u32x4 wv[RPL];
        [[maybe_unused]] TF16::Vec pv[RPL];     // HAD_OUT: the row's pre-scale chunk, fetched with its loads
        bool act[RPL];
        #pragma unroll
        for (int i = 0; i < RPL; ++i)
        {
            const int64_t row = r0 + (int64_t)i * SLOTS + slot;
            act[i] = lane_ok && row < a.rows;
            if (act[i])
            {
                xv[i] = load8s<XT>((const char*)a.x + row * a.ldx * XT::bytes, e);
                if constexpr (MODE == RMS_RES_IN || MODE == RMS_GATED)
                    rv[i] = load8s<RT>((const char*)a.r + row * a.ldr * RT::bytes, e);
                if (a.w) wv[i] = prefetch_w8(a.w, a.wt, weight_row<MODE>(a, row) + e);
                if constexpr ((HAD & HAD_OUT) != 0)
                    if (a.hpre[0]) pv[i] = load8<TF16>(a.hpre[0], pre_row(a, row) + e);
            }
        }
        #pragma unroll
        for (int i = 0; i < RPL; ++i)
        {
            const int64_t row = r0 + (int64_t)i * SLOTS + slot;
            double ss = 0.0;
            typename RmsCache<XT, RT, MODE>::Vec cv;
            if (act[i]) cv = rms_chunk1<XT, RT, MODE>(a, (char*)a.r + row * a.ldr * RT::bytes, e, true, xv[i], rv[i], ss);
            if constexpr (MF)
            {
                ss += dpp64<DPP_QUAD_XOR1>(ss);
                ss += dpp64<DPP_QUAD_XOR2>(ss);
                ss = sum_xor32(sum_xor16(ss));
            }
            else
                ss = group_sum64<LPR>(ss);
            const float rmf = rms_factor(ss, a.dim, a.eps) * a.cs;
            if constexpr (MF)
            {
                // The f16 norm output and its pre-scale product (zeros in the rows past the end, whose
                // lanes still take part in the MFMAs), the transform, then the stores of live rows.
                TF16::Vec v = {};
                if (act[i])
                {
                    v = rms_out8<XT, YT, RT, MODE, false>(a, e, weight_row<MODE>(a, row), cv, rv[i], wv[i], rmf);
                    if (a.y) store8<YT>((char*)a.y + row * a.ldy * YT::bytes, e, v);
                    if (a.hpre[0])
                    {
                        #pragma unroll
                        for (int q = 0; q < 4; ++q) v.a[q] = hmul2(v.a[q], pv[i].a[q]);
                    }
                }
                MfmaOut m;
                had128_mfma_issue_w(hw, v, m);
                mfma_wait(m);
                float f[8];
                had128_mfma_finish(m, f, l64, a.hr);
                if (act[i]) store8<TF16>((char*)a.hout[0] + row * a.ldh * 2, e, pack8<TF16>(f));
            }
            else if constexpr ((HAD & HAD_OUT) != 0)
            {
                // the butterfly on the row's 16-lane block groups (one output), as rms_chunk2 does it
                static_assert(YT::code == DT_F16, "the Hadamard prologue follows an f16 norm output");
                if (act[i])
                {
                    TF16::Vec v = rms_out8<XT, YT, RT, MODE, false>(a, e, weight_row<MODE>(a, row), cv, rv[i], wv[i], rmf);
                    if (a.y) store8<YT>((char*)a.y + row * a.ldy * YT::bytes, e, v);
                    if (a.hpre[0])
                    {
                        #pragma unroll
                        for (int q = 0; q < 4; ++q) v.a[q] = hmul2(v.a[q], pv[i].a[q]);
                    }
                    with_carried<true>(zero_lane16(v), a.hr, [&](auto C) {
                        float f[8];
                        butterfly128_f16<decltype(C)::value>(v, f, lane & 15, a.hr);
                        store8<TF16>((char*)a.hout[0] + row * a.ldh * 2, e, pack8<TF16>(f));
                    });
                }
            }
            else if (act[i])
                rms_chunk2<XT, YT, RT, MODE, HAD>(a, row, (char*)a.y + row * a.ldy * YT::bytes, e,
                                                      weight_row<MODE>(a, row), cv, rv[i], wv[i], rmf);
        }
    }
}

template <class XT, class YT, class RT, int MODE, int HAD = 0>
void launch_rms_rows(const RmsArgs& a, hipStream_t s)
{
    const int nc = a.dim >> 3;
    auto go = [&](auto L) {
        constexpr int LPR = decltype(L)::value;
        // One-wave workgroups (same process, both orders, us for 64 / 256 lanes at [131072, 128]: gated
        // norm 24.8 / 25.2, with the o_proj rotation on the matrix cores 28.6 / 29.5, butterfly 28.9 / 29.1).
        constexpr int kThreads = 64;
        constexpr int SLOTS = kThreads / LPR;
        const int tuned = tuning().rms_rows_rpl;
        // One row per lane: at 62 VGPRs (f32 gate) 8 waves per SIMD keep the loads in flight.  Measured
        // on MI355X, gated norm [131072, 128] bf16 x / f32 g / f16 y: 1 row per lane 25.2 us, 2 rows
        // 30.6 us, 4 rows (156 VGPRs) 33.4 us; a workgroup per row 63 us.
        const int rpl = (tuned == 1 || tuned == 2 || tuned == 4) ? tuned : 1;
        int64_t blocks = (a.rows + (int64_t)SLOTS * rpl - 1) / ((int64_t)SLOTS * rpl);
        if (blocks > kMaxGridX) blocks = kMaxGridX;
        if (rpl == 4) launch(k_rms_rows<XT, YT, RT, LPR, 4, MODE, HAD>, (unsigned)blocks, kThreads, 0, s, a);
        else if (rpl == 2) launch(k_rms_rows<XT, YT, RT, LPR, 2, MODE, HAD>, (unsigned)blocks, kThreads, 0, s, a);
        else launch(k_rms_rows<XT, YT, RT, LPR, 1, MODE, HAD>, (unsigned)blocks, kThreads, 0, s, a);
    };
    if constexpr ((HAD & HAD_MFMA) != 0)
        go(std::integral_constant<int, 16>{});   // rows of one block (the caller checks dim == 128)
    else if (nc <= 8) go(std::integral_constant<int, 8>{});
    else if (nc <= 16) go(std::integral_constant<int, 16>{});
    else if (nc <= 32) go(std::integral_constant<int, 32>{});
    else go(std::integral_constant<int, 64>{});
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
            if (MODE != RMS_GATHER && MODE != RMS_GATED && xt == DT_F16) v = clamp_f16(v);
            if (MODE == RMS_GATED && a.gfirst) v = v * gate_act(a.gact, load1(a.r, rt, row * a.ldr + j));
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
                if (MODE != RMS_GATHER && MODE != RMS_GATED && xt == DT_F16) v = clamp_f16(v);
            }
            const float ga = MODE == RMS_GATED ? gate_act(a.gact, load1(a.r, rt, row * a.ldr + j)) : 1.0f;
            if (MODE == RMS_GATED && a.gfirst) v = v * ga;
            float o;
            if (a.w)
            {
                float wf = load1(a.w, a.wt, weight_row<MODE>(a, row) + j);
                if (a.cb != 0.0f) wf = wf + a.cb;
                o = (v * wf) * rmf;
            }
            else
                o = v * rmf;
            if (MODE == RMS_GATED && !a.gfirst) o = o * ga;
            store1(a.y, yt, row * a.ldy + j, o);
        }
        __syncthreads();
    }
}

// ---------------------------------------------------------------------------------------------
// Host-side launch.

// Launch shape: a workgroup per row, MAXV chunks per lane, and when the weight is fetched.
//   Latency-bound launches (<= 1024 rows) spread a row over up to 1024 lanes, weight fetched early.
//   Streaming residual norms (RES_IN, no Hadamard outputs): up to 512 chunks one per lane; longer rows
//   two chunks per lane on a power-of-two wave count (512 lanes up to 1024 chunks), so that 32 / waves
//   workgroups fill a CU's 32 wave slots with no idle wave; weight fetched late.  MI355X, [8192, 5120]
//   bf16 (us): 2 x 320 57.2, 2 x 384 56.3, 2 x 512 54.9, 1 x 640 57.3, 3 x 256 58.3, 1 x 1024 62.1; the
//   f16 x / f32 r / f16 y mix 2 x 384 92.4, 2 x 512 88.6, 1 x 640 89.2.
//   Other streaming norms keep the rule fitted to a sweep of the residual norm over hidden sizes 2048 to
//   8192 before the weight moved (one chunk per lane up to 512 lanes, else two chunks on at least 384
//   lanes; 320 for the Hadamard kernels, whose chunks carry up to four butterflies), with the weight
//   fetched mid-row (plain; gather and Hadamard kernels: early, where fetching it later measured no gain).
//   Split chunks (rows of whole 512-element spans, plain and residual norms without Hadamard outputs,
//   streaming launches with an f32 operand): one chunk per lane up to 1024 chunks, else two, weight
//   fetched mid-row.  MI355X, f16 x / f32 r / f16 y at [8192, 5120] (us), 4-element quads per lane
//   standing in for split chunks: 640 lanes x 2 quads 82.0 mid / 82.5 late, 320 x 4 85.1 / 83.8,
//   256 x 5 83.7 / 85.8; contiguous chunks 2 x 512 late 89.3.
struct RmsShape
{
    int maxv;
    int threads;
    int wmode;
    bool split = false;
};

// wide: an f32 operand (x, r or y).
inline RmsShape rms_shape(int nc, int64_t rows, int mode, int had, bool wide = false)
{
    auto thr = [&](int m) { int t = (nc + m - 1) / m; return ((t + 63) / 64) * 64; };
    auto pick = [&](int m) { return m <= 1 ? 1 : m <= 2 ? 2 : m <= 4 ? 4 : 8; };
    const bool split_ok = !had && (mode == RMS_PLAIN || mode == RMS_RES_IN) && nc % 64 == 0 && nc <= 2048;
    auto split_shape = [&](int wm) { return RmsShape{ nc <= 1024 ? 1 : 2, nc <= 1024 ? nc : thr(2), wm, true }; };
#ifdef EXL3R_TUNING
    const int split_mode = tuning().rms_split;
    const int split_wm = tuning().rms_split_wm == W_LATE ? W_LATE : W_MID;
#else
    constexpr int split_mode = 0, split_wm = W_MID;
#endif
    if (split_ok && (split_mode == 1 || (split_mode == 0 && wide && rows > 1024))) return split_shape(split_wm);
#ifdef EXL3R_TUNING
    const Tuning& tu = tuning();
    RmsShape sh{ 0, 0, W_EARLY };
    if ((tu.rms_maxv == 1 || tu.rms_maxv == 2 || tu.rms_maxv == 4 || tu.rms_maxv == 8) &&
        (tu.rms_threads == 0 || (tu.rms_threads % 64 == 0 && tu.rms_threads <= 1024)))
    {
        sh.maxv = tu.rms_maxv;
        sh.threads = tu.rms_threads > 0 ? tu.rms_threads : thr(tu.rms_maxv);
        sh.wmode = rows > 1024 && !had ? (mode == RMS_RES_IN ? W_LATE : mode == RMS_PLAIN ? W_MID : W_EARLY) : W_EARLY;
        return sh;
    }
#endif
#ifdef EXL3R_TUNING
    if (rows > 1024 && !had && (mode == RMS_RES_IN || mode == RMS_PLAIN) && tuning().rms_wmode > 0)
    {
        // the automatic lane shape with the weight fetched early (1), mid-row (2) or late (3)
        Tuning t = tuning();
        t.rms_wmode = 0;
        const Tuning saved = tuning();
        tuning() = t;
        RmsShape sh = rms_shape(nc, rows, mode, had, wide);
        tuning() = saved;
        sh.wmode = saved.rms_wmode - 1;
        return sh;
    }
#endif
    if (rows > 1024 && mode == RMS_RES_IN && !had)
    {
        if (nc <= 512) return { 1, thr(1), W_LATE };
        int waves = 1;
        while (waves < 16 && waves * 128 < nc) waves *= 2;
        while (waves > 1 && (waves - 1) * 64 >= nc) waves /= 2;
        const int m = (nc + waves * 64 - 1) / (waves * 64);
        return { pick(m), waves * 64, W_LATE };
    }
    if (rows > 1024)
    {
        const int wm = !had && mode == RMS_PLAIN ? W_MID : W_EARLY;
        if (thr(1) <= 512) return { 1, thr(1), wm };
        if (thr(2) <= 1024) return { 2, thr(2) > 384 || had ? thr(2) : 384, wm };
    }
    static const int opts[3] = { 1, 2, 4 };
    for (int m : opts)
        if (thr(m) <= 1024) return { m, thr(m), W_EARLY };
    return { 8, thr(8), W_EARLY };   // <= 1024 (rms_vec_ok bounds the row at 8192 chunks)
}

template <class XT, class YT, class RT, int MODE, int HAD, int WM, bool SPLIT = false, class ACC = double>
void launch_rms_acc(const RmsArgs& a0, const RmsShape& sh, hipStream_t s)
{
    // Launches of more than kMaxGridX rows go out in blocks of kMaxGridX rows (row0 offsets the block).
    for (int64_t r0 = 0; r0 < a0.rows; r0 += kMaxGridX)
    {
        RmsArgs a = a0;
        a.row0 = r0;
        const dim3 grid((unsigned)(a0.rows - r0 < kMaxGridX ? a0.rows - r0 : kMaxGridX));
        switch (sh.maxv)
        {
            case 1: launch(k_rms_norm<XT, YT, RT, 1, MODE, HAD, WM, SPLIT, ACC>, grid, sh.threads, 0, s, a); break;
            case 2: launch(k_rms_norm<XT, YT, RT, 2, MODE, HAD, WM, SPLIT, ACC>, grid, sh.threads, 0, s, a); break;
            case 4:
                if constexpr (!SPLIT) launch(k_rms_norm<XT, YT, RT, 4, MODE, HAD, WM, false, ACC>, grid, sh.threads, 0, s, a);
                break;
            default:
                if constexpr (!SPLIT) launch(k_rms_norm<XT, YT, RT, 8, MODE, HAD, WM, false, ACC>, grid, sh.threads, 0, s, a);
                break;
        }
    }
}

template <class XT, class YT, class RT, int MODE, int HAD, int WM, bool SPLIT = false>
void launch_rms_wm(const RmsArgs& a0, const RmsShape& sh, hipStream_t s)
{
#ifdef EXL3R_TUNING
    if (HAD == 0 && (MODE == RMS_PLAIN || MODE == RMS_RES_IN) && tuning().rms_sum32 == 1)
        return launch_rms_acc<XT, YT, RT, MODE, HAD, WM, SPLIT, float>(a0, sh, s);
#endif
    launch_rms_acc<XT, YT, RT, MODE, HAD, WM, SPLIT, double>(a0, sh, s);
}

template <class XT, class YT, class RT>
constexpr bool rms_wide = XT::code == DT_F32 || YT::code == DT_F32 || RT::code == DT_F32;

// The resident-grid form: workgroups per CU from the occupancy of the instance (once per instance).
template <class XT, class YT, class RT, int MAXV, int MODE, class ACC>
void launch_rms_pipe(const RmsArgs& a, int threads, int per_cu, hipStream_t s)
{
    static const int resident = [&] {
        int nb = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&nb, k_rms_norm_pipe<XT, YT, RT, MAXV, MODE, ACC>, threads, 0) !=
                hipSuccess || nb < 1)
            nb = 1;
        return nb;
    }();
    int64_t blocks = (int64_t)(per_cu > 0 && per_cu < resident ? per_cu : resident) * device_cus();
    if (blocks > a.rows) blocks = a.rows;
    launch(k_rms_norm_pipe<XT, YT, RT, MAXV, MODE, ACC>, (unsigned)blocks, threads, 0, s, a);
}

template <class XT, class YT, class RT, int MODE, int HAD = 0>
void launch_rms_vec(const RmsArgs& a, hipStream_t s)
{
    const RmsShape sh = rms_shape(a.dim / 8, a.rows, MODE, HAD, rms_wide<XT, YT, RT>);
#ifdef EXL3R_TUNING
    if constexpr (HAD == 0 && (MODE == RMS_RES_IN || MODE == RMS_PLAIN))
    {
        if (tuning().rms_pipe > 0 && !sh.split && a.rows <= kMaxGridX && (sh.maxv == 1 || sh.maxv == 2))
        {
            const int pc = tuning().rms_pipe;   // 1: as many as fit, else that many per CU
            auto go = [&](auto M) {
                constexpr int MV = decltype(M)::value;
                if (tuning().rms_sum32 == 1) launch_rms_pipe<XT, YT, RT, MV, MODE, float>(a, sh.threads, pc - 1, s);
                else launch_rms_pipe<XT, YT, RT, MV, MODE, double>(a, sh.threads, pc - 1, s);
            };
            if (sh.maxv == 1) go(std::integral_constant<int, 1>{});
            else go(std::integral_constant<int, 2>{});
            return;
        }
    }
#endif
    if constexpr (HAD == 0 && (MODE == RMS_RES_IN || MODE == RMS_PLAIN))
    {
        if (sh.split)
        {
            if (sh.wmode == W_LATE) return launch_rms_wm<XT, YT, RT, MODE, HAD, W_LATE, true>(a, sh, s);
            return launch_rms_wm<XT, YT, RT, MODE, HAD, W_MID, true>(a, sh, s);
        }
    }
    if constexpr (HAD == 0 && (MODE == RMS_RES_IN || MODE == RMS_PLAIN))
    {
        if (sh.wmode == W_LATE) return launch_rms_wm<XT, YT, RT, MODE, HAD, W_LATE>(a, sh, s);
        if (sh.wmode == W_MID) return launch_rms_wm<XT, YT, RT, MODE, HAD, W_MID>(a, sh, s);
    }
    launch_rms_wm<XT, YT, RT, MODE, HAD, W_EARLY>(a, sh, s);
}

// The vector kernel needs 16-byte aligned rows of whole chunks and a launch shape that covers the row
// (at most 1024 lanes x 8 chunks).
inline bool rms_vec_ok(const RmsArgs& a, int xt, int yt, int rt, bool has_r, int mode, int had)
{
    if (a.dim % 8 != 0 || a.dim / 8 > 8 * 1024) return false;
    auto ok = [](const void* p, int64_t ld, int dt) {
        return p == nullptr || (aligned16(p) && (ld * dtype_bytes(dt)) % 16 == 0);
    };
    if (!ok(a.x, a.ldx, xt) || !ok(a.y, a.ldy, yt)) return false;
    if (has_r && !ok(a.r, a.ldr, rt)) return false;
    if (a.w && !aligned16(a.w)) return false;
    const bool wide = xt == DT_F32 || yt == DT_F32 || (has_r && rt == DT_F32);
    const RmsShape sh = rms_shape(a.dim / 8, a.rows, mode, had, wide);
    return (int64_t)sh.maxv * sh.threads >= a.dim / 8 && sh.threads <= 1024 && sh.threads % 64 == 0;
}

}  // namespace exl3r
