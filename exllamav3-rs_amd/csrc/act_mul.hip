// Gated activations z = act(x) * y for gfx950: exl3r_silu_mul / exl3r_gelu_mul (replace
// exl3_shim_silu_mul / exl3_shim_gelu_mul, reference csrc/exl3_shim.cpp:151-152 ->
// kernels/activation.cu:24-98, 181-255).
//
// Semantics are the reference's fp32 path (act_mul_kernel_f, kernels/activation_kernels.cuh:189-252)
// applied to upcast inputs: act in fp32, optional act_limit clamps (237-245), product in fp32, one
// round-to-nearest-even to z's dtype, f16 z clamped to +-65504 (2-7, 249-251).
//   silu(x) = x / (1 + exp(-x))                                   (activation_kernels.cuh:34-39)
//   gelu(x) = 0.5 x (1 + tanh(sqrt(2/pi) (x + 0.044715 x^3)))      (activation_kernels.cuh:52-58)
// both evaluated as x * sigmoid(z) by act_f (common.cuh).
//
// Streaming layout: 8-element chunks (16 bytes per 16-bit tensor) per lane, UNROLL chunks in flight
// per thread, strided by blockDim so each wave-wide access is 1 KiB contiguous.  Contiguous
// operands are flattened to one row; strided rows use gridDim.y over rows.
//
// exl3r_act_mul_had feeds the f16 activation straight into the next EXL3 linear's input rotation
// (GatedMlp::forward -> Linear::forward, src/modules.rs:932-940, 224-227): 16 consecutive lanes
// hold the 16 chunks of one 128-element block, so the block's butterfly runs in registers
// (hadamard.cuh) and the activation never returns to memory.
#include "abi.hpp"
#include "common.cuh"
#include "hadamard.cuh"

namespace exl3r {

struct ActArgs
{
    const void* x;
    const void* y;
    void* z;
    int64_t ldx, ldy, ldz;   // row strides (elements)
    int64_t rows;
    int64_t cols;            // elements per row
    float limit;
    // HAD kernels: out = had_r_128(z, hpre) at row stride ldh (f16), hr = scale / sqrt(128); z
    // (the f16 activation) is stored only when non-null.
    const void* hpre;
    void* hout;
    int64_t ldh;
    float hr;
    // AH_IN_X / AH_IN_Y kernels: f16 x / y are first given their projection's output rotation
    // had_r_128(v) * post (xpost / ypost: f16 per column, or null).
    const void* xpost;
    const void* ypost;
};

// Hadamard flags of the act-mul kernels (exl3r_act_mul_had).
constexpr int AH_OUT = 1;    // the f16 activation goes through the next projection's input rotation
constexpr int AH_IN_X = 2;   // x rotated on load
constexpr int AH_IN_Y = 4;   // y rotated on load

template <int ACT, bool LIMIT>
__device__ __forceinline__ float act_mul1(float g, float u, float limit)
{
    float a = act_f<ACT>(g);
    if constexpr (LIMIT)
    {
        if (u < -limit) u = -limit;
        if (u > limit) u = limit;
        if (a > limit) a = limit;
    }
    return a * u;
}

// act_chunk packed to OT, with one wave-uniform test: when no active lane's chunk has an element in
// act_f's tail (t > 64, x < -44.4 for SiLU), every element takes act_f_short -- the operations act_f
// performs there, without the tail's selects -- else act_f.  The results are act_chunk's in both
// cases (a NaN t takes the same operations on either path; fmaxf drops it from the chunk's maximum).
// Each path packs its own results, so that the f16 clamp's negation folds into the conversion.
// Lanes outside the exec mask take no part in the test.
template <int ACT, class OT, bool LIMIT>
__device__ __forceinline__ typename OT::Vec act_pack_wave(const float (&g)[8], const float (&u)[8], float limit)
{
    float t[8], n[8];
    #pragma unroll
    for (int j = 0; j < 8; ++j) t[j] = act_t<ACT>(g[j]);
    const float tmax = fmaxf(fmaxf(fmaxf(t[0], t[1]), fmaxf(t[2], t[3])), fmaxf(fmaxf(t[4], t[5]), fmaxf(t[6], t[7])));
    if (__builtin_amdgcn_ballot_w64(tmax > 64.0f) == 0)
    {
        #pragma unroll
        for (int j = 0; j < 8; ++j)
        {
            float a = act_f_short<ACT>(g[j], t[j]);
            float v = u[j];
            if constexpr (LIMIT)
            {
                if (v < -limit) v = -limit;
                if (v > limit) v = limit;
                if (a > limit) a = limit;
            }
            n[j] = OT::code == DT_F16 ? -nclamp_f16(a * v) : a * v;
        }
        return pack8<OT>(n);
    }
    #pragma unroll
    for (int j = 0; j < 8; ++j)
    {
        const float p = act_mul1<ACT, LIMIT>(g[j], u[j], limit);
        n[j] = OT::code == DT_F16 ? -nclamp_f16(p) : p;
    }
    return pack8<OT>(n);
}

template <int ACT, bool LIMIT>
__device__ __forceinline__ TF16::Vec act_chunk_wave_f16(const float (&g)[8], const float (&u)[8], float limit)
{
    return act_pack_wave<ACT, TF16, LIMIT>(g, u, limit);
}

// The same from the input chunks as loaded.  SiLU of f16 x and u without act_limit takes its three
// products by x and u straight from the packed pairs (mul_f16_f32: the exact conversion and one fp32
// rounding, as the product of the unpacked values), so the short path converts nothing; the results are
// act_chunk_wave_f16's.
template <int ACT, bool LIMIT, class IT>
__device__ __forceinline__ TF16::Vec act_chunk_wave_in(const typename IT::Vec& xv, const typename IT::Vec& yv, float limit)
{
    if constexpr (ACT == ACT_SILU && !LIMIT && IT::code == DT_F16)
    {
        float t[8], n[8];
        #pragma unroll
        for (int j = 0; j < 8; j += 2)
        {
            t[j] = mul_f16_f32<false>(xv.a[j / 2], -kLog2e);
            t[j + 1] = mul_f16_f32<true>(xv.a[j / 2], -kLog2e);
        }
        const float tmax = fmaxf(fmaxf(fmaxf(t[0], t[1]), fmaxf(t[2], t[3])), fmaxf(fmaxf(t[4], t[5]), fmaxf(t[6], t[7])));
        if (__builtin_amdgcn_ballot_w64(tmax > 64.0f) == 0)
        {
            #pragma unroll
            for (int j = 0; j < 8; j += 2)
            {
                const float s0 = __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(t[j]));
                const float s1 = __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(t[j + 1]));
                // s0, s1 come straight from v_rcp_f32 (a transcendental): the first reads wait a state
                n[j] = -nclamp_f16(mul_f16_f32<false>(yv.a[j / 2], mul_f16_f32<false, true>(xv.a[j / 2], s0)));
                n[j + 1] = -nclamp_f16(mul_f16_f32<true>(yv.a[j / 2], mul_f16_f32<true, true>(xv.a[j / 2], s1)));
            }
            return pack8<TF16>(n);
        }
        float g[8], u[8];
        unpack8<IT>(xv, g);
        unpack8<IT>(yv, u);
        #pragma unroll
        for (int j = 0; j < 8; ++j) n[j] = -nclamp_f16(act_mul1<ACT, LIMIT>(g[j], u[j], limit));
        return pack8<TF16>(n);
    }
    else
    {
        float g[8], u[8];
        unpack8<IT>(xv, g);
        unpack8<IT>(yv, u);
        return act_chunk_wave_f16<ACT, LIMIT>(g, u, limit);
    }
}

template <int ACT, class OT, bool LIMIT>
__device__ __forceinline__ void act_chunk(const float (&g)[8], const float (&u)[8], float limit, float (&o)[8])
{
    #pragma unroll
    for (int j = 0; j < 8; ++j)
    {
        float p = act_mul1<ACT, LIMIT>(g[j], u[j], limit);
        if constexpr (OT::code == DT_F16) p = clamp_f16(p);
        o[j] = p;
    }
}

// SPLIT: split chunks (two quads 256 apart) for rows of whole 512-element spans with an f32 side, so
// that each wave-wide f32 access is one contiguous 1 KB.
template <int ACT, class IT, class OT, int UNROLL, bool LIMIT, int HAD = 0, bool SPLIT = false>
__global__ __launch_bounds__(256) void k_act_mul(ActArgs a)
{
    static_assert(!SPLIT || HAD == 0, "split chunks: no Hadamard blocks");
    const int64_t cpr = a.cols >> 3;   // chunks per row
    const int nt = blockDim.x;
    for (int64_t row = blockIdx.y; row < a.rows; row += gridDim.y)
    {
        const char* xr = (const char*)a.x + row * a.ldx * IT::bytes;
        const char* yr = (const char*)a.y + row * a.ldy * IT::bytes;
        char* zr = (char*)a.z + row * a.ldz * OT::bytes;
        for (int64_t base = (int64_t)blockIdx.x * nt * UNROLL + threadIdx.x; base < cpr;
             base += (int64_t)gridDim.x * nt * UNROLL)
        {
            typename IT::Vec xv[UNROLL], yv[UNROLL];
            #pragma unroll
            for (int u = 0; u < UNROLL; ++u)
            {
                const int64_t c = base + (int64_t)u * nt;
                if (c < cpr)
                {
                    if constexpr (SPLIT)
                    {
                        xv[u] = load8s_split<IT>(xr, chunk_elem<true>(c));
                        yv[u] = load8s_split<IT>(yr, chunk_elem<true>(c));
                    }
                    else
                    {
                        xv[u] = load8s<IT>(xr, c * 8);
                        yv[u] = load8s<IT>(yr, c * 8);
                    }
                }
            }
            if constexpr (HAD == 0)
            {
                #pragma unroll
                for (int u = 0; u < UNROLL; ++u)
                {
                    const int64_t c = base + (int64_t)u * nt;
                    if (c < cpr)
                    {
                        float g[8], v[8];
                        unpack8<IT>(xv[u], g);
                        unpack8<IT>(yv[u], v);
                        const typename OT::Vec o = act_pack_wave<ACT, OT, LIMIT>(g, v, a.limit);
                        if constexpr (SPLIT) store8_split<OT>(zr, chunk_elem<true>(c), o);
                        else store8<OT>(zr, c * 8, o);
                    }
                }
            }
            else if constexpr ((HAD & (AH_IN_X | AH_IN_Y)) == 0)
            {
                // The output rotation alone: the exact stages, block by block (with the carried-sign
                // stages, and with the blocks of a step rotated together, [8192, 17408] f16 ran 161-164
                // against 148-153 us: this kernel's time is not the butterfly's).
                #pragma unroll
                for (int u = 0; u < UNROLL; ++u)
                {
                    const int64_t c = base + (int64_t)u * nt;
                    if (c < cpr)
                    {
                        static_assert(OT::code == DT_F16, "the Hadamard prologue follows an f16 activation");
                        float g[8], v[8], o[8];
                        unpack8<IT>(xv[u], g);
                        unpack8<IT>(yv[u], v);
                        act_chunk<ACT, OT, LIMIT>(g, v, a.limit, o);
                        TF16::Vec hv = pack8<TF16>(o);
                        if (a.z) store8<TF16>(zr, c * 8, hv);
                        if (a.hpre)
                        {
                            const TF16::Vec p = load8<TF16>(a.hpre, c * 8);
                            #pragma unroll
                            for (int q = 0; q < 4; ++q) hv.a[q] = hmul2(hv.a[q], p.a[q]);
                        }
                        float f[8];
                        butterfly128_f16<false>(hv, f, (int)(c & 15), a.hr);
                        store8<TF16>((char*)a.hout + row * a.ldh * 2, c * 8, pack8<TF16>(f));
                    }
                }
            }
            else
            {
                // The group of 16 lanes holding chunks c & ~15 .. c | 15 is one 128-column block (the
                // row length is a multiple of 128 and nt * UNROLL of 16), all active together.  One
                // wave-uniform choice of butterfly stages (hadamard.cuh) covers every block of a step.
                static_assert(OT::code == DT_F16, "the Hadamard prologue follows an f16 activation");
                // With the input rotations the three butterflies per element set the time: the
                // carried-sign stages where valid (MI355X, [8192, 17408] f16: 248-252 vs 270-272 us).
                bool live[UNROLL];
                #pragma unroll
                for (int u = 0; u < UNROLL; ++u) live[u] = base + (int64_t)u * nt < cpr;
                if constexpr ((HAD & (AH_IN_X | AH_IN_Y)) != 0)
                {
                    // Input rotations: x / y get their projections' output rotations first.
                    static_assert(IT::code == DT_F16, "input rotations take f16 x and y");
                    bool zero = false;
                    #pragma unroll
                    for (int u = 0; u < UNROLL; ++u)
                        if (live[u])
                        {
                            if constexpr ((HAD & AH_IN_X) != 0) zero |= zero_lane16(xv[u]);
                            if constexpr ((HAD & AH_IN_Y) != 0) zero |= zero_lane16(yv[u]);
                        }
                    with_carried<true>(zero, 0.0883883461356163f, [&](auto C) {
                        #pragma unroll
                        for (int u = 0; u < UNROLL; ++u)
                            if (live[u])
                            {
                                const int64_t c = base + (int64_t)u * nt;
                                if constexpr ((HAD & AH_IN_X) != 0) output_rotation8<decltype(C)::value>(xv[u], a.xpost, c * 8);
                                if constexpr ((HAD & AH_IN_Y) != 0) output_rotation8<decltype(C)::value>(yv[u], a.ypost, c * 8);
                            }
                    });
                }
                TF16::Vec hvs[UNROLL];
                bool zero = false;
                #pragma unroll
                for (int u = 0; u < UNROLL; ++u)
                {
                    const int64_t c = base + (int64_t)u * nt;
                    if (live[u])
                    {
                        float g[8], v[8], o[8];
                        unpack8<IT>(xv[u], g);
                        unpack8<IT>(yv[u], v);
                        act_chunk<ACT, OT, LIMIT>(g, v, a.limit, o);
                        TF16::Vec hv = pack8<TF16>(o);
                        if (a.z) store8<TF16>(zr, c * 8, hv);
                        if (a.hpre)
                        {
                            const TF16::Vec p = load8<TF16>(a.hpre, c * 8);
                            #pragma unroll
                            for (int q = 0; q < 4; ++q) hv.a[q] = hmul2(hv.a[q], p.a[q]);
                        }
                        hvs[u] = hv;
                        zero |= zero_lane16(hv);
                    }
                }
                with_carried<true>(zero, a.hr, [&](auto C) {
                    #pragma unroll
                    for (int u = 0; u < UNROLL; ++u)
                        if (live[u])
                        {
                            const int64_t c = base + (int64_t)u * nt;
                            float f[8];
                            butterfly128_f16<decltype(C)::value>(hvs[u], f, (int)(c & 15), a.hr);
                            store8<TF16>((char*)a.hout + row * a.ldh * 2, c * 8, pack8<TF16>(f));
                        }
                });
            }
        }
    }
}

// The activation -> Hadamard kernels with the transforms on the matrix cores (had128_mfma, hadamard.cuh).
// A wave takes a span of 64 chunks (4 blocks) in UNROLL consecutive rows, lane l holding chunk
// mfma_chunk(l) of the span in each row; the (row group, span) items of the tensor (counted in 32 bits)
// are dealt to the waves of the grid in turn.  The span's scale chunks are loaded once for its rows.
// Every access goes through a row's bounded buffer descriptor, so the chunks past a row's last block
// (whole blocks: cols is a multiple of 128) and the rows past the last one load zeros and store
// nothing, with no per-lane branch; loop bounds are wave-uniform, so every MFMA runs with the whole
// wave.  Same rounding points as the butterfly kernel (hadamard.cuh documents how the transform's sums
// may differ).
template <int ACT, class IT, int HAD, bool LIMIT, int UNROLL>
__global__ __launch_bounds__(256) void k_act_mul_had_mfma(ActArgs a)
{
    static_assert((HAD & AH_OUT) != 0, "the input rotations come with the output rotation");
    constexpr bool IN_X = (HAD & AH_IN_X) != 0, IN_Y = (HAD & AH_IN_Y) != 0;
    static_assert(!(IN_X || IN_Y) || IT::code == DT_F16, "input rotations take f16 x and y");
    const int lane = threadIdx.x & 63;
    const uint32_t cpr = (uint32_t)(a.cols >> 3);
    const uint32_t spr = (cpr + 63) >> 6;
    const uint32_t rows = (uint32_t)a.rows;
    const uint32_t items = ((rows + UNROLL - 1) / UNROLL) * spr;
    const uint32_t in_bytes = (uint32_t)a.cols * IT::bytes, out_bytes = (uint32_t)a.cols * 2;
    // wave-uniform item, row and span indices (scalar registers: the descriptors are scalar)
    const uint32_t wave = __builtin_amdgcn_readfirstlane((blockIdx.x * blockDim.x + threadIdx.x) >> 6);
    const uint32_t nwaves = (gridDim.x * blockDim.x) >> 6;
    const HadMfmaWords hw = had_mfma_words(lane);
    const uint32_t lc = (uint32_t)mfma_chunk(lane);
    const brsrc xpost = row_rsrc(a.xpost, a.xpost ? out_bytes : 0), ypost = row_rsrc(a.ypost, a.ypost ? out_bytes : 0);
    const brsrc hpre = row_rsrc(a.hpre, a.hpre ? out_bytes : 0);
    for (uint32_t it = wave; it < items; it += nwaves)
    {
        const uint32_t rg = it / spr, sp = it - rg * spr;
        const uint32_t c = sp * 64 + lc;                                  // the lane's chunk in each row
        const uint32_t off_in = c * (8 * IT::bytes), off16 = c * 16;     // its byte offsets
        typename IT::Vec xv[UNROLL], yv[UNROLL];
        brsrc zr[UNROLL], hr[UNROLL];
        #pragma unroll
        for (int u = 0; u < UNROLL; ++u)
        {
            const uint32_t row = rg * UNROLL + u;
            const bool in = row < rows;
            const int64_t r = in ? row : 0;
            xv[u] = bload8s<IT>(row_rsrc((const char*)a.x + r * a.ldx * IT::bytes, in ? in_bytes : 0), off_in);
            yv[u] = bload8s<IT>(row_rsrc((const char*)a.y + r * a.ldy * IT::bytes, in ? in_bytes : 0), off_in);
            zr[u] = row_rsrc((char*)a.z + r * a.ldz * 2, in && a.z ? out_bytes : 0);
            hr[u] = row_rsrc((char*)a.hout + r * a.ldh * 2, in ? out_bytes : 0);
        }
        TF16::Vec px, py, pp;
        if constexpr (IN_X) px.a = bload16(xpost, off16);
        if constexpr (IN_Y) py.a = bload16(ypost, off16);
        if (a.hpre) pp.a = bload16(hpre, off16);
        if constexpr (IN_X || IN_Y)
        {
            // the input rotations of every row in flight, their MFMAs issued together; each transform,
            // one rounding to f16, then the half post-scale
            constexpr int NX = IN_X ? UNROLL : 0, NY = IN_Y ? UNROLL : 0;
            TF16::Vec in[NX + NY];
            #pragma unroll
            for (int u = 0; u < UNROLL; ++u)
            {
                if constexpr (IN_X) in[u] = xv[u];
                if constexpr (IN_Y) in[NX + u] = yv[u];
            }
            MfmaOut m[NX + NY];
            had128_mfma_issue_w(hw, in, m);
            mfma_wait_all(m);
            auto finish = [&](const MfmaOut& mo, const TF16::Vec& p, bool on) {
                float f[8];
                had128_mfma_finish(mo, f, lane, 0.0883883461356163f);
                TF16::Vec v = pack8<TF16>(f);
                if (on)
                {
                    #pragma unroll
                    for (int q = 0; q < 4; ++q) v.a[q] = hmul2(v.a[q], p.a[q]);
                }
                return v;
            };
            #pragma unroll
            for (int u = 0; u < UNROLL; ++u)
            {
                if constexpr (IN_X) xv[u] = finish(m[u], px, a.xpost != nullptr);
                if constexpr (IN_Y) yv[u] = finish(m[NX + u], py, a.ypost != nullptr);
            }
        }
        TF16::Vec hv[UNROLL];
        #pragma unroll
        for (int u = 0; u < UNROLL; ++u)
        {
            hv[u] = act_chunk_wave_in<ACT, LIMIT, IT>(xv[u], yv[u], a.limit);
            if (a.z) bstore16(zr[u], off16, hv[u].a);
            if (a.hpre)
            {
                #pragma unroll
                for (int q = 0; q < 4; ++q) hv[u].a[q] = hmul2(hv[u].a[q], pp.a[q]);
            }
        }
        MfmaOut m[UNROLL];
        had128_mfma_issue_w(hw, hv, m);
        mfma_wait_all(m);
        #pragma unroll
        for (int u = 0; u < UNROLL; ++u)
        {
            float f[8];
            had128_mfma_finish(m[u], f, lane, a.hr);
            bstore16(hr[u], off16, pack8<TF16>(f).a);
        }
    }
}

// Short strided rows (at most 64 chunks, e.g. the gate of one 128-wide head read in place from an
// interleaved q | g projection): (row, chunk) items flattened over the whole grid, so a workgroup
// covers several rows instead of idling most of its lanes on one.  UNROLL items per thread in flight.
template <int ACT, class IT, class OT, int UNROLL, bool LIMIT>
__global__ __launch_bounds__(256) void k_act_mul_short(ActArgs a)
{
    const uint32_t cpr = (uint32_t)(a.cols >> 3);
    const uint32_t n = (uint32_t)a.rows * cpr;
    const uint32_t nt = blockDim.x;
    for (uint32_t base = blockIdx.x * nt * UNROLL + threadIdx.x; base < n; base += gridDim.x * nt * UNROLL)
    {
        typename IT::Vec xv[UNROLL], yv[UNROLL];
        uint32_t r[UNROLL], c[UNROLL];
        #pragma unroll
        for (int u = 0; u < UNROLL; ++u)
        {
            const uint32_t i = base + u * nt;
            r[u] = i / cpr;
            c[u] = i - r[u] * cpr;
            if (i < n)
            {
                xv[u] = load8s<IT>((const char*)a.x + (int64_t)r[u] * a.ldx * IT::bytes, (int64_t)c[u] * 8);
                yv[u] = load8s<IT>((const char*)a.y + (int64_t)r[u] * a.ldy * IT::bytes, (int64_t)c[u] * 8);
            }
        }
        #pragma unroll
        for (int u = 0; u < UNROLL; ++u)
        {
            if (base + u * nt >= n) continue;
            float g[8], v[8];
            unpack8<IT>(xv[u], g);
            unpack8<IT>(yv[u], v);
            store8<OT>((char*)a.z + (int64_t)r[u] * a.ldz * OT::bytes, (int64_t)c[u] * 8,
                       act_pack_wave<ACT, OT, LIMIT>(g, v, a.limit));
        }
    }
}

// Generic fallback: any shape, stride and alignment, one element per thread.
template <int ACT>
__global__ __launch_bounds__(256) void k_act_mul_generic(ActArgs a, int it, int ot)
{
    const int64_t n = a.rows * a.cols;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
    {
        const int64_t r = i / a.cols, c = i - r * a.cols;
        const float g = load1(a.x, it, r * a.ldx + c);
        const float u = load1(a.y, it, r * a.ldy + c);
        float p = a.limit != 0.0f ? act_mul1<ACT, true>(g, u, a.limit) : act_mul1<ACT, false>(g, u, a.limit);
        if (ot == DT_F16) p = clamp_f16(p);
        store1(a.z, ot, r * a.ldz + c, p);
    }
}

template <int ACT, class IT, class OT, int HAD = 0>
static void launch_act_vec(const ActArgs& a, hipStream_t s)
{
    const Tuning& tu = tuning();
    // Streaming launches take two chunks per thread: in one-wave workgroups from 32M elements (C3 bf16,
    // same process, us: 2 x 64 lanes 130.8 GELU / 131.0 SiLU against 134.0 / 134.9 with 2 x 128 and
    // 131.7 / 132.0 with 2 x 192; 1 x 64 133.8 / 134.5, 4 x 64 134.6 / 135.0; SiLU bf16 at [8192, 13824 ..
    // 25600] and [16384, 4096] 1-4% faster), in 128-thread workgroups below that (16.8M elements: SiLU
    // 18.38 against 18.60, the in-place sigmoid gate 18.19 against 18.65; 33.6M: the same); the
    // butterfly Hadamard forms at [8192, 17408] alike (145.1 against 147.0, with the input rotations
    // 222.0 against 222.9; each pair timed alternately).  Up to 8M elements one chunk per thread in 256-thread
    // workgroups (HIP graph, us, [rows, 17408] f16: 64 rows 3.15 vs 3.46, 256 rows 5.03 vs 5.41;
    // [512, 3072] 3.24 vs 3.54; from 1024 rows the streaming shape wins, 16.9 vs 18.8).
    const bool small = a.rows * a.cols <= ((int64_t)8 << 20);
    const int unroll = (tu.act_unroll == 1 || tu.act_unroll == 2 || tu.act_unroll == 4 || tu.act_unroll == 8) ? tu.act_unroll
                       : small ? 1 : 2;
    const bool one_wave = a.rows * a.cols >= ((int64_t)1 << 25);
    const int threads = (tu.act_threads > 0 && tu.act_threads % 64 == 0 && tu.act_threads <= 256) ? tu.act_threads
                        : small ? 256 : one_wave ? 64 : 128;
    const int64_t cpr = a.cols >> 3;
    if constexpr (HAD == 0)
    {
        // Rows of at most 64 chunks: one workgroup per row would idle most of its lanes (a 128-wide
        // strided gate: 52 us against 17 us for the same bytes as one flat row).
        if (a.rows > 1 && cpr <= 64 && a.rows * cpr < ((int64_t)1 << 31))
        {
            const int64_t n = a.rows * cpr;
            int64_t blocks = (n + 256 * 2 - 1) / (256 * 2);
            if (blocks > kMaxGridX) blocks = kMaxGridX;
            if (a.limit != 0.0f) launch(k_act_mul_short<ACT, IT, OT, 2, true>, (unsigned)blocks, 256, 0, s, a);
            else launch(k_act_mul_short<ACT, IT, OT, 2, false>, (unsigned)blocks, 256, 0, s, a);
            return;
        }
    }
    const int per = a.limit != 0.0f ? 2 : unroll;
    int64_t bx = (cpr + (int64_t)threads * per - 1) / ((int64_t)threads * per);
    if (tu.act_blocks_per_cu > 0)
    {
        const int64_t cap = (int64_t)tu.act_blocks_per_cu * device_cus() / (a.rows < 65535 ? (a.rows > 0 ? a.rows : 1) : 65535);
        if (bx > cap) bx = cap > 0 ? cap : 1;
    }
    if (bx > kMaxGridX) bx = kMaxGridX;
    const dim3 grid((unsigned)bx, (unsigned)(a.rows < 65535 ? a.rows : 65535));
    if constexpr (HAD == 0 && (IT::code == DT_F32 || OT::code == DT_F32))
    {
        if (a.cols % 512 == 0 && tu.rms_split != -1)
        {
            // two chunks per thread (the grid-stride loop covers the row whatever the grid)
            if (a.limit != 0.0f) launch(k_act_mul<ACT, IT, OT, 2, true, 0, true>, grid, threads, 0, s, a);
            else launch(k_act_mul<ACT, IT, OT, 2, false, 0, true>, grid, threads, 0, s, a);
            return;
        }
    }
    if (a.limit != 0.0f)
        launch(k_act_mul<ACT, IT, OT, 2, true, HAD>, grid, threads, 0, s, a);
    else
    {
        switch (unroll)
        {
            case 1: launch(k_act_mul<ACT, IT, OT, 1, false, HAD>, grid, threads, 0, s, a); break;
            case 2: launch(k_act_mul<ACT, IT, OT, 2, false, HAD>, grid, threads, 0, s, a); break;
            case 8: launch(k_act_mul<ACT, IT, OT, 8, false, HAD>, grid, threads, 0, s, a); break;
            default: launch(k_act_mul<ACT, IT, OT, 4, false, HAD>, grid, threads, 0, s, a); break;
        }
    }
}

// Grid of the matrix-core kernel: one wave per item (a span in UNROLL rows), no cap
// (kHadMfmaBlocksPerCu <= 0); the tuning build sweeps UNROLL and a looping grid of that many workgroups
// per CU.
constexpr int kHadMfmaBlocksPerCu = -1;

template <int ACT, class IT, int HAD, int UNROLL>
static void launch_act_had_mfma_u(const ActArgs& a, int per_cu, hipStream_t s)
{
    const int64_t items = (a.rows + UNROLL - 1) / UNROLL * ((a.cols / 8 + 63) / 64);
    const int threads = had_threads();
    const int wpb = threads / 64;
    int64_t blocks = (items + wpb - 1) / wpb;
    if (per_cu > 0 && blocks > (int64_t)per_cu * device_cus()) blocks = (int64_t)per_cu * device_cus();
    if (blocks > kMaxGridX) blocks = kMaxGridX;
    if (a.limit != 0.0f) launch(k_act_mul_had_mfma<ACT, IT, HAD, true, UNROLL>, (unsigned)blocks, threads, 0, s, a);
    else launch(k_act_mul_had_mfma<ACT, IT, HAD, false, UNROLL>, (unsigned)blocks, threads, 0, s, a);
}

template <int ACT, class IT, int HAD>
static void launch_act_had_mfma(const ActArgs& a, hipStream_t s)
{
#ifdef EXL3R_TUNING
    const Tuning& tu = tuning();
    const int per_cu = tu.had_mfma_per_cu != 0 ? tu.had_mfma_per_cu : kHadMfmaBlocksPerCu;   // <= 0: no cap
    if (tu.had_mfma_unroll == 1) launch_act_had_mfma_u<ACT, IT, HAD, 1>(a, per_cu, s);
    else if (tu.had_mfma_unroll == 4) launch_act_had_mfma_u<ACT, IT, HAD, 4>(a, per_cu, s);
    else launch_act_had_mfma_u<ACT, IT, HAD, 2>(a, per_cu, s);
#else
    launch_act_had_mfma_u<ACT, IT, HAD, 2>(a, kHadMfmaBlocksPerCu, s);
#endif
}

extern "C" int exl3r_had_r_128(const void* x, int dtype, int64_t ldx, void* out, int64_t ldo, int64_t rows,
                               int64_t cols, const void* pre_scale, const void* post_scale, float scale, void* stream);

template <int ACT>
static int act_mul_entry(const char* op, const void* x, const void* y, int it, void* z, int ot,
                         int64_t rows, int64_t cols, int64_t ldx, int64_t ldy, int64_t ldz,
                         float limit, void* stream);

// Activation -> Hadamard: the vector kernel with HAD when every row is 16-byte aligned, else the
// activation into z (or into out) and had_r_128 over it in place.
template <int ACT>
static int act_had_entry(const char* op, const void* x, const void* y, int it, int64_t ldx, int64_t ldy,
                         void* z, int64_t ldz, const void* pre, void* out, int64_t ldo,
                         int64_t rows, int64_t cols, float limit, float had_scale, int rotate_in,
                         const void* x_post, const void* y_post, void* stream)
{
    begin_call();
    if (!is_float_dtype(it)) return set_error(EXL3R_EDTYPE, "%s: unsupported input dtype %s", op, dtype_name(it));
    const bool exact = (rotate_in & EXL3R_HAD_EXACT) != 0;
    rotate_in &= ~EXL3R_HAD_EXACT;
    if (rotate_in & ~3) return set_error(EXL3R_EINVAL, "%s: rotate_in takes bits 0 (x) and 1 (y) and EXL3R_HAD_EXACT", op);
    if (rotate_in && it != EXL3R_F16) return set_error(EXL3R_EDTYPE, "%s: rotated inputs are f16", op);
    if ((x_post && !(rotate_in & 1)) || (y_post && !(rotate_in & 2)))
        return set_error(EXL3R_EINVAL, "%s: a post-scale without its input rotation", op);
    if (rows < 0 || cols <= 0 || cols % 128 || (rows > 1 && (ldx < cols || ldy < cols || ldo < cols || (z && ldz < cols))))
        return set_error(EXL3R_EINVAL, "%s: invalid shape rows=%lld cols=%lld (a multiple of 128) or row strides", op,
                         (long long)rows, (long long)cols);
    if (rows == 0) return EXL3R_OK;
    if (!x || !y || !out) return set_error(EXL3R_EINVAL, "%s: x, y and out must be non-null", op);
    if (out == x || out == y || out == z || (z && (z == x || z == y)))
        return set_error(EXL3R_EINVAL, "%s: out and z must not alias the inputs or each other", op);
    const int64_t lx = rows > 1 ? ldx : cols, ly = rows > 1 ? ldy : cols, lo = rows > 1 ? ldo : cols;
    const int64_t lz = z ? (rows > 1 ? ldz : cols) : cols;
    hipStream_t s = (hipStream_t)stream;
    const int eb = dtype_bytes(it);
    const bool vec = aligned16(x) && aligned16(y) && aligned16(out) && (!z || aligned16(z)) && (!pre || aligned16(pre)) &&
                     (!x_post || aligned16(x_post)) && (!y_post || aligned16(y_post)) &&
                     (lx * eb) % 16 == 0 && (ly * eb) % 16 == 0 && (lo * 2) % 16 == 0 && (lz * 2) % 16 == 0;
    // The matrix-core transforms unless the caller asks for the reference's butterfly; items are counted
    // in 32 bits, and a row's bytes in a buffer descriptor's 32-bit length.
    const bool mfma = !exact && rows * ((cols / 8 + 63) / 64) < ((int64_t)1 << 31) && cols * eb < ((int64_t)1 << 31);
    if (vec && mfma)
    {
        ActArgs a{ x, y, z, lx, ly, lz, rows, cols, limit, pre, out, lo, had_scale * 0.0883883461356163f, x_post, y_post };
        if (rotate_in == 3) launch_act_had_mfma<ACT, TF16, AH_OUT | AH_IN_X | AH_IN_Y>(a, s);
        else if (rotate_in == 1) launch_act_had_mfma<ACT, TF16, AH_OUT | AH_IN_X>(a, s);
        else if (rotate_in == 2) launch_act_had_mfma<ACT, TF16, AH_OUT | AH_IN_Y>(a, s);
        else with_float_type(it, [&](auto I) { launch_act_had_mfma<ACT, decltype(I), AH_OUT>(a, s); });
        return launch_status(op);
    }
    if (vec)
    {
        ActArgs a{ x, y, z, lx, ly, lz, rows, cols, limit, pre, out, lo, had_scale * 0.0883883461356163f, x_post, y_post };
        if (rotate_in == 3) launch_act_vec<ACT, TF16, TF16, AH_OUT | AH_IN_X | AH_IN_Y>(a, s);
        else if (rotate_in == 1) launch_act_vec<ACT, TF16, TF16, AH_OUT | AH_IN_X>(a, s);
        else if (rotate_in == 2) launch_act_vec<ACT, TF16, TF16, AH_OUT | AH_IN_Y>(a, s);
        else with_float_type(it, [&](auto I) { launch_act_vec<ACT, decltype(I), TF16, AH_OUT>(a, s); });
        return launch_status(op);
    }
    // The input rotations have no buffer of their own to go through outside the fused kernel.
    if (rotate_in) return set_error(EXL3R_EINVAL, "%s: rotated inputs need 16-byte aligned rows", op);
    void* dst = z ? z : out;
    const int64_t ld = z ? lz : lo;
    int rc = act_mul_entry<ACT>(op, x, y, it, dst, EXL3R_F16, rows, cols, lx, ly, ld, limit, stream);
    if (rc == EXL3R_OK) rc = exl3r_had_r_128(dst, EXL3R_F16, ld, out, lo, rows, cols, pre, nullptr, had_scale, stream);
    return rc;
}

template <int ACT>
static int act_mul_entry(const char* op, const void* x, const void* y, int it, void* z, int ot,
                         int64_t rows, int64_t cols, int64_t ldx, int64_t ldy, int64_t ldz,
                         float limit, void* stream)
{
    if (rows < 0 || cols < 0) return set_error(EXL3R_EINVAL, "%s: invalid shape rows=%lld cols=%lld", op, (long long)rows, (long long)cols);
    if (rows > 1 && (ldx < cols || ldy < cols || ldz < cols))
        return set_error(EXL3R_EINVAL, "%s: row strides must be >= cols", op);
    if (!is_float_dtype(it) || !is_float_dtype(ot))
        return set_error(EXL3R_EDTYPE, "%s: unsupported dtypes in=%s z=%s", op, dtype_name(it), dtype_name(ot));
    if (rows == 0 || cols == 0) return EXL3R_OK;
    if (!x || !y || !z) return set_error(EXL3R_EINVAL, "%s: x, y and z must be non-null", op);
    if ((z == x && (ot != it || ldz != ldx)) || (z == y && (ot != it || ldz != ldy)))
        return set_error(EXL3R_EINVAL, "%s: in-place z needs the aliased operand's dtype and stride", op);

    ActArgs a{ x, y, z, ldx, ldy, ldz, rows, cols, limit };
    if (rows == 1 || (ldx == cols && ldy == cols && ldz == cols))
    {
        a.cols = rows * cols;
        a.rows = 1;
        a.ldx = a.ldy = a.ldz = a.cols;
    }
    hipStream_t s = (hipStream_t)stream;

    const bool rows_ok = a.rows == 1 || ((a.ldx * dtype_bytes(it)) % 16 == 0 && (a.ldy * dtype_bytes(it)) % 16 == 0 &&
                                         (a.ldz * dtype_bytes(ot)) % 16 == 0 && a.cols % 8 == 0);
    const bool vec = rows_ok && aligned16(x) && aligned16(y) && aligned16(z) && a.cols >= 8;
    if (vec)
    {
        const int64_t body = a.cols & ~(int64_t)7;
        ActArgs b = a;
        b.cols = body;
        with_float_type(it, [&](auto I) {
            with_float_type(ot, [&](auto O) { launch_act_vec<ACT, decltype(I), decltype(O)>(b, s); });
        });
        if (body != a.cols)   // flat tail of < 8 elements
        {
            ActArgs t = a;
            t.x = (const char*)a.x + body * dtype_bytes(it);
            t.y = (const char*)a.y + body * dtype_bytes(it);
            t.z = (char*)a.z + body * dtype_bytes(ot);
            t.cols = a.cols - body;
            t.ldx = t.ldy = t.ldz = t.cols;
            launch(k_act_mul_generic<ACT>, 1, 64, 0, s, t, it, ot);
        }
    }
    else
    {
        const int64_t n = a.rows * a.cols;
        int64_t blocks = (n + 255) / 256;
        if (blocks > kMaxGridX) blocks = kMaxGridX;
        launch(k_act_mul_generic<ACT>, (unsigned)blocks, 256, 0, s, a, it, ot);
    }
    return launch_status(op);
}

}  // namespace exl3r

using namespace exl3r;

extern "C" int exl3r_silu_mul(const void* x, const void* y, int in_dtype, void* z, int z_dtype,
                              int64_t rows, int64_t cols, int64_t ldx, int64_t ldy, int64_t ldz,
                              float act_limit, void* stream)
{
    begin_call();
    return act_mul_entry<ACT_SILU>("exl3r_silu_mul", x, y, in_dtype, z, z_dtype, rows, cols, ldx, ldy, ldz, act_limit, stream);
}

extern "C" int exl3r_gelu_mul(const void* x, const void* y, int in_dtype, void* z, int z_dtype,
                              int64_t rows, int64_t cols, int64_t ldx, int64_t ldy, int64_t ldz,
                              float act_limit, void* stream)
{
    begin_call();
    return act_mul_entry<ACT_GELU>("exl3r_gelu_mul", x, y, in_dtype, z, z_dtype, rows, cols, ldx, ldy, ldz, act_limit, stream);
}

extern "C" int exl3r_act_mul_had(int act, const void* x, const void* y, int in_dtype, int64_t ldx, int64_t ldy,
                                 void* z, int64_t ldz, const void* pre_scale, void* out, int64_t ldo,
                                 int64_t rows, int64_t cols, float act_limit, float had_scale, int rotate_in,
                                 const void* x_post_scale, const void* y_post_scale, void* stream)
{
    begin_call();
    const char* op = "exl3r_act_mul_had";
    switch (act)
    {
        case EXL3R_ACT_SILU:
            return act_had_entry<ACT_SILU>(op, x, y, in_dtype, ldx, ldy, z, ldz, pre_scale, out, ldo, rows, cols,
                                           act_limit, had_scale, rotate_in, x_post_scale, y_post_scale, stream);
        case EXL3R_ACT_GELU:
            return act_had_entry<ACT_GELU>(op, x, y, in_dtype, ldx, ldy, z, ldz, pre_scale, out, ldo, rows, cols,
                                           act_limit, had_scale, rotate_in, x_post_scale, y_post_scale, stream);
        case EXL3R_ACT_MUL_SIGMOID:
        {
            if (act_limit != 0.0f) return set_error(EXL3R_EINVAL, "%s: act_limit applies to silu / gelu only", op);
            // The kernels take the gate first: x and y, their rotations and post-scales swap.
            const int bits = rotate_in & ~EXL3R_HAD_EXACT;
            const int swapped = bits & ~3 ? rotate_in
                                          : (((bits & 1) << 1) | ((bits >> 1) & 1) | (rotate_in & EXL3R_HAD_EXACT));
            return act_had_entry<ACT_SIGMOID>(op, y, x, in_dtype, ldy, ldx, z, ldz, pre_scale, out, ldo, rows, cols,
                                              0.0f, had_scale, swapped, y_post_scale, x_post_scale, stream);
        }
        default: return set_error(EXL3R_EINVAL, "%s: unknown act %d", op, act);
    }
}

// z = x * sigmoid(y): the act-mul kernels with the gate and value operands exchanged.
extern "C" int exl3r_mul_sigmoid(const void* x, const void* y, int in_dtype, void* z, int z_dtype,
                                 int64_t rows, int64_t cols, int64_t ldx, int64_t ldy, int64_t ldz, void* stream)
{
    begin_call();
    return act_mul_entry<ACT_SIGMOID>("exl3r_mul_sigmoid", y, x, in_dtype, z, z_dtype, rows, cols, ldy, ldx, ldz, 0.0f,
                                      stream);
}
