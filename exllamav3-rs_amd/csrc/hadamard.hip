// Random-Hadamard row transform for gfx950: exl3r_had_r_128 (replaces exl3_shim_had_r_128, reference
// csrc/exl3_shim.cpp:158-160 -> had_r_128, kernels/quant/hadamard.cu:88-170; the EXL3 linear's prefill
// input and output rotations, src/modules.rs:224-231).
//
// Every 128-element block of a row becomes r * H128 (x o pre) o post with H128 the Sylvester Hadamard
// matrix and r = fl32(scale * fl32(1/sqrt(128))).  Rounding points are the reference's: an f16
// pre-scale product is a half multiply, the transform runs in fp32 as the in-place butterfly over
// index bits 0..6 in that order ((a, b) -> (a + b, a - b), a the lower index), the result times r
// is rounded once to the I/O type, and an f16 post-scale is another half multiply.  f32 I/O uses
// fp32 scale products.  The same butterfly order on every path makes the results bit-identical.
//
// Layout: a block is held by 16 lanes, 8 elements (one 16-byte f16 chunk, two for f32) per lane, so
// index bits 0..2 are in-lane stages and bits 3..6 lane exchanges at xor 1, 2 (DPP quad_perm) and
// xor 4, 8 (ds_swizzle bit mode); a wave holds 4 blocks, a workgroup 16.  Rows that are not 16-byte
// aligned take a workgroup-per-block kernel that runs the same butterfly through LDS.
#include "abi.hpp"
#include "common.cuh"
#include "hadamard.cuh"

namespace exl3r {

struct HadArgs
{
    const char* x;
    char* out;
    int64_t ldx, ldo;        // row strides, bytes
    int64_t rows, nb;        // rows, 128-blocks per row
    const uint16_t* pre;     // f16 [nb * 128] or nullptr
    const uint16_t* post;
    float r;                 // scale / sqrt(128), rounded to fp32
};

template <class IO, bool PRE, bool POST>
__device__ __forceinline__ void had_block(const HadArgs& a, int64_t blk, int l16, typename IO::Vec v)
{
    #pragma clang fp contract(off)
    const int64_t row = blk / a.nb;
    const int64_t e0 = (blk - row * a.nb) * 128 + l16 * 8;
    float f[8];
    if constexpr (IO::code == DT_F16)
    {
        if constexpr (PRE)
        {
            const TF16::Vec p = load8<TF16>(a.pre, e0);
            #pragma unroll
            for (int i = 0; i < 4; ++i) v.a[i] = hmul2(v.a[i], p.a[i]);
        }
        butterfly128_f16<false>(v, f, l16, a.r);
    }
    else
    {
        unpack8<IO>(v, f);
        if constexpr (PRE)
        {
            float p[8];
            unpack8<TF16>(load8<TF16>(a.pre, e0), p);
            #pragma unroll
            for (int j = 0; j < 8; ++j) f[j] = f[j] * p[j];
        }
        butterfly128(f, l16, a.r);
    }
    if constexpr (IO::code == DT_F16)
    {
        v = pack8<IO>(f);
        if constexpr (POST)
        {
            const TF16::Vec p = load8<TF16>(a.post, e0);
            #pragma unroll
            for (int i = 0; i < 4; ++i) v.a[i] = hmul2(v.a[i], p.a[i]);
        }
    }
    else
    {
        if constexpr (POST)
        {
            float p[8];
            unpack8<TF16>(load8<TF16>(a.post, e0), p);
            #pragma unroll
            for (int j = 0; j < 8; ++j) f[j] = f[j] * p[j];
        }
        v = pack8<IO>(f);
    }
    store8<IO>(a.out + row * a.ldo, e0, v);
}

// U consecutive blocks per 16-lane group, all loads issued first (whole groups leave together, so
// the lane exchanges never see a finished partner).
template <class IO, bool PRE, bool POST, int U>
__global__ __launch_bounds__(256) void k_had(HadArgs a)
{
    const int l16 = threadIdx.x & 15;
    const int64_t blk0 = ((int64_t)blockIdx.x * (blockDim.x >> 4) + (threadIdx.x >> 4)) * U;
    const int64_t nblk = a.rows * a.nb;
    typename IO::Vec v[U];
    #pragma unroll
    for (int u = 0; u < U; ++u)
    {
        const int64_t blk = blk0 + u;
        if (blk < nblk)
        {
            const int64_t row = blk / a.nb;
            v[u] = load8s<IO>(a.x + row * a.ldx, (blk - row * a.nb) * 128 + l16 * 8);
        }
    }
    #pragma unroll
    for (int u = 0; u < U; ++u)
        if (blk0 + u < nblk) had_block<IO, PRE, POST>(a, blk0 + u, l16, v[u]);
}

// The same transform on the matrix cores (had128_mfma, hadamard.cuh), f16 only.  A wave takes spans of
// 4 blocks of a row, lane l holding chunk mfma_chunk(l) of its span; the spans of the tensor (rows *
// spans_per_row, counted in 32 bits) are dealt to the waves in turn, UN per wave in flight.  Loop
// bounds are wave-uniform (every MFMA runs with the whole wave); lanes past a row's last block carry
// zeros and store nothing.  A span's loads all complete before its MFMAs, so out may equal x.
template <bool PRE, bool POST, int UN>
__global__ __launch_bounds__(256) void k_had_mfma(HadArgs a)
{
    const int lane = threadIdx.x & 63;
    const uint32_t cpr = (uint32_t)(a.nb * 16);
    const uint32_t spr = (uint32_t)((a.nb + 3) / 4);
    const uint32_t nspans = (uint32_t)a.rows * spr;
    const uint32_t wave = __builtin_amdgcn_readfirstlane((blockIdx.x * blockDim.x + threadIdx.x) >> 6);
    const uint32_t nwaves = (gridDim.x * blockDim.x) >> 6;
    const HadMfma H = had_mfma_operands(lane);
    const uint32_t lc = (uint32_t)mfma_chunk(lane);
    for (uint32_t s0 = wave * UN; s0 < nspans; s0 += nwaves * UN)
    {
        TF16::Vec v[UN];
        uint32_t row[UN], c[UN];
        bool live[UN];
        #pragma unroll
        for (int u = 0; u < UN; ++u)
        {
            const uint32_t sp = s0 + u;
            row[u] = sp / spr;
            c[u] = (sp - row[u] * spr) * 64 + lc;
            live[u] = sp < nspans && c[u] < cpr;
            if (live[u]) v[u] = load8s<TF16>(a.x + (int64_t)row[u] * a.ldx, (int64_t)c[u] * 8);
            else v[u].a = u32x4{ 0u, 0u, 0u, 0u };
        }
        MfmaOut m[UN];
        #pragma unroll
        for (int u = 0; u < UN; ++u)
        {
            if constexpr (PRE)
            {
                if (live[u])
                {
                    const TF16::Vec p = load8<TF16>(a.pre, (int64_t)c[u] * 8);
                    #pragma unroll
                    for (int i = 0; i < 4; ++i) v[u].a[i] = hmul2(v[u].a[i], p.a[i]);
                }
            }
            m[u] = had128_mfma_issue(H, v[u]);
        }
        mfma_wait_all(m);
        #pragma unroll
        for (int u = 0; u < UN; ++u)
        {
            float f[8];
            had128_mfma_finish(m[u], f, lane, a.r);
            TF16::Vec o = pack8<TF16>(f);
            if (live[u])
            {
                if constexpr (POST)
                {
                    const TF16::Vec p = load8<TF16>(a.post, (int64_t)c[u] * 8);
                    #pragma unroll
                    for (int i = 0; i < 4; ++i) o.a[i] = hmul2(o.a[i], p.a[i]);
                }
                store8<TF16>(a.out + (int64_t)row[u] * a.ldo, (int64_t)c[u] * 8, o);
            }
        }
    }
}

// Any alignment: a 128-lane workgroup per block, the same butterfly through LDS.
__global__ __launch_bounds__(128) void k_had_generic(HadArgs a, int dt)
{
    #pragma clang fp contract(off)
    __shared__ float s[128];
    const int k = threadIdx.x;
    for (int64_t blk = blockIdx.x; blk < a.rows * a.nb; blk += gridDim.x)
    {
        const int64_t row = blk / a.nb;
        const int64_t e = (blk - row * a.nb) * 128 + k;
        float v = load1(a.x + row * a.ldx, dt, e);
        if (a.pre)
        {
            const float p = (float)((const _Float16*)a.pre)[e];
            v = dt == DT_F16 ? round_f16(v * p) : v * p;      // f16: the exact product rounded once
        }
        s[k] = v;
        for (int h = 1; h < 128; h <<= 1)
        {
            __syncthreads();
            const float mine = s[k], other = s[k ^ h];
            __syncthreads();
            s[k] = (k & h) ? other - mine : mine + other;
        }
        __syncthreads();
        float o = s[k] * a.r;
        if (dt == DT_F16) o = round_f16(o);
        if (a.post)
        {
            const float p = (float)((const _Float16*)a.post)[e];
            o = dt == DT_F16 ? round_f16(o * p) : o * p;
        }
        store1(a.out + row * a.ldo, dt, e, o);
        __syncthreads();
    }
}

}  // namespace exl3r

using namespace exl3r;

extern "C" int exl3r_had_r_128(const void* x, int dtype, int64_t ldx, void* out, int64_t ldo, int64_t rows,
                               int64_t cols, const void* pre_scale, const void* post_scale, float scale, void* stream)
{
    begin_call();
    const char* op = "exl3r_had_r_128";
    if (dtype != EXL3R_F16 && dtype != EXL3R_F32)
        return set_error(EXL3R_EDTYPE, "%s: x / out must be f16 or f32, got %s", op, dtype_name(dtype));
    if (rows < 0 || cols < 0 || cols % 128 || (rows > 1 && (ldx < cols || ldo < cols)))
        return set_error(EXL3R_EINVAL, "%s: invalid shape rows=%lld cols=%lld (a multiple of 128) ldx=%lld ldo=%lld", op,
                         (long long)rows, (long long)cols, (long long)ldx, (long long)ldo);
    if (pre_scale && post_scale)
        return set_error(EXL3R_EINVAL, "%s: give at most one of pre_scale / post_scale", op);
    if (rows == 0 || cols == 0) return EXL3R_OK;
    if (!x || !out) return set_error(EXL3R_EINVAL, "%s: x and out must be non-null", op);
    const int es = dtype_bytes(dtype);
    HadArgs a{ (const char*)x, (char*)out, (rows > 1 ? ldx : cols) * es, (rows > 1 ? ldo : cols) * es, rows, cols / 128,
               (const uint16_t*)pre_scale, (const uint16_t*)post_scale, scale * 0.0883883461356163f };
    hipStream_t s = (hipStream_t)stream;
    const void* sc = pre_scale ? pre_scale : post_scale;
    const bool vec = aligned16(x) && aligned16(out) && a.ldx % 16 == 0 && a.ldo % 16 == 0 && (!sc || aligned16(sc));
    const int64_t blocks = rows * a.nb;
    if (vec)
    {
        const int u = tuning().had_unroll == 2 || tuning().had_unroll == 4 ? tuning().had_unroll : 1;
        const int threads = had_threads(), gpb = threads / 16 * u;   // 16-lane groups (x blocks each) per workgroup
        const int64_t grid = (blocks + gpb - 1) / gpb;
        if (grid > 0x7fffffffLL) return set_error(EXL3R_EINVAL, "%s: too many blocks", op);
        auto go = [&](auto T, auto U) {
            using IO = decltype(T);
            constexpr int UN = decltype(U)::value;
            if (pre_scale) launch(k_had<IO, true, false, UN>, (unsigned)grid, threads, 0, s, a);
            else if (post_scale) launch(k_had<IO, false, true, UN>, (unsigned)grid, threads, 0, s, a);
            else launch(k_had<IO, false, false, UN>, (unsigned)grid, threads, 0, s, a);
        };
        auto go_u = [&](auto T) {
            if (u == 4) go(T, std::integral_constant<int, 4>{});
            else if (u == 2) go(T, std::integral_constant<int, 2>{});
            else go(T, std::integral_constant<int, 1>{});
        };
        if (dtype == EXL3R_F16) go_u(TF16{});
        else go_u(TF32{});
    }
    else
        launch(k_had_generic, (unsigned)(blocks < kMaxGridX ? blocks : kMaxGridX), 128, 0, s, a, dtype);
    return launch_status(op);
}

// exl3r_had_r_128 with the transform on the matrix cores (f16; the kernel the fused Hadamard entry
// points use unless EXL3R_HAD_EXACT).  Rows that are not 16-byte aligned take exl3r_had_r_128's
// butterfly, which is within the same tolerance.
extern "C" int exl3r_had_r_128_mfma(const void* x, int dtype, int64_t ldx, void* out, int64_t ldo, int64_t rows,
                                    int64_t cols, const void* pre_scale, const void* post_scale, float scale,
                                    void* stream)
{
    begin_call();
    const char* op = "exl3r_had_r_128_mfma";
    if (dtype != EXL3R_F16) return set_error(EXL3R_EDTYPE, "%s: x / out must be f16, got %s", op, dtype_name(dtype));
    if (rows < 0 || cols < 0 || cols % 128 || (rows > 1 && (ldx < cols || ldo < cols)))
        return set_error(EXL3R_EINVAL, "%s: invalid shape rows=%lld cols=%lld (a multiple of 128) ldx=%lld ldo=%lld", op,
                         (long long)rows, (long long)cols, (long long)ldx, (long long)ldo);
    if (pre_scale && post_scale)
        return set_error(EXL3R_EINVAL, "%s: give at most one of pre_scale / post_scale", op);
    if (rows == 0 || cols == 0) return EXL3R_OK;
    if (!x || !out) return set_error(EXL3R_EINVAL, "%s: x and out must be non-null", op);
    const int64_t lx = (rows > 1 ? ldx : cols) * 2, lo = (rows > 1 ? ldo : cols) * 2;
    const void* sc = pre_scale ? pre_scale : post_scale;
    const int64_t spans = rows * ((cols / 128 + 3) / 4);
    const bool vec = aligned16(x) && aligned16(out) && lx % 16 == 0 && lo % 16 == 0 && (!sc || aligned16(sc));
    if (!vec || spans >= ((int64_t)1 << 31))
        return exl3r_had_r_128(x, dtype, ldx, out, ldo, rows, cols, pre_scale, post_scale, scale, stream);
    HadArgs a{ (const char*)x, (char*)out, lx, lo, rows, cols / 128, (const uint16_t*)pre_scale,
               (const uint16_t*)post_scale, scale * 0.0883883461356163f };
    hipStream_t s = (hipStream_t)stream;
    constexpr int UN = 2;
    // one wave per UN spans (the grid does not loop; see the act -> Hadamard kernels' launch shape)
    const int per_cu = tuning().had_mfma_per_cu;
    const int threads = had_threads(), spb = threads / 64 * UN;   // spans per workgroup
    int64_t blocks = (spans + spb - 1) / spb;
    if (per_cu > 0 && blocks > (int64_t)per_cu * device_cus()) blocks = (int64_t)per_cu * device_cus();
    if (blocks > kMaxGridX) blocks = kMaxGridX;
    if (pre_scale) launch(k_had_mfma<true, false, UN>, (unsigned)blocks, threads, 0, s, a);
    else if (post_scale) launch(k_had_mfma<false, true, UN>, (unsigned)blocks, threads, 0, s, a);
    else launch(k_had_mfma<false, false, UN>, (unsigned)blocks, threads, 0, s, a);
    return launch_status(op);
}
