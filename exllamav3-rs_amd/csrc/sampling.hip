// Row argmax for gfx950: exl3r_argmax_sample (replaces exl3_shim_argmax_sample, reference
// csrc/exl3_shim.cpp:229-231 -> argmax_sample, kernels/generator/sampling_basic.cu:65-92, 151-172, and
// the generator's batched tch argmax over [bsz, vocab] logits, src/generator.rs:1596, draft.rs:121).
//
// Rule (torch.argmax's): the first index of the row maximum among indices < max_logit, NaN counting
// as the maximum (the first NaN wins) and -0 equal to +0.
//
// Layout, fewer than 512 rows (decode): a row is cut into slices of 2048 or 8192 elements, a 256-lane
// workgroup per slice (grid (slices, rows)), so a single decode row of 152k logits still spreads over
// ~75 CUs.  512 rows and more: a workgroup per row, the index written directly.  Each lane keeps its best candidate
// as one 64-bit key -- an order-preserving image of the value in the high word, the complement of
// the index in the low word -- so "larger key" is exactly "larger value, then lower index".  The
// workgroup's maximum key (DPP butterfly, one LDS hop) goes to the row's int64 output with one
// atomicMax; a clear
// kernel before and a convert kernel after turn that slot into the index.  Capture-safe: no memset.
#include "abi.hpp"
#include "common.cuh"

namespace exl3r {

struct ArgArgs
{
    const char* x;
    int64_t ld;          // row stride, bytes
    int64_t n;           // candidates per row (masked length)
    int64_t rows;
    uint64_t* ids;
};

// Order-preserving 32-bit image of a float (larger float -> larger key); -0 maps with +0 and every
// NaN to the top key.
__device__ __forceinline__ uint32_t order_key(float v)
{
    if (v != v) return 0xffffffffu;
    const uint32_t u = __builtin_bit_cast(uint32_t, v + 0.0f);   // -0 + +0 = +0
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

__device__ __forceinline__ uint64_t cand_key(float v, int64_t idx)
{
    return ((uint64_t)order_key(v) << 32) | (uint64_t)(0xffffffffu - (uint32_t)idx);
}

__device__ __forceinline__ uint64_t max_u64(uint64_t a, uint64_t b) { return a > b ? a : b; }

template <int CTRL>
__device__ __forceinline__ uint64_t dpp_u64(uint64_t v)
{
    const int lo = __builtin_amdgcn_update_dpp(0, (int)(uint32_t)v, CTRL, 0xf, 0xf, false);
    const int hi = __builtin_amdgcn_update_dpp(0, (int)(uint32_t)(v >> 32), CTRL, 0xf, 0xf, false);
    return ((uint64_t)(uint32_t)hi << 32) | (uint32_t)lo;
}

// Maximum over the wave, valid in lane 0 (and every lane).
__device__ __forceinline__ uint64_t wave_max_u64(uint64_t v)
{
    v = max_u64(v, dpp_u64<DPP_QUAD_XOR1>(v));
    v = max_u64(v, dpp_u64<DPP_QUAD_XOR2>(v));
    v = max_u64(v, dpp_u64<DPP_ROW_HALF_MIRROR>(v));
    v = max_u64(v, dpp_u64<DPP_ROW_MIRROR>(v));
    v = max_u64(v, __shfl_xor(v, 16));
    v = max_u64(v, __shfl_xor(v, 32));
    return v;
}

__global__ __launch_bounds__(256) void k_argmax_clear(uint64_t* ids, int64_t rows)
{
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < rows) ids[i] = 0;
}

__global__ __launch_bounds__(256) void k_argmax_convert(uint64_t* ids, int64_t rows)
{
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < rows)
    {
        const uint64_t k = ids[i];
        ids[i] = k ? (uint64_t)(0xffffffffu - (uint32_t)k) : 0;
    }
}

// A workgroup of 256 lanes reduces a slice of UNROLL * 2048 elements (UNROLL chunks of 8 per lane in
// flight) to one key, so a row takes only vocab / slice atomics: same-address atomics from many
// workgroups (and XCDs) serialize.  VEC: 16-byte aligned rows, whole chunks loaded as vectors (a
// chunk crossing n is read element by element); otherwise every element is read on its own.
template <class IT, bool VEC, int UNROLL>
__global__ __launch_bounds__(256) void k_argmax(ArgArgs a)
{
    __shared__ uint64_t part[4];
    const int tid = threadIdx.x;
    const int64_t start = (int64_t)blockIdx.x * UNROLL * 2048;
    for (int64_t row = blockIdx.y; row < a.rows; row += gridDim.y)
    {
        const char* base = a.x + row * a.ld;
        uint64_t best = 0;
        typename IT::Vec v[UNROLL];
        #pragma unroll
        for (int u = 0; u < UNROLL; ++u)
        {
            const int64_t c = start + u * 2048 + tid * 8;
            if (VEC && c + 8 <= a.n) v[u] = load8s<IT>(base, c);
        }
        #pragma unroll
        for (int u = 0; u < UNROLL; ++u)
        {
            const int64_t c = start + u * 2048 + tid * 8;
            if (VEC && c + 8 <= a.n)
            {
                float f[8];
                unpack8<IT>(v[u], f);
                #pragma unroll
                for (int j = 0; j < 8; ++j) best = max_u64(best, cand_key(f[j], c + j));
            }
            else
            {
                for (int j = 0; j < 8 && c + j < a.n; ++j)
                    best = max_u64(best, cand_key(load1(base, IT::code, c + j), c + j));
            }
        }
        best = wave_max_u64(best);
        if ((tid & 63) == 0) part[tid >> 6] = best;
        __syncthreads();
        if (tid == 0)
        {
            best = max_u64(max_u64(part[0], part[1]), max_u64(part[2], part[3]));
            if (best) atomicMax((unsigned long long*)(a.ids + row), (unsigned long long)best);
        }
        __syncthreads();
    }
}

// Many rows: a workgroup owns a row, walks it 2048 elements per step with 4 chunks per lane in
// flight, and writes the index itself (no atomics, no clear / convert launches).
template <class IT, bool VEC>
__global__ __launch_bounds__(256) void k_argmax_rows(ArgArgs a)
{
    __shared__ uint64_t part[4];
    const int tid = threadIdx.x;
    for (int64_t row = blockIdx.x; row < a.rows; row += gridDim.x)
    {
        const char* base = a.x + row * a.ld;
        uint64_t best = 0;
        for (int64_t s0 = 0; s0 < a.n; s0 += 4 * 2048)
        {
            typename IT::Vec v[4];
            #pragma unroll
            for (int u = 0; u < 4; ++u)
            {
                const int64_t c = s0 + u * 2048 + tid * 8;
                if (VEC && c + 8 <= a.n) v[u] = load8s<IT>(base, c);
            }
            #pragma unroll
            for (int u = 0; u < 4; ++u)
            {
                const int64_t c = s0 + u * 2048 + tid * 8;
                if (VEC && c + 8 <= a.n)
                {
                    float f[8];
                    unpack8<IT>(v[u], f);
                    #pragma unroll
                    for (int j = 0; j < 8; ++j) best = max_u64(best, cand_key(f[j], c + j));
                }
                else
                {
                    for (int j = 0; j < 8 && c + j < a.n; ++j)
                        best = max_u64(best, cand_key(load1(base, IT::code, c + j), c + j));
                }
            }
        }
        best = wave_max_u64(best);
        if ((tid & 63) == 0) part[tid >> 6] = best;
        __syncthreads();
        if (tid == 0)
        {
            best = max_u64(max_u64(part[0], part[1]), max_u64(part[2], part[3]));
            a.ids[row] = best ? (uint64_t)(0xffffffffu - (uint32_t)best) : 0;
        }
        __syncthreads();
    }
}

}  // namespace exl3r

using namespace exl3r;

extern "C" int exl3r_argmax_sample(const void* logits, int dtype, int64_t rows, int64_t vocab, int64_t ld,
                                   int max_logit, int64_t* ids, void* stream)
{
    const char* op = "exl3r_argmax_sample";
    if (!is_float_dtype(dtype)) return set_error(EXL3R_EDTYPE, "%s: unsupported logits dtype %s", op, dtype_name(dtype));
    if (rows < 0 || vocab <= 0 || vocab > 0xffffffffLL || (rows > 1 && ld < vocab))
        return set_error(EXL3R_EINVAL, "%s: invalid shape rows=%lld vocab=%lld ld=%lld", op, (long long)rows,
                         (long long)vocab, (long long)ld);
    if (rows == 0) return EXL3R_OK;
    if (!logits || !ids) return set_error(EXL3R_EINVAL, "%s: logits and ids must be non-null", op);
    const int64_t n = (max_logit <= 0 || max_logit > vocab) ? vocab : max_logit;
    const int es = dtype_bytes(dtype);
    ArgArgs a{ (const char*)logits, (rows > 1 ? ld : vocab) * es, n, rows, (uint64_t*)ids };
    hipStream_t s = (hipStream_t)stream;
    const bool vec = aligned16(logits) && a.ld % 16 == 0;
    if (rows >= 512)
    {
        const unsigned grid = (unsigned)(rows < kMaxGridX ? rows : kMaxGridX);
        with_float_type(dtype, [&](auto T) {
            if (vec) k_argmax_rows<decltype(T), true><<<grid, 256, 0, s>>>(a);
            else k_argmax_rows<decltype(T), false><<<grid, 256, 0, s>>>(a);
        });
        return launch_status(op);
    }
    const unsigned small = (unsigned)((rows + 255) / 256);
    k_argmax_clear<<<small, 256, 0, s>>>(a.ids, rows);
    // Slices of 8192 elements (19 per 152k-token row); decode batches of a few rows take 2048-element
    // slices so the row still spreads over enough CUs.
    const int unroll = rows >= 16 ? 4 : 1;
    const int64_t slice = (int64_t)unroll * 2048;
    const dim3 grid((unsigned)((n + slice - 1) / slice), (unsigned)rows);
    with_float_type(dtype, [&](auto T) {
        using Ty = decltype(T);
        if (unroll == 4)
        {
            if (vec) k_argmax<Ty, true, 4><<<grid, 256, 0, s>>>(a);
            else k_argmax<Ty, false, 4><<<grid, 256, 0, s>>>(a);
        }
        else
        {
            if (vec) k_argmax<Ty, true, 1><<<grid, 256, 0, s>>>(a);
            else k_argmax<Ty, false, 1><<<grid, 256, 0, s>>>(a);
        }
    });
    k_argmax_convert<<<small, 256, 0, s>>>(a.ids, rows);
    return launch_status(op);
}
