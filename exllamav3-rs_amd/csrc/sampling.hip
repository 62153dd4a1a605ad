// Row sampling for gfx950.
//
// exl3r_argmax_sample replaces exl3_shim_argmax_sample (reference csrc/exl3_shim.cpp:229-231 ->
// argmax_sample, kernels/generator/sampling_basic.cu:65-92, 151-172) and the generator's batched tch
// argmax over [bsz, vocab] logits (src/generator.rs:1596, draft.rs:121).  Rule (torch.argmax's): the
// first index of the row maximum among indices < max_logit, NaN counting as the maximum (the first
// NaN wins) and -0 equal to +0.
//
// exl3r_gumbel_sample / exl3r_gumbel_noise take the role of exl3_shim_gumbel_sample and
// exl3_shim_gumbel_noise_f32 (exl3_shim.cpp:232-237; sampling_basic.cu:94-128, gumbel.cu:45-62): a
// Gumbel-max draw, the argmax of logits + Gumbel(0, 1) noise, which picks index i with probability
// softmax(logits)_i.  The noise stream is this library's own, a function of (seed, row, column) only:
//   bits = Philox4x32-10(counter {column >> 2, row low, row high, 0}, key {seed, 0}), word column & 3
//   u    = ((bits >> 9) + 0.5) * 2^-23          exact, in [2^-24, 1 - 2^-24]
//   g    = -log(-log(u))                         log_f32 below, correctly ordered fp32 operations
// Philox4x32-10 is the published generator of Salmon, Moraes, Dror and Shaw ("Parallel random
// numbers: as easy as 1, 2, 3", SC 2011).
//
// Layout, few rows (decode): a row is cut into slices of 2048 or 8192 elements, a 256-lane
// workgroup per slice (grid (slices, rows)), so a single decode row of 152k logits still spreads over
// ~75 CUs.  From 128 rows (argmax) or 384 rows (Gumbel draw): a workgroup of 512 or 1024 lanes per
// row, the index written directly.  Each lane keeps its
// best candidate as one 64-bit key -- an order-preserving image of the value in the high word, the
// complement of the index in the low word -- so "larger key" is exactly "larger value, then lower
// index".  With slices, the workgroup's maximum key (DPP butterfly, one LDS hop) goes to the row's
// int64 output with one atomicMax; a clear kernel before and a convert kernel after turn that slot
// into the index.  Capture-safe: no memset.
#include <mutex>

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
    uint32_t seed;       // Gumbel noise key
};

// Philox4x32-10: ten rounds of two 32 x 32 -> 64-bit products with the published multipliers,
// the key advanced by the published Weyl increments between rounds.
__device__ __forceinline__ void philox4x32_10(uint32_t c0, uint32_t c1, uint32_t c2, uint32_t c3, uint32_t k0,
                                              uint32_t k1, uint32_t (&out)[4])
{
    #pragma unroll
    for (int round = 0; round < 10; ++round)
    {
        const uint64_t p0 = (uint64_t)0xD2511F53u * c0, p1 = (uint64_t)0xCD9E8D57u * c2;
        // three-way xor in one gfx950 bitop3 (truth table 0x96 = a ^ b ^ c)
        const uint32_t n0 = __builtin_amdgcn_bitop3_b32((uint32_t)(p1 >> 32), c1, k0, 0x96);
        const uint32_t n2 = __builtin_amdgcn_bitop3_b32((uint32_t)(p0 >> 32), c3, k1, 0x96);
        c1 = (uint32_t)p1;
        c3 = (uint32_t)p0;
        c0 = n0;
        c2 = n2;
        k0 += 0x9E3779B9u;
        k1 += 0xBB67AE85u;
    }
    out[0] = c0; out[1] = c1; out[2] = c2; out[3] = c3;
}

// Natural log of a positive normal float in plain fp32 operations and explicit fmas, so that any
// IEEE implementation of the same steps gives the same bits.  x = 2^e m, m in [sqrt(1/2), sqrt(2))
// (0x3f3504f3 is sqrt(1/2)); f = m - 1 exactly; log(1 + f) = 2 atanh(s), s = f / (2 + f), arranged as
// f - (f^2/2 - s (f^2/2 + R)) with R = sum_k 2 s^2k / (2k + 1) through k = 5.  s enters only the
// correction term, so 1/(2 + f) comes from the linear minimax seed on [2 - 0.2929, 2 + 0.4143]
// (relative error 1.49e-2) and two Newton steps (5.0e-8) instead of an IEEE divide.  e ln2 is split
// so that e * ln2_hi is exact (15-bit ln2_hi, |e| < 2^9); ln2_lo is the float nearest ln2 - ln2_hi.
// Error: under 0.72 ulp on a sweep of normal floats.
__device__ __forceinline__ float log_f32(float x)
{
    #pragma clang fp contract(off)
    const uint32_t ix = __builtin_bit_cast(uint32_t, x);
    const int32_t e = ((int32_t)(ix - 0x3f3504f3u)) >> 23;
    const float m = __builtin_bit_cast(float, ix - ((uint32_t)e << 23));
    const float f = m - 1.0f;
    const float d = 2.0f + f;
    float y = __builtin_fmaf(d, -0x1.e9813ap-3f, 0x1.f859fcp-1f);
    y = __builtin_fmaf(y, __builtin_fmaf(-d, y, 1.0f), y);
    y = __builtin_fmaf(y, __builtin_fmaf(-d, y, 1.0f), y);
    const float s = f * y;
    const float z = s * s;
    const float R = z * __builtin_fmaf(z, __builtin_fmaf(z, __builtin_fmaf(z, __builtin_fmaf(z, 0x1.745d18p-3f,
                    0x1.c71c72p-3f), 0x1.24924ap-2f), 0x1.99999ap-2f), 0x1.555556p-1f);
    const float hfsq = 0.5f * f * f;
    const float ef = (float)e;
    return __builtin_fmaf(ef, 0x1.62e4p-1f, -((hfsq - __builtin_fmaf(s, hfsq + R, ef * 0x1.7f7d1cp-20f)) - f));
}

__device__ __forceinline__ float gumbel_of_bits(uint32_t b)
{
    #pragma clang fp contract(off)
    const float u = ((float)(b >> 9) + 0.5f) * 1.1920928955078125e-07f;    // 2^-23
    return -log_f32(-log_f32(u));
}

// Noise for columns c .. c+7 of `row`, c a multiple of 4.
__device__ __forceinline__ void gumbel8(uint32_t seed, int64_t row, int64_t c, float (&g)[8])
{
    uint32_t w[4];
    #pragma unroll
    for (int h = 0; h < 2; ++h)
    {
        philox4x32_10((uint32_t)(c >> 2) + h, (uint32_t)row, (uint32_t)((uint64_t)row >> 32), 0u, seed, 0u, w);
        #pragma unroll
        for (int j = 0; j < 4; ++j) g[4 * h + j] = gumbel_of_bits(w[j]);
    }
}

__device__ __forceinline__ float gumbel1(uint32_t seed, int64_t row, int64_t c)
{
    uint32_t w[4];
    philox4x32_10((uint32_t)(c >> 2), (uint32_t)row, (uint32_t)((uint64_t)row >> 32), 0u, seed, 0u, w);
    const int j = (int)(c & 3);
    return gumbel_of_bits(j == 0 ? w[0] : j == 1 ? w[1] : j == 2 ? w[2] : w[3]);
}

// Candidate value: the logit, plus its noise for a Gumbel draw.
template <bool GUMBEL>
__device__ __forceinline__ void candidates8(float (&f)[8], const ArgArgs& a, int64_t row, int64_t c)
{
    #pragma clang fp contract(off)
    if constexpr (GUMBEL)
    {
        float g[8];
        gumbel8(a.seed, row, c, g);
        #pragma unroll
        for (int j = 0; j < 8; ++j) f[j] = f[j] + g[j];
    }
}

template <bool GUMBEL>
__device__ __forceinline__ float candidate1(const char* base, int dt, const ArgArgs& a, int64_t row, int64_t c)
{
    #pragma clang fp contract(off)
    const float x = load1(base, dt, c);
    if constexpr (GUMBEL) return x + gumbel1(a.seed, row, c);
    else return x;
}

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

// A lane's running best over candidates seen in increasing index order: a candidate replaces the
// best when none is held yet, when it is larger, or when it is the first NaN (a NaN best is final);
// ties keep the earlier index.  Float compares per element; the 64-bit key is formed once.
struct LaneBest
{
    float v = 0.0f;
    uint32_t i = 0;
    bool has = false;

    __device__ __forceinline__ void consider(float x, int64_t idx)
    {
        const bool take = (!has) | (x > v) | ((x != x) & (v == v));    // no short circuit: selects, no branches
        v = take ? x : v;
        i = take ? (uint32_t)idx : i;
        has = true;
    }
    __device__ __forceinline__ uint64_t key() const { return has ? cand_key(v, i) : 0; }
};

// f16 logits without noise: a lane keeps its best chunk of 8 instead of its best element.  The chunk's
// maximum cm comes from NaN-propagating packed maxima (v_pk_maximum3_f16: a NaN anywhere in the chunk
// makes cm NaN); the chunk replaces the held one when it is the lane's first chunk, when cm is larger
// (-0 and +0 compare equal, so the earlier chunk stays), or when cm is the first NaN (a NaN best is
// final).  The held chunk's data is kept and its element found once at the end: the first one equal
// to the maximum, or the first NaN when the maximum is NaN, which is the element LaneBest keeps over
// the same elements in the same order.  Per 8 elements: 3 maxima, 3 compares and 6 selects instead of
// 8 x LaneBest::consider.
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));

struct LaneBestF16
{
    _Float16 m = 0;
    uint32_t c = 0;     // first element of the held chunk
    u32x4 d = {};       // its data
    bool has = false;

    // FIRST: the lane's first chunk (taken unconditionally).
    template <bool FIRST>
    __device__ __forceinline__ void consider8(const u32x4& w, uint32_t c0)
    {
        // (uint32_t) casts: the operand of a bit_cast must be a value, not a vector element -- this
        // compiler lowers __builtin_bit_cast of an ext_vector element lvalue as a read of element 0.
        const f16x2 p = __builtin_elementwise_maximum(
            __builtin_elementwise_maximum(__builtin_bit_cast(f16x2, (uint32_t)w[0]), __builtin_bit_cast(f16x2, (uint32_t)w[1])),
            __builtin_elementwise_maximum(__builtin_bit_cast(f16x2, (uint32_t)w[2]), __builtin_bit_cast(f16x2, (uint32_t)w[3])));
        const _Float16 cm = __builtin_elementwise_maximum(p[0], p[1]);
        const bool take = FIRST || (cm > m) || ((cm != cm) & (m == m));
        m = take ? cm : m;
        c = take ? c0 : c;
        #pragma unroll
        for (int q = 0; q < 4; ++q) d[q] = take ? w[q] : d[q];
        has = FIRST || has;
    }

    __device__ __forceinline__ LaneBest lane_best() const
    {
        LaneBest lb;
        int j = 7;
        #pragma unroll
        for (int q = 7; q >= 0; --q)
        {
            const _Float16 x = __builtin_bit_cast(f16x2, (uint32_t)d[q >> 1])[q & 1];
            j = ((x == m) | ((x != x) & (m != m))) ? q : j;
        }
        lb.v = (float)m;
        lb.i = c + (uint32_t)j;
        lb.has = has;
        return lb;
    }
};

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

// One lane's best candidate over its UNROLL chunks of the slice starting at `start` of `row`.  VEC:
// 16-byte aligned rows, whole chunks loaded as vectors (a chunk crossing n is read element by
// element); otherwise every element is read on its own.
template <class IT, bool VEC, int UNROLL, bool GUMBEL>
__device__ __forceinline__ uint64_t slice_lane_key(const ArgArgs& a, int64_t row, int64_t start, int tid)
{
    const char* base = a.x + row * a.ld;
    LaneBest lb;
    typename IT::Vec v[UNROLL];
    #pragma unroll
    for (int u = 0; u < UNROLL; ++u)
    {
        const int64_t c = start + u * 2048 + tid * 8;
        if (VEC && c + 8 <= a.n) v[u] = load8s<IT>(base, c);
    }
    if constexpr (VEC && IT::code == DT_F16 && !GUMBEL)
    {
        // whole chunks by LaneBestF16 (a chunk is whole only when every earlier one of the lane is)
        LaneBestF16 hb;
        #pragma unroll
        for (int u = 0; u < UNROLL; ++u)
        {
            const int64_t c = start + u * 2048 + tid * 8;
            if (c + 8 <= a.n)
            {
                if (u == 0) hb.consider8<true>(v[u].a, (uint32_t)c);
                else hb.consider8<false>(v[u].a, (uint32_t)c);
            }
        }
        lb = hb.lane_best();
    }
    #pragma unroll
    for (int u = 0; u < UNROLL; ++u)
    {
        const int64_t c = start + u * 2048 + tid * 8;
        if (VEC && c + 8 <= a.n)
        {
            if constexpr (IT::code == DT_F16 && !GUMBEL) continue;   // taken above
            float f[8];
            unpack8<IT>(v[u], f);
            candidates8<GUMBEL>(f, a, row, c);
            #pragma unroll
            for (int j = 0; j < 8; ++j) lb.consider(f[j], c + j);
        }
        else
        {
            for (int j = 0; j < 8 && c + j < a.n; ++j)
                lb.consider(candidate1<GUMBEL>(base, IT::code, a, row, c + j), c + j);
        }
    }
    return lb.key();
}

// A workgroup of 256 lanes reduces a slice of UNROLL * 2048 elements (UNROLL chunks of 8 per lane in
// flight) to one key, so a row takes only vocab / slice atomics: same-address atomics from many
// workgroups (and XCDs) serialize.
template <class IT, bool VEC, int UNROLL, bool GUMBEL>
__global__ __launch_bounds__(256) void k_argmax(ArgArgs a)
{
    __shared__ uint64_t part[4];
    const int tid = threadIdx.x;
    const int64_t start = (int64_t)blockIdx.x * UNROLL * 2048;
    for (int64_t row = blockIdx.y; row < a.rows; row += gridDim.y)
    {
        uint64_t best = wave_max_u64(slice_lane_key<IT, VEC, UNROLL, GUMBEL>(a, row, start, tid));
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

// The same slices in one launch with a workspace (exl3r_argmax_sample_ws, exl3r_gumbel_sample_ws):
// each workgroup folds its slice's key into the row's slot with atomicMax and then counts itself in
// count[row]; the workgroup whose count completes the row takes the slot with an atomic exchange
// (which also resets it to 0), writes the index and resets the count, so the workspace is zero again
// when the launch ends and nothing is cleared per call.  Ordering comes from completion, not fences:
// a workgroup issues its count only after its atomicMax has returned, so every slot update is
// performed before the last count, and the exchange after that (atomics on one address are
// serialized where they are performed, across XCDs too).  (Release / acquire
// fences at device scope write back and invalidate the L2 for every workgroup: 28.8 against 10.2 us
// for the three launches at 64 x 151936.)  No workgroup waits for another.
template <class IT, bool VEC, int UNROLL, bool GUMBEL>
__global__ __launch_bounds__(256) void k_argmax_ws(ArgArgs a, uint32_t* count, uint64_t* slot)
{
    __shared__ uint64_t wpart[4];
    const int tid = threadIdx.x;
    const uint32_t slices = gridDim.x;
    const int64_t start = (int64_t)blockIdx.x * UNROLL * 2048;
    for (int64_t row = blockIdx.y; row < a.rows; row += gridDim.y)
    {
        uint64_t best = wave_max_u64(slice_lane_key<IT, VEC, UNROLL, GUMBEL>(a, row, start, tid));
        if ((tid & 63) == 0) wpart[tid >> 6] = best;
        __syncthreads();
        if (tid == 0)
        {
            best = max_u64(max_u64(wpart[0], wpart[1]), max_u64(wpart[2], wpart[3]));
            // The returning form, its value consumed: the count below is issued only once the slot's
            // update has been performed and answered.
            const unsigned long long prev = atomicMax((unsigned long long*)(slot + row), (unsigned long long)best);
            asm volatile("" : : "v"(prev) : "memory");
            if (atomicAdd(count + row, 1u) + 1 == slices)
            {
                const uint64_t k = atomicExch((unsigned long long*)(slot + row), 0ull);
                a.ids[row] = k ? (uint64_t)(0xffffffffu - (uint32_t)k) : 0;
                atomicExch(count + row, 0u);
            }
        }
        __syncthreads();
    }
}

// Many rows: a workgroup of THREADS lanes owns a row, walks it THREADS * 8 elements per chunk round
// with 4 chunks per lane in flight, and writes the index itself (no atomics, no clear / convert
// launches).
template <class IT, bool VEC, bool GUMBEL, int THREADS>
__global__ __launch_bounds__(THREADS) void k_argmax_rows(ArgArgs a)
{
    constexpr int WAVES = THREADS / 64;
    constexpr int STEP = THREADS * 8;          // elements per chunk round
    __shared__ uint64_t part[WAVES];
    const int tid = threadIdx.x;
    for (int64_t row = blockIdx.x; row < a.rows; row += gridDim.x)
    {
        const char* base = a.x + row * a.ld;
        LaneBest lb;
        if constexpr (VEC && IT::code == DT_F16 && !GUMBEL)
        {
            // whole chunks by LaneBestF16, then the elements of a partial last chunk (after every whole
            // one) by the lane that holds it
            const int64_t nw = a.n & ~(int64_t)7;
            LaneBestF16 hb;
            auto round = [&](int64_t s0, auto FIRST) __attribute__((always_inline)) {
                u32x4 v[4];
                #pragma unroll
                for (int u = 0; u < 4; ++u)
                {
                    const int64_t c = s0 + u * STEP + tid * 8;
                    if (c < nw) v[u] = load8s<TF16>(base, c).a;
                }
                #pragma unroll
                for (int u = 0; u < 4; ++u)
                {
                    const int64_t c = s0 + u * STEP + tid * 8;
                    if (c < nw)
                    {
                        if (decltype(FIRST)::value && u == 0) hb.consider8<true>(v[u], (uint32_t)c);
                        else hb.consider8<false>(v[u], (uint32_t)c);
                    }
                }
            };
            if (nw > 0) round((int64_t)0, std::true_type{});
            for (int64_t s0 = 4 * STEP; s0 < nw; s0 += 4 * STEP) round(s0, std::false_type{});
            lb = hb.lane_best();
            if (nw < a.n && tid * 8 == nw % STEP)
                for (int64_t c = nw; c < a.n; ++c) lb.consider(load1(base, DT_F16, c), c);
        }
        else for (int64_t s0 = 0; s0 < a.n; s0 += 4 * STEP)
        {
            typename IT::Vec v[4];
            #pragma unroll
            for (int u = 0; u < 4; ++u)
            {
                const int64_t c = s0 + u * STEP + tid * 8;
                if (VEC && c + 8 <= a.n) v[u] = load8s<IT>(base, c);
            }
            #pragma unroll
            for (int u = 0; u < 4; ++u)
            {
                const int64_t c = s0 + u * STEP + tid * 8;
                if (VEC && c + 8 <= a.n)
                {
                    float f[8];
                    unpack8<IT>(v[u], f);
                    candidates8<GUMBEL>(f, a, row, c);
                    #pragma unroll
                    for (int j = 0; j < 8; ++j) lb.consider(f[j], c + j);
                }
                else
                {
                    for (int j = 0; j < 8 && c + j < a.n; ++j)
                        lb.consider(candidate1<GUMBEL>(base, IT::code, a, row, c + j), c + j);
                }
            }
        }
        uint64_t best = wave_max_u64(lb.key());
        if ((tid & 63) == 0) part[tid >> 6] = best;
        __syncthreads();
        if (tid == 0)
        {
            best = part[0];
            #pragma unroll
            for (int w = 1; w < WAVES; ++w) best = max_u64(best, part[w]);
            a.ids[row] = best ? (uint64_t)(0xffffffffu - (uint32_t)best) : 0;
        }
        __syncthreads();
    }
}

// out[r, c] = x[r, c] + g(seed, r, c): a lane per 8 columns (grid (column chunks, rows)).  VEC: 16-byte
// aligned rows of x and out; otherwise element by element.
struct NoiseArgs
{
    const char* x;
    char* out;
    int64_t ldx, ldo;    // bytes
    int64_t rows, cols;
    uint32_t seed;
};

template <class IT, class OT, bool VEC>
__global__ __launch_bounds__(256) void k_gumbel_noise(NoiseArgs a)
{
    #pragma clang fp contract(off)
    const int64_t c = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 8;
    if (c >= a.cols) return;
    for (int64_t row = blockIdx.y; row < a.rows; row += gridDim.y)
    {
        const char* xr = a.x + row * a.ldx;
        char* orow = a.out + row * a.ldo;
        if (VEC && c + 8 <= a.cols)
        {
            float f[8], g[8];
            unpack8<IT>(load8s<IT>(xr, c), f);
            gumbel8(a.seed, row, c, g);
            #pragma unroll
            for (int j = 0; j < 8; ++j) f[j] = f[j] + g[j];
            store8<OT>(orow, c, pack8<OT>(f));
        }
        else
        {
            for (int64_t j = c; j < c + 8 && j < a.cols; ++j)
                store1(orow, OT::code, j, load1(xr, IT::code, j) + gumbel1(a.seed, row, j));
        }
    }
}

}  // namespace exl3r

using namespace exl3r;

// exl3r_argmax_sample_noalloc's scratch: the one-launch kernel's row counters and slots for 384 rows
// (4608 bytes: the workspace of exl3r_argmax_sample_ws), one copy per GPU the library runs on, held
// until the process ends.  It is zero when the code object is loaded, and every completed call leaves
// it zero (the last workgroup of a row resets the row's counter and slot), so no call clears it.  Host
// code never uses the name as an address: scratch_of_current_device() asks the runtime for the
// current device's copy, once per device.
static __device__ __align__(256) unsigned char scratch[384 * 12];

namespace {

// Workspace of the single-launch sliced path: kWsMaxRows row counters (u32), then as many row slots
// (u64), all zero between calls.
constexpr int64_t kWsMaxRows = 384;
constexpr size_t kCountBytes = kWsMaxRows * 4;
constexpr size_t kWsBytes = kCountBytes + kWsMaxRows * 8;

// Elements per slice of the sliced kernels: 8192 (19 slices per 152k-token row); decode batches of a
// few rows take 2048-element slices so the row still spreads over enough CUs.
inline int slice_unroll(int64_t rows) { return rows >= 16 ? 4 : 1; }

struct Workspace
{
    void* base;      // nullptr: the three-launch path (ids as the reduction slot)
    size_t bytes;
    bool scratch;    // the library's scratch (looked up when the sliced kernel needs it); a call it cannot
                     // serve is an error, not the three-launch path
};

static_assert(sizeof(scratch) == kWsBytes, "the scratch is one workspace");

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// The current device's scratch address: hipGetSymbolAddress on the first call with that device
// current, kept per device.
int scratch_of_current_device(const char* op, void** out)
{
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return set_error((int)e, "%s: hipGetDevice: %s", op, hipGetErrorString(e));
    if (dev < 0 || dev >= kMaxDevices)
        return set_error(EXL3R_EINVAL, "%s: device %d is beyond the %d devices this entry point serves", op, dev,
                         kMaxDevices);
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[dev])
    {
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p)
            return set_error(e != hipSuccess ? (int)e : (int)hipErrorInvalidSymbol, "%s: hipGetSymbolAddress(scratch): %s",
                             op, hipGetErrorString(e != hipSuccess ? e : hipErrorInvalidSymbol));
        g_scratch_ptr[dev] = p;
    }
    *out = g_scratch_ptr[dev];
    return EXL3R_OK;
}

// Shared by the argmax and the Gumbel draw: validation, then the slice or row-per-workgroup kernels.
template <bool GUMBEL>
int sample_entry(const char* op, const void* logits, int dtype, int64_t rows, int64_t vocab, int64_t ld,
                 int max_logit, uint32_t seed, int64_t* ids, void* stream, Workspace ws = { nullptr, 0, false })
{

    if (!is_float_dtype(dtype)) return set_error(EXL3R_EDTYPE, "%s: unsupported logits dtype %s", op, dtype_name(dtype));
    if (rows < 0 || vocab <= 0 || vocab > 0xffffffffLL || (rows > 1 && ld < vocab))
        return set_error(EXL3R_EINVAL, "%s: invalid shape rows=%lld vocab=%lld ld=%lld", op, (long long)rows,
                         (long long)vocab, (long long)ld);
    if (rows == 0) return EXL3R_OK;
    if (!logits || !ids) return set_error(EXL3R_EINVAL, "%s: logits and ids must be non-null", op);
    const int64_t n = (max_logit <= 0 || max_logit > vocab) ? vocab : max_logit;
    const int es = dtype_bytes(dtype);
    ArgArgs a{ (const char*)logits, (rows > 1 ? ld : vocab) * es, n, rows, (uint64_t*)ids, seed };
    hipStream_t s = (hipStream_t)stream;
    const bool vec = aligned16(logits) && a.ld % 16 == 0;
    // Measured on MI355X over f16 [rows, 151936] logits (us; sliced / a workgroup per row with 512 /
    // 1024 lanes): argmax 64 rows 11.2 / 25.0 / 16.4, 128 rows 16.8 / 25.7 / 17.0, 192 rows 21.8 /
    // 26.3 / 17.4, 512 rows - / 32.0 / 33.5 (256 lanes 57.0), 1024 rows - / 62.3 / 64.5; the Gumbel
    // draw, compute-bound, keeps the sliced kernel longer: 256 rows 58.9 / 74.6 / 64.3, 512 rows
    // 147.6 (256 lanes) / 125.9 / 125.6, 1024 rows - / 225.3 / 246.3.
    const Tuning& tu = tuning();
    const int64_t rows_min = tu.sample_rows_min > 0 ? tu.sample_rows_min : GUMBEL ? 384 : 128;
    if (rows >= rows_min)
    {
        const unsigned grid = (unsigned)(rows < kMaxGridX ? rows : kMaxGridX);
        int threads = GUMBEL || rows >= 512 ? 512 : 1024;
        if (tu.sample_threads == 256 || tu.sample_threads == 512 || tu.sample_threads == 1024) threads = tu.sample_threads;
        with_float_type(dtype, [&](auto T) {
            using Ty = decltype(T);
            if (threads == 1024)
            {
                if (vec) launch(k_argmax_rows<Ty, true, GUMBEL, 1024>, grid, 1024, 0, s, a);
                else launch(k_argmax_rows<Ty, false, GUMBEL, 1024>, grid, 1024, 0, s, a);
            }
            else if (threads == 512)
            {
                if (vec) launch(k_argmax_rows<Ty, true, GUMBEL, 512>, grid, 512, 0, s, a);
                else launch(k_argmax_rows<Ty, false, GUMBEL, 512>, grid, 512, 0, s, a);
            }
            else
            {
                if (vec) launch(k_argmax_rows<Ty, true, GUMBEL, 256>, grid, 256, 0, s, a);
                else launch(k_argmax_rows<Ty, false, GUMBEL, 256>, grid, 256, 0, s, a);
            }
        });
        return launch_status(op);
    }
    const int unroll = slice_unroll(rows);
    const int64_t slice = (int64_t)unroll * 2048;
    const dim3 grid((unsigned)((n + slice - 1) / slice), (unsigned)rows);
    if (ws.scratch)
    {
        if (rows > kWsMaxRows)
            return set_error(EXL3R_EINVAL, "%s: %lld rows take the sliced kernel, whose scratch holds %lld rows", op,
                             (long long)rows, (long long)kWsMaxRows);
        const int rc = scratch_of_current_device(op, &ws.base);
        if (rc) return rc;
    }
    if (ws.base && rows <= kWsMaxRows)
    {
        // One launch: the slice keys and row counters in the workspace.
        if (((uintptr_t)ws.base & 255) || ws.bytes < kWsBytes)
            return set_error(EXL3R_EINVAL, "%s: the workspace must be 256-byte aligned and hold %zu bytes (%zu given)",
                             op, kWsBytes, ws.bytes);
        uint32_t* count = (uint32_t*)ws.base;
        uint64_t* part = (uint64_t*)((char*)ws.base + kCountBytes);
        with_float_type(dtype, [&](auto T) {
            using Ty = decltype(T);
            if (unroll == 4)
            {
                if (vec) launch(k_argmax_ws<Ty, true, 4, GUMBEL>, grid, 256, 0, s, a, count, part);
                else launch(k_argmax_ws<Ty, false, 4, GUMBEL>, grid, 256, 0, s, a, count, part);
            }
            else
            {
                if (vec) launch(k_argmax_ws<Ty, true, 1, GUMBEL>, grid, 256, 0, s, a, count, part);
                else launch(k_argmax_ws<Ty, false, 1, GUMBEL>, grid, 256, 0, s, a, count, part);
            }
        });
        return launch_status(op);
    }
    const unsigned small = (unsigned)((rows + 255) / 256);
    launch(k_argmax_clear, small, 256, 0, s, a.ids, rows);
    with_float_type(dtype, [&](auto T) {
        using Ty = decltype(T);
        if (unroll == 4)
        {
            if (vec) launch(k_argmax<Ty, true, 4, GUMBEL>, grid, 256, 0, s, a);
            else launch(k_argmax<Ty, false, 4, GUMBEL>, grid, 256, 0, s, a);
        }
        else
        {
            if (vec) launch(k_argmax<Ty, true, 1, GUMBEL>, grid, 256, 0, s, a);
            else launch(k_argmax<Ty, false, 1, GUMBEL>, grid, 256, 0, s, a);
        }
    });
    launch(k_argmax_convert, small, 256, 0, s, a.ids, rows);
    return launch_status(op);
}

}  // namespace

extern "C" int exl3r_argmax_sample_noalloc(const void* logits, int dtype, int64_t rows, int64_t vocab, int64_t ld,
                                           int max_logit, int64_t* ids, void* stream)
{
    begin_call();
    const char* op = "exl3r_argmax_sample_noalloc";
    return sample_entry<false>(op, logits, dtype, rows, vocab, ld, max_logit, 0u, ids, stream, { nullptr, kWsBytes, true });
}

extern "C" int exl3r_argmax_sample(const void* logits, int dtype, int64_t rows, int64_t vocab, int64_t ld,
                                   int max_logit, int64_t* ids, void* stream)
{
    begin_call();
    return sample_entry<false>("exl3r_argmax_sample", logits, dtype, rows, vocab, ld, max_logit, 0u, ids, stream);
}

extern "C" size_t exl3r_sample_workspace_bytes(void) { return kWsBytes; }

extern "C" int exl3r_argmax_sample_ws(const void* logits, int dtype, int64_t rows, int64_t vocab, int64_t ld,
                                      int max_logit, int64_t* ids, void* workspace, size_t workspace_bytes,
                                      void* stream)
{
    begin_call();
    if (!workspace) return set_error(EXL3R_EINVAL, "exl3r_argmax_sample_ws: workspace must be non-null");
    return sample_entry<false>("exl3r_argmax_sample_ws", logits, dtype, rows, vocab, ld, max_logit, 0u, ids, stream,
                               { workspace, workspace_bytes, false });
}

extern "C" int exl3r_gumbel_sample_ws(const void* logits, int dtype, int64_t rows, int64_t vocab, int64_t ld,
                                      int max_logit, uint32_t random, int64_t* ids, void* workspace,
                                      size_t workspace_bytes, void* stream)
{
    begin_call();
    if (!workspace) return set_error(EXL3R_EINVAL, "exl3r_gumbel_sample_ws: workspace must be non-null");
    return sample_entry<true>("exl3r_gumbel_sample_ws", logits, dtype, rows, vocab, ld, max_logit, random, ids,
                              stream, { workspace, workspace_bytes, false });
}

extern "C" int exl3r_gumbel_sample(const void* logits, int dtype, int64_t rows, int64_t vocab, int64_t ld,
                                   int max_logit, uint32_t random, int64_t* ids, void* stream)
{
    begin_call();
    return sample_entry<true>("exl3r_gumbel_sample", logits, dtype, rows, vocab, ld, max_logit, random, ids, stream);
}

extern "C" int exl3r_gumbel_noise(const void* x, int x_dtype, int64_t ldx, void* out, int out_dtype, int64_t ldo,
                                  int64_t rows, int64_t cols, uint32_t random, void* stream)
{
    begin_call();
    const char* op = "exl3r_gumbel_noise";
    if (!is_float_dtype(x_dtype) || !is_float_dtype(out_dtype))
        return set_error(EXL3R_EDTYPE, "%s: unsupported dtypes x=%s out=%s", op, dtype_name(x_dtype),
                         dtype_name(out_dtype));
    if (rows < 0 || cols < 0 || cols > 0xffffffffLL * 4 || (rows > 1 && (ldx < cols || ldo < cols)))
        return set_error(EXL3R_EINVAL, "%s: invalid shape rows=%lld cols=%lld ldx=%lld ldo=%lld", op, (long long)rows,
                         (long long)cols, (long long)ldx, (long long)ldo);
    if (rows == 0 || cols == 0) return EXL3R_OK;
    if (!x || !out) return set_error(EXL3R_EINVAL, "%s: x and out must be non-null", op);
    const int xs = dtype_bytes(x_dtype), os = dtype_bytes(out_dtype);
    NoiseArgs a{ (const char*)x, (char*)out, (rows > 1 ? ldx : cols) * xs, (rows > 1 ? ldo : cols) * os, rows, cols,
                 random };
    const bool vec = aligned16(x) && aligned16(out) && a.ldx % 16 == 0 && a.ldo % 16 == 0;
    const dim3 grid((unsigned)((cols + 2047) / 2048), (unsigned)(rows < 65535 ? rows : 65535));
    hipStream_t s = (hipStream_t)stream;
    with_float_type(x_dtype, [&](auto TI) {
        with_float_type(out_dtype, [&](auto TO) {
            if (vec) launch(k_gumbel_noise<decltype(TI), decltype(TO), true>, grid, 256, 0, s, a);
            else launch(k_gumbel_noise<decltype(TI), decltype(TO), false>, grid, 256, 0, s, a);
        });
    });
    return launch_status(op);
}
