// Naive unfused baseline kernels (see naive_baseline.h): the textbook one-op-per-launch form the
// fused kernels are measured against, plus a plain copy kernel for counter calibration.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "abi.hpp"
#include "naive_baseline.h"

using exl3r::launch;

typedef _Float16 half_t;

__global__ void k_naive_add(const half_t* x, const half_t* r, half_t* h, int64_t n)
{
    int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) h[i] = (half_t)((float)x[i] + (float)r[i]);
}

__global__ __launch_bounds__(1024) void k_naive_rms(const half_t* x, const half_t* w, half_t* y, int dim, float eps)
{
    __shared__ float red[1024];
    const half_t* xr = x + (int64_t)blockIdx.x * dim;
    half_t* yr = y + (int64_t)blockIdx.x * dim;
    float s = 0.0f;
    for (int j = threadIdx.x; j < dim; j += blockDim.x) { float v = (float)xr[j]; s += v * v; }
    red[threadIdx.x] = s;
    __syncthreads();
    for (int st = blockDim.x / 2; st > 0; st >>= 1)
    {
        if ((int)threadIdx.x < st) red[threadIdx.x] += red[threadIdx.x + st];
        __syncthreads();
    }
    const float rmf = rsqrtf(red[0] / (float)dim + eps);
    for (int j = threadIdx.x; j < dim; j += blockDim.x) yr[j] = (half_t)((float)xr[j] * (float)w[j] * rmf);
}

__global__ __launch_bounds__(1024) void k_naive_head_norm(half_t* x, const half_t* w, int hd, float eps)
{
    __shared__ float red[1024];
    half_t* xr = x + (int64_t)blockIdx.x * hd;
    float v = (int)threadIdx.x < hd ? (float)xr[threadIdx.x] : 0.0f;
    red[threadIdx.x] = v * v;
    __syncthreads();
    for (int st = blockDim.x / 2; st > 0; st >>= 1)
    {
        if ((int)threadIdx.x < st) red[threadIdx.x] += red[threadIdx.x + st];
        __syncthreads();
    }
    const float rmf = rsqrtf(red[0] / (float)hd + eps);
    if ((int)threadIdx.x < hd) xr[threadIdx.x] = (half_t)(v * rmf * (float)w[threadIdx.x]);
}

__global__ void k_naive_rope(half_t* x, const float* inv_freq, const int32_t* positions, int64_t tokens,
                             int64_t seq_len, int heads, int hd)
{
    const int half = hd / 2;
    int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= tokens * heads * half) return;
    const int t = (int)(i % half);
    const int64_t th = i / half;
    const int64_t tok = th / heads;
    const int pos = positions[tok / seq_len] + (int)(tok % seq_len);
    float s, c;
    sincosf(inv_freq[t] * (float)pos, &s, &c);
    half_t* hp = x + th * hd;
    const float v1 = (float)hp[t], v2 = (float)hp[t + half];
    hp[t] = (half_t)(v1 * c - v2 * s);
    hp[t + half] = (half_t)(v2 * c + v1 * s);
}

__global__ void k_naive_silu(const half_t* g, half_t* z, int64_t n)
{
    int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) { float v = (float)g[i]; z[i] = (half_t)(v / (1.0f + expf(-v))); }
}

__global__ void k_naive_mul(const half_t* a, const half_t* b, half_t* z, int64_t n)
{
    int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) z[i] = (half_t)((float)a[i] * (float)b[i]);
}

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

// One 16-byte chunk per thread, non-temporal load and store: the fastest copy measured on MI355X
// (6.6 TB/s for 1 GiB), used both as the practical bandwidth reference and to calibrate counters.
__global__ __launch_bounds__(128) void k_calib_copy(const u32x4* src, u32x4* dst, int64_t n16)
{
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n16) __builtin_nontemporal_store(__builtin_nontemporal_load(src + i), dst + i);
}

// Same copy with ordinary (cached) loads and stores: calibrates counters for kernels whose loads are
// cached (the embedding table rows).
__global__ __launch_bounds__(128) void k_calib_copy_cached(const u32x4* src, u32x4* dst, int64_t n16)
{
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n16) dst[i] = src[i];
}

// Unfused paged KV-cache append (the separate launch that follows RoPE in paged attention): one
// 16-byte vector of k and of v per thread, pages of page_size tokens through the block table.
// Positions are assumed valid (as the reference's kernel assumes them).
__global__ void k_naive_paged_kv(const u32x4* k, const u32x4* v, u32x4* kc, u32x4* vc, const int32_t* block_table,
                                 const int32_t* seqlens, int64_t seq_len, int heads, int vecs, int64_t max_blocks,
                                 int page_size, int64_t total)
{
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total; i += (int64_t)gridDim.x * blockDim.x)
    {
        const int64_t row = i / vecs;                   // (token, head)
        const int64_t tok = row / heads;
        const int64_t b = tok / seq_len;
        const int64_t pos = (int64_t)seqlens[b] + (tok - b * seq_len);
        const int64_t page = block_table[b * max_blocks + pos / page_size];
        const int64_t dst = ((page * page_size + pos % page_size) * heads + (row - tok * heads)) * vecs + (i - row * vecs);
        kc[dst] = k[i];
        vc[dst] = v[i];
    }
}

static unsigned blocks_for(int64_t n, int threads)
{
    int64_t b = (n + threads - 1) / threads;
    return (unsigned)(b > (1 << 30) ? (1 << 30) : (b > 0 ? b : 1));
}

extern "C" int naive_add_f16(const void* x, const void* r, void* h, int64_t n, void* stream)
{
    return launch(k_naive_add, blocks_for(n, 256), 256, 0, (hipStream_t)stream, (const half_t*)x, (const half_t*)r, (half_t*)h, n);
}

extern "C" int naive_rms_norm_f16(const void* x, const void* w, void* y, int64_t rows, int dim, float eps, void* stream)
{
    return launch(k_naive_rms, (unsigned)rows, 1024, 0, (hipStream_t)stream, (const half_t*)x, (const half_t*)w, (half_t*)y, dim, eps);
}

extern "C" int naive_head_norm_f16(void* x, const void* w, int64_t tokens, int heads, int hd, float eps, void* stream)
{
    int threads = 64;
    while (threads < hd) threads *= 2;
    return launch(k_naive_head_norm, (unsigned)(tokens * heads), threads, 0, (hipStream_t)stream, (half_t*)x, (const half_t*)w, hd, eps);
}

extern "C" int naive_rope_neox_f16(void* x, const float* inv_freq, const int32_t* positions, int64_t tokens,
                                   int64_t seq_len, int heads, int hd, void* stream)
{
    const int64_t n = tokens * heads * (hd / 2);
    return launch(k_naive_rope, blocks_for(n, 256), 256, 0, (hipStream_t)stream, (half_t*)x, inv_freq, positions, tokens, seq_len, heads, hd);
}

extern "C" int naive_silu_f16(const void* g, void* z, int64_t n, void* stream)
{
    return launch(k_naive_silu, blocks_for(n, 256), 256, 0, (hipStream_t)stream, (const half_t*)g, (half_t*)z, n);
}

extern "C" int naive_mul_f16(const void* a, const void* b, void* z, int64_t n, void* stream)
{
    return launch(k_naive_mul, blocks_for(n, 256), 256, 0, (hipStream_t)stream, (const half_t*)a, (const half_t*)b, (half_t*)z, n);
}

extern "C" int calib_copy(const void* src, void* dst, int64_t nbytes, void* stream)
{
    if (nbytes % 16) return -1;
    const int64_t n16 = nbytes / 16;
    if (n16 > ((int64_t)1 << 37)) return -1;
    return launch(k_calib_copy, (unsigned)((n16 + 127) / 128), 128, 0, (hipStream_t)stream, (const u32x4*)src, (u32x4*)dst, n16);
}

extern "C" int calib_copy_cached(const void* src, void* dst, int64_t nbytes, void* stream)
{
    if (nbytes % 16) return -1;
    const int64_t n16 = nbytes / 16;
    if (n16 > ((int64_t)1 << 37)) return -1;
    return launch(k_calib_copy_cached, (unsigned)((n16 + 127) / 128), 128, 0, (hipStream_t)stream, (const u32x4*)src, (u32x4*)dst, n16);
}

extern "C" int naive_paged_kv_update_f16(const void* k, const void* v, void* k_cache, void* v_cache,
                                         const int32_t* block_table, const int32_t* cache_seqlens, int64_t bsz,
                                         int64_t seq_len, int heads, int hd, int64_t max_blocks, int page_size,
                                         void* stream)
{
    if (hd % 8 || bsz <= 0 || seq_len <= 0) return -1;
    const int64_t total = bsz * seq_len * heads * (hd / 8);
    const unsigned grid = (unsigned)((total + 255) / 256 < 65535 ? (total + 255) / 256 : 65535);
    return launch(k_naive_paged_kv, grid, 256, 0, (hipStream_t)stream, (const u32x4*)k, (const u32x4*)v, (u32x4*)k_cache,
                                                           (u32x4*)v_cache, block_table, cache_seqlens, seq_len, heads,
                                                           hd / 8, max_blocks, page_size, total);
}
