/* Naive unfused HIP baseline for the decode-step comparison (bench only, not part of the drop-in
 * ABI): one element per thread, scalar 2-byte accesses, LDS tree reductions, one op per launch.
 * All tensors are f16, contiguous.  Returns 0 or a hipError_t. */
#ifndef EXL3R_NAIVE_BASELINE_H
#define EXL3R_NAIVE_BASELINE_H
#include <stdint.h>
#include "../../include/exl3r/rowops.h"
#ifdef __cplusplus
extern "C" {
#endif
/* h = x + r (elementwise) */
EXL3R_API int naive_add_f16(const void* x, const void* r, void* h, int64_t n, void* stream);
/* y = rmsnorm(x) * w over rows of dim (one 1024-thread block per row, LDS tree reduce) */
EXL3R_API int naive_rms_norm_f16(const void* x, const void* w, void* y, int64_t rows, int dim, float eps, void* stream);
/* per-head rmsnorm in place over [tokens, heads, hd] (one block per head) */
EXL3R_API int naive_head_norm_f16(void* x, const void* w, int64_t tokens, int heads, int hd, float eps, void* stream);
/* NeoX rotary in place over [tokens, heads, hd], full rotary; pos = positions[t / seq_len] + t % seq_len */
EXL3R_API int naive_rope_neox_f16(void* x, const float* inv_freq, const int32_t* positions, int64_t tokens,
                                   int64_t seq_len, int heads, int hd, void* stream);
/* z = silu(g) */
EXL3R_API int naive_silu_f16(const void* g, void* z, int64_t n, void* stream);
/* z = a * b */
EXL3R_API int naive_mul_f16(const void* a, const void* b, void* z, int64_t n, void* stream);
/* Paged KV-cache append as a separate launch: k, v [bsz, seq_len, heads, hd] into caches
 * [pages, page_size, heads, hd] at cache_seqlens[b] + s through block_table [bsz, max_blocks]. */
EXL3R_API int naive_paged_kv_update_f16(const void* k, const void* v, void* k_cache, void* v_cache,
                                        const int32_t* block_table, const int32_t* cache_seqlens, int64_t bsz,
                                        int64_t seq_len, int heads, int hd, int64_t max_blocks, int page_size,
                                        void* stream);
/* Non-temporal 16-byte-per-lane copy of nbytes (multiple of 16): bandwidth reference and rocprof
 * counter calibration. */
EXL3R_API int calib_copy(const void* src, void* dst, int64_t nbytes, void* stream);
/* The same copy with ordinary (cached) loads and stores. */
EXL3R_API int calib_copy_cached(const void* src, void* dst, int64_t nbytes, void* stream);
#ifdef __cplusplus
}
#endif
#endif
