/* Launch-shape overrides for tests and benchmarking sweeps -- not part of the drop-in ABI and not
 * exported by the product library (lib/libexl3rowops.so).  They exist only in the sweep/test build
 * lib/libexl3rowops_tune.so (the same sources compiled with EXL3R_TUNING), where the tests use them
 * to force each RoPE kernel on the same inputs.  0 restores the automatic choice.
 * Process-global, not thread-safe: set them before launching. */
#ifndef EXL3R_TUNING_H
#define EXL3R_TUNING_H
#include "../../include/exl3r/rowops.h"
#ifdef __cplusplus
extern "C" {
#endif
EXL3R_API void exl3r_tune_rms(int maxv, int threads);
/* short-row RMSNorm kernel: rows per lane in flight (1, 2, 4; 0 auto) */
EXL3R_API void exl3r_tune_rms_rows(int rows_per_lane);
/* plain / residual RMSNorm with split chunks (rows of whole 512-element spans): -1 never, 0 auto,
 * 1 always; the weight fetched mid-row (1) or late (2) in split launches */
EXL3R_API void exl3r_tune_rms_split(int split, int wmode);
/* streaming plain / residual RMSNorm: fp32 row sum (sum32 = 1; 0 fp64), weight fetched early / mid / late
 * (wmode 1 / 2 / 3; 0 auto), resident grid (pipe 1: as many workgroups per CU as fit, n > 1: n - 1);
 * Hadamard norms: cached residual stores (r_cached = 1) */
EXL3R_API void exl3r_tune_rms_mode(int sum32, int wmode, int r_cached, int pipe);
EXL3R_API void exl3r_tune_act(int unroll, int threads, int blocks_per_cu);
/* heads per lane: 1, 2 or 4 */
EXL3R_API void exl3r_tune_rope(int iters);
/* wave-per-token RoPE kernel: use 0 auto / 1 never / 2 always; heads per lane in flight 2, 4, 6, 8 (0 auto) */
EXL3R_API void exl3r_tune_rope_tok(int use, int hpl, int wgs_per_cu);
/* NeoX RoPE at head_dim = rotary_dim = 128, 8 lanes per head: 0 auto, -1 never, 1..3 always with that many
 * 8-head passes per wave */
EXL3R_API void exl3r_tune_rope_nx(int passes);
/* the same kernel: items (8-head passes) a wave takes in a row, its token's angles evaluated once per
 * token within them (1..16; 0 auto) */
EXL3R_API void exl3r_tune_rope_nx_run(int run);
/* the same kernel: the head norm's sum of squares in fp32 (1) instead of fp64 (0) */
EXL3R_API void exl3r_tune_rope_ss32(int on);
/* argmax / Gumbel sampling: rows from which a workgroup owns a whole row (0: 512), and its lanes (256, 512, 1024) */
EXL3R_API void exl3r_tune_sample(int rows_min, int threads);
/* Hadamard: 128-blocks per 16-lane group (1, 2, 4; 0 auto) */
EXL3R_API void exl3r_tune_had(int blocks_per_group);
/* matrix-core Hadamard kernels: spans (act-mul: rows of a span) per wave in flight (1, 2, 4; 0 auto),
 * workgroups per CU of a looping grid (0 auto, < 0 one item per wave) */
EXL3R_API void exl3r_tune_had_mfma(int unroll, int blocks_per_cu);
/* lanes per workgroup of the Hadamard kernels k_had, k_had_mfma and k_act_mul_had_mfma (64, 128, 256; 0 auto) */
EXL3R_API void exl3r_tune_had_threads(int threads);
EXL3R_API void exl3r_tune_embed(int threads);
#ifdef __cplusplus
}
#endif
#endif
