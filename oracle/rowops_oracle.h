/*
 * CPU oracle for the fused row ops — TEST INFRASTRUCTURE ONLY.
 *
 * A plain-C restatement of the reference semantics of exllamav3-rs's RMSNorm, SiLU/GELU-gated
 * multiply, q/k head-norm + rotary embedding and embedding gather (each function cites the
 * reference file:line it follows).  Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load it, and only as the checker or the timed CPU baseline; the product path
 * (the HIP library) never calls it.
 *
 * Arguments mirror include/exl3r/rowops.h, but pointers are HOST pointers and every function takes
 * an OpenMP thread count (<= 0 means 1).  Dtype codes are the EXL3R_* codes of that header.
 *
 * Parity pins (tests/test_oracle_*.py): exhaustive/ random conversion checks against numpy/torch,
 * fp64 closed forms and torch-CPU library routines (committed fixtures under tests/golden/),
 * invariants and special cases; `oracle_mutation` plants known mistakes so the tests can show that
 * each pin catches them.
 */
#ifndef EXL3R_ROWOPS_ORACLE_H
#define EXL3R_ROWOPS_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define OR_F32  0
#define OR_F16  1
#define OR_BF16 2
#define OR_I32  3
#define OR_I64  4

#define OR_ROPE_GPTJ 1
#define OR_ROPE_NEOX 2

#define OR_ACT_SILU 0
#define OR_ACT_GELU 1
#define OR_ACT_SIGMOID 2

/* Planted-mistake switch for the oracle's own tests (0 = faithful). */
extern int oracle_mutation;
#define ORM_NONE              0
#define ORM_RMS_NO_EPS        1  /* eps dropped from the mean square */
#define ORM_RMS_NO_CLAMP      2  /* f16 x not clamped to +-65504 on read */
#define ORM_RES_NO_ROUND      3  /* residual sum not rounded to r's dtype before the norm */
#define ORM_RMS_NO_BIAS       4  /* constant_bias ignored */
#define ORM_RMS_DIM_OFF       5  /* mean taken over dim - 1 */
#define ORM_SILU_SIGN         6  /* silu uses exp(+x) */
#define ORM_GELU_NO_CUBIC     7  /* gelu drops the 0.044715 x^3 term */
#define ORM_ACT_NO_LIMIT_Y    8  /* act_limit does not clamp y */
#define ORM_ROPE_SIGN         9  /* r1 = v1 cos + v2 sin */
#define ORM_ROPE_SWAP_SINCOS 10  /* sin and cos exchanged */
#define ORM_ROPE_POS_OFF     11  /* position off by one */
#define ORM_ROPE_NEOX_PAIR   12  /* NeoX pairs (2t, 2t+1) like GPT-J */
#define ORM_HEADNORM_1ROUND  13  /* f16-weight head norm rounded once instead of twice */
#define ORM_EMBED_OFF        14  /* gathers row ids[i] + 1 */
#define ORM_ROPE_NORM_AFTER  15  /* head norm applied after the rotation */
#define ORM_PAGE_OFF         16  /* paged append writes one row past the cache position */
#define ORM_GATED_WGROUP     17  /* gated norm ignores w_groups (always weight row 0) */
#define ORM_GATED_ORDER      18  /* gate_first handled as gate-after */
#define ORM_SIGMOID_SIGN     19  /* sigmoid uses exp(+x) */
#define ORM_QG_SWAP          20  /* deinterleave returns q and g exchanged */
#define ORM_ARGMAX_LAST_TIE  21  /* argmax ties go to the last index */
#define ORM_ARGMAX_NO_MASK   22  /* argmax ignores max_logit */
#define ORM_PHILOX_NO_BUMP   23  /* Philox key not advanced between rounds */
#define ORM_LOG_NO_LN2LO     24  /* log drops the low part of e * ln2 */
#define ORM_GUMBEL_NO_ROW    25  /* Gumbel noise ignores the row (every row draws the same noise) */
#define ORM_TABLE_ROW_OFF    26  /* angle table read one row past the position */
#define ORM_HAD_NO_PRE_ROUND 27  /* f16 pre-scale product kept in fp32 instead of rounded to half */
#define ORM_HAD_SIGN         28  /* butterfly stage 6 computes b - a instead of a - b */

/* Conversions (round to nearest even; NaN -> canonical quiet NaN). */
uint16_t oracle_f32_to_f16(float f);
float    oracle_f16_to_f32(uint16_t h);
uint16_t oracle_f32_to_bf16(float f);
float    oracle_bf16_to_f32(uint16_t h);
/* Round a double to the value set of dtype (F32/F16/BF16), RNE, overflow -> inf. */
double   oracle_round(double v, int dtype);
void     oracle_f32_to_f16_array(const float* in, uint16_t* out, int64_t n);
void     oracle_f32_to_bf16_array(const float* in, uint16_t* out, int64_t n);

int oracle_rms_norm(const void* x, int x_dtype, int64_t ldx,
                    const void* w, int w_dtype,
                    void* y, int y_dtype, int64_t ldy,
                    void* r /* NULL: plain RMSNorm */, int r_dtype, int64_t ldr,
                    int64_t rows, int64_t dim,
                    float eps, float constant_bias, float constant_scale, int nthreads);

int oracle_act_mul(int act, const void* x, const void* y, int in_dtype, void* z, int z_dtype,
                   int64_t rows, int64_t cols, int64_t ldx, int64_t ldy, int64_t ldz,
                   float act_limit, int nthreads);

int oracle_rope(const void* q, void* out_q, int64_t q_tok_stride, int64_t q_head_stride, int num_heads_q,
                const void* k, void* out_k, int64_t k_tok_stride, int64_t k_head_stride, int num_heads_k,
                int dtype, int64_t bsz, int64_t seq_len, int head_dim,
                const float* inv_freq, int rotary_dim,
                int32_t position, const int32_t* positions, const int32_t* position_ids,
                const void* q_norm, const void* k_norm, int norm_dtype,
                float norm_eps, float norm_constant_bias,
                int rope_mode, float attn_factor, int nthreads);

/*
 * oracle_rope with an angle table in place of inv_freq (RoPE::apply's freq_table, src/rope.rs:225-260;
 * rope.cu:69-83): the angle of frequency t for token s of sequence b at position pos is
 * table[b * table_bstride + pos * R/2 + t] (table_bstride 0: one table for every sequence); a
 * position outside [0, table_rows) stores 1 to *err (when given) and rotates by angle 0.
 */
int oracle_rope_table(const void* q, void* out_q, int64_t q_tok_stride, int64_t q_head_stride, int hq,
                      const void* k, void* out_k, int64_t k_tok_stride, int64_t k_head_stride, int hk,
                      int dt, int64_t bsz, int64_t seq_len, int hd,
                      const float* table, int64_t table_rows, int64_t table_bstride, int R,
                      int32_t position, const int32_t* positions, const int32_t* position_ids,
                      const void* q_norm, const void* k_norm, int nwt,
                      float eps, float cb, int mode, float attn_factor, int32_t* err, int nthreads);

/*
 * Gated RMSNorm (gated_rms_norm_kernel, reference kernels/norm.cu:482-581; host checks 591-668):
 *   a = act(g) in fp32 (gate_act 0 silu, 1 sigmoid);
 *   gate_first: v = fl32(x * a) and the row sum is over v; otherwise v = x;
 *   rmf = 1 / sqrtf(sum(v^2) / dim + eps);  w row = row % w_groups, plus constant_bias when it is != 0;
 *   y = (v * w) * rmf (gate_first) or ((x * w) * rmf) * a, rounded once to y's dtype.
 * x, w, g, y: F16 / BF16 / F32 (w may be NULL: no weight); x is not clamped.
 */
int oracle_gated_rms_norm(const void* x, int x_dtype, int64_t ldx, const void* w, int w_dtype, int w_groups,
                          void* y, int y_dtype, int64_t ldy, const void* g, int g_dtype, int64_t ldg,
                          int64_t rows, int64_t dim, float eps, float constant_bias, int gate_first, int gate_act,
                          int nthreads);

/*
 * Split per-head interleaved rows [rows, heads, 2 * head_dim] into q [rows, heads, head_dim] and
 * g [rows, heads * head_dim] (deinterleave_qg, reference kernels/activation.cu:721-779); row strides in
 * elements.  A bit copy of 16-bit elements.
 */
int oracle_deinterleave_qg(const void* qg, int64_t ldqg, void* q, int64_t ldq, void* g, int64_t ldg,
                           int64_t rows, int heads, int head_dim, int nthreads);

/*
 * Row argmax of logits [rows, vocab] (row stride ld; F16 / BF16 / F32) into int64 ids[rows]: the
 * first index of the maximum among indices < max_logit (max_logit <= 0 or > vocab: the whole row),
 * NaN counting as the maximum (the first NaN wins), -0 equal to +0 -- torch.argmax's rule, the batched
 * argmax of the generator (src/generator.rs:1596) that exl3_shim_argmax_sample
 * (kernels/generator/sampling_basic.cu:65-92, 151-172) also serves.
 */
int oracle_argmax(const void* logits, int dtype, int64_t rows, int64_t vocab, int64_t ld, int max_logit,
                  int64_t* ids, int nthreads);

/*
 * Random-Hadamard row transform had_r_128 (kernels/quant/hadamard.cu:88-170, inner
 * hadamard_inner.cuh:96-200): every 128-element block of each row of x [rows, cols] (cols % 128 == 0)
 * becomes y = r * H128 (x o pre) o post, H128 the Sylvester Hadamard matrix, r = fl32(scale *
 * fl32(1/sqrt(128))).  F16: the pre-scale product is a half multiply (rounded to half), the transform
 * runs in fp32 as the in-place butterfly with stages over index bits 0..6 in that order, each pair
 * (a, b) -> (a + b, a - b); the result times r is rounded to half once, then the post-scale half
 * multiply.  F32: the same with fp32 scale products.  pre and post are f16 [cols] or NULL; at most
 * one is given.  out may be x.
 */
int oracle_had_r_128(const void* x, int dt, int64_t ldx, void* out, int64_t ldo, int64_t rows, int64_t cols,
                     const uint16_t* pre, const uint16_t* post, float scale, int nthreads);

/*
 * Gumbel-max sampling (the role of exl3_shim_gumbel_sample / exl3_shim_gumbel_noise_f32,
 * kernels/generator/sampling_basic.cu:94-128, 174-197 and gumbel.cu:45-62).  The reference draws
 * its uniforms from cuRAND's Philox stream; this build defines its own stream over the published
 * Philox4x32-10 generator (Salmon, Moraes, Dror, Shaw, "Parallel random numbers: as easy as 1, 2,
 * 3", SC 2011):
 *   bits(r, c) = Philox4x32-10(counter = {c >> 2, r mod 2^32, r >> 32, 0}, key = {seed, 0})[c & 3]
 *   u = ((bits >> 9) + 0.5) * 2^-23                  (exact; 2^-24 <= u <= 1 - 2^-24)
 *   g = -log(-log(u))                                 (log_f32 below, fp32)
 *   noisy(r, c) = fl32(x(r, c) + g)
 * so the noise of an element depends only on (seed, row, column), never on the launch shape.
 */
void oracle_philox4x32_10(const uint32_t ctr[4], const uint32_t key[2], uint32_t out[4]);
/* The fp32 natural log both sides evaluate (argument reduction to [sqrt(1/2), sqrt(2)), Cody-Waite
 * split of e*ln2, log(1+f) = f - (f^2/2 - s (f^2/2 + R(s^2))) with s = f/(2+f) from a Newton
 * reciprocal and R the atanh series through s^10), for positive normal x. */
float oracle_log_f32(float x);
/* g[i] = -log(-log(u(bits[i]))) for raw Philox words. */
void oracle_gumbel_of_bits(const uint32_t* bits, float* g, int64_t n);
/* out[r, c] = x[r, c] + g(seed, r, c), every column; in F16/BF16/F32, out F16/BF16/F32 (one rounding). */
int oracle_gumbel_noise(const void* x, int xt, int64_t ldx, void* out, int ot, int64_t ldo, int64_t rows,
                        int64_t cols, uint32_t seed, int nthreads);
/* ids[r] = argmax over c < max_logit of fl32(x[r, c] + g(seed, r, c)) (oracle_argmax's rule). */
int oracle_gumbel_sample(const void* logits, int dtype, int64_t rows, int64_t vocab, int64_t ld, int max_logit,
                         uint32_t seed, int64_t* ids, int nthreads);

/*
 * Paged KV-cache append (paged_kv_update_vec8_kernel, reference kernels/generator/cache.cu:143-243):
 * for each sequence b, token s and kv head h, with pos = cache_seqlens[b] + s,
 *   k_cache[page, pos % page_size, h, :] = k[b, s, h, :]   (v likewise),
 *   page = block_table[b * max_blocks + pos / page_size].
 * Caches are contiguous [num_pages, page_size, num_heads_kv, head_dim] of k's dtype (F16 / BF16).
 * A position outside the block table or a page outside the pool is skipped and sets *err_flag
 * (the reference does not check them).  k or v may be NULL (that cache is not written).
 */
int oracle_paged_kv_append(const void* k, int64_t k_tok_stride, int64_t k_head_stride,
                           const void* v, int64_t v_tok_stride, int64_t v_head_stride,
                           int num_heads_kv, int dtype, int64_t bsz, int64_t seq_len, int head_dim,
                           void* k_cache, void* v_cache, int page_size, int64_t num_pages,
                           const int32_t* block_table, int64_t max_blocks, const int32_t* cache_seqlens,
                           int32_t* err_flag, int nthreads);

int oracle_embedding(const void* table, int table_dtype, int64_t vocab, int64_t hidden, int64_t ldt,
                     const void* ids, int ids_dtype, int64_t n,
                     void* out, int out_dtype, int64_t ldo,
                     int32_t* err_flag, int nthreads);

int oracle_embedding_rms_norm(const void* table, int table_dtype, int64_t vocab, int64_t hidden, int64_t ldt,
                              const void* ids, int ids_dtype, int64_t n,
                              void* h, int h_dtype, int64_t ldh,
                              const void* w, int w_dtype,
                              void* y, int y_dtype, int64_t ldy,
                              float eps, float constant_bias, float constant_scale,
                              int32_t* err_flag, int nthreads);

#ifdef __cplusplus
}
#endif

#endif
