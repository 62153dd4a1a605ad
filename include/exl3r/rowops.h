/*
 * exl3r rowops — C ABI of the MI355X (gfx950) fused per-layer row kernels.
 *
 * Drop-in replacement for the `at::Tensor*` shim entry points of exllamav3-rs that cover
 * RMSNorm, residual-fused RMSNorm, SiLU/GELU-gated multiply, q/k head-norm + rotary, and the
 * token-embedding gather.  Every entry point takes raw device pointers, element counts and row
 * strides (in ELEMENTS, not bytes), dtype codes and an explicit HIP stream (`hipStream_t`
 * passed as `void*`; NULL = the null stream).
 *
 * Common contract of every `int exl3r_*` entry point:
 *   - returns EXL3R_OK (0) on success, a negative EXL3R_E* code for an invalid argument (nothing is
 *     launched), or a positive hipError_t when the launch itself failed;
 *   - on failure exl3r_last_error() returns a message for the calling thread;
 *   - the status covers this call's own launches only: the thread's HIP last-error state
 *     (hipGetLastError / hipPeekAtLastError) is neither read nor cleared, so an error another
 *     caller left pending stays pending (a launch that fails sets it, as any failing HIP call does);
 *   - never allocates, never synchronises the host, never throws or exits;
 *   - is stateless and thread-safe; work is enqueued on `stream` only (capture-safe: the
 *     device-resident position/id buffers are read by the kernels, so a captured graph can be
 *     replayed after their contents change);
 *   - arguments are validated before any HIP call, so validation errors are reported even on a
 *     machine without a GPU;
 *   - a call with no rows / tokens / ids validates its shapes and dtypes and returns EXL3R_OK
 *     without launching; its data pointers may then be NULL (empty tensors carry none).
 *
 * Reference entry points replaced (apiplant/exllamav3-rs, cited file:line):
 *   exl3r_rms_norm          <- exl3_shim_rms_norm         csrc/exl3_shim.cpp:76-80   (ffi.rs:43-50, 293-296)
 *   exl3r_rms_norm_res_in   <- exl3_shim_rms_norm_res_in  csrc/exl3_shim.cpp:139-142 (ffi.rs:114-117, 464-468)
 *   exl3r_silu_mul          <- exl3_shim_silu_mul         csrc/exl3_shim.cpp:151     (ffi.rs:125, 492-495)
 *   exl3r_gelu_mul          <- exl3_shim_gelu_mul         csrc/exl3_shim.cpp:152     (ffi.rs:126, 496-499)
 *   exl3r_rope              <- exl3_shim_rope             csrc/exl3_shim.cpp:87-98   (ffi.rs:51-65, 298-333)
 *   exl3r_rope_table        <- exl3_shim_rope with a [max_pos, rotary_dim/2] (or per-sequence
 *                              [bsz, max_pos, rotary_dim/2]) angle table as inv_freq, RoPE::apply's
 *                              freq_table  src/rope.rs:225-260, kernels/rope.cu:69-83, 340-347
 *   exl3r_rope_cs_table,    <- exl3_shim_rope with its per-layer sin / cos evaluation (kernels/rope.cu:69-85)
 *   exl3r_rope_cs              hoisted into one table per forward pass, as RoPE::angle_table hoists the
 *                              angles (src/rope.rs:225-260, 294-301)
 *   exl3r_rope_paged_kv     <- exl3_shim_rope followed by exl3_shim_paged_kv_cache_update
 *                              csrc/exl3_shim.cpp:87-98, 109-112 (ffi.rs:298-350; call sites modules.rs:666-704)
 *   exl3r_rope_qg           <- exl3_shim_deinterleave_qg then exl3_shim_rope on q (gated attention,
 *                              src/modules.rs:637-646 then 669-681)
 *   exl3r_gated_rms_norm    <- exl3_shim_gated_rms_norm   csrc/exl3_shim.cpp:143-147 (ffi.rs:118-124, 479-483)
 *   exl3r_mul_sigmoid       <- exl3_shim_mul_sigmoid_     csrc/exl3_shim.cpp:167     (ffi.rs:166, 616-618)
 *   exl3r_deinterleave_qg   <- exl3_shim_deinterleave_qg  csrc/exl3_shim.cpp:168-171 (ffi.rs:167, 622-624)
 *   exl3r_argmax_sample     <- exl3_shim_argmax_sample    csrc/exl3_shim.cpp:229-231 (ffi.rs:136, 521-525) and the
 *                              generator's batched tch argmax over [bsz, vocab] logits  src/generator.rs:1596
 *   exl3r_gumbel_sample     <- exl3_shim_gumbel_sample    csrc/exl3_shim.cpp:232-234 (ffi.rs:137, 526-530)
 *   exl3r_gumbel_noise      <- exl3_shim_gumbel_noise_f32 csrc/exl3_shim.cpp:235-237 (ffi.rs:138, 531-535)
 *   exl3r_had_r_128         <- exl3_shim_had_r_128        csrc/exl3_shim.cpp:158-160 (ffi.rs:162-164, 604-608;
 *                              call sites modules.rs:224-231)
 *   exl3r_rms_norm_had      <- RmsNorm::forward / forward_res followed by each projection's had_r_128
 *                              input rotation  src/modules.rs:372-411, 224-227
 *   exl3r_embedding         <- Embedding::forward's tch index_select + to_kind   src/modules.rs:430-436
 *   exl3r_embedding_rms_norm<- embed followed by RmsNorm::forward (MTP head)    src/mtp.rs:189-190
 */
#ifndef EXL3R_ROWOPS_H
#define EXL3R_ROWOPS_H

#include <stddef.h>
#include <stdint.h>

#if defined(__GNUC__) || defined(__clang__)
#define EXL3R_API __attribute__((visibility("default")))
#else
#define EXL3R_API
#endif

#ifdef __cplusplus
extern "C" {
#endif

/* dtype codes */
#define EXL3R_F32  0
#define EXL3R_F16  1
#define EXL3R_BF16 2
#define EXL3R_I32  3
#define EXL3R_I64  4

/* status codes (positive values are hipError_t) */
#define EXL3R_OK            0
#define EXL3R_EINVAL      (-1) /* null pointer, bad shape, stride or scalar argument */
#define EXL3R_EDTYPE      (-2) /* unsupported dtype or dtype combination */

/* rotary styles: same values as ROPESTYLE_* (kernels/rope.cuh:6-8) and ffi::ROPE_* (src/ffi.rs:217-219) */
/* activations of exl3r_act_mul_had */
#define EXL3R_ACT_SILU        0 /* silu(x) * y */
#define EXL3R_ACT_GELU        1 /* gelu(x) * y */
#define EXL3R_ACT_MUL_SIGMOID 2 /* x * sigmoid(y) */

/* Flag of the fused Hadamard entry points (exl3r_act_mul_had's rotate_in, exl3r_rms_norm_had's rotate_x,
 * the rope_mode of exl3r_rope_had / exl3r_rope_paged_kv_had, exl3r_rope_desc's rotate,
 * exl3r_gated_rms_norm_had's gate_act): the 128-point
 * transforms as the reference's fp32 butterfly (bit-identical to the unfused calls) instead of the
 * matrix-core form (within the stated rounding tolerance of it). */
#define EXL3R_HAD_EXACT 16

#define EXL3R_ROPE_NONE 0
#define EXL3R_ROPE_GPTJ 1
#define EXL3R_ROPE_NEOX 2

/* ABI version: major * 10000 + minor * 100 + patch */
EXL3R_API int exl3r_version(void);

/* Message describing the last failing call on this thread ("" if none). */
EXL3R_API const char* exl3r_last_error(void);

/*
 * RMSNorm over the last dimension:
 *   y[i, :] = (x[i, :] * (w + constant_bias)) * (constant_scale / sqrt(mean(x[i, :]^2) + eps))
 * Replaces exl3_shim_rms_norm (csrc/exl3_shim.cpp:76-80) -> rms_norm RES_NONE (kernels/norm.cu:434-448).
 *   x: [rows, dim] with row stride ldx; dtype F16 (clamped to +-65504 on read), BF16 or F32.
 *   w: [dim] contiguous, F16/BF16/F32, or NULL for no weight.
 *   y: [rows, dim] with row stride ldy; F16/BF16/F32.  y == x (in place) is allowed when the
 *      element sizes and strides agree.
 */
EXL3R_API int exl3r_rms_norm(const void* x, int x_dtype, int64_t ldx,
                   const void* w, int w_dtype,
                   void* y, int y_dtype, int64_t ldy,
                   int64_t rows, int64_t dim,
                   float eps, float constant_bias, float constant_scale,
                   void* stream);

/*
 * Pre-norm residual add fused with RMSNorm:
 *   r[i, :] <- round_r(x[i, :] + r[i, :])   (in place, rounded to r's dtype like an unfused add)
 *   y[i, :]  = RMSNorm(r[i, :])             (as exl3r_rms_norm, no clamp on the sum)
 * Replaces exl3_shim_rms_norm_res_in (csrc/exl3_shim.cpp:139-142) -> rms_norm RES_IN
 * (kernels/norm.cu:467-479, kernel 198-223).  r: [rows, dim], row stride ldr, F16/BF16/F32.
 */
EXL3R_API int exl3r_rms_norm_res_in(const void* x, int x_dtype, int64_t ldx,
                          const void* w, int w_dtype,
                          void* y, int y_dtype, int64_t ldy,
                          void* r, int r_dtype, int64_t ldr,
                          int64_t rows, int64_t dim,
                          float eps, float constant_bias, float constant_scale,
                          void* stream);

/*
 * Gated activations, z = act(x) * y, computed in fp32 and rounded once to z's dtype:
 *   silu(x) = x / (1 + exp(-x));   gelu(x) = 0.5 x (1 + tanh(sqrt(2/pi) (x + 0.044715 x^3)))
 * With act_limit != 0: act(x) is clamped from above and y to [-act_limit, act_limit] first.
 * An F16 z is clamped to +-65504 (NaN -> 65504), as the reference's fp32 path does.
 * Replaces exl3_shim_silu_mul / exl3_shim_gelu_mul (csrc/exl3_shim.cpp:151-152 ->
 * kernels/activation.cu:24-98, 181-255).
 *   x, y: [rows, cols], row strides ldx, ldy; both of in_dtype (F16/BF16/F32).
 *   z:    [rows, cols], row stride ldz; F16/BF16/F32.  z may alias x or y exactly.
 */
EXL3R_API int exl3r_silu_mul(const void* x, const void* y, int in_dtype, void* z, int z_dtype,
                   int64_t rows, int64_t cols, int64_t ldx, int64_t ldy, int64_t ldz,
                   float act_limit, void* stream);
EXL3R_API int exl3r_gelu_mul(const void* x, const void* y, int in_dtype, void* z, int z_dtype,
                   int64_t rows, int64_t cols, int64_t ldx, int64_t ldy, int64_t ldz,
                   float act_limit, void* stream);

/*
 * Gated RMSNorm (the Qwen3.5 gated-delta-net output norm, src/qwen3_5.rs:212; Mamba2 group norm):
 *   a = act(g) with act = silu (gate_act 0) or sigmoid (gate_act 1), in fp32;
 *   gate_first == 0: y = ((x * w') * rmf) * a,   rmf = 1 / sqrt(mean(x^2) + eps);
 *   gate_first != 0: y = (v * w') * rmf with v = x * a and rmf over v;
 *   w' = w + constant_bias, row i using weight row i % w_groups (w holds w_groups * dim values;
 *   w == NULL: no weight); one rounding to y's dtype; x is not clamped.
 * Replaces exl3_shim_gated_rms_norm (csrc/exl3_shim.cpp:143-147) -> gated_rms_norm
 * (kernels/norm.cu:482-668), which takes bf16 x, f32/bf16 w, bf16/f32 g and f16/f32 y.
 *   x: [rows, dim] F16/BF16/F32, row stride ldx;  g: [rows, dim] F16/BF16/F32, row stride ldg;
 *   y: [rows, dim] F16/BF16/F32, row stride ldy (y may equal x, not g).
 */
EXL3R_API int exl3r_gated_rms_norm(const void* x, int x_dtype, int64_t ldx, const void* w, int w_dtype, int w_groups,
                         void* y, int y_dtype, int64_t ldy, const void* g, int g_dtype, int64_t ldg,
                         int64_t rows, int64_t dim, float eps, float constant_bias,
                         int gate_first, int gate_act, void* stream);

/*
 * exl3r_gated_rms_norm with an f16 output that feeds the next EXL3 projection's input rotation, in one
 * pass: the Qwen3.5 gated-delta-net output norm, then o_proj's had_r_128(y, pre_scale)
 * (src/qwen3_5.rs:208-214 -> src/modules.rs:224-227).
 *   out = had_r_128(y, pre_scale) with scale had_scale: f16 [rows, dim] at row stride ldo (y, out
 *         and the rows of the projection input share one layout); y (f16, the norm output) is written
 *         only when y != NULL.
 *   pre_scale: the projection's f16 suh or NULL; norm row r uses pre_scale[(r % pre_rows) * dim ..] --
 *         with the usual layout (rows = tokens * heads of dim = head_dim, dense) pre_rows = heads and
 *         pre_scale is [heads * head_dim]; pre_rows > 1 needs rows % pre_rows == 0 and ldo == ldy == dim.
 *   gate_act: as exl3r_gated_rms_norm, | EXL3R_HAD_EXACT for the reference's butterfly.
 * dim % 128 == 0; out and y alias nothing.  Rows of dim 128 (16-bit x, f32 or bf16 gate, 16-byte
 * aligned) run the transform on the matrix cores: bit-identical to exl3r_gated_rms_norm with an f16 y
 * followed by exl3r_had_r_128_mfma over the [rows / pre_rows, pre_rows * dim] projection rows.  With
 * EXL3R_HAD_EXACT, and at other row lengths, bit-identical to it followed by exl3r_had_r_128;
 * unaligned or f32-x rows run those calls.
 */
EXL3R_API int exl3r_gated_rms_norm_had(const void* x, int x_dtype, int64_t ldx, const void* w, int w_dtype,
                             int w_groups, const void* g, int g_dtype, int64_t ldg, void* y, int64_t ldy,
                             const void* pre_scale, int pre_rows, void* out, int64_t ldo, int64_t rows,
                             int64_t dim, float eps, float constant_bias, int gate_first, int gate_act,
                             float had_scale, void* stream);

/*
 * Sigmoid gate: z = x * sigmoid(y), in fp32, rounded once to z's dtype (the gated-attention
 * output gate, src/modules.rs:785-787).  Replaces exl3_shim_mul_sigmoid_ (csrc/exl3_shim.cpp:167 ->
 * mul_sigmoid_, kernels/activation.cu:532-568, in place on f16 with half arithmetic).
 *   x, y: [rows, cols] of in_dtype (F16/BF16/F32), row strides ldx, ldy; z of z_dtype, row stride
 *   ldz; z may equal x (the reference's in-place form) or y.
 */
EXL3R_API int exl3r_mul_sigmoid(const void* x, const void* y, int in_dtype, void* z, int z_dtype,
                      int64_t rows, int64_t cols, int64_t ldx, int64_t ldy, int64_t ldz, void* stream);

/*
 * Split a per-head interleaved projection (rows of [heads, q | g], 2 * head_dim per head) into
 * q [rows, heads, head_dim] and g [rows, heads * head_dim], bit for bit.  Replaces
 * exl3_shim_deinterleave_qg (csrc/exl3_shim.cpp:168-171 -> deinterleave_qg,
 * kernels/activation.cu:721-779).  Row strides in elements; dtype F16/BF16/F32 (copied as bits).
 */
EXL3R_API int exl3r_deinterleave_qg(const void* qg, int64_t ld_qg, void* q, int64_t ld_q, void* g, int64_t ld_g,
                          int dtype, int64_t rows, int heads, int head_dim, void* stream);

/*
 * Fused per-head RMSNorm (optional) + rotary embedding on q and (optional) k.
 * Replaces exl3_shim_rope (csrc/exl3_shim.cpp:87-98) -> rope (kernels/rope.cu:279-467).
 *   q, out_q: [bsz, seq_len, num_heads_q, head_dim] of dtype (F16/BF16); element (b, s, h, d) at
 *             (b*seq_len + s)*q_tok_stride + h*q_head_stride + d.  out_q may equal q (in place);
 *             out_q uses q's strides.
 *   k, out_k: same for num_heads_k key heads (k == NULL: q only, as RoPE::apply_one).
 *   inv_freq: [rotary_dim / 2] float32; rotary_dim even, 2 <= rotary_dim <= head_dim.  Dimensions
 *             >= rotary_dim pass through (normed if a norm is applied).
 *   position / positions / position_ids: rotary position of token s of sequence b is
 *             position + s, or positions[b] + s (int32 [bsz], device), or position_ids[b*seq_len + s]
 *             (int32 [bsz*seq_len], device).  At most one of positions/position_ids is non-NULL.
 *   q_norm, k_norm: [head_dim] contiguous norm weights of norm_dtype (F16/BF16/F32) or NULL.  A
 *             norm is applied iff q_norm != NULL; then k_norm is required when k != NULL.
 *   rope_mode: EXL3R_ROPE_GPTJ (pairs 2t, 2t+1) or EXL3R_ROPE_NEOX (pairs t, t + rotary_dim/2).
 *   sin and cos of angle = fl32(inv_freq[t] * (float)pos) are evaluated in double precision, rounded
 *   once to fp32 and scaled by attn_factor (supported for |angle| < 2^52).
 */
EXL3R_API int exl3r_rope(const void* q, void* out_q, int64_t q_tok_stride, int64_t q_head_stride, int num_heads_q,
               const void* k, void* out_k, int64_t k_tok_stride, int64_t k_head_stride, int num_heads_k,
               int dtype, int64_t bsz, int64_t seq_len, int head_dim,
               const float* inv_freq, int rotary_dim,
               int32_t position, const int32_t* positions, const int32_t* position_ids,
               const void* q_norm, const void* k_norm, int norm_dtype,
               float norm_eps, float norm_constant_bias,
               int rope_mode, float attn_factor,
               void* stream);

/*
 * exl3r_rope with precomputed rotation angles (MRoPE, the vision tower's 2-D RoPE): the angle of
 * frequency t for token s of sequence b at position pos (from position / positions / position_ids as
 * in exl3r_rope) is angle_table[b*table_batch_stride + pos*(rotary_dim/2) + t]; sin and cos of it
 * are evaluated as in exl3r_rope.  table_batch_stride 0 shares one [table_rows, rotary_dim/2] table
 * between sequences; table_rows*rotary_dim/2 gives each sequence its own.  Replaces exl3_shim_rope
 * called with a 2-D / 3-D inv_freq (kernels/rope.cu:69-83, 340-347, where the 2-D form is only
 * valid for bsz 1).
 *   err_flag: NULL or a device int32; a position outside [0, table_rows) is rotated by angle 0 and
 *             1 is stored to *err_flag (the reference reads outside the table).
 */
EXL3R_API int exl3r_rope_table(const void* q, void* out_q, int64_t q_tok_stride, int64_t q_head_stride, int num_heads_q,
                     const void* k, void* out_k, int64_t k_tok_stride, int64_t k_head_stride, int num_heads_k,
                     int dtype, int64_t bsz, int64_t seq_len, int head_dim,
                     const float* angle_table, int64_t table_rows, int64_t table_batch_stride, int rotary_dim,
                     int32_t position, const int32_t* positions, const int32_t* position_ids,
                     const void* q_norm, const void* k_norm, int norm_dtype,
                     float norm_eps, float norm_constant_bias, int rope_mode, float attn_factor,
                     int32_t* err_flag, void* stream);

/*
 * exl3r_deinterleave_qg followed by exl3r_rope on its q, in one pass (gated attention's q projection,
 * src/modules.rs:637-646, then RoPE::apply, src/modules.rs:669-681): head h of token (b, s) is read
 * from the q half of the interleaved pair at qg + (b*seq_len + s)*qg_tok_stride + h*2*head_dim and
 * written roped (and normed) to a dense out_q [bsz, seq_len, num_heads_q, head_dim].  Bit-identical to
 * the two calls.  The gate is left in qg (g of head h at + h*2*head_dim + head_dim): with a dense qg
 * (qg_tok_stride = num_heads_q*2*head_dim), exl3r_mul_sigmoid over rows = tokens*num_heads_q and
 * cols = head_dim reads it with ldy = 2*head_dim, so the deinterleave copy disappears.  out_q must not
 * overlap qg; every other argument as exl3r_rope.
 */
EXL3R_API int exl3r_rope_qg(const void* qg, int64_t qg_tok_stride, void* out_q, int num_heads_q, const void* k,
                            void* out_k, int64_t k_tok_stride, int64_t k_head_stride, int num_heads_k, int dtype,
                            int64_t bsz, int64_t seq_len, int head_dim, const float* inv_freq, int rotary_dim,
                            int32_t position, const int32_t* positions, const int32_t* position_ids,
                            const void* q_norm, const void* k_norm, int norm_dtype, float norm_eps,
                            float norm_constant_bias, int rope_mode, float attn_factor, void* stream);

/*
 * {cos, sin} * attn_factor of every token's rotary frequencies, for exl3r_rope_cs: the positions of a
 * forward pass are the same in every layer, so one table serves all of its RoPE calls (the reference
 * evaluates sin / cos in every layer's kernel, kernels/rope.cu:69-85; RoPE::angle_table hoists only the
 * angles, src/rope.rs:294-301).
 *   cs_table: [bsz*seq_len, rotary_dim/2] pairs of float32 {cos, sin} (8 * bsz*seq_len * rotary_dim/2
 *             bytes, 8-byte aligned); row b*seq_len + s holds token s of sequence b.
 *   inv_freq, rotary_dim, position / positions / position_ids, attn_factor: as exl3r_rope; each pair
 *             is the value exl3r_rope evaluates for that token and frequency.
 */
EXL3R_API int exl3r_rope_cs_table(int64_t bsz, int64_t seq_len, const float* inv_freq, int rotary_dim,
                                  int32_t position, const int32_t* positions, const int32_t* position_ids,
                                  float attn_factor, void* cs_table, void* stream);

/*
 * exl3r_rope with the rotary pairs read from a table that exl3r_rope_cs_table filled for the same
 * bsz, seq_len, inv_freq, rotary_dim, positions and attn_factor: bit-identical to exl3r_rope, and every
 * other argument as there.  The kernels copy a token's table row where exl3r_rope evaluates it.
 */
EXL3R_API int exl3r_rope_cs(const void* q, void* out_q, int64_t q_tok_stride, int64_t q_head_stride, int num_heads_q,
                            const void* k, void* out_k, int64_t k_tok_stride, int64_t k_head_stride, int num_heads_k,
                            int dtype, int64_t bsz, int64_t seq_len, int head_dim, const void* cs_table,
                            int rotary_dim, const void* q_norm, const void* k_norm, int norm_dtype, float norm_eps,
                            float norm_constant_bias, int rope_mode, void* stream);

/*
 * exl3r_rope preceded by the q / k projections' output rotation, in one pass at prefill: the EXL3
 * linear's had_r_128(y, y, NULL, svh, 1.0) (src/modules.rs:231) on each projection output, then
 * RoPE::apply on it (src/rope.rs:233-260).  q, k: f16 [tokens, heads * head_dim] rows with heads
 * packed (head stride = head_dim), heads * head_dim a multiple of 128; q_post_scale / k_post_scale:
 * f16 [heads * head_dim] (the projections' svh) or NULL.  Other arguments as exl3r_rope.  q and k are
 * only read when out_q / out_k differ from them.  head_dim 128 (NeoX at rotary_dim 128, or GPT-J at a
 * rotary_dim multiple of 4), 16-byte aligned: one fused launch, whose transforms run on the matrix cores:
 * bit-identical to exl3r_had_r_128_mfma on q and k followed by exl3r_rope (each rotated value the
 * butterfly's or its f16 neighbour, as exl3r_had_r_128_mfma states); with EXL3R_HAD_EXACT in rope_mode,
 * the reference's butterfly, bit-identical to exl3r_had_r_128 followed by exl3r_rope.  Otherwise the
 * rotations run (as exl3r_had_r_128) into out_q / out_k and exl3r_rope in place there.
 *   cs_table: NULL, or a {cos, sin} table that exl3r_rope_cs_table filled for the same positions,
 *             inv_freq, rotary_dim and attn_factor; the rotary pairs are then read from it (inv_freq
 *             may be NULL; the results are the same bits).
 */
EXL3R_API int exl3r_rope_had(const void* q, void* out_q, int64_t q_tok_stride, int num_heads_q,
                   const void* k, void* out_k, int64_t k_tok_stride, int num_heads_k,
                   int dtype, int64_t bsz, int64_t seq_len, int head_dim,
                   const float* inv_freq, int rotary_dim,
                   int32_t position, const int32_t* positions, const int32_t* position_ids,
                   const void* q_norm, const void* k_norm, int norm_dtype,
                   float norm_eps, float norm_constant_bias, int rope_mode, float attn_factor,
                   const void* q_post_scale, const void* k_post_scale, const void* cs_table, void* stream);

/*
 * exl3r_rope_paged_kv preceded by the q / k / v projections' output rotation at prefill: each
 * projection output first becomes had_r_128(y, y, NULL, svh, 1.0) (src/modules.rs:231), then RoPE::apply
 * and paged_kv_cache_update (src/modules.rs:669-704).  q, k, v: f16 with heads packed (head stride =
 * head_dim), heads * head_dim a multiple of 128; *_post_scale: f16 [heads * head_dim] (svh) or NULL.
 * Other arguments as exl3r_rope_paged_kv.  head_dim 128 (NeoX at rotary_dim 128, or GPT-J at a
 * rotary_dim multiple of 4), 16-byte aligned: one fused launch that writes only out_q, out_k (if given)
 * and the caches, its transforms on the matrix cores (bit-identical to exl3r_had_r_128_mfma on q, k and
 * v followed by exl3r_rope_paged_kv) or, with EXL3R_HAD_EXACT in rope_mode, as the reference's butterfly
 * (bit-identical to exl3r_had_r_128 followed by exl3r_rope_paged_kv).  Otherwise the rotations run first
 * (as exl3r_had_r_128) -- q into out_q, k into out_k (into k itself when out_k is NULL) and v in place --
 * then exl3r_rope_paged_kv.  cs_table: as exl3r_rope_had.
 */
EXL3R_API int exl3r_rope_paged_kv_had(const void* q, void* out_q, int64_t q_tok_stride, int num_heads_q,
                            const void* k, void* out_k, int64_t k_tok_stride, const void* v,
                            int64_t v_tok_stride, int num_heads_kv, int dtype, int64_t bsz,
                            int64_t seq_len, int head_dim, const float* inv_freq, int rotary_dim,
                            int32_t position, const int32_t* positions, const int32_t* position_ids,
                            const void* q_norm, const void* k_norm, int norm_dtype,
                            float norm_eps, float norm_constant_bias, int rope_mode, float attn_factor,
                            void* k_cache, void* v_cache, int page_size, int64_t num_pages,
                            const int32_t* block_table, int64_t max_blocks_per_seq,
                            const int32_t* cache_seqlens, int32_t* err_flag,
                            const void* q_post_scale, const void* k_post_scale, const void* v_post_scale,
                            const void* cs_table, void* stream);

/*
 * exl3r_rope fused with the paged KV-cache append that follows it in paged attention
 * (Attention::forward, src/modules.rs:666-704: rope in place, then paged_kv_cache_update,
 * kernels/generator/cache.cu:143-243):
 *   q, k: as exl3r_rope (q -> out_q); the roped k heads are written to out_k when out_k != NULL
 *         (may equal k) and, for each token, to k_cache;
 *   v:    [bsz, seq_len, num_heads_kv, head_dim] of dtype, row (b*seq_len + s)*v_tok_stride +
 *         h*v_head_stride, copied unchanged to v_cache;
 *   k_cache, v_cache: contiguous [num_pages, page_size, num_heads_kv, head_dim] of dtype; token s of
 *         sequence b goes to page block_table[b*max_blocks_per_seq + pos / page_size], row
 *         pos % page_size, with pos = cache_seqlens[b] + s (int32 device arrays).  page_size is a
 *         power of two (the reference's pages hold 256 tokens).
 *   err_flag: NULL or a device int32; a token whose pos is negative or past the block table, or whose
 *         page is outside [0, num_pages), is not appended and 1 is stored to *err_flag (the
 *         reference does not check).  k heads are still written to out_k.
 * The rotary position arguments are independent of cache_seqlens (the paged path passes the same
 * per-sequence lengths to both: positions = cache_seqlens).
 *   cs_table: NULL, or a {cos, sin} table that exl3r_rope_cs_table filled for the same positions,
 *         inv_freq, rotary_dim and attn_factor: the rotary pairs are read from it (inv_freq may be
 *         NULL), bit-identical to evaluating them.  One table serves every layer of a forward pass.
 */
EXL3R_API int exl3r_rope_paged_kv(const void* q, void* out_q, int64_t q_tok_stride, int64_t q_head_stride, int num_heads_q,
                        const void* k, void* out_k, int64_t k_tok_stride, int64_t k_head_stride,
                        const void* v, int64_t v_tok_stride, int64_t v_head_stride, int num_heads_kv,
                        int dtype, int64_t bsz, int64_t seq_len, int head_dim,
                        const float* inv_freq, int rotary_dim,
                        int32_t position, const int32_t* positions, const int32_t* position_ids,
                        const void* q_norm, const void* k_norm, int norm_dtype,
                        float norm_eps, float norm_constant_bias, int rope_mode, float attn_factor,
                        void* k_cache, void* v_cache, int page_size, int64_t num_pages,
                        const int32_t* block_table, int64_t max_blocks_per_seq, const int32_t* cache_seqlens,
                        int32_t* err_flag, const void* cs_table, void* stream);

/*
 * Every RoPE variant above through one descriptor: the variant follows from the fields that are set,
 * so a further fusion adds fields here instead of another entry point.  No counterpart in the
 * reference (its RoPE is one shim, exl3_shim_rope); for callers that build their arguments once per
 * layer and for bindings that would otherwise mirror eight signatures.  Semantics, results and errors
 * are those of the entry point it selects:
 *   rotate = 1 or 1 | EXL3R_HAD_EXACT (the projections' output rotations; q_post_scale / k_post_scale /
 *                      v_post_scale; the flag goes to rope_mode)
 *                      -> exl3r_rope_paged_kv_had with k_cache, else exl3r_rope_had (heads packed);
 *   k_cache != NULL    -> exl3r_rope_paged_kv (v, caches, block table, cache_seqlens, err_flag);
 *   angle_table        -> exl3r_rope_table (table_rows, table_batch_stride, err_flag);
 *   out_q in its own layout (q_head_stride = 2 * head_dim, out_q dense: the gated q | g split)
 *                      -> exl3r_rope_qg;
 *   cs_table           -> exl3r_rope_cs;
 *   otherwise          -> exl3r_rope.
 * One rotation source: inv_freq, angle_table or cs_table (rotate and k_cache accept cs_table with
 * inv_freq too, as their entry points do).  out_q_tok_stride and out_q_head_stride of 0 mean q's.
 * struct_size must be at least sizeof(exl3r_rope_desc) as this header declares it.  attn_factor must be
 * set (1.0 for the unscaled rotation): 0 or NaN, which a zero-initialised descriptor would pass, is
 * refused with EXL3R_EINVAL.
 */
typedef struct exl3r_rope_desc
{
    int32_t struct_size;
    int32_t dtype;
    int64_t bsz, seq_len;
    int32_t head_dim, rotary_dim;
    int32_t rope_mode;
    float attn_factor;
    const void* q;
    void* out_q;
    int64_t q_tok_stride, q_head_stride, out_q_tok_stride, out_q_head_stride;
    int32_t num_heads_q, num_heads_k;
    const void* k;
    void* out_k;
    int64_t k_tok_stride, k_head_stride;
    const float* inv_freq;
    const float* angle_table;
    int64_t table_rows, table_batch_stride;
    const void* cs_table;
    const int32_t* positions;
    const int32_t* position_ids;
    int32_t position;
    int32_t norm_dtype;
    const void* q_norm;
    const void* k_norm;
    float norm_eps, norm_constant_bias;
    int32_t rotate, page_size;
    const void* q_post_scale;
    const void* k_post_scale;
    const void* v_post_scale;
    const void* v;
    int64_t v_tok_stride, v_head_stride;
    void* k_cache;
    void* v_cache;
    int64_t num_pages, max_blocks_per_seq;
    const int32_t* block_table;
    const int32_t* cache_seqlens;
    int32_t* err_flag;
} exl3r_rope_desc;

EXL3R_API int exl3r_rope_run(const exl3r_rope_desc* d, void* stream);

/*
 * Row argmax of logits [rows, vocab] (row stride ld elements; F16/BF16/F32) into int64 ids[rows]:
 * the first index of the row maximum among indices < max_logit (max_logit <= 0 or > vocab: the whole
 * row), NaN counting as the maximum (the first NaN wins), -0 equal to +0 (torch.argmax's rule).
 * Replaces exl3_shim_argmax_sample (csrc/exl3_shim.cpp:229-231 -> kernels/generator/sampling_basic.cu:
 * 65-92, 151-172; for an odd max_logit its pairwise mask, 57-60, also drops index max_logit - 1;
 * here the mask is exact)
 * and the generator's batched tch argmax (src/generator.rs:1596).  ids must be 8-byte aligned.  Below
 * 128 rows ids is the reduction slot during the call (three launches on `stream`); from 128 rows a
 * single launch writes it directly.
 */
EXL3R_API int exl3r_argmax_sample(const void* logits, int dtype, int64_t rows, int64_t vocab, int64_t ld,
                        int max_logit, int64_t* ids, void* stream);

/*
 * Gumbel-max categorical draw: ids[r] = the exl3r_argmax_sample index (same rule and mask) of
 * fl32(logits[r, c] + g(random, r, c)), so that index i is drawn with probability
 * softmax(logits[r, :max_logit])_i.  Replaces exl3_shim_gumbel_sample (csrc/exl3_shim.cpp:232-234 ->
 * kernels/generator/sampling_basic.cu:94-128, 174-197).  The noise is Gumbel(0, 1) from this
 * library's own stream, a function of (random, r, c) only:
 *   bits = Philox4x32-10(counter {c >> 2, r mod 2^32, r >> 32, 0}, key {random, 0}), word c & 3
 *   u = ((bits >> 9) + 0.5) * 2^-23,  g = -log(-log(u))  (fp32, finite: -2.82 < g < 16.64)
 * The reference draws from cuRAND's Philox stream instead; draws agree in distribution, not in bits.
 */
EXL3R_API int exl3r_gumbel_sample(const void* logits, int dtype, int64_t rows, int64_t vocab, int64_t ld,
                        int max_logit, uint32_t random, int64_t* ids, void* stream);

/*
 * exl3r_argmax_sample / exl3r_gumbel_sample in one launch below 128 / 384 rows (decode batches): each
 * slice's workgroup folds its key into the row's slot in the workspace and the last one to finish a
 * row writes the index, instead of three launches through the ids slot.  Same rule, mask and noise;
 * the ids are identical.  workspace: exl3r_sample_workspace_bytes() bytes of device memory (row
 * counters and row slots for up to 384 rows), 256-byte aligned and zero before its first use; every
 * completed call leaves it zero again, so a workspace is cleared once, when it is allocated.  Calls
 * that share a workspace must not overlap (one stream, or ordered by events).  From 128 / 384 rows
 * the workgroup-per-row kernel runs and the workspace is not touched.  Same call sites as
 * exl3r_argmax_sample (src/generator.rs:1596) and exl3r_gumbel_sample (ffi.rs:526-530), for callers
 * that keep a workspace per stream.
 */
EXL3R_API size_t exl3r_sample_workspace_bytes(void);
EXL3R_API int exl3r_argmax_sample_ws(const void* logits, int dtype, int64_t rows, int64_t vocab, int64_t ld,
                        int max_logit, int64_t* ids, void* workspace, size_t workspace_bytes, void* stream);
EXL3R_API int exl3r_gumbel_sample_ws(const void* logits, int dtype, int64_t rows, int64_t vocab, int64_t ld,
                        int max_logit, uint32_t random, int64_t* ids, void* workspace,
                        size_t workspace_bytes, void* stream);

/*
 * exl3r_argmax_sample_ws without a workspace argument: the library's own scratch, a fixed
 * exl3r_sample_workspace_bytes()-byte array per GPU (384 rows) held until the process ends, serves as
 * the workspace, so the call allocates nothing, ever: no hipMalloc, hipFree or allocating library
 * routine (the device address is looked up once per device, on the first call with it current).
 * No counterpart in the reference: it is for callers that cannot allocate (code under HIP graph
 * capture, tight serving loops, harnesses that forbid allocation).  The ids equal
 * exl3r_argmax_sample's.  Calls that overlap on one GPU (several streams, or several graph replays in
 * flight) share the scratch and race; a call that would need more rows of it than it holds is
 * refused with EXL3R_EINVAL (below 128 rows the sliced kernel runs; from 128 the workgroup-per-row
 * kernel, which needs no scratch).
 */
EXL3R_API int exl3r_argmax_sample_noalloc(const void* logits, int dtype, int64_t rows, int64_t vocab, int64_t ld,
                        int max_logit, int64_t* ids, void* stream);

/*
 * out[r, c] = x[r, c] + g(random, r, c) over every column (the noise of exl3r_gumbel_sample), rounded
 * once to out_dtype; out may be x.  x and out: [rows, cols], row strides ldx / ldo elements,
 * F16/BF16/F32.  With an F32 out, exl3r_argmax_sample of out equals exl3r_gumbel_sample of x.
 * Replaces exl3_shim_gumbel_noise_f32 (csrc/exl3_shim.cpp:235-237 -> kernels/generator/gumbel.cu:
 * 44-62, 114-137), which adds noise over the flattened tensor.
 */
EXL3R_API int exl3r_gumbel_noise(const void* x, int x_dtype, int64_t ldx, void* out, int out_dtype, int64_t ldo,
                       int64_t rows, int64_t cols, uint32_t random, void* stream);

/*
 * Random-Hadamard row transform: every 128-element block of each row of x [rows, cols]
 * (cols % 128 == 0, row strides ldx / ldo elements) becomes r * H128 (x o pre_scale) o post_scale,
 * H128 the Sylvester Hadamard matrix, r = scale / sqrt(128) in fp32; out may equal x.  dtype F16 or
 * F32 (x and out alike); pre_scale / post_scale are f16 [cols] (EXL3's suh / svh) or NULL, and at most
 * one of them is given (the reference silently drops post_scale when both are).  Rounding follows
 * kernels/quant/hadamard_inner.cuh:96-200: an f16 pre-scale product is a half multiply, the transform
 * is an fp32 butterfly over index bits 0..6 in order, the result times r is rounded once, an f16
 * post-scale is a half multiply.  Replaces exl3_shim_had_r_128 (csrc/exl3_shim.cpp:158-160 ->
 * had_r_128, kernels/quant/hadamard.cu:88-170).
 */
EXL3R_API int exl3r_had_r_128(const void* x, int dtype, int64_t ldx, void* out, int64_t ldo, int64_t rows,
                    int64_t cols, const void* pre_scale, const void* post_scale, float scale, void* stream);

/*
 * exl3r_had_r_128 with the 128-point transform on the matrix cores (v_mfma_f32_16x16x32_f16 against
 * +-1 f16 operands, fp32 sums): the transform the fused Hadamard entry points use unless
 * EXL3R_HAD_EXACT.  Same arguments, dtype F16 only, same pre / post-scale roundings.  The sums are
 * grouped differently from the reference's butterfly, so each f16 result is exl3r_had_r_128's or its
 * f16 neighbour, or within 2^-17 * r * sum|input| of it where the transform cancels (r = scale /
 * sqrt(128), the sum over the 128 pre-scaled inputs of the block); zero results are +0.  Rows that
 * are not 16-byte aligned run exl3r_had_r_128.  No counterpart in the reference (same call site,
 * src/modules.rs:224-231, for callers that take the tolerance for the speed).
 */
EXL3R_API int exl3r_had_r_128_mfma(const void* x, int dtype, int64_t ldx, void* out, int64_t ldo, int64_t rows,
                    int64_t cols, const void* pre_scale, const void* post_scale, float scale, void* stream);

/*
 * RMSNorm whose f16 output feeds the random-Hadamard input rotation of 1..4 EXL3 projections, in one
 * pass (the prefill path of RmsNorm::forward / forward_res, src/modules.rs:372-411, then
 * had_r_128(y, suh) per projection, src/modules.rs:224-227):
 *   r == NULL: y = RMSNorm(x) as exl3r_rms_norm; else r += x in place and y = RMSNorm(r) as
 *              exl3r_rms_norm_res_in; y is f16 and written only when y != NULL (row stride ldy);
 *   outs[i] = had_r_128(y, pre_scales[i]) with scale had_scale, f16 [rows, dim] at row stride ldo;
 *              pre_scales[i] is f16 [dim] (the projection's suh) or NULL.
 *   rotate_x = 1: x (f16, the raw output of the previous EXL3 projection) is first replaced by that
 *              projection's output rotation had_r_128(x, x, NULL, x_post_scale, 1.0)
 *              (src/modules.rs:231; x_post_scale is its f16 [dim] svh, or NULL); x is not written.
 *              | EXL3R_HAD_EXACT: see below.
 * dim % 128 == 0; n_out in 1..4; outputs alias nothing.  The transforms run on the matrix cores, as
 * exl3r_had_r_128_mfma: each result is the unfused calls' (exl3r_had_r_128) or its f16 neighbour, or
 * within 2^-17 * r * sum|input| of it where the transform cancels.  With EXL3R_HAD_EXACT in rotate_x
 * the transforms are the reference's butterfly and the results are bit-identical to the unfused
 * calls.  Rows that are not 16-byte aligned run the unfused calls (the rotated x and the norm go to y
 * or to outs[0]).
 */
EXL3R_API int exl3r_rms_norm_had(const void* x, int x_dtype, int64_t ldx, const void* w, int w_dtype,
                       void* r, int r_dtype, int64_t ldr, void* y, int64_t ldy,
                       int n_out, const void* const* pre_scales, void* const* outs, int64_t ldo,
                       int64_t rows, int64_t dim, float eps, float constant_bias, float constant_scale,
                       float had_scale, int rotate_x, const void* x_post_scale, void* stream);

/*
 * Gated activation whose f16 output feeds the random-Hadamard input rotation of the next EXL3
 * projection, in one pass (GatedMlp::forward's silu_mul -> down_proj, src/modules.rs:932-940, and the
 * Qwen3.5 attention gate -> o_proj; then had_r_128(z, suh), src/modules.rs:224-227):
 *   z   = act(x, y) as exl3r_silu_mul / exl3r_gelu_mul / exl3r_mul_sigmoid with an f16 z
 *         (act = EXL3R_ACT_*; act_limit as exl3r_silu_mul, 0 for EXL3R_ACT_MUL_SIGMOID), written
 *         only when z != NULL (row stride ldz);
 *   out = had_r_128(z, pre_scale) with scale had_scale: f16 [rows, cols], row stride ldo;
 *         pre_scale is f16 [cols] (the projection's suh) or NULL.
 *   rotate_in: bit 0 / bit 1 -- x / y (f16, the raw output of an EXL3 projection: gate_proj and up_proj
 *         in the MLP) is first given that projection's output rotation had_r_128(v, v, NULL, post, 1.0)
 *         (src/modules.rs:231) with post = x_post_scale / y_post_scale (f16 [cols] svh, or NULL); x and y
 *         are not written.  Needs 16-byte aligned rows.  | EXL3R_HAD_EXACT: see below.
 * x, y: [rows, cols] of in_dtype (F16/BF16/F32), row strides ldx, ldy; cols % 128 == 0; out and z
 * alias nothing.  Rows that are not 16-byte aligned run the unfused calls.
 * The 128-point transforms run on the matrix cores (v_mfma_f32_16x16x32_f16: f16 operands, fp32
 * sums grouped differently from the reference's butterfly).  Each f16 result of a transform is then
 * the unfused call's result or its f16 neighbour, or within 2^-17 * r * sum|input| of it where the
 * transform cancels (r = had_scale / sqrt(128), the sum over the 128 inputs of the block); zero
 * results are +0.  With EXL3R_HAD_EXACT in rotate_in the transforms are the reference's fp32 butterfly
 * and the results are bit-identical to the unfused calls.
 */
EXL3R_API int exl3r_act_mul_had(int act, const void* x, const void* y, int in_dtype, int64_t ldx, int64_t ldy,
                      void* z, int64_t ldz, const void* pre_scale, void* out, int64_t ldo,
                      int64_t rows, int64_t cols, float act_limit, float had_scale, int rotate_in,
                      const void* x_post_scale, const void* y_post_scale, void* stream);

/*
 * Token-embedding gather: out[i, :] = table[ids[i], :], bit-exact (same dtype) or exactly upcast to
 * F32.  Replaces Embedding::forward's index_select + to_kind(Float) (src/modules.rs:430-436).
 *   table: [vocab, hidden], row stride ldt, F16/BF16/F32.
 *   ids:   [n] I32 or I64, device.
 *   out:   [n, hidden], row stride ldo; dtype == table dtype, or F32.
 *   err_flag: NULL or an int32 in device memory; a row whose id is outside [0, vocab) is written as
 *             zeros and 1 is stored to *err_flag (never cleared by the kernel).
 */
EXL3R_API int exl3r_embedding(const void* table, int table_dtype, int64_t vocab, int64_t hidden, int64_t ldt,
                    const void* ids, int ids_dtype, int64_t n,
                    void* out, int out_dtype, int64_t ldo,
                    int32_t* err_flag, void* stream);

/*
 * Embedding gather fused with the RMSNorm that follows it (src/mtp.rs:189-190 applies
 * pre_fc_norm_embedding to embed(t)):
 *   h[i, :] = table[ids[i], :]   (optional output, exact as exl3r_embedding; h == NULL skips it)
 *   y[i, :] = RMSNorm(h[i, :]) with weight w (NULL: none), eps, constant_bias, constant_scale.
 */
EXL3R_API int exl3r_embedding_rms_norm(const void* table, int table_dtype, int64_t vocab, int64_t hidden, int64_t ldt,
                             const void* ids, int ids_dtype, int64_t n,
                             void* h, int h_dtype, int64_t ldh,
                             const void* w, int w_dtype,
                             void* y, int y_dtype, int64_t ldy,
                             float eps, float constant_bias, float constant_scale,
                             int32_t* err_flag, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* EXL3R_ROWOPS_H */
