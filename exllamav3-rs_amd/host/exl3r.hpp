// exl3r host layer: the C++ counterpart of the reference's Rust side for the fused row ops.
//
// The reference binds its kernels through `src/ffi.rs` (safe wrappers over `extern "C"` shim
// functions taking tch tensors) and calls them from `src/modules.rs` / `src/rope.rs`.  This layer
// keeps those names and argument meanings over the pointer/shape/stride C ABI of
// include/exl3r/rowops.h, with a small HIP device-buffer/stream type in place of tch:
//
//   exl3r::ffi::rms_norm / rms_norm_res_in / silu_mul / gelu_mul / rope  <- src/ffi.rs:293-333, 464-503
//   exl3r::ffi::gated_rms_norm / mul_sigmoid_ / deinterleave_qg          <- src/ffi.rs:479-483, 616-624
//   exl3r::ffi::rope_paged_kv                                            <- rope + paged append, src/modules.rs:666-704
//   exl3r::ffi::argmax_sample / gumbel_sample / gumbel_noise             <- src/ffi.rs:521-535, src/generator.rs:1596
//   exl3r::ffi::had_r_128 / rms_norm_had / act_mul_had / rope_had        <- src/ffi.rs:606-607, src/modules.rs:224-231
//   exl3r::ffi::rope_cs_table / rope_cs                                  <- rope() with the sin / cos hoisted per forward
//   exl3r::ffi::rope_qg                                                  <- deinterleave_qg + rope, src/modules.rs:637-681
//   exl3r::ffi::embedding                                                <- index_select, src/modules.rs:430-436
//   exl3r::RmsNorm::forward / forward_res                                <- src/modules.rs:342-412
//   exl3r::Embedding::forward                                            <- src/modules.rs:418-437
//   exl3r::GatedMlp::activate                                            <- src/modules.rs:932-940 (silu_mul step)
//   exl3r::RoPE (params of every rope_type, apply, apply_one, apply_paged) <- src/rope.rs:33-220, 225-292, 309-317
//
// Error behaviour: the reference panics / throws (TORCH_CHECK) on invalid input; here every failure
// throws exl3r::Error carrying the C ABI status and message.  Kernels are enqueued on the given
// Stream; nothing here synchronises except the explicit host copies.
#pragma once

#include <hip/hip_runtime_api.h>

#include <cstddef>
#include <cstdint>
#include <stdexcept>
#include <string>
#include <vector>

#include "../../include/exl3r/rowops.h"

namespace exl3r {

enum class DType : int { F32 = EXL3R_F32, F16 = EXL3R_F16, BF16 = EXL3R_BF16, I32 = EXL3R_I32, I64 = EXL3R_I64 };
enum class RopeStyle : int { None = EXL3R_ROPE_NONE, GptJ = EXL3R_ROPE_GPTJ, NeoX = EXL3R_ROPE_NEOX };

size_t dtype_size(DType dt);

class Error : public std::runtime_error
{
public:
    Error(int code, const std::string& what) : std::runtime_error(what), code_(code) {}
    int code() const { return code_; }

private:
    int code_;
};

// Owning HIP stream (default priority).  Stream() wraps the null stream.
class Stream
{
public:
    Stream() = default;
    static Stream create();
    ~Stream();
    Stream(Stream&& o) noexcept;
    Stream& operator=(Stream&& o) noexcept;
    Stream(const Stream&) = delete;
    Stream& operator=(const Stream&) = delete;
    hipStream_t get() const { return s_; }
    void synchronize() const;

private:
    hipStream_t s_ = nullptr;
    bool owned_ = false;
};

// Owning device allocation (hipMalloc / hipFree).
class DeviceBuffer
{
public:
    DeviceBuffer() = default;
    explicit DeviceBuffer(size_t bytes);
    ~DeviceBuffer();
    DeviceBuffer(DeviceBuffer&& o) noexcept;
    DeviceBuffer& operator=(DeviceBuffer&& o) noexcept;
    DeviceBuffer(const DeviceBuffer&) = delete;
    DeviceBuffer& operator=(const DeviceBuffer&) = delete;
    void* data() const { return p_; }
    size_t bytes() const { return n_; }
    void upload(const void* host, size_t bytes, const Stream& s);     // async H2D, then stream sync
    void download(void* host, size_t bytes, const Stream& s) const;   // async D2H, then stream sync

private:
    void* p_ = nullptr;
    size_t n_ = 0;
};

// Non-owning strided view of device memory (the role tch::Tensor plays at the reference's FFI).
// Strides are in elements; the innermost dimension must be dense for every op here.
struct Tensor
{
    void* data = nullptr;
    DType dtype = DType::F16;
    std::vector<int64_t> shape;
    std::vector<int64_t> strides;

    Tensor() = default;
    Tensor(void* d, DType t, std::vector<int64_t> shp);                              // contiguous
    Tensor(void* d, DType t, std::vector<int64_t> shp, std::vector<int64_t> str);    // strided
    int64_t numel() const;
    int dim() const { return (int)shape.size(); }
    int64_t size(int i) const { return shape[i < 0 ? i + dim() : i]; }
    int64_t stride(int i) const { return strides[i < 0 ? i + dim() : i]; }
    bool is_contiguous() const;
    // View as [rows, last] with one row stride (throws if the leading dims do not collapse).
    void rows_view(int64_t& rows, int64_t& cols, int64_t& ld) const;
};

// Tensor with its own storage (one hipMalloc; for weights and long-lived buffers, not per-call outputs).
struct OwnedTensor
{
    DeviceBuffer buf;
    Tensor t;
    static OwnedTensor empty(DType dt, std::vector<int64_t> shape);
};

// Device memory for module outputs, reserved once (one hipMalloc at construction) and handed out by
// bumping an offset (256-byte aligned): a module call then allocates, frees and synchronises nothing, so
// it can run inside a captured HIP graph or a tight decode loop.  This is the role tch's caching
// allocator plays for the reference's modules (src/modules.rs:376, 400, 937 take `empty_like` outputs).
// reset() hands the whole arena out again: the caller resets once no earlier output is read any more
// (after each decode step, say).  An arena is not thread-safe.
class Arena
{
public:
    explicit Arena(size_t bytes);
    // A contiguous tensor of `shape` carved from the arena; throws exl3r::Error (EXL3R_EINVAL) when it
    // does not fit.
    Tensor empty(DType dt, std::vector<int64_t> shape);
    void reset() { off_ = 0; }
    size_t used() const { return off_; }
    size_t capacity() const { return buf_.bytes(); }

private:
    DeviceBuffer buf_;
    size_t off_ = 0;
};

namespace ffi {

// src/ffi.rs:293-296: y = RMSNorm(x) over the last dim; w may be null.
void rms_norm(const Tensor& x, const Tensor* w, const Tensor& y, float eps, float constant_bias,
              float constant_scale, const Stream& s);
// src/ffi.rs:464-468: r += x (in place, rounded to r's dtype), y = RMSNorm(r).
void rms_norm_res_in(const Tensor& x, const Tensor* w, const Tensor& y, const Tensor& r, float eps, float bias,
                     float scale, const Stream& s);
// src/ffi.rs:492-499: z = act(x) * y; act_limit 0 disables clamping.
void silu_mul(const Tensor& x, const Tensor& y, const Tensor& z, float act_limit, const Stream& s);
void gelu_mul(const Tensor& x, const Tensor& y, const Tensor& z, float act_limit, const Stream& s);
// src/ffi.rs:479-483: y = RMSNorm(x) * (w + bias) * act(g), or RMSNorm(x * act(g)) * (w + bias) with
// gate_first; act = silu (gate_act 0) or sigmoid (1); w may be null or hold w_groups rows of dim.
void gated_rms_norm(const Tensor& x, const Tensor* w, const Tensor& y, const Tensor& g, float eps, float bias,
                    int w_groups, bool gate_first, int gate_act, const Stream& s);
// gated_rms_norm into an f16 y (optional) that feeds o_proj's input rotation: out = had_r_128(y, pre_scale)
// (src/qwen3_5.rs:208-214 -> src/modules.rs:224-227), one pass.
// Norm row r uses pre_scale[(r % pre_rows) * dim ..] (rows = tokens * heads of head_dim: pre_rows = heads).
// Rows of 128 run the transform on the matrix cores; exact: the reference's butterfly (EXL3R_HAD_EXACT).
void gated_rms_norm_had(const Tensor& x, const Tensor* w, const Tensor& g, const Tensor& out, const Tensor* y,
                        const Tensor* pre_scale, float eps, float bias, int w_groups, bool gate_first, int gate_act,
                        float had_scale, const Stream& s, int pre_rows = 1, bool exact = false);
// src/ffi.rs:616-618: x *= sigmoid(y), in place.
void mul_sigmoid_(const Tensor& x, const Tensor& y, const Stream& s);
// src/ffi.rs:622-624: split [.., heads * 2 * head_dim] interleaved (q | g) rows into q [.., heads, head_dim] and
// g [.., heads * head_dim].
void deinterleave_qg(const Tensor& qg, const Tensor& q, const Tensor& g, int64_t head_dim, const Stream& s);
// src/ffi.rs:298-333: fused (optional) q/k head RMSNorm + RoPE on (bsz, seq, heads, head_dim)
// tensors; positions (int32 [bsz]) or position_ids (int32 [bsz, seq]) override position.  As in the
// reference (rope.cu:340-347), a 2-D [max_pos, R/2] (shared by every sequence) or 3-D
// [bsz, max_pos, R/2] inv_freq is a table of precomputed angles; a position outside it stores 1 to
// err_flag (device int32) when given.
void rope(const Tensor& q, const Tensor& out_q, const Tensor* k, const Tensor* out_k, const Tensor& inv_freq,
          int64_t position, const Tensor* positions, const Tensor* q_norm, const Tensor* k_norm, float norm_eps,
          float norm_constant_bias, RopeStyle rope_mode, float attn_factor, const Stream& s,
          const Tensor* position_ids = nullptr, int32_t* err_flag = nullptr);
// deinterleave_qg() then rope() on its q in one pass (gated attention, src/modules.rs:637-646 then 669-681):
// qg (bsz, seq, heads, 2 * head_dim) holds each head's [q | g]; out_q (bsz, seq, heads, head_dim) dense gets
// the roped q.  The gate stays in qg for mul_sigmoid_ with a row stride of 2 * head_dim.
void rope_qg(const Tensor& qg, const Tensor& out_q, const Tensor* k, const Tensor* out_k, const Tensor& inv_freq,
             int64_t position, const Tensor* positions, const Tensor* q_norm, const Tensor* k_norm, float norm_eps,
             float norm_constant_bias, RopeStyle rope_mode, float attn_factor, const Stream& s,
             const Tensor* position_ids = nullptr);
// {cos, sin} * attn_factor of every token's rotary frequencies into cs_table (float32 [bsz * seq, R/2, 2]),
// as rope() evaluates them for the same positions: built once per forward pass for every layer's rope_cs()
// (the reference evaluates them in each layer's kernel, kernels/rope.cu:69-85).
void rope_cs_table(int64_t bsz, int64_t seq_len, const Tensor& inv_freq, int64_t position, const Tensor* positions,
                   const Tensor* position_ids, float attn_factor, const Tensor& cs_table, const Stream& s);
// rope() with the rotary pairs read from a rope_cs_table() of the same positions: bit-identical to rope().
void rope_cs(const Tensor& q, const Tensor& out_q, const Tensor* k, const Tensor* out_k, const Tensor& cs_table,
             const Tensor* q_norm, const Tensor* k_norm, float norm_eps, float norm_constant_bias, RopeStyle rope_mode,
             const Stream& s);
// rope_had, rope_paged_kv and rope_paged_kv_had take an optional cs_table (a rope_cs_table() of the same
// positions) that the kernels read in place of evaluating sin / cos; the results are the same bits.
// rope() on the raw f16 outputs of the q / k projections (heads packed), each first given its projection's
// output rotation had_r_128(y, y, None, svh) (src/modules.rs:231); q_post_scale / k_post_scale are the
// projections' f16 svh or null.
void rope_had(const Tensor& q, const Tensor& out_q, const Tensor* k, const Tensor* out_k, const Tensor& inv_freq,
              int64_t position, const Tensor* positions, const Tensor* q_norm, const Tensor* k_norm, float norm_eps,
              float norm_constant_bias, RopeStyle rope_mode, float attn_factor, const Tensor* q_post_scale,
              const Tensor* k_post_scale, const Stream& s, const Tensor* position_ids = nullptr,
              const Tensor* cs_table = nullptr, bool exact = false);
// rope_paged_kv() on the raw f16 outputs of the q / k / v projections (heads packed), each first given its
// projection's output rotation had_r_128(y, y, None, svh); outside the fused launch v (and k without out_k)
// are rotated in place.  (rope_had and rope_paged_kv_had: the fused launch runs the transforms on the
// matrix cores; exact: the reference's butterfly, EXL3R_HAD_EXACT.)
void rope_paged_kv_had(const Tensor& q, const Tensor& out_q, const Tensor& k, const Tensor* out_k, const Tensor& v,
                       const Tensor& inv_freq, int64_t position, const Tensor* positions, const Tensor* q_norm,
                       const Tensor* k_norm, float norm_eps, float norm_constant_bias, RopeStyle rope_mode,
                       float attn_factor, const Tensor& k_cache, const Tensor& v_cache, const Tensor& block_table,
                       const Tensor& cache_seqlens, int32_t* err_flag, const Tensor* q_post_scale,
                       const Tensor* k_post_scale, const Tensor* v_post_scale, const Stream& s,
                       const Tensor* cs_table = nullptr, bool exact = false);
// rope() fused with the paged KV-cache append that follows it in paged attention (src/modules.rs:666-704,
// ffi.rs:337-350): the roped k (also written to out_k when given) and v go to k_cache / v_cache
// [pages, page_size, kv_heads, head_dim] at cache_seqlens[b] + s through block_table [bsz, max_blocks].
void rope_paged_kv(const Tensor& q, const Tensor& out_q, const Tensor& k, const Tensor* out_k, const Tensor& v,
                   const Tensor& inv_freq, int64_t position, const Tensor* positions, const Tensor* q_norm,
                   const Tensor* k_norm, float norm_eps, float norm_constant_bias, RopeStyle rope_mode, float attn_factor,
                   const Tensor& k_cache, const Tensor& v_cache, const Tensor& block_table, const Tensor& cache_seqlens,
                   int32_t* err_flag, const Stream& s, const Tensor* cs_table = nullptr);
// src/ffi.rs:521-525 (and the generator's batched argmax, src/generator.rs:1596): ids[i] = first index of the
// maximum of logits[i, :max_logit] (whole row when max_logit <= 0), NaN maximal; ids int64 [rows].
void argmax_sample(const Tensor& logits, const Tensor& ids, int max_logit, const Stream& s);
// src/ffi.rs:526-530: a draw from softmax(logits[i, :max_logit]) per row (Gumbel-max over this library's
// Philox4x32-10 stream keyed by `random`); ids int64 [rows].
void gumbel_sample(const Tensor& logits, const Tensor& ids, int max_logit, uint32_t random, const Stream& s);
// argmax_sample / gumbel_sample in one launch below 128 / 384 rows, with a workspace of
// exl3r_sample_workspace_bytes() bytes (zero before its first use, left zero by every call; one per
// stream): the same ids.
void argmax_sample_ws(const Tensor& logits, const Tensor& ids, int max_logit, const DeviceBuffer& workspace,
                      const Stream& s);
void gumbel_sample_ws(const Tensor& logits, const Tensor& ids, int max_logit, uint32_t random,
                      const DeviceBuffer& workspace, const Stream& s);
// src/ffi.rs:531-535: out = x + the Gumbel noise gumbel_sample adds (out may be x).
void gumbel_noise(const Tensor& x, const Tensor& out, uint32_t random, const Stream& s);
// src/ffi.rs:606-607: the EXL3 linear's random-Hadamard rotation of [rows, cols] f16 / f32 x into out
// (cols % 128 == 0; out may be x), with an optional f16 [cols] pre_scale (suh) or post_scale (svh).
void had_r_128(const Tensor& x, const Tensor& out, const Tensor* pre_scale, const Tensor* post_scale, float scale,
               const Stream& s);
// RMSNorm (r == nullptr) or residual RMSNorm (r += x) whose f16 output feeds had_r_128(y, pre_scales[i]) of
// 1..4 projections (src/modules.rs:372-411 then 224-227), in one pass; outs are f16 like x; y (f16) is
// written only when given; pre_scales[i] may be null.  rotate_x: f16 x is first taken through its
// producer's output rotation had_r_128(x, post_scale = x_post_scale) (src/modules.rs:231).
// The transforms run on the matrix cores; exact: the reference's butterfly (EXL3R_HAD_EXACT).
void rms_norm_had(const Tensor& x, const Tensor* w, const Tensor* r, const Tensor* y,
                  const std::vector<const Tensor*>& outs, const std::vector<const Tensor*>& pre_scales, float eps,
                  float constant_bias, float constant_scale, float had_scale, const Stream& s,
                  bool rotate_x = false, const Tensor* x_post_scale = nullptr, bool exact = false);
// Gated activation whose f16 output feeds the next projection's had_r_128(z, pre_scale)
// (src/modules.rs:932-940 then 224-227): silu(x) * y, gelu(x) * y or x * sigmoid(y); z kept when given.
enum class HadAct : int { Silu = EXL3R_ACT_SILU, Gelu = EXL3R_ACT_GELU, MulSigmoid = EXL3R_ACT_MUL_SIGMOID };
// rotate_x / rotate_y: the f16 input is first given its projection's output rotation (post-scale x_post /
// y_post, or none).
// The transforms run on the matrix cores; exact: the reference's butterfly (EXL3R_HAD_EXACT).
void act_mul_had(HadAct act, const Tensor& x, const Tensor& y, const Tensor& out, const Tensor* pre_scale,
                 const Tensor* z, float act_limit, float had_scale, const Stream& s, bool rotate_x = false,
                 bool rotate_y = false, const Tensor* x_post = nullptr, const Tensor* y_post = nullptr,
                 bool exact = false);
// Embedding gather: out[i] = table[ids[i]] (bit-exact, or exact upcast to f32); err_flag optional.
void embedding(const Tensor& table, const Tensor& ids, const Tensor& out, int32_t* err_flag, const Stream& s);
// Gather fused with the following RMSNorm; h optional.
void embedding_rms_norm(const Tensor& table, const Tensor& ids, const Tensor* h, const Tensor* w, const Tensor& y,
                        float eps, float constant_bias, float constant_scale, int32_t* err_flag, const Stream& s);

}  // namespace ffi

// src/modules.rs:342-412.  No call allocates: the output comes from an Arena or from the caller.
class RmsNorm
{
public:
    RmsNorm(Tensor weight, float eps, float constant_bias = 0.0f, float constant_scale = 1.0f)
        : weight_(std::move(weight)), eps_(eps), constant_bias_(constant_bias), constant_scale_(constant_scale) {}
    // y = norm(x) in f16 (every call site in the Qwen3 tree), same shape as x.
    Tensor forward(const Tensor& x, Arena& arena, const Stream& s) const;
    void forward_into(const Tensor& x, const Tensor& y, const Stream& s) const;
    // Pre-norm residual add fused with the norm: r += add (in place), returns norm(r) in f16.
    // add == nullptr: plain forward(r).  A residual that is not contiguous takes the reference's
    // unfused path (src/modules.rs:393-395): y = norm(r + add) and r is left unchanged.  r + add is
    // then formed in `scratch` (contiguous, r's dtype and shape; from the arena in forward_res): r is
    // copied into it (2-D copies, no allocation) and the fused kernel updates the copy instead of r.
    // Such a residual needs a dense last dim.
    Tensor forward_res(const Tensor& r, const Tensor* add, Arena& arena, const Stream& s) const;
    void forward_res_into(const Tensor& r, const Tensor* add, const Tensor& y, const Stream& s,
                          const Tensor* scratch = nullptr) const;
    const Tensor& weight() const { return weight_; }

private:
    Tensor weight_;
    float eps_, constant_bias_, constant_scale_;
};

// src/modules.rs:418-437: f32 rows out of an f16/bf16 table (the residual stream is f32).
class Embedding
{
public:
    explicit Embedding(Tensor weight, DType out_kind = DType::F32) : weight_(std::move(weight)), out_kind_(out_kind) {}
    // ids: [b, s] int64 -> [b, s, hidden] of out_kind (from the arena, or into the caller's out).
    Tensor forward(const Tensor& ids, Arena& arena, const Stream& s) const;
    void forward_into(const Tensor& ids, const Tensor& out, const Stream& s) const;

private:
    Tensor weight_;
    DType out_kind_;
};

// The activation step of src/modules.rs:932-940 (gate/up/down Linear layers are outside this path).
struct GatedMlp
{
    enum class Act { Silu, Gelu };
    // a = act(g) * u, same shape and dtype as g (from the arena, or into the caller's a).
    static Tensor activate(const Tensor& g, const Tensor& u, Act act, float act_limit, Arena& arena, const Stream& s);
    static void activate_into(const Tensor& g, const Tensor& u, const Tensor& a, Act act, float act_limit,
                              const Stream& s);
};

// src/rope.rs:33-86, 233-292, 309-317: inv_freq producer (default and linear scaling) and the
// in-place apply / apply_one.
// config.json rope_scaling (src/rope.rs:15-26, 45-67): the rope_type and the fields its producer reads.
struct RopeScaling
{
    enum class Type { Default, Linear, Llama3, Yarn, LongRope, Proportional };
    Type type = Type::Default;
    double factor = 0.0;                       // 0: absent (linear, yarn, proportional 1; llama3 8)
    double low_freq_factor = 1.0;              // llama3
    double high_freq_factor = 4.0;             // llama3
    double original_max_position_embeddings = 0.0;  // llama3 (8192 when 0), yarn, longrope
    int64_t max_position_embeddings = 0;       // yarn, longrope
    double beta_fast = 32.0, beta_slow = 1.0;  // yarn
    bool truncate = true;                      // yarn
    bool has_attention_factor = false;         // yarn: attention_factor given
    double attention_factor = 1.0;
    std::vector<double> long_factor, short_factor;   // longrope: one factor per frequency
    int head_dim = 0;                          // proportional
    double partial_rotary_factor = 1.0;        // proportional
};

class RoPE
{
public:
    struct Params
    {
        std::vector<float> inv_freq;
        double attn_factor;
    };
    // inv_freq and attn_factor of every rope_type the reference knows (RoPE::new, src/rope.rs:45-67;
    // default / mrope 82-86, linear 55-59, llama3 88-108, proportional 110-131, yarn 133-191,
    // longrope 193-220).  rotary_dim is ignored by "proportional", which spans head_dim with zero
    // frequencies past partial_rotary_factor.  Throws exl3r::Error on a missing or invalid field.
    static Params params(double theta, int rotary_dim, const RopeScaling& sc);
    RoPE(double theta, int rotary_dim, RopeStyle style, const RopeScaling& sc);
    // inv_freq[i] = 1 / exp((2i / rotary_dim) * ln(theta)) in fp32 (rope.rs:39-42, 82-86, 309-317),
    // divided by `linear_factor` for rope_type "linear" (rope.rs:55-59).
    RoPE(double theta, int rotary_dim, RopeStyle style, double attn_factor = 1.0, double linear_factor = 1.0);
    static std::vector<float> default_inv_freq(double theta, int rotary_dim, double linear_factor = 1.0);
    // freq_table: optional [max_pos, rotary_dim/2] f32 precomputed angles used in place of inv_freq
    // (rope.rs:225-260: MRoPE, the vision tower's 2-D RoPE).
    void apply(const Tensor& q, const Tensor& k, int64_t position, const Tensor* positions, const Tensor* q_norm,
               const Tensor* k_norm, float norm_eps, float norm_constant_bias, const Stream& s,
               const Tensor* freq_table = nullptr) const;
    void apply_one(const Tensor& x, int64_t position, const Tensor* positions, const Tensor* norm, float norm_eps,
                   float norm_constant_bias, const Stream& s) const;
    // apply() on q and k in place, then k and v appended to the paged caches (one launch); the rotary
    // positions are the cache lengths, as in the paged attention path (src/modules.rs:666-681).
    void apply_paged(const Tensor& q, const Tensor& k, const Tensor& v, const Tensor& k_cache, const Tensor& v_cache,
                     const Tensor& block_table, const Tensor& cache_seqlens, const Tensor* q_norm, const Tensor* k_norm,
                     float norm_eps, float norm_constant_bias, int32_t* err_flag, const Stream& s) const;
    const std::vector<float>& inv_freq_host() const { return inv_freq_host_; }
    int rotary_dim() const { return rotary_dim_; }

private:
    std::vector<float> inv_freq_host_;
    DeviceBuffer inv_freq_;
    Tensor inv_freq_t_;
    int rotary_dim_;
    RopeStyle style_;
    float attn_factor_;
};

}  // namespace exl3r
