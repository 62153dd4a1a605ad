// exl3r host layer implementation (see exl3r.hpp).
#include "exl3r.hpp"

#include <cmath>
#include <utility>

namespace exl3r {

namespace {

void check_abi(int rc)
{
    if (rc != EXL3R_OK) throw Error(rc, exl3r_last_error());
}

void check_hip(hipError_t e, const char* what)
{
    if (e != hipSuccess) throw Error((int)e, std::string(what) + ": " + hipGetErrorString(e));
}

void require(bool ok, const std::string& msg)
{
    if (!ok) throw Error(EXL3R_EINVAL, msg);
}

// Literal messages (every check on the launch path): the string is built only when the check fails,
// not on each call.
void require(bool ok, const char* msg)
{
    if (!ok) throw Error(EXL3R_EINVAL, std::string(msg));
}

int code(DType t) { return (int)t; }
int code_or(const Tensor* t, DType dflt) { return t ? (int)t->dtype : (int)dflt; }
const void* ptr(const Tensor* t) { return t ? t->data : nullptr; }

std::vector<int64_t> contiguous_strides(const std::vector<int64_t>& shape)
{
    std::vector<int64_t> st(shape.size());
    int64_t acc = 1;
    for (int i = (int)shape.size() - 1; i >= 0; --i)
    {
        st[i] = acc;
        acc *= shape[i];
    }
    return st;
}

}  // namespace

size_t dtype_size(DType dt)
{
    switch (dt)
    {
        case DType::F32: case DType::I32: return 4;
        case DType::F16: case DType::BF16: return 2;
        case DType::I64: return 8;
    }
    return 0;
}

// ------------------------------------------------------------------------------------------------
// Stream / DeviceBuffer

Stream Stream::create()
{
    Stream s;
    check_hip(hipStreamCreate(&s.s_), "hipStreamCreate");
    s.owned_ = true;
    return s;
}

Stream::~Stream()
{
    if (owned_ && s_) (void)hipStreamDestroy(s_);
}

Stream::Stream(Stream&& o) noexcept : s_(o.s_), owned_(o.owned_)
{
    o.s_ = nullptr;
    o.owned_ = false;
}

Stream& Stream::operator=(Stream&& o) noexcept
{
    if (this != &o)
    {
        if (owned_ && s_) (void)hipStreamDestroy(s_);
        s_ = o.s_;
        owned_ = o.owned_;
        o.s_ = nullptr;
        o.owned_ = false;
    }
    return *this;
}

void Stream::synchronize() const { check_hip(hipStreamSynchronize(s_), "hipStreamSynchronize"); }

DeviceBuffer::DeviceBuffer(size_t bytes) : n_(bytes)
{
    if (bytes) check_hip(hipMalloc(&p_, bytes), "hipMalloc");
}

DeviceBuffer::~DeviceBuffer()
{
    if (p_) (void)hipFree(p_);
}

DeviceBuffer::DeviceBuffer(DeviceBuffer&& o) noexcept : p_(o.p_), n_(o.n_)
{
    o.p_ = nullptr;
    o.n_ = 0;
}

DeviceBuffer& DeviceBuffer::operator=(DeviceBuffer&& o) noexcept
{
    if (this != &o)
    {
        if (p_) (void)hipFree(p_);
        p_ = o.p_;
        n_ = o.n_;
        o.p_ = nullptr;
        o.n_ = 0;
    }
    return *this;
}

void DeviceBuffer::upload(const void* host, size_t bytes, const Stream& s)
{
    require(bytes <= n_, "DeviceBuffer::upload: too many bytes");
    check_hip(hipMemcpyAsync(p_, host, bytes, hipMemcpyHostToDevice, s.get()), "hipMemcpyAsync H2D");
    s.synchronize();
}

void DeviceBuffer::download(void* host, size_t bytes, const Stream& s) const
{
    require(bytes <= n_, "DeviceBuffer::download: too many bytes");
    check_hip(hipMemcpyAsync(host, p_, bytes, hipMemcpyDeviceToHost, s.get()), "hipMemcpyAsync D2H");
    s.synchronize();
}

// ------------------------------------------------------------------------------------------------
// Tensor

Tensor::Tensor(void* d, DType t, std::vector<int64_t> shp) : data(d), dtype(t), shape(std::move(shp))
{
    strides = contiguous_strides(shape);
}

Tensor::Tensor(void* d, DType t, std::vector<int64_t> shp, std::vector<int64_t> str)
    : data(d), dtype(t), shape(std::move(shp)), strides(std::move(str))
{
    require(shape.size() == strides.size(), "Tensor: shape and strides differ in rank");
}

int64_t Tensor::numel() const
{
    int64_t n = 1;
    for (int64_t s : shape) n *= s;
    return n;
}

bool Tensor::is_contiguous() const { return strides == contiguous_strides(shape); }

void Tensor::rows_view(int64_t& rows, int64_t& cols, int64_t& ld) const
{
    require(dim() >= 1, "expected at least a 1-D tensor");
    cols = shape.back();
    require(cols <= 1 || strides.back() == 1, "last dimension must be contiguous");
    rows = 1;
    for (int i = 0; i < dim() - 1; ++i) rows *= shape[i];
    ld = dim() >= 2 ? strides[dim() - 2] : cols;
    // leading dims must collapse into one stride: stride[i] == stride[i+1] * shape[i+1]
    for (int i = 0; i + 2 < dim(); ++i)
        if (shape[i] > 1) require(strides[i] == strides[i + 1] * shape[i + 1], "leading dimensions must collapse to one row stride");
    if (rows <= 1) ld = cols;
}

OwnedTensor OwnedTensor::empty(DType dt, std::vector<int64_t> shape)
{
    OwnedTensor o;
    int64_t n = 1;
    for (int64_t s : shape) n *= s;
    o.buf = DeviceBuffer((size_t)n * dtype_size(dt));
    o.t = Tensor(o.buf.data(), dt, std::move(shape));
    return o;
}

Arena::Arena(size_t bytes) : buf_(bytes) {}

Tensor Arena::empty(DType dt, std::vector<int64_t> shape)
{
    int64_t n = 1;
    for (int64_t d : shape)
    {
        require(d >= 0, "Arena::empty: negative dimension");
        n *= d;
    }
    const size_t bytes = (size_t)n * dtype_size(dt);
    const size_t off = (off_ + 255) & ~(size_t)255;
    require(off + bytes <= buf_.bytes(), "Arena::empty: " + std::to_string(bytes) + " bytes do not fit (" +
                                             std::to_string(buf_.bytes() - off_) + " free)");
    off_ = off + bytes;
    return Tensor((char*)buf_.data() + off, dt, std::move(shape));
}

// ------------------------------------------------------------------------------------------------
// ffi

namespace ffi {

void rms_norm(const Tensor& x, const Tensor* w, const Tensor& y, float eps, float constant_bias, float constant_scale,
              const Stream& s)
{
    int64_t rows, dim, ldx, ry, dy, ldy;
    x.rows_view(rows, dim, ldx);
    y.rows_view(ry, dy, ldy);
    require(ry == rows && dy == dim, "rms_norm: x and y shapes differ");
    check_abi(exl3r_rms_norm(x.data, code(x.dtype), ldx, ptr(w), code_or(w, DType::F16), y.data, code(y.dtype), ldy,
                             rows, dim, eps, constant_bias, constant_scale, s.get()));
}

void rms_norm_res_in(const Tensor& x, const Tensor* w, const Tensor& y, const Tensor& r, float eps, float bias,
                     float scale, const Stream& s)
{
    int64_t rows, dim, ldx, ry, dy, ldy, rr, dr, ldr;
    x.rows_view(rows, dim, ldx);
    y.rows_view(ry, dy, ldy);
    r.rows_view(rr, dr, ldr);
    require(ry == rows && dy == dim && rr == rows && dr == dim, "rms_norm_res_in: x, y and r shapes differ");
    check_abi(exl3r_rms_norm_res_in(x.data, code(x.dtype), ldx, ptr(w), code_or(w, DType::F16), y.data,
                                    code(y.dtype), ldy, r.data, code(r.dtype), ldr, rows, dim, eps, bias, scale,
                                    s.get()));
}

static void act(int which, const Tensor& x, const Tensor& y, const Tensor& z, float act_limit, const Stream& s)
{
    int64_t rows, cols, ldx, ry, cy, ldy, rz, cz, ldz;
    x.rows_view(rows, cols, ldx);
    y.rows_view(ry, cy, ldy);
    z.rows_view(rz, cz, ldz);
    require(ry == rows && cy == cols && rz == rows && cz == cols, "act_mul: x, y and z shapes differ");
    require(x.dtype == y.dtype, "act_mul: x and y must share a dtype");
    auto fn = which == 0 ? exl3r_silu_mul : exl3r_gelu_mul;
    check_abi(fn(x.data, y.data, code(x.dtype), z.data, code(z.dtype), rows, cols, ldx, ldy, ldz, act_limit, s.get()));
}

void silu_mul(const Tensor& x, const Tensor& y, const Tensor& z, float act_limit, const Stream& s) { act(0, x, y, z, act_limit, s); }
void gelu_mul(const Tensor& x, const Tensor& y, const Tensor& z, float act_limit, const Stream& s) { act(1, x, y, z, act_limit, s); }

void gated_rms_norm(const Tensor& x, const Tensor* w, const Tensor& y, const Tensor& g, float eps, float bias,
                    int w_groups, bool gate_first, int gate_act, const Stream& s)
{
    int64_t rows, dim, ldx, ry, dy, ldy, rg, dg, ldg;
    x.rows_view(rows, dim, ldx);
    y.rows_view(ry, dy, ldy);
    g.rows_view(rg, dg, ldg);
    require(ry == rows && dy == dim && rg == rows && dg == dim, "gated_rms_norm: x, y and g shapes differ");
    require(!w || w->numel() == (int64_t)w_groups * dim, "gated_rms_norm: w must hold w_groups * dim values");
    check_abi(exl3r_gated_rms_norm(x.data, code(x.dtype), ldx, ptr(w), code_or(w, DType::F32), w_groups, y.data,
                                   code(y.dtype), ldy, g.data, code(g.dtype), ldg, rows, dim, eps, bias, gate_first ? 1 : 0,
                                   gate_act, s.get()));
}

void gated_rms_norm_had(const Tensor& x, const Tensor* w, const Tensor& g, const Tensor& out, const Tensor* y,
                        const Tensor* pre_scale, float eps, float bias, int w_groups, bool gate_first, int gate_act,
                        float had_scale, const Stream& s, int pre_rows, bool exact)
{
    int64_t rows, dim, ldx, rg, dg, ldg, ro, dout, ldo, ldy = 0;
    x.rows_view(rows, dim, ldx);
    g.rows_view(rg, dg, ldg);
    out.rows_view(ro, dout, ldo);
    require(rg == rows && dg == dim && ro == rows && dout == dim && out.dtype == DType::F16,
            "gated_rms_norm_had: g like x, out f16 like x");
    if (y)
    {
        int64_t ry, dy;
        y->rows_view(ry, dy, ldy);
        require(ry == rows && dy == dim && y->dtype == DType::F16, "gated_rms_norm_had: y is f16 like x");
    }
    require(!w || w->numel() == (int64_t)w_groups * dim, "gated_rms_norm_had: w must hold w_groups * dim values");
    check_abi(exl3r_gated_rms_norm_had(x.data, code(x.dtype), ldx, ptr(w), code_or(w, DType::F32), w_groups, g.data,
                                       code(g.dtype), ldg, y ? y->data : nullptr, ldy, ptr(pre_scale), pre_rows,
                                       out.data, ldo,
                                       rows, dim, eps, bias, gate_first ? 1 : 0, gate_act | (exact ? EXL3R_HAD_EXACT : 0),
                                       had_scale, s.get()));
}

void mul_sigmoid_(const Tensor& x, const Tensor& y, const Stream& s)
{
    int64_t rows, cols, ldx, ry, cy, ldy;
    x.rows_view(rows, cols, ldx);
    y.rows_view(ry, cy, ldy);
    require(ry == rows && cy == cols && x.dtype == y.dtype, "mul_sigmoid_: x and y must share shape and dtype");
    check_abi(exl3r_mul_sigmoid(x.data, y.data, code(x.dtype), x.data, code(x.dtype), rows, cols, ldx, ldy, ldx, s.get()));
}

void deinterleave_qg(const Tensor& qg, const Tensor& q, const Tensor& g, int64_t head_dim, const Stream& s)
{
    require(head_dim > 0 && qg.size(-1) % (2 * head_dim) == 0, "deinterleave_qg: qg's last dim must be heads * 2 * head_dim");
    require(qg.is_contiguous() && q.is_contiguous() && g.is_contiguous(), "deinterleave_qg: tensors must be contiguous");
    const int64_t heads = qg.size(-1) / (2 * head_dim), rows = qg.numel() / qg.size(-1);
    require(q.numel() == rows * heads * head_dim && g.numel() == q.numel(), "deinterleave_qg: size mismatch");
    require(q.dtype == qg.dtype && g.dtype == qg.dtype, "deinterleave_qg: qg, q and g must share a dtype");
    check_abi(exl3r_deinterleave_qg(qg.data, 2 * heads * head_dim, q.data, heads * head_dim, g.data, heads * head_dim,
                                    code(qg.dtype), rows, (int)heads, (int)head_dim, s.get()));
}

void had_r_128(const Tensor& x, const Tensor& out, const Tensor* pre_scale, const Tensor* post_scale, float scale,
               const Stream& s)
{
    int64_t rows, cols, ldx, ro, co, ldo;
    x.rows_view(rows, cols, ldx);
    out.rows_view(ro, co, ldo);
    require(ro == rows && co == cols && out.dtype == x.dtype, "had_r_128: x and out must share shape and dtype");
    for (const Tensor* sc : { pre_scale, post_scale })
        require(!sc || (sc->dtype == DType::F16 && sc->numel() == cols), "had_r_128: scales are f16 [cols]");
    check_abi(exl3r_had_r_128(x.data, code(x.dtype), ldx, out.data, ldo, rows, cols, ptr(pre_scale), ptr(post_scale),
                              scale, s.get()));
}

void rms_norm_had(const Tensor& x, const Tensor* w, const Tensor* r, const Tensor* y,
                  const std::vector<const Tensor*>& outs, const std::vector<const Tensor*>& pre_scales, float eps,
                  float constant_bias, float constant_scale, float had_scale, const Stream& s, bool rotate_x,
                  const Tensor* x_post_scale, bool exact)
{
    int64_t rows, dim, ldx, ldr = 0, ldy = 0, ldo = -1;
    x.rows_view(rows, dim, ldx);
    require(!outs.empty() && outs.size() <= 4 && pre_scales.size() == outs.size(),
            "rms_norm_had: 1..4 outputs, one pre_scale (or null) each");
    std::vector<const void*> pre(outs.size());
    std::vector<void*> out(outs.size());
    for (size_t i = 0; i < outs.size(); ++i)
    {
        int64_t ro, co, lo;
        require(outs[i] != nullptr, "rms_norm_had: outputs must be given");
        outs[i]->rows_view(ro, co, lo);
        require(ro == rows && co == dim && outs[i]->dtype == DType::F16 && (ldo < 0 || lo == ldo),
                "rms_norm_had: outputs are f16 shaped like x with one row stride");
        ldo = lo;
        out[i] = outs[i]->data;
        pre[i] = ptr(pre_scales[i]);
    }
    if (r)
    {
        int64_t rr, dr;
        r->rows_view(rr, dr, ldr);
        require(rr == rows && dr == dim, "rms_norm_had: r must be shaped like x");
    }
    if (y)
    {
        int64_t ry, dy;
        y->rows_view(ry, dy, ldy);
        require(ry == rows && dy == dim && y->dtype == DType::F16, "rms_norm_had: y is f16 shaped like x");
    }
    check_abi(exl3r_rms_norm_had(x.data, code(x.dtype), ldx, ptr(w), code_or(w, DType::F16), r ? r->data : nullptr,
                                 r ? code(r->dtype) : EXL3R_F16, ldr, y ? y->data : nullptr, ldy, (int)outs.size(),
                                 pre.data(), out.data(), ldo, rows, dim, eps, constant_bias, constant_scale, had_scale,
                                 (rotate_x ? 1 : 0) | (exact ? EXL3R_HAD_EXACT : 0), ptr(x_post_scale), s.get()));
}

void act_mul_had(HadAct act, const Tensor& x, const Tensor& y, const Tensor& out, const Tensor* pre_scale,
                 const Tensor* z, float act_limit, float had_scale, const Stream& s, bool rotate_x, bool rotate_y,
                 const Tensor* x_post, const Tensor* y_post, bool exact)
{
    int64_t rows, cols, ldx, ry, cy, ldy, ro, co, ldo, ldz = 0;
    x.rows_view(rows, cols, ldx);
    y.rows_view(ry, cy, ldy);
    out.rows_view(ro, co, ldo);
    require(ry == rows && cy == cols && y.dtype == x.dtype, "act_mul_had: x and y must share shape and dtype");
    require(ro == rows && co == cols && out.dtype == DType::F16, "act_mul_had: out is f16 shaped like x");
    if (z)
    {
        int64_t rz, cz;
        z->rows_view(rz, cz, ldz);
        require(rz == rows && cz == cols && z->dtype == DType::F16, "act_mul_had: z is f16 shaped like x");
    }
    check_abi(exl3r_act_mul_had((int)act, x.data, y.data, code(x.dtype), ldx, ldy, z ? z->data : nullptr, ldz,
                                ptr(pre_scale), out.data, ldo, rows, cols, act_limit, had_scale,
                                (rotate_x ? 1 : 0) | (rotate_y ? 2 : 0) | (exact ? EXL3R_HAD_EXACT : 0), ptr(x_post),
                                ptr(y_post), s.get()));
}

void argmax_sample(const Tensor& logits, const Tensor& ids, int max_logit, const Stream& s)
{
    int64_t rows, vocab, ld;
    logits.rows_view(rows, vocab, ld);
    require(ids.dtype == DType::I64 && ids.numel() == rows && ids.is_contiguous(),
            "argmax_sample: ids must be contiguous int64 with one entry per logits row");
    check_abi(exl3r_argmax_sample(logits.data, code(logits.dtype), rows, vocab, ld, max_logit,
                                  static_cast<int64_t*>(ids.data), s.get()));
}

void gumbel_sample(const Tensor& logits, const Tensor& ids, int max_logit, uint32_t random, const Stream& s)
{
    int64_t rows, vocab, ld;
    logits.rows_view(rows, vocab, ld);
    require(ids.dtype == DType::I64 && ids.numel() == rows && ids.is_contiguous(),
            "gumbel_sample: ids must be contiguous int64 with one entry per logits row");
    check_abi(exl3r_gumbel_sample(logits.data, code(logits.dtype), rows, vocab, ld, max_logit, random,
                                  static_cast<int64_t*>(ids.data), s.get()));
}

void argmax_sample_ws(const Tensor& logits, const Tensor& ids, int max_logit, const DeviceBuffer& workspace,
                      const Stream& s)
{
    int64_t rows, vocab, ld;
    logits.rows_view(rows, vocab, ld);
    require(ids.dtype == DType::I64 && ids.numel() == rows && ids.is_contiguous(),
            "argmax_sample_ws: ids must be contiguous int64 with one entry per logits row");
    check_abi(exl3r_argmax_sample_ws(logits.data, code(logits.dtype), rows, vocab, ld, max_logit,
                                     static_cast<int64_t*>(ids.data), workspace.data(), workspace.bytes(), s.get()));
}

void gumbel_sample_ws(const Tensor& logits, const Tensor& ids, int max_logit, uint32_t random,
                      const DeviceBuffer& workspace, const Stream& s)
{
    int64_t rows, vocab, ld;
    logits.rows_view(rows, vocab, ld);
    require(ids.dtype == DType::I64 && ids.numel() == rows && ids.is_contiguous(),
            "gumbel_sample_ws: ids must be contiguous int64 with one entry per logits row");
    check_abi(exl3r_gumbel_sample_ws(logits.data, code(logits.dtype), rows, vocab, ld, max_logit, random,
                                     static_cast<int64_t*>(ids.data), workspace.data(), workspace.bytes(), s.get()));
}

void gumbel_noise(const Tensor& x, const Tensor& out, uint32_t random, const Stream& s)
{
    int64_t rows, cols, ldx, ro, co, ldo;
    x.rows_view(rows, cols, ldx);
    out.rows_view(ro, co, ldo);
    require(ro == rows && co == cols, "gumbel_noise: x and out shapes differ");
    check_abi(exl3r_gumbel_noise(x.data, code(x.dtype), ldx, out.data, code(out.dtype), ldo, rows, cols, random, s.get()));
}

void rope_qg(const Tensor& qg, const Tensor& out_q, const Tensor* k, const Tensor* out_k, const Tensor& inv_freq,
             int64_t position, const Tensor* positions, const Tensor* q_norm, const Tensor* k_norm, float norm_eps,
             float norm_constant_bias, RopeStyle rope_mode, float attn_factor, const Stream& s, const Tensor* position_ids)
{
    require(qg.dim() == 4 && out_q.dim() == 4, "rope_qg: qg and out_q must be (bsz, seq_len, heads, 2 * head_dim / head_dim)");
    const int64_t bsz = qg.size(0), seq = qg.size(1), hq = qg.size(2), hd = qg.size(3) / 2;
    require(qg.size(3) % 2 == 0 && qg.stride(3) == 1 && qg.stride(2) == 2 * hd, "rope_qg: qg must hold dense [q | g] heads");
    require(bsz <= 1 || seq <= 1 || qg.stride(0) == seq * qg.stride(1), "rope_qg: qg batch stride must be seq_len * token stride");
    require(out_q.is_contiguous() && out_q.size(0) == bsz && out_q.size(1) == seq && out_q.size(2) == hq && out_q.size(3) == hd,
            "rope_qg: out_q must be a dense (bsz, seq_len, heads, head_dim)");
    int64_t hk = 0, kts = 0, khs = 0;
    if (k)
    {
        require(out_k && k->dim() == 4 && k->size(0) == bsz && k->size(1) == seq && k->size(3) == hd,
                "rope_qg: k is incorrect shape");
        require(k->stride(3) == 1 && out_k->strides == k->strides, "rope_qg: out_k must share k's layout");
        hk = k->size(2);
        kts = k->stride(1);
        khs = k->stride(2);
    }
    require(inv_freq.dtype == DType::F32 && inv_freq.dim() == 1, "rope_qg: inv_freq must be float32 [R/2]");
    require(!positions || positions->dtype == DType::I32, "rope_qg: positions must be int32");
    require(!position_ids || position_ids->dtype == DType::I32, "rope_qg: position_ids must be int32");
    const Tensor* nw = q_norm ? q_norm : k_norm;
    check_abi(exl3r_rope_qg(qg.data, qg.stride(1), out_q.data, (int)hq, k ? k->data : nullptr, out_k ? out_k->data : nullptr,
                            kts, khs, (int)hk, code(qg.dtype), bsz, seq, (int)hd, (const float*)inv_freq.data,
                            (int)(inv_freq.size(0) * 2), (int32_t)position, (const int32_t*)ptr(positions),
                            (const int32_t*)ptr(position_ids), ptr(q_norm), ptr(k_norm), code_or(nw, DType::F16), norm_eps,
                            norm_constant_bias, (int)rope_mode, attn_factor, s.get()));
}

void rope_cs_table(int64_t bsz, int64_t seq_len, const Tensor& inv_freq, int64_t position, const Tensor* positions,
                   const Tensor* position_ids, float attn_factor, const Tensor& cs_table, const Stream& s)
{
    require(inv_freq.dtype == DType::F32 && inv_freq.dim() == 1, "rope_cs_table: inv_freq must be float32 [R/2]");
    require(!positions || positions->dtype == DType::I32, "rope_cs_table: positions must be int32");
    require(!position_ids || position_ids->dtype == DType::I32, "rope_cs_table: position_ids must be int32");
    require(cs_table.dtype == DType::F32 && cs_table.is_contiguous() && cs_table.dim() == 3 &&
                cs_table.size(0) == bsz * seq_len && cs_table.size(1) == inv_freq.size(0) && cs_table.size(2) == 2,
            "rope_cs_table: cs_table must be contiguous float32 [bsz * seq_len, R/2, 2]");
    check_abi(exl3r_rope_cs_table(bsz, seq_len, (const float*)inv_freq.data, (int)(inv_freq.size(0) * 2),
                                  (int32_t)position, (const int32_t*)ptr(positions), (const int32_t*)ptr(position_ids),
                                  attn_factor, cs_table.data, s.get()));
}

void rope_cs(const Tensor& q, const Tensor& out_q, const Tensor* k, const Tensor* out_k, const Tensor& cs_table,
             const Tensor* q_norm, const Tensor* k_norm, float norm_eps, float norm_constant_bias, RopeStyle rope_mode,
             const Stream& s)
{
    require(q.dim() == 4, "rope_cs: q must be (bsz, seq_len, heads, head_dim)");
    require(q.stride(3) == 1 && out_q.strides == q.strides && out_q.shape == q.shape,
            "rope_cs: q innermost dim must be dense and out_q must share q's layout");
    const int64_t bsz = q.size(0), seq = q.size(1), hd = q.size(3);
    require(bsz <= 1 || seq <= 1 || q.stride(0) == seq * q.stride(1), "rope_cs: q batch stride must be seq_len * token stride");
    int64_t hk = 0, kts = 0, khs = 0;
    if (k)
    {
        require(out_k && k->dim() == 4 && k->size(0) == bsz && k->size(1) == seq && k->size(3) == hd,
                "rope_cs: k is incorrect shape");
        require(k->stride(3) == 1 && out_k->strides == k->strides, "rope_cs: out_k must share k's layout");
        hk = k->size(2);
        kts = k->stride(1);
        khs = k->stride(2);
    }
    require(cs_table.dtype == DType::F32 && cs_table.is_contiguous() && cs_table.dim() == 3 &&
                cs_table.size(0) == bsz * seq && cs_table.size(2) == 2,
            "rope_cs: cs_table must be contiguous float32 [bsz * seq_len, R/2, 2]");
    const Tensor* nw = q_norm ? q_norm : k_norm;
    check_abi(exl3r_rope_cs(q.data, out_q.data, q.stride(1), q.stride(2), (int)q.size(2), k ? k->data : nullptr,
                            out_k ? out_k->data : nullptr, kts, khs, (int)hk, code(q.dtype), bsz, seq, (int)hd,
                            cs_table.data, (int)(cs_table.size(1) * 2), ptr(q_norm), ptr(k_norm),
                            code_or(nw, DType::F16), norm_eps, norm_constant_bias, (int)rope_mode, s.get()));
}

void rope(const Tensor& q, const Tensor& out_q, const Tensor* k, const Tensor* out_k, const Tensor& inv_freq,
          int64_t position, const Tensor* positions, const Tensor* q_norm, const Tensor* k_norm, float norm_eps,
          float norm_constant_bias, RopeStyle rope_mode, float attn_factor, const Stream& s, const Tensor* position_ids,
          int32_t* err_flag)
{
    require(q.dim() == 4, "rope: q must be (bsz, seq_len, heads, head_dim)");
    require(q.stride(3) == 1 && out_q.strides == q.strides && out_q.shape == q.shape,
            "rope: q innermost dim must be dense and out_q must share q's layout");
    const int64_t bsz = q.size(0), seq = q.size(1), hd = q.size(3);
    require(bsz <= 1 || seq <= 1 || q.stride(0) == seq * q.stride(1), "rope: q batch stride must be seq_len * token stride");
    int64_t hk = 0, kts = 0, khs = 0;
    if (k)
    {
        require(out_k && k->dim() == 4 && k->size(0) == bsz && k->size(1) == seq && k->size(3) == hd,
                "rope: k is incorrect shape");
        require(k->stride(3) == 1 && out_k->strides == k->strides, "rope: out_k must share k's layout");
        hk = k->size(2);
        kts = k->stride(1);
        khs = k->stride(2);
    }
    require(inv_freq.dtype == DType::F32, "rope: inv_freq must be float32");
    require(!positions || positions->dtype == DType::I32, "rope: positions must be int32");
    require(!position_ids || position_ids->dtype == DType::I32, "rope: position_ids must be int32");
    const Tensor* nw = q_norm ? q_norm : k_norm;
    if (inv_freq.dim() > 1)
    {
        require(inv_freq.dim() <= 3 && inv_freq.is_contiguous(), "rope: an angle table must be contiguous [max_pos, R/2] or [bsz, max_pos, R/2]");
        require(inv_freq.dim() == 2 || inv_freq.size(0) >= bsz, "rope: a per-sequence angle table needs bsz tables");
        const int64_t rows = inv_freq.size(-2), half = inv_freq.size(-1);
        check_abi(exl3r_rope_table(q.data, out_q.data, q.stride(1), q.stride(2), (int)q.size(2), k ? k->data : nullptr,
                                   out_k ? out_k->data : nullptr, kts, khs, (int)hk, code(q.dtype), bsz, seq, (int)hd,
                                   (const float*)inv_freq.data, rows, inv_freq.dim() == 3 ? rows * half : 0, (int)(half * 2),
                                   (int32_t)position, (const int32_t*)ptr(positions), (const int32_t*)ptr(position_ids),
                                   ptr(q_norm), ptr(k_norm), code_or(nw, DType::F16), norm_eps, norm_constant_bias,
                                   (int)rope_mode, attn_factor, err_flag, s.get()));
        return;
    }
    check_abi(exl3r_rope(q.data, out_q.data, q.stride(1), q.stride(2), (int)q.size(2), k ? k->data : nullptr,
                         out_k ? out_k->data : nullptr, kts, khs, (int)hk, code(q.dtype), bsz, seq, (int)hd,
                         (const float*)inv_freq.data, (int)(inv_freq.numel() * 2), (int32_t)position,
                         (const int32_t*)ptr(positions), (const int32_t*)ptr(position_ids), ptr(q_norm), ptr(k_norm),
                         code_or(nw, DType::F16), norm_eps, norm_constant_bias, (int)rope_mode, attn_factor, s.get()));
}

// rotary_dim of the entry points that take inv_freq [R/2] and optionally a rope_cs_table() {cos, sin} table
// [tokens, R/2, 2] (tokens = bsz * seq_len).  Their kernels index the table by token, so a table built for
// fewer tokens (one kept across forward passes of different lengths) is rejected before the launch.
static int rotary_dim_of(const char* op, const Tensor& inv_freq, const Tensor* cs_table, int64_t tokens)
{
    require(inv_freq.dtype == DType::F32 && inv_freq.dim() == 1, std::string(op) + ": inv_freq must be float32 [R/2]");
    if (cs_table)
        require(cs_table->dtype == DType::F32 && cs_table->is_contiguous() && cs_table->dim() == 3 &&
                    cs_table->size(0) == tokens && cs_table->size(1) == inv_freq.size(0) && cs_table->size(2) == 2,
                std::string(op) + ": cs_table must be contiguous float32 [bsz * seq_len, R/2, 2] with R/2 = inv_freq's length");
    return (int)(inv_freq.size(0) * 2);
}

void rope_had(const Tensor& q, const Tensor& out_q, const Tensor* k, const Tensor* out_k, const Tensor& inv_freq,
              int64_t position, const Tensor* positions, const Tensor* q_norm, const Tensor* k_norm, float norm_eps,
              float norm_constant_bias, RopeStyle rope_mode, float attn_factor, const Tensor* q_post_scale,
              const Tensor* k_post_scale, const Stream& s, const Tensor* position_ids, const Tensor* cs_table,
              bool exact)
{
    require(q.dim() == 4 && q.dtype == DType::F16, "rope_had: q must be f16 (bsz, seq_len, heads, head_dim)");
    const int64_t bsz = q.size(0), seq = q.size(1), hd = q.size(3);
    require(q.stride(3) == 1 && q.stride(2) == hd && out_q.strides == q.strides && out_q.shape == q.shape,
            "rope_had: q heads must be packed and out_q must share q's layout");
    require(bsz <= 1 || seq <= 1 || q.stride(0) == seq * q.stride(1), "rope_had: q batch stride must be seq_len * token stride");
    int64_t hk = 0, kts = 0;
    if (k)
    {
        require(out_k && k->dim() == 4 && k->size(0) == bsz && k->size(1) == seq && k->size(3) == hd &&
                    k->stride(3) == 1 && k->stride(2) == hd && out_k->strides == k->strides,
                "rope_had: k must be packed like q, out_k sharing its layout");
        hk = k->size(2);
        kts = k->stride(1);
    }
    const int rdim = rotary_dim_of("rope_had", inv_freq, cs_table, bsz * seq);
    require(!positions || positions->dtype == DType::I32, "rope_had: positions must be int32");
    require(!position_ids || position_ids->dtype == DType::I32, "rope_had: position_ids must be int32");
    const Tensor* nw = q_norm ? q_norm : k_norm;
    check_abi(exl3r_rope_had(q.data, out_q.data, q.stride(1), (int)q.size(2), k ? k->data : nullptr,
                             out_k ? out_k->data : nullptr, kts, (int)hk, code(q.dtype), bsz, seq, (int)hd,
                             (const float*)inv_freq.data, rdim, (int32_t)position,
                             (const int32_t*)ptr(positions), (const int32_t*)ptr(position_ids), ptr(q_norm),
                             ptr(k_norm), code_or(nw, DType::F16), norm_eps, norm_constant_bias,
                             (int)rope_mode | (exact ? EXL3R_HAD_EXACT : 0), attn_factor, ptr(q_post_scale),
                             ptr(k_post_scale), ptr(cs_table), s.get()));
}

void rope_paged_kv(const Tensor& q, const Tensor& out_q, const Tensor& k, const Tensor* out_k, const Tensor& v,
                   const Tensor& inv_freq, int64_t position, const Tensor* positions, const Tensor* q_norm,
                   const Tensor* k_norm, float norm_eps, float norm_constant_bias, RopeStyle rope_mode, float attn_factor,
                   const Tensor& k_cache, const Tensor& v_cache, const Tensor& block_table, const Tensor& cache_seqlens,
                   int32_t* err_flag, const Stream& s, const Tensor* cs_table)
{
    require(q.dim() == 4 && k.dim() == 4 && v.dim() == 4, "rope_paged_kv: q, k, v must be (bsz, seq_len, heads, head_dim)");
    require(q.stride(3) == 1 && out_q.strides == q.strides && out_q.shape == q.shape,
            "rope_paged_kv: q innermost dim must be dense and out_q must share q's layout");
    const int64_t bsz = q.size(0), seq = q.size(1), hd = q.size(3), hk = k.size(2);
    require(k.shape == v.shape && k.size(0) == bsz && k.size(1) == seq && k.size(3) == hd,
            "rope_paged_kv: k and v must be (bsz, seq_len, kv_heads, head_dim)");
    require(k.stride(3) == 1 && v.stride(3) == 1 && (!out_k || out_k->strides == k.strides),
            "rope_paged_kv: dense k / v rows; out_k must share k's layout");
    for (const Tensor* t : { &q, &k, &v })
        require(bsz <= 1 || seq <= 1 || t->stride(0) == seq * t->stride(1),
                "rope_paged_kv: batch stride must be seq_len * token stride");
    require(k_cache.dim() == 4 && k_cache.shape == v_cache.shape && k_cache.size(2) == hk && k_cache.size(3) == hd &&
                k_cache.is_contiguous() && v_cache.is_contiguous(),
            "rope_paged_kv: caches must be contiguous (pages, page_size, kv_heads, head_dim)");
    require(block_table.dim() == 2 && block_table.dtype == DType::I32 && cache_seqlens.dtype == DType::I32,
            "rope_paged_kv: block_table (bsz, max_blocks) and cache_seqlens (bsz) must be int32");
    const int rdim = rotary_dim_of("rope_paged_kv", inv_freq, cs_table, bsz * seq);
    require(!positions || positions->dtype == DType::I32, "rope_paged_kv: positions must be int32");
    const Tensor* nw = q_norm ? q_norm : k_norm;
    check_abi(exl3r_rope_paged_kv(q.data, out_q.data, q.stride(1), q.stride(2), (int)q.size(2), k.data,
                                  out_k ? out_k->data : nullptr, k.stride(1), k.stride(2), v.data, v.stride(1), v.stride(2),
                                  (int)hk, code(q.dtype), bsz, seq, (int)hd, (const float*)inv_freq.data,
                                  rdim, (int32_t)position, (const int32_t*)ptr(positions), nullptr,
                                  ptr(q_norm), ptr(k_norm), code_or(nw, DType::F16), norm_eps, norm_constant_bias,
                                  (int)rope_mode, attn_factor, k_cache.data, v_cache.data, (int)k_cache.size(1),
                                  k_cache.size(0), (const int32_t*)block_table.data, block_table.size(1),
                                  (const int32_t*)cache_seqlens.data, err_flag, ptr(cs_table), s.get()));
}

void rope_paged_kv_had(const Tensor& q, const Tensor& out_q, const Tensor& k, const Tensor* out_k, const Tensor& v,
                       const Tensor& inv_freq, int64_t position, const Tensor* positions, const Tensor* q_norm,
                       const Tensor* k_norm, float norm_eps, float norm_constant_bias, RopeStyle rope_mode,
                       float attn_factor, const Tensor& k_cache, const Tensor& v_cache, const Tensor& block_table,
                       const Tensor& cache_seqlens, int32_t* err_flag, const Tensor* q_post_scale,
                       const Tensor* k_post_scale, const Tensor* v_post_scale, const Stream& s,
                       const Tensor* cs_table, bool exact)
{
    require(q.dim() == 4 && k.dim() == 4 && v.dim() == 4 && q.dtype == DType::F16,
            "rope_paged_kv_had: q, k, v must be f16 (bsz, seq_len, heads, head_dim)");
    const int64_t bsz = q.size(0), seq = q.size(1), hd = q.size(3), hk = k.size(2);
    require(out_q.strides == q.strides && out_q.shape == q.shape, "rope_paged_kv_had: out_q must share q's layout");
    require(k.shape == v.shape && k.size(0) == bsz && k.size(1) == seq && k.size(3) == hd &&
                (!out_k || out_k->strides == k.strides),
            "rope_paged_kv_had: k and v must be (bsz, seq_len, kv_heads, head_dim); out_k shares k's layout");
    for (const Tensor* t : { &q, &k, &v })
        require(t->stride(3) == 1 && t->stride(2) == hd && (bsz <= 1 || seq <= 1 || t->stride(0) == seq * t->stride(1)),
                "rope_paged_kv_had: packed heads and batch stride seq_len * token stride");
    require(k_cache.dim() == 4 && k_cache.shape == v_cache.shape && k_cache.size(2) == hk && k_cache.size(3) == hd &&
                k_cache.is_contiguous() && v_cache.is_contiguous(),
            "rope_paged_kv_had: caches must be contiguous (pages, page_size, kv_heads, head_dim)");
    require(block_table.dim() == 2 && block_table.dtype == DType::I32 && cache_seqlens.dtype == DType::I32,
            "rope_paged_kv_had: block_table (bsz, max_blocks) and cache_seqlens (bsz) must be int32");
    const int rdim = rotary_dim_of("rope_paged_kv_had", inv_freq, cs_table, bsz * seq);
    require(!positions || positions->dtype == DType::I32, "rope_paged_kv_had: positions must be int32");
    const Tensor* nw = q_norm ? q_norm : k_norm;
    check_abi(exl3r_rope_paged_kv_had(q.data, out_q.data, q.stride(1), (int)q.size(2), k.data,
                                      out_k ? out_k->data : nullptr, k.stride(1), v.data, v.stride(1), (int)hk,
                                      code(q.dtype), bsz, seq, (int)hd, (const float*)inv_freq.data,
                                      rdim, (int32_t)position, (const int32_t*)ptr(positions),
                                      nullptr, ptr(q_norm), ptr(k_norm), code_or(nw, DType::F16), norm_eps,
                                      norm_constant_bias, (int)rope_mode | (exact ? EXL3R_HAD_EXACT : 0), attn_factor,
                                      k_cache.data, v_cache.data, (int)k_cache.size(1), k_cache.size(0),
                                      (const int32_t*)block_table.data, block_table.size(1),
                                      (const int32_t*)cache_seqlens.data, err_flag, ptr(q_post_scale),
                                      ptr(k_post_scale), ptr(v_post_scale), ptr(cs_table), s.get()));
}

void embedding(const Tensor& table, const Tensor& ids, const Tensor& out, int32_t* err_flag, const Stream& s)
{
    require(table.dim() == 2 && table.stride(1) == 1, "embedding: table must be [vocab, hidden] with dense rows");
    int64_t rows, hidden, ldo;
    out.rows_view(rows, hidden, ldo);
    require(rows == ids.numel() && hidden == table.size(1), "embedding: out must be [ids.numel(), hidden]");
    require(ids.is_contiguous(), "embedding: ids must be contiguous");
    check_abi(exl3r_embedding(table.data, code(table.dtype), table.size(0), table.size(1), table.stride(0), ids.data,
                              code(ids.dtype), ids.numel(), out.data, code(out.dtype), ldo, err_flag, s.get()));
}

void embedding_rms_norm(const Tensor& table, const Tensor& ids, const Tensor* h, const Tensor* w, const Tensor& y,
                        float eps, float constant_bias, float constant_scale, int32_t* err_flag, const Stream& s)
{
    require(table.dim() == 2 && table.stride(1) == 1, "embedding_rms_norm: table must be [vocab, hidden]");
    require(ids.is_contiguous(), "embedding_rms_norm: ids must be contiguous");
    int64_t rows, hidden, ldy, rh = 0, hh = 0, ldh = table.size(1);
    y.rows_view(rows, hidden, ldy);
    require(rows == ids.numel() && hidden == table.size(1), "embedding_rms_norm: y must be [ids.numel(), hidden]");
    if (h)
    {
        h->rows_view(rh, hh, ldh);
        require(rh == rows && hh == hidden, "embedding_rms_norm: h must be [ids.numel(), hidden]");
    }
    check_abi(exl3r_embedding_rms_norm(table.data, code(table.dtype), table.size(0), table.size(1), table.stride(0),
                                       ids.data, code(ids.dtype), ids.numel(), h ? h->data : nullptr,
                                       code_or(h, DType::F32), ldh, ptr(w), code_or(w, DType::F16), y.data,
                                       code(y.dtype), ldy, eps, constant_bias, constant_scale, err_flag, s.get()));
}

}  // namespace ffi

// ------------------------------------------------------------------------------------------------
// Modules

Tensor RmsNorm::forward(const Tensor& x, Arena& arena, const Stream& s) const
{
    Tensor y = arena.empty(DType::F16, x.shape);
    forward_into(x, y, s);
    return y;
}

void RmsNorm::forward_into(const Tensor& x, const Tensor& y, const Stream& s) const
{
    ffi::rms_norm(x, &weight_, y, eps_, constant_bias_, constant_scale_, s);
}

Tensor RmsNorm::forward_res(const Tensor& r, const Tensor* add, Arena& arena, const Stream& s) const
{
    Tensor y = arena.empty(DType::F16, r.shape);
    if (add && !r.is_contiguous())
    {
        const Tensor scratch = arena.empty(r.dtype, r.shape);
        forward_res_into(r, add, y, s, &scratch);
    }
    else
        forward_res_into(r, add, y, s);
    return y;
}

// dst (contiguous, src's dtype and shape) = src, whose last dim is dense: one 2-D copy per index of the
// dims before the last two.
static void copy_to_contiguous(const Tensor& src, const Tensor& dst, const Stream& s)
{
    require(dst.dtype == src.dtype && dst.shape == src.shape && dst.is_contiguous(),
            "RmsNorm::forward_res: scratch must be contiguous with the residual's dtype and shape");
    const int nd = src.dim();
    require(nd >= 1 && src.stride(-1) == 1, "RmsNorm::forward_res: a non-contiguous residual needs a dense last dim");
    if (src.numel() == 0) return;
    const size_t es = dtype_size(src.dtype);
    const int64_t cols = src.size(-1);
    const int64_t inner = nd >= 2 ? src.size(-2) : 1;
    const int64_t pitch = inner > 1 ? src.stride(-2) : cols;
    require(pitch >= cols, "RmsNorm::forward_res: residual rows overlap");
    int64_t outer = 1;
    for (int i = 0; i + 2 < nd; ++i) outer *= src.shape[i];
    for (int64_t o = 0; o < outer; ++o)
    {
        int64_t rem = o, off = 0;
        for (int i = nd - 3; i >= 0; --i)
        {
            off += (rem % src.shape[i]) * src.strides[i];
            rem /= src.shape[i];
        }
        check_hip(hipMemcpy2DAsync((char*)dst.data + (size_t)(o * inner * cols) * es, (size_t)cols * es,
                                   (const char*)src.data + (size_t)off * es, (size_t)pitch * es, (size_t)cols * es,
                                   (size_t)inner, hipMemcpyDeviceToDevice, s.get()),
                  "hipMemcpy2DAsync residual");
    }
}

void RmsNorm::forward_res_into(const Tensor& r, const Tensor* add, const Tensor& y, const Stream& s,
                               const Tensor* scratch) const
{
    if (!add) return forward_into(r, y, s);
    require(add->shape == r.shape, "RmsNorm::forward_res: add and residual shapes differ");
    if (r.is_contiguous())
        return ffi::rms_norm_res_in(*add, &weight_, y, r, eps_, constant_bias_, constant_scale_, s);
    // src/modules.rs:393-395: forward(r + add), r unchanged.
    require(scratch != nullptr, "RmsNorm::forward_res: a non-contiguous residual needs a scratch tensor");
    copy_to_contiguous(r, *scratch, s);
    ffi::rms_norm_res_in(*add, &weight_, y, *scratch, eps_, constant_bias_, constant_scale_, s);
}

Tensor Embedding::forward(const Tensor& ids, Arena& arena, const Stream& s) const
{
    std::vector<int64_t> shape = ids.shape;
    shape.push_back(weight_.size(1));
    Tensor out = arena.empty(out_kind_, shape);
    forward_into(ids, out, s);
    return out;
}

void Embedding::forward_into(const Tensor& ids, const Tensor& out, const Stream& s) const
{
    ffi::embedding(weight_, ids, out, nullptr, s);
}

Tensor GatedMlp::activate(const Tensor& g, const Tensor& u, Act act, float act_limit, Arena& arena, const Stream& s)
{
    Tensor a = arena.empty(g.dtype, g.shape);
    activate_into(g, u, a, act, act_limit, s);
    return a;
}

void GatedMlp::activate_into(const Tensor& g, const Tensor& u, const Tensor& a, Act act, float act_limit,
                             const Stream& s)
{
    if (act == Act::Silu) ffi::silu_mul(g, u, a, act_limit, s);
    else ffi::gelu_mul(g, u, a, act_limit, s);
}

RoPE::RoPE(double theta, int rotary_dim, RopeStyle style, double attn_factor, double linear_factor)
    : rotary_dim_(rotary_dim), style_(style), attn_factor_((float)attn_factor)
{
    inv_freq_host_ = default_inv_freq(theta, rotary_dim, linear_factor);
    inv_freq_ = DeviceBuffer(inv_freq_host_.size() * sizeof(float));
    check_hip(hipMemcpy(inv_freq_.data(), inv_freq_host_.data(), inv_freq_.bytes(), hipMemcpyHostToDevice), "hipMemcpy inv_freq");
    inv_freq_t_ = Tensor(inv_freq_.data(), DType::F32, { (int64_t)inv_freq_host_.size() });
}

RoPE::RoPE(double theta, int rotary_dim, RopeStyle style, const RopeScaling& sc)
    : style_(style)
{
    Params p = params(theta, rotary_dim, sc);
    inv_freq_host_ = std::move(p.inv_freq);
    rotary_dim_ = (int)inv_freq_host_.size() * 2;
    attn_factor_ = (float)p.attn_factor;
    inv_freq_ = DeviceBuffer(inv_freq_host_.size() * sizeof(float));
    check_hip(hipMemcpy(inv_freq_.data(), inv_freq_host_.data(), inv_freq_.bytes(), hipMemcpyHostToDevice), "hipMemcpy inv_freq");
    inv_freq_t_ = Tensor(inv_freq_.data(), DType::F32, { (int64_t)inv_freq_host_.size() });
}

RoPE::Params RoPE::params(double theta, int rotary_dim, const RopeScaling& sc)
{
    using T = RopeScaling::Type;
    require(theta > 0.0, "RoPE: theta must be positive");
    const double pi = 3.14159265358979323846;
    const double factor_or_1 = sc.factor > 0.0 ? sc.factor : 1.0;
    if (sc.type == T::Default) return { default_inv_freq(theta, rotary_dim), 1.0 };
    if (sc.type == T::Linear) return { default_inv_freq(theta, rotary_dim, factor_or_1), 1.0 };
    if (sc.type == T::Proportional)
    {
        // inv_freq over head_dim / 2 frequencies: theta^(-2i / head_dim) for the first
        // partial_rotary_factor * head_dim / 2, zero after (those dims keep angle 0), all / factor.
        require(sc.head_dim >= 2 && sc.head_dim % 2 == 0, "RoPE proportional: head_dim must be even");
        const int angles = (int)(sc.partial_rotary_factor * sc.head_dim / 2.0);
        require(angles >= 0 && angles <= sc.head_dim / 2, "RoPE proportional: partial_rotary_factor out of range");
        std::vector<float> inv(sc.head_dim / 2, 0.0f);
        for (int i = 0; i < angles; ++i)
            inv[i] = (float)(std::exp(-(2.0 * i / sc.head_dim) * std::log(theta)) / factor_or_1);
        return { inv, 1.0 };
    }
    require(rotary_dim >= 2 && rotary_dim % 2 == 0, "RoPE: rotary_dim must be even and >= 2");
    const int half = rotary_dim / 2;
    const std::vector<float> base = default_inv_freq(theta, rotary_dim);
    std::vector<float> inv(half);
    if (sc.type == T::Llama3)
    {
        // Wavelengths 2 pi / f above old_ctx / low_freq_factor are divided by factor, those below
        // old_ctx / high_freq_factor kept, and the band between blended with
        // smooth = (old_ctx / wavelen - low) / (high - low).
        const double factor = sc.factor > 0.0 ? sc.factor : 8.0;
        const double old_ctx = sc.original_max_position_embeddings > 0.0 ? sc.original_max_position_embeddings : 8192.0;
        require(sc.high_freq_factor > sc.low_freq_factor, "RoPE llama3: high_freq_factor must exceed low_freq_factor");
        const double low_wl = old_ctx / sc.low_freq_factor, high_wl = old_ctx / sc.high_freq_factor;
        for (int i = 0; i < half; ++i)
        {
            const double f = base[i], wl = 2.0 * pi / f;
            const double scaled = wl > low_wl ? f / factor : f;
            if (wl >= high_wl && wl <= low_wl)
            {
                const double smooth = (old_ctx / wl - sc.low_freq_factor) / (sc.high_freq_factor - sc.low_freq_factor);
                inv[i] = (float)((scaled / factor) * (1.0 - smooth) + scaled * smooth);
            }
            else
                inv[i] = (float)scaled;
        }
        return { inv, 1.0 };
    }
    if (sc.type == T::Yarn)
    {
        require(sc.max_position_embeddings > 0, "RoPE yarn: max_position_embeddings is required");
        double orig_max, factor;
        if (sc.original_max_position_embeddings > 0.0)
        {
            orig_max = sc.original_max_position_embeddings;
            factor = (double)sc.max_position_embeddings / orig_max;
        }
        else
        {
            orig_max = (double)sc.max_position_embeddings;
            factor = factor_or_1;
        }
        require(factor > 0.0, "RoPE yarn: factor must be positive");
        auto find = [&](double rot) { return rotary_dim * std::log(orig_max / (rot * 2.0 * pi)) / (2.0 * std::log(theta)); };
        double low = find(sc.beta_fast), high = find(sc.beta_slow);
        if (sc.truncate)
        {
            low = std::floor(low);
            high = std::ceil(high);
        }
        low = std::max(low, 0.0);
        high = std::min(high, rotary_dim - 1.0);
        if (low == high) high += 0.001;
        for (int i = 0; i < half; ++i)
        {
            const double pos_freq = std::exp((2.0 * i / rotary_dim) * std::log(theta));
            const double ramp = std::min(std::max((i - low) / (high - low), 0.0), 1.0);
            const double extrap = 1.0 - ramp;
            inv[i] = (float)((1.0 / (factor * pos_freq)) * (1.0 - extrap) + (1.0 / pos_freq) * extrap);
        }
        const double attn = sc.has_attention_factor ? sc.attention_factor
                                                    : (factor <= 1.0 ? 1.0 : 0.1 * std::log(factor) + 1.0);
        return { inv, attn };
    }
    // LongRope / "su": per-frequency extension factors, long_factor when the context is extended.
    const double a = (double)sc.max_position_embeddings, b = sc.original_max_position_embeddings;
    require(a > 0.0 && b > 0.0, "RoPE longrope: max_position_embeddings and original_max_position_embeddings are required");
    const std::vector<double>& ext = a > b ? sc.long_factor : sc.short_factor;
    require((int)ext.size() == half, "RoPE longrope: one factor per frequency (rotary_dim / 2) is required");
    for (int i = 0; i < half; ++i)
        inv[i] = (float)(1.0 / (ext[i] * std::exp((2.0 * i / rotary_dim) * std::log(theta))));
    return { inv, a > b ? std::sqrt(1.0 + std::log(a / b) / std::log(b)) : 1.0 };
}

std::vector<float> RoPE::default_inv_freq(double theta, int rotary_dim, double linear_factor)
{
    require(rotary_dim >= 2 && rotary_dim % 2 == 0, "RoPE: rotary_dim must be even and >= 2");
    require(theta > 0.0 && linear_factor > 0.0, "RoPE: theta and the scaling factor must be positive");
    const float ln_theta = (float)std::log(theta);
    std::vector<float> inv(rotary_dim / 2);
    for (int i = 0; i < rotary_dim / 2; ++i)
    {
        const float t = (float)(2 * i) / (float)rotary_dim;     // arange(0, d, 2) / d
        float f = 1.0f / std::exp(t * ln_theta);                 // 1 / exp(t * ln theta)
        if (linear_factor != 1.0) f = f / (float)linear_factor;
        inv[i] = f;
    }
    return inv;
}

void RoPE::apply(const Tensor& q, const Tensor& k, int64_t position, const Tensor* positions, const Tensor* q_norm,
                 const Tensor* k_norm, float norm_eps, float norm_constant_bias, const Stream& s,
                 const Tensor* freq_table) const
{
    ffi::rope(q, q, &k, &k, freq_table ? *freq_table : inv_freq_t_, position, positions, q_norm, k_norm, norm_eps,
              norm_constant_bias, style_, attn_factor_, s);
}

void RoPE::apply_paged(const Tensor& q, const Tensor& k, const Tensor& v, const Tensor& k_cache, const Tensor& v_cache,
                       const Tensor& block_table, const Tensor& cache_seqlens, const Tensor* q_norm, const Tensor* k_norm,
                       float norm_eps, float norm_constant_bias, int32_t* err_flag, const Stream& s) const
{
    ffi::rope_paged_kv(q, q, k, &k, v, inv_freq_t_, 0, &cache_seqlens, q_norm, k_norm, norm_eps, norm_constant_bias,
                       style_, attn_factor_, k_cache, v_cache, block_table, cache_seqlens, err_flag, s);
}

void RoPE::apply_one(const Tensor& x, int64_t position, const Tensor* positions, const Tensor* norm, float norm_eps,
                     float norm_constant_bias, const Stream& s) const
{
    ffi::rope(x, x, nullptr, nullptr, inv_freq_t_, position, positions, norm, nullptr, norm_eps, norm_constant_bias,
              style_, attn_factor_, s);
}

}  // namespace exl3r
