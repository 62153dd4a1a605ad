// GPU checks of the C++ host layer: each module (RmsNorm, Embedding, GatedMlp, RoPE) runs through
// the C ABI on a HIP stream and is compared with the CPU oracle on the same bits.
#include "exl3r.hpp"
#include "rowops_oracle.h"

#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <vector>

using namespace exl3r;

static int failures = 0;
static uint64_t rng_state = 0x9e3779b97f4a7c15ull;

static uint64_t splitmix()
{
    uint64_t z = (rng_state += 0x9e3779b97f4a7c15ull);
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
}

static float normal(float mean, float std)
{
    const double u1 = ((splitmix() >> 11) + 1) * 0x1.0p-53, u2 = (splitmix() >> 11) * 0x1.0p-53;
    return (float)(mean + std * std::sqrt(-2.0 * std::log(u1)) * std::cos(2.0 * M_PI * u2));
}

// Host storage of n elements of dtype dt with N(mean, std) values rounded to dt.
static std::vector<uint8_t> host_normal(DType dt, size_t n, float mean, float std)
{
    std::vector<uint8_t> b(n * dtype_size(dt));
    for (size_t i = 0; i < n; ++i)
    {
        const float v = normal(mean, std);
        if (dt == DType::F32) std::memcpy(&b[i * 4], &v, 4);
        else
        {
            const uint16_t h = dt == DType::F16 ? oracle_f32_to_f16(v) : oracle_f32_to_bf16(v);
            std::memcpy(&b[i * 2], &h, 2);
        }
    }
    return b;
}

static OwnedTensor upload(const std::vector<uint8_t>& h, DType dt, std::vector<int64_t> shape, const Stream& s)
{
    OwnedTensor t = OwnedTensor::empty(dt, shape);
    t.buf.upload(h.data(), h.size(), s);
    return t;
}

static std::vector<uint8_t> download(const OwnedTensor& t, const Stream& s)
{
    std::vector<uint8_t> h(t.buf.bytes());
    t.buf.download(h.data(), h.size(), s);
    return h;
}

static void hip_ok(hipError_t e, const char* what)
{
    if (e != hipSuccess)
    {
        std::printf("FAIL %s: %s\n", what, hipGetErrorString(e));
        std::exit(1);
    }
}

// A contiguous view's bytes (arena outputs).
static std::vector<uint8_t> download(const Tensor& t, const Stream& s)
{
    std::vector<uint8_t> h((size_t)t.numel() * dtype_size(t.dtype));
    hip_ok(hipMemcpyAsync(h.data(), t.data, h.size(), hipMemcpyDeviceToHost, s.get()), "hipMemcpyAsync D2H");
    s.synchronize();
    return h;
}

static int64_t ordered16(uint16_t b) { return (b & 0x8000) ? -(int64_t)(b & 0x7fff) : (int64_t)b; }

// Max ulp distance of two 16-bit storage arrays.
static int64_t max_ulp16(const std::vector<uint8_t>& a, const std::vector<uint8_t>& b)
{
    int64_t worst = 0;
    for (size_t i = 0; i + 1 < a.size(); i += 2)
    {
        uint16_t x, y;
        std::memcpy(&x, &a[i], 2);
        std::memcpy(&y, &b[i], 2);
        const int64_t d = std::llabs(ordered16(x) - ordered16(y));
        worst = d > worst ? d : worst;
    }
    return worst;
}

static void report(const char* what, bool ok, const char* detail)
{
    std::printf("%s %s: %s\n", ok ? "ok  " : "FAIL", what, detail);
    if (!ok) ++failures;
}

int main()
{
    Stream s = Stream::create();
    char msg[256];
    Arena arena(64 << 20);   // module outputs (no allocation inside a module call)

    // RmsNorm::forward on a 3-D f16 tensor (rows collapse to 21 x 512), f16 weight.
    {
        auto xh = host_normal(DType::F16, 3 * 7 * 512, 0.f, 1.f);
        auto wh = host_normal(DType::F16, 512, 1.f, 0.1f);
        auto x = upload(xh, DType::F16, { 3, 7, 512 }, s);
        auto w = upload(wh, DType::F16, { 512 }, s);
        RmsNorm norm(w.t, 1e-6f);
        auto y = norm.forward(x.t, arena, s);
        auto yh = download(y, s);
        std::vector<uint8_t> ey(yh.size());
        oracle_rms_norm(xh.data(), OR_F16, 512, wh.data(), OR_F16, ey.data(), OR_F16, 512, nullptr, OR_F32, 512, 21, 512,
                        1e-6f, 0.f, 1.f, 1);
        const int64_t u = max_ulp16(yh, ey);
        std::snprintf(msg, sizeof msg, "max ulp %lld", (long long)u);
        report("RmsNorm::forward f16 [3,7,512]", u <= 1, msg);
    }
    // RmsNorm::forward_res: f32 residual stream + f16 sublayer output (the Qwen3 path, norm.cu:403).
    {
        auto rh = host_normal(DType::F32, 8 * 1024, 0.f, 4.f);
        auto ah = host_normal(DType::F16, 8 * 1024, 0.f, 1.f);
        auto wh = host_normal(DType::F16, 1024, 1.f, 0.1f);
        auto r = upload(rh, DType::F32, { 1, 8, 1024 }, s);
        auto add = upload(ah, DType::F16, { 1, 8, 1024 }, s);
        auto w = upload(wh, DType::F16, { 1024 }, s);
        RmsNorm norm(w.t, 1e-6f, 1.0f);
        auto y = norm.forward_res(r.t, &add.t, arena, s);
        auto yh = download(y, s), rh2 = download(r, s);
        std::vector<uint8_t> ey(yh.size()), er = rh;
        oracle_rms_norm(ah.data(), OR_F16, 1024, wh.data(), OR_F16, ey.data(), OR_F16, 1024, er.data(), OR_F32, 1024, 8,
                        1024, 1e-6f, 1.0f, 1.f, 1);
        const int64_t u = max_ulp16(yh, ey);
        const bool r_ok = std::memcmp(rh2.data(), er.data(), er.size()) == 0;
        std::snprintf(msg, sizeof msg, "y max ulp %lld, residual bit-exact %s", (long long)u, r_ok ? "yes" : "no");
        report("RmsNorm::forward_res f32 residual", u <= 1 && r_ok, msg);
    }
    // RmsNorm::forward_res with a residual that is not contiguous (tokens 1..3 of each sequence of a
    // [2, 5, 256] f32 buffer): the reference's unfused path, y = norm(r + add) with r unchanged
    // (src/modules.rs:393-395), formed in a scratch tensor from the arena.
    {
        const int64_t B = 2, S = 5, T = 3, D = 256;
        auto bh = host_normal(DType::F32, B * S * D, 0.f, 4.f);
        auto ah = host_normal(DType::F16, B * T * D, 0.f, 1.f);
        auto wh = host_normal(DType::F16, D, 1.f, 0.1f);
        auto big = upload(bh, DType::F32, { B, S, D }, s);
        auto add = upload(ah, DType::F16, { B, T, D }, s);
        auto w = upload(wh, DType::F16, { D }, s);
        const Tensor r((char*)big.t.data + D * 4, DType::F32, { B, T, D }, { S * D, D, 1 });
        RmsNorm norm(w.t, 1e-6f);
        auto y = norm.forward_res(r, &add.t, arena, s);
        auto yh = download(y, s), bh2 = download(big, s);
        std::vector<uint8_t> rc((size_t)(B * T * D) * 4), ey(yh.size());
        for (int64_t b = 0; b < B; ++b)
            std::memcpy(&rc[(size_t)(b * T * D) * 4], &bh[(size_t)((b * S + 1) * D) * 4], (size_t)(T * D) * 4);
        oracle_rms_norm(ah.data(), OR_F16, D, wh.data(), OR_F16, ey.data(), OR_F16, D, rc.data(), OR_F32, D, B * T, D,
                        1e-6f, 0.f, 1.f, 1);
        const int64_t u = max_ulp16(yh, ey);
        const bool r_ok = std::memcmp(bh2.data(), bh.data(), bh.size()) == 0;
        std::snprintf(msg, sizeof msg, "y max ulp %lld, residual buffer unchanged %s", (long long)u, r_ok ? "yes" : "no");
        report("RmsNorm::forward_res non-contiguous residual (unfused path)", u <= 1 && r_ok && y.shape == r.shape, msg);
    }
    // Embedding::forward: bf16 table -> f32 rows (exact upcast), ids [2, 5] int64.
    {
        auto th = host_normal(DType::BF16, 100 * 64, 0.f, 0.02f);
        std::vector<int64_t> ids = { 3, 99, 0, 3, 50, 1, 2, 97, 42, 7 };
        auto table = upload(th, DType::BF16, { 100, 64 }, s);
        OwnedTensor idt = OwnedTensor::empty(DType::I64, { 2, 5 });
        idt.buf.upload(ids.data(), ids.size() * 8, s);
        Embedding emb(table.t);
        auto out = emb.forward(idt.t, arena, s);
        auto oh = download(out, s);
        std::vector<uint8_t> eo(oh.size());
        int32_t err = 0;
        oracle_embedding(th.data(), OR_BF16, 100, 64, 64, ids.data(), OR_I64, 10, eo.data(), OR_F32, 64, &err, 1);
        const bool ok = out.shape == std::vector<int64_t>({ 2, 5, 64 }) && std::memcmp(oh.data(), eo.data(), eo.size()) == 0;
        report("Embedding::forward bf16 -> f32", ok, ok ? "bit-exact" : "mismatch");
    }
    // GatedMlp::activate (SiLU and GELU), bf16 [16, 256].
    for (int act = 0; act < 2; ++act)
    {
        auto gh = host_normal(DType::BF16, 16 * 256, 0.f, 2.f);
        auto uh = host_normal(DType::BF16, 16 * 256, 0.f, 1.f);
        auto g = upload(gh, DType::BF16, { 16, 256 }, s);
        auto u = upload(uh, DType::BF16, { 16, 256 }, s);
        auto a = GatedMlp::activate(g.t, u.t, act ? GatedMlp::Act::Gelu : GatedMlp::Act::Silu, 0.f, arena, s);
        auto ah = download(a, s);
        std::vector<uint8_t> ea(ah.size());
        oracle_act_mul(act ? OR_ACT_GELU : OR_ACT_SILU, gh.data(), uh.data(), OR_BF16, ea.data(), OR_BF16, 16, 256, 256,
                       256, 256, 0.f, 1);
        const int64_t d = max_ulp16(ah, ea);
        std::snprintf(msg, sizeof msg, "max ulp %lld", (long long)d);
        report(act ? "GatedMlp::activate gelu" : "GatedMlp::activate silu", d <= 1, msg);
    }
    // RoPE::apply (NeoX, f16 heads, f16 head-norm weights, per-sequence positions) and apply_one.
    {
        const int bsz = 2, seq = 3, hq = 4, hk = 2, hd = 64;
        auto qh = host_normal(DType::F16, bsz * seq * hq * hd, 0.f, 1.f);
        auto kh = host_normal(DType::F16, bsz * seq * hk * hd, 0.f, 1.f);
        auto qnh = host_normal(DType::F16, hd, 1.f, 0.1f), knh = host_normal(DType::F16, hd, 1.f, 0.1f);
        std::vector<int32_t> pos = { 17, 30000 };
        auto q = upload(qh, DType::F16, { bsz, seq, hq, hd }, s);
        auto k = upload(kh, DType::F16, { bsz, seq, hk, hd }, s);
        auto qn = upload(qnh, DType::F16, { hd }, s), kn = upload(knh, DType::F16, { hd }, s);
        OwnedTensor pd = OwnedTensor::empty(DType::I32, { bsz });
        pd.buf.upload(pos.data(), pos.size() * 4, s);
        RoPE rope(1e6, hd, RopeStyle::NeoX);
        rope.apply(q.t, k.t, 0, &pd.t, &qn.t, &kn.t, 1e-6f, 0.f, s);
        auto qo = download(q, s), ko = download(k, s);
        std::vector<uint8_t> eq(qh.size()), ek(kh.size());
        oracle_rope(qh.data(), eq.data(), hq * hd, hd, hq, kh.data(), ek.data(), hk * hd, hd, hk, OR_F16, bsz, seq, hd,
                    rope.inv_freq_host().data(), hd, 0, pos.data(), nullptr, qnh.data(), knh.data(), OR_F16, 1e-6f, 0.f,
                    OR_ROPE_NEOX, 1.f, 1);
        const int64_t dq = max_ulp16(qo, eq), dk = max_ulp16(ko, ek);
        std::snprintf(msg, sizeof msg, "q max ulp %lld, k max ulp %lld", (long long)dq, (long long)dk);
        report("RoPE::apply neox f16 + head norm", dq <= 2 && dk <= 2, msg);

        auto xh = host_normal(DType::F16, seq * hq * hd, 0.f, 1.f);
        auto x = upload(xh, DType::F16, { 1, seq, hq, hd }, s);
        RoPE gptj(1e4, 32, RopeStyle::GptJ);
        gptj.apply_one(x.t, 5, nullptr, nullptr, 1e-6f, 0.f, s);
        auto xo = download(x, s);
        std::vector<uint8_t> ex(xh.size());
        oracle_rope(xh.data(), ex.data(), hq * hd, hd, hq, nullptr, nullptr, 0, 0, 0, OR_F16, 1, seq, hd,
                    gptj.inv_freq_host().data(), 32, 5, nullptr, nullptr, nullptr, nullptr, OR_F16, 1e-6f, 0.f,
                    OR_ROPE_GPTJ, 1.f, 1);
        const int64_t dx = max_ulp16(xo, ex);
        std::snprintf(msg, sizeof msg, "max ulp %lld", (long long)dx);
        report("RoPE::apply_one gptj partial rotary", dx <= 2, msg);

        // RoPE::apply with a freq_table of arbitrary angles (MRoPE-style), [50, hd/2], shared by both sequences.
        std::vector<float> table(50 * hd / 2);
        for (size_t i = 0; i < table.size(); ++i) table[i] = normal(0.f, 300.f);
        OwnedTensor tab = OwnedTensor::empty(DType::F32, { 50, hd / 2 });
        tab.buf.upload(table.data(), table.size() * 4, s);
        std::vector<int32_t> tpos = { 3, 40 };
        pd.buf.upload(tpos.data(), tpos.size() * 4, s);
        auto q2 = upload(qh, DType::F16, { bsz, seq, hq, hd }, s);
        auto k2 = upload(kh, DType::F16, { bsz, seq, hk, hd }, s);
        rope.apply(q2.t, k2.t, 0, &pd.t, &qn.t, &kn.t, 1e-6f, 0.f, s, &tab.t);
        auto q2o = download(q2, s), k2o = download(k2, s);
        int32_t terr = 0;
        oracle_rope_table(qh.data(), eq.data(), hq * hd, hd, hq, kh.data(), ek.data(), hk * hd, hd, hk, OR_F16, bsz, seq,
                          hd, table.data(), 50, 0, hd, 0, tpos.data(), nullptr, qnh.data(), knh.data(), OR_F16, 1e-6f,
                          0.f, OR_ROPE_NEOX, 1.f, &terr, 1);
        const int64_t tq = max_ulp16(q2o, eq), tk = max_ulp16(k2o, ek);
        std::snprintf(msg, sizeof msg, "q max ulp %lld, k max ulp %lld", (long long)tq, (long long)tk);
        report("RoPE::apply with freq_table", tq <= 2 && tk <= 2 && terr == 0, msg);
    }
    // RoPE::apply_paged: rope + paged KV append (16-token pages, positions = cache lengths).
    {
        const int bsz = 2, seq = 5, hq = 4, hk = 2, hd = 64, page = 16, pages = 9, max_blocks = 4;
        auto qh = host_normal(DType::F16, bsz * seq * hq * hd, 0.f, 1.f);
        auto kh = host_normal(DType::F16, bsz * seq * hk * hd, 0.f, 1.f);
        auto vh = host_normal(DType::F16, bsz * seq * hk * hd, 0.f, 1.f);
        auto kch = host_normal(DType::F16, (size_t)pages * page * hk * hd, 0.f, 1.f);
        auto vch = host_normal(DType::F16, (size_t)pages * page * hk * hd, 0.f, 1.f);
        auto qnh = host_normal(DType::F16, hd, 1.f, 0.1f), knh = host_normal(DType::F16, hd, 1.f, 0.1f);
        std::vector<int32_t> lens = { 14, 40 }, table = { 3, 0, 7, 5, 1, 8, 2, 6 };
        auto q = upload(qh, DType::F16, { bsz, seq, hq, hd }, s);
        auto k = upload(kh, DType::F16, { bsz, seq, hk, hd }, s);
        auto v = upload(vh, DType::F16, { bsz, seq, hk, hd }, s);
        auto kc = upload(kch, DType::F16, { pages, page, hk, hd }, s);
        auto vc = upload(vch, DType::F16, { pages, page, hk, hd }, s);
        auto qn = upload(qnh, DType::F16, { hd }, s), kn = upload(knh, DType::F16, { hd }, s);
        OwnedTensor ld = OwnedTensor::empty(DType::I32, { bsz }), bt = OwnedTensor::empty(DType::I32, { bsz, max_blocks });
        ld.buf.upload(lens.data(), lens.size() * 4, s);
        bt.buf.upload(table.data(), table.size() * 4, s);
        RoPE rope(1e6, hd, RopeStyle::NeoX);
        rope.apply_paged(q.t, k.t, v.t, kc.t, vc.t, bt.t, ld.t, &qn.t, &kn.t, 1e-6f, 0.f, nullptr, s);
        auto qo = download(q, s), ko = download(k, s), kco = download(kc, s), vco = download(vc, s);
        std::vector<uint8_t> eq(qh.size()), ek(kh.size());
        oracle_rope(qh.data(), eq.data(), hq * hd, hd, hq, kh.data(), ek.data(), hk * hd, hd, hk, OR_F16, bsz, seq, hd,
                    rope.inv_freq_host().data(), hd, 0, lens.data(), nullptr, qnh.data(), knh.data(), OR_F16, 1e-6f, 0.f,
                    OR_ROPE_NEOX, 1.f, 1);
        oracle_paged_kv_append(ek.data(), hk * hd, hd, vh.data(), hk * hd, hd, hk, OR_F16, bsz, seq, hd, kch.data(),
                               vch.data(), page, pages, table.data(), max_blocks, lens.data(), nullptr, 1);
        const int64_t dq = max_ulp16(qo, eq), dk = max_ulp16(ko, ek);
        const bool caches = kco == kch && vco == vch;
        std::snprintf(msg, sizeof msg, "q max ulp %lld, k max ulp %lld, caches %s", (long long)dq, (long long)dk,
                      caches ? "bitwise" : "DIFFER");
        report("RoPE::apply_paged neox f16 + paged append", dq == 0 && dk == 0 && caches, msg);
    }
    // Gated ops: gated_rms_norm (bf16 x, f32 gate and weight, f16 y), mul_sigmoid_, deinterleave_qg.
    {
        const int rows = 40, dim = 128, heads = 4, hd = 32;
        auto xh = host_normal(DType::BF16, rows * dim, 0.f, 1.f);
        auto gh = host_normal(DType::F32, rows * dim, 0.f, 2.f);
        auto wh = host_normal(DType::F32, dim, 1.f, 0.1f);
        auto x = upload(xh, DType::BF16, { rows, dim }, s), g = upload(gh, DType::F32, { rows, dim }, s);
        auto w = upload(wh, DType::F32, { dim }, s);
        OwnedTensor y = OwnedTensor::empty(DType::F16, { rows, dim });
        ffi::gated_rms_norm(x.t, &w.t, y.t, g.t, 1e-6f, 0.f, 1, false, 0, s);
        auto yo = download(y, s);
        std::vector<uint8_t> ey(yo.size());
        oracle_gated_rms_norm(xh.data(), OR_BF16, dim, wh.data(), OR_F32, 1, ey.data(), OR_F16, dim, gh.data(), OR_F32,
                              dim, rows, dim, 1e-6f, 0.f, 0, 0, 1);
        const int64_t dy = max_ulp16(yo, ey);
        std::snprintf(msg, sizeof msg, "max ulp %lld", (long long)dy);
        report("ffi::gated_rms_norm silu gate", dy <= 1, msg);

        auto ah = host_normal(DType::F16, rows * dim, 0.f, 2.f), bh = host_normal(DType::F16, rows * dim, 0.f, 3.f);
        auto av = upload(ah, DType::F16, { rows, dim }, s), bv = upload(bh, DType::F16, { rows, dim }, s);
        ffi::mul_sigmoid_(av.t, bv.t, s);
        auto ao = download(av, s);
        std::vector<uint8_t> ea(ao.size());
        oracle_act_mul(OR_ACT_SIGMOID, bh.data(), ah.data(), OR_F16, ea.data(), OR_F16, rows, dim, dim, dim, dim, 0.f, 1);
        const int64_t da = max_ulp16(ao, ea);
        std::snprintf(msg, sizeof msg, "max ulp %lld", (long long)da);
        report("ffi::mul_sigmoid_", da <= 1, msg);

        auto qgh = host_normal(DType::F16, rows * heads * 2 * hd, 0.f, 1.f);
        auto qg = upload(qgh, DType::F16, { rows, heads * 2 * hd }, s);
        OwnedTensor q = OwnedTensor::empty(DType::F16, { rows, heads, hd }), gg = OwnedTensor::empty(DType::F16, { rows, heads * hd });
        ffi::deinterleave_qg(qg.t, q.t, gg.t, hd, s);
        auto qo = download(q, s), go = download(gg, s);
        std::vector<uint8_t> eq(qo.size()), eg(go.size());
        oracle_deinterleave_qg(qgh.data(), heads * 2 * hd, eq.data(), heads * hd, eg.data(), heads * hd, rows, heads, hd, 1);
        report("ffi::deinterleave_qg", qo == eq && go == eg, qo == eq && go == eg ? "bitwise" : "DIFFER");
    }
    // argmax_sample: bf16 logits [6, 9000] with planted ties, masked to the first 8001 columns.
    {
        const int rows = 6, vocab = 9000, mask = 8001;
        auto lh = host_normal(DType::BF16, rows * vocab, 0.f, 2.f);
        const uint16_t big = oracle_f32_to_bf16(40.f);
        for (int r = 0; r < rows; ++r)
        {
            std::memcpy(&lh[(r * vocab + 100 * r + 7) * 2], &big, 2);
            std::memcpy(&lh[(r * vocab + 7900) * 2], &big, 2);
            std::memcpy(&lh[(r * vocab + 8500) * 2], &big, 2);
        }
        auto l = upload(lh, DType::BF16, { rows, vocab }, s);
        auto ids = OwnedTensor::empty(DType::I64, { rows });
        ffi::argmax_sample(l.t, ids.t, mask, s);
        auto got = download(ids, s);
        std::vector<int64_t> want(rows);
        oracle_argmax(lh.data(), OR_BF16, rows, vocab, vocab, mask, want.data(), 1);
        const bool ok = std::memcmp(got.data(), want.data(), rows * 8) == 0 && want[3] == 307;
        report("ffi::argmax_sample bf16 masked", ok, ok ? "exact" : "DIFFER");
        // The one-launch form with a workspace (zeroed once), twice in a row on one workspace.
        DeviceBuffer ws(exl3r_sample_workspace_bytes());
        hip_ok(hipMemsetAsync(ws.data(), 0, ws.bytes(), s.get()), "hipMemsetAsync");
        auto ids_ws = OwnedTensor::empty(DType::I64, { rows });
        bool ok_ws = true;
        for (int rep = 0; rep < 2; ++rep)
        {
            ffi::argmax_sample_ws(l.t, ids_ws.t, mask, ws, s);
            ok_ws = ok_ws && std::memcmp(download(ids_ws, s).data(), want.data(), rows * 8) == 0;
        }
        report("ffi::argmax_sample_ws bf16 masked, workspace reused", ok_ws, ok_ws ? "exact" : "DIFFER");
    }
    // gumbel_noise (f16 -> f32) and gumbel_sample on the same logits: bitwise noise, equal ids, and the
    // sample equals the argmax of the noisy logits.
    {
        const int rows = 5, vocab = 3001;
        const uint32_t seed = 0xC0FFEEu;
        auto lh = host_normal(DType::F16, rows * vocab, 0.f, 3.f);
        auto l = upload(lh, DType::F16, { rows, vocab }, s);
        auto noisy = OwnedTensor::empty(DType::F32, { rows, vocab });
        auto ids = OwnedTensor::empty(DType::I64, { rows });
        auto ids2 = OwnedTensor::empty(DType::I64, { rows });
        ffi::gumbel_noise(l.t, noisy.t, seed, s);
        ffi::gumbel_sample(l.t, ids.t, 0, seed, s);
        ffi::argmax_sample(noisy.t, ids2.t, 0, s);
        auto gn = download(noisy, s), gi = download(ids, s), gi2 = download(ids2, s);
        std::vector<uint8_t> en(gn.size());
        std::vector<int64_t> ei(rows);
        oracle_gumbel_noise(lh.data(), OR_F16, vocab, en.data(), OR_F32, vocab, rows, vocab, seed, 1);
        oracle_gumbel_sample(lh.data(), OR_F16, rows, vocab, vocab, 0, seed, ei.data(), 1);
        const bool ok = gn == en && std::memcmp(gi.data(), ei.data(), rows * 8) == 0 && gi == gi2;
        report("ffi::gumbel_noise / gumbel_sample", ok, ok ? "noise bitwise, ids exact" : "DIFFER");
    }
    // had_r_128 with suh, then the fused residual norm -> q/k/v inputs and the fused SiLU -> down_proj
    // input, each bitwise against the oracle composition.
    {
        const int rows = 12, dim = 512;
        std::vector<uint8_t> sh(dim * 2);
        for (int i = 0; i < dim; ++i)
        {
            const uint16_t v = (splitmix() & 1) ? 0xbc00 : 0x3c00;   // -1.0 / +1.0 in f16
            std::memcpy(&sh[i * 2], &v, 2);
        }
        auto suh = upload(sh, DType::F16, { dim }, s);
        auto xh = host_normal(DType::F16, rows * dim, 0.f, 1.f);
        auto x = upload(xh, DType::F16, { rows, dim }, s);
        auto hx = OwnedTensor::empty(DType::F16, { rows, dim });
        ffi::had_r_128(x.t, hx.t, &suh.t, nullptr, 1.f, s);
        std::vector<uint8_t> eh(xh.size());
        oracle_had_r_128(xh.data(), OR_F16, dim, eh.data(), dim, rows, dim, (const uint16_t*)sh.data(), nullptr, 1.f, 1);
        bool ok = download(hx, s) == eh;
        report("ffi::had_r_128 f16 with suh", ok, ok ? "bitwise" : "DIFFER");

        auto rh = host_normal(DType::F32, rows * dim, 0.f, 4.f);
        auto wh = host_normal(DType::F16, dim, 1.f, 0.1f);
        auto r = upload(rh, DType::F32, { rows, dim }, s);
        auto w = upload(wh, DType::F16, { dim }, s);
        auto o0 = OwnedTensor::empty(DType::F16, { rows, dim }), o1 = OwnedTensor::empty(DType::F16, { rows, dim });
        ffi::rms_norm_had(x.t, &w.t, &r.t, nullptr, { &o0.t, &o1.t }, { &suh.t, nullptr }, 1e-6f, 0.f, 1.f, 1.f, s,
                          false, nullptr, true);
        std::vector<uint8_t> ey(xh.size()), er = rh, e0(xh.size()), e1(xh.size());
        oracle_rms_norm(xh.data(), OR_F16, dim, wh.data(), OR_F16, ey.data(), OR_F16, dim, er.data(), OR_F32, dim, rows, dim,
                        1e-6f, 0.f, 1.f, 1);
        oracle_had_r_128(ey.data(), OR_F16, dim, e0.data(), dim, rows, dim, (const uint16_t*)sh.data(), nullptr, 1.f, 1);
        oracle_had_r_128(ey.data(), OR_F16, dim, e1.data(), dim, rows, dim, nullptr, nullptr, 1.f, 1);
        ok = download(o0, s) == e0 && download(o1, s) == e1 && download(r, s) == er;
        report("ffi::rms_norm_had residual, 2 outputs", ok, ok ? "bitwise" : "DIFFER");

        auto gh = host_normal(DType::F16, rows * dim, 0.f, 2.f);
        auto g = upload(gh, DType::F16, { rows, dim }, s);
        auto z = OwnedTensor::empty(DType::F16, { rows, dim }), hz = OwnedTensor::empty(DType::F16, { rows, dim });
        ffi::act_mul_had(ffi::HadAct::Silu, g.t, x.t, hz.t, &suh.t, &z.t, 0.f, 1.f, s, false, false, nullptr, nullptr,
                         true);
        auto zh = download(z, s);
        std::vector<uint8_t> ez(zh.size()), ehz(zh.size());
        oracle_act_mul(0, gh.data(), xh.data(), OR_F16, ez.data(), OR_F16, rows, dim, dim, dim, dim, 0.f, 1);
        oracle_had_r_128(zh.data(), OR_F16, dim, ehz.data(), dim, rows, dim, (const uint16_t*)sh.data(), nullptr, 1.f, 1);
        const int64_t u = max_ulp16(zh, ez);
        ok = u <= 1 && download(hz, s) == ehz;
        std::snprintf(msg, sizeof msg, "z max ulp %lld, rotation of z bitwise", (long long)u);
        report("ffi::act_mul_had silu -> had", ok, ok ? msg : "DIFFER");
    }
    // rope_had (exact: the butterfly): the q / k output rotations then head-norm + NeoX RoPE, equal to
    // had_r_128 then rope.
    {
        const int T = 1100, hq = 4, hk = 2, hd = 128;
        auto qh = host_normal(DType::F16, T * hq * hd, 0.f, 2.f), kh = host_normal(DType::F16, T * hk * hd, 0.f, 2.f);
        auto nh = host_normal(DType::F16, hd, 1.f, 0.1f);
        std::vector<uint8_t> sq(hq * hd * 2);
        for (int i = 0; i < hq * hd; ++i)
        {
            const uint16_t v = (splitmix() & 1) ? 0xbc00 : 0x3c00;
            std::memcpy(&sq[i * 2], &v, 2);
        }
        std::vector<float> fh(hd / 2);
        for (int i = 0; i < hd / 2; ++i) fh[i] = (float)(1.0 / std::pow(1e6, 2.0 * i / hd));
        std::vector<uint8_t> fb(fh.size() * 4);
        std::memcpy(fb.data(), fh.data(), fb.size());
        auto q = upload(qh, DType::F16, { 1, T, hq, hd }, s), k = upload(kh, DType::F16, { 1, T, hk, hd }, s);
        auto q2 = upload(qh, DType::F16, { 1, T, hq, hd }, s), k2 = upload(kh, DType::F16, { 1, T, hk, hd }, s);
        auto qn = upload(nh, DType::F16, { hd }, s), svq = upload(sq, DType::F16, { hq * hd }, s);
        auto f = upload(fb, DType::F32, { hd / 2 }, s);
        ffi::rope_had(q.t, q.t, &k.t, &k.t, f.t, 5, nullptr, &qn.t, &qn.t, 1e-6f, 0.f, RopeStyle::NeoX, 1.f, &svq.t,
                      nullptr, s, nullptr, nullptr, true);
        Tensor q2v(q2.t.data, DType::F16, { T, hq * hd }), k2v(k2.t.data, DType::F16, { T, hk * hd });
        ffi::had_r_128(q2v, q2v, nullptr, &svq.t, 1.f, s);
        ffi::had_r_128(k2v, k2v, nullptr, nullptr, 1.f, s);
        ffi::rope(q2.t, q2.t, &k2.t, &k2.t, f.t, 5, nullptr, &qn.t, &qn.t, 1e-6f, 0.f, RopeStyle::NeoX, 1.f, s);
        const bool ok = download(q, s) == download(q2, s) && download(k, s) == download(k2, s);
        report("ffi::rope_had exact == had_r_128 + rope", ok, ok ? "bitwise" : "DIFFER");
    }
    // rope_cs: RoPE from a {cos, sin} table built once, bitwise equal to rope() evaluating sin / cos.
    {
        const int T = 1200, hq = 8, hk = 2, hd = 128;
        auto qh = host_normal(DType::BF16, T * hq * hd, 0.f, 1.f), kh = host_normal(DType::BF16, T * hk * hd, 0.f, 1.f);
        auto nh = host_normal(DType::F32, hd, 1.f, 0.1f);
        std::vector<float> fh(hd / 2);
        for (int i = 0; i < hd / 2; ++i) fh[i] = (float)(1.0 / std::pow(1e6, 2.0 * i / hd));
        std::vector<uint8_t> fb(fh.size() * 4);
        std::memcpy(fb.data(), fh.data(), fb.size());
        auto q = upload(qh, DType::BF16, { 1, T, hq, hd }, s), k = upload(kh, DType::BF16, { 1, T, hk, hd }, s);
        auto q2 = upload(qh, DType::BF16, { 1, T, hq, hd }, s), k2 = upload(kh, DType::BF16, { 1, T, hk, hd }, s);
        auto qn = upload(nh, DType::F32, { hd }, s), f = upload(fb, DType::F32, { hd / 2 }, s);
        auto cs = OwnedTensor::empty(DType::F32, { T, hd / 2, 2 });
        ffi::rope_cs_table(1, T, f.t, 3000, nullptr, nullptr, 1.f, cs.t, s);
        ffi::rope_cs(q.t, q.t, &k.t, &k.t, cs.t, &qn.t, &qn.t, 1e-6f, 0.f, RopeStyle::NeoX, s);
        ffi::rope(q2.t, q2.t, &k2.t, &k2.t, f.t, 3000, nullptr, &qn.t, &qn.t, 1e-6f, 0.f, RopeStyle::NeoX, 1.f, s);
        const bool ok = download(q, s) == download(q2, s) && download(k, s) == download(k2, s);
        report("ffi::rope_cs_table + rope_cs == rope", ok, ok ? "bitwise" : "DIFFER");
    }
    // rope_qg: q read from the interleaved q | g projection, bitwise equal to deinterleave_qg + rope.
    {
        const int T = 1100, hq = 4, hk = 2, hd = 128;
        auto qgh = host_normal(DType::F16, T * hq * 2 * hd, 0.f, 1.f), kh = host_normal(DType::F16, T * hk * hd, 0.f, 1.f);
        auto nh = host_normal(DType::F16, hd, 0.f, 0.1f);
        std::vector<float> fh(hd / 2);
        for (int i = 0; i < hd / 2; ++i) fh[i] = (float)(1.0 / std::pow(1e6, 2.0 * i / hd));
        std::vector<uint8_t> fb(fh.size() * 4);
        std::memcpy(fb.data(), fh.data(), fb.size());
        auto qg = upload(qgh, DType::F16, { 1, T, hq, 2 * hd }, s);
        auto k = upload(kh, DType::F16, { 1, T, hk, hd }, s), k2 = upload(kh, DType::F16, { 1, T, hk, hd }, s);
        auto qn = upload(nh, DType::F16, { hd }, s), f = upload(fb, DType::F32, { hd / 2 }, s);
        auto oq = OwnedTensor::empty(DType::F16, { 1, T, hq, hd }), q = OwnedTensor::empty(DType::F16, { 1, T, hq, hd });
        auto g = OwnedTensor::empty(DType::F16, { 1, T, hq * hd });
        ffi::rope_qg(qg.t, oq.t, &k.t, &k.t, f.t, 9, nullptr, &qn.t, &qn.t, 1e-6f, 1.f, RopeStyle::NeoX, 1.f, s);
        Tensor qgv(qg.t.data, DType::F16, { 1, T, hq * 2 * hd });
        ffi::deinterleave_qg(qgv, q.t, g.t, hd, s);
        ffi::rope(q.t, q.t, &k2.t, &k2.t, f.t, 9, nullptr, &qn.t, &qn.t, 1e-6f, 1.f, RopeStyle::NeoX, 1.f, s);
        const bool ok = download(oq, s) == download(q, s) && download(k, s) == download(k2, s);
        report("ffi::rope_qg == deinterleave_qg + rope", ok, ok ? "bitwise" : "DIFFER");
    }
    // gated_rms_norm_had: the GDN output norm (8 tokens x 4 heads of 128, one o_proj row per token)
    // into o_proj's input rotation (exact: the butterfly), bitwise equal to the gated norm followed by had_r_128.
    {
        const int heads = 4, rows = 8 * heads, dim = 128;
        auto xh = host_normal(DType::BF16, rows * dim, 0.f, 1.f), gh = host_normal(DType::F32, rows * dim, 0.f, 2.f);
        auto wh = host_normal(DType::F32, dim, 1.f, 0.1f);
        std::vector<uint8_t> sh(heads * dim * 2);
        for (int i = 0; i < heads * dim; ++i)
        {
            const uint16_t v = (splitmix() & 1) ? 0xbc00 : 0x3c00;
            std::memcpy(&sh[i * 2], &v, 2);
        }
        auto x = upload(xh, DType::BF16, { rows, dim }, s), g = upload(gh, DType::F32, { rows, dim }, s);
        auto w = upload(wh, DType::F32, { dim }, s), sv = upload(sh, DType::F16, { heads * dim }, s);
        auto out = OwnedTensor::empty(DType::F16, { rows, dim }), y = OwnedTensor::empty(DType::F16, { rows, dim });
        auto ref = OwnedTensor::empty(DType::F16, { rows / heads, heads * dim });
        ffi::gated_rms_norm_had(x.t, &w.t, g.t, out.t, nullptr, &sv.t, 1e-6f, 0.f, 1, false, 1, 1.f, s, heads, true);
        ffi::gated_rms_norm(x.t, &w.t, y.t, g.t, 1e-6f, 0.f, 1, false, 1, s);
        Tensor yv(y.t.data, DType::F16, { rows / heads, heads * dim });
        ffi::had_r_128(yv, ref.t, &sv.t, nullptr, 1.f, s);
        const bool ok = download(out, s) == download(ref, s);
        report("ffi::gated_rms_norm_had exact == gated norm + had_r_128", ok, ok ? "bitwise" : "DIFFER");
    }
    // Graph capture: RmsNorm::forward_res (output from an arena) and RoPE::apply (positions read from device
    // memory) recorded into a HIP graph in the strict (global) capture mode, which fails any allocation or
    // synchronisation inside the calls; replayed three times with new inputs and positions uploaded eagerly
    // between the replays, every replay checked against the oracle.
    {
        const int T = 8, H = 512, hq = 4, hk = 2, hd = 128;
        Stream cs = Stream::create();
        OwnedTensor r = OwnedTensor::empty(DType::F32, { T, H }), add = OwnedTensor::empty(DType::F16, { T, H });
        OwnedTensor q = OwnedTensor::empty(DType::F16, { T, 1, hq, hd }), k = OwnedTensor::empty(DType::F16, { T, 1, hk, hd });
        OwnedTensor pos = OwnedTensor::empty(DType::I32, { T });
        auto wh = host_normal(DType::F16, H, 1.f, 0.1f);
        auto qnh = host_normal(DType::F16, hd, 1.f, 0.1f), knh = host_normal(DType::F16, hd, 1.f, 0.1f);
        auto w = upload(wh, DType::F16, { H }, cs);
        auto qn = upload(qnh, DType::F16, { hd }, cs), kn = upload(knh, DType::F16, { hd }, cs);
        RmsNorm norm(w.t, 1e-6f, 1.0f);
        RoPE rope(1e6, hd, RopeStyle::NeoX);
        Arena garena(1 << 20);
        hipGraph_t graph = nullptr;
        hipGraphExec_t exec = nullptr;
        hip_ok(hipStreamBeginCapture(cs.get(), hipStreamCaptureModeGlobal), "hipStreamBeginCapture");
        Tensor y = norm.forward_res(r.t, &add.t, garena, cs);
        rope.apply(q.t, k.t, 0, &pos.t, &qn.t, &kn.t, 1e-6f, 0.f, cs);
        hip_ok(hipStreamEndCapture(cs.get(), &graph), "hipStreamEndCapture");
        hip_ok(hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0), "hipGraphInstantiate");
        bool all_ok = true;
        for (int rep = 0; rep < 3; ++rep)
        {
            auto rh = host_normal(DType::F32, T * H, 0.f, 4.f), ah = host_normal(DType::F16, T * H, 0.f, 1.f);
            auto qh = host_normal(DType::F16, T * hq * hd, 0.f, 1.f), kh = host_normal(DType::F16, T * hk * hd, 0.f, 1.f);
            std::vector<int32_t> ph(T);
            for (int i = 0; i < T; ++i) ph[i] = (int32_t)((splitmix() >> 40) % 40000);
            r.buf.upload(rh.data(), rh.size(), cs);
            add.buf.upload(ah.data(), ah.size(), cs);
            q.buf.upload(qh.data(), qh.size(), cs);
            k.buf.upload(kh.data(), kh.size(), cs);
            pos.buf.upload(ph.data(), ph.size() * 4, cs);
            hip_ok(hipGraphLaunch(exec, cs.get()), "hipGraphLaunch");
            cs.synchronize();
            auto yo = download(y, cs), ro = download(r, cs), qo = download(q, cs), ko = download(k, cs);
            std::vector<uint8_t> ey(yo.size()), er = rh, eq(qh.size()), ek(kh.size());
            oracle_rms_norm(ah.data(), OR_F16, H, wh.data(), OR_F16, ey.data(), OR_F16, H, er.data(), OR_F32, H, T, H,
                            1e-6f, 1.0f, 1.f, 1);
            oracle_rope(qh.data(), eq.data(), hq * hd, hd, hq, kh.data(), ek.data(), hk * hd, hd, hk, OR_F16, T, 1, hd,
                        rope.inv_freq_host().data(), hd, 0, ph.data(), nullptr, qnh.data(), knh.data(), OR_F16, 1e-6f,
                        0.f, OR_ROPE_NEOX, 1.f, 1);
            const int64_t dy = max_ulp16(yo, ey), dq = max_ulp16(qo, eq), dk = max_ulp16(ko, ek);
            const bool r_ok = std::memcmp(ro.data(), er.data(), er.size()) == 0;
            std::snprintf(msg, sizeof msg, "replay %d: y max ulp %lld, residual bit-exact %s, q/k max ulp %lld/%lld", rep,
                          (long long)dy, r_ok ? "yes" : "no", (long long)dq, (long long)dk);
            const bool ok = dy <= 1 && r_ok && dq <= 2 && dk <= 2;
            report("captured forward_res + RoPE::apply", ok, msg);
            all_ok = all_ok && ok;
        }
        hip_ok(hipGraphExecDestroy(exec), "hipGraphExecDestroy");
        hip_ok(hipGraphDestroy(graph), "hipGraphDestroy");
        report("graph capture of the module layer (no allocation inside the calls)", all_ok && garena.used() > 0,
               all_ok ? "3 replays" : "mismatch");
    }

    std::printf(failures ? "test_host_gpu: %d failures\n" : "test_host_gpu: all passed\n", failures);
    return failures ? 1 : 0;
}
