// CPU checks of the C++ host layer: argument validation throws exl3r::Error with the C ABI's
// status before any device work, and the default inv_freq producer matches theta^(-2i/d).
// Device pointers are fake (never dereferenced: every call fails validation first).
#include "exl3r.hpp"

#include <cmath>
#include <cstdio>
#include <functional>
#include <string>

using namespace exl3r;

static int failures = 0;

static void expect_error(const char* what, int code, const std::function<void()>& fn)
{
    try
    {
        fn();
        std::printf("FAIL %s: no exception\n", what);
        ++failures;
    }
    catch (const Error& e)
    {
        if (e.code() != code)
        {
            std::printf("FAIL %s: code %d (%s), expected %d\n", what, e.code(), e.what(), code);
            ++failures;
        }
        else
            std::printf("ok   %s: %s\n", what, e.what());
    }
}

int main()
{
    void* fake = (void*)0x1000;
    Stream s;
    Tensor x(fake, DType::F16, { 4, 64 }), y(fake, DType::F16, { 4, 32 }), w(fake, DType::F16, { 64 });
    expect_error("rms_norm shape mismatch", EXL3R_EINVAL, [&] { ffi::rms_norm(x, &w, y, 1e-6f, 0.f, 1.f, s); });
    Tensor xi(fake, DType::I32, { 4, 64 }), y2(Tensor((char*)fake + 4096, DType::F16, { 4, 64 }));
    expect_error("rms_norm bad dtype", EXL3R_EDTYPE, [&] { ffi::rms_norm(xi, &w, y2, 1e-6f, 0.f, 1.f, s); });
    Tensor strided(fake, DType::F16, { 2, 3, 64 }, { 1000, 64, 1 });
    expect_error("rows that do not collapse", EXL3R_EINVAL, [&] { ffi::rms_norm(strided, &w, strided, 1e-6f, 0.f, 1.f, s); });
    Tensor q(fake, DType::F16, { 1, 3, 4, 64 }), k(fake, DType::F16, { 1, 3, 2, 32 }), inv(fake, DType::F32, { 32 });
    expect_error("rope k shape", EXL3R_EINVAL, [&] { ffi::rope(q, q, &k, &k, inv, 0, nullptr, nullptr, nullptr, 1e-6f, 0.f, RopeStyle::NeoX, 1.f, s); });
    Tensor k2(fake, DType::F16, { 1, 3, 2, 64 });
    expect_error("rope style none", EXL3R_EINVAL, [&] { ffi::rope(q, q, &k2, &k2, inv, 0, nullptr, nullptr, nullptr, 1e-6f, 0.f, RopeStyle::None, 1.f, s); });
    expect_error("rope q_norm without k_norm", EXL3R_EINVAL, [&] { ffi::rope(q, q, &k2, &k2, inv, 0, nullptr, &w, nullptr, 1e-6f, 0.f, RopeStyle::NeoX, 1.f, s); });
    Tensor q3(fake, DType::F16, { 3, 4, 64 });
    expect_error("rope q rank", EXL3R_EINVAL, [&] { ffi::rope(q3, q3, nullptr, nullptr, inv, 0, nullptr, nullptr, nullptr, 1e-6f, 0.f, RopeStyle::NeoX, 1.f, s); });
    Tensor table(fake, DType::F32, { 10, 64 }), ids(fake, DType::I64, { 2, 3 }), out16(fake, DType::F16, { 6, 64 });
    expect_error("embedding lossy out dtype", EXL3R_EDTYPE, [&] { ffi::embedding(table, ids, out16, nullptr, s); });
    Tensor out_bad(fake, DType::F32, { 5, 64 });
    expect_error("embedding out rows", EXL3R_EINVAL, [&] { ffi::embedding(table, ids, out_bad, nullptr, s); });
    Tensor g(fake, DType::BF16, { 8, 128 }), u(fake, DType::F16, { 8, 128 }), z(fake, DType::BF16, { 8, 128 });
    expect_error("act dtype mismatch", EXL3R_EINVAL, [&] { ffi::silu_mul(g, u, z, 0.f, s); });
    expect_error("RoPE odd rotary_dim", EXL3R_EINVAL, [&] { RoPE::default_inv_freq(1e6, 63); });
    // RmsNorm::forward_res_into with a residual that is not contiguous takes the reference's unfused path
    // through a caller's scratch: refused without one, with a scratch of another dtype, or for a residual
    // whose last dim is not dense.
    {
        RmsNorm norm(w, 1e-6f);
        Tensor rs(fake, DType::F32, { 2, 3, 64 }, { 1000, 64, 1 }), add(fake, DType::F16, { 2, 3, 64 });
        Tensor yy(fake, DType::F16, { 2, 3, 64 }), sc16(fake, DType::F16, { 2, 3, 64 }), sc(fake, DType::F32, { 2, 3, 64 });
        Tensor rt(fake, DType::F32, { 2, 3, 64 }, { 1000, 1, 3 });
        expect_error("forward_res non-contiguous residual without scratch", EXL3R_EINVAL,
                     [&] { norm.forward_res_into(rs, &add, yy, s); });
        expect_error("forward_res scratch dtype", EXL3R_EINVAL, [&] { norm.forward_res_into(rs, &add, yy, s, &sc16); });
        expect_error("forward_res residual last dim not dense", EXL3R_EINVAL,
                     [&] { norm.forward_res_into(rt, &add, yy, s, &sc); });
    }

    // {cos, sin} tables must cover the call's bsz * seq_len tokens (the kernels index them by token) and
    // match inv_freq's R/2; an angle table is rope()'s input only.
    {
        Tensor q4(fake, DType::F16, { 1, 3, 4, 128 }), k4(fake, DType::F16, { 1, 3, 2, 128 }), v4(fake, DType::F16, { 1, 3, 2, 128 });
        Tensor inv64(fake, DType::F32, { 64 }), angles(fake, DType::F32, { 16, 64 });
        Tensor cs_short(fake, DType::F32, { 2, 64, 2 }), cs_rdim(fake, DType::F32, { 3, 32, 2 }), cs_f16(fake, DType::F16, { 3, 64, 2 });
        Tensor kc(fake, DType::F16, { 4, 256, 2, 128 }), bt(fake, DType::I32, { 1, 2 }), sl(fake, DType::I32, { 1 });
        auto had = [&](const Tensor& inv, const Tensor* cs) {
            ffi::rope_had(q4, q4, &k4, &k4, inv, 0, nullptr, nullptr, nullptr, 1e-6f, 0.f, RopeStyle::NeoX, 1.f, nullptr,
                          nullptr, s, nullptr, cs);
        };
        auto paged = [&](const Tensor& inv, const Tensor* cs) {
            ffi::rope_paged_kv(q4, q4, k4, nullptr, v4, inv, 0, nullptr, nullptr, nullptr, 1e-6f, 0.f, RopeStyle::NeoX, 1.f,
                               kc, kc, bt, sl, nullptr, s, cs);
        };
        auto paged_had = [&](const Tensor& inv, const Tensor* cs) {
            ffi::rope_paged_kv_had(q4, q4, k4, nullptr, v4, inv, 0, nullptr, nullptr, nullptr, 1e-6f, 0.f, RopeStyle::NeoX,
                                   1.f, kc, kc, bt, sl, nullptr, nullptr, nullptr, nullptr, s, cs);
        };
        const std::function<void(const Tensor&, const Tensor*)> ops[3] = { had, paged, paged_had };
        const char* names[3] = { "rope_had", "rope_paged_kv", "rope_paged_kv_had" };
        for (int i = 0; i < 3; ++i)
        {
            const std::string n = names[i];
            expect_error((n + " short cs_table").c_str(), EXL3R_EINVAL, [&] { ops[i](inv64, &cs_short); });
            expect_error((n + " cs_table R/2 != inv_freq").c_str(), EXL3R_EINVAL, [&] { ops[i](inv64, &cs_rdim); });
            expect_error((n + " f16 cs_table").c_str(), EXL3R_EINVAL, [&] { ops[i](inv64, &cs_f16); });
            expect_error((n + " angle table as inv_freq").c_str(), EXL3R_EINVAL, [&] { ops[i](angles, nullptr); });
        }
    }

    // inv_freq: 1 / exp((2i/d) ln theta) in fp32 equals theta^(-2i/d) to a few fp32 ulps.
    const std::vector<float> inv_freq = RoPE::default_inv_freq(1e6, 128);
    double worst = 0.0;
    for (size_t i = 0; i < inv_freq.size(); ++i)
    {
        const double ref = std::pow(1e6, -2.0 * (double)i / 128.0);
        worst = std::fmax(worst, std::fabs(inv_freq[i] - ref) / ref);
    }
    const std::vector<float> lin = RoPE::default_inv_freq(1e4, 64, 4.0);
    const bool lin_ok = std::fabs(lin[5] * 4.0 - std::pow(1e4, -10.0 / 64.0)) < 1e-6 * std::pow(1e4, -10.0 / 64.0);
    std::printf("%s inv_freq max rel err %.3g (theta 1e6, d 128); linear scaling %s\n", worst < 2e-6 ? "ok  " : "FAIL",
                worst, lin_ok ? "ok" : "FAIL");
    if (worst >= 2e-6 || !lin_ok) ++failures;

    // rope_type producers (RoPE::params, src/rope.rs:45-220): the structure each one fixes.
    {
        auto check = [&](const char* what, bool ok) {
            std::printf("%s %s\n", ok ? "ok  " : "FAIL", what);
            if (!ok) ++failures;
        };
        auto near = [](double a, double b, double rel) { return std::fabs(a - b) <= rel * std::fabs(b); };
        using T = RopeScaling::Type;
        const double pi = 3.14159265358979323846;

        // llama3 (Llama 3.1: theta 5e5, factor 8, low 1, high 4, 8192): wavelengths below 8192/4 kept,
        // above 8192 divided by 8, the band between strictly between the two, monotone overall.
        const std::vector<float> b5 = RoPE::default_inv_freq(5e5, 128);
        RopeScaling l3;
        l3.type = T::Llama3;
        l3.factor = 8.0;
        l3.original_max_position_embeddings = 8192.0;
        const RoPE::Params p3 = RoPE::params(5e5, 128, l3);
        bool kept = true, divided = true, between = true, mono = true;
        int nk = 0, nd = 0, nm = 0;
        for (size_t i = 0; i < b5.size(); ++i)
        {
            const double wl = 2.0 * pi / b5[i];
            if (wl < 2048.0) { kept = kept && p3.inv_freq[i] == b5[i]; ++nk; }
            else if (wl > 8192.0) { divided = divided && near(p3.inv_freq[i], b5[i] / 8.0, 1e-6); ++nd; }
            else { between = between && p3.inv_freq[i] < b5[i] && p3.inv_freq[i] > b5[i] / 8.0; ++nm; }
            if (i) mono = mono && p3.inv_freq[i] < p3.inv_freq[i - 1];
        }
        check("llama3: high band kept, low band / factor, middle band between, monotone",
              kept && divided && between && mono && nk && nd && nm && p3.attn_factor == 1.0);
        RopeScaling l3d = l3;
        l3d.factor = 0.0;                 // absent: the reference's default factor 8
        check("llama3: absent factor means 8", RoPE::params(5e5, 128, l3d).inv_freq == p3.inv_freq);

        // yarn (DeepSeek-V2 style: theta 1e4, d 64, 163840 positions over 4096 -> factor 40): the first
        // frequencies extrapolated (unchanged), the last interpolated (/ 40), monotone between;
        // attn_factor 0.1 ln 40 + 1 unless given.
        const std::vector<float> b4 = RoPE::default_inv_freq(1e4, 64);
        RopeScaling y;
        y.type = T::Yarn;
        y.max_position_embeddings = 163840;
        y.original_max_position_embeddings = 4096.0;
        const RoPE::Params py = RoPE::params(1e4, 64, y);
        bool ymono = true, yrange = true;
        for (size_t i = 1; i < b4.size(); ++i) ymono = ymono && py.inv_freq[i] < py.inv_freq[i - 1];
        for (size_t i = 0; i < b4.size(); ++i)
            yrange = yrange && py.inv_freq[i] <= b4[i] * (1 + 2e-6) && py.inv_freq[i] >= b4[i] / 40.0 * (1 - 2e-6);
        check("yarn: extrapolated head, interpolated tail, monotone, mscale 0.1 ln(factor) + 1",
              near(py.inv_freq[0], b4[0], 2e-6) && near(py.inv_freq.back(), b4.back() / 40.0, 2e-6) && ymono && yrange &&
              near(py.attn_factor, 0.1 * std::log(40.0) + 1.0, 1e-12));
        RopeScaling y2 = y;
        y2.has_attention_factor = true;
        y2.attention_factor = 0.7;
        check("yarn: attention_factor overrides mscale", RoPE::params(1e4, 64, y2).attn_factor == 0.7);

        // longrope: unit factors give the default frequencies, constant 2 halves them (as linear 2);
        // extended context uses long_factor with scale sqrt(1 + ln(a/b) / ln(b)), else short_factor, 1.
        RopeScaling lr;
        lr.type = T::LongRope;
        lr.max_position_embeddings = 131072;
        lr.original_max_position_embeddings = 4096.0;
        lr.long_factor.assign(32, 2.0);
        lr.short_factor.assign(32, 1.0);
        const RoPE::Params pl = RoPE::params(1e4, 64, lr);
        const std::vector<float> lin2 = RoPE::default_inv_freq(1e4, 64, 2.0);
        bool lr_ok = true;
        for (size_t i = 0; i < lin2.size(); ++i) lr_ok = lr_ok && near(pl.inv_freq[i], lin2[i], 2e-6);
        RopeScaling lrs = lr;
        lrs.max_position_embeddings = 4096;
        const RoPE::Params ps = RoPE::params(1e4, 64, lrs);
        bool sh_ok = ps.attn_factor == 1.0;
        for (size_t i = 0; i < b4.size(); ++i) sh_ok = sh_ok && near(ps.inv_freq[i], b4[i], 2e-6);
        check("longrope: long / short factors and the extended-context scale",
              lr_ok && sh_ok && near(pl.attn_factor, std::sqrt(1.0 + std::log(32.0) / std::log(4096.0)), 1e-12));

        // proportional: head_dim 256 with a quarter rotated: 32 frequencies of the head-dim ramp, zeros
        // after, all divided by factor.
        RopeScaling pr;
        pr.type = T::Proportional;
        pr.head_dim = 256;
        pr.partial_rotary_factor = 0.25;
        pr.factor = 2.0;
        const RoPE::Params pp = RoPE::params(1e6, 0, pr);
        const std::vector<float> b256 = RoPE::default_inv_freq(1e6, 256);
        bool pp_ok = pp.inv_freq.size() == 128;
        for (size_t i = 0; pp_ok && i < 128; ++i)
            pp_ok = i < 32 ? near(pp.inv_freq[i], b256[i] / 2.0, 2e-6) : pp.inv_freq[i] == 0.0f;
        check("proportional: partial head-dim ramp, zero tail, / factor", pp_ok);

        RopeScaling bad = l3;
        bad.high_freq_factor = 0.5;
        expect_error("llama3 high <= low", EXL3R_EINVAL, [&] { RoPE::params(5e5, 128, bad); });
        RopeScaling ybad;
        ybad.type = T::Yarn;
        expect_error("yarn without max_position_embeddings", EXL3R_EINVAL, [&] { RoPE::params(1e4, 64, ybad); });
        RopeScaling lbad = lr;
        lbad.long_factor.resize(5);
        expect_error("longrope factor count", EXL3R_EINVAL, [&] { RoPE::params(1e4, 64, lbad); });
    }
    std::printf(failures ? "test_host_cpu: %d failures\n" : "test_host_cpu: all passed\n", failures);
    return failures ? 1 : 0;
}
