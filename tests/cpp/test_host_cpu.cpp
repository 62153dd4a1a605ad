// CPU checks of the C++ host layer: argument validation throws exl3r::Error with the C ABI's
// status before any device work, and the default inv_freq producer matches theta^(-2i/d).
// Device pointers are fake (never dereferenced: every call fails validation first).
#include "exl3r.hpp"

#include <cmath>
#include <cstdio>
#include <functional>

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
    std::printf(failures ? "test_host_cpu: %d failures\n" : "test_host_cpu: all passed\n", failures);
    return failures ? 1 : 0;
}
