// Eager timing of one 64-row decode layer's row ops, issued from compiled code -- the regime of the
// reference's batched decode, which is not graph-captured (its generator launches every op from Rust on
// one stream, src/generator.rs:1512-1607).
//
//   fused: exl3r::ffi::rms_norm_res_in -> rope (q/k head-norm + NeoX, per-sequence positions) ->
//          rms_norm_res_in -> silu_mul: 4 launches through the C++ host layer, argument checks included,
//          as the reference's ffi.rs wrappers would issue them;
//   naive: the unfused HIP baseline (libexl3r_naive.so): add, norm, 2 head norms, 2 RoPE, add, norm,
//          silu, mul: 10 launches through its C entry points.
//
// Shapes: T = 64 rows, hidden 5120, intermediate 17408, 64 / 8 heads of 128, f16.  Each window enqueues
// `iters` layers back to back on one stream between two HIP events; windows alternate between the two
// variants and the median window is reported, with the host's enqueue time per layer beside it (when it
// is below the device time, the GPU is the bound).  One JSON line on stdout.
//
//   exl3r_bench_decode [iters=2000] [windows=7]
#include "exl3r.hpp"

#include "../csrc/naive_baseline.h"

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <functional>
#include <vector>

using namespace exl3r;

namespace {

void hip_ok(hipError_t e, const char* what)
{
    if (e != hipSuccess)
    {
        std::fprintf(stderr, "%s: %s\n", what, hipGetErrorString(e));
        std::exit(1);
    }
}

void rc_ok(int rc, const char* what)
{
    if (rc != 0)
    {
        std::fprintf(stderr, "%s failed: %d\n", what, rc);
        std::exit(1);
    }
}

// fp32 -> IEEE binary16, round to nearest even (finite inputs of moderate range only).
uint16_t to_half(float f)
{
    uint32_t x;
    std::memcpy(&x, &f, 4);
    const uint32_t sign = (x >> 16) & 0x8000u;
    const int exp = (int)((x >> 23) & 0xff) - 127 + 15;
    uint32_t man = x & 0x7fffffu;
    if (exp <= 0)
    {
        if (exp < -10) return (uint16_t)sign;
        man |= 0x800000u;
        const int shift = 14 - exp;
        uint32_t h = man >> shift;
        const uint32_t rem = man & ((1u << shift) - 1), half = 1u << (shift - 1);
        if (rem > half || (rem == half && (h & 1))) ++h;
        return (uint16_t)(sign | h);
    }
    uint32_t h = ((uint32_t)exp << 10) | (man >> 13);
    const uint32_t rem = man & 0x1fffu;
    if (rem > 0x1000u || (rem == 0x1000u && (h & 1))) ++h;
    return (uint16_t)(sign | h);
}

// Seeded N(mean, std) values (Box-Muller over a 64-bit LCG) in f16.
std::vector<uint16_t> normal_f16(size_t n, float mean, float stdv, uint64_t seed)
{
    std::vector<uint16_t> v(n);
    uint64_t st = seed * 6364136223846793005ull + 1442695040888963407ull;
    auto uni = [&]() {
        st = st * 6364136223846793005ull + 1442695040888963407ull;
        return ((st >> 11) + 0.5) * (1.0 / 9007199254740992.0);
    };
    for (size_t i = 0; i < n; ++i)
    {
        const double z = std::sqrt(-2.0 * std::log(uni())) * std::cos(6.283185307179586 * uni());
        v[i] = to_half((float)(mean + stdv * z));
    }
    return v;
}

struct Buf
{
    DeviceBuffer b;
    Tensor t;
    Buf(DType dt, std::vector<int64_t> shape) : b(0)
    {
        int64_t n = 1;
        for (int64_t d : shape) n *= d;
        b = DeviceBuffer((size_t)n * dtype_size(dt));
        t = Tensor(b.data(), dt, shape);
    }
};

}  // namespace

int main(int argc, char** argv)
{
    const int iters = argc > 1 ? std::atoi(argv[1]) : 2000;
    const int windows = argc > 2 ? std::atoi(argv[2]) : 7;
    const int64_t T = 64, H = 5120, I = 17408, HQ = 64, HK = 8, HD = 128;
    Stream s = Stream::create();

    Buf resid(DType::F16, { T, H }), a_out(DType::F16, { T, H }), m_out(DType::F16, { T, H }), y(DType::F16, { T, H });
    Buf w1(DType::F16, { H }), w2(DType::F16, { H }), qn(DType::F16, { HD }), kn(DType::F16, { HD });
    Buf q(DType::F16, { T, 1, HQ, HD }), k(DType::F16, { T, 1, HK, HD });
    Buf gate(DType::F16, { T, I }), up(DType::F16, { T, I }), act(DType::F16, { T, I }), tmp(DType::F16, { T, I });
    Buf pos(DType::I32, { T }), inv(DType::F32, { HD / 2 });

    auto fill = [&](Buf& b, float mean, float stdv, uint64_t seed) {
        const std::vector<uint16_t> h = normal_f16((size_t)b.t.numel(), mean, stdv, seed);
        b.b.upload(h.data(), h.size() * 2, s);
    };
    fill(resid, 0, 4, 1);
    fill(a_out, 0, 1, 2);
    fill(m_out, 0, 1, 3);
    fill(w1, 1, 0.1f, 4);
    fill(w2, 1, 0.1f, 5);
    fill(qn, 1, 0.1f, 6);
    fill(kn, 1, 0.1f, 7);
    fill(q, 0, 1, 8);
    fill(k, 0, 1, 9);
    fill(gate, 0, 1, 10);
    fill(up, 0, 1, 11);
    std::vector<int32_t> hpos(T);
    for (int64_t i = 0; i < T; ++i) hpos[i] = (int32_t)((i * 2654435761u) % 32768u);
    pos.b.upload(hpos.data(), hpos.size() * 4, s);
    const std::vector<float> hinv = RoPE::default_inv_freq(1e6, (int)HD);
    inv.b.upload(hinv.data(), hinv.size() * 4, s);

    hipStream_t hs = s.get();
    const std::function<void()> fused = [&] {
        ffi::rms_norm_res_in(a_out.t, &w1.t, y.t, resid.t, 1e-6f, 0.0f, 1.0f, s);
        ffi::rope(q.t, q.t, &k.t, &k.t, inv.t, 0, &pos.t, &qn.t, &kn.t, 1e-6f, 0.0f, RopeStyle::NeoX, 1.0f, s);
        ffi::rms_norm_res_in(m_out.t, &w2.t, y.t, resid.t, 1e-6f, 0.0f, 1.0f, s);
        ffi::silu_mul(gate.t, up.t, act.t, 0.0f, s);
    };
    const std::function<void()> naive = [&] {
        rc_ok(naive_add_f16(a_out.b.data(), resid.b.data(), resid.b.data(), T * H, hs), "naive_add");
        rc_ok(naive_rms_norm_f16(resid.b.data(), w1.b.data(), y.b.data(), T, (int)H, 1e-6f, hs), "naive_rms_norm");
        rc_ok(naive_head_norm_f16(q.b.data(), qn.b.data(), T, (int)HQ, (int)HD, 1e-6f, hs), "naive_head_norm q");
        rc_ok(naive_head_norm_f16(k.b.data(), kn.b.data(), T, (int)HK, (int)HD, 1e-6f, hs), "naive_head_norm k");
        rc_ok(naive_rope_neox_f16(q.b.data(), (const float*)inv.b.data(), (const int32_t*)pos.b.data(), T, 1, (int)HQ,
                                  (int)HD, hs), "naive_rope q");
        rc_ok(naive_rope_neox_f16(k.b.data(), (const float*)inv.b.data(), (const int32_t*)pos.b.data(), T, 1, (int)HK,
                                  (int)HD, hs), "naive_rope k");
        rc_ok(naive_add_f16(m_out.b.data(), resid.b.data(), resid.b.data(), T * H, hs), "naive_add");
        rc_ok(naive_rms_norm_f16(resid.b.data(), w2.b.data(), y.b.data(), T, (int)H, 1e-6f, hs), "naive_rms_norm");
        rc_ok(naive_silu_f16(gate.b.data(), tmp.b.data(), T * I, hs), "naive_silu");
        rc_ok(naive_mul_f16(tmp.b.data(), up.b.data(), act.b.data(), T * I, hs), "naive_mul");
    };

    hipEvent_t e0, e1;
    hip_ok(hipEventCreate(&e0), "hipEventCreate");
    hip_ok(hipEventCreate(&e1), "hipEventCreate");
    // Returns {device us per layer, host enqueue us per layer} of one window.
    auto window = [&](const std::function<void()>& fn) {
        hip_ok(hipEventRecord(e0, hs), "hipEventRecord");
        const auto t0 = std::chrono::steady_clock::now();
        for (int i = 0; i < iters; ++i) fn();
        const auto t1 = std::chrono::steady_clock::now();
        hip_ok(hipEventRecord(e1, hs), "hipEventRecord");
        hip_ok(hipEventSynchronize(e1), "hipEventSynchronize");
        float ms = 0.0f;
        hip_ok(hipEventElapsedTime(&ms, e0, e1), "hipEventElapsedTime");
        const double host_us = std::chrono::duration<double, std::micro>(t1 - t0).count() / iters;
        return std::pair<double, double>(ms * 1000.0 / iters, host_us);
    };
    for (int i = 0; i < 50; ++i)
    {
        fused();
        naive();
    }
    s.synchronize();
    std::vector<double> fd, fh, nd, nh;
    for (int w = 0; w < windows; ++w)
    {
        auto f = window(fused);
        auto n = window(naive);
        fd.push_back(f.first);
        fh.push_back(f.second);
        nd.push_back(n.first);
        nh.push_back(n.second);
    }
    auto median = [](std::vector<double> v) {
        std::sort(v.begin(), v.end());
        return v[v.size() / 2];
    };
    const double f_us = median(fd), n_us = median(nd);
    std::printf("{\"fused_us\": %.3f, \"naive_us\": %.3f, \"speedup\": %.3f, \"fused_host_enqueue_us\": %.3f, "
                "\"naive_host_enqueue_us\": %.3f, \"iters\": %d, \"windows\": %d, \"fused_min_us\": %.3f, "
                "\"naive_min_us\": %.3f}\n",
                f_us, n_us, n_us / f_us, median(fh), median(nh), iters, windows, *std::min_element(fd.begin(), fd.end()),
                *std::min_element(nd.begin(), nd.end()));
    hip_ok(hipEventDestroy(e0), "hipEventDestroy");
    hip_ok(hipEventDestroy(e1), "hipEventDestroy");
    return 0;
}
