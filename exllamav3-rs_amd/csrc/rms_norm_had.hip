// C ABI: exl3r_rms_norm_had -- RMSNorm (plain, or with the residual add folded in) whose f16 output
// feeds the random-Hadamard input rotation of one to four EXL3 projections, in one pass: the norm of
// RmsNorm::forward / forward_res (src/modules.rs:372-411) followed by each consumer's
// had_r_128(y, suh) (src/modules.rs:224-227; kernels/quant/hadamard.cu:88-170).  With rotate_x, x
// is first given the producing projection's own output rotation had_r_128(x, x, None, svh)
// (src/modules.rs:231).  The transforms run on the matrix cores (had128_mfma), or with EXL3R_HAD_EXACT in
// rotate_x as the reference's butterfly, bit-identical to those calls made one after another.
#include "rms_norm_kernel.cuh"
#include "rms_norm_launch.hpp"

using namespace exl3r;

extern "C" int exl3r_had_r_128(const void* x, int dtype, int64_t ldx, void* out, int64_t ldo, int64_t rows,
                               int64_t cols, const void* pre_scale, const void* post_scale, float scale, void* stream);

extern "C" int exl3r_rms_norm_had(const void* x, int xt, int64_t ldx, const void* w, int wt,
                                  void* r, int rt, int64_t ldr, void* y, int64_t ldy,
                                  int n_out, const void* const* pre_scales, void* const* outs, int64_t ldo,
                                  int64_t rows, int64_t dim, float eps, float constant_bias, float constant_scale,
                                  float had_scale, int rotate_x, const void* x_post_scale, void* stream)
{
    begin_call();
    const char* op = "exl3r_rms_norm_had";
    const bool exact = (rotate_x & EXL3R_HAD_EXACT) != 0;
    rotate_x &= ~EXL3R_HAD_EXACT;
    if (rotate_x & ~1) return set_error(EXL3R_EINVAL, "%s: rotate_x takes 0 or 1 (and EXL3R_HAD_EXACT)", op);
    if (rotate_x && xt != EXL3R_F16) return set_error(EXL3R_EDTYPE, "%s: rotate_x takes f16 x", op);
    if (!rotate_x && x_post_scale) return set_error(EXL3R_EINVAL, "%s: x_post_scale without rotate_x", op);
    if (!is_float_dtype(xt) || (w && !is_float_dtype(wt)) || (r && !is_float_dtype(rt)))
        return set_error(EXL3R_EDTYPE, "%s: unsupported x / w / r dtype", op);
    if (rows < 0 || dim <= 0 || dim % 128 || dim > 65536 || (rows > 1 && (ldx < dim || ldo < dim)) ||
        (r && rows > 1 && ldr < dim) || (y && rows > 1 && ldy < dim))
        return set_error(EXL3R_EINVAL, "%s: invalid shape rows=%lld dim=%lld (a multiple of 128) or row strides", op,
                         (long long)rows, (long long)dim);
    if (n_out < 1 || n_out > 4 || !outs || !pre_scales)
        return set_error(EXL3R_EINVAL, "%s: n_out must be 1..4 with outs and pre_scales arrays", op);
    if (rows == 0) return EXL3R_OK;
    if (!x) return set_error(EXL3R_EINVAL, "%s: x must be non-null", op);
    for (int i = 0; i < n_out; ++i)
    {
        if (!outs[i]) return set_error(EXL3R_EINVAL, "%s: outs[%d] must be non-null", op, i);
        if (outs[i] == x || outs[i] == r || outs[i] == y) return set_error(EXL3R_EINVAL, "%s: outs[%d] aliases an input", op, i);
        for (int j = 0; j < i; ++j)
            if (outs[j] == outs[i]) return set_error(EXL3R_EINVAL, "%s: outs[%d] and outs[%d] alias", op, j, i);
    }
    if (y && (y == x || y == r)) return set_error(EXL3R_EINVAL, "%s: y must not alias x or r", op);
    if (r && x == r && (rotate_x || xt != rt || ldx != ldr))
        return set_error(EXL3R_EINVAL, "%s: x == r needs equal dtypes and strides, and no rotate_x", op);

    RmsArgs a{};
    a.x = x; a.ldx = rows > 1 ? ldx : dim; a.w = w; a.wt = wt; a.y = y; a.ldy = y ? (rows > 1 ? ldy : dim) : dim;
    a.r = r; a.ldr = r ? (rows > 1 ? ldr : dim) : 0;
    a.rows = rows; a.dim = (int)dim; a.eps = eps; a.cb = constant_bias; a.cs = constant_scale;
    a.nh = n_out; a.ldh = rows > 1 ? ldo : dim; a.hr = had_scale * 0.0883883461356163f;
    a.hxpost = x_post_scale;
#ifdef EXL3R_TUNING
    a.r_cached = tuning().rms_r_cached;
#endif
    bool aligned = (a.ldh * 2) % 16 == 0;
    for (int i = 0; i < n_out; ++i)
    {
        a.hpre[i] = pre_scales[i];
        a.hout[i] = outs[i];
        aligned = aligned && aligned16(outs[i]) && (!pre_scales[i] || aligned16(pre_scales[i]));
    }
    aligned = aligned && (!x_post_scale || aligned16(x_post_scale));
    hipStream_t s = (hipStream_t)stream;
    if (aligned && rms_vec_ok(a, xt, EXL3R_F16, r ? rt : EXL3R_F16, r != nullptr, r ? RMS_RES_IN : RMS_PLAIN, HAD_OUT))
    {
        auto go = [&](auto M) {
            constexpr int F = decltype(M)::value;   // HAD_MFMA or 0 (the butterfly)
            if (rotate_x)
            {
                if (!r) launch_rms_vec<TF16, TF16, TNone, RMS_PLAIN, HAD_IN | HAD_OUT | F>(a, s);
                else with_float_type(rt, [&](auto R) { launch_rms_vec<TF16, TF16, decltype(R), RMS_RES_IN, HAD_IN | HAD_OUT | F>(a, s); });
            }
            else
                with_float_type(xt, [&](auto X) {
                    if (!r) launch_rms_vec<decltype(X), TF16, TNone, RMS_PLAIN, HAD_OUT | F>(a, s);
                    else with_float_type(rt, [&](auto R) { launch_rms_vec<decltype(X), TF16, decltype(R), RMS_RES_IN, HAD_OUT | F>(a, s); });
                });
        };
        if (exact) go(std::integral_constant<int, 0>{});
        else go(std::integral_constant<int, HAD_MFMA>{});
        return launch_status(op);
    }
    // Unaligned rows: the calls one after another.  A rotated x goes to the first output, the norm
    // into y (or into the first output, in place), then one transform per output, the first output
    // last so that it may be transformed in place.
    const void* xin = x;
    int64_t ldxin = ldx;
    int rc = EXL3R_OK;
    if (rotate_x)
    {
        rc = exl3r_had_r_128(x, EXL3R_F16, ldx, outs[0], ldo, rows, dim, nullptr, x_post_scale, 1.0f, stream);
        xin = outs[0];
        ldxin = ldo;
    }
    void* dst = y ? y : outs[0];
    const int64_t ldd = y ? a.ldy : a.ldh;
    if (rc == EXL3R_OK)
        rc = r ? exl3r_rms_norm_res_in(xin, xt, ldxin, w, wt, dst, EXL3R_F16, ldd, r, rt, ldr, rows, dim, eps,
                                       constant_bias, constant_scale, stream)
               : exl3r_rms_norm(xin, xt, ldxin, w, wt, dst, EXL3R_F16, ldd, rows, dim, eps, constant_bias,
                                constant_scale, stream);
    for (int i = n_out - 1; i >= 0 && rc == EXL3R_OK; --i)
        rc = exl3r_had_r_128(dst, EXL3R_F16, ldd, outs[i], a.ldh, rows, dim, pre_scales[i], nullptr, had_scale, stream);
    return rc;
}
