// C ABI: exl3r_rms_norm_res_in (replaces exl3_shim_rms_norm_res_in, reference
// csrc/exl3_shim.cpp:139-142 -> rms_norm_res_in, kernels/norm.cu:467-479).
#include "rms_norm_kernel.cuh"
#include "rms_norm_launch.hpp"

using namespace exl3r;

extern "C" int exl3r_rms_norm_res_in(const void* x, int xt, int64_t ldx, const void* w, int wt,
                                     void* y, int yt, int64_t ldy, void* r, int rt, int64_t ldr,
                                     int64_t rows, int64_t dim,
                                     float eps, float constant_bias, float constant_scale, void* stream)
{
    begin_call();
    const char* op = "exl3r_rms_norm_res_in";
    int rc = check_rms_common(op, x, xt, ldx, w, wt, y, yt, ldy, rows, dim);
    if (rc) return rc;
    if (!is_float_dtype(rt)) return set_error(EXL3R_EDTYPE, "%s: unsupported residual dtype %s", op, dtype_name(rt));
    if (ldr < dim) return set_error(EXL3R_EINVAL, "%s: residual row stride %lld < dim %lld", op, (long long)ldr, (long long)dim);
    if (rows == 0) return EXL3R_OK;
    if (!r) return set_error(EXL3R_EINVAL, "%s: residual r must be non-null", op);
    if (r == y) return set_error(EXL3R_EINVAL, "%s: y must not alias the residual", op);
    if (x == r && (xt != rt || ldx != ldr)) return set_error(EXL3R_EINVAL, "%s: x == r needs equal dtypes and strides", op);

    RmsArgs a{};
    a.x = x; a.ldx = ldx; a.w = w; a.wt = wt; a.y = y; a.ldy = ldy; a.r = r; a.ldr = ldr;
    a.rows = rows; a.dim = (int)dim; a.eps = eps; a.cb = constant_bias; a.cs = constant_scale;
    hipStream_t s = (hipStream_t)stream;

    if (rms_vec_ok(a, xt, yt, rt, true, RMS_RES_IN, 0))
    {
        with_float_type(xt, [&](auto X) {
            with_float_type(rt, [&](auto R) {
                with_float_type(yt, [&](auto Y) {
                    launch_rms_vec<decltype(X), decltype(Y), decltype(R), RMS_RES_IN>(a, s);
                });
            });
        });
    }
    else
    {
        const unsigned grid = (unsigned)(rows < kMaxGridX ? rows : kMaxGridX);
        launch(k_rms_norm_generic<RMS_RES_IN>, grid, 256, 0, s, a, xt, yt, rt);
    }
    return launch_status(op);
}
