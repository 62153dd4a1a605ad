// C ABI: exl3r_rms_norm (replaces exl3_shim_rms_norm, reference csrc/exl3_shim.cpp:76-80) and the
// shared argument checks of the RMSNorm family.
#include "rms_norm_kernel.cuh"
#include "rms_norm_launch.hpp"

namespace exl3r {

int check_rms_common(const char* op, const void* x, int xt, int64_t ldx, const void* w, int wt,
                     const void* y, int yt, int64_t ldy, int64_t rows, int64_t dim)
{
    if (rows > 0 && (!x || !y)) return set_error(EXL3R_EINVAL, "%s: x and y must be non-null", op);
    if (rows < 0 || dim <= 0 || dim > (int64_t)1 << 30)
        return set_error(EXL3R_EINVAL, "%s: invalid shape rows=%lld dim=%lld", op, (long long)rows, (long long)dim);
    if (ldx < dim || ldy < dim)
        return set_error(EXL3R_EINVAL, "%s: row strides (%lld, %lld) must be >= dim %lld", op,
                         (long long)ldx, (long long)ldy, (long long)dim);
    if (!is_float_dtype(xt) || !is_float_dtype(yt) || (w && !is_float_dtype(wt)))
        return set_error(EXL3R_EDTYPE, "%s: unsupported dtypes x=%s y=%s w=%s", op, dtype_name(xt),
                         dtype_name(yt), w ? dtype_name(wt) : "none");
    if (rows > 0 && x == y && (xt != yt || ldx != ldy))
        return set_error(EXL3R_EINVAL, "%s: in-place y == x needs equal dtypes and strides", op);
    return EXL3R_OK;
}

}  // namespace exl3r

using namespace exl3r;

extern "C" int exl3r_rms_norm(const void* x, int xt, int64_t ldx, const void* w, int wt,
                              void* y, int yt, int64_t ldy, int64_t rows, int64_t dim,
                              float eps, float constant_bias, float constant_scale, void* stream)
{
    begin_call();
    int rc = check_rms_common("exl3r_rms_norm", x, xt, ldx, w, wt, y, yt, ldy, rows, dim);
    if (rc) return rc;
    if (rows == 0) return EXL3R_OK;

    RmsArgs a{};
    a.x = x; a.ldx = ldx; a.w = w; a.wt = wt; a.y = y; a.ldy = ldy;
    a.rows = rows; a.dim = (int)dim; a.eps = eps; a.cb = constant_bias; a.cs = constant_scale;
    hipStream_t s = (hipStream_t)stream;

    if (rms_vec_ok(a, xt, yt, 0, false, RMS_PLAIN, 0))
    {
        with_float_type(xt, [&](auto X) {
            with_float_type(yt, [&](auto Y) {
                launch_rms_vec<decltype(X), decltype(Y), TNone, RMS_PLAIN>(a, s);
            });
        });
    }
    else
    {
        const unsigned grid = (unsigned)(rows < kMaxGridX ? rows : kMaxGridX);
        launch(k_rms_norm_generic<RMS_PLAIN>, grid, 256, 0, s, a, xt, yt, 0);
    }
    return launch_status("exl3r_rms_norm");
}
