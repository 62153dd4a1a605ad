// C ABI: exl3r_gated_rms_norm (replaces exl3_shim_gated_rms_norm, reference csrc/exl3_shim.cpp:143-147 ->
// gated_rms_norm, kernels/norm.cu:482-668; the Qwen3.5 gated-delta-net output norm, src/qwen3_5.rs:212).
//
// y = RMSNorm(x) * w * act(g) with act = silu or sigmoid, or RMSNorm(x * act(g)) * w with gate_first,
// the weight cycling over w_groups rows (Mamba2 group norm).  The RMSNorm kernel family's register-
// resident row (rms_norm_kernel.cuh, mode RMS_GATED) carries the gate through its second operand.
#include "rms_norm_kernel.cuh"
#include "rms_norm_launch.hpp"

using namespace exl3r;

extern "C" int exl3r_gated_rms_norm(const void* x, int xt, int64_t ldx, const void* w, int wt, int w_groups,
                                    void* y, int yt, int64_t ldy, const void* g, int gt, int64_t ldg,
                                    int64_t rows, int64_t dim, float eps, float constant_bias,
                                    int gate_first, int gate_act, void* stream)
{
    begin_call();
    const char* op = "exl3r_gated_rms_norm";
    int rc = check_rms_common(op, x, xt, ldx, w, wt, y, yt, ldy, rows, dim);
    if (rc) return rc;
    if (!is_float_dtype(gt)) return set_error(EXL3R_EDTYPE, "%s: unsupported gate dtype %s", op, dtype_name(gt));
    if (ldg < dim) return set_error(EXL3R_EINVAL, "%s: gate row stride %lld < dim %lld", op, (long long)ldg, (long long)dim);
    if (w_groups < 1) return set_error(EXL3R_EINVAL, "%s: w_groups must be >= 1", op);
    if (gate_act != 0 && gate_act != 1) return set_error(EXL3R_EINVAL, "%s: gate_act must be 0 (silu) or 1 (sigmoid)", op);
    if (rows == 0) return EXL3R_OK;
    if (!g) return set_error(EXL3R_EINVAL, "%s: gate g must be non-null", op);
    if (g == y) return set_error(EXL3R_EINVAL, "%s: y must not alias the gate", op);

    RmsArgs a{};
    a.x = x; a.ldx = ldx; a.w = w; a.wt = wt; a.y = y; a.ldy = ldy; a.r = const_cast<void*>(g); a.ldr = ldg;
    a.rows = rows; a.dim = (int)dim; a.eps = eps; a.cb = constant_bias; a.cs = 1.0f;
    a.gact = gate_act; a.gfirst = gate_first != 0; a.w_groups = w_groups;
    hipStream_t s = (hipStream_t)stream;

    // Short rows (head-dim rows of the gated-delta-net output) take the lanes-per-row kernel for the
    // reference's gate types (bf16 / f32); everything else the workgroup-per-row kernel.
    const bool short_rows = dim <= 512 && (gt == EXL3R_F32 || gt == EXL3R_BF16);
    if (xt != EXL3R_F32 && rms_vec_ok(a, xt, yt, gt, true, RMS_GATED, 0))
    {
        auto go_x = [&](auto X) {
            with_float_type(yt, [&](auto Y) {
                using XTy = decltype(X);
                using YTy = decltype(Y);
                if (short_rows)
                {
                    if (gt == EXL3R_F32) launch_rms_rows<XTy, YTy, TF32, RMS_GATED>(a, s);
                    else launch_rms_rows<XTy, YTy, TBF16, RMS_GATED>(a, s);
                    return;
                }
                with_float_type(gt, [&](auto G) { launch_rms_vec<XTy, YTy, decltype(G), RMS_GATED>(a, s); });
            });
        };
        if (xt == EXL3R_F16) go_x(TF16{});
        else go_x(TBF16{});
    }
    else
    {
        const unsigned grid = (unsigned)(rows < kMaxGridX ? rows : kMaxGridX);
        launch(k_rms_norm_generic<RMS_GATED>, grid, 256, 0, s, a, xt, yt, gt);
    }
    return launch_status(op);
}

extern "C" int exl3r_had_r_128(const void* x, int dtype, int64_t ldx, void* out, int64_t ldo, int64_t rows,
                               int64_t cols, const void* pre_scale, const void* post_scale, float scale, void* stream);

// exl3r_gated_rms_norm with an f16 output feeding the next EXL3 projection's input rotation, in one
// pass: the gated-delta-net output norm, then o_proj's had_r_128(y, suh) (src/qwen3_5.rs:208-214,
// src/modules.rs:224-227).  A 128-column block of the rotation is 16 lanes of one row's lane group; rows
// of one block (head_dim 128) run the transform on the matrix cores unless EXL3R_HAD_EXACT is in
// gate_act (then, and at other row lengths, the reference's butterfly).
extern "C" int exl3r_gated_rms_norm_had(const void* x, int xt, int64_t ldx, const void* w, int wt, int w_groups,
                                        const void* g, int gt, int64_t ldg, void* y, int64_t ldy,
                                        const void* pre_scale, int pre_rows, void* out, int64_t ldo, int64_t rows,
                                        int64_t dim, float eps, float constant_bias, int gate_first, int gate_act,
                                        float had_scale, void* stream)
{
    begin_call();
    const char* op = "exl3r_gated_rms_norm_had";
    const bool exact = (gate_act & EXL3R_HAD_EXACT) != 0;
    gate_act &= ~EXL3R_HAD_EXACT;
    if (dim <= 0 || dim % 128) return set_error(EXL3R_EINVAL, "%s: dim %lld must be a multiple of 128", op, (long long)dim);
    int rc = check_rms_common(op, x, xt, ldx, w, wt, out, EXL3R_F16, ldo, rows, dim);
    if (rc) return rc;
    if (!is_float_dtype(gt)) return set_error(EXL3R_EDTYPE, "%s: unsupported gate dtype %s", op, dtype_name(gt));
    if (ldg < dim || (y && rows > 1 && ldy < dim))
        return set_error(EXL3R_EINVAL, "%s: gate / y row stride below dim %lld", op, (long long)dim);
    if (w_groups < 1) return set_error(EXL3R_EINVAL, "%s: w_groups must be >= 1", op);
    if (pre_rows < 1) return set_error(EXL3R_EINVAL, "%s: pre_rows must be >= 1", op);
    if (gate_act != 0 && gate_act != 1) return set_error(EXL3R_EINVAL, "%s: gate_act must be 0 (silu) or 1 (sigmoid)", op);
    if (rows == 0) return EXL3R_OK;
    if (!g) return set_error(EXL3R_EINVAL, "%s: gate g must be non-null", op);
    if (pre_rows > 1 && (rows % pre_rows || ldo != dim || (y && ldy != dim)))
        return set_error(EXL3R_EINVAL, "%s: pre_rows > 1 needs whole projection rows of dense norm rows", op);
    if (out == x || out == g || out == y || (y && (y == x || y == g)))
        return set_error(EXL3R_EINVAL, "%s: out and y must not alias the inputs or each other", op);

    RmsArgs a{};
    a.x = x; a.ldx = ldx; a.w = w; a.wt = wt; a.y = y; a.ldy = y ? ldy : dim; a.r = const_cast<void*>(g); a.ldr = ldg;
    a.rows = rows; a.dim = (int)dim; a.eps = eps; a.cb = constant_bias; a.cs = 1.0f;
    a.gact = gate_act; a.gfirst = gate_first != 0; a.w_groups = w_groups;
    a.nh = 1; a.hpre[0] = pre_scale; a.hpre_rows = pre_rows; a.hout[0] = out; a.ldh = rows > 1 ? ldo : dim;
    a.hr = had_scale * 0.0883883461356163f;
    hipStream_t s = (hipStream_t)stream;
    const bool short_rows = dim <= 512 && (gt == EXL3R_F32 || gt == EXL3R_BF16);
    const bool aligned = aligned16(out) && (a.ldh * 2) % 16 == 0 && (!pre_scale || aligned16(pre_scale));
    if (xt != EXL3R_F32 && aligned && rms_vec_ok(a, xt, EXL3R_F16, gt, true, RMS_GATED, HAD_OUT))
    {
        auto go_x = [&](auto X) {
            using XTy = decltype(X);
            if (short_rows)
            {
                // rows of one block: the transform on the matrix cores unless exact
                if (dim == 128 && !exact)
                {
                    if (gt == EXL3R_F32) launch_rms_rows<XTy, TF16, TF32, RMS_GATED, HAD_OUT | HAD_MFMA>(a, s);
                    else launch_rms_rows<XTy, TF16, TBF16, RMS_GATED, HAD_OUT | HAD_MFMA>(a, s);
                }
                else if (gt == EXL3R_F32) launch_rms_rows<XTy, TF16, TF32, RMS_GATED, HAD_OUT>(a, s);
                else launch_rms_rows<XTy, TF16, TBF16, RMS_GATED, HAD_OUT>(a, s);
                return;
            }
            with_float_type(gt, [&](auto G) { launch_rms_vec<XTy, TF16, decltype(G), RMS_GATED, HAD_OUT>(a, s); });
        };
        if (xt == EXL3R_F16) go_x(TF16{});
        else go_x(TBF16{});
        return launch_status(op);
    }
    // Otherwise the calls one after another: the norm into y (or into out), then the rotation.
    void* dst = y ? y : out;
    const int64_t ldd = y ? a.ldy : a.ldh;
    rc = exl3r_gated_rms_norm(x, xt, ldx, w, wt, w_groups, dst, EXL3R_F16, ldd, g, gt, ldg, rows, dim, eps, constant_bias,
                              gate_first, gate_act, stream);
    // With pre_rows > 1 the norm rows are dense, so pre_rows of them form one projection row.
    const int64_t prow = rows / pre_rows, pcols = dim * pre_rows;
    if (rc == EXL3R_OK)
        rc = exl3r_had_r_128(dst, EXL3R_F16, pre_rows > 1 ? pcols : ldd, out, pre_rows > 1 ? pcols : a.ldh,
                             pre_rows > 1 ? prow : rows, pre_rows > 1 ? pcols : dim, pre_scale, nullptr, had_scale, stream);
    return rc;
}
