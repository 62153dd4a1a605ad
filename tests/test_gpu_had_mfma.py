"""GPU parity of the matrix-core 128-point Hadamard transform (v_mfma_f32_16x16x32_f16 against +-1 f16
operands): exl3r_had_r_128_mfma against the oracle's had_r_128 (the reference's fp32 butterfly,
kernels/quant/hadamard_inner.cuh:96-200) within the stated tolerance -- each f16 result the butterfly's
or its neighbour, or within 2^-17 * r * sum|input| where the transform cancels, and nearly all of them
identical -- at the C3 shape, with pre- and post-scales, a scalar scale, partial spans, strided rows,
special values (inf, NaN, zeros of both signs, subnormals, overflow); then exl3r_act_mul_had in its
default (matrix-core) form bit for bit against the unfused matrix-core calls (activation into z, then
exl3r_had_r_128_mfma; the input rotations as exl3r_had_r_128_mfma with the post-scale), and against the
oracle composition within the tolerance."""
import numpy as np
import pytest
import torch

import exl3r.ffi as ffi
from _gpu import NTHREADS, assert_bitwise, assert_close_ulp, assert_had_close, dev_normal, from_dev, to_dev
from oracle import oracle as orc
from test_gpu_act_had import oracle_act, suh

pytestmark = pytest.mark.gpu

F16, BF16, F32 = orc.F16, orc.BF16, orc.F32
R0 = 0.0883883461356163


def f32(bits):
    return orc.to_f32(np.ascontiguousarray(bits), F16).astype(np.float64)


def had_case(x, pre=None, post=None, scale=1.0, out=None):
    out = torch.empty_like(x) if out is None else out
    ffi.had_r_128(x, out, pre, post, scale, mfma=True)
    torch.cuda.synchronize()
    xh = np.ascontiguousarray(from_dev(x))
    ph = from_dev(pre) if pre is not None else None
    qh = from_dev(post) if post is not None else None
    exp = orc.had_r_128(xh, F16, pre=ph, post=qh, scale=scale, nthreads=NTHREADS)
    xin = f32(xh) * (f32(ph)[None, :] if ph is not None else 1.0)
    # a post-scale multiplies the transform (and its tolerance) column by column
    r = R0 * scale
    return from_dev(out), exp, xin if qh is None else xin * np.abs(f32(qh)).max(), r, 2 if qh is not None else 1


@pytest.mark.parametrize("shape,pre,post,scale", [
    ((2048, 5120), True, False, 1.0),      # a C3-sized input rotation (suh)
    ((517, 17408), False, True, 1.0),      # an output rotation (svh) of the MLP width
    ((37, 1024), False, False, 0.5),       # scalar scale
    ((3, 384), True, False, 1.0),          # 3 blocks: one partial span per row
    ((1, 128), False, False, -2.0),        # one block, negative scale
])
def test_had_mfma_vs_oracle(shape, pre, post, scale):
    x = dev_normal(shape, 0, 1, F16, 41)
    p = suh(shape[1], 42) if pre else None
    q = suh(shape[1], 43) if post else None
    got, exp, xin, r, mu = had_case(x, p, q, scale)
    assert_had_close(got, exp, xin, r, what=f"had_r_128_mfma {shape} pre{int(pre)} post{int(post)} s{scale}",
                     max_ulp=mu)


def test_had_mfma_strided_in_place_and_unaligned():
    base = dev_normal((64, 1280), 0, 1, F16, 44)
    x = base[:, :1024]
    ref = x.clone()
    got, exp, xin, r, _ = had_case(ref, out=x)    # strided rows, written over x's storage
    assert_had_close(got, exp, xin, r, what="strided in place")
    assert torch.equal(base[:, 1024:], dev_normal((64, 1280), 0, 1, F16, 44)[:, 1024:])
    u = dev_normal((9, 259), 0, 1, F16, 45)[:, 1:257]     # unaligned rows: the butterfly, bit for bit
    out = torch.empty((9, 256), device="cuda", dtype=torch.float16)
    ffi.had_r_128(u, out, mfma=True)
    torch.cuda.synchronize()
    assert_bitwise(from_dev(out), orc.had_r_128(np.ascontiguousarray(from_dev(u)), F16, nthreads=NTHREADS),
                   what="unaligned -> butterfly")


def special_rows(cols, seed):
    rng = np.random.default_rng(seed)
    x = (rng.standard_normal((16, cols)) * 3).astype(np.float16)
    x[0, 5] = np.inf                                   # one inf: the block is +-inf
    x[1, 7] = -np.inf
    x[1, 9] = np.inf                                   # inf - inf: NaN
    x[2, 100] = np.nan
    x[3] = 0.0
    x[4] = -0.0
    x[5, :128] = -0.0
    x[5, 3] = 1.0                                      # one non-zero among -0s
    x[6] = (rng.integers(-8, 9, cols) * 2.0 ** -24).astype(np.float16)   # subnormals
    x[7] = 60000.0                                     # the transform overflows to inf
    x[8, :128] = np.where(np.arange(128) % 2, 1.0, -1.0)                 # exact cancellations
    x[9] = rng.integers(-2, 3, cols).astype(np.float16)
    return to_dev(x.view(np.uint16), F16)


def test_had_mfma_special_values():
    x = special_rows(512, 46)
    got, exp, xin, r, _ = had_case(x)
    xin = np.where(np.isfinite(xin), xin, 0.0)
    assert_had_close(got, exp, xin, r, what="special values", min_exact=0.9)
    g = f32(got)
    # one inf: every result of its block infinite; +inf and -inf: NaN where their signs meet, else inf
    assert np.isinf(g[0, :128]).all() and np.isnan(g[2, :128]).all()
    assert (np.isnan(g[1, :128]) | np.isinf(g[1, :128])).all() and np.isnan(g[1, :128]).any()
    assert (g[3] == 0).all() and (g[4] == 0).all() and np.isinf(g[7, ::128]).all()


def unfused_mfma(act, x, y, pre, limit, had_scale, rot=(False, False), posts=(None, None)):
    """The matrix-core path as separate calls: input rotations, activation into z, input rotation of z."""
    rx, ry = x, y
    if rot[0]:
        rx = torch.empty_like(x)
        ffi.had_r_128(x, rx, None, posts[0], mfma=True)
    if rot[1]:
        ry = torch.empty_like(y)
        ffi.had_r_128(y, ry, None, posts[1], mfma=True)
    z = torch.empty(x.shape, device="cuda", dtype=torch.float16)
    if act == "mul_sigmoid":
        ffi.mul_sigmoid(rx, ry, z)
    else:
        {"silu": ffi.silu_mul, "gelu": ffi.gelu_mul}[act](rx, ry, z, limit)
    out = torch.empty_like(z)
    ffi.had_r_128(z, out, pre, None, had_scale, mfma=True)
    return rx, ry, z, out


def run(act, rows, cols, it, limit=0.0, pre=True, had_scale=1.0, rot=(False, False), posts=True, seed=0,
        with_z=True):
    x = dev_normal((rows, cols), 0, 2, it, seed)
    y = dev_normal((rows, cols), 0, 1, it, seed + 1)
    p = suh(cols, seed + 2) if pre else None
    ps = tuple(suh(cols, seed + 3 + i) if rot[i] and posts else None for i in range(2))
    z = torch.empty((rows, cols), device="cuda", dtype=torch.float16) if with_z else None
    out = torch.empty((rows, cols), device="cuda", dtype=torch.float16)
    ffi.act_mul_had(act, x, y, out, p, z, limit, had_scale, rotate_x=rot[0], rotate_y=rot[1],
                    x_post_scale=ps[0], y_post_scale=ps[1])
    rx, ry, ez, eout = unfused_mfma(act, x, y, p, limit, had_scale, rot, ps)
    torch.cuda.synchronize()
    tag = f"{act}_had mfma {rows}x{cols} in{it} L{limit} rot{rot}"
    assert_bitwise(from_dev(out), from_dev(eout), what=tag + " vs unfused matrix-core calls")
    if with_z:
        assert_bitwise(from_dev(z), from_dev(ez), what=tag + " z vs unfused")
    # against the oracle: the activation of the (matrix-core) rotated inputs, then the butterfly of z
    gz = from_dev(ez)
    assert_close_ulp(gz, oracle_act(act, rx, ry, it, limit), F16, 1, what=tag + " z vs oracle")
    pz = f32(gz) * (f32(from_dev(p))[None, :] if p is not None else 1.0)
    exp = orc.had_r_128(np.ascontiguousarray(gz), F16, pre=from_dev(p) if p is not None else None, scale=had_scale,
                        nthreads=NTHREADS)
    assert_had_close(from_dev(out), exp, pz, R0 * had_scale, what=tag + " out vs oracle had_r_128(z)")


def test_mlp_tail_c3():
    """The C3 MLP tail from the raw gate_proj / up_proj outputs (both rotated on load), 2048 x 17408."""
    run("silu", 2048, 17408, F16, rot=(True, True), seed=51)


@pytest.mark.parametrize("act", ["silu", "gelu", "mul_sigmoid"])
@pytest.mark.parametrize("it", [F16, BF16, F32])
def test_acts_and_dtypes(act, it):
    run(act, 37, 1024, it, seed=52)


@pytest.mark.parametrize("act,rot", [("silu", (True, False)), ("gelu", (False, True)), ("mul_sigmoid", (True, True))])
def test_rotated_inputs(act, rot):
    run(act, 33, 1152, F16, rot=rot, posts=act != "gelu", seed=53)


def test_limit_scale_partial_spans_no_pre_no_z():
    run("silu", 65, 2048, BF16, limit=2.5, had_scale=0.5, seed=54)
    run("gelu", 9, 384, F16, pre=False, with_z=False, seed=55)
    run("silu", 1, 128, F16, rot=(True, True), seed=56)


def test_exact_flag_is_the_butterfly():
    """EXL3R_HAD_EXACT selects the reference's butterfly: bit for bit the oracle's had_r_128 of z."""
    x = dev_normal((48, 1024), 0, 2, F16, 57)
    y = dev_normal((48, 1024), 0, 1, F16, 58)
    p = suh(1024, 59)
    z = torch.empty_like(x)
    out = torch.empty_like(x)
    ffi.act_mul_had("silu", x, y, out, p, z, exact=True)
    torch.cuda.synchronize()
    exp = orc.had_r_128(np.ascontiguousarray(from_dev(z)), F16, pre=from_dev(p), nthreads=NTHREADS)
    assert_bitwise(from_dev(out), exp, what="exact flag")


def run_norm(rows, dim, xt, rt=None, wt=F16, n_out=3, with_y=True, rotate_x=False, cb=0.0, had_scale=1.0, seed=0):
    """exl3r_rms_norm_had in its default (matrix-core) form: bit for bit the unfused matrix-core calls
    (the input rotation exl3r_had_r_128_mfma, the norm, one exl3r_had_r_128_mfma per output); the norm
    bit for bit the oracle's on the same (rotated) input; each output within the tolerance of the oracle's
    butterfly of that norm."""
    x = dev_normal((rows, dim), 0, 1, xt, seed)
    r = dev_normal((rows, dim), 0, 4, rt, seed + 1) if rt is not None else None
    r2 = r.clone() if r is not None else None
    w = dev_normal((dim,), 1, 0.1, wt, seed + 2)
    y = torch.empty((rows, dim), device="cuda", dtype=torch.float16) if with_y else None
    outs = [torch.empty((rows, dim), device="cuda", dtype=torch.float16) for _ in range(n_out)]
    pres = [suh(dim, seed + 10 + i) if i != 1 else None for i in range(n_out)]
    xsv = suh(dim, seed + 30) if rotate_x else None
    rh = np.ascontiguousarray(from_dev(r)).copy() if r is not None else None
    ffi.rms_norm_had(x, w, outs, pres, 1e-6, cb, 1.0, r=r, y=y, had_scale=had_scale, rotate_x=rotate_x,
                     x_post_scale=xsv)
    xin = x
    if rotate_x:
        xin = torch.empty_like(x)
        ffi.had_r_128(x, xin, None, xsv, mfma=True)
    y2 = torch.empty((rows, dim), device="cuda", dtype=torch.float16)
    if r is not None:
        ffi.rms_norm_res_in(xin, w, y2, r2, 1e-6, cb, 1.0)
    else:
        ffi.rms_norm(xin, w, y2, 1e-6, cb, 1.0)
    sep = []
    for p in pres:
        o = torch.empty_like(y2)
        ffi.had_r_128(y2, o, p, None, had_scale, mfma=True)
        sep.append(o)
    torch.cuda.synchronize()
    tag = f"norm_had mfma {rows}x{dim} x{xt} r{rt} rot{int(rotate_x)}"
    if with_y:
        assert_bitwise(from_dev(y), from_dev(y2), what=tag + " y vs unfused")
    if r is not None:
        assert_bitwise(from_dev(r), from_dev(r2), what=tag + " residual vs unfused")
    for i, (a, b) in enumerate(zip(outs, sep)):
        assert_bitwise(from_dev(a), from_dev(b), what=f"{tag} out{i} vs unfused matrix-core calls")
    xh = np.ascontiguousarray(from_dev(xin))
    ey = orc.rms_norm(xh, xt, from_dev(w), wt, F16, 1e-6, cb, 1.0, r=rh, rt=rt if rt is not None else F32,
                      nthreads=NTHREADS) if r is not None else \
        orc.rms_norm(xh, xt, from_dev(w), wt, F16, 1e-6, cb, 1.0, nthreads=NTHREADS)
    assert_bitwise(from_dev(y2), ey, what=tag + " norm vs oracle")
    for i, (o, p) in enumerate(zip(outs, pres)):
        ph = from_dev(p) if p is not None else None
        exp = orc.had_r_128(ey, F16, pre=ph, scale=had_scale, nthreads=NTHREADS)
        xin_t = f32(ey) * (f32(ph)[None, :] if ph is not None else 1.0)
        assert_had_close(from_dev(o), exp, xin_t, R0 * had_scale, what=f"{tag} out{i} vs oracle")


def test_norm_had_qwen3_attention_input():
    """f16 x into the f32 residual, three projection inputs (q, k, v), the C3 hidden size."""
    run_norm(2048, 5120, F16, F32, n_out=3, with_y=False, seed=61)


def test_norm_had_rotated_layer_boundary():
    """o_proj / down_proj output rotated on load, then the residual norm and three projection inputs."""
    run_norm(1024, 5120, F16, F32, n_out=3, with_y=True, rotate_x=True, seed=62)


@pytest.mark.parametrize("xt,rt,wt", [(F16, None, F16), (BF16, None, BF16), (F32, F16, F32), (BF16, BF16, F16)])
def test_norm_had_dtypes(xt, rt, wt):
    run_norm(67, 1152, xt, rt, wt, n_out=2, cb=1.0, had_scale=0.5, seed=63)


def test_norm_had_wide_rows():
    """Rows over 32768 columns: 8 chunks on each of 1024 lanes (the instances that spill to scratch)."""
    run_norm(3, 40960, F16, F32, n_out=3, with_y=True, rotate_x=True, seed=66)
    run_norm(2, 65536, BF16, None, BF16, n_out=2, seed=67)


def test_norm_had_partial_spans():
    """dim 384: 3 blocks, so the last wave span of a row is part empty (those lanes carry zeros)."""
    run_norm(33, 384, F16, F32, n_out=4, seed=64)
    run_norm(5, 128, F16, None, n_out=1, rotate_x=True, seed=65)


@pytest.mark.parametrize("act,rot", [("silu", (True, True)), ("gelu", (False, False))])
def test_strided_rows_padding_untouched(act, rot):
    """Strided x, y, z and out (row strides past cols): the matrix-core kernel reaches every row through a
    descriptor bounded at the row's bytes, so the padding columns keep their sentinel and every result
    equals the contiguous call's, bit for bit -- also for an odd row count (a row group with a missing
    row) and cols not a multiple of 512 (a span with missing blocks)."""
    rows, cols, ld = 67, 1152, 1152 + 72
    sentinel = 0x7E5A                                  # an f16 NaN pattern no result takes

    def padded(v):
        t = torch.full((rows, ld), 0.0, device="cuda", dtype=torch.float16)
        t[:, :cols] = v
        return t
    x = dev_normal((rows, cols), 0, 2, F16, 91)
    y = dev_normal((rows, cols), 0, 1, F16, 92)
    p = suh(cols, 93)
    ps = tuple(suh(cols, 94 + i) if rot[i] else None for i in range(2))
    zc, oc = torch.empty_like(x), torch.empty_like(x)
    ffi.act_mul_had(act, x, y, oc, p, zc, rotate_x=rot[0], rotate_y=rot[1], x_post_scale=ps[0], y_post_scale=ps[1])
    xs, ys = padded(x), padded(y)
    zs = torch.full((rows, ld), 0.0, device="cuda", dtype=torch.float16).view(torch.int16).fill_(sentinel).view(torch.float16)
    os_ = torch.full((rows, ld), 0.0, device="cuda", dtype=torch.float16).view(torch.int16).fill_(sentinel).view(torch.float16)
    ffi.act_mul_had(act, xs[:, :cols], ys[:, :cols], os_[:, :cols], p, zs[:, :cols], rotate_x=rot[0], rotate_y=rot[1],
                    x_post_scale=ps[0], y_post_scale=ps[1])
    torch.cuda.synchronize()
    for name, got, exp in (("out", os_, oc), ("z", zs, zc)):
        g = got.view(torch.int16).cpu().numpy()
        assert (g[:, cols:] == sentinel).all(), f"{act} {name}: padding written"
        assert_bitwise(np.ascontiguousarray(g[:, :cols]), from_dev(exp).view(np.int16), what=f"{act} {name} strided")
