"""GPU parity of exl3r_rms_norm_had with EXL3R_HAD_EXACT (RMSNorm, optionally with the residual add,
feeding the random-Hadamard input rotation of up to four EXL3 projections in one pass; the matrix-core
default is covered by test_gpu_had_mfma.py) against the oracle
composition -- oracle_rms_norm to an f16 y, then oracle_had_r_128 per projection, after
oracle_had_r_128(x, post=svh) when x is rotated on load -- bit for bit, and against the unfused GPU
calls: the Qwen3 attention-input case (f16 x, f32 residual, three
projections), plain norms, Qwen3.5's constant bias, a scalar transform scale, the unaligned fallback
with and without y, zero rows and the argument errors."""
import numpy as np
import pytest
import torch

import exl3r
import exl3r.ffi as ffi
from _gpu import NTHREADS, TORCH_DT, assert_bitwise, dev_normal, from_dev, to_dev
from oracle import oracle as orc

pytestmark = pytest.mark.gpu

F32, F16, BF16 = orc.F32, orc.F16, orc.BF16


def suh(dim, seed):
    rng = np.random.default_rng(seed)
    return torch.from_numpy(np.where(rng.random(dim) < 0.5, -1.0, 1.0).astype(np.float16)).cuda()


def run(rows, dim, xt, rt=None, wt=F16, n_out=3, with_y=True, cb=0.0, had_scale=1.0, ld=None, seed=0, pre_none=(),
        rotate_x=False, svh=True):
    ld = ld or dim
    x = dev_normal((rows, ld), 0, 1, xt, seed)[:, :dim]
    r = dev_normal((rows, ld), 0, 4, rt, seed + 1)[:, :dim] if rt is not None else None
    w = dev_normal((dim,), 1, 0.1, wt, seed + 2)
    y = torch.empty((rows, dim), device="cuda", dtype=torch.float16) if with_y else None
    outs = [torch.empty((rows, dim), device="cuda", dtype=torch.float16) for _ in range(n_out)]
    pres = [None if i in pre_none else suh(dim, seed + 10 + i) for i in range(n_out)]
    xh = np.ascontiguousarray(from_dev(x))
    rh = np.ascontiguousarray(from_dev(r)).copy() if r is not None else None
    wh = from_dev(w)
    xsv = suh(dim, seed + 30) if rotate_x and svh else None
    ffi.rms_norm_had(x, w, outs, pres, 1e-6, cb, 1.0, r=r, y=y, had_scale=had_scale, rotate_x=rotate_x,
                     x_post_scale=xsv, exact=True)
    torch.cuda.synchronize()
    if rotate_x:      # the producer's output rotation, had_r_128(x, x, None, svh), before the norm
        xh = orc.had_r_128(xh, F16, post=from_dev(xsv) if xsv is not None else None, nthreads=NTHREADS)
    ey = orc.rms_norm(xh, xt, wh, wt, F16, 1e-6, cb, 1.0, r=rh, rt=rt if rt is not None else F32, nthreads=NTHREADS) \
        if r is not None else orc.rms_norm(xh, xt, wh, wt, F16, 1e-6, cb, 1.0, nthreads=NTHREADS)
    tag = f"norm_had {rows}x{dim} x{xt} r{rt} out{n_out} y{int(with_y)} rot{int(rotate_x)}"
    if with_y:
        assert_bitwise(from_dev(y), ey, what=tag + " y")
    if r is not None:
        assert_bitwise(np.ascontiguousarray(from_dev(r)), rh, what=tag + " residual")
    for i, o in enumerate(outs):
        exp = orc.had_r_128(ey, F16, pre=from_dev(pres[i]) if pres[i] is not None else None, scale=had_scale,
                            nthreads=NTHREADS)
        assert_bitwise(from_dev(o), exp, what=f"{tag} out{i}")
    return x, r, w, outs, pres


def test_qwen3_attention_input_prefill():
    """f16 sublayer output into the f32 residual stream, three projection inputs (q, k, v)."""
    run(2048, 5120, F16, F32, n_out=3, with_y=False, seed=1)


@pytest.mark.parametrize("xt,rt,wt", [(F16, None, F16), (BF16, None, BF16), (F32, F16, F32), (BF16, BF16, F16)])
def test_dtypes_plain_and_residual(xt, rt, wt):
    run(67, 1024, xt, rt, wt, n_out=2, seed=2)


def test_four_outputs_bias_scale_and_missing_pre():
    run(33, 2048, F16, F32, n_out=4, cb=1.0, had_scale=0.5, pre_none=(1,), seed=3)


def test_rotated_input_qwen3_layer_boundary():
    """o_proj / down_proj output (raw f16, before its svh rotation) into the f32 residual, then the
    next norm's three projection inputs: one pass for had(svh) -> residual add -> norm -> 3 x had(suh)."""
    run(2048, 5120, F16, F32, n_out=3, with_y=False, rotate_x=True, seed=11)


@pytest.mark.parametrize("rt", [None, F32, F16, BF16])
def test_rotated_input_variants(rt):
    run(45, 1024, F16, rt, F32, n_out=2, with_y=True, rotate_x=True, svh=rt != F16, cb=1.0, seed=12)


def test_wide_rows():
    """Rows over 32768 columns (8 chunks on each of 1024 lanes, the instances that spill), the butterfly."""
    run(3, 40960, F16, F32, n_out=3, with_y=True, rotate_x=True, seed=15)
    run(2, 65536, F32, F32, F32, n_out=1, with_y=True, seed=16)


def test_rotated_input_unaligned_fallback():
    run(9, 256, F16, F32, n_out=2, with_y=False, ld=259, rotate_x=True, seed=13)
    run(9, 256, F16, None, n_out=1, with_y=True, ld=259, rotate_x=True, seed=14)


def test_unaligned_fallback():
    run(9, 256, F16, F32, n_out=2, with_y=True, ld=259, seed=4)
    run(9, 256, F16, None, n_out=3, with_y=False, ld=259, seed=5)


def test_fused_equals_unfused_gpu_calls():
    rows, dim = 512, 4096
    x = dev_normal((rows, dim), 0, 1, F16, 6)
    r1 = dev_normal((rows, dim), 0, 4, F32, 7)
    r2 = r1.clone()
    w = dev_normal((dim,), 1, 0.1, F16, 8)
    pres = [suh(dim, 20 + i) for i in range(3)]
    fused = [torch.empty((rows, dim), device="cuda", dtype=torch.float16) for _ in range(3)]
    ffi.rms_norm_had(x, w, fused, pres, 1e-6, r=r1, exact=True)
    y = torch.empty((rows, dim), device="cuda", dtype=torch.float16)
    ffi.rms_norm_res_in(x, w, y, r2, 1e-6)
    sep = [torch.empty_like(y) for _ in range(3)]
    for o, p in zip(sep, pres):
        ffi.had_r_128(y, o, p)
    torch.cuda.synchronize()
    assert torch.equal(r1, r2)
    for a, b in zip(fused, sep):
        assert torch.equal(a.view(torch.int16), b.view(torch.int16))


def test_zero_rows_and_errors():
    z = torch.empty((0, 256), device="cuda", dtype=torch.float16)
    ffi.rms_norm_had(z, None, [torch.empty_like(z)], [None], 1e-6)
    x = dev_normal((4, 256), 0, 1, F16, 9)
    o = torch.empty_like(x)
    with pytest.raises(exl3r.Exl3rError):
        bad = dev_normal((4, 200), 0, 1, F16, 10)
        ffi.rms_norm_had(bad, None, [torch.empty_like(bad)], [None], 1e-6)
    with pytest.raises(exl3r.Exl3rError):
        ffi.rms_norm_had(x, None, [x], [None], 1e-6)                  # output aliases x
    with pytest.raises(ValueError):
        ffi.rms_norm_had(x, None, [o] * 5, [None] * 5, 1e-6)
    with pytest.raises(exl3r.Exl3rError):
        ffi.rms_norm_had(x, None, [o, o], [None, None], 1e-6)          # outputs alias each other
    with pytest.raises(exl3r.Exl3rError):
        xb = x.to(torch.bfloat16)
        ffi.rms_norm_had(xb, None, [o], [None], 1e-6, rotate_x=True)   # the rotation takes f16 x
    with pytest.raises(exl3r.Exl3rError):
        ffi.rms_norm_had(x, None, [o], [None], 1e-6, x_post_scale=suh(256, 1))   # post-scale without rotate_x
    torch.cuda.synchronize()


def test_zero_signs_of_the_rotations():
    """Norm outputs whose rotations produce exact zeros (x in {-1, 0, 1}, unit weights, +-1 pre-scales:
    whole blocks cancel), rows of +0 and of -0, a lane of -0 among non-zero values: the fused
    butterflies (carried-sign lane stages where valid, else exact) against the oracle, bit for bit,
    signs of zeros included."""
    rows, dim = 24, 1024
    rng = np.random.default_rng(41)
    xh = rng.integers(-1, 2, (rows, dim)).astype(np.float16)
    xh[1] = 0.0
    xh[2] = -0.0
    xh[3, :8] = -0.0
    xh[4].reshape(-1, 128)[:, :64] = 0.0
    xh[5, 128:256] = -0.0
    xh[6] = 1.0
    x = to_dev(xh.view(np.uint16), F16)
    w = torch.ones(dim, device="cuda", dtype=torch.float16)
    y = torch.empty((rows, dim), device="cuda", dtype=torch.float16)
    outs = [torch.empty((rows, dim), device="cuda", dtype=torch.float16) for _ in range(3)]
    pres = [suh(dim, 50 + i) for i in range(3)]
    ffi.rms_norm_had(x, w, outs, pres, 1e-6, 0.0, 1.0, y=y, exact=True)
    torch.cuda.synchronize()
    ey = orc.rms_norm(xh.view(np.uint16), F16, from_dev(w), F16, F16, 1e-6, 0.0, 1.0, nthreads=NTHREADS)
    assert_bitwise(from_dev(y), ey, what="zero signs: y")
    nzero = 0
    for i, o in enumerate(outs):
        exp = orc.had_r_128(ey, F16, pre=from_dev(pres[i]), nthreads=NTHREADS)
        nzero += int(((exp & 0x7fff) == 0).sum())
        assert_bitwise(from_dev(o), exp, what=f"zero signs: out{i}")
    assert nzero > 1000    # the cancellations are there
