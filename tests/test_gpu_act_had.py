"""GPU parity of exl3r_act_mul_had (the gated activation feeding the next EXL3 projection's
random-Hadamard input rotation in one pass: silu_mul -> down_proj, src/modules.rs:932-940, and the
Qwen3.5 attention gate -> o_proj), with EXL3R_HAD_EXACT (the reference's butterfly; the matrix-core
default is covered by test_gpu_had_mfma.py).  The activation z is checked against the oracle at the
activation's own tolerance (<= 1 ulp of f16); the projection input is checked bit for bit against
the oracle's had_r_128 of that z, and against the unfused GPU calls (exl3r_silu_mul / gelu_mul /
mul_sigmoid into an f16 z, then exl3r_had_r_128).  Covers the MLP prefill shape of Qwen3-32B, every
input dtype, act_limit, a missing pre-scale, a scalar transform scale, strided and unaligned rows
(the unfused fallback), zero rows and the argument errors; and with x and / or y given their producing
projection's output rotation on load (the MLP from the raw gate_proj / up_proj outputs), checked
bitwise against the rotations run first."""
import numpy as np
import pytest
import torch

import exl3r
import exl3r.ffi as ffi
from _gpu import NTHREADS, assert_bitwise, assert_close_ulp, dev_normal, from_dev, to_dev
from oracle import oracle as orc

pytestmark = pytest.mark.gpu

F32, F16, BF16 = orc.F32, orc.F16, orc.BF16
UNFUSED = {"silu": ffi.silu_mul, "gelu": ffi.gelu_mul}


def suh(cols, seed):
    rng = np.random.default_rng(seed)
    return torch.from_numpy((np.where(rng.random(cols) < 0.5, -1.0, 1.0) *
                             (1 + 0.01 * rng.standard_normal(cols))).astype(np.float16)).cuda()


def oracle_act(act, x, y, it, limit):
    xh, yh = np.ascontiguousarray(from_dev(x)), np.ascontiguousarray(from_dev(y))
    if act == "mul_sigmoid":
        return orc.mul_sigmoid(xh, yh, it, F16, nthreads=NTHREADS)
    code = orc.ACT_SILU if act == "silu" else orc.ACT_GELU
    return orc.act_mul(code, xh, yh, it, F16, limit, nthreads=NTHREADS)


def unfused(act, x, y, pre, limit, had_scale):
    z = torch.empty(x.shape, device="cuda", dtype=torch.float16)
    if act == "mul_sigmoid":
        ffi.mul_sigmoid(x, y, z)
    else:
        UNFUSED[act](x, y, z, limit)
    out = torch.empty_like(z)
    ffi.had_r_128(z, out, pre, None, had_scale)
    return z, out


def run(act, rows, cols, it, limit=0.0, with_z=True, pre=True, had_scale=1.0, ld=None, off=0, seed=0):
    ld = ld or cols
    x = dev_normal((rows, ld + off), 0, 2, it, seed)[:, off:off + cols]
    y = dev_normal((rows, ld + off), 0, 1, it, seed + 1)[:, off:off + cols]
    p = suh(cols, seed + 2) if pre else None
    z = torch.empty((rows, cols), device="cuda", dtype=torch.float16) if with_z else None
    out = torch.empty((rows, cols), device="cuda", dtype=torch.float16)
    ffi.act_mul_had(act, x, y, out, p, z, limit, had_scale, exact=True)
    ez, eout = unfused(act, x, y, p, limit, had_scale)
    torch.cuda.synchronize()
    tag = f"{act}_had {rows}x{cols} in{it} L{limit} z{int(with_z)} pre{int(pre)} ld{ld} off{off}"
    assert_bitwise(from_dev(out), from_dev(eout), what=tag + " vs unfused")
    if with_z:
        gz = from_dev(z)
        assert_bitwise(gz, from_dev(ez), what=tag + " z vs unfused")
        assert_close_ulp(gz, oracle_act(act, x, y, it, limit), F16, 1, what=tag + " z vs oracle")
        exp = orc.had_r_128(np.ascontiguousarray(gz), F16, pre=from_dev(p) if p is not None else None,
                            scale=had_scale, nthreads=NTHREADS)
        assert_bitwise(from_dev(out), exp, what=tag + " out vs oracle had_r_128(z)")


def test_qwen3_down_proj_input_prefill():
    """silu(gate) * up of Qwen3-32B prefill, 2048 x 25600 f16, into down_proj's input rotation."""
    run("silu", 2048, 25600, F16, seed=1)


@pytest.mark.parametrize("act", ["silu", "gelu", "mul_sigmoid"])
@pytest.mark.parametrize("it", [F16, BF16, F32])
def test_acts_and_dtypes(act, it):
    run(act, 37, 1024, it, seed=3)


def test_limit_scale_missing_pre_and_no_z():
    run("silu", 65, 2048, BF16, limit=2.5, had_scale=0.5, seed=4)
    run("gelu", 65, 2048, F16, pre=False, with_z=False, seed=5)
    run("silu", 1, 384, F16, with_z=False, seed=6)


def test_strided_and_unaligned_rows():
    run("silu", 19, 512, F16, ld=520, seed=7)                       # strided, vector kernel
    run("gelu", 19, 512, F16, ld=515, seed=8)                       # unaligned stride: unfused fallback
    run("mul_sigmoid", 7, 256, BF16, off=1, with_z=False, seed=9)    # unaligned base: fallback into out


def run_rotated(act, rows, cols, rot_x, rot_y, posts=True, with_z=True, seed=0):
    """x / y are raw projection outputs: the fused call rotates them on load; the reference path rotates
    them first (had_r_128 with post-scale), then runs the unfused activation and input rotation."""
    x = dev_normal((rows, cols), 0, 2, F16, seed)
    y = dev_normal((rows, cols), 0, 1, F16, seed + 1)
    p = suh(cols, seed + 2)
    xs = suh(cols, seed + 3) if rot_x and posts else None
    ys = suh(cols, seed + 4) if rot_y and posts else None
    z = torch.empty((rows, cols), device="cuda", dtype=torch.float16) if with_z else None
    out = torch.empty((rows, cols), device="cuda", dtype=torch.float16)
    ffi.act_mul_had(act, x, y, out, p, z, rotate_x=rot_x, rotate_y=rot_y, x_post_scale=xs, y_post_scale=ys, exact=True)
    rx, ry = x, y
    if rot_x:
        rx = torch.empty_like(x)
        ffi.had_r_128(x, rx, None, xs)
    if rot_y:
        ry = torch.empty_like(y)
        ffi.had_r_128(y, ry, None, ys)
    ez, eout = unfused(act, rx, ry, p, 0.0, 1.0)
    torch.cuda.synchronize()
    tag = f"{act}_had rotated x{int(rot_x)} y{int(rot_y)} {rows}x{cols}"
    assert_bitwise(from_dev(out), from_dev(eout), what=tag + " vs unfused")
    if with_z:
        assert_bitwise(from_dev(z), from_dev(ez), what=tag + " z vs unfused")
        # the rotated inputs against the oracle's rotation, bit for bit
        ox = orc.had_r_128(np.ascontiguousarray(from_dev(x)), F16, post=from_dev(xs) if xs is not None else None,
                           nthreads=NTHREADS) if rot_x else from_dev(x)
        oy = orc.had_r_128(np.ascontiguousarray(from_dev(y)), F16, post=from_dev(ys) if ys is not None else None,
                           nthreads=NTHREADS) if rot_y else from_dev(y)
        assert_bitwise(from_dev(rx), ox, what=tag + " rotated x")
        assert_bitwise(from_dev(ry), oy, what=tag + " rotated y")
        assert_close_ulp(from_dev(z), oracle_act(act, rx, ry, F16, 0.0), F16, 1, what=tag + " z vs oracle")


def test_mlp_tail_rotated_gate_and_up():
    """The Qwen3-32B MLP at prefill from the raw gate_proj / up_proj outputs: their svh rotations, silu(g) * u
    and down_proj's input rotation in one pass."""
    run_rotated("silu", 1024, 25600, True, True, with_z=False, seed=21)


@pytest.mark.parametrize("act,rx,ry", [("silu", True, False), ("gelu", False, True), ("mul_sigmoid", False, True),
                                       ("mul_sigmoid", True, True)])
def test_rotated_inputs(act, rx, ry):
    run_rotated(act, 33, 1024, rx, ry, posts=act != "gelu", seed=22)


def test_zero_rows_and_errors():
    z0 = torch.empty((0, 256), device="cuda", dtype=torch.float16)
    ffi.act_mul_had("silu", z0, z0, torch.empty_like(z0))
    x = dev_normal((4, 256), 0, 1, F16, 10)
    y = dev_normal((4, 256), 0, 1, F16, 11)
    with pytest.raises(exl3r.Exl3rError):
        bad = dev_normal((4, 200), 0, 1, F16, 12)
        ffi.act_mul_had("silu", bad, bad.clone(), torch.empty_like(bad))
    with pytest.raises(exl3r.Exl3rError):
        ffi.act_mul_had("silu", x, y, x)                                     # out aliases x
    with pytest.raises(exl3r.Exl3rError):
        ffi.act_mul_had("mul_sigmoid", x, y, torch.empty_like(x), act_limit=1.0)
    rc = exl3r.load().exl3r_act_mul_had(7, x.data_ptr(), y.data_ptr(), F16, 256, 256, None, 0, None,
                                        torch.empty_like(x).data_ptr(), 256, 4, 256, 0.0, 1.0, 0, None, None, None)
    assert rc == exl3r.EINVAL
    with pytest.raises(exl3r.Exl3rError):                                   # rotated inputs are f16
        xb = x.to(torch.bfloat16)
        ffi.act_mul_had("silu", xb, xb.clone(), torch.empty_like(x), rotate_x=True)
    with pytest.raises(exl3r.Exl3rError):                                   # post-scale without its rotation
        ffi.act_mul_had("silu", x, y, torch.empty_like(x), y_post_scale=suh(256, 1))
    with pytest.raises(exl3r.Exl3rError):                                   # unaligned rows cannot rotate inputs
        xs = dev_normal((4, 259), 0, 1, F16, 13)[:, :256]
        ffi.act_mul_had("silu", xs, xs, torch.empty_like(x), rotate_x=True)
    torch.cuda.synchronize()


def zero_sign_rows(rows, cols, seed):
    """f16 rows built to exercise the signs of exact zeros in the rotations: small integers (exact
    cancellations inside the butterflies), rows of +0, rows of -0, rows whose first 128-block has one
    16-lane chunk (8 values) of -0 among non-zero values, and blocks half +0, half non-zero."""
    rng = np.random.default_rng(seed)
    x = rng.integers(-2, 3, (rows, cols)).astype(np.float16)
    x[1] = 0.0
    x[2] = -0.0
    x[3, :8] = -0.0
    x[4].reshape(-1, 128)[:, :64] = 0.0
    x[5].reshape(-1, 128)[:, 64:] = -0.0
    x[6, 128:256] = -0.0
    return to_dev(x.view(np.uint16), F16)


@pytest.mark.parametrize("act", ["silu", "mul_sigmoid"])
def test_rotated_inputs_zero_signs(act):
    """x / y rotated on load where the rotations produce exact zeros: the fused kernel's butterflies
    (the carried-sign lane stages, or the exact ones for a wave holding 8 zeros with a -0 in one lane)
    against the unfused exact calls, bit for bit, signs of zeros included; and the rotations themselves
    against the oracle."""
    rows, cols = 40, 1024
    x, y = zero_sign_rows(rows, cols, 31), zero_sign_rows(rows, cols, 32)
    y[2:4] = y[2:4].neg()
    p = torch.from_numpy(np.where(np.random.default_rng(33).random(cols) < 0.5, -1.0, 1.0).astype(np.float16)).cuda()
    z = torch.empty((rows, cols), device="cuda", dtype=torch.float16)
    out = torch.empty((rows, cols), device="cuda", dtype=torch.float16)
    ffi.act_mul_had(act, x, y, out, p, z, rotate_x=True, rotate_y=True, exact=True)
    rx, ry = torch.empty_like(x), torch.empty_like(y)
    ffi.had_r_128(x, rx, None, None)
    ffi.had_r_128(y, ry, None, None)
    ez, eout = unfused(act, rx, ry, p, 0.0, 1.0)
    torch.cuda.synchronize()
    assert_bitwise(from_dev(rx), orc.had_r_128(np.ascontiguousarray(from_dev(x)), F16, nthreads=NTHREADS), what="rotated x")
    assert_bitwise(from_dev(ry), orc.had_r_128(np.ascontiguousarray(from_dev(y)), F16, nthreads=NTHREADS), what="rotated y")
    zeros = (from_dev(rx) & 0x7fff) == 0
    assert zeros.sum() > 1000 and (from_dev(rx)[zeros] == 0x8000).any()    # the cases are there
    assert_bitwise(from_dev(z), from_dev(ez), what=f"{act} zero signs: z")
    assert_bitwise(from_dev(out), from_dev(eout), what=f"{act} zero signs: out")
