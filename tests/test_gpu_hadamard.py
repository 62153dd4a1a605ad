"""GPU parity of exl3r_had_r_128 (the EXL3 linear's random-Hadamard input / output rotation,
src/modules.rs:224-231) against the CPU oracle, itself pinned to scipy's Sylvester matrix: bit-exact
on both kernels (16-byte aligned rows, and any alignment through LDS) for f16 and f32, with the
pre-scale (suh), the post-scale (svh) or neither, a scalar scale, strided rows, in place, the
prefill shape of a Qwen3-32B projection, zero-size calls and the argument errors."""
import numpy as np
import pytest
import torch

import exl3r
import exl3r.ffi as ffi
from _gpu import NTHREADS, assert_bitwise, dev_normal, from_dev
from oracle import oracle as orc

pytestmark = pytest.mark.gpu

F16, F32 = orc.F16, orc.F32


def scales(cols, seed):
    rng = np.random.default_rng(seed)
    s = np.where(rng.random(cols) < 0.5, -1.0, 1.0) * (1 + 0.02 * rng.standard_normal(cols))
    return torch.from_numpy(s.astype(np.float16)).cuda()


def run(x, dt, pre=None, post=None, scale=1.0, out=None, what=""):
    out = torch.empty_like(x) if out is None else out
    xh = np.ascontiguousarray(from_dev(x))
    ffi.had_r_128(x, out, pre, post, scale)
    torch.cuda.synchronize()
    exp = orc.had_r_128(xh, dt, pre=from_dev(pre) if pre is not None else None,
                        post=from_dev(post) if post is not None else None, scale=scale, nthreads=NTHREADS)
    got = np.ascontiguousarray(from_dev(out))
    assert_bitwise(got.view(np.uint32) if dt == F32 else got, exp.view(np.uint32) if dt == F32 else exp, what=what)


def test_prefill_projection_input():
    """8192 tokens x 5120 (a Qwen3-32B q/k/v/gate/up input) with suh, f16."""
    run(dev_normal((8192, 5120), 0, 1, F16, 1), F16, pre=scales(5120, 2), what="had f16 [8192,5120] suh")


@pytest.mark.parametrize("dt", [F16, F32])
@pytest.mark.parametrize("mode", ["pre", "post", "none"])
def test_dtypes_and_scales(dt, mode):
    x = dev_normal((77, 1024), 0, 3, dt, 3)
    s = scales(1024, 4)
    run(x, dt, pre=s if mode == "pre" else None, post=s if mode == "post" else None, scale=0.75,
        what=f"had dt{dt} {mode}")


def test_in_place_strided_and_unaligned():
    base = dev_normal((33, 640 + 8), 0, 1, F16, 5)
    run(base[:, :640], F16, pre=scales(640, 6), what="strided rows (vector kernel)")
    x = base[:, :640].clone()
    xh = from_dev(x)
    ffi.had_r_128(x, x, None, scales(640, 7))
    torch.cuda.synchronize()
    assert_bitwise(from_dev(x), orc.had_r_128(xh, F16, post=from_dev(scales(640, 7))), what="in place")
    odd = dev_normal((9, 257), 0, 1, F32, 8)
    run(odd[:, 1:], F32, pre=scales(256, 9), what="unaligned rows (generic kernel)")
    run(dev_normal((5, 384 + 3), 0, 1, F16, 10)[:, :384], F16, what="odd stride (generic kernel)")


def test_signed_zeros_and_special_values():
    """Zero blocks of either sign (an exact zero's sign follows the butterfly's order: (-0) + (-0) = -0,
    (+0) - (+0) = +0), infinities, overflow to infinity, NaN and f16 subnormals, with a sign-flipping
    pre-scale.  Finite
    and infinite results are compared bit for bit; NaN positions must agree (a NaN's sign and payload
    are the arithmetic unit's own)."""
    cols = 256
    x = np.zeros((8, cols), np.float16)
    x[1] = -0.0
    x[2, ::3] = -0.0
    x[3, 5] = np.inf
    x[4, 7] = np.nan
    x[5] = 60000.0
    x[6, 3], x[6, 9] = np.inf, -np.inf
    # f16 subnormals of both signs next to zeros (the first butterfly stage converts the packed halves itself)
    x[7] = (np.random.default_rng(3).integers(-1023, 1024, cols) * 2.0 ** -24).astype(np.float16)
    pre = np.where(np.arange(cols) % 5 == 0, -1.0, 1.0).astype(np.float16)
    xd = torch.from_numpy(x.view(np.int16)).view(torch.float16).cuda()
    pd = torch.from_numpy(pre.view(np.int16)).view(torch.float16).cuda()
    for p_ in (None, pd):
        out = torch.empty_like(xd)
        ffi.had_r_128(xd, out, p_)
        torch.cuda.synchronize()
        got = from_dev(out).view(np.float16)
        exp = orc.had_r_128(x.view(np.uint16), F16, pre=pre.view(np.uint16) if p_ is not None else None).view(np.float16)
        gn, en = np.isnan(got), np.isnan(exp)
        assert np.array_equal(gn, en), "NaN positions differ"
        assert np.array_equal(got.view(np.uint16)[~gn], exp.view(np.uint16)[~en]), "non-NaN results differ bitwise"
        if p_ is None:
            # an all -0 block: only the all-plus row of H sums -0 + -0 ...; every other output is +0
            assert np.array_equal(np.nonzero(np.signbit(got[1]))[0], [0, 128])
            # one infinity spreads over its whole block (the other block stays zero); a constant block
            # of 60000 sums to 60000 * sqrt(128) at output 0 -- past the f16 range -- and to zero elsewhere
            assert np.isinf(got[3, :128]).all() and not got[3, 128:].any()
            assert np.isinf(got[5, [0, 128]]).all() and not np.delete(got[5], [0, 128]).any()


def test_involution_on_device():
    x = dev_normal((64, 512), 0, 1, F32, 11)
    y = torch.empty_like(x)
    ffi.had_r_128(x, y)
    ffi.had_r_128(y, y)
    torch.cuda.synchronize()
    assert torch.max(torch.abs(y - x)).item() < 1e-5


def test_zero_size_and_errors():
    z = torch.empty((0, 256), device="cuda", dtype=torch.float16)
    ffi.had_r_128(z, z)
    x = dev_normal((2, 256), 0, 1, F16, 12)
    with pytest.raises(exl3r.Exl3rError):
        ffi.had_r_128(x, x, scales(256, 13), scales(256, 14))
    bad = dev_normal((2, 200), 0, 1, F16, 15)
    with pytest.raises(exl3r.Exl3rError):
        ffi.had_r_128(bad, bad)
    with pytest.raises(exl3r.Exl3rError):
        ffi.had_r_128(x.to(torch.bfloat16), x.to(torch.bfloat16))
    torch.cuda.synchronize()
