"""GPU parity of exl3r_silu_mul / exl3r_gelu_mul against the CPU oracle: <= 1 ulp for 16-bit z,
max abs err <= 2e-3 of the output scale (one ulp for bf16).  An f32 z (an extension: the
reference writes f16) carries the fp32 evaluation error of the GPU (v_exp_f32 / v_rcp_f32 are
1-ulp approximations, and the fp32 rounding of the exponent argument t = x (K1 + K2 x^2) shifts
exp2(t) by ~|t| 2^-23 ln 2 relative, with |t| <= ~150 before the result underflows; the oracle
evaluates in fp64): elementwise relative error <= 2^-15 (plus a few denormal ulps)."""
import numpy as np
import pytest
import torch

import exl3r.ffi as ffi
from _gpu import NTHREADS, TORCH_DT, assert_close_rel, assert_close_ulp, dev_normal, from_dev
from oracle import oracle as orc

pytestmark = pytest.mark.gpu

F16, BF16, F32 = orc.F16, orc.BF16, orc.F32
ACTS = {"silu": (ffi.silu_mul, orc.ACT_SILU), "gelu": (ffi.gelu_mul, orc.ACT_GELU)}


def run(act, rows, cols, it, zt, limit=0.0, seed=0, ld=None, std=1.0):
    fn, code = ACTS[act]
    ld = ld or cols
    xs = dev_normal((rows, ld), 0.0, std, it, seed)
    ys = dev_normal((rows, ld), 0.0, 1.0, it, seed + 1)
    x, y = xs[:, :cols], ys[:, :cols]
    z = torch.empty((rows, cols), device="cuda", dtype=TORCH_DT[zt])
    fn(x, y, z, limit)
    torch.cuda.synchronize()
    exp = orc.act_mul(code, np.ascontiguousarray(from_dev(x)), np.ascontiguousarray(from_dev(y)), it, zt, limit,
                      nthreads=NTHREADS)
    what = f"{act} {rows}x{cols} in={it} z={zt} L={limit}"
    if zt == F32:
        assert_close_rel(from_dev(z), exp, 2.0 ** -15, what=what)
    else:
        assert_close_ulp(from_dev(z), exp, zt, 1, what=what)


@pytest.mark.parametrize("act", ["silu", "gelu"])
def test_c1_f16(act):
    """Config 1(2): gate, up [512, 3072] f16 ~ N(0, 1)."""
    run(act, 512, 3072, F16, F16)


@pytest.mark.parametrize("act", ["silu", "gelu"])
def test_c3_bf16_full(act):
    """Config 3(2)/(3): gate, up [8192, 17408] bf16 ~ N(0, 1) (full size)."""
    run(act, 8192, 17408, BF16, BF16, seed=3)


@pytest.mark.parametrize("act", ["silu", "gelu"])
@pytest.mark.parametrize("it", [F16, BF16, F32])
@pytest.mark.parametrize("zt", [F16, BF16, F32])
def test_dtype_matrix(act, it, zt):
    run(act, 13, 1000, it, zt, seed=it * 3 + zt, std=4.0)


@pytest.mark.parametrize("act", ["silu", "gelu"])
def test_wide_range_and_limit(act):
    run(act, 64, 4096, F16, F16, std=8.0, seed=11)
    run(act, 64, 4096, BF16, BF16, std=30.0, seed=12)
    run(act, 64, 4096, F16, F16, limit=7.0, std=8.0, seed=13)


@pytest.mark.parametrize("act", ["silu", "gelu"])
def test_strided_odd_and_tail(act):
    run(act, 64, 1024, BF16, BF16, ld=2048, seed=21)     # gate/up as column slices of [T, 2I]
    run(act, 7, 1001, F16, F16, seed=22)                  # flat, 7007 % 8 != 0 -> vector body + tail
    run(act, 7, 1001, F16, F16, ld=1003, seed=23)         # strided odd rows -> generic kernel
    run(act, 1, 5, F16, F16, seed=24)                     # smaller than one chunk
    run(act, 4099, 128, F16, F16, ld=256, seed=25)        # short strided rows: the flattened short-row kernel
    run(act, 33, 512, BF16, F32, ld=520, limit=3.0, seed=26)   # 64 chunks per row, act_limit


@pytest.mark.parametrize("act", ["silu", "gelu"])
@pytest.mark.parametrize("it,zt", [(F32, F16), (F16, F32), (F32, F32), (BF16, F32)])
def test_split_chunks_f32(act, it, zt):
    """An f32 side with rows of whole 512-element spans: split chunks (two quads 256 apart per lane),
    contiguous, strided (gate / up as column slices) and with act_limit."""
    run(act, 40, 2048, it, zt, seed=31 + it + zt, std=4.0)
    run(act, 24, 1024, it, zt, ld=2048, seed=32 + it + zt)
    run(act, 9, 4608, it, zt, limit=5.0, std=6.0, seed=33 + it + zt)


def test_in_place_and_specials():
    x = torch.tensor([[0.0, -0.0, 60.0, -60.0, float("inf"), float("-inf"), float("nan"), 300.0]], device="cuda")
    y = torch.tensor([[5.0, 5.0, 3.0, 3.0, 1.0, 1.0, 1.0, 300.0]], device="cuda")
    for act, (fn, code) in ACTS.items():
        xs, ys = x.clone(), y.clone()
        exp = orc.act_mul(code, from_dev(xs), from_dev(ys), F32, F16)
        z = torch.empty(x.shape, device="cuda", dtype=torch.float16)
        fn(xs, ys, z)
        assert_close_ulp(from_dev(z), exp, F16, 0, rel=0.0, what=f"{act} specials")
        xh = x.half().contiguous()
        exp2 = orc.act_mul(code, from_dev(xh), from_dev(y.half()), F16, F16)
        fn(xh, y.half(), xh)                                # z == x in place
        assert_close_ulp(from_dev(xh), exp2, F16, 0, rel=0.0, what=f"{act} in place")


def test_zero_rows():
    x = torch.empty((0, 17408), device="cuda", dtype=torch.bfloat16)
    ffi.silu_mul(x, x, torch.empty_like(x))
    ffi.gelu_mul(x, x, torch.empty_like(x))
    torch.cuda.synchronize()
