"""GPU parity of the gated row ops against the CPU oracle: exl3r_gated_rms_norm (Qwen3.5 gated-delta
output norm, Mamba2 group norm), exl3r_mul_sigmoid (gated-attention output gate) and
exl3r_deinterleave_qg (q | g split).  The gate activation is an fp32 evaluation (v_exp_f32 /
v_rcp_f32, 1-ulp approximations) against the oracle's fp64 one, so 16-bit outputs are within 1 ulp
and f32 outputs within 2^-15 relative (as for the act-mul kernels); the deinterleave is bit-exact."""
import numpy as np
import pytest
import torch

import exl3r.ffi as ffi
from _gpu import NTHREADS, TORCH_DT, assert_bitwise, assert_close_rel, assert_close_ulp, dev_normal, from_dev
from oracle import oracle as orc

pytestmark = pytest.mark.gpu

F16, BF16, F32 = orc.F16, orc.BF16, orc.F32


def check(got, exp, code, what):
    if code == F32:
        assert_close_rel(got, exp, 2.0 ** -15, what=what)
    else:
        assert_close_ulp(got, exp, code, 1, what=what)


def run_gated(rows, dim, xt=BF16, gt=F32, wt=F32, yt=F16, w_groups=1, gate_first=False, gate_act=0, cb=0.0,
              with_w=True, seed=0, ld=None):
    ld = ld or dim
    x = dev_normal((rows, ld), 0, 1, xt, seed)[:, :dim]
    g = dev_normal((rows, ld), 0, 2, gt, seed + 1)[:, :dim]
    w = dev_normal((w_groups * dim,), 1, 0.1, wt, seed + 2) if with_w else None
    y = torch.empty((rows, dim), device="cuda", dtype=TORCH_DT[yt])
    ffi.gated_rms_norm(x, w, y, g, 1e-6, cb, w_groups, gate_first, gate_act)
    torch.cuda.synchronize()
    exp = orc.gated_rms_norm(np.ascontiguousarray(from_dev(x)), xt, np.ascontiguousarray(from_dev(g)), gt, yt,
                             w=from_dev(w) if with_w else None, wt=wt, w_groups=w_groups, eps=1e-6, cb=cb,
                             gate_first=gate_first, gate_act=gate_act, nthreads=NTHREADS)
    check(from_dev(y), exp, yt, f"gated {rows}x{dim} x{xt} g{gt} w{wt if with_w else '-'} y{yt} G{w_groups} "
                                f"first{int(gate_first)} act{gate_act}")


@pytest.mark.parametrize("gate_act", [0, 1])
@pytest.mark.parametrize("gate_first", [False, True])
def test_qwen35_gdn_output_norm(gate_act, gate_first):
    # 4096 tokens x 32 value heads, head_dim 128: bf16 core, f32 gate, f32 weight, f16 out (qwen3_5.rs:209-212)
    run_gated(4096 * 32, 128, gate_first=gate_first, gate_act=gate_act, seed=gate_act + 2 * gate_first)


@pytest.mark.parametrize("xt,gt,wt,yt", [(BF16, BF16, BF16, F32), (F16, F16, F16, F16), (BF16, F32, BF16, BF16),
                                         (F32, F32, F32, F32), (F16, BF16, F32, F32)])
def test_dtypes(xt, gt, wt, yt):
    run_gated(37, 256, xt, gt, wt, yt, seed=11)


@pytest.mark.parametrize("rows,dim", [(1, 128), (3, 4096), (5, 8192), (9, 24), (4, 100)])
def test_shapes_groups_bias(rows, dim):
    run_gated(rows, dim, w_groups=3 if rows > 1 else 1, cb=1.0, gate_first=True, gate_act=1, seed=rows + dim)
    run_gated(rows, dim, with_w=False, seed=rows)


@pytest.mark.parametrize("xt,gt,wt,yt", [(F16, F32, F32, F32), (F16, F16, F16, F16), (BF16, BF16, F32, F16)])
def test_wide_rows(xt, gt, wt, yt):
    """Rows over 32768 columns: 8 chunks on each of 1024 lanes (the instances that spill to scratch)."""
    run_gated(2, 65536, xt, gt, wt, yt, gate_act=1, seed=80)
    run_gated(3, 40960, xt, gt, wt, yt, gate_first=True, cb=1.0, seed=81)


def test_strided_rows_generic_path():
    run_gated(11, 128, ld=136, seed=21)                      # 16-byte-aligned rows: vector kernel
    run_gated(11, 128, xt=BF16, gt=BF16, ld=131, seed=22)    # unaligned rows: generic kernel


@pytest.mark.parametrize("it,zt", [(F16, F16), (BF16, BF16), (F16, F32), (F32, F32)])
def test_mul_sigmoid(it, zt):
    x = dev_normal((4096, 4096), 0, 2, it, 31)
    y = dev_normal((4096, 4096), 0, 3, it, 32)
    z = torch.empty_like(x, dtype=TORCH_DT[zt])
    ffi.mul_sigmoid(x, y, z)
    torch.cuda.synchronize()
    exp = orc.mul_sigmoid(from_dev(x), from_dev(y), it, zt, nthreads=NTHREADS)
    check(from_dev(z), exp, zt, f"mul_sigmoid in{it} z{zt}")


def test_mul_sigmoid_gate_read_in_place_from_qg():
    """The attention output gate read in place from an interleaved q | g projection (32 heads of 128 per
    token: rows of 128 with a 256-element stride, the short-row kernel), o updated in place."""
    qg = dev_normal((3000 * 32, 256), 0, 2, F16, 40)
    o = dev_normal((3000 * 32, 128), 0, 1, F16, 41)
    oh, gh = from_dev(o).copy(), np.ascontiguousarray(from_dev(qg)[:, 128:])
    ffi.mul_sigmoid_(o, qg[:, 128:])
    torch.cuda.synchronize()
    check(from_dev(o), orc.mul_sigmoid(oh, gh, F16, F16, nthreads=NTHREADS), F16, "mul_sigmoid_ gate from qg")


def test_mul_sigmoid_in_place_and_tail():
    x = dev_normal((3, 1001), 0, 2, F16, 33)
    y = dev_normal((3, 1001), 0, 3, F16, 34)
    xh, yh = from_dev(x), from_dev(y)
    ffi.mul_sigmoid_(x, y)
    torch.cuda.synchronize()
    check(from_dev(x), orc.mul_sigmoid(xh, yh, F16, F16), F16, "mul_sigmoid_ in place, odd cols")


@pytest.mark.parametrize("dt,heads,hd,rows", [(F16, 32, 128, 4096), (BF16, 8, 64, 33), (F16, 3, 20, 7), (F32, 4, 16, 5)])
def test_deinterleave_qg(dt, heads, hd, rows):
    qg = dev_normal((rows, heads * 2 * hd), 0, 1, dt, 41)
    q = torch.empty((rows, heads, hd), device="cuda", dtype=TORCH_DT[dt])
    g = torch.empty((rows, heads * hd), device="cuda", dtype=TORCH_DT[dt])
    ffi.deinterleave_qg(qg, q, g, hd)
    torch.cuda.synchronize()
    eq, eg = (orc.deinterleave_qg(from_dev(qg), heads, hd) if dt != F32 else
              (from_dev(qg).reshape(rows, heads, 2, hd)[:, :, 0].reshape(rows, -1),
               from_dev(qg).reshape(rows, heads, 2, hd)[:, :, 1].reshape(rows, -1)))
    assert_bitwise(from_dev(q).reshape(rows, -1), eq, what=f"deinterleave q {dt} {heads}x{hd}")
    assert_bitwise(from_dev(g), eg, what=f"deinterleave g {dt} {heads}x{hd}")


def test_zero_rows():
    x = torch.empty((0, 128), device="cuda", dtype=torch.bfloat16)
    ffi.gated_rms_norm(x, None, torch.empty((0, 128), device="cuda", dtype=torch.float16),
                       torch.empty((0, 128), device="cuda", dtype=torch.float32), 1e-6)
    ffi.mul_sigmoid_(torch.empty((0, 64), device="cuda", dtype=torch.float16),
                     torch.empty((0, 64), device="cuda", dtype=torch.float16))
    ffi.deinterleave_qg(torch.empty((0, 256), device="cuda", dtype=torch.float16),
                        torch.empty((0, 1, 128), device="cuda", dtype=torch.float16),
                        torch.empty((0, 128), device="cuda", dtype=torch.float16), 128)
    torch.cuda.synchronize()
