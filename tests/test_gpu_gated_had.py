"""GPU parity of exl3r_gated_rms_norm_had: the Qwen3.5 gated-delta-net output norm whose f16 output feeds
o_proj's random-Hadamard input rotation in one pass (src/qwen3_5.rs:208-214 -> src/modules.rs:224-227).
The rotated output is checked bit for bit against the unfused GPU calls with the same form of the
transform (exl3r_gated_rms_norm into an f16 y, then exl3r_had_r_128_mfma for rows of 128 on the
short-row kernel, exl3r_had_r_128 with EXL3R_HAD_EXACT and elsewhere) and against the oracle's rotation
of that y (bitwise with the butterfly, within the matrix-core transform's tolerance otherwise); y itself
against the oracle at the gated norm's tolerance (<= 1 ulp of f16).  Covers the Qwen3.5 prefill shape
(head_dim-128 rows on the short-row kernel) in both forms, row counts that end inside a wave's 4 rows,
longer rows (the workgroup kernel), both gates before and after the norm, weight groups, a bias, a
missing pre-scale, the unaligned fallback, zero rows and the errors."""
import numpy as np
import pytest
import torch

import exl3r
import exl3r.ffi as ffi
from _gpu import NTHREADS, assert_bitwise, assert_close_ulp, assert_had_close, dev_normal, from_dev
from oracle import oracle as orc
from test_gpu_act_had import suh

pytestmark = pytest.mark.gpu

F32, F16, BF16 = orc.F32, orc.F16, orc.BF16


def run(rows, dim, xt=BF16, gt=F32, wt=F32, w_groups=1, gate_first=False, gate_act=0, cb=0.0, with_w=True,
        with_y=True, pre=True, had_scale=1.0, ld=None, heads=1, seed=0, exact=False):
    """`heads` norm rows of dim form one projection input row (pre_rows): the projection's suh has
    heads * dim entries and the reference rotates the [rows / heads, heads * dim] projection rows.  The
    matrix-core transform runs where the short-row kernel takes rows of 128 (16-bit x, f32 or bf16 gate,
    aligned rows) unless exact."""
    ld = ld or dim
    x = dev_normal((rows, ld), 0, 1, xt, seed)[:, :dim]
    g = dev_normal((rows, ld), 0, 2, gt, seed + 1)[:, :dim]
    w = dev_normal((w_groups * dim,), 1, 0.1, wt, seed + 2) if with_w else None
    p = suh(heads * dim, seed + 3) if pre else None
    y = torch.empty((rows, dim), device="cuda", dtype=torch.float16) if with_y else None
    out = torch.empty((rows, dim), device="cuda", dtype=torch.float16)
    mf = not exact and dim == 128 and xt != F32 and gt in (F32, BF16) and ld % 8 == 0
    ffi.gated_rms_norm_had(x, w, g, out, 1e-6, p, y, cb, w_groups, gate_first, gate_act, had_scale, pre_rows=heads,
                           exact=exact)
    uy = torch.empty((rows, dim), device="cuda", dtype=torch.float16)
    ffi.gated_rms_norm(x, w, uy, g, 1e-6, cb, w_groups, gate_first, gate_act)
    uout = torch.empty_like(out)
    ffi.had_r_128(uy.view(rows // heads, heads * dim), uout.view(rows // heads, heads * dim), p, None, had_scale,
                  mfma=mf)
    torch.cuda.synchronize()
    tag = (f"gated_had {rows}x{dim} x{xt} g{gt} G{w_groups} first{int(gate_first)} act{gate_act} y{int(with_y)} "
           f"{'mfma' if mf else 'exact'}")
    assert_bitwise(from_dev(out), from_dev(uout), what=tag + " vs unfused")
    if with_y:
        assert_bitwise(from_dev(y), from_dev(uy), what=tag + " y vs unfused")
    ey = orc.gated_rms_norm(np.ascontiguousarray(from_dev(x)), xt, np.ascontiguousarray(from_dev(g)), gt, F16,
                            w=from_dev(w) if with_w else None, wt=wt, w_groups=w_groups, eps=1e-6, cb=cb,
                            gate_first=gate_first, gate_act=gate_act, nthreads=NTHREADS)
    assert_close_ulp(from_dev(uy), ey, F16, 1, what=tag + " y vs oracle")
    yin = np.ascontiguousarray(from_dev(uy)).reshape(rows // heads, heads * dim)
    eo = orc.had_r_128(yin, F16, pre=from_dev(p) if p is not None else None, scale=had_scale, nthreads=NTHREADS)
    got = from_dev(out).reshape(rows // heads, heads * dim)
    if mf:
        xin = orc.to_f32(yin, F16).astype(np.float64) * (orc.to_f32(from_dev(p), F16).astype(np.float64)[None, :]
                                                         if p is not None else 1.0)
        assert_had_close(got, eo, xin, 0.0883883461356163 * had_scale, what=tag + " out vs oracle had_r_128(y)")
    else:
        assert_bitwise(got, eo, what=tag + " out vs oracle had_r_128(y)")


@pytest.mark.parametrize("gate_act", [0, 1])
@pytest.mark.parametrize("gate_first", [False, True])
def test_qwen35_gdn_output_into_o_proj(gate_act, gate_first):
    """2048 tokens x 32 value heads of 128: bf16 core, f32 gate, f32 weight, the short-row kernel (its
    matrix-core form; the butterfly with EXL3R_HAD_EXACT for one of the gates)."""
    run(2048 * 32, 128, gate_first=gate_first, gate_act=gate_act, with_y=False, heads=32,
        seed=gate_act + 2 * gate_first)
    if gate_act == 0:
        run(512 * 32, 128, gate_first=gate_first, gate_act=gate_act, with_y=False, heads=32, seed=20 + gate_first,
            exact=True)


@pytest.mark.parametrize("rows", [1, 3, 5, 4 * 16 + 2, 4097])
def test_row_counts_inside_a_span(rows):
    """Row counts that end inside a wave's 4 rows (the rows past the end take part in the MFMAs with
    zeros and store nothing), with y written, bf16 gate and weight, f16 x."""
    run(rows, 128, xt=F16, gt=BF16, wt=BF16, had_scale=-0.75, seed=30 + rows)


@pytest.mark.parametrize("xt,gt,wt", [(F16, BF16, F16), (BF16, BF16, BF16), (F16, F32, F32)])
def test_dtypes_and_row_lengths(xt, gt, wt):
    run(36, 256, xt, gt, wt, heads=4, seed=5)         # short rows, two blocks per row
    run(19, 1024, xt, gt, wt, w_groups=2, seed=6)     # workgroup kernel
    run(7, 384, xt, F16, wt, heads=7, seed=7)         # f16 gate: workgroup kernel


def test_wide_rows():
    """Rows over 32768 columns: 8 chunks on each of 1024 lanes (the instances that spill to scratch)."""
    run(2, 65536, F16, F32, F32, gate_act=1, seed=11)
    run(3, 40960, BF16, BF16, BF16, gate_first=True, seed=12)


def test_bias_scale_missing_pre_and_fallback():
    run(33, 128, cb=1.0, had_scale=0.5, pre=False, seed=8)
    run(9, 256, ld=259, seed=9)                       # unaligned rows: the unfused calls
    run(8, 256, xt=F32, heads=2, seed=10)             # f32 x: the unfused calls


def test_zero_rows_and_errors():
    z = torch.empty((0, 128), device="cuda", dtype=torch.bfloat16)
    ffi.gated_rms_norm_had(z, None, z.float(), torch.empty((0, 128), device="cuda", dtype=torch.float16), 1e-6)
    x = dev_normal((4, 128), 0, 1, BF16, 11)
    g = dev_normal((4, 128), 0, 1, F32, 12)
    with pytest.raises(exl3r.Exl3rError):
        x2 = dev_normal((4, 100), 0, 1, BF16, 13)
        ffi.gated_rms_norm_had(x2, None, g[:, :100], torch.empty((4, 100), device="cuda", dtype=torch.float16), 1e-6)
    with pytest.raises(exl3r.Exl3rError):
        o = torch.empty((4, 128), device="cuda", dtype=torch.float16)
        ffi.gated_rms_norm_had(x, None, g, o, 1e-6, y=o)       # y aliases out
    with pytest.raises(exl3r.Exl3rError):
        ffi.gated_rms_norm_had(x, None, g, torch.empty((4, 128), device="cuda", dtype=torch.float16), 1e-6,
                               gate_act=3)
    with pytest.raises(exl3r.Exl3rError):                       # 4 rows are not whole groups of 3
        ffi.gated_rms_norm_had(x, None, g, torch.empty((4, 128), device="cuda", dtype=torch.float16), 1e-6,
                               pre_rows=3)
    torch.cuda.synchronize()
