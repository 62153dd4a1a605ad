"""Pins the oracle's RMSNorm (plain and RES_IN) against torch-CPU float64 fixtures, closed forms and
invariants; planted mistakes in the oracle must each fail one of these checks."""
import numpy as np
import pytest

from _util import load_cases, round64, ulp_dist
from oracle import oracle as orc


def golden_ok(case):
    x = case["x"].reshape(case["rows"], case["dim"])
    r = case["r"].reshape(x.shape).copy() if "r" in case else None
    y = orc.rms_norm(x, case["xt"], case["w"], case["wt"], case["yt"], case["eps"], case["cb"], case["cs"],
                     r=r, rt=case["rt"] if r is not None else orc.F32)
    exp = round64(case["y64"], case["yt"])
    d = ulp_dist(y, exp, case["yt"])
    if case["yt"] == orc.F32:   # three fp32 roundings (x*w, rmf, *rmf) before the f32 output
        ok = d.max() <= 3
    else:                       # one RNE to a 16-bit format dominates
        ok = d.max() <= 1 and np.mean(d == 0) > 0.99
    if r is not None:
        ok = ok and np.array_equal(r, case["h"])
    return ok


CASES = load_cases("rmsnorm.npz")


@pytest.mark.parametrize("i", range(len(CASES)))
def test_golden(i):
    assert golden_ok(CASES[i])


def closed_form_ok():
    """x = c * ones, w = 1, eps: y = c / sqrt(c^2 + eps) for every element."""
    dim = 256
    cs = np.array([1.0, -3.0, 1e-3, 250.0], np.float32)
    x = np.repeat(cs[:, None], dim, 1).astype(np.float32)
    w = orc.to_bits(np.ones(dim, np.float32), orc.F16)
    y = orc.rms_norm(x, orc.F32, w, orc.F16, orc.F32, 1e-2)
    exp = cs.astype(np.float64) / np.sqrt(cs.astype(np.float64) ** 2 + 1e-2)
    return np.allclose(y, exp[:, None], rtol=3e-7, atol=0)


def test_closed_form():
    assert closed_form_ok()


def test_scale_invariance_eps0():
    rng = np.random.default_rng(4)
    x = rng.standard_normal((8, 384)).astype(np.float32)
    w = orc.to_bits(rng.standard_normal(384).astype(np.float32) * 0.1 + 1, orc.BF16)
    y1 = orc.rms_norm(x, orc.F32, w, orc.BF16, orc.F16, 0.0)
    y2 = orc.rms_norm(x * np.float32(64.0), orc.F32, w, orc.BF16, orc.F16, 0.0)
    assert np.array_equal(y1, y2)


def test_zero_row_and_residual_cancel():
    rng = np.random.default_rng(5)
    x = orc.to_bits(rng.standard_normal((3, 64)).astype(np.float32), orc.F16)
    r = x.copy() ^ np.uint16(0x8000)          # r = -x exactly
    w = orc.to_bits(np.ones(64, np.float32), orc.F16)
    y = orc.rms_norm(x, orc.F16, w, orc.F16, orc.F16, 1e-6, r=r, rt=orc.F16)
    assert np.all(orc.to_f32(y, orc.F16) == 0) and np.all(orc.to_f32(r, orc.F16) == 0)


def res_in_rounding_ok():
    """The residual written back and normalised is round_r(x + r), computed here with numpy."""
    rng = np.random.default_rng(6)
    x = orc.to_bits(rng.standard_normal((4, 128)).astype(np.float32), orc.F16)
    r = orc.to_bits(rng.standard_normal((4, 128)).astype(np.float32) * 4, orc.F16)
    h = (orc.to_f32(x, orc.F16) + orc.to_f32(r, orc.F16)).astype(np.float16).view(np.uint16)
    w = orc.to_bits(np.ones(128, np.float32), orc.F16)
    r2 = r.copy()
    y = orc.rms_norm(x, orc.F16, w, orc.F16, orc.F32, 0.0, r=r2, rt=orc.F16)
    y_plain = orc.rms_norm(h, orc.F16, w, orc.F16, orc.F32, 0.0)
    return np.array_equal(r2, h) and np.array_equal(y, y_plain)


def test_res_in_rounding():
    assert res_in_rounding_ok()


def clamp_ok():
    """f16 x: +-inf -> +-65504, NaN -> 65504 before the norm (CLAMP_FP16)."""
    x = orc.to_bits(np.array([[1.0, np.inf, -np.inf, np.nan, 2.0, 3.0, 4.0, 5.0]], np.float32), orc.F16)
    xc = orc.to_bits(np.array([[1.0, 65504.0, -65504.0, 65504.0, 2.0, 3.0, 4.0, 5.0]], np.float32), orc.F16)
    y = orc.rms_norm(x, orc.F16, None, orc.F16, orc.F32, 1e-6)
    yc = orc.rms_norm(xc, orc.F16, None, orc.F16, orc.F32, 1e-6)
    return np.array_equal(y, yc) and np.all(np.isfinite(y))


def test_f16_clamp():
    assert clamp_ok()


def bias_ok():
    rng = np.random.default_rng(7)
    x = rng.standard_normal((4, 96)).astype(np.float32)
    w = (rng.standard_normal(96) * 0.1).astype(np.float32)
    y1 = orc.rms_norm(x, orc.F32, w, orc.F32, orc.F32, 1e-6, cb=1.0)
    y2 = orc.rms_norm(x, orc.F32, w + np.float32(1.0), orc.F32, orc.F32, 1e-6, cb=0.0)
    return np.array_equal(y1, y2) and not np.array_equal(y1, orc.rms_norm(x, orc.F32, w, orc.F32, orc.F32, 1e-6))


def test_constant_bias():
    assert bias_ok()


def test_constant_scale_power_of_two():
    rng = np.random.default_rng(8)
    x = orc.to_bits(rng.standard_normal((4, 200)).astype(np.float32), orc.BF16)
    w = orc.to_bits(rng.standard_normal(200).astype(np.float32) * 0.1 + 1, orc.BF16)
    y1 = orc.to_f32(orc.rms_norm(x, orc.BF16, w, orc.BF16, orc.BF16, 1e-6, cs=1.0), orc.BF16)
    y2 = orc.to_f32(orc.rms_norm(x, orc.BF16, w, orc.BF16, orc.BF16, 1e-6, cs=0.25), orc.BF16)
    assert np.array_equal(y1 * np.float32(0.25), y2)


@pytest.mark.parametrize("mutation", [1, 2, 3, 4, 5])
def test_planted_mistakes_are_caught(mutation):
    """Each planted mistake fails at least one of the pins above."""
    orc.set_mutation(mutation)
    results = [all(golden_ok(c) for c in CASES), closed_form_ok(), res_in_rounding_ok(), clamp_ok(), bias_ok()]
    assert not all(results), f"mutation {mutation} not caught"
