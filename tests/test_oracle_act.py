"""Pins the oracle's gated activations against 60-digit mpmath fixtures (cross-checked with torch's
float64 F.silu / F.gelu where they do not cancel), closed forms, the odd-part identity
act(x) - act(-x) = x, special values and the act_limit / f16 clamps."""
import numpy as np
import pytest

from _util import load_cases, round64, ulp_dist
from oracle import oracle as orc

CASES = load_cases("act.npz")


def golden_ok(case):
    x = case["x"].reshape(case["rows"], case["cols"])
    y = case["y"].reshape(x.shape)
    z = orc.act_mul(case["act"], x, y, case["it"], case["zt"], case["limit"])
    exp = round64(case["z64"], case["zt"])
    d = ulp_dist(z, exp, case["zt"])
    if case["zt"] == orc.F32:
        return d.max() <= 4
    return d.max() <= 1 and np.mean(d == 0) > 0.98


@pytest.mark.parametrize("i", range(len(CASES)))
def test_golden(i):
    assert golden_ok(CASES[i])


@pytest.mark.parametrize("i", range(len(CASES)))
def test_fixture_agrees_with_torch_where_torch_is_accurate(i):
    c = CASES[i]
    xf = orc.to_f32(c["x"], c["it"]).reshape(c["rows"], c["cols"])
    m = np.abs(xf) <= 4
    assert np.allclose(c["z64"][m], c["z_torch64"][m], rtol=1e-9, atol=1e-300)


def odd_identity_ok(act):
    """act(x) - act(-x) == x for silu and tanh-gelu (their even parts cancel)."""
    x = np.linspace(-12, 12, 2001, dtype=np.float32)[None, :]
    one = np.ones_like(x)
    zp = orc.act_mul(act, x, one, orc.F32, orc.F32)
    zn = orc.act_mul(act, -x, one, orc.F32, orc.F32)
    return np.allclose(zp.astype(np.float64) - zn, x, rtol=0, atol=4e-6 * np.maximum(1, np.abs(x)))


@pytest.mark.parametrize("act", [orc.ACT_SILU, orc.ACT_GELU])
def test_odd_identity(act):
    assert odd_identity_ok(act)


def special_values_ok(act):
    x = np.array([[0.0, -0.0, 60.0, -60.0, 1.0, 2.0]], np.float32)
    y = np.array([[5.0, 5.0, 3.0, 3.0, 0.0, 1.0]], np.float32)
    z = orc.act_mul(act, x, y, orc.F32, orc.F32)[0]
    silu2 = 2.0 / (1.0 + np.exp(-2.0))
    c = np.sqrt(2 / np.pi) * (2.0 + 0.044715 * 8.0)
    gelu2 = 2.0 * 0.5 * (1.0 + np.tanh(c))
    neg60 = -60.0 * 3.0 / (1.0 + np.exp(60.0)) if act == orc.ACT_SILU else 0.0   # gelu(-60) underflows
    ok = z[0] == 0 and z[1] == 0 and z[2] == 180.0 and np.isclose(z[3], neg60, rtol=1e-6, atol=0) and z[4] == 0
    ok = ok and abs(z[5] - (silu2 if act == orc.ACT_SILU else gelu2)) <= 2e-7 * 2
    return bool(ok)


@pytest.mark.parametrize("act", [orc.ACT_SILU, orc.ACT_GELU])
def test_special_values(act):
    assert special_values_ok(act)


def limit_ok():
    """act_limit L: y clamped to [-L, L], act(x) clamped from above (x = 10 -> silu ~ 10 -> L)."""
    x = np.array([[10.0, 10.0, -10.0, 1.0]], np.float32)
    y = np.array([[1.0, -100.0, 100.0, 100.0]], np.float32)
    z = orc.act_mul(orc.ACT_SILU, x, y, orc.F32, orc.F32, limit=3.0)[0]
    s1 = np.float32(1.0 / (1.0 + np.exp(-1.0)))
    s_10 = np.float32(-10.0 / (1.0 + np.exp(10.0)))
    return bool(z[0] == 3.0 and z[1] == -9.0 and np.isclose(z[2], s_10 * 3.0, rtol=1e-6) and np.isclose(z[3], s1 * 3.0, rtol=1e-6))


def test_limit():
    assert limit_ok()


def test_f16_output_clamp():
    x = np.array([[300.0, 300.0, np.nan, -300.0]], np.float32)
    y = np.array([[300.0, -300.0, 1.0, 1.0]], np.float32)
    z = orc.to_f32(orc.act_mul(orc.ACT_SILU, x, y, orc.F32, orc.F16), orc.F16)[0]
    assert z[0] == 65504.0 and z[1] == -65504.0 and z[2] == 65504.0 and z[3] == 0.0


@pytest.mark.parametrize("mutation", [6, 7, 8])
def test_planted_mistakes_are_caught(mutation):
    orc.set_mutation(mutation)
    results = [all(golden_ok(c) for c in CASES), odd_identity_ok(orc.ACT_SILU), odd_identity_ok(orc.ACT_GELU),
               special_values_ok(orc.ACT_SILU), special_values_ok(orc.ACT_GELU), limit_ok()]
    assert not all(results), f"mutation {mutation} not caught"
