"""Pins the oracle's RNE conversions: exhaustively against numpy's binary16 and by brute force
against torch's bfloat16 rounding, including every tie."""
import numpy as np
import pytest
import torch

from oracle import oracle as orc


def test_f16_to_f32_exhaustive():
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    ref = bits.view(np.float16).astype(np.float32)
    lib = orc.load()
    got = np.array([lib.oracle_f16_to_f32(int(b)) for b in bits], np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), ref[~nan].view(np.uint32))


def _f16_probe_values():
    """Every finite f16, the midpoints between neighbours (ties) and points just off them,
    overflow boundaries, specials."""
    h = np.arange(0, 0x7C00, dtype=np.uint16).view(np.float16).astype(np.float64)
    mids = (h[:-1] + h[1:]) / 2.0
    off = np.concatenate([np.nextafter(mids.astype(np.float32), np.float32(np.inf)),
                          np.nextafter(mids.astype(np.float32), np.float32(-np.inf))]).astype(np.float64)
    extra = np.array([65504.0, 65519.0, 65519.99, 65520.0, 65536.0, 1e10, 2.0 ** -25, 2.0 ** -24, 3 * 2.0 ** -26,
                      2.0 ** -26, 1e-30, 0.0])
    v = np.concatenate([h, mids, off, extra]).astype(np.float32)
    return np.concatenate([v, -v, np.array([np.inf, -np.inf, np.nan], np.float32)])


def test_f32_to_f16_matches_numpy():
    v = _f16_probe_values()
    got = orc.f32_to_f16_bits(v)
    ref = v.astype(np.float16).view(np.uint16)
    nan = np.isnan(v)
    assert np.array_equal(got[~nan], ref[~nan])
    assert np.all((got[nan] & 0x7C00) == 0x7C00) and np.all(got[nan] & 0x3FF)


def test_f32_to_f16_random():
    rng = np.random.default_rng(1)
    u = rng.integers(0, 2 ** 32, 2_000_000, dtype=np.uint64).astype(np.uint32)
    v = u.view(np.float32)
    v = v[~np.isnan(v)]
    assert np.array_equal(orc.f32_to_f16_bits(v), v.astype(np.float16).view(np.uint16))


def test_f32_to_bf16_matches_torch():
    rng = np.random.default_rng(2)
    u = rng.integers(0, 2 ** 32, 2_000_000, dtype=np.uint64).astype(np.uint32)
    # exact ties and neighbours of ties
    ties = (rng.integers(0, 2 ** 16, 100_000, dtype=np.uint64).astype(np.uint32) << 16) | 0x8000
    u = np.concatenate([u, ties, ties + 1, ties - 1])
    v = u.view(np.float32)
    keep = ~np.isnan(v)
    ref = torch.from_numpy(v[keep].copy()).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(orc.f32_to_bf16_bits(v[keep]), ref)
    nanbits = orc.f32_to_bf16_bits(v[~keep])
    assert np.all(np.isnan(orc.to_f32(nanbits, orc.BF16)))


def test_bf16_to_f32_exhaustive():
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    ref = torch.from_numpy(bits.view(np.int16).copy()).view(torch.bfloat16).float().numpy()
    got = orc.to_f32(bits, orc.BF16)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), ref[~nan].view(np.uint32))


@pytest.mark.parametrize("code", [orc.F16, orc.BF16])
def test_round_f64_agrees_with_f32_path(code):
    """oracle_round(double) == the bitwise f32 conversion for values exact in f32, and rounds
    double ties the IEEE way."""
    rng = np.random.default_rng(3)
    v = (rng.standard_normal(20000) * 10.0 ** rng.integers(-6, 5, 20000)).astype(np.float32)
    lib = orc.load()
    r = np.array([lib.oracle_round(float(t), code) for t in v], np.float64).astype(np.float32)
    assert np.array_equal(orc.to_bits(r, code), orc.to_bits(v, code))
    # 1 + 2^-11 is the f16 tie between 1 and 1 + 2^-10 (even: 1); 1 + 2^-11 + 2^-40 rounds up.
    assert lib.oracle_round(1.0 + 2.0 ** -11, orc.F16) == 1.0
    assert lib.oracle_round(1.0 + 2.0 ** -11 + 2.0 ** -40, orc.F16) == 1.0 + 2.0 ** -10
    assert lib.oracle_round(65519.999, orc.F16) == 65504.0
    assert np.isinf(lib.oracle_round(65520.0, orc.F16))
