"""The oracle's row argmax (the generator's batched argmax, src/generator.rs:1596, and
exl3_shim_argmax_sample, kernels/generator/sampling_basic.cu:65-172) pinned against numpy.argmax, an
independent implementation of the same rule (first maximal index; NaN is maximal), on random rows,
ties, signed zeros, infinities, NaNs and the max_logit mask, plus planted mistakes."""
import numpy as np
import pytest

from oracle import oracle as orc

F32, F16, BF16 = orc.F32, orc.F16, orc.BF16
ORM_ARGMAX_LAST_TIE, ORM_ARGMAX_NO_MASK = 21, 22


def ref(x, max_logit=0):
    n = x.shape[1] if max_logit <= 0 or max_logit > x.shape[1] else max_logit
    return np.argmax(x[:, :n], axis=1)


@pytest.mark.parametrize("dt", [F16, BF16, F32])
def test_random_rows_match_numpy(dt):
    rng = np.random.default_rng(1)
    x = orc.to_bits((rng.standard_normal((33, 1000)) * 4).astype(np.float32), dt)
    xf = orc.to_f32(x, dt)
    assert np.array_equal(orc.argmax(x, dt), ref(xf))
    for m in (1, 2, 499, 999, 1000, 5000):
        assert np.array_equal(orc.argmax(x, dt, m), ref(xf, m))


def test_ties_zeros_infinities_nans():
    rows = np.array([[1.0, 3.0, 3.0, 2.0],            # tie -> first
                     [-0.0, 0.0, -1.0, -0.0],         # -0 == +0 -> index 0
                     [-np.inf, -np.inf, -np.inf, -np.inf],
                     [1.0, np.inf, 5.0, np.inf],
                     [1.0, np.nan, 9.0, np.nan],      # first NaN wins
                     [np.nan, 1.0, 2.0, 3.0],
                     [7.0, 7.0, 7.0, 7.0]], np.float32)
    assert np.array_equal(orc.argmax(rows, F32), np.argmax(rows, axis=1))
    assert list(orc.argmax(rows, F32)) == [1, 0, 0, 1, 1, 0, 0]


@pytest.mark.parametrize("mutation", [ORM_ARGMAX_LAST_TIE, ORM_ARGMAX_NO_MASK])
def test_planted_mistakes_are_caught(mutation):
    x = np.array([[1.0, 3.0, 3.0, 2.0, 9.0]], np.float32)
    clean = orc.argmax(x, F32, 4)
    orc.set_mutation(mutation)
    try:
        bad = orc.argmax(x, F32, 4)
    finally:
        orc.set_mutation(0)
    assert not np.array_equal(clean, bad)
