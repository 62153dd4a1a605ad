"""The oracle's Gumbel-max sampler (the role of exl3_shim_gumbel_sample / exl3_shim_gumbel_noise_f32,
kernels/generator/sampling_basic.cu:94-128 and gumbel.cu:45-62), pinned piece by piece:

- Philox4x32-10 against the known-answer vectors published with the Random123 library
  (Salmon et al., SC 2011);
- the fp32 log against float64 numpy.log on a sweep of normal floats;
- the transform -log(-log(u)) exhaustively over all 2^23 uniforms the stream can produce;
- the noise's distribution (Gumbel(0, 1): mean = Euler's gamma, variance = pi^2/6, CDF
  exp(-exp(-g))) and the independence of rows and columns;
- the Gumbel-max theorem: draws over identical rows follow softmax(logits);
- sample == argmax of (logits + noise) over the masked prefix;
plus planted mistakes that each of these must catch.

The reference draws its uniforms from cuRAND; that stream is not reproduced (its draws are parity
unpinned against the reference by design; the distribution is what both share)."""
import math

import numpy as np
import pytest

from oracle import oracle as orc

F32, F16, BF16 = orc.F32, orc.F16, orc.BF16
ORM_PHILOX_NO_BUMP, ORM_LOG_NO_LN2LO, ORM_GUMBEL_NO_ROW = 23, 24, 25
EULER_GAMMA = 0.5772156649015329

# Random123 kat_vectors, philox4x32 with 10 rounds: counter, key -> output
KAT = [
    ([0, 0, 0, 0], [0, 0], [0x6627E8D5, 0xE169C58D, 0xBC57AC4C, 0x9B00DBD8]),
    ([0xFFFFFFFF] * 4, [0xFFFFFFFF] * 2, [0x408F276D, 0x41C83B0E, 0xA20BC7C6, 0x6D5451FD]),
    ([0x243F6A88, 0x85A308D3, 0x13198A2E, 0x03707344], [0xA4093822, 0x299F31D0],
     [0xD16CFE09, 0x94FDCCEB, 0x5001E420, 0x24126EA1]),
]


@pytest.fixture
def mutation():
    yield lambda m: orc.set_mutation(m)
    orc.set_mutation(0)


def test_philox_known_answers():
    for ctr, key, out in KAT:
        assert list(orc.philox4x32_10(ctr, key)) == out


def test_philox_mutation_caught(mutation):
    mutation(ORM_PHILOX_NO_BUMP)
    assert list(orc.philox4x32_10(*KAT[0][:2])) != KAT[0][2]


def ulps(got, exact):
    return np.abs(got.astype(np.float64) - exact) / np.spacing(np.abs(exact).astype(np.float32)).astype(np.float64)


def test_log_f32_accuracy():
    rng = np.random.default_rng(3)
    xs = rng.integers(0x00800000, 0x7F800000, 60000, dtype=np.uint32).view(np.float32)
    xs = np.concatenate([xs, np.float32([1.0, 2.0, 0.5, 0.70710677, 0.7071068, 1.4142135, 1.4142137,
                                         5.9604645e-08, 0.99999994, 16.635532])])
    got = np.array([orc.log_f32(x) for x in xs], np.float32)
    exact = np.log(xs.astype(np.float64))
    nz = exact != 0
    assert ulps(got[nz], exact[nz]).max() <= 1.0
    assert orc.log_f32(1.0) == 0.0


def exhaustive_transform():
    k = np.arange(1 << 23, dtype=np.uint32)
    g = orc.gumbel_of_bits(k << 9).astype(np.float64)
    u = (k.astype(np.float64) + 0.5) * 2.0 ** -23
    return g, -np.log(-np.log(u))


def test_gumbel_transform_exhaustive():
    # Every uniform the stream can produce: u = (k + 0.5) 2^-23, k < 2^23.  Bound: 1.5 ulp of g, or
    # 1.2e-7 absolute (one ulp of 1.0) near g = 0, where -log(u) ~ 1 has been rounded to fp32.
    g, exact = exhaustive_transform()
    tol = np.maximum(1.5 * np.spacing(np.abs(exact).astype(np.float32)).astype(np.float64), 1.2e-7)
    assert np.all(np.abs(g - exact) <= tol)
    assert g.min() > -2.82 and g.max() < 16.64            # u never reaches 0 or 1: g is always finite
    # the 9 low bits of the Philox word are not used
    assert orc.gumbel_of_bits(np.uint32([0x12345600]))[0] == orc.gumbel_of_bits(np.uint32([0x123457FF]))[0]


def test_log_mutation_caught(mutation):
    mutation(ORM_LOG_NO_LN2LO)
    g, exact = exhaustive_transform()
    tol = np.maximum(1.5 * np.spacing(np.abs(exact).astype(np.float32)).astype(np.float64), 1.2e-7)
    assert not np.all(np.abs(g - exact) <= tol)


def test_stream_layout():
    """Noise depends on (seed, row, column) only: the element (r, c) is word c & 3 of the Philox
    block at counter (c >> 2, r, 0, 0), key (seed, 0)."""
    zeros = np.zeros((7, 37), np.float32)
    n7 = orc.gumbel_noise(zeros, F32, 1234)
    n3 = orc.gumbel_noise(zeros[:3], F32, 1234)
    assert np.array_equal(n7[:3], n3)
    for r, c in [(0, 0), (2, 5), (6, 36), (5, 11)]:
        bits = orc.philox4x32_10([c >> 2, r, 0, 0], [1234, 0])
        assert n7[r, c] == orc.gumbel_of_bits(bits[c & 3:(c & 3) + 1])[0]
    assert not np.any(n7 == orc.gumbel_noise(zeros, F32, 1235))
    assert len(np.unique(n7)) == n7.size


def test_noise_distribution():
    rows, cols = 1000, 4096
    g = orc.gumbel_noise(np.zeros((rows, cols), np.float32), F32, 7, nthreads=8).astype(np.float64)
    n = g.size
    var = math.pi ** 2 / 6
    assert abs(g.mean() - EULER_GAMMA) < 5 * math.sqrt(var / n)
    assert abs(g.var() - var) < 0.005 * var
    s = np.sort(g.ravel())
    cdf = np.exp(-np.exp(-s))
    ks = max(np.max(np.arange(1, n + 1) / n - cdf), np.max(cdf - np.arange(n) / n))
    assert ks < 1.63 / math.sqrt(n)                          # Kolmogorov-Smirnov at the 1% level
    for a, b in [(g[:, :-1], g[:, 1:]), (g[:, :-4], g[:, 4:]), (g[:-1], g[1:])]:
        assert abs(np.corrcoef(a.ravel(), b.ravel())[0, 1]) < 5 / math.sqrt(a.size)


def chi2_of_draws(logits, ids):
    p = np.exp(logits - logits.max())
    p /= p.sum()
    counts = np.bincount(ids, minlength=len(logits)).astype(np.float64)
    live = p > 0
    assert counts[~live].sum() == 0
    e = p[live] * len(ids)
    return float(((counts[live] - e) ** 2 / e).sum()), int(live.sum() - 1)


def test_gumbel_max_follows_softmax():
    logits = np.float32([0.0, 1.0, 2.0, -1.0, 0.5, 3.0, -np.inf, 2.0, -4.0])
    rows = 200000
    ids = orc.gumbel_sample(np.tile(logits, (rows, 1)), F32, 99, nthreads=8)
    chi2, dof = chi2_of_draws(logits, ids)
    assert chi2 < dof + 6 * math.sqrt(2 * dof), chi2          # ~ p < 1e-6 under the null


def test_row_mutation_caught(mutation):
    mutation(ORM_GUMBEL_NO_ROW)
    logits = np.float32([0.0, 1.0, 2.0, -1.0])
    ids = orc.gumbel_sample(np.tile(logits, (20000, 1)), F32, 99, nthreads=8)
    chi2, dof = chi2_of_draws(logits, ids)
    assert chi2 > dof + 6 * math.sqrt(2 * dof)


@pytest.mark.parametrize("dt", [F16, BF16, F32])
def test_sample_is_argmax_of_noise(dt):
    rng = np.random.default_rng(11)
    x = (rng.standard_normal((40, 3001)) * 3).astype(np.float32)
    x[3, 100] = np.inf
    x[4, :] = -np.inf
    x[5, 77] = np.nan
    x[6, [10, 2000]] = 60.0
    xb = orc.to_bits(x, dt)
    noisy = orc.gumbel_noise(xb, dt, 5)
    for m in (0, 1, 2, 1500, 3001, 9999):
        ids = orc.gumbel_sample(xb, dt, 5, m)
        assert np.array_equal(ids, orc.argmax(noisy, F32, m))
        if 0 < m < 3001:
            assert ids.max() < m
    assert orc.gumbel_sample(xb, dt, 5)[3] == 100 and orc.gumbel_sample(xb, dt, 5)[5] == 77


def test_noise_output_dtypes():
    rng = np.random.default_rng(12)
    x = orc.to_bits((rng.standard_normal((5, 64)) * 3).astype(np.float32), F16)
    f32 = orc.gumbel_noise(x, F16, 21)
    for dt in (F16, BF16):
        assert np.array_equal(orc.gumbel_noise(x, F16, 21, out_dt=dt), orc.to_bits(f32, dt))
