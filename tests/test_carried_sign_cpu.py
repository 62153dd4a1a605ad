"""CPU model of the carried-sign Hadamard butterfly (hadamard.cuh butterfly128_t<true>) against the exact
butterfly, in numpy float32: the 128-point block as 16 lanes x 8 slots, in-lane stages over index bits
0..2, then the lane stages xor 1, 2, 4, 8 where every lane keeps v + c * partner (c = -1 in the upper
lane, one rounding), and the final scale fma(v, (-1)^popcount(lane) r, +0).  It pins the argument the
kernels rely on: the result equals the exact butterfly bit for bit -- signed zeros, infinities and NaN
positions included -- whenever no lane holds 8 zero inputs with a -0 among them (and r > 0); and the
model shows the exception that makes the kernels take the exact stages for such waves.  The GPU tests
check the kernels themselves against the oracle; this checks the reasoning on inputs chosen to break
it (cancellations to exact zero, signed zeros, infinities, NaN, overflow)."""
import numpy as np

R = np.float32(0.0883883461356163)


def exact(x, r=R):
    f = x.astype(np.float32).copy()
    h = 1
    while h < 128:
        idx = np.arange(128)
        lo = idx[(idx & h) == 0]
        a, b = f[lo].copy(), f[lo | h].copy()
        f[lo], f[lo | h] = a + b, a - b
        h <<= 1
    return f * np.float32(r)


def fma_zero(v, s):
    """fma(v, s, +0) in fp32: the exact product (double holds it) plus +0, rounded once."""
    p = v.astype(np.float64) * s.astype(np.float64)
    return (p + 0.0).astype(np.float32)


def carried(x, r=R):
    f = x.astype(np.float32).reshape(16, 8).copy()       # [lane, slot]
    for h in (1, 2, 4):
        j = np.arange(8)
        lo = j[(j & h) == 0]
        a, b = f[:, lo].copy(), f[:, lo | h].copy()
        f[:, lo], f[:, lo | h] = a + b, a - b
    lanes = np.arange(16)
    for m in (1, 2, 4, 8):
        c = np.where(lanes & m, np.float32(-1), np.float32(1))[:, None]
        f = (f.astype(np.float64) + f[lanes ^ m].astype(np.float64) * c).astype(np.float32)
    sign = np.array([(-1) ** bin(l).count("1") for l in lanes], np.float32)[:, None]
    return fma_zero(f, np.broadcast_to(sign * np.float32(r), f.shape)).reshape(128)


def zero_lane(x):
    bits = x.astype(np.float32).reshape(16, 8).view(np.uint32)
    return bool((np.bitwise_or.reduce(bits, axis=1) == 0x80000000).any())


def same(a, b):
    na, nb = np.isnan(a), np.isnan(b)
    return np.array_equal(na, nb) and np.array_equal(a.view(np.uint32)[~na], b.view(np.uint32)[~nb])


def blocks(rng, n):
    for t in range(n):
        kind = t % 8
        x = rng.standard_normal(128).astype(np.float16).astype(np.float32)
        if kind == 1:
            x[rng.random(128) < 0.4] = 0.0                       # +0 inputs
        elif kind == 2:
            x = rng.integers(-2, 3, 128).astype(np.float32)       # cancellations to exact zero
        elif kind == 3:
            x = np.repeat(rng.integers(-1, 2, 16).astype(np.float32), 8)
        elif kind == 4:
            x[rng.integers(0, 128, 3)] = np.inf
            x[rng.integers(0, 128, 2)] = -np.inf
        elif kind == 5:
            x[rng.integers(0, 128, 2)] = np.nan
        elif kind == 6:
            x *= np.float32(3e37)                                 # overflow inside the butterfly
        elif kind == 7:
            x = rng.integers(-1, 2, 128).astype(np.float32)
            x[x == 0] = -0.0                                      # -0 inputs mixed with non-zeros
        yield x


def test_carried_equals_exact_unless_a_lane_is_zero_with_a_negative_zero():
    rng = np.random.default_rng(2024)
    checked = 0
    with np.errstate(all="ignore"):
        for x in blocks(rng, 4000):
            if zero_lane(x):
                continue
            assert same(carried(x), exact(x)), x
            checked += 1
    assert checked > 3500


def test_all_zero_blocks():
    """A block of +0 gives +0 everywhere either way; a block with -0 inputs gives -0 at some outputs
    in the exact butterfly, which the carried stages cannot reproduce -- the case the wave's ballot
    (a lane of 8 zeros with a -0) sends to the exact stages."""
    z = np.zeros(128, np.float32)
    assert same(carried(z), exact(z)) and not zero_lane(z)
    nz = np.full(128, -0.0, np.float32)
    assert zero_lane(nz)
    e = exact(nz)
    assert (e.view(np.uint32) == 0x80000000).any()               # the reference keeps some -0
    assert not same(carried(nz), e)


def test_a_negative_zero_among_nonzeros_changes_nothing():
    """-0 inputs in lanes that also hold non-zero values: no result depends only on zeros, so every
    zero result is +0 and the carried stages stay exact (no ballot hit for these blocks)."""
    rng = np.random.default_rng(7)
    with np.errstate(all="ignore"):
        for _ in range(500):
            x = rng.integers(-1, 2, 128).astype(np.float32)
            x[rng.random(128) < 0.3] = -0.0
            lanes = x.reshape(16, 8)
            lanes[(lanes == 0).all(axis=1), 0] = 1.0               # no all-zero lane
            assert not zero_lane(x)
            assert same(carried(x), exact(x))


def test_scale_sign_is_folded_exactly():
    """fma(v, +-r, +0) rounds every non-zero product as r * v does (underflow to a signed zero
    included), and gives +0 for a zero v of either sign."""
    rng = np.random.default_rng(11)
    v = (rng.standard_normal(20000) * np.exp2(rng.integers(-160, 120, 20000))).astype(np.float32)
    v[:50] = 0.0
    v[50:100] = -0.0
    for s in (R, -R):
        got = fma_zero(v, np.full_like(v, s))
        want = (v.astype(np.float64) * np.float64(s)).astype(np.float32)
        nz = v != 0
        assert np.array_equal(got[nz].view(np.uint32), want[nz].view(np.uint32))
        assert (got[~nz].view(np.uint32) == 0).all()
