"""Pins the oracle's random-Hadamard row transform (had_r_128, kernels/quant/hadamard.cu:88-170 and
hadamard_inner.cuh:96-200) against an independent construction: scipy.linalg.hadamard's Sylvester
matrix applied in float64.  Also: a unit vector gives exactly +-fl32(1/sqrt(128)) (one nonzero
term, no rounding); the transform is its own inverse; blocks are independent; the f16 pre-scale
product is rounded to half before the transform, as __hmul2 rounds it; the post scale applies after
the rounded transform.  Planted mistakes (pre-scale not rounded, a sign flipped in the last
butterfly stage) fail."""
import numpy as np
import pytest
from scipy.linalg import hadamard

from oracle import oracle as orc

F16, F32 = orc.F16, orc.F32
ORM_HAD_NO_PRE_ROUND, ORM_HAD_SIGN = 27, 28
H = hadamard(128).astype(np.float64)
R = float(np.float32(1.0 / np.sqrt(128.0)))


def exact(x64, pre=None):
    rows, cols = x64.shape
    blocks = x64.reshape(rows, cols // 128, 128)
    if pre is not None:
        blocks = blocks * pre.reshape(cols // 128, 128)
    return (blocks @ H.T * R).reshape(rows, cols)


@pytest.fixture
def mutation():
    yield lambda m: orc.set_mutation(m)
    orc.set_mutation(0)


def test_f32_against_sylvester_matrix():
    rng = np.random.default_rng(0)
    x = (rng.standard_normal((37, 512)) * 3).astype(np.float32)
    got = orc.had_r_128(x, F32).astype(np.float64)
    ex = exact(x.astype(np.float64))
    # seven fp32 butterfly levels: error below 8 ulps of the largest partial sum
    assert np.max(np.abs(got - ex)) <= 8 * 2.0 ** -24 * np.max(np.abs(x)) * 128 * R


def test_f16_against_sylvester_matrix_with_pre_scale():
    rng = np.random.default_rng(1)
    x = (rng.standard_normal((29, 1024))).astype(np.float16)
    suh = np.where(rng.random(1024) < 0.5, -1.0, 1.0) * (1 + 0.01 * rng.standard_normal(1024))
    pre = suh.astype(np.float16)
    got = orc.had_r_128(x.view(np.uint16), F16, pre=pre.view(np.uint16)).view(np.float16).astype(np.float64)
    xs = (x * pre).astype(np.float64)                                    # numpy's half multiply rounds once
    ex = exact(xs)
    ulp = np.spacing(np.abs(ex).astype(np.float16)).astype(np.float64)
    assert np.all(np.abs(got - ex) <= ulp * 1.0 + 2.0 ** -24)              # within one half ulp step


def test_unit_vectors_exact_and_blocks_independent():
    x = np.zeros((128, 256), np.float32)
    x[np.arange(128), np.arange(128)] = 1.0
    got = orc.had_r_128(x, F32)
    assert np.array_equal(got[:, :128], (H[:, np.arange(128)].T * R).astype(np.float32))
    assert not got[:, 128:].any()


def test_signed_zeros_follow_the_butterfly():
    """IEEE rules fix the sign of an exact zero: (-0) + (-0) = -0 and every difference of equal zeros
    is +0.  An all -0 block therefore gives -0 only at output 0 (the all-plus row of H, reached by
    additions alone) and +0 elsewhere; an all +0 block gives +0 everywhere."""
    x = np.zeros((2, 256), np.float16)
    x[1] = -0.0
    o = orc.had_r_128(x.view(np.uint16), F16).view(np.float16)
    assert not np.signbit(o[0]).any()
    assert np.array_equal(np.nonzero(np.signbit(o[1]))[0], [0, 128])
    assert not o.any()


def test_involution():
    x = np.random.default_rng(2).standard_normal((8, 384)).astype(np.float32)
    back = orc.had_r_128(orc.had_r_128(x, F32), F32)
    assert np.max(np.abs(back - x)) < 1e-5


def test_post_scale_and_scalar_scale():
    rng = np.random.default_rng(3)
    x = rng.standard_normal((5, 256)).astype(np.float16)
    svh = (1 + 0.05 * rng.standard_normal(256)).astype(np.float16)
    plain = orc.had_r_128(x.view(np.uint16), F16).view(np.float16)
    post = orc.had_r_128(x.view(np.uint16), F16, post=svh.view(np.uint16)).view(np.float16)
    assert np.array_equal(post, (plain * svh).astype(np.float16))
    halved = orc.had_r_128(x.view(np.uint16), F16, scale=0.5).view(np.float16)
    assert np.array_equal(halved, (plain.astype(np.float32) * 0.5).astype(np.float16))   # power of two: exact


def test_pre_and_post_together_rejected():
    x = np.zeros((1, 128), np.float32)
    with pytest.raises(ValueError):
        orc.had_r_128(x, F32, pre=np.zeros(128, np.uint16), post=np.zeros(128, np.uint16))


def test_mutations_caught(mutation):
    rng = np.random.default_rng(4)
    x = rng.standard_normal((16, 256)).astype(np.float16)
    pre = (1 + 0.3 * rng.standard_normal(256)).astype(np.float16)
    ref = orc.had_r_128(x.view(np.uint16), F16, pre=pre.view(np.uint16))
    mutation(ORM_HAD_NO_PRE_ROUND)
    assert not np.array_equal(orc.had_r_128(x.view(np.uint16), F16, pre=pre.view(np.uint16)), ref)
    mutation(ORM_HAD_SIGN)
    xf = rng.standard_normal((4, 128)).astype(np.float32)
    assert np.max(np.abs(orc.had_r_128(xf, F32).astype(np.float64) - exact(xf.astype(np.float64)))) > 0.1
