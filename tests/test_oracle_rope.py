"""Pins the oracle's head-norm + rotary embedding: float64 fixtures (torch F.rms_norm + half ops for
the norm, a complex product for the rotation), and the invariants a rotation must satisfy -- pos 0 is
the identity, pair norms are preserved, NeoX is GPT-J conjugated by the half/interleave permutation,
dimensions past rotary_dim pass through, and the three position sources agree."""
import numpy as np
import pytest

from _util import load_cases, round64, ulp_dist
from oracle import oracle as orc

CASES = load_cases("rope.npz")


def spacing(v, code):
    """ulp of the 16-bit format at |v|."""
    mant = 11 if code == orc.F16 else 8
    emin = -14 if code == orc.F16 else -126
    e = np.floor(np.log2(np.maximum(np.abs(v), 2.0 ** emin)))
    return 2.0 ** (np.maximum(e, emin) - (mant - 1))


def pair_magnitude(out64, R, mode):
    """sqrt(r1^2 + r2^2) of each element's rotation pair (the element itself past R)."""
    mag = np.abs(out64).copy()
    t = np.arange(R // 2)
    i1 = t if mode == orc.ROPE_NEOX else 2 * t
    i2 = t + R // 2 if mode == orc.ROPE_NEOX else 2 * t + 1
    m = np.hypot(out64[..., i1], out64[..., i2])
    mag[..., i1] = m
    mag[..., i2] = m
    return mag


def run_case(c, position=None):
    pos = c["position"] if position is None else position
    nw = c["nwt"] if c["nwt"] >= 0 else orc.F16
    return orc.rope(c["q"], c["k"], c["dt"], c["inv_freq"], c["mode"], position=pos,
                    positions=c.get("positions"), position_ids=c.get("position_ids"),
                    q_norm=c.get("q_norm"), k_norm=c.get("k_norm"), nwt=nw, eps=c["eps"], cb=c["cb"],
                    attn=c["attn"])


def golden_ok(c):
    oq, ok_ = run_case(c)
    good = True
    for out, key in ((oq, "q64"), (ok_, "k64")):
        exp64 = c[key]
        exp = round64(exp64, c["dt"])
        d = ulp_dist(out, exp, c["dt"])
        err = np.abs(orc.to_f32(out, c["dt"]).astype(np.float64) - exp64)
        bound = 2 * spacing(pair_magnitude(exp64, c["R"], c["mode"]), c["dt"])
        good = good and bool(np.all(err <= bound)) and np.mean(d <= 1) > 0.99
    return good


def headnorm_ok(c):
    """With the rotation at position 0 (identity) the output is the normed head itself."""
    if c["nwt"] < 0:
        return True
    z = dict(c)
    z.pop("positions", None)
    z.pop("position_ids", None)
    z["position"] = 0
    z["attn"] = 1.0
    z["q"] = c["q"][:, :1].copy()
    z["k"] = c["k"][:, :1].copy()
    oq, ok_ = run_case(z)
    good = True
    for out, key in ((oq, "qn"), (ok_, "kn")):
        d = ulp_dist(out, c[key][:, :1], c["dt"])
        good = good and d.max() <= 1 and np.mean(d == 0) > 0.99
    return good


@pytest.mark.parametrize("i", range(len(CASES)))
def test_golden(i):
    assert golden_ok(CASES[i])


@pytest.mark.parametrize("i", range(len(CASES)))
def test_golden_head_norm(i):
    assert headnorm_ok(CASES[i])


def _inputs(rng, bsz, seq, hq, hk, hd, dt):
    q = orc.to_bits(rng.standard_normal((bsz, seq, hq, hd)).astype(np.float32), dt)
    k = orc.to_bits(rng.standard_normal((bsz, seq, hk, hd)).astype(np.float32), dt)
    return q, k


def _inv_freq(R, theta=1e6):
    return (1.0 / theta ** (np.arange(0, R, 2) / R)).astype(np.float32)


def identity_ok():
    rng = np.random.default_rng(9)
    q, k = _inputs(rng, 1, 1, 3, 2, 64, orc.F16)
    ok = True
    for mode in (orc.ROPE_NEOX, orc.ROPE_GPTJ):
        oq, ok_ = orc.rope(q, k, orc.F16, _inv_freq(64), mode, position=0)
        ok = ok and np.array_equal(oq, q) and np.array_equal(ok_, k)
    return ok


def test_position_zero_is_identity():
    assert identity_ok()


def norm_preserved_ok():
    rng = np.random.default_rng(10)
    q = rng.standard_normal((1, 64, 2, 128)).astype(np.float32)
    q16 = orc.to_bits(q, orc.BF16)
    ok = True
    for mode in (orc.ROPE_NEOX, orc.ROPE_GPTJ):
        oq, _ = orc.rope(q16, None, orc.BF16, _inv_freq(128, 1e4), mode, position=17)
        a, b = orc.to_f32(q16, orc.BF16).astype(np.float64), orc.to_f32(oq, orc.BF16).astype(np.float64)
        t = np.arange(64)
        i1 = t if mode == orc.ROPE_NEOX else 2 * t
        i2 = t + 64 if mode == orc.ROPE_NEOX else 2 * t + 1
        ma, mb = np.hypot(a[..., i1], a[..., i2]), np.hypot(b[..., i1], b[..., i2])
        ok = ok and np.allclose(ma, mb, rtol=2 ** -7, atol=1e-3) and not np.allclose(a, b, atol=1e-2)
    return ok


def test_pair_norm_preserved():
    assert norm_preserved_ok()


def neox_gptj_ok():
    """NeoX(x) == P^-1 GPTJ(P x), P: (x[t], x[t + hd/2]) -> (x[2t], x[2t+1]); weights permuted alike."""
    rng = np.random.default_rng(11)
    hd = 128
    q, k = _inputs(rng, 2, 3, 4, 2, hd, orc.F16)
    wq = orc.to_bits(rng.standard_normal(hd).astype(np.float32) * 0.1 + 1, orc.F16)
    wk = orc.to_bits(rng.standard_normal(hd).astype(np.float32) * 0.1 + 1, orc.F16)
    perm = np.empty(hd, np.int64)
    perm[0::2] = np.arange(hd // 2)
    perm[1::2] = np.arange(hd // 2) + hd // 2
    inv = np.argsort(perm)
    pos = np.array([5, 30000], np.int32)
    a = orc.rope(q, k, orc.F16, _inv_freq(hd), orc.ROPE_NEOX, positions=pos, q_norm=wq, k_norm=wk, nwt=orc.F16)
    b = orc.rope(np.ascontiguousarray(q[..., perm]), np.ascontiguousarray(k[..., perm]), orc.F16, _inv_freq(hd),
                 orc.ROPE_GPTJ, positions=pos, q_norm=np.ascontiguousarray(wq[perm]),
                 k_norm=np.ascontiguousarray(wk[perm]), nwt=orc.F16)
    return np.array_equal(a[0], b[0][..., inv]) and np.array_equal(a[1], b[1][..., inv])


def test_neox_is_permuted_gptj():
    assert neox_gptj_ok()


def test_partial_rotary_passthrough():
    rng = np.random.default_rng(12)
    q, k = _inputs(rng, 1, 4, 2, 2, 128, orc.BF16)
    for mode in (orc.ROPE_NEOX, orc.ROPE_GPTJ):
        oq, ok_ = orc.rope(q, k, orc.BF16, _inv_freq(64), mode, position=100)
        assert np.array_equal(oq[..., 64:], q[..., 64:]) and np.array_equal(ok_[..., 64:], k[..., 64:])
        assert not np.array_equal(oq[..., :64], q[..., :64])


def test_position_sources_agree():
    rng = np.random.default_rng(13)
    q, k = _inputs(rng, 1, 7, 2, 1, 64, orc.F16)
    f = _inv_freq(64)
    a = orc.rope(q, k, orc.F16, f, orc.ROPE_NEOX, position=1234)
    b = orc.rope(q, k, orc.F16, f, orc.ROPE_NEOX, positions=np.array([1234], np.int32))
    c = orc.rope(q, k, orc.F16, f, orc.ROPE_NEOX, position_ids=np.arange(1234, 1241, dtype=np.int32))
    assert all(np.array_equal(x[0], y[0]) and np.array_equal(x[1], y[1]) for x, y in ((a, b), (a, c)))


@pytest.mark.parametrize("mutation", [9, 10, 11, 12, 13, 15])
def test_planted_mistakes_are_caught(mutation):
    orc.set_mutation(mutation)
    results = [all(golden_ok(c) for c in CASES), all(headnorm_ok(c) for c in CASES), identity_ok(),
               norm_preserved_ok(), neox_gptj_ok()]
    assert not all(results), f"mutation {mutation} not caught"
