"""Shared helpers for the tests: ulp distances, fixture loading, seeded inputs, torch<->storage."""
import os

import numpy as np

from oracle import oracle as orc

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def load_cases(name):
    z = np.load(os.path.join(GOLDEN, name), allow_pickle=False)
    n = int(z["n"])
    cases = [{} for _ in range(n)]
    for key in z.files:
        if key == "n":
            continue
        i, k = key.split("/", 1)
        v = z[key]
        cases[int(i)][k] = v.item() if v.ndim == 0 else v
    return cases


def ordered(bits, code):
    """Storage array -> int64 ordered so that adjacent representable values differ by 1."""
    if code == orc.F32:
        u = np.asarray(bits, np.float32).view(np.int32).astype(np.int64)
        return np.where(u < 0, -(u & 0x7FFFFFFF), u)
    u = np.asarray(bits, np.uint16).astype(np.int64)
    return np.where(u & 0x8000, -(u & 0x7FFF), u)


def isnan_bits(bits, code):
    return np.isnan(orc.to_f32(bits, code))


def ulp_dist(a, b, code):
    """Elementwise ulp distance between two storage arrays of dtype `code` (NaN == NaN -> 0,
    NaN vs number -> huge)."""
    da = ordered(a, code)
    db = ordered(b, code)
    d = np.abs(da - db)
    na, nb = isnan_bits(a, code), isnan_bits(b, code)
    d = np.where(na & nb, 0, d)
    d = np.where(na ^ nb, 1 << 40, d)
    return d


def round64(v, code):
    """float64 values -> storage of dtype `code`, one RNE."""
    v = np.asarray(v, np.float64)
    r = np.vectorize(lambda t: orc.load().oracle_round(float(t), code), otypes=[np.float64])(v)
    return orc.to_bits(r.astype(np.float32), code)


def max_rel_err(a, b, code):
    """max |a - b| / max |b| over finite elements (the 'relative to the output scale' bound)."""
    fa, fb = orc.to_f32(a, code).astype(np.float64), orc.to_f32(b, code).astype(np.float64)
    m = np.isfinite(fa) & np.isfinite(fb)
    if not m.any():
        return 0.0
    scale = np.max(np.abs(fb[m]))
    return float(np.max(np.abs(fa[m] - fb[m])) / scale) if scale > 0 else float(np.max(np.abs(fa[m])))


def normal(rng, shape, mean, std, code):
    """Seeded N(mean, std) in fp32, rounded RNE to `code` (the bench/test input convention)."""
    v = (rng.standard_normal(shape, dtype=np.float32) * np.float32(std) + np.float32(mean)).astype(np.float32)
    return orc.to_bits(v, code)
