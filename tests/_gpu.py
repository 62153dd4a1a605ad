"""GPU-side test helpers: move storage arrays (fp32 / raw 16-bit bits) to and from torch tensors,
seeded device-side input generation, and the parity assertions of the north-star tolerances."""
import numpy as np
import torch

from _util import max_rel_err, ulp_dist
from oracle import oracle as orc

TORCH_DT = {orc.F32: torch.float32, orc.F16: torch.float16, orc.BF16: torch.bfloat16, orc.I32: torch.int32,
            orc.I64: torch.int64}
NTHREADS = 8


def to_dev(a, code, device="cuda"):
    a = np.ascontiguousarray(a)
    if code in (orc.F16, orc.BF16):
        return torch.from_numpy(a.view(np.int16)).view(TORCH_DT[code]).to(device)
    return torch.from_numpy(a).to(device)


def from_dev(t):
    t = t.detach().cpu().contiguous()
    if t.dtype in (torch.float16, torch.bfloat16):
        return t.view(torch.int16).numpy().view(np.uint16)
    return t.numpy()


def code_of(t):
    return {v: k for k, v in TORCH_DT.items()}[t.dtype]


def dev_normal(shape, mean, std, code, seed, device="cuda"):
    """Seeded N(mean, std) generated in fp32 on the GPU and rounded RNE to `code`."""
    g = torch.Generator(device=device).manual_seed(seed)
    v = torch.randn(shape, generator=g, device=device, dtype=torch.float32) * std + mean
    return v.to(TORCH_DT[code])


def rel_bound(code):
    """Max abs error relative to the output scale (max |oracle|).  2e-3 for f16/f32 outputs; for
    bf16 one ulp is already 2^-8..2^-7 of the value, so a 1-ulp difference at the largest element
    can reach 2^-7 of the scale and the ulp bound is the binding one."""
    return 2.0 ** -7 if code == orc.BF16 else 2e-3


def assert_close_ulp(got, exp, code, max_ulp, rel=None, what=""):
    """GPU vs oracle: elementwise ulp distance <= max_ulp and max abs err <= rel * output scale."""
    if rel is None:
        rel = rel_bound(code)
    d = ulp_dist(got, exp, code)
    mre = max_rel_err(got, exp, code)
    stats = f"{what}: max_ulp={int(d.max()) if d.size else 0} exact={np.mean(d == 0) if d.size else 1:.6f} max_rel_err={mre:.3e}"
    print(stats)
    assert d.size == 0 or d.max() <= max_ulp, stats
    assert mre <= rel, stats
    return d


def assert_close_rel(got, exp, rel, what=""):
    """f32 outputs: elementwise |got - exp| <= rel * |exp| + 2^-146 (a few fp32 denormal ulps;
    NaN must match NaN)."""
    g = np.asarray(got, np.float64)
    e = np.asarray(exp, np.float64)
    nan_ok = np.array_equal(np.isnan(g), np.isnan(e))
    m = ~np.isnan(e)
    inf_ok = np.array_equal(g[m & np.isinf(e)], e[m & np.isinf(e)])
    f = m & np.isfinite(e)
    err = np.maximum(np.abs(g[f] - e[f]) - 2.0 ** -146, 0.0) / np.maximum(np.abs(e[f]), 2.0 ** -149)
    worst = float(err.max()) if err.size else 0.0
    stats = f"{what}: max_elem_rel_err={worst:.3e} nan_ok={nan_ok} inf_ok={inf_ok}"
    print(stats)
    assert nan_ok and inf_ok and worst <= rel, stats


def assert_bitwise(got, exp, what=""):
    same = np.array_equal(np.ascontiguousarray(got).view(np.uint8), np.ascontiguousarray(exp).view(np.uint8))
    print(f"{what}: bitwise={'yes' if same else 'NO'}")
    assert same, what


def had_abs_tol(xin, r):
    """Per element: 2^-17 * |r| * (sum of |input| over the element's 128-block), xin [rows, cols] floats.
    The matrix-core and butterfly fp32 transforms are each within a few 2^-24 * sum|input| of the exact
    one (32-term MFMA sums plus 2 stages, against 7 butterfly stages), so their difference before the f16
    rounding is well inside this."""
    a = np.abs(np.asarray(xin, np.float64))
    rows, cols = a.shape
    s = a.reshape(rows, cols // 128, 128).sum(-1)
    return np.repeat(2.0 ** -17 * abs(r) * s, 128, axis=1)


def assert_had_close(got, exp, xin, r, what="", min_exact=0.98, max_ulp=1):
    """Matrix-core Hadamard results against the butterfly's (f16 storage [rows, cols]): each element is
    the same value (+0 and -0 equal), within max_ulp f16 steps (1: the neighbour; 2 after an f16
    post-scale product, which rounds a second time), or within had_abs_tol (where the transform
    cancels); NaN only where the other is NaN; and at least min_exact of the elements are identical."""
    got = np.ascontiguousarray(got)
    exp = np.ascontiguousarray(exp)
    g = orc.to_f32(got, orc.F16).astype(np.float64)
    e = orc.to_f32(exp, orc.F16).astype(np.float64)
    d = ulp_dist(got, exp, orc.F16)
    with np.errstate(invalid="ignore"):
        diff = np.abs(g - e)
        ok = (d <= max_ulp) | (diff <= had_abs_tol(xin, r))
    same = d == 0
    bad = int((~ok).sum())
    stats = (f"{what}: identical={same.mean():.6f} neighbour={np.mean(d == 1):.6f} "
             f"beyond_neighbour={np.mean(d > 1):.6f} outside_tolerance={bad}")
    print(stats)
    assert bad == 0, stats
    assert same.mean() >= min_exact, stats



def assert_head_close(got, exp, hd, what="", rel=2.0 ** -8, max_ulp=2, min_exact=0.97):
    """f16 heads of hd elements computed from the matrix-core output rotation against the oracle's
    composition with the butterfly: each element within max_ulp f16 steps of the oracle, or within rel
    times its head's largest |oracle value| (a last-place difference of the transform moves through the
    head norm's statistic and RoPE's differences, which can cancel to a small result); NaN only where
    the oracle has NaN; at least min_exact of the elements identical.  A wrong index, sign or operand
    moves results by the order of the head's scale, far outside this."""
    got = np.ascontiguousarray(got).reshape(-1, hd)
    exp = np.ascontiguousarray(exp).reshape(-1, hd)
    g = orc.to_f32(got, orc.F16).astype(np.float64)
    e = orc.to_f32(exp, orc.F16).astype(np.float64)
    d = ulp_dist(got, exp, orc.F16)
    with np.errstate(invalid="ignore"):
        scale = np.nanmax(np.where(np.isfinite(e), np.abs(e), 0.0), axis=1, keepdims=True)
        ok = (d <= max_ulp) | (np.abs(g - e) <= rel * scale)
    same = d == 0
    bad = int((~ok).sum())
    stats = (f"{what}: identical={same.mean():.6f} within_2ulp={np.mean(d <= 2):.6f} "
             f"outside_tolerance={bad} of {d.size}")
    print(stats)
    assert bad == 0, stats
    assert same.mean() >= min_exact, stats
