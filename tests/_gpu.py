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
