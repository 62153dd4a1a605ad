"""The oracle's gated RMSNorm (reference kernels/norm.cu:482-668), sigmoid gate multiply
(activation.cu:532-568) and q/g deinterleave (activation.cu:721-779), pinned by relations that hold
exactly in floating point, by torch float64 evaluations, and by planted mistakes.

  - A sigmoid gate of 30 is exactly 1.0 in fp32, so gate-after and gate-first both reduce to the
    plain RMSNorm oracle (itself pinned by torch fixtures), bitwise.
  - A sigmoid gate of 0 is exactly 0.5: gate-after halves the f32 output exactly.
  - Gate-first with eps = 0 and a constant gate of 0.5 scales x by 2^-1; the power-of-two scalings
    cancel exactly in sqrt and divide, so the output equals the plain norm bitwise.
  - w_groups = k equals row-by-row calls with the row's own weight slice.
  - The deinterleave equals a numpy reshape of [rows, heads, 2, hd]."""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import oracle as orc
from _util import ulp_dist

F32, F16, BF16 = orc.F32, orc.F16, orc.BF16
ORM_GATED_WGROUP, ORM_GATED_ORDER, ORM_SIGMOID_SIGN, ORM_QG_SWAP = 17, 18, 19, 20


def bits(rng, shape, mean, std, dt):
    return orc.to_bits((rng.standard_normal(shape, dtype=np.float32) * std + mean).astype(np.float32), dt)


def setup(seed=0, rows=7, dim=96, xt=BF16, gt=F32, wt=F32, w_groups=1):
    rng = np.random.default_rng(seed)
    return (bits(rng, (rows, dim), 0, 1, xt), bits(rng, (rows, dim), 0, 2, gt),
            bits(rng, (w_groups * dim,), 1, 0.1, wt))


def f32(a, dt):
    return orc.to_f32(a, dt)


@pytest.mark.parametrize("gate_first", [False, True])
def test_unit_sigmoid_gate_is_plain_rms_norm(gate_first):
    x, _, w = setup(1)
    g = np.full(x.shape, 30.0, np.float32)
    y = orc.gated_rms_norm(x, BF16, g, F32, F32, w=w, wt=F32, gate_first=gate_first, gate_act=1)
    ref = orc.rms_norm(x, BF16, w, F32, F32, eps=1e-6)
    assert np.array_equal(y.view(np.uint32), ref.view(np.uint32))


def test_half_sigmoid_gate_halves_exactly():
    x, _, w = setup(2)
    g = np.zeros(x.shape, np.float32)
    y = orc.gated_rms_norm(x, BF16, g, F32, F32, w=w, gate_act=1)
    ref = orc.rms_norm(x, BF16, w, F32, F32, eps=1e-6)
    assert np.array_equal(y, ref * np.float32(0.5))
    assert not np.any(orc.gated_rms_norm(x, BF16, g, F32, F32, w=w, gate_act=0))      # silu(0) = 0


def test_gate_first_power_of_two_gate_cancels():
    x, _, w = setup(3)
    g = np.zeros(x.shape, np.float32)   # sigmoid(0) = 0.5
    y = orc.gated_rms_norm(x, BF16, g, F32, F32, w=w, gate_first=True, gate_act=1, eps=0.0)
    ref = orc.rms_norm(x, BF16, w, F32, F32, eps=0.0)
    assert np.array_equal(y.view(np.uint32), ref.view(np.uint32))


def test_w_groups_equal_row_slices():
    x, g, w = setup(4, rows=9, w_groups=3)
    y = orc.gated_rms_norm(x, BF16, g, F32, F32, w=w, w_groups=3)
    dim = x.shape[1]
    for i in range(x.shape[0]):
        yi = orc.gated_rms_norm(x[i:i + 1], BF16, g[i:i + 1], F32, F32, w=w[(i % 3) * dim:(i % 3 + 1) * dim].copy())
        assert np.array_equal(y[i], yi[0])


@pytest.mark.parametrize("gate_act", [0, 1])
@pytest.mark.parametrize("gate_first", [False, True])
def test_against_torch_float64(gate_act, gate_first):
    x, g, w = setup(5 + gate_act + 2 * gate_first, rows=16, dim=256)
    xf, gf, wf = (torch.from_numpy(f32(a, dt).astype(np.float64)) for a, dt in ((x, BF16), (g, F32), (w, F32)))
    a = torch.sigmoid(gf) if gate_act else F.silu(gf)
    v = xf * a if gate_first else xf
    n = F.rms_norm(v, (256,), eps=1e-6) * wf
    ref = (n if gate_first else n * a).numpy()
    y = orc.gated_rms_norm(x, BF16, g, F32, F16, w=w, gate_first=gate_first, gate_act=gate_act)
    d = ulp_dist(y, orc.to_bits(ref.astype(np.float32), F16), F16)
    assert d.max() <= 1, d.max()


def test_mul_sigmoid_against_torch_and_special_values():
    rng = np.random.default_rng(9)
    x, y = bits(rng, (33, 64), 0, 2, F16), bits(rng, (33, 64), 0, 4, F16)
    z = orc.mul_sigmoid(x, y, F16, F16)
    ref = (torch.from_numpy(f32(x, F16).astype(np.float64)) * torch.sigmoid(torch.from_numpy(f32(y, F16).astype(np.float64)))).numpy()
    assert ulp_dist(z, orc.to_bits(ref.astype(np.float32), F16), F16).max() <= 1
    xs = orc.to_bits(np.array([[3.0, -5.0, 7.0, 1.0]], np.float32), F16)
    ys = orc.to_bits(np.array([[0.0, 60.0, -60.0, float("inf")]], np.float32), F16)
    assert list(f32(orc.mul_sigmoid(xs, ys, F16, F32), F32)[0]) == [1.5, -5.0, pytest.approx(7.0 * np.exp(-60.0), rel=1e-6), 1.0]


def test_deinterleave_is_a_reshape():
    rng = np.random.default_rng(10)
    rows, heads, hd = 5, 6, 64
    qg = rng.integers(0, 65535, (rows, heads * 2 * hd)).astype(np.uint16)
    q, g = orc.deinterleave_qg(qg, heads, hd)
    r = qg.reshape(rows, heads, 2, hd)
    assert np.array_equal(q, r[:, :, 0].reshape(rows, -1)) and np.array_equal(g, r[:, :, 1].reshape(rows, -1))


@pytest.mark.parametrize("mutation", [ORM_GATED_WGROUP, ORM_GATED_ORDER, ORM_SIGMOID_SIGN, ORM_QG_SWAP])
def test_planted_mistakes_are_caught(mutation):
    x, g, w = setup(11, rows=6, w_groups=2)
    qg = np.random.default_rng(12).integers(0, 65535, (4, 2 * 2 * 32)).astype(np.uint16)
    clean = (orc.gated_rms_norm(x, BF16, g, F32, F32, w=w, w_groups=2, gate_first=True, gate_act=1),
             orc.deinterleave_qg(qg, 2, 32))
    orc.set_mutation(mutation)
    try:
        bad = (orc.gated_rms_norm(x, BF16, g, F32, F32, w=w, w_groups=2, gate_first=True, gate_act=1),
               orc.deinterleave_qg(qg, 2, 32))
    finally:
        orc.set_mutation(0)
    differs = not np.array_equal(clean[0], bad[0]) or not all(np.array_equal(a, b) for a, b in zip(clean[1], bad[1]))
    assert differs
