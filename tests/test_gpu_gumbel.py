"""GPU parity of exl3r_gumbel_noise and exl3r_gumbel_sample against the CPU oracle (itself pinned by
the Philox known-answer vectors, an exhaustive accuracy check of the noise transform and the
Gumbel-max distribution): bit-exact noise and exactly equal token ids on decode and prefill logits,
every dtype, the max_logit mask, unaligned rows, special values, zero rows, and the identity
gumbel_sample(x) == argmax_sample(gumbel_noise(x)) on the device."""
import math

import numpy as np
import pytest
import torch

import exl3r.ffi as ffi
from _gpu import NTHREADS, TORCH_DT, dev_normal, from_dev, to_dev
from oracle import oracle as orc

pytestmark = pytest.mark.gpu

F16, BF16, F32 = orc.F16, orc.BF16, orc.F32


def run_sample(logits, dt, seed, max_logit=0):
    ids = torch.full((logits.shape[0],), -7, dtype=torch.int64, device="cuda")
    ffi.gumbel_sample(logits, ids, max_logit, seed)
    torch.cuda.synchronize()
    exp = orc.gumbel_sample(np.ascontiguousarray(from_dev(logits)), dt, seed, max_logit, nthreads=NTHREADS)
    got = ids.cpu().numpy()
    assert np.array_equal(got, exp), f"rows differing: {np.nonzero(got != exp)[0][:8]}"
    return got


def run_noise(x, dt, seed, out_dt):
    out = torch.empty(x.shape, dtype=TORCH_DT[out_dt], device="cuda")
    ffi.gumbel_noise(x, out, seed)
    torch.cuda.synchronize()
    exp = orc.gumbel_noise(np.ascontiguousarray(from_dev(x)), dt, seed, out_dt, nthreads=NTHREADS)
    got = from_dev(out)
    same = (got.view(np.uint32) == exp.view(np.uint32)) if out_dt == F32 else (got == exp)
    assert same.all(), f"{(~same).sum()} elements differ, first at {np.argwhere(~same)[:4].tolist()}"


@pytest.mark.parametrize("rows", [1, 8, 64])
def test_sample_decode_vocab(rows):
    run_sample(dev_normal((rows, 151936), 0, 3, F16, 40 + rows), F16, 1234 + rows)


@pytest.mark.parametrize("dt", [BF16, F32])
def test_sample_prefill_rows(dt):
    run_sample(dev_normal((600, 32000), 0, 3, dt, 41), dt, 77)          # row-per-workgroup kernel


@pytest.mark.parametrize("rows", [383, 384])
def test_sample_kernel_switch(rows):
    run_sample(dev_normal((rows, 9001), 0, 3, F16, 49), F16, 78)


@pytest.mark.parametrize("m", [1, 2, 151643, 151936, 200000])
def test_sample_mask(m):
    ids = run_sample(dev_normal((4, 151936), 0, 1, F16, 42), F16, 5, m)
    assert ids.max() < min(m, 151936)


def test_sample_special_values_and_unaligned():
    x = np.full((6, 3001), -1.0, np.float32)
    x[0, :] = -np.inf
    x[1, 2500] = np.inf
    x[2, [7, 2999]] = np.nan
    x[3, 1500] = 40.0               # 40 - 2.82 beats -1 + 16.64: always drawn
    x[5, :] = 0.0
    for dt in (F16, F32):
        got = run_sample(to_dev(orc.to_bits(x, dt), dt), dt, 9)
        assert list(got[:4]) == [got[0], 2500, 7, 1500]
    base = dev_normal((5, 4097), 0, 3, BF16, 43)
    run_sample(base[:, 1:], BF16, 10)                  # 2 bytes off 16-byte alignment: element path
    run_sample(base[:, :4001], BF16, 11, 3999)         # odd stride 4097


@pytest.mark.parametrize("seed", [0, 0xFFFFFFFF])
def test_sample_seeds(seed):
    run_sample(dev_normal((16, 50000), 0, 2, F16, 44), F16, seed)


@pytest.mark.parametrize("xt,ot", [(F16, F32), (BF16, F32), (F32, F32), (F16, F16), (F32, BF16)])
def test_noise_dtypes(xt, ot):
    run_noise(dev_normal((9, 8200), 0, 3, xt, 45), xt, 31337, ot)


def test_noise_unaligned_odd_and_in_place():
    base = dev_normal((7, 1001), 0, 3, F32, 46)
    run_noise(base[:, 1:], F32, 3, F32)
    run_noise(base[:, :999], F32, 4, F16)
    x = dev_normal((3, 4096), 0, 3, F32, 47)
    exp = orc.gumbel_noise(from_dev(x), F32, 8, F32)
    ffi.gumbel_noise(x, x, 8)
    torch.cuda.synchronize()
    assert np.array_equal(from_dev(x).view(np.uint32), exp.view(np.uint32))


def test_sample_equals_argmax_of_noise_on_device():
    x = dev_normal((64, 151936), 0, 3, F16, 48)
    noisy = torch.empty(x.shape, dtype=torch.float32, device="cuda")
    ffi.gumbel_noise(x, noisy, 2024)
    a = torch.empty(64, dtype=torch.int64, device="cuda")
    b = torch.empty(64, dtype=torch.int64, device="cuda")
    ffi.argmax_sample(noisy, a, 100000)
    ffi.gumbel_sample(x, b, 100000, 2024)
    torch.cuda.synchronize()
    assert torch.equal(a, b)


def test_draws_follow_softmax():
    logits = torch.tensor([0.0, 1.0, 2.0, -1.0, 0.5, 3.0, float("-inf"), 2.0, -4.0], device="cuda")
    rows = 200000
    ids = torch.empty(rows, dtype=torch.int64, device="cuda")
    ffi.gumbel_sample(logits.expand(rows, -1).contiguous(), ids, 0, 99)
    counts = torch.bincount(ids, minlength=9).double().cpu().numpy()
    p = torch.softmax(logits.double(), 0).cpu().numpy()
    live = p > 0
    assert counts[~live].sum() == 0
    e = p[live] * rows
    chi2 = float(((counts[live] - e) ** 2 / e).sum())
    dof = int(live.sum()) - 1
    assert chi2 < dof + 6 * math.sqrt(2 * dof), chi2


def test_zero_rows_and_cols():
    ids = torch.empty(0, dtype=torch.int64, device="cuda")
    ffi.gumbel_sample(torch.empty((0, 100), device="cuda", dtype=torch.float16), ids, 0, 1)
    x = torch.empty((0, 64), device="cuda")
    ffi.gumbel_noise(x, x, 1)
    y = torch.empty((4, 0), device="cuda")
    ffi.gumbel_noise(y, y, 1)
    torch.cuda.synchronize()
