"""GPU parity of exl3r_argmax_sample against the CPU oracle (itself pinned to numpy.argmax): bit-exact
token ids on decode and prefill logits, every dtype, the max_logit mask (odd and even), ties that
span slices (lowest index wins across waves), NaN / inf / signed-zero rows, unaligned rows and an
unpadded vocab."""
import numpy as np
import pytest
import torch

import exl3r.ffi as ffi
from _gpu import NTHREADS, TORCH_DT, dev_normal, from_dev, to_dev
from oracle import oracle as orc

pytestmark = pytest.mark.gpu

F16, BF16, F32 = orc.F16, orc.BF16, orc.F32


def run(logits, dt, max_logit=0):
    ids = torch.full((logits.shape[0],), -7, dtype=torch.int64, device="cuda")
    ffi.argmax_sample(logits, ids, max_logit)
    torch.cuda.synchronize()
    exp = orc.argmax(np.ascontiguousarray(from_dev(logits)), dt, max_logit, nthreads=NTHREADS)
    got = ids.cpu().numpy()
    assert np.array_equal(got, exp), f"rows differing: {np.nonzero(got != exp)[0][:8]}"


@pytest.mark.parametrize("rows", [1, 8, 64])
def test_decode_vocab(rows):
    run(dev_normal((rows, 151936), 0, 3, F16, rows), F16)


@pytest.mark.parametrize("dt", [BF16, F32])
def test_prefill_rows_dtypes(dt):
    run(dev_normal((300, 32000), 0, 3, dt, 5), dt)


@pytest.mark.parametrize("m", [1, 2, 151643, 151644, 151936, 200000, 0])
def test_mask(m):
    run(dev_normal((4, 151936), 0, 3, F16, 6 + (m % 7)), F16, m)


def test_ties_across_slices():
    x = np.zeros((5, 20000), np.float32)
    x[0, [3000, 17000]] = 5.0          # two slices, same value -> 3000
    x[1, [19999, 512, 8]] = 2.0        # -> 8
    x[2, :] = 1.0                      # all equal -> 0
    x[3, [1024, 1023]] = 4.0           # slice boundary -> 1023
    x[4, 10000] = 1e-30                # a single positive -> 10000
    for dt in (F16, BF16, F32):
        run(to_dev(orc.to_bits(x, dt), dt), dt)


def test_special_values():
    x = np.full((6, 3000), -1.0, np.float32)
    x[0, :] = -np.inf
    x[1, [5, 2500]] = np.inf
    x[2, [7, 2999]] = np.nan
    x[3, :] = -0.0
    x[3, 1500] = 0.0
    x[4, [100, 200]] = [np.nan, np.inf]
    x[5, 2999] = -0.5
    for dt in (F16, F32):
        run(to_dev(orc.to_bits(x, dt), dt), dt)


def test_unaligned_and_unpadded():
    base = dev_normal((7, 50001), 0, 3, F16, 8)
    run(base[:, 1:], F16)              # rows start 2 bytes off 16-byte alignment: element path
    run(base[:, :50001], F16)          # odd vocab, stride 50001
    run(dev_normal((3, 13), 0, 3, F32, 9), F32, 12)


@pytest.mark.parametrize("rows", [127, 128, 383, 384, 511, 512, 1500])
def test_many_rows(rows):
    run(dev_normal((rows, 20000), 0, 3, F16, rows), F16)
    run(dev_normal((rows, 5003), 0, 3, BF16, rows + 1)[:, 1:], BF16, 4000)


def test_zero_rows():
    ids = torch.empty(0, dtype=torch.int64, device="cuda")
    ffi.argmax_sample(torch.empty((0, 100), device="cuda", dtype=torch.float16), ids)
    torch.cuda.synchronize()


@pytest.mark.parametrize("rows", [6, 130])
def test_f16_chunk_path_special_values(rows):
    """f16 logits take the chunk-wise path (packed NaN-propagating maxima per 8 logits, the held chunk
    searched once): the element rule must still hold inside a chunk, across chunks and in a partial
    last chunk, on both kernels (6 rows: sliced; 130: a workgroup per row)."""
    n = 4104                                   # 513 whole chunks; masks below cut partial ones
    x = np.full((rows, n), -3.0, np.float32)
    x[0, [16, 17]] = [-0.0, 0.0]               # -0 then +0 in one chunk, both maximal -> 16
    x[0, :16] = -1.0
    x[1, [9, 40]] = [0.0, -0.0]                # +0 in an earlier chunk than -0 -> 9
    x[2, [2, 11]] = [np.inf, np.nan]           # a NaN after an inf -> the NaN
    x[3, [13, 4000, 4001]] = [np.nan, np.nan, np.nan]   # the first NaN
    x[4, [7, 8]] = [5.0, 5.0]                  # equal maxima across a chunk boundary -> 7
    x[5, [6, 5]] = [9.0, 9.0]                  # within one chunk -> 5
    x[:, n - 1] = np.where(np.arange(rows) >= 6, 100.0, x[:, n - 1])  # rows >= 6: the last logit
    bits = orc.to_bits(x, F16)
    bits[3, 13] = 0xFE00                       # a negative-signed NaN is a NaN (still the first)
    dev = to_dev(bits, F16)
    run(dev, F16)
    run(dev, F16, n - 3)                       # a partial last chunk, row maxima cut off
    y = np.full((rows, n), -np.inf, np.float32)   # all -inf -> 0; one finite value in a partial chunk
    y[1, 4100] = -70000.0                      # -inf in f16 after rounding: still all -inf -> 0
    y[2, 4101] = 1.0
    run(to_dev(orc.to_bits(y, F16), F16), F16, 4102)
