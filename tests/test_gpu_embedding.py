"""GPU parity of exl3r_embedding (bit-exact) and exl3r_embedding_rms_norm (h bit-exact, y <= 1 ulp)
against the CPU oracle, at configs 1(4) and 5, with both id dtypes and out-of-range ids."""
import numpy as np
import pytest
import torch

import exl3r.ffi as ffi
from _gpu import NTHREADS, TORCH_DT, assert_bitwise, assert_close_ulp, dev_normal, from_dev
from oracle import oracle as orc

pytestmark = pytest.mark.gpu

F16, BF16, F32, I32, I64 = orc.F16, orc.BF16, orc.F32, orc.I32, orc.I64


def zipf_ids(n, vocab, seed, s=1.1, repeat=0.05):
    """Config 5 ids: Zipf(s) ranks over the vocab (id = rank - 1), each position repeating the
    previous id with probability `repeat`."""
    rng = np.random.default_rng(seed)
    ranks = np.arange(1, vocab + 1, dtype=np.float64)
    p = ranks ** -s
    p /= p.sum()
    ids = rng.choice(vocab, size=n, p=p)
    rep = rng.random(n) < repeat
    for i in np.nonzero(rep)[0]:
        if i > 0:
            ids[i] = ids[i - 1]
    return ids.astype(np.int64)


def check_gather(table, tt, ids, idt, ot):
    ids_d = torch.from_numpy(ids.astype(np.int64 if idt == I64 else np.int32)).cuda()
    out = torch.empty((ids.size, table.shape[1]), device="cuda", dtype=TORCH_DT[ot])
    err = torch.zeros(1, dtype=torch.int32, device="cuda")
    ffi.embedding(table, ids_d, out, err)
    torch.cuda.synchronize()
    th = from_dev(table)
    exp, eflag = orc.embedding(th, tt, ids_d.cpu().numpy(), idt, ot, nthreads=NTHREADS)
    assert_bitwise(from_dev(out), exp, what=f"gather {table.shape} n={ids.size} t={tt} o={ot} id={idt}")
    assert int(err.item()) == eflag


def test_c1_gather():
    """Config 1(4): table [151936, 1024] f16 ~ N(0, 0.02), 512 uniform ids; f16 and exact f32 out."""
    table = dev_normal((151936, 1024), 0.0, 0.02, F16, 0)
    ids = np.random.default_rng(0).integers(0, 151936, 512)
    check_gather(table, F16, ids, I64, F16)
    check_gather(table, F16, ids, I32, F32)


def test_c5_gather_zipf():
    """Config 5 gather: table [151936, 5120] bf16 ~ N(0, 0.02), 16384 Zipf(1.1) ids with 5% repeats."""
    table = dev_normal((151936, 5120), 0.0, 0.02, BF16, 1)
    ids = zipf_ids(16384, 151936, 1)
    check_gather(table, BF16, ids, I64, BF16)


@pytest.mark.parametrize("tt,ot", [(BF16, F32), (F32, F32), (F16, F16)])
def test_small_tables(tt, ot):
    table = dev_normal((1000, 72), 0.0, 0.02, tt, 2)
    ids = np.random.default_rng(3).integers(0, 1000, 300)
    check_gather(table, tt, ids, I32, ot)
    table2 = dev_normal((50, 13), 0.0, 0.02, tt, 4)    # hidden % 8 != 0 -> generic kernel
    check_gather(table2, tt, np.arange(50)[::-1].copy(), I64, ot)


@pytest.mark.parametrize("tt,ot,hidden", [(BF16, F32, 5120), (F32, F32, 2048), (F16, F32, 512)])
def test_split_chunks_f32(tt, ot, hidden):
    """An f32 side with rows of whole 512-element spans: split chunks (two quads 256 apart per lane),
    with out-of-range ids zeroing their rows."""
    table = dev_normal((3000, hidden), 0.0, 0.02, tt, 6)
    ids = np.random.default_rng(7).integers(0, 3000, 700)
    ids[[5, 300]] = [-2, 3000]
    check_gather(table, tt, ids, I64, ot)


def test_out_of_range_ids():
    table = dev_normal((100, 256), 0.0, 0.02, BF16, 5)
    check_gather(table, BF16, np.array([3, -1, 100, 99, 1 << 40, 0]), I64, BF16)


def test_nan_payloads_bit_exact():
    raw = torch.tensor([[0x7FC1, -127, 1, -32768] * 4], dtype=torch.int16)  # NaN payloads, denormal, -0
    table = raw.view(torch.bfloat16).cuda()
    check_gather(table, BF16, np.array([0, 0, 0]), I32, BF16)


def run_fused(n, vocab, hidden, tt, ht, yt, wt, seed, ids=None):
    table = dev_normal((vocab, hidden), 0.0, 0.02, tt, seed)
    w = dev_normal((hidden,), 1.0, 0.1, wt, seed + 1)
    ids = zipf_ids(n, vocab, seed) if ids is None else ids
    ids_d = torch.from_numpy(ids).cuda()
    y = torch.empty((n, hidden), device="cuda", dtype=TORCH_DT[yt])
    h = torch.empty((n, hidden), device="cuda", dtype=TORCH_DT[ht]) if ht is not None else None
    err = torch.zeros(1, dtype=torch.int32, device="cuda")
    ffi.embedding_rms_norm(table, ids_d, h, w, y, 1e-6, 0.0, 1.0, err)
    torch.cuda.synchronize()
    eh, ey, eflag = orc.embedding_rms_norm(from_dev(table), tt, ids, I64, from_dev(w), wt, yt, ht=ht, eps=1e-6,
                                           nthreads=NTHREADS)
    if ht is not None:
        assert_bitwise(from_dev(h), eh, what="fused h")
    assert_close_ulp(from_dev(y), ey, yt, 3 if yt == F32 else 1, what=f"fused y n={n} hidden={hidden}")
    assert int(err.item()) == eflag


def test_c5_gather_rms_norm():
    """Config 5: gathered rows then RMSNorm (eps 1e-6, w ~ N(1, 0.1)), writing h and y (bf16)."""
    run_fused(16384, 151936, 5120, BF16, BF16, BF16, BF16, seed=7)


@pytest.mark.parametrize("tt,ht,yt,wt", [(F16, F32, F16, F16), (BF16, None, BF16, BF16), (F32, F32, F16, F16)])
def test_fused_variants(tt, ht, yt, wt):
    run_fused(257, 3000, 1024, tt, ht, yt, wt, seed=8)


def test_fused_bad_ids_and_generic():
    run_fused(4, 64, 256, BF16, BF16, BF16, BF16, seed=9, ids=np.array([1, -5, 64, 2], np.int64))
    run_fused(6, 64, 100, F16, F16, F16, F16, seed=10)


def test_zero_ids():
    table = torch.zeros((16, 64), device="cuda", dtype=torch.bfloat16)
    ids = torch.empty(0, device="cuda", dtype=torch.int64)
    ffi.embedding(table, ids, torch.empty((0, 64), device="cuda", dtype=torch.float32))
    y = torch.empty((0, 64), device="cuda", dtype=torch.bfloat16)
    ffi.embedding_rms_norm(table, ids, None, None, y, 1e-6)
    torch.cuda.synchronize()
