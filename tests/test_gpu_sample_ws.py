"""GPU parity of the one-launch sampling forms exl3r_argmax_sample_ws / exl3r_gumbel_sample_ws (row
counters and slots in a caller's workspace, the last workgroup of a row writing the index) against
the CPU oracle and the three-launch entry points: exactly equal token ids at decode shapes, every
dtype, the max_logit mask, ties across slices, NaN / inf rows, unaligned rows, the kernel switch to a
workgroup per row, and one workspace reused by calls of different shapes (its counters and slots
must come back to zero after every call, which the next call's ids depend on)."""
import numpy as np
import pytest
import torch

import exl3r.ffi as ffi
from _gpu import NTHREADS, dev_normal, from_dev, to_dev
from oracle import oracle as orc

pytestmark = pytest.mark.gpu

F16, BF16, F32 = orc.F16, orc.BF16, orc.F32


def workspace(*_):
    return torch.zeros(ffi.sample_workspace_bytes(), dtype=torch.uint8, device="cuda")


def argmax_ws(logits, ws, max_logit=0):
    ids = torch.full((logits.shape[0],), -7, dtype=torch.int64, device="cuda")
    ffi.argmax_sample_ws(logits, ids, ws, max_logit)
    return ids


def check_argmax(logits, dt, ws, max_logit=0):
    ids = argmax_ws(logits, ws, max_logit)
    ref = torch.full_like(ids, -9)
    ffi.argmax_sample(logits, ref, max_logit)
    torch.cuda.synchronize()
    exp = orc.argmax(np.ascontiguousarray(from_dev(logits)), dt, max_logit, nthreads=NTHREADS)
    got = ids.cpu().numpy()
    assert np.array_equal(got, exp), f"rows differing: {np.nonzero(got != exp)[0][:8]}"
    assert np.array_equal(got, ref.cpu().numpy())


def check_gumbel(logits, dt, ws, seed, max_logit=0):
    ids = torch.full((logits.shape[0],), -7, dtype=torch.int64, device="cuda")
    ffi.gumbel_sample_ws(logits, ids, ws, max_logit, seed)
    ref = torch.full_like(ids, -9)
    ffi.gumbel_sample(logits, ref, max_logit, seed)
    torch.cuda.synchronize()
    exp = orc.gumbel_sample(np.ascontiguousarray(from_dev(logits)), dt, seed, max_logit, nthreads=NTHREADS)
    got = ids.cpu().numpy()
    assert np.array_equal(got, exp), f"rows differing: {np.nonzero(got != exp)[0][:8]}"
    assert np.array_equal(got, ref.cpu().numpy())


@pytest.mark.parametrize("rows", [1, 2, 8, 15, 16, 64, 127])
def test_argmax_decode_vocab(rows):
    check_argmax(dev_normal((rows, 151936), 0, 3, F16, 900 + rows), F16, workspace(rows, 151936))


@pytest.mark.parametrize("dt", [BF16, F32])
def test_argmax_dtypes_and_mask(dt):
    x = dev_normal((24, 151936), 0, 3, dt, 910)
    for m in (0, 1, 2, 8191, 8192, 151643):
        check_argmax(x, dt, workspace(24, 151936, m), m)


def test_argmax_ties_specials_unaligned():
    x = np.full((8, 20000), -1.0, np.float32)
    x[0, [3000, 17000]] = 5.0          # equal maxima in two slices -> 3000
    x[1, :] = 1.0                      # all equal -> 0
    x[2, [2047, 2048]] = 4.0           # slice boundary -> 2047
    x[3, [7, 19999]] = np.nan          # first NaN
    x[4, [100, 200]] = [np.nan, np.inf]
    x[5, :] = -np.inf
    x[6, :] = -0.0
    x[6, 12345] = 0.0
    x[7, 19999] = 3.0
    ws = workspace(8, 20000)
    for dt in (F16, F32):
        check_argmax(to_dev(orc.to_bits(x, dt), dt), dt, ws)
    base = dev_normal((5, 50001), 0, 3, F16, 911)
    check_argmax(base[:, 1:], F16, workspace(5, 50000))      # element path (rows 2 bytes off alignment)


@pytest.mark.parametrize("rows", [128, 300])
def test_argmax_row_kernel_ignores_workspace(rows):
    check_argmax(dev_normal((rows, 20000), 0, 3, F16, 912), F16, workspace(1, 16))


def test_workspace_reused_across_shapes():
    """One workspace, calls of different shapes back to back on one stream: each call's counters start
    at zero only if the previous call left them so."""
    ws = workspace(127, 151936)
    for k, (rows, vocab, m) in enumerate([(64, 151936, 0), (3, 151936, 0), (127, 32000, 0), (64, 151936, 100000),
                                          (1, 151936, 0), (64, 151936, 0)]):
        check_argmax(dev_normal((rows, vocab), 0, 3, F16, 920 + k), F16, ws, m)
        check_gumbel(dev_normal((rows, vocab), 0, 1, F16, 930 + k), F16, ws, 55 + k, m)
    assert int(ws.count_nonzero()) == 0


@pytest.mark.parametrize("rows", [1, 8, 64, 383])
def test_gumbel_decode(rows):
    check_gumbel(dev_normal((rows, 151936 if rows < 100 else 9001), 0, 1, F16, 940 + rows), F16,
                 workspace(rows, 151936), 4242 + rows)


def test_gumbel_dtypes_mask_and_row_kernel():
    check_gumbel(dev_normal((12, 32000), 0, 1, BF16, 950), BF16, workspace(12, 32000), 7, 31999)
    check_gumbel(dev_normal((12, 32000), 0, 1, F32, 951), F32, workspace(12, 32000), 8)
    check_gumbel(dev_normal((400, 5000), 0, 1, F16, 952), F16, workspace(1, 16), 9)      # row kernel


def test_small_workspace_is_an_error():
    x = dev_normal((4, 151936), 0, 3, F16, 960)
    ws = torch.zeros(ffi.sample_workspace_bytes() - 256, dtype=torch.uint8, device="cuda")
    ids = torch.empty(4, dtype=torch.int64, device="cuda")
    with pytest.raises(Exception, match="workspace"):
        ffi.argmax_sample_ws(x, ids, ws)


def test_graph_replays_reuse_the_workspace():
    """argmax_sample_ws and gumbel_sample_ws captured in one HIP graph on one workspace, replayed with new
    logits written between replays: every replay's ids equal the oracle's (the workspace must be back at
    zero after each replay, since nothing in the graph clears it)."""
    rows, vocab = 64, 151936
    x = dev_normal((rows, vocab), 0, 3, F16, 980)
    ws = workspace()
    ids_a = torch.empty(rows, dtype=torch.int64, device="cuda")
    ids_g = torch.empty(rows, dtype=torch.int64, device="cuda")
    side = torch.cuda.Stream()
    with torch.cuda.stream(side):
        ffi.argmax_sample_ws(x, ids_a, ws)                  # warm-up outside capture
        ffi.gumbel_sample_ws(x, ids_g, ws, 0, 11)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        ffi.argmax_sample_ws(x, ids_a, ws)
        ffi.gumbel_sample_ws(x, ids_g, ws, 0, 11)
    torch.cuda.synchronize()
    for rep in range(4):
        x.copy_(dev_normal((rows, vocab), 0, 3, F16, 981 + rep))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        xh = np.ascontiguousarray(from_dev(x))
        assert np.array_equal(ids_a.cpu().numpy(), orc.argmax(xh, F16, 0, nthreads=NTHREADS)), f"replay {rep} argmax"
        assert np.array_equal(ids_g.cpu().numpy(), orc.gumbel_sample(xh, F16, 11, 0, nthreads=NTHREADS)), \
            f"replay {rep} gumbel"
    assert int(ws.count_nonzero()) == 0
