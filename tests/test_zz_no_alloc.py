"""GPU check of exl3r_argmax_sample_noalloc (the allocation-free argmax: the library's own per-GPU
scratch as the one-launch kernel's workspace) through the C ABI against exl3r_argmax_sample_ws with a
caller's workspace, token ids exactly equal (and equal to the CPU oracle), on two calls in a row, the
second with a smaller input -- the scratch keeps the first call's contents, which must be back at
zero -- and a third at 200 rows, which takes the workgroup-per-row kernel and no scratch."""
import ctypes

import numpy as np
import pytest
import torch

import exl3r
import exl3r._lib as L
from _gpu import NTHREADS, dev_normal, from_dev
from oracle import oracle as orc

pytestmark = pytest.mark.gpu

F16 = orc.F16


def ids_noalloc(x):
    lib = L.load()
    ids = torch.full((x.shape[0],), -7, dtype=torch.int64, device="cuda")
    st = torch.cuda.current_stream().cuda_stream
    rc = lib.exl3r_argmax_sample_noalloc(x.data_ptr(), L.F16, x.shape[0], x.shape[1], x.stride(0), 0, ids.data_ptr(), st)
    assert rc == 0, L.load().exl3r_last_error()
    return ids


def ids_ws(x):
    lib = L.load()
    ws = torch.zeros(lib.exl3r_sample_workspace_bytes(), dtype=torch.uint8, device="cuda")
    ids = torch.full((x.shape[0],), -9, dtype=torch.int64, device="cuda")
    st = torch.cuda.current_stream().cuda_stream
    rc = lib.exl3r_argmax_sample_ws(x.data_ptr(), L.F16, x.shape[0], x.shape[1], x.stride(0), 0, ids.data_ptr(),
                                    ws.data_ptr(), ws.numel(), st)
    assert rc == 0, L.load().exl3r_last_error()
    return ids


def test_noalloc_matches_workspace_entry_point():
    for k, (rows, vocab) in enumerate([(64, 151936), (5, 32000), (200, 20000)]):
        x = dev_normal((rows, vocab), 0, 3, F16, 970 + k)
        got = ids_noalloc(x)
        ref = ids_ws(x)
        torch.cuda.synchronize()
        exp = orc.argmax(np.ascontiguousarray(from_dev(x)), F16, 0, nthreads=NTHREADS)
        print(f"noalloc call {k}: rows={rows} vocab={vocab}", flush=True)
        assert np.array_equal(got.cpu().numpy(), ref.cpu().numpy()), f"call {k}: differs from exl3r_argmax_sample_ws"
        assert np.array_equal(got.cpu().numpy(), exp), f"call {k}: differs from the oracle"


def test_noalloc_in_graph_replays():
    """The allocation-free argmax captured in a HIP graph (after one eager call on the device, which looks
    up the scratch), replayed with new logits written between replays, each replay against the
    workspace entry point's ids."""
    rows, vocab = 32, 151936
    x = dev_normal((rows, vocab), 0, 3, F16, 990)
    side = torch.cuda.Stream()
    with torch.cuda.stream(side):
        ids = ids_noalloc(x)
    torch.cuda.synchronize()
    lib = L.load()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        st = torch.cuda.current_stream().cuda_stream
        rc = lib.exl3r_argmax_sample_noalloc(x.data_ptr(), L.F16, rows, vocab, vocab, 0, ids.data_ptr(), st)
    assert rc == 0
    torch.cuda.synchronize()
    for rep in range(3):
        x.copy_(dev_normal((rows, vocab), 0, 3, F16, 991 + rep))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        ref = ids_ws(x)
        torch.cuda.synchronize()
        assert np.array_equal(ids.cpu().numpy(), ref.cpu().numpy()), f"replay {rep}"
