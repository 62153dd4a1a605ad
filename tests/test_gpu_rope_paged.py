"""GPU parity of exl3r_rope_paged_kv (q/k head norm + RoPE fused with the paged KV-cache append,
reference src/modules.rs:666-704 -> kernels/rope.cu + kernels/generator/cache.cu:143-243) against
the CPU oracle run as the reference runs it: rope, then the append.  q, the optional in-place k
and the whole k / v caches are compared bitwise, on both RoPE kernels."""
import numpy as np
import pytest
import torch

import exl3r
import exl3r._lib as L
import exl3r.ffi as ffi
from _gpu import NTHREADS, assert_bitwise, assert_close_ulp, dev_normal, from_dev
from oracle import oracle as orc

pytestmark = pytest.mark.gpu

F16, BF16 = orc.F16, orc.BF16


def inv_freq(R, theta=1e6):
    return (1.0 / theta ** (np.arange(0, R, 2, dtype=np.float64) / R)).astype(np.float32)


def run(bsz, seq, hq, hk, hd, R, mode, dt, page, pages, max_blocks, seqlens, bt, norm=True, with_out_k=True, seed=0):
    q = dev_normal((bsz, seq, hq, hd), 0, 1, dt, seed)
    k = dev_normal((bsz, seq, hk, hd), 0, 1, dt, seed + 1)
    v = dev_normal((bsz, seq, hk, hd), 0, 1, dt, seed + 2)
    kc = dev_normal((pages, page, hk, hd), 0, 1, dt, seed + 3)
    vc = dev_normal((pages, page, hk, hd), 0, 1, dt, seed + 4)
    qn = dev_normal((hd,), 1, 0.1, dt, seed + 5) if norm else None
    kn = dev_normal((hd,), 1, 0.1, dt, seed + 6) if norm else None
    qh, kh, vh, kch, vch = from_dev(q), from_dev(k), from_dev(v), from_dev(kc), from_dev(vc)
    f = inv_freq(R)
    sl = torch.from_numpy(seqlens.astype(np.int32)).cuda()
    btd = torch.from_numpy(bt.astype(np.int32)).cuda()
    err = torch.zeros(1, dtype=torch.int32, device="cuda")
    ffi.rope_paged_kv(q, q, k, k if with_out_k else None, v, torch.from_numpy(f).cuda(), 0, sl, qn, kn, 1e-6, 0.0,
                      mode, 1.0, kc, vc, btd, sl, err_flag=err)
    torch.cuda.synchronize()
    eq, ek = orc.rope(qh, kh, dt, f, mode, positions=seqlens.astype(np.int32), q_norm=from_dev(qn) if norm else None,
                      k_norm=from_dev(kn) if norm else None, nwt=dt, eps=1e-6, nthreads=NTHREADS)
    e_err = orc.paged_kv_append(ek, vh, dt, kch, vch, bt, seqlens, nthreads=NTHREADS)
    tag = f"paged b{bsz} s{seq} h{hq}/{hk} d{hd} R{R} mode{mode} dt{dt} page{page}"
    assert_close_ulp(from_dev(q), eq, dt, 0, what=tag + " q")
    if with_out_k:
        assert_close_ulp(from_dev(k), ek, dt, 0, what=tag + " k")
    else:
        assert_bitwise(from_dev(k), kh, what=tag + " k untouched")
    assert_bitwise(from_dev(kc), kch, what=tag + " k_cache")
    assert_bitwise(from_dev(vc), vch, what=tag + " v_cache")
    assert int(err.item()) == e_err, tag + " err flag"


def layout(bsz, seq, page, max_blocks, seed, pages=None):
    rng = np.random.default_rng(seed)
    pages = pages or bsz * max_blocks + 3
    bt = rng.permutation(pages)[: bsz * max_blocks].reshape(bsz, max_blocks).astype(np.int32)
    seqlens = rng.integers(0, max_blocks * page - seq + 1, bsz).astype(np.int32)
    return pages, bt, seqlens


@pytest.fixture
def tune():
    """Forces the RoPE kernel (0 auto, 1 never the wave-per-token kernel, 2 always) through the sweep/test
    build of the library, which the wrappers call inside the fixture."""
    with L.tuned() as lib:
        yield lambda use: lib.exl3r_tune_rope_tok(use, 0, 0)


@pytest.mark.parametrize("use", [0, 1, 2])
def test_decode_batch(tune, use):
    tune(use)
    pages, bt, sl = layout(64, 1, 256, 8, 1)
    run(64, 1, 16, 4, 128, 128, exl3r.ROPE_NEOX, F16, 256, pages, 8, sl, bt, seed=1)


@pytest.mark.parametrize("use", [0, 1, 2])
def test_prefill_chunk_crossing_pages(tune, use):
    tune(use)
    pages, bt, sl = layout(2, 600, 256, 6, 2)
    run(2, 600, 16, 4, 128, 128, exl3r.ROPE_NEOX, F16, 256, pages, 6, sl, bt, seed=2)


@pytest.mark.parametrize("dt,mode,R,page,hd", [(BF16, exl3r.ROPE_NEOX, 128, 16, 128), (F16, exl3r.ROPE_GPTJ, 64, 32, 128),
                                               (BF16, exl3r.ROPE_GPTJ, 256, 64, 256), (F16, exl3r.ROPE_NEOX, 64, 8, 64),
                                               (F16, exl3r.ROPE_NEOX, 100, 16, 100)])
def test_dtypes_modes_page_sizes(dt, mode, R, page, hd):
    pages, bt, sl = layout(3, 45, page, 12, 3)
    run(3, 45, 8, 2, hd, R, mode, dt, page, pages, 12, sl, bt, seed=3)


def test_no_out_k_no_norm_large_prefill():
    pages, bt, sl = layout(1, 1500, 256, 8, 4)
    run(1, 1500, 32, 8, 128, 128, exl3r.ROPE_NEOX, F16, 256, pages, 8, sl, bt, norm=False, with_out_k=False, seed=4)


@pytest.mark.parametrize("use", [1, 2])
def test_bad_positions_and_pages_flagged(tune, use):
    tune(use)
    pages, bt, sl = layout(4, 20, 16, 4, 5)
    bt[1, :] = pages + 7           # sequence 1: pages outside the pool
    sl[2] = 4 * 16 - 10            # sequence 2 runs past its block table
    sl[3] = -3                     # negative position
    run(4, 20, 8, 2, 128, 128, exl3r.ROPE_NEOX, F16, 16, pages, 4, sl, bt, seed=5)


def test_zero_tokens():
    z = torch.empty((1, 0, 8, 128), device="cuda", dtype=torch.float16)
    zk = torch.empty((1, 0, 2, 128), device="cuda", dtype=torch.float16)
    kc = torch.zeros((4, 16, 2, 128), device="cuda", dtype=torch.float16)
    bt = torch.zeros((1, 4), device="cuda", dtype=torch.int32)
    sl = torch.zeros(1, device="cuda", dtype=torch.int32)
    ffi.rope_paged_kv(z, z, zk, zk, zk, torch.from_numpy(inv_freq(128)).cuda(), 0, sl, None, None, 1e-6, 0.0,
                      exl3r.ROPE_NEOX, 1.0, kc, kc.clone(), bt, sl)
    torch.cuda.synchronize()
    assert torch.count_nonzero(kc).item() == 0
