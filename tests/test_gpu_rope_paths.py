"""Both vector RoPE kernels (the wave-per-token NeoX prefill kernel and the flattened kernel)
forced through the launch-shape hook of the sweep/test build (libexl3rowops_tune.so, the same
sources with the overrides compiled in) on the same cases, each checked against the CPU oracle: every
batch width and grid shape of the prefill kernel, head dims 64 / 128 / 256, partial rotary, q only,
strided rows and every position source, so parity does not depend on which kernel the size
heuristic picks (GPT-J always takes the flattened kernel)."""
import ctypes

import numpy as np
import pytest
import torch

import exl3r
import exl3r._lib as L
from test_gpu_rope import run

pytestmark = pytest.mark.gpu

F16, BF16, F32 = exl3r.F16, exl3r.BF16, exl3r.F32


@pytest.fixture
def tune():
    """Kernel choice, heads per lane and grid of the sweep/test build, which the wrappers call inside the
    fixture."""
    with L.tuned() as lib:
        def set_(use, hpl=0, wpc=0):
            lib.exl3r_tune_rope_tok(use, hpl, wpc)
        yield set_


@pytest.mark.parametrize("hpl,wpc", [(2, 0), (3, 0), (2, 1), (3, 1), (2, 4), (3, 4)])
def test_prefill_kernel_batches_and_grids(tune, hpl, wpc):
    tune(2, hpl, wpc)
    rng = np.random.default_rng(hpl * 10 + wpc)
    pid = rng.integers(0, 40000, (1, 300)).astype(np.int32)
    run(1, 300, 20, 6, 128, 128, exl3r.ROPE_NEOX, F16, position_ids=pid, seed=hpl + wpc)
    run(2, 77, 9, 3, 128, 128, exl3r.ROPE_NEOX, BF16, nwt=BF16, positions=np.array([5, 31000], np.int32), seed=7)


@pytest.mark.parametrize("use", [1, 2])
@pytest.mark.parametrize("hd,R,mode,dt,nwt", [(64, 64, exl3r.ROPE_NEOX, F16, F16), (256, 256, exl3r.ROPE_NEOX, BF16, F32),
                                              (128, 64, exl3r.ROPE_NEOX, F16, BF16), (128, 96, exl3r.ROPE_GPTJ, F16, F16),
                                              (128, 128, exl3r.ROPE_GPTJ, BF16, BF16), (64, 32, exl3r.ROPE_GPTJ, F16, F32)])
def test_both_kernels_shapes(tune, use, hd, R, mode, dt, nwt):
    tune(use, 3, 0)
    run(1, 130, 7, 3, hd, R, mode, dt, nwt=nwt, position=1234, seed=hd + R + use)


@pytest.mark.parametrize("use", [1, 2])
def test_both_kernels_no_norm_q_only_out_of_place(tune, use):
    tune(use)
    run(1, 65, 8, 0, 128, 128, exl3r.ROPE_NEOX, F16, norm=False, with_k=False, position=70000)
    run(3, 21, 8, 2, 128, 128, exl3r.ROPE_NEOX, F16, norm=True, position=11, out_of_place=True, attn=0.5, cb=1.0)


@pytest.mark.parametrize("use", [1, 2])
@pytest.mark.parametrize("hq,hk,hd", [(128, 8, 128), (6, 3, 128), (1, 1, 128), (40, 0, 128), (50, 10, 64),
                                      (9, 3, 256)])
def test_both_kernels_head_counts(tune, use, hq, hk, hd):
    """Many heads (128 + 8), a lane group that mixes q and k heads (6 + 3), single heads, q only, and the
    64 / 256 head dims."""
    tune(use)
    run(2, 50, hq, hk, hd, hd, exl3r.ROPE_NEOX, F16, position=321, with_k=hk > 0, seed=hq + hk)
    run(1, 33, hq, hk, hd, hd // 2, exl3r.ROPE_GPTJ, BF16, nwt=F32, position=9, with_k=hk > 0, seed=hq * hk + 1)
