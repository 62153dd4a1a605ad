"""Seeded randomized parity: every entry point on shapes, dtypes, row strides, alignments and
arguments drawn at random inside each op's documented domain (rows and dims that are not multiples
of the vector width, padded rows, every dtype combination, every position source, odd masks),
each case checked against the CPU oracle at the same tolerance as the op's own tests.  The cases
are fixed by their seeds, so a failure names a reproducible configuration."""
import os

import numpy as np
import pytest
import torch

import exl3r
import exl3r.ffi as ffi
from _gpu import NTHREADS, TORCH_DT, assert_bitwise, dev_normal, from_dev
from oracle import oracle as orc
from test_gpu_act import run as run_act
from test_gpu_act_had import run as run_act_had, run_rotated as run_act_had_rotated
from test_gpu_argmax import run as run_argmax
from test_gpu_embedding import check_gather, run_fused
from test_gpu_gated import check as check_gate, run_gated
from test_gpu_gated_had import run as run_gated_had
from test_gpu_gumbel import run_noise, run_sample
from test_gpu_hadamard import run as run_had, scales
from test_gpu_rms_norm import run_plain, run_res
from test_gpu_rms_norm_had import run as run_norm_had
from test_gpu_rope import run as run_rope
from test_gpu_rope_had import run as run_rope_had
from test_gpu_rope_paged import layout, run as run_paged
from test_gpu_rope_table import run as run_rope_table

pytestmark = pytest.mark.gpu

F32, F16, BF16, I32, I64 = orc.F32, orc.F16, orc.BF16, orc.I32, orc.I64
FLOATS = [F32, F16, BF16]
# EXL3R_FUZZ_CASES widens the sweep for a longer run (the default keeps the suite at seconds).
CASES = range(int(os.environ.get("EXL3R_FUZZ_CASES", "24")))


def pick(rng, seq):
    return seq[int(rng.integers(len(seq)))]


def dim_of(rng, lo, hi):
    """A dimension, half the time a multiple of 8 (vector kernels), else anything (generic kernels)."""
    d = int(rng.integers(lo, hi + 1))
    return max(8, d - d % 8) if rng.random() < 0.5 else d


@pytest.mark.parametrize("case", CASES)
def test_fuzz_rms_norm(case):
    rng = np.random.default_rng(1000 + case)
    rows, dim = int(rng.integers(1, 300)), dim_of(rng, 2, 9000)
    xt, wt, yt = pick(rng, FLOATS), pick(rng, FLOATS), pick(rng, FLOATS)
    pad = int(rng.integers(0, 3)) * 8
    run_plain(rows, dim, xt, wt, yt, eps=float(pick(rng, [1e-6, 1e-5, 0.1])), cb=float(pick(rng, [0.0, 1.0])),
              cs=float(pick(rng, [1.0, 0.5, 3.0])), seed=case, ldx=dim + pad, ldy=dim + pad,
              weight=bool(rng.random() < 0.8))
    run_res(int(rng.integers(1, 200)), dim_of(rng, 8, 9000), pick(rng, FLOATS), pick(rng, FLOATS), pick(rng, FLOATS),
            pick(rng, FLOATS), seed=case + 50, cb=float(pick(rng, [0.0, 1.0])))


@pytest.mark.parametrize("case", CASES)
def test_fuzz_act_mul(case):
    rng = np.random.default_rng(2000 + case)
    rows, cols = int(rng.integers(1, 200)), dim_of(rng, 1, 20000)
    it, zt = pick(rng, FLOATS), pick(rng, FLOATS)
    run_act(pick(rng, ["silu", "gelu"]), rows, cols, it, zt, limit=float(pick(rng, [0.0, 0.0, 2.5, 40.0])),
            seed=case, ld=cols + int(rng.integers(0, 3)) * 8, std=float(pick(rng, [1.0, 4.0, 30.0])))


@pytest.mark.parametrize("case", CASES)
def test_fuzz_gated_rms_norm(case):
    rng = np.random.default_rng(3000 + case)
    dim = pick(rng, [64, 128, 256, 512, dim_of(rng, 8, 4096)])
    rows = int(rng.integers(1, 400))
    run_gated(rows, dim, pick(rng, FLOATS), pick(rng, FLOATS), pick(rng, FLOATS), pick(rng, FLOATS),
              w_groups=int(pick(rng, [1, 1, 2, 4])), gate_first=bool(rng.random() < 0.5), gate_act=int(rng.integers(2)),
              cb=float(pick(rng, [0.0, 1.0])), with_w=bool(rng.random() < 0.85), seed=case,
              ld=dim + int(rng.integers(0, 2)) * 8)
    hdim = 128 * int(pick(rng, [1, 1, 2, 3, 8]))
    heads = int(pick(rng, [1, 2, 8, 32]))
    run_gated_had(heads * int(rng.integers(1, 40)), hdim, pick(rng, [F16, BF16]), pick(rng, FLOATS), pick(rng, FLOATS),
                  w_groups=int(pick(rng, [1, 1, 2])), gate_first=bool(rng.random() < 0.5), gate_act=int(rng.integers(2)),
                  cb=float(pick(rng, [0.0, 1.0])), with_w=bool(rng.random() < 0.85), with_y=bool(rng.random() < 0.5),
                  pre=bool(rng.random() < 0.85), heads=heads, seed=case + 1)


@pytest.mark.parametrize("case", CASES)
def test_fuzz_gate_and_split(case):
    rng = np.random.default_rng(3500 + case)
    rows, cols = int(rng.integers(1, 300)), dim_of(rng, 1, 9000)
    it, zt = pick(rng, FLOATS), pick(rng, FLOATS)
    ld = cols + int(rng.integers(0, 2)) * int(pick(rng, [1, 8]))
    x = dev_normal((rows, ld), 0, 2, it, case)[:, :cols]
    y = dev_normal((rows, ld), 0, 3, it, case + 1)[:, :cols]
    z = torch.empty((rows, cols), device="cuda", dtype=TORCH_DT[zt])
    ffi.mul_sigmoid(x, y, z)
    torch.cuda.synchronize()
    exp = orc.mul_sigmoid(np.ascontiguousarray(from_dev(x)), np.ascontiguousarray(from_dev(y)), it, zt,
                          nthreads=NTHREADS)
    check_gate(from_dev(z), exp, zt, f"mul_sigmoid {rows}x{cols} in{it} z{zt}")
    dt = pick(rng, [F16, BF16])
    heads, hd = int(rng.integers(1, 40)), int(pick(rng, [16, 20, 64, 128, 256]))
    rows = int(rng.integers(1, 500))
    qg = dev_normal((rows, heads * 2 * hd), 0, 1, dt, case + 2)
    q = torch.empty((rows, heads, hd), device="cuda", dtype=TORCH_DT[dt])
    g = torch.empty((rows, heads * hd), device="cuda", dtype=TORCH_DT[dt])
    ffi.deinterleave_qg(qg, q, g, hd)
    torch.cuda.synchronize()
    eq, eg = orc.deinterleave_qg(from_dev(qg), heads, hd)
    assert_bitwise(from_dev(q).reshape(rows, -1), eq, what=f"deinterleave q {dt} {rows}x{heads}x{hd}")
    assert_bitwise(from_dev(g), eg, what=f"deinterleave g {dt} {rows}x{heads}x{hd}")


def rope_shape(rng):
    hd = pick(rng, [64, 96, 128, 128, 256, 100, 72])
    R = pick(rng, [hd, hd, hd // 2, max(2, (hd // 4) * 2)])
    R -= R % 2
    return hd, max(R, 2)


def position_source(rng, bsz, seq):
    k = int(rng.integers(3))
    if k == 0:
        return dict(position=int(rng.integers(0, 50000)))
    if k == 1:
        return dict(positions=rng.integers(0, 50000, bsz).astype(np.int32))
    return dict(position_ids=rng.integers(0, 50000, (bsz, seq)).astype(np.int32))


@pytest.mark.parametrize("case", CASES)
def test_fuzz_rope(case):
    rng = np.random.default_rng(4000 + case)
    hd, R = rope_shape(rng)
    bsz = int(rng.integers(1, 5))
    seq = int(pick(rng, [1, int(rng.integers(1, 40)), int(rng.integers(200, 700))]))
    norm = bool(rng.random() < 0.7)
    run_rope(bsz, seq, int(rng.integers(1, 20)), int(rng.integers(1, 6)), hd, R,
             pick(rng, [exl3r.ROPE_NEOX, exl3r.ROPE_GPTJ]), pick(rng, [F16, BF16]), nwt=pick(rng, FLOATS), norm=norm,
             cb=float(pick(rng, [0.0, 1.0])), attn=float(pick(rng, [1.0, 0.7])), seed=case,
             with_k=bool(rng.random() < 0.85), out_of_place=bool(rng.random() < 0.3), **position_source(rng, bsz, seq))


@pytest.mark.parametrize("case", CASES)
def test_fuzz_rope_table(case):
    rng = np.random.default_rng(5000 + case)
    hd, R = rope_shape(rng)
    bsz, seq = int(rng.integers(1, 4)), int(rng.integers(1, 300))
    rows = int(rng.integers(1, 400))
    shared = bool(rng.random() < 0.5)
    table = rng.uniform(-500, 500, (rows, R // 2) if shared else (bsz, rows, R // 2)).astype(np.float32)
    pid = rng.integers(0, rows, (bsz, seq)).astype(np.int32)
    run_rope_table(bsz, seq, int(rng.integers(1, 12)), int(rng.integers(1, 4)), hd, table,
                   pick(rng, [exl3r.ROPE_NEOX, exl3r.ROPE_GPTJ]), pick(rng, [F16, BF16]), nwt=pick(rng, FLOATS),
                   norm=bool(rng.random() < 0.7), position_ids=pid, seed=case)


@pytest.mark.parametrize("case", CASES)
def test_fuzz_rope_paged(case):
    rng = np.random.default_rng(6000 + case)
    hd, R = rope_shape(rng)
    bsz, seq = int(rng.integers(1, 5)), int(pick(rng, [1, int(rng.integers(2, 300))]))
    page = int(pick(rng, [8, 16, 64, 256]))
    max_blocks = (seq + 300) // page + 2
    pages, bt, sl = layout(bsz, seq, page, max_blocks, case)
    run_paged(bsz, seq, int(rng.integers(1, 12)), int(rng.integers(1, 4)), hd, R,
              pick(rng, [exl3r.ROPE_NEOX, exl3r.ROPE_GPTJ]), pick(rng, [F16, BF16]), page, pages, max_blocks, sl, bt,
              norm=bool(rng.random() < 0.7), with_out_k=bool(rng.random() < 0.5), seed=case)


@pytest.mark.parametrize("case", CASES)
def test_fuzz_embedding(case):
    rng = np.random.default_rng(7000 + case)
    vocab, hidden = int(rng.integers(2, 5000)), dim_of(rng, 1, 6000)
    tt = pick(rng, FLOATS)
    ot = pick(rng, [tt, F32])
    table = dev_normal((vocab, hidden), 0.0, 0.02, tt, case)
    ids = rng.integers(-3, vocab + 3, int(rng.integers(1, 500)))
    check_gather(table, tt, ids, pick(rng, [I32, I64]), ot)
    tt2 = pick(rng, FLOATS)
    run_fused(int(rng.integers(1, 300)), vocab, dim_of(rng, 8, 4096), tt2, pick(rng, [None, tt2, F32]),
              pick(rng, FLOATS), pick(rng, FLOATS), seed=case + 7)


@pytest.mark.parametrize("case", CASES)
def test_fuzz_sampling(case):
    rng = np.random.default_rng(8000 + case)
    rows, vocab = int(pick(rng, [1, int(rng.integers(2, 130)), int(rng.integers(130, 700))])), int(rng.integers(1, 160000))
    dt = pick(rng, FLOATS)
    x = dev_normal((rows, vocab + int(rng.integers(0, 2))), 0.0, float(pick(rng, [0.5, 3.0, 20.0])), dt, case)
    off = int(rng.integers(0, 2))
    logits = x[:, off:off + vocab] if x.shape[1] > vocab else x[:, :vocab]
    mask = int(pick(rng, [0, 0, int(rng.integers(1, vocab + 1)), vocab + 5]))
    run_argmax(logits, dt, mask)
    run_sample(logits, dt, int(rng.integers(0, 2 ** 32)), mask)
    cols = min(vocab, 5000)
    run_noise(logits[:, :cols], dt, int(rng.integers(0, 2 ** 32)), pick(rng, FLOATS))


@pytest.mark.parametrize("case", CASES)
def test_fuzz_hadamard(case):
    rng = np.random.default_rng(9000 + case)
    rows, cols = int(rng.integers(1, 400)), 128 * int(rng.integers(1, 48))
    dt = pick(rng, [F16, F32])
    pad = int(pick(rng, [0, 0, 8, 3]))
    x = dev_normal((rows, cols + pad), 0, float(pick(rng, [1.0, 30.0])), dt, case)[:, :cols]
    mode = pick(rng, ["pre", "post", "none"])
    s = scales(cols, case + 1)
    run_had(x, dt, pre=s if mode == "pre" else None, post=s if mode == "post" else None,
            scale=float(pick(rng, [1.0, 0.5, 1.7])), what=f"fuzz had {rows}x{cols}+{pad} dt{dt} {mode}")
    n_out = int(rng.integers(1, 5))
    rot = bool(rng.random() < 0.4)
    run_norm_had(int(rng.integers(1, 300)), 128 * int(rng.integers(1, 40)), F16 if rot else pick(rng, FLOATS),
                 pick(rng, [None, F32, F16, BF16]), pick(rng, FLOATS), n_out=n_out, with_y=bool(rng.random() < 0.5),
                 cb=float(pick(rng, [0.0, 1.0])), had_scale=float(pick(rng, [1.0, 0.25])),
                 pre_none=tuple(i for i in range(n_out) if rng.random() < 0.3), seed=case + 3, rotate_x=rot,
                 svh=bool(rng.random() < 0.8))
    run_act_had(pick(rng, ["silu", "gelu", "mul_sigmoid"]), int(rng.integers(1, 300)), 128 * int(rng.integers(1, 80)),
                pick(rng, FLOATS), with_z=bool(rng.random() < 0.6), pre=bool(rng.random() < 0.8),
                ld=None if rng.random() < 0.7 else 128 * int(rng.integers(81, 90)) + int(pick(rng, [0, 8, 3])), seed=case + 5)
    rx = bool(rng.random() < 0.7)
    run_act_had_rotated(pick(rng, ["silu", "gelu", "mul_sigmoid"]), int(rng.integers(1, 200)),
                        128 * int(rng.integers(1, 60)), rx, (not rx) or bool(rng.random() < 0.6),
                        posts=bool(rng.random() < 0.8), with_z=bool(rng.random() < 0.6), seed=case + 6)


@pytest.mark.parametrize("case", CASES)
def test_fuzz_rope_had(case):
    rng = np.random.default_rng(9500 + case)
    hd = int(pick(rng, [128, 128, 128, 64, 256]))
    hq, hk = 2 * int(rng.integers(1, 20)), 2 * int(rng.integers(1, 4))
    bsz = int(rng.integers(1, 3))
    seq = int(pick(rng, [int(rng.integers(1, 64)), int(rng.integers(520, 1500))]))
    R = int(pick(rng, [hd, hd, hd // 2]))
    with_k = bool(rng.random() < 0.85)
    run_rope_had(bsz, seq, hq, hk if with_k else 0, hd, R, pick(rng, [exl3r.ROPE_NEOX, exl3r.ROPE_NEOX, exl3r.ROPE_GPTJ]),
                 nwt=pick(rng, FLOATS), norm=bool(rng.random() < 0.7), with_k=with_k, q_post=bool(rng.random() < 0.8),
                 k_post=bool(rng.random() < 0.8), position=int(rng.integers(0, 30000)),
                 out_of_place=bool(rng.random() < 0.3), seed=case)
