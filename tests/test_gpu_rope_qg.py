"""GPU parity of exl3r_rope_qg: gated attention's q | g split (exl3r_deinterleave_qg, src/modules.rs:637-646)
and the q / k head-norm + RoPE that follows (src/modules.rs:669-681) in one pass, q read straight from the
interleaved projection output and written dense.  Checked against the CPU oracle's composition
(oracle deinterleave_qg, then oracle rope on its q: <= 2 ulp, the RoPE bound), and bit for bit against
exl3r_deinterleave_qg then exl3r_rope, with qg left unwritten, and the output
gate read in place from qg (exl3r_mul_sigmoid with a 2 * head_dim row stride) against the gate from the
deinterleave.  Covers the wave-per-token prefill kernel (f16 and bf16, head_dim 128 and 256 with partial
rotary), decode-sized launches, GPT-J, a strided qg, the generic kernel, and the errors."""
import numpy as np
import pytest
import torch

import exl3r
import exl3r.ffi as ffi
from _gpu import NTHREADS, assert_close_ulp, dev_normal, from_dev
from oracle import oracle as orc
from test_gpu_rope import inv_freq, ragged_position_ids

pytestmark = pytest.mark.gpu

F16, BF16, F32 = orc.F16, orc.BF16, orc.F32


def same(a, b):
    return torch.equal(a.contiguous().view(torch.int16), b.contiguous().view(torch.int16))


def run(bsz, seq, hq, hk, hd, R, mode, dt, nwt=None, cb=0.0, position=0, positions=None, position_ids=None, pad=0,
        seed=0):
    qg_full = dev_normal((bsz, seq, hq * 2 * hd + pad), 0.0, 1.0, dt, seed)
    qg = qg_full[..., :hq * 2 * hd].view(bsz, seq, hq, 2 * hd) if pad else qg_full.view(bsz, seq, hq, 2 * hd)
    k = dev_normal((bsz, seq, hk, hd), 0.0, 1.0, dt, seed + 1)
    qn = dev_normal((hd,), 1.0, 0.1, nwt, seed + 2) if nwt is not None else None
    kn = dev_normal((hd,), 1.0, 0.1, nwt, seed + 3) if nwt is not None else None
    f = torch.from_numpy(inv_freq(R)).cuda()
    pos_d = torch.from_numpy(positions).cuda() if positions is not None else None
    pid_d = torch.from_numpy(position_ids).cuda() if position_ids is not None else None
    before = from_dev(qg_full).copy()
    kh = from_dev(k)
    # reference: the split, then RoPE in place on the dense q
    q = torch.empty((bsz, seq, hq, hd), device="cuda", dtype=qg.dtype)
    g = torch.empty((bsz, seq, hq * hd), device="cuda", dtype=qg.dtype)
    ffi.deinterleave_qg(qg.reshape(bsz, seq, hq * 2 * hd) if not pad else qg_full[..., :hq * 2 * hd], q, g, hd)
    ek = k.clone()
    ffi.rope(q, q, ek, ek, f, position, pos_d, qn, kn, 1e-6, cb, mode, 1.0, position_ids=pid_d)
    # fused
    oq = torch.empty((bsz, seq, hq, hd), device="cuda", dtype=qg.dtype)
    ok = k.clone()
    ffi.rope_qg(qg, oq, ok, ok, f, position, pos_d, qn, kn, 1e-6, cb, mode, 1.0, position_ids=pid_d)
    torch.cuda.synchronize()
    tag = f"rope_qg b{bsz} s{seq} h{hq}/{hk} d{hd} R{R} mode{mode} {dt} w{nwt} pad{pad}"
    # the oracle: split the interleaved rows, then rope the q half (and k)
    oq_h, _ = orc.deinterleave_qg(np.ascontiguousarray(before.reshape(bsz * seq, -1)[:, :hq * 2 * hd]), hq, hd,
                                  nthreads=NTHREADS)
    eq_o, ek_o = orc.rope(oq_h.reshape(bsz, seq, hq, hd), kh, dt, inv_freq(R), mode, position=position,
                          positions=positions,
                          position_ids=position_ids.reshape(-1) if position_ids is not None else None,
                          q_norm=from_dev(qn) if qn is not None else None,
                          k_norm=from_dev(kn) if kn is not None else None,
                          nwt=nwt if nwt is not None else F16, eps=1e-6, cb=cb, nthreads=NTHREADS)
    assert_close_ulp(from_dev(oq), eq_o, dt, 2, what=tag + " q vs oracle")
    assert_close_ulp(from_dev(ok), ek_o, dt, 2, what=tag + " k vs oracle")
    assert same(oq, q), tag + " q vs deinterleave + rope"
    assert same(ok, ek), tag + " k vs rope"
    assert np.array_equal(from_dev(qg_full), before), tag + " qg must not be written"
    # the output gate read in place from qg
    if not pad:
        n = bsz * seq * hq
        o = dev_normal((n, hd), 0.0, 1.0, dt, seed + 4)
        z_ref, z = torch.empty_like(o), torch.empty_like(o)
        ffi.mul_sigmoid(o, g.view(n, hd), z_ref)
        ffi.mul_sigmoid(o, qg.reshape(n, 2 * hd)[:, hd:], z)
        torch.cuda.synchronize()
        assert same(z, z_ref), tag + " gate from qg"


def test_qwen35_prefill():
    """2048 tokens, 32 q heads of 128 (q | g = 256 per head), 4 kv heads, f16 head norm with bias 1."""
    run(1, 2048, 32, 4, 128, 128, exl3r.ROPE_NEOX, F16, nwt=F16, cb=1.0, position=11, seed=1)


def test_partial_rotary_hd256_ragged_bf16():
    pid = ragged_position_ids(2)[None, :]
    run(1, pid.size, 16, 2, 256, 64, exl3r.ROPE_NEOX, BF16, nwt=BF16, cb=1.0, position_ids=pid, seed=2)


@pytest.mark.parametrize("case", ["decode", "gptj", "strided", "generic", "no_norm"])
def test_other_kernels(case):
    if case == "decode":
        pos = np.random.default_rng(3).integers(0, 40000, 64).astype(np.int32)
        run(64, 1, 32, 4, 128, 128, exl3r.ROPE_NEOX, F16, nwt=F16, positions=pos, seed=3)
    elif case == "gptj":
        run(2, 700, 8, 2, 128, 64, exl3r.ROPE_GPTJ, BF16, nwt=F32, position=5, seed=4)
    elif case == "strided":          # a padded projection row: qg token stride beyond heads * 2 * head_dim
        run(1, 1300, 8, 2, 128, 128, exl3r.ROPE_NEOX, F16, nwt=F16, position=7, pad=64, seed=5)
    elif case == "generic":          # head_dim 100: the generic kernel
        run(2, 40, 4, 2, 100, 100, exl3r.ROPE_NEOX, F16, nwt=F16, position=9, seed=6)
    else:
        run(1, 1500, 16, 4, 128, 128, exl3r.ROPE_NEOX, F16, position=100, seed=7)


def test_errors():
    f = torch.from_numpy(inv_freq(128)).cuda()
    qg = dev_normal((1, 4, 4, 256), 0, 1, F16, 8)
    with pytest.raises(exl3r.Exl3rError):                      # out_q inside qg
        inside = torch.as_strided(qg, (1, 4, 4, 128), (2048, 512, 128, 1))
        ffi.rope_qg(qg, inside, None, None, f, 0, None, None, None, 1e-6, 0.0, exl3r.ROPE_NEOX, 1.0)
    with pytest.raises(ValueError):                             # out_q not (.., heads, head_dim)
        ffi.rope_qg(qg, torch.empty((1, 4, 4, 256), device="cuda", dtype=torch.float16), None, None, f, 0, None,
                    None, None, 1e-6, 0.0, exl3r.ROPE_NEOX, 1.0)
    z = torch.empty((1, 0, 4, 256), device="cuda", dtype=torch.float16)
    ffi.rope_qg(z, torch.empty((1, 0, 4, 128), device="cuda", dtype=torch.float16), None, None, f, 0, None, None,
                None, 1e-6, 0.0, exl3r.ROPE_NEOX, 1.0)
    torch.cuda.synchronize()
