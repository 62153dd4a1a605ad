"""GPU parity of exl3r_rope_had: RoPE (with the optional head RMSNorm) on the raw f16 outputs of the
q / k projections, each first given its projection's output rotation had_r_128(y, y, None, svh)
(Linear::forward, src/modules.rs:231, then RoPE::apply).  Checked bitwise against the unfused GPU calls
made with the same form of the transform (exl3r_had_r_128_mfma, or exl3r_had_r_128 with
EXL3R_HAD_EXACT and outside the 8-lane kernel, on q and k, then exl3r_rope), and against the oracle
composition (oracle_had_r_128, then oracle_rope): at RoPE's own tolerance (<= 2 ulp) for the
butterfly, within the matrix-core transform's tolerance carried through the head (assert_head_close)
otherwise.  Covers the fused launch at the Qwen3-32B prefill shape in both forms, every norm weight
dtype, missing post-scales, q without k, out of place, ragged positions, the fallback (partial NeoX
rotary, head_dim 64 and 256), GPT-J, decode sizes and the errors."""
import numpy as np
import pytest
import torch

import exl3r
import exl3r.ffi as ffi
from _gpu import NTHREADS, assert_close_ulp, assert_head_close, dev_normal, from_dev
from oracle import oracle as orc
from test_gpu_rope import inv_freq, ragged_position_ids

pytestmark = pytest.mark.gpu

F16, BF16, F32 = orc.F16, orc.BF16, orc.F32


def svh(n, seed):
    rng = np.random.default_rng(seed)
    return torch.from_numpy((np.where(rng.random(n) < 0.5, -1.0, 1.0) *
                             (1 + 0.02 * rng.standard_normal(n))).astype(np.float16)).cuda()


def nx_rotation(hd, R, mode, heads=0):
    """Whether exl3r_rope_had / exl3r_rope_paged_kv_had take the 8-lane kernel, whose default transform
    runs on the matrix cores: heads of 128, NeoX over the full width or GPT-J over a multiple of 4, at
    most 192 heads (q + k, + v with the cache) for the post-scales in LDS (16-byte aligned post-scales,
    evaluated or {cos, sin} rotations; the tests' tensors are aligned)."""
    return hd == 128 and (R == 128 if mode == exl3r.ROPE_NEOX else R % 4 == 0) and heads <= 192


def run(bsz, seq, hq, hk, hd, R, mode, nwt=F16, norm=True, with_k=True, q_post=True, k_post=True, position=0,
        position_ids=None, out_of_place=False, seed=0, exact=False):
    q = dev_normal((bsz, seq, hq, hd), 0.0, 2.0, F16, seed)
    k = dev_normal((bsz, seq, hk, hd), 0.0, 2.0, F16, seed + 1) if with_k else None
    qn = dev_normal((hd,), 1.0, 0.1, nwt, seed + 2) if norm else None
    kn = dev_normal((hd,), 1.0, 0.1, nwt, seed + 3) if norm and with_k else None
    qs = svh(hq * hd, seed + 4) if q_post else None
    ks = svh(hk * hd, seed + 5) if with_k and k_post else None
    f = inv_freq(R)
    fd = torch.from_numpy(f).cuda()
    pid_d = torch.from_numpy(position_ids).cuda() if position_ids is not None else None
    qh, kh = from_dev(q), (from_dev(k) if with_k else None)
    mf = not exact and nx_rotation(hd, R, mode, hq + (hk if with_k else 0))
    # unfused GPU reference: the output rotations (in the fused launch's form), then exl3r_rope in place
    uq = torch.empty_like(q)
    ffi.had_r_128(q.view(bsz * seq, hq * hd), uq.view(bsz * seq, hq * hd), None, qs, mfma=mf)
    uk = None
    if with_k:
        uk = torch.empty_like(k)
        ffi.had_r_128(k.view(bsz * seq, hk * hd), uk.view(bsz * seq, hk * hd), None, ks, mfma=mf)
    ffi.rope(uq, uq, uk, uk, fd, position, None, qn, kn, 1e-6, 0.0, mode, 1.0, position_ids=pid_d)
    oq = torch.empty_like(q) if out_of_place else q
    ok = (torch.empty_like(k) if out_of_place else k) if with_k else None
    ffi.rope_had(q, oq, k, ok, fd, position, None, qn, kn, 1e-6, 0.0, mode, 1.0, q_post_scale=qs, k_post_scale=ks,
                 position_ids=pid_d, exact=exact)
    torch.cuda.synchronize()
    tag = f"rope_had b{bsz} s{seq} h{hq}/{hk} d{hd} R{R} mode{mode} w{nwt if norm else '-'} {'mfma' if mf else 'exact'}"
    assert torch.equal(oq.view(torch.int16), uq.view(torch.int16)), tag + " q vs unfused"
    if with_k:
        assert torch.equal(ok.view(torch.int16), uk.view(torch.int16)), tag + " k vs unfused"
    if out_of_place:
        assert np.array_equal(from_dev(q), qh), tag + " q must not be written"
    # oracle composition
    n = bsz * seq
    rq = orc.had_r_128(np.ascontiguousarray(qh.reshape(n, hq * hd)), F16,
                       post=from_dev(qs) if qs is not None else None, nthreads=NTHREADS).reshape(qh.shape)
    rk = orc.had_r_128(np.ascontiguousarray(kh.reshape(n, hk * hd)), F16,
                       post=from_dev(ks) if ks is not None else None, nthreads=NTHREADS).reshape(kh.shape) \
        if with_k else None
    eq, ek = orc.rope(rq, rk, F16, f, mode, position=position,
                      position_ids=position_ids.reshape(-1) if position_ids is not None else None,
                      q_norm=from_dev(qn) if norm else None, k_norm=from_dev(kn) if kn is not None else None,
                      nwt=nwt, eps=1e-6, nthreads=NTHREADS)
    if mf:
        assert_head_close(from_dev(oq), eq, hd, what=tag + " q vs oracle")
        if with_k:
            assert_head_close(from_dev(ok), ek, hd, what=tag + " k vs oracle")
    else:
        assert_close_ulp(from_dev(oq), eq, F16, 2, what=tag + " q vs oracle")
        if with_k:
            assert_close_ulp(from_dev(ok), ek, F16, 2, what=tag + " k vs oracle")


@pytest.mark.parametrize("exact", [False, True])
def test_qwen3_32b_prefill_fused(exact):
    """64 q / 8 kv heads of 128, 2048 tokens, f16 head norm: the fused launch, on the matrix cores and
    (exact) as the reference's butterfly."""
    run(1, 2048, 64, 8, 128, 128, exl3r.ROPE_NEOX, position=17, seed=1, exact=exact)


@pytest.mark.parametrize("exact", [False, True])
def test_ragged_positions_out_of_place(exact):
    pid = ragged_position_ids(3)
    run(1, pid.size, 32, 4, 128, 128, exl3r.ROPE_NEOX, nwt=F32, position_ids=pid[None, :], out_of_place=True, seed=2,
        exact=exact)


@pytest.mark.parametrize("nwt,norm", [(BF16, True), (F16, False)])
def test_norm_kinds_and_missing_post_scales(nwt, norm):
    run(2, 600, 8, 2, 128, 128, exl3r.ROPE_NEOX, nwt=nwt, norm=norm, q_post=False, position=1000, seed=3)


def test_q_only_and_partial_rotary():
    run(1, 1100, 12, 0, 128, 64, exl3r.ROPE_NEOX, with_k=False, seed=4)


def test_odd_head_counts():
    """Passes whose 8 heads are partly past the end (5 q + 1 k heads: the lanes of heads 6 and 7 repeat
    head 5), and q heads ending inside a 4-head span of the matrix-core placement."""
    run(3, 333, 5, 1, 128, 128, exl3r.ROPE_NEOX, position=3, seed=11)
    run(1, 700, 6, 0, 128, 128, exl3r.ROPE_NEOX, with_k=False, nwt=F32, seed=12)


def test_head_counts_at_the_post_scale_bound():
    """192 heads: the 8-lane kernel with every post-scale in LDS (48 KB, lower occupancy); 200 heads: the
    wave-per-token kernel and its butterfly."""
    run(1, 96, 184, 8, 128, 128, exl3r.ROPE_NEOX, position=9, seed=13)
    run(1, 96, 192, 8, 128, 128, exl3r.ROPE_NEOX, position=9, seed=14)


@pytest.mark.parametrize("case", ["decode", "gptj", "gptj_exact", "hd64", "hd256"])
def test_fallback_shapes(case):
    if case == "decode":
        run(64, 1, 64, 8, 128, 128, exl3r.ROPE_NEOX, position=4000, seed=5)
    elif case.startswith("gptj"):
        run(1, 1200, 8, 2, 128, 64, exl3r.ROPE_GPTJ, seed=6, exact=case == "gptj_exact")
    elif case == "hd64":
        run(1, 1200, 8, 2, 64, 64, exl3r.ROPE_NEOX, out_of_place=True, seed=7)
    else:
        run(2, 300, 4, 1, 256, 256, exl3r.ROPE_NEOX, seed=8)


def test_zero_tokens_and_errors():
    f = torch.from_numpy(inv_freq(128)).cuda()
    z = torch.empty((1, 0, 4, 128), device="cuda", dtype=torch.float16)
    ffi.rope_had(z, z, None, None, f, 0, None, None, None, 1e-6, 0.0, exl3r.ROPE_NEOX, 1.0)
    qb = dev_normal((1, 4, 4, 128), 0, 1, BF16, 9)
    with pytest.raises(exl3r.Exl3rError):
        ffi.rope_had(qb, qb, None, None, f, 0, None, None, None, 1e-6, 0.0, exl3r.ROPE_NEOX, 1.0)
    q3 = dev_normal((1, 4, 3, 64), 0, 1, F16, 10)                 # 3 * 64 columns: not whole blocks
    with pytest.raises(exl3r.Exl3rError):
        ffi.rope_had(q3, q3, None, None, torch.from_numpy(inv_freq(64)).cuda(), 0, None, None, None, 1e-6, 0.0,
                     exl3r.ROPE_NEOX, 1.0)
    torch.cuda.synchronize()
