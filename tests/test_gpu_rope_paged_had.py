"""GPU parity of exl3r_rope_paged_kv_had: RoPE and the paged KV-cache append on the raw f16 outputs of
the q / k / v projections, each first given its projection's output rotation had_r_128(y, y, None, svh)
(src/modules.rs:231, then src/modules.rs:669-704).  Checked against the CPU oracle's composition
(oracle had_r_128 of q, k and v with their post-scales, oracle rope, oracle paged_kv_append) and bitwise
against the unfused GPU calls with the same form of the transform (exl3r_had_r_128_mfma for the 8-lane
kernel's default, exl3r_had_r_128 with EXL3R_HAD_EXACT and on the other paths, on q, k and v, then
exl3r_rope_paged_kv): q, the optional out_k, the whole k / v caches and the error flag, on the fused
launches and on the fallback, with and without post-scales and head norms, pages crossed, a bad
block-table entry, and the errors.  Against the oracle: bitwise with the butterfly, within the
matrix-core transform's tolerance carried through the head (assert_head_close) otherwise."""
import numpy as np
import pytest
import torch

import exl3r
import exl3r._lib as L
import exl3r.ffi as ffi
from _gpu import NTHREADS, assert_bitwise, assert_close_ulp, assert_head_close, dev_normal, from_dev
from oracle import oracle as orc
from test_gpu_rope import inv_freq
from test_gpu_rope_had import svh
from test_gpu_rope_paged import layout

pytestmark = pytest.mark.gpu

F16 = orc.F16


def same(a, b):
    return torch.equal(a.view(torch.int16), b.view(torch.int16))


def run(bsz, seq, hq, hk, page, max_blocks, norm=True, with_out_k=True, posts=(True, True, True), bad_entry=False,
        seed=0, exact=False, forced=False):
    """forced: a test build setting forces a kernel other than the 8-lane one (the butterfly there)."""
    hd = 128
    pages, bt, sl = layout(bsz, seq, page, max_blocks, seed)
    if bad_entry:
        bt[0, int(sl[0]) // page] = pages + 7
    q = dev_normal((bsz, seq, hq, hd), 0, 2, F16, seed)
    k = dev_normal((bsz, seq, hk, hd), 0, 2, F16, seed + 1)
    v = dev_normal((bsz, seq, hk, hd), 0, 2, F16, seed + 2)
    kc = dev_normal((pages, page, hk, hd), 0, 1, F16, seed + 3)
    vc = dev_normal((pages, page, hk, hd), 0, 1, F16, seed + 4)
    qn = dev_normal((hd,), 1, 0.1, F16, seed + 5) if norm else None
    kn = dev_normal((hd,), 1, 0.1, F16, seed + 6) if norm else None
    sq = svh(hq * hd, seed + 7) if posts[0] else None
    sk = svh(hk * hd, seed + 8) if posts[1] else None
    sv = svh(hk * hd, seed + 9) if posts[2] else None
    f = torch.from_numpy(inv_freq(hd)).cuda()
    sld = torch.from_numpy(sl.astype(np.int32)).cuda()
    btd = torch.from_numpy(bt.astype(np.int32)).cuda()
    # unfused: rotations into copies, then the paged RoPE on them
    n = bsz * seq
    ukc_in, uvc_in = kc.clone(), vc.clone()
    uq, uk, uv, ukc, uvc = q.clone(), k.clone(), v.clone(), kc.clone(), vc.clone()
    mf = not exact and not forced
    ffi.had_r_128(uq.view(n, hq * hd), uq.view(n, hq * hd), None, sq, mfma=mf)
    ffi.had_r_128(uk.view(n, hk * hd), uk.view(n, hk * hd), None, sk, mfma=mf)
    ffi.had_r_128(uv.view(n, hk * hd), uv.view(n, hk * hd), None, sv, mfma=mf)
    uerr = torch.zeros(1, dtype=torch.int32, device="cuda")
    ffi.rope_paged_kv(uq, uq, uk, uk, uv, f, 0, sld, qn, kn, 1e-6, 0.0, exl3r.ROPE_NEOX, 1.0, ukc, uvc, btd, sld,
                      err_flag=uerr)
    # fused
    oq = torch.empty_like(q)
    ok = torch.empty_like(k) if with_out_k else None
    k_in = k.clone()
    err = torch.zeros(1, dtype=torch.int32, device="cuda")
    ffi.rope_paged_kv_had(q, oq, k_in, ok, v.clone(), f, 0, sld, qn, kn, 1e-6, 0.0, exl3r.ROPE_NEOX, 1.0, kc, vc, btd,
                          sld, q_post_scale=sq, k_post_scale=sk, v_post_scale=sv, err_flag=err, exact=exact)
    torch.cuda.synchronize()
    tag = (f"paged_had b{bsz} s{seq} h{hq}/{hk} page{page} norm{int(norm)} outk{int(with_out_k)} posts{posts} "
           f"{'mfma' if mf else 'exact'}")
    # the oracle: each projection's output rotation, RoPE at the cache positions, the paged append
    def rot(t, heads, post):
        return orc.had_r_128(from_dev(t).reshape(n, heads * hd), F16, post=from_dev(post) if post is not None else None,
                             nthreads=NTHREADS).reshape(bsz, seq, heads, hd)
    eq, ek = orc.rope(rot(q, hq, sq), rot(k, hk, sk), F16, inv_freq(hd), exl3r.ROPE_NEOX, positions=sl.astype(np.int32),
                      q_norm=from_dev(qn) if norm else None, k_norm=from_dev(kn) if norm else None, nwt=F16, eps=1e-6,
                      nthreads=NTHREADS)
    ekc, evc = from_dev(ukc_in), from_dev(uvc_in)
    e_err = orc.paged_kv_append(ek, rot(v, hk, sv), F16, ekc, evc, bt, sl, nthreads=NTHREADS)
    if mf:
        assert_head_close(from_dev(oq), eq, hd, what=tag + " q vs oracle")
        if with_out_k:
            assert_head_close(from_dev(ok), ek, hd, what=tag + " out_k vs oracle")
        assert_head_close(from_dev(kc), ekc, hd, what=tag + " k_cache vs oracle")
        assert_head_close(from_dev(vc), evc, hd, what=tag + " v_cache vs oracle")
    else:
        assert_close_ulp(from_dev(oq), eq, F16, 0, what=tag + " q vs oracle")
        if with_out_k:
            assert_close_ulp(from_dev(ok), ek, F16, 0, what=tag + " out_k vs oracle")
        assert_bitwise(from_dev(kc), ekc, what=tag + " k_cache vs oracle")
        assert_bitwise(from_dev(vc), evc, what=tag + " v_cache vs oracle")
    assert int(err.item()) == e_err, tag + " err flag vs oracle"
    assert same(oq, uq), tag + " q"
    if with_out_k:
        assert same(ok, uk), tag + " out_k"
    assert same(kc, ukc), tag + " k_cache"
    assert same(vc, uvc), tag + " v_cache"
    assert int(err.item()) == int(uerr.item()) == (1 if bad_entry else 0), tag + " err flag"


@pytest.fixture
def tune():
    """Forces the RoPE kernel (0 auto, 1 never the wave-per-token kernel, 2 always) through the sweep/test
    build of the library, which the wrappers call inside the fixture."""
    with L.tuned() as lib:
        yield lambda use: lib.exl3r_tune_rope_tok(use, 0, 0)


@pytest.mark.parametrize("exact", [False, True])
def test_qwen3_32b_prefill_fused(exact):
    """64 q / 8 kv heads of 128, 2 x 1100 tokens crossing 256-token pages: the fused launch, on the matrix
    cores and (exact) as the reference's butterfly."""
    run(2, 1100, 64, 8, 256, 6, seed=1, exact=exact)


def test_default_paths_partial_passes():
    """The 8-lane kernel's default form with passes partly past the last head (5 q + 2 k + 2 v heads),
    no out_k, missing post-scales and a bad block-table entry."""
    run(1, 700, 5, 2, 64, 14, norm=False, with_out_k=False, posts=(True, False, True), seed=12)
    run(3, 300, 8, 2, 16, 24, posts=(False, True, False), bad_entry=True, seed=13)


@pytest.mark.parametrize("use", [1, 2])
def test_fused_and_fallback_paths(tune, use):
    tune(use)                     # 1: the fallback (rotations, then the paged RoPE); 2: the wave-per-token kernel
    run(1, 700, 16, 4, 64, 14, norm=False, with_out_k=False, posts=(True, False, True), seed=2, forced=True)
    run(3, 300, 8, 2, 16, 24, posts=(False, True, False), bad_entry=True, seed=3, forced=True)


def test_errors():
    f = torch.from_numpy(inv_freq(128)).cuda()
    q = dev_normal((1, 4, 2, 128), 0, 1, F16, 9)
    kc = torch.zeros((4, 16, 2, 128), dtype=torch.float16, device="cuda")
    bt = torch.zeros((1, 4), dtype=torch.int32, device="cuda")
    sl = torch.zeros(1, dtype=torch.int32, device="cuda")
    qb = q.to(torch.bfloat16)
    with pytest.raises(exl3r.Exl3rError):
        ffi.rope_paged_kv_had(qb, qb, qb, None, qb, f, 0, sl, None, None, 1e-6, 0.0, exl3r.ROPE_NEOX, 1.0,
                              kc.to(torch.bfloat16), kc.to(torch.bfloat16), bt, sl)
    q3 = dev_normal((1, 4, 3, 64), 0, 1, F16, 10)
    kc3 = torch.zeros((4, 16, 3, 64), dtype=torch.float16, device="cuda")
    with pytest.raises(exl3r.Exl3rError):
        ffi.rope_paged_kv_had(q3, q3, q3.clone(), None, q3.clone(), torch.from_numpy(inv_freq(64)).cuda(), 0, sl, None,
                              None, 1e-6, 0.0, exl3r.ROPE_NEOX, 1.0, kc3, kc3.clone(), bt, sl)
    torch.cuda.synchronize()
