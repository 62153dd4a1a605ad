"""GPU check of exl3r_rope_run: each variant reached through the descriptor is bit-identical to its
own entry point on the same inputs -- plain, the {cos, sin} table, an angle table, the gated q | g split,
the output rotations, the paged append, and both together.  (The entry points themselves are checked
against the CPU oracle in their own test files.)"""
import numpy as np
import pytest
import torch

import exl3r
import exl3r.ffi as ffi
from _gpu import dev_normal
from oracle import oracle as orc
from test_gpu_rope import inv_freq
from test_gpu_rope_had import svh
from test_gpu_rope_paged import layout

pytestmark = pytest.mark.gpu

F16, BF16 = orc.F16, orc.BF16
NEOX, GPTJ = exl3r.ROPE_NEOX, exl3r.ROPE_GPTJ


def same(a, b):
    return torch.equal(a.contiguous().view(torch.int16), b.contiguous().view(torch.int16))


def common(q, k, hd, R, mode, qn, kn, attn=1.0):
    bsz, seq, hq, _ = q.shape
    return dict(dtype=exl3r.F16 if q.dtype == torch.float16 else exl3r.BF16, bsz=bsz, seq_len=seq, head_dim=hd,
                rotary_dim=R, rope_mode=mode, attn_factor=attn, q_tok_stride=q.stride(1), q_head_stride=q.stride(2),
                num_heads_q=hq, num_heads_k=k.shape[2] if k is not None else 0,
                k_tok_stride=k.stride(1) if k is not None else 0, k_head_stride=k.stride(2) if k is not None else 0,
                q_norm=qn, k_norm=kn, norm_dtype=exl3r.F16, norm_eps=1e-6,
                norm_constant_bias=0.0)


@pytest.mark.parametrize("bsz,seq,mode,R,dt", [(1, 1100, NEOX, 128, F16), (3, 40, GPTJ, 64, BF16), (64, 1, NEOX, 128, F16)])
def test_plain_and_cs(bsz, seq, mode, R, dt):
    hq, hk, hd = 16, 4, 128
    q, k = dev_normal((bsz, seq, hq, hd), 0, 1, dt, 1), dev_normal((bsz, seq, hk, hd), 0, 1, dt, 2)
    qn, kn = dev_normal((hd,), 1, 0.1, F16, 3), dev_normal((hd,), 1, 0.1, F16, 4)
    f = torch.from_numpy(inv_freq(R)).cuda()
    pos = torch.from_numpy(np.random.default_rng(5).integers(0, 30000, bsz).astype(np.int32)).cuda()
    q1, k1, q2, k2 = q.clone(), k.clone(), q.clone(), k.clone()
    ffi.rope(q1, q1, k1, k1, f, 0, pos, qn, kn, 1e-6, 0.0, mode, 0.9)
    ffi.rope_run(q=q2, out_q=q2, k=k2, out_k=k2, inv_freq=f, positions=pos, **common(q, k, hd, R, mode, qn, kn, 0.9))
    torch.cuda.synchronize()
    assert same(q1, q2) and same(k1, k2)
    cs = ffi.rope_cs_table(bsz, seq, f, 0, pos, None, 0.9)
    q3, k3, q4, k4 = q.clone(), k.clone(), q.clone(), k.clone()
    ffi.rope_cs(q3, q3, k3, k3, cs, qn, kn, 1e-6, 0.0, mode)
    ffi.rope_run(q=q4, out_q=q4, k=k4, out_k=k4, cs_table=cs, **common(q, k, hd, R, mode, qn, kn, 0.9))
    torch.cuda.synchronize()
    assert same(q3, q4) and same(k3, k4)
    assert same(q1, q3)     # the table reproduces the evaluated pairs


def test_angle_table_and_qg():
    bsz, seq, hq, hk, hd = 2, 50, 8, 2, 128
    q, k = dev_normal((bsz, seq, hq, hd), 0, 1, F16, 11), dev_normal((bsz, seq, hk, hd), 0, 1, F16, 12)
    qn, kn = dev_normal((hd,), 1, 0.1, F16, 13), dev_normal((hd,), 1, 0.1, F16, 14)
    table = torch.from_numpy((np.arange(200, dtype=np.float32)[:, None] * inv_freq(hd)[None, :]).astype(np.float32)).cuda()
    pos = torch.tensor([3, 100], dtype=torch.int32, device="cuda")
    q1, k1, q2, k2 = q.clone(), k.clone(), q.clone(), k.clone()
    ffi.rope(q1, q1, k1, k1, table, 0, pos, qn, kn, 1e-6, 0.0, NEOX, 1.0)
    ffi.rope_run(q=q2, out_q=q2, k=k2, out_k=k2, angle_table=table, table_rows=200, table_batch_stride=0, positions=pos,
                 **common(q, k, hd, hd, NEOX, qn, kn))
    torch.cuda.synchronize()
    assert same(q1, q2) and same(k1, k2)
    # the gated q | g split: q read from the q halves of qg, written dense
    qg = dev_normal((bsz, seq, hq, 2 * hd), 0, 1, F16, 15)
    f = torch.from_numpy(inv_freq(hd)).cuda()
    o1, o2 = torch.empty((bsz, seq, hq, hd), device="cuda", dtype=torch.float16), torch.empty((bsz, seq, hq, hd), device="cuda", dtype=torch.float16)
    k3, k4 = k.clone(), k.clone()
    ffi.rope_qg(qg, o1, k3, k3, f, 7, None, qn, kn, 1e-6, 0.0, NEOX, 1.0)
    c = common(qg, k, hd, hd, NEOX, qn, kn)
    ffi.rope_run(q=qg, out_q=o2, out_q_tok_stride=hq * hd, out_q_head_stride=hd, k=k4, out_k=k4, inv_freq=f, position=7, **c)
    torch.cuda.synchronize()
    assert same(o1, o2) and same(k3, k4)


@pytest.mark.parametrize("tokens", [1100, 40])
def test_rotations_and_paged(tokens):
    bsz, seq = (1, tokens) if tokens > 100 else (2, tokens // 2)
    hq, hk, hd, page, mb = 16, 4, 128, 64, 24
    q, k, v = (dev_normal((bsz, seq, h, hd), 0, 2, F16, s) for h, s in ((hq, 21), (hk, 22), (hk, 23)))
    qn, kn = dev_normal((hd,), 1, 0.1, F16, 24), dev_normal((hd,), 1, 0.1, F16, 25)
    sq, sk, sv = svh(hq * hd, 26), svh(hk * hd, 27), svh(hk * hd, 28)
    f = torch.from_numpy(inv_freq(hd)).cuda()
    pages, bt, sl = layout(bsz, seq, page, mb, 29)
    btd, sld = torch.from_numpy(bt).cuda(), torch.from_numpy(sl).cuda()
    # the output rotations alone
    o1, o2, ok1, ok2 = (torch.empty_like(t) for t in (q, q, k, k))
    ffi.rope_had(q, o1, k, ok1, f, 0, sld, qn, kn, 1e-6, 0.0, NEOX, 1.0, q_post_scale=sq, k_post_scale=sk)
    c = common(q, k, hd, hd, NEOX, qn, kn)
    ffi.rope_run(q=q, out_q=o2, k=k, out_k=ok2, inv_freq=f, positions=sld, rotate=1, q_post_scale=sq, k_post_scale=sk, **c)
    torch.cuda.synchronize()
    assert same(o1, o2) and same(ok1, ok2)
    # the reference's butterfly: EXL3R_HAD_EXACT in rotate
    ffi.rope_had(q, o1, k, ok1, f, 0, sld, qn, kn, 1e-6, 0.0, NEOX, 1.0, q_post_scale=sq, k_post_scale=sk, exact=True)
    ffi.rope_run(q=q, out_q=o2, k=k, out_k=ok2, inv_freq=f, positions=sld, rotate=1 | ffi.HAD_EXACT, q_post_scale=sq,
                 k_post_scale=sk, **c)
    torch.cuda.synchronize()
    assert same(o1, o2) and same(ok1, ok2), "rotate | EXL3R_HAD_EXACT"
    # the paged append, then with the rotations
    for rotate in (0, 1):
        kc1, vc1 = dev_normal((pages, page, hk, hd), 0, 1, F16, 30), dev_normal((pages, page, hk, hd), 0, 1, F16, 31)
        kc2, vc2 = kc1.clone(), vc1.clone()
        qa, ka, qb, kb = q.clone(), k.clone(), q.clone(), k.clone()
        e1, e2 = torch.zeros(1, dtype=torch.int32, device="cuda"), torch.zeros(1, dtype=torch.int32, device="cuda")
        if rotate:
            ffi.rope_paged_kv_had(q, qa, k.clone(), ka, v.clone(), f, 0, sld, qn, kn, 1e-6, 0.0, NEOX, 1.0, kc1, vc1,
                                  btd, sld, q_post_scale=sq, k_post_scale=sk, v_post_scale=sv, err_flag=e1)
            ffi.rope_run(q=q, out_q=qb, k=k.clone(), out_k=kb, v=v.clone(), v_tok_stride=v.stride(1),
                         v_head_stride=v.stride(2), inv_freq=f, positions=sld, rotate=1, q_post_scale=sq,
                         k_post_scale=sk, v_post_scale=sv, k_cache=kc2, v_cache=vc2, page_size=page,
                         num_pages=pages, block_table=btd, max_blocks_per_seq=mb, cache_seqlens=sld, err_flag=e2, **c)
        else:
            ffi.rope_paged_kv(qa, qa, ka, ka, v, f, 0, sld, qn, kn, 1e-6, 0.0, NEOX, 1.0, kc1, vc1, btd, sld, err_flag=e1)
            ffi.rope_run(q=qb, out_q=qb, k=kb, out_k=kb, v=v, v_tok_stride=v.stride(1), v_head_stride=v.stride(2),
                         inv_freq=f, positions=sld, k_cache=kc2, v_cache=vc2, page_size=page, num_pages=pages,
                         block_table=btd, max_blocks_per_seq=mb, cache_seqlens=sld, err_flag=e2, **c)
        torch.cuda.synchronize()
        tag = f"paged rotate={rotate} tokens={tokens}"
        assert same(qa, qb) and same(ka, kb), tag
        assert same(kc1, kc2) and same(vc1, vc2), tag
        assert int(e1.item()) == int(e2.item()) == 0, tag
