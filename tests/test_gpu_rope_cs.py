"""GPU parity of exl3r_rope_cs_table + exl3r_rope_cs: RoPE (with the optional head RMSNorm) whose
per-layer sin / cos evaluation (kernels/rope.cu:69-85) is hoisted into one {cos, sin} table per forward
pass.  exl3r_rope_cs is checked against the CPU oracle's rope (<= 2 ulp, the RoPE bound; the oracle
evaluates cos / sin itself, in double, of the same fp32 angles) and bit for bit against exl3r_rope on the
same inputs, on every kernel it shares with it: the wave-per-token prefill kernel (NeoX,
f16 and bf16), the flattened kernel (decode, GPT-J, head_dim 64 / 256) and the generic one (head_dim
not a multiple of 8), with each position source, attn_factor, q without k, out of place and batches.
The table itself is checked against the closed form: fl32(cos / sin of the fp32 angle
fl32(inv_freq[t] * pos)) * attn_factor, to <= 1 ulp of fp32, and bitwise on exactly representable
angles (pos 0)."""
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
    return torch.equal(a.view(torch.int16), b.view(torch.int16))


def run(bsz, seq, hq, hk, hd, R, mode, dt, nwt=None, position=0, positions=None, position_ids=None, attn=1.0,
        with_k=True, out_of_place=False, seed=0):
    q = dev_normal((bsz, seq, hq, hd), 0.0, 1.0, dt, seed)
    k = dev_normal((bsz, seq, hk, hd), 0.0, 1.0, dt, seed + 1) if with_k else None
    qn = dev_normal((hd,), 1.0, 0.1, nwt, seed + 2) if nwt is not None else None
    kn = dev_normal((hd,), 1.0, 0.1, nwt, seed + 3) if nwt is not None and with_k else None
    f = torch.from_numpy(inv_freq(R)).cuda()
    pos_d = torch.from_numpy(positions).cuda() if positions is not None else None
    pid_d = torch.from_numpy(position_ids).cuda() if position_ids is not None else None
    eq, ek = q.clone(), (k.clone() if with_k else None)
    ffi.rope(eq, eq, ek, ek, f, position, pos_d, qn, kn, 1e-6, 0.0, mode, attn, position_ids=pid_d)
    cs = ffi.rope_cs_table(bsz, seq, f, position, pos_d, pid_d, attn)
    oq = torch.empty_like(q) if out_of_place else q
    ok = (torch.empty_like(k) if out_of_place else k) if with_k else None
    qh = from_dev(q)
    kh = from_dev(k) if with_k else None
    ffi.rope_cs(q, oq, k, ok, cs, qn, kn, 1e-6, 0.0, mode)
    torch.cuda.synchronize()
    tag = f"rope_cs b{bsz} s{seq} h{hq}/{hk} d{hd} R{R} mode{mode} {dt} w{nwt}"
    eq_o, ek_o = orc.rope(qh, kh, dt, inv_freq(R), mode, position=position, positions=positions,
                          position_ids=position_ids.reshape(-1) if position_ids is not None else None,
                          q_norm=from_dev(qn) if qn is not None else None, k_norm=from_dev(kn) if kn is not None else None,
                          nwt=nwt if nwt is not None else F16, eps=1e-6, attn=attn, nthreads=NTHREADS)
    assert_close_ulp(from_dev(oq), eq_o, dt, 2, what=tag + " q vs oracle")
    if with_k:
        assert_close_ulp(from_dev(ok), ek_o, dt, 2, what=tag + " k vs oracle")
    assert same(oq, eq), tag + " q vs exl3r_rope"
    if with_k:
        assert same(ok, ek), tag + " k vs exl3r_rope"
    if out_of_place:
        assert np.array_equal(from_dev(q), qh), tag + " q must not be written"
    return cs


def token_positions(bsz, seq, position, positions, position_ids):
    if position_ids is not None:
        return position_ids.reshape(-1).astype(np.int64)
    base = positions.astype(np.int64) if positions is not None else np.full(bsz, position, np.int64)
    return (base[:, None] + np.arange(seq)[None, :]).reshape(-1)


def test_c4_prefill_wave_per_token():
    """Config 4's ragged prefill (~4.6k tokens, positions up to ~33k), 64 q / 8 kv heads of 128, NeoX."""
    pid = ragged_position_ids(0)[None, :]
    run(1, pid.size, 64, 8, 128, 128, exl3r.ROPE_NEOX, F16, nwt=F16, position_ids=pid, seed=1)
    run(1, pid.size, 64, 8, 128, 128, exl3r.ROPE_NEOX, BF16, nwt=BF16, position_ids=pid, seed=2)


def test_table_closed_form():
    """cos / sin of the fp32 angle evaluated in fp64 and rounded once, times attn_factor: within 1 ulp of
    numpy's double-precision cos / sin of the same fp32 angle rounded to fp32 (the kernel's own fp64
    evaluation may sit on the other side of a rounding boundary), bitwise at position 0."""
    bsz, seq, R, attn = 3, 700, 128, 0.75
    positions = np.array([0, 5000, 31000], np.int32)
    cs = from_dev(run(bsz, seq, 8, 2, 128, R, exl3r.ROPE_NEOX, F16, nwt=F32, positions=positions, attn=attn,
                      seed=3))
    pos = token_positions(bsz, seq, 0, positions, None)
    f = inv_freq(R)
    ang = (f[None, :] * pos[:, None].astype(np.float32)).astype(np.float32)
    ec = (np.cos(ang.astype(np.float64)).astype(np.float32) * np.float32(attn)).astype(np.float32)
    es = (np.sin(ang.astype(np.float64)).astype(np.float32) * np.float32(attn)).astype(np.float32)
    for got, exp, what in ((cs[..., 0], ec, "cos"), (cs[..., 1], es, "sin")):
        ulp = np.abs(got.view(np.int32).astype(np.int64) - exp.view(np.int32).astype(np.int64))
        sign_ok = (np.sign(got) == np.sign(exp)) | (got == 0) | (exp == 0)
        assert sign_ok.all() and ulp[got != 0].max() <= 1, what
        assert np.array_equal(got[0], exp[0]), what + " at position 0"
    assert np.array_equal(cs[0, :, 0], np.full(R // 2, attn, np.float32))


@pytest.mark.parametrize("case", ["decode", "gptj", "hd64", "hd256", "generic", "q_only", "position"])
def test_flattened_and_generic_kernels(case):
    if case == "decode":          # 64 sequences x 1 token at per-sequence positions: the flattened kernel
        pos = np.random.default_rng(4).integers(0, 40000, 64).astype(np.int32)
        run(64, 1, 64, 8, 128, 128, exl3r.ROPE_NEOX, F16, nwt=F16, positions=pos, seed=4)
    elif case == "gptj":
        pid = ragged_position_ids(5)[None, :]
        run(1, pid.size, 16, 4, 128, 64, exl3r.ROPE_GPTJ, BF16, nwt=F32, position_ids=pid, seed=5)
    elif case == "hd64":
        run(2, 600, 8, 2, 64, 64, exl3r.ROPE_NEOX, F16, nwt=F16, position=123, out_of_place=True, seed=6)
    elif case == "hd256":
        run(2, 300, 4, 1, 256, 128, exl3r.ROPE_NEOX, BF16, position=7, seed=7)
    elif case == "generic":       # head_dim 100: not 8-element lane chunks
        run(2, 50, 4, 2, 100, 100, exl3r.ROPE_NEOX, F16, nwt=F16, position=9, seed=8)
    elif case == "q_only":
        run(1, 1500, 12, 0, 128, 128, exl3r.ROPE_NEOX, F16, with_k=False, position=3, attn=1.25, seed=9)
    else:
        run(4, 1100, 8, 8, 128, 128, exl3r.ROPE_NEOX, F16, nwt=BF16, position=20000, seed=10)


def test_zero_tokens_and_errors():
    f = torch.from_numpy(inv_freq(128)).cuda()
    z = torch.empty((1, 0, 4, 128), device="cuda", dtype=torch.float16)
    cs0 = ffi.rope_cs_table(1, 0, f, 0)
    assert cs0.shape == (0, 64, 2)
    ffi.rope_cs(z, z, None, None, cs0, None, None, 1e-6, 0.0, exl3r.ROPE_NEOX)
    q = dev_normal((1, 4, 4, 128), 0, 1, F16, 11)
    cs = ffi.rope_cs_table(1, 4, f, 0)
    with pytest.raises(ValueError):                                 # table of another token count
        ffi.rope_cs(q, q, None, None, cs[:3], None, None, 1e-6, 0.0, exl3r.ROPE_NEOX)
    with pytest.raises(exl3r.Exl3rError):                           # rotary_dim beyond head_dim
        q64 = dev_normal((1, 4, 4, 64), 0, 1, F16, 12)
        ffi.rope_cs(q64, q64, None, None, cs, None, None, 1e-6, 0.0, exl3r.ROPE_NEOX)
    torch.cuda.synchronize()


def paged_case(bsz, seq, hq, hk, page, max_blocks, had, tune_use=0, seed=0):
    """exl3r_rope_paged_kv / exl3r_rope_paged_kv_had with a {cos, sin} table against the same call evaluating
    sin / cos: q, out_k, both whole caches and the error flag bitwise."""
    import exl3r._lib as L
    from test_gpu_rope_paged import layout
    from test_gpu_rope_had import svh
    hd = 128
    pages, bt, sl = layout(bsz, seq, page, max_blocks, seed)
    q = dev_normal((bsz, seq, hq, hd), 0, 2, F16, seed)
    k = dev_normal((bsz, seq, hk, hd), 0, 2, F16, seed + 1)
    v = dev_normal((bsz, seq, hk, hd), 0, 2, F16, seed + 2)
    kc = dev_normal((pages, page, hk, hd), 0, 1, F16, seed + 3)
    vc = dev_normal((pages, page, hk, hd), 0, 1, F16, seed + 4)
    qn = dev_normal((hd,), 1, 0.1, F16, seed + 5)
    kn = dev_normal((hd,), 1, 0.1, F16, seed + 6)
    f = torch.from_numpy(inv_freq(hd)).cuda()
    sld = torch.from_numpy(sl.astype(np.int32)).cuda()
    btd = torch.from_numpy(bt.astype(np.int32)).cuda()
    cs = ffi.rope_cs_table(bsz, seq, f, 0, sld)
    posts = dict(q_post_scale=svh(hq * hd, seed + 7), k_post_scale=svh(hk * hd, seed + 8),
                 v_post_scale=svh(hk * hd, seed + 9)) if had else {}
    outs = []
    with L.tuned() as lib:
        lib.exl3r_tune_rope_tok(tune_use, 0, 0)
        for table in (None, cs):
            oq, ok, vv, kcc, vcc = torch.empty_like(q), torch.empty_like(k), v.clone(), kc.clone(), vc.clone()
            err = torch.zeros(1, dtype=torch.int32, device="cuda")
            fn = ffi.rope_paged_kv_had if had else ffi.rope_paged_kv
            fn(q, oq, k.clone(), ok, vv, f if table is None else None, 0, sld, qn, kn, 1e-6, 0.0, exl3r.ROPE_NEOX, 1.0,
               kcc, vcc, btd, sld, err_flag=err, cs_table=table, **posts)
            outs.append((oq, ok, kcc, vcc, err))
        torch.cuda.synchronize()
    tag = f"paged{'_had' if had else ''} cs b{bsz} s{seq} h{hq}/{hk} use{tune_use}"
    for a, b, what in zip(outs[0], outs[1], ("q", "out_k", "k_cache", "v_cache", "err")):
        assert same(a, b) if a.dtype == torch.float16 else torch.equal(a, b), tag + " " + what


@pytest.mark.parametrize("had", [False, True])
@pytest.mark.parametrize("use", [0, 1])
def test_paged_append_with_table(had, use):
    """The wave-per-token kernel (prefill, 2 x 1100 tokens crossing 256-token pages; with the output rotation
    of q / k / v when `had`), and with use=1 the flattened kernel / the rotations followed by the paged RoPE."""
    paged_case(2, 1100, 16, 4, 256, 6, had, tune_use=use, seed=21 + had + 2 * use)


def test_paged_append_with_table_decode():
    paged_case(16, 1, 32, 8, 16, 64, False, seed=25)


@pytest.mark.parametrize("tok", [True, False])
def test_rope_had_with_table(tok):
    """exl3r_rope_had with a {cos, sin} table against the same call evaluating sin / cos: the fused launch
    (1100 tokens) and the fallback (the rotations, then exl3r_rope_cs)."""
    from test_gpu_rope_had import svh
    bsz, seq, hq, hk, hd = (1, 1100, 16, 4, 128) if tok else (8, 1, 16, 4, 128)
    q = dev_normal((bsz, seq, hq, hd), 0, 2, F16, 30)
    k = dev_normal((bsz, seq, hk, hd), 0, 2, F16, 31)
    qn = dev_normal((hd,), 1, 0.1, BF16, 32)
    kn = dev_normal((hd,), 1, 0.1, BF16, 33)
    qs, ks = svh(hq * hd, 34), svh(hk * hd, 35)
    f = torch.from_numpy(inv_freq(hd)).cuda()
    pos = torch.from_numpy(np.arange(bsz, dtype=np.int32) * 977 + 5).cuda()
    cs = ffi.rope_cs_table(bsz, seq, f, 0, pos)
    res = []
    for table in (None, cs):
        oq, ok = torch.empty_like(q), torch.empty_like(k)
        ffi.rope_had(q, oq, k, ok, f, 0, pos, qn, kn, 1e-6, 0.0, exl3r.ROPE_NEOX, 1.0, q_post_scale=qs, k_post_scale=ks,
                     cs_table=table)
        res.append((oq, ok))
    torch.cuda.synchronize()
    assert same(res[0][0], res[1][0]) and same(res[0][1], res[1][1]), f"rope_had cs tok={tok}"
