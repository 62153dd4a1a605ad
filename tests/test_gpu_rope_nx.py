"""GPU parity of the head_dim-128 RoPE kernel with 8 lanes per head (k_rope_nx: every rotary pair in one
lane, items of one or two 8-head passes walked by a resident grid), forced through the launch-shape hook
of the sweep/test build on shapes the size rule would not give it: few tokens, head counts that mix q and
k heads inside a pass or leave a pass part-empty, q only, GPT-J at several rotary dims, every weight
dtype, no norm, out of place, packed q/k/v views, each position source, grids of 1 and 2 workgroups per
CU (so each wave walks many items), runs of consecutive items per wave (a token's angles evaluated
once per run, runs crossing tokens), the {cos, sin} table, out_q in its own layout (exl3r_rope_qg), the
paged append (exl3r_rope_paged_kv) and the projections' output rotations (exl3r_rope_had,
exl3r_rope_paged_kv_had).  Each case is checked against the CPU oracle (<= 2 ulp, the RoPE bound; the
caches bit for bit)."""
import numpy as np
import pytest
import torch

import exl3r
import exl3r._lib as L
import exl3r.ffi as ffi
from _gpu import NTHREADS, assert_close_ulp, dev_normal, from_dev, to_dev
from oracle import oracle as orc
from test_gpu_rope import inv_freq, ragged_position_ids, run

pytestmark = pytest.mark.gpu

F16, BF16, F32 = orc.F16, orc.BF16, orc.F32


@pytest.fixture
def nx():
    """Forces the 8-lane kernel with `passes` (1, 2) passes per item on a grid of `wpc` workgroups per CU
    (0: the resident grid), each wave taking `run` consecutive items at a time (0: the automatic choice)."""
    with L.tuned() as lib:
        def set_(passes, wpc=0, run=0):
            lib.exl3r_tune_rope_nx(passes)
            lib.exl3r_tune_rope_tok(0, 0, wpc)
            lib.exl3r_tune_rope_nx_run(run)
        yield set_


@pytest.mark.parametrize("passes", [1, 2])
@pytest.mark.parametrize("hq,hk", [(64, 8), (6, 3), (1, 1), (12, 0), (20, 7), (9, 8)])
def test_head_counts(nx, passes, hq, hk):
    """(6, 3), (20, 7): q and k heads inside one pass; (1, 1), (9, 8): mostly empty passes; (12, 0): q only."""
    nx(passes)
    run(2, 61, hq, hk, 128, 128, exl3r.ROPE_NEOX, F16, position=300, with_k=hk > 0, seed=hq * 10 + hk)
    run(1, 45, hq, hk, 128, 64, exl3r.ROPE_GPTJ, BF16, nwt=F32, position=7, with_k=hk > 0, seed=hq + hk + 1)


@pytest.mark.parametrize("passes", [1, 2])
@pytest.mark.parametrize("R,mode", [(128, exl3r.ROPE_NEOX), (128, exl3r.ROPE_GPTJ), (64, exl3r.ROPE_GPTJ),
                                    (96, exl3r.ROPE_GPTJ), (4, exl3r.ROPE_GPTJ)])
@pytest.mark.parametrize("dt,nwt", [(F16, F16), (F16, F32), (F16, BF16), (BF16, BF16), (BF16, F16)])
def test_modes_and_dtypes(nx, passes, R, mode, dt, nwt):
    nx(passes)
    run(1, 130, 10, 2, 128, R, mode, dt, nwt=nwt, position=1234, cb=1.0 if nwt != F32 else 0.5, seed=R + dt + nwt)


@pytest.mark.parametrize("passes", [1, 2])
def test_no_norm_out_of_place_attn(nx, passes):
    nx(passes)
    run(1, 70, 8, 2, 128, 128, exl3r.ROPE_NEOX, F16, norm=False, position=5000, out_of_place=True, attn=0.75)
    run(3, 20, 8, 0, 128, 64, exl3r.ROPE_GPTJ, BF16, norm=False, with_k=False, positions=np.array([0, 1, 40000], np.int32))


@pytest.mark.parametrize("passes,wpc", [(1, 1), (2, 1), (2, 2), (1, 0)])
def test_c4_grids(nx, passes, wpc):
    """Config 4's ragged prefill (~4.6k tokens, 64 / 8 heads) on small persistent grids: every wave walks
    dozens of items through both buffers."""
    nx(passes, wpc)
    pid = ragged_position_ids(3)[None, :]
    run(1, pid.size, 64, 8, 128, 128, exl3r.ROPE_NEOX, F16, position_ids=pid, seed=31 + passes)
    run(1, pid.size, 64, 8, 128, 64, exl3r.ROPE_GPTJ, F16, position_ids=pid, seed=33 + passes)


@pytest.mark.parametrize("passes", [1, 2])
def test_packed_qkv_views(nx, passes):
    """q and k as views into one [bsz, seq, hq + 2 hk, hd] projection output; the v heads stay unwritten."""
    nx(passes)
    bsz, seq, hq, hk, hd = 2, 37, 16, 4, 128
    qkv = dev_normal((bsz, seq, hq + 2 * hk, hd), 0.0, 1.0, F16, 21)
    qn, kn = dev_normal((hd,), 1.0, 0.1, F16, 22), dev_normal((hd,), 1.0, 0.1, F16, 23)
    before = from_dev(qkv)
    q, k = qkv[:, :, :hq], qkv[:, :, hq:hq + hk]
    f = inv_freq(128)
    pos = np.array([3, 20000], np.int32)
    ffi.rope(q, q, k, k, torch.from_numpy(f).cuda(), 0, torch.from_numpy(pos).cuda(), qn, kn, 1e-6, 0.0,
             exl3r.ROPE_NEOX, 1.0)
    torch.cuda.synchronize()
    eq, ek = orc.rope(np.ascontiguousarray(before[:, :, :hq]), np.ascontiguousarray(before[:, :, hq:hq + hk]), F16, f,
                      exl3r.ROPE_NEOX, positions=pos, q_norm=from_dev(qn), k_norm=from_dev(kn), nwt=F16, eps=1e-6,
                      nthreads=NTHREADS)
    after = from_dev(qkv)
    assert_close_ulp(after[:, :, :hq], eq, F16, 2, what="packed q")
    assert_close_ulp(after[:, :, hq:hq + hk], ek, F16, 2, what="packed k")
    assert np.array_equal(after[:, :, hq + hk:], before[:, :, hq + hk:]), "v heads modified"


@pytest.mark.parametrize("passes", [1, 2])
@pytest.mark.parametrize("mode,R", [(exl3r.ROPE_NEOX, 128), (exl3r.ROPE_GPTJ, 64)])
def test_cs_table(nx, passes, mode, R):
    """exl3r_rope_cs on the forced kernel against the oracle (the table row read per item)."""
    nx(passes)
    cs_case(mode, R, f"nx{passes}")


def cs_case(mode, R, tag):
    bsz, seq, hq, hk, hd = 3, 90, 10, 3, 128
    q = dev_normal((bsz, seq, hq, hd), 0, 1, F16, 40)
    k = dev_normal((bsz, seq, hk, hd), 0, 1, F16, 41)
    qn, kn = dev_normal((hd,), 1, 0.1, F16, 42), dev_normal((hd,), 1, 0.1, F16, 43)
    f = inv_freq(R)
    pos = np.array([7, 900, 31000], np.int32)
    qh, kh = from_dev(q), from_dev(k)
    cs = ffi.rope_cs_table(bsz, seq, torch.from_numpy(f).cuda(), 0, torch.from_numpy(pos).cuda(), None, 0.8)
    ffi.rope_cs(q, q, k, k, cs, qn, kn, 1e-6, 0.0, mode)
    torch.cuda.synchronize()
    eq, ek = orc.rope(qh, kh, F16, f, mode, positions=pos, q_norm=from_dev(qn), k_norm=from_dev(kn), nwt=F16,
                      eps=1e-6, attn=0.8, nthreads=NTHREADS)
    assert_close_ulp(from_dev(q), eq, F16, 2, what=f"rope_cs {tag} mode{mode} q")
    assert_close_ulp(from_dev(k), ek, F16, 2, what=f"rope_cs {tag} mode{mode} k")


@pytest.mark.parametrize("passes", [1, 2])
def test_qg_out_layout(nx, passes):
    """exl3r_rope_qg (q read from the q halves of [q | g] heads, written to a dense out_q) on the forced
    kernel against the oracle's deinterleave then rope."""
    nx(passes)
    bsz, seq, hq, hk, hd = 1, 200, 12, 2, 128
    qg = dev_normal((bsz, seq, hq, 2 * hd), 0, 1, F16, 50)
    k = dev_normal((bsz, seq, hk, hd), 0, 1, F16, 51)
    qn, kn = dev_normal((hd,), 1, 0.1, F16, 52), dev_normal((hd,), 1, 0.1, F16, 53)
    f = inv_freq(128)
    qgh, kh = from_dev(qg), from_dev(k)
    oq = torch.empty((bsz, seq, hq, hd), device="cuda", dtype=torch.float16)
    ffi.rope_qg(qg, oq, k, k, torch.from_numpy(f).cuda(), 9, None, qn, kn, 1e-6, 1.0, exl3r.ROPE_NEOX, 1.0)
    torch.cuda.synchronize()
    qh, _ = orc.deinterleave_qg(qgh.reshape(bsz * seq, -1), hq, hd, nthreads=NTHREADS)
    eq, ek = orc.rope(qh.reshape(bsz, seq, hq, hd), kh, F16, f, exl3r.ROPE_NEOX, position=9, q_norm=from_dev(qn),
                      k_norm=from_dev(kn), nwt=F16, eps=1e-6, cb=1.0, nthreads=NTHREADS)
    assert_close_ulp(from_dev(oq), eq, F16, 2, what=f"rope_qg nx{passes} q")
    assert_close_ulp(from_dev(k), ek, F16, 2, what=f"rope_qg nx{passes} k")
    assert np.array_equal(from_dev(qg), qgh), "qg modified"


@pytest.mark.parametrize("case", ["neox_f16", "gptj_bf16", "mixed_passes", "no_norm_no_out_k", "bad_entries"])
def test_paged_append(nx, case):
    """exl3r_rope_paged_kv on the forced kernel (v heads after the k heads in the item space, k and v
    rows written to the paged caches) against the oracle's rope then paged_kv_append."""
    import test_gpu_rope_paged as P
    nx(1)
    if case == "neox_f16":
        pages, bt, sl = P.layout(2, 45, 16, 8, 61)
        P.run(2, 45, 16, 4, 128, 128, exl3r.ROPE_NEOX, F16, 16, pages, 8, sl, bt, seed=61)
    elif case == "gptj_bf16":
        pages, bt, sl = P.layout(3, 30, 32, 4, 62)
        P.run(3, 30, 8, 2, 128, 64, exl3r.ROPE_GPTJ, BF16, 32, pages, 4, sl, bt, seed=62)
    elif case == "mixed_passes":     # 12 q / 3 kv heads: passes holding q and k, and k and v heads
        pages, bt, sl = P.layout(2, 37, 16, 8, 63)
        P.run(2, 37, 12, 3, 128, 128, exl3r.ROPE_NEOX, F16, 16, pages, 8, sl, bt, seed=63)
    elif case == "no_norm_no_out_k":
        pages, bt, sl = P.layout(1, 90, 64, 4, 64)
        P.run(1, 90, 16, 8, 128, 128, exl3r.ROPE_NEOX, F16, 64, pages, 4, sl, bt, norm=False, with_out_k=False,
              seed=64)
    else:
        pages, bt, sl = P.layout(4, 20, 16, 4, 65)
        bt[1, :] = pages + 7
        sl[2] = 4 * 16 - 10
        sl[3] = -3
        P.run(4, 20, 8, 2, 128, 128, exl3r.ROPE_NEOX, F16, 16, pages, 4, sl, bt, seed=65)


@pytest.mark.parametrize("case", ["neox", "gptj", "no_norm_missing_posts", "q_only", "out_of_place_bf16w"])
def test_output_rotation(nx, case):
    """exl3r_rope_had on the forced kernel: each head's output rotation on the 8-lane layout (bits 0-2 and 6
    in-lane, bits 3-5 across the group), against the unfused calls and the oracle's had_r_128 then rope."""
    import test_gpu_rope_had as RH
    nx(1)
    if case == "neox":
        RH.run(1, 70, 12, 3, 128, 128, exl3r.ROPE_NEOX, position=21, seed=71)
    elif case == "gptj":
        RH.run(2, 30, 8, 2, 128, 64, exl3r.ROPE_GPTJ, nwt=F32, position=5, seed=72)
    elif case == "no_norm_missing_posts":
        RH.run(1, 40, 16, 4, 128, 128, exl3r.ROPE_NEOX, norm=False, q_post=False, seed=73)
    elif case == "q_only":
        RH.run(1, 33, 10, 0, 128, 128, exl3r.ROPE_NEOX, with_k=False, position=300, seed=74)
    else:
        RH.run(2, 25, 8, 8, 128, 128, exl3r.ROPE_NEOX, nwt=BF16, k_post=False, out_of_place=True, seed=75)


@pytest.mark.parametrize("case", ["qwen3_shape", "mixed_passes_no_out_k", "bad_entry_posts"])
def test_paged_output_rotation(nx, case):
    """exl3r_rope_paged_kv_had on the forced kernel: q / k / v rotated, q / k normed and roped, k / v
    appended; against the oracle composition and the unfused calls."""
    import test_gpu_rope_paged_had as PH
    nx(1)
    if case == "qwen3_shape":
        PH.run(1, 80, 64, 8, 16, 8, seed=81)
    elif case == "mixed_passes_no_out_k":
        PH.run(2, 30, 12, 3, 16, 4, with_out_k=False, posts=(True, False, True), seed=82)
    else:
        PH.run(3, 25, 8, 2, 16, 4, norm=False, posts=(False, True, False), bad_entry=True, seed=83)


@pytest.mark.parametrize("passes,length,wpc", [(1, 2, 0), (1, 3, 1), (1, 5, 0), (2, 3, 0), (1, 9, 2), (2, 16, 1)])
def test_runs(nx, passes, length, wpc):
    """Each wave taking `length` consecutive items: the token's angles are evaluated once per token within
    a run, runs that cross token boundaries re-evaluate them, and small grids make every wave walk many
    runs.  Ragged position ids (consecutive tokens of different sequences rotate by unrelated angles),
    mixed q / k passes, GPT-J, per-sequence positions, and with one pass per item the {cos, sin} table,
    the paged append and the output rotations, each against the oracle."""
    import test_gpu_rope_had as RH
    import test_gpu_rope_paged as P
    import test_gpu_rope_paged_had as PH
    nx(passes, wpc, length)
    pid = ragged_position_ids(5)[None, :700]
    run(1, pid.size, 20, 7, 128, 128, exl3r.ROPE_NEOX, F16, position_ids=pid, seed=90 + length)
    run(1, pid.size, 64, 8, 128, 64, exl3r.ROPE_GPTJ, BF16, position_ids=pid, seed=91 + length)
    run(3, 41, 9, 8, 128, 128, exl3r.ROPE_NEOX, F16, positions=np.array([3, 20000, 77], np.int32), seed=92 + length)
    if passes == 1:
        cs_case(exl3r.ROPE_NEOX, 128, f"run{length}")
        pages, bt, sl = P.layout(2, 45, 16, 8, 93)
        P.run(2, 45, 12, 3, 128, 128, exl3r.ROPE_NEOX, F16, 16, pages, 8, sl, bt, seed=93)
        RH.run(1, 70, 12, 3, 128, 128, exl3r.ROPE_NEOX, position=21, seed=94)
        PH.run(2, 40, 16, 4, 16, 8, seed=95)


@pytest.mark.parametrize("passes", [1, 2])
def test_rotation_f16_special_values(nx, passes):
    """The f16 NeoX rotation forms its fp32 products straight from the packed f16 pairs (a mixed-precision
    fma with a -0 addend): f16 subnormals, signed zeros, the f16 maximum (products past it round to
    infinity) and position 0 (sin = 0: every second product is a zero of either sign), without the head
    norm so that the raw inputs reach the products.  Against the oracle (<= 2 ulp), and every result the
    oracle gives as a zero carries the oracle's sign."""
    nx(passes)
    seq, hq, hk = 48, 12, 5
    rng = np.random.default_rng(123)
    vals = np.array([0.0, -0.0, 6e-8, -6e-8, 3.0e-5, -2.4e-5, 65504.0, -65504.0, 1.0, -1.0, 0.5, 1e-3],
                    np.float16)
    qh = rng.choice(vals, (1, seq, hq, 128)).astype(np.float16).view(np.uint16)
    kh = rng.choice(vals, (1, seq, hk, 128)).astype(np.float16).view(np.uint16)
    pid = np.concatenate([np.zeros(16, np.int32), rng.integers(1, 40000, seq - 16).astype(np.int32)])[None, :]
    f = inv_freq(128)
    q, k = to_dev(qh, F16), to_dev(kh, F16)
    ffi.rope(q, q, k, k, torch.from_numpy(f).cuda(), 0, None, None, None, 1e-6, 0.0, exl3r.ROPE_NEOX, 1.0,
             position_ids=torch.from_numpy(pid).cuda())
    torch.cuda.synchronize()
    eq, ek = orc.rope(qh, kh, F16, f, exl3r.ROPE_NEOX, position_ids=pid.reshape(-1), q_norm=None, k_norm=None,
                      nwt=F16, eps=1e-6, cb=0.0, attn=1.0, nthreads=NTHREADS)
    for got, exp, what in ((from_dev(q), eq, "q"), (from_dev(k), ek, "k")):
        assert_close_ulp(got, exp, F16, 2, what=f"f16 specials {what} passes={passes}")
        zero = (exp & 0x7FFF) == 0
        assert zero.sum() > 100, "the case must hold zero results"
        assert np.array_equal(got[zero], exp[zero]), f"zero signs differ ({what})"
