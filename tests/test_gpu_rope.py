"""GPU parity of exl3r_rope (head RMSNorm + NeoX / GPT-J rotary) against the CPU oracle: <= 2 ulp
with sin/cos in fp32, at the configs' shapes, position sources, dtypes and the generic path."""
import numpy as np
import pytest
import torch

import exl3r
import exl3r.ffi as ffi
from _gpu import NTHREADS, TORCH_DT, assert_close_ulp, dev_normal, from_dev, to_dev
from oracle import oracle as orc

pytestmark = pytest.mark.gpu

F16, BF16, F32 = orc.F16, orc.BF16, orc.F32


def inv_freq(R, theta=1e6):
    return (1.0 / theta ** (np.arange(0, R, 2, dtype=np.float64) / R)).astype(np.float32)


def run(bsz, seq, hq, hk, hd, R, mode, dt, nwt=F16, norm=True, position=0, positions=None, position_ids=None,
        cb=0.0, attn=1.0, seed=0, with_k=True, out_of_place=False):
    q = dev_normal((bsz, seq, hq, hd), 0.0, 1.0, dt, seed)
    k = dev_normal((bsz, seq, hk, hd), 0.0, 1.0, dt, seed + 1) if with_k else None
    qn = dev_normal((hd,), 1.0, 0.1, nwt, seed + 2) if norm else None
    kn = dev_normal((hd,), 1.0, 0.1, nwt, seed + 3) if norm and with_k else None
    f = inv_freq(R)
    qh, kh = from_dev(q), (from_dev(k) if with_k else None)
    pos_d = torch.from_numpy(positions).cuda() if positions is not None else None
    pid_d = torch.from_numpy(position_ids).cuda() if position_ids is not None else None
    oq = torch.empty_like(q) if out_of_place else q
    ok = (torch.empty_like(k) if out_of_place else k) if with_k else None
    ffi.rope(q, oq, k, ok, torch.from_numpy(f).cuda(), position, pos_d, qn, kn, 1e-6, cb, mode, attn,
             position_ids=pid_d)
    torch.cuda.synchronize()
    eq, ek = orc.rope(qh, kh, dt, f, mode, position=position, positions=positions,
                      position_ids=position_ids.reshape(-1) if position_ids is not None else None,
                      q_norm=from_dev(qn) if norm else None, k_norm=from_dev(kn) if kn is not None else None,
                      nwt=nwt, eps=1e-6, cb=cb, attn=attn, nthreads=NTHREADS)
    tag = f"rope b{bsz} s{seq} h{hq}/{hk} d{hd} R{R} mode{mode} dt{dt} w{nwt if norm else '-'}"
    assert_close_ulp(from_dev(oq), eq, dt, 2, what=tag + " q")
    if with_k:
        assert_close_ulp(from_dev(ok), ek, dt, 2, what=tag + " k")


def test_c1_qwen3_06b():
    """Config 1(3): 16 q / 8 kv heads, head_dim 128, theta 1e6, positions 0..511, f16 head norm."""
    run(1, 512, 16, 8, 128, 128, exl3r.ROPE_NEOX, F16, position=0)


def ragged_position_ids(seed):
    rng = np.random.default_rng(seed)
    lens = rng.integers(64, 513, 16)
    starts = rng.integers(0, 32768, 16)
    return np.concatenate([s + np.arange(n) for s, n in zip(starts, lens)]).astype(np.int32)


def test_c4_paged_neox():
    """Config 4: 16 ragged sequences (~4096 tokens), 64 q / 8 kv heads, hd 128, starts in [0, 32768)."""
    pid = ragged_position_ids(0)
    run(1, pid.size, 64, 8, 128, 128, exl3r.ROPE_NEOX, F16, position_ids=pid[None, :], seed=4)


def test_c4_gptj_partial():
    """Config 4 GPT-J variant: rotary_dim 64 of 128 (partial)."""
    pid = ragged_position_ids(1)
    run(1, pid.size, 64, 8, 128, 64, exl3r.ROPE_GPTJ, F16, position_ids=pid[None, :], seed=5)


def test_decode_batch_positions():
    """64-row decode: bsz 64, q_len 1, per-sequence positions (the paged decode call)."""
    pos = np.random.default_rng(2).integers(0, 32768, 64).astype(np.int32)
    run(64, 1, 64, 8, 128, 128, exl3r.ROPE_NEOX, F16, positions=pos, seed=6)


@pytest.mark.parametrize("dt,nwt", [(F16, F16), (F16, BF16), (F16, F32), (BF16, BF16), (BF16, F16), (BF16, F32)])
@pytest.mark.parametrize("mode", [exl3r.ROPE_NEOX, exl3r.ROPE_GPTJ])
def test_dtypes(dt, nwt, mode):
    run(2, 37, 6, 2, 128, 128, mode, dt, nwt=nwt, position=100, cb=1.0 if nwt == BF16 else 0.0, seed=dt + 3 * nwt)


@pytest.mark.parametrize("hd,R,mode", [(64, 64, exl3r.ROPE_NEOX), (256, 256, exl3r.ROPE_NEOX), (128, 32, exl3r.ROPE_NEOX),
                                       (96, 96, exl3r.ROPE_NEOX), (96, 64, exl3r.ROPE_GPTJ), (80, 32, exl3r.ROPE_NEOX),
                                       (100, 40, exl3r.ROPE_NEOX), (30, 30, exl3r.ROPE_GPTJ), (512, 512, exl3r.ROPE_GPTJ)])
def test_head_dims(hd, R, mode):
    run(1, 40, 5, 3, hd, R, mode, BF16, nwt=BF16, position=7, seed=hd + R)


def test_no_norm_q_only_out_of_place_attn():
    run(1, 33, 8, 0, 128, 128, exl3r.ROPE_NEOX, F16, norm=False, with_k=False, position=5000)
    run(2, 9, 8, 2, 128, 128, exl3r.ROPE_GPTJ, F16, norm=True, position=77, out_of_place=True, attn=0.75)
    run(3, 5, 4, 4, 64, 64, exl3r.ROPE_NEOX, BF16, norm=False, positions=np.array([0, 1, 40000], np.int32))


def test_large_positions():
    run(1, 64, 4, 2, 128, 128, exl3r.ROPE_NEOX, F16, position=1_000_000, seed=9)


def test_packed_qkv_views():
    """q and k as views into one [bsz, seq, hq + 2 hk, hd] QKV projection output (token stride
    (hq + 2 hk) hd), rotated in place; the V heads between and after them stay bit-identical."""
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


def test_zero_tokens():
    q = torch.empty((1, 0, 8, 128), device="cuda", dtype=torch.float16)
    k = torch.empty((1, 0, 2, 128), device="cuda", dtype=torch.float16)
    ffi.rope(q, q, k, k, torch.from_numpy(inv_freq(128)).cuda(), 0, None, None, None, 1e-6, 0.0,
             exl3r.ROPE_NEOX, 1.0)
    torch.cuda.synchronize()
