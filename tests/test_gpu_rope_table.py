"""GPU parity of exl3r_rope_table (RoPE with precomputed angles: RoPE::apply's freq_table, MRoPE and
the vision tower's 2-D RoPE) against the CPU oracle, on every kernel (the launch-shape hook forces
the wave-per-token and flattened kernels; odd head dims take the generic kernel), plus two
device-side identities: a table whose row p is fl32(p) * inv_freq gives exl3r_rope's result bit for
bit, and a per-sequence [bsz, rows, R/2] ramp table equals per-sequence start positions."""
import numpy as np
import pytest
import torch

import exl3r
import exl3r._lib as L
import exl3r.ffi as ffi
from _gpu import NTHREADS, assert_close_ulp, dev_normal, from_dev
from oracle import oracle as orc

pytestmark = pytest.mark.gpu

F16, BF16, F32 = exl3r.F16, exl3r.BF16, exl3r.F32


@pytest.fixture
def tune():
    """Forces the RoPE kernel (0 auto, 1 never the wave-per-token kernel, 2 always) through the sweep/test
    build of the library, which the wrappers call inside the fixture."""
    with L.tuned() as lib:
        yield lambda use: lib.exl3r_tune_rope_tok(use, 0, 0)


def inv_freq(R, theta=1e6):
    return (1.0 / theta ** (np.arange(0, R, 2, dtype=np.float64) / R)).astype(np.float32)


def ramp_table(rows, R, start=0):
    p = (np.arange(rows, dtype=np.float64) + start).astype(np.float32)
    return (p[:, None] * inv_freq(R)[None, :]).astype(np.float32)


def run(bsz, seq, hq, hk, hd, table, mode, dt, nwt=F16, norm=True, position=0, positions=None, position_ids=None,
        seed=0, expect_err=0):
    q = dev_normal((bsz, seq, hq, hd), 0.0, 1.0, dt, seed)
    k = dev_normal((bsz, seq, hk, hd), 0.0, 1.0, dt, seed + 1)
    qn = dev_normal((hd,), 1.0, 0.1, nwt, seed + 2) if norm else None
    kn = dev_normal((hd,), 1.0, 0.1, nwt, seed + 3) if norm else None
    qh, kh = from_dev(q), from_dev(k)
    err = torch.zeros(1, dtype=torch.int32, device="cuda")
    pos_d = torch.from_numpy(positions).cuda() if positions is not None else None
    pid_d = torch.from_numpy(position_ids).cuda() if position_ids is not None else None
    ffi.rope(q, q, k, k, torch.from_numpy(table).cuda(), position, pos_d, qn, kn, 1e-6, 0.0, mode, 1.0,
             position_ids=pid_d, err_flag=err)
    torch.cuda.synchronize()
    eq, ek, eerr = orc.rope_table(qh, kh, dt, table, mode, position=position, positions=positions,
                                  position_ids=position_ids.reshape(-1) if position_ids is not None else None,
                                  q_norm=from_dev(qn) if norm else None, k_norm=from_dev(kn) if norm else None,
                                  nwt=nwt, nthreads=NTHREADS)
    tag = f"rope_table b{bsz} s{seq} h{hq}/{hk} d{hd} R{table.shape[-1] * 2} mode{mode} dt{dt}"
    assert_close_ulp(from_dev(q), eq, dt, 2, what=tag + " q")
    assert_close_ulp(from_dev(k), ek, dt, 2, what=tag + " k")
    assert int(err.item()) == eerr == expect_err
    return q, k


@pytest.mark.parametrize("use", [1, 2])
@pytest.mark.parametrize("mode,R,dt,nwt", [(exl3r.ROPE_NEOX, 128, F16, F16), (exl3r.ROPE_GPTJ, 64, F16, F16),
                                           (exl3r.ROPE_NEOX, 128, BF16, F32), (exl3r.ROPE_GPTJ, 128, BF16, BF16)])
def test_mrope_like_random_angles(tune, use, mode, R, dt, nwt):
    """Arbitrary angles (as an MRoPE table holds), ragged per-token positions, both kernels."""
    tune(use)
    table = np.random.default_rng(R + use).uniform(-3000.0, 3000.0, (2048, R // 2)).astype(np.float32)
    pid = np.random.default_rng(7).integers(0, 2048, (1, 1100)).astype(np.int32)
    run(1, 1100, 8, 2, 128, table, mode, dt, nwt=nwt, position_ids=pid, seed=R)


def test_per_sequence_tables_and_shared_table():
    tables = np.random.default_rng(2).uniform(-50.0, 50.0, (3, 40, 64)).astype(np.float32)
    run(3, 40, 4, 2, 128, tables, exl3r.ROPE_NEOX, F16, seed=11)                            # [bsz, rows, R/2]
    run(3, 20, 4, 2, 128, tables[1], exl3r.ROPE_NEOX, F16, positions=np.array([0, 5, 20], np.int32), seed=12)


def test_out_of_table_positions_flagged():
    pid = np.array([[0, 1, 99, 100, 5000, -1, 3, 99]], np.int32)
    run(1, 8, 4, 2, 128, ramp_table(100, 128), exl3r.ROPE_NEOX, F16, position_ids=pid, seed=13, expect_err=1)


def test_odd_head_dims():
    """head_dim 100 (generic kernel) and 96 with rotary 48."""
    run(2, 9, 3, 1, 100, ramp_table(64, 100), exl3r.ROPE_NEOX, F16, positions=np.array([3, 40], np.int32), seed=14)
    run(1, 5, 2, 2, 96, ramp_table(32, 48), exl3r.ROPE_GPTJ, BF16, nwt=F32, position=7, seed=15)


@pytest.mark.parametrize("use", [1, 2])
def test_ramp_table_equals_inv_freq_on_device(tune, use):
    """The reference's own plain angle table (rope.rs:294-300) must reproduce exl3r_rope bit for bit."""
    tune(use)
    T = 1500
    q = dev_normal((1, T, 16, 128), 0.0, 1.0, F16, 20)
    k = dev_normal((1, T, 4, 128), 0.0, 1.0, F16, 21)
    qn, kn = dev_normal((128,), 1.0, 0.1, F16, 22), dev_normal((128,), 1.0, 0.1, F16, 23)
    pid = torch.from_numpy(np.random.default_rng(24).integers(0, 40000, (1, T)).astype(np.int32)).cuda()
    q2, k2 = q.clone(), k.clone()
    ffi.rope(q, q, k, k, torch.from_numpy(inv_freq(128)).cuda(), 0, None, qn, kn, 1e-6, 0.0, exl3r.ROPE_NEOX, 1.0,
             position_ids=pid)
    ffi.rope(q2, q2, k2, k2, torch.from_numpy(ramp_table(40000, 128)).cuda(), 0, None, qn, kn, 1e-6, 0.0,
             exl3r.ROPE_NEOX, 1.0, position_ids=pid)
    torch.cuda.synchronize()
    assert torch.equal(q.view(torch.int16), q2.view(torch.int16))
    assert torch.equal(k.view(torch.int16), k2.view(torch.int16))
    s = torch.from_numpy(np.array([100, 7], np.int32)).cuda()
    x = dev_normal((2, 30, 4, 128), 0.0, 1.0, F16, 25)
    y = x.clone()
    ffi.rope(x, x, None, None, torch.from_numpy(inv_freq(128)).cuda(), 0, s, None, None, 1e-6, 0.0, exl3r.ROPE_NEOX, 1.0)
    t3 = np.stack([ramp_table(30, 128, 100), ramp_table(30, 128, 7)])
    ffi.rope(y, y, None, None, torch.from_numpy(t3).cuda(), 0, None, None, None, 1e-6, 0.0, exl3r.ROPE_NEOX, 1.0)
    torch.cuda.synchronize()
    assert torch.equal(x.view(torch.int16), y.view(torch.int16))


def test_zero_tokens_and_bad_arguments():
    z = torch.empty((1, 0, 4, 128), device="cuda", dtype=torch.float16)
    ffi.rope(z, z, None, None, torch.zeros((10, 64), device="cuda"), 0, None, None, None, 1e-6, 0.0,
             exl3r.ROPE_NEOX, 1.0)
    with pytest.raises(exl3r.Exl3rError):
        lib = L.load()
        q = dev_normal((1, 2, 4, 128), 0.0, 1.0, F16, 30)
        rc = lib.exl3r_rope_table(q.data_ptr(), q.data_ptr(), 512, 128, 4, None, None, 0, 0, 0, F16, 1, 2, 128,
                                  torch.zeros(64, device="cuda").data_ptr(), 0, 0, 128, 0, None, None, None, None, F16,
                                  1e-6, 0.0, exl3r.ROPE_NEOX, 1.0, None, None)
        L.check(rc)
