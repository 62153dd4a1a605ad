"""Pins the oracle's angle-table RoPE (RoPE::apply's freq_table, src/rope.rs:225-260, 294-300;
rope.cu:69-83) against the already pinned inv_freq RoPE: a table whose row p holds fl32(p) *
inv_freq -- the reference's own angle_table, an fp32 [max_pos, 1] x [1, R/2] product -- must give
the inv_freq result bit for bit; permuting the table rows and remapping the positions changes
nothing; a [bsz, rows, R/2] table of per-sequence ramps equals per-sequence start positions; a
position outside the table is flagged and rotated by angle 0.  A mutation that reads the next row
fails."""
import numpy as np
import pytest

from oracle import oracle as orc

F16, BF16, F32 = orc.F16, orc.BF16, orc.F32
ORM_TABLE_ROW_OFF = 26


def inv_freq(R, theta=1e6):
    return (1.0 / theta ** (np.arange(0, R, 2, dtype=np.float64) / R)).astype(np.float32)


def ramp_table(rows, R, start=0):
    p = (np.arange(rows, dtype=np.float64) + start).astype(np.float32)
    return (p[:, None] * inv_freq(R)[None, :]).astype(np.float32)      # fp32 products, one rounding


def heads(bsz, seq, hq, hk, hd, dt, seed):
    rng = np.random.default_rng(seed)
    q = orc.to_bits(rng.standard_normal((bsz, seq, hq, hd)).astype(np.float32), dt)
    k = orc.to_bits(rng.standard_normal((bsz, seq, hk, hd)).astype(np.float32), dt)
    qn = orc.to_bits((1 + 0.1 * rng.standard_normal(hd)).astype(np.float32), F16)
    kn = orc.to_bits((1 + 0.1 * rng.standard_normal(hd)).astype(np.float32), F16)
    return q, k, qn, kn


@pytest.mark.parametrize("mode,R,dt,norm", [(orc.ROPE_NEOX, 128, F16, True), (orc.ROPE_GPTJ, 64, F16, True),
                                            (orc.ROPE_NEOX, 64, BF16, False), (orc.ROPE_GPTJ, 128, BF16, True)])
def test_ramp_table_equals_inv_freq(mode, R, dt, norm):
    q, k, qn, kn = heads(2, 37, 4, 2, 128, dt, R)
    kw = dict(q_norm=qn if norm else None, k_norm=kn if norm else None, nwt=F16)
    pos = np.array([5, 3000], np.int32)
    eq, ek = orc.rope(q, k, dt, inv_freq(R), mode, positions=pos, **kw)
    tq, tk, err = orc.rope_table(q, k, dt, ramp_table(4000, R), mode, positions=pos, **kw)
    assert err == 0 and np.array_equal(tq, eq) and np.array_equal(tk, ek)
    pid = np.random.default_rng(1).integers(0, 4000, 2 * 37).astype(np.int32)
    eq, ek = orc.rope(q, k, dt, inv_freq(R), mode, position_ids=pid, **kw)
    tq, tk, err = orc.rope_table(q, k, dt, ramp_table(4000, R), mode, position_ids=pid, **kw)
    assert err == 0 and np.array_equal(tq, eq) and np.array_equal(tk, ek)


def test_permuted_rows_with_remapped_positions():
    q, k, qn, kn = heads(1, 50, 3, 1, 128, F16, 3)
    table = ramp_table(200, 128)
    perm = np.random.default_rng(4).permutation(200)
    inv = np.argsort(perm)                        # table[perm][inv[p]] == table[p]
    pid = np.random.default_rng(5).integers(0, 200, 50).astype(np.int32)
    a = orc.rope_table(q, k, F16, table, orc.ROPE_NEOX, position_ids=pid, q_norm=qn, k_norm=kn)
    b = orc.rope_table(q, k, F16, table[perm], orc.ROPE_NEOX, position_ids=inv[pid].astype(np.int32),
                       q_norm=qn, k_norm=kn)
    assert np.array_equal(a[0], b[0]) and np.array_equal(a[1], b[1])


def test_per_sequence_table():
    q, k, qn, kn = heads(3, 20, 2, 2, 128, BF16, 6)
    starts = [0, 777, 31000]
    table3 = np.stack([ramp_table(20, 128, s) for s in starts])              # [bsz, rows, R/2]
    eq, ek = orc.rope(q, k, BF16, inv_freq(128), orc.ROPE_NEOX, positions=np.array(starts, np.int32),
                      q_norm=qn, k_norm=kn, nwt=F16)
    tq, tk, err = orc.rope_table(q, k, BF16, table3, orc.ROPE_NEOX, q_norm=qn, k_norm=kn, nwt=F16)
    assert err == 0 and np.array_equal(tq, eq) and np.array_equal(tk, ek)


def test_out_of_table_positions_flagged_and_unrotated():
    q, k, qn, kn = heads(1, 10, 2, 1, 128, F16, 7)
    pid = np.array([0, 1, 99, 100, 5000, -1, 3, 99, 100, 2], np.int32)
    tq, tk, err = orc.rope_table(q, k, F16, ramp_table(100, 128), orc.ROPE_NEOX, position_ids=pid,
                                 q_norm=qn, k_norm=kn)
    assert err == 1
    eq, ek = orc.rope(q, k, F16, inv_freq(128), orc.ROPE_NEOX, position_ids=np.where((pid >= 0) & (pid < 100), pid, 0)
                      .astype(np.int32), q_norm=qn, k_norm=kn)
    assert np.array_equal(tq, eq) and np.array_equal(tk, ek)
    _, _, err = orc.rope_table(q, k, F16, ramp_table(100, 128), orc.ROPE_NEOX, position_ids=np.clip(pid, 0, 99)
                               .astype(np.int32), q_norm=qn, k_norm=kn)
    assert err == 0


def test_row_mutation_caught():
    q, k, qn, kn = heads(1, 16, 2, 1, 128, F16, 8)
    eq, _ = orc.rope(q, k, F16, inv_freq(128), orc.ROPE_NEOX, position=40, q_norm=qn, k_norm=kn)
    orc.set_mutation(ORM_TABLE_ROW_OFF)
    try:
        tq, _, _ = orc.rope_table(q, k, F16, ramp_table(100, 128), orc.ROPE_NEOX, position=40, q_norm=qn, k_norm=kn)
    finally:
        orc.set_mutation(0)
    assert not np.array_equal(tq, eq)
