"""Pins the oracle's embedding gather by brute force (numpy fancy indexing, bit patterns) and its
fused gather + RMSNorm by composition with the separately pinned RMSNorm."""
import numpy as np
import pytest

from oracle import oracle as orc


def _table(rng, vocab, hidden, code):
    return orc.to_bits((rng.standard_normal((vocab, hidden)) * 0.02).astype(np.float32), code)


def gather_ok():
    rng = np.random.default_rng(14)
    ok = True
    for tt, ot in ((orc.BF16, orc.BF16), (orc.F16, orc.F16), (orc.BF16, orc.F32), (orc.F16, orc.F32), (orc.F32, orc.F32)):
        table = _table(rng, 97, 40, tt)
        for idt, npt in ((orc.I32, np.int32), (orc.I64, np.int64)):
            ids = rng.integers(0, 97, 33).astype(npt)
            ids[5] = ids[4]                          # repeated id
            out, err = orc.embedding(table, tt, ids, idt, ot)
            exp = table[ids]
            if ot != tt:
                exp = orc.to_f32(exp, tt)
            ok = ok and err == 0 and np.array_equal(out.view(np.uint8), np.ascontiguousarray(exp).view(np.uint8))
    return ok


def test_gather_brute_force():
    assert gather_ok()


def test_out_of_range_ids_zero_row_and_flag():
    rng = np.random.default_rng(15)
    table = _table(rng, 10, 16, orc.BF16)
    ids = np.array([1, -1, 10, 3], np.int64)
    out, err = orc.embedding(table, orc.BF16, ids, orc.I64, orc.BF16)
    assert err == 1
    assert np.all(out[1] == 0) and np.all(out[2] == 0)
    assert np.array_equal(out[0], table[1]) and np.array_equal(out[3], table[3])


def test_nan_payload_copied_bitwise():
    table = np.array([[0x7FC1, 0xFF81, 0x0001, 0x8000]], np.uint16)   # NaNs with payloads, denormal, -0
    out, _ = orc.embedding(table, orc.BF16, np.array([0, 0], np.int32), orc.I32, orc.BF16)
    assert np.array_equal(out, np.repeat(table, 2, 0))


def fused_ok():
    rng = np.random.default_rng(16)
    ok = True
    for tt, ht, yt in ((orc.BF16, orc.BF16, orc.BF16), (orc.F16, orc.F32, orc.F16), (orc.BF16, None, orc.F32)):
        table = _table(rng, 50, 64, tt)
        ids = rng.integers(0, 50, 20).astype(np.int32)
        w = orc.to_bits((rng.standard_normal(64) * 0.1 + 1).astype(np.float32), orc.BF16)
        h, y, err = orc.embedding_rms_norm(table, tt, ids, orc.I32, w, orc.BF16, yt, ht=ht, eps=1e-6)
        g, _ = orc.embedding(table, tt, ids, orc.I32, tt)
        y2 = orc.rms_norm(orc.to_f32(g, tt), orc.F32, w, orc.BF16, yt, 1e-6)   # f32 input: no clamp
        ok = ok and err == 0 and np.array_equal(y, y2)
        if ht is not None:
            ok = ok and np.array_equal(h, g if ht == tt else orc.to_f32(g, tt))
    return ok


def test_fused_gather_norm_is_composition():
    assert fused_ok()


@pytest.mark.parametrize("mutation", [14])
def test_planted_mistakes_are_caught(mutation):
    orc.set_mutation(mutation)
    assert not gather_ok()
