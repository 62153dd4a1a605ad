"""The oracle's paged KV-cache append (reference kernels/generator/cache.cu:143-243), pinned by
properties of a paged store rather than by its own index formula: every appended row reads back
through the block table at its logical position, nothing else in the pool changes, appends that
cross a page boundary land on two pages, bad positions / pages are flagged and skipped, and a
planted one-row offset is caught."""
import numpy as np
import pytest

from oracle import oracle as orc
from _util import normal as _normal

ORM_PAGE_OFF = 16   # oracle/rowops_oracle.h


def normal(shape, mean, std, dt, seed):
    return _normal(np.random.default_rng(seed), shape, mean, std, dt)

F16, BF16 = orc.F16, orc.BF16


def setup(bsz=3, seq=5, hk=2, hd=16, page=8, pages=12, seed=0, dt=F16):
    rng = np.random.default_rng(seed)
    k = normal((bsz, seq, hk, hd), 0, 1, dt, seed)
    v = normal((bsz, seq, hk, hd), 0, 1, dt, seed + 1)
    kc = normal((pages, page, hk, hd), 0, 1, dt, seed + 2)
    vc = normal((pages, page, hk, hd), 0, 1, dt, seed + 3)
    max_blocks = 4
    bt = rng.permutation(pages)[: bsz * max_blocks].reshape(bsz, max_blocks).astype(np.int32)
    seqlens = rng.integers(0, max_blocks * page - seq, bsz).astype(np.int32)
    return k, v, kc, vc, bt, seqlens


def read_back(cache, bt, b, pos):
    page = cache.shape[1]
    return cache[bt[b, pos // page], pos % page]


@pytest.mark.parametrize("dt", [F16, BF16])
def test_rows_read_back_and_nothing_else_changes(dt):
    k, v, kc, vc, bt, seqlens = setup(dt=dt, seed=4)
    kc0, vc0 = kc.copy(), vc.copy()
    assert orc.paged_kv_append(k, v, dt, kc, vc, bt, seqlens) == 0
    touched = np.zeros(kc.shape[:2], bool)
    for b in range(k.shape[0]):
        for s in range(k.shape[1]):
            pos = int(seqlens[b]) + s
            assert np.array_equal(read_back(kc, bt, b, pos), k[b, s])
            assert np.array_equal(read_back(vc, bt, b, pos), v[b, s])
            touched[bt[b, pos // kc.shape[1]], pos % kc.shape[1]] = True
    assert np.array_equal(kc[~touched], kc0[~touched]) and np.array_equal(vc[~touched], vc0[~touched])
    assert touched.sum() == k.shape[0] * k.shape[1]


def test_append_crossing_a_page_boundary():
    k, v, kc, vc, bt, _ = setup(bsz=1, seq=6, page=8, seed=5)
    seqlens = np.array([5], np.int32)           # positions 5..10: pages bt[0,0] and bt[0,1]
    orc.paged_kv_append(k, v, F16, kc, vc, bt, seqlens)
    assert np.array_equal(kc[bt[0, 0], 5:8], k[0, 0:3]) and np.array_equal(kc[bt[0, 1], 0:3], k[0, 3:6])


def test_k_only_and_v_only():
    k, v, kc, vc, bt, seqlens = setup(seed=6)
    vc0 = vc.copy()
    orc.paged_kv_append(k, None, F16, kc, None, bt, seqlens)
    assert np.array_equal(vc, vc0)
    assert np.array_equal(read_back(kc, bt, 0, int(seqlens[0])), k[0, 0])


def test_out_of_range_positions_and_pages_are_flagged_and_skipped():
    k, v, kc, vc, bt, seqlens = setup(bsz=2, seq=3, seed=7)
    bt[1, :] = -1                                 # sequence 1 has no pages
    seqlens[0] = 4 * 8 - 1                        # token 1 of sequence 0 runs past the block table
    kc0 = kc.copy()
    err = orc.paged_kv_append(k, v, F16, kc, vc, bt, seqlens)
    assert err == 1
    assert np.array_equal(read_back(kc, bt, 0, int(seqlens[0])), k[0, 0])
    changed = np.any(kc != kc0, axis=(2, 3)).sum()
    assert changed == 1


def test_planted_mistake_is_caught():
    k, v, kc, vc, bt, seqlens = setup(seed=8)
    orc.set_mutation(ORM_PAGE_OFF)
    orc.paged_kv_append(k, v, F16, kc, vc, bt, seqlens)
    orc.set_mutation(0)
    assert not np.array_equal(read_back(kc, bt, 0, int(seqlens[0])), k[0, 0])
