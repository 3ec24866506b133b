"""CPU tests of the paged-pool bookkeeping (q3attn/pages.py): page accounting under random grow/release
sequences, all-or-nothing exhaustion, the scratch seat, and the device-side block-table / slot views against
the host page lists (the identity-table special case reproduces the reference's seat * seat_len + pos)."""
import numpy as np
import pytest
import torch

from q3attn.pages import PagePool, PoolExhausted


def test_random_grow_release_keeps_accounting():
    rng = np.random.default_rng(0)
    pool = PagePool(num_pages=200, max_seats=12, max_pages_per_seat=20, device="cpu")
    lengths = np.zeros(12, np.int64)
    for step in range(400):
        s = int(rng.integers(12))
        if rng.random() < 0.15:
            pool.release(s)
            lengths[s] = 0
        else:
            n = int(min(lengths[s] + rng.integers(1, 40), pool.seat_len))
            try:
                pool.grow(s, n)
                lengths[s] = n
            except PoolExhausted:
                pass
        assert pool.capacity(s) >= lengths[s]
        if step % 25 == 0:
            pool.check()
    pool.check()


def test_grow_is_all_or_nothing():
    pool = PagePool(num_pages=9, max_seats=4, max_pages_per_seat=8, device="cpu")   # 8 usable pages
    pool.grow([0, 1], [64, 32])                                                        # 4 + 2 pages
    before = (pool.free_pages, pool.pages_of(2), pool.table.clone())
    with pytest.raises(PoolExhausted):
        pool.grow([2, 3], [32, 32])                                                    # needs 4, 2 free
    assert pool.free_pages == before[0] and pool.pages_of(2) == before[1]
    assert torch.equal(pool.table, before[2])
    pool.release(0)
    pool.grow([2, 3], [32, 32])
    pool.check()


def test_pages_are_reused_after_release():
    pool = PagePool(num_pages=5, max_seats=2, max_pages_per_seat=4, device="cpu")
    pool.grow(0, 64)
    first = pool.pages_of(0)
    pool.release(0)
    pool.grow(1, 64)
    assert sorted(pool.pages_of(1)) == sorted(first)
    assert (pool.table[0] == -1).all()
    pool.check()


def test_scratch_seat_and_bounds():
    pool = PagePool(num_pages=10, max_seats=3, max_pages_per_seat=4, device="cpu")
    assert (pool.table[pool.scratch_seat] == PagePool.SCRATCH_PAGE).all()
    with pytest.raises(IndexError):
        pool.grow(3, 1)
    with pytest.raises(ValueError):
        pool.grow(0, pool.seat_len + 1)
    with pytest.raises(ValueError):
        PagePool(num_pages=10, max_seats=3, max_pages_per_seat=4, page_size=24, device="cpu")


def test_slot_and_block_table_views():
    pool = PagePool(num_pages=64, max_seats=5, max_pages_per_seat=6, device="cpu")
    rng = np.random.default_rng(1)
    lens = rng.integers(1, pool.seat_len, size=5)
    pool.release(range(5))
    for s in rng.permutation(5):
        pool.grow(int(s), int(lens[s]))
    seat = torch.tensor([3, 0, 4, 4, 1], dtype=torch.long)
    pos = torch.tensor([int(lens[3]) - 1, 0, int(lens[4]) - 1, 5, int(lens[1]) // 2], dtype=torch.long)
    slots = pool.slot(seat, pos)
    for i in range(len(seat)):
        pl = pool.pages_of(int(seat[i]))
        assert int(slots[i]) == pl[int(pos[i]) // 16] * 16 + int(pos[i]) % 16
    bt = pool.block_table(seat)
    assert bt.dtype == torch.int32 and bt.shape == (5, 6)
    for i in range(len(seat)):
        pl = pool.pages_of(int(seat[i]))
        assert bt[i, : len(pl)].tolist() == pl and (bt[i, len(pl):] == -1).all()


def test_identity_layout_reproduces_reference_slot():
    """Seats growing in order on a fresh pool get consecutive pages; with page_size == seat_len the slot is the
    reference's seat * seat_len + pos (engine/talker.py:109) shifted by the reserved scratch page."""
    pool = PagePool(num_pages=1 + 4, max_seats=4, max_pages_per_seat=1, page_size=256, device="cpu")
    for s in range(4):
        pool.grow(s, 256)
    seat = torch.arange(4).repeat_interleave(3)
    pos = torch.tensor([0, 17, 255] * 4)
    assert torch.equal(pool.slot(seat, pos), (seat + 1) * 256 + pos)
