"""Paged KV pool bookkeeping: 16-token pages handed out to seats from a free list.

The reference gives every seat a fixed, contiguous slice of the KV pool (pages of 256 positions and an identity
``seat_pages`` table, engine/talker.py:23-31, 42; append slot ``seat * seat_len + pos``, engine/talker.py:109).
Here the pool is shared: a seat owns only the pages its tokens occupy, taken from a free list as it grows and
returned when it is released, so memory follows the live contexts instead of ``n_seats * seat_len``.

* ``table`` is a device-resident ``[max_seats + 1, max_pages_per_seat]`` int32 block table (row ``max_seats`` is the
  scratch seat that padded rows use, engine/talker.py:27, 110-111; all its entries point at the reserved scratch
  page).  Unallocated entries hold -1 (the decode kernels treat out-of-range page ids as "no tokens").
* ``grow`` / ``release`` run on the host between frames and push only the changed table entries to the device
  (one indexed write per call).
* ``block_table(seat)`` and ``slot(seat, pos)`` are plain tensor ops on device tensors, so a captured frame graph
  computes its rows' tables and append slots from the device-resident seat ids and positions, as
  ``Talker._frame`` does (engine/talker.py:107-112).

The pool tensors themselves (``[num_pages, page_size, kv_heads, head_dim]`` per layer) are the caller's; this class
only decides which page ids hold which seat's tokens.
"""
from __future__ import annotations

import numpy as np
import torch


class PoolExhausted(RuntimeError):
    """No free page is left for a seat that must grow."""


class PagePool:
    SCRATCH_PAGE = 0

    def __init__(self, num_pages: int, max_seats: int, max_pages_per_seat: int, page_size: int = 16,
                 device="cuda"):
        if page_size < 16 or page_size & (page_size - 1):
            raise ValueError(f"page_size {page_size} must be a power of two >= 16")
        if num_pages < 2 or max_seats < 1 or max_pages_per_seat < 1:
            raise ValueError("need num_pages >= 2 (one is the scratch page), max_seats >= 1, max_pages_per_seat >= 1")
        self.num_pages, self.max_seats, self.max_pages, self.page_size = num_pages, max_seats, max_pages_per_seat, page_size
        self.scratch_seat = max_seats
        self.device = torch.device(device)
        # Free list as a stack; low page ids are handed out first.
        self._free = list(range(num_pages - 1, self.SCRATCH_PAGE, -1))
        self._pages = [[] for _ in range(max_seats)]          # host copy of each seat's page list
        host = np.full((max_seats + 1, max_pages_per_seat), -1, np.int32)
        host[max_seats, :] = self.SCRATCH_PAGE
        self.table = torch.from_numpy(host).to(self.device)

    # ------------------------------------------------------------------ host-side bookkeeping
    @property
    def seat_len(self) -> int:
        """Positions one seat can hold."""
        return self.max_pages * self.page_size

    @property
    def free_pages(self) -> int:
        return len(self._free)

    def pages_of(self, seat: int) -> list:
        return list(self._pages[seat])

    def capacity(self, seat: int) -> int:
        """Positions seat ``seat`` can hold with its current pages."""
        return len(self._pages[seat]) * self.page_size

    def grow(self, seats, lengths) -> None:
        """Give each seat enough pages for ``length`` positions (0..length-1).  All-or-nothing: raises
        PoolExhausted (changing nothing) when the free list cannot cover the request."""
        seats = [int(s) for s in np.atleast_1d(seats)]
        lengths = [int(n) for n in np.atleast_1d(lengths)]
        if len(seats) != len(lengths):
            raise ValueError("seats and lengths differ in length")
        need = {}
        for s, n in zip(seats, lengths):
            if not 0 <= s < self.max_seats:
                raise IndexError(f"seat {s} outside [0, {self.max_seats})")
            if n > self.seat_len:
                raise ValueError(f"seat {s}: length {n} exceeds {self.seat_len} positions")
            want = -(-max(n, 0) // self.page_size)
            need[s] = max(need.get(s, 0), want)
        extra = sum(max(0, w - len(self._pages[s])) for s, w in need.items())
        if extra > len(self._free):
            raise PoolExhausted(f"{extra} pages needed, {len(self._free)} free")
        rows, cols, vals = [], [], []
        for s, w in need.items():
            pl = self._pages[s]
            while len(pl) < w:
                p = self._free.pop()
                rows.append(s)
                cols.append(len(pl))
                vals.append(p)
                pl.append(p)
        self._write(rows, cols, vals)

    def release(self, seats) -> None:
        """Return the seats' pages to the free list and clear their table rows."""
        rows, cols, vals = [], [], []
        for s in (int(x) for x in np.atleast_1d(seats)):
            if not 0 <= s < self.max_seats:
                raise IndexError(f"seat {s} outside [0, {self.max_seats})")
            pl = self._pages[s]
            for i in range(len(pl)):
                rows.append(s)
                cols.append(i)
                vals.append(-1)
            self._free.extend(reversed(pl))
            self._pages[s] = []
        self._write(rows, cols, vals)

    def _write(self, rows, cols, vals) -> None:
        if not rows:
            return
        idx_r = torch.tensor(rows, dtype=torch.long)
        idx_c = torch.tensor(cols, dtype=torch.long)
        v = torch.tensor(vals, dtype=torch.int32)
        if self.device.type != "cpu":
            idx_r, idx_c, v = (t.pin_memory().to(self.device, non_blocking=True) for t in (idx_r, idx_c, v))
        self.table.index_put_((idx_r, idx_c), v)

    def check(self) -> None:
        """Invariant check (tests and debugging): every page is free, scratch, or owned by exactly one seat, and
        the device table matches the host lists."""
        owned = [p for pl in self._pages for p in pl]
        all_ids = owned + self._free + [self.SCRATCH_PAGE]
        if sorted(all_ids) != list(range(self.num_pages)):
            raise AssertionError("page accounting broken: pages lost or handed out twice")
        host = self.table.cpu().numpy()
        for s, pl in enumerate(self._pages):
            row = host[s]
            if list(row[: len(pl)]) != pl or (row[len(pl):] != -1).any():
                raise AssertionError(f"device table row {s} differs from the host page list")

    # ------------------------------------------------------------------ device-side views (graph-capturable)
    def block_table(self, seat: torch.Tensor) -> torch.Tensor:
        """Rows of the block table for a batch of seat ids (int64 device tensor) -> [B, max_pages] int32."""
        return self.table.index_select(0, seat)

    def slot(self, seat: torch.Tensor, pos: torch.Tensor) -> torch.Tensor:
        """Flat append slot (page * page_size + offset) of position ``pos`` of each seat, int64: the index the
        reference computes as ``seat * seat_len + pos`` (engine/talker.py:109) for its identity table."""
        page = self.table[seat, torch.div(pos, self.page_size, rounding_mode="floor")].long()
        return page * self.page_size + pos % self.page_size
