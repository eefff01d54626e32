"""CPU side of the device page-table advance.

(1) Pins oracle.page_table.advance_table: after k steps a row that started
    with L tokens holds ceil((L+k)/ps) pages, its last page is filled to
    (L+k) - ps*(pages-1), and step s wrote position L+s into slot
    (pages[(L+s) // ps], (L+s) % ps), with new pages taken in order.
(2) The generator's reserve feeder against a model of the device ring:
    the ring is refilled ahead of every page a row takes, a refill never
    changes a page the device has not taken yet, uploads happen about once
    per page of steps, and the table grown from the ring equals the host
    pool's own table at the end.
"""

import numpy as np
import pytest
import torch

from oracle import page_table as opt
from pagelora_amd.generation import _ReserveFeeder
from pagelora_amd.kv_pool import PagedKVPool, Request


def _rows(lengths, ps, start=1000):
    rows, nxt = [], start
    for L in lengths:
        n = -(-L // ps)
        rows.append([(nxt + i, 0, ps if i < n - 1 else L - ps * (n - 1)) for i in range(n)])
        nxt += n
    return rows, nxt


@pytest.mark.parametrize("ps", [1, 4, 16])
def test_oracle_advance_closed_form(ps):
    rng = np.random.default_rng(ps)
    lengths = [0, ps, ps + 1, 2 * ps - 1] + rng.integers(0, 5 * ps, size=8).tolist()
    rows, nxt = _rows(lengths, ps)
    indptr, indices, last = opt.build_batch_page_table(rows, ps)
    steps = 3 * ps + 2
    new = [list(range(nxt + 100 * b, nxt + 100 * b + 50)) for b in range(len(lengths))]
    pages = [[s[0] for s in r] for r in rows]
    for s in range(steps):
        q = [list(x) for x in new]
        indptr, indices, last, pos, pid, off = opt.advance_table(indptr, indices, last, ps, q)
        for b, L in enumerate(lengths):
            taken = len(new[b]) - len(q[b])
            pages[b] += new[b][:taken]
            new[b] = q[b]
            t = L + s  # the token this step wrote
            assert pos[b] == t
            assert (pid[b], off[b]) == (pages[b][t // ps], t % ps)
    for b, L in enumerate(lengths):
        n = -(-(L + steps) // ps)
        assert indptr[b + 1] - indptr[b] == n == len(pages[b])
        assert indices[indptr[b]:indptr[b + 1]] == pages[b]
        assert last[b] == (L + steps) - ps * (n - 1)


class _RingModel:
    """The device side of PageReserve: ring, head cursor, the advance."""

    def __init__(self, batch, slots):
        self.batch, self.slots = batch, slots
        self.ring = np.full((batch, slots), -1, dtype=np.int32)
        self.head = [0] * batch
        self.uploads = 0

    def upload(self, snap):
        for b in range(self.batch):
            for s in range(self.slots):
                if self.ring[b, s] >= 0:  # a page not taken yet must be repeated as is
                    assert snap[b, s] == self.ring[b, s], (b, s)
        self.ring = snap.copy()
        self.uploads += 1

    def take(self, b):
        s = self.head[b] % self.slots
        page = int(self.ring[b, s])
        assert page >= 0, f"row {b} found no reserved page"
        self.ring[b, s] = -1
        self.head[b] += 1
        return page


@pytest.mark.parametrize("slots", [2, 3, 5])
def test_feeder_keeps_rings_ahead(slots):
    ps = 16
    pool = PagedKVPool(num_layers=1, capacity_pages=512, page_size=ps, num_kv_heads=1, head_dim=8,
                       dtype=torch.float32, device="cpu")
    prefix = Request()
    pool.reserve(prefix, 32)  # two shared full pages
    reqs = []
    for n in (0, 1, 15, 16, 17, 40):
        r = Request(prefix_pages=list(prefix.own_pages), prefix_len=32, length=32)
        pool.reserve(r, n)
        reqs.append(r)
    reqs.append(Request())  # a row with no tokens at all
    indptr, indices, last = (a.tolist() for a in pool.tables(reqs))
    lengths0 = [r.length for r in reqs]
    steps = 100
    ring = _RingModel(len(reqs), slots)
    feeder = _ReserveFeeder(pool, reqs, ring, steps)
    for s in range(steps):
        feeder.before_step(s)
        takers = [[ring.take(b)] if (lengths0[b] + s) % ps == 0 else [] for b in range(len(reqs))]
        indptr, indices, last, *_ = opt.advance_table(indptr, indices, last, ps, takers)
        assert all(not t for t in takers)  # every page given was taken
    assert [r.length for r in reqs] == [L + steps for L in lengths0]
    ip, ind, ls = pool.tables(reqs)
    assert ip.tolist() == indptr and ind.tolist() == indices and ls.tolist() == last
    # a refill covers (slots - 1) pages of steps and comes when less than a
    # page of steps is left: one upload per (slots - 2) pages of steps
    if slots > 2:
        assert ring.uploads <= -(-steps // ((slots - 2) * ps)) + 1, ring.uploads
    assert ring.uploads <= steps
