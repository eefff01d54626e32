"""Device-side page-table advance (pl_page_table_advance) against the oracle.

Each case builds a ragged batch table (empty rows, rows ending on a full
page, rows mid-page), advances it step after step on the device and checks
every step bit-exactly against oracle.page_table.advance_table (the
reference's reserve_spans(1) + repack): indptr, indices, last_page_len, the
token positions and KV slots, and the consumed reserve slots.  Sizes cover
one-tile and many-tile moves (8192 entries per tile) and the 4096-row
maximum.  Error cases are forced from the host (an empty reserve slot, a
full indices buffer, a malformed table): the kernel reports them in status
and leaves the table unchanged.
"""

import numpy as np
import pytest
import torch

from oracle import page_table as opt
from pagelora_amd.page_table import (ADVANCE_BAD_TABLE, ADVANCE_MISSING_PAGE, ADVANCE_NO_ROOM, PageReserve,
                                     page_table_advance)

pytestmark = pytest.mark.gpu


def _table(lengths, ps, rng):
    pages = [-(-L // ps) for L in lengths]
    ids = rng.permutation(sum(pages) + 10 * len(lengths) + 1000).astype(np.int64)
    rows, used = [], 0
    for L, n in zip(lengths, pages):
        row = ids[used:used + n].tolist()
        used += n
        rows.append([(p, 0, ps if i < n - 1 else L - ps * (n - 1)) for i, p in enumerate(row)])
    indptr, indices, last = opt.build_batch_page_table(rows, ps)
    return indptr, indices, last, ids[used:].tolist()


class _Device:
    def __init__(self, dev, indptr, indices, last, capacity, slots, batch):
        self.indptr = torch.tensor(indptr, dtype=torch.int32, device=dev)
        self.indices = torch.zeros(capacity, dtype=torch.int32, device=dev)
        self.indices[: len(indices)] = torch.tensor(indices, dtype=torch.int32)
        # rows without pages carry an arbitrary fill: the kernel must not read it
        self.last = torch.tensor([x if x else 7 for x in last], dtype=torch.int32, device=dev)
        self.reserve = torch.full((batch, slots), -1, dtype=torch.int32, device=dev)
        self.head = torch.zeros(batch, dtype=torch.int32, device=dev)
        self.pos = torch.full((batch,), -5, dtype=torch.int64, device=dev)
        self.pid = torch.full((batch,), -5, dtype=torch.int64, device=dev)
        self.off = torch.full((batch,), -5, dtype=torch.int64, device=dev)
        self.status = torch.zeros(1, dtype=torch.int32, device=dev)

    def advance(self, ps):
        page_table_advance(self.indptr, self.indices, self.last, ps, self.reserve, self.head, self.pos, self.pid,
                           self.off, self.status)


def _run_steps(dev, lengths, ps, steps, slots, seed, head0=None):
    """Advance `steps` times, refilling each row's ring from the host before
    every step; compare everything with the oracle after each step."""
    rng = np.random.default_rng(seed)
    B = len(lengths)
    indptr, indices, last, free = _table(lengths, ps, rng)
    need = [max(0, -(-(L + steps) // ps) - (-(-L // ps))) for L in lengths]
    capacity = len(indices) + sum(need) + 3
    d = _Device(dev, indptr, indices, last, capacity, slots, B)
    head = np.zeros(B, dtype=np.int64) if head0 is None else np.asarray(head0, dtype=np.int64)
    d.head.copy_(torch.tensor(head, dtype=torch.int32))
    queues = []  # the pages each row will take, in order
    for n in need:
        queues.append(free[:n])
        free = free[n:]
    taken = [0] * B
    for step in range(steps):
        # host refill: the next `slots` pages of every row at slot (head + k) % slots
        ring = np.full((B, slots), -1, dtype=np.int32)
        for b in range(B):
            for k in range(taken[b], min(len(queues[b]), taken[b] + slots)):
                ring[b, (head[b] + k - taken[b]) % slots] = queues[b][k]
        d.reserve.copy_(torch.from_numpy(ring))
        oracle_pages = [list(queues[b][taken[b]:]) for b in range(B)]
        before = [len(q) for q in oracle_pages]
        indptr, indices, last, pos, pid, off = opt.advance_table(indptr, indices, last, ps, oracle_pages)
        d.advance(ps)
        torch.cuda.synchronize()
        assert int(d.status.item()) == 0, f"step {step}: status {int(d.status.item())}"
        tot = indptr[-1]
        assert d.indptr.tolist() == indptr, f"step {step}: indptr"
        assert d.indices[:tot].tolist() == indices, f"step {step}: indices"
        got_last = d.last.tolist()
        assert got_last == last, f"step {step}: last_page_len"
        assert d.pos.tolist() == pos and d.pid.tolist() == pid and d.off.tolist() == off, f"step {step}: slots"
        for b in range(B):
            grew = before[b] - len(oracle_pages[b])
            if grew:
                slot = head[b] % slots
                assert int(d.reserve[b, slot]) == -1, "a taken slot is cleared"
                head[b] += 1
                taken[b] += 1
        assert d.head.tolist() == head.tolist()
    return indptr, indices, last


def test_advance_small_ragged(gpu_device):
    # empty rows, full last pages, mid-page rows, one-token rows
    lengths = [0, 1, 15, 16, 17, 32, 0, 33, 5, 48]
    _run_steps(gpu_device, lengths, 16, steps=40, slots=3, seed=1)


@pytest.mark.parametrize("ps", [1, 3, 16])
def test_advance_page_sizes(gpu_device, ps):
    rng = np.random.default_rng(ps)
    lengths = rng.integers(0, 60, size=37).tolist()
    _run_steps(gpu_device, lengths, ps, steps=2 * ps + 5, slots=2, seed=ps)


def test_advance_ring_wraps_from_any_head(gpu_device):
    rng = np.random.default_rng(5)
    lengths = rng.integers(0, 100, size=20).tolist()
    _run_steps(gpu_device, lengths, 4, steps=30, slots=3, seed=5, head0=rng.integers(0, 1000, size=20).tolist())


def test_advance_many_tiles(gpu_device):
    # batch 64 of the ragged headline shape: ~20k entries = 3 move tiles; 40 steps
    rng = np.random.default_rng(11)
    lengths = rng.integers(128, 8193, size=64).tolist()
    lengths[::7] = [16 * (x // 16) for x in lengths[::7]]  # some rows end on a full page
    _run_steps(gpu_device, lengths, 16, steps=20, slots=2, seed=11)


def test_advance_max_rows(gpu_device):
    rng = np.random.default_rng(12)
    lengths = rng.integers(0, 300, size=4096).tolist()
    lengths[::3] = [16 * (x // 16) for x in lengths[::3]]
    _run_steps(gpu_device, lengths, 16, steps=3, slots=2, seed=12)


def _snapshot(d):
    return d.indptr.tolist(), d.indices.tolist(), d.last.tolist()


def test_advance_missing_page_leaves_table(gpu_device):
    rng = np.random.default_rng(2)
    indptr, indices, last, free = _table([16, 5, 32], 16, rng)
    d = _Device(gpu_device, indptr, indices, last, 64, 2, 3)
    d.reserve[0, 0] = free[0]  # row 0 has its page, row 2 (also full) has none
    before = _snapshot(d)
    d.advance(16)
    torch.cuda.synchronize()
    assert int(d.status.item()) == ADVANCE_MISSING_PAGE
    assert _snapshot(d) == before
    assert d.pid.tolist() == [-1, -1, -1] and d.off.tolist() == [-1, -1, -1]
    assert d.head.tolist() == [0, 0, 0] and int(d.reserve[0, 0]) == free[0]


def test_advance_no_room(gpu_device):
    rng = np.random.default_rng(3)
    indptr, indices, last, free = _table([16, 5], 16, rng)
    d = _Device(gpu_device, indptr, indices, last, len(indices), 1, 2)  # full buffer
    d.reserve[0, 0] = free[0]
    before = _snapshot(d)
    d.advance(16)
    torch.cuda.synchronize()
    assert int(d.status.item()) == ADVANCE_NO_ROOM
    assert _snapshot(d) == before
    # a mid-page row alone needs no room: advancing row 1 only works
    d2 = _Device(gpu_device, [0, 1], indices[1:2], last[1:2], 1, 1, 1)
    d2.advance(16)
    torch.cuda.synchronize()
    assert int(d2.status.item()) == 0 and d2.last.tolist() == [6]


@pytest.mark.parametrize("bad", ["last0", "last_big", "decreasing", "beyond"])
def test_advance_malformed_table(gpu_device, bad):
    indptr, indices, last = [0, 2, 3], [4, 5, 6], [16, 3]
    if bad == "last0":
        last = [0, 3]
    elif bad == "last_big":
        last = [17, 3]
    elif bad == "decreasing":
        indptr = [0, 3, 2]
    else:
        indptr = [0, 2, 9]
    d = _Device(gpu_device, indptr, indices, last, 8, 1, 2)
    d.last.copy_(torch.tensor(last, dtype=torch.int32))
    d.reserve[:, 0] = 40
    before = _snapshot(d)
    d.advance(16)
    torch.cuda.synchronize()
    assert int(d.status.item()) & ADVANCE_BAD_TABLE
    assert _snapshot(d) == before
    assert d.pid.tolist() == [-1, -1]


def test_advance_host_validation(gpu_device):
    d = _Device(gpu_device, [0, 1], [3], [2], 4, 1, 1)
    with pytest.raises(ValueError):
        page_table_advance(d.indptr, d.indices, d.last, 16, d.reserve.view(-1), d.head, d.pos, d.pid, d.off,
                           d.status)
    with pytest.raises(ValueError):
        page_table_advance(d.indptr, d.indices, d.last, 16, d.reserve, d.head, d.pos.int(), d.pid, d.off,
                           d.status)
    with pytest.raises(ValueError):
        page_table_advance(d.indptr, d.indices, d.last, 0, d.reserve, d.head, d.pos, d.pid, d.off, d.status)
    big = 4097
    with pytest.raises(NotImplementedError):
        page_table_advance(torch.zeros(big + 1, dtype=torch.int32, device=gpu_device), d.indices,
                           torch.ones(big, dtype=torch.int32, device=gpu_device), 16,
                           torch.zeros((big, 1), dtype=torch.int32, device=gpu_device),
                           torch.zeros(big, dtype=torch.int32, device=gpu_device),
                           *(torch.zeros(big, dtype=torch.int64, device=gpu_device) for _ in range(3)), d.status)


def test_page_reserve_check_raises(gpu_device):
    r = PageReserve(2, 2, gpu_device)
    r.check()
    r.status.fill_(ADVANCE_MISSING_PAGE | ADVANCE_NO_ROOM)
    with pytest.raises(RuntimeError, match="no reserved page"):
        r.check()
    r.reset()
    r.check()
    r.upload(np.array([[3, -1], [4, 5]], dtype=np.int32))
    assert r.reserve.tolist() == [[3, -1], [4, 5]]
