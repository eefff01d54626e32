"""Page-table packing: per-row KV page spans -> (indptr, indices, last_page_len).

Same contract as the reference's ``model/kvcache/flashinfer_page_table.py``:
``indptr[B+1]`` is the prefix sum of pages per row, ``indices`` lists each
row's physical page ids in logical order, ``last_page_len[B]`` is the fill of
each row's final page; every span must start at page offset 0 and only the
last page of a row may be partial (``_validate_and_collect_page_table``,
flashinfer_page_table.py:200-221, after merging adjacent slices of one page,
``_coalesce_block_spans`` :184-197).

The MI355X difference is the upload: tables are packed into reusable pinned
host staging buffers and copied to persistent device buffers with one
asynchronous H2D per tensor, instead of ``torch.tensor(list, device=cuda)``
from pageable memory every step (flashinfer_page_table.py:106-116).
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Iterable, Sequence

import numpy as np
import torch


@dataclass(frozen=True)
class KVBlockSpan:
    """A slice [start, start + length) of physical KV page ``block_id``.

    Same fields as the reference's ``KVBlockSpan`` (model/kvcache/radix_types.py:31-36).
    """

    block_id: int
    start: int
    length: int


@dataclass(frozen=True)
class PageTable:
    """Page-table tensors handed to ``plan_decode`` (flashinfer_page_table.py:12-18)."""

    paged_kv_indptr: torch.Tensor
    paged_kv_indices: torch.Tensor
    paged_kv_last_page_len: torch.Tensor


def _row_pages(spans: Iterable[KVBlockSpan], page_size: int) -> tuple[list[int], int]:
    """Validate one row's spans; return (page ids, fill of the last page).

    Adjacent slices of the same page are merged first, so a page written in
    two appends (prefix part + decode token) counts once.
    """

    if page_size <= 0:
        raise ValueError("page_size must be positive")
    pages: list[int] = []
    fills: list[int] = []
    for span in spans:
        if span.length <= 0:
            continue
        if pages and pages[-1] == span.block_id and fills[-1] == span.start:
            fills[-1] += span.length  # continues the previous slice of this page
            continue
        if span.start != 0:
            raise ValueError("page spans must start at page offset 0")
        pages.append(int(span.block_id))
        fills.append(int(span.length))
    for i, fill in enumerate(fills):
        if fill <= 0 or fill > page_size:
            raise ValueError("page span length is out of range")
        if i < len(fills) - 1 and fill != page_size:
            raise ValueError("non-last page spans must be full pages")
    return pages, (fills[-1] if fills else 0)


def pack_rows(batch_spans: Sequence[Sequence[KVBlockSpan]], page_size: int) -> tuple[np.ndarray, np.ndarray, np.ndarray]:
    """Pack rows into int32 numpy arrays (indptr, indices, last_page_len)."""

    counts = np.zeros(len(batch_spans) + 1, dtype=np.int64)
    all_pages: list[int] = []
    last = np.zeros(len(batch_spans), dtype=np.int32)
    for b, spans in enumerate(batch_spans):
        pages, fill = _row_pages(spans, page_size)
        all_pages.extend(pages)
        counts[b + 1] = len(pages)
        last[b] = fill
    indptr = np.cumsum(counts).astype(np.int32)
    return indptr, np.asarray(all_pages, dtype=np.int32), last


def build_page_table(
    spans: Sequence[KVBlockSpan],
    *,
    page_size: int,
    device: torch.device | str = "cpu",
    pin_memory: bool = False,
) -> PageTable:
    """Single-row table (flashinfer_page_table.py:137-157)."""

    return build_batch_page_table([spans], page_size=page_size, device=device, pin_memory=pin_memory)


def build_batch_page_table(
    batch_spans: Sequence[Sequence[KVBlockSpan]],
    *,
    page_size: int,
    device: torch.device | str = "cpu",
    pin_memory: bool = False,
) -> PageTable:
    """Batched table built into fresh tensors (flashinfer_page_table.py:160-181)."""

    indptr, indices, last = pack_rows(batch_spans, page_size)
    device = torch.device(device)

    def to_tensor(a: np.ndarray) -> torch.Tensor:
        t = torch.from_numpy(a.copy())
        if pin_memory and device.type == "cpu":
            t = t.pin_memory()
        return t.to(device) if device.type != "cpu" else t

    return PageTable(to_tensor(indptr), to_tensor(indices), to_tensor(last))


class BatchPageTableBuffer:
    """Reusable batched page-table buffers (flashinfer_page_table.py:68-134).

    Device buffers grow by doubling; a growth replaces the tensors (and so
    their data pointers, which is why graph keys include them).  Host
    staging buffers are pinned so each update is three asynchronous copies
    on the current stream.  A staging buffer is not rewritten until the copy
    that reads it has completed (an event per buffer generation).
    """

    def __init__(
        self,
        *,
        page_size: int,
        device: torch.device | str,
        initial_rows: int = 2,
        initial_pages: int = 16,
    ) -> None:
        if page_size <= 0:
            raise ValueError("page_size must be positive")
        self.page_size = int(page_size)
        self.device = torch.device(device)
        self._rows = max(1, int(initial_rows))
        self._pages = max(1, int(initial_pages))
        self._alloc_rows()
        self._alloc_pages()
        self._stage = None
        self._stage_event = None

    # Row and page capacities grow independently, as in the reference
    # (_ensure_row_capacity / _ensure_page_capacity, :123-134).
    def _alloc_rows(self) -> None:
        self.paged_kv_indptr = torch.zeros(self._rows + 1, dtype=torch.int32, device=self.device)
        self.paged_kv_last_page_len = torch.zeros(self._rows, dtype=torch.int32, device=self.device)

    def _alloc_pages(self) -> None:
        self.paged_kv_indices = torch.zeros(self._pages, dtype=torch.int32, device=self.device)

    def signature(self) -> tuple[int, int, int]:
        return (
            self.paged_kv_indptr.data_ptr(),
            self.paged_kv_indices.data_ptr(),
            self.paged_kv_last_page_len.data_ptr(),
        )

    def update_from_batch_spans(self, batch_spans: Sequence[Sequence[KVBlockSpan]]) -> PageTable:
        indptr, indices, last = pack_rows(batch_spans, self.page_size)
        return self.update_from_arrays(indptr, indices, last)

    def update_from_spans(self, spans: Sequence[KVBlockSpan]) -> PageTable:
        return self.update_from_batch_spans([spans])

    def update_from_arrays(self, indptr: np.ndarray, indices: np.ndarray, last: np.ndarray) -> PageTable:
        rows = len(last)
        pages = len(indices)
        if rows > self._rows:
            self._rows = max(rows, self._rows * 2)
            self._alloc_rows()
        if pages > self._pages:
            self._pages = max(pages, self._pages * 2)
            self._alloc_pages()
        if self.device.type == "cpu":
            self.paged_kv_indptr[: rows + 1].copy_(torch.from_numpy(indptr))
            self.paged_kv_last_page_len[:rows].copy_(torch.from_numpy(last))
            self.paged_kv_indices[:pages].copy_(torch.from_numpy(indices))
        else:
            stage = self._staging(rows, pages)
            n_ip, n_pg, n_ls = rows + 1, pages, rows
            stage[0][:n_ip].numpy()[:] = indptr
            stage[1][:n_pg].numpy()[:] = indices
            stage[2][:n_ls].numpy()[:] = last
            self.paged_kv_indptr[:n_ip].copy_(stage[0][:n_ip], non_blocking=True)
            if n_pg:
                self.paged_kv_indices[:n_pg].copy_(stage[1][:n_pg], non_blocking=True)
            self.paged_kv_last_page_len[:n_ls].copy_(stage[2][:n_ls], non_blocking=True)
            self._stage_event = torch.cuda.Event()
            self._stage_event.record(torch.cuda.current_stream(self.device))
        return PageTable(
            self.paged_kv_indptr[: rows + 1],
            self.paged_kv_indices[:pages],
            self.paged_kv_last_page_len[:rows],
        )

    def _staging(self, rows: int, pages: int):
        if self._stage_event is not None:
            self._stage_event.synchronize()  # previous upload still reads the staging buffers
        if self._stage is None or self._stage[0].numel() < rows + 1 or self._stage[1].numel() < max(pages, 1):
            cap_rows = max(rows, self._rows)
            cap_pages = max(pages, self._pages, 1)
            self._stage = (
                torch.empty(cap_rows + 1, dtype=torch.int32, pin_memory=True),
                torch.empty(cap_pages, dtype=torch.int32, pin_memory=True),
                torch.empty(cap_rows, dtype=torch.int32, pin_memory=True),
            )
        return self._stage


class PageTableBuffer(BatchPageTableBuffer):
    """Single-request variant (flashinfer_page_table.py:21-65)."""

    def __init__(self, *, page_size: int, device: torch.device | str, initial_capacity: int = 16) -> None:
        super().__init__(page_size=page_size, device=device, initial_rows=1, initial_pages=initial_capacity)


# ------------------------------------------------ device-side advance ---
# Status bits written by pl_page_table_advance.
ADVANCE_MISSING_PAGE = 1  # a row needed a page and its reserve slot held -1
ADVANCE_NO_ROOM = 2       # the table would outgrow its indices buffer
ADVANCE_BAD_TABLE = 4     # indptr decreasing / out of range, or a bad last_page_len

MAX_ADVANCE_ROWS = 4096


def _need(t: torch.Tensor, name: str, dtype: torch.dtype, shape=None, min_numel: int = 0) -> None:
    if t.device.type != "cuda":
        raise RuntimeError(f"{name} must be on a ROCm device")
    if t.dtype != dtype:
        raise ValueError(f"{name} must be {dtype}, got {t.dtype}")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")
    if shape is not None and tuple(t.shape) != tuple(shape):
        raise ValueError(f"{name} must have shape {tuple(shape)}, got {tuple(t.shape)}")
    if t.numel() < min_numel:
        raise ValueError(f"{name} needs at least {min_numel} elements")


def page_table_advance(
    paged_kv_indptr: torch.Tensor,
    paged_kv_indices: torch.Tensor,
    paged_kv_last_page_len: torch.Tensor,
    page_size: int,
    reserve: torch.Tensor,
    reserve_head: torch.Tensor,
    positions: torch.Tensor,
    page_id: torch.Tensor,
    page_offset: torch.Tensor,
    status: torch.Tensor,
) -> None:
    """Append one decode token to every row of a device page table, in place.

    The device-side replacement of the reference's per-step
    ``reserve_chunk(request, 1)`` + ``update_from_batch_spans`` (generation.py:
    1011-1035; paged_kv_store.py:113-190; flashinfer_page_table.py:89-121):
    a row whose last page is full (or that has none) takes its next page from
    ``reserve[b, reserve_head[b] % slots]`` (int32, the slot is then set to
    -1); every row's token position and KV slot go to ``positions`` /
    ``page_id`` / ``page_offset`` (int64 [B]).  Errors found on the device
    set bits of ``status[0]`` (ADVANCE_*) and leave the table unchanged.
    Enqueued on the current stream; nothing is read back.
    """
    from . import _lib

    lib = _lib.load()
    batch = paged_kv_last_page_len.numel()
    if batch > MAX_ADVANCE_ROWS:
        raise NotImplementedError(f"batch {batch} exceeds {MAX_ADVANCE_ROWS} rows")
    _need(paged_kv_indptr, "paged_kv_indptr", torch.int32, (batch + 1,))
    _need(paged_kv_indices, "paged_kv_indices", torch.int32, min_numel=1)
    _need(paged_kv_last_page_len, "paged_kv_last_page_len", torch.int32, (batch,))
    if reserve.dim() != 2 or reserve.shape[0] != batch or reserve.shape[1] < 1:
        raise ValueError(f"reserve must be [batch={batch}, slots >= 1], got {tuple(reserve.shape)}")
    _need(reserve, "reserve", torch.int32)
    _need(reserve_head, "reserve_head", torch.int32, (batch,))
    for name, t in (("positions", positions), ("page_id", page_id), ("page_offset", page_offset)):
        _need(t, name, torch.int64, (batch,))
    _need(status, "status", torch.int32, min_numel=1)
    st = lib.pl_page_table_advance(
        paged_kv_indptr.data_ptr(), paged_kv_indices.data_ptr(), paged_kv_indices.numel(),
        paged_kv_last_page_len.data_ptr(), batch, int(page_size), reserve.data_ptr(), reserve.shape[1],
        reserve_head.data_ptr(), positions.data_ptr(), page_id.data_ptr(), page_offset.data_ptr(),
        status.data_ptr(), _lib.stream_handle(paged_kv_indptr.device),
    )
    _lib.check(st, "pl_page_table_advance")


class PageReserve:
    """Per-row rings of pages the device takes as decode rows grow.

    ``reserve[b, s]`` holds a page id or -1, ``head[b]`` counts the pages
    row b has taken (its next page is slot ``head[b] % slots``), ``status``
    collects the ADVANCE_* bits.  The host writes whole ring snapshots with
    :meth:`upload` (one asynchronous copy from pinned memory); a snapshot
    must repeat every page the device has not taken yet, in its slot.
    """

    def __init__(self, batch: int, slots: int, device) -> None:
        if batch < 1 or slots < 1:
            raise ValueError("batch and slots must be >= 1")
        self.batch, self.slots = int(batch), int(slots)
        self.device = torch.device(device)
        self.reserve = torch.full((self.batch, self.slots), -1, dtype=torch.int32, device=self.device)
        self.head = torch.zeros(self.batch, dtype=torch.int32, device=self.device)
        self.status = torch.zeros(1, dtype=torch.int32, device=self.device)
        self._stage = [torch.empty((self.batch, self.slots), dtype=torch.int32, pin_memory=True) for _ in range(2)]
        self._events: list = [None, None]
        self._next = 0

    def reset(self) -> None:
        """Empty rings, zero heads and status (enqueued on the current stream)."""
        self.reserve.fill_(-1)
        self.head.zero_()
        self.status.zero_()

    def upload(self, ring: np.ndarray) -> None:
        """Copy a host snapshot [batch, slots] of the rings to the device."""
        i = self._next
        self._next ^= 1
        if self._events[i] is not None:
            self._events[i].synchronize()  # the copy that last read this staging buffer has run
        self._stage[i].numpy()[:] = ring
        self.reserve.copy_(self._stage[i], non_blocking=True)
        ev = torch.cuda.Event()
        ev.record(torch.cuda.current_stream(self.device))
        self._events[i] = ev

    def check(self) -> None:
        """Raise if any advance since the last reset failed (reads back: synchronizes)."""
        bits = int(self.status.item())
        if bits:
            what = [n for b, n in ((ADVANCE_MISSING_PAGE, "a row found no reserved page"),
                                   (ADVANCE_NO_ROOM, "the page table outgrew its buffer"),
                                   (ADVANCE_BAD_TABLE, "the page table was malformed")) if bits & b]
            raise RuntimeError("device page-table advance failed: " + "; ".join(what))
