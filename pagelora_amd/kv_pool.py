"""Paged KV pool, page allocator and per-request spans.

Layout of the pool (``model/kvcache/paged_kv_store.py:559-570``): one dense
tensor ``[num_layers, capacity_pages, 2, page_size, num_kv_heads, head_dim]``;
``pool[l]`` is the NHD layer view the decode kernels read, with K at index
0 and V at index 1 of dim 2 (``layer_runner.py:411-412``).

Size the pool for the whole workload up front (288 GB of HBM makes that
the normal case): its data pointer then stays fixed and a captured decode
graph replays for the life of the engine.  When it does run out, it grows
as the reference's does (``paged_kv_store.py:304-330, 543-579``): a new
tensor of ``max(16, 2 x capacity, required)`` pages, or exactly
``max_pages`` when capped, with the old pages copied in place, so every
page id stays valid.  The move changes the pool's data pointer, which is
part of every decode graph key, so the next step recaptures once.

Requests own page spans (``KVBlockSpan``); rows may share prefix pages
(``paged_kvcache_manager.py:324-333``), which are read-only to decode.
"""

from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np
import torch

from .page_table import KVBlockSpan, pack_rows


class PageAllocator:
    """Free-list page allocator (paged_kv_allocator.py:22-73 semantics:
    allocate n pages or fail atomically, free returns pages to the list).

    Page 0 is never handed out: it is the scratch slot that graph warm-up
    runs append their (discarded) K/V into.  ``grow(required_pages)``, when
    given, is called when the free list runs short; it returns the new
    capacity, whose pages join the free list (lowest ids handed out first).
    """

    def __init__(self, capacity: int, grow=None) -> None:
        self.capacity = int(capacity)
        self._free = list(range(self.capacity - 1, 0, -1))
        self._grow = grow

    @property
    def free_pages(self) -> int:
        return len(self._free)

    def allocate(self, n: int) -> list[int]:
        if n > len(self._free):
            if self._grow is None:
                raise RuntimeError(f"paged KV pool exhausted: need {n} pages, {len(self._free)} free")
            new_cap = int(self._grow(self.capacity + n - len(self._free)))
            self._free = list(range(new_cap - 1, self.capacity - 1, -1)) + self._free
            self.capacity = new_cap
        out = [self._free.pop() for _ in range(n)]
        return out

    def free(self, pages) -> None:
        self._free.extend(int(p) for p in pages)


@dataclass
class Request:
    """One sequence's pages: shared prefix pages (read-only) + own pages."""

    prefix_pages: list[int] = field(default_factory=list)
    prefix_len: int = 0          # tokens held by the prefix pages (a multiple of page_size)
    own_pages: list[int] = field(default_factory=list)
    length: int = 0              # total tokens (prefix + own)

    def pages(self) -> list[int]:
        return self.prefix_pages + self.own_pages

    def spans(self, page_size: int) -> list[KVBlockSpan]:
        out = []
        remaining = self.length
        for p in self.pages():
            n = min(page_size, remaining)
            if n <= 0:
                break
            out.append(KVBlockSpan(p, 0, n))
            remaining -= n
        return out

    def slot(self, position: int, page_size: int) -> tuple[int, int]:
        """(page id, offset) that holds logical token ``position``."""
        return self.pages()[position // page_size], position % page_size


class PagedKVPool:
    """Paged KV pool for all layers plus its allocator.

    ``max_pages``: 0 grows without bound (the reference's default), > 0
    grows straight to that many pages and no further, None never grows (an
    exhausted pool raises RuntimeError).
    """

    def __init__(
        self,
        *,
        num_layers: int,
        capacity_pages: int,
        page_size: int,
        num_kv_heads: int,
        head_dim: int,
        dtype: torch.dtype,
        device: torch.device | str,
        max_pages: int | None = 0,
    ) -> None:
        if max_pages is not None and max_pages > 0 and max_pages < capacity_pages:
            raise ValueError(f"max_pages {max_pages} < capacity_pages {capacity_pages}")
        self.num_layers = num_layers
        self.page_size = page_size
        self.num_kv_heads = num_kv_heads
        self.head_dim = head_dim
        self.cache = torch.empty(
            (num_layers, capacity_pages, 2, page_size, num_kv_heads, head_dim), dtype=dtype, device=device
        )
        self.max_pages = max_pages
        self.version = 0      # bumped whenever the pool tensor moves
        self.grow_count = 0
        self.allocator = PageAllocator(capacity_pages, grow=None if max_pages is None else self._grow)

    def _grow(self, required_pages: int) -> int:
        """Move the pool to a larger tensor, copying every page (ids unchanged)
        (paged_kv_store.py:543-579: max(16, 2 x capacity, required), or
        exactly max_pages when capped).  Stream-ordered: work queued earlier
        on the current stream finishes with the old tensor first."""
        cap = self.capacity_pages
        if self.max_pages:
            if required_pages > self.max_pages:
                raise RuntimeError(f"paged KV pool capacity exceeded: {required_pages} pages > max_pages "
                                   f"{self.max_pages}")
            new_cap = self.max_pages
        else:
            new_cap = max(16, 2 * cap, required_pages)
        old = self.cache
        new = torch.empty((old.shape[0], new_cap) + tuple(old.shape[2:]), dtype=old.dtype, device=old.device)
        new[:, :cap].copy_(old)
        self.cache = new
        self.version += 1
        self.grow_count += 1
        return new_cap

    @property
    def capacity_pages(self) -> int:
        return self.cache.shape[1]

    def layer_cache(self, layer: int) -> torch.Tensor:
        return self.cache[layer]

    def reserve(self, request: Request, new_tokens: int) -> None:
        """Grow the request by ``new_tokens`` tokens, allocating pages as needed."""
        need = -(-(request.length + new_tokens - request.prefix_len) // self.page_size) - len(request.own_pages)
        if need > 0:
            request.own_pages += self.allocator.allocate(need)
        request.length += new_tokens

    def release(self, request: Request) -> None:
        self.allocator.free(request.own_pages)
        request.own_pages = []

    def tables(self, requests) -> tuple[np.ndarray, np.ndarray, np.ndarray]:
        """int32 (indptr, indices, last_page_len) for the batch."""
        return pack_rows([r.spans(self.page_size) for r in requests], self.page_size)
