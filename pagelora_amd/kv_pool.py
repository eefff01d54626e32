"""Paged KV pool, page allocator and per-request spans.

Layout of the pool (``model/kvcache/paged_kv_store.py:559-570``): one dense
tensor ``[num_layers, capacity_pages, 2, page_size, num_kv_heads, head_dim]``;
``pool[l]`` is the NHD layer view the decode kernels read, with K at index
0 and V at index 1 of dim 2 (``layer_runner.py:411-412``).

The MI355X pool is allocated once at its full capacity (288 GB of HBM makes
that the normal case): the reference grows it by doubling
(``paged_kv_store.py:543-579``), which moves the tensor and forces every
captured decode graph to be recaptured.  A fixed pool keeps one data
pointer for the life of the engine.

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
    runs append their (discarded) K/V into.
    """

    def __init__(self, capacity: int) -> None:
        self.capacity = int(capacity)
        self._free = list(range(self.capacity - 1, 0, -1))

    @property
    def free_pages(self) -> int:
        return len(self._free)

    def allocate(self, n: int) -> list[int]:
        if n > len(self._free):
            raise RuntimeError(f"paged KV pool exhausted: need {n} pages, {len(self._free)} free")
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
    """Fixed-capacity paged KV pool for all layers plus its allocator."""

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
    ) -> None:
        self.num_layers = num_layers
        self.page_size = page_size
        self.num_kv_heads = num_kv_heads
        self.head_dim = head_dim
        self.cache = torch.empty(
            (num_layers, capacity_pages, 2, page_size, num_kv_heads, head_dim), dtype=dtype, device=device
        )
        self.allocator = PageAllocator(capacity_pages)

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
