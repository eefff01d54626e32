"""hipGraph capture and replay of the batched decode step.

Counterpart of the reference's ``FlashInferBatchDecodeCudaGraphRunner``
(model/flashinfer/cuda_graph.py:307-543): graph-owned input buffers
(tokens, positions, KV slot page/offset, adapter ids), one warmup on a
side stream, then capture of embed -> layers -> final norm -> lm_head ->
argmax (cuda_graph.py:222-234, 475-493); a capture failure disables graphs
and the caller falls back to eager (cuda_graph.py:204-210, 420-426).

The key (``DecodeGraphKey``, cuda_graph.py:76-93) differs on purpose: it has
no ``page_table_pages`` and no host plan, and its adapter version changes
only when the adapter stacks move (``DecoderWeights.adapter_version``):
writing new adapter values into a slot keeps every address a graph reads.
The decode plan lives on the device and the KV pool moves only when it
grows, so a graph captured for a batch size replays for every later step
while the rows grow; the reference recaptures on every new page.  torch's
CUDAGraph is hipGraph on ROCm.
"""

from __future__ import annotations

import gc

from collections import OrderedDict
from dataclasses import dataclass

import torch

from .attention_backend import PagedDecodeAttention
from .decoder import DecodeContext, DecoderWeights, decode_step_static
from .kv_pool import PagedKVPool


@dataclass(frozen=True)
class DecodeGraphKey:
    model_id: int
    backend_signature: tuple
    cache_data_ptr: int
    cache_shape: tuple
    cache_dtype: torch.dtype
    batch: int
    adapter_version: int
    reserve_ptrs: tuple = ()  # device page-table advance captured in (its ring buffers)
    uniform_adapter: int = -1  # >= 0: one adapter bound to every row, baked into the kernels


@dataclass
class DecodeGraphEntry:
    graph: torch.cuda.CUDAGraph
    ctx: DecodeContext
    logits: torch.Tensor


class BatchDecodeGraphRunner:
    """Capture once per key, replay every step."""

    def __init__(self, weights: DecoderWeights, pool: PagedKVPool, backend: PagedDecodeAttention,
                 max_entries: int = 32) -> None:
        self.weights = weights
        self.pool = pool
        self.backend = backend
        self.max_entries = max_entries
        self.disabled_reason: str | None = None
        self.capture_count = 0
        self.replay_count = 0
        self._graphs: OrderedDict[DecodeGraphKey, DecodeGraphEntry] = OrderedDict()

    def key(self, batch: int, reserve=None, uniform_adapter: int = -1) -> DecodeGraphKey:
        cache = self.pool.cache
        ptrs = () if reserve is None else (reserve.reserve.data_ptr(), reserve.head.data_ptr(),
                                           reserve.status.data_ptr())
        return DecodeGraphKey(
            model_id=id(self.weights),
            backend_signature=self.backend.decode_graph_signature(),
            cache_data_ptr=cache.data_ptr(),
            cache_shape=tuple(cache.shape),
            cache_dtype=cache.dtype,
            batch=batch,
            adapter_version=self.weights.adapter_version,
            reserve_ptrs=ptrs,
            uniform_adapter=uniform_adapter,
        )

    def entry(self, batch: int, reserve=None, uniform_adapter: int = -1) -> DecodeGraphEntry | None:
        """The graph for ``batch``: captured on first use (needs a current plan).

        With a :class:`PageReserve` the graph starts with the device-side
        page-table advance and re-plan, so a replay needs no host input.
        """
        if self.disabled_reason is not None:
            return None
        k = self.key(batch, reserve, uniform_adapter)
        e = self._graphs.get(k)
        if e is not None:
            self._graphs.move_to_end(k)
            return e
        # graphs of a pool tensor that has since moved are never replayed again
        for stale in [x for x in self._graphs if x.cache_data_ptr != k.cache_data_ptr]:
            del self._graphs[stale]
        try:
            e = self._capture(batch, reserve, uniform_adapter)
        except Exception as exc:  # capture failure: fall back to eager for good
            self.disabled_reason = f"{type(exc).__name__}: {exc}"
            self._graphs.clear()
            return None
        while len(self._graphs) >= self.max_entries:
            self._graphs.popitem(last=False)
        self._graphs[k] = e
        self.capture_count += 1
        return e

    def _capture(self, batch: int, reserve=None, uniform_adapter: int = -1) -> DecodeGraphEntry:
        dev = self.pool.cache.device
        ctx = DecodeContext(batch, dev)
        ctx.uniform_adapter = uniform_adapter
        # Warm up once on a side stream (allocator pools, library workspaces),
        # writing to a slot nobody reads: page 0 of the pool is never handed out.
        cur = torch.cuda.current_stream(dev)
        side = torch.cuda.Stream(device=dev)
        side.wait_stream(cur)
        with torch.cuda.stream(side):
            decode_step_static(self.weights, self.pool, self.backend, ctx)
        cur.wait_stream(side)
        graph = torch.cuda.CUDAGraph()
        # No Python garbage collection while the stream captures (torch's
        # graph context no longer collects first): a collected object that
        # owns pinned host memory or an event, such as an earlier generation's
        # staging buffers, would make HIP calls from its destructor that are
        # illegal during capture, and the error raised there aborts the process.
        gc.collect()
        gc_was_enabled = gc.isenabled()
        gc.disable()
        try:
            with torch.cuda.graph(graph):
                if reserve is not None:  # not in the warm-up: it would grow the rows
                    self.backend.advance_decode(reserve, ctx.positions, ctx.page_id, ctx.page_offset)
                logits = decode_step_static(self.weights, self.pool, self.backend, ctx)
        finally:
            if gc_was_enabled:
                gc.enable()
        return DecodeGraphEntry(graph=graph, ctx=ctx, logits=logits)

    @property
    def adapter_version(self) -> int:
        """The weights' adapter-layout version the graph keys carry."""
        return self.weights.adapter_version

    def replay(self, entry: DecodeGraphEntry) -> torch.Tensor:
        entry.graph.replay()
        self.replay_count += 1
        return entry.logits

    def clear(self) -> None:
        self._graphs.clear()
