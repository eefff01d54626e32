"""Batched greedy decode loop with hipGraph replay.

The driver of the decode path, after the reference's
``generate_batch_with_flashinfer_kvcache`` (model/flashinfer/generation.py:872-1132):
per step it reserves each row's KV slot (``reserve_chunk``), packs the page
table and plans the decode (``_plan_decode_batch``, :221-247), copies the
step inputs into the graph-owned buffers and replays the captured step
(cuda_graph.py:350-418), falling back to eager when capture failed.

Differences on MI355X: the next token never leaves the device (the graph
writes the argmax into the buffer the next step reads), the page table goes
up as one asynchronous copy from pinned memory with no read-back (the plan
runs on the device), and the graph is not recaptured as rows grow.
tok/s follows the reference's definition: generated tokens / decode seconds
(test/inference/common.py:59-60).
"""

from __future__ import annotations

import time
from dataclasses import dataclass, field

import numpy as np
import torch

from .attention_backend import PagedDecodeAttention
from .decode_graph import BatchDecodeGraphRunner
from .decoder import DecodeContext, DecoderWeights, decode_step_static, prefill, prefill_backend
from .kv_pool import PagedKVPool, Request
from .page_table import PageReserve


@dataclass
class GenerateResult:
    tokens: torch.Tensor             # [B, steps] generated ids (host)
    decode_seconds: float
    prefill_seconds: float
    steps: int
    batch: int
    used_graph: bool
    graph_captures: int = 0
    graph_replays: int = 0
    first_logits: torch.Tensor | None = None
    extra: dict = field(default_factory=dict)
    generated_tokens: int | None = None  # when rows retire early (EOS): the tokens actually decoded

    @property
    def decode_tokens_per_s(self) -> float:
        n = self.batch * self.steps if self.generated_tokens is None else self.generated_tokens
        return n / self.decode_seconds if self.decode_seconds > 0 else 0.0


class _PinnedRing:
    """Pinned host staging slots reused round-robin; a slot is rewritten only
    after the copy that read it has run (event per slot)."""

    def __init__(self, slots: int, shape, dtype) -> None:
        self.bufs = [torch.empty(shape, dtype=dtype, pin_memory=True) for _ in range(slots)]
        self.events: list[torch.cuda.Event | None] = [None] * slots
        self.i = 0

    def next(self) -> tuple[torch.Tensor, int]:
        i = self.i
        self.i = (self.i + 1) % len(self.bufs)
        if self.events[i] is not None:
            self.events[i].synchronize()
        return self.bufs[i], i

    def record(self, i: int) -> None:
        ev = torch.cuda.Event()
        ev.record()
        self.events[i] = ev


class _ReserveFeeder:
    """Keeps each row's reserve ring a window of steps ahead of the device.

    Rows grow by exactly one token per step, so the host knows without a
    read-back which step makes row b take its k-th new page: with L0 tokens
    and n0 pages at the start, the pages taken by steps < s number
    ``max(0, ceil((L0 + s) / ps) - n0)``.  Every refill reserves the tokens
    of the next ``window`` steps in the pool (allocating pages as needed)
    and uploads one snapshot of the rings: pages taken earlier are gone from
    the device ring, the rest sit at slot ``k % slots``.  A window of
    ``(slots - 1) * ps`` steps holds at most ``slots - 1`` new pages per row,
    so a snapshot never overwrites a page the device has not taken yet.
    """

    def __init__(self, pool: PagedKVPool, requests: list[Request], reserve: PageReserve, steps: int) -> None:
        self.pool, self.requests, self.reserve, self.steps = pool, requests, reserve, steps
        ps = pool.page_size
        self.ps = ps
        self.L0 = [r.length for r in requests]
        self.n0 = [-(-L // ps) for L in self.L0]
        self.window = (reserve.slots - 1) * ps
        self.reserved_until = 0  # steps whose tokens are reserved in the pool
        self.uploads = 0

    def taken_before(self, b: int, s: int) -> int:
        return max(0, -(-(self.L0[b] + s) // self.ps) - self.n0[b])

    def before_step(self, s: int) -> None:
        """Refill (enqueued before step ``s``) when a row's window runs short."""
        if s >= self.reserved_until or any(
                self.taken_before(b, min(self.steps, s + self.ps)) > self.taken_before(b, self.reserved_until)
                for b in range(len(self.requests))):
            self._refill(s)

    def _refill(self, s: int) -> None:
        end = min(self.steps, s + self.window)
        ring = np.full((len(self.requests), self.reserve.slots), -1, dtype=np.int32)
        for b, r in enumerate(self.requests):
            if end > self.reserved_until:
                self.pool.reserve(r, end - self.reserved_until)
            pages = r.pages()
            for k in range(self.taken_before(b, s), self.taken_before(b, end)):
                ring[b, k % self.reserve.slots] = pages[self.n0[b] + k]
        self.reserved_until = max(self.reserved_until, end)
        self.reserve.upload(ring)
        self.uploads += 1


class BatchGenerator:
    """Owns the backend, graph runner and pinned staging for one model + pool."""

    def __init__(self, weights: DecoderWeights, pool: PagedKVPool, *, workspace_mb: int = 128,
                 use_graph: bool = True) -> None:
        cfg = weights.cfg
        self.weights = weights
        self.pool = pool
        # Rows that share prefix pages list them once each, so a batch's
        # logical page count can exceed the pool; size the persistent table
        # for that up front so the decode graph's buffers never move.
        self.backend = PagedDecodeAttention(
            device=pool.cache.device, workspace_mb=workspace_mb, num_qo_heads=cfg.num_qo_heads,
            num_kv_heads=cfg.num_kv_heads, head_dim=cfg.head_dim, page_size=pool.page_size,
            max_pages=4 * pool.capacity_pages,
        )
        self.use_graph = use_graph
        self.graphs = BatchDecodeGraphRunner(weights, pool, self.backend)
        self._tables = _PinnedRing(4, (3, 4 * pool.capacity_pages + 1), torch.int32)
        self._inputs = _PinnedRing(4, (4, 4096), torch.int64)
        self._reserves: dict[int, PageReserve] = {}  # batch -> rings (their pointers are in the graphs)
        self.reserve_slots = 3

    def _plan(self, requests) -> None:
        indptr, indices, last = self.pool.tables(requests)
        if len(indices) + 1 > self._tables.bufs[0].shape[1]:
            torch.cuda.synchronize(self.pool.cache.device)  # every staged copy has run
            self._tables = _PinnedRing(4, (3, 2 * len(indices) + 1), torch.int32)
        buf, slot = self._tables.next()
        B, n = len(requests), len(indices)
        buf[0, : B + 1].numpy()[:] = indptr
        buf[1, :n].numpy()[:] = indices
        buf[2, :B].numpy()[:] = last
        self.backend.plan_decode(paged_kv_indptr=buf[0, : B + 1], paged_kv_indices=buf[1, :n],
                                 paged_kv_last_page_len=buf[2, :B])
        self._tables.record(slot)

    def _stage_inputs(self, ctx: DecodeContext, requests, adapters) -> None:
        """Reserve each row's slot for its next token; upload position/slot/adapter."""
        B = len(requests)
        buf, slot = self._inputs.next()
        ps = self.pool.page_size
        for b, r in enumerate(requests):
            pos = r.length
            self.pool.reserve(r, 1)
            page, off = r.slot(pos, ps)
            buf[0, b], buf[1, b], buf[2, b], buf[3, b] = pos, page, off, adapters[b]
        ctx.positions.copy_(buf[0, :B], non_blocking=True)
        ctx.page_id.copy_(buf[1, :B], non_blocking=True)
        ctx.page_offset.copy_(buf[2, :B], non_blocking=True)
        ctx.adapter_ids.copy_(buf[3, :B], non_blocking=True)
        self._inputs.record(slot)

    @torch.no_grad()
    def generate(self, requests: list[Request], first_tokens: torch.Tensor, steps: int,
                 adapters: list[int] | None = None, device_tables: bool = False,
                 keep_logits: bool = False, eos_token_id: int | None = None) -> GenerateResult:
        """Decode ``steps`` greedy tokens for rows whose prompts are prefilled.

        first_tokens: [B] int64 on the device, the token each row decodes
        first (the greedy pick of the prefill logits).  With
        ``device_tables`` the page table is uploaded once and then grown on
        the device inside the step (pl_page_table_advance); the host only
        refills the page reserve about once per page of steps.
        ``keep_logits`` keeps every step's logits ([steps, B, vocab] on the
        device, in ``extra["logits"]``).  With ``eos_token_id`` a row stops
        at its first pick of that token (see :meth:`_generate_until_eos`).
        """
        if eos_token_id is not None:
            if device_tables:
                raise ValueError("rows retiring at EOS re-plan the batch on the host every step; "
                                 "use device_tables=False")
            return self._generate_until_eos(requests, first_tokens, steps, adapters, int(eos_token_id),
                                            keep_logits)
        if device_tables:
            return self._generate_device_tables(requests, first_tokens, steps, adapters, keep_logits)
        B = len(requests)
        dev = self.pool.cache.device
        adapters = adapters or [0] * B
        uniform = self._uniform_adapter(adapters)
        history = torch.empty((steps, B), dtype=torch.int64, device=dev)
        entry = entry_key = None
        kept = []
        ctx = DecodeContext(B, dev)
        ctx.uniform_adapter = uniform
        torch.cuda.synchronize(dev)
        t0 = time.perf_counter()
        capture_s = 0.0
        for step in range(steps):
            if step == 0:
                staging = ctx
                self._stage_inputs(staging, requests, adapters)
                self._plan(requests)
                if self.use_graph:
                    tc = time.perf_counter()
                    n_before = self.graphs.capture_count
                    entry = self.graphs.entry(B, uniform_adapter=uniform)
                    entry_key = self.graphs.key(B, uniform_adapter=uniform)
                    if self.graphs.capture_count != n_before:
                        torch.cuda.synchronize(dev)
                        capture_s = time.perf_counter() - tc
                if entry is not None:
                    ctx = entry.ctx
                    for name in ("positions", "page_id", "page_offset", "adapter_ids"):
                        getattr(ctx, name).copy_(getattr(staging, name))
                ctx.tokens.copy_(first_tokens)
            else:
                self._stage_inputs(ctx, requests, adapters)
                self._plan(requests)  # ctx.tokens holds the last pick (the step wrote it)
                if entry is not None and self.graphs.key(B, uniform_adapter=uniform) != entry_key:
                    # the plan moved the persistent page-table buffers (the
                    # batch's page list outgrew them) or the slot reservation
                    # grew the pool: the captured graph reads the old ones,
                    # so take the graph of the new key
                    tc = time.perf_counter()
                    n_before = self.graphs.capture_count
                    new = self.graphs.entry(B, uniform_adapter=uniform)
                    if self.graphs.capture_count != n_before:
                        torch.cuda.synchronize(dev)
                        capture_s += time.perf_counter() - tc
                    if new is None:  # capture failed: continue eagerly on the staged buffers
                        entry = None
                    else:
                        for name in ("positions", "page_id", "page_offset", "adapter_ids", "tokens"):
                            getattr(new.ctx, name).copy_(getattr(ctx, name))
                        entry, ctx = new, new.ctx
                    entry_key = self.graphs.key(B, uniform_adapter=uniform)
            if entry is not None:
                logits = self.graphs.replay(entry)
            else:
                logits = decode_step_static(self.weights, self.pool, self.backend, ctx)
            history[step].copy_(ctx.next_tokens)
            if keep_logits:
                kept.append(logits.clone())
        torch.cuda.synchronize(dev)
        dt = time.perf_counter() - t0 - capture_s
        extra = {"capture_seconds": capture_s}
        if keep_logits:
            extra["logits"] = torch.stack(kept)
        return GenerateResult(tokens=history.t().cpu(), decode_seconds=dt, prefill_seconds=0.0, steps=steps,
                              batch=B, used_graph=entry is not None, graph_captures=self.graphs.capture_count,
                              graph_replays=self.graphs.replay_count, extra=extra)


    def _generate_until_eos(self, requests, first_tokens, steps, adapters, eos, keep_logits=False) -> GenerateResult:
        """The reference's batched loop with rows retiring at EOS
        (generation.py:967-1086): a row whose pick is ``eos`` keeps that token
        as its last and is not decoded again; the others go on as a smaller
        batch, whose graph is captured once for that batch size (the batch
        is part of the graph key, cuda_graph.py:525-526).  A row whose first
        token is ``eos`` is not decoded at all.  The picks come back to the
        host every step, as the reference's sampler does.

        ``tokens`` is [B, steps] with -1 after a row's last token;
        ``extra["lengths"]`` the tokens each row decoded, ``extra["batch"]``
        the batch size of each step, ``generated_tokens`` their sum (tok/s
        counts those).
        """
        B = len(requests)
        dev = self.pool.cache.device
        adapters = list(adapters or [0] * B)
        out = torch.full((B, steps), -1, dtype=torch.int64)
        first = first_tokens.reshape(-1).cpu().tolist()
        active = [b for b in range(B) if first[b] != eos]
        cur = torch.tensor([first[b] for b in active], dtype=torch.int64)
        kept = None
        eager: dict[int, DecodeContext] = {}
        batches: list[int] = []
        used_graph = False
        torch.cuda.synchronize(dev)
        t0 = time.perf_counter()
        capture_s = 0.0
        for step in range(steps):
            if not active:
                break
            reqs = [requests[b] for b in active]
            ads = [adapters[b] for b in active]
            Ba, uniform = len(reqs), self._uniform_adapter(ads)
            staging = eager.get(Ba)
            if staging is None:
                staging = eager[Ba] = DecodeContext(Ba, dev)
            staging.uniform_adapter = uniform
            self._stage_inputs(staging, reqs, ads)
            self._plan(reqs)
            entry = None
            if self.use_graph:
                tc = time.perf_counter()
                n_before = self.graphs.capture_count
                entry = self.graphs.entry(Ba, uniform_adapter=uniform)
                if self.graphs.capture_count != n_before:
                    torch.cuda.synchronize(dev)
                    capture_s += time.perf_counter() - tc
            if entry is not None:
                ctx = entry.ctx
                for name in ("positions", "page_id", "page_offset", "adapter_ids"):
                    getattr(ctx, name).copy_(getattr(staging, name))
            else:
                ctx = staging
            ctx.tokens.copy_(cur)
            if entry is not None:
                logits = self.graphs.replay(entry)
                used_graph = True
            else:
                logits = decode_step_static(self.weights, self.pool, self.backend, ctx)
            picks = ctx.next_tokens.cpu()
            if keep_logits:
                if kept is None:
                    kept = torch.full((steps, B, logits.shape[1]), float("nan"), dtype=logits.dtype, device=dev)
                kept[step, torch.tensor(active, device=dev)] = logits
            out[active, step] = picks
            batches.append(Ba)
            go_on = picks != eos
            active = [b for b, g in zip(active, go_on.tolist()) if g]
            cur = picks[go_on]
        torch.cuda.synchronize(dev)
        dt = time.perf_counter() - t0 - capture_s
        lengths = (out >= 0).sum(dim=1).tolist()
        extra = {"capture_seconds": capture_s, "lengths": lengths, "batch": batches}
        if keep_logits:
            extra["logits"] = kept
        return GenerateResult(tokens=out, decode_seconds=dt, prefill_seconds=0.0, steps=steps, batch=B,
                              used_graph=used_graph, graph_captures=self.graphs.capture_count,
                              graph_replays=self.graphs.replay_count, extra=extra,
                              generated_tokens=int(sum(batches)))

    def _uniform_adapter(self, adapters) -> int:
        """The one adapter every row uses, else -1 (per-row ids)."""
        a = adapters[0] if adapters and all(x == adapters[0] for x in adapters) else -1
        return a if 0 <= a < self.weights.n_adapters else -1

    def _generate_device_tables(self, requests, first_tokens, steps, adapters, keep_logits=False) -> GenerateResult:
        B = len(requests)
        dev = self.pool.cache.device
        adapters = adapters or [0] * B
        uniform = self._uniform_adapter(adapters)
        history = torch.empty((steps, B), dtype=torch.int64, device=dev)
        reserve = self._reserves.get(B)
        if reserve is None:
            reserve = self._reserves[B] = PageReserve(B, self.reserve_slots, dev)
        reserve.reset()
        feeder = _ReserveFeeder(self.pool, requests, reserve, steps)
        torch.cuda.synchronize(dev)
        t0 = time.perf_counter()
        capture_s = 0.0
        self._plan(requests)  # the table of the prompts; the device grows it from here
        entry = None
        if self.use_graph:
            tc = time.perf_counter()
            n_before = self.graphs.capture_count
            entry = self.graphs.entry(B, reserve, uniform)
            if self.graphs.capture_count != n_before:
                torch.cuda.synchronize(dev)
                capture_s = time.perf_counter() - tc
        if entry is not None:
            ctx = entry.ctx
        else:
            ctx = DecodeContext(B, dev)
            ctx.uniform_adapter = uniform
        ctx.adapter_ids.copy_(torch.tensor(adapters, dtype=torch.int32))
        ctx.tokens.copy_(first_tokens)
        entry_key = self.graphs.key(B, reserve, uniform) if entry is not None else None
        kept = []
        for step in range(steps):
            feeder.before_step(step)  # ctx.tokens holds the last pick (the step wrote it)
            if entry is not None and self.graphs.key(B, reserve, uniform) != entry_key:
                # the refill grew the pool (a new tensor, the same page ids):
                # capture the step once more on the new pool and carry the
                # step inputs over (positions and slots come from the
                # in-graph advance)
                tc = time.perf_counter()
                n_before = self.graphs.capture_count
                new = self.graphs.entry(B, reserve, uniform)
                if self.graphs.capture_count != n_before:
                    torch.cuda.synchronize(dev)
                    capture_s += time.perf_counter() - tc
                if new is None:  # capture failed: continue eagerly on the current buffers
                    entry = None
                else:
                    for name in ("tokens", "adapter_ids"):
                        getattr(new.ctx, name).copy_(getattr(ctx, name))
                    entry, ctx = new, new.ctx
                entry_key = self.graphs.key(B, reserve, uniform)
            if entry is not None:
                logits = self.graphs.replay(entry)
            else:
                self.backend.advance_decode(reserve, ctx.positions, ctx.page_id, ctx.page_offset)
                logits = decode_step_static(self.weights, self.pool, self.backend, ctx)
            history[step].copy_(ctx.next_tokens)
            if keep_logits:
                kept.append(logits.clone())
        torch.cuda.synchronize(dev)
        dt = time.perf_counter() - t0 - capture_s
        reserve.check()
        extra = {"capture_seconds": capture_s, "reserve_uploads": feeder.uploads}
        if keep_logits:
            extra["logits"] = torch.stack(kept)
        return GenerateResult(tokens=history.t().cpu(), decode_seconds=dt, prefill_seconds=0.0, steps=steps,
                              batch=B, used_graph=entry is not None, graph_captures=self.graphs.capture_count,
                              graph_replays=self.graphs.replay_count, extra=extra)


def prefill_requests(weights: DecoderWeights, pool: PagedKVPool, prompts: list[torch.Tensor],
                     shared_prefix: torch.Tensor | None = None, adapters: list[int] | None = None):
    """Prefill rows (optionally behind one shared prefix held in shared pages).

    Returns (requests, first_tokens [B] on the device, first-step logits [B, V]).
    The shared prefix must fill whole pages so rows can list its pages
    read-only (paged_kvcache_manager.py:324-333).
    """
    dev = pool.cache.device
    ps = pool.page_size
    adapters = adapters or [0] * len(prompts)
    backend = prefill_backend(weights.cfg, ps, dev)
    prefix_pages, prefix_len = [], 0
    if shared_prefix is not None and shared_prefix.numel():
        if shared_prefix.numel() % ps:
            raise ValueError("a shared prefix must fill whole pages")
        owner = Request()
        pool.reserve(owner, shared_prefix.numel())
        prefill(weights, pool, owner, shared_prefix.to(dev), adapter=adapters[0], backend=backend)
        prefix_pages, prefix_len = list(owner.own_pages), owner.length
    requests, logits = [], []
    for p, a in zip(prompts, adapters):
        r = Request(prefix_pages=list(prefix_pages), prefix_len=prefix_len, length=prefix_len)
        pool.reserve(r, p.numel())
        logits.append(prefill(weights, pool, r, p.to(dev), adapter=a, backend=backend))
        requests.append(r)
    logits = torch.cat(logits, dim=0)
    return requests, torch.argmax(logits, dim=-1), logits
