"""Paged decode attention behind the reference's plan()/run() surface.

``PagedDecodeAttention`` keeps the constructor, methods and attributes of the
reference's ``FlashInferAttentionBackend`` (model/flashinfer/attention_backend.py:18-292)
that its callers use -- ``plan_decode``, ``run_decode``, ``decode_graph_signature``,
``workspace_buffer``, ``page_size``, ``query_rescale``, ``decode_use_tensor_cores``,
``use_flashinfer_qk_norm`` -- and runs the gfx950 kernels of libpagelora_amd.so:

* ``plan_decode`` copies the page table into persistent device buffers and
  enqueues the device-side split-KV plan.  Nothing is read back to the host,
  so the plan can also be captured into the decode graph.
* ``run_decode`` launches the split-KV decode kernel (+ merge) on the
  current stream.  Its grid depends only on the batch size, so one captured
  hipGraph replays across steps while the rows grow
  (``decode_graph_signature`` does not change with sequence length).

Mathematics: ``o = softmax(q . K^T / sqrt(D)) . V`` per (row, q head), kv head
``hq // (Hq / Hkv)``.  The reference divides q by 16 and multiplies the scale
by 16 (attention_backend.py:37-41, 97, 128) to dodge FlashInfer's finite
``-5e4`` mask sentinel; the kernels here mask with ``-inf`` selects, so that
workaround is not needed and ``query_rescale`` is 1.0.
"""

from __future__ import annotations

import ctypes
import math
import os
import weakref
from collections import deque
from typing import Sequence

import torch

from . import _lib

# Split-KV sizing.  The decode grid is (target_items + batch) x kv heads
# waves whatever the lengths (so one captured graph replays as rows grow), and
# the device plan cuts rows into chunks of max(min_chunk, total/target_items)
# pages.  The default item count was measured on MI355X (1,024 SIMDs), step
# time of plan + decode + merge:
#   - batch <= 32: 128 items (4 x 2114 and 1 x 32K tokens, GQA 4: 1,024 waves,
#     one per SIMD; 256 or 64 items were 5-10% slower; re-checked end to end
#     on the 36-layer 1 x 32K step with q/k/v folded in: 226.1 tok/s at 128
#     items, 210.3 at 192, 215.8 at 256);
#   - GQA 4 with head_dim 128 (scores on MFMA) at any batch: 128 items
#     (bf16, 8 kv heads: 64 x 2048 90.9 us against 92.0 at 256 items,
#     128 x 2048 166.6 vs 170.8, 64 x 8192 325.1 vs 326.1; 192 items, an
#     uneven count of waves per SIMD, 105.7 / 170.2 / 382.1);
#   - other larger batches with 8 kv heads: 256 items (64 x 2048 GQA 4 on
#     the VALU scores: 99 us against 118 us at 1,024 items; ragged
#     64 x U[128, 8192]: 204 vs 217 us);
#   - larger batches with >= 16 kv heads: 192 items, i.e. 6 waves per SIMD
#     (ragged batch-64 MHA: 713.5 us against 729 us at 256 items).
_ENV_TARGET_WAVES = os.environ.get("PAGELORA_DECODE_TARGET_WAVES")
# The minimum chunk binds only for short rows (a chunk is otherwise
# total / target_items pages).  1 x 2048 tokens bf16, GQA 4 (32 items at 4
# pages, 64 at 2), plan-less step in a graph: 21.2 -> 20.2 us warm, 23.3 ->
# 22.3 us cold at 2 pages.
_DEFAULT_MIN_CHUNK_PAGES = int(os.environ.get("PAGELORA_DECODE_MIN_CHUNK_PAGES", "2"))


def default_target_items(batch: int, num_kv_heads: int, num_qo_heads: int | None = None,
                         head_dim: int | None = None) -> int:
    if _ENV_TARGET_WAVES:
        return max(1, int(_ENV_TARGET_WAVES) // num_kv_heads)
    if batch <= 32 or (num_qo_heads == 4 * num_kv_heads and head_dim == 128):
        return 128
    return 192 if num_kv_heads >= 16 else 256


def _validate_host_table(indptr: torch.Tensor, indices: torch.Tensor, last: torch.Tensor, page_size: int) -> int:
    """Check a host-side page table; returns the largest page id (or -1)."""

    ip = indptr.tolist()
    if ip and ip[0] != 0:
        raise ValueError("paged_kv_indptr must start at 0")
    if any(b < a for a, b in zip(ip, ip[1:])):
        raise ValueError("paged_kv_indptr must be non-decreasing")
    if ip and ip[-1] > indices.numel():
        raise ValueError(f"paged_kv_indptr[-1]={ip[-1]} exceeds paged_kv_indices length {indices.numel()}")
    lens = last.tolist()
    for b, (a, e) in enumerate(zip(ip, ip[1:])):
        if e > a and not (1 <= lens[b] <= page_size):
            raise ValueError(f"paged_kv_last_page_len[{b}]={lens[b]} outside [1, {page_size}]")
    used = indices[: ip[-1]] if ip else indices[:0]
    if used.numel() and int(used.min()) < 0:
        raise ValueError("paged_kv_indices holds a negative page id")
    return int(used.max()) if used.numel() else -1


def _cache_geometry(cache, num_kv_heads: int, head_dim: int, page_size: int):
    """(k_tensor, v_tensor_or_ptr_source, page_stride, token_stride, head_stride, num_pages)."""

    if isinstance(cache, (tuple, list)):
        k, v = cache
        if k.shape != v.shape or k.stride() != v.stride() or k.dtype != v.dtype:
            raise ValueError("K and V caches must have the same shape, strides and dtype")
        if k.dim() != 4 or tuple(k.shape[1:]) != (page_size, num_kv_heads, head_dim):
            raise ValueError(f"K/V caches must be [P, {page_size}, {num_kv_heads}, {head_dim}] (NHD), got {tuple(k.shape)}")
        if k.stride(3) != 1:
            raise ValueError("head_dim must be contiguous in the KV cache")
        return k, v, k.stride(0), k.stride(1), k.stride(2), k.shape[0]
    if cache.dim() != 5 or tuple(cache.shape[1:]) != (2, page_size, num_kv_heads, head_dim):
        raise ValueError(
            f"paged KV cache layer must be [P, 2, {page_size}, {num_kv_heads}, {head_dim}] (NHD), got {tuple(cache.shape)}"
        )
    if cache.stride(4) != 1:
        raise ValueError("head_dim must be contiguous in the KV cache")
    return cache[:, 0], cache[:, 1], cache.stride(0), cache.stride(2), cache.stride(3), cache.shape[0]


class PagedDecodeAttention:
    """gfx950 paged decode attention with the FlashInferAttentionBackend surface.

    ``share_prefix``: when a host-table plan finds every row of a batch of 2..4
    rows starting with the same pages (a shared prompt prefix), the folded
    q/k/v run attends those pages once for all rows
    (``pl_decode_plan_shared``); False reads them once per row.
    """

    share_prefix = True
    # pages per prefix item: 32 tokens, one MFMA step of the prefix kernel path
    _PREFIX_TOKENS = 32
    # With a shared prefix: own items per row the grid is sized for, and the
    # own items' minimum chunk in pages (None: the prefix item's).  4 rows x
    # (2048 shared + 64+) end to end, alternating: 4 items of >= 2 pages
    # 1000.1 tok/s, 8 of >= 2 1002.2, 8 of >= 1 1003.2, 16 of >= 1 1003.5.
    _SHARED_OWN_ITEMS_PER_ROW = 8
    _SHARED_OWN_MIN_CHUNK: int | None = 1

    def __init__(
        self,
        *,
        device: torch.device | str,
        workspace_mb: int,
        num_qo_heads: int,
        num_kv_heads: int,
        head_dim: int,
        page_size: int,
        target_waves: int | None = None,
        min_chunk_pages: int | None = None,
        max_pages: int = 0,
    ) -> None:
        self.device = torch.device(device)
        self.workspace_mb = max(1, int(workspace_mb))
        self.num_qo_heads = int(num_qo_heads)
        self.num_kv_heads = int(num_kv_heads)
        self.head_dim = int(head_dim)
        self.page_size = int(page_size)
        if self.num_kv_heads <= 0 or self.num_qo_heads % self.num_kv_heads:
            raise ValueError("Q head count must be divisible by KV head count")
        self.query_rescale = 1.0
        self.sm_scale = 1.0 / math.sqrt(self.head_dim)
        # One code path for every GQA ratio (the reference switches to
        # FlashInfer's tensor-core kernel for ratios outside {1,2,4,8}); groups
        # above 8 run as several waves of at most 8 query heads per kv head.
        self.decode_use_tensor_cores = False
        self.use_flashinfer_qk_norm = False
        self.target_waves = int(target_waves) if target_waves else None  # None: default_target_items(...)
        # the minimum split chunk is 32 tokens (2 pages of 16) whatever the page size
        default_chunk = _DEFAULT_MIN_CHUNK_PAGES if self.page_size >= 16 else \
            -(-_DEFAULT_MIN_CHUNK_PAGES * 16 // max(1, self.page_size))
        self.min_chunk_pages = int(min_chunk_pages or default_chunk)
        if self.device.type == "cuda":
            self._lib = _lib.load()  # fails loudly when the extension is not built
        else:
            self._lib = None
        self.workspace_buffer = torch.empty(self.workspace_mb * 1024 * 1024, dtype=torch.uint8, device=self.device)
        if self._lib is not None:
            # the library's direct plan for this workspace dies with it, so a
            # later tensor at the same address starts without one
            weakref.finalize(self.workspace_buffer, self._lib.pl_decode_forget,
                             ctypes.c_void_p(self.workspace_buffer.data_ptr()))
        # Initial capacity of the persistent indices buffer.  A capacity that
        # covers every page a batch can list (e.g. the pool size) means the
        # buffers, and so decode_graph_signature(), never change as rows grow.
        self.max_pages = int(max_pages)
        self._decode_graph_buffers: tuple[torch.Tensor, torch.Tensor, torch.Tensor] | None = None
        self._decode_host_uploads: deque = deque()
        self._plan: dict | None = None

    # ------------------------------------------------------------ planning
    def plan_decode(
        self,
        *,
        paged_kv_indptr: torch.Tensor,
        paged_kv_indices: torch.Tensor,
        paged_kv_last_page_len: torch.Tensor,
        q_data_type: torch.dtype | None = None,
        kv_data_type: torch.dtype | None = None,
        non_blocking: bool | None = None,
    ) -> None:
        """Upload one step's page table and enqueue the device-side plan.

        Shared by every decoder layer of the step (attention_backend.py:63-118).
        Host tables are validated here; device tables are trusted (the kernels
        still clamp every index into its buffer).
        """

        if paged_kv_indptr.dim() != 1 or paged_kv_last_page_len.dim() != 1 or paged_kv_indices.dim() != 1:
            raise ValueError("page-table tensors must be 1-D")
        batch = paged_kv_last_page_len.numel()
        if paged_kv_indptr.numel() != batch + 1:
            raise ValueError("paged_kv_indptr must have batch + 1 entries")
        for t in (paged_kv_indptr, paged_kv_indices, paged_kv_last_page_len):
            if t.dtype != torch.int32:
                raise ValueError("page-table tensors must be int32")
        max_page = None
        if paged_kv_indptr.device.type == "cpu":
            max_page = _validate_host_table(paged_kv_indptr, paged_kv_indices, paged_kv_last_page_len, self.page_size)
        if self.device.type != "cuda":
            raise RuntimeError("PagedDecodeAttention.plan_decode needs a ROCm device")

        self._ensure_graph_safe_decode_buffers(paged_kv_indptr, paged_kv_indices, paged_kv_last_page_len)
        indptr_buf, indices_buf, last_buf = self._decode_graph_buffers
        host = (paged_kv_indptr, paged_kv_indices, paged_kv_last_page_len)
        async_host = all(t.device.type == "cpu" and t.is_pinned() for t in host)
        if async_host:
            # A pinned source must stay alive until its upload has run; keep at
            # most 8 in flight (attention_backend.py:79-88, 114-118).
            while self._decode_host_uploads and self._decode_host_uploads[0][0].query():
                self._decode_host_uploads.popleft()
            if len(self._decode_host_uploads) >= 8:
                self._decode_host_uploads[0][0].synchronize()
                self._decode_host_uploads.popleft()
        nb = bool(async_host if non_blocking is None else non_blocking)
        indptr_buf[: batch + 1].copy_(paged_kv_indptr, non_blocking=nb)
        if paged_kv_indices.numel():
            indices_buf[: paged_kv_indices.numel()].copy_(paged_kv_indices, non_blocking=nb)
        last_buf[:batch].copy_(paged_kv_last_page_len, non_blocking=nb)
        if async_host:
            ev = torch.cuda.Event()
            ev.record(torch.cuda.current_stream(self.device))
            self._decode_host_uploads.append((ev, host))

        target_items = self._target_items(batch)
        shared = 0
        if paged_kv_indptr.device.type == "cpu":
            shared = self._shared_prefix_pages(paged_kv_indptr, paged_kv_indices, batch, target_items)
            if shared:
                # the rows' own pages past the prefix are few: a few items each
                # (a grid sized for 128 would be mostly idle workgroups)
                target_items = min(target_items, self._SHARED_OWN_ITEMS_PER_ROW * batch)
        self._plan = {
            "batch": batch,
            "target_items": target_items,
            "q_data_type": q_data_type,
            "kv_data_type": kv_data_type,
            "max_page": max_page,
            "shared": shared,
        }
        self._launch_plan(batch, target_items)

    def replan_decode(self) -> None:
        """Re-run the device-side plan on the current buffers (same batch).

        For callers that update the persistent page-table buffers on the
        device (e.g. inside a captured step) instead of calling plan_decode.
        """

        if self._plan is None:
            raise RuntimeError("plan_decode has not been called")
        self._launch_plan(self._plan["batch"], self._plan["target_items"])

    def advance_decode(self, reserve, positions: torch.Tensor, page_id: torch.Tensor,
                       page_offset: torch.Tensor) -> None:
        """Grow every planned row by one decode token on the device, then re-plan.

        ``reserve`` is a :class:`~pagelora_amd.page_table.PageReserve` of the
        plan's batch; the token positions and KV slots land in ``positions`` /
        ``page_id`` / ``page_offset``.  Two kernels, no host table and no
        read-back, so a captured decode step can start with it
        (generation.py:1011-1035 does this on the host every step).
        """

        from .page_table import page_table_advance

        if self._plan is None:
            raise RuntimeError("plan_decode has not been called")
        batch = self._plan["batch"]
        if reserve.batch != batch:
            raise ValueError(f"reserve holds {reserve.batch} rows but the plan has {batch}")
        indptr_buf, indices_buf, last_buf = self._decode_graph_buffers
        page_table_advance(indptr_buf, indices_buf, last_buf[:batch], self.page_size, reserve.reserve,
                           reserve.head, positions, page_id, page_offset, reserve.status)
        self._plan["max_page"] = None  # pages now come from the reserve; the kernels clamp them
        self._launch_plan(batch, self._plan["target_items"])

    def _launch_plan(self, batch: int, target_items: int) -> None:
        indptr_buf, indices_buf, _ = self._decode_graph_buffers
        shared = (self._plan or {}).get("shared", 0)
        pchunk = self._prefix_chunk_pages()
        status = self._lib.pl_decode_plan_shared(
            indptr_buf.data_ptr(),
            batch,
            indices_buf.numel(),
            self.num_qo_heads,
            self.head_dim,
            target_items,
            # own items as short as the prefix items when a prefix is shared
            (self._SHARED_OWN_MIN_CHUNK or pchunk) if shared else self.min_chunk_pages,
            shared,
            pchunk if shared else 1,
            self.workspace_buffer.data_ptr(),
            self.workspace_buffer.numel(),
            _lib.stream_handle(self.device),
        )
        _lib.check(status, "pl_decode_plan_shared")

    def _prefix_chunk_pages(self) -> int:
        return max(1, self._PREFIX_TOKENS // self.page_size)

    def _shared_prefix_pages(self, indptr: torch.Tensor, indices: torch.Tensor, batch: int,
                             target_items: int) -> int:
        """Leading pages every row of the batch lists (whole prefix items,
        each row keeping at least one page of its own), where the folded
        run can share them; 0 otherwise."""
        pchunk = self._prefix_chunk_pages()
        if (not self.share_prefix or not 2 <= batch <= 4 or pchunk * self.page_size != self._PREFIX_TOKENS
                or self.num_qo_heads != 4 * self.num_kv_heads or self.head_dim != 128):
            return 0
        ip = indptr.tolist()
        lens = [ip[b + 1] - ip[b] for b in range(batch)]
        limit = min(lens) - 1
        if limit < 2 * pchunk:
            return 0
        import numpy as np

        idx = indices.numpy()
        first = idx[ip[0]: ip[0] + limit]
        same = np.ones(limit, dtype=bool)
        for b in range(1, batch):
            same &= idx[ip[b]: ip[b] + limit] == first
        common = limit if same.all() else int(np.argmin(same))
        shared = common // pchunk * pchunk
        if shared < 2 * pchunk:
            return 0
        need = self._lib.pl_decode_workspace_size_shared(batch, target_items, self.num_qo_heads, self.head_dim,
                                                         shared, pchunk)
        return shared if need <= self.workspace_buffer.numel() else 0

    def _target_items(self, batch: int) -> int:
        """Work items per step (target_waves / kv heads if set, else the
        measured default), within the workspace."""

        if self.target_waves:
            t = max(1, self.target_waves // self.num_kv_heads)
        else:
            t = default_target_items(batch, self.num_kv_heads, self.num_qo_heads, self.head_dim)
        cap = self.workspace_buffer.numel()
        while t > 1 and self._lib.pl_decode_workspace_size(batch, t, self.num_qo_heads, self.head_dim) > cap:
            t //= 2
        if self._lib.pl_decode_workspace_size(batch, t, self.num_qo_heads, self.head_dim) > cap:
            raise _lib.WorkspaceTooSmallError(
                f"workspace of {self.workspace_mb} MiB cannot hold a decode plan for batch {batch}"
            )
        return t

    def _ensure_graph_safe_decode_buffers(self, indptr, indices, last_page_len) -> None:
        """Persistent device page-table buffers (attention_backend.py:198-221 policy):
        rebuilt when the batch changes or the indices outgrow a power-of-two capacity."""

        buffers = self._decode_graph_buffers
        if buffers is not None and buffers[0].numel() == indptr.numel() and buffers[1].numel() >= indices.numel():
            return
        capacity = max(16, self.max_pages, 1 << max(0, indices.numel() - 1).bit_length())
        self._decode_graph_buffers = (
            torch.zeros(indptr.numel(), dtype=torch.int32, device=self.device),
            torch.zeros(capacity, dtype=torch.int32, device=self.device),
            torch.ones(last_page_len.numel(), dtype=torch.int32, device=self.device),
        )

    def decode_graph_signature(self):
        """Everything a captured run_decode bakes in (attention_backend.py:223-227).

        Sequence lengths are not part of it: the plan lives on the device.
        """

        bufs = self._decode_graph_buffers
        ptrs = tuple(b.data_ptr() for b in bufs) if bufs is not None else ()
        plan = self._plan or {}
        return (id(self), plan.get("batch"), plan.get("target_items"), plan.get("shared", 0), ptrs,
                self.workspace_buffer.data_ptr())

    # ----------------------------------------------------------------- run
    def run_decode(self, q: torch.Tensor, paged_kv_cache_layer) -> torch.Tensor:
        """One layer of paged decode attention; returns ``[B, Hq, 1, D]``
        (attention_backend.py:120-131)."""

        q_nhd = q.squeeze(2) if q.dim() == 4 and q.size(2) == 1 else q
        out = torch.empty(q_nhd.shape, dtype=q_nhd.dtype, device=q_nhd.device)
        self.run_decode_into(q_nhd, paged_kv_cache_layer, out)
        return out.unsqueeze(2) if out.dim() == 3 else out

    def run_decode_into(
        self,
        q: torch.Tensor,
        paged_kv_cache_layer,
        out: torch.Tensor,
        lse: torch.Tensor | None = None,
        *,
        flags: int = 0,
    ) -> torch.Tensor:
        """Allocation-free variant: writes ``out`` ([B, Hq, D]) and optionally
        ``lse`` ([B, Hq] fp32, natural log).  ``flags`` (PL_DECODE_SKIP_MERGE /
        PL_DECODE_MERGE_ONLY) launches only one of the two run kernels."""

        plan = self._plan
        if plan is None:
            raise RuntimeError("plan_decode must be called before run_decode")
        if q.dim() != 3 or tuple(q.shape[1:]) != (self.num_qo_heads, self.head_dim):
            raise ValueError(f"q must be [B, {self.num_qo_heads}, {self.head_dim}], got {tuple(q.shape)}")
        batch = q.shape[0]
        if batch != plan["batch"]:
            raise ValueError(f"q has batch {batch} but the plan has {plan['batch']}")
        if q.stride(2) != 1 or out.stride(2) != 1 or tuple(out.shape) != tuple(q.shape) or out.dtype != q.dtype:
            raise ValueError("q and out must match in shape/dtype with a contiguous head_dim")
        if q.device.type != "cuda":
            raise RuntimeError("run_decode needs tensors on a ROCm device")
        k, v, page_stride, token_stride, head_stride, num_pages = _cache_geometry(
            paged_kv_cache_layer, self.num_kv_heads, self.head_dim, self.page_size
        )
        if k.dtype != q.dtype:
            raise ValueError(f"q dtype {q.dtype} != KV cache dtype {k.dtype}")
        if plan["max_page"] is not None and plan["max_page"] >= num_pages:
            raise ValueError(f"page id {plan['max_page']} is outside the {num_pages}-page KV pool")
        if lse is not None and (lse.dtype != torch.float32 or tuple(lse.shape) != (batch, self.num_qo_heads) or not lse.is_contiguous()):
            raise ValueError("lse must be a contiguous fp32 [B, Hq] tensor")
        _, indices_buf, last_buf = self._decode_graph_buffers
        status = self._lib.pl_decode_run(
            q.data_ptr(), q.stride(0), q.stride(1),
            k.data_ptr(), v.data_ptr(), page_stride, token_stride, head_stride,
            num_pages,
            indices_buf.data_ptr(), last_buf.data_ptr(),
            out.data_ptr(), out.stride(0), out.stride(1),
            lse.data_ptr() if lse is not None else None,
            batch, self.num_qo_heads, self.num_kv_heads, self.head_dim, self.page_size,
            self.sm_scale, _lib.dtype_code(q.dtype), plan["target_items"], int(flags),
            self.workspace_buffer.data_ptr(), self.workspace_buffer.numel(),
            _lib.stream_handle(q.device),
        )
        _lib.check(status, "pl_decode_run")
        return out

    def run_decode_qkv_into(
        self,
        qkv: torch.Tensor,
        paged_kv_cache_layer,
        out: torch.Tensor,
        *,
        q_norm_weight: torch.Tensor | None,
        k_norm_weight: torch.Tensor | None,
        rope_cos_sin: torch.Tensor,
        page_id: torch.Tensor,
        page_offset: torch.Tensor,
        eps: float,
        lora=None,
        adapter_ids: torch.Tensor | None = None,
        lse: torch.Tensor | None = None,
        o_shrink=None,
    ) -> torch.Tensor:
        """``run_decode_into`` from the packed q/k/v projection rows
        (pl_decode_run_qkv): the kernel forms q (LoRA delta, head norm, RoPE
        with ``rope_cos_sin`` from ``fused_ops.rope_cos_sin``), appends each
        row's new k/v at ``(page_id, page_offset)`` and attends.  ``lora`` is
        the (q, k, v) ``fused_ops.LoraUp`` triple or None.  Built for 16-bit
        caches, head_dim 128, 4 q heads per kv head, LoRA rank 0/8/16.

        ``o_shrink`` = (``_lib.LoraARows`` of o_proj, ``linear.LoraPartials``
        [B, parts, rank], n_adapters): the merge also writes o_proj's LoRA
        shrink partials of the attention output (pl_decode_run_qkv_oshrink);
        ``parts`` is :meth:`oshrink_parts`."""

        from .fused_ops import _lora_args, _rows2d

        plan = self._plan
        if plan is None:
            raise RuntimeError("plan_decode must be called before run_decode")
        _rows2d(qkv, "qkv")
        batch = qkv.shape[0]
        if batch != plan["batch"]:
            raise ValueError(f"qkv has batch {batch} but the plan has {plan['batch']}")
        if tuple(out.shape) != (batch, self.num_qo_heads, self.head_dim) or out.stride(2) != 1 or out.dtype != qkv.dtype:
            raise ValueError(f"out must be [{batch}, {self.num_qo_heads}, {self.head_dim}] of qkv's dtype")
        if qkv.device.type != "cuda":
            raise RuntimeError("run_decode needs tensors on a ROCm device")
        k, v, page_stride, token_stride, head_stride, num_pages = _cache_geometry(
            paged_kv_cache_layer, self.num_kv_heads, self.head_dim, self.page_size
        )
        if k.dtype != qkv.dtype:
            raise ValueError(f"qkv dtype {qkv.dtype} != KV cache dtype {k.dtype}")
        if plan["max_page"] is not None and plan["max_page"] >= num_pages:
            raise ValueError(f"page id {plan['max_page']} is outside the {num_pages}-page KV pool")
        for t, n in ((page_id, "page_id"), (page_offset, "page_offset")):
            if t.dtype != torch.int64 or t.numel() != batch:
                raise ValueError(f"{n} must be int64 [B]")
        if (rope_cos_sin.dtype != torch.float32 or tuple(rope_cos_sin.shape) != (batch, self.head_dim // 2, 2)
                or not rope_cos_sin.is_contiguous()):
            raise ValueError(f"rope_cos_sin must be a contiguous fp32 [{batch}, {self.head_dim // 2}, 2] tensor")
        if lse is not None and (lse.dtype != torch.float32 or tuple(lse.shape) != (batch, self.num_qo_heads) or not lse.is_contiguous()):
            raise ValueError("lse must be a contiguous fp32 [B, Hq] tensor")
        arr, ids, n = (None, None, 1)
        if lora is not None:
            if len(lora) != 3:
                raise ValueError("lora must be (q, k, v)")
            arr, ids, n = _lora_args(lora, adapter_ids, batch)
        _, indices_buf, last_buf = self._decode_graph_buffers
        args = (
            qkv.data_ptr(), qkv.stride(0), arr, ids, n,
            q_norm_weight.data_ptr() if q_norm_weight is not None else None,
            k_norm_weight.data_ptr() if k_norm_weight is not None else None,
            rope_cos_sin.data_ptr(), page_id.data_ptr(), page_offset.data_ptr(), float(eps),
            k.data_ptr(), v.data_ptr(), page_stride, token_stride, head_stride, num_pages,
            indices_buf.data_ptr(), last_buf.data_ptr(),
            out.data_ptr(), out.stride(0), out.stride(1),
            lse.data_ptr() if lse is not None else None,
            batch, self.num_qo_heads, self.num_kv_heads, self.head_dim, self.page_size,
            self.sm_scale, _lib.dtype_code(qkv.dtype), plan["target_items"], 0,
            self.workspace_buffer.data_ptr(), self.workspace_buffer.numel(),
        )
        if o_shrink is None:
            _lib.check(self._lib.pl_decode_run_qkv(*args, _lib.stream_handle(qkv.device)), "pl_decode_run_qkv")
            return out
        a_rows, parts, n_o = o_shrink
        if parts.partials.shape[0] != batch or parts.parts != self.oshrink_parts(batch):
            raise ValueError(f"o_proj partials must be [{batch}, {self.oshrink_parts(batch)}, rank]")
        if lora is None:
            if a_rows.adapter < 0 and (adapter_ids is None or adapter_ids.dtype != torch.int32
                                       or adapter_ids.numel() != batch):
                raise ValueError("per-row adapters need int32 adapter_ids [B]")
            args = args[:3] + (adapter_ids.data_ptr() if adapter_ids is not None else None, int(n_o)) + args[5:]
        elif n_o != n:
            raise ValueError("o_proj and q/k/v must stack the same adapters")
        p = parts.struct()
        _lib.check(self._lib.pl_decode_run_qkv_oshrink(*args, ctypes.byref(a_rows), ctypes.byref(p),
                                                       _lib.stream_handle(qkv.device)),
                   "pl_decode_run_qkv_oshrink")
        return out

    def oshrink_parts(self, batch: int) -> int:
        """Partial sums per row of the o_proj shrink the merge forms: one per
        (head, dim slice), with the merge's dim split for this batch."""
        pairs = batch * self.num_qo_heads
        ds = 4 if self.head_dim % 32 == 0 and pairs * 4 <= 256 else (2 if self.head_dim % 16 == 0 and pairs * 2 <= 256 else 1)
        return self.num_qo_heads * ds

    # ------------------------------------------------------------- prefill
    def plan_prefill(
        self,
        *,
        qo_indptr: torch.Tensor,
        paged_kv_indptr: torch.Tensor,
        paged_kv_indices: torch.Tensor,
        paged_kv_last_page_len: torch.Tensor,
        causal: bool = True,
        q_data_type: torch.dtype | None = None,
        kv_data_type: torch.dtype | None = None,
    ) -> None:
        """Plan packed multi-token attention (attention_backend.py:133-170).

        Request r owns query rows ``qo_indptr[r] .. qo_indptr[r+1]``, the last
        ``qo_len`` positions of its paged sequence; with ``causal`` query j
        sees kv positions ``<= kv_len - qo_len + j``.  The work list is built
        on the host (the tables are read there, as FlashInfer's prefill plan
        does), then tables and work list are uploaded on the current stream.
        """

        tables = (qo_indptr, paged_kv_indptr, paged_kv_indices, paged_kv_last_page_len)
        if any(t.dim() != 1 for t in tables):
            raise ValueError("prefill tables must be 1-D")
        batch = paged_kv_last_page_len.numel()
        if qo_indptr.numel() != batch + 1 or paged_kv_indptr.numel() != batch + 1:
            raise ValueError("qo_indptr and paged_kv_indptr must have batch + 1 entries")
        host = [t.detach().to("cpu", torch.int32).contiguous() for t in tables]
        qo_h, kv_h, ind_h, last_h = host
        max_page = _validate_host_table(kv_h, ind_h, last_h, self.page_size)
        if self.device.type != "cuda":
            raise RuntimeError("PagedDecodeAttention.plan_prefill needs a ROCm device")
        n = ctypes.c_int(0)
        args = (qo_h.data_ptr(), kv_h.data_ptr(), last_h.data_ptr(), batch, self.num_qo_heads, self.num_kv_heads,
                self.page_size, int(bool(causal)))
        _lib.check(self._lib.pl_prefill_plan(*args, None, 0, ctypes.byref(n)), "pl_prefill_plan")
        items_h = torch.empty(max(1, 2 * n.value), dtype=torch.int32)
        _lib.check(self._lib.pl_prefill_plan(*args, items_h.data_ptr(), n.value, ctypes.byref(n)), "pl_prefill_plan")
        dev = [t.to(self.device, non_blocking=False) for t in (qo_h, kv_h, ind_h, last_h, items_h)]
        self._prefill_plan = {
            "batch": batch,
            "tokens": int(qo_h[-1]) if batch else 0,
            "num_items": n.value,
            "causal": bool(causal),
            "max_page": max_page,
            "tables": dev,
            "q_data_type": q_data_type,
            "kv_data_type": kv_data_type,
        }

    def run_prefill(self, q: torch.Tensor, paged_kv_cache_layer) -> torch.Tensor:
        """One layer of paged prefill attention (attention_backend.py:172-190).

        ``q`` is packed ``[tokens, Hq, D]`` (returns the same shape) or
        ``[B, Hq, S, D]`` with S tokens per request (returns ``[B, Hq, S, D]``).
        """

        if q.dim() == 4:
            bsz, heads, seqlen, head_dim = q.shape
            out4 = torch.empty((bsz, heads, seqlen, head_dim), dtype=q.dtype, device=q.device)
            if bsz == 1:
                # [1, H, S, D] seen as [S, H, D]: strided views, no copies
                self.run_prefill_into(q[0].transpose(0, 1), paged_kv_cache_layer, out4[0].transpose(0, 1))
                return out4
            q_nhd = q.transpose(1, 2).reshape(bsz * seqlen, heads, head_dim)
            out = self.run_prefill_into(q_nhd, paged_kv_cache_layer, torch.empty_like(q_nhd))
            return out.reshape(bsz, seqlen, heads, head_dim).transpose(1, 2).contiguous()
        out = torch.empty(q.shape, dtype=q.dtype, device=q.device)
        return self.run_prefill_into(q, paged_kv_cache_layer, out)

    def run_prefill_into(self, q: torch.Tensor, paged_kv_cache_layer, out: torch.Tensor) -> torch.Tensor:
        """Writes ``out`` ([tokens, Hq, D], head_dim contiguous) for packed ``q``."""

        plan = getattr(self, "_prefill_plan", None)
        if plan is None:
            raise RuntimeError("plan_prefill must be called before run_prefill")
        if q.dim() != 3 or tuple(q.shape[1:]) != (self.num_qo_heads, self.head_dim):
            raise ValueError(f"q must be [tokens, {self.num_qo_heads}, {self.head_dim}], got {tuple(q.shape)}")
        if q.shape[0] != plan["tokens"]:
            raise ValueError(f"q has {q.shape[0]} tokens but the plan has {plan['tokens']}")
        if tuple(out.shape) != tuple(q.shape) or out.dtype != q.dtype or q.stride(2) != 1 or out.stride(2) != 1:
            raise ValueError("q and out must match in shape/dtype with a contiguous head_dim")
        if q.device.type != "cuda":
            raise RuntimeError("run_prefill needs tensors on a ROCm device")
        k, v, page_stride, token_stride, head_stride, num_pages = _cache_geometry(
            paged_kv_cache_layer, self.num_kv_heads, self.head_dim, self.page_size
        )
        if k.dtype != q.dtype:
            raise ValueError(f"q dtype {q.dtype} != KV cache dtype {k.dtype}")
        if plan["max_page"] >= num_pages:
            raise ValueError(f"page id {plan['max_page']} is outside the {num_pages}-page KV pool")
        qo_d, kv_d, ind_d, last_d, items_d = plan["tables"]
        status = self._lib.pl_prefill_run(
            q.data_ptr(), q.stride(0), q.stride(1),
            k.data_ptr(), v.data_ptr(), page_stride, token_stride, head_stride,
            num_pages,
            qo_d.data_ptr(), kv_d.data_ptr(), ind_d.data_ptr(), last_d.data_ptr(),
            items_d.data_ptr(), plan["num_items"],
            out.data_ptr(), out.stride(0), out.stride(1),
            plan["batch"], self.num_qo_heads, self.num_kv_heads, self.head_dim, self.page_size,
            int(plan["causal"]), self.sm_scale, _lib.dtype_code(q.dtype),
            _lib.stream_handle(q.device),
        )
        _lib.check(status, "pl_prefill_run")
        return out


# The reference's class name, for drop-in imports.
FlashInferAttentionBackend = PagedDecodeAttention


def kv_append(
    cache_layer,
    k: torch.Tensor,
    v: torch.Tensor,
    page_id: torch.Tensor,
    page_offset: torch.Tensor,
    *,
    num_kv_heads: int,
    head_dim: int,
    page_size: int,
) -> None:
    """Write one decode token per row into its page: the graph-safe append
    that replaces ``_append_decode_kv_static`` (layer_runner.py:399-412)."""

    kc, vc, page_stride, token_stride, head_stride, num_pages = _cache_geometry(
        cache_layer, num_kv_heads, head_dim, page_size
    )
    if k.dim() != 3 or k.shape != v.shape or tuple(k.shape[1:]) != (num_kv_heads, head_dim):
        raise ValueError(f"k and v must be [B, {num_kv_heads}, {head_dim}]")
    if k.stride(2) != 1 or v.stride(2) != 1:
        raise ValueError("k and v need a contiguous head_dim")
    if k.dtype != kc.dtype or v.dtype != kc.dtype:
        raise ValueError("k/v dtype must match the cache")
    batch = k.shape[0]
    if page_id.dtype != torch.int64 or page_offset.dtype != torch.int64:
        raise ValueError("page_id and page_offset must be int64")
    if page_id.numel() != batch or page_offset.numel() != batch:
        raise ValueError("page_id / page_offset must have one entry per row")
    lib = _lib.load()
    status = lib.pl_kv_append(
        k.data_ptr(), v.data_ptr(), k.stride(0), k.stride(1), v.stride(0), v.stride(1),
        kc.data_ptr(), vc.data_ptr(), page_stride, token_stride, head_stride,
        num_pages, page_size,
        page_id.data_ptr(), page_offset.data_ptr(),
        batch, num_kv_heads, head_dim, _lib.dtype_code(k.dtype), _lib.stream_handle(k.device),
    )
    _lib.check(status, "pl_kv_append")
