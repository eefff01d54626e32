"""torch fp32 CPU restatement of the decode hot path, for the CPU baseline.

The float64 numpy modules of this package are the checker; this module is
the same arithmetic in torch float32 on the host's cores, the speed a CPU
implementation of the path reaches (all threads).  It is timed next to the
GPU kernels and is itself checked against the float64 oracle
(tests/test_oracle_torch_cpu.py).

  paged_decode  the reference's run_decode arithmetic
                (model/flashinfer/attention_backend.py:120-131): per row,
                gather the row's pages from the NHD pool [P, 2, page, Hkv, D]
                (K at index 0, V at 1: layer_runner.py:411-412), upcast to
                fp32, o = softmax(q . K^T / sqrt(D)) . V per q head, kv head
                h // (Hq / Hkv); rows hold full pages except the last,
                which holds last_page_len tokens (flashinfer_page_table.py:200-221).
  lora_delta    the no-merge delta of LoRALinear.forward / _lora_delta
                (multilora/linear.py:226-231, model/flashinfer/packed_ops.py:534-553):
                (x A^T) B^T * scale per token, x A^T rounded to the 16-bit
                input type as F.linear returns it, adapter ids[t] per token.

Test infrastructure only (imported by tests/ and bench.py's cpu_baseline).
"""

from __future__ import annotations

import math

import torch


def paged_decode(q: torch.Tensor, cache: torch.Tensor, indptr, indices, last_page_len, rows=None) -> torch.Tensor:
    """o [B, Hq, D] fp32 for q [B, Hq, D] and a host pool [P, 2, page, Hkv, D]
    (any float type).  ``rows`` restricts the work to a subset of rows."""
    B, hq, d = q.shape
    ps, hkv = cache.shape[2], cache.shape[3]
    g = hq // hkv
    scale = 1.0 / math.sqrt(d)
    out = torch.zeros((B, hq, d), dtype=torch.float32)
    ip = [int(v) for v in indptr]
    for b in (range(B) if rows is None else rows):
        n = ip[b + 1] - ip[b]
        if n == 0:
            continue
        L = (n - 1) * ps + int(last_page_len[b])
        pages = torch.as_tensor(indices[ip[b]: ip[b + 1]], dtype=torch.long)
        kv = cache.index_select(0, pages)                      # [n, 2, ps, Hkv, D], one gather per row
        k = kv[:, 0].reshape(n * ps, hkv, d)[:L].float()       # [L, Hkv, D]
        v = kv[:, 1].reshape(n * ps, hkv, d)[:L].float()
        qh = q[b].float().reshape(hkv, g, d)                   # q heads grouped by kv head
        s = torch.matmul(qh, k.permute(1, 2, 0)) * scale       # [Hkv, g, L]
        p = torch.softmax(s, dim=-1)
        out[b] = torch.matmul(p, v.permute(1, 0, 2)).reshape(hq, d)
    return out


def _round(t: torch.Tensor, dtype: torch.dtype | None) -> torch.Tensor:
    return t if dtype is None else t.to(dtype).float()


def lora_delta(x: torch.Tensor, ids, a_stack: torch.Tensor, b_stack: torch.Tensor, scale: float,
               intermediate: torch.dtype | None = None) -> torch.Tensor:
    """[T, out] fp32: row t is (x_t A[ids[t]]^T) B[ids[t]]^T * scale (0 for ids
    outside [0, n)); tokens are grouped by adapter so each adapter is two GEMMs."""
    x = x.float()
    n = a_stack.shape[0]
    ids = torch.as_tensor(ids, dtype=torch.long)
    out = torch.zeros((x.shape[0], b_stack.shape[1]), dtype=torch.float32)
    for a in range(n):
        sel = (ids == a).nonzero().flatten()
        if sel.numel() == 0:
            continue
        down = _round(x.index_select(0, sel) @ a_stack[a].float().t(), intermediate)
        out.index_copy_(0, sel, down @ b_stack[a].float().t() * scale)
    return out
