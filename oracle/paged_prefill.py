"""float64 numpy restatement of paged prefill (multi-query) attention.

The reference's prefill attention (model/flashinfer/attention_backend.py:133-190)
is FlashInfer's BatchPrefillWithPagedKVCacheWrapper planned with
``qo_indptr`` / ``paged_kv_indptr`` / ``paged_kv_indices`` /
``paged_kv_last_page_len``, ``causal=True`` (generation.py:266-275,
300-308) and run on q/16 with sm_scale 16/sqrt(D).  Request r's queries
are rows qo_indptr[r] .. qo_indptr[r+1] of the packed q and are the LAST
qo_len positions of its kv_len-token sequence: the reference appends a
segment's K/V into the pages before attention reads them
(layer_runner.py:85-102), so kv_len counts prefix + segment.  The causal
mask is aligned to the bottom right: query j (0-based within the request)
sees kv positions 0 .. kv_len - qo_len + j.  GQA: q head h reads kv head
h // (Hq / Hkv).

Test infrastructure only.
"""

from __future__ import annotations

import numpy as np

from .paged_decode import _f64, gather_row_kv


def prefill_request(q_req, k, v, sm_scale, causal=True):
    """Attention of one request's queries.

    q_req [qo_len, Hq, D]; k, v [kv_len, Hkv, D].  Returns o [qo_len, Hq, D]
    (float64).  With ``causal`` query j sees kv positions <= kv_len - qo_len + j.
    """
    q_req = _f64(q_req)
    qo_len, hq, d = q_req.shape
    kv_len, hkv, _ = k.shape
    g = hq // hkv
    o = np.zeros((qo_len, hq, d))
    if qo_len == 0 or kv_len == 0:
        return o
    kh = np.repeat(_f64(k), g, axis=1)  # [kv_len, Hq, D]
    vh = np.repeat(_f64(v), g, axis=1)
    s = np.einsum("jhd,lhd->hjl", q_req, kh) * sm_scale  # [Hq, qo_len, kv_len]
    if causal:
        limit = kv_len - qo_len + np.arange(qo_len)  # last visible position per query
        visible = np.arange(kv_len)[None, :] <= limit[:, None]
        s = np.where(visible[None], s, -np.inf)
    m = s.max(axis=2, keepdims=True)
    p = np.exp(s - m)
    p /= p.sum(axis=2, keepdims=True)
    return np.einsum("hjl,lhd->jhd", p, vh)


def paged_prefill(q, cache, qo_indptr, kv_indptr, kv_indices, kv_last_page_len, sm_scale=None, causal=True,
                  requests=None):
    """Packed paged prefill: q [tokens, Hq, D] -> o [tokens, Hq, D] (float64).

    ``requests`` restricts the work to a subset of requests (other rows stay 0).
    """
    q = np.asarray(q)
    tokens, hq, d = q.shape
    if sm_scale is None:
        sm_scale = 1.0 / np.sqrt(d)
    o = np.zeros((tokens, hq, d))
    batch = len(kv_last_page_len)
    for r in (range(batch) if requests is None else requests):
        a, b = int(qo_indptr[r]), int(qo_indptr[r + 1])
        k, v = gather_row_kv(cache, kv_indptr, kv_indices, kv_last_page_len, r)
        o[a:b] = prefill_request(q[a:b], k, v, sm_scale, causal)
    return o


def prefill_flops(qo_indptr, kv_indptr, kv_last_page_len, page_size, num_qo_heads, head_dim, causal=True):
    """Multiply-add FLOPs (2 per MAC) of Q K^T and P V over the visible pairs."""
    pairs = 0
    for r in range(len(kv_last_page_len)):
        qo_len = int(qo_indptr[r + 1] - qo_indptr[r])
        n = int(kv_indptr[r + 1] - kv_indptr[r])
        kv_len = (n - 1) * page_size + int(kv_last_page_len[r]) if n else 0
        if causal:
            first = kv_len - qo_len + 1  # positions seen by query 0
            pairs += qo_len * first + qo_len * (qo_len - 1) // 2
        else:
            pairs += qo_len * kv_len
    return 4 * pairs * num_qo_heads * head_dim
