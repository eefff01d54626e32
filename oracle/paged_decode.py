"""float64 numpy restatement of paged decode attention and the decode KV append.

The reference's decode attention (model/flashinfer/attention_backend.py:120-131)
is FlashInfer's BatchDecodeWithPagedKVCacheWrapper.run on q/16 with
sm_scale = 16/sqrt(D) (:97, :128): per row b and query head h,
    o[b, h] = softmax((q[b, h] / 16) . K_b[:, h // g]^T * 16 / sqrt(D)) . V_b
with g = Hq / Hkv, and K_b / V_b the tokens of pages
indices[indptr[b]:indptr[b+1]] (NHD pool [P, 2, page, Hkv, D], K at index 0
and V at index 1 of dim 1: layer_runner.py:411-412, paged_kv_store.py:559-570),
all pages full except the last which holds last_page_len[b] tokens
(flashinfer_page_table.py:200-221).  The /16 and *16 cancel exactly in real
arithmetic, so the oracle computes softmax(q . K^T / sqrt(D)) . V in float64.

Test infrastructure only.
"""

from __future__ import annotations

import numpy as np


def _f64(a):
    a = np.asarray(a)
    return a.astype(np.float64, copy=False)


def gather_row_kv(cache, indptr, indices, last_page_len, b):
    """Dense K, V of row b: ([L, Hkv, D], [L, Hkv, D]) from an NHD pool.

    cache: [P, 2, page, Hkv, D] array, or a (k_pages, v_pages) pair each
    [P, page, Hkv, D].
    """
    if isinstance(cache, (tuple, list)):
        kp, vp = cache
    else:
        kp, vp = cache[:, 0], cache[:, 1]
    page_size = kp.shape[1]
    pages = list(indices[indptr[b]:indptr[b + 1]])
    if not pages:
        shape = (0,) + tuple(kp.shape[2:])
        return np.zeros(shape), np.zeros(shape)
    ks, vs = [], []
    for i, p in enumerate(pages):
        n = page_size if i < len(pages) - 1 else int(last_page_len[b])
        ks.append(_f64(kp[p, :n]))
        vs.append(_f64(vp[p, :n]))
    return np.concatenate(ks, 0), np.concatenate(vs, 0)


def decode_row(q_row, k, v, sm_scale):
    """softmax(q . K^T * sm_scale) . V for one row.

    q_row [Hq, D]; k, v [L, Hkv, D].  Returns (o [Hq, D], lse [Hq]) with lse
    the natural-log log-sum-exp of the scaled scores (-inf, and o = 0, for L = 0).
    """
    q_row = _f64(q_row)
    hq, d = q_row.shape
    L, hkv, _ = k.shape
    g = hq // hkv
    if L == 0:
        return np.zeros((hq, d)), np.full(hq, -np.inf)
    kh = np.repeat(k, g, axis=1)            # [L, Hq, D]: q head h reads kv head h // g
    vh = np.repeat(v, g, axis=1)
    s = np.einsum("hd,lhd->hl", q_row, kh) * sm_scale
    m = s.max(axis=1, keepdims=True)
    p = np.exp(s - m)
    denom = p.sum(axis=1, keepdims=True)
    o = np.einsum("hl,lhd->hd", p / denom, vh)
    lse = (m + np.log(denom))[:, 0]
    return o, lse


def paged_decode(q, cache, indptr, indices, last_page_len, sm_scale=None, rows=None):
    """Batched paged decode: returns (o [B, Hq, D], lse [B, Hq]) in float64.

    q [B, Hq, D] (or [B, Hq, 1, D]).  ``rows`` restricts the work to a subset
    of rows (the others stay zero / -inf) for large checks.
    """
    q = np.asarray(q)
    if q.ndim == 4:
        q = q[:, :, 0]
    B, hq, d = q.shape
    if sm_scale is None:
        sm_scale = 1.0 / np.sqrt(d)
    o = np.zeros((B, hq, d))
    lse = np.full((B, hq), -np.inf)
    for b in (range(B) if rows is None else rows):
        k, v = gather_row_kv(cache, indptr, indices, last_page_len, b)
        o[b], lse[b] = decode_row(q[b], k, v, sm_scale)
    return o, lse


def kv_append(cache, page_id, offset, k, v):
    """cache[page_id[b], 0, offset[b]] = k[b]; cache[page_id[b], 1, offset[b]] = v[b].

    The graph-static decode append of layer_runner.py:399-412 (index_put_
    with kv_key_index 0 and kv_value_index 1).  Modifies and returns ``cache``.
    """
    for b in range(len(page_id)):
        cache[page_id[b], 0, offset[b]] = k[b]
        cache[page_id[b], 1, offset[b]] = v[b]
    return cache


def algorithmic_bytes(indptr, last_page_len, page_size, num_qo_heads, num_kv_heads, head_dim, kv_bytes, q_bytes):
    """Bytes a decode call must move: K+V of every valid token, q in, o out, tables."""
    B = len(last_page_len)
    tokens = 0
    for b in range(B):
        n = indptr[b + 1] - indptr[b]
        if n:
            tokens += (n - 1) * page_size + int(last_page_len[b])
    kv = 2 * tokens * num_kv_heads * head_dim * kv_bytes
    qo = 2 * B * num_qo_heads * head_dim * q_bytes
    tables = 4 * (2 * B + 1 + int(indptr[-1]))
    return kv + qo + tables
