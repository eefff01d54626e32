"""Host-side prefill plan (pl_prefill_plan): work items, order and errors.

pl_prefill_plan reads host tables only, so it runs without a GPU.
"""

from __future__ import annotations

import ctypes

import numpy as np
import pytest

from pagelora_amd import _lib

ROWS_PER_ITEM = 64
TILE = 64  # kv tokens per unit of the plan's work estimate (kPlanTile)


def _plan(qo_indptr, kv_indptr, last, hq, hkv, page_size, causal=True, max_items=None):
    lib = _lib.load()
    qo = np.ascontiguousarray(qo_indptr, dtype=np.int32)
    kv = np.ascontiguousarray(kv_indptr, dtype=np.int32)
    la = np.ascontiguousarray(last, dtype=np.int32)
    n = ctypes.c_int(-1)
    args = (qo.ctypes.data, kv.ctypes.data, la.ctypes.data, len(la), hq, hkv, page_size, int(causal))
    _lib.check(lib.pl_prefill_plan(*args, None, 0, ctypes.byref(n)), "pl_prefill_plan")
    count = n.value
    cap = count if max_items is None else max_items
    items = np.zeros(max(1, 2 * cap), dtype=np.int32)
    _lib.check(lib.pl_prefill_plan(*args, items.ctypes.data, cap, ctypes.byref(n)), "pl_prefill_plan")
    assert n.value == count
    return items[: 2 * count].reshape(-1, 2)


def _expected_items(qo_lens, kv_lens, g, causal=True):
    out = []
    for r, (n, L) in enumerate(zip(qo_lens, kv_lens)):
        rows = n * g
        for r0 in range(0, rows, ROWS_PER_ITEM):
            last_row = min(r0 + ROWS_PER_ITEM, rows) - 1
            max_pos = L - n + last_row // g if causal else L - 1
            out.append((max_pos // TILE + 1, r, r0))
    return out


def _tables(qo_lens, kv_lens, ps):
    pages = [-(-L // ps) for L in kv_lens]
    qo = np.concatenate([[0], np.cumsum(qo_lens)])
    kv = np.concatenate([[0], np.cumsum(pages)])
    last = [L - ps * (p - 1) for L, p in zip(kv_lens, pages)]
    return qo, kv, last


@pytest.mark.parametrize("g", [1, 4])
@pytest.mark.parametrize("causal", [True, False])
def test_items_cover_every_row_once_longest_first(g, causal):
    qo_lens, kv_lens = [100, 0, 7, 300], [2148, 5, 7, 300]
    qo, kv, last = _tables(qo_lens, kv_lens, 16)
    items = _plan(qo, kv, last, 8 * g, 8, 16, causal)
    exp = _expected_items(qo_lens, kv_lens, g, causal)
    assert sorted(map(tuple, items.tolist())) == sorted((r, r0) for _, r, r0 in exp)
    work = {(r, r0): w for w, r, r0 in exp}
    ws = [work[tuple(it)] for it in items.tolist()]
    assert ws == sorted(ws, reverse=True)


def test_empty_batch_and_no_queries():
    assert _plan([0], [0], [], 4, 4, 16).shape == (0, 2)
    assert _plan([0, 0], [0, 1], [3], 4, 4, 16).shape == (0, 2)


def test_rejects_causal_query_longer_than_kv():
    qo, kv, last = _tables([9], [8], 4)
    with pytest.raises(ValueError, match="exceeds kv_len"):
        _plan(qo, kv, last, 2, 2, 4, causal=True)
    assert len(_plan(qo, kv, last, 2, 2, 4, causal=False)) == 1


@pytest.mark.parametrize("bad_last", [0, 5])
def test_rejects_last_page_len_out_of_range(bad_last):
    with pytest.raises(ValueError, match="last_page_len"):
        _plan([0, 1], [0, 1], [bad_last], 2, 2, 4)


def test_rejects_bad_head_ratio_and_decreasing_indptr():
    with pytest.raises(ValueError, match="multiple"):
        _plan([0, 1], [0, 1], [1], 6, 4, 4)
    with pytest.raises(ValueError, match="non-decreasing"):
        _plan([0, 2, 1], [0, 1, 2], [4, 4], 2, 2, 4)


def test_too_few_items_is_a_workspace_error():
    qo, kv, last = _tables([200], [200], 16)
    with pytest.raises(_lib.WorkspaceTooSmallError):
        _plan(qo, kv, last, 4, 1, 16, max_items=2)
