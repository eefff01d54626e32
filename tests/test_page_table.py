"""Host page-table packing (pagelora_amd.page_table) against the oracle and
the reference's vectors; buffer reuse semantics on CPU."""

import json
import random
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import page_table as opt
from pagelora_amd.page_table import (
    BatchPageTableBuffer,
    KVBlockSpan,
    PageTableBuffer,
    build_batch_page_table,
    build_page_table,
    pack_rows,
)

VECTORS = json.loads((Path(__file__).parent / "golden" / "reference_vectors.json").read_text())


def _spans(row):
    return [KVBlockSpan(*s) for s in row]


@pytest.mark.parametrize("case", VECTORS["page_table"], ids=lambda c: c["source"][:60])
def test_reference_vectors(case):
    table = build_batch_page_table([_spans(r) for r in case["rows"]], page_size=case["page_size"], device="cpu")
    assert table.paged_kv_indptr.tolist() == case["indptr"]
    assert table.paged_kv_indices.tolist() == case["indices"]
    assert table.paged_kv_last_page_len.tolist() == case["last_page_len"]
    assert table.paged_kv_indptr.dtype == torch.int32


@pytest.mark.parametrize("case", VECTORS["page_table_rejects"], ids=lambda c: c["source"][:60])
def test_reference_rejects(case):
    with pytest.raises(ValueError):
        build_batch_page_table([_spans(r) for r in case["rows"]], page_size=case["page_size"], device="cpu")


def test_single_row_builder():
    t = build_page_table([KVBlockSpan(11, 0, 2), KVBlockSpan(12, 0, 1)], page_size=2, device="cpu")
    assert (t.paged_kv_indptr.tolist(), t.paged_kv_indices.tolist(), t.paged_kv_last_page_len.tolist()) == ([0, 2], [11, 12], [1])


def _random_rows(rng, page_size):
    rows = []
    for _ in range(rng.randint(0, 6)):
        n_pages = rng.randint(0, 5)
        row = []
        for p in range(n_pages):
            pid = rng.randint(0, 50)
            full = p < n_pages - 1
            length = page_size if full else rng.randint(1, page_size)
            if rng.random() < 0.3 and length > 1:  # split a page into two adjacent slices
                cut = rng.randint(1, length - 1)
                row += [(pid, 0, cut), (pid, cut, length - cut)]
            else:
                row.append((pid, 0, length))
            if rng.random() < 0.1:
                row.append((pid, 0, 0))  # empty span
        if rng.random() < 0.1 and row:  # malformed: a non-full middle page or offset start
            i = rng.randrange(len(row))
            b, s, l = row[i]
            row[i] = (b, s + 1, l) if rng.random() < 0.5 else (b, s, max(1, l - 1))
        rows.append(row)
    return rows


@pytest.mark.parametrize("page_size", [1, 2, 16, 32])
def test_random_rows_match_oracle(page_size):
    rng = random.Random(1000 + page_size)
    for _ in range(300):
        rows = _random_rows(rng, page_size)
        try:
            want = opt.build_batch_page_table(rows, page_size)
        except ValueError:
            with pytest.raises(ValueError):
                pack_rows([[KVBlockSpan(*s) for s in r] for r in rows], page_size)
            continue
        indptr, indices, last = pack_rows([[KVBlockSpan(*s) for s in r] for r in rows], page_size)
        assert (indptr.tolist(), indices.tolist(), last.tolist()) == want


def test_single_buffer_reuses_tensors():
    # test_paged_kvcache_manager.py:483-500
    buf = PageTableBuffer(page_size=2, device="cpu", initial_capacity=1)
    first = buf.update_from_spans([KVBlockSpan(11, 0, 1)])
    second = buf.update_from_spans([KVBlockSpan(11, 0, 2), KVBlockSpan(12, 0, 1)])
    assert second.paged_kv_indptr.data_ptr() == first.paged_kv_indptr.data_ptr()
    assert second.paged_kv_last_page_len.data_ptr() == first.paged_kv_last_page_len.data_ptr()
    assert second.paged_kv_indptr.tolist() == [0, 2]
    assert second.paged_kv_indices.tolist() == [11, 12]
    assert second.paged_kv_last_page_len.tolist() == [1]


def test_batch_buffer_reuses_tensors_until_growth():
    # test_paged_kvcache_manager.py:503-543
    buf = BatchPageTableBuffer(page_size=4, device="cpu", initial_rows=2, initial_pages=4)
    first = buf.update_from_batch_spans([[KVBlockSpan(2, 0, 3)], [KVBlockSpan(4, 0, 4)]])
    sig = buf.signature()
    second = buf.update_from_batch_spans([[KVBlockSpan(2, 0, 4)], [KVBlockSpan(4, 0, 4), KVBlockSpan(5, 0, 1)]])
    assert buf.signature() == sig
    assert first.paged_kv_indptr.data_ptr() == second.paged_kv_indptr.data_ptr()
    assert second.paged_kv_indptr.tolist() == [0, 1, 3]
    assert second.paged_kv_indices.tolist() == [2, 4, 5]
    assert second.paged_kv_last_page_len.tolist() == [4, 1]
    # Growth past capacity replaces the buffers (new data pointers).
    buf.update_from_batch_spans([[KVBlockSpan(i, 0, 4)] for i in range(5)])
    assert buf.signature() != sig

