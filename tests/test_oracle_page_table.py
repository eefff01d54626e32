"""Pin the page-table oracle to the reference's own test vectors."""

import json
from pathlib import Path

import pytest

from oracle import page_table as opt

VECTORS = json.loads((Path(__file__).parent / "golden" / "reference_vectors.json").read_text())


@pytest.mark.parametrize("case", VECTORS["page_table"], ids=lambda c: c["source"][:60])
def test_oracle_matches_reference_vectors(case):
    indptr, indices, last = opt.build_batch_page_table([[tuple(s) for s in row] for row in case["rows"]], case["page_size"])
    assert indptr == case["indptr"]
    assert indices == case["indices"]
    assert last == case["last_page_len"]


@pytest.mark.parametrize("case", VECTORS["page_table_rejects"], ids=lambda c: c["source"][:60])
def test_oracle_rejects_reference_cases(case):
    with pytest.raises(ValueError):
        opt.build_batch_page_table([[tuple(s) for s in row] for row in case["rows"]], case["page_size"])


def test_oracle_coalesces_split_page_slices():
    # A page filled by a prefix slice and a decode slice counts once
    # (flashinfer_page_table.py:184-197): [5(0,1), 5(1,1)] -> one page of 2.
    assert opt.build_batch_page_table([[(5, 0, 1), (5, 1, 1)]], 4) == ([0, 1], [5], [2])
    # A gap does not merge, and then the second slice starts mid-page -> reject.
    with pytest.raises(ValueError):
        opt.build_batch_page_table([[(5, 0, 1), (5, 2, 1)]], 4)
    # Zero-length spans vanish; an empty row packs to zero pages.
    assert opt.build_batch_page_table([[(3, 0, 0)], [(4, 0, 3)]], 4) == ([0, 0, 1], [4], [0, 3])


def test_oracle_rejects_bad_lengths():
    with pytest.raises(ValueError):
        opt.build_batch_page_table([[(1, 0, 5)]], 4)   # longer than a page
    with pytest.raises(ValueError):
        opt.build_batch_page_table([[(1, 0, 2)]], 0)   # bad page size
