"""Pure-Python restatement of the reference's page-table packing.

Follows model/kvcache/flashinfer_page_table.py:
  coalesce_block_spans            :184-197
  validate_and_collect_page_table :200-221
  build_batch_page_table          :160-181 (and :137-157 for one row)
Spans are (block_id, start, length) triples, as KVBlockSpan (radix_types.py:31-36).
Test infrastructure only.
"""

from __future__ import annotations


def coalesce_block_spans(spans):
    """Merge adjacent slices of the same physical page; drop empty spans (:184-197)."""
    merged = []
    for block_id, start, length in spans:
        if length <= 0:
            continue
        if merged:
            pb, ps, pl = merged[-1]
            if pb == block_id and ps + pl == start:
                merged[-1] = (pb, ps, pl + length)
                continue
        merged.append((block_id, start, length))
    return merged


def validate_and_collect_page_table(spans, page_size):
    """Return (page ids, last_page_len) or raise ValueError (:200-221)."""
    if page_size <= 0:
        raise ValueError("page_size must be positive")
    coalesced = coalesce_block_spans(spans)
    indices = []
    last = 0
    for i, (block_id, start, length) in enumerate(coalesced):
        if start != 0:
            raise ValueError("spans must start at page offset 0")
        if length <= 0 or length > page_size:
            raise ValueError("span length out of range")
        if i < len(coalesced) - 1 and length != page_size:
            raise ValueError("non-last spans must be full pages")
        indices.append(block_id)
        last = length
    return indices, last


def build_batch_page_table(batch_spans, page_size):
    """Return (indptr, indices, last_page_len) as Python lists (:160-181)."""
    indptr = [0]
    indices = []
    lasts = []
    for spans in batch_spans:
        row, last = validate_and_collect_page_table(spans, page_size)
        indices.extend(row)
        indptr.append(len(indices))
        lasts.append(last)
    return indptr, indices, lasts
