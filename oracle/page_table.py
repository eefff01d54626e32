"""Pure-Python restatement of the reference's page-table packing.

Follows model/kvcache/flashinfer_page_table.py:
  coalesce_block_spans            :184-197
  validate_and_collect_page_table :200-221
  build_batch_page_table          :160-181 (and :137-157 for one row)
and the per-step growth of a decode row, model/kvcache/paged_kv_store.py:
  reserve_one_token               reserve_spans :113-190 with one token
  advance_table                   one decode step of a batch (generation.py:1011-1035)
Spans are (block_id, start, length) triples, as KVBlockSpan (radix_types.py:31-36).
Pinning: the packing against the reference's own vectors (tests/golden);
the advance against the closed form of a row of L tokens (pages
ceil(L/ps), fill L - ps*(pages-1), slot (pages[L // ps], L % ps)).
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


def reserve_one_token(spans, page_size, take_page):
    """Append one token to a row's spans (paged_kv_store.py:113-190 with
    token_count 1): extend the last span if its page has room (:138-147),
    else allocate a page and append the span (page, 0, 1) (:149-164).

    ``take_page()`` returns the next page id of the row.  Returns the new
    span list and the chunk span written, as (page, offset).
    """
    spans = list(spans)
    if spans and spans[-1][2] < page_size:
        block_id, start, length = spans[-1]
        spans[-1] = (block_id, start, length + 1)
        return spans, (block_id, length)
    page = take_page()
    spans.append((page, 0, 1))
    return spans, (page, 0)


def table_to_spans(indptr, indices, last_page_len, page_size):
    """Per-row spans of a packed table: full pages, the last one filled to
    last_page_len (the inverse of build_batch_page_table)."""
    rows = []
    for b in range(len(indptr) - 1):
        pages = indices[indptr[b]:indptr[b + 1]]
        rows.append([(p, 0, page_size if i < len(pages) - 1 else last_page_len[b]) for i, p in enumerate(pages)])
    return rows


def advance_table(indptr, indices, last_page_len, page_size, new_pages):
    """One decode step of every row on a packed table: reserve one token per
    row (reserve_one_token) and repack (build_batch_page_table), as the
    batched decode loop does per step (generation.py:1011-1035).

    ``new_pages[b]`` is a list of page ids row b may take, in order; taken
    pages are popped from its front.  Returns (indptr, indices, last,
    positions, page_ids, offsets).
    """
    rows = table_to_spans(indptr, indices, last_page_len, page_size)
    out_rows, positions, page_ids, offsets = [], [], [], []
    for b, spans in enumerate(rows):
        positions.append(sum(s[2] for s in spans))
        spans, (page, off) = reserve_one_token(spans, page_size, lambda: new_pages[b].pop(0))
        out_rows.append(spans)
        page_ids.append(page)
        offsets.append(off)
    ip, ind, last = build_batch_page_table(out_rows, page_size)
    return ip, ind, last, positions, page_ids, offsets
