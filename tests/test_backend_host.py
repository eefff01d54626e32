"""Host-side behaviour of the drop-in backend that needs no GPU: constructor
checks and page-table validation (attention_backend.py:44-45 raises
ValueError for a bad head ratio; flashinfer_page_table.py:205-218 for bad
tables)."""

import pytest
import torch

from pagelora_amd.attention_backend import FlashInferAttentionBackend, PagedDecodeAttention


def _backend(**kw):
    args = dict(device=torch.device("cpu"), workspace_mb=1, num_qo_heads=28, num_kv_heads=4, head_dim=128,
                page_size=16)
    args.update(kw)
    return PagedDecodeAttention(**args)


def test_alias_and_attributes():
    assert FlashInferAttentionBackend is PagedDecodeAttention
    be = _backend()
    assert be.page_size == 16 and be.workspace_buffer.numel() == 1 << 20
    assert be.query_rescale == 1.0 and be.sm_scale == pytest.approx(128 ** -0.5)
    assert be.decode_use_tensor_cores is False and be.use_flashinfer_qk_norm is False


def test_head_ratio_must_divide():
    with pytest.raises(ValueError):
        _backend(num_qo_heads=30, num_kv_heads=4)
    with pytest.raises(ValueError):
        _backend(num_kv_heads=0)


@pytest.mark.parametrize(
    "indptr,indices,last",
    [
        ([1, 2], [0, 0], [1]),        # indptr must start at 0
        ([0, 2, 1], [0, 0], [1, 1]),  # non-decreasing
        ([0, 3], [0, 0], [1]),        # points past indices
        ([0, 1], [0], [17]),          # last_page_len > page_size
        ([0, 1], [0], [0]),           # last_page_len < 1 on a non-empty row
        ([0, 1], [-3], [4]),          # negative page id
    ],
)
def test_bad_host_tables_raise_before_any_device_work(indptr, indices, last):
    be = _backend()
    with pytest.raises(ValueError):
        be.plan_decode(paged_kv_indptr=torch.tensor(indptr, dtype=torch.int32),
                       paged_kv_indices=torch.tensor(indices, dtype=torch.int32),
                       paged_kv_last_page_len=torch.tensor(last, dtype=torch.int32))


def test_wrong_dtype_or_shape_raises():
    be = _backend()
    with pytest.raises(ValueError):
        be.plan_decode(paged_kv_indptr=torch.tensor([0, 1]), paged_kv_indices=torch.tensor([0]),
                       paged_kv_last_page_len=torch.tensor([1]))  # int64, not int32
    with pytest.raises(ValueError):
        be.plan_decode(paged_kv_indptr=torch.tensor([0, 1, 2], dtype=torch.int32),
                       paged_kv_indices=torch.tensor([0, 1], dtype=torch.int32),
                       paged_kv_last_page_len=torch.tensor([1], dtype=torch.int32))  # B+1 mismatch


def test_cpu_backend_refuses_to_plan_a_valid_table():
    be = _backend()
    with pytest.raises(RuntimeError):
        be.plan_decode(paged_kv_indptr=torch.tensor([0, 1], dtype=torch.int32),
                       paged_kv_indices=torch.tensor([3], dtype=torch.int32),
                       paged_kv_last_page_len=torch.tensor([5], dtype=torch.int32))


def _i32(x):
    return torch.tensor(x, dtype=torch.int32)


@pytest.mark.parametrize(
    "qo,indptr,indices,last",
    [
        ([0, 1], [0, 1, 2], [0, 0], [1]),  # qo_indptr / kv_indptr lengths differ from the batch
        ([0, 1], [0, 3], [0, 0], [1]),     # kv_indptr points past indices
        ([0, 1], [0, 1], [0], [17]),       # last_page_len > page_size
        ([0, 1], [0, 1], [-3], [4]),       # negative page id
    ],
)
def test_bad_prefill_tables_raise_before_any_device_work(qo, indptr, indices, last):
    be = _backend()
    with pytest.raises(ValueError):
        be.plan_prefill(qo_indptr=_i32(qo), paged_kv_indptr=_i32(indptr), paged_kv_indices=_i32(indices),
                        paged_kv_last_page_len=_i32(last))


def test_cpu_backend_refuses_to_plan_or_run_prefill():
    be = _backend()
    with pytest.raises(RuntimeError):
        be.plan_prefill(qo_indptr=_i32([0, 2]), paged_kv_indptr=_i32([0, 1]), paged_kv_indices=_i32([0]),
                        paged_kv_last_page_len=_i32([2]))
    with pytest.raises(RuntimeError, match="plan_prefill"):
        be.run_prefill(torch.ones(2, 28, 128), torch.zeros(1, 2, 16, 4, 128))


def _prefix_backend(**kw):
    """A CPU-constructed backend with the library loaded for its size query
    (the detection is host logic; nothing runs on a device)."""
    from pagelora_amd import _lib

    be = PagedDecodeAttention(device="cpu", workspace_mb=64, num_qo_heads=32, num_kv_heads=8, head_dim=128,
                              page_size=16, **kw)
    be._lib = _lib.load()
    return be


def _table(rows):
    indptr = [0]
    for r in rows:
        indptr.append(indptr[-1] + len(r))
    return torch.tensor(indptr, dtype=torch.int32), torch.tensor([p for r in rows for p in r], dtype=torch.int32)


@pytest.mark.parametrize("rows,want", [
    # 4 rows behind 10 shared pages: whole 2-page prefix items (10)
    ([list(range(10)) + [100 + b, 200 + b] for b in range(4)], 10),
    # an odd shared count rounds down to whole items
    ([list(range(9)) + [100 + b] for b in range(3)], 8),
    # every row keeps its last page (the one being appended to) as its own
    ([list(range(12)) for _ in range(2)], 10),
    # rows that differ from the third page on: below two items, nothing shared
    ([[0, 1, 2 + b, 3, 4, 5] for b in range(2)], 0),
    # one row, or more than 4: no sharing
    ([list(range(10)) + [100]], 0),
    ([list(range(10)) + [100 + b] for b in range(5)], 0),
])
def test_shared_prefix_detection(rows, want):
    be = _prefix_backend()
    indptr, indices = _table(rows)
    assert be._shared_prefix_pages(indptr, indices, len(rows), 16) == want


def test_shared_prefix_needs_gqa4_head128_and_32_token_items():
    rows = [list(range(10)) + [100 + b] for b in range(4)]
    indptr, indices = _table(rows)
    be = _prefix_backend()
    be.share_prefix = False
    assert be._shared_prefix_pages(indptr, indices, 4, 16) == 0
    from pagelora_amd import _lib
    for kw in (dict(num_qo_heads=8, num_kv_heads=8, head_dim=128), dict(num_qo_heads=32, num_kv_heads=8, head_dim=64)):
        b2 = PagedDecodeAttention(device="cpu", workspace_mb=64, page_size=16, **kw)
        b2._lib = _lib.load()
        assert b2._shared_prefix_pages(indptr, indices, 4, 16) == 0
    b3 = PagedDecodeAttention(device="cpu", workspace_mb=64, num_qo_heads=32, num_kv_heads=8, head_dim=128,
                              page_size=12)
    b3._lib = _lib.load()
    assert b3._shared_prefix_pages(indptr, indices, 4, 16) == 0
