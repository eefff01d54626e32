"""Pin the paged-decode oracle: closed forms, invariances, a library routine."""

import json
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import paged_decode as opd

VECTORS = json.loads((Path(__file__).parent / "golden" / "reference_vectors.json").read_text())


def _random_case(rng, B=3, hq=8, hkv=2, d=16, ps=4, pool=40, max_len=30):
    lens = rng.integers(1, max_len + 1, size=B)
    n_pages = (lens + ps - 1) // ps
    perm = rng.permutation(pool)[: n_pages.sum()]
    indptr = np.concatenate([[0], np.cumsum(n_pages)]).astype(np.int64)
    last = (lens - ps * (n_pages - 1)).astype(np.int64)
    cache = rng.standard_normal((pool, 2, ps, hkv, d))
    q = rng.standard_normal((B, hq, d))
    return q, cache, indptr, perm, last, lens


def test_reference_decode_vector():
    # test_flashinfer_backend.py:157-177 restated: equal huge-magnitude scores.
    case = VECTORS["decode"][0]
    ps = 2
    cache = np.zeros((1, 2, ps, 1, 1))
    cache[0, 0, :, 0, 0] = case["k"]
    cache[0, 1, :, 0, 0] = case["v"]
    q = np.full((2, 1, 1), case["q"])
    o, _ = opd.paged_decode(q, cache, [0, 1, 2], [0, 0], case["rows_tokens"])
    assert o[:, 0, 0].tolist() == pytest.approx(case["expected"], abs=1e-12)


def test_single_token_returns_its_value():
    rng = np.random.default_rng(0)
    cache = rng.standard_normal((3, 2, 16, 2, 8))
    q = rng.standard_normal((1, 4, 8)) * 50
    o, lse = opd.paged_decode(q, cache, [0, 1], [2], [1])
    np.testing.assert_allclose(o[0], np.repeat(cache[2, 1, 0], 2, axis=0), atol=1e-12)
    # lse of one score is the score itself
    s = np.einsum("hd,hd->h", q[0], np.repeat(cache[2, 0, 0], 2, axis=0)) / np.sqrt(8)
    np.testing.assert_allclose(lse[0], s, atol=1e-10)


def test_equal_keys_average_values():
    rng = np.random.default_rng(1)
    ps, L = 16, 37
    cache = np.zeros((4, 2, ps, 1, 8))
    cache[:, 0] = rng.standard_normal(8)  # every key identical
    cache[:, 1] = rng.standard_normal((4, ps, 1, 8))
    q = rng.standard_normal((1, 1, 8))
    pages = [3, 0, 2]
    o, lse = opd.paged_decode(q, cache, [0, 3], pages, [L - 2 * ps])
    vals = np.concatenate([cache[3, 1], cache[0, 1], cache[2, 1, : L - 2 * ps]])
    np.testing.assert_allclose(o[0, 0], vals[:, 0].mean(0), atol=1e-12)
    s = q[0, 0] @ cache[0, 0, 0, 0] / np.sqrt(8)
    np.testing.assert_allclose(lse[0, 0], s + np.log(L), atol=1e-10)


def test_matches_torch_sdpa_float64():
    rng = np.random.default_rng(2)
    q, cache, indptr, idx, last, lens = _random_case(rng)
    o, _ = opd.paged_decode(q, cache, indptr, idx, last)
    for b in range(len(lens)):
        k, v = opd.gather_row_kv(cache, indptr, idx, last, b)
        assert k.shape[0] == lens[b]
        g = q.shape[1] // k.shape[1]
        kt = torch.from_numpy(np.repeat(k, g, axis=1)).permute(1, 0, 2)  # [Hq, L, D]
        vt = torch.from_numpy(np.repeat(v, g, axis=1)).permute(1, 0, 2)
        qt = torch.from_numpy(q[b])[:, None, :]                            # [Hq, 1, D]
        ref = torch.nn.functional.scaled_dot_product_attention(qt, kt, vt)[:, 0]
        np.testing.assert_allclose(o[b], ref.numpy(), atol=1e-12)


def test_brute_force_tiny():
    rng = np.random.default_rng(3)
    q, cache, indptr, idx, last, lens = _random_case(rng, B=2, hq=2, hkv=1, d=3, ps=2, pool=8, max_len=5)
    o, _ = opd.paged_decode(q, cache, indptr, idx, last, sm_scale=0.7)
    for b in range(2):
        toks = []
        pages = idx[indptr[b]:indptr[b + 1]]
        for i, p in enumerate(pages):
            n = 2 if i < len(pages) - 1 else last[b]
            toks += [(p, t) for t in range(n)]
        for h in range(2):
            w = [np.exp(0.7 * sum(q[b, h, j] * cache[p, 0, t, 0, j] for j in range(3))) for p, t in toks]
            want = [sum(wi * cache[p, 1, t, 0, j] for wi, (p, t) in zip(w, toks)) / sum(w) for j in range(3)]
            np.testing.assert_allclose(o[b, h], want, atol=1e-12)


def test_page_permutation_invariance_and_pool_padding():
    rng = np.random.default_rng(4)
    q, cache, indptr, idx, last, _ = _random_case(rng)
    o1, l1 = opd.paged_decode(q, cache, indptr, idx, last)
    perm = rng.permutation(cache.shape[0])          # new physical position of each page
    cache2 = np.empty_like(cache)
    cache2[perm] = cache
    cache2 = np.concatenate([cache2, np.full((5,) + cache.shape[1:], np.nan)])  # padded pool
    o2, l2 = opd.paged_decode(q, cache2, indptr, perm[idx], last)
    np.testing.assert_allclose(o1, o2, atol=1e-13)
    np.testing.assert_allclose(l1, l2, atol=1e-13)


def test_gqa_equals_mha_with_repeated_heads():
    rng = np.random.default_rng(5)
    q, cache, indptr, idx, last, _ = _random_case(rng, hq=8, hkv=2)
    o_gqa, _ = opd.paged_decode(q, cache, indptr, idx, last)
    o_mha, _ = opd.paged_decode(q, np.repeat(cache, 4, axis=3), indptr, idx, last)
    np.testing.assert_allclose(o_gqa, o_mha, atol=1e-13)


def test_split_kv_tuple_layout_equals_pool_layout():
    rng = np.random.default_rng(6)
    q, cache, indptr, idx, last, _ = _random_case(rng)
    o1, _ = opd.paged_decode(q, cache, indptr, idx, last)
    o2, _ = opd.paged_decode(q, (cache[:, 0], cache[:, 1]), indptr, idx, last)
    np.testing.assert_array_equal(o1, o2)


def test_nan_outside_valid_tokens_is_never_read():
    rng = np.random.default_rng(7)
    q, cache, indptr, idx, last, _ = _random_case(rng)
    o1, _ = opd.paged_decode(q, cache, indptr, idx, last)
    poisoned = cache.copy()
    used = set(idx.tolist())
    for p in range(cache.shape[0]):
        if p not in used:
            poisoned[p] = np.nan
    for b in range(len(last)):
        lastp = idx[indptr[b + 1] - 1]
        poisoned[lastp, :, last[b]:] = np.nan
    o2, _ = opd.paged_decode(q, poisoned, indptr, idx, last)
    np.testing.assert_array_equal(o1, o2)


def test_kv_append_matches_index_put():
    rng = np.random.default_rng(8)
    cache = rng.standard_normal((6, 2, 4, 2, 8))
    k = rng.standard_normal((3, 2, 8))
    v = rng.standard_normal((3, 2, 8))
    pid, off = np.array([5, 0, 2]), np.array([3, 0, 1])
    want = torch.from_numpy(cache.copy())
    want.index_put_((torch.from_numpy(pid), torch.zeros(3, dtype=torch.long), torch.from_numpy(off)), torch.from_numpy(k))
    want.index_put_((torch.from_numpy(pid), torch.ones(3, dtype=torch.long), torch.from_numpy(off)), torch.from_numpy(v))
    got = opd.kv_append(cache.copy(), pid, off, k, v)
    np.testing.assert_array_equal(got, want.numpy())


def test_algorithmic_bytes_formula():
    # 2 rows: 3 pages (last 5 of 16) and 1 page (7): 37 + 7 tokens.
    n = opd.algorithmic_bytes([0, 3, 4], [5, 7], 16, 32, 8, 128, 2, 2)
    assert n == 2 * 44 * 8 * 128 * 2 + 2 * 2 * 32 * 128 * 2 + 4 * (2 * 2 + 1 + 4)
