"""Pin the paged-prefill oracle: the reference's known answer, the decode
oracle row by row, chunking consistency, torch's SDPA, GQA = repeated MHA."""

from __future__ import annotations

import json
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import paged_decode as opd
from oracle import paged_prefill as opp

VECTORS = json.loads((Path(__file__).parent / "golden" / "reference_vectors.json").read_text())


def _random_pool(rng, kv_lens, page_size, hkv, d, spare=3):
    """Pages for each request in a shuffled pool; returns cache, kv_indptr, kv_indices, last."""
    n_pages = [-(-L // page_size) for L in kv_lens]
    total = sum(n_pages) + spare
    perm = rng.permutation(total)
    cache = rng.standard_normal((total, 2, page_size, hkv, d))
    indptr = np.concatenate([[0], np.cumsum(n_pages)]).astype(np.int64)
    indices = perm[: indptr[-1]]
    last = np.array([L - page_size * (n - 1) for L, n in zip(kv_lens, n_pages)])
    return cache, indptr, indices, last


def test_reference_prefill_vector():
    """test_flashinfer_backend.py:157-177 in its own form: causal [1, 5]."""
    case = VECTORS["prefill"][0]
    ps, d = case["page_size"], case["head_dim"]
    cache = np.zeros((1, 2, ps, 1, d))
    cache[0, 0, :, 0, 0] = case["k"]
    cache[0, 1, :, 0, 0] = case["v"]
    q = np.array(case["q"]).reshape(-1, 1, d)
    o = opp.paged_prefill(q, cache, case["qo_indptr"], case["kv_indptr"], case["kv_indices"],
                          case["kv_last_page_len"], causal=case["causal"])
    np.testing.assert_allclose(o[:, 0, 0], case["expected"], rtol=0, atol=1e-12)


@pytest.mark.parametrize("g", [1, 4])
def test_each_query_equals_decode_over_its_visible_prefix(g):
    """Query j of a request with kv_len L and qo_len n sees exactly the first
    L - n + j + 1 tokens: one decode row over a table truncated to them."""
    rng = np.random.default_rng(7)
    ps, hkv, d = 4, 2, 8
    kv_lens, qo_lens = [13, 9, 4], [5, 9, 1]
    cache, indptr, indices, last = _random_pool(rng, kv_lens, ps, hkv, d)
    qo_indptr = np.concatenate([[0], np.cumsum(qo_lens)])
    q = rng.standard_normal((qo_indptr[-1], hkv * g, d))
    o = opp.paged_prefill(q, cache, qo_indptr, indptr, indices, last)
    for r, (L, n) in enumerate(zip(kv_lens, qo_lens)):
        pages = indices[indptr[r]:indptr[r + 1]]
        for j in range(n):
            visible = L - n + j + 1
            np_ = -(-visible // ps)
            od, _ = opd.paged_decode(q[qo_indptr[r] + j][None], cache, [0, np_], pages[:np_],
                                     [visible - ps * (np_ - 1)])
            np.testing.assert_allclose(o[qo_indptr[r] + j], od[0], rtol=0, atol=1e-12)


def test_chunked_prefill_matches_full_prefill():
    """Prefilling the last m tokens after the first L - m are cached gives the
    same rows as prefilling all L at once (the reference's segmented prefill)."""
    rng = np.random.default_rng(11)
    ps, hkv, d, L = 8, 1, 16, 37
    cache, indptr, indices, last = _random_pool(rng, [L], ps, hkv, d)
    q = rng.standard_normal((L, 2, d))
    full = opp.paged_prefill(q, cache, [0, L], indptr, indices, last)
    for m in (1, 5, 16, 36):
        part = opp.paged_prefill(q[L - m:], cache, [0, m], indptr, indices, last)
        np.testing.assert_allclose(part, full[L - m:], rtol=0, atol=1e-12)


@pytest.mark.parametrize("causal", [True, False])
def test_matches_torch_sdpa(causal):
    """Square causal prefill is torch's is_causal SDPA; non-causal is plain SDPA
    over qo_len != kv_len (torch's routine, float64, on the CPU)."""
    rng = np.random.default_rng(3)
    ps, hq, d = 16, 4, 32
    L = 45
    qo = L if causal else 7
    cache, indptr, indices, last = _random_pool(rng, [L], ps, hq, d)
    q = rng.standard_normal((qo, hq, d))
    o = opp.paged_prefill(q, cache, [0, qo], indptr, indices, last, causal=causal)
    k, v = opd.gather_row_kv(cache, indptr, indices, last, 0)
    ref = torch.nn.functional.scaled_dot_product_attention(
        torch.from_numpy(q).transpose(0, 1), torch.from_numpy(k).transpose(0, 1),
        torch.from_numpy(v).transpose(0, 1), is_causal=causal,
    ).transpose(0, 1).numpy()
    np.testing.assert_allclose(o, ref, rtol=0, atol=1e-12)


def test_gqa_equals_mha_with_repeated_kv():
    rng = np.random.default_rng(5)
    ps, hkv, g, d = 4, 2, 4, 8
    cache, indptr, indices, last = _random_pool(rng, [10, 3], ps, hkv, d)
    qo_indptr = [0, 6, 9]
    q = rng.standard_normal((9, hkv * g, d))
    o_gqa = opp.paged_prefill(q, cache, qo_indptr, indptr, indices, last)
    o_mha = opp.paged_prefill(q, np.repeat(cache, g, axis=3), qo_indptr, indptr, indices, last)
    np.testing.assert_allclose(o_gqa, o_mha, rtol=0, atol=1e-12)


def test_empty_requests_and_untouched_pool_pages():
    rng = np.random.default_rng(9)
    ps, hkv, d = 4, 1, 8
    cache, indptr, indices, last = _random_pool(rng, [5, 6], ps, hkv, d, spare=4)
    qo_indptr = [0, 0, 3]  # request 0 has no queries this step
    q = rng.standard_normal((3, 1, d))
    o1 = opp.paged_prefill(q, cache, qo_indptr, indptr, indices, last)
    used = set(indices.tolist())
    poisoned = cache.copy()
    for p in range(cache.shape[0]):
        if p not in used:
            poisoned[p] = np.nan
    poisoned[indices[indptr[1]:indptr[2]][-1], :, last[1]:] = np.nan  # tail of the last page
    o2 = opp.paged_prefill(q, poisoned, qo_indptr, indptr, indices, last)
    np.testing.assert_array_equal(o1, o2)


def test_top_left_alignment_is_rejected_by_the_decode_check():
    """A plausible mistake (causal mask aligned to the top left, as torch's
    is_causal for qo_len < kv_len) differs from the oracle's rows."""
    rng = np.random.default_rng(13)
    ps, d, L, n = 4, 8, 11, 4
    cache, indptr, indices, last = _random_pool(rng, [L], ps, 1, d)
    q = rng.standard_normal((n, 1, d))
    o = opp.paged_prefill(q, cache, [0, n], indptr, indices, last)
    k, v = opd.gather_row_kv(cache, indptr, indices, last, 0)
    wrong = torch.nn.functional.scaled_dot_product_attention(
        torch.from_numpy(q).transpose(0, 1), torch.from_numpy(k).transpose(0, 1),
        torch.from_numpy(v).transpose(0, 1), is_causal=True,
    ).transpose(0, 1).numpy()
    assert np.abs(o - wrong).max() > 1e-3


def test_prefill_flops_counts_visible_pairs():
    qo_indptr, kv_indptr, last = [0, 3, 5], [0, 2, 3], [2, 4]
    ps, hq, d = 4, 2, 8
    # request 0: kv 6, qo 3 -> sees 4, 5, 6; request 1: kv 4, qo 2 -> sees 3, 4
    pairs = (4 + 5 + 6) + (3 + 4)
    assert opp.prefill_flops(qo_indptr, kv_indptr, last, ps, hq, d) == 4 * pairs * hq * d
    assert opp.prefill_flops(qo_indptr, kv_indptr, last, ps, hq, d, causal=False) == 4 * (18 + 8) * hq * d
