"""Seeded paged-decode inputs shared by the GPU tests, smoke() and bench.py."""

from __future__ import annotations

import math

import numpy as np
import torch


def ragged_case(
    *,
    lens,
    hq: int,
    hkv: int,
    head_dim: int,
    page_size: int,
    dtype,
    device,
    seed: int,
    pool_extra: int = 0,
    poison: bool = True,
    q_scale: float = 1.0,
    shared_prefix_pages: int = 0,
):
    """Build a paged KV pool, page table and q for rows of the given lengths.

    Physical pages are a seeded random permutation of the pool.  With
    ``poison`` every slot that no row may read (unused pages, the tail of
    each last page) holds NaN, so a stray read shows up in the output.
    ``shared_prefix_pages`` > 0 makes every row start with the same physical
    pages (a radix-shared prefix).
    """
    lens = [int(x) for x in lens]
    B = len(lens)
    gen = torch.Generator().manual_seed(seed)
    n_pages = [max(0, math.ceil(L / page_size)) for L in lens]
    shared = shared_prefix_pages
    own = [max(0, n - shared) if shared else n for n in n_pages]
    total_unique = shared + sum(own)
    pool = total_unique + pool_extra
    perm = torch.randperm(pool, generator=gen).tolist()
    shared_ids = perm[:shared]
    cursor = shared
    indices, indptr, last = [], [0], []
    for b in range(B):
        row = (shared_ids[: min(shared, n_pages[b])] if shared else []) + perm[cursor: cursor + own[b]]
        cursor += own[b]
        indices += row
        indptr.append(len(indices))
        last.append(lens[b] - page_size * (n_pages[b] - 1) if n_pages[b] else 0)
    fill = float("nan") if poison else 0.0
    cache = torch.full((pool, 2, page_size, hkv, head_dim), fill, dtype=torch.float32)
    used = torch.zeros(pool, page_size, dtype=torch.bool)
    for b in range(B):
        pages = indices[indptr[b]: indptr[b + 1]]
        for i, p in enumerate(pages):
            n = page_size if i < len(pages) - 1 else last[b]
            used[p, :n] = True
    vals = torch.randn((pool, 2, page_size, hkv, head_dim), generator=gen)
    mask = used[:, None, :, None, None].expand_as(cache)
    cache[mask] = vals[mask]
    q = torch.randn((B, hq, head_dim), generator=gen) * q_scale
    cache = cache.to(dtype)
    q = q.to(dtype)
    tables = (
        torch.tensor(indptr, dtype=torch.int32),
        torch.tensor(indices, dtype=torch.int32),
        torch.tensor(last, dtype=torch.int32),
    )
    return {
        "q": q.to(device),
        "cache": cache.to(device),
        "indptr": tables[0],
        "indices": tables[1],
        "last": tables[2],
        "q_host": q,
        "cache_host": cache,
        "lens": lens,
    }


def uniform_lens(B, lo, hi, seed):
    rng = np.random.default_rng(seed)
    return rng.integers(lo, hi + 1, size=B).tolist()
