"""Paged decode attention on the GPU vs the float64 oracle.

Tolerances: fp32 inputs 2e-5 max-abs; fp16/bf16 inputs 2e-3 max-abs against
the oracle evaluated on the same rounded inputs (the bar of the path's
parity requirement), plus one unit of the output type's rounding
(2^-11 for fp16, 2^-8 for bf16, relative) since the kernel must store its
fp32 result in that type.
"""

import math
import zlib

import numpy as np
import pytest
import torch

from oracle import paged_decode as opd
from pagelora_amd.attention_backend import PagedDecodeAttention, kv_append
from tests.gpu_cases import ragged_case, uniform_lens

pytestmark = pytest.mark.gpu

TOL = {torch.float32: (2e-5, 0.0), torch.float16: (2e-3, 2.0**-11), torch.bfloat16: (2e-3, 2.0**-8)}


def _run(case, hq, hkv, d, ps, dtype, device, lse=False, **kw):
    be = PagedDecodeAttention(device=device, workspace_mb=kw.pop("workspace_mb", 64), num_qo_heads=hq,
                              num_kv_heads=hkv, head_dim=d, page_size=ps, **kw)
    be.plan_decode(paged_kv_indptr=case["indptr"], paged_kv_indices=case["indices"],
                   paged_kv_last_page_len=case["last"], q_data_type=dtype, kv_data_type=dtype)
    if lse:
        out = torch.empty_like(case["q"])
        lse_t = torch.empty(case["q"].shape[:2], dtype=torch.float32, device=device)
        be.run_decode_into(case["q"], case["cache"], out, lse_t)
        torch.cuda.synchronize()
        return out, lse_t, be
    out = be.run_decode(case["q"], case["cache"])
    torch.cuda.synchronize()
    return out[:, :, 0], None, be


def _oracle(case, rows=None):
    return opd.paged_decode(case["q_host"].float().numpy(), case["cache_host"].float().numpy(),
                            case["indptr"].numpy(), case["indices"].numpy(), case["last"].numpy(), rows=rows)


def _check(out, ref, dtype, rows=None):
    atol, rtol = TOL[dtype]
    got = out.float().cpu().numpy()
    if rows is not None:
        got, ref = got[rows], ref[rows]
    err = np.abs(got - ref)
    bound = atol + rtol * np.abs(ref)
    assert np.isfinite(got).all(), "non-finite output"
    assert (err <= bound).all(), f"max err {err.max():.3e} (bound {bound.max():.3e})"
    return float(err.max())


def test_fp32_batch4_512_gqa4(gpu_device):
    # B=4, 32/8 heads, D=128, page 16, 512 tokens per row, 128 of 256 pages.
    case = ragged_case(lens=[512] * 4, hq=32, hkv=8, head_dim=128, page_size=16, dtype=torch.float32,
                       device=gpu_device, seed=1234, pool_extra=128)
    out, _, _ = _run(case, 32, 8, 128, 16, torch.float32, gpu_device)
    ref, _ = _oracle(case)
    _check(out, ref, torch.float32)


def test_bf16_qwen3_layer_1x2048(gpu_device):
    case = ragged_case(lens=[2048], hq=32, hkv=8, head_dim=128, page_size=16, dtype=torch.bfloat16,
                       device=gpu_device, seed=1235, pool_extra=4096 - 128)
    out, _, _ = _run(case, 32, 8, 128, 16, torch.bfloat16, gpu_device)
    ref, _ = _oracle(case)
    err = _check(out, ref, torch.bfloat16)
    assert err <= 2e-3


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("heads", [(4, 4), (8, 4), (16, 4), (7, 1), (24, 3), (40, 8), (8, 1)])
@pytest.mark.parametrize("head_dim", [64, 128, 256])
def test_random_shapes(gpu_device, dtype, heads, head_dim):
    hq, hkv = heads
    seed = zlib.crc32(f"{dtype}-{hq}-{hkv}-{head_dim}".encode()) % 10000
    lens = [1, 15, 16, 17, 33, 200, 64] + uniform_lens(3, 1, 300, seed)
    case = ragged_case(lens=lens, hq=hq, hkv=hkv, head_dim=head_dim, page_size=16, dtype=dtype,
                       device=gpu_device, seed=seed, pool_extra=7)
    ref, ref_lse = _oracle(case)
    # Few work items -> rows split into many chunks; many -> mostly whole rows.
    for tw in (8, 100000):
        out, lse, _ = _run(case, hq, hkv, head_dim, 16, dtype, gpu_device, lse=True, target_waves=tw,
                           min_chunk_pages=1)
        _check(out, ref, dtype)
        np.testing.assert_allclose(lse.cpu().numpy(), ref_lse, atol=2e-3 if dtype != torch.float32 else 1e-4)


def test_large_batch_plan(gpu_device):
    """2,500 rows: the plan kernel's threads each own several rows (its
    per-thread row loop and the size-class stash), and the rows' short last
    chunks fill many size classes; split and unsplit plans."""
    lens = [0, 1, 16, 17] + uniform_lens(2496, 0, 200, 77)
    case = ragged_case(lens=lens, hq=8, hkv=2, head_dim=64, page_size=16, dtype=torch.float16,
                       device=gpu_device, seed=78, pool_extra=9)
    ref, ref_lse = _oracle(case)
    for tw in (2 * 600, 2 * 20000):
        out, lse, _ = _run(case, 8, 2, 64, 16, torch.float16, gpu_device, lse=True, target_waves=tw,
                           min_chunk_pages=1, workspace_mb=128)
        _check(out, ref, torch.float16)
        np.testing.assert_allclose(lse.cpu().numpy(), ref_lse, atol=2e-3)


def test_plan_coarse_size_classes(gpu_device):
    """Chunks longer than the plan's 1,024 size classes (one or two items for
    the whole batch): the short chunks are ordered by coarse classes."""
    lens = [16 * 2900, 16 * 100 + 5, 16 * 1500, 0, 16 * 2999 + 1, 7]
    case = ragged_case(lens=lens, hq=4, hkv=1, head_dim=64, page_size=16, dtype=torch.float16,
                       device=gpu_device, seed=79, pool_extra=5)
    ref, _ = _oracle(case)
    for tw in (1, 2, 3):
        out, _, _ = _run(case, 4, 1, 64, 16, torch.float16, gpu_device, target_waves=tw, min_chunk_pages=1)
        _check(out, ref, torch.float16)


@pytest.mark.parametrize("page_size", [16, 32, 64])
def test_page_sizes(gpu_device, page_size):
    lens = [1, page_size - 1, page_size, page_size + 1, 5 * page_size + 3, 700]
    case = ragged_case(lens=lens, hq=32, hkv=8, head_dim=128, page_size=page_size, dtype=torch.bfloat16,
                       device=gpu_device, seed=page_size, pool_extra=3)
    out, _, _ = _run(case, 32, 8, 128, page_size, torch.bfloat16, gpu_device, target_waves=64, min_chunk_pages=1)
    ref, _ = _oracle(case)
    _check(out, ref, torch.bfloat16)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("page_size", [1, 2, 3, 4, 5, 8, 12, 24])
@pytest.mark.parametrize("heads,head_dim", [((32, 8), 128), ((8, 8), 64), ((16, 2), 256), ((6, 2), 128)])
def test_small_page_sizes(gpu_device, dtype, page_size, heads, head_dim):
    """Pages that are not a multiple of 16 tokens: a 16-token block spans
    several pages and each lane looks up its own rows' pages (the MFMA-score
    wave at 32/8 heads, D=128, 16-bit; the VALU wave otherwise).  Split and
    unsplit plans; unread slots hold NaN."""
    hq, hkv = heads
    seed = zlib.crc32(f"small-{dtype}-{page_size}-{hq}-{head_dim}".encode()) % 10000
    lens = [1, page_size - 1, page_size, page_size + 1, 5 * page_size + 3, 15, 16, 17, 33, 300]
    lens = [x for x in lens if x > 0] + uniform_lens(3, 1, 400, seed)
    case = ragged_case(lens=lens, hq=hq, hkv=hkv, head_dim=head_dim, page_size=page_size, dtype=dtype,
                       device=gpu_device, seed=seed, pool_extra=5)
    ref, ref_lse = _oracle(case)
    for tw in (8, 100000):
        out, lse, _ = _run(case, hq, hkv, head_dim, page_size, dtype, gpu_device, lse=True, target_waves=tw,
                           min_chunk_pages=1)
        _check(out, ref, dtype)
        np.testing.assert_allclose(lse.cpu().numpy(), ref_lse, atol=2e-3 if dtype != torch.float32 else 1e-4)


def test_small_pages_default_chunking(gpu_device):
    """Default plan on 2-token pages: the minimum chunk is scaled to the
    page size (32 tokens), the rows still match the oracle."""
    case = ragged_case(lens=[2048, 100, 1], hq=32, hkv=8, head_dim=128, page_size=2, dtype=torch.bfloat16,
                       device=gpu_device, seed=31, pool_extra=11)
    out, _, be = _run(case, 32, 8, 128, 2, torch.bfloat16, gpu_device)
    assert be.min_chunk_pages == 16
    ref, _ = _oracle(case)
    _check(out, ref, torch.bfloat16)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("heads", [(16, 1), (32, 2), (12, 1), (11, 1), (40, 4), (64, 4), (48, 2)])
@pytest.mark.parametrize("page_size", [16, 4])
def test_gqa_groups_above_8(gpu_device, dtype, heads, page_size):
    """GQA groups of more than 8 query heads (FlashInfer routes them to its
    tensor-core kernel, attention_backend.py:46-55): each kv head is served by
    several waves of at most 8 query heads (16 -> 2 x 8, 12 -> 2 x 6,
    11 -> 11 x 1, 10 -> 2 x 5, 24 -> 3 x 8)."""
    hq, hkv = heads
    seed = zlib.crc32(f"gqa-{dtype}-{hq}-{hkv}-{page_size}".encode()) % 10000
    lens = [1, 17, 64, 300] + uniform_lens(4, 1, 500, seed)
    case = ragged_case(lens=lens, hq=hq, hkv=hkv, head_dim=128, page_size=page_size, dtype=dtype,
                       device=gpu_device, seed=seed, pool_extra=3)
    ref, ref_lse = _oracle(case)
    for tw in (8, 100000):
        out, lse, _ = _run(case, hq, hkv, 128, page_size, dtype, gpu_device, lse=True, target_waves=tw,
                           min_chunk_pages=1)
        _check(out, ref, dtype)
        np.testing.assert_allclose(lse.cpu().numpy(), ref_lse, atol=2e-3 if dtype != torch.float32 else 1e-4)


def test_reference_page_tables_on_4_token_pages(gpu_device):
    """The second table of test_paged_kvcache_manager.py:503-543 (page size
    4: indptr [0,1,3], indices [2,4,5], last [4,1]) run through decode vs the
    oracle."""
    d, hq, hkv = 64, 4, 2
    gen = torch.Generator().manual_seed(3)
    cache = torch.randn((8, 2, 4, hkv, d), generator=gen).to(torch.float16)
    q = torch.randn((2, hq, d), generator=gen).to(torch.float16)
    indptr = torch.tensor([0, 1, 3], dtype=torch.int32)
    indices = torch.tensor([2, 4, 5], dtype=torch.int32)
    last = torch.tensor([4, 1], dtype=torch.int32)
    be = PagedDecodeAttention(device=gpu_device, workspace_mb=1, num_qo_heads=hq, num_kv_heads=hkv, head_dim=d,
                              page_size=4)
    be.plan_decode(paged_kv_indptr=indptr, paged_kv_indices=indices, paged_kv_last_page_len=last)
    out = be.run_decode(q.to(gpu_device), cache.to(gpu_device))[:, :, 0]
    ref, _ = opd.paged_decode(q.float().numpy(), cache.float().numpy(), indptr.numpy(), indices.numpy(),
                              last.numpy())
    _check(out, ref, torch.float16)


def test_reference_decode_vector_2_token_page(gpu_device):
    """test_flashinfer_backend.py:157-177 on its own 2-token page: q = -1000,
    k = 100 on both tokens, v = [1, 9]; the row that sees one token returns
    1, the row that sees both returns their mean 5."""
    d = 64
    cache = torch.zeros((1, 2, 2, 1, d), dtype=torch.float32)
    cache[0, 0, :, 0, 0] = 100.0
    cache[0, 1, 0, 0, 0] = 1.0
    cache[0, 1, 1, 0, 0] = 9.0
    q = torch.zeros((2, 1, d))
    q[:, 0, 0] = -1000.0
    be = PagedDecodeAttention(device=gpu_device, workspace_mb=1, num_qo_heads=1, num_kv_heads=1, head_dim=d,
                              page_size=2)
    be.plan_decode(paged_kv_indptr=torch.tensor([0, 1, 2], dtype=torch.int32),
                   paged_kv_indices=torch.tensor([0, 0], dtype=torch.int32),
                   paged_kv_last_page_len=torch.tensor([1, 2], dtype=torch.int32))
    out = be.run_decode(q.to(gpu_device), cache.to(gpu_device))
    assert out[:, 0, 0, 0].cpu().tolist() == [1.0, 5.0]


def test_shared_prefix_pages(gpu_device):
    # Rows listing the same physical pages (radix-shared prefix) read them concurrently.
    case = ragged_case(lens=[2048 + 64] * 4, hq=32, hkv=8, head_dim=128, page_size=16, dtype=torch.bfloat16,
                       device=gpu_device, seed=77, shared_prefix_pages=128)
    assert case["indices"][:128].tolist() == case["indices"][132:260].tolist()
    out, _, _ = _run(case, 32, 8, 128, 16, torch.bfloat16, gpu_device)
    ref, _ = _oracle(case)
    _check(out, ref, torch.bfloat16)


def test_split_kv_tuple_layout(gpu_device):
    case = ragged_case(lens=[100, 37], hq=8, hkv=2, head_dim=128, page_size=16, dtype=torch.float16,
                       device=gpu_device, seed=5)
    be = PagedDecodeAttention(device=gpu_device, workspace_mb=8, num_qo_heads=8, num_kv_heads=2, head_dim=128,
                              page_size=16)
    be.plan_decode(paged_kv_indptr=case["indptr"], paged_kv_indices=case["indices"],
                   paged_kv_last_page_len=case["last"])
    k = case["cache"][:, 0].contiguous()
    v = case["cache"][:, 1].contiguous()
    out_tuple = be.run_decode(case["q"], (k, v))
    out_pool = be.run_decode(case["q"], case["cache"])
    torch.cuda.synchronize()
    assert torch.equal(out_tuple, out_pool)


def test_reference_decode_vector(gpu_device):
    # test_flashinfer_backend.py:157-177 restated: q=-1000, k=100 -> equal scores.
    d = 64
    cache = torch.zeros((2, 2, 16, 1, d), dtype=torch.float32)
    cache[:, 0, :, 0, 0] = 100.0
    cache[0, 1, 0, 0, 0] = 1.0
    cache[0, 1, 1, 0, 0] = 9.0
    q = torch.zeros((2, 1, d))
    q[:, 0, 0] = -1000.0
    be = PagedDecodeAttention(device=gpu_device, workspace_mb=1, num_qo_heads=1, num_kv_heads=1, head_dim=d,
                              page_size=16)
    be.plan_decode(paged_kv_indptr=torch.tensor([0, 1, 2], dtype=torch.int32),
                   paged_kv_indices=torch.tensor([0, 0], dtype=torch.int32),
                   paged_kv_last_page_len=torch.tensor([1, 2], dtype=torch.int32))
    out = be.run_decode(q.to(gpu_device), cache.to(gpu_device))
    assert out[:, 0, 0, 0].cpu().tolist() == [1.0, 5.0]


def test_empty_row_gives_zeros(gpu_device):
    case = ragged_case(lens=[0, 40, 0], hq=8, hkv=8, head_dim=128, page_size=16, dtype=torch.float16,
                       device=gpu_device, seed=9, pool_extra=2)
    out, lse, _ = _run(case, 8, 8, 128, 16, torch.float16, gpu_device, lse=True)
    ref, _ = _oracle(case)
    _check(out, ref, torch.float16)
    assert torch.isinf(lse[0]).all() and torch.isinf(lse[2]).all()


def test_ragged_batch64_mha_full_size(gpu_device):
    # Llama-2-7B shape: 32/32 heads, fp16, 64 rows with lengths U[128, 8192].
    torch.manual_seed(0)
    lens = uniform_lens(64, 128, 8192, 1236)
    ps, h, d = 16, 32, 128
    n_pages = [math.ceil(L / ps) for L in lens]
    total = sum(n_pages)
    pool = total + 1024
    gen = torch.Generator(device=gpu_device).manual_seed(1236)
    cache = torch.randn((pool, 2, ps, h, d), device=gpu_device, dtype=torch.float16, generator=gen)
    q = (torch.randn((64, h, d), device=gpu_device, generator=gen) / math.sqrt(d)).to(torch.float16)
    perm = torch.randperm(pool, generator=torch.Generator().manual_seed(1236))[:total].to(torch.int32)
    indptr = torch.tensor(np.concatenate([[0], np.cumsum(n_pages)]), dtype=torch.int32)
    last = torch.tensor([L - ps * (n - 1) for L, n in zip(lens, n_pages)], dtype=torch.int32)
    be = PagedDecodeAttention(device=gpu_device, workspace_mb=128, num_qo_heads=h, num_kv_heads=h, head_dim=d,
                              page_size=ps)
    be.plan_decode(paged_kv_indptr=indptr, paged_kv_indices=perm, paged_kv_last_page_len=last)
    out = be.run_decode(q, cache)[:, :, 0]
    torch.cuda.synchronize()
    # (1) the oracle on every one of the 64 rows, one row's pages at a time
    # (~7 s of float64 CPU work for the 285k tokens)
    q_host = q.float().cpu().numpy()
    atol, rtol = TOL[torch.float16]
    got_all = out.float().cpu().numpy()
    for b in range(64):
        pages = perm[indptr[b]: indptr[b + 1]].long()
        sub = cache[pages.to(gpu_device)].float().cpu().numpy()
        n = n_pages[b]
        o, _ = opd.paged_decode(q_host[b: b + 1], sub, [0, n], np.arange(n), [int(last[b])])
        err = np.abs(got_all[b] - o[0])
        assert (err <= atol + rtol * np.abs(o[0])).all(), f"row {b} ({lens[b]} tokens): max err {err.max():.3e}"
    # (2) physical-page permutation invariance: bit-identical output
    new_pos = torch.randperm(pool, generator=torch.Generator().manual_seed(99))
    cache2 = torch.empty_like(cache)
    cache2[new_pos.to(gpu_device)] = cache
    del cache
    be.plan_decode(paged_kv_indptr=indptr, paged_kv_indices=new_pos[perm.long()].to(torch.int32),
                   paged_kv_last_page_len=last)
    out2 = be.run_decode(q, cache2)[:, :, 0]
    torch.cuda.synchronize()
    assert torch.equal(out, out2)


def test_graph_replay_across_growing_rows(gpu_device):
    """One captured run_decode replays while rows grow; every replay matches eager."""
    hq, hkv, d, ps = 32, 8, 128, 16
    B = 4
    pool = 600
    gen = torch.Generator(device=gpu_device).manual_seed(3)
    cache = torch.randn((pool, 2, ps, hkv, d), device=gpu_device, dtype=torch.bfloat16, generator=gen)
    q = torch.randn((B, hq, d), device=gpu_device, dtype=torch.bfloat16, generator=gen)
    perm = torch.randperm(pool, generator=torch.Generator().manual_seed(4)).to(torch.int32)
    be = PagedDecodeAttention(device=gpu_device, workspace_mb=32, num_qo_heads=hq, num_kv_heads=hkv, head_dim=d,
                              page_size=ps, max_pages=pool)

    def table(lens):
        n = [math.ceil(L / ps) for L in lens]
        indptr = torch.tensor(np.concatenate([[0], np.cumsum(n)]), dtype=torch.int32)
        idx = perm[: sum(n)].clone()
        last = torch.tensor([L - ps * (k - 1) for L, k in zip(lens, n)], dtype=torch.int32)
        return indptr.pin_memory(), idx.pin_memory(), last.pin_memory()

    lens = [100, 530, 16, 2000]
    ip, ix, la = table(lens)
    be.plan_decode(paged_kv_indptr=ip, paged_kv_indices=ix, paged_kv_last_page_len=la)
    out = torch.empty((B, hq, d), device=gpu_device, dtype=torch.bfloat16)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        be.run_decode_into(q, cache, out)
    torch.cuda.current_stream().wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        be.run_decode_into(q, cache, out)
    sig = be.decode_graph_signature()
    for step in range(8):
        lens = [L + 37 * step for L in lens]
        ip, ix, la = table(lens)
        be.plan_decode(paged_kv_indptr=ip, paged_kv_indices=ix, paged_kv_last_page_len=la)
        assert be.decode_graph_signature() == sig  # no recapture needed while rows grow
        graph.replay()
        torch.cuda.synchronize()
        replayed = out.clone()
        eager = be.run_decode(q, cache)[:, :, 0]
        torch.cuda.synchronize()
        assert torch.equal(replayed, eager), f"step {step}"


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_kv_append_matches_oracle(gpu_device, dtype):
    pool, ps, hkv, d, B = 12, 16, 8, 128, 5
    cache = torch.randn((pool, 2, ps, hkv, d), dtype=dtype)
    k = torch.randn((B, hkv, d), dtype=dtype)
    v = torch.randn((B, hkv, d), dtype=dtype)
    pid = torch.tensor([3, 11, 0, 7, 5])
    off = torch.tensor([0, 15, 7, 1, 9])
    want = opd.kv_append(cache.float().numpy().copy(), pid.numpy(), off.numpy(), k.float().numpy(), v.float().numpy())
    dev = cache.to(gpu_device)
    kv_append(dev, k.to(gpu_device), v.to(gpu_device), pid.to(gpu_device), off.to(gpu_device),
              num_kv_heads=hkv, head_dim=d, page_size=ps)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(dev.float().cpu().numpy(), want)


def test_bad_inputs_raise(gpu_device):
    be = PagedDecodeAttention(device=gpu_device, workspace_mb=1, num_qo_heads=8, num_kv_heads=2, head_dim=128,
                              page_size=16)
    with pytest.raises(ValueError):  # last_page_len outside [1, page_size]
        be.plan_decode(paged_kv_indptr=torch.tensor([0, 1], dtype=torch.int32),
                       paged_kv_indices=torch.tensor([0], dtype=torch.int32),
                       paged_kv_last_page_len=torch.tensor([17], dtype=torch.int32))
    be.plan_decode(paged_kv_indptr=torch.tensor([0, 1], dtype=torch.int32),
                   paged_kv_indices=torch.tensor([9], dtype=torch.int32),
                   paged_kv_last_page_len=torch.tensor([3], dtype=torch.int32))
    cache = torch.zeros((4, 2, 16, 2, 128), device=gpu_device, dtype=torch.float16)
    q = torch.zeros((1, 8, 128), device=gpu_device, dtype=torch.float16)
    with pytest.raises(ValueError):  # page 9 outside a 4-page pool
        be.run_decode(q, cache)
    with pytest.raises(ValueError):  # dtype mismatch
        be.run_decode(q.float(), torch.zeros((10, 2, 16, 2, 128), device=gpu_device, dtype=torch.float16))
    with pytest.raises(ValueError):  # batch mismatch
        be.run_decode(torch.zeros((2, 8, 128), device=gpu_device, dtype=torch.float16),
                      torch.zeros((10, 2, 16, 2, 128), device=gpu_device, dtype=torch.float16))
