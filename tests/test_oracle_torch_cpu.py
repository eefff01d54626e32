"""Pin the torch fp32 CPU path (the CPU baseline) to the float64 oracle.

The float64 oracle is itself pinned (test_oracle_decode.py,
test_oracle_lora.py); here the fp32 restatement must agree with it on
ragged, GQA and MHA cases, on a single-token closed form, and a planted
mistake (a transposed GQA head mapping) must fail the same comparison.
"""

import numpy as np
import torch

from oracle import lora as ol
from oracle import paged_decode as opd
from oracle import torch_cpu as tc


def _case(seed, B, hq, hkv, d, ps, max_len, pool_extra=5):
    rng = np.random.default_rng(seed)
    lens = rng.integers(0, max_len + 1, size=B)
    n_pages = (lens + ps - 1) // ps
    pool = int(n_pages.sum()) + pool_extra
    perm = rng.permutation(pool)[: n_pages.sum()]
    indptr = np.concatenate([[0], np.cumsum(n_pages)])
    last = np.where(n_pages > 0, lens - ps * (n_pages - 1), 0)
    cache = rng.standard_normal((pool, 2, ps, hkv, d)).astype(np.float32)
    q = rng.standard_normal((B, hq, d)).astype(np.float32)
    return q, cache, indptr, perm, last


def test_paged_decode_matches_float64_oracle():
    for seed, (B, hq, hkv, d, ps, L) in enumerate([(5, 8, 2, 64, 16, 70), (3, 4, 4, 128, 4, 33),
                                                    (4, 32, 8, 128, 16, 300), (2, 12, 1, 32, 1, 9)]):
        q, cache, indptr, perm, last = _case(seed, B, hq, hkv, d, ps, L)
        want, _ = opd.paged_decode(q, cache, indptr, perm, last)
        got = tc.paged_decode(torch.from_numpy(q), torch.from_numpy(cache), indptr, perm, last)
        assert np.abs(got.numpy() - want).max() <= 2e-5


def test_paged_decode_single_token_is_its_value():
    rng = np.random.default_rng(1)
    cache = torch.from_numpy(rng.standard_normal((4, 2, 16, 2, 8)).astype(np.float32))
    q = torch.from_numpy(rng.standard_normal((1, 4, 8)).astype(np.float32))
    got = tc.paged_decode(q, cache, [0, 1], [3], [1])
    want = cache[3, 1, 0].repeat_interleave(2, dim=0)  # q heads 0,1 -> kv head 0; 2,3 -> 1
    assert torch.allclose(got[0], want, atol=0, rtol=0)


def test_planted_head_mapping_mistake_is_caught():
    # kv head h % Hkv instead of h // g would pass an MHA case; it must fail GQA
    q, cache, indptr, perm, last = _case(7, 2, 8, 2, 16, 4, 20)
    want, _ = opd.paged_decode(q, cache, indptr, perm, last)
    bad_q = q.reshape(2, 2, 4, 16).transpose(0, 2, 1, 3).reshape(2, 8, 16).copy()
    got = tc.paged_decode(torch.from_numpy(bad_q), torch.from_numpy(cache), indptr, perm, last).numpy()
    got = got.reshape(2, 4, 2, 16).transpose(0, 2, 1, 3).reshape(2, 8, 16)
    assert np.abs(got - want).max() > 1e-2


def test_lora_delta_matches_float64_oracle():
    rng = np.random.default_rng(3)
    T, fin, fout, r, n = 24, 96, 40, 8, 3
    ids = rng.integers(-1, n, size=T)
    x = torch.from_numpy(rng.standard_normal((T, fin)).astype(np.float32)).to(torch.bfloat16)
    A = torch.from_numpy(rng.standard_normal((n, r, fin)).astype(np.float32) * 0.1).to(torch.bfloat16)
    B = torch.from_numpy(rng.standard_normal((n, fout, r)).astype(np.float32) * 0.1).to(torch.bfloat16)
    for inter, tag in ((None, None), (torch.bfloat16, "bf16")):
        got = tc.lora_delta(x, ids, A, B, 2.0, intermediate=inter).numpy()
        want = ol.multi_adapter_delta(x.float().numpy(), ids.tolist(), A.float().numpy(), B.float().numpy(), 2.0,
                                      intermediate=tag)
        # bf16 intermediate: a rounding may land on the other side of a tie in fp32 vs float64
        assert np.abs(got - want).max() <= (1e-4 if inter is None else 2e-2)
        assert np.array_equal(got[ids < 0], np.zeros_like(got[ids < 0]))
