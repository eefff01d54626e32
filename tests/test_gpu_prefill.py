"""Paged prefill attention on the GPU vs the float64 oracle.

Tolerances as for decode: 2e-3 max-abs against the oracle evaluated on the
same rounded inputs, plus one unit of the output type's rounding (2^-11
relative for fp16, 2^-8 for bf16), since the kernel stores its fp32 result
in that type.  At full prompt sizes the oracle runs on sampled query rows:
query j of a request is one decode row over its visible prefix (the oracle
tests pin that identity).
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import paged_decode as opd
from oracle import paged_prefill as opp
from pagelora_amd.attention_backend import PagedDecodeAttention
from tests.gpu_cases import ragged_case

pytestmark = pytest.mark.gpu

TOL = {torch.float16: (2e-3, 2.0**-11), torch.bfloat16: (2e-3, 2.0**-8)}


def _case(qo_lens, kv_lens, hq, hkv, d, ps, dtype, device, seed, shared_prefix_pages=0):
    case = ragged_case(lens=kv_lens, hq=hq, hkv=hkv, head_dim=d, page_size=ps, dtype=dtype, device=device,
                       seed=seed, pool_extra=3, shared_prefix_pages=shared_prefix_pages)
    gen = torch.Generator().manual_seed(seed + 7)
    qo_indptr = np.concatenate([[0], np.cumsum(qo_lens)]).astype(np.int32)
    q = torch.randn((int(qo_indptr[-1]), hq, d), generator=gen).to(dtype)
    case.update(q_host=q, q=q.to(device), qo_indptr=torch.from_numpy(qo_indptr), qo_lens=list(qo_lens))
    return case


def _backend(case, hq, hkv, d, ps, device, causal=True):
    be = PagedDecodeAttention(device=device, workspace_mb=8, num_qo_heads=hq, num_kv_heads=hkv, head_dim=d,
                              page_size=ps)
    be.plan_prefill(qo_indptr=case["qo_indptr"], paged_kv_indptr=case["indptr"], paged_kv_indices=case["indices"],
                    paged_kv_last_page_len=case["last"], causal=causal)
    return be


def _oracle(case, causal=True):
    return opp.paged_prefill(case["q_host"].float().numpy(), case["cache_host"].float().numpy(),
                             case["qo_indptr"].numpy(), case["indptr"].numpy(), case["indices"].numpy(),
                             case["last"].numpy(), causal=causal)


def _check(got, ref, dtype):
    atol, rtol = TOL[dtype]
    got = got.float().cpu().numpy() if isinstance(got, torch.Tensor) else got
    assert np.isfinite(got).all(), "non-finite output"
    err = np.abs(got - ref)
    bound = atol + rtol * np.abs(ref)
    assert (err <= bound).all(), f"max err {err.max():.3e} (bound at worst {bound.flat[np.argmax(err - bound)]:.3e})"
    return float(err.max())


def _sampled_rows_oracle(case, r, rows):
    """Oracle output of query rows `rows` of request r, each as one decode row."""
    cache = case["cache_host"].float().numpy()
    ip, ind, last = case["indptr"].numpy(), case["indices"].numpy(), case["last"].numpy()
    k, v = opd.gather_row_kv(cache, ip, ind, last, r)
    kv_len, n = k.shape[0], case["qo_lens"][r]
    q0 = int(case["qo_indptr"][r])
    q = case["q_host"].float().numpy()
    d = q.shape[-1]
    hkv = k.shape[1]
    g = q.shape[1] // hkv
    out = np.zeros((len(rows), q.shape[1], d))
    for i, j in enumerate(rows):
        vis = kv_len - n + j + 1
        for h in range(hkv):  # one kv head at a time keeps the oracle's GQA repeat small
            o, _ = opd.decode_row(q[q0 + j, h * g:(h + 1) * g], k[:vis, h:h + 1], v[:vis, h:h + 1],
                                  1.0 / math.sqrt(d))
            out[i, h * g:(h + 1) * g] = o
    return out


def test_reference_prefill_vector(gpu_device):
    """test_flashinfer_backend.py:157-177 at head_dim 64: causal [1, 5]."""
    d, ps = 64, 16
    cache = torch.zeros((2, 2, ps, 1, d), dtype=torch.bfloat16)
    cache[1, 0, :2, 0, 0] = 100.0
    cache[1, 1, 0, 0, :] = 1.0
    cache[1, 1, 1, 0, :] = 9.0
    q = torch.zeros((2, 1, d), dtype=torch.bfloat16)
    q[:, 0, 0] = -1000.0
    be = PagedDecodeAttention(device=gpu_device, workspace_mb=1, num_qo_heads=1, num_kv_heads=1, head_dim=d,
                              page_size=ps)
    i32 = lambda x: torch.tensor(x, dtype=torch.int32)  # noqa: E731
    be.plan_prefill(qo_indptr=i32([0, 2]), paged_kv_indptr=i32([0, 1]), paged_kv_indices=i32([1]),
                    paged_kv_last_page_len=i32([2]))
    out = be.run_prefill(q.to(gpu_device), cache.to(gpu_device))
    torch.cuda.synchronize()
    assert out[:, 0].float().cpu().numpy().tolist() == [[1.0] * d, [5.0] * d]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("heads", [(4, 4), (8, 2), (32, 8)])
@pytest.mark.parametrize("head_dim", [64, 128, 256])
@pytest.mark.parametrize("causal", [True, False])
def test_ragged_requests_vs_oracle(gpu_device, dtype, heads, head_dim, causal):
    hq, hkv = heads
    qo_lens = [37, 0, 5, 1, 70]
    kv_lens = [37, 20, 100, 17, 133]
    case = _case(qo_lens, kv_lens, hq, hkv, head_dim, 16, dtype, gpu_device, seed=hq * 31 + head_dim)
    be = _backend(case, hq, hkv, head_dim, 16, gpu_device, causal)
    out = be.run_prefill(case["q"], case["cache"])
    torch.cuda.synchronize()
    _check(out, _oracle(case, causal), dtype)


@pytest.mark.parametrize("page_size", [1, 5, 16, 64])
def test_page_sizes(gpu_device, page_size):
    case = _case([50, 9], [50, 77], 8, 2, 128, page_size, torch.bfloat16, gpu_device, seed=page_size)
    be = _backend(case, 8, 2, 128, page_size, gpu_device)
    out = be.run_prefill(case["q"], case["cache"])
    torch.cuda.synchronize()
    _check(out, _oracle(case), torch.bfloat16)


def test_shared_prefix_pages(gpu_device):
    """Requests listing the same physical prefix pages (a radix-shared prefix)."""
    case = _case([16, 16, 3], [96 + 16, 96 + 16, 96 + 3], 8, 2, 128, 16, torch.bfloat16, gpu_device, seed=5,
                 shared_prefix_pages=6)
    ip, ind = case["indptr"].tolist(), case["indices"].tolist()
    assert ind[ip[0]:ip[0] + 6] == ind[ip[1]:ip[1] + 6] == ind[ip[2]:ip[2] + 6]
    be = _backend(case, 8, 2, 128, 16, gpu_device)
    out = be.run_prefill(case["q"], case["cache"])
    torch.cuda.synchronize()
    _check(out, _oracle(case), torch.bfloat16)


def test_bhsd_queries_match_packed(gpu_device):
    """run_prefill on [B, H, S, D] (attention_backend.py:178-185) equals the packed call."""
    for bsz in (1, 3):
        S = 24
        case = _case([S] * bsz, [S + 40] * bsz, 8, 2, 128, 16, torch.bfloat16, gpu_device, seed=40 + bsz)
        be = _backend(case, 8, 2, 128, 16, gpu_device)
        packed = be.run_prefill(case["q"], case["cache"])
        q4 = case["q"].reshape(bsz, S, 8, 128).transpose(1, 2).contiguous()
        out4 = be.run_prefill(q4, case["cache"])
        torch.cuda.synchronize()
        assert out4.shape == (bsz, 8, S, 128)
        assert torch.equal(out4.transpose(1, 2).reshape(bsz * S, 8, 128), packed)


def test_chunked_prefill_equals_full_prefill_bitwise(gpu_device):
    """The last m queries prefilled on their own give exactly the full prompt's rows."""
    L, hq, hkv, d, ps = 300, 8, 2, 128, 16
    case = _case([L], [L], hq, hkv, d, ps, torch.bfloat16, gpu_device, seed=9)
    be = _backend(case, hq, hkv, d, ps, gpu_device)
    full = be.run_prefill(case["q"], case["cache"])
    for m in (1, 17, 64, 129):
        be.plan_prefill(qo_indptr=torch.tensor([0, m], dtype=torch.int32), paged_kv_indptr=case["indptr"],
                        paged_kv_indices=case["indices"], paged_kv_last_page_len=case["last"])
        part = be.run_prefill(case["q"][L - m:].contiguous(), case["cache"])
        torch.cuda.synchronize()
        assert torch.equal(part, full[L - m:]), f"m={m}"


def test_last_query_matches_decode_kernel(gpu_device):
    """A request's last query attends to its whole sequence: the decode kernel's result."""
    case = _case([33, 1, 200], [533, 64, 800], 32, 8, 128, 16, torch.bfloat16, gpu_device, seed=12)
    be = _backend(case, 32, 8, 128, 16, gpu_device)
    out = be.run_prefill(case["q"], case["cache"])
    be.plan_decode(paged_kv_indptr=case["indptr"], paged_kv_indices=case["indices"],
                   paged_kv_last_page_len=case["last"])
    last_rows = case["qo_indptr"][1:].long() - 1
    dec = be.run_decode(case["q"][last_rows.to(gpu_device)].contiguous(), case["cache"])[:, :, 0]
    torch.cuda.synchronize()
    assert (out[last_rows.to(gpu_device)].float() - dec.float()).abs().max().item() <= 4e-3


@pytest.mark.parametrize("prompt", [2112, 32768])
def test_qwen3_shape_long_prompt_sampled_rows(gpu_device, prompt):
    """Qwen3-8B attention shape (32/8 heads, D 128, bf16) over a whole prompt;
    rows checked against the oracle at tile and item boundaries."""
    hq, hkv, d, ps = 32, 8, 128, 16
    case = _case([prompt], [prompt], hq, hkv, d, ps, torch.bfloat16, gpu_device, seed=prompt)
    be = _backend(case, hq, hkv, d, ps, gpu_device)
    out = be.run_prefill(case["q"], case["cache"])
    torch.cuda.synchronize()
    rows = sorted({0, 1, 15, 16, 31, 32, 33, 63, 64, 1000, prompt // 2, prompt - 2, prompt - 1})
    ref = _sampled_rows_oracle(case, 0, rows)
    _check(out[rows].float().cpu().numpy(), ref, torch.bfloat16)


def test_bad_inputs_raise(gpu_device):
    case = _case([8], [8], 4, 4, 64, 16, torch.bfloat16, gpu_device, seed=1)
    be = PagedDecodeAttention(device=gpu_device, workspace_mb=1, num_qo_heads=4, num_kv_heads=4, head_dim=64,
                              page_size=16)
    with pytest.raises(RuntimeError, match="plan_prefill"):
        be.run_prefill(case["q"], case["cache"])
    with pytest.raises(ValueError, match="exceeds kv_len"):
        be.plan_prefill(qo_indptr=torch.tensor([0, 9], dtype=torch.int32), paged_kv_indptr=case["indptr"],
                        paged_kv_indices=case["indices"], paged_kv_last_page_len=case["last"])
    be.plan_prefill(qo_indptr=case["qo_indptr"], paged_kv_indptr=case["indptr"], paged_kv_indices=case["indices"],
                    paged_kv_last_page_len=case["last"])
    with pytest.raises(ValueError, match="tokens"):
        be.run_prefill(case["q"][:7], case["cache"])
    with pytest.raises(ValueError, match="dtype"):
        be.run_prefill(case["q"].half(), case["cache"])
