"""Decode attention with the q/k/v epilogue folded in (pl_decode_run_qkv)
against the two-call path (pl_qk_norm_rope_append(_lora) + pl_decode_run)
on the same inputs, and against the float64 oracle.

What the folded kernel must reproduce:
  - the v appended into each row's new slot: bit-identical (same arithmetic);
  - the appended k: within one bf16/fp16 rounding of the value plus one of
    the row's largest element (its head norm sums the squares in another
    order, and the rotation can cancel);
  - the attention output: 2e-3 + one output rounding from the oracle fed with
    the two-call path's q and cache (the path's parity bar).
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

from oracle import paged_decode as opd
from pagelora_amd import fused_ops
from pagelora_amd.attention_backend import PagedDecodeAttention
from tests.gpu_cases import ragged_case

pytestmark = pytest.mark.gpu

HQ, HKV, D, PS = 32, 8, 128, 16
THETA = 1e6


def _case(device, dtype, lens, seed, rank, n_adapters, bound, shared=0, ps=PS):
    case = ragged_case(lens=lens, hq=HQ, hkv=HKV, head_dim=D, page_size=ps, dtype=dtype, device=device, seed=seed,
                       pool_extra=4, poison=False, shared_prefix_pages=shared)
    case["ps"] = ps
    B = len(lens)
    gen = torch.Generator().manual_seed(seed + 1)
    cols = (HQ + 2 * HKV) * D
    ycols = 3 * n_adapters * rank
    qkv = (torch.randn((B, cols + ycols), generator=gen) * 2).to(dtype).to(device)
    qn = (1 + 0.1 * torch.randn(D, generator=gen)).to(dtype).to(device)
    kn = (1 + 0.1 * torch.randn(D, generator=gen)).to(dtype).to(device)
    indptr, indices, last = case["indptr"].tolist(), case["indices"].tolist(), case["last"].tolist()
    # the new token is each row's last one (the plan counts it)
    page_id = torch.tensor([indices[indptr[b + 1] - 1] for b in range(B)], dtype=torch.int64, device=device)
    offset = torch.tensor([last[b] - 1 for b in range(B)], dtype=torch.int64, device=device)
    positions = torch.tensor([L - 1 for L in lens], dtype=torch.int64, device=device)
    lora, ids = None, None
    if rank:
        outs = (HQ * D, HKV * D, HKV * D)
        Bs = [(torch.randn((n_adapters, o, rank), generator=gen) * 0.05).to(dtype).to(device) for o in outs]
        lora = tuple(fused_ops.LoraUp(qkv, cols + m * n_adapters * rank, Bs[m], 2.0, adapter=bound)
                     for m in range(3))
        ids = torch.tensor([(b % (n_adapters + 1)) - 1 for b in range(B)], dtype=torch.int32, device=device)
    return case, qkv, qn, kn, page_id, offset, positions, lora, ids


def _backend(case, device, tw, share=False):
    be = PagedDecodeAttention(device=device, workspace_mb=64, num_qo_heads=HQ, num_kv_heads=HKV, head_dim=D,
                              page_size=case["ps"], target_waves=tw, min_chunk_pages=1)
    be.share_prefix = share
    be.plan_decode(paged_kv_indptr=case["indptr"], paged_kv_indices=case["indices"],
                   paged_kv_last_page_len=case["last"])
    return be


def _two_call(case, be, qkv, qn, kn, page_id, offset, positions, lora, ids, cache):
    cols = (HQ + 2 * HKV) * D
    q = fused_ops.qk_norm_rope_append(qkv[:, :cols], qn, kn, positions, page_id, offset, cache, num_qo_heads=HQ,
                                      num_kv_heads=HKV, head_dim=D, page_size=case["ps"], rope_theta=THETA, eps=1e-6,
                                      lora=lora, adapter_ids=ids)
    out = torch.empty_like(q)
    be.run_decode_into(q, cache, out)
    return q, out


def _folded(case, be, qkv, qn, kn, page_id, offset, positions, lora, ids, cache):
    cols = (HQ + 2 * HKV) * D
    rope = fused_ops.rope_cos_sin(positions, head_dim=D, rope_theta=THETA)
    out = torch.empty((qkv.shape[0], HQ, D), dtype=qkv.dtype, device=qkv.device)
    be.run_decode_qkv_into(qkv[:, :cols], cache, out, q_norm_weight=qn, k_norm_weight=kn, rope_cos_sin=rope,
                           page_id=page_id, page_offset=offset, eps=1e-6, lora=lora, adapter_ids=ids)
    return out


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("lora_mode", ["none", "ids", "bound"])
@pytest.mark.parametrize("tw", [8, 100000])
def test_folded_matches_two_call_path(gpu_device, dtype, lora_mode, tw):
    lens = [1, 16, 17, 33, 300, 1024, 2049]
    rank, n_ad, bound = {"none": (0, 1, -1), "ids": (16, 2, -1), "bound": (16, 2, 1)}[lora_mode]
    case, qkv, qn, kn, page_id, offset, positions, lora, ids = _case(gpu_device, dtype, lens, 7 + tw % 5, rank,
                                                                      n_ad, bound)
    be = _backend(case, gpu_device, tw)
    cache_a, cache_b = case["cache"].clone(), case["cache"].clone()
    q_ref, out_ref = _two_call(case, be, qkv, qn, kn, page_id, offset, positions, lora, ids, cache_a)
    out = _folded(case, be, qkv, qn, kn, page_id, offset, positions, lora, ids, cache_b)
    torch.cuda.synchronize()
    rel = 2.0**-8 if dtype == torch.bfloat16 else 2.0**-11
    pid, off = page_id.cpu(), offset.cpu()
    for b in range(len(lens)):
        ka, kb = cache_a[pid[b], 0, off[b]].float(), cache_b[pid[b], 0, off[b]].float()
        va, vb = cache_a[pid[b], 1, off[b]], cache_b[pid[b], 1, off[b]]
        assert torch.equal(va, vb), f"row {b}: appended v differs"
        # one unit of the value (up to 2*rel relative) plus one of the row's
        # largest element: the rotation's a*cos - c*sin can cancel
        tol = 2 * rel * ka.abs() + rel * ka.abs().max()
        assert ((ka - kb).abs() <= tol).all(), f"row {b}: appended k beyond one rounding"
    # every other slot untouched and equal
    cb = cache_b.clone()
    cb[pid.to(cb.device), :, off.to(cb.device)] = cache_a[pid.to(cb.device), :, off.to(cb.device)]
    assert torch.equal(cache_a, cb)
    # the output against the oracle fed with the two-call path's q and cache
    ref, _ = opd.paged_decode(q_ref.float().cpu().numpy(), cache_a.float().cpu().numpy(), case["indptr"].numpy(),
                              case["indices"].numpy(), case["last"].numpy())
    got = out.float().cpu().numpy()
    assert np.isfinite(got).all()
    err = np.abs(got - ref)
    assert (err <= 2e-3 + rel * np.abs(ref)).all(), f"max err {err.max():.3e}"
    # and against the two-call output: the same up to q's rounding
    assert np.abs(got - out_ref.float().cpu().numpy()).max() <= 2e-3 + 4 * rel


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("lora_mode", ["none", "bound", "ids"])
@pytest.mark.parametrize("lens,ps", [([2112, 2112, 2112, 2112], 16), ([700, 900, 1210], 16), ([100, 130], 16),
                                     ([2112, 2150, 2200, 2300], 32), ([100, 130], 32), ([97, 96], 32)])
def test_shared_prefix_matches_unshared(gpu_device, dtype, lora_mode, lens, ps):
    """Rows that begin with the same pages: the folded run attending the
    prefix once for all rows (pl_decode_plan_shared: prefix items of 32
    tokens, two 16-token pages or one 32-token page, scoring every row's
    heads as MFMA columns, P.V on MFMA) against the same run reading the
    prefix per row, and both against the oracle fed with the two-call
    path's q and cache (2e-3 + one output rounding).  The appended k/v are
    the own items' and stay bit-identical.  Per-token adapters fall back to
    the unshared run.  [97, 96] on 32-token pages: the shorter row holds
    exactly one page past the prefix."""
    rank, n_ad, bound = {"none": (0, 1, -1), "ids": (16, 2, -1), "bound": (16, 2, 1)}[lora_mode]
    shared = (min(lens) + ps - 1) // ps - 1
    pchunk = 32 // ps
    case, qkv, qn, kn, page_id, offset, positions, lora, ids = _case(gpu_device, dtype, lens, 11 + len(lens), rank,
                                                                      n_ad, bound, shared=shared, ps=ps)
    be_s = _backend(case, gpu_device, None, share=True)
    be_p = _backend(case, gpu_device, None, share=False)
    assert be_s._plan["shared"] == shared // pchunk * pchunk and be_p._plan["shared"] == 0
    cache_r, cache_s, cache_p = case["cache"].clone(), case["cache"].clone(), case["cache"].clone()
    q_ref, _ = _two_call(case, be_p, qkv, qn, kn, page_id, offset, positions, lora, ids, cache_r)
    out_s = _folded(case, be_s, qkv, qn, kn, page_id, offset, positions, lora, ids, cache_s)
    out_p = _folded(case, be_p, qkv, qn, kn, page_id, offset, positions, lora, ids, cache_p)
    torch.cuda.synchronize()
    assert torch.equal(cache_s, cache_p)
    rel = 2.0**-8 if dtype == torch.bfloat16 else 2.0**-11
    ref, _ = opd.paged_decode(q_ref.float().cpu().numpy(), cache_r.float().cpu().numpy(), case["indptr"].numpy(),
                              case["indices"].numpy(), case["last"].numpy())
    for name, out in (("shared", out_s), ("per-row", out_p)):
        got = out.float().cpu().numpy()
        assert np.isfinite(got).all(), name
        err = np.abs(got - ref)
        assert (err <= 2e-3 + rel * np.abs(ref)).all(), f"{name}: max err {err.max():.3e}"
    assert np.abs(out_s.float().cpu().numpy() - out_p.float().cpu().numpy()).max() <= 2e-3 + 4 * rel


def test_out_of_pool_slot_is_skipped(gpu_device):
    dtype = torch.bfloat16
    lens = [40, 70]
    case, qkv, qn, kn, page_id, offset, positions, lora, ids = _case(gpu_device, dtype, lens, 3, 16, 1, 0)
    be = _backend(case, gpu_device, 100000)
    bad = page_id.clone()
    bad[0] = -1  # row 0's slot is outside the pool: nothing is written for it
    cache = case["cache"].clone()
    _folded(case, be, qkv, qn, kn, bad, offset, positions, lora, ids, cache)
    torch.cuda.synchronize()
    assert torch.equal(cache[page_id[0].item(), :, offset[0].item()], case["cache"][page_id[0].item(), :, offset[0].item()])
    assert not torch.equal(cache[page_id[1].item(), :, offset[1].item()], case["cache"][page_id[1].item(), :, offset[1].item()])


def test_rope_table_matches_angles(gpu_device):
    pos = torch.tensor([0, 1, 2047, 32767, 131071], dtype=torch.int64, device=gpu_device)
    t = fused_ops.rope_cos_sin(pos, head_dim=D, rope_theta=THETA).cpu().double().numpy()
    inv = fused_ops.rope_inv_freq(D, THETA, 1.0, "cpu").numpy()
    ang = (pos.cpu().numpy().astype(np.float32)[:, None] * inv[None, :]).astype(np.float32).astype(np.float64)
    assert np.abs(t[..., 0] - np.cos(ang)).max() < 2e-6
    assert np.abs(t[..., 1] - np.sin(ang)).max() < 2e-6


def test_unsupported_shapes_raise(gpu_device):
    case = ragged_case(lens=[20], hq=8, hkv=8, head_dim=128, page_size=16, dtype=torch.bfloat16, device=gpu_device,
                       seed=1)
    be = PagedDecodeAttention(device=gpu_device, workspace_mb=8, num_qo_heads=8, num_kv_heads=8, head_dim=128,
                              page_size=16)
    be.plan_decode(paged_kv_indptr=case["indptr"], paged_kv_indices=case["indices"],
                   paged_kv_last_page_len=case["last"])
    qkv = torch.zeros((1, 24 * 128), dtype=torch.bfloat16, device=gpu_device)
    z = torch.zeros(1, dtype=torch.int64, device=gpu_device)
    rope = fused_ops.rope_cos_sin(z, head_dim=128, rope_theta=THETA)
    with pytest.raises(NotImplementedError):
        be.run_decode_qkv_into(qkv, case["cache"], torch.empty((1, 8, 128), dtype=torch.bfloat16, device=gpu_device),
                               q_norm_weight=None, k_norm_weight=None, rope_cos_sin=rope, page_id=z, page_offset=z,
                               eps=1e-6)
