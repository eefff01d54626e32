"""The decode layer's post-attention fusion, kernel by kernel, through the C ABI:

  - pl_linear_shuffled_norm (RMSNorm in the GEMM's prologue): the normalized
    rows it reports against the float64 RMSNorm (one rounding), and its
    output bit for bit against pl_linear_shuffled on those rows (the same
    MFMA sequence and reduction order);
  - pl_linear_shuffled_add (projection + LoRA delta from partial sums + the
    residual add): its base output bit for bit against pl_linear_shuffled,
    and the residual against the float64 oracle of the reference's
    ``hidden + round(x W^T + s (x A^T) B^T)`` on the same y, with the bar of
    three roundings (base output, module output, sum) plus y's own rounding
    carried through B;
  - pl_decode_run_qkv_oshrink (o_proj's LoRA shrink in the merge): the
    attention output and the appended K/V bit for bit against
    pl_decode_run_qkv (single-item rows go through the merge with one
    partial, which reproduces the direct write exactly), and the partial
    sums against the float64 product of the stored output with A.
"""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from oracle import fused as of
from oracle import lora as ol
from pagelora_amd import _lib, fused_ops
from pagelora_amd.attention_backend import _cache_geometry
from pagelora_amd.linear import (LoraPartials, ShuffledWeight, linear_shuffled, linear_shuffled_add,
                                 linear_shuffled_norm, lora_a_rows)
from tests.test_gpu_decode_qkv import HKV, HQ, D, THETA, _backend, _case

pytestmark = pytest.mark.gpu

REL = {torch.bfloat16: 2.0**-8, torch.float16: 2.0**-11}


def _np(t):
    return t.double().cpu().numpy()


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("tokens", [1, 2, 3, 4, 5, 8])
@pytest.mark.parametrize("shape", [(6192, 4096), (24608, 4096), (48, 512), (1000, 1024)])
def test_norm_gemm(gpu_device, dtype, tokens, shape):
    n, k = shape
    if tokens * k > 32768:
        pytest.skip("beyond the prologue's 32768 elements per token tile")
    g = torch.Generator().manual_seed(n + k + tokens)
    x = (torch.randn((tokens, k), generator=g) * 3).to(dtype)
    w = (1 + 0.1 * torch.randn(k, generator=g)).to(dtype)
    W = (torch.randn((n, k), generator=g) * k ** -0.5).to(dtype)
    sw = ShuffledWeight(W.to(gpu_device))
    xd = x.to(gpu_device)
    xn = torch.empty_like(xd)
    out = linear_shuffled_norm(xd, w.to(gpu_device), 1e-6, sw, x_norm_out=xn)
    ref = linear_shuffled(xn, sw)
    torch.cuda.synchronize()
    want = of.rmsnorm(_np(x), _np(w), 1e-6)
    err = np.abs(_np(xn) - want)
    assert (err <= REL[dtype] * np.abs(want) + 1e-6).all(), f"norm: max err {err.max():.3e}"
    assert torch.equal(out, ref), "the GEMM on the LDS rows differs from the GEMM on the reported rows"


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("tokens", [1, 4, 9, 16])
@pytest.mark.parametrize("shape,parts", [((24608, 4096), 256), ((6192, 4096), 256), ((48, 1024), 37),
                                         ((1000, 2048), 600)])
def test_norm_gemm_from_squares(gpu_device, dtype, tokens, shape, parts):
    """The sums of squares given in pieces (as pl_linear_shuffled_add writes
    them): the normalized rows against the float64 RMSNorm, the output bit
    for bit against pl_linear_shuffled on those rows."""
    n, k = shape
    g = torch.Generator().manual_seed(n + k + tokens + parts)
    x = (torch.randn((tokens, k), generator=g) * 3).to(dtype)
    w = (1 + 0.1 * torch.randn(k, generator=g)).to(dtype)
    W = (torch.randn((n, k), generator=g) * k ** -0.5).to(dtype)
    xf = x.double().numpy()
    sq = np.zeros((tokens, (parts + 3) // 4 * 4), dtype=np.float32)
    edges = np.linspace(0, k, parts + 1).astype(int)
    for j in range(parts):
        sq[:, j] = (xf[:, edges[j]:edges[j + 1]] ** 2).sum(axis=1)
    sw = ShuffledWeight(W.to(gpu_device))
    xd = x.to(gpu_device)
    xn = torch.empty_like(xd)
    sqd = torch.from_numpy(sq).to(gpu_device)[:, :parts] if parts % 4 == 0 else torch.from_numpy(sq).to(gpu_device)
    if parts % 4:
        # the pieces are read 4 at a time: the row pitch is a multiple of 4, the count `parts`
        out = torch.empty((tokens, n), dtype=dtype, device=gpu_device)
        lib = _lib.load()
        _lib.check(lib.pl_linear_shuffled_norm(xd.data_ptr(), xd.stride(0), tokens, k, w.to(gpu_device).data_ptr(),
                                               1e-6, sqd.data_ptr(), sqd.stride(0), parts, sw.data.data_ptr(), n,
                                               out.data_ptr(), out.stride(0), xn.data_ptr(), xn.stride(0),
                                               _lib.dtype_code(dtype), _lib.stream_handle(xd.device)),
                   "pl_linear_shuffled_norm")
    else:
        out = linear_shuffled_norm(xd, w.to(gpu_device), 1e-6, sw, x_norm_out=xn, sq=sqd)
    ref = linear_shuffled(xn, sw)
    torch.cuda.synchronize()
    want = of.rmsnorm(xf, _np(w), 1e-6)
    err = np.abs(_np(xn) - want)
    assert (err <= REL[dtype] * np.abs(want) + 1e-6).all(), f"norm: max err {err.max():.3e}"
    assert torch.equal(out, ref), "the GEMM on the normalized operands differs from the GEMM on the reported rows"


def test_norm_gemm_strided_rows(gpu_device):
    """x as a column slice of a wider buffer; no x_norm_out."""
    g = torch.Generator().manual_seed(5)
    big = (torch.randn((4, 4096 + 64), generator=g)).to(torch.bfloat16).to(gpu_device)
    w = (1 + 0.1 * torch.randn(4096, generator=g)).to(torch.bfloat16).to(gpu_device)
    W = (torch.randn((512, 4096), generator=g) * 0.02).to(torch.bfloat16)
    sw = ShuffledWeight(W.to(gpu_device))
    a = linear_shuffled_norm(big[:, :4096], w, 1e-6, sw)
    b = linear_shuffled_norm(big[:, :4096].contiguous(), w, 1e-6, sw)
    torch.cuda.synchronize()
    assert torch.equal(a, b)


def _add_case(gpu_device, dtype, tokens, rank, parts, n_ad, bound, layout, n=4096, k=4096, seed=0):
    g = torch.Generator().manual_seed(seed + tokens * 7 + parts + rank)
    x = (torch.randn((tokens, k), generator=g)).to(dtype)
    W = (torch.randn((n + 48, k), generator=g) * k ** -0.5).to(dtype)  # 48 more rows: stacked A rows, not read
    B = (torch.randn((n_ad, n, rank), generator=g) * 0.05).to(dtype)
    yp = (torch.randn((tokens, parts, rank), generator=g) * 0.3).float()
    hid = (torch.randn((tokens, n), generator=g)).to(dtype)
    ids = torch.tensor([(t % (n_ad + 1)) - 1 for t in range(tokens)], dtype=torch.int32)  # -1: no adapter
    sw = ShuffledWeight(W.to(gpu_device))
    Bd = B.to(gpu_device)
    if layout == "chunk8":
        Bd = fused_ops.lora_b_chunk8(Bd)
    lora = fused_ops.LoraUp(None, 0, Bd, 2.0, bound)
    return x, W, B, yp, hid, ids, sw, lora


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("tokens,parts", [(1, 128), (4, 64), (4, 6), (3, 40), (16, 32), (1, 1)])
@pytest.mark.parametrize("rank", [8, 16])
@pytest.mark.parametrize("mode", ["ids", "bound", "chunk8"])
def test_add_gemm(gpu_device, dtype, tokens, parts, rank, mode):
    _check_add_gemm(gpu_device, dtype, tokens, parts, rank, mode)


# K = 12288 (down_proj: six weight batches per wave, two in flight), a K that
# splits into no whole batches per wave, and a grid of more than one
# workgroup per CU (both take the one-batch loop)
@pytest.mark.parametrize("n,k", [(4096, 12288), (4096, 4608), (5120, 4096), (64, 12288)])
def test_add_gemm_shapes(gpu_device, n, k):
    _check_add_gemm(gpu_device, torch.bfloat16, 4, 24, 16, "bound", n=n, k=k)


def _check_add_gemm(gpu_device, dtype, tokens, parts, rank, mode, n=4096, k=4096):
    n_ad = 2
    bound = 1 if mode == "bound" else -1
    x, W, B, yp, hid, ids, sw, lora = _add_case(gpu_device, dtype, tokens, rank, parts, n_ad, bound,
                                                "chunk8" if mode == "chunk8" else "rows", n=n, k=k)
    res = hid.to(gpu_device)
    base = torch.empty_like(res)
    ids_d = ids.to(gpu_device)
    nblk = (n + 15) // 16
    sq = torch.full((tokens, nblk + 4), float("nan"), device=gpu_device)
    linear_shuffled_add(x.to(gpu_device), sw, n, res, lora, LoraPartials(yp.to(gpu_device)),
                        ids_d if bound < 0 else None, out=base, sq_out=sq)
    ref = linear_shuffled(x.to(gpu_device), sw)[:, :n]
    torch.cuda.synchronize()
    assert torch.equal(base, ref), "base output differs from pl_linear_shuffled"
    # the squares of the stored residual per 16 columns (fp32 sums of 16 terms)
    r64 = _np(res).reshape(tokens, nblk, 16)
    sq_want = (r64 ** 2).sum(axis=2)
    sq_got = sq[:, :nblk].double().cpu().numpy()
    assert (np.abs(sq_got - sq_want) <= 1e-5 * sq_want + 1e-30).all(), "sums of squares"
    assert torch.isnan(sq[:, nblk:]).all(), "sq_out written past its blocks"
    rel = REL[dtype]
    y = yp.double().sum(dim=1).numpy()
    ok_id = np.array([bound] * tokens) if bound >= 0 else ids.numpy()
    want = np.empty((tokens, n))
    carry = np.empty((tokens, n))
    b_base = _np(base)
    for t in range(tokens):
        a = ok_id[t]
        if 0 <= a < n_ad:
            yr = ol.round_to(y[t], "bf16" if dtype == torch.bfloat16 else "f16")
            d = ol.up_projection(yr[None], _np(B[a]), 2.0)[0]
            carry[t] = np.abs(b_base[t] + d) + rel * 2.0 * (np.abs(yr) @ np.abs(_np(B[a])).T)
        else:
            d = 0.0
            carry[t] = np.abs(b_base[t])
        mod = ol.round_to(b_base[t] + d, "bf16" if dtype == torch.bfloat16 else "f16")
        want[t] = _np(hid)[t] + mod
    got = _np(res)
    err = np.abs(got - want)
    bound_ = 2e-3 + rel * (np.abs(want) + carry)
    assert (err <= bound_).all(), f"residual: worst err/bound {(err / bound_).max():.2f}"


def test_add_gemm_without_lora(gpu_device):
    g = torch.Generator().manual_seed(11)
    x = torch.randn((4, 4096), generator=g).to(torch.bfloat16).to(gpu_device)
    W = (torch.randn((4096, 4096), generator=g) * 0.015).to(torch.bfloat16)
    hid = torch.randn((4, 4096), generator=g).to(torch.bfloat16).to(gpu_device)
    sw = ShuffledWeight(W.to(gpu_device))
    res = hid.clone()
    linear_shuffled_add(x, sw, 4096, res)
    ref = linear_shuffled(x, sw)
    torch.cuda.synchronize()
    want = (hid.float() + ref.float()).to(torch.bfloat16)  # one rounding of the exact bf16 sum
    assert torch.equal(res, want)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("lora_mode", ["ids", "bound"])
@pytest.mark.parametrize("rank", [8, 16])
@pytest.mark.parametrize("lens", [[2049], [1, 16, 17, 300], [1, 16, 17, 33, 300, 1024, 2049, 5, 40]])
def test_oshrink_matches_plain_run(gpu_device, dtype, lora_mode, rank, lens):
    n_ad, bound = (2, -1) if lora_mode == "ids" else (2, 1)
    case, qkv, qn, kn, page_id, offset, positions, lora, ids = _case(gpu_device, dtype, lens, 3 + rank, rank, n_ad,
                                                                      bound)
    be = _backend(case, gpu_device, 100000)
    B = len(lens)
    K = HQ * D
    g = torch.Generator().manual_seed(21 + rank)
    Wo = (torch.randn((K + n_ad * rank + 5, K), generator=g) * 0.02).to(dtype)  # [W_o; A_o; 5 spare rows]
    sw = ShuffledWeight(Wo.to(gpu_device))
    rope = fused_ops.rope_cos_sin(positions, head_dim=D, rope_theta=THETA)
    cols = (HQ + 2 * HKV) * D
    caches = [case["cache"].clone(), case["cache"].clone()]
    outs = [torch.empty((B, HQ, D), dtype=dtype, device=gpu_device) for _ in range(2)]
    parts = LoraPartials(torch.full((B, be.oshrink_parts(B), rank), float("nan"), device=gpu_device))
    for i, o_shrink in enumerate((None, (lora_a_rows(sw, K, rank, bound), parts, n_ad))):
        be.run_decode_qkv_into(qkv[:, :cols], caches[i], outs[i], q_norm_weight=qn, k_norm_weight=kn,
                               rope_cos_sin=rope, page_id=page_id, page_offset=offset, eps=1e-6, lora=lora,
                               adapter_ids=ids, o_shrink=o_shrink)
    torch.cuda.synchronize()
    assert torch.equal(outs[0], outs[1]), "attention output differs with the o shrink"
    assert torch.equal(caches[0], caches[1]), "appended K/V differ with the o shrink"
    attn = _np(outs[1]).reshape(B, K)
    A = _np(Wo[K:K + n_ad * rank]).reshape(n_ad, rank, K)
    ids_h = ids.cpu().numpy() if bound < 0 else np.full(B, bound)
    got = parts.sum().cpu().numpy()
    for b in range(B):
        a = ids_h[b] if 0 <= ids_h[b] < n_ad else 0
        want = A[a] @ attn[b]
        bar = 1e-6 + 2e-5 * (np.abs(A[a]) @ np.abs(attn[b]))
        assert (np.abs(got[b] - want) <= bar).all(), f"row {b}: shrink partials off by {np.abs(got[b] - want).max():.3e}"


def test_oshrink_rejects_a_skipped_merge(gpu_device):
    """The shrink lives in the merge: flags that skip it are refused."""
    case, qkv, qn, kn, page_id, offset, positions, lora, ids = _case(gpu_device, torch.bfloat16, [300, 40], 4, 16,
                                                                      2, 1)
    be = _backend(case, gpu_device, 100000)
    K = HQ * D
    sw = ShuffledWeight(torch.zeros((K + 32, K), dtype=torch.bfloat16, device=gpu_device))
    parts = LoraPartials(torch.empty((2, be.oshrink_parts(2), 16), device=gpu_device))
    rows = lora_a_rows(sw, K, 16, 1)
    lib = _lib.load()
    arr, ids_p, n = fused_ops._lora_args(lora, ids, 2)
    k, v, ps_, ts, hs, npg = _cache_geometry(case["cache"], HKV, D, case["ps"])
    rope = fused_ops.rope_cos_sin(positions, head_dim=D, rope_theta=THETA)
    out = torch.empty((2, HQ, D), dtype=torch.bfloat16, device=gpu_device)
    _, ind, last = be._decode_graph_buffers
    p = parts.struct()
    st = lib.pl_decode_run_qkv_oshrink(
        qkv.data_ptr(), qkv.stride(0), arr, ids_p, n, qn.data_ptr(), kn.data_ptr(), rope.data_ptr(),
        page_id.data_ptr(), offset.data_ptr(), 1e-6, k.data_ptr(), v.data_ptr(), ps_, ts, hs, npg, ind.data_ptr(),
        last.data_ptr(), out.data_ptr(), out.stride(0), out.stride(1), None, 2, HQ, HKV, D, case["ps"], be.sm_scale,
        _lib.PL_DTYPE_BF16, be._plan["target_items"], _lib.PL_DECODE_SKIP_MERGE, be.workspace_buffer.data_ptr(),
        be.workspace_buffer.numel(), ctypes.byref(rows), ctypes.byref(p), None)
    assert st == _lib.PL_ERR_INVALID


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("rows", [1, 4, 9])
@pytest.mark.parametrize("rank,down_rank", [(16, 16), (8, 16), (16, 8)])
@pytest.mark.parametrize("inter,bound", [(12288, 1), (12288, -1), (1056, -1)])
def test_silu_shrink_matches_plain_silu(gpu_device, dtype, rows, rank, down_rank, inter, bound):
    """SiLU*up with down_proj's LoRA shrink (pl_silu_mul_lora_shrink): its
    output bit for bit against pl_silu_mul_lora, and the partial sums (one
    per 256 columns) against the float64 product of that output with the
    row's adapter's A rows."""
    n_ad = 2
    g = torch.Generator().manual_seed(rows * 13 + rank + down_rank + inter)
    gu = (torch.randn((rows, 2 * inter + 2 * n_ad * rank), generator=g)).to(dtype).to(gpu_device)
    Bg = (torch.randn((n_ad, inter, rank), generator=g) * 0.05).to(dtype).to(gpu_device)
    Bu = (torch.randn((n_ad, inter, rank), generator=g) * 0.05).to(dtype).to(gpu_device)
    lora = (fused_ops.LoraUp(gu, 2 * inter, Bg, 2.0, bound), fused_ops.LoraUp(gu, 2 * inter + n_ad * rank, Bu, 2.0, bound))
    ids = torch.tensor([(b % (n_ad + 1)) - 1 for b in range(rows)], dtype=torch.int32, device=gpu_device)
    hidden = 256
    Wd = (torch.randn((hidden + n_ad * down_rank, inter), generator=g) * 0.02).to(dtype)
    sw = ShuffledWeight(Wd.to(gpu_device))
    parts = LoraPartials(torch.full((rows, -(-inter // 256), down_rank), float("nan"), device=gpu_device))
    act = fused_ops.silu_mul(gu[:, : 2 * inter], lora=lora, adapter_ids=ids,
                             down_shrink=(lora_a_rows(sw, hidden, down_rank, bound), parts))
    ref = fused_ops.silu_mul(gu[:, : 2 * inter], lora=lora, adapter_ids=ids)
    torch.cuda.synchronize()
    assert torch.equal(act, ref), "SiLU*up output differs with the down shrink"
    A = _np(Wd[hidden:]).reshape(n_ad, down_rank, inter)
    ids_h = ids.cpu().numpy() if bound < 0 else np.full(rows, bound)
    got = parts.sum().cpu().numpy()
    x = _np(act)
    for b in range(rows):
        a = ids_h[b] if 0 <= ids_h[b] < n_ad else 0
        want = A[a] @ x[b]
        bar = 1e-6 + 2e-5 * (np.abs(A[a]) @ np.abs(x[b]))
        assert (np.abs(got[b] - want) <= bar).all(), f"row {b}: shrink partials off by {np.abs(got[b] - want).max():.3e}"
