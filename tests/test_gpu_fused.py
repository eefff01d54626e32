"""Fused element-wise decode kernels vs the float64 oracle.

Bars: each kernel rounds its fp32 result once to the storage type, so the
bound is one rounding of the output (2^-8 relative for bf16, 2^-11 for
fp16, 1e-6 for fp32) plus 1e-5 absolute for the fp32 arithmetic.
"""

import numpy as np
import pytest
import torch

from oracle import fused as of
from oracle import lora as ol
from pagelora_amd import fused_ops

pytestmark = pytest.mark.gpu

REL = {torch.float32: 1e-6, torch.float16: 2.0**-11, torch.bfloat16: 2.0**-8}


def _check(got, want, dtype, extra_abs=1e-5):
    got = got.float().cpu().numpy()
    err = np.abs(got - want)
    bound = extra_abs + REL[dtype] * np.abs(want)
    assert (err <= bound).all(), f"max err {err.max():.3e}, worst ratio {(err / bound).max():.2f}"


def _round(dtype):
    if dtype == torch.bfloat16:
        return ol.round_bf16
    if dtype == torch.float16:
        return lambda a: np.asarray(a).astype(np.float16).astype(np.float64)
    return lambda a: np.asarray(a).astype(np.float32).astype(np.float64)


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("hidden", [128, 4096, 12288])
def test_rmsnorm_and_add_rmsnorm(gpu_device, dtype, hidden):
    g = torch.Generator().manual_seed(hidden)
    x = torch.randn((5, hidden), generator=g).to(dtype)
    r = torch.randn((5, hidden), generator=g).to(dtype)
    w = (1 + 0.1 * torch.randn(hidden, generator=g)).to(dtype)
    xd, rd, wd = x.to(gpu_device), r.to(gpu_device), w.to(gpu_device)
    out = fused_ops.rmsnorm(xd, wd, 1e-6)
    _check(out, of.rmsnorm(x.double().numpy(), w.double().numpy(), 1e-6), dtype)
    out2 = fused_ops.add_rmsnorm(rd, xd, wd, 1e-6)
    torch.cuda.synchronize()
    new_r, want = of.add_rmsnorm(r.double().numpy(), x.double().numpy(), w.double().numpy(), 1e-6,
                                 round_sum=_round(dtype))
    np.testing.assert_array_equal(rd.double().cpu().numpy(), new_r)  # the stored sum is the rounded sum
    _check(out2, want, dtype)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_silu_mul(gpu_device, dtype):
    g = torch.Generator().manual_seed(1)
    gu = (torch.randn((4, 2 * 12288), generator=g) * 3).to(dtype)
    out = fused_ops.silu_mul(gu.to(gpu_device))
    _check(out, of.silu_mul(gu.double().numpy()), dtype)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("head_dim", [64, 128, 256])
def test_qk_norm_rope_append(gpu_device, dtype, head_dim):
    hq, hkv, ps, pool, B = 8, 2, 16, 10, 4
    g = torch.Generator().manual_seed(head_dim)
    qkv = torch.randn((B, (hq + 2 * hkv) * head_dim), generator=g).to(dtype)
    qw = (1 + 0.1 * torch.randn(head_dim, generator=g)).to(dtype)
    kw = (1 + 0.1 * torch.randn(head_dim, generator=g)).to(dtype)
    positions = torch.tensor([0, 17, 4095, 40000])
    page_id = torch.tensor([3, 9, 0, 5])
    offset = torch.tensor([0, 15, 7, 1])
    cache = torch.zeros((pool, 2, ps, hkv, head_dim), dtype=dtype)
    dev = gpu_device
    cd = cache.to(dev)
    q = fused_ops.qk_norm_rope_append(qkv.to(dev), qw.to(dev), kw.to(dev), positions.to(dev), page_id.to(dev),
                                      offset.to(dev), cd, num_qo_heads=hq, num_kv_heads=hkv, head_dim=head_dim,
                                      page_size=ps, rope_theta=1e6, eps=1e-6)
    torch.cuda.synchronize()
    # the oracle rotates with the kernel's own fp32 inverse-frequency table:
    # a 1-ulp table difference moves the angle at position 40000 by ~5e-3 rad
    table = fused_ops.rope_inv_freq(head_dim, 1e6, 1.0, dev).cpu().numpy()
    np.testing.assert_allclose(table, of.inv_freq_f32(head_dim, 1e6), rtol=3e-7)
    wq, wk, wv = of.qk_norm_rope_append(qkv.double().numpy(), hq, hkv, head_dim, qw.double().numpy(),
                                        kw.double().numpy(), positions.numpy(), 1e-6, 1e6, inv_freq=table)
    _check(q, wq, dtype, extra_abs=2e-5)
    got = cd.cpu()
    for b in range(B):
        _check(got[page_id[b], 0, offset[b]], wk[b], dtype, extra_abs=2e-5)
        np.testing.assert_array_equal(got[page_id[b], 1, offset[b]].double().numpy(), wv[b])
    # nothing else in the pool was touched
    mask = torch.ones((pool, ps), dtype=torch.bool)
    mask[page_id, offset] = False
    assert (got[:, :, :][mask.nonzero(as_tuple=True)[0], :, mask.nonzero(as_tuple=True)[1]] == 0).all()
