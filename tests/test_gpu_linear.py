"""Decode-sized linear layer (pl_linear) with and without the fused LoRA
expand, vs float64 references on the same rounded inputs.

Bars: one rounding of the output to the storage type (2^-8 relative for
bf16, 2^-11 for fp16) plus 1e-3 absolute for the fp32 accumulation over K;
with LoRA the oracle rounds the rank-r intermediate like the reference's
F.linear (packed_ops.py:324) and the absolute bar is 2e-3.
"""

import numpy as np
import pytest
import torch

from oracle import lora as ol
from pagelora_amd.lora import lora_linear

pytestmark = pytest.mark.gpu

REL = {torch.bfloat16: 2.0**-8, torch.float16: 2.0**-11}


def _check(got, want, dtype, atol):
    got = got.float().cpu().numpy()
    err = np.abs(got - want)
    bound = atol + REL[dtype] * np.abs(want)
    assert np.isfinite(got).all()
    assert (err <= bound).all(), f"max err {err.max():.3e} worst ratio {(err / bound).max():.2f}"


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("T", [1, 4, 16, 17, 64])
@pytest.mark.parametrize("NK", [(6144, 4096), (4096, 12288), (1000, 256), (37, 64), (48, 40), (200, 264)])
def test_linear_matches_float64(gpu_device, dtype, T, NK):
    N, K = NK
    g = torch.Generator().manual_seed(N + K + T)
    x = torch.randn((T, K), generator=g).to(dtype)
    w = (torch.randn((N, K), generator=g) * 0.02).to(dtype)
    b = (torch.randn(N, generator=g) * 0.1).to(dtype)
    out = lora_linear(x.to(gpu_device), w.to(gpu_device), None, None, bias=b.to(gpu_device))
    want = x.double().numpy() @ w.double().numpy().T + b.double().numpy()
    _check(out, want, dtype, 1e-3)


@pytest.mark.parametrize("T", [1, 4, 16, 40])
@pytest.mark.parametrize("K", [512, 264])
def test_fused_lora_expand_matches_oracle(gpu_device, T, K):
    # K = 264: the k loops' last step holds only one 8-element group per row
    dtype = torch.bfloat16
    g = torch.Generator().manual_seed(T + K)
    outs, r, n = (256, 64, 64), 16, 3
    N = sum(outs)
    x = torch.randn((T, K), generator=g).to(dtype)
    w = (torch.randn((N, K), generator=g) * 0.02).to(dtype)
    ids = torch.randint(-1, n, (T,), generator=g, dtype=torch.int32)
    mods, host, col = [], [], 0
    for fout in outs:
        A = (torch.randn((n, r, K), generator=g) * K ** -0.5).to(dtype)
        B = (torch.randn((n, fout, r), generator=g) * 0.05).to(dtype)
        mods.append((A.to(gpu_device), B.to(gpu_device), col, 2.0))
        host.append((A, B, col, fout))
        col += fout
    out = lora_linear(x.to(gpu_device), w.to(gpu_device), mods, ids.to(gpu_device))
    torch.cuda.synchronize()
    want = x.double().numpy() @ w.double().numpy().T
    for A, B, c, fout in host:
        want[:, c:c + fout] += ol.multi_adapter_delta(x.float().numpy(), ids.tolist(), A.float().numpy(),
                                                      B.float().numpy(), 2.0, intermediate="bf16")
    _check(out, want, dtype, 2e-3)


def test_single_adapter_2d_lora_rank_2(gpu_device):
    # one adapter given as 2-D A/B (the reference's bound-adapter case), rank 2
    dtype = torch.bfloat16
    g = torch.Generator().manual_seed(9)
    T, K, N = 3, 64, 40
    x = torch.randn((T, K), generator=g).to(dtype)
    w = (torch.randn((N, K), generator=g) * 0.05).to(dtype)
    A = (torch.randn((2, K), generator=g) * 0.2).to(dtype)
    B = (torch.randn((N, 2), generator=g) * 0.2).to(dtype)
    ids = torch.zeros(T, dtype=torch.int32)
    out = lora_linear(x.to(gpu_device), w.to(gpu_device), [(A.to(gpu_device), B.to(gpu_device), 0, 2.0)],
                      ids.to(gpu_device))
    want = x.double().numpy() @ w.double().numpy().T + ol.lora_delta(
        x.float().numpy(), A.float().numpy(), B.float().numpy(), 2.0, intermediate="bf16")
    _check(out, want, dtype, 2e-3)
