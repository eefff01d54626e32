"""Pre-shuffled decode GEMM (pl_weight_shuffle + pl_linear_shuffled) vs the oracle.

The shuffle is data movement: checked bit-exactly against the documented
index map.  The GEMM is checked against the oracle's linear term (the LoRA
oracle at scale 0: x . W^T + bias in float64) with one rounding of the
output (2^-8 relative for bf16, 2^-11 for fp16) plus the fp32
accumulation's error, 2e-3 max-abs.
"""

import numpy as np
import pytest
import torch

from oracle import lora as ol
from pagelora_amd import _lib
from pagelora_amd.linear import ShuffledWeight, linear_shuffled

pytestmark = pytest.mark.gpu

REL = {torch.bfloat16: 2.0**-8, torch.float16: 2.0**-11}


def _oracle_linear(x, w, bias):
    zero_a = np.zeros((1, x.shape[1]))
    zero_b = np.zeros((w.shape[0], 1))
    return ol.lora_linear(x, w, bias, zero_a, zero_b, 0.0)


def test_shuffle_layout_matches_the_index_map(gpu_device):
    n, k = 37, 96  # rows padded to 48
    w = torch.arange(n * k, dtype=torch.int32).remainder(30000).to(torch.float32).to(torch.bfloat16).reshape(n, k)
    sw = ShuffledWeight(w.to(gpu_device))
    got = sw.data.cpu().view(torch.int16).numpy()
    wi = w.view(torch.int16).numpy()
    assert got.size == 48 * k
    ks = k // 32
    want = np.zeros(48 * k, dtype=np.int16)
    for nb in range(3):
        for s in range(ks):
            for lane in range(64):
                row, col = nb * 16 + lane % 16, s * 32 + (lane // 16) * 8
                base = ((nb * ks + s) * 64 + lane) * 8
                if row < n:
                    want[base:base + 8] = wi[row, col:col + 8]
    np.testing.assert_array_equal(got, want)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("tokens", [1, 4, 16, 17, 64])
@pytest.mark.parametrize("shape", [(6192, 4096), (4112, 12288), (1000, 256), (16, 32)])
def test_linear_shuffled_vs_oracle(gpu_device, dtype, tokens, shape):
    n, k = shape
    g = torch.Generator().manual_seed(n + k + tokens)
    x = torch.randn((tokens, k), generator=g).to(dtype)
    w = (torch.randn((n, k), generator=g) * k ** -0.5).to(dtype)
    bias = (torch.randn(n, generator=g) * 0.1).to(dtype) if n == 1000 else None
    sw = ShuffledWeight(w.to(gpu_device))
    out = linear_shuffled(x.to(gpu_device), sw, bias.to(gpu_device) if bias is not None else None)
    torch.cuda.synchronize()
    want = _oracle_linear(x.double().numpy(), w.double().numpy(), bias.double().numpy() if bias is not None else None)
    got = out.float().cpu().numpy()
    err = np.abs(got - want)
    bound = 2e-3 + REL[dtype] * np.abs(want)
    assert (err <= bound).all(), f"max err {err.max():.3e}"


def test_strided_x_and_out(gpu_device):
    """x and out as column slices of wider buffers (the decoder's views)."""
    g = torch.Generator().manual_seed(3)
    xs = torch.randn((4, 4096 + 64), generator=g).to(torch.bfloat16)
    w = (torch.randn((512, 4096), generator=g) * 0.02).to(torch.bfloat16)
    sw = ShuffledWeight(w.to(gpu_device))
    xd = xs.to(gpu_device)
    big = torch.full((4, 512 + 32), 7.0, dtype=torch.bfloat16, device=gpu_device)
    linear_shuffled(xd[:, :4096], sw, out=big[:, :512])
    ref = linear_shuffled(xd[:, :4096].contiguous(), sw)
    torch.cuda.synchronize()
    assert torch.equal(big[:, :512], ref)
    assert (big[:, 512:] == 7.0).all()


def test_bad_inputs_raise(gpu_device):
    w = torch.zeros((16, 48), dtype=torch.bfloat16, device=gpu_device)
    with pytest.raises(ValueError, match="multiple of 32"):
        ShuffledWeight(w)
    sw = ShuffledWeight(torch.zeros((16, 64), dtype=torch.bfloat16, device=gpu_device))
    with pytest.raises(ValueError):
        linear_shuffled(torch.zeros((4, 32), dtype=torch.bfloat16, device=gpu_device), sw)
    with pytest.raises(ValueError, match="at most"):
        linear_shuffled(torch.zeros((_lib.PL_LINEAR_MAX_TOKENS + 1, 64), dtype=torch.bfloat16, device=gpu_device), sw)


@pytest.mark.parametrize("splits", [1, 2, 3, 4])
@pytest.mark.parametrize("shape", [(4112, 4096), (4112, 12288), (6192, 4096), (48, 96)])
@pytest.mark.parametrize("tokens", [1, 4, 17])
def test_split_planes_sum_to_the_linear(gpu_device, splits, shape, tokens):
    """pl_linear_shuffled_split: the in-order sum of the planes, rounded, is the
    oracle's linear (same bar), and for one split it is pl_linear_shuffled."""
    from pagelora_amd.linear import linear_shuffled_split

    n, k = shape
    g = torch.Generator().manual_seed(n * 7 + k + tokens + splits)
    x = torch.randn((tokens, k), generator=g).to(torch.bfloat16)
    w = (torch.randn((n, k), generator=g) * k ** -0.5).to(torch.bfloat16)
    sw = ShuffledWeight(w.to(gpu_device))
    if splits > k // 32:  # fewer 32-wide k-steps than splits
        with pytest.raises(ValueError, match="splits"):
            linear_shuffled_split(x.to(gpu_device), sw, splits)
        return
    so = linear_shuffled_split(x.to(gpu_device), sw, splits)
    got = so.sum()
    torch.cuda.synchronize()
    assert so.partials.shape == (splits, tokens, (n + 7) // 8 * 8)
    want = _oracle_linear(x.double().numpy(), w.double().numpy(), None)
    err = np.abs(got.float().cpu().numpy() - want)
    assert (err <= 2e-3 + REL[torch.bfloat16] * np.abs(want)).all(), f"max err {err.max():.3e}"
    if splits == 1:
        assert torch.equal(got, linear_shuffled(x.to(gpu_device), sw))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("side_splits", [1, 3, 16])
@pytest.mark.parametrize("shape", [(4096 + 16, 4096, 4096), (4096 + 64, 12288, 4096), (6144 + 48, 4096, 6144),
                                   (48 + 8, 96, 48)])
@pytest.mark.parametrize("tokens", [1, 4, 17])
def test_side_planes_and_main_columns(gpu_device, side_splits, shape, tokens, dtype):
    """pl_linear_shuffled_side: the main columns are pl_linear_shuffled's,
    bit for bit (the same workgroups compute them); the side planes' in-order
    sum, rounded, is the oracle's linear over the side rows (the same bar)."""
    from pagelora_amd.linear import linear_shuffled_side

    n, k, main = shape
    g = torch.Generator().manual_seed(n * 3 + k + tokens + side_splits)
    x = torch.randn((tokens, k), generator=g).to(dtype)
    w = (torch.randn((n, k), generator=g) * k ** -0.5).to(dtype)
    sw = ShuffledWeight(w.to(gpu_device))
    if side_splits > k // 32:
        with pytest.raises(ValueError, match="side_splits"):
            linear_shuffled_side(x.to(gpu_device), sw, main, side_splits)
        return
    out, side = linear_shuffled_side(x.to(gpu_device), sw, main, side_splits)
    ref = linear_shuffled(x.to(gpu_device), sw)
    torch.cuda.synchronize()
    assert out.shape == (tokens, main)
    assert torch.equal(out, ref[:, :main])
    assert side.out_features == n - main and side.partials.shape == (side_splits, tokens, (n - main + 7) // 8 * 8)
    want = _oracle_linear(x.double().numpy(), w[main:].double().numpy(), None)
    got = side.sum().float().cpu().numpy()
    err = np.abs(got - want)
    assert (err <= 2e-3 + REL[dtype] * np.abs(want)).all(), f"max err {err.max():.3e}"


def test_side_bad_inputs_raise(gpu_device):
    from pagelora_amd.linear import linear_shuffled_side

    sw = ShuffledWeight(torch.zeros((48, 64), dtype=torch.bfloat16, device=gpu_device))
    x = torch.zeros((4, 64), dtype=torch.bfloat16, device=gpu_device)
    for main in (0, 8, 48, 64):  # not a positive multiple of 16 below out_features
        with pytest.raises(ValueError, match="main_features"):
            linear_shuffled_side(x, sw, main, 1)
    with pytest.raises(ValueError, match="side_splits"):
        linear_shuffled_side(x, sw, 32, 3)  # 2 k-steps


def _oracle_chunked(x, w_dev, rows=16384):
    """x . W^T in float64 with W copied to the host 16384 rows at a time."""
    want = np.empty((x.shape[0], w_dev.shape[0]))
    for lo in range(0, w_dev.shape[0], rows):
        want[:, lo: lo + rows] = x @ w_dev[lo: lo + rows].double().cpu().numpy().T
    return want


@pytest.mark.parametrize("tokens", [1, 4, 64])
@pytest.mark.parametrize("shape", [(151936, 4096), (24608, 4096)])
def test_linear_shuffled_decoder_shapes(gpu_device, shape, tokens):
    """The Qwen3-8B lm_head (vocabulary 151,936: 9,496 row blocks, the
    largest grid of the decode step) and gate_up with its two adapters' A
    rows (24,576 + 32 rows) against the oracle's linear term, same bar."""
    n, k = shape
    print(f"[shuffled gemm] {n} x {k}, {tokens} tokens", flush=True)
    g = torch.Generator(device=gpu_device).manual_seed(n + tokens)
    w = (torch.randn((n, k), generator=g, device=gpu_device) * k ** -0.5).to(torch.bfloat16)
    x = torch.randn((tokens, k), generator=g, device=gpu_device).to(torch.bfloat16)
    sw = ShuffledWeight(w)
    out = linear_shuffled(x, sw)
    torch.cuda.synchronize()
    want = _oracle_chunked(x.double().cpu().numpy(), w)
    err = np.abs(out.float().cpu().numpy() - want)
    assert (err <= 2e-3 + REL[torch.bfloat16] * np.abs(want)).all(), f"max err {err.max():.3e}"


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("shape", [(6144 + 48, 4096), (24576 + 32, 4096), (4096 + 16, 12288), (151936, 4096),
                                   (37, 96)])
def test_unshuffle_inverts_the_shuffle(gpu_device, shape, dtype):
    """pl_weight_unshuffle(pl_weight_shuffle(W)) == W bit for bit at the
    decoder's shapes (qkv, gate_up and down with their A rows, the lm_head)
    and a ragged one, into a fresh tensor and into the decoder's shared
    row-major scratch buffer (which the stage check's oracle weights and
    prefill's library GEMMs read)."""
    from pagelora_amd.decoder import unshuffled_scratch

    n, k = shape
    print(f"[unshuffle] {n} x {k} {dtype}", flush=True)
    g = torch.Generator(device=gpu_device).manual_seed(n * 3 + k)
    w = torch.randn((n, k), generator=g, device=gpu_device).to(dtype)
    sw = ShuffledWeight(w)
    fresh = sw.unshuffle()
    assert torch.equal(fresh.view(torch.int16), w.view(torch.int16))
    del fresh
    scratch = unshuffled_scratch(sw)
    assert torch.equal(scratch.view(torch.int16), w.view(torch.int16))
    # a row-strided target (the unshuffle writes only the [n, k] view)
    wide = torch.full((n, k + 64), 3.0, dtype=dtype, device=gpu_device)
    sw.unshuffle(wide[:, :k])
    assert torch.equal(wide[:, :k].view(torch.int16), w.view(torch.int16))
    assert (wide[:, k:] == 3.0).all()
