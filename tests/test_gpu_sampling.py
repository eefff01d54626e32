"""pl_greedy_argmax vs torch.argmax (the reference's greedy_argmax_token,
sampling.py:8-15), computed on the CPU from the same logits: identical
indices, including ties (first index), NaN (first NaN), rows of -inf, a
vocab that is not a multiple of the 16-byte chunk (padded row stride), and
the Qwen3 vocab."""

import pytest
import torch

from pagelora_amd import _lib, fused_ops

pytestmark = pytest.mark.gpu


def _check(logits_cpu, dev, ld=None):
    rows, vocab = logits_cpu.shape
    if ld is None:
        d = logits_cpu.to(dev)
    else:  # padded rows: a strided view of a wider buffer
        buf = torch.full((rows, ld), float("nan"), dtype=logits_cpu.dtype)
        buf[:, :vocab] = logits_cpu
        d = buf.to(dev)[:, :vocab]
    tokens = torch.full((rows,), -7, dtype=torch.int64, device=dev)
    got = fused_ops.greedy_argmax(d, tokens_out=tokens)
    want = torch.argmax(logits_cpu.float(), dim=-1)
    assert torch.equal(got.cpu(), want), (got.cpu()[:8], want[:8])
    assert torch.equal(tokens.cpu(), want)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("rows,vocab", [(1, 8), (4, 151936), (64, 32000), (3, 1000)])
def test_random_logits(gpu_device, dtype, rows, vocab):
    g = torch.Generator().manual_seed(rows * vocab)
    _check((torch.randn((rows, vocab), generator=g) * 4).to(dtype), gpu_device)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_ties_nan_and_inf(gpu_device, dtype):
    vocab = 5000
    x = torch.zeros((6, vocab), dtype=dtype)
    x[0, [17, 300, 4999]] = 2.0                # tie: the first index wins
    x[1] = float("-inf")                       # all -inf: index 0
    x[2, 1234] = float("nan")                  # a NaN beats every number
    x[2, 10] = 100.0
    x[3, [40, 41]] = float("nan")              # first NaN
    x[4, 4999] = float("inf")
    x[5] = 1.0                                 # all equal: index 0
    _check(x, gpu_device)


@pytest.mark.parametrize("dtype,vocab,ld", [(torch.bfloat16, 1003, 1008), (torch.float16, 9, 16), (torch.float32, 1001, 1004)])
def test_tail_and_padded_rows(gpu_device, dtype, vocab, ld):
    g = torch.Generator().manual_seed(vocab)
    x = torch.randn((5, vocab), generator=g).to(dtype)
    x[2, vocab - 1] = 50.0                     # the max in the tail past the last whole chunk
    _check(x, gpu_device, ld=ld)


def test_rejects_misaligned_rows(gpu_device):
    x = torch.zeros((2, 1003), dtype=torch.bfloat16, device=gpu_device)
    with pytest.raises(ValueError):
        fused_ops.greedy_argmax(x)             # row stride 1003 elements: rows not 16-byte aligned


def test_workspace_size_and_reuse(gpu_device):
    # slices of 2048 16-byte chunks: 151,936 bf16 logits -> 10 slices per row
    ws = fused_ops.greedy_argmax_workspace(4, 151936, torch.bfloat16, gpu_device)
    assert ws.numel() == 4 * 10 * 8
    g = torch.Generator().manual_seed(3)
    for _ in range(3):  # the same workspace serves consecutive calls
        x = torch.randn((4, 151936), generator=g).to(torch.bfloat16)
        got = fused_ops.greedy_argmax(x.to(gpu_device), workspace=ws)
        assert torch.equal(got.cpu(), torch.argmax(x.float(), dim=-1))
    with pytest.raises(_lib.WorkspaceTooSmallError):
        fused_ops.greedy_argmax(x.to(gpu_device), workspace=ws[:16])
