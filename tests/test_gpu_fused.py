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


# ---- the same kernels with the LoRA up-projection of their input applied first
# The producer GEMM's output row holds the base columns followed by every
# adapter's rank-space intermediate y; the module output is
# round(base + scale * y[a] . B[a]^T), restated here through the LoRA oracle
# (lora_delta with A = identity is exactly scale * y . B^T).  Token 3 carries
# an id outside [0, n_adapters): it gets no delta.  Bound: two roundings of
# the result (the module output's and the kernel's own).

IDS = [0, 2, 1, -1, 2]
N_ADAPTERS, RANK, SCALE = 3, 16, 2.0


def _lora_inputs(g, rows, base_cols, modules, dtype):
    """(full producer output [rows, base + n*r*len(modules)], {name: B}, {name: y_offset})."""
    full = torch.randn((rows, base_cols + N_ADAPTERS * RANK * len(modules)), generator=g).to(dtype)
    Bs, offs = {}, {}
    for j, (name, fout) in enumerate(modules):
        Bs[name] = (torch.randn((N_ADAPTERS, fout, RANK), generator=g) * 0.05).to(dtype)
        offs[name] = base_cols + j * N_ADAPTERS * RANK
    return full, Bs, offs


def _module_out(full, base_lo, base_hi, B, y_off, dtype):
    """Oracle of round(base + scale * y[a] . B[a]^T) for columns [base_lo, base_hi)."""
    f = full.double().numpy()
    base = f[:, base_lo:base_hi].copy()
    eye = np.eye(RANK)
    for t, a in enumerate(IDS):
        if 0 <= a < N_ADAPTERS:
            y = f[t:t + 1, y_off + a * RANK: y_off + (a + 1) * RANK]
            base[t] += ol.lora_delta(y, eye, B[a].double().numpy(), SCALE)[0]
    return _round(dtype)(base)


def _check2(got, want, dtype, extra_abs=1e-5):
    got = got.float().cpu().numpy() if isinstance(got, torch.Tensor) else got
    err = np.abs(got - want)
    bound = extra_abs + 2 * REL[dtype] * np.maximum(np.abs(want), 1e-3)
    assert np.isfinite(got).all()
    assert (err <= bound).all(), f"max err {err.max():.3e}, worst ratio {(err / bound).max():.2f}"


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("hidden", [256, 4096])
def test_add_rmsnorm_lora(gpu_device, dtype, hidden):
    g = torch.Generator().manual_seed(100 + hidden)
    rows = len(IDS)
    full, Bs, offs = _lora_inputs(g, rows, hidden, [("o", hidden)], dtype)
    r = torch.randn((rows, hidden), generator=g).to(dtype)
    w = (1 + 0.1 * torch.randn(hidden, generator=g)).to(dtype)
    fd, rd = full.to(gpu_device), r.to(gpu_device)
    ids = torch.tensor(IDS, dtype=torch.int32, device=gpu_device)
    up = fused_ops.LoraUp(fd, offs["o"], Bs["o"].to(gpu_device), SCALE)
    out = fused_ops.add_rmsnorm(rd, fd[:, :hidden], w.to(gpu_device), 1e-6, lora=up, adapter_ids=ids)
    torch.cuda.synchronize()
    x_eff = _module_out(full, 0, hidden, Bs["o"], offs["o"], dtype)
    new_r, want = of.add_rmsnorm(r.double().numpy(), x_eff, w.double().numpy(), 1e-6, round_sum=_round(dtype))
    _check2(rd, new_r, dtype)
    _check2(out, want, dtype)


@pytest.mark.parametrize("rank", [8, 32, 64])
@pytest.mark.parametrize("hidden", [4096, 12288])
def test_add_rmsnorm_lora_ranks(gpu_device, rank, hidden):
    # every built rank, through the single-chunk kernel (4096) and the general one (12288)
    dtype = torch.bfloat16
    g = torch.Generator().manual_seed(rank + hidden)
    rows = len(IDS)
    full = torch.randn((rows, hidden + N_ADAPTERS * rank), generator=g).to(dtype)
    B = (torch.randn((N_ADAPTERS, hidden, rank), generator=g) * 0.05).to(dtype)
    r = torch.randn((rows, hidden), generator=g).to(dtype)
    w = (1 + 0.1 * torch.randn(hidden, generator=g)).to(dtype)
    fd, rd = full.to(gpu_device), r.to(gpu_device)
    ids = torch.tensor(IDS, dtype=torch.int32, device=gpu_device)
    up = fused_ops.LoraUp(fd, hidden, B.to(gpu_device), SCALE)
    out = fused_ops.add_rmsnorm(rd, fd[:, :hidden], w.to(gpu_device), 1e-6, lora=up, adapter_ids=ids)
    torch.cuda.synchronize()
    f = full.double().numpy()
    x_eff = f[:, :hidden].copy()
    for t, a in enumerate(IDS):
        if 0 <= a < N_ADAPTERS:
            y = f[t:t + 1, hidden + a * rank: hidden + (a + 1) * rank]
            x_eff[t] += ol.lora_delta(y, np.eye(rank), B[a].double().numpy(), SCALE)[0]
    x_eff = _round(dtype)(x_eff)
    new_r, want = of.add_rmsnorm(r.double().numpy(), x_eff, w.double().numpy(), 1e-6, round_sum=_round(dtype))
    _check2(rd, new_r, dtype)
    _check2(out, want, dtype)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_silu_mul_lora(gpu_device, dtype):
    inter = 1024
    g = torch.Generator().manual_seed(7)
    rows = len(IDS)
    full, Bs, offs = _lora_inputs(g, rows, 2 * inter, [("gate", inter), ("up", inter)], dtype)
    fd = full.to(gpu_device)
    ids = torch.tensor(IDS, dtype=torch.int32, device=gpu_device)
    ups = (fused_ops.LoraUp(fd, offs["gate"], Bs["gate"].to(gpu_device), SCALE),
           fused_ops.LoraUp(fd, offs["up"], Bs["up"].to(gpu_device), SCALE))
    out = fused_ops.silu_mul(fd[:, : 2 * inter], lora=ups, adapter_ids=ids)
    torch.cuda.synchronize()
    gate = _module_out(full, 0, inter, Bs["gate"], offs["gate"], dtype)
    up = _module_out(full, inter, 2 * inter, Bs["up"], offs["up"], dtype)
    _check2(out, of.silu_mul(np.concatenate([gate, up], axis=1)), dtype)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("head_dim", [64, 128])
def test_qk_norm_rope_append_lora(gpu_device, dtype, head_dim):
    hq, hkv, ps, pool = 8, 2, 16, 10
    rows = len(IDS)
    qd, kd = hq * head_dim, hkv * head_dim
    g = torch.Generator().manual_seed(head_dim + 1)
    full, Bs, offs = _lora_inputs(g, rows, qd + 2 * kd, [("q", qd), ("k", kd), ("v", kd)], dtype)
    qw = (1 + 0.1 * torch.randn(head_dim, generator=g)).to(dtype)
    kw = (1 + 0.1 * torch.randn(head_dim, generator=g)).to(dtype)
    positions = torch.tensor([0, 17, 4095, 40000, 5])
    page_id = torch.tensor([3, 9, 0, 5, 7])
    offset = torch.tensor([0, 15, 7, 1, 2])
    dev = gpu_device
    cd = torch.zeros((pool, 2, ps, hkv, head_dim), dtype=dtype, device=dev)
    fd = full.to(dev)
    ids = torch.tensor(IDS, dtype=torch.int32, device=dev)
    ups = tuple(fused_ops.LoraUp(fd, offs[m], Bs[m].to(dev), SCALE) for m in ("q", "k", "v"))
    q = fused_ops.qk_norm_rope_append(fd[:, : qd + 2 * kd], qw.to(dev), kw.to(dev), positions.to(dev),
                                      page_id.to(dev), offset.to(dev), cd, num_qo_heads=hq, num_kv_heads=hkv,
                                      head_dim=head_dim, page_size=ps, rope_theta=1e6, eps=1e-6, lora=ups,
                                      adapter_ids=ids)
    torch.cuda.synchronize()
    qkv_eff = np.concatenate([_module_out(full, 0, qd, Bs["q"], offs["q"], dtype),
                              _module_out(full, qd, qd + kd, Bs["k"], offs["k"], dtype),
                              _module_out(full, qd + kd, qd + 2 * kd, Bs["v"], offs["v"], dtype)], axis=1)
    table = fused_ops.rope_inv_freq(head_dim, 1e6, 1.0, dev).cpu().numpy()
    wq, wk, wv = of.qk_norm_rope_append(qkv_eff, hq, hkv, head_dim, qw.double().numpy(), kw.double().numpy(),
                                        positions.numpy(), 1e-6, 1e6, inv_freq=table)
    _check2(q, wq, dtype, extra_abs=2e-5)
    got = cd.cpu()
    for b in range(rows):
        _check2(got[page_id[b], 0, offset[b]], wk[b], dtype, extra_abs=2e-5)
        _check2(got[page_id[b], 1, offset[b]], wv[b], dtype)


def test_lora_up_rejects_bad_layouts(gpu_device):
    x = torch.zeros((2, 64 + 16), dtype=torch.bfloat16, device=gpu_device)
    r = torch.zeros((2, 64), dtype=torch.bfloat16, device=gpu_device)
    w = torch.ones(64, dtype=torch.bfloat16, device=gpu_device)
    ids = torch.zeros(2, dtype=torch.int32, device=gpu_device)
    with pytest.raises(ValueError, match="out of range"):
        fused_ops.add_rmsnorm(r, x[:, :64], w, 1e-6,
                              lora=fused_ops.LoraUp(x, 72, torch.zeros((1, 64, 16), dtype=torch.bfloat16,
                                                                       device=gpu_device), 1.0), adapter_ids=ids)
    with pytest.raises(NotImplementedError, match="rank"):
        fused_ops.add_rmsnorm(r, x[:, :64], w, 1e-6,
                              lora=fused_ops.LoraUp(x, 64, torch.zeros((1, 64, 12), dtype=torch.bfloat16,
                                                                       device=gpu_device), 1.0), adapter_ids=ids)
    with pytest.raises(ValueError, match="output features"):
        fused_ops.add_rmsnorm(r, x[:, :64], w, 1e-6,
                              lora=fused_ops.LoraUp(x, 64, torch.zeros((1, 32, 16), dtype=torch.bfloat16,
                                                                       device=gpu_device), 1.0), adapter_ids=ids)


# ---- split-K inputs: a consumer fed fp32 partial planes equals the same
# consumer fed their in-order, rounded sum (bit-exact).

def _random_split(g, splits, rows, cols, dtype, device):
    from pagelora_amd.linear import SplitOutput

    ld = (cols + 7) // 8 * 8 + 8
    parts = (torch.randn((splits, rows, ld), generator=g) * 0.7).to(device)
    return SplitOutput(parts, cols, dtype)


# Splits 1-4 at hidden <= 8192 take the single-chunk decode kernel; 6 splits
# and hidden 12288 take the general one.
@pytest.mark.parametrize("splits,hidden", [(1, 4096), (2, 4096), (3, 4096), (4, 4096), (6, 4096), (3, 12288)])
def test_add_rmsnorm_lora_split_input_matches_summed_input(gpu_device, splits, hidden):
    rows = len(IDS)
    g = torch.Generator().manual_seed(splits)
    so = _random_split(g, splits, rows, hidden + N_ADAPTERS * RANK, torch.bfloat16, gpu_device)
    B = (torch.randn((N_ADAPTERS, hidden, RANK), generator=g) * 0.05).to(torch.bfloat16).to(gpu_device)
    r0 = torch.randn((rows, hidden), generator=g).to(torch.bfloat16).to(gpu_device)
    w = (1 + 0.1 * torch.randn(hidden, generator=g)).to(torch.bfloat16).to(gpu_device)
    ids = torch.tensor(IDS, dtype=torch.int32, device=gpu_device)
    dense = so.sum()
    r1, r2 = r0.clone(), r0.clone()
    out1 = fused_ops.add_rmsnorm(r1, so, w, 1e-6, lora=fused_ops.LoraUp(so, hidden, B, SCALE), adapter_ids=ids)
    out2 = fused_ops.add_rmsnorm(r2, dense[:, :hidden], w, 1e-6, lora=fused_ops.LoraUp(dense, hidden, B, SCALE),
                                 adapter_ids=ids)
    torch.cuda.synchronize()
    assert torch.equal(r1, r2) and torch.equal(out1, out2)


@pytest.mark.parametrize("splits", [2, 4])
def test_qk_norm_rope_append_lora_split_input_matches_summed_input(gpu_device, splits):
    hq, hkv, d, ps, pool = 8, 2, 128, 16, 10
    rows = len(IDS)
    qd, kd = hq * d, hkv * d
    g = torch.Generator().manual_seed(10 + splits)
    so = _random_split(g, splits, rows, qd + 2 * kd + 3 * N_ADAPTERS * RANK, torch.bfloat16, gpu_device)
    dense = so.sum()
    Bs = [(torch.randn((N_ADAPTERS, f, RANK), generator=g) * 0.05).to(torch.bfloat16).to(gpu_device)
          for f in (qd, kd, kd)]
    offs = [qd + 2 * kd + j * N_ADAPTERS * RANK for j in range(3)]
    qw = (1 + 0.1 * torch.randn(d, generator=g)).to(torch.bfloat16).to(gpu_device)
    kw = (1 + 0.1 * torch.randn(d, generator=g)).to(torch.bfloat16).to(gpu_device)
    pos = torch.tensor([0, 17, 4095, 40000, 5], device=gpu_device)
    pid = torch.tensor([3, 9, 0, 5, 7], device=gpu_device)
    off = torch.tensor([0, 15, 7, 1, 2], device=gpu_device)
    ids = torch.tensor(IDS, dtype=torch.int32, device=gpu_device)
    outs = []
    for src in (so, dense):
        cache = torch.zeros((pool, 2, ps, hkv, d), dtype=torch.bfloat16, device=gpu_device)
        ups = tuple(fused_ops.LoraUp(src, o, B, SCALE) for o, B in zip(offs, Bs))
        inp = src if src is so else dense[:, : qd + 2 * kd]
        q = fused_ops.qk_norm_rope_append(inp, qw, kw, pos, pid, off, cache, num_qo_heads=hq, num_kv_heads=hkv,
                                          head_dim=d, page_size=ps, rope_theta=1e6, eps=1e-6, lora=ups,
                                          adapter_ids=ids)
        outs.append((q, cache))
    torch.cuda.synchronize()
    assert torch.equal(outs[0][0], outs[1][0]) and torch.equal(outs[0][1], outs[1][1])


# The chunked B layout (PL_LORA_B_CHUNK8) holds the same values in another
# order: every consumer must give bit-identical results with it.
@pytest.mark.parametrize("hidden,splits", [(4096, 0), (4096, 3), (12288, 0), (256, 2)])
def test_lora_b_chunk8_add_rmsnorm_bitwise(gpu_device, hidden, splits):
    rows, dev = len(IDS), gpu_device
    g = torch.Generator().manual_seed(hidden + splits)
    cols = hidden + N_ADAPTERS * RANK
    if splits:
        y = _random_split(g, splits, rows, cols, torch.bfloat16, dev)
        x = y
    else:
        y = torch.randn((rows, cols), generator=g).to(torch.bfloat16).to(dev)
        x = y[:, :hidden]
    B = (torch.randn((N_ADAPTERS, hidden, RANK), generator=g) * 0.05).to(torch.bfloat16).to(dev)
    r0 = torch.randn((rows, hidden), generator=g).to(torch.bfloat16).to(dev)
    w = (1 + 0.1 * torch.randn(hidden, generator=g)).to(torch.bfloat16).to(dev)
    ids = torch.tensor(IDS, dtype=torch.int32, device=dev)
    outs = []
    for Bx in (B, fused_ops.lora_b_chunk8(B)):
        r = r0.clone()
        o = fused_ops.add_rmsnorm(r, x, w, 1e-6, lora=fused_ops.LoraUp(y, hidden, Bx, SCALE), adapter_ids=ids)
        outs.append((r, o))
    torch.cuda.synchronize()
    assert torch.equal(outs[0][0], outs[1][0]) and torch.equal(outs[0][1], outs[1][1])


def test_lora_b_chunk8_silu_and_qk_bitwise(gpu_device):
    rows, dev, dtype = len(IDS), gpu_device, torch.bfloat16
    g = torch.Generator().manual_seed(77)
    inter = 1024
    full, Bs, offs = _lora_inputs(g, rows, 2 * inter, [("gate", inter), ("up", inter)], dtype)
    fd = full.to(dev)
    ids = torch.tensor(IDS, dtype=torch.int32, device=dev)
    res = []
    for conv in (lambda b: b, fused_ops.lora_b_chunk8):
        ups = tuple(fused_ops.LoraUp(fd, offs[m], conv(Bs[m].to(dev)), SCALE) for m in ("gate", "up"))
        res.append(fused_ops.silu_mul(fd[:, : 2 * inter], lora=ups, adapter_ids=ids))
    assert torch.equal(res[0], res[1])

    hq, hkv, d, ps, pool = 8, 2, 128, 16, 10
    qd, kd = hq * d, hkv * d
    full, Bs, offs = _lora_inputs(g, rows, qd + 2 * kd, [("q", qd), ("k", kd), ("v", kd)], dtype)
    fd = full.to(dev)
    qw = torch.ones(d, dtype=dtype, device=dev)
    pos = torch.tensor([0, 17, 4095, 40000, 5], device=dev)
    pid = torch.tensor([3, 9, 0, 5, 7], device=dev)
    off = torch.tensor([0, 15, 7, 1, 2], device=dev)
    got = []
    for conv in (lambda b: b, fused_ops.lora_b_chunk8):
        cd = torch.zeros((pool, 2, ps, hkv, d), dtype=dtype, device=dev)
        ups = tuple(fused_ops.LoraUp(fd, offs[m], conv(Bs[m].to(dev)), SCALE) for m in ("q", "k", "v"))
        q = fused_ops.qk_norm_rope_append(fd[:, : qd + 2 * kd], qw, qw, pos, pid, off, cd, num_qo_heads=hq,
                                          num_kv_heads=hkv, head_dim=d, page_size=ps, rope_theta=1e6, eps=1e-6,
                                          lora=ups, adapter_ids=ids)
        got.append((q, cd))
    assert torch.equal(got[0][0], got[1][0]) and torch.equal(got[0][1], got[1][1])


# One adapter bound to every token (pl_lora_up.adapter >= 0, the reference's
# single active adapter) must equal per-token ids that all name it.
@pytest.mark.parametrize("hidden,splits", [(4096, 0), (4096, 3), (12288, 0)])
def test_uniform_adapter_add_rmsnorm_bitwise(gpu_device, hidden, splits):
    rows, dev = 5, gpu_device
    g = torch.Generator().manual_seed(hidden + splits + 1)
    cols = hidden + N_ADAPTERS * RANK
    if splits:
        y = _random_split(g, splits, rows, cols, torch.bfloat16, dev)
        x = y
    else:
        y = torch.randn((rows, cols), generator=g).to(torch.bfloat16).to(dev)
        x = y[:, :hidden]
    B = (torch.randn((N_ADAPTERS, hidden, RANK), generator=g) * 0.05).to(torch.bfloat16).to(dev)
    r0 = torch.randn((rows, hidden), generator=g).to(torch.bfloat16).to(dev)
    w = (1 + 0.1 * torch.randn(hidden, generator=g)).to(torch.bfloat16).to(dev)
    ids = torch.full((rows,), 2, dtype=torch.int32, device=dev)
    r1, r2 = r0.clone(), r0.clone()
    o1 = fused_ops.add_rmsnorm(r1, x, w, 1e-6, lora=fused_ops.LoraUp(y, hidden, B, SCALE), adapter_ids=ids)
    o2 = fused_ops.add_rmsnorm(r2, x, w, 1e-6, lora=fused_ops.LoraUp(y, hidden, B, SCALE, adapter=2))
    torch.cuda.synchronize()
    assert torch.equal(r1, r2) and torch.equal(o1, o2)


def test_uniform_adapter_silu_and_qk_bitwise(gpu_device):
    rows, dev, dtype = 5, gpu_device, torch.bfloat16
    g = torch.Generator().manual_seed(91)
    ids = torch.full((rows,), 1, dtype=torch.int32, device=dev)
    inter = 1024
    full, Bs, offs = _lora_inputs(g, rows, 2 * inter, [("gate", inter), ("up", inter)], dtype)
    fd = full.to(dev)
    res = []
    for a, i in ((-1, ids), (1, None)):
        ups = tuple(fused_ops.LoraUp(fd, offs[m], Bs[m].to(dev), SCALE, a) for m in ("gate", "up"))
        res.append(fused_ops.silu_mul(fd[:, : 2 * inter], lora=ups, adapter_ids=i))
    assert torch.equal(res[0], res[1])

    hq, hkv, d, ps, pool = 8, 2, 128, 16, 10
    qd, kd = hq * d, hkv * d
    full, Bs, offs = _lora_inputs(g, rows, qd + 2 * kd, [("q", qd), ("k", kd), ("v", kd)], dtype)
    fd = full.to(dev)
    qw = torch.ones(d, dtype=dtype, device=dev)
    pos = torch.tensor([0, 17, 4095, 40000, 5], device=dev)
    pid = torch.tensor([3, 9, 0, 5, 7], device=dev)
    off = torch.tensor([0, 15, 7, 1, 2], device=dev)
    got = []
    for a, i in ((-1, ids), (1, None)):
        cd = torch.zeros((pool, 2, ps, hkv, d), dtype=dtype, device=dev)
        ups = tuple(fused_ops.LoraUp(fd, offs[m], Bs[m].to(dev), SCALE, a) for m in ("q", "k", "v"))
        q = fused_ops.qk_norm_rope_append(fd[:, : qd + 2 * kd], qw, qw, pos, pid, off, cd, num_qo_heads=hq,
                                          num_kv_heads=hkv, head_dim=d, page_size=ps, rope_theta=1e6, eps=1e-6,
                                          lora=ups, adapter_ids=i)
        got.append((q, cd))
    assert torch.equal(got[0][0], got[1][0]) and torch.equal(got[0][1], got[1][1])


def test_uniform_adapter_validation(gpu_device):
    dev = gpu_device
    x = torch.zeros((2, 64 + 3 * 16), dtype=torch.bfloat16, device=dev)
    B = torch.zeros((3, 64, 16), dtype=torch.bfloat16, device=dev)
    r = torch.zeros((2, 64), dtype=torch.bfloat16, device=dev)
    w = torch.ones(64, dtype=torch.bfloat16, device=dev)
    with pytest.raises(ValueError):   # per-token mode without ids
        fused_ops.add_rmsnorm(r, x[:, :64], w, 1e-6, lora=fused_ops.LoraUp(x, 64, B, 1.0))
    with pytest.raises(ValueError):   # bound adapter outside the stack
        fused_ops.add_rmsnorm(r, x[:, :64], w, 1e-6, lora=fused_ops.LoraUp(x, 64, B, 1.0, adapter=3))
    gu = torch.zeros((2, 2 * 64 + 2 * 3 * 16), dtype=torch.bfloat16, device=dev)
    with pytest.raises(ValueError):   # modules of one call bind different adapters
        fused_ops.silu_mul(gu[:, :128], lora=(fused_ops.LoraUp(gu, 128, B, 1.0, 0), fused_ops.LoraUp(gu, 176, B, 1.0, 1)))


@pytest.mark.parametrize("planes", [1, 3, 16, 40])
@pytest.mark.parametrize("rank", [8, 16])
@pytest.mark.parametrize("hidden", [256, 4096])
@pytest.mark.parametrize("bound", [False, True])
def test_add_rmsnorm_lora_side_planes_match_summed_y(gpu_device, planes, rank, hidden, bound):
    """pl_add_rmsnorm_lora_side (y from side planes, summed in plane order by
    the workgroup) equals pl_add_rmsnorm_lora with y = the planes' in-order sum
    rounded (SplitOutput.sum), bit for bit."""
    rows = len(IDS)
    g = torch.Generator().manual_seed(planes * 31 + rank + hidden + bound)
    side = _random_split(g, planes, rows, N_ADAPTERS * rank, torch.bfloat16, gpu_device)
    dense_y = side.sum()
    x = torch.randn((rows, hidden), generator=g).to(torch.bfloat16).to(gpu_device)
    B = (torch.randn((N_ADAPTERS, hidden, rank), generator=g) * 0.05).to(torch.bfloat16).to(gpu_device)
    r0 = torch.randn((rows, hidden), generator=g).to(torch.bfloat16).to(gpu_device)
    w = (1 + 0.1 * torch.randn(hidden, generator=g)).to(torch.bfloat16).to(gpu_device)
    ids = None if bound else torch.tensor(IDS, dtype=torch.int32, device=gpu_device)
    adapter = 2 if bound else -1
    r1, r2 = r0.clone(), r0.clone()
    out1 = fused_ops.add_rmsnorm(r1, x, w, 1e-6, lora=fused_ops.LoraUp(side, 0, B, SCALE, adapter), adapter_ids=ids)
    out2 = fused_ops.add_rmsnorm(r2, x, w, 1e-6, lora=fused_ops.LoraUp(dense_y, 0, B, SCALE, adapter),
                                 adapter_ids=ids)
    torch.cuda.synchronize()
    assert torch.equal(r1, r2) and torch.equal(out1, out2)
    assert not torch.equal(r1, r0)
