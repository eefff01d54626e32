"""Pin the element-wise oracle (norm, SiLU*up, RoPE) to library routines and
closed forms."""

import numpy as np
import torch
import torch.nn.functional as F

from oracle import fused as of


def test_rmsnorm_matches_torch_rms_norm():
    rng = np.random.default_rng(0)
    x = rng.standard_normal((5, 64)) * 3
    w = rng.standard_normal(64)
    want = F.rms_norm(torch.from_numpy(x), (64,), torch.from_numpy(w), eps=1e-6).numpy()
    np.testing.assert_allclose(of.rmsnorm(x, w, 1e-6), want, rtol=1e-12, atol=1e-12)


def test_add_rmsnorm_is_add_then_norm():
    rng = np.random.default_rng(1)
    r, x, w = rng.standard_normal((3, 32)), rng.standard_normal((3, 32)), rng.standard_normal(32)
    nr, out = of.add_rmsnorm(r, x, w, 1e-5)
    np.testing.assert_allclose(nr, r + x)
    np.testing.assert_allclose(out, of.rmsnorm(r + x, w, 1e-5))


def test_silu_mul_matches_torch():
    # the reference's own check (test_flashinfer_packed_ops.py:360-366)
    rng = np.random.default_rng(2)
    gu = rng.standard_normal((4, 10))
    g, u = torch.from_numpy(gu).chunk(2, dim=-1)
    np.testing.assert_allclose(of.silu_mul(gu), (F.silu(g) * u).numpy(), rtol=1e-12, atol=1e-12)


def test_inv_freq_matches_torch_formula():
    for d, theta in ((128, 1e6), (64, 1e4), (256, 5e5)):
        want = 1.0 / (theta ** (torch.arange(0, d, 2, dtype=torch.int64).float() / d))
        np.testing.assert_allclose(of.inv_freq_f32(d, theta), want.numpy(), rtol=2e-7)


def test_rope_closed_forms():
    rng = np.random.default_rng(3)
    x = rng.standard_normal((6, 3, 16))
    pos = np.array([0, 1, 7, 100, 4095, 32767])
    y = of.rope(x, pos, 1e4)
    # position 0 is the identity
    np.testing.assert_allclose(y[0], x[0], atol=1e-15)
    # each (i, i + D/2) pair is rotated: norms are preserved
    np.testing.assert_allclose(np.hypot(y[..., :8], y[..., 8:]), np.hypot(x[..., :8], x[..., 8:]), rtol=1e-12)
    # as complex multiplication by exp(i * angle) (independent formulation)
    inv = of.inv_freq_f32(16, 1e4).astype(np.float64)
    ang = (pos.astype(np.float32)[:, None] * of.inv_freq_f32(16, 1e4)[None]).astype(np.float64)
    z = (x[..., :8] + 1j * x[..., 8:]) * np.exp(1j * ang)[:, None, :]
    np.testing.assert_allclose(y[..., :8], z.real, atol=1e-12)
    np.testing.assert_allclose(y[..., 8:], z.imag, atol=1e-12)
    assert inv[0] == 1.0


def test_rope_scores_depend_on_relative_position():
    rng = np.random.default_rng(4)
    q, k = rng.standard_normal((1, 1, 32)), rng.standard_normal((1, 1, 32))
    s1 = (of.rope(q, [10], 1e4) * of.rope(k, [3], 1e4)).sum()
    s2 = (of.rope(q, [27], 1e4) * of.rope(k, [20], 1e4)).sum()
    np.testing.assert_allclose(s1, s2, rtol=1e-5)


def test_qk_norm_rope_append_splits_heads():
    rng = np.random.default_rng(5)
    hq, hkv, d = 4, 2, 16
    qkv = rng.standard_normal((3, (hq + 2 * hkv) * d))
    qw, kw = rng.standard_normal(d), rng.standard_normal(d)
    q, k, v = of.qk_norm_rope_append(qkv, hq, hkv, d, qw, kw, [5, 6, 7], 1e-6, 1e6)
    np.testing.assert_allclose(v, qkv[:, (hq + hkv) * d:].reshape(3, hkv, d))
    np.testing.assert_allclose(q, of.rope(of.rmsnorm(qkv[:, : hq * d].reshape(3, hq, d), qw, 1e-6), [5, 6, 7], 1e6))
