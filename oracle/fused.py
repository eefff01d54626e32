"""float64 numpy restatement of the decode layer's element-wise ops.

  rmsnorm        model/flashinfer/norm.py:15-24, 60-65 (FlashInfer rmsnorm:
                 x * rsqrt(mean(x^2) + eps) * w)
  add_rmsnorm    norm.py:27-57 (residual = residual + x, then rmsnorm)
  silu_mul       packed_ops.py:230-239 (silu(gate) * up on the halves of gate_up)
  rope           projection.py:155-190 (apply_rope_pos_ids, non-interleaved:
                 x*cos + rotate_half(x)*sin, angle = pos / scale * theta^(-2i/D),
                 _rope_theta/_rope_scale :280-296)
  head_norm      projection.py:248-260 (per-head RMSNorm over head_dim)
  qk_norm_rope_append  head_norm + rope on q and k, then the decode append
                 of layer_runner.py:399-412

Test infrastructure only.
"""

from __future__ import annotations

import numpy as np


def _f64(a):
    return np.asarray(a).astype(np.float64, copy=False)


def rmsnorm(x, w, eps):
    x = _f64(x)
    return x / np.sqrt((x * x).mean(-1, keepdims=True) + eps) * _f64(w)


def add_rmsnorm(residual, x, w, eps, round_sum=None):
    """Returns (new residual, normed).  ``round_sum`` rounds the stored sum
    (the residual is kept in the model dtype)."""
    r = _f64(residual) + _f64(x)
    if round_sum is not None:
        r = round_sum(r)
    return r, rmsnorm(r, w, eps)


def silu_mul(gate_up):
    gu = _f64(gate_up)
    half = gu.shape[-1] // 2
    g, u = gu[..., :half], gu[..., half:]
    return g / (1.0 + np.exp(-g)) * u


def inv_freq_f32(d, theta, scale=1.0):
    """The reference's fp32 inverse frequencies: 1 / theta^(arange(0, d, 2)/d), / scale."""
    e = np.arange(0, d, 2, dtype=np.float32) / np.float32(d)
    inv = np.float32(1.0) / np.power(np.float32(theta), e, dtype=np.float32)
    return (inv / np.float32(scale)).astype(np.float32)


def rope(x, positions, theta, scale=1.0, inv_freq=None):
    """x [T, H, D], positions [T].  The angle is the fp32 product
    position * inv_freq (as the reference forms it); cos/sin in float64."""
    x = _f64(x)
    d = x.shape[-1]
    inv = inv_freq_f32(d, theta, scale) if inv_freq is None else np.asarray(inv_freq, dtype=np.float32)
    ang = (np.asarray(positions, dtype=np.float32)[:, None] * inv[None, :]).astype(np.float64)
    cos, sin = np.cos(ang)[:, None, :], np.sin(ang)[:, None, :]
    x1, x2 = x[..., : d // 2], x[..., d // 2:]
    return np.concatenate([x1 * cos - x2 * sin, x2 * cos + x1 * sin], axis=-1)


def qk_norm_rope_append(qkv, hq, hkv, d, q_norm_w, k_norm_w, positions, eps, theta, scale=1.0, inv_freq=None):
    """Returns (q [T, hq, d], k [T, hkv, d], v [T, hkv, d]) as written."""
    qkv = _f64(qkv)
    T = qkv.shape[0]
    q = qkv[:, : hq * d].reshape(T, hq, d)
    k = qkv[:, hq * d: (hq + hkv) * d].reshape(T, hkv, d)
    v = qkv[:, (hq + hkv) * d: (hq + 2 * hkv) * d].reshape(T, hkv, d)
    if q_norm_w is not None:
        q = rmsnorm(q, q_norm_w, eps)
    if k_norm_w is not None:
        k = rmsnorm(k, k_norm_w, eps)
    return rope(q, positions, theta, scale, inv_freq), rope(k, positions, theta, scale, inv_freq), v
