"""float64 numpy restatement of the no-merge LoRA delta and its merged comparator.

Reference formulas:
  LoRALinear.forward (multilora/linear.py:200-231), serve role, eval dropout:
      y = x W^T + b + (x A^T) B^T * scale,   scale = alpha / rank (linear.py:41, 71)
  _lora_delta (model/flashinfer/packed_ops.py:534-553): the delta term alone.
  _cached_packed_lora_delta (packed_ops.py:328-384): A_cat = concat_rows(A_i),
      B_bd = block_diag(scale_i * B_i); delta = (x A_cat^T) B_bd^T (:314-325).
  merged comparator: W_eff = W + scale * B A (linear.py:166-172,
      effective_weights.py:53-75, 78-129), y = x W_eff^T + b.
Multi-adapter: token t uses adapter ids[t]'s A/B (no reference counterpart:
the reference binds one adapter at a time, multilora/runtime.py:138-174);
tokens with ids outside [0, n) get no delta.

Test infrastructure only.
"""

from __future__ import annotations

import numpy as np


def _f64(a):
    return np.asarray(a).astype(np.float64, copy=False)


def round_bf16(a):
    """Round to the nearest bfloat16 (ties to even), returned as float64."""
    f = np.asarray(a, dtype=np.float32)
    u = f.view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) & 0xFFFF0000
    out = u.astype(np.uint32).view(np.float32).astype(np.float64)
    return np.where(np.isnan(f), np.nan, out)


def round_to(a, dtype):
    """Round float64 values to the storage type `dtype` ("bf16", "f16" or None)."""
    if dtype is None:
        return _f64(a)
    if dtype == "bf16":
        return round_bf16(a)
    if dtype == "f16":
        return np.asarray(a, dtype=np.float64).astype(np.float16).astype(np.float64)
    raise ValueError(dtype)


def linear(x, w):
    """F.linear without bias: x W^T (the base projection and the LoRA shrink)."""
    return _f64(x) @ _f64(w).T


def up_projection(down, b, scale):
    """The expand half of the delta: down B^T * scale (packed_ops.py:324-325,
    multilora/linear.py:227-228), for the rank-space intermediate ``down``."""
    return _f64(down) @ _f64(b).T * scale


def lora_delta(x, a, b, scale, intermediate=None):
    """(x A^T) B^T * scale for x [T, in], A [r, in], B [out, r].

    ``intermediate`` ("bf16" / "f16") rounds x A^T to that type first, as the
    reference's ``down = F.linear(x, A)`` returns it in the model dtype
    (packed_ops.py:324, 551; multilora/linear.py:227).
    """
    down = round_to(linear(x, a), intermediate)
    return up_projection(down, b, scale)


def lora_linear(x, w, bias, a, b, scale):
    """LoRALinear.forward in serve mode: x W^T + b + delta."""
    y = _f64(x) @ _f64(w).T
    if bias is not None:
        y = y + _f64(bias)
    return y + lora_delta(x, a, b, scale)


def merged_linear(x, w, bias, a, b, scale):
    """x (W + scale * B A)^T + b: the merged / effective-weights path."""
    w_eff = _f64(w) + scale * (_f64(b) @ _f64(a))
    y = _f64(x) @ w_eff.T
    if bias is not None:
        y = y + _f64(bias)
    return y


def pack_lora(mods):
    """Packed (A_cat [sum r, in], B_bd [sum out, sum r]) for [(A, B, scale), ...]."""
    a_cat = np.concatenate([_f64(a) for a, _, _ in mods], axis=0)
    outs = [np.asarray(b).shape[0] for _, b, _ in mods]
    ranks = [np.asarray(a).shape[0] for a, _, _ in mods]
    b_bd = np.zeros((sum(outs), sum(ranks)))
    oo = ro = 0
    for (a, b, s), o, r in zip(mods, outs, ranks):
        b_bd[oo:oo + o, ro:ro + r] = _f64(b) * s
        oo += o
        ro += r
    return a_cat, b_bd


def packed_lora_delta(x, mods):
    """delta for a packed group: (x A_cat^T) B_bd^T (packed_ops.py:314-325)."""
    a_cat, b_bd = pack_lora(mods)
    return (_f64(x) @ a_cat.T) @ b_bd.T


def multi_adapter_delta(x, ids, a_stack, b_stack, scale, intermediate=None):
    """Per-token adapter: row t gets (x_t A[ids[t]]^T) B[ids[t]]^T * scale.

    a_stack [n, r, in], b_stack [n, out, r]; rows with ids outside [0, n) are 0.
    ``intermediate`` as in lora_delta.
    """
    x = _f64(x)
    n = a_stack.shape[0]
    out = np.zeros((x.shape[0], b_stack.shape[1]))
    for t, a_id in enumerate(ids):
        if 0 <= a_id < n:
            down = round_to(x[t] @ _f64(a_stack[a_id]).T, intermediate)
            out[t] = down @ _f64(b_stack[a_id]).T * scale
    return out
