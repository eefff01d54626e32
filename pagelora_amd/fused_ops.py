"""Python entry points of the fused element-wise decode kernels.

``rmsnorm`` / ``add_rmsnorm`` replace the reference's ``apply_rmsnorm`` and
``add_residual_rmsnorm`` (model/flashinfer/norm.py:15-65), ``silu_mul`` its
``apply_gate_up_activation`` (packed_ops.py:230-239), and
``qk_norm_rope_append`` fuses the q/k head norm and RoPE of
``project_qkv_with_optional_norm`` (projection.py:34-190, 248-260) with the
decode token's page append (layer_runner.py:399-412).
"""

from __future__ import annotations

import ctypes
from dataclasses import dataclass
from typing import Sequence

import torch

from . import _lib
from .attention_backend import _cache_geometry
from .linear import SplitOutput


def _rows2d(t: torch.Tensor, name: str) -> None:
    if t.dim() != 2 or t.stride(1) != 1:
        raise ValueError(f"{name} must be 2-D with unit column stride")


def lora_b_chunk8(B: torch.Tensor) -> torch.Tensor:
    """B [n, out, r] (or [out, r]) in the consumer-coalesced layout
    PL_LORA_B_CHUNK8: [n, nblk, 8, r/8, 64, 8] with nblk = ceil(out/512) and
    element (a, j, i, k, l, e) = B[a][8(64j + l) + i][8k + e], zero past
    ``out``.  A wave whose threads own 8 output columns each reads its block
    as one contiguous region, each load instruction 1 KiB contiguous."""
    B3 = B if B.dim() == 3 else B.unsqueeze(0)
    n, out, r = B3.shape
    if out % 8 or r % 8:
        raise ValueError("chunked LoRA B needs out_features and rank multiples of 8")
    nblk = -(-out // 512)
    padded = B3.new_zeros((n, nblk * 512, r))
    padded[:, :out] = B3
    # [n, j, l, i, k, e] -> [n, j, i, k, l, e]
    return padded.reshape(n, nblk, 64, 8, r // 8, 8).permute(0, 1, 3, 4, 2, 5).contiguous()


@dataclass
class LoraUp:
    """The up-projection half of a no-merge LoRA module, applied by the kernel
    that consumes the module's output (``pl_lora_up``).

    ``y`` is the producer GEMM's output row block ``[T, *]`` (a GEMM on the
    base weight with the adapters' A rows stacked under it); adapter a's
    rank-space intermediate sits at columns ``y_offset + a*r .. + r``.  ``B``
    is ``[n_adapters, out, r]`` (row-major) or the same values from
    :func:`lora_b_chunk8` (5-D, the layout the kernels read fastest).  The
    module output is ``round(base + scale * y[a] . B[a]^T)``
    (multilora/linear.py:226-231).
    """

    y: "torch.Tensor | SplitOutput"
    y_offset: int
    B: torch.Tensor
    scale: float
    # >= 0: every token uses this adapter (the reference's one bound adapter
    # per batch) and adapter_ids may be omitted; -1: per-token adapter_ids
    adapter: int = -1

    def _b_shape(self) -> tuple[int, int, int, int]:
        """(n_adapters, out_features, rank, b_layout)."""
        B = self.B
        if B.dim() == 6:
            # padded to whole 512-column blocks: the pad holds zeros and the
            # kernels read only the columns they are asked for
            n, nblk, eight, rk, lanes, e = B.shape
            if eight != 8 or lanes != 64 or e != 8:
                raise ValueError("a 6-D LoraUp.B must be lora_b_chunk8 output [n, ceil(out/512), 8, r/8, 64, 8]")
            return n, nblk * 512, rk * 8, _lib.PL_LORA_B_CHUNK8
        B3 = B if B.dim() == 3 else B.unsqueeze(0)
        return B3.shape[0], B3.shape[1], B3.shape[2], _lib.PL_LORA_B_ROWS

    def struct(self) -> "_lib.LoraUp":
        n, out, r, layout = self._b_shape()
        B = self.B
        if isinstance(self.y, SplitOutput):  # read from the split planes by the kernel
            if not B.is_contiguous() or B.dtype != self.y.dtype:
                raise ValueError("LoraUp.B must be contiguous and of the model dtype")
            if self.y_offset < 0 or self.y_offset + n * r > self.y.ld:
                raise ValueError("LoraUp: y columns out of range")
            return _lib.LoraUp(None, 0, int(self.y_offset), B.data_ptr(), int(out), int(r), float(self.scale),
                               int(layout), int(self.adapter))
        if self.y.dim() != 2 or self.y.stride(1) != 1:
            raise ValueError("LoraUp.y must be 2-D with unit column stride")
        if not B.is_contiguous() or B.dtype != self.y.dtype:
            raise ValueError("LoraUp.B must be contiguous and of y's dtype")
        if self.y_offset < 0 or self.y_offset + n * r > self.y.shape[1]:
            raise ValueError("LoraUp: y columns out of range")
        return _lib.LoraUp(self.y.data_ptr(), self.y.stride(0), int(self.y_offset), B.data_ptr(), int(out), int(r),
                           float(self.scale), int(layout), int(self.adapter))

    @property
    def n_adapters(self) -> int:
        return self._b_shape()[0]


def _lora_args(lora: Sequence[LoraUp], adapter_ids: torch.Tensor | None, rows: int):
    n = lora[0].n_adapters
    if any(m.n_adapters != n for m in lora):
        raise ValueError("every LoRA module of a call must stack the same adapters")
    bound = lora[0].adapter
    if any(m.adapter != bound for m in lora):
        raise ValueError("every LoRA module of a call must bind the same adapter")
    if bound >= n or bound < -1:
        raise ValueError(f"adapter {bound} outside [-1, {n})")
    if bound < 0 and adapter_ids is None:
        raise ValueError("adapter_ids is required unless the modules bind one adapter")
    if adapter_ids is not None and (adapter_ids.dtype != torch.int32 or adapter_ids.numel() != rows):
        raise ValueError("adapter_ids must be int32 [rows]")
    for m in lora:
        y_rows = m.y.rows if isinstance(m.y, SplitOutput) else m.y.shape[0]
        if y_rows != rows:
            raise ValueError("LoraUp.y must have one row per token")
    arr = (_lib.LoraUp * len(lora))(*[m.struct() for m in lora])
    return arr, (adapter_ids.data_ptr() if adapter_ids is not None else None), n


def rmsnorm(x: torch.Tensor, weight: torch.Tensor, eps: float, out: torch.Tensor | None = None) -> torch.Tensor:
    _rows2d(x, "x")
    out = torch.empty_like(x) if out is None else out
    _rows2d(out, "out")
    if weight.numel() != x.shape[1] or weight.dtype != x.dtype or out.dtype != x.dtype:
        raise ValueError("weight/out must match x")
    lib = _lib.load()
    _lib.check(lib.pl_rmsnorm(x.data_ptr(), x.stride(0), weight.data_ptr(), out.data_ptr(), out.stride(0),
                              x.shape[0], x.shape[1], float(eps), _lib.dtype_code(x.dtype),
                              _lib.stream_handle(x.device)), "pl_rmsnorm")
    return out


def add_rmsnorm(residual: torch.Tensor, x: "torch.Tensor | SplitOutput", weight: torch.Tensor, eps: float,
                out: torch.Tensor | None = None, *, lora: LoraUp | None = None,
                adapter_ids: torch.Tensor | None = None) -> torch.Tensor:
    """In place ``residual += x``; returns ``rmsnorm(residual)``.

    With ``lora``, x is the base output of the module whose up-projection
    ``lora`` describes: ``residual += round(x + delta)`` (pl_add_rmsnorm_lora).
    x may then also be a :class:`SplitOutput` (split-K planes summed here),
    or x a tensor and ``lora.y`` the side planes of
    :func:`linear.linear_shuffled_side` (pl_add_rmsnorm_lora_side).
    """
    _rows2d(residual, "residual")
    rows, hidden = residual.shape
    split = isinstance(x, SplitOutput)
    if split:
        if lora is None:
            raise ValueError("a split-K input needs the module's lora")
        if x.rows != rows or x.out_features < hidden or x.dtype != residual.dtype:
            raise ValueError("x must match residual")
    else:
        _rows2d(x, "x")
        if x.shape != residual.shape or x.dtype != residual.dtype:
            raise ValueError("x must match residual")
    out = torch.empty_like(residual) if out is None else out
    lib = _lib.load()
    if lora is not None and not split and isinstance(lora.y, SplitOutput):
        # y from the side planes of linear_shuffled_side, x whole
        arr, ids, n = _lora_args([lora], adapter_ids, rows)
        _lib.check(lib.pl_add_rmsnorm_lora_side(residual.data_ptr(), residual.stride(0), x.data_ptr(), x.stride(0),
                                                ctypes.byref(lora.y.struct()), arr, ids, n, weight.data_ptr(),
                                                out.data_ptr(), out.stride(0), rows, hidden, float(eps),
                                                _lib.dtype_code(residual.dtype), _lib.stream_handle(residual.device)),
                   "pl_add_rmsnorm_lora_side")
        return out
    if lora is not None:
        arr, ids, n = _lora_args([lora], adapter_ids, rows)
        xs = ctypes.byref(x.struct()) if split else None
        _lib.check(lib.pl_add_rmsnorm_lora(residual.data_ptr(), residual.stride(0), None if split else x.data_ptr(),
                                           0 if split else x.stride(0), xs, arr, ids, n, weight.data_ptr(),
                                           out.data_ptr(), out.stride(0), rows, hidden, float(eps),
                                           _lib.dtype_code(residual.dtype), _lib.stream_handle(residual.device)),
                   "pl_add_rmsnorm_lora")
        return out
    _lib.check(lib.pl_add_rmsnorm(residual.data_ptr(), residual.stride(0), x.data_ptr(), x.stride(0),
                                  weight.data_ptr(), out.data_ptr(), out.stride(0), rows, hidden, float(eps),
                                  _lib.dtype_code(x.dtype), _lib.stream_handle(x.device)), "pl_add_rmsnorm")
    return out


def silu_mul(gate_up: torch.Tensor, out: torch.Tensor | None = None, *,
             lora: Sequence[LoraUp] | None = None, adapter_ids: torch.Tensor | None = None,
             down_shrink=None) -> torch.Tensor:
    """``silu(gate) * up`` of a packed ``[T, 2*inter]`` row block; with ``lora``
    (gate, up) the modules' LoRA deltas are added first (pl_silu_mul_lora).
    ``down_shrink`` = (``_lib.LoraARows`` of down_proj, ``linear.LoraPartials``
    [T, ceil(inter / 256), rank]): the kernel also writes down_proj's LoRA
    shrink partials of the output (pl_silu_mul_lora_shrink)."""
    _rows2d(gate_up, "gate_up")
    inter = gate_up.shape[1] // 2
    if gate_up.shape[1] != 2 * inter:
        raise ValueError("gate_up must have an even number of columns")
    out = torch.empty((gate_up.shape[0], inter), dtype=gate_up.dtype, device=gate_up.device) if out is None else out
    lib = _lib.load()
    rows = gate_up.shape[0]
    if down_shrink is not None:
        if lora is None or len(lora) != 2:
            raise ValueError("the down_proj shrink comes with the gate / up LoRA")
        arr, ids, n = _lora_args(lora, adapter_ids, rows)
        a_rows, parts = down_shrink
        if parts.partials.shape[0] != rows:
            raise ValueError("down_proj partials must have one row per token")
        p = parts.struct()
        _lib.check(lib.pl_silu_mul_lora_shrink(gate_up.data_ptr(), gate_up.stride(0), arr, ids, n, out.data_ptr(),
                                               out.stride(0), rows, inter, ctypes.byref(a_rows), ctypes.byref(p),
                                               _lib.dtype_code(gate_up.dtype), _lib.stream_handle(gate_up.device)),
                   "pl_silu_mul_lora_shrink")
        return out
    if lora is not None:
        if len(lora) != 2:
            raise ValueError("lora must be (gate, up)")
        arr, ids, n = _lora_args(lora, adapter_ids, rows)
        _lib.check(lib.pl_silu_mul_lora(gate_up.data_ptr(), gate_up.stride(0), arr, ids, n, out.data_ptr(),
                                        out.stride(0), rows, inter, _lib.dtype_code(gate_up.dtype),
                                        _lib.stream_handle(gate_up.device)), "pl_silu_mul_lora")
        return out
    _lib.check(lib.pl_silu_mul(gate_up.data_ptr(), gate_up.stride(0), out.data_ptr(), out.stride(0),
                               rows, inter, _lib.dtype_code(gate_up.dtype),
                               _lib.stream_handle(gate_up.device)), "pl_silu_mul")
    return out


_INV_FREQ: dict = {}


def rope_inv_freq(head_dim: int, theta: float, scale: float, device) -> torch.Tensor:
    """fp32 inverse frequencies as the reference's RoPE forms them
    (1 / theta^(arange(0, D, 2) / D), then / scale for linear scaling)."""
    key = (head_dim, float(theta), float(scale), str(device))
    t = _INV_FREQ.get(key)
    if t is None:
        t = 1.0 / (float(theta) ** (torch.arange(0, head_dim, 2, dtype=torch.int64).float() / head_dim))
        t = (t / float(scale)).to(device)
        _INV_FREQ[key] = t
    return t


def rope_cos_sin(positions: torch.Tensor, *, head_dim: int, rope_theta: float, rope_scale: float = 1.0,
                 out: torch.Tensor | None = None) -> torch.Tensor:
    """``[B, head_dim/2, 2]`` fp32: cos and sin of ``positions[b] * inv_freq[i]``
    (pl_rope_cos_sin) -- the RoPE angles every layer of one decode step shares,
    for :meth:`PagedDecodeAttention.run_decode_qkv_into`."""
    if positions.dtype != torch.int64 or positions.dim() != 1:
        raise ValueError("positions must be int64 [B]")
    B, half = positions.numel(), head_dim // 2
    out = torch.empty((B, half, 2), dtype=torch.float32, device=positions.device) if out is None else out
    if out.dtype != torch.float32 or tuple(out.shape) != (B, half, 2) or not out.is_contiguous():
        raise ValueError(f"out must be a contiguous fp32 [{B}, {half}, 2] tensor")
    inv_freq = rope_inv_freq(head_dim, rope_theta, rope_scale, positions.device)
    lib = _lib.load()
    _lib.check(lib.pl_rope_cos_sin(positions.data_ptr(), B, inv_freq.data_ptr(), half, out.data_ptr(),
                                   _lib.stream_handle(positions.device)), "pl_rope_cos_sin")
    return out


def qk_norm_rope_append(
    qkv: torch.Tensor,
    q_norm_weight: torch.Tensor | None,
    k_norm_weight: torch.Tensor | None,
    positions: torch.Tensor,
    page_id: torch.Tensor,
    page_offset: torch.Tensor,
    cache_layer,
    *,
    num_qo_heads: int,
    num_kv_heads: int,
    head_dim: int,
    page_size: int,
    rope_theta: float,
    rope_scale: float = 1.0,
    eps: float = 1e-6,
    q_out: torch.Tensor | None = None,
    lora: Sequence[LoraUp] | None = None,
    adapter_ids: torch.Tensor | None = None,
) -> torch.Tensor:
    """Returns the rotated q [B, Hq, D]; writes rotated k and v into the pages.

    With ``lora`` (q, k, v) the modules' LoRA deltas are added to the packed
    row first (pl_qk_norm_rope_append_lora); qkv may then also be a
    :class:`SplitOutput` (split-K planes summed here).
    """
    split = isinstance(qkv, SplitOutput)
    if split:
        if lora is None:
            raise ValueError("a split-K input needs the modules' lora")
        B = qkv.rows
    else:
        _rows2d(qkv, "qkv")
        B = qkv.shape[0]
    kc, vc, page_stride, token_stride, head_stride, num_pages = _cache_geometry(
        cache_layer, num_kv_heads, head_dim, page_size)
    if kc.dtype != qkv.dtype:
        raise ValueError("qkv dtype must match the KV cache")
    if split and qkv.out_features < (num_qo_heads + 2 * num_kv_heads) * head_dim:
        raise ValueError("qkv has fewer columns than q|k|v")
    for t, n in ((positions, "positions"), (page_id, "page_id"), (page_offset, "page_offset")):
        if t.dtype != torch.int64 or t.numel() != B:
            raise ValueError(f"{n} must be int64 [B]")
    q_out = torch.empty((B, num_qo_heads, head_dim), dtype=qkv.dtype, device=qkv.device) if q_out is None else q_out
    inv_freq = rope_inv_freq(head_dim, rope_theta, rope_scale, qkv.device)
    lib = _lib.load()
    if lora is not None:
        if len(lora) != 3:
            raise ValueError("lora must be (q, k, v)")
        arr, ids, n = _lora_args(lora, adapter_ids, B)
        _lib.check(lib.pl_qk_norm_rope_append_lora(
            None if split else qkv.data_ptr(), 0 if split else qkv.stride(0),
            ctypes.byref(qkv.struct()) if split else None, arr, ids, n,
            q_norm_weight.data_ptr() if q_norm_weight is not None else None,
            k_norm_weight.data_ptr() if k_norm_weight is not None else None,
            positions.data_ptr(), page_id.data_ptr(), page_offset.data_ptr(),
            q_out.data_ptr(), kc.data_ptr(), vc.data_ptr(), page_stride, token_stride, head_stride,
            num_pages, page_size, B, num_qo_heads, num_kv_heads, head_dim,
            inv_freq.data_ptr(), float(eps), _lib.dtype_code(qkv.dtype),
            _lib.stream_handle(qkv.device)), "pl_qk_norm_rope_append_lora")
        return q_out
    _lib.check(lib.pl_qk_norm_rope_append(
        qkv.data_ptr(), qkv.stride(0),
        q_norm_weight.data_ptr() if q_norm_weight is not None else None,
        k_norm_weight.data_ptr() if k_norm_weight is not None else None,
        positions.data_ptr(), page_id.data_ptr(), page_offset.data_ptr(),
        q_out.data_ptr(), kc.data_ptr(), vc.data_ptr(), page_stride, token_stride, head_stride,
        num_pages, page_size, B, num_qo_heads, num_kv_heads, head_dim,
        inv_freq.data_ptr(), float(eps), _lib.dtype_code(qkv.dtype),
        _lib.stream_handle(qkv.device)), "pl_qk_norm_rope_append")
    return q_out


def greedy_argmax(logits: torch.Tensor, out: torch.Tensor | None = None,
                  tokens_out: torch.Tensor | None = None, workspace: torch.Tensor | None = None) -> torch.Tensor:
    """``torch.argmax(logits, dim=-1)`` for 2-D logits on the device (``pl_greedy_argmax``):
    the first maximal index per row, a NaN counting as the largest value
    (sampling.py:8-15).  ``tokens_out`` (int64 [rows], optional) receives the
    same indices: the next decode step's input-token buffer.  ``workspace``
    (uint8, optional; see :func:`greedy_argmax_workspace`) holds the
    per-slice maxima."""
    _rows2d(logits, "logits")
    rows, vocab = logits.shape
    lib = _lib.load()
    if out is None:
        out = torch.empty(rows, dtype=torch.int64, device=logits.device)
    for name, t in (("out", out), ("tokens_out", tokens_out)):
        if t is not None and (t.dtype != torch.int64 or t.numel() != rows or not t.is_contiguous()):
            raise ValueError(f"{name} must be a contiguous int64 tensor of {rows} elements")
    if workspace is None:
        workspace = greedy_argmax_workspace(rows, vocab, logits.dtype, logits.device)
    st = lib.pl_greedy_argmax(logits.data_ptr(), logits.stride(0), rows, vocab, _lib.dtype_code(logits.dtype),
                              out.data_ptr(), tokens_out.data_ptr() if tokens_out is not None else None,
                              workspace.data_ptr(), workspace.numel(), _lib.stream_handle(logits.device))
    _lib.check(st, "pl_greedy_argmax")
    return out


def greedy_argmax_workspace(rows: int, vocab: int, dtype: torch.dtype, device) -> torch.Tensor:
    """A workspace for :func:`greedy_argmax` on [rows, vocab] logits of ``dtype``."""
    n = _lib.load().pl_greedy_argmax_workspace_size(rows, vocab, _lib.dtype_code(dtype))
    return torch.empty(max(int(n), 8), dtype=torch.uint8, device=device)
