"""No-merge LoRA delta on the gfx950 shrink/expand kernels.

``lora_delta_`` adds ``scale_m * B_m[a_t] . (A_m[a_t] . x_t)`` to the output
of every module m of a group sharing the input x, in place, for per-token
adapter ids ``a_t`` -- the delta term of the reference's no-merge path:

* packed q/k/v and gate/up: ``_packed_lora_delta`` / ``_cached_packed_lora_delta``
  (model/flashinfer/packed_ops.py:314-384) build ``A_cat`` and a block-diagonal
  ``B_bd`` with the scale folded in and run two ``F.linear``;
* o_proj / down_proj: ``LoRALinear.forward`` (multilora/linear.py:200-231) and
  ``_lora_delta`` (packed_ops.py:534-553).

Here one shrink launch reads x once for the whole group and one expand
launch accumulates every module's delta straight into its base output; the
block-diagonal zeros are never stored or read.  ``lora_delta_groups_`` runs
up to four groups with their own inputs in the same two launches.  Adapter
selection is per token (the reference binds one adapter for the whole
batch, multilora/runtime.py:138-174; a single adapter is the case
``ids == 0``).
"""

from __future__ import annotations

import ctypes
from typing import Sequence

import torch

from . import _lib

_WS: dict[int, torch.Tensor] = {}


def _workspace(device: torch.device, nbytes: int) -> torch.Tensor:
    """Per-device workspace for the shrink's partial sums, grown (never
    shrunk) on demand -- never inside a captured graph."""
    key = device.index if device.index is not None else torch.cuda.current_device()
    ws = _WS.get(key)
    if ws is None or ws.numel() < nbytes:
        if torch.cuda.is_current_stream_capturing():
            raise RuntimeError("LoRA workspace must be sized before graph capture (call reserve_workspace)")
        size = max(nbytes, 1 << 20)
        ws = torch.empty(size, dtype=torch.uint8, device=device)
        _WS[key] = ws
    return ws


def reserve_workspace(device: torch.device | str, nbytes: int) -> None:
    """Allocate ``nbytes`` of workspace ahead of a (possibly captured) call."""
    _workspace(torch.device(device), nbytes)


_DELTA_WS: dict[int, torch.Tensor] = {}


def _delta_workspace(device: torch.device, nbytes: int) -> torch.Tensor:
    """Per-device workspace of pl_lora_delta(_groups): zero-filled when
    allocated (its ticket area must start at zero; every call leaves it so)
    and used by no other entry point; grown on demand, never inside a
    captured graph."""
    key = device.index if device.index is not None else torch.cuda.current_device()
    ws = _DELTA_WS.get(key)
    if ws is None or ws.numel() < nbytes:
        if torch.cuda.is_current_stream_capturing():
            raise RuntimeError("LoRA workspace must be sized before graph capture (call reserve_delta_workspace)")
        ws = torch.zeros(max(nbytes, 1 << 20), dtype=torch.uint8, device=device)
        _DELTA_WS[key] = ws
    return ws


def reserve_delta_workspace(device: torch.device | str, nbytes: int) -> None:
    """Allocate ``nbytes`` of lora_delta_ workspace ahead of a captured call."""
    _delta_workspace(torch.device(device), nbytes)


def _module_structs(modules, x: torch.Tensor):
    """ctypes array of pl_lora_module for [(A, B, out, scale), ...]."""
    n = len(modules)
    if not 1 <= n <= _lib.PL_LORA_MAX_MODULES:
        raise ValueError(f"a LoRA group holds 1..{_lib.PL_LORA_MAX_MODULES} modules, got {n}")
    arr = (_lib.LoraModule * n)()
    n_adapters = None
    out_dtype = None
    for i, (A, B, out, scale) in enumerate(modules):
        if A.dim() == 2:
            A = A.unsqueeze(0)
        if B.dim() == 2:
            B = B.unsqueeze(0)
        if A.dim() != 3 or B.dim() != 3:
            raise ValueError("A must be [adapters, rank, in] and B [adapters, out, rank]")
        na, r, fin = A.shape
        nb, fout, rb = B.shape
        if na != nb or rb != r or fin != x.shape[1]:
            raise ValueError(f"module {i}: A {tuple(A.shape)} / B {tuple(B.shape)} do not match x {tuple(x.shape)}")
        if not (A.is_contiguous() and B.is_contiguous()):
            raise ValueError(f"module {i}: A and B must be contiguous")
        if A.dtype != x.dtype or B.dtype != x.dtype:
            raise ValueError(f"module {i}: A/B dtype must equal x dtype {x.dtype}")
        if out.dim() != 2 or out.shape[0] != x.shape[0] or out.shape[1] != fout or out.stride(1) != 1:
            raise ValueError(f"module {i}: out must be [T, {fout}] with unit column stride")
        if n_adapters is None:
            n_adapters, out_dtype = na, out.dtype
        elif na != n_adapters or out.dtype != out_dtype:
            raise ValueError("all modules of a group need the same adapter count and output dtype")
        for t in (A, B, out):
            if t.device != x.device:
                raise ValueError("x, A, B and out must be on one device")
        arr[i].A, arr[i].B, arr[i].out = A.data_ptr(), B.data_ptr(), out.data_ptr()
        arr[i].ldo, arr[i].out_features, arr[i].rank, arr[i].scale = out.stride(0), fout, r, float(scale)
    return arr, n_adapters, out_dtype


def lora_delta_(
    x: torch.Tensor,
    modules: Sequence[tuple[torch.Tensor, torch.Tensor, torch.Tensor, float]],
    adapter_ids: torch.Tensor,
) -> None:
    """In place: ``out += scale * B[ids] . (A[ids] . x)`` for each ``(A, B, out, scale)``.

    x: [T, in] (bf16 or fp16, unit column stride); A: [adapters, r, in] or
    [r, in]; B: [adapters, out, r] or [out, r]; out: [T, out] view of the
    base projection output (bf16, fp16 or fp32); adapter_ids: int32 [T] on
    the device (negative = no adapter).
    """
    if x.dim() != 2 or x.stride(1) != 1:
        raise ValueError("x must be [T, in] with unit column stride")
    if adapter_ids.dtype != torch.int32 or adapter_ids.numel() != x.shape[0] or adapter_ids.device != x.device:
        raise ValueError("adapter_ids must be int32 [T] on x's device")
    if x.shape[0] == 0:
        return
    arr, n_adapters, out_dtype = _module_structs(modules, x)
    lib = _lib.load()
    n = len(modules)
    grp = _lib.LoraGroup(x.data_ptr(), x.stride(0), x.shape[1], n, arr)
    nbytes = lib.pl_lora_delta_workspace_size(ctypes.byref(grp), 1, x.shape[0], n_adapters)
    if nbytes == 0:
        raise ValueError(f"invalid LoRA group: {_lib.last_error()}")
    ws = _delta_workspace(x.device, nbytes)
    status = lib.pl_lora_delta(
        x.data_ptr(), x.stride(0), x.shape[0], x.shape[1], arr, n,
        adapter_ids.data_ptr(), n_adapters, _lib.dtype_code(x.dtype), _lib.dtype_code(out_dtype),
        ws.data_ptr(), ws.numel(), _lib.stream_handle(x.device),
    )
    _lib.check(status, "pl_lora_delta")


def lora_delta_groups_(
    groups: Sequence[tuple[torch.Tensor, Sequence[tuple[torch.Tensor, torch.Tensor, torch.Tensor, float]]]],
    adapter_ids: torch.Tensor,
) -> None:
    """``lora_delta_`` for up to four groups ``(x, modules)`` with their own
    inputs and the same per-token adapter ids, in one pair of launches at
    decode sizes.  Every x has the same token count and dtype; groups must
    not write the same outputs."""
    if not 1 <= len(groups) <= _lib.PL_LORA_MAX_GROUPS:
        raise ValueError(f"1..{_lib.PL_LORA_MAX_GROUPS} groups, got {len(groups)}")
    x0 = groups[0][0]
    T = x0.shape[0]
    if adapter_ids.dtype != torch.int32 or adapter_ids.numel() != T or adapter_ids.device != x0.device:
        raise ValueError("adapter_ids must be int32 [T] on the inputs' device")
    descs = (_lib.LoraGroup * len(groups))()
    keep = []
    n_adapters = out_dtype = None
    for i, (x, modules) in enumerate(groups):
        if x.dim() != 2 or x.stride(1) != 1 or x.shape[0] != T or x.dtype != x0.dtype or x.device != x0.device:
            raise ValueError(f"group {i}: x must be [{T}, in] with unit column stride, {x0.dtype} on {x0.device}")
        arr, na, od = _module_structs(modules, x)
        if n_adapters is None:
            n_adapters, out_dtype = na, od
        elif na != n_adapters or od != out_dtype:
            raise ValueError("all groups need the same adapter count and output dtype")
        keep.append(arr)
        descs[i].x, descs[i].ldx, descs[i].in_features = x.data_ptr(), x.stride(0), x.shape[1]
        descs[i].num_modules, descs[i].modules = len(modules), arr
    if T == 0:
        return
    lib = _lib.load()
    nbytes = lib.pl_lora_delta_workspace_size(descs, len(groups), T, n_adapters)
    if nbytes == 0:
        raise ValueError(f"invalid LoRA groups: {_lib.last_error()}")
    ws = _delta_workspace(x0.device, nbytes)
    status = lib.pl_lora_delta_groups(
        descs, len(groups), T, adapter_ids.data_ptr(), n_adapters, _lib.dtype_code(x0.dtype),
        _lib.dtype_code(out_dtype), ws.data_ptr(), ws.numel(), _lib.stream_handle(x0.device),
    )
    _lib.check(status, "pl_lora_delta_groups")


def lora_linear(
    x: torch.Tensor,
    weight: torch.Tensor,
    lora_modules: Sequence[tuple[torch.Tensor, torch.Tensor, int, float]] | None,
    adapter_ids: torch.Tensor | None,
    *,
    bias: torch.Tensor | None = None,
    out: torch.Tensor | None = None,
) -> torch.Tensor:
    """``x . W^T (+ bias) + sum_m scale_m * B_m[ids] . (A_m[ids] . x)`` for
    decode-sized batches (T <= 64): the LoRA shrink, then one kernel that
    streams W and adds the expand in its epilogue (``pl_linear``).

    lora_modules: ``(A, B, col_offset, scale)`` per module, in rank order,
    ``col_offset`` being the module's first output column of W's output.
    """
    if x.dim() != 2 or x.stride(1) != 1:
        raise ValueError("x must be [T, in] with unit column stride")
    T, fin = x.shape
    if T > _lib.PL_LINEAR_MAX_TOKENS:
        raise ValueError(f"lora_linear takes at most {_lib.PL_LINEAR_MAX_TOKENS} tokens")
    if weight.dim() != 2 or weight.shape[1] != fin or weight.stride(1) != 1 or weight.dtype != x.dtype:
        raise ValueError("weight must be [out, in] matching x")
    N = weight.shape[0]
    out = torch.empty((T, N), dtype=x.dtype, device=x.device) if out is None else out
    if out.shape != (T, N) or out.stride(1) != 1 or out.dtype != x.dtype:
        raise ValueError("out must be [T, out] with unit column stride")
    if bias is not None and (bias.numel() != N or bias.dtype != x.dtype):
        raise ValueError("bias must be [out] of x's dtype")
    lib = _lib.load()
    stream = _lib.stream_handle(x.device)
    n = 0
    arr = None
    ws = None
    n_adapters = 1
    if lora_modules:
        n = len(lora_modules)
        group = []
        arr = (_lib.LinearLora * n)()
        for i, (A, B, col, scale) in enumerate(lora_modules):
            fout = B.shape[-2]
            group.append((A, B, out[:, col:col + fout], scale))
            Bc = B if B.dim() == 3 else B.unsqueeze(0)
            arr[i].B, arr[i].col_offset, arr[i].out_features = Bc.data_ptr(), int(col), int(fout)
            arr[i].rank, arr[i].scale = int(Bc.shape[2]), float(scale)
        if adapter_ids is None or adapter_ids.dtype != torch.int32 or adapter_ids.numel() != T:
            raise ValueError("adapter_ids must be int32 [T]")
        mods, n_adapters, _ = _module_structs(group, x)
        nbytes = lib.pl_lora_workspace_size(T, fin, mods, n)
        if nbytes == 0:
            raise ValueError(f"invalid LoRA group: {_lib.last_error()}")
        ws = _workspace(x.device, nbytes)
        _lib.check(lib.pl_lora_shrink(x.data_ptr(), x.stride(0), T, fin, mods, n, adapter_ids.data_ptr(),
                                      n_adapters, _lib.dtype_code(x.dtype), ws.data_ptr(), ws.numel(), stream),
                   "pl_lora_shrink")
    _lib.check(lib.pl_linear(
        x.data_ptr(), x.stride(0), T, fin, weight.data_ptr(), weight.stride(0), N,
        bias.data_ptr() if bias is not None else None, out.data_ptr(), out.stride(0),
        arr, n, adapter_ids.data_ptr() if n else None, n_adapters,
        ws.data_ptr() if ws is not None else None, ws.numel() if ws is not None else 0,
        _lib.dtype_code(x.dtype), stream), "pl_linear")
    return out
