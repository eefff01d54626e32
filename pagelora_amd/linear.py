"""Decode-sized linear layer on pre-shuffled weights (``pl_linear_shuffled``).

``ShuffledWeight`` re-lays a row-major ``[out, in]`` weight once into the
lane order of the MFMA B operand (1 KiB blocks of 16 rows x 32 k), so the
decode GEMM reads every weight byte with fully coalesced 1 KiB loads; it
replaces the base ``F.linear`` of the reference's projections
(model/flashinfer/packed_ops.py:143, 179, 251-265) at decode batch sizes.
"""

from __future__ import annotations

import ctypes

import torch

from . import _lib


class ShuffledWeight:
    """The shuffled copy of a ``[out_features, in_features]`` F16/BF16 weight."""

    def __init__(self, weight: torch.Tensor) -> None:
        if weight.dim() != 2 or weight.stride(1) != 1:
            raise ValueError("weight must be [out, in] with unit column stride")
        if weight.dtype not in (torch.bfloat16, torch.float16):
            raise ValueError("shuffled weights are bf16 or fp16")
        lib = _lib.load()
        n, k = weight.shape
        nbytes = lib.pl_weight_shuffled_bytes(n, k)
        if nbytes == 0:
            raise ValueError(f"in_features must be a positive multiple of 32 (got {k})")
        self.data = torch.empty(nbytes // weight.element_size(), dtype=weight.dtype, device=weight.device)
        _lib.check(lib.pl_weight_shuffle(weight.data_ptr(), weight.stride(0), n, k, self.data.data_ptr(), nbytes,
                                         _lib.dtype_code(weight.dtype), _lib.stream_handle(weight.device)),
                   "pl_weight_shuffle")
        self.out_features, self.in_features, self.dtype = n, k, weight.dtype

    @property
    def nbytes(self) -> int:
        return self.data.numel() * self.data.element_size()

    def unshuffle(self, out: torch.Tensor | None = None) -> torch.Tensor:
        """The row-major ``[out_features, in_features]`` weight (into ``out``,
        a tensor of that shape with unit column stride, when given)."""
        n, k = self.out_features, self.in_features
        if out is None:
            out = torch.empty((n, k), dtype=self.dtype, device=self.data.device)
        if out.shape != (n, k) or out.stride(1) != 1 or out.dtype != self.dtype:
            raise ValueError(f"out must be [{n}, {k}] of {self.dtype} with unit column stride")
        lib = _lib.load()
        _lib.check(lib.pl_weight_unshuffle(self.data.data_ptr(), self.nbytes, n, k, out.data_ptr(), out.stride(0),
                                           _lib.dtype_code(self.dtype), _lib.stream_handle(self.data.device)),
                   "pl_weight_unshuffle")
        return out

    def write_rows(self, rows: torch.Tensor, lo: int) -> None:
        """Replace rows ``lo .. lo + len(rows)`` with the row-major ``rows``
        when no row-major copy of the whole weight is kept: the 16-row blocks
        that hold them are unshuffled, patched and shuffled back."""
        hi = lo + rows.shape[0]
        if rows.dim() != 2 or rows.shape[1] != self.in_features or not 0 <= lo < hi <= self.out_features:
            raise ValueError(f"rows must be [n, {self.in_features}] inside 0..{self.out_features}")
        lo16, hi16 = lo // 16 * 16, min(-(-hi // 16) * 16, self.out_features)
        k, es = self.in_features, self.data.element_size()
        lib = _lib.load()
        stream = _lib.stream_handle(self.data.device)
        nbytes = lib.pl_weight_shuffled_bytes(hi16 - lo16, k)
        block = torch.empty((hi16 - lo16, k), dtype=self.dtype, device=self.data.device)
        base = self.data.data_ptr() + lo16 * k * es  # row block nb starts at element nb * 16 * K
        _lib.check(lib.pl_weight_unshuffle(base, nbytes, hi16 - lo16, k, block.data_ptr(), k,
                                           _lib.dtype_code(self.dtype), stream), "pl_weight_unshuffle")
        block[lo - lo16: hi - lo16].copy_(rows)
        _lib.check(lib.pl_weight_shuffle(block.data_ptr(), k, hi16 - lo16, k, base, nbytes,
                                         _lib.dtype_code(self.dtype), stream), "pl_weight_shuffle")

    def refresh_rows(self, weight: torch.Tensor, lo: int, hi: int) -> None:
        """Re-shuffle rows ``lo .. hi`` of the row-major ``weight`` this copy
        was made from (after they changed in place): the 16-row blocks that
        hold them are rewritten, nothing else."""
        if weight.shape != (self.out_features, self.in_features) or weight.dtype != self.dtype:
            raise ValueError("weight must be the [out, in] tensor this copy was shuffled from")
        if not 0 <= lo < hi <= self.out_features:
            raise ValueError(f"rows {lo}..{hi} outside 0..{self.out_features}")
        lo16, hi16 = lo // 16 * 16, min(-(-hi // 16) * 16, self.out_features)
        lib = _lib.load()
        k, es = self.in_features, weight.element_size()
        nbytes = lib.pl_weight_shuffled_bytes(hi16 - lo16, k)
        # row block nb starts at element nb * 16 * K of the shuffled copy
        _lib.check(lib.pl_weight_shuffle(weight.data_ptr() + lo16 * weight.stride(0) * es, weight.stride(0),
                                         hi16 - lo16, k, self.data.data_ptr() + lo16 * k * es, nbytes,
                                         _lib.dtype_code(weight.dtype), _lib.stream_handle(weight.device)),
                   "pl_weight_shuffle")


def linear_shuffled(x: torch.Tensor, weight: ShuffledWeight, bias: torch.Tensor | None = None,
                    out: torch.Tensor | None = None) -> torch.Tensor:
    """``x . W^T (+ bias)`` for up to 64 tokens from a :class:`ShuffledWeight`."""
    if x.dim() != 2 or x.stride(1) != 1 or x.shape[1] != weight.in_features or x.dtype != weight.dtype:
        raise ValueError(f"x must be [T, {weight.in_features}] of {weight.dtype} with unit column stride")
    T, N = x.shape[0], weight.out_features
    if T > _lib.PL_LINEAR_MAX_TOKENS:
        raise ValueError(f"linear_shuffled takes at most {_lib.PL_LINEAR_MAX_TOKENS} tokens")
    out = torch.empty((T, N), dtype=x.dtype, device=x.device) if out is None else out
    if out.shape != (T, N) or out.stride(1) != 1 or out.dtype != x.dtype:
        raise ValueError("out must be [T, out] with unit column stride")
    if bias is not None and (bias.numel() != N or bias.dtype != x.dtype):
        raise ValueError("bias must be [out] of x's dtype")
    lib = _lib.load()
    _lib.check(lib.pl_linear_shuffled(x.data_ptr(), x.stride(0), T, weight.in_features, weight.data.data_ptr(), N,
                                      bias.data_ptr() if bias is not None else None, out.data_ptr(), out.stride(0),
                                      _lib.dtype_code(x.dtype), _lib.stream_handle(x.device)),
               "pl_linear_shuffled")
    return out


class SplitOutput:
    """A decode GEMM output held as split-K partial planes ``[splits, T, ld]``
    (fp32).  Element (t, c) is the in-order sum over the planes, rounded to
    the model dtype: the value the unsplit GEMM would have written.  The
    kernels that consume the projection (``fused_ops.add_rmsnorm``,
    ``fused_ops.qk_norm_rope_append``) read it directly (``pl_split_out``)."""

    def __init__(self, partials: torch.Tensor, out_features: int, dtype: torch.dtype) -> None:
        self.partials = partials
        self.out_features = out_features
        self.dtype = dtype

    @property
    def splits(self) -> int:
        return self.partials.shape[0]

    @property
    def rows(self) -> int:
        return self.partials.shape[1]

    @property
    def ld(self) -> int:
        return self.partials.shape[2]

    @property
    def device(self) -> torch.device:
        return self.partials.device

    def struct(self) -> "_lib.SplitOut":
        p = self.partials
        return _lib.SplitOut(p.data_ptr(), p.shape[0], p.stride(1), p.stride(0))

    def sum(self) -> torch.Tensor:
        """The rounded output as a tensor (planes added in order, as the kernels do)."""
        acc = torch.zeros_like(self.partials[0])
        for s in range(self.splits):
            acc = acc + self.partials[s]
        return acc[:, : self.out_features].to(self.dtype)


def linear_shuffled_split(x: torch.Tensor, weight: ShuffledWeight, splits: int) -> SplitOutput:
    """``x . W^T`` with K split over ``splits`` workgroups per 16 output
    columns, returned as fp32 partial planes for a consuming kernel to sum."""
    if x.dim() != 2 or x.stride(1) != 1 or x.shape[1] != weight.in_features or x.dtype != weight.dtype:
        raise ValueError(f"x must be [T, {weight.in_features}] of {weight.dtype} with unit column stride")
    T, N = x.shape[0], weight.out_features
    if T > _lib.PL_LINEAR_MAX_TOKENS:
        raise ValueError(f"linear_shuffled_split takes at most {_lib.PL_LINEAR_MAX_TOKENS} tokens")
    ld = (N + 7) // 8 * 8
    partials = torch.empty((splits, T, ld), dtype=torch.float32, device=x.device)
    lib = _lib.load()
    _lib.check(lib.pl_linear_shuffled_split(x.data_ptr(), x.stride(0), T, weight.in_features, weight.data.data_ptr(),
                                            N, int(splits), partials.data_ptr(), ld, partials.stride(0),
                                            _lib.dtype_code(x.dtype), _lib.stream_handle(x.device)),
               "pl_linear_shuffled_split")
    return SplitOutput(partials, N, x.dtype)


def linear_shuffled_side(x: torch.Tensor, weight: ShuffledWeight, main_features: int,
                         side_splits: int) -> tuple[torch.Tensor, SplitOutput]:
    """``x . W^T`` with the rows from ``main_features`` on (the LoRA A rows
    stacked under W) split-K into fp32 planes: returns the first
    ``main_features`` outputs as a ``[T, main_features]`` tensor and the rest
    as a :class:`SplitOutput` of ``out_features - main_features`` columns
    (``pl_linear_shuffled_side``)."""
    if x.dim() != 2 or x.stride(1) != 1 or x.shape[1] != weight.in_features or x.dtype != weight.dtype:
        raise ValueError(f"x must be [T, {weight.in_features}] of {weight.dtype} with unit column stride")
    T, N = x.shape[0], weight.out_features
    if T > _lib.PL_LINEAR_MAX_TOKENS:
        raise ValueError(f"linear_shuffled_side takes at most {_lib.PL_LINEAR_MAX_TOKENS} tokens")
    if main_features <= 0 or main_features % 16 or main_features >= N:
        raise ValueError("main_features must be a positive multiple of 16 below out_features")
    side = N - main_features
    ld = (side + 7) // 8 * 8
    out = torch.empty((T, main_features), dtype=x.dtype, device=x.device)
    partials = torch.empty((side_splits, T, ld), dtype=torch.float32, device=x.device)
    lib = _lib.load()
    _lib.check(lib.pl_linear_shuffled_side(x.data_ptr(), x.stride(0), T, weight.in_features, weight.data.data_ptr(),
                                           N, int(main_features), out.data_ptr(), out.stride(0), int(side_splits),
                                           partials.data_ptr(), ld, partials.stride(0), _lib.dtype_code(x.dtype),
                                           _lib.stream_handle(x.device)),
               "pl_linear_shuffled_side")
    return out, SplitOutput(partials, side, x.dtype)


class LoraPartials:
    """fp32 partial sums ``[T, parts, rank]`` of a LoRA module's rank-space
    row y = x . A_a^T, for each token's own adapter a, written by the kernel
    that produces x (``pl_lora_partials``): y[t] is the sum over the parts,
    which the consuming kernel adds in a fixed order."""

    def __init__(self, partials: torch.Tensor) -> None:
        if partials.dim() != 3 or partials.dtype != torch.float32 or not partials.is_contiguous():
            raise ValueError("partials must be a contiguous fp32 [T, parts, rank] tensor")
        self.partials = partials

    @property
    def rank(self) -> int:
        return self.partials.shape[2]

    @property
    def parts(self) -> int:
        return self.partials.shape[1]

    def struct(self) -> "_lib.LoraPartials":
        p = self.partials
        return _lib.LoraPartials(p.data_ptr(), p.stride(0), p.shape[1], p.shape[2])

    def sum(self) -> torch.Tensor:
        """y [T, rank] in float64 (for checks)."""
        return self.partials.double().sum(dim=1)


def lora_a_rows(weight: ShuffledWeight, a_row0: int, rank: int, adapter: int = -1) -> "_lib.LoraARows":
    """``pl_lora_a_rows`` of a module whose adapters' A rows sit under W in
    the shuffled ``weight``: adapter a's rank r is row ``a_row0 + a*rank + r``."""
    if a_row0 < 0 or a_row0 + rank > weight.out_features:
        raise ValueError(f"A rows {a_row0}.. outside the weight's {weight.out_features} rows")
    return _lib.LoraARows(weight.data.data_ptr(), weight.in_features, weight.out_features, int(a_row0), int(rank),
                          int(adapter))


def linear_shuffled_norm(x: torch.Tensor, norm_weight: torch.Tensor, eps: float, weight: ShuffledWeight,
                         x_norm_out: torch.Tensor | None = None, sq: torch.Tensor | None = None) -> torch.Tensor:
    """``RMSNorm(x) . W^T`` in one launch (``pl_linear_shuffled_norm``): the
    normalized rows never go through memory (``x_norm_out``, when given,
    receives them too).  ``sq`` [T, parts] fp32: the rows' sums of squares in
    pieces, from the GEMM that wrote x (:func:`linear_shuffled_add`)."""
    if x.dim() != 2 or x.stride(1) != 1 or x.shape[1] != weight.in_features or x.dtype != weight.dtype:
        raise ValueError(f"x must be [T, {weight.in_features}] of {weight.dtype} with unit column stride")
    if norm_weight.numel() != weight.in_features or norm_weight.dtype != x.dtype or not norm_weight.is_contiguous():
        raise ValueError("norm_weight must be a contiguous [in_features] tensor of x's dtype")
    T, N = x.shape[0], weight.out_features
    out = torch.empty((T, N), dtype=x.dtype, device=x.device)
    if x_norm_out is not None and (tuple(x_norm_out.shape) != tuple(x.shape) or x_norm_out.stride(1) != 1
                                   or x_norm_out.dtype != x.dtype):
        raise ValueError("x_norm_out must be shaped like x with unit column stride")
    if sq is not None and (sq.dim() != 2 or sq.shape[0] != T or sq.dtype != torch.float32 or sq.stride(1) != 1):
        raise ValueError("sq must be fp32 [T, parts] with unit column stride")
    lib = _lib.load()
    _lib.check(lib.pl_linear_shuffled_norm(x.data_ptr(), x.stride(0), T, weight.in_features, norm_weight.data_ptr(),
                                           float(eps), sq.data_ptr() if sq is not None else None,
                                           sq.stride(0) if sq is not None else 0, sq.shape[1] if sq is not None else 0,
                                           weight.data.data_ptr(), N, out.data_ptr(), out.stride(0),
                                           x_norm_out.data_ptr() if x_norm_out is not None else None,
                                           x_norm_out.stride(0) if x_norm_out is not None else 0,
                                           _lib.dtype_code(x.dtype), _lib.stream_handle(x.device)),
               "pl_linear_shuffled_norm")
    return out


def linear_shuffled_add(x: torch.Tensor, weight: ShuffledWeight, main_features: int, residual: torch.Tensor,
                        lora=None, partials: LoraPartials | None = None, adapter_ids: torch.Tensor | None = None,
                        out: torch.Tensor | None = None, sq_out: torch.Tensor | None = None) -> torch.Tensor:
    """``residual += round(round(x . W^T) + delta)`` over the first
    ``main_features`` rows of ``weight`` (``pl_linear_shuffled_add``), with
    the LoRA up-projection delta of ``lora`` (a ``fused_ops.LoraUp``; its
    ``y`` is not read) on y from ``partials``.  ``out`` (optional) receives
    round(x . W^T); ``sq_out`` (optional, fp32 [T, >= main_features / 16])
    the new residual's sums of squares per 16 columns.  Returns
    ``residual``."""
    if x.dim() != 2 or x.stride(1) != 1 or x.shape[1] != weight.in_features or x.dtype != weight.dtype:
        raise ValueError(f"x must be [T, {weight.in_features}] of {weight.dtype} with unit column stride")
    T = x.shape[0]
    if not 0 < main_features <= weight.out_features:
        raise ValueError("main_features must be in 1..out_features")
    if tuple(residual.shape) != (T, main_features) or residual.stride(1) != 1 or residual.dtype != x.dtype:
        raise ValueError(f"residual must be [{T}, {main_features}] of x's dtype with unit column stride")
    if (lora is None) != (partials is None):
        raise ValueError("lora and partials are given together")
    lu = yp = None
    ids, n = None, 1
    if lora is not None:
        nad, outf, r, layout = lora._b_shape()
        if not lora.B.is_contiguous() or lora.B.dtype != x.dtype:
            raise ValueError("LoRA B must be contiguous and of x's dtype")
        if partials.partials.shape[0] != T:
            raise ValueError("partials must have one row per token")
        if lora.adapter < 0 and (adapter_ids is None or adapter_ids.dtype != torch.int32 or adapter_ids.numel() != T):
            raise ValueError("per-token adapters need int32 adapter_ids [T]")
        lu = _lib.LoraUp(None, 0, 0, lora.B.data_ptr(), int(outf), int(r), float(lora.scale), int(layout),
                         int(lora.adapter))
        yp = partials.struct()
        n = nad
        ids = adapter_ids.data_ptr() if adapter_ids is not None else None
    if out is not None and (tuple(out.shape) != (T, main_features) or out.stride(1) != 1 or out.dtype != x.dtype):
        raise ValueError("out must be shaped like residual")
    if sq_out is not None and (sq_out.dim() != 2 or sq_out.shape[0] != T or sq_out.shape[1] < -(-main_features // 16)
                               or sq_out.dtype != torch.float32 or sq_out.stride(1) != 1):
        raise ValueError(f"sq_out must be fp32 [T, >= {-(-main_features // 16)}] with unit column stride")
    lib = _lib.load()
    _lib.check(lib.pl_linear_shuffled_add(x.data_ptr(), x.stride(0), T, weight.in_features, weight.data.data_ptr(),
                                          int(main_features), residual.data_ptr(), residual.stride(0),
                                          ctypes.byref(lu) if lu is not None else None,
                                          ctypes.byref(yp) if yp is not None else None, ids, n,
                                          out.data_ptr() if out is not None else None,
                                          out.stride(0) if out is not None else 0,
                                          sq_out.data_ptr() if sq_out is not None else None,
                                          sq_out.stride(0) if sq_out is not None else 0,
                                          _lib.dtype_code(x.dtype), _lib.stream_handle(x.device)),
               "pl_linear_shuffled_add")
    return residual
