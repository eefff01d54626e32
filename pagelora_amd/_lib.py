"""ctypes binding of libpagelora_amd.so (declarations: include/pagelora.h).

Loading fails loudly when the library has not been built: there is no CPU
or torch fallback behind any entry point of this package.
"""

from __future__ import annotations

import ctypes
import threading
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libpagelora_amd.so"

PL_DTYPE_F32 = 0
PL_DTYPE_F16 = 1
PL_DTYPE_BF16 = 2

PL_OK = 0
PL_ERR_INVALID = 1
PL_ERR_UNSUPPORTED = 2
PL_ERR_WORKSPACE = 3
PL_ERR_HIP = 4

PL_LORA_MAX_MODULES = 4
PL_LORA_MAX_GROUPS = 4

PL_DECODE_SKIP_MERGE = 1
PL_DECODE_MERGE_ONLY = 2
PL_DECODE_NOALLOC_MAX_BYTES = 16 << 20


class ExtensionNotBuiltError(ImportError):
    """libpagelora_amd.so is missing: run ``__graft_entry__.build()``."""


class WorkspaceTooSmallError(RuntimeError):
    """The caller's workspace cannot hold the requested plan."""


class HipError(RuntimeError):
    """A HIP runtime call inside the library failed."""


class LoraModule(ctypes.Structure):
    """Mirror of ``pl_lora_module``."""

    _fields_ = [
        ("A", ctypes.c_void_p),
        ("B", ctypes.c_void_p),
        ("out", ctypes.c_void_p),
        ("ldo", ctypes.c_int64),
        ("out_features", ctypes.c_int),
        ("rank", ctypes.c_int),
        ("scale", ctypes.c_float),
    ]


class LoraGroup(ctypes.Structure):
    """Mirror of ``pl_lora_group``."""

    _fields_ = [
        ("x", ctypes.c_void_p),
        ("ldx", ctypes.c_int64),
        ("in_features", ctypes.c_int),
        ("num_modules", ctypes.c_int),
        ("modules", ctypes.POINTER(LoraModule)),
    ]


class LinearLora(ctypes.Structure):
    """Mirror of ``pl_linear_lora``."""

    _fields_ = [
        ("B", ctypes.c_void_p),
        ("col_offset", ctypes.c_int),
        ("out_features", ctypes.c_int),
        ("rank", ctypes.c_int),
        ("scale", ctypes.c_float),
    ]


class SplitOut(ctypes.Structure):
    """Mirror of ``pl_split_out``."""

    _fields_ = [
        ("partials", ctypes.c_void_p),
        ("splits", ctypes.c_int),
        ("ld", ctypes.c_int64),
        ("plane_stride", ctypes.c_int64),
    ]


class LoraUp(ctypes.Structure):
    """Mirror of ``pl_lora_up``."""

    _fields_ = [
        ("y", ctypes.c_void_p),
        ("ldy", ctypes.c_int64),
        ("y_offset", ctypes.c_int),
        ("B", ctypes.c_void_p),
        ("out_features", ctypes.c_int),
        ("rank", ctypes.c_int),
        ("scale", ctypes.c_float),
        ("b_layout", ctypes.c_int),
        ("adapter", ctypes.c_int),
    ]


class LoraPartials(ctypes.Structure):
    """Mirror of ``pl_lora_partials``."""

    _fields_ = [
        ("partials", ctypes.c_void_p),
        ("ld", ctypes.c_int64),
        ("parts", ctypes.c_int),
        ("rank", ctypes.c_int),
    ]


class LoraARows(ctypes.Structure):
    """Mirror of ``pl_lora_a_rows``."""

    _fields_ = [
        ("shuffled", ctypes.c_void_p),
        ("in_features", ctypes.c_int),
        ("out_features", ctypes.c_int),
        ("a_row0", ctypes.c_int),
        ("rank", ctypes.c_int),
        ("adapter", ctypes.c_int),
    ]


PL_LORA_B_ROWS = 0
PL_LORA_B_CHUNK8 = 1

PL_LINEAR_MAX_TOKENS = 64

_vp = ctypes.c_void_p
_i32 = ctypes.c_int
_i64 = ctypes.c_int64
_f32 = ctypes.c_float
_sz = ctypes.c_size_t

# name -> (restype, argtypes); the exact list of symbols the header declares.
SIGNATURES: dict[str, tuple[object, list[object]]] = {
    "pl_last_error": (ctypes.c_char_p, []),
    "pl_version": (_i32, []),
    "pl_decode_workspace_size": (_sz, [_i32, _i32, _i32, _i32]),
    "pl_decode_plan": (_i32, [_vp, _i32, _i32, _i32, _i32, _i32, _i32, _vp, _sz, _vp]),
    "pl_decode_workspace_size_shared": (_sz, [_i32, _i32, _i32, _i32, _i32, _i32]),
    "pl_decode_plan_shared": (_i32, [_vp, _i32, _i32, _i32, _i32, _i32, _i32, _i32, _i32, _vp, _sz, _vp]),
    "pl_decode_forget": (_i32, [_vp]),
    "pl_decode_run": (
        _i32,
        [
            _vp, _i64, _i64,            # q, strides
            _vp, _vp, _i64, _i64, _i64,  # k/v cache, page/token/head strides
            _i64,                        # num_pages
            _vp, _vp,                    # indices, last_page_len
            _vp, _i64, _i64,             # o, strides
            _vp,                         # lse
            _i32, _i32, _i32, _i32, _i32,  # batch, hq, hkv, head_dim, page_size
            _f32, _i32, _i32, _i32,      # sm_scale, dtype, target_items, flags
            _vp, _sz, _vp,               # workspace, bytes, stream
        ],
    ),
    "pl_decode_noalloc": (
        _i32,
        [
            _vp, _i64, _i64,            # q, strides
            _vp, _vp, _i64, _i64, _i64,  # k/v cache, page/token/head strides
            _i64,                        # num_pages
            _vp, _i32,                   # indptr, indices_capacity
            _vp, _vp,                    # indices, last_page_len
            _vp, _i64, _i64,             # o, strides
            _vp,                         # lse
            _i32, _i32, _i32, _i32, _i32,  # batch, hq, hkv, head_dim, page_size
            _f32, _i32, _i32, _i32,      # sm_scale, dtype, target_items, min_chunk_pages
            _vp,                         # stream
        ],
    ),
    "pl_kv_append": (
        _i32,
        [
            _vp, _vp, _i64, _i64, _i64, _i64,  # k, v, strides
            _vp, _vp, _i64, _i64, _i64,         # caches, page/token/head strides
            _i64, _i32,                         # num_pages, page_size
            _vp, _vp,                           # page_id, offset
            _i32, _i32, _i32, _i32, _vp,        # batch, hkv, head_dim, dtype, stream
        ],
    ),
    "pl_page_table_advance": (
        _i32,
        [
            _vp, _vp, _i64, _vp,          # indptr, indices, capacity, last_page_len
            _i32, _i32,                   # batch, page_size
            _vp, _i32, _vp,               # reserve, slots, reserve_head
            _vp, _vp, _vp, _vp, _vp,      # positions, page_id, page_offset, status, stream
        ],
    ),
    "pl_greedy_argmax_workspace_size": (_sz, [_i32, _i32, _i32]),
    "pl_greedy_argmax": (_i32, [_vp, _i64, _i32, _i32, _i32, _vp, _vp, _vp, _sz, _vp]),
    "pl_prefill_plan": (
        _i32,
        [
            _vp, _vp, _vp, _i32,         # qo_indptr, kv_indptr, last_page_len (host), batch
            _i32, _i32, _i32, _i32,      # hq, hkv, page_size, causal
            _vp, _i32, ctypes.POINTER(_i32),  # items (host), max_items, num_items
        ],
    ),
    "pl_prefill_run": (
        _i32,
        [
            _vp, _i64, _i64,             # q, strides
            _vp, _vp, _i64, _i64, _i64,  # k/v cache, page/token/head strides
            _i64,                        # num_pages
            _vp, _vp, _vp, _vp,          # qo_indptr, kv_indptr, kv_indices, last_page_len
            _vp, _i32,                   # items, num_items
            _vp, _i64, _i64,             # o, strides
            _i32, _i32, _i32, _i32, _i32, _i32,  # batch, hq, hkv, head_dim, page_size, causal
            _f32, _i32, _vp,             # sm_scale, dtype, stream
        ],
    ),
    "pl_rmsnorm": (_i32, [_vp, _i64, _vp, _vp, _i64, _i32, _i32, _f32, _i32, _vp]),
    "pl_add_rmsnorm_lora": (
        _i32,
        [_vp, _i64, _vp, _i64, ctypes.POINTER(SplitOut), ctypes.POINTER(LoraUp), _vp, _i32, _vp, _vp, _i64, _i32,
         _i32, _f32, _i32, _vp],
    ),
    "pl_add_rmsnorm_lora_side": (
        _i32,
        [_vp, _i64, _vp, _i64, ctypes.POINTER(SplitOut), ctypes.POINTER(LoraUp), _vp, _i32, _vp, _vp, _i64, _i32,
         _i32, _f32, _i32, _vp],
    ),
    "pl_silu_mul_lora": (_i32, [_vp, _i64, ctypes.POINTER(LoraUp), _vp, _i32, _vp, _i64, _i32, _i32, _i32, _vp]),
    "pl_silu_mul_lora_shrink": (_i32, [_vp, _i64, ctypes.POINTER(LoraUp), _vp, _i32, _vp, _i64, _i32, _i32,
                                       ctypes.POINTER(LoraARows), ctypes.POINTER(LoraPartials), _i32, _vp]),
    "pl_qk_norm_rope_append_lora": (
        _i32,
        [
            _vp, _i64, ctypes.POINTER(SplitOut),  # qkv, ld, split planes
            ctypes.POINTER(LoraUp), _vp, _i32,  # lora[3], ids, n_adapters
            _vp, _vp,                     # q/k norm weights
            _vp, _vp, _vp,                # positions, page_id, offset
            _vp, _vp, _vp,                # q_out, k_cache, v_cache
            _i64, _i64, _i64, _i64, _i32,  # page/token/head strides, num_pages, page_size
            _i32, _i32, _i32, _i32,       # batch, hq, hkv, head_dim
            _vp, _f32, _i32, _vp,         # inv_freq, eps, dtype, stream
        ],
    ),
    "pl_add_rmsnorm": (_i32, [_vp, _i64, _vp, _i64, _vp, _vp, _i64, _i32, _i32, _f32, _i32, _vp]),
    "pl_silu_mul": (_i32, [_vp, _i64, _vp, _i64, _i32, _i32, _i32, _vp]),
    "pl_qk_norm_rope_append": (
        _i32,
        [
            _vp, _i64, _vp, _vp,          # qkv, ld, q/k norm weights
            _vp, _vp, _vp,                # positions, page_id, offset
            _vp, _vp, _vp,                # q_out, k_cache, v_cache
            _i64, _i64, _i64, _i64, _i32,  # page/token/head strides, num_pages, page_size
            _i32, _i32, _i32, _i32,       # batch, hq, hkv, head_dim
            _vp, _f32, _i32, _vp,         # inv_freq, eps, dtype, stream
        ],
    ),
    "pl_rope_cos_sin": (
        _i32,
        [_vp, _i32, _vp, _i32, _vp, _vp],  # positions, batch, inv_freq, half_dim, out, stream
    ),
    "pl_decode_run_qkv": (
        _i32,
        [
            _vp, _i64, _vp, _vp, _i32,   # qkv, ld, lora (3 pl_lora_up), adapter_ids, num_adapters
            _vp, _vp, _vp,               # q/k norm weights, rope cos/sin
            _vp, _vp, _f32,              # page_id, offset, eps
            _vp, _vp, _i64, _i64, _i64,  # k/v cache, page/token/head strides
            _i64,                        # num_pages
            _vp, _vp,                    # indices, last_page_len
            _vp, _i64, _i64,             # o, strides
            _vp,                         # lse
            _i32, _i32, _i32, _i32, _i32,  # batch, hq, hkv, head_dim, page_size
            _f32, _i32, _i32, _i32,      # sm_scale, dtype, target_items, flags
            _vp, _sz, _vp,               # workspace, bytes, stream
        ],
    ),
    "pl_decode_run_qkv_oshrink": (
        _i32,
        [
            _vp, _i64, _vp, _vp, _i32,   # qkv, ld, lora (3 pl_lora_up), adapter_ids, num_adapters
            _vp, _vp, _vp,               # q/k norm weights, rope cos/sin
            _vp, _vp, _f32,              # page_id, offset, eps
            _vp, _vp, _i64, _i64, _i64,  # k/v cache, page/token/head strides
            _i64,                        # num_pages
            _vp, _vp,                    # indices, last_page_len
            _vp, _i64, _i64,             # o, strides
            _vp,                         # lse
            _i32, _i32, _i32, _i32, _i32,  # batch, hq, hkv, head_dim, page_size
            _f32, _i32, _i32, _i32,      # sm_scale, dtype, target_items, flags
            _vp, _sz,                    # workspace, bytes
            ctypes.POINTER(LoraARows), ctypes.POINTER(LoraPartials),  # o_proj A rows, partials
            _vp,                         # stream
        ],
    ),
    "pl_linear": (
        _i32,
        [_vp, _i64, _i32, _i32, _vp, _i64, _i32, _vp, _vp, _i64, ctypes.POINTER(LinearLora), _i32, _vp, _i32,
         _vp, _sz, _i32, _vp],
    ),
    "pl_weight_shuffled_bytes": (_sz, [_i32, _i32]),
    "pl_weight_shuffle": (_i32, [_vp, _i64, _i32, _i32, _vp, _sz, _i32, _vp]),
    "pl_weight_unshuffle": (_i32, [_vp, _sz, _i32, _i32, _vp, _i64, _i32, _vp]),
    "pl_linear_shuffled": (_i32, [_vp, _i64, _i32, _i32, _vp, _i32, _vp, _vp, _i64, _i32, _vp]),
    "pl_linear_shuffled_split": (_i32, [_vp, _i64, _i32, _i32, _vp, _i32, _i32, _vp, _i64, _i64, _i32, _vp]),
    "pl_linear_shuffled_side": (_i32, [_vp, _i64, _i32, _i32, _vp, _i32, _i32, _vp, _i64, _i32, _vp, _i64, _i64,
                                       _i32, _vp]),
    "pl_linear_shuffled_norm": (_i32, [_vp, _i64, _i32, _i32, _vp, _f32, _vp, _i64, _i32, _vp, _i32, _vp, _i64,
                                       _vp, _i64, _i32, _vp]),
    "pl_linear_shuffled_add": (_i32, [_vp, _i64, _i32, _i32, _vp, _i32, _vp, _i64, ctypes.POINTER(LoraUp),
                                      ctypes.POINTER(LoraPartials), _vp, _i32, _vp, _i64, _vp, _i64, _i32, _vp]),
    "pl_lora_workspace_size": (_sz, [_i32, _i32, ctypes.POINTER(LoraModule), _i32]),
    "pl_lora_delta": (
        _i32,
        [_vp, _i64, _i32, _i32, ctypes.POINTER(LoraModule), _i32, _vp, _i32, _i32, _i32, _vp, _sz, _vp],
    ),
    "pl_lora_delta_workspace_size": (_sz, [ctypes.POINTER(LoraGroup), _i32, _i32, _i32]),
    "pl_lora_delta_groups": (
        _i32,
        [ctypes.POINTER(LoraGroup), _i32, _i32, _vp, _i32, _i32, _i32, _vp, _sz, _vp],
    ),
    "pl_lora_shrink": (
        _i32,
        [_vp, _i64, _i32, _i32, ctypes.POINTER(LoraModule), _i32, _vp, _i32, _i32, _vp, _sz, _vp],
    ),
    "pl_lora_expand": (
        _i32,
        [_i32, _i32, ctypes.POINTER(LoraModule), _i32, _vp, _i32, _i32, _i32, _vp, _sz, _vp],
    ),
}

_lock = threading.Lock()
_lib: ctypes.CDLL | None = None


def load() -> ctypes.CDLL:
    """Return the loaded library, loading it on first use."""

    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not LIB_PATH.exists():
            raise ExtensionNotBuiltError(
                f"{LIB_PATH} is missing; build it with `python -c 'import __graft_entry__ as g; g.build()'`"
            )
        # torch first: its bundled HIP runtime then serves this library too
        # (one runtime per process, so torch streams are valid handles here).
        import torch  # noqa: F401

        lib = ctypes.CDLL(str(LIB_PATH))
        for name, (restype, argtypes) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = restype
            fn.argtypes = argtypes
        _lib = lib
        return lib


def last_error() -> str:
    msg = load().pl_last_error()
    return msg.decode() if msg else ""


def check(status: int, what: str) -> None:
    """Map a pl_status to the Python exception the reference would raise."""

    if status == PL_OK:
        return
    msg = f"{what}: {last_error()}"
    if status == PL_ERR_INVALID:
        raise ValueError(msg)
    if status == PL_ERR_UNSUPPORTED:
        raise NotImplementedError(msg)
    if status == PL_ERR_WORKSPACE:
        raise WorkspaceTooSmallError(msg)
    raise HipError(msg)


def dtype_code(dtype) -> int:
    import torch

    codes = {torch.float32: PL_DTYPE_F32, torch.float16: PL_DTYPE_F16, torch.bfloat16: PL_DTYPE_BF16}
    if dtype not in codes:
        raise NotImplementedError(f"dtype {dtype} is not supported (float32, float16, bfloat16)")
    return codes[dtype]


def stream_handle(device=None) -> int:
    """Raw hipStream_t of torch's current stream on ``device``."""

    import torch

    return torch.cuda.current_stream(device).cuda_stream
