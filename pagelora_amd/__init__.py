"""MI355X (gfx950) paged-decode + no-merge LoRA hot path of PageLoRA.

Host code in Python over PyTorch-ROCm; arithmetic in the hand-written HIP
kernels of libpagelora_amd.so (C ABI: include/pagelora.h).
"""

from .page_table import (  # noqa: F401
    BatchPageTableBuffer,
    KVBlockSpan,
    PageTable,
    PageTableBuffer,
    build_batch_page_table,
    build_page_table,
)

__all__ = [
    "BatchPageTableBuffer",
    "KVBlockSpan",
    "PageTable",
    "PageTableBuffer",
    "build_batch_page_table",
    "build_page_table",
]
