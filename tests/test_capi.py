"""The C-ABI library loads and exports exactly what include/pagelora.h declares.
No compute call is made (this runs without a GPU)."""

import ctypes
import re
from pathlib import Path

from pagelora_amd import _lib

HEADER = Path(__file__).resolve().parents[1] / "include" / "pagelora.h"


def _declared_functions():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(pl_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_the_binding_table():
    assert _declared_functions() == sorted(_lib.SIGNATURES)


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    for name in _declared_functions():
        assert hasattr(lib, name), name
    assert lib.pl_version() >> 16 == 1
    assert lib.pl_last_error() in (b"", None)


def test_workspace_size_query_is_host_only():
    lib = _lib.load()
    n = lib.pl_decode_workspace_size(64, 256, 32, 128)
    assert n >= (256 + 64) * 32 * 128 * 4
    assert lib.pl_decode_workspace_size(0, 0, 32, 128) == 0
    mods = (_lib.LoraModule * 3)()
    for m, out in zip(mods, (4096, 1024, 1024)):
        m.A = m.B = m.out = 256  # aligned dummy addresses: sizes only, never dereferenced
        m.ldo, m.out_features, m.rank, m.scale = 6144, out, 16, 2.0
    # fp32 partials [k-slices][T][sum(rank) padded to 32]: 64 tokens -> 4 slices, 4 tokens -> 8 slices
    assert lib.pl_lora_workspace_size(64, 4096, mods, 3) == 4 * 64 * 64 * 4
    assert lib.pl_lora_workspace_size(4, 4096, mods, 3) == 8 * 4 * 64 * 4


def test_lora_module_struct_layout():
    assert ctypes.sizeof(_lib.LoraModule) == 48
    assert _lib.LoraModule.ldo.offset == 24 and _lib.LoraModule.scale.offset == 40
