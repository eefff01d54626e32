"""Build libpagelora_amd.so (the HIP kernels and their C ABI) for gfx950.

Every ``csrc/*.hip`` file is compiled to an object with hipcc (in parallel),
then linked into one shared library next to this file.  The library has no
torch dependency: it links only the HIP runtime, so a non-Python host can
load it through the declarations in ``include/pagelora.h``.
"""

from __future__ import annotations

import concurrent.futures
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
CSRC = PKG_DIR / "csrc"
BUILD_DIR = PKG_DIR / "_build"
LIB_PATH = PKG_DIR / "libpagelora_amd.so"
ARCH = os.environ.get("PAGELORA_OFFLOAD_ARCH", "gfx950")

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    # No packed-fp32 instructions anywhere in the device code.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


# Per-source additions: MFMA accumulators in ordinary VGPRs rather than
# AGPRs.  paged_prefill: the softmax rescale then works on them in place (no
# copies between the register files each tile) and the kernel needs 158
# registers instead of 192 (three waves per SIMD instead of two).  lora: the
# shrink kernel 72 -> 56 registers, the expand 72 -> 66.
_MFMA_VGPR = ["-mllvm", "-amdgpu-mfma-vgpr-form"]
FILE_FLAGS = {
    "paged_prefill.hip": _MFMA_VGPR,
    "lora.hip": _MFMA_VGPR,
}


def _hipcc() -> str:
    found = shutil.which("hipcc")
    if found:
        return found
    rocm = Path(os.environ.get("ROCM_PATH", "/opt/rocm")) / "bin" / "hipcc"
    if rocm.exists():
        return str(rocm)
    raise RuntimeError("hipcc not found: the HIP toolchain is required to build libpagelora_amd.so")


def _run(cmd: list[str]) -> None:
    proc = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(
        line for line in proc.stdout.splitlines() if "packed-fp32-ops" not in line
    )
    if proc.returncode != 0:
        raise RuntimeError(f"command failed ({proc.returncode}): {' '.join(cmd)}\n{out}")
    if out.strip():
        print(out, file=sys.stderr)


def build(verbose: bool = True, jobs: int | None = None) -> Path:
    """Compile every kernel source and link the shared library; returns its path."""

    hipcc = _hipcc()
    BUILD_DIR.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    if not sources:
        raise RuntimeError(f"no HIP sources under {CSRC}")
    objects = [BUILD_DIR / (src.stem + ".o") for src in sources]
    jobs = jobs or min(len(sources), max(1, os.cpu_count() or 1), 16)

    def compile_one(pair):
        src, obj = pair
        _run([hipcc, *HIPCC_FLAGS, *FILE_FLAGS.get(src.name, []), "-c", str(src), "-o", str(obj)])
        return src.name

    with concurrent.futures.ThreadPoolExecutor(max_workers=jobs) as pool:
        for name in pool.map(compile_one, zip(sources, objects)):
            if verbose:
                print(f"[pagelora_amd] compiled {name}", file=sys.stderr)

    tmp = LIB_PATH.with_suffix(".so.tmp")
    _run([hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objects)])
    os.replace(tmp, LIB_PATH)
    if verbose:
        print(f"[pagelora_amd] linked {LIB_PATH}", file=sys.stderr)
    return LIB_PATH


if __name__ == "__main__":
    build()
