"""PAGELORA_DECODE_PLAN_KERNEL=1 (the plan kernel for every batch) with a
batch whose rows share their leading pages: plan_decode detects the shared
prefix on the host tables, and the library plans the batch unshared instead
of rejecting it (the shared-prefix path needs a direct plan).  The outputs
match the oracle (attention_backend.py:63-131 semantics).

The variable is read once per process, at the first plan, so the check runs
in a fresh child process that has it set before any GPU call.
"""

import os
import subprocess
import sys
from pathlib import Path

import pytest

pytestmark = pytest.mark.gpu

ROOT = Path(__file__).resolve().parents[1]

CHILD = r"""
import numpy as np, torch
from oracle import paged_decode as opd
from pagelora_amd.attention_backend import PagedDecodeAttention
from tests.gpu_cases import ragged_case

dev = torch.device("cuda:0")
for dtype in (torch.bfloat16, torch.float16):
    lens = [2048 + 64, 2048 + 70, 2048 + 1, 2048 + 33]
    print(f"[plan kernel forced] 4 rows with a 128-page shared prefix, {dtype}", flush=True)
    case = ragged_case(lens=lens, hq=32, hkv=8, head_dim=128, page_size=16, dtype=dtype, device=dev, seed=17,
                       pool_extra=4, shared_prefix_pages=128)
    be = PagedDecodeAttention(device=dev, workspace_mb=32, num_qo_heads=32, num_kv_heads=8, head_dim=128,
                              page_size=16)
    host = [t.pin_memory() for t in (case["indptr"], case["indices"], case["last"])]
    be.plan_decode(paged_kv_indptr=host[0], paged_kv_indices=host[1], paged_kv_last_page_len=host[2])
    assert be._plan["shared"] == 128, be._plan  # the prefix was found on the host tables
    out = be.run_decode(case["q"], case["cache"])[:, :, 0].float().cpu().numpy()
    ref, _ = opd.paged_decode(case["q_host"].float().numpy(), case["cache_host"].float().numpy(),
                              case["indptr"].numpy(), case["indices"].numpy(), case["last"].numpy())
    rel = 2.0**-8 if dtype == torch.bfloat16 else 2.0**-11
    err = np.abs(out - ref)
    bound = 2e-3 + rel * np.abs(ref)
    assert (err <= bound).all(), f"max err {err.max():.3e}"
    print(f"[plan kernel forced] {dtype}: max err {err.max():.2e}", flush=True)
print("CHILD OK", flush=True)
"""


def test_forced_plan_kernel_plans_shared_prefix_batches_unshared():
    env = dict(os.environ, PAGELORA_DECODE_PLAN_KERNEL="1")
    proc = subprocess.run([sys.executable, "-u", "-c", CHILD], cwd=ROOT, env=env, stdout=subprocess.PIPE,
                          stderr=subprocess.STDOUT, text=True, timeout=300)
    print(proc.stdout[-4000:])
    assert proc.returncode == 0, proc.stdout[-4000:]
    assert "CHILD OK" in proc.stdout
