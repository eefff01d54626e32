"""pl_decode_noalloc through the C ABI: the plan and run of one decode step
with the work list and split partials in the library's per-device scratch
array, against the existing pl_decode_plan + pl_decode_run on a caller
workspace.  Same kernels and plan, so outputs and LSE must be bit-identical;
checked on calls in a row (each smaller than the one before, so a stale work
list or partial would show): batches of 64 and 17 rows, planned by the plan
kernel into the scratch, then batches of up to 16 rows, whose items the
kernels derive from indptr.  A plan larger than the scratch maximum is
rejected before any launch.
"""

import math

import pytest
import torch

from pagelora_amd import _lib
from tests.gpu_cases import ragged_case, uniform_lens

pytestmark = pytest.mark.gpu

HQ, HKV, D, PS = 32, 8, 128, 16


def _tables(case, dev):
    return (case["indptr"].to(dev), case["indices"].to(dev), case["last"].to(dev))


def _args(case, tables, out, lse):
    q, cache = case["q"], case["cache"]
    indptr, indices, last = tables
    return dict(q=(q.data_ptr(), q.stride(0), q.stride(1)),
                kv=(cache[:, 0].data_ptr(), cache[:, 1].data_ptr(), cache.stride(0), cache.stride(2), cache.stride(3),
                    cache.shape[0]),
                o=(out.data_ptr(), out.stride(0), out.stride(1), lse.data_ptr()),
                tables=(indptr.data_ptr(), max(1, indices.numel()), indices.data_ptr(), last.data_ptr()),
                batch=q.shape[0], dtype=_lib.dtype_code(q.dtype))


def _noalloc(lib, a, target, stream):
    return lib.pl_decode_noalloc(*a["q"], *a["kv"], a["tables"][0], a["tables"][1], a["tables"][2], a["tables"][3],
                                 *a["o"], a["batch"], HQ, HKV, D, PS, 1.0 / math.sqrt(D), a["dtype"], target, 4,
                                 stream)


def _with_workspace(lib, a, target, ws, stream):
    st = lib.pl_decode_plan(a["tables"][0], a["batch"], a["tables"][1], HQ, D, target, 4, ws.data_ptr(), ws.numel(),
                            stream)
    if st:
        return st
    return lib.pl_decode_run(*a["q"], *a["kv"], a["tables"][2], a["tables"][3], *a["o"], a["batch"], HQ, HKV, D, PS,
                             1.0 / math.sqrt(D), a["dtype"], target, 0, ws.data_ptr(), ws.numel(), stream)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_noalloc_matches_workspace_entry(gpu_device, dtype):
    lib = _lib.load()
    stream = _lib.stream_handle(gpu_device)
    ws = torch.empty(64 << 20, dtype=torch.uint8, device=gpu_device)
    rows64 = uniform_lens(64, 1, 1024, seed=71)
    rows64[5] = 0
    calls = [  # (lens, target items): each call smaller than the one before
        # more than 16 rows: the plan kernel writes the work list, row table
        # and header into the scratch, and the next (smaller) plan must not
        # leave any of this one's items behind
        (rows64, 256),
        (uniform_lens(17, 1, 3000, seed=72), 128),
        ([4100, 1, 17, 300, 2047, 16, 0, 8192], 128),
        ([32768], 128),          # one row cut into many items: partials merged from the scratch
        ([700, 33, 5], 64),
    ]
    for i, (lens, target) in enumerate(calls):
        print(f"[noalloc] call {i}: lens {lens}, target {target}, {dtype}", flush=True)
        case = ragged_case(lens=lens, hq=HQ, hkv=HKV, head_dim=D, page_size=PS, dtype=dtype, device=gpu_device,
                           seed=40 + i, pool_extra=3)
        tables = _tables(case, gpu_device)
        outs = []
        for use_ws in (False, True):
            out = torch.full_like(case["q"], float("nan"))
            lse = torch.full(case["q"].shape[:2], float("nan"), dtype=torch.float32, device=gpu_device)
            a = _args(case, tables, out, lse)
            st = _with_workspace(lib, a, target, ws, stream) if use_ws else _noalloc(lib, a, target, stream)
            assert st == _lib.PL_OK, _lib.last_error()
            outs.append((out, lse))
        torch.cuda.synchronize()
        (o1, l1), (o2, l2) = outs
        assert torch.equal(o1, o2), f"call {i}: outputs differ"
        assert torch.equal(l1.isinf(), l2.isinf()) and torch.equal(l1[~l1.isinf()], l2[~l2.isinf()]), f"call {i}: lse"
        assert not torch.isnan(o1[torch.tensor(lens, device=gpu_device) > 0]).any()


def test_noalloc_rejects_plans_beyond_the_scratch(gpu_device):
    lib = _lib.load()
    batch, target = 4096, 256
    need = lib.pl_decode_workspace_size(batch, target, HQ, D)
    assert need > _lib.PL_DECODE_NOALLOC_MAX_BYTES
    st = lib.pl_decode_noalloc(None, 0, 0, None, None, 0, 0, 0, 1, None, 1, None, None, None, 0, 0, None, batch, HQ,
                               HKV, D, PS, 0.1, _lib.PL_DTYPE_BF16, target, 4, _lib.stream_handle(gpu_device))
    assert st == _lib.PL_ERR_WORKSPACE
    assert "maximum" in _lib.last_error()
