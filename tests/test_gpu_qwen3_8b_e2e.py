"""End-to-end decode at the Qwen3-8B shape (36 layers, hidden 4096, 32/8
heads, head_dim 128, intermediate 12288, vocab 151936, bf16, rank-16
no-merge LoRA on all seven modules, random init), on the two workloads the
end-to-end tok/s is quoted on:

  shared4  4 rows behind a 2048-token prefix held in shared pages, each with
           its own 64-token suffix, 16 greedy steps
  long32k  1 row at 32768 tokens, 4 greedy steps

For each:
  (a) hipGraph replay == eager: tokens and every step's logits bit-identical
      (the reference's eager-vs-graph gate, scripts/check_inference_correctness.py:17-61,
      here exact);
  (b) the page table grown on the device inside the captured step == the
      host-packed table: the same tokens, and the final device table equals
      the host's packing of the grown rows;
  (c) layer 0 (and layer 1's input) of the first decode step, stage by
      stage, against the float64 oracle applied to the kernels' own stored
      inputs of each stage (tests/stage_check.py; the stages of
      layer_runner.py:340-412).  Bar: 2e-3 + one bf16 rounding of the output
      (2^-8 relative), plus one rounding of an intermediate a stage rounds
      before its output, carried to the output.
"""

import gc

import pytest
import torch

from pagelora_amd.decoder import QWEN3_8B, DecoderWeights
from pagelora_amd.generation import BatchGenerator, prefill_requests
from pagelora_amd.kv_pool import PagedKVPool
from tests.stage_check import stage_check

pytestmark = [pytest.mark.gpu, pytest.mark.timeout(600)]

CFG = QWEN3_8B
PS = 16

WORKLOADS = {
    "shared4": dict(prefix_len=2048, suffix_len=64, rows=4, steps=16),
    "long32k": dict(prefix_len=0, suffix_len=32768, rows=1, steps=4),
}


@pytest.fixture(scope="module")
def weights(gpu_device):
    print("[qwen3-8b] building 36-layer random-init weights", flush=True)
    w = DecoderWeights(CFG, n_adapters=1, device=gpu_device, seed=0)
    torch.cuda.synchronize()
    yield w
    del w
    gc.collect()
    torch.cuda.empty_cache()


def _fresh(w, dev, prefix_len, suffix_len, rows, steps, seed=5):
    """A new pool with the workload's rows prefilled (deterministic: every
    call gives the same caches and first tokens)."""
    pages = (prefix_len + rows * (suffix_len + steps + 2 * PS)) // PS + 8 * rows + 8
    pool = PagedKVPool(num_layers=CFG.num_layers, capacity_pages=pages, page_size=PS, num_kv_heads=CFG.num_kv_heads,
                       head_dim=CFG.head_dim, dtype=torch.bfloat16, device=dev)
    g = torch.Generator().manual_seed(seed)
    prefix = torch.randint(0, CFG.vocab, (prefix_len,), generator=g) if prefix_len else None
    prompts = [torch.randint(0, CFG.vocab, (suffix_len,), generator=g) for _ in range(rows)]
    reqs, first, _ = prefill_requests(w, pool, prompts, shared_prefix=prefix)
    return pool, reqs, first


@pytest.mark.parametrize("workload", sorted(WORKLOADS))
def test_qwen3_8b_decode(weights, gpu_device, workload):
    kw = WORKLOADS[workload]
    steps = kw["steps"]
    dev = gpu_device
    print(f"[qwen3-8b] {workload}: stage check of layer 0", flush=True)
    pool, reqs, first = _fresh(weights, dev, **kw)
    stage_check(weights, pool, reqs, first, dev)
    del pool, reqs
    runs = {}
    for name, use_graph, device_tables in (("eager", False, False), ("graph", True, False),
                                           ("graph_device_tables", True, True)):
        print(f"[qwen3-8b] {workload}: {name}, {steps} steps", flush=True)
        pool, reqs, first = _fresh(weights, dev, **kw)
        gen = BatchGenerator(weights, pool, use_graph=use_graph)
        res = gen.generate(reqs, first, steps, device_tables=device_tables, keep_logits=True)
        assert res.used_graph == use_graph
        if use_graph:
            assert res.graph_captures == 1 and res.graph_replays == steps
        if device_tables:
            indptr, indices, last = pool.tables(reqs)
            ip_buf, ind_buf, last_buf = gen.backend._decode_graph_buffers
            assert ip_buf.tolist() == indptr.tolist()
            assert ind_buf[: indptr[-1]].tolist() == indices.tolist()
            assert last_buf.tolist() == last.tolist()
        runs[name] = (res.tokens, res.extra["logits"].cpu())
        del gen, pool, reqs, res
        gc.collect()
        torch.cuda.empty_cache()
    tok_e, log_e = runs["eager"]
    for name in ("graph", "graph_device_tables"):
        tok, log = runs[name]
        assert torch.equal(tok, tok_e), f"{name}: tokens differ from eager"
        assert torch.equal(log, log_e), f"{name}: logits differ from eager (max {(log - log_e).abs().max()})"
