"""Rows retiring at EOS in the batched decode loop (the reference's
generate_batch_with_flashinfer_kvcache, model/flashinfer/generation.py:
967-1086): a row whose greedy pick is the EOS token keeps it as its last
token and is not decoded again; the others go on as a smaller batch, whose
graph is captured once per batch size (cuda_graph.py:525-526).

Checked against a run without EOS on the same prefilled rows: each row's
tokens are that run's up to and including its first EOS pick, then -1.  The
rows are short enough that every batch size splits them into the same
2-page items, and each kernel computes a row independently of the others,
so the continuing rows' tokens match bit for bit, eager and under graph
replay.
"""

import pytest
import torch

from pagelora_amd.decoder import DecoderConfig, DecoderWeights
from pagelora_amd.generation import BatchGenerator, prefill_requests
from pagelora_amd.kv_pool import PagedKVPool

pytestmark = pytest.mark.gpu

SMALL = DecoderConfig(num_layers=2, hidden=256, num_qo_heads=8, num_kv_heads=2, head_dim=64, intermediate=512,
                      vocab=1000, lora_rank=16, lora_alpha=32.0)
STEPS = 12
ADAPTERS = [0, 1, 1]


def _setup(dev):
    w = DecoderWeights(SMALL, n_adapters=2, device=dev, seed=3)
    pool = PagedKVPool(num_layers=SMALL.num_layers, capacity_pages=64, page_size=16, num_kv_heads=2, head_dim=64,
                       dtype=torch.bfloat16, device=dev)
    g = torch.Generator().manual_seed(8)
    prefix = torch.randint(0, SMALL.vocab, (32,), generator=g)
    prompts = [torch.randint(0, SMALL.vocab, (n,), generator=g) for n in (5, 17, 1)]
    reqs, first, _ = prefill_requests(w, pool, prompts, shared_prefix=prefix, adapters=ADAPTERS)
    return w, pool, reqs, first


def _expected(first, tokens, eos):
    out = torch.full_like(tokens, -1)
    for b in range(tokens.shape[0]):
        if int(first[b]) == eos:
            continue
        row = tokens[b].tolist()
        n = row.index(eos) + 1 if eos in row else len(row)
        out[b, :n] = tokens[b, :n]
    return out


def _rewind(reqs, lengths):
    for r, n in zip(reqs, lengths):
        r.length -= n


def test_rows_retire_at_eos(gpu_device):
    w, pool, reqs, first = _setup(gpu_device)
    ref = BatchGenerator(w, pool, workspace_mb=8, use_graph=False).generate(reqs, first, STEPS, adapters=ADAPTERS)
    _rewind(reqs, [STEPS] * len(reqs))
    T0, first_h = ref.tokens, first.cpu()
    # an EOS that row 1 picks mid-run while rows 0 and 2 go on past it, and
    # one that is row 2's first token (row 2 is then never decoded)
    eos_mid = None
    for j in range(3, 9):
        t = int(T0[1, j])
        if t not in T0[1, :j].tolist() and t not in first_h.tolist() and \
                t not in T0[0, : j + 2].tolist() and t not in T0[2, : j + 2].tolist():
            eos_mid = t
            break
    assert eos_mid is not None, f"no usable EOS in {T0.tolist()}"
    cases = [eos_mid]
    if int(first_h[2]) not in first_h[:2].tolist():
        cases.append(int(first_h[2]))
    for eos in cases:
        want = _expected(first_h, T0, eos)
        for use_graph in (False, True):
            print(f"[eos] eos {eos}, graph {use_graph}", flush=True)
            gen = BatchGenerator(w, pool, workspace_mb=8, use_graph=use_graph)
            res = gen.generate(reqs, first, STEPS, adapters=ADAPTERS, eos_token_id=eos)
            _rewind(reqs, res.extra["lengths"])
            assert torch.equal(res.tokens, want), f"eos {eos} graph {use_graph}: {res.tokens.tolist()} != {want.tolist()}"
            sizes = res.extra["batch"]
            assert sizes == sorted(sizes, reverse=True) and sum(sizes) == res.generated_tokens
            assert res.extra["lengths"] == (want >= 0).sum(dim=1).tolist()
            if use_graph:
                assert res.used_graph and res.graph_captures == len(set(sizes))
    with pytest.raises(ValueError, match="device_tables"):
        BatchGenerator(w, pool, workspace_mb=8).generate(reqs, first, 2, eos_token_id=eos_mid, device_tables=True)
