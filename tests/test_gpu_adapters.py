"""Binding adapters into the fused decoder between generate() calls (the
reference's register_logical_adapter / set_active, multilora/runtime.py:
257-375), on the GPU:

* an update written in place into the active slot: the captured graph is
  replayed as it is (no recapture), and its tokens and logits equal an eager
  run of the same sequence bit for bit;
* a new adapter registered past the stacked slots (buffers move): exactly
  one new capture, again equal to eager;
* the shuffled decode weights after an in-place update equal a fresh shuffle
  of weights built with that adapter from the start;
* one decode step on the new adapter, stage by stage, against the oracle on
  the A/B that were bound (tests/stage_check.py).
"""

import pytest
import torch

from pagelora_amd.adapters import AdapterRegistry
from pagelora_amd.decoder import MODULES, DecoderConfig, DecoderWeights, projections
from pagelora_amd.generation import BatchGenerator, prefill_requests
from pagelora_amd.kv_pool import PagedKVPool
from tests.stage_check import stage_check

pytestmark = pytest.mark.gpu

# head_dim 128 and GQA 4: the decode layers fold the q/k/v epilogue into attention
CFG = DecoderConfig(num_layers=2, hidden=512, num_qo_heads=4, num_kv_heads=1, head_dim=128, intermediate=512,
                    vocab=1000, lora_rank=16, lora_alpha=32.0)


# rank 8: an adapter slot's A rows start inside a 16-row block of the
# shuffled weight (slot 1 of a module at rows base + 8 .. + 16), so a slot
# write patches part of a block
CFG_R8 = DecoderConfig(num_layers=2, hidden=512, num_qo_heads=4, num_kv_heads=1, head_dim=128, intermediate=512,
                       vocab=1000, lora_rank=8, lora_alpha=16.0)


def _adapter(seed, dev, modules=MODULES, scale=1.0, cfg=CFG):
    g = torch.Generator().manual_seed(seed)
    outs = {m: o for _, _, mods in projections(cfg) for m, o in mods}
    ins = {m: fin for _, fin, mods in projections(cfg) for m, _ in mods}
    r = cfg.lora_rank
    return {(l, m): ((torch.randn((r, ins[m]), generator=g) * ins[m] ** -0.5).to(torch.bfloat16).to(dev),
                     (torch.randn((outs[m], r), generator=g) * 0.02 * scale).to(torch.bfloat16).to(dev))
            for l in range(cfg.num_layers) for m in modules}


def _scenario(dev, use_graph):
    """prefill + 8 steps on "general", an in-place update of "general" + 8
    steps, a new adapter "tuned" (stacks grow) + 8 steps."""
    w = DecoderWeights(CFG, n_adapters=1, device=dev, seed=1)
    reg = AdapterRegistry(w)
    pool = PagedKVPool(num_layers=CFG.num_layers, capacity_pages=64, page_size=16, num_kv_heads=1, head_dim=128,
                       dtype=torch.bfloat16, device=dev)
    g = torch.Generator().manual_seed(3)
    prompts = [torch.randint(0, CFG.vocab, (n,), generator=g) for n in (21, 40, 3)]
    reqs, first, _ = prefill_requests(w, pool, prompts)
    gen = BatchGenerator(w, pool, workspace_mb=8, use_graph=use_graph)
    out = {}
    r1 = gen.generate(reqs, first, 8, adapters=reg.row_adapters(3), keep_logits=True)
    out["before"] = (r1.tokens, r1.extra["logits"].cpu(), r1.graph_captures)
    reg.update_adapter("general", _adapter(10, dev))
    r2 = gen.generate(reqs, r1.tokens[:, -1].to(dev), 8, adapters=reg.row_adapters(3), keep_logits=True)
    out["updated"] = (r2.tokens, r2.extra["logits"].cpu(), r2.graph_captures)
    tuned = _adapter(20, dev, modules=("q", "k", "v", "o"), scale=3.0)
    reg.register_logical_adapter("tuned", tuned)
    reg.set_active("tuned")
    r3 = gen.generate(reqs, r2.tokens[:, -1].to(dev), 8, adapters=reg.row_adapters(3), keep_logits=True)
    out["tuned"] = (r3.tokens, r3.extra["logits"].cpu(), r3.graph_captures)
    return out, (w, pool, reqs, r3.tokens[:, -1].to(dev), tuned)


def test_bound_adapters_graph_equals_eager(gpu_device):
    eager, _ = _scenario(gpu_device, use_graph=False)
    graph, (w, pool, reqs, last, tuned) = _scenario(gpu_device, use_graph=True)
    for phase in ("before", "updated", "tuned"):
        assert torch.equal(graph[phase][0], eager[phase][0]), f"{phase}: tokens"
        assert torch.equal(graph[phase][1], eager[phase][1]), f"{phase}: logits"
    # the in-place update reused the captured graph; the new slot captured exactly once more
    assert graph["before"][2] == 1 and graph["updated"][2] == 1 and graph["tuned"][2] == 2
    # one more step on "tuned", stage by stage, vs the oracle on the bound A/B
    stage_check(w, pool, reqs, last, gpu_device, slot=1, adapter=tuned)


@pytest.mark.parametrize("cfg,slots", [(CFG, 2), (CFG_R8, 3)], ids=["rank16", "rank8"])
def test_in_place_update_matches_a_fresh_shuffle(gpu_device, cfg, slots):
    w = DecoderWeights(cfg, n_adapters=slots, device=gpu_device, seed=4)
    new = _adapter(30, gpu_device, cfg=cfg)
    w.set_adapter(1, new)
    adapters = [{(l, m): (lw.lora[m][0][a], lw.lora[m][1][a]) for l, lw in enumerate(w.layers) for m in MODULES}
                for a in range(slots)]
    adapters[1] = new
    layers = []
    for lw in w.layers:
        d = {"input_norm": lw.input_norm, "post_norm": lw.post_norm, "q_norm": lw.q_norm, "k_norm": lw.k_norm}
        for proj, _, mods in projections(cfg):
            W, row = getattr(lw, f"w_{proj}"), 0
            for m, o in mods:
                d[m] = W[row:row + o]
                row += o
        layers.append(d)
    fresh = DecoderWeights.from_tensors(cfg, embed=w.embed, final_norm=w.final_norm, lm_head=w.lm_head,
                                        layers=layers, adapters=adapters, device=gpu_device)
    torch.cuda.synchronize()
    for a, b in zip(w.layers, fresh.layers):
        for proj in ("qkv", "o", "gate_up", "down"):
            assert torch.equal(a.shuffled[proj].data, b.shuffled[proj].data), proj
        for m in ("o", "down"):
            assert torch.equal(a.lora_b8[m], b.lora_b8[m]), m
