"""Adapter registry and weight binding on the host (CPU tensors, no shuffled
copies): where an adapter's A/B land in the stacked layout, zero deltas for
modules an adapter leaves out, growth of the stacks, and the registry's
reference-shaped API (multilora/runtime.py:257-375)."""

import pytest
import torch

from pagelora_amd.adapters import AdapterRegistry
from pagelora_amd.decoder import MODULES, DecoderConfig, DecoderWeights, projections

CFG = DecoderConfig(num_layers=2, hidden=64, num_qo_heads=4, num_kv_heads=2, head_dim=16, intermediate=96,
                    vocab=50, lora_rank=8, lora_alpha=16.0)


def _weights(n=1, seed=0):
    return DecoderWeights(CFG, n_adapters=n, device="cpu", dtype=torch.float32, seed=seed, shuffle=False)


def _adapter(seed, modules=MODULES, layers=range(CFG.num_layers)):
    g = torch.Generator().manual_seed(seed)
    outs = {m: o for _, _, mods in projections(CFG) for m, o in mods}
    ins = {m: fin for _, fin, mods in projections(CFG) for m, _ in mods}
    return {(l, m): (torch.randn((CFG.lora_rank, ins[m]), generator=g), torch.randn((outs[m], CFG.lora_rank), generator=g))
            for l in layers for m in modules}


def _base(w):
    layers = []
    for lw in w.layers:
        d = {"input_norm": lw.input_norm, "post_norm": lw.post_norm, "q_norm": lw.q_norm, "k_norm": lw.k_norm}
        for proj, _, mods in projections(CFG):
            W, row = getattr(lw, f"w_{proj}"), 0
            for m, o in mods:
                d[f"{m}_proj"] = W[row:row + o]
                row += o
        layers.append(d)
    return dict(embed=w.embed, final_norm=w.final_norm, lm_head=w.lm_head, layers=layers)


def test_from_tensors_reproduces_the_layout():
    w = _weights(n=2)
    adapters = [{(l, m): (lw.lora[m][0][a], lw.lora[m][1][a]) for l, lw in enumerate(w.layers) for m in MODULES}
                for a in range(2)]
    w2 = DecoderWeights.from_tensors(CFG, **_base(w), adapters=adapters, device="cpu", dtype=torch.float32,
                                     shuffle=False)
    for a, b in zip(w.layers, w2.layers):
        for proj, _, _ in projections(CFG):
            assert torch.equal(getattr(a, f"w_{proj}_ext"), getattr(b, f"w_{proj}_ext"))
        for m in MODULES:
            assert torch.equal(a.lora[m][1], b.lora[m][1])
            assert a.y_offset[m] == b.y_offset[m]


def test_set_adapter_in_place_writes_the_slot_rows():
    w = _weights(n=2)
    ext_ptr = w.layers[0].w_qkv_ext.data_ptr()
    before = [lw.w_qkv_ext.clone() for lw in w.layers]
    ad = _adapter(1)
    w.set_adapter(1, ad)
    r = CFG.lora_rank
    assert w.adapter_version == 0 and w.layers[0].w_qkv_ext.data_ptr() == ext_ptr  # in place
    for l, lw in enumerate(w.layers):
        for m in MODULES:
            A, B = ad[(l, m)]
            assert torch.equal(lw.lora[m][0][1], A) and torch.equal(lw.lora[m][1][1], B)
        # the A rows of slot 1 sit at y_offset + r .. + 2r of the stacked weight; slot 0 is untouched
        for m in ("q", "k", "v"):
            lo = lw.y_offset[m]
            assert torch.equal(lw.w_qkv_ext[lo + r: lo + 2 * r], ad[(l, m)][0])
            assert torch.equal(lw.w_qkv_ext[lo: lo + r], before[l][lo: lo + r])
        assert torch.equal(lw.w_qkv, before[l][: lw.w_qkv.shape[0]])


def test_modules_left_out_get_a_zero_delta():
    w = _weights(n=1)
    w.set_adapter(0, _adapter(2, modules=("q", "v")))  # the reference's default targets are a subset
    for lw in w.layers:
        for m in ("k", "o", "gate", "up", "down"):
            assert not lw.lora[m][0][0].any() and not lw.lora[m][1][0].any()
        assert lw.lora["q"][1][0].any()


def test_growth_keeps_values_and_changes_the_version():
    w = _weights(n=1)
    old = {(l, m): (lw.lora[m][0][0].clone(), lw.lora[m][1][0].clone()) for l, lw in enumerate(w.layers)
           for m in MODULES}
    base = [lw.w_gate_up.clone() for lw in w.layers]
    ad = _adapter(3)
    w.set_adapter(2, ad)
    assert w.n_adapters == 3 and w.adapter_version == 1
    for l, lw in enumerate(w.layers):
        assert torch.equal(lw.w_gate_up, base[l])
        for m in MODULES:
            assert torch.equal(lw.lora[m][0][0], old[(l, m)][0]) and torch.equal(lw.lora[m][1][0], old[(l, m)][1])
            assert not lw.lora[m][0][1].any() and not lw.lora[m][1][1].any()  # the skipped slot: zero
            assert torch.equal(lw.lora[m][0][2], ad[(l, m)][0])


def test_registry_mirrors_the_runtime_api():
    w = _weights(n=1)
    reg = AdapterRegistry(w)
    assert reg.list_logical_adapters() == ["general"] and reg.active_slot == 0
    ad = {(l, f"self_attn.{m}_proj"): v for (l, m), v in _adapter(4, modules=("q", "k", "v", "o")).items()}
    slot = reg.register_logical_adapter("tuned", ad)
    assert slot == 1 and reg.register_logical_adapter("tuned") == 1  # an existing name keeps its slot
    assert reg.flashinfer_graph_version == 1  # the stacks grew
    copy = reg.register_logical_adapter("copy", init_from="tuned")
    for lw in w.layers:
        for m in MODULES:
            assert torch.equal(lw.lora[m][0][copy], lw.lora[m][0][slot])
    reg.set_active("tuned")
    assert reg.row_adapters(3) == [1, 1, 1]
    reg.update_adapter("tuned", None)
    assert reg.adapter_versions["tuned"] == 1 and not w.layers[0].lora["q"][1][1].any()
    assert reg.flashinfer_graph_version == 2  # grew once more for "copy"; the update was in place
    with pytest.raises(KeyError):
        reg.set_active("missing")
    with pytest.raises(ValueError):
        w.set_adapter(0, {(0, "q"): (torch.zeros(3, 64), torch.zeros(64, 3))})  # wrong rank


def test_serve_state_export_and_load_round_trip():
    """export_serve_state / load_serve_state (multilora/runtime.py:570-607):
    the reference's keys, values of the adapter's slot, and a load into a new
    name registers it and reproduces the exported state exactly."""
    w = _weights(n=1)
    reg = AdapterRegistry(w)
    reg.update_adapter("general", _adapter(3))
    state = reg.export_serve_state("general")
    assert len(state) == CFG.num_layers * len(MODULES) * 2
    assert "layers.0.self_attn.q_proj.lora_serve_a" in state and "layers.1.mlp.down_proj.lora_serve_b" in state
    assert torch.equal(state["layers.1.mlp.gate_proj.lora_serve_a"], w.layers[1].lora["gate"][0][0])
    assert torch.equal(state["layers.0.self_attn.o_proj.lora_serve_b"], w.layers[0].lora["o"][1][0])
    v0 = w.adapter_version
    reg.load_serve_state("tuned", state)
    # registered from the default adapter (its version), then bumped by the load
    assert reg.list_logical_adapters() == ["general", "tuned"]
    assert reg.adapter_versions["tuned"] == reg.adapter_versions["general"] + 1
    assert w.adapter_version == v0 + 1  # the stacks grew to a second slot
    again = reg.export_serve_state("tuned")
    assert again.keys() == state.keys()
    for k in state:
        assert torch.equal(again[k], state[k]), k


def test_serve_state_load_partial_and_foreign_keys():
    """Keys of a known layer and module replace that A or B in place; the
    rest keep their values (a new name starts as a copy of the default
    adapter); keys the reference would skip are skipped."""
    w = _weights(n=2)
    reg = AdapterRegistry(w, logical_adapters=("general", "tuned"))
    reg.update_adapter("general", _adapter(4))
    reg.update_adapter("tuned", _adapter(5))
    before = reg.export_serve_state("tuned")
    g = torch.Generator().manual_seed(6)
    new_a = torch.randn(w.layers[1].lora["k"][0][1].shape, generator=g)
    new_b = torch.randn(w.layers[0].lora["up"][1][1].shape, generator=g)
    ptr = w.layers[1].lora["k"][0].data_ptr()
    reg.load_serve_state("tuned", {
        "layers.1.self_attn.k_proj.lora_serve_a": new_a,
        "layers.0.mlp.up_proj.lora_serve_b": new_b,
        "layers.0.mlp.up_proj.lora_serve_c": torch.zeros(1),   # unknown leaf
        "layers.7.self_attn.q_proj.lora_serve_a": torch.zeros(1),  # no such layer
        "layers.0.self_attn.rotary.lora_serve_a": torch.zeros(1),  # not a LoRA module
        "model.embed_tokens.weight": torch.zeros(1),
        "layers.x.mlp.up_proj.lora_serve_a": torch.zeros(1),
    })
    assert w.layers[1].lora["k"][0].data_ptr() == ptr  # written in place
    after = reg.export_serve_state("tuned")
    for k in before:
        if k == "layers.1.self_attn.k_proj.lora_serve_a":
            assert torch.equal(after[k], new_a)
        elif k == "layers.0.mlp.up_proj.lora_serve_b":
            assert torch.equal(after[k], new_b)
        else:
            assert torch.equal(after[k], before[k]), k
    # "general" is untouched; a new name starts from the default adapter
    reg.load_serve_state("third", {"layers.0.self_attn.v_proj.lora_serve_b": new_b[:, :0].new_zeros(
        w.layers[0].lora["v"][1][0].shape)})
    third, general = reg.export_serve_state("third"), reg.export_serve_state("general")
    for k in general:
        if k == "layers.0.self_attn.v_proj.lora_serve_b":
            assert not third[k].any()
        else:
            assert torch.equal(third[k], general[k]), k
