"""Logical LoRA adapters of the decoder: registry and active binding.

Counterpart of the serve side of the reference's ``LoRARuntime``
(multilora/runtime.py): ``register_logical_adapter`` (:257-292),
``set_active`` (:319-359) with its broadcast of the active adapter's A/B
into every wrapped module (``_broadcast_active``, :138-174), and the graph
version that invalidates captured decode graphs (:371-375, bumped by
``_clear_flashinfer_effective_weight_caches``, :697-713).

On MI355X every registered adapter stays resident in the decoder's stacked
layout (``DecoderWeights``: each adapter a slot of the A rows under the base
weights and of the B stacks), so:

* registering or updating an adapter writes its slot in place (A rows, their
  blocks of the shuffled decode weights, B and its chunked copy).  Graphs
  read weights by address, so graphs captured earlier stay valid and see the
  new values; only growing the stacks past their slots moves buffers, which
  changes ``DecoderWeights.adapter_version`` and so the graph key;
* switching the active adapter copies no weights: the decode kernels read
  the active slot (the bound adapter of the step, part of the graph key), so
  a switch replays the graph cached for that slot, or captures it once;
* rows of one batch may also use different adapters (per-row slots), which
  the reference's one-adapter runtime cannot express.
"""

from __future__ import annotations

from typing import Mapping

import torch

from .decoder import MODULES, DecoderWeights, module_key

# Module paths inside a decoder layer, as the reference's wrapped modules are
# named (layer.named_modules() of an HF Qwen3/Llama layer, runtime.py:100-115)
# in its serve-state keys "layers.{i}.{path}.lora_serve_a|b".
SERVE_STATE_MODULES = {"q": "self_attn.q_proj", "k": "self_attn.k_proj", "v": "self_attn.v_proj",
                       "o": "self_attn.o_proj", "gate": "mlp.gate_proj", "up": "mlp.up_proj",
                       "down": "mlp.down_proj"}


class AdapterRegistry:
    """Named adapters in the slots of one :class:`DecoderWeights`.

    ``logical_adapters`` name the weights' existing slots in order (slot 0 =
    the first name); they keep the values the weights hold.
    """

    def __init__(self, weights: DecoderWeights, logical_adapters=("general",),
                 default_logical_adapter: str = "general") -> None:
        if len(logical_adapters) > weights.n_adapters:
            raise ValueError(f"{len(logical_adapters)} names for {weights.n_adapters} adapter slots")
        self.weights = weights
        self.logical_adapter_names: list[str] = list(logical_adapters)
        self._slots = {name: i for i, name in enumerate(logical_adapters)}
        self.adapter_versions: dict[str, int] = {name: 0 for name in logical_adapters}
        if default_logical_adapter not in self._slots:
            raise KeyError(f"Unknown logical adapter: {default_logical_adapter}")
        self.default_logical_adapter = default_logical_adapter
        self.active_logical_adapter_name = default_logical_adapter

    # ------------------------------------------------------------ registry
    def slot(self, name: str) -> int:
        if name not in self._slots:
            raise KeyError(f"Unknown logical adapter: {name}")
        return self._slots[name]

    def list_logical_adapters(self) -> list[str]:
        return list(self.logical_adapter_names)

    def _values_of(self, slot: int) -> dict:
        return {(li, m): (lw.lora[m][0][slot], lw.lora[m][1][slot])
                for li, lw in enumerate(self.weights.layers) for m in MODULES}

    def register_logical_adapter(self, adapter_name: str, adapter: Mapping | None = None, *,
                                 init_from: str | None = None) -> int:
        """Register ``adapter_name`` in the next free slot and return the slot
        (runtime.py:257-292; an existing name keeps its slot and values).

        Values: ``adapter`` ({(layer, module): (A [r, in], B [out, r])},
        modules as "q".."down" or their *_proj names), else a copy of
        ``init_from``'s, else a zero delta (the reference's init_lora_pair
        makes B = 0, linear.py:234-254).
        """
        if adapter_name in self._slots:
            return self._slots[adapter_name]
        slot = len(self.logical_adapter_names)
        if adapter is None and init_from is not None:
            adapter = self._values_of(self.slot(init_from))
        self.weights.set_adapter(slot, self._normalized(adapter))
        self._slots[adapter_name] = slot
        self.logical_adapter_names.append(adapter_name)
        self.adapter_versions[adapter_name] = self.adapter_versions.get(init_from, 0) if init_from else 0
        return slot

    def update_adapter(self, adapter_name: str, adapter: Mapping | None) -> None:
        """Write new values for a registered adapter into its slot, in place
        (captured graphs stay valid; steps enqueued afterwards use them)."""
        self.weights.set_adapter(self.slot(adapter_name), self._normalized(adapter))
        self.adapter_versions[adapter_name] += 1

    # --------------------------------------------------------- serve state
    def export_serve_state(self, adapter_name: str) -> dict[str, torch.Tensor]:
        """One adapter's A/B as host tensors under the reference's keys
        "layers.{i}.{module path}.lora_serve_a" / "...lora_serve_b"
        (runtime.py:570-579): A [r, in], B [out, r] of every layer and module."""
        slot = self.slot(adapter_name)
        state: dict[str, torch.Tensor] = {}
        for li, lw in enumerate(self.weights.layers):
            for m in MODULES:
                prefix = f"layers.{li}.{SERVE_STATE_MODULES[m]}"
                state[f"{prefix}.lora_serve_a"] = lw.lora[m][0][slot].detach().cpu().clone()
                state[f"{prefix}.lora_serve_b"] = lw.lora[m][1][slot].detach().cpu().clone()
        return state

    def load_serve_state(self, adapter_name: str, state: Mapping[str, torch.Tensor]) -> None:
        """Load an adapter from such a state dict (runtime.py:581-607): an
        unknown name is registered first as a copy of the default adapter;
        keys that name a known layer and module replace that A or B, every
        other key is ignored (as the reference skips them); the values go
        into the adapter's slot in place and its version moves on."""
        if adapter_name not in self._slots:
            self.register_logical_adapter(adapter_name, init_from=self.default_logical_adapter)
        slot = self.slot(adapter_name)
        values = {key: list(ab) for key, ab in self._values_of(slot).items()}
        for key, tensor in state.items():
            parts = key.split(".")
            if len(parts) < 4 or parts[0] != "layers" or not parts[1].isdigit():
                continue
            leaf = parts[-1]
            try:
                module = module_key(".".join(parts[2:-1]))
            except KeyError:
                continue
            pair = values.get((int(parts[1]), module))
            if pair is None:
                continue
            if leaf == "lora_serve_a":
                pair[0] = torch.as_tensor(tensor)
            elif leaf == "lora_serve_b":
                pair[1] = torch.as_tensor(tensor)
        # set_adapter copies into the slot; the unchanged entries are views of
        # it, so cloned first
        self.weights.set_adapter(slot, {k: (A.clone(), B.clone()) for k, (A, B) in values.items()})
        self.adapter_versions[adapter_name] += 1

    @staticmethod
    def _normalized(adapter: Mapping | None) -> dict | None:
        if adapter is None:
            return None
        out = {}
        for key, (A, B) in adapter.items():
            layer, module = key
            out[(int(layer), module_key(module))] = (torch.as_tensor(A), torch.as_tensor(B))
        return out

    # -------------------------------------------------------------- active
    def set_active(self, adapter_name: str) -> None:
        """Make ``adapter_name`` the adapter every row decodes with
        (runtime.py:319-359, serve role)."""
        self.slot(adapter_name)
        self.active_logical_adapter_name = adapter_name

    @property
    def active_slot(self) -> int:
        return self._slots[self.active_logical_adapter_name]

    def row_adapters(self, batch: int) -> list[int]:
        """Per-row slots of a batch that decodes with the active adapter."""
        return [self.active_slot] * batch

    @property
    def flashinfer_graph_version(self) -> int:
        """Changes when captured decode graphs must be recaptured: only when
        the adapter stacks moved (a switch of the active adapter picks the
        graph of its slot instead)."""
        return self.weights.adapter_version
