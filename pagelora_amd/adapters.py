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
