"""Per-layer carried-state cache of the decoder (model/statesdictcache.py).

The reference's ``StatesDictCache`` (model/statesdictcache.py:128-187) is a
HuggingFace ``Cache`` subclass holding one states dict and one seen-token
counter per layer.  The KVM decoder makes three calls on it:

* ``get_seq_length(layer_idx)``: tokens the layer has consumed,
* ``get_states(layer_idx)``: that layer's states dict,
* ``update(layer_idx, offset, states_dict)``: merge entries into the dict and
  advance the counter by ``offset`` (model/statesdictcache.py:19-82).

The KVM mixer and the MLP only store fixed-size entries (the decode cache
object and final-token tensors), so the dynamic-window keys the reference
also handles for other mixers (``k``/``v``/``swa_*``/``bswa_*``,
model/statesdictcache.py:28-77) are stored as given.  No HuggingFace
dependency: the class is a plain container.
"""

from __future__ import annotations

from typing import Any


class StatesDictCache:
    """One states dict and one seen-token counter per layer."""

    def __init__(self):
        self.layers: list[dict[str, Any]] = []
        self.seen: list[int] = []

    def _ensure(self, layer_idx: int) -> None:
        while len(self.layers) <= layer_idx:
            self.layers.append({})
            self.seen.append(0)

    def get_seq_length(self, layer_idx: int = 0) -> int:
        """Tokens layer ``layer_idx`` has consumed (model/statesdictcache.py:141-145)."""
        if layer_idx >= len(self.layers):
            return 0
        return self.seen[layer_idx]

    def get_states(self, layer_idx: int) -> dict[str, Any]:
        """The layer's states dict (model/statesdictcache.py:147-148)."""
        return self.update(layer_idx, offset=0, states_dict=None)

    def update(self, layer_idx: int, offset: int = 1, states_dict: dict[str, Any] | None = None,
               **_: Any) -> dict[str, Any]:
        """Merge ``states_dict`` into the layer's dict and advance its counter
        by ``offset`` (model/statesdictcache.py:150-187, 19-82)."""
        self._ensure(layer_idx)
        if states_dict:
            self.layers[layer_idx].update(states_dict)
        self.seen[layer_idx] += int(offset)
        return self.layers[layer_idx]

    def reset(self) -> None:
        self.layers.clear()
        self.seen.clear()

    def __len__(self) -> int:
        return len(self.layers)


__all__ = ["StatesDictCache"]
