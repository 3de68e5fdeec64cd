"""Preallocated single-token decode state of the HIP KVM mixer.

Mirrors the carried-state container of the reference,
``TritonKVMDecodeCache`` (model/kvm_triton_decode.py:34-400), and its
snapshot type ``DecodeCacheSnapshot`` (:19-31): same constructor, same
``reset_`` / ``append_recent_`` / ``logical_recent`` / ``logical_state_dict``
/ ``persistent_metadata`` / ``state_length_after_cycle`` API and the eager
state-dict keys (model/kvm_mixer.py:518-525).

Layout (device, bf16 unless noted; rows = batch * kv_heads):
  state_k, state_v, state_k_attn, state_v_attn   [rows, capacity, D]
  state_vlen                                     [rows, capacity] fp32
  recent_k, recent_v                             [rows, W, D]   W = n_bswa * chunk_len
  recent_gate                                    [rows, W]
The window is a modular ring of exactly W rows: logical window row i sits at
ring row (recent_start + i) % W.  The reference double-maps a 2W ring so that
the window is contiguous for its kernels; the HIP kernels index modulo W
instead, so each new token is written once.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Any

import torch

from . import _lib
from .schedule import state_length_after_cycle as _cycle_len


@dataclass(frozen=True)
class DecodeCacheSnapshot:
    """Immutable tensors and scalar bookkeeping used to reset timed trials."""

    state_k: torch.Tensor       # [B, Hkv, S, D]
    state_v: torch.Tensor       # [B, Hkv, S, Dv]
    state_vlen: torch.Tensor    # [B, Hkv, S, 1]
    recent_k: torch.Tensor      # [B, Hkv, R, D]
    recent_v: torch.Tensor      # [B, Hkv, R, Dv]
    recent_gate: torch.Tensor   # [B, Hkv, R, 1]
    total_len: int
    state_coverage_len: int
    recent_begin: int


class KVMDecodeCache:
    """Optimized one-token cache used by the HIP KVM mixer.

    ``state_capacity`` is a capacity hint; adaptive schedules grow the state
    at an update boundary (model/kvm_triton_decode.py:202-239).  Ordinary
    token steps allocate nothing.
    """

    cache_representation = "preallocated modular window ring"

    def __init__(self, mixer: Any, snapshot: DecodeCacheSnapshot | None, *, state_capacity: int,
                 _device: torch.device | None = None, _batch: int | None = None) -> None:
        self.mixer = mixer
        if snapshot is not None:
            if not snapshot.state_k.is_cuda:
                raise RuntimeError("HIP KVM decode requires ROCm device tensors")
            device = snapshot.state_k.device
            self.batch = int(snapshot.state_k.size(0))
            self.dtype = snapshot.state_k.dtype
        else:
            device = _device
            self.batch = int(_batch)
            self.dtype = torch.bfloat16
        if self.dtype != torch.bfloat16:
            raise ValueError("the HIP KVM decode cache stores bfloat16 state")
        self.device = device
        self.kv_heads = int(mixer.num_key_value_heads)
        self.q_heads = int(mixer.num_attention_heads)
        self.head_dim = int(mixer.d_qk_head)
        self.value_dim = int(mixer.d_v_head)
        self.chunk_len = int(mixer.chunk_len)
        self.ring_capacity = int(mixer.n_bswa_chunks * mixer.chunk_len)
        self.state_capacity = int(state_capacity)
        self.kv_rows = self.batch * self.kv_heads
        if snapshot is not None:
            if self.state_capacity < int(snapshot.state_k.size(2)):
                raise ValueError("state capacity is smaller than the initial state")
            if int(snapshot.recent_k.size(2)) > self.ring_capacity:
                raise ValueError("initial recent front exceeds the ring capacity")

        self._alloc_state(self.state_capacity)
        W = self.ring_capacity
        bf = dict(device=device, dtype=torch.bfloat16)
        self.recent_k = torch.empty(self.kv_rows, W, self.head_dim, **bf)
        self.recent_v = torch.empty(self.kv_rows, W, self.value_dim, **bf)
        self.recent_gate = torch.empty(self.kv_rows, W, **bf)
        self.out = torch.empty(self.batch, self.q_heads, 1, self.value_dim, **bf)
        # Last update's routing: slot of every overflow token, append flags.
        self.route_by_token = torch.full((self.kv_rows, self.chunk_len), -1, device=device, dtype=torch.int32)
        self.append_by_token = torch.zeros((self.kv_rows, self.chunk_len), device=device, dtype=torch.int32)
        self.layer = mixer._layer_struct(self.batch, device)
        self.direct_layer = mixer._layer_struct(self.batch, device, gate_initial=False)
        lib = _lib.load()
        self.update_workspace = torch.empty(
            int(lib.kvm_update_workspace_bytes(self.layer.ref(), self.chunk_len)), device=device, dtype=torch.uint8)
        self._alloc_decode_workspace()
        self.total_len = 0
        self.state_len = 0
        self.state_coverage_len = 0
        self.recent_begin = 0
        self.recent_start = 0
        self.recent_len = 0
        self.update_count = 0
        if snapshot is not None:
            self.reset_(snapshot)

    # -- storage ------------------------------------------------------------
    def _alloc_state(self, cap: int) -> None:
        bf = dict(device=self.device, dtype=torch.bfloat16)
        self.state_k = torch.empty(self.kv_rows, cap, self.head_dim, **bf)
        self.state_v = torch.empty(self.kv_rows, cap, self.value_dim, **bf)
        self.state_k_attn = torch.empty_like(self.state_k)
        self.state_v_attn = torch.empty_like(self.state_v)
        self.state_vlen = torch.empty(self.kv_rows, cap, device=self.device, dtype=torch.float32)

    def _alloc_decode_workspace(self) -> None:
        lib = _lib.load()
        n = int(lib.kvm_decode_workspace_bytes(self.layer.ref(), self.state_capacity + self.ring_capacity))
        self.decode_workspace = torch.empty(max(n, 256), device=self.device, dtype=torch.uint8)

    def state_struct(self) -> _lib.KvmState:
        return _lib.state_struct(self.state_k, self.state_v, self.state_vlen, self.state_k_attn,
                                 self.state_v_attn, self.state_capacity)

    def _reserve_state_capacity(self, required: int) -> None:
        """Grow adaptive-state storage at a chunk boundary when necessary."""
        required = int(required)
        if required <= self.state_capacity:
            return
        if required > int(self.mixer.max_state_len):
            raise RuntimeError(
                f"HIP KVM decode requires {required} state rows, exceeding "
                f"the configured maximum {self.mixer.max_state_len}"
            )
        look = self.state_length_after_cycle(self.mixer, self.total_len + 1, required, self.ring_capacity)
        new_cap = min(int(self.mixer.max_state_len), max(required, look))
        old = (self.state_k, self.state_v, self.state_k_attn, self.state_v_attn, self.state_vlen)
        n = self.state_len
        self._alloc_state(new_cap)
        for dst, src in zip((self.state_k, self.state_v, self.state_k_attn, self.state_v_attn, self.state_vlen), old):
            dst[:, :n].copy_(src[:, :n])
        self.state_capacity = new_cap
        self._alloc_decode_workspace()

    @staticmethod
    def state_length_after_cycle(mixer: Any, total_len: int, state_len: int, cycle_len: int | None = None) -> int:
        """Return the required state capacity for a bounded decode interval."""
        return _cycle_len(mixer.state_budget, mixer.chunk_len, mixer.n_bswa_chunks, total_len, state_len, cycle_len)

    # -- state transitions ----------------------------------------------------
    def reset_(self, snapshot: DecodeCacheSnapshot) -> None:
        """Restore a snapshot; callers keep this outside measured GPU events."""
        S = int(snapshot.state_k.size(2))
        R = int(snapshot.recent_k.size(2))
        if S > self.state_capacity or R > self.ring_capacity:
            raise ValueError("snapshot does not fit the preallocated decode cache")
        rows = self.kv_rows
        self.state_k[:, :S].copy_(snapshot.state_k.reshape(rows, S, self.head_dim))
        self.state_v[:, :S].copy_(snapshot.state_v.reshape(rows, S, self.value_dim))
        self.state_vlen[:, :S].copy_(snapshot.state_vlen.reshape(rows, S).float())
        lib = _lib.load()
        st = self.state_struct()
        _lib.check(lib.kvm_state_refresh(self.layer.ref(), st, 0, S, _lib.stream_handle(self.device)),
                   "kvm_state_refresh")
        self.recent_k[:, :R].copy_(snapshot.recent_k.reshape(rows, R, self.head_dim))
        self.recent_v[:, :R].copy_(snapshot.recent_v.reshape(rows, R, self.value_dim))
        self.recent_gate[:, :R].copy_(snapshot.recent_gate.reshape(rows, R))
        self.total_len = int(snapshot.total_len)
        self.state_len = S
        self.state_coverage_len = int(snapshot.state_coverage_len)
        self.recent_begin = int(snapshot.recent_begin)
        self.recent_start = 0
        self.recent_len = R
        self.update_count = 0
        self.route_by_token.fill_(-1)
        self.append_by_token.zero_()

    def append_recent_(self, new_k: torch.Tensor, new_v: torch.Tensor, new_gate: torch.Tensor, *,
                       total_len: int, recent_begin: int) -> None:
        """Append one token to the window ring and update the bookkeeping."""
        evicted = int(recent_begin) - self.recent_begin
        if evicted < 0 or evicted > self.recent_len:
            raise AssertionError("invalid recent-window transition")
        if evicted:
            self.recent_start = (self.recent_start + evicted) % self.ring_capacity
            self.recent_len -= evicted
        if self.recent_len >= self.ring_capacity:
            raise AssertionError("recent ring append would exceed capacity")
        pos = (self.recent_start + self.recent_len) % self.ring_capacity
        seq, keep = _lib.seq4(new_k, new_v, new_gate)
        lib = _lib.load()
        _lib.check(lib.kvm_ring_write(self.layer.ref(), seq, self.recent_k.data_ptr(), self.recent_v.data_ptr(),
                                      self.recent_gate.data_ptr(), self.ring_capacity, pos,
                                      _lib.stream_handle(self.device)), "kvm_ring_write")
        del keep
        self.recent_len += 1
        self.total_len = int(total_len)
        self.recent_begin = int(recent_begin)

    # -- inspection -----------------------------------------------------------
    def _ring_rows(self, x: torch.Tensor) -> torch.Tensor:
        b, e = self.recent_start, self.recent_start + self.recent_len
        if e <= self.ring_capacity:
            return x[:, b:e]
        return torch.cat([x[:, b:], x[:, : e - self.ring_capacity]], dim=1)

    def logical_recent(self) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
        """The logical window (views, or copies when it wraps the ring)."""
        return (self._ring_rows(self.recent_k), self._ring_rows(self.recent_v), self._ring_rows(self.recent_gate))

    def logical_state_dict(self) -> dict[str, Any]:
        """The logical cache contents in the eager state-dict keys."""
        rk, rv, rg = self.logical_recent()
        m = self.mixer
        B, H, S, R = self.batch, self.kv_heads, self.state_len, self.recent_len
        return {
            m._CACHE_S_K: self.state_k[:, :S].reshape(B, H, S, self.head_dim),
            m._CACHE_S_V: self.state_v[:, :S].reshape(B, H, S, self.value_dim),
            m._CACHE_S_VLEN: self.state_vlen[:, :S].reshape(B, H, S, 1),
            m._CACHE_STATE_COVERAGE_LEN: self.state_coverage_len,
            m._CACHE_BSWA_BEGIN: self.recent_begin,
            m._CACHE_BSWA_K: rk.reshape(B, H, R, self.head_dim),
            m._CACHE_BSWA_V: rv.reshape(B, H, R, self.value_dim),
            m._CACHE_BSWA_MERGE_GATE: rg.reshape(B, H, R, 1),
        }

    def persistent_metadata(self) -> dict[str, Any]:
        return {
            "total_len": self.total_len,
            "active_state_len": self.state_len,
            "state_capacity": self.state_capacity,
            "state_coverage_len": self.state_coverage_len,
            "recent_begin": self.recent_begin,
            "recent_start": self.recent_start,
            "recent_len": self.recent_len,
            "recent_capacity": self.ring_capacity,
            "update_count": self.update_count,
            "cache_representation": self.cache_representation,
        }


# The reference's name for the same container.
TritonKVMDecodeCache = KVMDecodeCache

__all__ = ["KVMDecodeCache", "TritonKVMDecodeCache", "DecodeCacheSnapshot"]
