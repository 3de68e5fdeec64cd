"""Device-resident carried state for single-token KVM decode.

Public surface kept compatible with the reference's cache
(``TritonKVMDecodeCache``, model/kvm_triton_decode.py:34-400, and its
``DecodeCacheSnapshot``, :19-31): the constructor arguments, the method
names ``reset_``, ``append_recent_``, ``logical_recent``,
``logical_state_dict``, ``persistent_metadata``, ``state_length_after_cycle``
and the eager state-dict keys (model/kvm_mixer.py:518-525), so callers and
the reference's benchmark harness can drive either one.

Device tensors (bf16 unless noted; rows = batch * kv_heads):
  state_k, state_v, state_k_attn, state_v_attn   [rows, capacity, D]
  state_vlen                                     [rows, capacity] fp32
  recent_k, recent_v                             [rows, W, D]   W = n_bswa * chunk_len
  recent_gate                                    [rows, W]
The sliding window lives in a ring of exactly W rows.  Its bookkeeping is
(recent_start, recent_len): window token i is ring row
(recent_start + i) mod W.  Every kernel that reads the window takes the ring
start and wraps the index itself, so a decoded token is written to one row
only and the overflow chunk of a state update is read where it lies.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Any

import torch

from . import _lib
from .schedule import state_length_after_cycle as _cycle_len


@dataclass(frozen=True)
class DecodeCacheSnapshot:
    """A frozen copy of a layer's carried state: memory slots, window and
    counters.  A cache can be reset to it any number of times (benchmarks
    restore it before each timed trial)."""

    state_k: torch.Tensor       # [B, Hkv, S, D]
    state_v: torch.Tensor       # [B, Hkv, S, Dv]
    state_vlen: torch.Tensor    # [B, Hkv, S, 1]
    recent_k: torch.Tensor      # [B, Hkv, R, D]
    recent_v: torch.Tensor      # [B, Hkv, R, Dv]
    recent_gate: torch.Tensor   # [B, Hkv, R, 1]
    total_len: int
    state_coverage_len: int
    recent_begin: int


def _copy_rows(dst: torch.Tensor, src: torch.Tensor, n: int) -> None:
    """dst[:, :n] <- src reshaped to dst's row layout."""
    dst[:, :n].copy_(src.reshape(dst.size(0), n, *dst.shape[2:]).to(dst.dtype))


class KVMDecodeCache:
    """Carried state of one HIP KVM layer between decode steps.

    Buffers are allocated once.  A decode step allocates nothing; the only
    reallocation happens when a growing state budget needs more slots than
    ``state_capacity``, and then only at the state update that needs them
    (the reference grows at the same point, model/kvm_triton_decode.py:202-239).
    """

    cache_representation = "preallocated modular window ring"

    def __init__(self, mixer: Any, snapshot: DecodeCacheSnapshot | None, *, state_capacity: int,
                 _device: torch.device | None = None, _batch: int | None = None) -> None:
        self.mixer = mixer
        if snapshot is None:
            device, self.batch, self.dtype = _device, int(_batch), torch.bfloat16
        else:
            if not snapshot.state_k.is_cuda:
                raise RuntimeError("HIP KVM decode requires ROCm device tensors")
            device = snapshot.state_k.device
            self.batch = int(snapshot.state_k.size(0))
            self.dtype = snapshot.state_k.dtype
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
            if int(snapshot.state_k.size(2)) > self.state_capacity:
                raise ValueError("state capacity is smaller than the initial state")
            if int(snapshot.recent_k.size(2)) > self.ring_capacity:
                raise ValueError("initial recent front exceeds the ring capacity")

        self._alloc_state(self.state_capacity)
        rows, W = self.kv_rows, self.ring_capacity
        bf16 = dict(device=device, dtype=torch.bfloat16)
        self.recent_k = torch.empty(rows, W, self.head_dim, **bf16)
        self.recent_v = torch.empty(rows, W, self.value_dim, **bf16)
        self.recent_gate = torch.empty(rows, W, **bf16)
        self.out = torch.empty(self.batch, self.q_heads, 1, self.value_dim, **bf16)
        # Routing of the most recent state update: slot per overflow token
        # (-1 until an update has run) and whether the token was appended.
        i32 = dict(device=device, dtype=torch.int32)
        self.route_by_token = torch.full((rows, self.chunk_len), -1, **i32)
        self.append_by_token = torch.zeros((rows, self.chunk_len), **i32)
        self.layer = mixer._layer_struct(self.batch, device)
        self.direct_layer = mixer._layer_struct(self.batch, device, gate_initial=False)
        lib = _lib.load()
        self.update_workspace = torch.empty(
            int(lib.kvm_update_workspace_bytes(self.layer.ref(), self.chunk_len)), device=device, dtype=torch.uint8)
        self._alloc_decode_workspace()
        self._set_counters(total=0, state_len=0, coverage=0, begin=0, window=0)
        self.graph_ctl: int | None = None  # device counter record while a decode step is captured
        self.ring_row_written = False  # the prefix kernel wrote this step's ring row already
        if snapshot is not None:
            self.reset_(snapshot)

    def _set_counters(self, *, total: int, state_len: int, coverage: int, begin: int, window: int) -> None:
        self.total_len = int(total)
        self.state_len = int(state_len)
        self.state_coverage_len = int(coverage)
        self.recent_begin = int(begin)
        self.recent_start = 0
        self.recent_len = int(window)
        self.update_count = 0

    # -- storage ------------------------------------------------------------
    def _state_tensors(self) -> tuple[torch.Tensor, ...]:
        return (self.state_k, self.state_v, self.state_k_attn, self.state_v_attn, self.state_vlen)

    def _alloc_state(self, cap: int) -> None:
        rows = self.kv_rows
        bf16 = dict(device=self.device, dtype=torch.bfloat16)
        self.state_k = torch.empty(rows, cap, self.head_dim, **bf16)
        self.state_v = torch.empty(rows, cap, self.value_dim, **bf16)
        self.state_k_attn = torch.empty(rows, cap, self.head_dim, **bf16)
        self.state_v_attn = torch.empty(rows, cap, self.value_dim, **bf16)
        self.state_vlen = torch.empty(rows, cap, device=self.device, dtype=torch.float32)

    def _alloc_decode_workspace(self) -> None:
        lib = _lib.load()
        n = int(lib.kvm_decode_workspace_bytes(self.layer.ref(), self.state_capacity + self.ring_capacity))
        self.decode_workspace = torch.empty(max(n, 256), device=self.device, dtype=torch.uint8)

    def state_struct(self) -> _lib.KvmState:
        return _lib.state_struct(self.state_k, self.state_v, self.state_vlen, self.state_k_attn,
                                 self.state_v_attn, self.state_capacity)

    def _reserve_state_capacity(self, required: int) -> None:
        """Make room for ``required`` memory slots before an update appends.

        The new capacity also covers every update of the next window cycle,
        so a growing budget reallocates at most once per cycle, and never
        beyond the mixer's ``max_state_len``."""
        need = int(required)
        if need <= self.state_capacity:
            return
        limit = int(self.mixer.max_state_len)
        if need > limit:
            raise RuntimeError(
                f"HIP KVM decode requires {need} state rows, exceeding the configured maximum {limit}")
        ahead = self.state_length_after_cycle(self.mixer, self.total_len + 1, need, self.ring_capacity)
        grown = min(limit, max(need, ahead))
        keep, live = self._state_tensors(), self.state_len
        self._alloc_state(grown)
        for new, old in zip(self._state_tensors(), keep):
            new[:, :live].copy_(old[:, :live])
        self.state_capacity = grown
        self._alloc_decode_workspace()

    @staticmethod
    def state_length_after_cycle(mixer: Any, total_len: int, state_len: int, cycle_len: int | None = None) -> int:
        """State length after ``cycle_len`` more decoded tokens (one chunk
        when omitted), following the mixer's budget through every update the
        interval crosses; used to size the state ahead of time."""
        return _cycle_len(mixer.state_budget, mixer.chunk_len, mixer.n_bswa_chunks, total_len, state_len, cycle_len)

    # -- state transitions ----------------------------------------------------
    def reset_(self, snapshot: DecodeCacheSnapshot) -> None:
        """Load ``snapshot`` into the preallocated buffers.  The attention
        rows of the memory slots are recomputed on the device.  Not meant to
        be timed: it copies the whole state."""
        S, R = int(snapshot.state_k.size(2)), int(snapshot.recent_k.size(2))
        if S > self.state_capacity or R > self.ring_capacity:
            raise ValueError("snapshot does not fit the preallocated decode cache")
        _copy_rows(self.state_k, snapshot.state_k, S)
        _copy_rows(self.state_v, snapshot.state_v, S)
        _copy_rows(self.state_vlen, snapshot.state_vlen.float(), S)
        lib = _lib.load()
        _lib.check(lib.kvm_state_refresh(self.layer.ref(), self.state_struct(), 0, S,
                                         _lib.stream_handle(self.device)), "kvm_state_refresh")
        _copy_rows(self.recent_k, snapshot.recent_k, R)
        _copy_rows(self.recent_v, snapshot.recent_v, R)
        _copy_rows(self.recent_gate, snapshot.recent_gate, R)
        self._set_counters(total=snapshot.total_len, state_len=S, coverage=snapshot.state_coverage_len,
                           begin=snapshot.recent_begin, window=R)
        self.route_by_token.fill_(-1)
        self.append_by_token.zero_()

    def append_recent_(self, new_k: torch.Tensor, new_v: torch.Tensor, new_gate: torch.Tensor, *,
                       total_len: int, recent_begin: int, defer_write: bool = False) -> bool:
        """Slide the window to start at ``recent_begin`` and write the new
        token (k, v, gate of one token) behind its last row.  With
        ``defer_write`` the ring row is left unwritten where the next launch
        can write it instead (host counters, row not written yet): the caller
        must then pass the token to ``kvm_decode_step`` before anything else
        reads the ring.  Returns whether the write was deferred."""
        slide = int(recent_begin) - self.recent_begin
        if not 0 <= slide <= self.recent_len:
            raise AssertionError("invalid recent-window transition")
        kept = self.recent_len - slide
        if kept >= self.ring_capacity:
            raise AssertionError("recent ring append would exceed capacity")
        W = self.ring_capacity
        head = (self.recent_start + slide) % W
        deferred = defer_write and self.graph_ctl is None and not self.ring_row_written
        if not deferred:
            self._write_window_row(new_k, new_v, new_gate, (head + kept) % W)
        self.recent_start, self.recent_len = head, kept + 1
        self.total_len, self.recent_begin = int(total_len), int(recent_begin)
        return deferred

    def _write_window_row(self, k: torch.Tensor, v: torch.Tensor, gate: torch.Tensor, row: int) -> None:
        if self.ring_row_written:  # written by the prefix kernel of this captured step
            self.ring_row_written = False
            return
        seq, keep = _lib.seq4(k, v, gate)
        lib = _lib.load()
        if self.graph_ctl is not None:  # capture of a graph step: the row comes from the device counters
            _lib.check(lib.kvm_ring_write_dev(self.layer.ref(), seq, self.recent_k.data_ptr(),
                                              self.recent_v.data_ptr(), self.recent_gate.data_ptr(),
                                              self.ring_capacity, self.graph_ctl,
                                              _lib.stream_handle(self.device)), "kvm_ring_write_dev")
        else:
            _lib.check(lib.kvm_ring_write(self.layer.ref(), seq, self.recent_k.data_ptr(), self.recent_v.data_ptr(),
                                          self.recent_gate.data_ptr(), self.ring_capacity, row,
                                          _lib.stream_handle(self.device)), "kvm_ring_write")
        del keep

    # -- graph-captured decode ------------------------------------------------
    def graph_counters(self) -> list[int]:
        """Device counter record {active_state_len, ring_start, recent_len, 0}
        of the NEXT decode step (the values before its token is written)."""
        active = self.state_len if self.total_len + 1 > self.ring_capacity else 0
        return [active, self.recent_start, self.recent_len, 0]

    def graph_step_is_plain(self) -> bool:
        """Whether the next decode step only appends to the window ring (no
        direct-state append, no state update, no slide, the same active state
        length): the steps a captured graph replays."""
        m = self.mixer
        new_total = self.total_len + 1
        if m._bswa_begin_for_total_len(new_total) != self.recent_begin:
            return False
        direct_target = min(new_total, self.chunk_len)
        if max(direct_target, self.recent_begin) != self.state_coverage_len:
            return False
        if self.recent_len + 1 > self.ring_capacity:
            return False
        return self.total_len > self.ring_capacity  # active state length fixed (the whole state)

    def graph_advance_host_(self) -> None:
        """The host bookkeeping of one replayed plain step (append_recent_
        without a slide)."""
        self.recent_len += 1
        self.total_len += 1

    def graph_buffers(self) -> tuple:
        """Device addresses a captured step depends on."""
        return (self.state_k.data_ptr(), self.state_capacity, self.decode_workspace.data_ptr(),
                self.recent_k.data_ptr(), self.recent_v.data_ptr(), self.recent_gate.data_ptr())

    # -- inspection -----------------------------------------------------------
    def _window(self, ring: torch.Tensor) -> torch.Tensor:
        """The window rows of ``ring`` in token order: a view, or a copy when
        the window wraps past the ring's last row."""
        first = self.recent_start
        tail = first + self.recent_len - self.ring_capacity
        if tail <= 0:
            return ring[:, first:first + self.recent_len]
        return torch.cat([ring[:, first:], ring[:, :tail]], dim=1)

    def logical_recent(self) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
        """Window keys, values and merge gates in token order."""
        return self._window(self.recent_k), self._window(self.recent_v), self._window(self.recent_gate)

    def logical_state_dict(self) -> dict[str, Any]:
        """The carried state under the eager mixer's cache keys, shaped
        [B, Hkv, length, feature] as the eager cache holds it."""
        m = self.mixer
        B, H, S, R = self.batch, self.kv_heads, self.state_len, self.recent_len
        wk, wv, wg = self.logical_recent()
        return {
            m._CACHE_S_K: self.state_k[:, :S].reshape(B, H, S, self.head_dim),
            m._CACHE_S_V: self.state_v[:, :S].reshape(B, H, S, self.value_dim),
            m._CACHE_S_VLEN: self.state_vlen[:, :S].reshape(B, H, S, 1),
            m._CACHE_STATE_COVERAGE_LEN: self.state_coverage_len,
            m._CACHE_BSWA_BEGIN: self.recent_begin,
            m._CACHE_BSWA_K: wk.reshape(B, H, R, self.head_dim),
            m._CACHE_BSWA_V: wv.reshape(B, H, R, self.value_dim),
            m._CACHE_BSWA_MERGE_GATE: wg.reshape(B, H, R, 1),
        }

    def persistent_metadata(self) -> dict[str, Any]:
        """Scalar bookkeeping, under the key names the reference reports."""
        names = ("total_len", "state_capacity", "state_coverage_len", "recent_begin", "recent_start",
                 "recent_len", "update_count", "cache_representation")
        meta = {name: getattr(self, name) for name in names}
        meta["active_state_len"] = self.state_len
        meta["recent_capacity"] = self.ring_capacity
        return meta


# The reference's name for the same container.
TritonKVMDecodeCache = KVMDecodeCache

__all__ = ["KVMDecodeCache", "TritonKVMDecodeCache", "DecodeCacheSnapshot"]
