"""Host-side KVM schedule: window start, state budget, per-chunk prefill plan.

Integer bookkeeping of the reference, restated:
  * window start          model/kvm_mixer.py:167-172
  * state budget          model/kvm_mixer.py:131-165
  * prefill schedule      model/kernels/kvm_triton_training_kernels.py:85-171
    (the eager loop model/kvm_mixer.py:450-488 visits the same chunks)
  * decode capacity       model/kvm_triton_decode.py:241-262
"""

from __future__ import annotations

import math
from dataclasses import dataclass


def round_down_to_multiple(x: int, multiple: int) -> int:
    """model/kvm_mixer.py:25-28."""
    x = max(int(x), 0)
    m = max(int(multiple), 1)
    return (x // m) * m


def bswa_begin_for_total_len(total_len: int, chunk_len: int, n_bswa_chunks: int) -> int:
    """First token of the block-sliding window after ``total_len`` tokens."""
    end = round_down_to_multiple(int(total_len) + chunk_len - 1, chunk_len)
    return max(0, end - n_bswa_chunks * chunk_len)


@dataclass(frozen=True)
class StateBudget:
    """The state-budget attributes of the mixer (model/kvm_mixer.py:96-107)."""

    mode: str
    growth_factor: float
    growth_exponent: float
    round_down: int
    min_len: int
    saturation_n: int | None
    max_state_len: int

    def desired(self, ctx_len: int, available: int, current: int) -> int:
        """State length after an update (model/kvm_mixer.py:131-165)."""
        t = max(int(ctx_len), 0)
        avail = max(int(available), 0)
        cur = max(int(current), 0)
        if self.mode == "fixed":
            target = self.min_len
        elif self.mode == "power_law":
            target = int(math.floor(self.growth_factor * (float(t) ** self.growth_exponent)))
            target = max(round_down_to_multiple(target, self.round_down), self.min_len)
        elif self.mode == "kvm_saturation":
            n = float(self.saturation_n)
            target = int(math.floor((n * float(t)) / (n + float(t))))
            target = max(round_down_to_multiple(target, self.round_down), self.min_len)
        else:
            raise ValueError(f"Unsupported state_budget_mode={self.mode!r}")
        target = min(target, avail, self.max_state_len)
        return max(target, cur)


@dataclass(frozen=True)
class PrefillPlan:
    """Everything the prefill launch needs, as host integers."""

    seq_len: int
    chunk_len: int
    n_chunks: int
    front_len: int
    initial_state_len: int
    chunk_state_len: list[int]      # memory slots visible to query chunk m
    chunk_snapshot: list[int]       # updates applied before chunk m
    upd_token_begin: list[int]      # first token of each overflow chunk
    upd_ctx_len: list[int]
    upd_available: list[int]
    upd_state_before: list[int]
    upd_n_append: list[int]
    final_state_len: int
    final_coverage: int
    max_state_len: int

    @property
    def n_updates(self) -> int:
        return len(self.upd_token_begin)


def prefill_plan(T: int, chunk_len: int, n_bswa: int, budget: StateBudget) -> PrefillPlan:
    """Per-chunk plan of a T-token prefill.

    Chunk m (queries [mC, min(T, mC + C))) with m >= n attends to the state
    after the updates issued before it; after it, the overflow chunk
    [bswa_begin, next_bswa_begin) is folded into the state when the window
    advances (model/kvm_mixer.py:450-488).
    """
    T, C, n = int(T), int(chunk_len), int(n_bswa)
    if T < 1:
        raise ValueError("prefill needs at least one token")
    n_chunks = (T + C - 1) // C
    front = min(T, n * C)
    current = min(T, C)
    coverage = current
    chunk_state = [0] * n_chunks
    chunk_snap = [0] * n_chunks
    tb, ctx, avail, before, n_app = [], [], [], [], []
    for qb in range(front, T, C):
        m = qb // C
        qe = min(T, qb + C)
        begin = bswa_begin_for_total_len(qe, C, n)
        if begin != coverage:
            raise AssertionError("KVM prefill state coverage drifted from the active BSWA window.")
        chunk_state[m] = current
        chunk_snap[m] = len(tb)
        nxt = bswa_begin_for_total_len(min(T, qe + C), C, n)
        if nxt <= begin:
            continue
        want = budget.desired(qe, nxt, current)
        a = min(max(want - current, 0), nxt - begin)
        tb.append(begin)
        ctx.append(qe)
        avail.append(nxt)
        before.append(current)
        n_app.append(a)
        current += a
        coverage = nxt
    return PrefillPlan(
        seq_len=T, chunk_len=C, n_chunks=n_chunks, front_len=front,
        initial_state_len=min(T, C), chunk_state_len=chunk_state, chunk_snapshot=chunk_snap,
        upd_token_begin=tb, upd_ctx_len=ctx, upd_available=avail, upd_state_before=before,
        upd_n_append=n_app, final_state_len=current, final_coverage=coverage,
        max_state_len=current,
    )


def state_length_after_cycle(budget: StateBudget, chunk_len: int, n_bswa: int,
                             total_len: int, state_len: int, cycle_len: int | None = None) -> int:
    """State capacity a bounded decode interval needs (model/kvm_triton_decode.py:241-262)."""
    C = int(chunk_len)
    steps = C if cycle_len is None else int(cycle_len)
    coverage = max(min(int(total_len), C), bswa_begin_for_total_len(int(total_len), C, n_bswa))
    active = int(state_len)
    for step in range(1, steps + 1):
        nb = bswa_begin_for_total_len(int(total_len) + step, C, n_bswa)
        if nb <= coverage:
            continue
        active = budget.desired(n_bswa * C + coverage, coverage + C, active)
        coverage = nb
    return active
