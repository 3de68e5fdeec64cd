"""CPU checks of the training path's host side.

``snapshot_replay.replay_snapshot_rows`` rebuilds the memory snapshots from
the tokens and a forward's routes; the backward pulls the snapshot-row
gradients through it.  Here it is fed the routes the CPU oracle chose and
must reproduce the oracle's own state trajectory (fp32, every snapshot),
for fixed, growing (appends) and gated configurations."""

from __future__ import annotations

import math

import pytest
import torch
import torch.nn.functional as F

from oracle import kvm_oracle as O


def _routes_from_oracle(rec, plan, rows, C):
    """route_log / append_log [n_updates, rows, C] in the HIP prefill's format."""
    n = len(rec.updates)
    route = torch.full((max(n, 1), rows, C), -1, dtype=torch.int32)
    app = torch.zeros((max(n, 1), rows, C), dtype=torch.int32)
    for u, r in enumerate(rec.updates):
        ai = r.append_idx.reshape(rows, -1)
        mi = r.merge_idx.reshape(rows, -1)
        for row in range(rows):
            for j, t in enumerate(ai[row].tolist()):
                route[u, row, t] = plan.upd_state_before[u] + j
                app[u, row, t] = 1
            if r.route is not None:
                route[u, row, mi[row]] = r.route.reshape(rows, -1)[row].to(torch.int32)
    return route, app


@pytest.mark.parametrize("mode,factor,gates", [
    ("fixed", 1.0, (1, 1, 0, 0)),
    ("power_law", 6.0, (1, 1, 0, 0)),
    ("power_law", 6.0, (1, 0, 1, 1)),
])
def test_replay_reproduces_the_oracle_state(mode, factor, gates):
    from kvm_amd.schedule import StateBudget, prefill_plan
    from snapshot_replay import replay_snapshot_rows

    B, Hq, Hkv, D, C, T = 2, 4, 2, 64, 32, 300
    gk, gv, ga, gi = gates
    cfg = O.OracleConfig(q_heads=Hq, kv_heads=Hkv, head_dim=D, value_dim=D, chunk_len=C, n_bswa_chunks=2,
                         n_max_d_chunks=4, sink_len=1, rope_partial_dim=16, state_budget_mode=mode,
                         state_growth_factor=factor, state_min_len=C, gate_keys=bool(gk), gate_values=bool(gv),
                         gate_appends=bool(ga), gate_initial=bool(gi), append_tie_break="lower_index")
    gen = torch.Generator().manual_seed(7)
    p = O.OracleParams(ln_weight=1 + 0.1 * torch.randn(D, generator=gen), ln_bias=0.1 * torch.randn(D, generator=gen),
                       front_temp=torch.ones(Hq), state_temp=torch.ones(Hq))
    q = torch.randn(B, Hq, T, D, generator=gen) / math.sqrt(D)
    k = torch.randn(B, Hkv, T, D, generator=gen)
    v = torch.randn(B, Hkv, T, D, generator=gen)
    g = 1 + F.elu(torch.randn(B, Hkv, T, 1, generator=gen))
    rec = O.Recorder(keep_states=True)
    _, st = O.prefill(q, k, v, g, p, cfg, rec)
    budget = StateBudget(mode, factor, 0.5, 1, C, None, cfg.max_state_len)
    plan = prefill_plan(T, C, 2, budget)
    rows = B * Hkv
    route, app = _routes_from_oracle(rec, plan, rows, C)
    if mode != "fixed":
        assert sum(plan.upd_n_append) > 0
    snaps = replay_snapshot_rows(k.reshape(rows, T, D), v.reshape(rows, T, D), g.reshape(rows, T), p.ln_weight,
                                 p.ln_bias, plan, route, app,
                                 {"eps": 1e-5, "rope_partial_dim": 16, "gate_keys": bool(gk), "gate_values": bool(gv),
                                  "gate_appends": bool(ga), "gate_initial": bool(gi)})
    assert len(snaps) == plan.n_updates + 1
    states = [(u.s_k_before, u.s_v_before, u.s_vlen_before) for u in rec.updates]
    states.append((st[O.S_K], st[O.S_V], st[O.S_VLEN]))
    for s, ((ka, va), (sk, sv, vl)) in enumerate(zip(snaps, states)):
        want_k = O._ln(sk, p).reshape(rows, -1, D)
        want_v = (F.normalize(sv, dim=-1) * vl).reshape(rows, -1, D)
        assert ka.shape == want_k.shape, f"snapshot {s}: {tuple(ka.shape)} vs {tuple(want_k.shape)}"
        assert torch.allclose(ka, want_k, atol=2e-5, rtol=1e-5), f"snapshot {s} key rows"
        assert torch.allclose(va, want_v, atol=2e-5, rtol=1e-5), f"snapshot {s} value rows"
