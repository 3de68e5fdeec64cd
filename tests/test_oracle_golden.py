"""Pin the CPU oracle to the reference's own eager mixer via golden fixtures.

The fixtures were written by tests/golden/make_golden.py from
model.kvm_fp32_routing_reference.SequenceMixer (eager KVM with FP32 merge
routing).  On the torch build that wrote them the oracle must agree bit for
bit; on another torch build CPU kernels may round differently, so the check
falls back to a tolerance (and routes must still agree).
"""

import pytest
import torch

import golden_io
from oracle import kvm_oracle as O

SAME_TORCH = None


def _exact(fx):
    return fx["meta"]["torch_version"] == torch.__version__


def _route(u):
    """Slot per merged token; an update that appended every token has none."""
    if u.route is None:
        return torch.zeros(*u.merge_idx.shape[:-1], 0, dtype=torch.int32)
    return u.route.to(torch.int32)


def _cmp(a, b, exact, atol=2e-2):
    if exact:
        assert torch.equal(a, b), f"max diff {(a.float() - b.float()).abs().max()}"
    else:
        assert (a.float() - b.float()).abs().max() <= atol


@pytest.mark.parametrize("name", golden_io.names())
def test_prefill_matches_reference(name):
    fx = golden_io.load(name)
    m = fx["meta"]
    cfg, p = golden_io.oracle_setup(fx)
    T = m["T"]
    rec = O.Recorder()
    y, st = O.prefill(
        fx["in_q"][:, :, :T], fx["in_k"][:, :, :T], fx["in_v"][:, :, :T], fx["in_gate"][:, :, :T], p, cfg, rec
    )
    exact = _exact(fx)
    _cmp(y, fx["y_prefill"], exact)
    n_pre = m["n_prefill_updates"]
    assert len(rec.updates) == n_pre
    for i, u in enumerate(rec.updates):
        assert torch.equal(_route(u), fx[f"upd{i}_route"]), f"update {i} routes differ"
        if f"upd{i}_append_idx" in fx:
            assert torch.equal(u.append_idx.to(torch.int32), fx[f"upd{i}_append_idx"])
            assert torch.equal(u.merge_idx.to(torch.int32), fx[f"upd{i}_merge_idx"])
        else:
            assert u.n_append == 0


@pytest.mark.parametrize("name", golden_io.names())
def test_schedules_match_reference_state_lengths(name):
    """The state length after every update that the reference ran (recorded
    when it merged, prefill and decode updates alike) equals the oracle's
    schedule and the product's plan: this pins every budget branch (fixed,
    power law, saturation, round-down) to the reference's own arithmetic."""
    from kvm_amd.schedule import StateBudget, prefill_plan

    fx = golden_io.load(name)
    m = fx["meta"]
    cfg, _ = golden_io.oracle_setup(fx)
    T, C, n = m["T"], m["C"], m["n_bswa"]
    ref_after = [int(fx[f"upd{i}_state_len_at_merge"]) for i in range(m["n_updates"])]
    sched = O.prefill_schedule(cfg, T)
    assert [u[4] for u in sched["updates"]] == ref_after[:m["n_prefill_updates"]]
    budget = StateBudget(cfg.state_budget_mode, cfg.state_growth_factor, cfg.state_growth_exponent,
                         cfg.state_round_down, cfg.state_min_len, cfg.state_saturation_n, cfg.max_state_len)
    plan = prefill_plan(T, C, n, budget)
    assert [b + a for b, a in zip(plan.upd_state_before, plan.upd_n_append)] == ref_after[:m["n_prefill_updates"]]
    # Decode-time updates: one per chunk boundary the window crosses, each
    # with ctx = n*C + coverage and available = coverage + C (model/kvm_mixer.py:645-669).
    cur, cov = sched["final_state_len"], sched["final_coverage"]
    got = []
    for s in range(m.get("decode_steps", 0)):
        total = T + s + 1
        direct = min(total, C)
        if direct > cov:
            cur, cov = cur + 1, direct
        new_cov = max(direct, O.bswa_begin_for_total_len(total, C, n))
        if new_cov > cov:
            cur = budget.desired(n * C + cov, cov + C, cur)
            got.append(cur)
            cov = new_cov
    assert got == ref_after[m["n_prefill_updates"]:]


@pytest.mark.parametrize("name", golden_io.decode_names())
def test_decode_matches_reference(name):
    fx = golden_io.load(name)
    m = fx["meta"]
    cfg, p = golden_io.oracle_setup(fx)
    T, steps = m["T"], m["decode_steps"]
    rec = O.Recorder()
    q, k, v, g = fx["in_q"], fx["in_k"], fx["in_v"], fx["in_gate"]
    _, st = O.prefill(q[:, :, :T], k[:, :, :T], v[:, :, :T], g[:, :, :T], p, cfg, rec)
    outs = []
    for s in range(steps):
        t = T + s
        y, st = O.decode_step(st, t, q[:, :, t:t + 1], k[:, :, t:t + 1], v[:, :, t:t + 1], g[:, :, t:t + 1], p, cfg, rec)
        outs.append(y)
    exact = _exact(fx)
    _cmp(torch.cat(outs, dim=2), fx["y_decode"], exact)
    for key in (O.S_K, O.S_V, O.S_VLEN, O.BSWA_K, O.BSWA_V, O.BSWA_GATE):
        _cmp(st[key], fx["final_" + key], exact)
    assert st[O.COVERAGE] == int(fx["final_kvm_state_coverage_len"])
    assert st[O.BSWA_BEGIN] == int(fx["final_kvm_bswa_begin"])
    assert len(rec.updates) == m["n_updates"]
    for i, u in enumerate(rec.updates):
        assert torch.equal(_route(u), fx[f"upd{i}_route"]), f"update {i} routes differ"


@pytest.mark.parametrize("name,field", [
    ("no_merge_gate_bf16", "gate_keys"), ("no_merge_gate_bf16", "gate_values"),
    ("key_gate_only_growable_bf16", "gate_values"), ("no_head_temps_bf16", "use_head_temps"),
    ("bf16_routing_bf16", "fp32_routing"), ("no_vlens_bf16", "use_vlens"),
])
def test_flag_fixtures_pin_their_branch(name, field):
    """Each configuration-flag fixture decides its branch of the oracle: with
    the flag the reference ran, the prefill is bit-exact; with it flipped
    (the planted mistake), the output differs."""
    import dataclasses

    fx = golden_io.load(name)
    if not _exact(fx):
        pytest.skip("bit-exact comparison needs the torch build that wrote the fixture")
    T = fx["meta"]["T"]
    cfg, p = golden_io.oracle_setup(fx)
    args = (fx["in_q"][:, :, :T], fx["in_k"][:, :, :T], fx["in_v"][:, :, :T], fx["in_gate"][:, :, :T], p)
    y, _ = O.prefill(*args, cfg)
    assert torch.equal(y, fx["y_prefill"])
    flipped = dataclasses.replace(cfg, **{field: not getattr(cfg, field)})
    y_bad, _ = O.prefill(*args, flipped)
    assert not torch.equal(y_bad, fx["y_prefill"]), f"flipping {field} leaves the fixture's output unchanged"
