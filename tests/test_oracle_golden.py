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
        assert torch.equal(u.route.to(torch.int32), fx[f"upd{i}_route"]), f"update {i} routes differ"
        if f"upd{i}_append_idx" in fx:
            assert torch.equal(u.append_idx.to(torch.int32), fx[f"upd{i}_append_idx"])
            assert torch.equal(u.merge_idx.to(torch.int32), fx[f"upd{i}_merge_idx"])
        else:
            assert u.n_append == 0


@pytest.mark.parametrize("name", [n for n in golden_io.names() if n.startswith("decode")])
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
        assert torch.equal(u.route.to(torch.int32), fx[f"upd{i}_route"]), f"update {i} routes differ"
