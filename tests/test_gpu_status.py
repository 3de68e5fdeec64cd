"""The persistent update chain's failure path, forced from the host.

KVM_AMD_CHAIN_POLLS=0 gives every group wait of the chain a poll budget of
zero: each member gives up at its first barrier, before reading anything
another member wrote, and leaves normally.  The prefill must then never return
the incomplete state: the Python class, which reads the status word, repeats
the call on the per-update kernels (a RuntimeWarning, results equal to the
chain's); the C ABI in its synchronous mode returns KVM_EABORT; a deferred
check raises.  A later prefill with the normal budget must be correct again.
"""

from __future__ import annotations

import math

import pytest
import torch

import kvm_testlib as T

pytestmark = pytest.mark.gpu


def _inputs(B, Hq, Hkv, D, Tn, seed=0):
    gen = torch.Generator().manual_seed(seed)
    q = (torch.randn(B, Hq, Tn, D, generator=gen) / math.sqrt(D)).bfloat16().cuda()
    k = (torch.randn(B, Hkv, Tn, D, generator=gen) / math.sqrt(D)).bfloat16().cuda()
    v = (torch.randn(B, Hkv, Tn, D, generator=gen) / math.sqrt(D)).bfloat16().cuda()
    g = (1 + torch.nn.functional.elu(torch.randn(B, Hkv, Tn, 1, generator=gen))).bfloat16().cuda()
    return q, k, v, g


@pytest.mark.parametrize("mode", ["fixed", "power_law"])
def test_chain_timeout_is_reported_or_repeated(monkeypatch, mode):
    if not torch.cuda.is_available():
        pytest.skip("needs an MI355X")
    from kvm_amd import _lib

    B, Hq, Hkv, D, C, Tn = 1, 4, 2, 128, 64, 64 * 10
    cfg = T.mixer_config(Hq, Hkv, D, C, rope=32, mode=mode, min_len=C, n_max=4, factor=4.0, expo=0.5)
    mixer = T.make_mixer(cfg, torch.ones(D), torch.zeros(D), torch.ones(Hq), torch.ones(Hq))
    q, k, v, g = _inputs(B, Hq, Hkv, D, Tn)
    T.log(f"[status] {mode}: reference prefill B{B} Hq{Hq} Hkv{Hkv} D{D} C{C} T{Tn}")
    with torch.no_grad():
        good = mixer.prefill_raw(q, k, v, g)
        assert good["plan"].n_updates >= 2
        ref_out = good["out"].clone()
        T.log(f"[status] {mode}: prefill on the per-update kernels (KVM_PREFILL_NO_CHAIN)")
        nochain = mixer.prefill_raw(q, k, v, g, chain=False)
        for key in ("out", "state_k", "state_v", "state_vlen", "state_k_attn", "state_v_attn"):
            assert torch.equal(nochain[key], good[key]), key
        monkeypatch.setenv("KVM_AMD_CHAIN_POLLS", "0")
        T.log(f"[status] {mode}: prefill with a zero poll budget (every member leaves at its first wait)")
        with pytest.warns(RuntimeWarning, match="per-update kernels"):
            fallback = mixer.prefill_raw(q, k, v, g)
        for key in ("out", "state_k", "state_v", "state_vlen", "state_k_attn", "state_v_attn"):
            assert torch.equal(fallback[key], good[key]), key
        # The C ABI without a status word waits itself and returns KVM_EABORT.
        with pytest.raises(_lib.KvmLibraryError, match="timed out"):
            mixer.prefill_raw(q, k, v, g, check_status=None)
        # Deferred checking: the word is sticky across calls.
        mixer.prefill_raw(q, k, v, g, check_status=False)
        mixer.prefill_raw(q, k, v, g, check_status=False)
        with pytest.raises(RuntimeError, match="timed out"):
            mixer.check_prefill_status()
        monkeypatch.delenv("KVM_AMD_CHAIN_POLLS")
        T.log(f"[status] {mode}: prefill with the normal poll budget after the failures")
        again = mixer.prefill_raw(q, k, v, g)
        torch.cuda.synchronize()
    assert torch.equal(again["out"], ref_out), "a prefill after a reported failure must be exact again"
    mixer.check_prefill_status()  # clear


def test_forward_prefill_repeats_a_timed_out_chain(monkeypatch):
    """The mixer's forward reads the status word after queueing its output
    projection; a timed-out chain is still repeated on the per-update kernels
    before the result is returned (same output as the normal forward)."""
    if not torch.cuda.is_available():
        pytest.skip("needs an MI355X")
    import warnings

    B, Hq, Hkv, D, C, Tn = 1, 4, 2, 128, 64, 64 * 10
    cfg = T.mixer_config(Hq, Hkv, D, C, rope=32, mode="fixed", min_len=C, n_max=4, factor=4.0, expo=0.5)
    mixer = T.make_mixer(cfg, torch.ones(D), torch.zeros(D), torch.ones(Hq), torch.ones(Hq))
    q, k, v, g = _inputs(B, Hq, Hkv, D, Tn, seed=1)
    T.log(f"[status] forward_prefill B{B} Hq{Hq} Hkv{Hkv} D{D} C{C} T{Tn}: normal, then a zero poll budget")
    with torch.no_grad():
        with warnings.catch_warnings():
            warnings.simplefilter("error", RuntimeWarning)
            good = mixer.forward_prefill(q, k, v, g, None, None, None).clone()
        monkeypatch.setenv("KVM_AMD_CHAIN_POLLS", "0")
        with pytest.warns(RuntimeWarning, match="per-update kernels"):
            fallback = mixer.forward_prefill(q, k, v, g, None, None, None)
        monkeypatch.delenv("KVM_AMD_CHAIN_POLLS")
        torch.cuda.synchronize()
    assert torch.equal(fallback, good)
    mixer.check_prefill_status()  # the word was cleared by the forward's read


def test_training_backward_reports_a_timed_out_chain(monkeypatch):
    """The differentiable prefill queues its status read behind the forward's
    prefill; the backward waits for it and raises before using the forward's
    results.  With the normal budget the same forward / backward runs clean."""
    if not torch.cuda.is_available():
        pytest.skip("needs an MI355X")
    from kvm_amd import training

    B, Hq, Hkv, D, C, Tn = 1, 4, 2, 128, 64, 64 * 6
    cfg = T.mixer_config(Hq, Hkv, D, C, rope=32, mode="fixed", min_len=C, n_max=4, factor=4.0, expo=0.5)
    mixer = T.make_mixer(cfg, torch.ones(D), torch.zeros(D), torch.ones(Hq), torch.ones(Hq))
    q, k, v, g = _inputs(B, Hq, Hkv, D, Tn, seed=2)
    T.log(f"[status] training prefill B{B} Hq{Hq} Hkv{Hkv} D{D} C{C} T{Tn}: zero poll budget, then normal")
    monkeypatch.setenv("KVM_AMD_CHAIN_POLLS", "0")
    xs = [t.clone().requires_grad_(True) for t in (q, k, v, g)]
    y = training.prefill_with_grad(mixer, *xs)
    monkeypatch.delenv("KVM_AMD_CHAIN_POLLS")
    with pytest.raises(RuntimeError, match="timed out"):
        y.float().sum().backward()
    xs = [t.clone().requires_grad_(True) for t in (q, k, v, g)]
    y = training.prefill_with_grad(mixer, *xs)
    y.float().sum().backward()
    torch.cuda.synchronize()
    assert all(x.grad is not None and torch.isfinite(x.grad.float()).all() for x in xs)
    mixer.check_prefill_status()  # nothing left in the word
