"""Graph-captured decode (kvm_amd.backbone.DecodeGraph) against eager decode.

A small all-KVM decoder (2 layers, d_model 256, 4 heads of 64, chunk 64, two
window chunks, 64 fixed memory slots, token shift in the mixer and the MLP)
prefills 300 tokens and then decodes 100 teacher-forced tokens twice from the
same prefill: eagerly (one launch sequence per step, counters as kernel
arguments) and through DecodeGraph (the plain steps replayed from one captured
HIP graph with the counters in device memory, the two chunk-boundary steps of
the interval run eagerly).  Every step's logits and the carried state at the
end must be identical: the replayed kernels are the eager ones, with the same
operands, reading their counters from memory instead of arguments.
"""
from __future__ import annotations

import pytest
import torch

import kvm_testlib as T

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _model(seed):
    from kvm_amd.backbone import MixerConfig, RWKV7BackboneForCausalLM, init_random_

    cfg = MixerConfig(vocab_size=512, num_hidden_layers=2, num_attention_heads=4, hidden_size=256,
                      mup_base_dim=256, use_tokenshift_att=1, use_tokenshift_ffn=1, residual_scale=0.5,
                      rope_partial_dim=32, chunk_len=64, n_bswa_chunks=2, state_min_len=64,
                      state_budget_mode="fixed", sink_len=1)
    with torch.device("meta"):
        model = RWKV7BackboneForCausalLM(cfg)
    return init_random_(model.to_empty(device=DEV).to(torch.bfloat16), seed).eval()


def test_graph_decode_matches_eager():
    if not torch.cuda.is_available():
        pytest.skip("needs an MI355X")
    from kvm_amd.backbone import DecodeGraph, StatesDictCache

    B, Tp, n = 2, 300, 100
    model = _model(7)
    gen = torch.Generator(device=DEV).manual_seed(3)
    prompt = torch.randint(0, 512, (B, Tp), device=DEV, generator=gen)
    toks = torch.randint(0, 512, (n, B), device=DEV, generator=gen)
    T.log(f"[decode-graph] B{B} prompt {Tp}, {n} teacher-forced steps, eager vs graph")
    with torch.no_grad():
        eager_cache = StatesDictCache()
        model(input_ids=prompt, past_key_values=eager_cache, use_cache=True,
              cache_position=torch.arange(Tp, device=DEV), logits_to_keep=1)
        eager = []
        for s in range(n):
            out = model(input_ids=toks[s][:, None], past_key_values=eager_cache, use_cache=True,
                        cache_position=torch.tensor([Tp + s]), logits_to_keep=1)
            eager.append(out.logits[:, -1].clone())

        graph_cache = StatesDictCache()
        model(input_ids=prompt, past_key_values=graph_cache, use_cache=True,
              cache_position=torch.arange(Tp, device=DEV), logits_to_keep=1)
        runner = DecodeGraph(model, graph_cache)
        worst = 0.0
        for s in range(n):
            if s == n // 2:
                runner.close()  # released mid-way: the next plain step captures again
            got = runner.step(toks[s]).clone()
            d = float((got - eager[s]).abs().max())
            worst = max(worst, d)
            assert d == 0.0, f"step {s}: logits differ by {d:.3e} (replays so far {runner.replays})"
        torch.cuda.synchronize()
    T.log(f"[decode-graph] {runner.replays} replayed steps, {runner.eager_steps} eager steps, max |diff| {worst}")
    assert runner.replays >= 90 and runner.eager_steps >= 2
    assert graph_cache.get_seq_length(0) == eager_cache.get_seq_length(0) == Tp + n
    from kvm_amd.mixer import SequenceMixer

    for layer in range(2):
        a = eager_cache.get_states(layer)[SequenceMixer._CACHE_TRITON_DECODE]
        b = graph_cache.get_states(layer)[SequenceMixer._CACHE_TRITON_DECODE]
        assert a.persistent_metadata() == b.persistent_metadata()
        sa, sb = a.logical_state_dict(), b.logical_state_dict()
        for key, va in sa.items():
            vb = sb[key]
            if torch.is_tensor(va):
                assert torch.equal(va, vb), f"layer {layer} {key} differs"
            else:
                assert va == vb, f"layer {layer} {key}: {va} != {vb}"


def test_graph_decode_matches_eager_growing_state():
    """The same comparison with a growing memory (power-law budget, appends at
    chunk boundaries, GQA 4 query heads on 2 kv heads, chunk 32): boundary
    steps append to the state, the state is reallocated as it grows and the
    graph is captured again; every step's logits and the final carried state
    stay identical to eager decode."""
    if not torch.cuda.is_available():
        pytest.skip("needs an MI355X")
    from kvm_amd.backbone import DecodeGraph, MixerConfig, RWKV7BackboneForCausalLM, StatesDictCache, init_random_
    from kvm_amd.mixer import SequenceMixer

    cfg = MixerConfig(vocab_size=512, num_hidden_layers=2, num_attention_heads=4, num_key_value_heads=2,
                      hidden_size=256, mup_base_dim=256, use_tokenshift_att=1, use_tokenshift_ffn=1,
                      residual_scale=0.5, rope_partial_dim=32, chunk_len=32, n_bswa_chunks=2, n_max_d_chunks=3,
                      state_min_len=32, state_budget_mode="power_law", state_growth_factor=4.0,
                      state_growth_exponent=0.5, sink_len=2)
    with torch.device("meta"):
        model = RWKV7BackboneForCausalLM(cfg)
    model = init_random_(model.to_empty(device=DEV).to(torch.bfloat16), 11).eval()
    B, Tp, n = 2, 70, 160
    gen = torch.Generator(device=DEV).manual_seed(5)
    prompt = torch.randint(0, 512, (B, Tp), device=DEV, generator=gen)
    toks = torch.randint(0, 512, (n, B), device=DEV, generator=gen)
    T.log(f"[decode-graph] growing state: B{B} prompt {Tp}, {n} teacher-forced steps, eager vs graph")
    with torch.no_grad():
        eager_cache = StatesDictCache()
        model(input_ids=prompt, past_key_values=eager_cache, use_cache=True,
              cache_position=torch.arange(Tp, device=DEV), logits_to_keep=1)
        eager = []
        for s in range(n):
            out = model(input_ids=toks[s][:, None], past_key_values=eager_cache, use_cache=True,
                        cache_position=torch.tensor([Tp + s]), logits_to_keep=1)
            eager.append(out.logits[:, -1].clone())
        graph_cache = StatesDictCache()
        model(input_ids=prompt, past_key_values=graph_cache, use_cache=True,
              cache_position=torch.arange(Tp, device=DEV), logits_to_keep=1)
        runner = DecodeGraph(model, graph_cache)
        lens, sigs = [], set()
        for s in range(n):
            got = runner.step(toks[s]).clone()
            assert torch.equal(got, eager[s]), f"step {s}: logits differ (replays so far {runner.replays})"
            c = graph_cache.get_states(0)[SequenceMixer._CACHE_TRITON_DECODE]
            lens.append(c.state_len)
            sigs.add(c.graph_buffers())
        torch.cuda.synchronize()
    T.log(f"[decode-graph] state {lens[0]} -> {lens[-1]} slots, {len(sigs)} buffer sets, "
          f"{runner.replays} replays, {runner.eager_steps} eager steps")
    assert lens[-1] > lens[0], "the state did not grow"
    assert len(sigs) > 1, "the state was never reallocated"
    assert runner.replays > n // 2
    for layer in range(2):
        a = eager_cache.get_states(layer)[SequenceMixer._CACHE_TRITON_DECODE]
        b = graph_cache.get_states(layer)[SequenceMixer._CACHE_TRITON_DECODE]
        assert a.persistent_metadata() == b.persistent_metadata()
        sa, sb = a.logical_state_dict(), b.logical_state_dict()
        for key, va in sa.items():
            vb = sb[key]
            if torch.is_tensor(va):
                assert torch.equal(va, vb), f"layer {layer} {key} differs"
            else:
                assert va == vb, f"layer {layer} {key}: {va} != {vb}"


def test_graph_follows_weight_updates():
    """A parameter updated in place between replays (its version counter
    moves) makes DecodeGraph repack and recapture: every step's logits equal
    an eager step's with the same weights, before and after the update."""
    if not torch.cuda.is_available():
        pytest.skip("needs an MI355X")
    from kvm_amd.backbone import DecodeGraph, StatesDictCache

    B, Tp, n, s_upd = 2, 140, 40, 15
    model = _model(11)
    gen = torch.Generator(device=DEV).manual_seed(5)
    prompt = torch.randint(0, 512, (B, Tp), device=DEV, generator=gen)
    toks = torch.randint(0, 512, (n, B), device=DEV, generator=gen)
    T.log(f"[decode-graph-weights] B{B} prompt {Tp}, {n} steps, weights updated in place at step {s_upd}")
    with torch.no_grad():
        caches = [StatesDictCache(), StatesDictCache()]
        for c in caches:
            model(input_ids=prompt, past_key_values=c, use_cache=True,
                  cache_position=torch.arange(Tp, device=DEV), logits_to_keep=1)
        runner = DecodeGraph(model, caches[1])
        replays_before = 0
        for s in range(n):
            if s == s_upd:
                replays_before = runner.replays
                model.transformer.h[0].mlp.c_fc.weight.mul_(1.25)
                model.lm_head.weight.mul_(0.75)
            ref = model(input_ids=toks[s][:, None], past_key_values=caches[0], use_cache=True,
                        cache_position=torch.tensor([Tp + s]), logits_to_keep=1).logits[:, -1].clone()
            got = runner.step(toks[s]).clone()
            d = float((got - ref).abs().max())
            assert d == 0.0, f"step {s}: logits differ by {d:.3e} (replays {runner.replays})"
        torch.cuda.synchronize()
    T.log(f"[decode-graph-weights] {runner.replays} replays ({replays_before} before the update), "
          f"{runner.eager_steps} eager steps")
    assert replays_before >= 5 and runner.replays > replays_before + 5
