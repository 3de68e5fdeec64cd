"""CPU tests of the decoder around the KVM mixer (kvm_amd.backbone).

The whole-model golden fixtures (tests/golden/make_golden_backbone.py) hold
the reference's RWKV7BackboneForCausalLM with its eager FP32-routing KVM
mixer in every layer: prefill logits and a greedy decode.  Here the build's
decoder runs with ``tests/oracle_mixer.OracleSequenceMixer`` (the build's
own pre-boundary code + the CPU oracle after the boundary), so these tests
pin the decoder's host code and the mixer's projections / token shift /
value residual / RoPE / merge gate to the reference, bit for bit, without a
GPU.  The same fixtures are checked against the HIP mixer in
tests/test_gpu_backbone.py.
"""

from __future__ import annotations

import pytest
import torch

import golden_io
from kvm_amd import backbone as BB

ORACLE_MIXER = "oracle_mixer.OracleSequenceMixer"
NAMES = golden_io.backbone_names()


def test_fixtures_present():
    assert len(NAMES) >= 2


@pytest.mark.parametrize("name", NAMES)
def test_decoder_matches_reference_bit_exact(name):
    fx = golden_io.load_backbone(name)
    model = golden_io.backbone_model(fx, ORACLE_MIXER)
    ids, T = fx["input_ids"], fx["input_ids"].shape[1]
    cache = BB.StatesDictCache()
    with torch.no_grad():
        out = model(input_ids=ids, past_key_values=cache, use_cache=True, cache_position=torch.arange(T))
        assert out.logits.dtype == torch.float32
        assert torch.equal(out.logits, fx["prefill_logits"])
        # Teacher-forced decode: feed the reference's greedy tokens.
        toks = fx["decode_tokens"]
        for s in range(toks.shape[1]):
            lg = model(input_ids=toks[:, s:s + 1], past_key_values=cache, use_cache=True,
                       cache_position=torch.tensor([T + s])).logits[:, -1]
            assert torch.equal(lg, fx["decode_logits"][:, s]), f"decode step {s}"
    assert cache.get_seq_length(0) == T + toks.shape[1]


@pytest.mark.parametrize("name", NAMES)
def test_greedy_generation_matches_reference(name):
    fx = golden_io.load_backbone(name)
    model = golden_io.backbone_model(fx, ORACLE_MIXER)
    n = fx["decode_tokens"].shape[1]
    seen = []
    toks = model.generate_greedy(fx["input_ids"], n, on_step=lambda s, lg: seen.append(lg))
    assert torch.equal(toks, fx["decode_tokens"])
    assert torch.equal(seen[0], fx["prefill_logits"][:, -1])


def test_decode_after_prefill_equals_longer_prefill():
    """Invariant: logits of token T decoded after a prefill of T tokens equal
    the last logits of a prefill of T+1 tokens (same weights, same ids)."""
    fx = golden_io.load_backbone(NAMES[0])
    model = golden_io.backbone_model(fx, ORACLE_MIXER)
    ids = torch.cat([fx["input_ids"], fx["decode_tokens"][:, :1]], dim=1)
    T = fx["input_ids"].shape[1]
    with torch.no_grad():
        cache = BB.StatesDictCache()
        model(input_ids=ids[:, :T], past_key_values=cache, use_cache=True, cache_position=torch.arange(T))
        dec = model(input_ids=ids[:, T:], past_key_values=cache, use_cache=True,
                    cache_position=torch.tensor([T])).logits[:, -1]
        full = model(input_ids=ids).logits[:, -1]
    assert (dec - full).abs().max() <= 0.1, (dec - full).abs().max()
    assert torch.equal(dec.argmax(-1), full.argmax(-1))


def test_token_mixer_selection():
    cfg = BB.MixerConfig(token_mixer_class_path="model.kvm_triton_mixer.SequenceMixer")
    assert BB._resolve_mixer_path(cfg, 0) == "kvm_amd.mixer.SequenceMixer"
    for path in ("model.kvm_mixer.SequenceMixer", "model.kvm_fp32_routing_reference.SequenceMixer"):
        assert BB._resolve_mixer_path(BB.MixerConfig(token_mixer_class_path=path), 3) == "kvm_amd.mixer.SequenceMixer"
    assert BB._resolve_mixer_path(BB.MixerConfig(token_mixer="kvm"), 0) == "kvm_amd.mixer.SequenceMixer"
    with pytest.raises(ValueError, match="not part of this build"):
        BB._resolve_mixer_path(BB.MixerConfig(token_mixer="rwkv7"), 0)
    with pytest.raises(ValueError, match="alternating"):
        BB.RWKV7BackboneModel(BB.MixerConfig(alt_layer_every=2, kvm_use_vlens=1))


def test_input_validation():
    fx = golden_io.load_backbone(NAMES[0])
    model = golden_io.backbone_model(fx, ORACLE_MIXER)
    ids = fx["input_ids"][:, :8]
    with pytest.raises(ValueError, match="exactly one"):
        model()
    with pytest.raises(ValueError, match="Cannot infer"):
        model(input_ids=ids, past_key_values=BB.StatesDictCache())
    with pytest.raises(NotImplementedError):
        mask = torch.ones_like(ids)
        mask[0, 0] = 0
        model(input_ids=ids, attention_mask=mask)
    with pytest.raises(ValueError, match="inference"):
        model(input_ids=ids, labels=ids)


def test_config5_architecture_on_meta():
    """BASELINE config 5 (24 layers, d_model 2048, 16 heads of 128, vocab 65536,
    chunk 512, 512 fixed slots) builds with a HIP KVM mixer in every layer."""
    cfg = BB.MixerConfig(vocab_size=65536, num_hidden_layers=24, num_attention_heads=16, hidden_size=2048,
                         mup_base_dim=2048, use_tokenshift_att=1, use_tokenshift_ffn=1, residual_scale=0.5,
                         rope_partial_dim=64, chunk_len=512, state_min_len=512)
    with torch.device("meta"):
        model = BB.RWKV7BackboneForCausalLM(cfg)
    from kvm_amd.mixer import SequenceMixer

    mixers = [b.attn for b in model.transformer.h]
    assert len(mixers) == 24 and all(type(m) is SequenceMixer for m in mixers)
    assert {(m.d_qk_head, m.chunk_len, m.max_state_len, m.num_key_value_heads) for m in mixers} == {(128, 512, 512, 16)}
    d, V, r, ffn = 2048, 65536, 64, 8192
    per_layer = (4 * d * d + 3 * d + d + r * d + d * r + 4 * 128 + 2 * 128 + 16 * d + 2 * 16 + 4 * d
                 + 2 * ffn * d + d)
    assert sum(p.numel() for p in model.parameters()) == 24 * per_layer + 2 * V * d + 4 * d


HF_DIR = golden_io.BACKBONE / "hf_decoder_fixed_tokenshift"


def test_reference_hf_checkpoint_loads_bit_exact():
    """The checkpoint the reference's save_pretrained wrote (config.json +
    model.safetensors) gives the golden prefill and decode logits."""
    from kvm_amd.checkpoint import load_reference_checkpoint

    fx = golden_io.load_backbone("decoder_fixed_tokenshift")
    model = load_reference_checkpoint(HF_DIR, token_mixer_class_path=ORACLE_MIXER)
    assert model.config.num_hidden_layers == 2 and model.config.chunk_len == 32
    ids, T = fx["input_ids"], fx["input_ids"].shape[1]
    cache = BB.StatesDictCache()
    with torch.no_grad():
        lg = model(input_ids=ids, past_key_values=cache, use_cache=True, cache_position=torch.arange(T)).logits
        assert torch.equal(lg, fx["prefill_logits"])
        tok = fx["decode_tokens"][:, :1]
        lg = model(input_ids=tok, past_key_values=cache, use_cache=True, cache_position=torch.tensor([T])).logits
        assert torch.equal(lg[:, -1], fx["decode_logits"][:, 0])


def test_checkpoint_file_forms(tmp_path):
    """Trainer .pt checkpoints (torch.save of {step, model, optimizers},
    trainer.py:265-281), bare .safetensors / .pt state dicts and
    torch.compile / DDP key prefixes all load to the same tensors."""
    from safetensors.torch import save_file

    from kvm_amd.checkpoint import load_reference_checkpoint, read_state_dict

    ref = read_state_dict(HF_DIR)
    torch.save({"step": 10, "model": ref, "optimizers": []}, tmp_path / "model_step000010.pt")
    torch.save({"_orig_mod." + k: v for k, v in ref.items()}, tmp_path / "bare.pt")
    save_file({"module." + k: v.contiguous() for k, v in ref.items()}, str(tmp_path / "bare.safetensors"))
    (tmp_path / "config.json").write_text((HF_DIR / "config.json").read_text())
    for f in ("model_step000010.pt", "bare.pt", "bare.safetensors"):
        sd = read_state_dict(tmp_path / f)
        assert sd.keys() == ref.keys() and all(torch.equal(sd[k], ref[k]) for k in ref), f
    model = load_reference_checkpoint(tmp_path / "model_step000010.pt", token_mixer_class_path=ORACLE_MIXER)
    for k, v in model.state_dict().items():
        assert torch.equal(v, ref[k]), k


def test_snapshot_from_eager_states():
    """The eager carried-state dict (model/kvm_mixer.py:518-525) maps onto a
    DecodeCacheSnapshot with total_len = window begin + window length."""
    from kvm_amd.checkpoint import snapshot_from_states
    from oracle import kvm_oracle as O

    B, Hq, Hkv, D, C, Tn = 1, 2, 1, 64, 32, 150
    gen = torch.Generator().manual_seed(0)
    q = torch.randn(B, Hq, Tn, D, generator=gen).bfloat16()
    k = torch.randn(B, Hkv, Tn, D, generator=gen).bfloat16()
    v = torch.randn(B, Hkv, Tn, D, generator=gen).bfloat16()
    g = torch.ones(B, Hkv, Tn, 1).bfloat16()
    cfg = O.OracleConfig(q_heads=Hq, kv_heads=Hkv, head_dim=D, value_dim=D, chunk_len=C, state_min_len=C)
    p = O.OracleParams(ln_weight=torch.ones(D).bfloat16(), ln_bias=torch.zeros(D).bfloat16(),
                       front_temp=torch.ones(Hq).bfloat16(), state_temp=torch.ones(Hq).bfloat16())
    _, st = O.prefill(q, k, v, g, p, cfg)
    snap = snapshot_from_states(st)
    assert snap.total_len == Tn and snap.recent_begin == st[O.BSWA_BEGIN]
    assert snap.state_coverage_len == st[O.COVERAGE]
    assert snap.state_k is st[O.S_K] and snap.recent_gate is st[O.BSWA_GATE]
