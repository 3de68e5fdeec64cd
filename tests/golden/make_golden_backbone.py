"""Write the golden fixtures of the whole decoder (embedding -> KVM blocks -> LM head).

Runs ONLY in the build container, where the read-only reference checkout is
mounted (default ``/root/reference``, override with ``KVM_REFERENCE``).  It
imports the reference's ``model.rwkv7_backbone.RWKV7BackboneForCausalLM``
(``model/rwkv7_backbone.py:407-785``) with the eager FP32-routing KVM mixer
``model.kvm_fp32_routing_reference.SequenceMixer`` as every layer's token
mixer, fills every parameter with seeded random values (the reference's own
initialisation zeroes the output projections, which would hide the mixers),
and records, in bf16 on the CPU:

* the prefill logits of every position (``forward`` with ``cache_position``,
  ``model/rwkv7_backbone.py:458-480``),
* a greedy decode: each step feeds the previous argmax token as a single
  token with the layer caches (``forward_inference`` -> ``forward_single``,
  ``model/kvm_mixer.py:527-570``), and its logits.

The fixtures hold tensors only: the parameters (bf16 bits), the token ids,
the logits and the decoded tokens, plus the model config as JSON.

For the first case it also writes the checkpoint the reference's trainer
leaves at the end of a run (``raw_model.save_pretrained(logdir)``,
trainer.py:286): the model is saved into a temporary directory and only its
data files, ``config.json`` and ``model.safetensors``, are kept, under
``backbone/hf_<case>/`` (save_pretrained also copies code files; those are
not kept).  ``--checkpoint-only`` writes just that checkpoint.

The reference's ``StatesDictCache`` cannot be built with this container's
transformers (its layer class misses an abstract method), so the decode uses
a stand-in with the same three calls the model makes on it
(``get_seq_length``, ``get_states``, ``update``; ``model/statesdictcache.py:141-187``).

Usage:  python tests/golden/make_golden_backbone.py
"""

from __future__ import annotations

import json
import os
import shutil
import sys
import tempfile
from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent
OUT_DIR = HERE / "backbone"
REF = Path(os.environ.get("KVM_REFERENCE", "/root/reference"))

# Model configs: field names of model/rwkv7_backbone.py:276-405 (MixerConfigDataclass).
_COMMON = dict(
    token_mixer_class_path="model.kvm_fp32_routing_reference.SequenceMixer",
    rope_theta=10000.0, use_l2wrap=0, param_dtype="bfloat16",
    kvm_use_merge_gate_keys=1, kvm_use_merge_gate_values=1, kvm_use_head_temps=1,
    kvm_use_vlens=1, kvm_aotriton_forward_attention=0, state_round_down=1,
    state_saturation_n=None, kvm_value_residual_mode="rwkv", kvm_token_shift_mode="rwkv",
)

CASES = [
    # 350M-recipe style (configs/prolong/350M/kvm_*.yaml): token shift on both
    # mixers, value residual, residual_scale 0.5, fixed state.
    dict(
        name="decoder_fixed_tokenshift",
        B=2, T=150, decode_steps=40, seed=11,
        model=dict(
            vocab_size=96, num_hidden_layers=2, num_attention_heads=2, hidden_size=128,
            mup_base_dim=128, ffn_expansion=4.0, use_skip_connections=0, use_block_lambdas=0,
            logit_softcap=0.0, use_tokenshift_att=1, use_tokenshift_ffn=1, rope_partial_dim=32,
            sink_len=1, chunk_len=32, n_max_d_chunks=1, n_bswa_chunks=2, state_budget_mode="fixed",
            state_growth_factor=1.0, state_growth_exponent=0.5, state_min_len=32,
            use_value_residual=1, residual_scale=0.5,
            kvm_apply_merge_gate_to_initial_state=0, kvm_apply_merge_gate_to_appends=0,
        ),
    ),
    # GQA, U-net skip connections, block lambdas, logit soft cap, growing state.
    dict(
        name="decoder_gqa_skip_growth",
        B=1, T=200, decode_steps=30, seed=12,
        model=dict(
            vocab_size=80, num_hidden_layers=4, num_attention_heads=4, num_key_value_heads=2,
            d_head=64, hidden_size=128, mup_base_dim=128, ffn_expansion=2.0,
            use_skip_connections=1, use_block_lambdas=1, logit_softcap=30.0, use_tokenshift_att=1,
            use_tokenshift_ffn=0, rope_partial_dim=32, sink_len=2, chunk_len=32, n_max_d_chunks=3,
            n_bswa_chunks=2, state_budget_mode="power_law", state_growth_factor=4.0,
            state_growth_exponent=0.5, state_min_len=32, use_value_residual=1, residual_scale=None,
            kvm_apply_merge_gate_to_initial_state=1, kvm_apply_merge_gate_to_appends=1,
        ),
    ),
]


class LayerStatesCache:
    """Per-layer states dict plus a seen-token counter (the three calls the
    backbone and the KVM mixer make on their cache)."""

    def __init__(self):
        self.states, self.seen = {}, {}

    def get_seq_length(self, layer_idx=0):
        return self.seen.get(layer_idx, 0)

    def get_states(self, layer_idx):
        return self.states.setdefault(layer_idx, {})

    def update(self, layer_idx, offset=1, states_dict=None, **_):
        st = self.states.setdefault(layer_idx, {})
        if states_dict:
            st.update(states_dict)
        self.seen[layer_idx] = self.seen.get(layer_idx, 0) + offset
        return st


def randomize_(model: torch.nn.Module, seed: int) -> None:
    """Seeded random parameters: matrices ~ N(0, 1/fan_in), vectors perturbed
    around their initial value (LayerNorm weights stay near 1)."""
    gen = torch.Generator().manual_seed(seed)
    with torch.no_grad():
        for name, p in sorted(model.named_parameters()):
            if p.dim() >= 2:
                std = 1.0 if name.endswith("wte.weight") else p.shape[-1] ** -0.5
                p.copy_(torch.randn(p.shape, generator=gen) * std)
            else:
                p.add_(0.1 * torch.randn(p.shape, generator=gen))


def _bits(t: torch.Tensor) -> np.ndarray:
    return t.detach().contiguous().to(torch.bfloat16).view(torch.int16).numpy()


def build_model(case):
    sys.path.insert(0, str(REF))
    import utils.grad_cp as grad_cp  # noqa: E402
    from model.rwkv7_backbone import MixerConfig, RWKV7BackboneForCausalLM  # noqa: E402

    grad_cp.use_grad_cp = 0  # plain module calls (no checkpoint wrapper) at inference
    cfg = MixerConfig(**_COMMON, **case["model"])
    torch.manual_seed(case["seed"])
    model = RWKV7BackboneForCausalLM(cfg).to(torch.bfloat16).eval()
    randomize_(model, case["seed"])
    return cfg, model


def save_checkpoint(case):
    """config.json + model.safetensors exactly as the reference writes them."""
    _, model = build_model(case)
    out = OUT_DIR / f"hf_{case['name']}"
    out.mkdir(parents=True, exist_ok=True)
    with tempfile.TemporaryDirectory() as tmp:
        model.save_pretrained(tmp)
        for name in ("config.json", "model.safetensors"):
            shutil.copyfile(Path(tmp) / name, out / name)
    print(f"wrote {out.relative_to(HERE)}: " + ", ".join(
        f"{p.name} {p.stat().st_size / 1024:.0f} KiB" for p in sorted(out.iterdir())))


def run_case(case):
    cfg, model = build_model(case)

    B, T, n_dec = case["B"], case["T"], case["decode_steps"]
    gen = torch.Generator().manual_seed(case["seed"] + 1000)
    ids = torch.randint(0, cfg.vocab_size, (B, T), generator=gen)
    cache = LayerStatesCache()
    with torch.no_grad():
        out = model(input_ids=ids, past_key_values=cache, use_cache=False,
                    cache_position=torch.arange(T))
        prefill_logits = out.logits.float()
        tok = prefill_logits[:, -1].argmax(-1)
        dec_tokens, dec_logits = [], []
        for s in range(n_dec):
            dec_tokens.append(tok)
            o = model(input_ids=tok[:, None], past_key_values=cache, use_cache=False,
                      cache_position=torch.tensor([T + s]))
            lg = o.logits.float()[:, -1]
            dec_logits.append(lg)
            tok = lg.argmax(-1)
    data = {f"param.{k}": _bits(v) for k, v in model.state_dict().items()}
    data["input_ids"] = ids.numpy().astype(np.int64)
    data["prefill_logits"] = prefill_logits.numpy()
    data["decode_tokens"] = torch.stack(dec_tokens, 1).numpy().astype(np.int64)
    data["decode_logits"] = torch.stack(dec_logits, 1).numpy()
    meta = dict(name=case["name"], B=B, T=T, decode_steps=n_dec, seed=case["seed"],
                model={**_COMMON, **case["model"]}, torch_version=torch.__version__,
                reference="SmerkyG/KVM-paper model.rwkv7_backbone.RWKV7BackboneForCausalLM "
                          "+ model.kvm_fp32_routing_reference.SequenceMixer (CPU, bf16)")
    data["meta_json"] = np.array(json.dumps(meta))
    return data


def main():
    OUT_DIR.mkdir(exist_ok=True)
    save_checkpoint(CASES[0])
    if "--checkpoint-only" in sys.argv:
        return
    for case in CASES:
        data = run_case(case)
        path = OUT_DIR / f"{case['name']}.npz"
        np.savez_compressed(path, **data)
        print(f"wrote {path.relative_to(HERE)}: {path.stat().st_size / 1024:.0f} KiB, "
              f"{sum(1 for k in data if k.startswith('param.'))} parameter tensors")


if __name__ == "__main__":
    main()
