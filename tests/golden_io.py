"""Load the golden fixtures written by tests/golden/make_golden.py."""

from __future__ import annotations

import json
from pathlib import Path

import numpy as np
import torch

GOLDEN = Path(__file__).resolve().parent / "golden"


def names():
    return sorted(p.stem for p in GOLDEN.glob("*.npz"))


def product_names():
    """Fixtures of configurations the HIP mixer implements (fp32 routing,
    kvm_use_vlens 1); the others pin only the CPU oracle's branches."""
    return [n for n in names() if meta(n).get("routing", "fp32") == "fp32" and meta(n).get("vlens", 1) == 1]


def decode_names():
    """Fixtures that also hold cached single-token decode steps."""
    return [n for n in names() if meta(n).get("decode_steps", 0) > 0]


def meta(name: str) -> dict:
    z = np.load(GOLDEN / f"{name}.npz", allow_pickle=False)
    return json.loads(str(z["meta_json"]))


def _tensor(arr: np.ndarray, dtype: str) -> torch.Tensor:
    t = torch.from_numpy(np.array(arr))
    if dtype == "bf16" and t.dtype == torch.int16:
        return t.view(torch.bfloat16)
    return t


def load(name: str) -> dict:
    """Return {"meta": dict, tensors...} with bf16 arrays restored as bf16."""
    z = np.load(GOLDEN / f"{name}.npz", allow_pickle=False)
    meta = json.loads(str(z["meta_json"]))
    out = {"meta": meta}
    for key in z.files:
        if key == "meta_json":
            continue
        out[key] = _tensor(z[key], meta["dtype"])
    return out


def oracle_setup(fx: dict):
    """OracleConfig/OracleParams matching a fixture's reference mixer."""
    from oracle.kvm_oracle import OracleConfig, OracleParams

    m = fx["meta"]
    cfg = OracleConfig(
        q_heads=m["Hq"], kv_heads=m["Hkv"], head_dim=m["D"], value_dim=m["D"],
        chunk_len=m["C"], n_bswa_chunks=m["n_bswa"], n_max_d_chunks=m["n_max"],
        sink_len=m["sink"], rope_partial_dim=m["rope"] if m["rope"] > 0 else m["D"],
        state_budget_mode=m["mode"], state_growth_factor=m["factor"],
        state_growth_exponent=m["expo"], state_round_down=m.get("round_down", 1), state_min_len=m["min_len"],
        state_saturation_n=m.get("sat_n"),
        gate_appends=bool(m["gate_appends"]), gate_initial=bool(m["gate_initial"]),
        use_head_temps=bool(m["temps"]), gate_keys=bool(m.get("gate_keys", 1)),
        gate_values=bool(m.get("gate_values", 1)), use_vlens=bool(m.get("vlens", 1)),
        fp32_routing=m.get("routing", "fp32") == "fp32",
    )
    p = OracleParams(
        ln_weight=fx["in_ln_w"], ln_bias=fx["in_ln_b"],
        front_temp=fx["in_front_temp"], state_temp=fx["in_state_temp"],
    )
    return cfg, p


BACKBONE = GOLDEN / "backbone"


def backbone_names():
    return sorted(p.stem for p in BACKBONE.glob("*.npz"))


def load_backbone(name: str) -> dict:
    """Whole-decoder fixture of tests/golden/make_golden_backbone.py: meta,
    bf16 ``params`` (reference state_dict names), ``input_ids`` [B,T],
    fp32 ``prefill_logits`` [B,T,V], greedy ``decode_tokens`` [B,N] and
    ``decode_logits`` [B,N,V] (logits after feeding decode token s)."""
    z = np.load(BACKBONE / f"{name}.npz", allow_pickle=False)
    out = {"meta": json.loads(str(z["meta_json"]))}
    out["params"] = {k[len("param."):]: torch.from_numpy(np.array(z[k])).view(torch.bfloat16)
                     for k in z.files if k.startswith("param.")}
    for key in ("input_ids", "prefill_logits", "decode_tokens", "decode_logits"):
        out[key] = torch.from_numpy(np.array(z[key]))
    return out


def backbone_model(fx: dict, mixer_path: str | None = None, device="cpu"):
    """The build's decoder with a fixture's config and weights (bf16, eval).
    ``mixer_path`` overrides the token mixer class path; by default the
    reference's path in the fixture resolves to the HIP mixer."""
    from kvm_amd.backbone import MixerConfig, RWKV7BackboneForCausalLM

    m = dict(fx["meta"]["model"])
    if mixer_path is not None:
        m["token_mixer_class_path"] = mixer_path
    model = RWKV7BackboneForCausalLM(MixerConfig(**m)).to(torch.bfloat16)
    model.load_state_dict(fx["params"], strict=True)
    return model.to(device).eval()
