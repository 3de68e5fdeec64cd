"""Load the golden fixtures written by tests/golden/make_golden.py."""

from __future__ import annotations

import json
from pathlib import Path

import numpy as np
import torch

GOLDEN = Path(__file__).resolve().parent / "golden"


def names():
    return sorted(p.stem for p in GOLDEN.glob("*.npz"))


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
        state_growth_exponent=m["expo"], state_round_down=1, state_min_len=m["min_len"],
        gate_appends=bool(m["gate_appends"]), gate_initial=bool(m["gate_initial"]),
        use_head_temps=bool(m["temps"]),
    )
    p = OracleParams(
        ln_weight=fx["in_ln_w"], ln_bias=fx["in_ln_b"],
        front_temp=fx["in_front_temp"], state_temp=fx["in_state_temp"],
    )
    return cfg, p
