"""Shared helpers of the KVM tests: mixer construction, caches, tolerances."""

from __future__ import annotations

import os
from types import SimpleNamespace

import torch

# Output tolerance of the north star: bf16 outputs against the reference,
# max |err| <= 2e-2 and mean |err| <= 2e-3, errors measured in fp32.
MAX_ABS = 2e-2
MEAN_ABS = 2e-3


def gpu_available() -> bool:
    return torch.cuda.is_available()


def mixer_config(Hq, Hkv, D, C, n_bswa=2, sink=1, rope=32, mode="fixed", min_len=-1, n_max=1,
                 factor=1.0, expo=0.5, sat_n=None, temps=True, gate_appends=0, gate_initial=0,
                 gate_keys=1, gate_values=1, round_down=1):
    """Config namespace with every attribute the KVM mixer reads."""
    return SimpleNamespace(
        num_attention_heads=Hq, num_key_value_heads=Hkv, hidden_size=Hq * D, d_qk_head=D, d_v_head=D,
        d_head=None, num_hidden_layers=1, mup_base_dim=Hq * D, use_tokenshift_att=0, use_value_residual=0,
        kvm_value_residual_mode="rwkv", kvm_token_shift_mode="rwkv", rope_partial_dim=rope,
        sink_len=sink, chunk_len=C, n_max_d_chunks=n_max, n_bswa_chunks=n_bswa,
        state_budget_mode=mode, state_growth_factor=factor, state_growth_exponent=expo,
        state_round_down=round_down, state_min_len=min_len, state_saturation_n=sat_n,
        kvm_use_merge_gate_keys=gate_keys, kvm_use_merge_gate_values=gate_values,
        kvm_apply_merge_gate_to_appends=gate_appends, kvm_apply_merge_gate_to_initial_state=gate_initial,
        kvm_use_head_temps=int(temps), kvm_use_vlens=1, kvm_aotriton_forward_attention=0,
    )


def fixture_config(meta):
    return mixer_config(
        meta["Hq"], meta["Hkv"], meta["D"], meta["C"], n_bswa=meta["n_bswa"], sink=meta["sink"],
        rope=meta["rope"], mode=meta["mode"], min_len=meta["min_len"], n_max=meta["n_max"],
        factor=meta["factor"], expo=meta["expo"], temps=meta["temps"],
        gate_appends=meta["gate_appends"], gate_initial=meta["gate_initial"],
        sat_n=meta.get("sat_n"), round_down=meta.get("round_down", 1),
        gate_keys=meta.get("gate_keys", 1), gate_values=meta.get("gate_values", 1),
    )


def make_mixer(cfg, ln_w, ln_b, front_temp=None, state_temp=None, device="cuda"):
    from kvm_amd import SequenceMixer

    m = SequenceMixer(cfg, 0).to(device=device, dtype=torch.bfloat16).eval()
    with torch.no_grad():
        m.ln_s_k.weight.copy_(ln_w)
        m.ln_s_k.bias.copy_(ln_b)
        if cfg.kvm_use_head_temps:
            m.front_head_temp.copy_(front_temp)
            m.state_head_temp.copy_(state_temp)
    m.c_proj = torch.nn.Identity()
    return m


class LayerStatesCache:
    """Per-layer states dict plus a seen-token counter: the three calls the
    mixer makes on its cache (model/statesdictcache.py:141-187)."""

    def __init__(self):
        self.states, self.seen = {}, {}

    def get_seq_length(self, layer_idx):
        return self.seen.get(layer_idx, 0)

    def get_states(self, layer_idx):
        return self.states.setdefault(layer_idx, {})

    def update(self, layer_idx, offset=1, states_dict=None):
        st = self.states.setdefault(layer_idx, {})
        if states_dict:
            st.update(states_dict)
        self.seen[layer_idx] = self.seen.get(layer_idx, 0) + offset
        return st


def err_stats(a: torch.Tensor, b: torch.Tensor):
    d = (a.detach().float().cpu() - b.detach().float().cpu()).abs()
    return float(d.max()), float(d.mean())


def assert_close_bf16(a, b, what, max_abs=MAX_ABS, mean_abs=MEAN_ABS):
    mx, mean = err_stats(a, b)
    assert mx <= max_abs and mean <= mean_abs, f"{what}: max |err| {mx:.3e} (<= {max_abs}), mean {mean:.3e} (<= {mean_abs})"
    return mx, mean


def log(msg: str):
    print(msg, flush=True)
    if os.environ.get("KVM_TEST_LOG"):
        with open(os.environ["KVM_TEST_LOG"], "a") as f:
            f.write(msg + "\n")
