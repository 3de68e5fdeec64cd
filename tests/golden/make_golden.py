"""Write the golden KVM fixtures from the reference's own eager mixer.

Runs ONLY in the build container, where the read-only reference checkout is
mounted (default ``/root/reference``, override with ``KVM_REFERENCE``).  It
imports ``model.kvm_fp32_routing_reference.SequenceMixer`` (the eager KVM
mixer with FP32 merge routing; ``model/kvm_fp32_routing_reference.py:21-49``)
and the historical golden ``model.kvm_mixer.SequenceMixer``, runs
``forward_prefill`` (``model/kvm_mixer.py:403-516``) and cached single-token
decode (``model/kvm_mixer.py:572-713``) on seeded inputs, and saves inputs and
outputs as ``.npz`` fixtures next to this script.  Nothing of the reference's
source is stored: only tensors (inputs, outputs, per-update routing records).

Routing records are captured from the reference's own calls:
``kvm_mixer._split_append_merge_idx_by_maxsim`` is wrapped to record the
append/merge token split (kvm_mixer.py:44-75, called at :290), and
``torch.scatter`` is wrapped during ``_merge_into_state`` to record the chosen
slot per merged token (the ``best_s_idx`` argument, kvm_mixer.py:328-331 /
kvm_fp32_routing_reference.py:34-40).

Usage:  python tests/golden/make_golden.py
"""

from __future__ import annotations

import json
import os
import sys
import time
from pathlib import Path
from types import SimpleNamespace

import numpy as np
import torch
import torch.nn.functional as F

HERE = Path(__file__).resolve().parent
REF = Path(os.environ.get("KVM_REFERENCE", "/root/reference"))

# Fixture cases: (name, mixer/config overrides, shapes, dtype, decode steps)
CASES = [
    dict(
        name="fixed_bf16_gqa",
        dtype="bf16", B=1, Hq=4, Hkv=2, D=64, T=777, C=64, n_bswa=2,
        sink=1, rope=32, mode="fixed", min_len=64, n_max=1, factor=1.0, expo=0.5,
        decode_steps=0, temps=True, gate_appends=0, gate_initial=0,
    ),
    dict(
        name="growable_bf16",
        dtype="bf16", B=2, Hq=1, Hkv=1, D=64, T=1100, C=64, n_bswa=2,
        sink=1, rope=16, mode="power_law", min_len=64, n_max=3, factor=5.0, expo=0.5,
        decode_steps=0, temps=True, gate_appends=0, gate_initial=0,
    ),
    dict(
        name="fixed_fp32_cfg1shape",
        dtype="fp32", B=1, Hq=2, Hkv=2, D=64, T=640, C=64, n_bswa=2,
        sink=1, rope=32, mode="fixed", min_len=16, n_max=1, factor=1.0, expo=0.5,
        decode_steps=0, temps=False, gate_appends=0, gate_initial=0,
    ),
    dict(
        name="decode_growable_bf16",
        dtype="bf16", B=1, Hq=2, Hkv=1, D=64, T=150, C=32, n_bswa=2,
        sink=2, rope=32, mode="power_law", min_len=32, n_max=3, factor=4.0, expo=0.5,
        decode_steps=120, temps=True, gate_appends=1, gate_initial=1,
    ),
    dict(
        name="decode_short_prompt_bf16",
        dtype="bf16", B=1, Hq=2, Hkv=2, D=64, T=20, C=32, n_bswa=2,
        sink=1, rope=32, mode="fixed", min_len=32, n_max=1, factor=1.0, expo=0.5,
        decode_steps=90, temps=True, gate_appends=0, gate_initial=0,
    ),
    # The saturating budget floor(N t / (N + t)) of the paper's saturate runs
    # (configs/prolong/120M/kvm_swa_saturate1024_wd.yaml: state_min_len 1,
    # state_saturation_n): the state grows by a few slots at every update, so
    # most updates both append and merge; the decode steps cross further
    # boundaries of the same budget.
    dict(
        name="saturation_bf16",
        dtype="bf16", B=1, Hq=2, Hkv=2, D=64, T=1400, C=64, n_bswa=2,
        sink=1, rope=32, mode="kvm_saturation", min_len=1, n_max=10, factor=1.0, expo=0.5,
        sat_n=300, decode_steps=140, temps=True, gate_appends=0, gate_initial=0,
    ),
    # The same budget with state_round_down 16, GQA and gated appends / initial state.
    dict(
        name="saturation_round16_gqa_bf16",
        dtype="bf16", B=2, Hq=4, Hkv=2, D=64, T=1000, C=64, n_bswa=2,
        sink=2, rope=16, mode="kvm_saturation", min_len=1, n_max=8, factor=1.0, expo=0.5,
        sat_n=500, round_down=16, decode_steps=70, temps=True, gate_appends=1, gate_initial=1,
    ),
    # The paper's no-merge-gate ablation (configs/prolong/120M/ablation_kvm_no_merge_gate.yaml:
    # kvm_use_merge_gate_keys / kvm_use_merge_gate_values 0): routes and slot
    # sums use the ungated overflow streams (model/kvm_mixer.py:264-281).
    dict(
        name="no_merge_gate_bf16",
        dtype="bf16", B=1, Hq=4, Hkv=2, D=64, T=700, C=64, n_bswa=2,
        sink=1, rope=32, mode="fixed", min_len=64, n_max=1, factor=1.0, expo=0.5,
        decode_steps=80, temps=True, gate_appends=0, gate_initial=0, gate_keys=0, gate_values=0,
    ),
    # Only the key gate, with growth (appends keep their ungated rows).
    dict(
        name="key_gate_only_growable_bf16",
        dtype="bf16", B=1, Hq=2, Hkv=1, D=64, T=900, C=64, n_bswa=2,
        sink=1, rope=16, mode="power_law", min_len=64, n_max=3, factor=5.0, expo=0.5,
        decode_steps=0, temps=True, gate_appends=0, gate_initial=0, gate_keys=1, gate_values=0,
    ),
    # The no-head-temperature ablation (ablation_kvm_no_head_temps.yaml:
    # kvm_use_head_temps 0), with two sink slots.
    dict(
        name="no_head_temps_bf16",
        dtype="bf16", B=2, Hq=2, Hkv=2, D=64, T=600, C=64, n_bswa=2,
        sink=2, rope=32, mode="fixed", min_len=64, n_max=1, factor=1.0, expo=0.5,
        decode_steps=80, temps=False, gate_appends=0, gate_initial=0,
    ),
    # The historical golden's bf16 merge routing (model/kvm_mixer.py:321-331,
    # the mixer without the FP32 cast): pins the oracle's bf16-routing branch.
    # CPU oracle only: the HIP path always routes in fp32.
    dict(
        name="bf16_routing_bf16",
        dtype="bf16", B=1, Hq=2, Hkv=2, D=64, T=640, C=64, n_bswa=2,
        sink=1, rope=32, mode="fixed", min_len=64, n_max=1, factor=1.0, expo=0.5,
        decode_steps=0, temps=True, gate_appends=0, gate_initial=0, routing="bf16",
    ),
    # kvm_use_vlens 0 (slot counts instead of value norms, model/kvm_mixer.py:
    # 204-208, 337-338): pins the oracle's count branch.  CPU oracle only: the
    # reference's Triton mixer rejects it (model/kvm_triton_mixer.py:218-219),
    # and so does the HIP mixer.
    dict(
        name="no_vlens_bf16",
        dtype="bf16", B=1, Hq=2, Hkv=2, D=64, T=640, C=64, n_bswa=2,
        sink=1, rope=32, mode="fixed", min_len=64, n_max=1, factor=1.0, expo=0.5,
        decode_steps=40, temps=True, gate_appends=0, gate_initial=0, vlens=0,
    ),
]


class LayerStatesCache:
    """Per-layer states dict plus a seen-token counter.

    The three calls the KVM mixer makes on its cache
    (model/statesdictcache.py:141-187, used at kvm_mixer.py:501, 586-595, 699):
    ``get_seq_length``, ``get_states`` and ``update(layer_idx, offset,
    states_dict)``.  The reference's own ``StatesDictCache`` cannot be built
    with the container's transformers 5.15 (its layer class misses the
    abstract ``get_max_length``), so this stand-in carries the same contract.
    """

    def __init__(self):
        self.states = {}
        self.seen = {}

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


def _import_reference():
    sys.path.insert(0, str(REF))
    import model.kvm_mixer as eager  # noqa: E402
    import model.kvm_fp32_routing_reference as fp32ref  # noqa: E402

    return eager, fp32ref, LayerStatesCache


def _config(case):
    return SimpleNamespace(
        num_attention_heads=case["Hq"], num_key_value_heads=case["Hkv"],
        hidden_size=case["Hq"] * case["D"], d_qk_head=case["D"], d_v_head=case["D"], d_head=None,
        num_hidden_layers=1, mup_base_dim=case["Hq"] * case["D"],
        use_tokenshift_att=0, use_value_residual=0,
        kvm_value_residual_mode="rwkv", kvm_token_shift_mode="rwkv",
        rope_partial_dim=case["rope"], sink_len=case["sink"], chunk_len=case["C"],
        n_max_d_chunks=case["n_max"], n_bswa_chunks=case["n_bswa"],
        state_budget_mode=case["mode"], state_growth_factor=case["factor"],
        state_growth_exponent=case["expo"], state_round_down=case.get("round_down", 1),
        state_min_len=case["min_len"], state_saturation_n=case.get("sat_n"),
        kvm_use_merge_gate_keys=case.get("gate_keys", 1), kvm_use_merge_gate_values=case.get("gate_values", 1),
        kvm_apply_merge_gate_to_appends=case["gate_appends"],
        kvm_apply_merge_gate_to_initial_state=case["gate_initial"],
        kvm_use_head_temps=int(case["temps"]), kvm_use_vlens=case.get("vlens", 1),
        kvm_aotriton_forward_attention=0,
    )


def _inputs(case, gen):
    dt = torch.bfloat16 if case["dtype"] == "bf16" else torch.float32
    B, Hq, Hkv, D, T = case["B"], case["Hq"], case["Hkv"], case["D"], case["T"]
    n_dec = case["decode_steps"]
    q = torch.randn(B, Hq, T + n_dec, D, generator=gen).to(dt)
    k = torch.randn(B, Hkv, T + n_dec, D, generator=gen).to(dt)
    v = torch.randn(B, Hkv, T + n_dec, D, generator=gen).to(dt)
    gate = (1.0 + F.elu(torch.randn(B, Hkv, T + n_dec, 1, generator=gen))).to(dt)
    ln_w = (1.0 + 0.1 * torch.randn(D, generator=gen)).to(dt)
    ln_b = (0.1 * torch.randn(D, generator=gen)).to(dt)
    ft = (1.0 + 0.1 * torch.randn(Hq, generator=gen)).to(dt)
    st = (1.0 + 0.1 * torch.randn(Hq, generator=gen)).to(dt)
    return dict(q=q, k=k, v=v, gate=gate, ln_w=ln_w, ln_b=ln_b, front_temp=ft, state_temp=st)


def _as_np(t: torch.Tensor):
    if t.dtype == torch.bfloat16:
        return t.contiguous().view(torch.int16).numpy()
    return t.contiguous().numpy()


def _run_case(case, eager, fp32ref, StatesDictCache):
    gen = torch.Generator().manual_seed(1234 + len(case["name"]))
    inp = _inputs(case, gen)
    dt = inp["q"].dtype
    # The FP32-routing mixer, or the historical golden (bf16 routing) it derives from.
    mixer_cls = eager.SequenceMixer if case.get("routing") == "bf16" else fp32ref.SequenceMixer
    mixer = mixer_cls(_config(case), 0).to(dt).eval()
    with torch.no_grad():
        mixer.ln_s_k.weight.copy_(inp["ln_w"])
        mixer.ln_s_k.bias.copy_(inp["ln_b"])
        if case["temps"]:
            mixer.front_head_temp.copy_(inp["front_temp"])
            mixer.state_head_temp.copy_(inp["state_temp"])
    mixer.c_proj = torch.nn.Identity()

    records = []
    orig_split = eager._split_append_merge_idx_by_maxsim
    orig_scatter = torch.scatter
    orig_merge = mixer_cls._merge_into_state

    def split_wrapper(k_block, n_append, k_ref):
        app, mrg = orig_split(k_block, n_append, k_ref)
        records.append({"kind": "split", "append_idx": app.clone(), "merge_idx": mrg.clone(),
                         "state_len": int(k_ref.size(2)), "n_append": int(n_append)})
        return app, mrg

    def merge_wrapper(self, k_merge, v_merge, s_k, s_v, s_vlen, protected_slots):
        captured = {}

        def scatter_wrapper(inp_t, dim, index, src, *a, **kw):
            captured["route"] = index.clone()
            return orig_scatter(inp_t, dim, index, src, *a, **kw)

        torch.scatter = scatter_wrapper
        try:
            out = orig_merge(self, k_merge, v_merge, s_k, s_v, s_vlen, protected_slots)
        finally:
            torch.scatter = orig_scatter
        records.append({"kind": "merge", "route": captured["route"].squeeze(-1),
                        "state_len": int(s_k.size(2)), "protected": int(protected_slots)})
        return out

    eager._split_append_merge_idx_by_maxsim = split_wrapper
    mixer_cls._merge_into_state = merge_wrapper
    try:
        T = case["T"]
        cache = StatesDictCache() if case["decode_steps"] else None
        t0 = time.time()
        with torch.no_grad():
            y = mixer.forward_prefill(
                inp["q"][:, :, :T], inp["k"][:, :, :T], inp["v"][:, :, :T], inp["gate"][:, :, :T],
                None, None, None, cache,
            )
        prefill_s = time.time() - t0
        n_prefill_records = len(records)
        dec_out = []
        if cache is not None:
            with torch.no_grad():
                for s in range(case["decode_steps"]):
                    t = T + s
                    yd = mixer.forward_single(
                        inp["q"][:, :, t:t + 1], inp["k"][:, :, t:t + 1], inp["v"][:, :, t:t + 1],
                        inp["gate"][:, :, t:t + 1], None, None, None, cache,
                    )
                    dec_out.append(yd)
            st = cache.get_states(0)
        else:
            st = None
    finally:
        eager._split_append_merge_idx_by_maxsim = orig_split
        mixer_cls._merge_into_state = orig_merge

    out = {}
    for key, t in inp.items():
        out["in_" + key] = _as_np(t)
    B, Hq, D = case["B"], case["Hq"], case["D"]
    out["y_prefill"] = _as_np(y.view(B, T, Hq, D).transpose(1, 2))
    if dec_out:
        out["y_decode"] = _as_np(torch.cat(dec_out, dim=1).view(B, -1, Hq, D).transpose(1, 2))
        for key in ("kvm_s_k", "kvm_s_v", "kvm_s_vlen", "kvm_bswa_k", "kvm_bswa_v", "kvm_bswa_merge_gate"):
            out["final_" + key] = _as_np(st[key])
        out["final_kvm_state_coverage_len"] = np.array(int(st["kvm_state_coverage_len"]))
        out["final_kvm_bswa_begin"] = np.array(int(st["kvm_bswa_begin"]))
    # Per-update entries.  An update that appends starts with a split record
    # and merges afterwards unless every token was appended (then the
    # reference skips the merge, kvm_mixer.py:307-308); an update without
    # appends has only its merge record.  "state_len_at_merge" is the state
    # length after the update's appends.
    def per_update(recs):
        upd = []
        for r in recs:
            if r["kind"] == "split":
                n_merge = int(r["merge_idx"].size(-1))
                route = torch.zeros(*r["merge_idx"].shape[:-1], 0, dtype=torch.int64)
                upd.append({"append_idx": r["append_idx"], "merge_idx": r["merge_idx"], "route": route,
                            "state_len_at_merge": r["state_len"] + r["n_append"], "open": n_merge > 0})
            elif upd and upd[-1].get("open"):
                upd[-1]["route"] = r["route"]
                upd[-1]["open"] = False
                assert upd[-1]["state_len_at_merge"] == r["state_len"]
            else:
                upd.append({"route": r["route"], "state_len_at_merge": r["state_len"]})
        return upd

    upd = per_update(records)
    n_prefill_updates = len(per_update(records[:n_prefill_records]))
    for i, u in enumerate(upd):
        out[f"upd{i}_route"] = u["route"].numpy().astype(np.int32)
        out[f"upd{i}_state_len_at_merge"] = np.array(u["state_len_at_merge"])
        if "append_idx" in u:
            out[f"upd{i}_append_idx"] = u["append_idx"].numpy().astype(np.int32)
            out[f"upd{i}_merge_idx"] = u["merge_idx"].numpy().astype(np.int32)
    meta = dict(case)
    meta.update(
        n_updates=len(upd), n_prefill_updates=n_prefill_updates,
        torch_version=torch.__version__, prefill_seconds=prefill_s,
        reference=("SmerkyG/KVM-paper eager model.kvm_mixer.SequenceMixer (bf16 routing)"
                   if case.get("routing") == "bf16" else
                   "SmerkyG/KVM-paper eager model.kvm_fp32_routing_reference.SequenceMixer"),
    )
    out["meta_json"] = np.array(json.dumps(meta))
    return out


def main():
    """Write every case, or only the cases named on the command line."""
    eager, fp32ref, StatesDictCache = _import_reference()
    torch.manual_seed(0)
    wanted = set(sys.argv[1:])
    for case in CASES:
        if wanted and case["name"] not in wanted:
            continue
        data = _run_case(case, eager, fp32ref, StatesDictCache)
        path = HERE / f"{case['name']}.npz"
        np.savez_compressed(path, **data)
        meta = json.loads(str(data["meta_json"]))
        print(f"wrote {path.name}: {path.stat().st_size/1024:.0f} KiB, updates={meta['n_updates']}")


if __name__ == "__main__":
    main()
