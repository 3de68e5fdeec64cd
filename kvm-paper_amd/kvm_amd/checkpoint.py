"""Reference checkpoints and carried states into this build.

Weights.  The reference writes two checkpoint forms:

* at the end of a run, ``raw_model.save_pretrained(logdir)`` (trainer.py:286):
  ``config.json`` (the MixerConfig fields, model/rwkv7_backbone.py:276-405)
  and ``model.safetensors``, or ``model-*.safetensors`` shards listed in
  ``model.safetensors.index.json``;
* during a run, ``torch.save({"step", "model": state_dict, "optimizers"},
  "model_stepNNNNNN.pt")`` (trainer.py:265-281).

``examine_ckpt.py:16-19`` also reads bare state dicts from ``.safetensors``
or ``.pt`` files.  ``load_reference_checkpoint`` accepts all of these.
Parameter names are the reference's, so the state dict loads strictly.
``.pt`` files are read with ``torch.load(weights_only=True)``, which
executes nothing from the file.

Carried state.  The eager mixer keeps its decode state as a dict with the
keys ``kvm_s_k, kvm_s_v, kvm_s_vlen, kvm_state_coverage_len,
kvm_bswa_begin, kvm_bswa_k, kvm_bswa_v, kvm_bswa_merge_gate``
(model/kvm_mixer.py:518-525).  ``snapshot_from_states`` turns it into a
``DecodeCacheSnapshot``, from which ``SequenceMixer.make_decode_cache``
builds the HIP decode cache that continues the sequence.  The other
direction is ``KVMDecodeCache.logical_state_dict()``.
"""

from __future__ import annotations

import json
from pathlib import Path
from typing import Any

import torch

from .backbone import MixerConfig, RWKV7BackboneForCausalLM
from .decode_cache import DecodeCacheSnapshot

_WRAPPER_PREFIXES = ("_orig_mod.", "module.")


def _clean_key(key: str) -> str:
    """Drop wrapper prefixes that torch.compile / DDP put on parameter names."""
    changed = True
    while changed:
        changed = False
        for p in _WRAPPER_PREFIXES:
            if key.startswith(p):
                key, changed = key[len(p):], True
        key = key.replace("._orig_mod.", ".")
    return key


def _read_safetensors(path: Path) -> dict[str, torch.Tensor]:
    from safetensors.torch import load_file

    return load_file(str(path))


def read_state_dict(path: str | Path) -> dict[str, torch.Tensor]:
    """Model tensors of a checkpoint directory, ``.safetensors`` file or
    ``.pt`` file (a trainer checkpoint dict or a bare state dict)."""
    path = Path(path)
    if path.is_dir():
        index = path / "model.safetensors.index.json"
        if index.exists():
            files = sorted(set(json.loads(index.read_text())["weight_map"].values()))
            sd: dict[str, torch.Tensor] = {}
            for f in files:
                sd.update(_read_safetensors(path / f))
        elif (path / "model.safetensors").exists():
            sd = _read_safetensors(path / "model.safetensors")
        else:
            raise FileNotFoundError(f"{path}: no model.safetensors or model.safetensors.index.json")
    elif path.suffix == ".safetensors":
        sd = _read_safetensors(path)
    else:
        obj = torch.load(str(path), map_location="cpu", weights_only=True)
        sd = obj["model"] if isinstance(obj, dict) and isinstance(obj.get("model"), dict) else obj
        if not isinstance(sd, dict):
            raise ValueError(f"{path}: not a state dict or a trainer checkpoint")
    return {_clean_key(k): v for k, v in sd.items()}


def read_config(path: str | Path) -> MixerConfig:
    """MixerConfig from a checkpoint directory's config.json (or the file)."""
    path = Path(path)
    cfg_file = path / "config.json" if path.is_dir() else path
    return MixerConfig(**json.loads(cfg_file.read_text()))


def load_reference_checkpoint(path: str | Path, config: MixerConfig | dict | None = None, *,
                              token_mixer_class_path: str | None = None, device: Any = None,
                              dtype: torch.dtype = torch.bfloat16, strict: bool = True) -> RWKV7BackboneForCausalLM:
    """The decoder with a reference checkpoint's weights.

    ``config``: a MixerConfig or dict of its fields; by default the
    checkpoint directory's (or the ``.pt`` / ``.safetensors`` file's
    directory's) ``config.json``.  ``token_mixer_class_path`` overrides the
    config's mixer (the reference's KVM paths resolve to the HIP mixer).
    The model is built on the meta device and takes the checkpoint's tensors,
    so no initialisation runs."""
    path = Path(path)
    if config is None:
        config = read_config(path if path.is_dir() else path.parent)
    elif isinstance(config, dict):
        config = MixerConfig(**config)
    if token_mixer_class_path is not None:
        config.token_mixer_class_path = token_mixer_class_path
    sd = read_state_dict(path)
    with torch.device("meta"):
        model = RWKV7BackboneForCausalLM(config)
    model.load_state_dict(sd, strict=strict, assign=True)
    missing = [n for n, t in list(model.named_parameters()) + list(model.named_buffers()) if t.is_meta]
    if missing:
        raise ValueError(f"{path}: the checkpoint has no tensor for {missing[:8]}"
                         f"{' ...' if len(missing) > 8 else ''} (nothing to initialise them from)")
    model = model.to(dtype=dtype)
    if device is not None:
        model = model.to(device)
    return model.eval()


def snapshot_from_states(states: dict[str, Any]) -> DecodeCacheSnapshot:
    """DecodeCacheSnapshot of the eager mixer's carried-state dict
    (model/kvm_mixer.py:518-525).  The window holds tokens
    [kvm_bswa_begin, total_len), so total_len = kvm_bswa_begin + its length."""
    begin = int(states["kvm_bswa_begin"])
    bk = states["kvm_bswa_k"]
    return DecodeCacheSnapshot(
        state_k=states["kvm_s_k"], state_v=states["kvm_s_v"], state_vlen=states["kvm_s_vlen"],
        recent_k=bk, recent_v=states["kvm_bswa_v"], recent_gate=states["kvm_bswa_merge_gate"],
        total_len=begin + int(bk.size(2)), state_coverage_len=int(states["kvm_state_coverage_len"]),
        recent_begin=begin,
    )


__all__ = ["load_reference_checkpoint", "read_config", "read_state_dict", "snapshot_from_states"]
