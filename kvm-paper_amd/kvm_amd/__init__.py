"""MI355X-native Key-Value Means (KVM) attention forward path.

Public API:
  SequenceMixer            drop-in for model.kvm_triton_mixer.SequenceMixer
  KVMDecodeCache           carried decode state (TritonKVMDecodeCache API)
  DecodeCacheSnapshot      snapshot used to (re)initialise a decode cache
  RWKV7BackboneForCausalLM decoder whose token mixers are SequenceMixer
                           (model.rwkv7_backbone.RWKV7BackboneForCausalLM)
  MixerConfig              its config (the reference's field names/defaults)
  StatesDictCache          per-layer carried-state cache of the decoder
  DecodeGraph              the decoder's single-token step replayed from a HIP graph
  load_reference_checkpoint  the decoder from a reference checkpoint
                           (save_pretrained directory, trainer .pt, .safetensors)
  snapshot_from_states     DecodeCacheSnapshot from the eager mixer's state dict
  load_library             load libkvm_amd.so (raises if it is not built)
"""

from ._lib import load as load_library
from .backbone import DecodeGraph, MixerConfig, RWKV7BackboneForCausalLM, RWKV7BackboneModel, init_random_
from .checkpoint import load_reference_checkpoint, snapshot_from_states
from .decode_cache import DecodeCacheSnapshot, KVMDecodeCache, TritonKVMDecodeCache
from .mixer import SequenceMixer
from .states_cache import StatesDictCache

__all__ = ["SequenceMixer", "KVMDecodeCache", "TritonKVMDecodeCache", "DecodeCacheSnapshot", "load_library",
           "MixerConfig", "RWKV7BackboneForCausalLM", "RWKV7BackboneModel", "StatesDictCache", "init_random_",
           "load_reference_checkpoint", "snapshot_from_states", "DecodeGraph"]
