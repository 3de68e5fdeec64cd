"""MI355X-native Key-Value Means (KVM) attention forward path.

Public API:
  SequenceMixer            drop-in for model.kvm_triton_mixer.SequenceMixer
  KVMDecodeCache           carried decode state (TritonKVMDecodeCache API)
  DecodeCacheSnapshot      snapshot used to (re)initialise a decode cache
  load_library             load libkvm_amd.so (raises if it is not built)
"""

from ._lib import load as load_library
from .decode_cache import DecodeCacheSnapshot, KVMDecodeCache, TritonKVMDecodeCache
from .mixer import SequenceMixer

__all__ = ["SequenceMixer", "KVMDecodeCache", "TritonKVMDecodeCache", "DecodeCacheSnapshot", "load_library"]
