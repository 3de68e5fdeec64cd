"""ctypes binding of libkvm_amd.so, the C ABI declared in include/kvm_amd.h.

PyTorch is used only for device memory and the current HIP stream; every
computation of the KVM forward path runs in the HIP kernels of the library.
There is no fallback: when the library is missing or fails to load, every
entry point raises.
"""

from __future__ import annotations

import ctypes
import os
from pathlib import Path

import torch

LIB_NAME = "libkvm_amd.so"
LIB_PATH = Path(__file__).resolve().parent / LIB_NAME
ABI_VERSION = 12

KVM_OK = 0
KVM_EINVAL = -1
KVM_EHIP = -2
KVM_ESPACE = -3
KVM_EABORT = -4
KVM_STATUS_CHAIN_TIMEOUT = 1
KVM_PREFILL_NO_CHAIN = 1

_i64 = ctypes.c_int64
_vp = ctypes.c_void_p


class KvmLayer(ctypes.Structure):
    _fields_ = [
        ("batch", _i64), ("q_heads", _i64), ("kv_heads", _i64),
        ("head_dim", _i64), ("value_dim", _i64), ("chunk_len", _i64),
        ("n_bswa_chunks", _i64), ("sink_len", _i64), ("rope_partial_dim", _i64),
        ("gate_keys", _i64), ("gate_values", _i64), ("gate_appends", _i64),
        ("gate_initial", _i64), ("ln_eps", ctypes.c_double),
        ("ln_weight", _vp), ("ln_bias", _vp), ("state_temp", _vp), ("front_temp", _vp),
    ]


class KvmSeq(ctypes.Structure):
    _fields_ = [
        ("k", _vp), ("v", _vp), ("gate", _vp),
        ("k_sb", _i64), ("k_sh", _i64), ("k_st", _i64),
        ("v_sb", _i64), ("v_sh", _i64), ("v_st", _i64),
        ("g_sb", _i64), ("g_sh", _i64), ("g_st", _i64),
        ("ring", _i64),
    ]


class KvmState(ctypes.Structure):
    _fields_ = [
        ("s_k", _vp), ("s_v", _vp), ("s_vlen", _vp),
        ("s_k_attn", _vp), ("s_v_attn", _vp), ("capacity", _i64),
    ]


class KvmPrefillDesc(ctypes.Structure):
    _fields_ = [
        ("layer", KvmLayer),
        ("q", _vp), ("q_sb", _i64), ("q_sh", _i64), ("q_st", _i64),
        ("kv", KvmSeq),
        ("seq_len", _i64),
        ("out", _vp), ("o_sb", _i64), ("o_st", _i64), ("o_sh", _i64),
        ("state", KvmState),
        ("n_chunks", _i64),
        ("chunk_state_len", ctypes.POINTER(ctypes.c_int32)),
        ("chunk_snapshot", ctypes.POINTER(ctypes.c_int32)),
        ("n_updates", _i64),
        ("upd_token_begin", ctypes.POINTER(ctypes.c_int32)),
        ("upd_state_before", ctypes.POINTER(ctypes.c_int32)),
        ("upd_n_append", ctypes.POINTER(ctypes.c_int32)),
        ("max_state_len", _i64),
        ("snapshot_ring", _i64),
        ("workspace", _vp), ("workspace_bytes", _i64),
        ("route_log", _vp), ("append_log", _vp),
        ("events", _vp),
        ("status", _vp),
        ("lse", _vp),
        ("snap_k", _vp), ("snap_v", _vp),
        ("flags", _i64),
    ]


class KvmPrefillBwdDesc(ctypes.Structure):
    _fields_ = [
        ("layer", KvmLayer),
        ("q", _vp), ("q_sb", _i64), ("q_sh", _i64), ("q_st", _i64),
        ("kv", KvmSeq),
        ("seq_len", _i64),
        ("dout", _vp), ("do_sb", _i64), ("do_st", _i64), ("do_sh", _i64),
        ("lse", _vp), ("delta", _vp),
        ("out", _vp), ("o_sb", _i64), ("o_st", _i64), ("o_sh", _i64),
        ("snap_k", _vp), ("snap_v", _vp),
        ("max_state_len", _i64),
        ("n_chunks", _i64),
        ("chunk_state_len", ctypes.POINTER(ctypes.c_int32)),
        ("chunk_snapshot", ctypes.POINTER(ctypes.c_int32)),
        ("dq", _vp), ("dq_sb", _i64), ("dq_sh", _i64), ("dq_st", _i64),
        ("dk", _vp), ("dv", _vp),
        ("d_snap_k", _vp), ("d_snap_v", _vp),
        ("d_state_temp", _vp), ("d_front_temp", _vp),
        ("workspace", _vp), ("workspace_bytes", _i64),
    ]


class KvmStateBwdDesc(ctypes.Structure):
    _fields_ = [
        ("layer", KvmLayer),
        ("kv", KvmSeq),
        ("seq_len", _i64), ("initial_state_len", _i64), ("n_updates", _i64),
        ("upd_token_begin", ctypes.POINTER(ctypes.c_int32)),
        ("upd_state_before", ctypes.POINTER(ctypes.c_int32)),
        ("upd_n_append", ctypes.POINTER(ctypes.c_int32)),
        ("route_log", _vp), ("append_log", _vp),
        ("max_state_len", _i64),
        ("d_snap_k", _vp), ("d_snap_v", _vp),
        ("dk", _vp), ("dv", _vp), ("dgate", _vp),
        ("d_ln", _vp),
        ("workspace", _vp), ("workspace_bytes", _i64),
    ]


class KvmPrefixDesc(ctypes.Structure):
    _fields_ = [
        ("batch", _i64), ("seq_len", _i64), ("q_heads", _i64), ("kv_heads", _i64),
        ("head_dim", _i64), ("value_dim", _i64), ("value_residual_mode", _i64), ("token_shift", _i64),
        ("ln_eps", ctypes.c_double),
        ("q_lin", _vp), ("k_lin", _vp), ("v_lin", _vp), ("v_first", _vp), ("gate_lin", _vp), ("key_weight", _vp),
        ("q_prev", _vp), ("k_prev", _vp), ("v_prev", _vp),
        ("x_q", _vp), ("x_k", _vp), ("x_v", _vp), ("v_gate0", _vp), ("lamb", _vp),
        ("ln_q_w", _vp), ("ln_q_b", _vp), ("ln_k_w", _vp), ("ln_k_b", _vp),
        ("cos", _vp), ("sin", _vp), ("rope_sb", _i64), ("rope_st", _i64), ("qkv_st", _i64), ("kw_st", _i64),
        ("q_out", _vp), ("k_out", _vp), ("v_out", _vp), ("gate_out", _vp), ("v_last_out", _vp),
        ("q_last_out", _vp), ("k_last_out", _vp),
        ("ring_k", _vp), ("ring_v", _vp), ("ring_gate", _vp), ("ring_cap", _i64), ("ring_pos", _i64),
        ("ring_ctl", _vp),
    ]


class KvmAddNormDesc(ctypes.Structure):
    _fields_ = [
        ("x", _vp), ("y", _vp), ("alpha", ctypes.c_double), ("round_product", _i64),
        ("ln_w", _vp), ("ln_b", _vp), ("eps", ctypes.c_double),
        ("mix", _vp), ("prev", _vp),
        ("out_x", _vp), ("out_h", _vp), ("out_shift", _vp), ("state_out", _vp),
        ("batch", _i64), ("seq_len", _i64), ("width", _i64),
    ]


# Exported symbols and their signatures (include/kvm_amd.h).
_P = ctypes.POINTER
SIGNATURES = {
    "kvm_abi_version": (ctypes.c_int, []),
    "kvm_struct_size": (_i64, [ctypes.c_int]),
    "kvm_last_error": (ctypes.c_char_p, []),
    "kvm_prefill_workspace_bytes": (_i64, [_P(KvmPrefillDesc)]),
    "kvm_prefill": (ctypes.c_int, [_P(KvmPrefillDesc), _vp]),
    "kvm_prefill_backward_workspace_bytes": (_i64, [_P(KvmPrefillBwdDesc)]),
    "kvm_prefill_backward": (ctypes.c_int, [_P(KvmPrefillBwdDesc), _vp]),
    "kvm_state_backward_workspace_bytes": (_i64, [_P(KvmStateBwdDesc)]),
    "kvm_state_backward": (ctypes.c_int, [_P(KvmStateBwdDesc), _vp]),
    "kvm_prefix": (ctypes.c_int, [_P(KvmPrefixDesc), _vp]),
    "kvm_ring_write_dev": (ctypes.c_int, [_P(KvmLayer), _P(KvmSeq), _vp, _vp, _vp, _i64, _vp, _vp]),
    "kvm_decode_attention_dev": (ctypes.c_int, [_P(KvmLayer), _vp, _i64, _i64, _P(KvmState), _vp, ctypes.c_int32,
                                                _vp, _vp, _i64, _vp, _i64, _i64, _vp, _i64, _vp]),
    "kvm_decode_advance": (ctypes.c_int, [_vp, _i64, _vp]),
    "kvm_token_shift": (ctypes.c_int, [_vp, _vp, _vp, _vp, _i64, _i64, _i64, ctypes.c_int, _vp]),
    "kvm_relu_square": (ctypes.c_int, [_vp, _vp, _i64, _vp]),
    "kvm_gemm_small": (ctypes.c_int, [_vp, _i64, _vp, _i64, _vp, _i64, _i64, _i64, _i64, ctypes.c_int, _vp]),
    "kvm_add_norm": (ctypes.c_int, [_P(KvmAddNormDesc), _vp]),
    "kvm_gemm_small_tile_rows": (ctypes.c_int, [_i64, _i64]),
    "kvm_gemm_small_packed": (ctypes.c_int, [_vp, _i64, _vp, _vp, _i64, _i64, _i64, _i64, ctypes.c_int,
                                             ctypes.c_int, _vp]),
    "kvm_state_append_direct": (ctypes.c_int, [_P(KvmLayer), _P(KvmSeq), _i64, _i64, _P(KvmState), _i64, _vp]),
    "kvm_state_refresh": (ctypes.c_int, [_P(KvmLayer), _P(KvmState), _i64, _i64, _vp]),
    "kvm_update_workspace_bytes": (_i64, [_P(KvmLayer), _i64]),
    "kvm_state_update": (ctypes.c_int, [_P(KvmLayer), _P(KvmSeq), _i64, _i64, _i64, _i64, _P(KvmState),
                                        _vp, _vp, _vp, _i64, _vp, _vp, _vp]),
    "kvm_ring_write": (ctypes.c_int, [_P(KvmLayer), _P(KvmSeq), _vp, _vp, _vp, _i64, _i64, _vp]),
    "kvm_decode_workspace_bytes": (_i64, [_P(KvmLayer), _i64]),
    "kvm_decode_attention": (ctypes.c_int, [_P(KvmLayer), _vp, _i64, _i64, _P(KvmState), _i64, _vp, _vp,
                                            _i64, _i64, _i64, _vp, _i64, _i64, _vp, _i64, _vp]),
    "kvm_decode_step": (ctypes.c_int, [_P(KvmLayer), _vp, _i64, _i64, _P(KvmState), _i64, _P(KvmSeq), _vp, _vp,
                                       _vp, _i64, _i64, _i64, _vp, _i64, _i64, _vp, _i64, _vp]),
    "kvm_decode_attention_noalloc": (ctypes.c_int, [_P(KvmLayer), _vp, _i64, _i64, _P(KvmState), _i64, _vp,
                                                    _vp, _i64, _i64, _i64, _vp, _i64, _i64, _vp]),
}
# Library-owned scratch of kvm_decode_attention_noalloc per GPU (include/kvm_amd.h).
KVM_DECODE_SCRATCH_BYTES = 16 << 20

_LIB = None


class KvmLibraryError(RuntimeError):
    """The HIP library is missing, fails to load, or reports a HIP error."""


def load(path: str | os.PathLike | None = None):
    """Load libkvm_amd.so once and check its ABI; raise if it is unavailable."""
    global _LIB
    if _LIB is not None and path is None:
        return _LIB
    p = Path(path) if path is not None else LIB_PATH
    if not p.exists():
        raise KvmLibraryError(
            f"{p} is missing: build it with `python -c 'import __graft_entry__ as g; g.build()'` "
            "(hipcc --offload-arch=gfx950); there is no CPU fallback"
        )
    lib = ctypes.CDLL(str(p))
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    if lib.kvm_abi_version() != ABI_VERSION:
        raise KvmLibraryError(f"{p}: ABI version {lib.kvm_abi_version()} != {ABI_VERSION}")
    for i, st in enumerate((KvmLayer, KvmSeq, KvmState, KvmPrefillDesc, KvmPrefixDesc, KvmPrefillBwdDesc,
                              KvmStateBwdDesc, KvmAddNormDesc)):
        if lib.kvm_struct_size(i) != ctypes.sizeof(st):
            raise KvmLibraryError(f"{p}: struct {st.__name__} size mismatch")
    if path is None:
        _LIB = lib
    return lib


OPS_PATH = Path(__file__).resolve().parent / "libkvm_amd_torch.so"
_OPS = None


def ops():
    """``torch.ops.kvm_amd``: the torch operators (``prefill``,
    ``decode_step``) over libkvm_amd.so (csrc/kvm_torch_ops.cpp); loaded
    once, after the C library's ABI check.  Raises if it is not built."""
    global _OPS
    if _OPS is None:
        load()
        if not OPS_PATH.exists():
            raise KvmLibraryError(
                f"{OPS_PATH} is missing: build it with `python -c 'import __graft_entry__ as g; g.build()'`; "
                "there is no CPU fallback")
        torch.ops.load_library(str(OPS_PATH))
        _OPS = torch.ops.kvm_amd
    return _OPS


def call_op(op, *args):
    """Call a torch operator of the library: invalid arguments stay
    ValueError, any other failure it reports becomes KvmLibraryError (a
    RuntimeError, the reference's type for device-level errors)."""
    try:
        return op(*args)
    except ValueError:
        raise
    except RuntimeError as e:
        raise KvmLibraryError(str(e)) from e


def check(rc: int, what: str):
    """Raise the reference's exception type for a failed call."""
    if rc == KVM_OK:
        return
    msg = f"{what}: {load().kvm_last_error().decode(errors='replace')}"
    if rc == KVM_EINVAL:
        raise ValueError(msg)
    raise KvmLibraryError(msg)


def stream_handle(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()


def _bf16_view(t: torch.Tensor, name: str) -> torch.Tensor:
    if t.dtype != torch.bfloat16:
        raise ValueError(f"{name} must be bfloat16 (got {t.dtype})")
    if not t.is_cuda:
        raise RuntimeError(f"{name} must be a ROCm device tensor")
    if t.stride(-1) != 1 or t.data_ptr() % 16 or any(s % 8 for s in t.stride()[:-1]):
        t = t.contiguous()
    return t


def seq4(k: torch.Tensor, v: torch.Tensor, gate: torch.Tensor, ring: int = 0):
    """KvmSeq over [B, H, T, D] key / value views and a [B, H, T, 1] gate.

    Returns (struct, keepalive tensors)."""
    k = _bf16_view(k, "k")
    v = _bf16_view(v, "v")
    if gate.dtype != torch.bfloat16:
        gate = gate.to(torch.bfloat16)
    s = KvmSeq(
        k.data_ptr(), v.data_ptr(), gate.data_ptr(),
        k.stride(0), k.stride(1), k.stride(2),
        v.stride(0), v.stride(1), v.stride(2),
        gate.stride(0), gate.stride(1), gate.stride(2),
        int(ring),
    )
    return s, (k, v, gate)


def seq_rows(k: torch.Tensor, v: torch.Tensor, gate: torch.Tensor, kv_heads: int, ring: int = 0):
    """KvmSeq over row-major [rows, T, D] buffers (rows = batch * kv_heads)
    and a [rows, T] gate, e.g. the decode window ring."""
    rows, cap = int(k.size(0)), int(k.size(1))
    D = int(k.size(2))
    s = KvmSeq(
        k.data_ptr(), v.data_ptr(), gate.data_ptr(),
        kv_heads * cap * D, cap * D, D,
        kv_heads * cap * D, cap * D, D,
        kv_heads * cap, cap, 1,
        int(ring),
    )
    return s, (k, v, gate)


def state_struct(s_k, s_v, s_vlen, s_k_attn, s_v_attn, capacity: int) -> KvmState:
    return KvmState(ptr(s_k), ptr(s_v), ptr(s_vlen), ptr(s_k_attn), ptr(s_v_attn), int(capacity))


def int32_array(values):
    arr = (ctypes.c_int32 * max(len(values), 1))(*[int(v) for v in values])
    return arr
