"""Linear layers of the decoder's single-token decode step.

A decode step multiplies a few token rows (M <= 16) by each weight matrix, so
it is bound by reading the weights once; ``kvm_gemm_small`` streams them at
HBM speed where a general GEMM does not.  Everything else (prefill, training,
CPU tensors) goes to ``torch.nn.functional.linear``.
"""

from __future__ import annotations

import os
import weakref

import torch
import torch.nn.functional as F

from . import _lib


def linear(x: torch.Tensor, weight: torch.Tensor, bias: torch.Tensor | None = None, *,
           relu_square: bool = False) -> torch.Tensor:
    """``F.linear(x, weight, bias)``; bf16 inference on at most 16 rows runs
    ``kvm_gemm_small`` (fp32 accumulation, one bf16 rounding).  With
    ``relu_square`` the result is relu(y)^2 (the decoder MLP's activation),
    computed in the GEMM's epilogue or by ``kvm_relu_square``; that flag is
    for bf16 GPU inference only."""
    K = int(weight.shape[-1])
    small = not (bias is not None or not x.is_cuda or x.dtype != torch.bfloat16 or weight.dtype != torch.bfloat16
                 or K % 32 or x.shape[-1] != K
                 or (torch.is_grad_enabled() and (x.requires_grad or weight.requires_grad)))
    M = x.numel() // K if small else 0
    if not small or M < 1 or M > 16:
        y = F.linear(x, weight, bias)
        return _relu_square(y, out=y) if relu_square else y
    x2 = x.reshape(M, K)
    # The stride of a single row is meaningless to torch (it may be anything);
    # the kernel only needs K for it.
    x_st = K if M == 1 else int(x2.stride(0))
    if x2.stride(-1) != 1 or x_st % 8 or x_st < K or x2.data_ptr() % 16:
        # clone, not contiguous(): a contiguous but misaligned view (a split
        # of a wider row) would come back unchanged.
        x2 = x2.clone(memory_format=torch.contiguous_format)
        x_st = K
    N = int(weight.shape[0])
    y = torch.empty(M, N, device=x.device, dtype=torch.bfloat16)
    lib = _lib.load()
    rows = lib.kvm_gemm_small_tile_rows(M, N)
    wp = _packed(weight, rows)
    if wp is not None:
        _lib.check(lib.kvm_gemm_small_packed(x2.data_ptr(), x_st, wp.data_ptr(), y.data_ptr(), N, M, N, K, rows,
                                             int(relu_square), _lib.stream_handle(x.device)),
                   "kvm_gemm_small_packed")
        return y.view(*x.shape[:-1], N)
    w = weight
    w_st = K if N == 1 else int(w.stride(0))
    if w.stride(-1) != 1 or w_st % 8 or w_st < K or w.data_ptr() % 16:
        w = weight.clone(memory_format=torch.contiguous_format)
        w_st = K
    _lib.check(lib.kvm_gemm_small(x2.data_ptr(), x_st, w.data_ptr(), w_st, y.data_ptr(), N,
                                  M, N, K, int(relu_square), _lib.stream_handle(x.device)), "kvm_gemm_small")
    return y.view(*x.shape[:-1], N)


# Weights re-arranged for kvm_gemm_small_packed, per weight tensor (by id,
# dropped when the tensor is freed) and tile height, rebuilt when the weight
# changes (data pointer or version counter).
_PACKS: dict[int, dict] = {}


def _packed(weight: torch.Tensor, rows: int) -> torch.Tensor | None:
    """``weight`` [N, K] in the chunk layout of kvm_gemm_small_packed for
    ``rows``-row tiles (include/kvm_amd.h), made once per weight outside
    graph capture (a second copy of every decode weight in HBM); None where
    the layout does not apply (K not a multiple of the chunk width), while a
    graph is being captured and the weight has no current pack, or with
    KVM_AMD_PACK_WEIGHTS=0 (the plain kernel then runs)."""
    N, K = (int(d) for d in weight.shape)
    kc = 64 if rows == 8 else 32
    if K % kc or os.environ.get("KVM_AMD_PACK_WEIGHTS", "1") == "0":
        return None
    entry = _PACKS.get(id(weight))
    if entry is not None and entry["ref"]() is not weight:
        entry = None
    key = (weight.data_ptr(), weight._version)
    if entry is not None and entry["key"] == key and rows in entry:
        return entry[rows]
    if torch.cuda.is_current_stream_capturing():
        return None
    if entry is None:
        wid = id(weight)
        entry = {"ref": weakref.ref(weight), "key": key}
        _PACKS[wid] = entry
        weakref.finalize(weight, _PACKS.pop, wid, None)
    elif entry["key"] != key:
        entry.clear()
        entry.update(ref=weakref.ref(weight), key=key)
    nb = -(-N // rows)
    with torch.no_grad():
        w = torch.zeros(nb * rows, K, device=weight.device, dtype=torch.bfloat16)
        w[:N].copy_(weight)
        if rows == 16:  # [b, i, s, g, e] -> [b, s, g, i, e]
            p = w.view(nb, 16, K // 32, 4, 8).permute(0, 2, 3, 1, 4)
        else:  # [b, j, c, h, g, e] -> [b, c, g, h, j, e]
            p = w.view(nb, 8, K // 64, 2, 4, 8).permute(0, 2, 4, 3, 1, 5)
        entry[rows] = p.contiguous().view(-1)
    return entry[rows]


def _relu_square(h: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    """relu(h)^2 in one HIP launch (kvm_relu_square): bf16 GPU tensors only.
    ``out`` may be ``h`` itself (each element is read before it is written)."""
    if not h.is_cuda or h.dtype != torch.bfloat16 or h.numel() % 8:
        raise ValueError("relu_square runs on bf16 GPU tensors with a multiple of 8 elements")
    h = h.contiguous()
    if out is None or not out.is_contiguous() or out.shape != h.shape or out.dtype != h.dtype:
        out = torch.empty_like(h)
    _lib.check(_lib.load().kvm_relu_square(h.data_ptr(), out.data_ptr(), h.numel(), _lib.stream_handle(h.device)),
               "kvm_relu_square")
    return out


def module_linear(mod: torch.nn.Module, x: torch.Tensor) -> torch.Tensor:
    """``mod(x)``, through :func:`linear` when ``mod`` is an ``nn.Linear``
    (any other module, e.g. an ``nn.Identity`` a test puts in its place, is
    called as it is)."""
    if type(mod) is not torch.nn.Linear:
        return mod(x)
    return linear(x, mod.weight, mod.bias)


__all__ = ["linear", "module_linear"]
