"""The allocation-free decode entry point against the workspace one.

kvm_decode_attention_noalloc runs the same kernels as kvm_decode_attention
with the split-K partials in the library's own device scratch, so its output
must be bit-identical.  Two calls in a row, the second over fewer key rows
(and a smaller batch), so stale scratch contents of the first call cannot
leak into the second; then a call that needs more scratch than the library
holds must be refused with KVM_ESPACE.
"""

from __future__ import annotations

import math

import pytest
import torch

import kvm_testlib as T

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _case(lib, B, Hq, Hkv, D, S, W, R, start, seed):
    from kvm_amd import _lib

    rows = B * Hkv
    gen = torch.Generator(device=DEV).manual_seed(seed)
    ka = (0.5 * torch.randn(rows, S, D, device=DEV, generator=gen)).bfloat16()
    va = (0.5 * torch.randn(rows, S, D, device=DEV, generator=gen)).bfloat16()
    rk = torch.randn(rows, W, D, device=DEV, generator=gen).bfloat16()
    rv = torch.randn(rows, W, D, device=DEV, generator=gen).bfloat16()
    q = (torch.randn(B, Hq, 1, D, device=DEV, generator=gen) / math.sqrt(D)).bfloat16()
    cfg = T.mixer_config(Hq, Hkv, D, 64)
    m = T.make_mixer(cfg, torch.ones(D), torch.zeros(D), torch.ones(Hq), torch.ones(Hq))
    layer = m._layer_struct(B, torch.device(DEV))
    vlen = torch.ones(rows, S, device=DEV)
    st = _lib.state_struct(ka, va, vlen, ka, va, S)
    nws = int(lib.kvm_decode_workspace_bytes(layer.ref(), S + R))
    ws = torch.empty(nws, dtype=torch.uint8, device=DEV)
    ref = torch.empty(B, Hq, D, dtype=torch.bfloat16, device=DEV)
    got = torch.full_like(ref, float("nan"))
    common = (q.data_ptr(), q.stride(0), q.stride(1), st, S, rk.data_ptr(), rv.data_ptr(), W, start, R)
    _lib.check(lib.kvm_decode_attention(layer.ref(), *common, ref.data_ptr(), ref.stride(0), ref.stride(1),
                                        ws.data_ptr(), nws, 0), "kvm_decode_attention")
    _lib.check(lib.kvm_decode_attention_noalloc(layer.ref(), *common, got.data_ptr(), got.stride(0),
                                                got.stride(1), 0), "kvm_decode_attention_noalloc")
    torch.cuda.synchronize()
    return ref, got, nws


def test_noalloc_decode_matches_workspace_entry_point():
    if not torch.cuda.is_available():
        pytest.skip("needs an MI355X")
    from kvm_amd import _lib

    lib = _lib.load()
    # First call: config 4's shape (64 x 32 heads, 1024 slots + 385 window rows).
    T.log("[noalloc] call 1: B64 Hq32 Hkv32 D128 S1024 ring 1024 recent 385")
    ref, got, n1 = _case(lib, 64, 32, 32, 128, 1024, 1024, 385, 800, 5)
    assert n1 <= _lib.KVM_DECODE_SCRATCH_BYTES
    assert torch.equal(ref, got), "call 1: allocation-free output differs"
    # Second call: smaller batch, GQA, fewer rows; its partials cover a prefix of
    # what the first call left in the scratch.
    T.log("[noalloc] call 2: B3 Hq8 Hkv2 D64 S100 ring 128 recent 90")
    ref, got, n2 = _case(lib, 3, 8, 2, 64, 100, 128, 90, 60, 6)
    assert n2 < n1
    assert torch.equal(ref, got), "call 2: allocation-free output differs"
    T.log(f"[noalloc] outputs bit-identical to kvm_decode_attention (scratch {n1} then {n2} bytes)")


def test_noalloc_decode_rejects_oversized_calls():
    if not torch.cuda.is_available():
        pytest.skip("needs an MI355X")
    from kvm_amd import _lib

    lib = _lib.load()
    B, Hq, Hkv, D, S = 64, 64, 64, 128, 4096
    cfg = T.mixer_config(Hq, Hkv, D, 64)
    m = T.make_mixer(cfg, torch.ones(D), torch.zeros(D), torch.ones(Hq), torch.ones(Hq))
    layer = m._layer_struct(B, torch.device(DEV))
    assert int(lib.kvm_decode_workspace_bytes(layer.ref(), S + 512)) > _lib.KVM_DECODE_SCRATCH_BYTES
    dummy = torch.zeros(16, dtype=torch.bfloat16, device=DEV)
    st = _lib.state_struct(dummy, dummy, dummy, dummy, dummy, S)
    rc = lib.kvm_decode_attention_noalloc(layer.ref(), dummy.data_ptr(), 0, 0, st, S, dummy.data_ptr(),
                                          dummy.data_ptr(), 512, 0, 512, dummy.data_ptr(), 0, 0, 0)
    assert rc == _lib.KVM_ESPACE
    assert "scratch" in lib.kvm_last_error().decode()
