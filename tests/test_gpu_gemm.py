"""kvm_gemm_small (the decode step's linear layers) against an fp32 product.

Y = X W^T with fp32 accumulation and one rounding to bf16: every output is
within one bf16 ulp of the fp32 product of the same bf16 operands, plus the
fp32 summation bound K 2^-24 sum_k |x_k w_k| (two fp32 sums of K terms in
different orders; it dominates only where the result nearly cancels)."""
from __future__ import annotations

import pytest
import torch

import kvm_testlib as T

pytestmark = pytest.mark.gpu
DEV = "cuda"


@pytest.mark.parametrize("M,N,K", [(1, 48, 128), (3, 100, 384), (8, 2048, 64), (8, 6160, 2048), (8, 2048, 2048),
                                   (16, 2048, 8192), (8, 65536, 2048), (5, 300, 1152)])
def test_gemm_small_matches_fp32(M, N, K):
    if not torch.cuda.is_available():
        pytest.skip("needs an MI355X")
    from kvm_amd.linear import linear

    T.log(f"[gemm] M{M} N{N} K{K}")
    gen = torch.Generator(device=DEV).manual_seed(M * 7 + N)
    x = torch.randn(M, K, device=DEV, generator=gen).bfloat16()
    w = (torch.randn(N, K, device=DEV, generator=gen) / K ** 0.5).bfloat16()
    with torch.no_grad():
        got = linear(x, w).float()
    ref = x.float() @ w.float().t()
    ulp = torch.exp2(torch.floor(torch.log2(ref.abs().clamp_min(1e-30))) - 7)
    bound = ulp + K * 2.0 ** -24 * (x.float().abs() @ w.float().abs().t())
    excess = float(((got - ref).abs() / bound).max())
    T.log(f"[gemm] max |err| / (1 ulp + fp32 sum bound) = {excess:.3f}")
    assert excess <= 1.0, f"error {excess:.2f} x the bound"


@pytest.mark.parametrize("M,N,K", [(8, 8192, 2048), (3, 100, 384)])
def test_gemm_small_relu_square_epilogue(M, N, K):
    """epilogue 1 writes relu(y)^2 of the same bf16 product: bit-identical to
    the plain product followed by torch's relu().square() (which
    kvm_relu_square matches bit for bit)."""
    if not torch.cuda.is_available():
        pytest.skip("needs an MI355X")
    from kvm_amd.linear import linear

    T.log(f"[gemm] relu^2 epilogue M{M} N{N} K{K}")
    gen = torch.Generator(device=DEV).manual_seed(N + K)
    x = torch.randn(M, K, device=DEV, generator=gen).bfloat16()
    w = (torch.randn(N, K, device=DEV, generator=gen) / K ** 0.5).bfloat16()
    with torch.no_grad():
        fused = linear(x, w, relu_square=True)
        plain = torch.nn.functional.relu(linear(x, w)).square()
    assert torch.equal(fused, plain)
    assert bool((fused == 0).any()) and bool((fused > 0).any())


@pytest.mark.parametrize("M,N,K", [(8, 2048, 8192), (8, 6224, 2048), (3, 100, 384), (16, 300, 1152), (5, 2048, 64),
                                   (8, 65536, 2048)])
@pytest.mark.parametrize("epilogue", [0, 1])
def test_gemm_small_packed_matches_plain(M, N, K, epilogue):
    """kvm_gemm_small_packed (W re-arranged into per-load chunks) against
    kvm_gemm_small on the same operands: bit-identical (same lanes, same
    MFMA operands, same summation order)."""
    if not torch.cuda.is_available():
        pytest.skip("needs an MI355X")
    from kvm_amd import _lib
    from kvm_amd.linear import _packed

    T.log(f"[gemm] packed M{M} N{N} K{K} epilogue {epilogue}")
    lib = _lib.load()
    gen = torch.Generator(device=DEV).manual_seed(M + N + K)
    x = torch.randn(M, K, device=DEV, generator=gen).bfloat16()
    w = (torch.randn(N, K, device=DEV, generator=gen) / K ** 0.5).bfloat16()
    rows = lib.kvm_gemm_small_tile_rows(M, N)
    assert rows in (8, 16)
    wp = _packed(w, rows)
    if wp is None:
        assert K % (64 if rows == 8 else 32)
        pytest.skip("K does not fit the packed layout of this tile")
    assert wp.numel() == -(-N // rows) * rows * K
    st = _lib.stream_handle(x.device)
    plain = torch.empty(M, N, device=DEV, dtype=torch.bfloat16)
    packed = torch.empty_like(plain)
    _lib.check(lib.kvm_gemm_small(x.data_ptr(), K, w.data_ptr(), K, plain.data_ptr(), N, M, N, K, epilogue, st),
               "kvm_gemm_small")
    _lib.check(lib.kvm_gemm_small_packed(x.data_ptr(), K, wp.data_ptr(), packed.data_ptr(), N, M, N, K, rows,
                                         epilogue, st), "kvm_gemm_small_packed")
    torch.cuda.synchronize()
    assert torch.equal(plain, packed)
    with pytest.raises(ValueError, match="packed for"):
        _lib.check(lib.kvm_gemm_small_packed(x.data_ptr(), K, wp.data_ptr(), packed.data_ptr(), N, M, N, K,
                                             24 - rows, epilogue, st), "kvm_gemm_small_packed")
