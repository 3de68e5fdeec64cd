"""The decoder block's residual add + LayerNorm + MLP token shift kernel
(kvm_add_norm) against the torch ops it replaces (model/rwkv7_backbone.py
Block.forward and the MLP's token shift, model/tokenshift.py).

Bars:
* the residual x + s * y is bit-identical to Block._residual (a power-of-two
  s as one fused add, any other s with the product rounded first);
* the LayerNorm differs from torch's only in the fp32 reduction order, so
  every normalised value is within one bf16 ulp of F.layer_norm's, at least
  99 % of them equal, and within one ulp of the fp64 LayerNorm of the same
  bf16 residual;
* the token shift is bit-identical to the torch ops applied to the kernel's
  own normalised rows (carried row or zeros before token 0), and the carried
  row out is the last token's normalised row, also when written over the
  carried row in place (one token).
Widths cover one, two, four and eight 512-element chunks per lane and widths
that leave lanes idle; sequence lengths cover whole and partial runs of
tokens per wave.
"""
from __future__ import annotations

import pytest
import torch
import torch.nn.functional as F

import kvm_testlib as T

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _ulp(v):
    return torch.exp2(torch.floor(torch.log2(v.abs().clamp_min(2.0 ** -126))) - 7)


class _LN(torch.nn.Module):
    def __init__(self, d, gen):
        super().__init__()
        self.weight = torch.nn.Parameter((1 + 0.3 * torch.randn(d, device=DEV, generator=gen)).bfloat16(),
                                         requires_grad=False)
        self.bias = torch.nn.Parameter((0.1 * torch.randn(d, device=DEV, generator=gen)).bfloat16(),
                                       requires_grad=False)
        self.eps = 1e-5


@pytest.mark.parametrize("B,Tn,d,scale", [(3, 77, 2048, 0.5), (2, 9, 256, 1.0), (3, 1, 2048, 0.5),
                                          (2, 13, 200, 0.7), (1, 6, 4096, 0.25), (4, 5, 1024, 0.3)])
@pytest.mark.parametrize("with_prev", [False, True])
def test_add_norm_matches_torch(B, Tn, d, scale, with_prev):
    if not torch.cuda.is_available():
        pytest.skip("needs an MI355X")
    from kvm_amd.backbone import _add_norm

    T.log(f"[add_norm] B{B} T{Tn} d{d} scale {scale} prev {with_prev}")
    gen = torch.Generator(device=DEV).manual_seed(d + Tn)
    x = (3 * torch.randn(B, Tn, d, device=DEV, generator=gen) + 0.5).bfloat16()
    y = torch.randn(B, Tn, d, device=DEV, generator=gen).bfloat16()
    ln = _LN(d, gen)
    mix = torch.rand(1, 1, d, device=DEV, generator=gen).bfloat16()
    prev = torch.randn(B, 1, d, device=DEV, generator=gen).bfloat16() if with_prev else None
    with torch.no_grad():
        xs, h = _add_norm(x, y, scale, ln)
        xs2, sh = _add_norm(x, y, scale, ln, mix=mix, prev=prev,
                            state_out=torch.empty(B, 1, d, device=DEV, dtype=torch.bfloat16))
        # residual: Block._residual
        if scale > 0 and float(torch.tensor(scale).log2().frac()) == 0.0:
            ref_x = torch.add(x, y, alpha=scale)
        else:
            ref_x = x + y * scale
        assert torch.equal(xs, ref_x) and torch.equal(xs2, ref_x)
        # LayerNorm against torch and fp64
        ref_h = F.layer_norm(ref_x, (d,), ln.weight, ln.bias, ln.eps)
        diff = (h.float() - ref_h.float()).abs()
        assert float((diff / _ulp(ref_h.float())).max()) <= 1.0
        frac_eq = float((diff == 0).float().mean())
        r64 = ref_x.double()
        mu = r64.mean(-1, keepdim=True)
        var = ((r64 - mu) ** 2).mean(-1, keepdim=True)
        exact = (r64 - mu) / torch.sqrt(var + ln.eps) * ln.weight.double() + ln.bias.double()
        err64 = float(((h.double() - exact).abs() / _ulp(exact.float()).double()).max())
        T.log(f"[add_norm] equal to torch LN: {frac_eq:.5f}, max err vs fp64 {err64:.3f} ulp")
        assert frac_eq >= 0.99
        assert err64 <= 1.0
        # token shift of the kernel's own LN rows
        before = prev if prev is not None else torch.zeros(B, 1, d, device=DEV, dtype=torch.bfloat16)
        shifted = torch.cat([before, h[:, :-1]], dim=1)
        ref_sh = h + mix * (shifted - h)
    assert torch.equal(sh, ref_sh)


def test_add_norm_in_place_carried_row():
    """One token with state_out = prev: the carried row is read before it is
    overwritten with the new last row."""
    if not torch.cuda.is_available():
        pytest.skip("needs an MI355X")
    from kvm_amd.backbone import _add_norm

    B, d = 8, 2048
    gen = torch.Generator(device=DEV).manual_seed(5)
    x = torch.randn(B, 1, d, device=DEV, generator=gen).bfloat16()
    y = torch.randn(B, 1, d, device=DEV, generator=gen).bfloat16()
    ln = _LN(d, gen)
    mix = torch.rand(1, 1, d, device=DEV, generator=gen).bfloat16()
    prev = torch.randn(B, 1, d, device=DEV, generator=gen).bfloat16()
    prev0 = prev.clone()
    with torch.no_grad():
        _, h = _add_norm(x, y, 0.5, ln)
        _, sh = _add_norm(x, y, 0.5, ln, mix=mix, prev=prev, state_out=prev)
    assert torch.equal(sh, h + mix * (prev0 - h))
    assert torch.equal(prev, h)


def test_add_norm_rejects_bad_arguments():
    if not torch.cuda.is_available():
        pytest.skip("needs an MI355X")
    from kvm_amd.backbone import _add_norm

    gen = torch.Generator(device=DEV).manual_seed(1)
    ln = _LN(64, gen)
    x = torch.randn(2, 3, 64, device=DEV, generator=gen).bfloat16()
    prev = torch.zeros(2, 1, 64, device=DEV, dtype=torch.bfloat16)
    mix = torch.rand(64, device=DEV, generator=gen).bfloat16()
    with pytest.raises(ValueError, match="alias prev only when seq_len == 1"):
        _add_norm(x, x, 1.0, ln, mix=mix, prev=prev, state_out=prev)
    ln_wide = _LN(8192, gen)
    with pytest.raises(ValueError, match="width a multiple of 8"):
        _add_norm(torch.zeros(1, 1, 8192, device=DEV, dtype=torch.bfloat16), None, 1.0, ln_wide)
