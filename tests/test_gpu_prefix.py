"""GPU parity of the fused pre-boundary kernel (kvm_prefix) against the
mixer's torch op sequence, which is the reference's
(model/value_residual_mixin.py:173-237, model/kvm_mixer.py:367-401).

Both run on the same GPU from the same projections.  Every reference op
rounds to bf16 and the kernel keeps those rounding points; the fp32 results
of the sigmoid / elu / LayerNorm reductions may differ in their last bit, so
a LayerNorm output may differ by one bf16 ulp, and RoPE (a sum of two
rounded products, which may cancel) carries that into at most two ulps of
the larger of |value| and 1.  Bar: at least 99% of the elements of every
output equal, every difference at most 2^-6 * max(|value|, 1), cache entries
equal.  Covered: every value-residual mode, token shift on /
off, head_dim 64 / 128, GQA, merge gate on / off, a prefill followed by two
cached single-token steps (previous-token rows from the cache).
"""
from __future__ import annotations

import pytest
import torch

import kvm_testlib as T

pytestmark = pytest.mark.gpu
DEV = "cuda"


@pytest.fixture(scope="module")
def lib():
    if not torch.cuda.is_available():
        pytest.skip("needs an MI355X")
    from kvm_amd import _lib

    return _lib.load()


def _compare(a, b, what):
    a, b = a.float(), b.float()
    assert a.shape == b.shape, what
    diff = (a - b).abs()
    unit = torch.maximum(torch.maximum(a.abs(), b.abs()), torch.ones_like(a)) * 2.0 ** -7
    eq = float((diff == 0).float().mean())
    worst = float((diff / unit).max())
    T.log(f"[prefix] {what}: equal {eq * 100:.3f}%, worst {worst:.2f} units of 2^-7 max(|x|, 1)")
    assert eq >= 0.99 and worst <= 2.0 + 1e-6, f"{what}: equal {eq:.4f}, worst {worst:.2f}"


CASES = [
    # mode, token shift, D, Hq, Hkv, T, merge gate
    ("rwkv", 1, 128, 4, 4, 300, 1),
    ("rwkv", 0, 128, 8, 2, 257, 1),
    ("linear", 1, 64, 4, 2, 130, 1),
    ("none", 1, 64, 2, 2, 99, 0),
    ("rwkv_post_tokenshift", 1, 128, 4, 2, 200, 1),
]


@pytest.mark.parametrize("mode,shift,D,Hq,Hkv,Tn,gate", CASES)
def test_fused_prefix_matches_torch_ops(lib, mode, shift, D, Hq, Hkv, Tn, gate):
    from kvm_amd.backbone import RotaryEmbedding, StatesDictCache, init_random_
    from kvm_amd.mixer import SequenceMixer

    T.log(f"[prefix] mode={mode} shift={shift} D={D} Hq={Hq} Hkv={Hkv} T={Tn} gate={gate}")
    cfg = T.mixer_config(Hq, Hkv, D, 64, gate_keys=gate, gate_values=gate)
    cfg.use_value_residual = int(mode != "none")
    cfg.kvm_value_residual_mode = mode if mode != "none" else "rwkv"
    cfg.use_tokenshift_att = shift
    cfg.hidden_size = 3 * 64
    cfg.num_hidden_layers = 4
    m = SequenceMixer(cfg, 1)
    init_random_(m, seed=7)
    m = m.to(DEV, torch.bfloat16).eval()
    B = 2
    gen = torch.Generator(device=DEV).manual_seed(3)
    x = torch.randn(B, Tn + 2, cfg.hidden_size, device=DEV, generator=gen).bfloat16()
    v_first = torch.randn(B, Tn + 2, Hkv * D, device=DEV, generator=gen).bfloat16()
    rot = RotaryEmbedding(D, 32)
    pos = torch.arange(Tn + 2, device=DEV).unsqueeze(0)
    cos, sin = rot(pos)
    caches = (StatesDictCache(), StatesDictCache())
    # separate projection GEMMs here, as in the torch sequence: the comparison
    # isolates the elementwise kernel; the concatenated GEMM is checked below
    m._CONCAT_PROJ = False
    with torch.no_grad():
        steps = [(0, Tn)] + [(Tn + i, Tn + i + 1) for i in range(2)]
        for a, b in steps:
            pe = (cos[:, a:b], sin[:, a:b])
            args = (x[:, a:b], v_first[:, a:b], pe)
            fused = m._fused_prefix(*args, caches[0])
            ref = m._torch_prefix(*args, caches[1])
            for c in caches:
                c.update(1, offset=b - a)
            for name, f, r in zip(("q", "k", "v", "gate"), fused, ref):
                _compare(f.to(r.dtype) if name == "gate" else f, r, f"tokens [{a},{b}) {name}")
            st0, st1 = caches[0].get_states(1), caches[1].get_states(1)
            for key in st1:
                assert torch.equal(st0[key], st1[key]), f"cache entry {key} after tokens [{a},{b})"


def test_concatenated_projection_matches_separate_gemms(lib):
    """The fused path's single concatenated projection GEMM against separate
    GEMMs: the same products, rounded by different GEMM kernels, so outputs
    agree to within bf16 rounding of the projections."""
    from kvm_amd.backbone import RotaryEmbedding, init_random_
    from kvm_amd.mixer import SequenceMixer

    Hq, Hkv, D, Tn = 8, 2, 128, 200
    cfg = T.mixer_config(Hq, Hkv, D, 64)
    cfg.use_value_residual, cfg.use_tokenshift_att, cfg.hidden_size, cfg.num_hidden_layers = 1, 1, 256, 4
    m = SequenceMixer(cfg, 1)
    init_random_(m, seed=9)
    m = m.to(DEV, torch.bfloat16).eval()
    gen = torch.Generator(device=DEV).manual_seed(4)
    x = torch.randn(2, Tn, 256, device=DEV, generator=gen).bfloat16()
    v_first = torch.randn(2, Tn, Hkv * D, device=DEV, generator=gen).bfloat16()
    pe = RotaryEmbedding(D, 32)(torch.arange(Tn, device=DEV).unsqueeze(0))
    with torch.no_grad():
        m._CONCAT_PROJ = True
        a = m._fused_prefix(x, v_first, pe, None)
        m._CONCAT_PROJ = False
        b = m._fused_prefix(x, v_first, pe, None)
    for name, u, w in zip(("q", "k", "v", "gate"), a, b):
        mx, mean = T.err_stats(u, w)
        T.log(f"[prefix] concatenated vs separate projections, {name}: max {mx:.2e} mean {mean:.2e}")
        assert mx <= 0.1 and mean <= 2e-3, (name, mx, mean)


@pytest.mark.parametrize("with_prev", [False, True])
def test_mlp_kernels_match_torch_ops(lib, with_prev):
    """The decoder MLP's token shift (fallback "zero", or a carried previous
    token) and relu^2 kernels against the torch ops on the same GPU: bit-exact
    (elementwise, same bf16 rounding points)."""
    from kvm_amd.backbone import _kernel_token_shift, token_shift_delta
    from kvm_amd.linear import _relu_square

    gen = torch.Generator(device=DEV).manual_seed(8)
    B, Tn, d = 3, 77, 256
    x = torch.randn(B, Tn, d, device=DEV, generator=gen).bfloat16()
    mix = torch.rand(1, 1, d, device=DEV, generator=gen).bfloat16()
    prev = torch.randn(B, 1, d, device=DEV, generator=gen).bfloat16() if with_prev else None
    with torch.no_grad():
        got = _kernel_token_shift(x, prev, mix)
        ref = x + mix * token_shift_delta(x, prev, fallback="zero")
        assert torch.equal(got, ref), float((got.float() - ref.float()).abs().max())
        h = torch.randn(B, Tn, 4 * d, device=DEV, generator=gen).bfloat16()
        assert torch.equal(_relu_square(h), torch.nn.functional.relu(h).square())
        # in place (out is the input): the same values
        h2 = h.clone()
        assert torch.equal(_relu_square(h2, out=h2), torch.nn.functional.relu(h).square())


def test_mlp_row_chunks_match_whole_input(lib):
    """MLP.ffn runs inputs of more than _FFN_CHUNK rows in row chunks (each
    chunk's hidden activations stay in the last-level cache); rows are
    independent, so the chunked result is compared with the same ops on the
    whole input, here with a ragged last chunk."""
    from kvm_amd.backbone import MLP
    from kvm_amd.linear import linear
    from types import SimpleNamespace

    gen = torch.Generator(device=DEV).manual_seed(9)
    d = 256
    cfg = SimpleNamespace(ffn_expansion=4.0, hidden_size=d, use_tokenshift_ffn=0, num_hidden_layers=2)
    mlp = MLP(cfg, 0).to(DEV, torch.bfloat16).eval()
    with torch.no_grad():
        mlp.c_proj.weight.copy_((torch.randn(d, 4 * d, device=DEV, generator=gen) / 32).bfloat16())
        rows = 2 * MLP._FFN_CHUNK + 1234
        x = torch.randn(1, rows, d, device=DEV, generator=gen).bfloat16()
        got = mlp.ffn(x)
        ref = torch.nn.functional.linear(linear(x, mlp.c_fc.weight, relu_square=True), mlp.c_proj.weight)
    assert got.shape == ref.shape
    diff = (got.float() - ref.float()).abs()
    eq = float((diff == 0).float().mean())
    T.log(f"[mlp-chunks] rows {rows}: equal {eq * 100:.3f}%, max |diff| {float(diff.max()):.3e}")
    # The same GEMMs per row; only a different kernel choice for the chunk
    # shape could reorder the K sums (one bf16 rounding of the output).
    assert torch.allclose(got.float(), ref.float(), rtol=2 ** -7, atol=1e-3)
    assert eq >= 0.99
