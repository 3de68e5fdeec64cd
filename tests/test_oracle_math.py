"""Pin the CPU oracle where the reference's golden fixtures leave it open:
textbook formulas in fp64, brute force on small inputs, invariants, and the
append tie order of the reference."""

from __future__ import annotations

import math

import pytest
import torch
import torch.nn.functional as F

import golden_io
from oracle import kvm_oracle as O


def _params(D, Hq, seed=0):
    g = torch.Generator().manual_seed(seed)
    return O.OracleParams(
        ln_weight=(1 + 0.1 * torch.randn(D, generator=g)).bfloat16(),
        ln_bias=(0.1 * torch.randn(D, generator=g)).bfloat16(),
        front_temp=(1 + 0.1 * torch.randn(Hq, generator=g)).bfloat16(),
        state_temp=(1 + 0.1 * torch.randn(Hq, generator=g)).bfloat16(),
    )


# Hand-computed state budgets (model/kvm_mixer.py:131-165): budget, ctx_len,
# available, current -> state length.  Saturation values are
# floor(N t / (N + t)) worked out by hand: 1024*1024/2048 = 512 exactly;
# 1024*3072/4096 = 768 exactly; 1024*1023/2047 = 511.75 -> 511 (a formula
# that rounds instead of flooring gives 512); 300*192/492 = 117.07 -> 117;
# 500*1000/1500 = 333.3 -> 333, rounded down to 16 -> 320; 1024*1e6/(1e6+1024)
# = 1022.95 -> 1022.  Power law: floor(16 * sqrt(4096)) = 1024; floor(5 *
# sqrt(1000)) = floor(158.11) = 158; floor(1 * sqrt(65535)) = 255 (sqrt is
# 255.998).
BUDGET_TABLE = [
    # (mode, factor, exponent, round_down, min_len, saturation_n, max_state_len)
    (("kvm_saturation", 1.0, 0.5, 1, 1, 1024, 10**6), 1024, 10**6, 0, 512),
    (("kvm_saturation", 1.0, 0.5, 1, 1, 1024, 10**6), 3072, 10**6, 0, 768),
    (("kvm_saturation", 1.0, 0.5, 1, 1, 1024, 10**6), 1023, 10**6, 0, 511),
    (("kvm_saturation", 1.0, 0.5, 1, 1, 1024, 10**6), 1, 10**6, 0, 1),          # floor 0, raised to min_len 1
    (("kvm_saturation", 1.0, 0.5, 1, 1, 300, 640), 192, 128, 64, 117),
    (("kvm_saturation", 1.0, 0.5, 1, 1, 300, 640), 192, 100, 64, 100),         # capped by the available context
    (("kvm_saturation", 1.0, 0.5, 1, 1, 300, 640), 192, 1000, 130, 130),       # never below the current length
    (("kvm_saturation", 1.0, 0.5, 16, 1, 500, 512), 1000, 10**6, 0, 320),
    (("kvm_saturation", 1.0, 0.5, 16, 1, 500, 256), 1000, 10**6, 0, 256),      # capped by max_state_len
    (("kvm_saturation", 1.0, 0.5, 1, 1, 1024, 10**7), 10**6, 10**7, 0, 1022),
    (("power_law", 16.0, 0.5, 1, -1, None, 1024), 4096, 10**6, 0, 1024),
    (("power_law", 5.0, 0.5, 1, 64, None, 192), 1000, 10**6, 0, 158),
    (("power_law", 5.0, 0.5, 32, 64, None, 192), 1000, 10**6, 0, 128),
    (("power_law", 1.0, 0.5, 1, -1, None, 1024), 65535, 10**6, 0, 255),
    (("power_law", 1.0, 0.5, 1, 300, None, 1024), 65535, 10**6, 0, 300),       # min_len floor
    (("fixed", 1.0, 0.5, 1, 256, None, 512), 32768, 10**6, 512, 512),          # current 512 > floor 256
    (("fixed", 1.0, 0.5, 1, 64, None, 256), 4096, 10**6, 0, 64),
]


@pytest.mark.parametrize("budget,ctx,avail,cur,want", BUDGET_TABLE)
def test_state_budget_closed_forms(budget, ctx, avail, cur, want):
    from kvm_amd.schedule import StateBudget

    mode, f, e, rd, mn, sat, mx = budget
    assert StateBudget(mode, f, e, rd, mn, sat, mx).desired(ctx, avail, cur) == want
    C = 64
    cfg = O.OracleConfig(q_heads=1, kv_heads=1, head_dim=64, value_dim=64, chunk_len=C, n_max_d_chunks=1,
                         state_budget_mode=mode, state_growth_factor=f, state_growth_exponent=e,
                         state_round_down=rd, state_min_len=mn, state_saturation_n=sat)
    cfg_max = type(cfg).max_state_len
    try:
        type(cfg).max_state_len = property(lambda self: mx)
        assert O.desired_state_len(cfg, ctx, avail, cur) == want
    finally:
        type(cfg).max_state_len = cfg_max


def test_saturation_budget_properties():
    """floor(N t / (N + t)) rises with t, stays below N and below t, and
    reaches N - 1 only for t > N (N - 1) (brute force over t)."""
    from kvm_amd.schedule import StateBudget

    N = 97
    b = StateBudget("kvm_saturation", 1.0, 0.5, 1, 0, N, 10**9)
    prev = 0
    for t in range(0, 20000):
        s = b.desired(t, 10**9, 0)
        assert prev <= s < N and s <= t
        assert (s == N - 1) == (N * t >= (N - 1) * (N + t))
        prev = s


def test_prep_k_is_layernorm_of_rope_zeroed_key():
    D, r = 64, 24
    p = _params(D, 1)
    k = torch.randn(3, 2, 17, D).bfloat16()
    got = O.prep_k(k, p, r).double()
    z = k.double().clone()
    z[..., :r] = 0
    mu = z.mean(-1, keepdim=True)
    var = ((z - mu) ** 2).mean(-1, keepdim=True)
    ref = (z - mu) / torch.sqrt(var + 1e-5) * p.ln_weight.double() + p.ln_bias.double()
    # one bf16 rounding of the fp32 result
    assert (got - ref).abs().max() <= 2 ** -7 * ref.abs().max()
    # rope-zeroed dims do not influence the result
    k2 = k.clone()
    k2[..., :r] = torch.randn(3, 2, 17, r).bfloat16()
    assert torch.equal(O.prep_k(k2, p, r), O.prep_k(k, p, r))


def test_attend_matches_fp64_softmax():
    B, Hq, Hkv, D, S, W, L = 1, 4, 2, 64, 13, 40, 9
    cfg = O.OracleConfig(q_heads=Hq, kv_heads=Hkv, head_dim=D, value_dim=D)
    p = _params(D, Hq, 1)
    g = torch.Generator().manual_seed(2)
    q = torch.randn(B, Hq, L, D, generator=g).bfloat16()
    bk = torch.randn(B, Hkv, W, D, generator=g).bfloat16()
    bv = torch.randn(B, Hkv, W, D, generator=g).bfloat16()
    s_k = torch.randn(B, Hkv, S, D, generator=g).bfloat16()
    s_v = torch.randn(B, Hkv, S, D, generator=g).bfloat16()
    s_vlen = torch.rand(B, Hkv, S, 1, generator=g) + 0.5
    got = O.attend(q, bk, bv, s_k, s_v, s_vlen, p, cfg)
    grp = Hq // Hkv
    ln = F.layer_norm(s_k.double(), (D,), p.ln_weight.double(), p.ln_bias.double(), 1e-5)
    keys = torch.cat([ln.repeat_interleave(grp, 1) * p.state_temp.double().view(1, Hq, 1, 1),
                      bk.double().repeat_interleave(grp, 1) * p.front_temp.double().view(1, Hq, 1, 1)], 2)
    vals = torch.cat([(s_v.double() / s_v.double().norm(dim=-1, keepdim=True) * s_vlen.double()).repeat_interleave(grp, 1),
                      bv.double().repeat_interleave(grp, 1)], 2)
    # lower-right causal: window key j visible to query i iff j <= i + (W - L)
    vis = torch.ones(L, S + W, dtype=torch.bool)
    vis[:, S:] = torch.arange(W).view(1, -1) <= torch.arange(L).view(-1, 1) + (W - L)
    ref = O.brute_force_attention(q, keys, vals, vis)
    assert (got.double() - ref).abs().max() < 3e-2
    assert (got.double() - ref).abs().mean() < 3e-3


def test_route_merge_is_first_argmax_over_non_sink_slots():
    g = torch.Generator().manual_seed(4)
    km = torch.randn(2, 3, 50, 32, generator=g).bfloat16()
    sk = torch.randn(2, 3, 20, 32, generator=g).bfloat16()
    for protected in (0, 1, 3):
        got = O.route_merge(km, sk, protected, fp32_routing=True).squeeze(-1)
        ex = O.exact_logits(km, sk)
        ex[..., :protected] = float("-inf")
        top2 = ex.topk(2, dim=-1).values
        bound = O.fp32_dot_error_bound(km, sk).max(-1).values
        clear = (top2[..., 0] - top2[..., 1]) > 2 * bound
        assert clear.float().mean() > 0.95
        assert torch.equal(got[clear], ex.argmax(-1)[clear])
        assert bool((got >= protected).all())
    # exact ties resolve to the first index
    km = torch.ones(1, 1, 1, 4).bfloat16()
    sk = torch.ones(1, 1, 5, 4).bfloat16()
    assert int(O.route_merge(km, sk, 2, True)) == 2


def test_split_append_merge_brute_force():
    g = torch.Generator().manual_seed(5)
    kb = torch.randn(1, 2, 30, 16, generator=g).bfloat16()
    kr = torch.randn(1, 2, 7, 16, generator=g).bfloat16()
    app, mrg = O.split_append_merge(kb, 6, kr, stable=True)
    scores = torch.matmul(kb, kr.transpose(-1, -2)).float().max(-1).values
    for h in range(2):
        order = sorted(range(30), key=lambda t: (float(scores[0, h, t]), t))
        assert app[0, h].tolist() == sorted(order[:6])
        assert mrg[0, h].tolist() == sorted(order[6:])


def test_fixed_state_invariants():
    """Sink slots never change; the state length follows the schedule; vlen is
    the norm of the slot's first value (vlens=1, model/kvm_mixer.py:337-338)."""
    B, H, D, C, T = 1, 2, 64, 32, 300
    cfg = O.OracleConfig(q_heads=H, kv_heads=H, head_dim=D, value_dim=D, chunk_len=C, sink_len=2,
                         rope_partial_dim=16, state_min_len=C)
    p = _params(D, H, 3)
    g = torch.Generator().manual_seed(6)
    q, k, v = (torch.randn(B, H, T, D, generator=g).bfloat16() for _ in range(3))
    gate = (1 + F.elu(torch.randn(B, H, T, 1, generator=g))).bfloat16()
    rec = O.Recorder()
    _, st = O.prefill(q, k, v, gate, p, cfg, rec)
    s0_k = O.prep_k(k[:, :, :C], p, cfg.rope_partial_dim)
    assert torch.equal(st[O.S_K][:, :, :2], s0_k[:, :, :2])
    assert torch.equal(st[O.S_V][:, :, :2], v[:, :, :2])
    assert torch.allclose(st[O.S_VLEN], v[:, :, :C].float().norm(dim=-1, keepdim=True))
    for u in rec.updates:
        assert bool((u.route >= 2).all())
    sched = O.prefill_schedule(cfg, T)
    assert st[O.S_K].size(2) == sched["final_state_len"] == C


def test_decode_continues_prefill():
    """Decoding token T after a prefill of T tokens equals position T of a
    prefill of T + 1 tokens (same state, same window)."""
    B, H, D, C = 1, 2, 64, 32
    cfg = O.OracleConfig(q_heads=H, kv_heads=H, head_dim=D, value_dim=D, chunk_len=C, rope_partial_dim=16,
                         state_min_len=C)
    p = _params(D, H, 7)
    g = torch.Generator().manual_seed(8)
    for T in (100, 127, 130):
        q, k, v = (torch.randn(B, H, T + 1, D, generator=g).bfloat16() for _ in range(3))
        gate = (1 + F.elu(torch.randn(B, H, T + 1, 1, generator=g))).bfloat16()
        y_full, _ = O.prefill(q, k, v, gate, p, cfg)
        _, st = O.prefill(q[:, :, :T], k[:, :, :T], v[:, :, :T], gate[:, :, :T], p, cfg)
        yd, _ = O.decode_step(st, T, q[:, :, T:], k[:, :, T:], v[:, :, T:], gate[:, :, T:], p, cfg)
        assert (yd.float() - y_full[:, :, T:].float()).abs().max() < 2e-2


def test_reference_append_ties_differ_only_at_the_cut():
    """The reference ranks bf16 novelty scores with an unstable argsort; its
    choice among equal scores at the cut is the only place where it departs
    from the lower-index rule of the HIP kernels."""
    fx = golden_io.load("growable_bf16")
    cfg, p = golden_io.oracle_setup(fx)
    m = fx["meta"]
    T, C = m["T"], m["C"]
    q, k, v, g = (fx["in_" + x][:, :, :T] for x in ("q", "k", "v", "gate"))
    rec = O.Recorder(keep_states=True)
    O.prefill(q, k, v, g, p, cfg, rec)
    sched = O.prefill_schedule(cfg, T)["updates"]
    n_tie_cases = 0
    for i, u in enumerate(rec.updates):
        if u.n_append == 0:
            continue
        tb = sched[i][0] * C
        pk = O.prep_k(k[:, :, tb:tb + C], p, cfg.rope_partial_dim)
        app_ref, _ = O.split_append_merge(pk, u.n_append, O._ln(u.s_k_before, p), stable=False)
        app_low, _ = O.split_append_merge(pk, u.n_append, O._ln(u.s_k_before, p), stable=True)
        assert torch.equal(app_ref, u.append_idx)  # the oracle reproduces the reference
        nov = torch.matmul(pk, O._ln(u.s_k_before, p).transpose(-1, -2)).float().max(-1).values
        for b in range(m["B"]):
            for h in range(m["Hkv"]):
                a, l = set(app_ref[b, h].tolist()), set(app_low[b, h].tolist())
                if a != l:
                    n_tie_cases += 1
                    cut = torch.sort(nov[b, h]).values[u.n_append - 1]
                    for t in a ^ l:
                        assert nov[b, h, t] == cut
    assert n_tie_cases > 0  # the fixture does exercise the tie rule
