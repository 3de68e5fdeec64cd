"""GPU backward of the prefill against fp32 torch autograd of the same
fixed-route forward.

The HIP path (``kvm_amd.training.KVMPrefillFunction``): the forward on the
HIP library, the attention backward in HIP kernels, the memory-state chain
rule replayed under the forward's routes.  The reference here is an
independent fp32 restatement of the forward (model/kvm_mixer.py:403-516,
merge sums as one-hot products, :321-340) with the routes the HIP forward
chose, differentiated by torch autograd; the argmax and the append ranking
are fixed metadata, as in the reference's training function
(model/kvm_triton_mixer.py:24-195).

Bar (bf16 forward and bf16 MFMA operands in the backward): for every
gradient, max |err| <= 5e-2 * max |ref| and mean |err| <= 2e-2 * mean |ref|.
"""

from __future__ import annotations

import math

import pytest
import torch
import torch.nn.functional as F

import kvm_testlib as T
from snapshot_replay import replay_snapshot_rows

pytestmark = pytest.mark.gpu
DEV = "cuda"


def fixed_route_forward(q, k, v, g, lnw, lnb, ts, tf, plan, route_log, append_log, cfg, n_bswa):
    """fp32 KVM prefill output [B, Hq, T, D] with the given routes."""
    B, Hq, Tn, D = q.shape
    Hkv = k.size(1)
    grp = Hq // Hkv
    C = plan.chunk_len
    r = cfg["rope"]
    kz = torch.cat([torch.zeros_like(k[..., :r]), k[..., r:]], dim=-1)
    prep = F.layer_norm(kz, (D,), lnw, lnb, 1e-5)
    gk = prep * g if cfg["gate_keys"] else prep
    gv = v * g if cfg["gate_values"] else v
    ak, av = (gk, gv) if cfg["gate_appends"] else (prep, v)
    L0 = plan.initial_state_len
    s_k = (prep * g if cfg["gate_initial"] else prep)[:, :, :L0]
    s_v = (v * g if cfg["gate_initial"] else v)[:, :, :L0]
    vlen = v[:, :, :L0].norm(dim=-1, keepdim=True)
    snaps = [(s_k, s_v, vlen)]
    for u in range(plan.n_updates):
        tb, before, n_app = plan.upd_token_begin[u], plan.upd_state_before[u], plan.upd_n_append[u]
        route = route_log[u].view(B, Hkv, C).long()
        app = append_log[u].view(B, Hkv, C).bool()
        if n_app:
            new_k, new_v = [], []
            for b in range(B):
                for h in range(Hkv):
                    idx = app[b, h].nonzero().flatten() + tb
                    new_k.append(ak[b, h, idx])
                    new_v.append(av[b, h, idx])
            nk = torch.stack(new_k).view(B, Hkv, n_app, D)
            nv = torch.stack(new_v).view(B, Hkv, n_app, D)
            s_k = torch.cat([s_k, nk], dim=2)
            s_v = torch.cat([s_v, nv], dim=2)
            vlen = torch.cat([vlen, nv.norm(dim=-1, keepdim=True)], dim=2)
        S = before + n_app
        onehot = F.one_hot(route.clamp_min(0), S).to(q.dtype) * (~app).unsqueeze(-1).to(q.dtype)
        s_k = s_k + onehot.transpose(-1, -2) @ gk[:, :, tb:tb + C]
        s_v = s_v + onehot.transpose(-1, -2) @ gv[:, :, tb:tb + C]
        snaps.append((s_k, s_v, vlen))
    outs = []
    rep = lambda x: x.repeat_interleave(grp, dim=1)  # noqa: E731
    for m in range(plan.n_chunks):
        qb, qe = m * C, min(Tn, (m + 1) * C)
        wb = max(0, (m - n_bswa + 1) * C)
        kw, vw = rep(k[:, :, wb:qe]) * tf.view(1, Hq, 1, 1), rep(v[:, :, wb:qe])
        qi = torch.arange(qb, qe, device=q.device).view(-1, 1)
        kj = torch.arange(wb, qe, device=q.device).view(1, -1)
        vis = kj <= qi
        if m >= n_bswa:
            sk, sv, sl = snaps[plan.chunk_snapshot[m]]
            Sm = plan.chunk_state_len[m]
            ka = rep(F.layer_norm(sk[:, :, :Sm], (D,), lnw, lnb, 1e-5)) * ts.view(1, Hq, 1, 1)
            va = rep(F.normalize(sv[:, :, :Sm], dim=-1) * sl[:, :, :Sm])
            kw, vw = torch.cat([ka, kw], dim=2), torch.cat([va, vw], dim=2)
            vis = torch.cat([torch.ones(qe - qb, Sm, dtype=torch.bool, device=q.device), vis], dim=1)
        s = (q[:, :, qb:qe] @ kw.transpose(-1, -2)) / math.sqrt(D)
        s = s.masked_fill(~vis, float("-inf"))
        outs.append(torch.softmax(s, dim=-1) @ vw)
    return torch.cat(outs, dim=2)


def test_mixer_forward_trains_through_the_hip_prefill():
    """SequenceMixer.forward (projections -> post-QKV prefill -> c_proj) with
    gradients on: the mixer routes the prefill through the differentiable HIP
    path, and a training step's gradients reach every parameter."""
    if not torch.cuda.is_available():
        pytest.skip("needs an MI355X")
    from kvm_amd import SequenceMixer

    Hq, Hkv, D, C, Tn = 4, 2, 64, 64, 260
    cfg = T.mixer_config(Hq, Hkv, D, C, rope=16, mode="power_law", min_len=C, n_max=4, factor=8.0)
    torch.manual_seed(3)
    m = SequenceMixer(cfg, 0).to(DEV, torch.bfloat16).train()
    with torch.no_grad():  # the output projection starts at zero, which would stop every gradient upstream
        m.c_proj.weight.normal_(0.0, 0.02)
    x = (torch.randn(2, Tn, Hq * D, device=DEV) * 0.5).bfloat16().requires_grad_(True)
    T.log(f"[backward] mixer.forward B2 T{Tn} Hq{Hq} Hkv{Hkv} D{D} with gradients")
    ang = torch.arange(Tn, device=DEV).view(1, Tn, 1, 1) * torch.linspace(0.01, 1.0, D, device=DEV)
    pe = (ang.cos().bfloat16(), ang.sin().bfloat16())
    y = m(x, None, pe, None)
    (y.float() ** 2).mean().backward()
    torch.cuda.synchronize()
    assert x.grad is not None and bool(torch.isfinite(x.grad.float()).all())
    for name in ("c_q.weight", "c_k.weight", "c_v.weight", "c_proj.weight", "ln_s_k.weight", "ln_s_k.bias",
                 "state_head_temp", "front_head_temp"):
        p = dict(m.named_parameters())[name]
        assert p.grad is not None and bool(torch.isfinite(p.grad.float()).all()), name
        assert float(p.grad.float().abs().max()) > 0, f"{name}: zero gradient"


@pytest.mark.parametrize("B,Hq,Hkv,D,C,Tn,mode,factor,gates,extra", [
    (1, 4, 2, 64, 64, 300, "fixed", 1.0, (1, 1, 0, 0), {}),
    (2, 4, 2, 64, 64, 450, "power_law", 8.0, (1, 1, 0, 0), {}),
    (1, 2, 1, 128, 128, 700, "power_law", 8.0, (1, 0, 1, 1), {}),
    (1, 2, 2, 64, 32, 230, "fixed", 1.0, (1, 1, 0, 0), {}),  # chunks shorter than a 64-row block
    # the saturation budget with state_round_down 16, GQA and two sinks
    (2, 4, 2, 64, 64, 600, "kvm_saturation", 1.0, (1, 1, 1, 0),
     {"sat_n": 500, "round_down": 16, "min_len": 1, "n_max": 8, "sink": 2}),
    # kvm_use_head_temps 0 (no temperature parameters), two sinks, no merge gates
    (2, 2, 2, 64, 64, 400, "fixed", 1.0, (0, 0, 0, 0), {"temps": False, "sink": 2}),
])
def test_backward_matches_fp32_autograd(B, Hq, Hkv, D, C, Tn, mode, factor, gates, extra):
    if not torch.cuda.is_available():
        pytest.skip("needs an MI355X")
    from kvm_amd import training

    gk_, gv_, ga_, gi_ = gates
    temps = extra.get("temps", True)
    T.log(f"[backward] B{B} Hq{Hq} Hkv{Hkv} D{D} C{C} T{Tn} {mode} gates {gates} {extra}")
    cfg = T.mixer_config(Hq, Hkv, D, C, rope=16, mode=mode, min_len=extra.get("min_len", C),
                         n_max=extra.get("n_max", 4), factor=factor, expo=0.5, sat_n=extra.get("sat_n"),
                         round_down=extra.get("round_down", 1), sink=extra.get("sink", 1), temps=temps,
                         gate_keys=gk_, gate_values=gv_, gate_appends=ga_, gate_initial=gi_)
    gen = torch.Generator().manual_seed(11)
    lnw = (1 + 0.1 * torch.randn(D, generator=gen)).bfloat16()
    lnb = (0.1 * torch.randn(D, generator=gen)).bfloat16()
    tfh = (1 + 0.2 * torch.randn(Hq, generator=gen)).bfloat16()
    tsh = (1 + 0.2 * torch.randn(Hq, generator=gen)).bfloat16()
    m = T.make_mixer(cfg, lnw, lnb, tfh, tsh)
    m.train()
    q = torch.randn(B, Hq, Tn, D, generator=gen).bfloat16()
    k = torch.randn(B, Hkv, Tn, D, generator=gen).bfloat16()
    v = torch.randn(B, Hkv, Tn, D, generator=gen).bfloat16()
    g = (1 + F.elu(torch.randn(B, Hkv, Tn, 1, generator=gen))).bfloat16()
    dout = (torch.randn(B, Tn, Hq, D, generator=gen) * 0.1).bfloat16()
    # HIP
    xs = [t.to(DEV).requires_grad_(True) for t in (q, k, v, g)]
    y = training.prefill_with_grad(m, *xs)
    y.backward(dout.to(DEV))
    torch.cuda.synchronize()
    hip = {"q": xs[0].grad, "k": xs[1].grad, "v": xs[2].grad, "gate": xs[3].grad,
           "ln_w": m.ln_s_k.weight.grad, "ln_b": m.ln_s_k.bias.grad}
    if temps:
        hip.update(tau_state=m.state_head_temp.grad, tau_front=m.front_head_temp.grad)
    else:
        assert not hasattr(m, "state_head_temp") and not hasattr(m, "front_head_temp")
    # Routes of the HIP forward (deterministic: the same call again).
    with torch.no_grad():
        res = m.prefill_raw(*(t.to(DEV) for t in (q, k, v, g)), route_log=True)
    plan = res["plan"]
    if mode != "fixed":
        assert sum(plan.upd_n_append) > 0
    # Sinks are never merge targets.
    merged = res["append_log"] == 0
    assert bool((res["route_log"][merged] >= cfg.sink_len).all())
    # fp32 reference with the same routes (temperatures 1, without gradient, when the mixer has none)
    f32 = [t.to(DEV).float().requires_grad_(True) for t in (q, k, v, g, lnw, lnb, tsh, tfh)]
    if not temps:
        f32[6], f32[7] = torch.ones(Hq, device=DEV), torch.ones(Hq, device=DEV)
    rcfg = {"rope": 16, "gate_keys": gk_, "gate_values": gv_, "gate_appends": ga_, "gate_initial": gi_}
    yr = fixed_route_forward(*f32, plan, res["route_log"], res["append_log"], rcfg, cfg.n_bswa_chunks)
    T.assert_close_bf16(y.detach().float().transpose(1, 2), yr.detach(), "forward vs fp32 fixed-route forward")
    names = ["q", "k", "v", "gate", "ln_w", "ln_b"] + (["tau_state", "tau_front"] if temps else [])
    grads = torch.autograd.grad(yr.transpose(1, 2), f32[:len(names)], dout.to(DEV).float(), allow_unused=True)
    worst = []
    for name, ref in zip(names, grads):
        got = hip[name].float()
        if ref is None:  # an input the configuration does not use (the gate with every gate off)
            assert float(got.abs().max()) == 0.0, f"d{name} should be zero"
            worst.append(f"{name} unused (0)")
            continue
        assert got.shape == ref.shape, f"{name}: {tuple(got.shape)} vs {tuple(ref.shape)}"
        err = (got - ref).abs()
        rmax = float(err.max() / ref.abs().max().clamp_min(1e-12))
        rmean = float(err.mean() / ref.abs().mean().clamp_min(1e-12))
        worst.append(f"{name} {rmax:.1e}/{rmean:.1e}")
        assert rmax <= 5e-2 and rmean <= 2e-2, f"d{name}: relative max {rmax:.3e}, mean {rmean:.3e}"
    T.log(f"[backward] relative max/mean error per gradient: {', '.join(worst)}")


@pytest.mark.parametrize("B,Hkv,D,C,Tn,mode,gates", [
    (2, 2, 64, 64, 640, "power_law", (1, 1, 0, 0)),
    (1, 2, 128, 128, 1300, "power_law", (1, 0, 1, 1)),
    (1, 1, 64, 64, 400, "fixed", (0, 1, 1, 0)),
])
def test_state_backward_matches_replay_autograd(B, Hkv, D, C, Tn, mode, gates):
    """kvm_state_backward against torch autograd through replay_snapshot_rows
    (both fp32, the same routes): random snapshot-row gradients pulled back to
    k, v, the gate and the LayerNorm parameters (dk / dv start from zero, so
    they hold the state's share alone)."""
    if not torch.cuda.is_available():
        pytest.skip("needs an MI355X")
    from kvm_amd import training

    gk_, gv_, ga_, gi_ = gates
    Hq = Hkv
    T.log(f"[state-backward] B{B} Hkv{Hkv} D{D} C{C} T{Tn} {mode} gates {gates}")
    cfg = T.mixer_config(Hq, Hkv, D, C, rope=16, mode=mode, min_len=C, n_max=4, factor=8.0, expo=0.5,
                         gate_keys=gk_, gate_values=gv_, gate_appends=ga_, gate_initial=gi_)
    gen = torch.Generator().manual_seed(5)
    lnw = (1 + 0.1 * torch.randn(D, generator=gen)).bfloat16()
    lnb = (0.1 * torch.randn(D, generator=gen)).bfloat16()
    ones = torch.ones(Hq).bfloat16()
    m = T.make_mixer(cfg, lnw, lnb, ones, ones)
    q = torch.randn(B, Hq, Tn, D, generator=gen).bfloat16()
    k = torch.randn(B, Hkv, Tn, D, generator=gen).bfloat16()
    v = torch.randn(B, Hkv, Tn, D, generator=gen).bfloat16()
    g = (1 + F.elu(torch.randn(B, Hkv, Tn, 1, generator=gen))).bfloat16()
    with torch.no_grad():
        res = m.prefill_raw(*(t.to(DEV) for t in (q, k, v, g)), route_log=True)
    plan = res["plan"]
    rows = B * Hkv
    assert plan.n_updates > 0
    if mode != "fixed":
        assert sum(plan.upd_n_append) > 0
    n_snap = plan.n_updates + 1
    shape = (n_snap, rows, plan.max_state_len, D)
    dsk = torch.randn(shape, generator=gen).to(DEV)
    dsv = torch.randn(shape, generator=gen).to(DEV)
    lcfg = {"eps": 1e-5, "rope_partial_dim": 16, "gate_keys": gk_, "gate_values": gv_, "gate_appends": ga_,
            "gate_initial": gi_}
    kd, vd, gd = (x.to(DEV) for x in (k, v, g))
    dk = torch.zeros(B, Hkv, Tn, D, device=DEV)
    dv = torch.zeros(B, Hkv, Tn, D, device=DEV)
    dgate, d_ln = training.state_backward(m, kd, vd, gd, res, dsk, dsv, dk, dv)
    torch.cuda.synchronize()
    got = (dk.view(rows, Tn, D), dv.view(rows, Tn, D), dgate.view(rows, Tn), d_ln[0], d_ln[1])
    leaves = [x.float().requires_grad_(True) for x in (kd.reshape(rows, Tn, D), vd.reshape(rows, Tn, D),
                                                         gd.reshape(rows, Tn), lnw.to(DEV), lnb.to(DEV))]
    snaps = replay_snapshot_rows(*leaves, plan, res["route_log"], res["append_log"], lcfg)
    total = sum((ka * dsk[s, :, :ka.size(1)]).sum() + (va * dsv[s, :, :va.size(1)]).sum()
                for s, (ka, va) in enumerate(snaps))
    ref = torch.autograd.grad(total, leaves)
    worst = []
    for name, a, b in zip(["k", "v", "gate", "ln_w", "ln_b"], got, ref):
        assert a.shape == b.shape, name
        err = (a - b).abs()
        rmax = float(err.max() / b.abs().max().clamp_min(1e-12))
        rmean = float(err.mean() / b.abs().mean().clamp_min(1e-12))
        worst.append(f"{name} {rmax:.1e}/{rmean:.1e}")
        assert rmax <= 2e-3 and rmean <= 2e-4, f"d{name}: relative max {rmax:.3e}, mean {rmean:.3e}"
    T.log(f"[state-backward] relative max/mean error: {', '.join(worst)}")
