"""Parity at the BASELINE configurations' full sizes, through properties that
do not depend on running the CPU oracle at that size:

* the persistent update chain and the per-update kernels give bit-identical
  routes, appends, state and outputs over a whole 32K / 64K-token prefill
  (two independent implementations of the routing recurrence);
* routing invariants: sink slots are never merge targets, every target lies
  below the state length of its update, and appended rows are marked -1;
* vlens = 1: the attention value row of every slot has norm vlen;
* attention of the last query chunk (sampled heads) against fp64 softmax over
  the final state and the window;
* decode attention at config 4's full size (2048 rows, 1024 slots, wrapped
  1024-row window ring) on sampled rows against fp64.
"""
from __future__ import annotations

import math

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


def _gpu_inputs(B, Hq, Hkv, Tn, D, seed, clustered=False):
    """q/k/v ~ N(0,1)/sqrt(D), gate 1+elu(N(0,1)).  clustered:
    10% of the keys are one of 8 centres shared by every head, N(0,1)/sqrt(D),
    plus N(0, 0.05^2)/sqrt(D) noise, which stresses routing with near-equal keys."""
    gen = torch.Generator(device=DEV).manual_seed(seed)
    q = (torch.randn(B, Hq, Tn, D, device=DEV, generator=gen) / math.sqrt(D)).bfloat16()
    kf = torch.randn(B, Hkv, Tn, D, device=DEV, generator=gen)
    if clustered:
        centres = torch.randn(8, D, device=DEV, generator=gen)
        pick = torch.randint(0, 8, (B, Hkv, Tn), device=DEV, generator=gen)
        sel = torch.rand(B, Hkv, Tn, device=DEV, generator=gen) < 0.1
        noisy = centres[pick] + 0.05 * torch.randn(B, Hkv, Tn, D, device=DEV, generator=gen)
        kf = torch.where(sel.unsqueeze(-1), noisy, kf)
    k = (kf / math.sqrt(D)).bfloat16()
    v = (torch.randn(B, Hkv, Tn, D, device=DEV, generator=gen) / math.sqrt(D)).bfloat16()
    g = (1.0 + torch.nn.functional.elu(torch.randn(B, Hkv, Tn, 1, device=DEV, generator=gen))).bfloat16()
    return q, k, v, g


def _fp64_attention(q, keys, values, visible):
    s = (q.double() @ keys.double().transpose(-1, -2)) / math.sqrt(q.size(-1))
    s = s.masked_fill(~visible, float("-inf"))
    return torch.softmax(s, dim=-1) @ values.double()


@pytest.mark.parametrize("name,B,Hq,Hkv,Tn,D,C,mode,n_max,factor", [
    # config 2: fixed memory of 512 slots, 61 updates
    ("config2", 1, 32, 32, 32768, 128, 512, "fixed", 1, 1.0),
    # config 3, growth-exercising variant: power_law f=16, e=0.5, n_max_d_chunks=2 (S 512 -> 1024)
    ("config3-growth", 2, 16, 16, 65536, 128, 512, "power_law", 2, 16.0),
])
def test_full_size_prefill(lib, monkeypatch, name, B, Hq, Hkv, Tn, D, C, mode, n_max, factor):
    T.log(f"[full-size] {name}: B{B} Hq{Hq} Hkv{Hkv} T{Tn} D{D} C{C} {mode}")
    cfg = T.mixer_config(Hq, Hkv, D, C, mode=mode, min_len=C, n_max=n_max, factor=factor, expo=0.5)
    gen = torch.Generator().manual_seed(23)
    ln_w = (1 + 0.1 * torch.randn(D, generator=gen)).bfloat16()
    ln_b = (0.1 * torch.randn(D, generator=gen)).bfloat16()
    ft = (1 + 0.1 * torch.randn(Hq, generator=gen)).bfloat16()
    stt = (1 + 0.1 * torch.randn(Hq, generator=gen)).bfloat16()
    m = T.make_mixer(cfg, ln_w, ln_b, ft, stt)
    q, k, v, g = _gpu_inputs(B, Hq, Hkv, Tn, D, 29, clustered=name.startswith("config3"))
    plan = m.make_plan(Tn)
    res = {}
    for which, chain in (("chain", "1"), ("per-update", "0")):
        monkeypatch.setenv("KVM_AMD_CHAIN", chain)
        with torch.no_grad():
            res[which] = m.prefill_raw(q, k, v, g, route_log=True)
        torch.cuda.synchronize()
    a, b = res["chain"], res["per-update"]
    S = plan.final_state_len
    for key in ("route_log", "append_log", "out"):
        assert torch.equal(a[key], b[key]), f"{name}: {key} differs between the chain and the per-update kernels"
    for key in ("state_k", "state_v", "state_vlen", "state_k_attn", "state_v_attn"):
        assert torch.equal(a[key][:, :S], b[key][:, :S]), f"{name}: {key}"
    assert bool(torch.isfinite(a["out"].float()).all())

    # Routing invariants over every update.
    route, app = a["route_log"], a["append_log"]  # [n_updates, rows, C]
    before = torch.tensor(plan.upd_state_before, device=DEV, dtype=torch.int32).view(-1, 1, 1)
    n_app = torch.tensor(plan.upd_n_append, device=DEV, dtype=torch.int32).view(-1, 1, 1)
    merged = app == 0
    sink = int(cfg.sink_len)
    assert bool((route[merged] >= sink).all()), "a sink slot received a merge"
    assert bool(((route < before + n_app) | ~merged).all()), "a merge target lies past the state"
    # Appended tokens take the new slots S_before .. S_before + n_append - 1, in token order.
    assert torch.equal(app.sum(dim=2), n_app.view(-1, 1).expand(-1, app.size(1)).to(app.dtype))
    for u in range(plan.n_updates):
        na = int(plan.upd_n_append[u])
        if na == 0:
            continue
        got = route[u][app[u] == 1].view(app.size(1), na)
        want = plan.upd_state_before[u] + torch.arange(na, device=DEV, dtype=route.dtype)
        assert torch.equal(got, want.expand_as(got)), f"update {u}: appended slots"
    # vlens = 1: ||s_v_attn_j|| == vlen_j (bf16 rows)
    va = a["state_v_attn"][:, :S].float()
    vl = a["state_vlen"][:, :S].float()
    rel = ((va.norm(dim=-1) - vl).abs() / vl.clamp_min(1e-6)).max().item()
    assert rel < 1e-2, f"attention value norms differ from vlen by {rel:.2e}"

    # Last query chunk, sampled heads, against fp64 over the final state and the window.
    mlast = plan.n_chunks - 1
    assert plan.chunk_state_len[mlast] == S
    qb, qe = mlast * C, Tn
    wb = max(0, (mlast - cfg.n_bswa_chunks + 1) * C)
    grp = Hq // Hkv
    worst = (0.0, 0.0)
    for bi in sorted({0, B - 1}):
        for hq in (0, Hq // 2 + 1, Hq - 1):
            hk = hq // grp
            row = bi * Hkv + hk
            ka = a["state_k_attn"][row, :S].cpu()
            vs = a["state_v_attn"][row, :S].cpu()
            kw = k[bi, hk, wb:qe].cpu()
            vw = v[bi, hk, wb:qe].cpu()
            keys = torch.cat([(ka.float() * stt[hq].float()).bfloat16(), (kw.float() * ft[hq].float()).bfloat16()])
            vals = torch.cat([vs, vw])
            qpos = torch.arange(qb, qe).view(-1, 1)
            kpos = torch.cat([torch.full((S,), -1), torch.arange(wb, qe)]).view(1, -1)
            ref = _fp64_attention(q[bi, hq, qb:qe].cpu(), keys, vals, kpos <= qpos)
            got = a["out"][bi, qb:qe, hq].cpu()
            mx, mean = T.assert_close_bf16(got, ref, f"{name} last chunk b{bi} h{hq}", max_abs=8e-3, mean_abs=6e-4)
            worst = (max(worst[0], mx), max(worst[1], mean))
    n_merged = int(merged.sum())
    T.log(f"[full-size] {name}: {plan.n_updates} updates, S={S}, {n_merged} merged and "
          f"{int(app.sum())} appended tokens; chain == per-update; last chunk max {worst[0]:.2e} "
          f"mean {worst[1]:.2e}; vlen rel {rel:.1e}")


def test_full_size_decode_attention(lib):
    """Config 4 shape: B64 H32 D128, 1024 memory slots, 1024-row window ring
    holding 385 rows that wrap around its end."""
    from kvm_amd import _lib

    B, Hq, Hkv, D, S, W, R, start = 64, 32, 32, 128, 1024, 1024, 385, 800
    T.log(f"[full-size] decode B{B} Hq{Hq} D{D} S{S} ring {W} recent {R} start {start}")
    rows = B * Hkv
    gen = torch.Generator(device=DEV).manual_seed(31)
    ka = (0.5 * torch.randn(rows, S, D, device=DEV, generator=gen)).bfloat16()
    va = (0.5 * torch.randn(rows, S, D, device=DEV, generator=gen)).bfloat16()
    rk = torch.randn(rows, W, D, device=DEV, generator=gen).bfloat16()
    rv = torch.randn(rows, W, D, device=DEV, generator=gen).bfloat16()
    q = (torch.randn(B, Hq, 1, D, device=DEV, generator=gen) / math.sqrt(D)).bfloat16()
    gt = torch.Generator().manual_seed(37)
    ts = (1 + 0.2 * torch.randn(Hq, generator=gt)).float()
    tf = (1 + 0.2 * torch.randn(Hq, generator=gt)).float()
    cfg = T.mixer_config(Hq, Hkv, D, 256)
    m = T.make_mixer(cfg, torch.ones(D), torch.zeros(D), tf, ts)
    layer = m._layer_struct(B, torch.device(DEV))
    vlen = torch.ones(rows, S, device=DEV)
    st = _lib.state_struct(ka, va, vlen, ka, va, S)
    nws = int(lib.kvm_decode_workspace_bytes(layer.ref(), S + R))
    ws = torch.empty(nws, dtype=torch.uint8, device=DEV)
    out = torch.empty(B, Hq, D, dtype=torch.bfloat16, device=DEV)
    _lib.check(lib.kvm_decode_attention(layer.ref(), q.data_ptr(), q.stride(0), q.stride(1), st, S,
                                        rk.data_ptr(), rv.data_ptr(), W, start, R, out.data_ptr(),
                                        out.stride(0), out.stride(1), ws.data_ptr(), nws, 0), "decode")
    torch.cuda.synchronize()
    assert bool(torch.isfinite(out.float()).all())
    idx = (start + torch.arange(R)) % W
    ts_b, tf_b = m.state_head_temp.float().cpu(), m.front_head_temp.float().cpu()
    worst = (0.0, 0.0)
    for bi in (0, 37, B - 1):
        for hq in (0, 13, Hq - 1):
            row = bi * Hkv + hq * Hkv // Hq
            keys = torch.cat([(ka[row].cpu().float() * ts_b[hq]).bfloat16(),
                              (rk[row].cpu()[idx].float() * tf_b[hq]).bfloat16()])
            vals = torch.cat([va[row].cpu(), rv[row].cpu()[idx]])
            ref = _fp64_attention(q[bi, hq].cpu(), keys, vals, torch.ones(1, S + R, dtype=torch.bool))
            mx, mean = T.assert_close_bf16(out[bi, hq].cpu().view(1, D), ref, f"decode b{bi} h{hq}",
                                           max_abs=1e-2, mean_abs=1e-3)
            worst = (max(worst[0], mx), max(worst[1], mean))
    T.log(f"[full-size] decode sampled rows: max {worst[0]:.2e} mean {worst[1]:.2e}")
