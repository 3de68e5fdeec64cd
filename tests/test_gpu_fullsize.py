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


def _rows(x):
    return x.reshape(-1, x.size(-2), x.size(-1))

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


@pytest.mark.parametrize("name,B,Hq,Hkv,Tn,D,C,mode,n_max,factor", [
    ("config2", 1, 32, 32, 32768, 128, 512, "fixed", 1, 1.0),
    ("config3-growth", 2, 16, 16, 65536, 128, 512, "power_law", 2, 16.0),
])
def test_full_size_prefill_matches_oracle(lib, name, B, Hq, Hkv, Tn, D, C, mode, n_max, factor):
    """The whole full-size prefill against the CPU oracle on the same inputs
    (config 2: 61 updates, ~1M merge routes; config 3: 125 updates with
    appends, clustered keys): routes and append sets (logged: the first update
    with a difference), output within the bf16 tolerance, state rows; and, for
    the first, middle, last and first-differing updates, one update from the
    oracle's own state, where every differing route must be an fp32 near tie
    or a bf16 operand rounding (test_gpu_parity.update_parity)."""
    from oracle import kvm_oracle as O

    T.log(f"[full-size-oracle] {name}: B{B} Hq{Hq} Hkv{Hkv} T{Tn} D{D} C{C} {mode}")
    cfg = T.mixer_config(Hq, Hkv, D, C, mode=mode, min_len=C, n_max=n_max, factor=factor, expo=0.5)
    gen = torch.Generator().manual_seed(23)
    ln_w = (1 + 0.1 * torch.randn(D, generator=gen)).bfloat16()
    ln_b = (0.1 * torch.randn(D, generator=gen)).bfloat16()
    ft = (1 + 0.1 * torch.randn(Hq, generator=gen)).bfloat16()
    stt = (1 + 0.1 * torch.randn(Hq, generator=gen)).bfloat16()
    m = T.make_mixer(cfg, ln_w, ln_b, ft, stt)
    q, k, v, g = _gpu_inputs(B, Hq, Hkv, Tn, D, 29, clustered=name.startswith("config3"))
    with torch.no_grad():
        res = m.prefill_raw(q, k, v, g, route_log=True)
    torch.cuda.synchronize()
    ocfg = O.OracleConfig(
        q_heads=Hq, kv_heads=Hkv, head_dim=D, value_dim=D, chunk_len=C, n_bswa_chunks=cfg.n_bswa_chunks,
        n_max_d_chunks=n_max, sink_len=cfg.sink_len, rope_partial_dim=cfg.rope_partial_dim,
        state_budget_mode=mode, state_growth_factor=factor, state_growth_exponent=0.5, state_min_len=C,
        append_tie_break="lower_index")
    p = O.OracleParams(ln_weight=ln_w, ln_bias=ln_b, front_temp=ft, state_temp=stt)
    rec = O.Recorder(keep_states=True)
    torch.set_num_threads(min(16, torch.get_num_threads()))
    qc, kc, vc, gc = q.cpu(), k.cpu(), v.cpu(), g.cpu()
    y_ref, st = O.prefill(qc, kc, vc, gc, p, ocfg, rec)
    rows = B * Hkv
    assert len(rec.updates) == res["plan"].n_updates
    sched = O.prefill_schedule(ocfg, Tn)["updates"]
    first = None          # first update whose routes or appends differ
    n_diff = n_route = n_app_diff = 0
    for i, u in enumerate(rec.updates):
        gr = res["route_log"][i].cpu()
        ga = res["append_log"][i].cpu()
        ai = u.append_idx.reshape(rows, -1)
        app_ok = all(torch.equal(ga[r].nonzero().flatten(), ai[r]) for r in range(rows))
        if u.route is None:
            mism = torch.zeros(rows, 0, dtype=torch.bool)
        else:
            mi = u.merge_idx.reshape(rows, -1)
            g_sel = torch.gather(gr, 1, mi)
            mism = g_sel != u.route.reshape(rows, -1).to(torch.int32)
            n_diff += int(mism.sum())
            n_route += mism.numel()
        if first is None and (not app_ok or bool(mism.any())):
            first = i
        n_app_diff += 0 if app_ok else 1
    # Route exactness from an identical state at full size: the first update with a
    # difference (where the trajectories part), the first, middle and last updates.
    from kvm_amd import _lib
    from test_gpu_parity import update_parity

    layer = m._layer_struct(B, torch.device(DEV))
    seq, keep = _lib.seq4(k, v, g)
    nu = len(rec.updates)
    pc = [0, 0, 0, 0]
    for i in sorted({0, nu // 2, nu - 1} | ({first} if first is not None else set())):
        u = rec.updates[i]
        nxt = rec.updates[i + 1] if i + 1 < nu else None
        ref_next = (nxt.s_k_before, nxt.s_v_before) if nxt is not None else (st[O.S_K], st[O.S_V])
        c = update_parity(lib, layer, seq, u, sched[i][0] * C, kc, gc, p, ocfg, C, D, ref_next, f"{name} update {i}")
        pc = [x + y for x, y in zip(pc, c)]
    del keep
    T.log(f"[full-size-oracle] {name}: sampled updates from the oracle's state: {pc[0]} merged tokens, "
          f"{pc[1]} route mismatches ({pc[2]} fp32 near ties, {pc[3]} bf16 operand roundings)")
    S = res["plan"].final_state_len
    out = res["out"].cpu().transpose(1, 2)
    mx, mean = T.assert_close_bf16(out, y_ref, f"{name} full-size output")
    T.log(f"[full-size-oracle] {name}: {len(rec.updates)} updates, {n_route} merge routes, {n_diff} differ, "
          f"{n_app_diff} updates with a different append set; bit-exact through update "
          f"{len(rec.updates) - 1 if first is None else first - 1}; out max {mx:.2e} mean {mean:.2e}")
    # The two sides sum each slot's tokens in different orders (the reference's bf16
    # one-hot matmul, the kernels' token-order fp32 sums), so their states may differ by
    # a bf16 ulp and a route near a tie may flip; from there the trajectories differ in
    # the slots involved, most with config 3's clustered keys (near-identical slots).
    # Measured: config 2 0.015% of the routes (bit-exact through update 37 of 61),
    # config 3 1.0% (through update 15 of 125).  Bar: append sets equal, at most 2% of
    # the routes, outputs within the bf16 tolerance (checked above).
    assert n_app_diff == 0 and n_diff <= n_route // 50
    # After a near tie the two trajectories hold different sums in the slots involved; everywhere
    # else the state agrees: at least 99% of the slot rows within the bf16 tolerance.
    sk = res["state_k"][:, :S].cpu().view(B, Hkv, S, D).float()
    ref_sk = st[O.S_K].float()
    scale = float(ref_sk.abs().max())
    row_err = (sk - ref_sk).abs().amax(-1)
    frac = float((row_err <= 2e-2 * scale).float().mean())
    assert frac >= 0.99, f"{name}: only {frac:.4f} of the state rows agree"
    if first is None:
        assert n_diff == 0
