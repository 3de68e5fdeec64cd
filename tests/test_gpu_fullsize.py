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


def test_config1_exact_shape(lib):
    """BASELINE config 1 at its own shape: B1 H4 D64 T4096, chunk 256, n_bswa 2,
    fixed memory of 64 configured slots (the first chunk fills the state, so 256
    are live), rope_partial_dim 32, q/k/v ~ N(0,1) in fp32, unit LayerNorm and
    temperatures.  The HIP path computes in bf16 (as the reference's Triton path
    does), so it runs on the bf16-rounded inputs and is checked two ways:
      * against the bf16 oracle on the same bf16 inputs (the exactness claim):
        every update re-run from the oracle's state with every route mismatch
        classified (test_gpu_parity.update_parity), outputs within the bf16
        tolerance (max 2e-2, mean 2e-3);
      * against the fp32 oracle on the fp32 inputs (the reference's own CPU
        configuration).  Rounding the inputs to bf16 moves routing scores by
        ~2^-8 relative, so routes near a tie go elsewhere and the memory state
        takes another trajectory; the output difference this causes is a
        property of the algorithm in bf16, measured by the bf16 oracle against
        the fp32 oracle.  Bar: the HIP output is no further from fp32 than
        that (max and mean within 1.25x, plus 2e-3)."""
    from kvm_amd import _lib
    from oracle import kvm_oracle as O
    from test_gpu_parity import ParityCounts, update_parity

    B, H, D, Tn, C = 1, 4, 64, 4096, 256
    T.log(f"[config1] B{B} H{H} D{D} T{Tn} C{C} fixed 64 (256 live) rope 32")
    cfg = T.mixer_config(H, H, D, C, rope=32, mode="fixed", min_len=64, n_max=1)
    ones_d, zeros_d, ones_h = torch.ones(D), torch.zeros(D), torch.ones(H)
    m = T.make_mixer(cfg, ones_d, zeros_d, ones_h, ones_h)
    gen = torch.Generator().manual_seed(1)
    q32, k32, v32 = (torch.randn(B, H, Tn, D, generator=gen) for _ in range(3))
    g32 = 1 + torch.nn.functional.elu(torch.randn(B, H, Tn, 1, generator=gen))
    q16, k16, v16, g16 = (x.bfloat16() for x in (q32, k32, v32, g32))
    with torch.no_grad():
        res = m.prefill_raw(*(x.to(DEV) for x in (q16, k16, v16, g16)), route_log=True)
    torch.cuda.synchronize()
    out = res["out"].cpu().transpose(1, 2).float()
    # 16 chunks: chunks 2..15 read snapshots 0..13, so 13 updates run
    assert res["plan"].n_updates == 13 and res["plan"].final_state_len == 256

    def setup(dtype):
        c = O.OracleConfig(q_heads=H, kv_heads=H, head_dim=D, value_dim=D, chunk_len=C, n_bswa_chunks=2,
                           sink_len=1, rope_partial_dim=32, state_min_len=64, append_tie_break="lower_index")
        p = O.OracleParams(ln_weight=ones_d.to(dtype), ln_bias=zeros_d.to(dtype),
                           front_temp=ones_h.to(dtype), state_temp=ones_h.to(dtype))
        return c, p

    c32, p32 = setup(torch.float32)
    rec32 = O.Recorder()
    y32, _ = O.prefill(q32, k32, v32, g32, p32, c32, rec32)
    c16, p16 = setup(torch.bfloat16)
    rec = O.Recorder(keep_states=True)
    y16, st16 = O.prefill(q16, k16, v16, g16, p16, c16, rec)
    mx16, mean16 = T.assert_close_bf16(out, y16, "config 1 HIP vs bf16 oracle")
    mx32, mean32 = T.err_stats(out, y32)
    algo_mx, algo_mean = T.err_stats(y16, y32)
    assert mx32 <= 1.25 * algo_mx + 2e-3 and mean32 <= 1.25 * algo_mean + 2e-3, (
        f"config 1 HIP vs fp32 oracle: max {mx32:.3e} mean {mean32:.3e}; the bf16 oracle itself: "
        f"max {algo_mx:.3e} mean {algo_mean:.3e}")
    layer = m._layer_struct(B, torch.device(DEV))
    seq, keep = _lib.seq4(k16.to(DEV), v16.to(DEV), g16.to(DEV))
    sched = O.prefill_schedule(c16, Tn)["updates"]
    tot = ParityCounts()
    for i, u in enumerate(rec.updates):
        nxt = rec.updates[i + 1] if i + 1 < len(rec.updates) else None
        ref_next = (nxt.s_k_before, nxt.s_v_before) if nxt is not None else (st16[O.S_K], st16[O.S_V])
        tot.add(update_parity(lib, layer, seq, u, sched[i][0] * C, k16, g16, p16, c16, C, D, ref_next,
                              f"config 1 update {i}", v=v16))
    del keep
    # Routes of the HIP trajectory against the fp32 reference's: the bf16-rounded
    # inputs move the scores by ~2^-8 relative, so routes near a tie differ (logged).
    agree = total = 0
    for i, u in enumerate(rec32.updates):
        mi = u.merge_idx.reshape(B * H, -1)
        g_sel = torch.gather(res["route_log"][i].cpu(), 1, mi)
        agree += int((g_sel == u.route.reshape(B * H, -1).to(torch.int32)).sum())
        total += g_sel.numel()
    T.log(f"[config1] vs fp32 oracle: out max {mx32:.2e} mean {mean32:.2e} (bf16 oracle vs fp32 oracle: max "
          f"{algo_mx:.2e} mean {algo_mean:.2e}), routes {agree}/{total} equal; "
          f"vs bf16 oracle: out max {mx16:.2e} mean {mean16:.2e}; per update from the oracle's state: {tot}")
    assert tot.mismatch == tot.near_tie + tot.operand


@pytest.mark.parametrize("name,B,Hq,Hkv,Tn,D,C,mode,n_max,factor", [
    # config 2: fixed memory of 512 slots, 61 updates
    ("config2", 1, 32, 32, 32768, 128, 512, "fixed", 1, 1.0),
    # config 3, growth-exercising variant: power_law f=16, e=0.5, n_max_d_chunks=2 (S 512 -> 1024)
    ("config3-growth", 2, 16, 16, 65536, 128, 512, "power_law", 2, 16.0),
    # config 3 as written: floor(sqrt(t)) slots capped at 1024, which never passes the
    # 512 slots the first chunk fills (125 updates, no appends)
    ("config3-literal", 2, 16, 16, 65536, 128, 512, "power_law", 2, 1.0),
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
            # head temperature on the exact score (the kernels' form)
            keys = torch.cat([ka[row].cpu().double() * ts_b[hq], rk[row].cpu()[idx].double() * tf_b[hq]])
            vals = torch.cat([va[row].cpu(), rv[row].cpu()[idx]])
            ref = _fp64_attention(q[bi, hq].cpu(), keys, vals, torch.ones(1, S + R, dtype=torch.bool))
            mx, mean = T.assert_close_bf16(out[bi, hq].cpu().view(1, D), ref, f"decode b{bi} h{hq}",
                                           max_abs=1e-2, mean_abs=1e-3)
            worst = (max(worst[0], mx), max(worst[1], mean))
    T.log(f"[full-size] decode sampled rows: max {worst[0]:.2e} mean {worst[1]:.2e}")


def test_config4_decode_update_full_size(lib):
    """BASELINE config 4's decode-time state update at its real shape: 2048 rows
    (B64 x 32 heads) x 256 overflow tokens x 1024 slots, run by the decode cache
    on the first token after a 128K-context snapshot, then that token's
    attention.  Rows of three sequences (96 rows) are checked against the oracle
    run from the same snapshot:
      * every merge route equals the oracle's, or is classified: with identical
        operands an fp32 near tie (fp64 scores within twice the fp32 error
        bound); with operands that round differently (the GPU's LayerNorm of the
        token or of a slot, one bf16 ulp per element at most) the GPU's slot must
        be the first argmax for its own operands;
      * the updated sums of every row without a differing route are within 5
        bf16 ulps of the oracle's; the decode output within the bf16 tolerance."""
    import kvm_amd
    from oracle import kvm_oracle as O

    B, H, D, C, n, S, total = 64, 32, 128, 256, 2, 1024, 131072
    W = n * C
    T.log(f"[config4-update] B{B} H{H} D{D} C{C} S{S} total {total}: one decode step with its state update")
    cfg = T.mixer_config(H, H, D, C, rope=64, mode="fixed", min_len=S, n_max=4)
    m = T.make_mixer(cfg, torch.ones(D), torch.zeros(D), torch.ones(H), torch.ones(H))
    gen = torch.Generator(device=DEV).manual_seed(1)
    cnt = torch.randint(1, 4097, (B, H, S, 1), generator=gen, device=DEV).float()
    mean_k = torch.randn(B, H, S, D, generator=gen, device=DEV) * math.sqrt(0.5)
    mean_v = torch.randn(B, H, S, D, generator=gen, device=DEV) * math.sqrt(0.5)
    begin = max(0, (total + C - 1) // C * C - W)
    R = total - begin
    vlen16 = mean_v.norm(dim=-1, keepdim=True).bfloat16()
    snap = kvm_amd.DecodeCacheSnapshot(
        state_k=(mean_k * cnt).bfloat16(), state_v=(mean_v * cnt).bfloat16(), state_vlen=vlen16.float(),
        recent_k=(torch.randn(B, H, R, D, generator=gen, device=DEV) / math.sqrt(D)).bfloat16(),
        recent_v=(torch.randn(B, H, R, D, generator=gen, device=DEV) / math.sqrt(D)).bfloat16(),
        recent_gate=(1 + torch.nn.functional.elu(torch.randn(B, H, R, 1, generator=gen, device=DEV))).bfloat16(),
        total_len=total, state_coverage_len=max(min(total, C), begin), recent_begin=begin)
    q = (torch.randn(B, H, 1, D, generator=gen, device=DEV) / math.sqrt(D)).bfloat16()
    k = (torch.randn(B, H, 1, D, generator=gen, device=DEV) / math.sqrt(D)).bfloat16()
    v = (torch.randn(B, H, 1, D, generator=gen, device=DEV) / math.sqrt(D)).bfloat16()
    g = (1 + torch.nn.functional.elu(torch.randn(B, H, 1, 1, generator=gen, device=DEV))).bfloat16()
    cache = m.make_decode_cache(snap, state_capacity=S)
    ka_before = cache.state_k_attn.clone()
    with torch.no_grad():
        y = m._decode_one_token(q, k, v, g, cache).clone()
    torch.cuda.synchronize()
    assert cache.update_count == 1
    rows = B * H
    A = (rows * C * D * 2 + 255) // 256 * 256
    ws = cache.update_workspace
    g_gk = ws[A:A + rows * C * D * 2].view(torch.bfloat16).view(rows, C, D)

    bsel = [0, 37, B - 1]
    ocfg = O.OracleConfig(q_heads=H, kv_heads=H, head_dim=D, value_dim=D, chunk_len=C, n_bswa_chunks=n,
                          n_max_d_chunks=4, sink_len=cfg.sink_len, rope_partial_dim=64, state_min_len=S,
                          append_tie_break="lower_index")
    p = O.OracleParams(ln_weight=torch.ones(D).bfloat16(), ln_bias=torch.zeros(D).bfloat16(),
                       front_temp=torch.ones(H).bfloat16(), state_temp=torch.ones(H).bfloat16())
    sub = lambda t: t[bsel].cpu()  # noqa: E731
    ost = {O.S_K: sub(snap.state_k), O.S_V: sub(snap.state_v), O.S_VLEN: sub(vlen16),
           O.COVERAGE: snap.state_coverage_len, O.BSWA_BEGIN: begin,
           O.BSWA_K: sub(snap.recent_k), O.BSWA_V: sub(snap.recent_v), O.BSWA_GATE: sub(snap.recent_gate)}
    rec = O.Recorder()
    torch.set_num_threads(min(16, torch.get_num_threads()))
    oy, ost2 = O.decode_step(ost, total, sub(q), sub(k), sub(v), sub(g), p, ocfg, rec)
    assert len(rec.updates) == 1 and rec.updates[0].n_append == 0
    u = rec.updates[0]
    o_route = u.route.reshape(len(bsel) * H, -1).to(torch.int32)  # every token merges (no appends)
    ov_tb = u.merge_idx.reshape(len(bsel) * H, -1)
    assert bool((ov_tb == torch.arange(C)).all())
    o_ka = O._ln(ost[O.S_K], p).reshape(-1, S, D)
    lo = snap.state_coverage_len - begin  # the overflow chunk: window tokens [lo, lo + C)
    o_pk = O.prep_k(ost[O.BSWA_K][:, :, lo:lo + C], p, 64).reshape(-1, C, D)
    o_gk = o_pk * ost[O.BSWA_GATE][:, :, lo:lo + C].reshape(-1, C, 1)
    # The GPU's routing operands against exact (fp64) LayerNorms rounded once: the
    # slot rows LayerNorm(s_k) it refreshed from the snapshot and the overflow
    # tokens' prep(k); each within one bf16 ulp.
    from test_gpu_parity import layernorm_excess, ulp_distance
    rsel =torch.tensor([b * H + h for b in bsel for h in range(H)]).to(DEV)
    g_pk = ws[:rows * C * D * 2].view(torch.bfloat16).view(rows, C, D)[rsel].cpu()
    ex_ka, ka_ulps, _ = layernorm_excess(ka_before[rsel].cpu()[:, :S], o_ka, ost[O.S_K].reshape(-1, S, D), p, 0)
    ex_pk, pk_ulps, _ = layernorm_excess(g_pk, o_pk, ost[O.BSWA_K][:, :, lo:lo + C].reshape(-1, C, D), p, 64)
    assert ex_ka <= 0.0 and ex_pk <= 0.0, f"GPU LayerNorms beyond the rounding bar: slots {ex_ka:.2e}, tokens {ex_pk:.2e}"
    n_mis = n_tie = n_operand = 0
    bad_rows = set()
    for j, b in enumerate(bsel):
        for h in range(H):
            r, ro = b * H + h, j * H + h
            gr = cache.route_by_token[r].cpu()
            assert int(cache.append_by_token[r].sum()) == 0
            kg = ka_before[r].cpu()
            ag_all = g_gk[r].cpu()
            for t in (gr != o_route[ro]).nonzero().flatten().tolist():
                n_mis += 1
                bad_rows.add(ro)
                gb, ob = int(gr[t]), int(o_route[ro, t])
                a, ag = o_gk[ro, t], ag_all[t]
                same = torch.equal(a, ag) and torch.equal(kg[[ob, gb]], o_ka[ro, [ob, gb]])
                if same:
                    la, lb = float(a.double() @ o_ka[ro, ob].double()), float(a.double() @ o_ka[ro, gb].double())
                    bound = float(O.fp32_dot_error_bound(a.view(1, D), o_ka[ro, [ob, gb]]).max())
                    assert abs(la - lb) <= 2 * bound, f"row {r} token {t}: margin {la - lb:.3e} > {2 * bound:.3e}"
                    n_tie += 1
                else:
                    # (the GPU's operands are checked against exact LayerNorms below)
                    sc = kg[ocfg.sink_len:].double() @ ag.double()
                    gbound = float(O.fp32_dot_error_bound(ag.view(1, D), kg).max())
                    assert float(kg[gb].double() @ ag.double()) >= float(sc.max()) - 2 * gbound, (
                        f"row {r} token {t}: GPU slot {gb} is not the argmax for its own operands")
                    n_operand += 1
    worst = 0.0
    for j, b in enumerate(bsel):
        for h in range(H):
            ro, r = j * H + h, b * H + h
            if ro in bad_rows:
                continue
            for nm, got, ref, old in (("s_k", cache.state_k[r], ost2[O.S_K][j, h], ost[O.S_K][j, h]),
                                      ("s_v", cache.state_v[r], ost2[O.S_V][j, h], ost[O.S_V][j, h])):
                ul = float(ulp_distance(got.cpu()[:S], ref, old).max())
                worst = max(worst, ul)
                assert ul <= 5.0, f"row {r} {nm}: {ul:.1f} ulps (bar 5, test_gpu_parity.update_parity)"
    mx, mean = T.assert_close_bf16(y[bsel].cpu().view(len(bsel), H, 1, D), oy, "config 4 decode output after the update")
    T.log(f"[config4-update] {len(bsel) * H} rows x {C} tokens: {n_mis} route mismatches ({n_tie} fp32 near ties, "
          f"{n_operand} operand roundings); GPU LayerNorms within {max(ka_ulps, pk_ulps):.1f} ulp of exact; "
          f"sums within {worst:.1f} ulp of the oracle's in {len(bsel) * H - len(bad_rows)} rows; "
          f"output max {mx:.2e} mean {mean:.2e}")


@pytest.mark.parametrize("name,B,Hq,Hkv,Tn,D,C,mode,n_max,factor", [
    ("config2", 1, 32, 32, 32768, 128, 512, "fixed", 1, 1.0),
    ("config3-growth", 2, 16, 16, 65536, 128, 512, "power_law", 2, 16.0),
    ("config3-literal", 2, 16, 16, 65536, 128, 512, "power_law", 2, 1.0),
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
    # Route exactness from an identical state at full size, for EVERY update: each
    # update runs once more on the GPU from the oracle's own state before it, and every
    # differing route must be a classified fp32 near tie or operand rounding
    # (test_gpu_parity.update_parity states the bars).
    from kvm_amd import _lib
    from test_gpu_parity import ParityCounts, update_parity

    layer = m._layer_struct(B, torch.device(DEV))
    seq, keep = _lib.seq4(k, v, g)
    nu = len(rec.updates)
    tot = ParityCounts()
    for i in range(nu):
        u = rec.updates[i]
        nxt = rec.updates[i + 1] if i + 1 < nu else None
        ref_next = (nxt.s_k_before, nxt.s_v_before) if nxt is not None else (st[O.S_K], st[O.S_V])
        tot.add(update_parity(lib, layer, seq, u, sched[i][0] * C, kc, gc, p, ocfg, C, D, ref_next,
                              f"{name} update {i}", v=vc))
        if i % 16 == 15:
            T.log(f"[full-size-oracle] {name}: updates 0..{i} from the oracle's state: {tot}")
    del keep
    T.log(f"[full-size-oracle] {name}: every update from the oracle's state: {tot}")
    assert tot.updates == nu and tot.mismatch == tot.near_tie + tot.operand
    S = res["plan"].final_state_len
    out = res["out"].cpu().transpose(1, 2)
    mx, mean = T.assert_close_bf16(out, y_ref, f"{name} full-size output")
    T.log(f"[full-size-oracle] {name}: {len(rec.updates)} updates, {n_route} merge routes, {n_diff} differ, "
          f"{n_app_diff} updates with a different append set; bit-exact through update "
          f"{len(rec.updates) - 1 if first is None else first - 1}; out max {mx:.2e} mean {mean:.2e}")
    # End to end, the two trajectories are compared as well.  The two sides sum each
    # slot's tokens in different orders (the reference's bf16 one-hot matmul, the
    # kernels' token-order fp32 sums), so their states may differ by a bf16 ulp and a
    # route near a tie may flip; from there the trajectories hold different sums in the
    # slots involved, most with config 3's clustered keys (near-identical slots).  The
    # exactness claim is the per-update check above; here the bar is that the
    # trajectories stay close: append sets equal, at most 2% of the routes differing,
    # outputs within the bf16 tolerance (checked above).
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
