"""GPU parity of the HIP KVM path against the CPU oracle and the reference's
golden fixtures (tests/golden/*.npz, written from the reference's eager
mixer with FP32 routing).

Bars (north star):
  * routing: the slot of every overflow token equals the reference's, except
    (a) near-ties whose fp32 similarity margin is below the fp32 summation
    error bound (reported), and (b) tokens whose bf16 LayerNorm operand
    differs from the CPU's by rounding (reported);
  * outputs and carried state: bf16, max |err| <= 2e-2 and mean <= 2e-3
    (errors in fp32).
Every call goes through the C ABI of libkvm_amd.so.
"""

from __future__ import annotations

import ctypes
import math

import pytest
import torch

import golden_io
import kvm_testlib as T
from oracle import kvm_oracle as O

pytestmark = pytest.mark.gpu

DEV = "cuda"
# Fixtures of configurations the HIP mixer implements (the others pin only the CPU oracle).
BF16_FIXTURES = [n for n in golden_io.product_names() if golden_io.load(n)["meta"]["dtype"] == "bf16"]


@pytest.fixture(scope="module")
def lib():
    if not torch.cuda.is_available():
        pytest.skip("needs an MI355X")
    from kvm_amd import _lib

    return _lib.load()


def _rows(x):
    """[B, H, S, D] -> [B*H, S, D]."""
    return x.reshape(-1, x.size(-2), x.size(-1))


def _align256(n):
    return (n + 255) // 256 * 256


def bf16_ulp(x: torch.Tensor) -> torch.Tensor:
    """Spacing of bf16 numbers at |x| (8 significant bits): 2^(e - 7) for
    2^e <= |x| < 2^(e+1); the subnormal spacing 2^-133 below 2^-126."""
    a = x.double().abs().clamp_min(2.0 ** -126)
    return torch.exp2(torch.floor(torch.log2(a)) - 7)


def ulp_distance(got: torch.Tensor, ref: torch.Tensor, *scales: torch.Tensor) -> torch.Tensor:
    """|got - ref| in bf16 ulps of the largest magnitude among got, ref and
    `scales` (elementwise)."""
    mag = torch.maximum(got.double().abs(), ref.double().abs())
    for sc in scales:
        mag = torch.maximum(mag, sc.double().abs())
    return (got.double() - ref.double()).abs() / bf16_ulp(mag)


def layernorm_excess(got, other, x, p, zero_dims):
    """A bf16 LayerNorm output against the exact one.

    y = (x - mu) / sqrt(var + eps) * w + b computed exactly (fp64) after zeroing
    the first `zero_dims` features.  A correct fp32 evaluation rounded to bf16
    lies within ulp(y) + 2^-20 (|xhat w| + |b|) of y: half an ulp of rounding,
    half an ulp more where fp32 noise crosses a rounding boundary, and the fp32
    error of the terms themselves, which is many ulps of y only where they
    nearly cancel (y close to zero).  Returns (largest excess over that bar, the
    largest distance of `got` and of `other` from bf16(y) in ulps)."""
    xd = x.double().clone()
    xd[..., :zero_dims] = 0.0
    mu = xd.mean(-1, keepdim=True)
    var = ((xd - mu) ** 2).mean(-1, keepdim=True)
    xw = (xd - mu) / torch.sqrt(var + p.ln_eps) * p.ln_weight.double()
    y = xw + p.ln_bias.double()
    tol = bf16_ulp(y) + 2.0 ** -20 * (xw.abs() + p.ln_bias.double().abs())
    excess = float(((got.double() - y).abs() - tol).max())
    yb = y.bfloat16()
    return excess, float(ulp_distance(got, yb).max()), float(ulp_distance(other, yb).max())


class ParityCounts:
    """Route classification of update_parity, summed over updates."""

    def __init__(self):
        self.merged = self.mismatch = self.near_tie = self.operand = self.operand_tokens = 0
        self.max_tie_margin = 0.0      # largest |margin| / bound of a near-tie flip
        self.max_operand_margin = 0.0  # largest reference margin of an operand-rounding flip
        self.max_state_ulps = 0.0      # largest GPU distance (ulps) from the exact sums when routes agree
        self.max_oracle_ulps = 0.0     # the same for the CPU oracle's sums
        self.max_pk_ulps = 0.0         # GPU prep(k) vs the exact LayerNorm (ulps)
        self.max_oracle_pk_ulps = 0.0  # CPU oracle's prep(k) vs the exact LayerNorm
        self.updates = 0

    def add(self, o: "ParityCounts"):
        for k in ("merged", "mismatch", "near_tie", "operand", "operand_tokens", "updates"):
            setattr(self, k, getattr(self, k) + getattr(o, k))
        for k in ("max_tie_margin", "max_operand_margin", "max_state_ulps", "max_oracle_ulps",
                  "max_pk_ulps", "max_oracle_pk_ulps"):
            setattr(self, k, max(getattr(self, k), getattr(o, k)))
        return self

    def __str__(self):
        return (f"{self.updates} updates, {self.merged} merged tokens, {self.mismatch} route mismatches "
                f"({self.near_tie} fp32 near ties, max |margin| {self.max_tie_margin:.2f} x bound; "
                f"{self.operand} on a bf16 operand rounding, max reference margin {self.max_operand_margin:.2e}); "
                f"{self.operand_tokens} tokens with a rounded-differently operand (prep(k) from the exact "
                f"LayerNorm: GPU {self.max_pk_ulps:.1f} ulp, CPU oracle {self.max_oracle_pk_ulps:.1f} ulp); "
                f"updated sums within {self.max_state_ulps:.1f} ulp of exact (CPU oracle's: "
                f"{self.max_oracle_ulps:.1f} ulp)")


def update_parity(lib, layer, seq, u, tb, k, g, p, ocfg, C, D, ref_next, what, v=None):
    """One kvm_state_update from the oracle's state before update `u` (an
    O.UpdateRecord kept with keep_states=True) on tokens [tb, tb + C), against
    the oracle's decisions.  Returns a ParityCounts.

    Bars (every mismatch is classified, none is excused wholesale):
      * append sets are equal except at an exact tie of the bf16 novelty cut,
        or for a token whose GPU routing operand prep(k) rounds differently;
      * a differing merge route with identical operands is an fp32 near tie:
        the exact (fp64) scores of the two slots are within twice the fp32
        dot-product error bound;
      * a differing merge route on a token whose GPU operand rounds
        differently (one bf16 ulp in some element of LayerNorm's output) must
        be the first argmax for the GPU's operand (within the fp32 bound), and
        the reference's margin must be explained by the operand difference:
        margin <= sum_i |a_gpu_i - a_ref_i| |k_ref_i - k_gpu_i| + 2 bound;
      * when every route and append agrees (and `v` is given), each updated
        state element is within 3 bf16 ulps of the correctly rounded result
        recomputed exactly (fp64) from the agreed routes (derivation at the
        check below)."""
    from kvm_amd import _lib

    rows = int(u.s_k_before.size(0) * u.s_k_before.size(1))
    before = u.state_len_before
    after = before + u.n_append
    cap = after
    s_k = torch.zeros(rows, cap, D, dtype=torch.bfloat16)
    s_v = torch.zeros_like(s_k)
    vlen = torch.zeros(rows, cap)
    s_k[:, :before] = _rows(u.s_k_before)
    s_v[:, :before] = _rows(u.s_v_before)
    vlen[:, :before] = u.s_vlen_before.reshape(rows, before)
    ka = torch.zeros_like(s_k)
    va = torch.zeros_like(s_k)
    ka[:, :before] = _rows(O._ln(u.s_k_before, p))
    va[:, :before] = _rows(O.state_values_for_attention(u.s_v_before, u.s_vlen_before, ocfg))
    dev = [t.to(DEV).contiguous() for t in (s_k, s_v, vlen, ka, va)]
    out_k, out_v = torch.empty_like(dev[3]), torch.empty_like(dev[4])
    state = _lib.state_struct(*dev, cap)
    nws = int(lib.kvm_update_workspace_bytes(layer.ref(), C))
    ws = torch.zeros(nws, dtype=torch.uint8, device=DEV)
    route = torch.full((rows, C), -7, dtype=torch.int32, device=DEV)
    app = torch.full((rows, C), -7, dtype=torch.int32, device=DEV)
    _lib.check(lib.kvm_state_update(layer.ref(), seq, tb, C, before, u.n_append, state,
                                    out_k.data_ptr(), out_v.data_ptr(), ws.data_ptr(), nws,
                                    route.data_ptr(), app.data_ptr(), 0), "update")
    torch.cuda.synchronize()
    route, app = route.cpu(), app.cpu()
    o_app = torch.zeros(rows, C, dtype=torch.int32)
    o_route = torch.full((rows, C), -1, dtype=torch.int32)
    ai = u.append_idx.reshape(rows, -1)
    mi = u.merge_idx.reshape(rows, -1)
    for r in range(rows):
        o_app[r, ai[r]] = 1
        o_route[r, ai[r]] = before + torch.arange(ai.size(1), dtype=torch.int32)
        if u.route is not None:
            o_route[r, mi[r]] = u.route.reshape(rows, -1)[r].to(torch.int32)
    # GPU streams of the overflow tokens (workspace layout of include/kvm_amd.h).
    A = _align256(rows * C * D * 2)
    wsc = ws.cpu()
    g_pk = wsc[:A][: rows * C * D * 2].view(torch.bfloat16).view(rows, C, D)
    g_gk = wsc[A:2 * A][: rows * C * D * 2].view(torch.bfloat16).view(rows, C, D)
    o_pk = _rows(O.prep_k(k[:, :, tb:tb + C], p, ocfg.rope_partial_dim))
    o_gk = o_pk * _rows(g[:, :, tb:tb + C]) if ocfg.gate_keys else o_pk
    pk_diff_tok = (g_pk != o_pk).any(-1) | (g_gk != o_gk).any(-1)
    cnt = ParityCounts()
    cnt.updates = 1
    cnt.operand_tokens = int(pk_diff_tok.sum())
    if u.n_append > 0:
        nov = torch.matmul(o_pk.unsqueeze(0), _rows(O._ln(u.s_k_before, p)).transpose(-1, -2).unsqueeze(0))
        nov = nov.squeeze(0).float().max(-1).values  # bf16 scores as the reference ranks them
        for r in range(rows):
            diff = (app[r] != o_app[r]).nonzero().flatten()
            if len(diff):
                cut = torch.sort(nov[r]).values[u.n_append - 1]
                for t in diff.tolist():
                    assert nov[r, t] == cut or bool(pk_diff_tok[r, t]), f"{what} row {r}: append set differs at token {t} (no tie)"
    s_attn_gpu = dev[3].cpu()  # the rows routing read: oracle rows + appended rows written by the GPU
    merged = (app == 0) & (o_app == 0)
    cnt.merged = int(merged.sum())
    for r, t in ((merged & (route != o_route)).nonzero().tolist()):
        cnt.mismatch += 1
        gb, ob = int(route[r, t]), int(o_route[r, t])
        kr = s_attn_gpu[r].double()
        a = o_gk[r, t].double()
        la, lb = float(a @ kr[ob]), float(a @ kr[gb])
        bound = float(O.fp32_dot_error_bound(o_gk[r, t:t + 1], s_attn_gpu[r, [ob, gb]]).max())
        if bool(pk_diff_tok[r, t]):
            # (the GPU operand itself is checked against the exact LayerNorm below)
            ag = g_gk[r, t].double()
            gbound = float(O.fp32_dot_error_bound(g_gk[r, t:t + 1], s_attn_gpu[r]).max())
            lo = max(ocfg.sink_len, 0)
            best = float((kr[lo:after] @ ag).max())
            assert float(ag @ kr[gb]) >= best - 2 * gbound, (
                f"{what} row {r} token {t}: GPU slot {gb} is not the argmax for the GPU's own operand")
            explained = float(((ag - a).abs() * (kr[ob] - kr[gb]).abs()).sum())
            assert la - lb <= explained + 2 * bound, (
                f"{what} row {r} token {t}: reference margin {la - lb:.3e} exceeds what the operand "
                f"rounding explains ({explained:.3e} + 2 x {bound:.3e})")
            cnt.operand += 1
            cnt.max_operand_margin = max(cnt.max_operand_margin, la - lb)
            continue
        assert abs(la - lb) <= 2 * bound + 1e-6 * max(abs(la), 1.0), (
            f"{what} row {r} token {t}: GPU slot {gb} vs reference {ob}, margin {la - lb:.3e} > bound {bound:.3e}")
        cnt.near_tie += 1
        cnt.max_tie_margin = max(cnt.max_tie_margin, abs(la - lb) / max(bound, 1e-30))
    if v is not None:
        # The merge operands.  prep(k) is a LayerNorm: the GPU's must be within
        # one bf16 ulp of the exact (fp64) LayerNorm rounded once (the CPU's own
        # bf16 LayerNorm kernel is logged against the same exact value: near zero
        # its output may sit several ulps away).  The gated key and value are
        # single rounded products of bf16 numbers, so they must be bit-equal to
        # bf16(prep * gate) and bf16(v * gate) of the GPU's own prep.
        ov = _rows(v[:, :, tb:tb + C])
        gt = _rows(g[:, :, tb:tb + C])
        g_gv = wsc[2 * A:3 * A][: rows * C * D * 2].view(torch.bfloat16).view(rows, C, D)
        excess, pk_ulps, opk_ulps = layernorm_excess(g_pk, o_pk, _rows(k[:, :, tb:tb + C]), p,
                                                     ocfg.rope_partial_dim)
        cnt.max_pk_ulps = max(cnt.max_pk_ulps, pk_ulps)
        cnt.max_oracle_pk_ulps = max(cnt.max_oracle_pk_ulps, opk_ulps)
        assert excess <= 0.0, f"{what}: GPU prep(k) exceeds the LayerNorm rounding bar by {excess:.3e}"
        want_gk = g_pk * gt if ocfg.gate_keys else g_pk
        want_gv = ov * gt if ocfg.gate_values else ov
        assert bool(torch.equal(g_gk, want_gk)), f"{what}: GPU merge key is not bf16(prep * gate)"
        assert bool(torch.equal(g_gv, want_gv)), f"{what}: GPU merge value is not bf16(v * gate)"
        o_gv = want_gv
    if cnt.mismatch == 0 and bool((app == o_app).all()) and v is not None:
        # The merge arithmetic, against an exact recomputation from the agreed
        # routes and the GPU's own operands (a token whose LayerNorm output rounds
        # one ulp differently moves a small sum by many of ITS ulps, which is the
        # operand check above, not the summation): slot j holds base_j (its old
        # sum, or the appended token's row) and gains X_j, the exact (fp64) sum of
        # the merge rows routed to it; the correctly rounded result is
        # bf16(base_j + bf16(X_j)).  The kernels sum in fp32 in token order, exact
        # unless the terms' exponents spread over more than fp32's precision, so
        # their delta may differ from bf16(X_j) by one ulp(X_j) <= 2 ulp(M) near a
        # rounding boundary, and the final rounding adds one ulp(M): bar 3 ulps of
        # M (the largest of base, result and GPU).  The CPU oracle's distance from
        # the exact sums of ITS operands is logged alongside.
        app_k, app_v = (g_gk, g_gv) if ocfg.gate_appends else (g_pk, ov)
        o_app_k, o_app_v = (o_gk, o_gv) if ocfg.gate_appends else (o_pk, ov)
        ref_k, ref_v = _rows(ref_next[0]), _rows(ref_next[1])
        for nm, got_s, old_s, rows_m, rows_a, ref_s, o_rows_m, o_rows_a in (
                ("s_k", dev[0], s_k, g_gk, app_k, ref_k, o_gk, o_app_k),
                ("s_v", dev[1], s_v, g_gv, app_v, ref_v, o_gv, o_app_v)):
            def exact_update(m_rows, a_rows):
                base = old_s[:, :after].clone()
                X = torch.zeros(rows, after, D, dtype=torch.float64)
                for r in range(rows):
                    base[r, before:after] = a_rows[r, ai[r]]
                    sel = merged[r].nonzero().flatten()
                    X[r].index_add_(0, o_route[r, sel].long(), m_rows[r, sel].double())
                touched = (X != 0).any(-1, keepdim=True)
                return torch.where(touched, (base.double() + X.bfloat16().double()).bfloat16(), base), base

            exact, base = exact_update(rows_m, rows_a)
            worst = float(ulp_distance(got_s.cpu()[:, :after], exact, base).max())
            cnt.max_state_ulps = max(cnt.max_state_ulps, worst)
            o_exact, o_base = exact_update(o_rows_m, o_rows_a)
            cnt.max_oracle_ulps = max(cnt.max_oracle_ulps,
                                      float(ulp_distance(ref_s[:, :after], o_exact, o_base).max()))
            assert worst <= 3.0, f"{what} {nm}: an element is {worst:.1f} bf16 ulps from the exact sum (bar 3)"
    return cnt


def _fixture_mixer(fx):
    cfg = T.fixture_config(fx["meta"])
    m = T.make_mixer(cfg, fx["in_ln_w"], fx["in_ln_b"], fx["in_front_temp"], fx["in_state_temp"])
    return cfg, m


@pytest.mark.parametrize("name", BF16_FIXTURES)
def test_update_routing_matches_oracle(lib, name):
    """One kvm_state_update per recorded update, from the oracle's state."""
    from kvm_amd import _lib

    fx = golden_io.load(name)
    meta = fx["meta"]
    T.log(f"[update-parity] {name}")
    ocfg, p = golden_io.oracle_setup(fx)
    ocfg.append_tie_break = "lower_index"
    Tn = meta["T"]
    q, k, v, g = (fx["in_" + x][:, :, :Tn] for x in ("q", "k", "v", "gate"))
    rec = O.Recorder(keep_states=True)
    _, st_final = O.prefill(q, k, v, g, p, ocfg, rec)
    plan_tb = O.prefill_schedule(ocfg, Tn)["updates"]
    _, mixer = _fixture_mixer(fx)
    layer = mixer._layer_struct(meta["B"], torch.device(DEV))
    kd, vd, gd = k.to(DEV), v.to(DEV), g.to(DEV)
    seq, keep = _lib.seq4(kd, vd, gd)
    C, D = meta["C"], meta["D"]
    rows = meta["B"] * meta["Hkv"]
    tot = ParityCounts()
    for i, u in enumerate(rec.updates):
        nxt = rec.updates[i + 1] if i + 1 < len(rec.updates) else None
        ref_next = (nxt.s_k_before, nxt.s_v_before) if nxt is not None else (st_final[O.S_K], st_final[O.S_V])
        tot.add(update_parity(lib, layer, seq, u, plan_tb[i][0] * C, k, g, p, ocfg, C, D, ref_next, f"update {i}",
                              v=v))
    T.log(f"[update-parity] {name}: {tot}")
    assert tot.mismatch == tot.near_tie + tot.operand


def _prefill_gpu(fx, route_log=True):
    meta = fx["meta"]
    cfg, mixer = _fixture_mixer(fx)
    Tn = meta["T"]
    q, k, v, g = (fx["in_" + x][:, :, :Tn].to(DEV) for x in ("q", "k", "v", "gate"))
    with torch.no_grad():
        res = mixer.prefill_raw(q, k, v, g, route_log=route_log)
    torch.cuda.synchronize()
    return mixer, res


def _oracle_lower_index(fx):
    """The oracle with the lower-index append tie rule of the HIP kernels."""
    cfg, p = golden_io.oracle_setup(fx)
    cfg.append_tie_break = "lower_index"
    return cfg, p


@pytest.mark.parametrize("name", BF16_FIXTURES)
def test_prefill_matches_golden(lib, name):
    """GPU prefill vs the oracle on the fixture inputs (and vs the reference's
    recorded output whenever the oracle's trajectory is the reference's)."""
    fx = golden_io.load(name)
    meta = fx["meta"]
    T.log(f"[prefill-golden] {name} B{meta['B']} Hq{meta['Hq']} Hkv{meta['Hkv']} T{meta['T']} C{meta['C']}")
    mixer, res = _prefill_gpu(fx)
    ocfg, p = _oracle_lower_index(fx)
    Tn = meta["T"]
    rec = O.Recorder()
    y_ref, _ = O.prefill(*(fx["in_" + x][:, :, :Tn] for x in ("q", "k", "v", "gate")), p, ocfg, rec)
    same = torch.equal(y_ref, fx["y_prefill"])
    out = res["out"].cpu().transpose(1, 2)  # [B, Hq, T, D]
    mx, mean = T.assert_close_bf16(out, y_ref, f"{name} prefill output")
    if same:
        T.assert_close_bf16(out, fx["y_prefill"], f"{name} prefill output vs reference")
    plan = res["plan"]
    assert plan.n_updates == meta["n_prefill_updates"] == len(rec.updates)
    rows = meta["B"] * meta["Hkv"]
    agree = total = 0
    for i, u in enumerate(rec.updates):
        gr = res["route_log"][i].cpu()
        ga = res["append_log"][i].cpu()
        mi = u.merge_idx.reshape(rows, -1)
        ai = u.append_idx.reshape(rows, -1)
        for r in range(rows):
            assert torch.equal(ga[r].nonzero().flatten(), ai[r]), f"update {i} row {r}: append sets differ"
        if u.route is None:  # every token of this update was appended
            continue
        g_sel = torch.stack([gr[r, mi[r]] for r in range(rows)])
        ref_route = u.route.reshape(rows, -1).to(torch.int32)
        agree += int((g_sel == ref_route).sum())
        total += ref_route.numel()
    T.log(f"[prefill-golden] {name}: out max {mx:.2e} mean {mean:.2e}; routes {agree}/{total} agree; "
          f"oracle trajectory {'is' if same else 'differs from'} the reference's (append ties)")
    assert agree >= total - max(2, total // 200)


@pytest.mark.parametrize("name", [n for n in BF16_FIXTURES if n in golden_io.decode_names()])
def test_decode_matches_golden(lib, name):
    fx = golden_io.load(name)
    meta = fx["meta"]
    T.log(f"[decode-golden] {name} T{meta['T']} steps {meta['decode_steps']}")
    cfg, mixer = _fixture_mixer(fx)
    Tn, steps = meta["T"], meta["decode_steps"]
    ocfg, p = _oracle_lower_index(fx)
    cq, ck, cv, cg = (fx["in_" + x] for x in ("q", "k", "v", "gate"))
    _, ost = O.prefill(cq[:, :, :Tn], ck[:, :, :Tn], cv[:, :, :Tn], cg[:, :, :Tn], p, ocfg)
    oys = []
    for s in range(steps):
        t = Tn + s
        yd, ost = O.decode_step(ost, t, cq[:, :, t:t + 1], ck[:, :, t:t + 1], cv[:, :, t:t + 1], cg[:, :, t:t + 1], p, ocfg)
        oys.append(yd)
    y_ref = torch.cat(oys, 2)
    same = torch.equal(y_ref, fx["y_decode"])
    q, k, v, g = (fx["in_" + x].to(DEV) for x in ("q", "k", "v", "gate"))
    cache = T.LayerStatesCache()
    with torch.no_grad():
        mixer.forward_prefill(q[:, :, :Tn], k[:, :, :Tn], v[:, :, :Tn], g[:, :, :Tn], None, None, None, cache)
        outs = []
        for s in range(steps):
            t = Tn + s
            y = mixer.forward_single(q[:, :, t:t + 1], k[:, :, t:t + 1], v[:, :, t:t + 1], g[:, :, t:t + 1],
                                     None, None, None, cache)
            outs.append(y.float().cpu())
    torch.cuda.synchronize()
    y = torch.cat(outs, dim=1).view(meta["B"], steps, meta["Hq"], meta["D"]).transpose(1, 2)
    mx, mean = T.assert_close_bf16(y, y_ref, f"{name} decode outputs")
    if same:
        T.assert_close_bf16(y, fx["y_decode"], f"{name} decode outputs vs reference")
    dc = cache.get_states(0)[mixer._CACHE_TRITON_DECODE]
    sd = dc.logical_state_dict()
    ulp_log = []
    for key in (O.S_K, O.S_V, O.S_VLEN, O.BSWA_K, O.BSWA_V, O.BSWA_GATE):
        ref = ost[key]
        got = sd[key].cpu()
        assert got.shape == ref.shape, f"{key}: {tuple(got.shape)} vs {tuple(ref.shape)}"
        if key == O.S_VLEN:
            assert torch.allclose(got.float(), ref.float(), rtol=1e-5, atol=1e-5), key
        elif key in (O.S_K, O.S_V):
            # Carried sums: the bar is relative to the element's magnitude.  Each update
            # adds the same tokens in another order (fp32) and rounds to bf16 twice, so an
            # element may move by a bf16 ulp per update that touched it; the final state
            # must stay within 4 ulps everywhere (sums reach |x| ~ 8 here, where one ulp
            # is 2^-4, so an absolute 2e-2 bar would be below one ulp).
            ulps = ulp_distance(got, ref)
            ulp_log.append(f"{key} max {float(ulps.max()):.1f} ulp, {float((ulps > 0).float().mean()):.2e} of elements differ")
            assert float(ulps.max()) <= 4.0, f"{name} final {key}: {float(ulps.max()):.1f} bf16 ulps (bar 4)"
        else:
            T.assert_close_bf16(got, ref, f"{name} final {key}")
    assert sd[O.COVERAGE] == int(fx["final_kvm_state_coverage_len"]) == ost[O.COVERAGE]
    assert sd[O.BSWA_BEGIN] == int(fx["final_kvm_bswa_begin"]) == ost[O.BSWA_BEGIN]
    T.log(f"[decode-golden] {name}: out max {mx:.2e} mean {mean:.2e}; {dc.update_count} decode updates; "
          f"oracle trajectory {'is' if same else 'differs from'} the reference's; state {'; '.join(ulp_log)}")


# ---------------------------------------------------------------------------
# Attention numerics against fp64 on the GPU's own state.

def _fp64_attention(q, keys, values, visible):
    s = (q.double() @ keys.double().transpose(-1, -2)) / math.sqrt(q.size(-1))
    s = s.masked_fill(~visible, float("-inf"))
    return torch.softmax(s, dim=-1) @ values.double()


def _random_inputs(B, Hq, Hkv, Tn, D, seed):
    gen = torch.Generator().manual_seed(seed)
    q = (torch.randn(B, Hq, Tn, D, generator=gen) / math.sqrt(D)).bfloat16()
    k = (torch.randn(B, Hkv, Tn, D, generator=gen) / math.sqrt(D)).bfloat16()
    v = (torch.randn(B, Hkv, Tn, D, generator=gen) / math.sqrt(D)).bfloat16()
    g = (1.0 + torch.nn.functional.elu(torch.randn(B, Hkv, Tn, 1, generator=gen))).bfloat16()
    return q, k, v, g


@pytest.mark.parametrize("B,Hq,Hkv,Tn,D,C,mode", [
    (1, 4, 2, 1000, 128, 128, "fixed"),
    (2, 2, 2, 777, 64, 64, "power_law"),
    (1, 4, 2, 1300, 128, 256, "fixed"),
    (1, 2, 2, 1700, 64, 512, "power_law"),
])
def test_last_chunk_attention_exact(lib, B, Hq, Hkv, Tn, D, C, mode):
    """The last query chunk attends to the final state: compare with fp64."""
    T.log(f"[attn-exact] B{B} Hq{Hq} Hkv{Hkv} T{Tn} D{D} C{C} {mode}")
    cfg = T.mixer_config(Hq, Hkv, D, C, mode=mode, min_len=C, n_max=3, factor=6.0)
    gen = torch.Generator().manual_seed(7)
    ln_w = (1 + 0.1 * torch.randn(D, generator=gen)).bfloat16()
    ln_b = (0.1 * torch.randn(D, generator=gen)).bfloat16()
    ft = (1 + 0.1 * torch.randn(Hq, generator=gen)).bfloat16()
    stt = (1 + 0.1 * torch.randn(Hq, generator=gen)).bfloat16()
    m = T.make_mixer(cfg, ln_w, ln_b, ft, stt)
    q, k, v, g = _random_inputs(B, Hq, Hkv, Tn, D, 11)
    with torch.no_grad():
        res = m.prefill_raw(q.to(DEV), k.to(DEV), v.to(DEV), g.to(DEV))
    torch.cuda.synchronize()
    plan = res["plan"]
    S = plan.final_state_len
    mlast = plan.n_chunks - 1
    assert plan.chunk_state_len[mlast] == S
    qb, qe = mlast * C, Tn
    wb = max(0, (mlast - cfg.n_bswa_chunks + 1) * C)
    grp = Hq // Hkv
    ka = res["state_k_attn"].cpu()[:, :S].view(B, Hkv, S, D).repeat_interleave(grp, 1)
    va = res["state_v_attn"].cpu()[:, :S].view(B, Hkv, S, D).repeat_interleave(grp, 1)
    kw = k[:, :, wb:qe].repeat_interleave(grp, 1)
    vw = v[:, :, wb:qe].repeat_interleave(grp, 1)
    keys = torch.cat([(ka.float() * stt.float().view(1, Hq, 1, 1)).bfloat16(),
                      (kw.float() * ft.float().view(1, Hq, 1, 1)).bfloat16()], 2)
    vals = torch.cat([va, vw], 2)
    qpos = torch.arange(qb, qe).view(-1, 1)
    kpos = torch.cat([torch.full((S,), -1), torch.arange(wb, qe)]).view(1, -1)
    ref = _fp64_attention(q[:, :, qb:qe], keys, vals, kpos <= qpos)
    got = res["out"].cpu()[:, qb:qe].transpose(1, 2)
    mx, mean = T.assert_close_bf16(got, ref, "last-chunk attention", max_abs=8e-3, mean_abs=6e-4)
    T.log(f"[attn-exact] max {mx:.2e} mean {mean:.2e}")


@pytest.mark.parametrize("B,Hq,Hkv,D,S,R,W,start", [
    (4, 8, 8, 128, 1000, 300, 512, 400),
    (2, 8, 2, 64, 37, 120, 128, 100),
    (3, 4, 4, 128, 0, 60, 64, 10),
])
def test_decode_attention_exact(lib, B, Hq, Hkv, D, S, R, W, start):
    """kvm_decode_attention against fp64, including a wrapped window ring."""
    from kvm_amd import _lib

    T.log(f"[decode-exact] B{B} Hq{Hq} Hkv{Hkv} D{D} S{S} R{R} W{W} start{start}")
    gen = torch.Generator().manual_seed(3)
    rows = B * Hkv
    cap = max(S, 1) + 5
    ka = torch.randn(rows, cap, D, generator=gen).bfloat16()
    va = (0.5 * torch.randn(rows, cap, D, generator=gen)).bfloat16()
    rk = torch.randn(rows, W, D, generator=gen).bfloat16()
    rv = torch.randn(rows, W, D, generator=gen).bfloat16()
    q = (torch.randn(B, Hq, 1, D, generator=gen) / math.sqrt(D)).bfloat16()
    ts = (1 + 0.2 * torch.randn(Hq, generator=gen)).float()
    tf = (1 + 0.2 * torch.randn(Hq, generator=gen)).float()
    cfg = T.mixer_config(Hq, Hkv, D, 64)
    m = T.make_mixer(cfg, torch.ones(D), torch.zeros(D), tf, ts)
    layer = m._layer_struct(B, torch.device(DEV))
    dev = {n: t.to(DEV) for n, t in dict(ka=ka, va=va, rk=rk, rv=rv, q=q).items()}
    st = _lib.state_struct(dev["ka"], dev["va"], dev["va"][:, :, :1].contiguous(), dev["ka"], dev["va"], cap)
    nws = int(lib.kvm_decode_workspace_bytes(layer.ref(), S + R))
    ws = torch.empty(nws, dtype=torch.uint8, device=DEV)
    out = torch.empty(B, Hq, D, dtype=torch.bfloat16, device=DEV)
    _lib.check(lib.kvm_decode_attention(layer.ref(), dev["q"].data_ptr(), dev["q"].stride(0), dev["q"].stride(1),
                                        st, S, dev["rk"].data_ptr(), dev["rv"].data_ptr(), W, start, R,
                                        out.data_ptr(), out.stride(0), out.stride(1), ws.data_ptr(), nws, 0), "decode")
    torch.cuda.synchronize()
    grp = Hq // Hkv
    idx = (start + torch.arange(R)) % W
    ts_b, tf_b = m.state_head_temp.float().cpu(), m.front_head_temp.float().cpu()
    # The head temperature scales the exact score (the kernels' form; the same
    # as scaling the unrounded keys).
    keys = torch.cat([ka[:, :S].view(B, Hkv, S, D).repeat_interleave(grp, 1).double() * ts_b.view(1, Hq, 1, 1),
                      rk[:, idx].view(B, Hkv, R, D).repeat_interleave(grp, 1).double() * tf_b.view(1, Hq, 1, 1)], 2)
    vals = torch.cat([va[:, :S].view(B, Hkv, S, D).repeat_interleave(grp, 1), rv[:, idx].view(B, Hkv, R, D).repeat_interleave(grp, 1)], 2)
    ref = _fp64_attention(q, keys, vals, torch.ones(1, S + R, dtype=torch.bool)).squeeze(2)
    mx, mean = T.assert_close_bf16(out.cpu(), ref, "decode attention", max_abs=1e-2, mean_abs=1e-3)
    T.log(f"[decode-exact] max {mx:.2e} mean {mean:.2e}")


@pytest.mark.parametrize("B,Hq,Hkv,D,S,R,W,start", [
    (4, 8, 8, 128, 1000, 300, 512, 400),
    (2, 8, 2, 64, 37, 120, 128, 100),
    (3, 4, 4, 128, 0, 60, 64, 10),
    (2, 16, 4, 128, 0, 1, 64, 63),
])
def test_decode_step_matches_write_then_attend(lib, B, Hq, Hkv, D, S, R, W, start):
    """kvm_decode_step (ring write folded into the attention launches) gives
    the output and ring contents of kvm_ring_write + kvm_decode_attention,
    bit for bit; the token's row is the last of the R window rows."""
    from kvm_amd import _lib

    T.log(f"[decode-step] B{B} Hq{Hq} Hkv{Hkv} D{D} S{S} R{R} W{W} start{start}")
    gen = torch.Generator().manual_seed(5)
    rows = B * Hkv
    cap = max(S, 1) + 5
    t = dict(ka=torch.randn(rows, cap, D, generator=gen), va=0.5 * torch.randn(rows, cap, D, generator=gen),
             rk=torch.randn(rows, W, D, generator=gen), rv=torch.randn(rows, W, D, generator=gen),
             rg=1 + torch.rand(rows, W, generator=gen),
             q=torch.randn(B, Hq, 1, D, generator=gen) / math.sqrt(D),
             nk=torch.randn(B, Hkv, 1, D, generator=gen), nv=torch.randn(B, Hkv, 1, D, generator=gen),
             ng=1 + torch.rand(B, Hkv, 1, 1, generator=gen))
    dev = {n: x.bfloat16().to(DEV) for n, x in t.items()}
    cfg = T.mixer_config(Hq, Hkv, D, 64)
    m = T.make_mixer(cfg, torch.ones(D), torch.zeros(D), 1 + 0.2 * torch.randn(Hq, generator=gen),
                     1 + 0.2 * torch.randn(Hq, generator=gen))
    layer = m._layer_struct(B, torch.device(DEV))
    st = _lib.state_struct(dev["ka"], dev["va"], dev["va"][:, :, :1].contiguous(), dev["ka"], dev["va"], cap)
    seq, keep = _lib.seq4(dev["nk"], dev["nv"], dev["ng"])
    nws = int(lib.kvm_decode_workspace_bytes(layer.ref(), S + R))
    ws = torch.empty(nws, dtype=torch.uint8, device=DEV)
    q = dev["q"]
    res = {}
    for fused in (False, True):
        rk, rv, rg = dev["rk"].clone(), dev["rv"].clone(), dev["rg"].clone()
        out = torch.empty(B, Hq, D, dtype=torch.bfloat16, device=DEV)
        if fused:
            _lib.check(lib.kvm_decode_step(layer.ref(), q.data_ptr(), q.stride(0), q.stride(1), st, S, seq,
                                           rk.data_ptr(), rv.data_ptr(), rg.data_ptr(), W, start, R, out.data_ptr(),
                                           out.stride(0), out.stride(1), ws.data_ptr(), nws, 0), "decode step")
        else:
            _lib.check(lib.kvm_ring_write(layer.ref(), seq, rk.data_ptr(), rv.data_ptr(), rg.data_ptr(), W,
                                          (start + R - 1) % W, 0), "ring write")
            _lib.check(lib.kvm_decode_attention(layer.ref(), q.data_ptr(), q.stride(0), q.stride(1), st, S,
                                                rk.data_ptr(), rv.data_ptr(), W, start, R, out.data_ptr(),
                                                out.stride(0), out.stride(1), ws.data_ptr(), nws, 0), "decode")
        torch.cuda.synchronize()
        res[fused] = [x.cpu() for x in (out, rk, rv, rg)]
    del keep
    for name, a, b in zip(("out", "ring_k", "ring_v", "ring_gate"), res[False], res[True]):
        assert torch.equal(a, b), f"decode step {name} differs from ring write + attention"
    pos = (start + R - 1) % W
    assert torch.equal(res[True][1][:, pos], t["nk"].bfloat16().reshape(rows, D))
    T.log("[decode-step] output and ring bit-identical")


def test_decode_step_rejects_bad_window(lib):
    """kvm_decode_step refuses an empty window (the token must be its last row)."""
    from kvm_amd import _lib

    cfg = T.mixer_config(4, 4, 64, 64)
    m = T.make_mixer(cfg, torch.ones(64), torch.zeros(64), torch.ones(4), torch.ones(4))
    layer = m._layer_struct(1, torch.device(DEV))
    x = torch.zeros(4, 8, 64, dtype=torch.bfloat16, device=DEV)
    st = _lib.state_struct(x, x, x[:, :, :1].contiguous(), x, x, 8)
    tok = torch.zeros(1, 4, 1, 64, dtype=torch.bfloat16, device=DEV)
    seq, keep = _lib.seq4(tok, tok, tok[..., :1])
    rc = lib.kvm_decode_step(layer.ref(), tok.data_ptr(), 256, 64, st, 4, seq, x.data_ptr(), x.data_ptr(),
                             x.data_ptr(), 8, 0, 0, tok.data_ptr(), 256, 64, x.data_ptr(), x.numel() * 2, 0)
    assert rc != 0 and b"last window row" in lib.kvm_last_error()
    del keep


def test_prefill_deterministic(lib):
    """Two prefills of the same input are bit-identical (no atomics anywhere)."""
    B, Hq, Hkv, Tn, D, C = 1, 8, 8, 4096, 128, 256
    T.log(f"[determinism] B{B} H{Hq} T{Tn} C{C}")
    cfg = T.mixer_config(Hq, Hkv, D, C, min_len=C)
    m = T.make_mixer(cfg, torch.ones(D), torch.zeros(D), torch.ones(Hq), torch.ones(Hq))
    q, k, v, g = (t.to(DEV) for t in _random_inputs(B, Hq, Hkv, Tn, D, 5))
    with torch.no_grad():
        a = m.prefill_raw(q, k, v, g, route_log=True)
        b = m.prefill_raw(q, k, v, g, route_log=True)
    torch.cuda.synchronize()
    for key in ("out", "state_k", "state_v", "state_k_attn", "state_v_attn", "route_log"):
        assert torch.equal(a[key], b[key]), key
    assert bool(torch.isfinite(a["out"].float()).all())


@pytest.mark.parametrize("B,Hq,Hkv,Tn,D,C,mode", [
    (1, 4, 2, 1300, 128, 256, "fixed"),
    (1, 2, 1, 1700, 64, 512, "power_law"),
])
def test_prefill_wide_chunks_match_oracle(lib, B, Hq, Hkv, Tn, D, C, mode):
    """Whole prefill (every query chunk, every update) at chunk lengths that
    span several 128-query attention tiles per chunk, against the CPU oracle."""
    T.log(f"[prefill-wide] B{B} Hq{Hq} Hkv{Hkv} T{Tn} D{D} C{C} {mode}")
    cfg = T.mixer_config(Hq, Hkv, D, C, mode=mode, min_len=C, n_max=2, factor=6.0)
    gen = torch.Generator().manual_seed(5)
    ln_w = (1 + 0.1 * torch.randn(D, generator=gen)).bfloat16()
    ln_b = (0.1 * torch.randn(D, generator=gen)).bfloat16()
    ft = (1 + 0.1 * torch.randn(Hq, generator=gen)).bfloat16()
    stt = (1 + 0.1 * torch.randn(Hq, generator=gen)).bfloat16()
    m = T.make_mixer(cfg, ln_w, ln_b, ft, stt)
    q, k, v, g = _random_inputs(B, Hq, Hkv, Tn, D, 13)
    with torch.no_grad():
        res = m.prefill_raw(q.to(DEV), k.to(DEV), v.to(DEV), g.to(DEV))
    torch.cuda.synchronize()
    ocfg = O.OracleConfig(
        q_heads=Hq, kv_heads=Hkv, head_dim=D, value_dim=D, chunk_len=C, n_bswa_chunks=cfg.n_bswa_chunks,
        n_max_d_chunks=cfg.n_max_d_chunks, sink_len=cfg.sink_len, rope_partial_dim=cfg.rope_partial_dim,
        state_budget_mode=mode, state_growth_factor=cfg.state_growth_factor,
        state_growth_exponent=cfg.state_growth_exponent, state_round_down=1, state_min_len=C,
        append_tie_break="lower_index")
    p = O.OracleParams(ln_weight=ln_w, ln_bias=ln_b, front_temp=ft, state_temp=stt)
    y_ref, st = O.prefill(q, k, v, g, p, ocfg)
    got = res["out"].cpu().transpose(1, 2)
    mx, mean = T.assert_close_bf16(got, y_ref, "wide-chunk prefill output")
    S = res["plan"].final_state_len
    sk = res["state_k"].cpu()[:, :S].view(B, Hkv, S, D)
    # state sums: bf16 values of magnitude up to ~C; relative bound of a few bf16 ulps
    scale = float(st[O.S_K].float().abs().max())
    smx, smean = T.err_stats(sk, st[O.S_K])
    assert smx <= 2e-2 * scale and smean <= 2e-3 * scale, f"final s_k: max {smx:.3e}, mean {smean:.3e}, scale {scale:.3e}"
    T.log(f"[prefill-wide] out max {mx:.2e} mean {mean:.2e}; S={S}; s_k max {smx:.2e} mean {smean:.2e} (scale {scale:.2e})")


@pytest.mark.parametrize("B,Hq,Hkv,Tn,D,C,mode,sink,gate_app,budget", [
    (1, 8, 8, 4096, 128, 256, "fixed", 1, 0, None),
    (2, 4, 2, 3000, 64, 128, "power_law", 1, 0, None),
    (1, 4, 2, 2000, 128, 100, "power_law", 3, 1, None),
    (1, 32, 32, 8192, 128, 512, "fixed", 1, 0, None),
    (1, 4, 4, 6000, 64, 256, "power_law", 2, 0, 3),
    # more rows than one launch keeps resident (45 rows: launches over rows 0-31 and 32-44)
    (9, 10, 5, 2600, 128, 512, "fixed", 1, 0, None),
    (9, 5, 5, 1500, 64, 128, "power_law", 2, 0, None),
])
def test_chain_matches_per_update_kernels(lib, monkeypatch, B, Hq, Hkv, Tn, D, C, mode, sink, gate_app,
                                          budget):
    """The persistent update chains (slot-owner routing for batches without
    appends, token-split routing otherwise) and the per-update kernels give
    bit-identical routes, appends, state and outputs (same fp32 scores, same
    token-order sums); `budget` snapshots force several chain launches."""
    T.log(f"[chain] B{B} Hq{Hq} Hkv{Hkv} T{Tn} D{D} C{C} {mode} sink {sink} ring {budget}")
    cfg = T.mixer_config(Hq, Hkv, D, C, mode=mode, sink=sink, min_len=C, n_max=4, factor=6.0,
                         gate_appends=gate_app)
    gen = torch.Generator().manual_seed(11)
    ln_w = (1 + 0.1 * torch.randn(D, generator=gen)).bfloat16()
    ln_b = (0.1 * torch.randn(D, generator=gen)).bfloat16()
    m = T.make_mixer(cfg, ln_w, ln_b, torch.ones(Hq), torch.ones(Hq))
    q, k, v, g = (t.to(DEV) for t in _random_inputs(B, Hq, Hkv, Tn, D, 17))
    plan = m.make_plan(Tn)
    snap_bytes = None
    if budget is not None:
        snap_bytes = budget * 2 * B * Hkv * plan.max_state_len * D * 2
    res = {}
    for name, chain, fixed in (("owner", "1", "1"), ("token", "1", "0"), ("per-update", "0", "1")):
        monkeypatch.setenv("KVM_AMD_CHAIN", chain)
        monkeypatch.setenv("KVM_AMD_CHAIN_FIXED", fixed)
        with torch.no_grad():
            res[name] = m.prefill_raw(q, k, v, g, route_log=True, snapshot_budget=snap_bytes)
        torch.cuda.synchronize()
    b = res["per-update"]
    S = plan.final_state_len
    assert plan.n_updates > 0
    for name in ("owner", "token"):
        a = res[name]
        for key in ("route_log", "append_log", "out"):
            assert torch.equal(a[key], b[key]), f"{name} chain: {key}"
        for key in ("state_k", "state_v", "state_vlen", "state_k_attn", "state_v_attn"):
            assert torch.equal(a[key][:, :S], b[key][:, :S]), f"{name} chain: {key}"
    a = res["owner"]
    n_app = int(a["append_log"].sum())
    T.log(f"[chain] {plan.n_updates} updates, S={S}, {n_app} appended tokens: identical")


@pytest.mark.parametrize("C,D,n_keys", [(128, 128, 12), (100, 64, 5)])
def test_chain_append_ties_match_per_update_kernels(lib, monkeypatch, C, D, n_keys):
    """Exact novelty ties: every key is one of n_keys vectors per head, so
    many tokens of a chunk have the same novelty (and many slots the same
    key).  The appending chain (a bitonic sort of novelty-and-index keys)
    must select the same least-novel tokens as the per-update kernels, ties
    to the lower index, and route to the same lowest slots among equal
    scores: routes, appends, state and outputs bit for bit."""
    B, Hq, Hkv = 1, 4, 2
    Tn = C * 11 + C // 3
    T.log(f"[chain-ties] C{C} D{D} {n_keys} distinct keys per head, T{Tn}")
    cfg = T.mixer_config(Hq, Hkv, D, C, mode="power_law", sink=1, min_len=C, n_max=4, factor=6.0)
    gen = torch.Generator().manual_seed(29)
    ln_w = (1 + 0.1 * torch.randn(D, generator=gen)).bfloat16()
    ln_b = (0.1 * torch.randn(D, generator=gen)).bfloat16()
    m = T.make_mixer(cfg, ln_w, ln_b, torch.ones(Hq), torch.ones(Hq))
    q, _, v, g = _random_inputs(B, Hq, Hkv, Tn, D, 31)
    base = (torch.randn(B, Hkv, n_keys, D, generator=gen) / math.sqrt(D)).bfloat16()
    pick = torch.randint(0, n_keys, (B, Hkv, Tn), generator=gen)
    k = torch.gather(base, 2, pick.unsqueeze(-1).expand(B, Hkv, Tn, D))
    q, k, v, g = (t.to(DEV) for t in (q, k, v, g))
    plan = m.make_plan(Tn)
    assert sum(plan.upd_n_append) > 0
    res = {}
    for name, chain in (("chain", "1"), ("per-update", "0")):
        monkeypatch.setenv("KVM_AMD_CHAIN", chain)
        with torch.no_grad():
            res[name] = m.prefill_raw(q, k, v, g, route_log=True)
        torch.cuda.synchronize()
    a, b = res["chain"], res["per-update"]
    S = plan.final_state_len
    for key in ("route_log", "append_log", "out"):
        assert torch.equal(a[key], b[key]), key
    for key in ("state_k", "state_v", "state_vlen", "state_k_attn", "state_v_attn"):
        assert torch.equal(a[key][:, :S], b[key][:, :S]), key
    # The append sets against the oracle with the same lower-index tie rule.
    ocfg = O.OracleConfig(
        q_heads=Hq, kv_heads=Hkv, head_dim=D, value_dim=D, chunk_len=C, n_bswa_chunks=cfg.n_bswa_chunks,
        n_max_d_chunks=cfg.n_max_d_chunks, sink_len=cfg.sink_len, rope_partial_dim=cfg.rope_partial_dim,
        state_budget_mode="power_law", state_growth_factor=cfg.state_growth_factor,
        state_growth_exponent=cfg.state_growth_exponent, state_round_down=1, state_min_len=C,
        append_tie_break="lower_index")
    p = O.OracleParams(ln_weight=ln_w, ln_bias=ln_b, front_temp=torch.ones(Hq).bfloat16(),
                       state_temp=torch.ones(Hq).bfloat16())
    rec = O.Recorder()
    O.prefill(q.cpu(), k.cpu(), v.cpu(), g.cpu(), p, ocfg, rec)
    alog = a["append_log"].cpu()
    assert len(rec.updates) == plan.n_updates
    checked = 0
    for i, u in enumerate(rec.updates):
        for r in range(B * Hkv):
            want = sorted(u.append_idx[r // Hkv, r % Hkv].tolist()) if u.append_idx is not None else []
            got = torch.nonzero(alog[i, r]).flatten().tolist()
            assert got == want, f"update {i} row {r}: appended {got} against the oracle's {want}"
            checked += len(want)
    T.log(f"[chain-ties] {plan.n_updates} updates, S={S}, {checked} appended tokens: identical to the "
          f"per-update kernels and to the oracle")


@pytest.mark.parametrize("B,Hkv,Tn,D,min_len,skew", [
    (1, 32, 8192, 128, 768, False),   # 96 owned slots per member
    (1, 32, 8192, 128, 1024, False),  # 128 owned slots per member
    (2, 16, 6144, 64, 1024, False),
    (4, 8, 8192, 128, 1024, True),    # most tokens to a few slots: several staged rounds per half
])
def test_chain_wide_state_matches_per_update_kernels(lib, monkeypatch, B, Hkv, Tn, D, min_len, skew):
    """A fixed budget above the first chunk: the first update appends up to
    `min_len` slots (appending chain), every later one appends nothing, so
    the launch is split there and the rest runs on the slot-owner chain with
    more than 64 slots per member (up to 128 at 8 members).  Routes, state
    and outputs must equal the per-update kernels bit for bit."""
    C, Hq = 512, Hkv
    T.log(f"[chain-wide] B{B} Hkv{Hkv} T{Tn} D{D} C{C} min_len {min_len} skew {skew}")
    cfg = T.mixer_config(Hq, Hkv, D, C, mode="fixed", sink=1, min_len=min_len, n_max=4, factor=6.0)
    gen = torch.Generator().manual_seed(5)
    ln_w = (1 + 0.1 * torch.randn(D, generator=gen)).bfloat16()
    ln_b = (0.1 * torch.randn(D, generator=gen)).bfloat16()
    m = T.make_mixer(cfg, ln_w, ln_b, torch.ones(Hq), torch.ones(Hq))
    q, k, v, g = _random_inputs(B, Hq, Hkv, Tn, D, 23)
    if skew:
        d = torch.randn(D, generator=gen)
        k = (d / d.norm() + 0.02 * torch.randn(B, Hkv, Tn, D, generator=gen) / math.sqrt(D)).bfloat16()
    q, k, v, g = (t.to(DEV) for t in (q, k, v, g))
    plan = m.make_plan(Tn)
    S = plan.final_state_len
    assert S == min_len and plan.upd_n_append[0] > 0 and not any(plan.upd_n_append[1:])
    res = {}
    for name, chain, fixed in (("owner", "1", "1"), ("per-update", "0", "1")):
        monkeypatch.setenv("KVM_AMD_CHAIN", chain)
        monkeypatch.setenv("KVM_AMD_CHAIN_FIXED", fixed)
        with torch.no_grad():
            res[name] = m.prefill_raw(q, k, v, g, route_log=True)
        torch.cuda.synchronize()
    a, b = res["owner"], res["per-update"]
    for key in ("route_log", "append_log", "out"):
        assert torch.equal(a[key], b[key]), f"{key}"
    for key in ("state_k", "state_v", "state_vlen", "state_k_attn", "state_v_attn"):
        assert torch.equal(a[key][:, :S], b[key][:, :S]), f"{key}"
    r = b["route_log"][1: plan.n_updates].long()
    mem = torch.where(r >= 0, (r // 16) % 8, 8).flatten(0, 1)
    busiest = float(torch.stack([torch.bincount(x, minlength=9)[:8] for x in mem.cpu()]).max(dim=1).values
                    .float().mean())
    T.log(f"[chain-wide] {plan.n_updates} updates, S={S}: identical; busiest member takes {busiest:.0f} tokens")
    if skew:
        assert busiest > 96, "inputs did not skew the routes past one staged round"


@pytest.mark.parametrize("B,Hkv,Tn,D,C", [
    (4, 8, 8192, 128, 512),  # 32 rows: one launch
    (9, 5, 4096, 64, 256),   # 45 rows: two row batches
])
def test_chain_skewed_routes_match_per_update_kernels(lib, monkeypatch, B, Hkv, Tn, D, C):
    """Keys close to one shared direction send most of a chunk's tokens to
    the slots of one or two members of the slot-owner chain (which member
    changes from update to update), so members run far apart in time; the
    chain must still equal the barrier-synchronised per-update kernels
    bit for bit, on every one of three runs.  (A merge buffer reused one
    update too early showed up only under such skew.)"""
    Hq = Hkv
    T.log(f"[chain-skew] B{B} Hkv{Hkv} T{Tn} D{D} C{C}")
    cfg = T.mixer_config(Hq, Hkv, D, C, mode="fixed", sink=1, min_len=C, n_max=4, factor=6.0)
    gen = torch.Generator().manual_seed(3)
    ln_w = (1 + 0.1 * torch.randn(D, generator=gen)).bfloat16()
    ln_b = (0.1 * torch.randn(D, generator=gen)).bfloat16()
    m = T.make_mixer(cfg, ln_w, ln_b, torch.ones(Hq), torch.ones(Hq))
    q, _, v, g = _random_inputs(B, Hq, Hkv, Tn, D, 29)
    d = torch.randn(D, generator=gen)
    k = (d / d.norm() + 0.02 * torch.randn(B, Hkv, Tn, D, generator=gen) / math.sqrt(D)).bfloat16()
    q, k, v, g = (t.to(DEV) for t in (q, k, v, g))
    plan = m.make_plan(Tn)
    S = plan.final_state_len
    keys = ("route_log", "out", "state_k", "state_v", "state_vlen", "state_k_attn", "state_v_attn")
    monkeypatch.setenv("KVM_AMD_CHAIN", "0")
    with torch.no_grad():
        ref = m.prefill_raw(q, k, v, g, route_log=True)
    torch.cuda.synchronize()
    # the skew this test depends on: the busiest member's share of a row's chunk, averaged
    G = 8
    r = ref["route_log"][: plan.n_updates].long()
    mem = torch.where(r >= 0, (r // 16) % G, G).flatten(0, 1)  # [update * row, token]
    counts = torch.stack([torch.bincount(x, minlength=G + 1)[:G] for x in mem.cpu()])
    busiest = float(counts.max(dim=1).values.float().mean()) / C
    T.log(f"[chain-skew] {plan.n_updates} updates, S={S}; the busiest member takes {busiest:.0%} of a chunk on average")
    assert busiest >= 0.4, f"inputs did not skew the routes (busiest member {busiest:.0%})"
    monkeypatch.setenv("KVM_AMD_CHAIN", "1")
    monkeypatch.setenv("KVM_AMD_CHAIN_FIXED", "1")
    for run in range(3):
        with torch.no_grad():
            a = m.prefill_raw(q, k, v, g, route_log=True)
        torch.cuda.synchronize()
        for key in keys:
            x, y = a[key], ref[key]
            if key.startswith("state"):
                x, y = x[:, :S], y[:, :S]
            assert torch.equal(x, y), f"run {run}: {key}"


@pytest.mark.parametrize("Tn", [1, 5, 63, 64, 65, 128, 129, 191, 300])
def test_prefill_ragged_lengths_match_oracle(lib, Tn):
    """Prompt lengths around the chunk and window boundaries (C = 64, window
    2C): no update, the first update, partial last chunks; batch 3 with GQA.
    Output against the CPU oracle, then one cached decode step from the
    prefill's cache (output, state coverage and s_k) against the oracle's."""
    B, Hq, Hkv, D, C = 3, 2, 1, 64, 64
    T.log(f"[prefill-ragged] B{B} Hq{Hq} Hkv{Hkv} T{Tn} D{D} C{C}")
    cfg = T.mixer_config(Hq, Hkv, D, C, mode="fixed", min_len=C)
    gen = torch.Generator().manual_seed(Tn)
    ln_w = (1 + 0.1 * torch.randn(D, generator=gen)).bfloat16()
    ln_b = (0.1 * torch.randn(D, generator=gen)).bfloat16()
    ft = (1 + 0.1 * torch.randn(Hq, generator=gen)).bfloat16()
    stt = (1 + 0.1 * torch.randn(Hq, generator=gen)).bfloat16()
    m = T.make_mixer(cfg, ln_w, ln_b, ft, stt)
    q, k, v, g = _random_inputs(B, Hq, Hkv, Tn + 1, D, 100 + Tn)
    ocfg = O.OracleConfig(
        q_heads=Hq, kv_heads=Hkv, head_dim=D, value_dim=D, chunk_len=C, n_bswa_chunks=cfg.n_bswa_chunks,
        n_max_d_chunks=cfg.n_max_d_chunks, sink_len=cfg.sink_len, rope_partial_dim=cfg.rope_partial_dim,
        state_min_len=C, append_tie_break="lower_index")
    p = O.OracleParams(ln_weight=ln_w, ln_bias=ln_b, front_temp=ft, state_temp=stt)
    cache = T.LayerStatesCache()
    dq, dk, dv, dg = (x.to(DEV) for x in (q, k, v, g))
    with torch.no_grad():
        y = m.forward_prefill(dq[:, :, :Tn], dk[:, :, :Tn], dv[:, :, :Tn], dg[:, :, :Tn], None, None, None, cache)
        y_dec = m.forward_single(dq[:, :, Tn:], dk[:, :, Tn:], dv[:, :, Tn:], dg[:, :, Tn:], None, None, None, cache)
    torch.cuda.synchronize()
    y_ref, st = O.prefill(q[:, :, :Tn], k[:, :, :Tn], v[:, :, :Tn], g[:, :, :Tn], p, ocfg)
    T.assert_close_bf16(y.cpu().view(B, Tn, Hq, D).transpose(1, 2), y_ref, f"T={Tn} prefill output")
    dec_ref, st = O.decode_step(st, Tn, q[:, :, Tn:], k[:, :, Tn:], v[:, :, Tn:], g[:, :, Tn:], p, ocfg)
    T.assert_close_bf16(y_dec.cpu().view(B, 1, Hq, D).transpose(1, 2), dec_ref, f"T={Tn} decode step")
    c = cache.get_states(0)[m._CACHE_TRITON_DECODE]
    got = c.logical_state_dict()
    S = int(st[O.S_K].size(2))
    assert int(got["kvm_state_coverage_len"]) == int(st[O.COVERAGE])
    scale = max(1.0, float(st[O.S_K].float().abs().max()))
    smx, _ = T.err_stats(got["kvm_s_k"][:, :, :S].cpu(), st[O.S_K])
    assert smx <= 2e-2 * scale, f"T={Tn}: state s_k after the decode step: max err {smx:.3e} (scale {scale:.2e})"


@pytest.mark.parametrize("Tn", [100, 127, 191, 300])
def test_decode_after_prefill_matches_longer_prefill(lib, Tn):
    """One cached decode step after a prefill of T tokens gives the last row
    of a prefill of T + 1 tokens (the oracle's invariant, decode after
    prefill(T) = prefill(T + 1)), with head temperatures away from 1: the
    prefill and decode kernels apply them the same way (on the fp32 score).
    T = 127 and 191 put the decoded token at a chunk boundary (the decode
    step runs a state update).  The two paths sum the softmax in different
    orders and round the softmax weights differently, so the bar is a few
    bf16 ulps of each output row."""
    B, Hq, Hkv, D, C = 2, 4, 2, 128, 64
    T.log(f"[decode-vs-prefill] B{B} Hq{Hq} Hkv{Hkv} T{Tn} D{D} C{C}")
    cfg = T.mixer_config(Hq, Hkv, D, C, mode="fixed", min_len=C)
    gen = torch.Generator().manual_seed(500 + Tn)
    ln_w = (1 + 0.1 * torch.randn(D, generator=gen)).bfloat16()
    ln_b = (0.1 * torch.randn(D, generator=gen)).bfloat16()
    ft = (1 + 0.3 * torch.randn(Hq, generator=gen)).bfloat16()
    stt = (1 + 0.3 * torch.randn(Hq, generator=gen)).bfloat16()
    assert bool((ft != 1).all() and (stt != 1).all())
    m = T.make_mixer(cfg, ln_w, ln_b, ft, stt)
    q, k, v, g = (x.to(DEV) for x in _random_inputs(B, Hq, Hkv, Tn + 1, D, 600 + Tn))
    cache = T.LayerStatesCache()
    with torch.no_grad():
        y_long = m.forward_prefill(q, k, v, g, None, None, None, T.LayerStatesCache())
        m.forward_prefill(q[:, :, :Tn], k[:, :, :Tn], v[:, :, :Tn], g[:, :, :Tn], None, None, None, cache)
        y_dec = m.forward_single(q[:, :, Tn:], k[:, :, Tn:], v[:, :, Tn:], g[:, :, Tn:], None, None, None, cache)
    torch.cuda.synchronize()
    last = y_long.view(B, Tn + 1, Hq * D)[:, Tn].float().cpu()
    dec = y_dec.view(B, Hq * D).float().cpu()
    diff = (last - dec).abs()
    # One bf16 ulp of each head's output row, taken at the row's largest
    # magnitude: the prefill rounds the softmax weights to bf16 for its PV
    # product and the decode kernel keeps them in fp32, so elements near zero
    # differ by an ulp of the row, not of themselves.
    row_ulp = last.view(B, Hq, D).abs().amax(-1, keepdim=True).expand(B, Hq, D).reshape(B, Hq * D) * 2.0 ** -8
    ratio = float((diff / row_ulp).max())
    T.log(f"[decode-vs-prefill] max {float(diff.max()):.3e} mean {float(diff.mean()):.3e} "
          f"max / row ulp {ratio:.2f}")
    assert ratio <= 4.0, "decode step and the longer prefill's last row differ beyond 4 ulps of the row"
    assert float(diff.mean()) <= 2e-5


def test_prefill_saturation_budget_matches_oracle(lib):
    """The saturation budget (state_budget_mode "kvm_saturation",
    floor(N t / (N + t)), model/kvm_mixer.py:131-165) grows the state with
    appends over the prefill: state length, output and final state against
    the CPU oracle."""
    B, Hq, Hkv, D, C, Tn = 1, 4, 2, 64, 64, 1000
    cfg = T.mixer_config(Hq, Hkv, D, C, mode="kvm_saturation", min_len=C, n_max=4, sat_n=2000)
    T.log(f"[prefill-saturation] B{B} Hq{Hq} Hkv{Hkv} T{Tn} D{D} C{C} N=2000 cap {C * 4}")
    gen = torch.Generator().manual_seed(41)
    ln_w = (1 + 0.1 * torch.randn(D, generator=gen)).bfloat16()
    ln_b = (0.1 * torch.randn(D, generator=gen)).bfloat16()
    ft = (1 + 0.1 * torch.randn(Hq, generator=gen)).bfloat16()
    stt = (1 + 0.1 * torch.randn(Hq, generator=gen)).bfloat16()
    m = T.make_mixer(cfg, ln_w, ln_b, ft, stt)
    q, k, v, g = _random_inputs(B, Hq, Hkv, Tn, D, 43)
    with torch.no_grad():
        res = m.prefill_raw(q.to(DEV), k.to(DEV), v.to(DEV), g.to(DEV), route_log=True)
    torch.cuda.synchronize()
    ocfg = O.OracleConfig(
        q_heads=Hq, kv_heads=Hkv, head_dim=D, value_dim=D, chunk_len=C, n_bswa_chunks=cfg.n_bswa_chunks,
        n_max_d_chunks=4, sink_len=cfg.sink_len, rope_partial_dim=cfg.rope_partial_dim,
        state_budget_mode="kvm_saturation", state_min_len=C, state_saturation_n=2000,
        append_tie_break="lower_index")
    p = O.OracleParams(ln_weight=ln_w, ln_bias=ln_b, front_temp=ft, state_temp=stt)
    rec = O.Recorder()
    y_ref, st = O.prefill(q, k, v, g, p, ocfg, rec)
    S = res["plan"].final_state_len
    assert S == int(st[O.S_K].size(2)) and S > C, (S, int(st[O.S_K].size(2)))
    assert sum(u.n_append for u in rec.updates) == S - C
    T.assert_close_bf16(res["out"].cpu().transpose(1, 2), y_ref, "saturation prefill output")
    # append sets and merge routes of every update against the oracle's
    rows = B * Hkv
    n_diff = total = 0
    for i, u in enumerate(rec.updates):
        gr = res["route_log"][i].cpu()
        ga = res["append_log"][i].cpu()
        mi = u.merge_idx.reshape(rows, -1)
        if u.append_idx is not None:
            ai = u.append_idx.reshape(rows, -1)
            for r in range(rows):
                assert torch.equal(ga[r].nonzero().flatten(), ai[r]), f"update {i} row {r}: append sets differ"
        if u.route is None:  # every token of this update was appended
            assert mi.size(1) == 0
            continue
        g_sel = torch.stack([gr[r, mi[r]] for r in range(rows)])
        n_diff += int((g_sel != u.route.reshape(rows, -1).to(torch.int32)).sum())
        total += g_sel.numel()
    T.log(f"[prefill-saturation] S {C} -> {S}, {len(rec.updates)} updates, {n_diff}/{total} merge routes differ")
    assert n_diff == 0
