"""Benchmark of the MI355X KVM forward path (one GPU).

Workloads:
  prefill  config 2: one KVM layer, B1 Hq=Hkv=32 D128, T=32768, chunk 512,
           n_bswa 2, fixed memory (state_min_len 256; the first chunk fills
           the state, so 512 slots are live), q/k/v ~ N(0,1)/sqrt(128),
           gate 1+elu(N(0,1)), bf16, fp32 routing/accumulation.
           A step = one prefill at the post-QKV boundary (q/k/v/gate
           resident in HBM -> [B, T, Hq*D] output + final state).
  decode   config 4: B64 Hq=Hkv=32 D128, chunk 256, n_bswa 2 (512-token
           window), 1024 memory slots at total length 131072; a step =
           one token for all 64 sequences (ring write, the state update when
           a chunk boundary is crossed, split-K attention).  The timed
           region is `--decode-steps` consecutive tokens from a fresh
           snapshot, so the one update per 256 tokens is included.
  config3  config 3: B2 H16 D128 T65536 chunk 512, floor(sqrt(tokens seen)) slots capped
           at 1024, clustered keys; the budget as written and a growth
           variant (factor 16, 512 -> 1024 slots by appends); reported in the
           "prefill_config3" object.
  decoder  config 5: random-init 24-layer all-KVM decoder (d_model 2048,
           16 heads of 128, vocab 65536, chunk 512, 512 fixed slots):
           prefill 16384 random token ids at batch 8, then greedy decode
           (`--e2e-decode` steps); reported in the "decoder_e2e" object.

Prints ONE JSON line: value = prefill tokens/s; the decode figures are in
the "decode" object.  roofline: achieved algorithmic FLOP/s of the prefill's
dominant kernel (by event time: the update chain or the attention; both, and
the whole path, are in roofline.per_kernel / roofline.whole_path) against
the bf16 MFMA peak, and bytes/s of the decode attention against HBM, all
timed with HIP events on the launch stream.  --evict also times every
prefill after streaming 512 MiB (the reference's cache-eviction protocol).
cpu_baseline: the CPU oracle (an eager
restatement of the reference, pinned to it by golden fixtures) on a bounded
sample of the prefill workload.
"""

from __future__ import annotations

import argparse
import gc
import json
import math
import os
import sys
import time
from pathlib import Path
from types import SimpleNamespace

ROOT = Path(__file__).resolve().parent
for _p in (ROOT, ROOT / "kvm-paper_amd"):
    if str(_p) not in sys.path:
        sys.path.insert(0, str(_p))

PEAK_BF16_FLOPS = 2.5e15   # MI355X dense bf16 MFMA
PEAK_HBM_BYTES = 8.0e12    # MI355X HBM3E


def measured_traffic(kernel, workload):
    """HBM bytes per launch of `kernel` on `workload` as the committed
    rocprofv3 FETCH_SIZE/WRITE_SIZE runs measured them (scaled by the
    plain-copy calibration), or None when no such measurement is recorded."""
    path = ROOT / "profiles" / "hbm_traffic.txt"
    if not path.exists():
        return None
    for line in path.read_text().splitlines():
        f = line.split()
        if len(f) == 4 and not line.startswith("#") and f[0] == kernel and f[1] == workload:
            return int(f[2]) + int(f[3])
    return None


def _config(Hq, Hkv, D, C, n_bswa, min_len, n_max, mode="fixed", factor=1.0):
    return SimpleNamespace(
        num_attention_heads=Hq, num_key_value_heads=Hkv, hidden_size=Hq * D, d_qk_head=D, d_v_head=D,
        d_head=None, num_hidden_layers=1, mup_base_dim=Hq * D, use_tokenshift_att=0, use_value_residual=0,
        kvm_value_residual_mode="rwkv", kvm_token_shift_mode="rwkv", rope_partial_dim=64, sink_len=1,
        chunk_len=C, n_max_d_chunks=n_max, n_bswa_chunks=n_bswa, state_budget_mode=mode,
        state_growth_factor=factor, state_growth_exponent=0.5, state_round_down=1, state_min_len=min_len,
        state_saturation_n=None, kvm_use_merge_gate_keys=1, kvm_use_merge_gate_values=1,
        kvm_apply_merge_gate_to_appends=0, kvm_apply_merge_gate_to_initial_state=0, kvm_use_head_temps=1,
        kvm_use_vlens=1, kvm_aotriton_forward_attention=0,
    )


def attention_pairs(plan, n_bswa):
    """Sum over queries of visible keys (state slots + window, causal)."""
    C, T = plan.chunk_len, plan.seq_len
    total = 0
    for m in range(plan.n_chunks):
        qb, qe = m * C, min(T, (m + 1) * C)
        S = plan.chunk_state_len[m]
        wb = max(0, (m - n_bswa + 1) * C)
        L = qe - qb
        # query t sees S + (t - wb + 1) keys
        total += L * S + sum(t - wb + 1 for t in (qb, qe - 1)) * L // 2
    return total


def routing_pairs(plan):
    return sum(plan.chunk_len * (b + a) for b, a in zip(plan.upd_state_before, plan.upd_n_append))


def bench_prefill(args, torch, kvm_amd):
    B, H, D, T, C = 1, 32, 128, 32768, 512
    cfg = _config(H, H, D, C, 2, 256, 1)
    dev = torch.device("cuda:0")
    mixer = kvm_amd.SequenceMixer(cfg, 0).to(dev, torch.bfloat16).eval()
    gen = torch.Generator(device=dev).manual_seed(0)
    q = torch.randn(B, H, T, D, generator=gen, device=dev, dtype=torch.float32).div_(math.sqrt(D)).bfloat16()
    k = torch.randn(B, H, T, D, generator=gen, device=dev, dtype=torch.float32).div_(math.sqrt(D)).bfloat16()
    v = torch.randn(B, H, T, D, generator=gen, device=dev, dtype=torch.float32).div_(math.sqrt(D)).bfloat16()
    g = (1 + torch.nn.functional.elu(torch.randn(B, H, T, 1, generator=gen, device=dev))).bfloat16()
    plan = mixer.make_plan(T)
    with torch.no_grad():
        for _ in range(args.warmup):
            mixer.prefill_raw(q, k, v, g, plan=plan)
        torch.cuda.synchronize()
        # Timed steps: one event pair around all of them, nothing inside.  The
        # device status word is sticky, so it is read once after the timed
        # steps (a failed update chain raises there).
        start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        start.record()
        for i in range(args.steps):
            mixer.prefill_raw(q, k, v, g, plan=plan, check_status=False)
        end.record()
        torch.cuda.synchronize()
        wall = time.perf_counter() - t0
        mixer.check_prefill_status()
        # Breakdown (update chain, attention launches) from separate steps whose
        # events kvm_prefill records on its launch stream.
        evs = [[torch.cuda.Event(enable_timing=True) for _ in range(4)] for _ in range(args.steps)]
        for e in evs:  # every event recorded once, whatever kvm_prefill marks
            for x in e:
                x.record()
        for i in range(args.steps):
            mixer.prefill_raw(q, k, v, g, plan=plan, events=evs[i], check_status=False)
        torch.cuda.synchronize()
        mixer.check_prefill_status()
        # Optional cache-evicting timing (the reference's protocol,
        # scripts/kvm_benchmark/common.py:283-295): a 512 MiB buffer is
        # streamed before every timed prefill, outside its event pair.
        evict_ms = None
        if getattr(args, "evict", False):
            flush = torch.empty(512 << 20, dtype=torch.uint8, device=dev)
            pairs = []
            for i in range(args.steps):
                flush.add_(1)
                a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                a.record()
                mixer.prefill_raw(q, k, v, g, plan=plan, check_status=False)
                b.record()
                pairs.append((a, b))
            torch.cuda.synchronize()
            mixer.check_prefill_status()
            evict_ms = sum(a.elapsed_time(b) for a, b in pairs) / args.steps
            del flush
    ms = start.elapsed_time(end) / args.steps
    attn_ms = sum(e[2].elapsed_time(e[3]) for e in evs) / args.steps
    chain_ms = sum(e[0].elapsed_time(e[1]) for e in evs) / args.steps
    attn_flop = 4 * D * H * B * attention_pairs(plan, 2)
    route_flop = 2 * D * H * B * routing_pairs(plan)
    return dict(
        ms=ms, wall_ms=wall * 1e3 / args.steps, tok_s=B * T / (ms * 1e-3), attn_ms=attn_ms, chain_ms=chain_ms,
        evict_ms=evict_ms,
        attn_flop=attn_flop, route_flop=route_flop, plan=plan, inputs=(q, k, v, g), mixer=mixer,
    )


def bench_prefill_config3(args, torch, kvm_amd):
    """B2 H16 D128 T65536 C512, slots floor(sqrt(tokens seen)) capped at 1024 (the reference's
    power-law budget floors, model/kvm_mixer.py:141-147; BASELINE.json writes ceil)
    (power-law budget, n_max_d_chunks 2), 10 % of the keys drawn from 8 shared centres.  As
    written the budget never passes the 512 slots the first chunk fills ("literal": 125 updates,
    no appends); the growth variant (factor 16) grows the state 512 -> 1024 through appends."""
    B, H, D, T, C = 2, 16, 128, 65536, 512
    dev = torch.device("cuda:0")
    gen = torch.Generator(device=dev).manual_seed(3)
    q = (torch.randn(B, H, T, D, generator=gen, device=dev) / math.sqrt(D)).bfloat16()
    kf = torch.randn(B, H, T, D, generator=gen, device=dev)
    centres = torch.randn(8, D, generator=gen, device=dev)
    pick = torch.randint(0, 8, (B, H, T), generator=gen, device=dev)
    sel = torch.rand(B, H, T, generator=gen, device=dev) < 0.1
    kf = torch.where(sel.unsqueeze(-1), centres[pick] + 0.05 * torch.randn(B, H, T, D, generator=gen, device=dev),
                     kf)
    k = (kf / math.sqrt(D)).bfloat16()
    del kf
    v = (torch.randn(B, H, T, D, generator=gen, device=dev) / math.sqrt(D)).bfloat16()
    g = (1 + torch.nn.functional.elu(torch.randn(B, H, T, 1, generator=gen, device=dev))).bfloat16()
    out = {}
    for name, factor in (("literal", 1.0), ("growth_f16", 16.0)):
        mixer = kvm_amd.SequenceMixer(_config(H, H, D, C, 2, C, 2, "power_law", factor), 0).to(dev, torch.bfloat16)
        mixer.eval()
        plan = mixer.make_plan(T)
        with torch.no_grad():
            for _ in range(args.warmup):
                mixer.prefill_raw(q, k, v, g, plan=plan)
            torch.cuda.synchronize()
            start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            start.record()
            for _ in range(args.steps):
                mixer.prefill_raw(q, k, v, g, plan=plan, check_status=False)
            end.record()
            torch.cuda.synchronize()
            mixer.check_prefill_status()
        ms = start.elapsed_time(end) / args.steps
        flop = 4 * D * H * B * attention_pairs(plan, 2) + 2 * D * H * B * routing_pairs(plan)
        out[name] = {"ms_per_step": round(ms, 3), "tokens_per_s": round(B * T / (ms * 1e-3), 1),
                     "updates": plan.n_updates, "final_slots": plan.final_state_len,
                     "appended_per_row": int(sum(plan.upd_n_append)), "algorithmic_flop": flop,
                     "frac_of_mfma_peak": round(flop / (ms * 1e-3) / 2.5e15, 4)}
        del mixer
    return out


def bench_backward(args, torch, kvm_amd, pf):
    """Config 2 training step of the KVM layer at the post-QKV boundary: the
    differentiable prefill (routes fixed by the forward) and its backward.
    Reports the whole step and the HIP attention backward alone."""
    from kvm_amd import training

    mixer = pf["mixer"]
    q, k, v, g = (x.detach().requires_grad_(True) for x in pf["inputs"])
    B, H, T, D = q.shape
    dout = (torch.randn(B, T, H, D, device=q.device) * 0.05).bfloat16()
    for p in mixer.parameters():
        p.requires_grad_(True)

    params = [q, k, v, g, *mixer.parameters()]

    def step():
        for t in params:  # zero_grad(set_to_none=True), as an optimizer step leaves them
            t.grad = None
        y = training.prefill_with_grad(mixer, q, k, v, g)
        y.backward(dout)

    step()
    torch.cuda.synchronize()
    steps = max(1, min(args.steps, 3))
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(steps):
        step()
    e1.record()
    torch.cuda.synchronize()
    step_ms = e0.elapsed_time(e1) / steps
    with torch.no_grad():
        res = mixer.prefill_raw(q, k, v, g, route_log=True, keep_snapshots=True, want_lse=True)
        a0, a1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a0.record()
        for _ in range(steps):
            training.attention_backward(mixer, q, k, v, g, res, dout)
        a1.record()
        torch.cuda.synchronize()
    return dict(step_ms=step_ms, attn_bwd_ms=a0.elapsed_time(a1) / steps, steps=steps)


def bench_decode(args, torch, kvm_amd):
    B, H, D, C, n = 64, 32, 128, 256, 2
    S, total = 1024, 131072
    W = n * C
    cfg = _config(H, H, D, C, n, S, 4)
    dev = torch.device("cuda:0")
    mixer = kvm_amd.SequenceMixer(cfg, 0).to(dev, torch.bfloat16).eval()
    gen = torch.Generator(device=dev).manual_seed(1)
    cnt = torch.randint(1, 4097, (B, H, S, 1), generator=gen, device=dev).float()
    mean_k = torch.randn(B, H, S, D, generator=gen, device=dev) * math.sqrt(0.5)
    mean_v = torch.randn(B, H, S, D, generator=gen, device=dev) * math.sqrt(0.5)
    begin = max(0, (total + C - 1) // C * C - W)
    R = total - begin
    snap = kvm_amd.DecodeCacheSnapshot(
        state_k=(mean_k * cnt).bfloat16(), state_v=(mean_v * cnt).bfloat16(),
        state_vlen=mean_v.norm(dim=-1, keepdim=True),
        recent_k=(torch.randn(B, H, R, D, generator=gen, device=dev) / math.sqrt(D)).bfloat16(),
        recent_v=(torch.randn(B, H, R, D, generator=gen, device=dev) / math.sqrt(D)).bfloat16(),
        recent_gate=(1 + torch.nn.functional.elu(torch.randn(B, H, R, 1, generator=gen, device=dev))).bfloat16(),
        total_len=total, state_coverage_len=max(min(total, C), begin), recent_begin=begin,
    )
    steps = args.decode_steps
    qs = (torch.randn(steps, B, H, 1, D, generator=gen, device=dev) / math.sqrt(D)).bfloat16()
    ks = (torch.randn(steps, B, H, 1, D, generator=gen, device=dev) / math.sqrt(D)).bfloat16()
    vs = (torch.randn(steps, B, H, 1, D, generator=gen, device=dev) / math.sqrt(D)).bfloat16()
    gs = (1 + torch.nn.functional.elu(torch.randn(steps, B, H, 1, 1, generator=gen, device=dev))).bfloat16()
    cache = mixer.make_decode_cache(snap, state_capacity=S)

    def run(inner):
        """One event pair per token (the reference's protocol); with `inner`,
        a second pair around each attention launch (for the attention time)."""
        cache.reset_(snap)
        torch.cuda.synchronize()
        ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(steps)]
        ea = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(steps)]
        for i in range(steps):
            ev[i][0].record()
            # The token's ring row is written by the attention launch
            # (kvm_decode_step), as in the mixer's own decode step.
            fresh = mixer._decode_advance(ks[i], vs[i], gs[i], cache, defer_ring_write=True)
            if inner:
                ea[i][0].record()
            mixer._decode_attention(qs[i], cache, fresh)
            if inner:
                ea[i][1].record()
            ev[i][1].record()
        torch.cuda.synchronize()
        return ev, ea

    with torch.no_grad():
        for _ in range(max(1, args.warmup)):
            run(False)
        ev, _ = run(False)
        _, ea = run(True)
    step_ms = [a.elapsed_time(b) for a, b in ev]
    attn_ms = [a.elapsed_time(b) for a, b in ea]
    total_ms = sum(step_ms)
    rows = B * H
    # Algorithmic bytes per attention launch: each key and value row read
    # once, q read and out written, and the token's ring row (k, v, gate) written.
    active = S
    bytes_per = []
    for i in range(steps):
        t = total + 1 + i
        rb = max(0, (t + C - 1) // C * C - W)
        bytes_per.append(rows * (active + (t - rb)) * (2 * D) * 2 + 2 * rows * D * 2 + rows * (2 * D + 1) * 2)
    return dict(
        ms_per_step=total_ms / steps, tok_s=B * steps / (total_ms * 1e-3), attn_ms=sum(attn_ms) / steps,
        bytes=sum(bytes_per) / steps, update_step_ms=step_ms[0], other_step_ms=sum(step_ms[1:]) / max(steps - 1, 1),
        steps=steps,
    )


def bench_e2e(args, torch, kvm_amd):
    """Config 5: random-init 24-layer all-KVM decoder (d_model 2048, 16 heads
    of 128, vocab 65536, bf16, chunk 512, 512 fixed slots); prefill 16384
    random token ids at batch 8, then greedy decode.  One untimed warm-up
    (prefill + 8 decode steps), then the timed prefill and decode, then two
    more timed prefills: the reported prefill is the median of the three."""
    from kvm_amd.backbone import DecodeGraph, MixerConfig, RWKV7BackboneForCausalLM, StatesDictCache, init_random_

    # The earlier workloads' cached allocator blocks are returned first, so
    # that the decoder's buffers are laid out as in a process of its own.
    torch.cuda.empty_cache()
    cfg = MixerConfig(vocab_size=65536, num_hidden_layers=24, num_attention_heads=16, hidden_size=2048,
                      mup_base_dim=2048, use_tokenshift_att=1, use_tokenshift_ffn=1, residual_scale=0.5,
                      rope_partial_dim=64, chunk_len=512, n_bswa_chunks=2, state_min_len=512,
                      state_budget_mode="fixed", sink_len=1)
    with torch.device("meta"):
        model = RWKV7BackboneForCausalLM(cfg)
    model = init_random_(model.to_empty(device="cuda").to(torch.bfloat16), 0).eval()
    B, T, n_dec = 8, 16384, args.e2e_decode
    gen = torch.Generator(device="cuda").manual_seed(1)
    ids = torch.randint(0, cfg.vocab_size, (B, T), device="cuda", generator=gen)

    def run(n, graph):
        # The previous run's cache and HIP graph are released here, outside
        # the timed region, not by a garbage collection inside it.
        gc.collect()
        cache = StatesDictCache()
        e = [torch.cuda.Event(enable_timing=True) for _ in range(3)]
        torch.cuda.synchronize()
        e[0].record()
        lg = model(input_ids=ids, past_key_values=cache, use_cache=True,
                   cache_position=torch.arange(T, device="cuda"), logits_to_keep=1).logits[:, -1]
        e[1].record()
        runner = DecodeGraph(model, cache) if graph else None
        for s in range(n):
            tok = lg.argmax(-1)
            if runner is not None:
                lg = runner.step(tok)
            else:
                lg = model(input_ids=tok[:, None], past_key_values=cache, use_cache=True,
                           cache_position=torch.tensor([T + s]), logits_to_keep=1).logits[:, -1]
        e[2].record()
        torch.cuda.synchronize()
        if runner is not None:
            runner.close()
        return e[0].elapsed_time(e[1]), e[1].elapsed_time(e[2])

    def breakdown():
        """One more prefill with HIP events around each stage of every layer
        (separate from the timed run): the mixer's projections + fused
        prefix, its KVM prefill (update chain / per-update kernels, then the
        attention launches, from kvm_prefill's own event marks), its output
        projection (the rest of the mixer), the MLP (hipBLASLt GEMMs +
        relu^2) and the fused residual-add + LayerNorm launches; "other" is
        the rest of the prefill (embedding, LM head on the last token)."""
        import kvm_amd.backbone as bb

        rec = {k: [] for k in ("mixer", "prefix", "kvm", "mlp", "add_norm")}
        ev = lambda: torch.cuda.Event(enable_timing=True)  # noqa: E731

        def timed(fn, key):
            def w(*a, **kw):
                e0, e1 = ev(), ev()
                e0.record()
                r = fn(*a, **kw)
                e1.record()
                rec[key].append((e0, e1))
                return r
            return w

        def kvm_timed(fn):
            def w(*a, **kw):
                es = [ev() for _ in range(4)]
                for e in es:  # every event recorded once, whatever the call marks
                    e.record()
                kw["events"] = es
                r = fn(*a, **kw)
                rec["kvm"].append(es)
                return r
            return w

        saved_add_norm = bb._add_norm
        for blk in model.transformer.h:
            m = blk.attn
            m.forward_inference = timed(m.forward_inference, "mixer")
            m.forward_prefix = timed(m.forward_prefix, "prefix")
            m.prefill_raw = kvm_timed(m.prefill_raw)
            blk.mlp.ffn = timed(blk.mlp.ffn, "mlp")
        bb._add_norm = timed(saved_add_norm, "add_norm")
        try:
            cache = StatesDictCache()
            e0, e1 = ev(), ev()
            torch.cuda.synchronize()
            e0.record()
            model(input_ids=ids, past_key_values=cache, use_cache=True,
                  cache_position=torch.arange(T, device="cuda"), logits_to_keep=1)
            e1.record()
            torch.cuda.synchronize()
        finally:
            bb._add_norm = saved_add_norm
            for blk in model.transformer.h:
                for name in ("forward_inference", "forward_prefix", "prefill_raw"):
                    blk.attn.__dict__.pop(name, None)
                blk.mlp.__dict__.pop("ffn", None)
        tot = lambda key: sum(a.elapsed_time(b) for a, b in rec[key])  # noqa: E731
        upd = sum(es[0].elapsed_time(es[1]) for es in rec["kvm"])
        att = sum(es[2].elapsed_time(es[3]) for es in rec["kvm"])
        total = e0.elapsed_time(e1)
        mixer, prefix, mlp, an = tot("mixer"), tot("prefix"), tot("mlp"), tot("add_norm")
        return {"total": total, "mixer_projections_and_prefix": prefix, "kvm_updates": upd,
                "kvm_attention": att, "mixer_output_projection_and_rest": mixer - prefix - upd - att,
                "mlp": mlp, "add_norm": an, "other": total - mixer - mlp - an}

    n_eager = min(n_dec, args.e2e_eager_steps)
    with torch.no_grad():
        run(8, True)
        pre_ms, dec_ms = run(n_dec, True)
        # Two more prefills alone: the reported prefill is the median of three.
        pre_samples = [pre_ms] + [run(0, False)[0] for _ in range(2)]
        pre_ms = sorted(pre_samples)[1]
        eager_ms = run(n_eager, False)[1] if n_eager > 0 else None
        stages = breakdown()
    del model
    torch.cuda.empty_cache()
    return dict(prefill_ms=pre_ms, prefill_samples_ms=[round(x, 2) for x in pre_samples],
                prefill_tok_s=B * T / (pre_ms * 1e-3), decode_ms_per_step=dec_ms / n_dec,
                decode_tok_s=B * n_dec / (dec_ms * 1e-3), decode_steps=n_dec, decode_path="hip_graph",
                eager_decode_ms_per_step=eager_ms / n_eager if n_eager > 0 else None, prefill_stages_ms=stages)


def _cpu_prefill_inputs(torch, B, H, D, T, dtype, seed):
    gen = torch.Generator().manual_seed(seed)
    q = (torch.randn(B, H, T, D, generator=gen) / math.sqrt(D)).to(dtype)
    k = (torch.randn(B, H, T, D, generator=gen) / math.sqrt(D)).to(dtype)
    v = (torch.randn(B, H, T, D, generator=gen) / math.sqrt(D)).to(dtype)
    g = (1 + torch.nn.functional.elu(torch.randn(B, H, T, 1, generator=gen))).to(dtype)
    return q, k, v, g


def _time_cpu(fn, runs=3):
    """One untimed warm-up, then the median of `runs` timed calls (seconds)."""
    fn()
    times = []
    for _ in range(runs):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    return sorted(times)[len(times) // 2], times


def cpu_baseline(torch, sample_T):
    """The CPU oracle (eager restatement of model/kvm_mixer.py with fp32
    routing) on the host cores of this process: the first sample_T tokens of
    the config-2 prefill (bf16), and BASELINE config 1 (fp32, B1 H4 D64
    T4096 C256, 64 configured slots -> 256 effective, rope_partial_dim 32)."""
    from oracle import kvm_oracle as O

    threads = len(os.sched_getaffinity(0))
    torch.set_num_threads(threads)

    def params(D, H, dtype):
        return O.OracleParams(ln_weight=torch.ones(D).to(dtype), ln_bias=torch.zeros(D).to(dtype),
                              front_temp=torch.ones(H).to(dtype), state_temp=torch.ones(H).to(dtype))

    B, H, D, C = 1, 32, 128, 512
    x2 = _cpu_prefill_inputs(torch, B, H, D, sample_T, torch.bfloat16, 0)
    cfg2 = O.OracleConfig(q_heads=H, kv_heads=H, head_dim=D, value_dim=D, chunk_len=C, n_bswa_chunks=2,
                          sink_len=1, rope_partial_dim=64, state_min_len=256)
    p2 = params(D, H, torch.bfloat16)
    sec2, all2 = _time_cpu(lambda: O.prefill(*x2, p2, cfg2))
    x1 = _cpu_prefill_inputs(torch, 1, 4, 64, 4096, torch.float32, 0)
    cfg1 = O.OracleConfig(q_heads=4, kv_heads=4, head_dim=64, value_dim=64, chunk_len=256, n_bswa_chunks=2,
                          sink_len=1, rope_partial_dim=32, state_min_len=64)
    p1 = params(64, 4, torch.float32)
    sec1, all1 = _time_cpu(lambda: O.prefill(*x1, p1, cfg1))
    quota = None
    try:
        q_, per = open("/sys/fs/cgroup/cpu.max").read().split()[:2]
        quota = None if q_ == "max" else round(int(q_) / int(per), 2)
    except (OSError, ValueError):
        pass
    return dict(value=B * sample_T / sec2, unit="tokens/s", cores=threads, kind="port",
                sample=f"CPU oracle (eager restatement of model/kvm_mixer.py, fp32 routing) prefill of "
                       f"{sample_T} tokens of the config-2 layer (B1 H32 D128 C512, 512 slots, bf16) on "
                       f"{threads} threads (all cores in this process's affinity): 1 warm-up, median of "
                       f"3 runs {sec2:.2f} s (runs {', '.join(f'{t:.2f}' for t in all2)} s)",
                host={"affinity_cpus": threads, "os_cpu_count": os.cpu_count(), "cgroup_cpu_quota": quota,
                      "omp_num_threads": os.environ.get("OMP_NUM_THREADS")},
                config1={"value": 4096 / sec1, "unit": "tokens/s", "dtype": "f32", "seconds": round(sec1, 4),
                         "sample": "BASELINE config 1 whole: B1 H4 D64 T4096 C256 fp32, 64 configured slots "
                                   "(256 effective), rope_partial_dim 32; 1 warm-up, median of 3"})


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=30)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--decode-steps", type=int, default=256)
    ap.add_argument("--cpu-sample", type=int, default=32768,
                    help="tokens of the prefill workload the CPU baseline runs (default: all)")
    ap.add_argument("--skip-cpu", action="store_true")
    ap.add_argument("--skip-decode", action="store_true")
    ap.add_argument("--skip-e2e", action="store_true")
    ap.add_argument("--skip-backward", action="store_true")
    ap.add_argument("--skip-config3", action="store_true")
    ap.add_argument("--e2e-decode", type=int, default=512,
                    help="greedy decode steps of the config-5 decoder run (default 512)")
    ap.add_argument("--e2e-eager-steps", type=int, default=64,
                    help="decode steps of the config-5 decoder also run without the HIP graph, "
                         "for comparison (default 64; 0 skips)")
    ap.add_argument("--only", choices=["prefill", "decode", "copy", "e2e", "backward", "config3"], default=None,
                    help="run one workload (profiling); 'copy' streams a known number of bytes "
                         "through a plain device copy to calibrate the FETCH_SIZE/WRITE_SIZE counters")
    ap.add_argument("--copy-mib", type=int, default=1024)
    ap.add_argument("--evict", action="store_true",
                    help="also time every prefill after streaming 512 MiB through the caches (the reference's "
                         "protocol); reported as prefill.evicted_ms_per_step")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU: this build has no multi-GPU path (asked for --gpus {args.gpus}).",
              file=sys.stderr)
        sys.exit(2)
    import torch
    import kvm_amd

    kvm_amd.load_library()
    if args.only == "copy":
        n = args.copy_mib << 19  # bf16 elements
        src = torch.randn(n, device="cuda:0").bfloat16()
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_bytes_read": 2 * n, "copy_bytes_written": 2 * n, "launches": 3}))
        return
    if args.only == "e2e":
        print(json.dumps(bench_e2e(args, torch, kvm_amd)))
        return
    if args.only == "config3":
        print(json.dumps(bench_prefill_config3(args, torch, kvm_amd)))
        return
    if args.only == "decode":
        dec = bench_decode(args, torch, kvm_amd)
        print(json.dumps({k: v for k, v in dec.items()}))
        return
    print("bench: prefill config 2 ...", file=sys.stderr, flush=True)
    pf = bench_prefill(args, torch, kvm_amd)
    if args.only == "prefill":
        print(json.dumps({"ms": pf["ms"], "attention_ms": pf["attn_ms"], "chain_ms": pf["chain_ms"],
                          "evicted_ms": pf["evict_ms"]}))
        return
    if args.only == "backward":
        print(json.dumps(bench_backward(args, torch, kvm_amd, pf)))
        return
    print(f"bench: prefill {pf['ms']:.3f} ms/step (attention {pf['attn_ms']:.3f} ms, updates {pf['chain_ms']:.3f} ms)",
          file=sys.stderr, flush=True)
    bwd = None
    if not args.skip_backward:
        print("bench: config 2 training step (differentiable prefill + backward) ...", file=sys.stderr, flush=True)
        bwd = bench_backward(args, torch, kvm_amd, pf)
        print(f"bench: training step {bwd['step_ms']:.2f} ms (HIP attention backward {bwd['attn_bwd_ms']:.2f} ms)",
              file=sys.stderr, flush=True)
    pf3 = None
    if not args.skip_config3:
        print("bench: prefill config 3 (growable memory, two budgets) ...", file=sys.stderr, flush=True)
        pf3 = bench_prefill_config3(args, torch, kvm_amd)
        print("bench: config 3 " + ", ".join(f"{k} {v['ms_per_step']:.2f} ms" for k, v in pf3.items()),
              file=sys.stderr, flush=True)
    dec = None
    if not args.skip_decode:
        print("bench: decode config 4 ...", file=sys.stderr, flush=True)
        dec = bench_decode(args, torch, kvm_amd)
        print(f"bench: decode {dec['ms_per_step']:.3f} ms/token-step (attention {dec['attn_ms']:.3f} ms)",
              file=sys.stderr, flush=True)
    e2e = None
    if not args.skip_e2e:
        print("bench: config 5 decoder (24 layers, B8 T16384 prefill + greedy decode) ...", file=sys.stderr, flush=True)
        e2e = bench_e2e(args, torch, kvm_amd)
        print(f"bench: decoder prefill {e2e['prefill_ms']:.1f} ms, decode {e2e['decode_ms_per_step']:.2f} ms/step",
              file=sys.stderr, flush=True)
    cpu = None
    if not args.skip_cpu:
        print("bench: cpu baseline ...", file=sys.stderr, flush=True)
        cpu = cpu_baseline(torch, args.cpu_sample)
    # Per-kernel rooflines of the prefill (algorithmic FLOP of the launch over
    # its event time), the dominant kernel's as the line's `roofline`, and
    # the whole path's.
    attn_achieved = pf["attn_flop"] / (pf["attn_ms"] * 1e-3)
    chain_achieved = pf["route_flop"] / (pf["chain_ms"] * 1e-3)
    path_achieved = (pf["attn_flop"] + pf["route_flop"]) / (pf["ms"] * 1e-3)
    per_kernel = {
        "k_attn_prefill": {"bound": "mfma", "ms": round(pf["attn_ms"], 4), "flop": pf["attn_flop"],
                           "achieved": round(attn_achieved / 1e12, 2), "frac": round(attn_achieved / PEAK_BF16_FLOPS, 4),
                           "traffic": measured_traffic("k_attn_prefill", "config2")},
        "k_chain_fixed": {"bound": "mfma (latency of the update recurrence in practice)", "ms": round(pf["chain_ms"], 4),
                          "flop": pf["route_flop"], "achieved": round(chain_achieved / 1e12, 2),
                          "frac": round(chain_achieved / PEAK_BF16_FLOPS, 4),
                          "traffic": measured_traffic("k_chain_fixed", "config2")},
    }
    dominant = max(per_kernel, key=lambda n: per_kernel[n]["ms"])
    dk = per_kernel[dominant]
    line = {
        "metric": "KVM prefill tokens/s @32K and decode tokens/s @128K; % MFMA/HBM roofline",
        "value": round(pf["tok_s"], 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(pf["ms"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded Gaussian q/k/v, 1+elu gates; random-init layer parameters)",
        "config": {"workload": "config 2: KVM layer prefill B1 H32 D128 T32768 C512 fixed memory (512 live slots)",
                   "global_batch": 1, "seq_len": 32768, "parallelism": "none (1 GPU)"},
        "prefill": {
            "ms_per_step": round(pf["ms"], 4), "attention_ms": round(pf["attn_ms"], 4),
            "update_chain_ms": round(pf["chain_ms"], 4), "algorithmic_flop": pf["attn_flop"] + pf["route_flop"],
            "attention_flop": pf["attn_flop"], "routing_flop": pf["route_flop"],
            "whole_path_frac_of_mfma_peak": round((pf["attn_flop"] + pf["route_flop"]) / (pf["ms"] * 1e-3) / PEAK_BF16_FLOPS, 4),
        },
        "roofline": {
            "bound": "mfma", "kernel": dominant, "achieved": dk["achieved"],
            "peak": PEAK_BF16_FLOPS / 1e12, "unit": "TFLOP/s", "frac": dk["frac"], "traffic": dk["traffic"],
            "per_kernel": per_kernel,
            "whole_path": {"achieved": round(path_achieved / 1e12, 2), "frac": round(path_achieved / PEAK_BF16_FLOPS, 4),
                           "ms": round(pf["ms"], 4), "flop": pf["attn_flop"] + pf["route_flop"]},
        },
    }
    if pf["evict_ms"] is not None:
        line["prefill"]["evicted_ms_per_step"] = round(pf["evict_ms"], 4)
        line["prefill"]["evicted_tokens_per_s"] = round(32768 / (pf["evict_ms"] * 1e-3), 1)
    if dec is not None:
        bw = dec["bytes"] / (dec["attn_ms"] * 1e-3)
        line["decode"] = {
            "workload": "config 4: B64 H32 D128, 1024 slots + 512-token window at 128K context, "
                        f"{dec['steps']} tokens from a fresh snapshot (one state update included)",
            "value": round(dec["tok_s"], 1), "unit": "tokens/s", "ms_per_step": round(dec["ms_per_step"], 4),
            "attention_ms": round(dec["attn_ms"], 4), "update_step_ms": round(dec["update_step_ms"], 4),
            "other_step_ms": round(dec["other_step_ms"], 4),
            "roofline": {"bound": "hbm", "kernel": "k_decode_partial+k_decode_combine",
                         "achieved": round(bw / 1e9, 1), "peak": PEAK_HBM_BYTES / 1e9, "unit": "GB/s",
                         "frac": round(bw / PEAK_HBM_BYTES, 4),
                         "traffic": measured_traffic("k_decode_partial", "config4")},
        }
    if bwd is not None:
        line["backward"] = {
            "workload": "config 2 training step of the KVM layer at the post-QKV boundary: differentiable "
                        "prefill (routes fixed by the forward) + backward of q, k, v, gate, ln_s_k and the "
                        "head temperatures",
            "step_ms": round(bwd["step_ms"], 3), "attention_backward_ms": round(bwd["attn_bwd_ms"], 3),
            "tokens_per_s": round(32768 / (bwd["step_ms"] * 1e-3), 1),
        }
    if pf3 is not None:
        line["prefill_config3"] = {
            "workload": "config 3: KVM layer prefill B2 H16 D128 T65536 C512, floor(sqrt(tokens seen)) slots (the reference's power-law budget) capped at 1024, "
                        "10% of keys from 8 shared centres; 'literal' is the budget as written (never passes the "
                        "512 slots of the first chunk), 'growth_f16' grows 512 -> 1024 slots through appends",
            **pf3,
        }
    if e2e is not None:
        line["decoder_e2e"] = {
            "workload": "config 5: random-init 24-layer all-KVM decoder, d_model 2048, 16 heads of 128, vocab 65536, "
                        f"bf16, chunk 512, 512 fixed slots; prefill 16384 random token ids at batch 8, then "
                        f"{e2e['decode_steps']} greedy decode steps replayed from a HIP graph (projections, MLP "
                        "and LM head: hipBLASLt in the prefill, kvm_gemm_small in decode)",
            "prefill_tokens_per_s": round(e2e["prefill_tok_s"], 1), "prefill_ms": round(e2e["prefill_ms"], 2),
            "prefill_samples_ms": e2e["prefill_samples_ms"],
            "decode_tokens_per_s": round(e2e["decode_tok_s"], 1),
            "decode_ms_per_step": round(e2e["decode_ms_per_step"], 3),
            "decode_path": e2e["decode_path"],
            "eager_decode_ms_per_step": (round(e2e["eager_decode_ms_per_step"], 3)
                                         if e2e["eager_decode_ms_per_step"] is not None else None),
            "prefill_stages_ms": {k: round(v, 2) for k, v in e2e["prefill_stages_ms"].items()},
        }
    line["cpu_baseline"] = cpu
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
