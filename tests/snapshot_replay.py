"""Torch restatement of the memory snapshots a prefill's attention reads,
rebuilt in fp32 from the tokens and the forward's routes: the reference the
HIP state backward (kvm_state_backward) is tested against.  Test
infrastructure only; the product never imports it."""

from __future__ import annotations

import torch
import torch.nn.functional as F


def replay_snapshot_rows(k, v, gate, ln_w, ln_b, plan, route_log, append_log, cfg):
    """Attention rows of every snapshot, rebuilt in fp32 from the tokens and
    the forward's routes (differentiable in k, v, gate, ln_w, ln_b).

    k, v: [rows, T, D]; gate: [rows, T]; route_log / append_log:
    [n_updates, rows, C] (slot of every overflow token; 1 if appended).
    ``cfg`` carries eps, rope_partial_dim, gate_keys, gate_values,
    gate_appends, gate_initial.  Returns a list of (k_rows, v_rows), one per
    snapshot, each [rows, S_snapshot, D].  The state follows
    model/kvm_mixer.py:434-447 (initial state), :231-248 (append) and
    :321-340 (merge sums) with the routes given.
    """
    rows, T, D = k.shape
    C = plan.chunk_len
    r = int(cfg["rope_partial_dim"])
    kz = torch.cat([torch.zeros_like(k[..., :r]), k[..., r:]], dim=-1)
    prep = F.layer_norm(kz, (D,), ln_w, ln_b, cfg["eps"])
    g = gate.unsqueeze(-1)
    gk = prep * g if cfg["gate_keys"] else prep
    gv = v * g if cfg["gate_values"] else v
    ak, av = (gk, gv) if cfg["gate_appends"] else (prep, v)

    def attn_rows(s_k, s_v, vlen):
        return (F.layer_norm(s_k, (D,), ln_w, ln_b, cfg["eps"]),
                F.normalize(s_v, dim=-1) * vlen.unsqueeze(-1))

    L0 = plan.initial_state_len
    s_k = (prep * g if cfg["gate_initial"] else prep)[:, :L0]
    s_v = (v * g if cfg["gate_initial"] else v)[:, :L0]
    vlen = v[:, :L0].norm(dim=-1)
    snaps = [attn_rows(s_k, s_v, vlen)]
    ridx = torch.arange(rows, device=k.device).unsqueeze(1)
    for u in range(plan.n_updates):
        tb, before, n_app = plan.upd_token_begin[u], plan.upd_state_before[u], plan.upd_n_append[u]
        route = route_log[u].long()                 # [rows, C]
        app = append_log[u].bool()
        after = before + n_app
        if n_app:
            # Appended tokens take slots before .. after - 1 in token order.
            tok = app.nonzero()[:, 1].view(rows, n_app) + tb
            new_k = ak[ridx, tok]
            new_v = av[ridx, tok]
            s_k = torch.cat([s_k, new_k], dim=1)
            s_v = torch.cat([s_v, new_v], dim=1)
            vlen = torch.cat([vlen, new_v.norm(dim=-1)], dim=1)
        merged = ~app
        flat = (ridx * after + route).masked_select(merged)
        tok_rows = (ridx * T + tb + torch.arange(C, device=k.device)).masked_select(merged)
        dk = torch.zeros(rows * after, D, device=k.device, dtype=k.dtype).index_add(
            0, flat, gk.reshape(rows * T, D).index_select(0, tok_rows))
        dv = torch.zeros(rows * after, D, device=k.device, dtype=k.dtype).index_add(
            0, flat, gv.reshape(rows * T, D).index_select(0, tok_rows))
        s_k = s_k + dk.view(rows, after, D)
        s_v = s_v + dv.view(rows, after, D)
        snaps.append(attn_rows(s_k, s_v, vlen))
    return snaps
