"""Training path of the HIP KVM mixer: the prefill as a differentiable op.

Reference: ``_KvmTritonTrainingFunction`` (model/kvm_triton_mixer.py:24-195)
with ``run_training_backward_reconstruct_live_state``
(model/kernels/kvm_triton_training_kernels.py:3621-4153).  As there, the
routing decisions of the forward (which slot every overflow token was
appended to or merged into) are fixed metadata: the argmax and the append
ranking are not differentiated, and the bf16 roundings of the forward are
taken as the identity in the backward.

Forward: ``kvm_prefill`` on the HIP library, keeping every memory snapshot
the query chunks read, the routes of every update and the log-sum-exp of
every query.

Backward:
  * attention (HIP, ``kvm_prefill_backward``): dq, the window keys' and
    values' gradients, the gradients of every snapshot's key and value rows,
    and the two head temperatures' gradients;
  * memory state (HIP, ``kvm_state_backward``): the snapshot rows are
    functions of the tokens through LayerNorm_s(s_k), normalize(s_v) * vlen,
    the merge sums under the fixed routes and the token rows (LayerNorm_s of
    the rope-zeroed keys, the values, the merge gate's products); the kernel
    pulls the snapshot-row gradients back through all of it to k, v (added
    to the window gradients), the gate and the ln_s_k parameters.

"""

from __future__ import annotations

import ctypes

import torch

from . import _lib


def attention_backward(mixer, q, k, v, gate, res, dout):
    """The HIP attention backward of one prefill (kvm_prefill_backward).

    Returns dq [B,Hq,T,D] bf16, dk / dv of the window tokens [B,Hkv,T,D]
    fp32, d_snap_k / d_snap_v [n_snap, B*Hkv, S_max, D] fp32 and the
    temperature gradients [Hq] fp32."""
    B, Hq, T, D = q.shape
    Hkv = k.size(1)
    plan = res["plan"]
    dev = q.device
    out = res["out"]                                  # [B, T, Hq, D] bf16
    dout = dout.to(torch.bfloat16).contiguous()
    delta = torch.empty(B, Hq, T, device=dev, dtype=torch.float32)  # rowsum(dout * out), filled by the library
    qv = _lib._bf16_view(q, "q")
    seq, keep = _lib.seq4(k, v, gate)
    layer = mixer._layer_struct(B, dev)
    dq = torch.empty(B, Hq, T, D, device=dev, dtype=torch.bfloat16)
    f32 = dict(device=dev, dtype=torch.float32)
    dk = torch.empty(B, Hkv, T, D, **f32)
    dv = torch.empty(B, Hkv, T, D, **f32)
    snap_k, snap_v = res["snap_k"], res["snap_v"]
    d_snap_k = torch.empty(snap_k.shape, **f32)
    d_snap_v = torch.empty(snap_v.shape, **f32)
    d_ts = torch.empty(Hq, **f32)
    d_tf = torch.empty(Hq, **f32)
    arrs = [_lib.int32_array(a) for a in (plan.chunk_state_len, plan.chunk_snapshot)]
    d = _lib.KvmPrefillBwdDesc()
    d.layer = layer.struct
    d.q, d.q_sb, d.q_sh, d.q_st = qv.data_ptr(), qv.stride(0), qv.stride(1), qv.stride(2)
    d.kv = seq
    d.seq_len = T
    d.dout, d.do_sb, d.do_st, d.do_sh = dout.data_ptr(), dout.stride(0), dout.stride(1), dout.stride(2)
    d.lse, d.delta = res["lse"].data_ptr(), delta.data_ptr()
    d.out, d.o_sb, d.o_st, d.o_sh = out.data_ptr(), out.stride(0), out.stride(1), out.stride(2)
    d.snap_k, d.snap_v = snap_k.data_ptr(), snap_v.data_ptr()
    d.max_state_len = plan.max_state_len
    d.n_chunks = plan.n_chunks
    d.chunk_state_len, d.chunk_snapshot = arrs[0], arrs[1]
    d.dq, d.dq_sb, d.dq_sh, d.dq_st = dq.data_ptr(), dq.stride(0), dq.stride(1), dq.stride(2)
    d.dk, d.dv = dk.data_ptr(), dv.data_ptr()
    d.d_snap_k, d.d_snap_v = d_snap_k.data_ptr(), d_snap_v.data_ptr()
    d.d_state_temp, d.d_front_temp = d_ts.data_ptr(), d_tf.data_ptr()
    lib = _lib.load()
    nws = int(lib.kvm_prefill_backward_workspace_bytes(ctypes.byref(d)))
    if nws < 0:
        raise ValueError("invalid backward descriptor: " + lib.kvm_last_error().decode())
    ws = torch.empty(max(nws, 16), device=dev, dtype=torch.uint8)
    d.workspace, d.workspace_bytes = ws.data_ptr(), nws
    _lib.check(lib.kvm_prefill_backward(ctypes.byref(d), _lib.stream_handle(dev)), "kvm_prefill_backward")
    del keep, ws
    return dq, dk, dv, d_snap_k, d_snap_v, d_ts, d_tf


class KVMPrefillFunction(torch.autograd.Function):
    """y = prefill(q, k, v, gate; ln_s_k, temperatures) at the post-QKV
    boundary, differentiable in all of them (routes fixed by the forward).
    Returns the attention output [B, T, Hq, Dv] bf16 (before c_proj)."""

    @staticmethod
    def forward(ctx, mixer, q, k, v, gate, ln_w, ln_b, state_temp, front_temp):
        with torch.no_grad():
            # No status read here (a host synchronisation per layer and step):
            # a copy of the word into host memory is queued behind the
            # prefill, and the backward waits for that copy (long complete by
            # then, so without draining the stream) before using anything the
            # forward produced.
            res = mixer.prefill_raw(q, k, v, gate, route_log=True, keep_snapshots=True, want_lse=True,
                                    check_status=False)
            ctx.status = mixer._status_pending(q.device)
        ctx.mixer = mixer
        ctx.res = res
        ctx.save_for_backward(q, k, v, gate, ln_w, ln_b, state_temp, front_temp)
        return res["out"]

    @staticmethod
    def backward(ctx, dout):
        q, k, v, gate, ln_w, ln_b, state_temp, front_temp = ctx.saved_tensors
        mixer, res = ctx.mixer, ctx.res
        mixer._raise_status(ctx.status())  # a timed-out update chain raises here, before its results are used
        plan = res["plan"]
        dq, dk_w, dv_w, d_snap_k, d_snap_v, d_ts, d_tf = attention_backward(mixer, q, k, v, gate, res, dout)
        if plan.n_chunks > mixer.config.n_bswa_chunks:  # some query chunk read the memory state
            dgate, d_ln = state_backward(mixer, k, v, gate, res, d_snap_k, d_snap_v, dk_w, dv_w)
            glw, glb = d_ln[0], d_ln[1]
        else:
            dgate = torch.zeros(gate.shape, device=gate.device, dtype=torch.float32)
            glw, glb = torch.zeros_like(ln_w, dtype=torch.float32), torch.zeros_like(ln_b, dtype=torch.float32)
        return (None, dq.to(q.dtype), dk_w.to(k.dtype), dv_w.to(v.dtype), dgate.view(gate.shape).to(gate.dtype),
                glw.to(ln_w.dtype), glb.to(ln_b.dtype), d_ts.to(state_temp.dtype), d_tf.to(front_temp.dtype))


def state_backward(mixer, k, v, gate, res, d_snap_k, d_snap_v, dk, dv):
    """The memory state's share of the backward (``kvm_state_backward``).

    k, v: [B, Hkv, T, D] bf16 and gate [B, Hkv, T, 1] as the forward read
    them; ``res`` the forward's ``prefill_raw`` result (plan, route_log,
    append_log); d_snap_k / d_snap_v the snapshot-row gradients; dk / dv
    fp32 [B, Hkv, T, D] contiguous, to which the state's share is added in
    place.  Returns dgate fp32 [B, Hkv, T] and the ln_s_k gradients [2, D].
    Reference: _live_state_dkdv_to_raw_grad_kernel, _reverse_route_scatter_grad_split_kernel,
    _initial_state_grad_kernel (model/kernels/kvm_triton_training_kernels.py:2093-2745)."""
    B, Hkv, T, D = k.shape
    dev = k.device
    plan = res["plan"]
    nu = plan.n_updates
    for name, t in (("dk", dk), ("dv", dv)):
        if t.dtype != torch.float32 or not t.is_contiguous() or tuple(t.shape) != (B, Hkv, T, D):
            raise ValueError(f"{name} must be contiguous fp32 [B, Hkv, T, D]")
    seq, keep = _lib.seq4(k, v, gate)
    layer = mixer._layer_struct(B, dev)
    dgate = torch.zeros(B, Hkv, T, device=dev, dtype=torch.float32)
    d_ln = torch.empty(2, D, device=dev, dtype=torch.float32)
    d = _lib.KvmStateBwdDesc()
    d.layer = layer.struct
    d.kv = seq
    d.seq_len, d.initial_state_len, d.n_updates = T, plan.initial_state_len, nu
    sched = [_lib.int32_array(a) for a in (plan.upd_token_begin, plan.upd_state_before, plan.upd_n_append)]
    d.upd_token_begin, d.upd_state_before, d.upd_n_append = sched
    if nu:
        rl = res["route_log"].to(torch.int32).contiguous()
        al = res["append_log"].to(torch.int32).contiguous()
        d.route_log, d.append_log = rl.data_ptr(), al.data_ptr()
    d.max_state_len = plan.max_state_len
    d.d_snap_k, d.d_snap_v = d_snap_k.data_ptr(), d_snap_v.data_ptr()
    d.dk, d.dv, d.dgate, d.d_ln = dk.data_ptr(), dv.data_ptr(), dgate.data_ptr(), d_ln.data_ptr()
    lib = _lib.load()
    nws = int(lib.kvm_state_backward_workspace_bytes(ctypes.byref(d)))
    if nws < 0:
        raise ValueError("invalid state-backward descriptor: " + lib.kvm_last_error().decode())
    ws = torch.empty(max(nws, 16), device=dev, dtype=torch.uint8)
    d.workspace, d.workspace_bytes = ws.data_ptr(), nws
    _lib.check(lib.kvm_state_backward(ctypes.byref(d), _lib.stream_handle(dev)), "kvm_state_backward")
    del keep, ws
    return dgate, d_ln


def prefill_with_grad(mixer, q, k, v, gate):
    """Differentiable post-QKV prefill of ``mixer`` (routes fixed by the forward)."""
    Hq = mixer.num_attention_heads
    dev = q.device
    ones = torch.ones(Hq, device=dev, dtype=torch.float32)
    temps = bool(mixer.config.kvm_use_head_temps)
    ts = mixer.state_head_temp.view(-1) if temps else ones
    tf = mixer.front_head_temp.view(-1) if temps else ones
    return KVMPrefillFunction.apply(mixer, q, k, v, gate, mixer.ln_s_k.weight, mixer.ln_s_k.bias, ts, tf)


__all__ = ["KVMPrefillFunction", "prefill_with_grad", "attention_backward",
           "state_backward"]
