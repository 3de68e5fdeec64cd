"""Drop-in KVM ``SequenceMixer`` running the forward path on MI355X HIP kernels.

Selection: ``model.token_mixer_class_path: kvm_amd.mixer.SequenceMixer``
(with ``kvm-paper_amd/`` on ``sys.path``) in place of
``model.kvm_triton_mixer.SequenceMixer`` (configs/prolong/kvm_triton.yaml:4).
The constructor ``SequenceMixer(config, layer_idx)``, the parameter names and
labels, the ``forward`` / ``forward_inference`` / ``forward_prefix`` /
``forward_prefill`` / ``forward_single`` / ``_decode_one_token`` signatures
and the carried-state cache entry follow the reference:
  * model/value_residual_mixin.py:14-295   heads, projections, value residual
  * model/kvm_mixer.py:78-118, 342-401     KVM parameters, forward_prefix
  * model/kvm_triton_mixer.py:198-757      prefill / decode at the QKV boundary

Everything after the post-QKV boundary (window + memory attention, the
block-boundary memory update, decode) runs in libkvm_amd.so through its C ABI
(include/kvm_amd.h).  The projections before the boundary are plain torch
modules, as in the reference.  Training: a prefill that needs gradients runs
through ``training.KVMPrefillFunction`` (the HIP forward keeping its
snapshots, routes and log-sum-exp; the HIP attention and state backward),
with the forward's routes as fixed metadata, as in the reference's training
function (model/kvm_triton_mixer.py:24-195).  Only the cached decode path is
inference-only.
"""

from __future__ import annotations

import warnings

import argparse
import ctypes
import math
import os
import weakref

import torch
import torch.nn.functional as F
from torch import nn

from . import _lib
from .linear import linear, module_linear
from .decode_cache import DecodeCacheSnapshot, KVMDecodeCache
from .schedule import (
    PrefillPlan,
    StateBudget,
    bswa_begin_for_total_len,
    prefill_plan,
    state_length_after_cycle,
)

# Snapshot memory budget of one prefill (bytes); the snapshot ring is sized to
# hold every snapshot when they fit, otherwise attention launches are batched.
_SNAPSHOT_BUDGET = int(os.environ.get("KVM_AMD_SNAPSHOT_BYTES", str(8 << 30)))


def set_label(label, module, mup_d_in_ratio=None):
    """Optimizer label of parameters (utils/opt.py:4-10)."""
    if isinstance(module, torch.Tensor):
        module.label = label
        module.mup_d_in_ratio = mup_d_in_ratio
    else:
        for p in module.parameters():
            set_label(label, p, mup_d_in_ratio)
    return module


def _store_states(cache, layer_idx, states, new_states):
    """Carry per-token states to the next step: copies (a view would keep
    the whole [B, T, d] source alive), written in place into the previous
    step's tensors when the cache asks for fixed addresses (a captured decode
    step reads and writes the same buffers on every replay)."""
    if getattr(cache, "static_states", False):
        fresh = {}
        for key, val in new_states.items():
            old = states.get(key)
            if old is not None and old.shape == val.shape and old.dtype == val.dtype:
                old.copy_(val)
            else:
                fresh[key] = val.clone()
        if fresh:
            cache.update(layer_idx, offset=0, states_dict=fresh)
        return
    cache.update(layer_idx, offset=0, states_dict={key: val.clone() for key, val in new_states.items()})


def apply_rotary_embeddings(x_BTHD, position_embeddings):
    """Interleaved-pair RoPE (model/rwkv7_backbone.py:76-88)."""
    cos, sin = position_embeddings
    assert cos.size(1) == x_BTHD.size(1), f"{cos.size()} {x_BTHD.size()}"
    x_flip = x_BTHD.view(*x_BTHD.shape[:-1], x_BTHD.shape[-1] // 2, 2).flip(-1).view(x_BTHD.shape)
    return cos * x_BTHD + sin * x_flip


def _token_shift(x, scale, prev=None):
    """RWKV token shift (model/tokenshift.py:11-37, fallback "first")."""
    if prev is None:
        prev = x[:, :1]
    elif prev.dtype != x.dtype or prev.device != x.device:
        prev = prev.to(device=x.device, dtype=x.dtype)
    return x + scale * (torch.cat([prev, x[:, :-1]], dim=1) - x)


class _LayerHandle:
    """A KvmLayer struct plus the fp32 parameter copies it points to."""

    def __init__(self, struct: _lib.KvmLayer, keep):
        self.struct = struct
        self.keep = keep

    def ref(self):
        return ctypes.byref(self.struct)

    def op_args(self):
        """(cfg integers, ln_eps, ln_w, ln_b, state_temp, front_temp): the
        layer as the torch operators take it (csrc/kvm_torch_ops.cpp)."""
        s = self.struct
        cfg = [s.batch, s.q_heads, s.kv_heads, s.head_dim, s.value_dim, s.chunk_len, s.n_bswa_chunks,
               s.sink_len, s.rope_partial_dim, s.gate_keys, s.gate_values, s.gate_appends, s.gate_initial]
        return (cfg, float(s.ln_eps), *self.keep)


# The schedule's int32 arrays of a plan as ctypes arrays (and as one host
# int32 tensor for the torch operator), made once per plan object (a
# prefill loop that passes one plan pays the conversion once).
_PLAN_ARRAYS: dict[int, tuple] = {}


def _plan_arrays(plan: PrefillPlan) -> list:
    hit = _PLAN_ARRAYS.get(id(plan))
    if hit is not None and hit[0]() is plan:
        return hit[1]
    parts = (plan.chunk_state_len, plan.chunk_snapshot, plan.upd_token_begin, plan.upd_state_before,
             plan.upd_n_append)
    arrs = [_lib.int32_array(a) for a in parts]
    arrs.append(torch.tensor([int(x) for a in parts for x in a], dtype=torch.int32))
    pid = id(plan)
    _PLAN_ARRAYS[pid] = (weakref.ref(plan), arrs)
    weakref.finalize(plan, _PLAN_ARRAYS.pop, pid, None)
    return arrs


class SequenceMixer(nn.Module):
    """KVM token mixer (post-QKV path on HIP kernels)."""

    _CACHE_S_K = "kvm_s_k"
    _CACHE_S_V = "kvm_s_v"
    _CACHE_S_VLEN = "kvm_s_vlen"
    _CACHE_STATE_COVERAGE_LEN = "kvm_state_coverage_len"
    _CACHE_BSWA_BEGIN = "kvm_bswa_begin"
    _CACHE_BSWA_K = "kvm_bswa_k"
    _CACHE_BSWA_V = "kvm_bswa_v"
    _CACHE_BSWA_MERGE_GATE = "kvm_bswa_merge_gate"
    # Same cache key as the reference mixer (model/kvm_triton_mixer.py:214).
    _CACHE_TRITON_DECODE = "kvm_triton_decode_cache"
    _CACHE_Q_FINAL = "att_q_final_token"
    _CACHE_K_FINAL = "att_k_final_token"
    _CACHE_V_FINAL = "att_v_final_token"
    _CACHE_X_FINAL = "att_x_final_token"

    def __init__(self, config, layer_idx: int):
        super().__init__()
        # --- heads and projections (model/value_residual_mixin.py:15-166) ---
        self.layer_idx = layer_idx
        self.config = config
        self.num_attention_heads = config.num_attention_heads
        self.num_key_value_heads = (
            config.num_key_value_heads if config.num_key_value_heads is not None else config.num_attention_heads
        )
        if self.num_key_value_heads <= 0:
            raise ValueError("num_key_value_heads must be positive")
        if self.num_attention_heads % self.num_key_value_heads:
            raise ValueError("num_attention_heads must be divisible by num_key_value_heads")
        self.kv_group_size = self.num_attention_heads // self.num_key_value_heads
        self.hidden_size = config.hidden_size
        self.d_qk_head = config.d_qk_head or config.d_head or (config.hidden_size // config.num_attention_heads)
        self.d_v_head = config.d_v_head or config.d_head or (config.hidden_size // config.num_attention_heads)
        d_q = self.num_attention_heads * self.d_qk_head
        d_k = self.num_key_value_heads * self.d_qk_head
        d_v = self.num_key_value_heads * self.d_v_head
        d_out = self.num_attention_heads * self.d_v_head
        self.q_projection_size, self.k_projection_size = d_q, d_k
        self.value_projection_size, self.attention_output_size = d_v, d_out
        self.rwkv_tokenshift_fallback = "first"
        self.tokenshift_mode = config.kvm_token_shift_mode if config.use_tokenshift_att else "none"
        if self.tokenshift_mode == "rwkv":
            ratio = 1.0 - (layer_idx / config.num_hidden_layers)
            ddd_q = torch.arange(d_q, dtype=torch.float32) / d_q
            ddd_k = torch.arange(d_k, dtype=torch.float32) / d_k
            ddd_v = torch.arange(d_v, dtype=torch.float32) / d_v
            self.x_q = set_label("scalars", nn.Parameter(1.0 - torch.pow(ddd_q, 0.2 * ratio)))
            self.x_k = set_label("scalars", nn.Parameter(1.0 - torch.pow(ddd_k, 0.7 * ratio)))
            self.x_v = set_label("scalars", nn.Parameter(1.0 - torch.pow(ddd_v, 0.7 * ratio)))
        self.c_q = set_label("matrix_params", nn.Linear(self.hidden_size, d_q, bias=False))
        self.c_k = set_label("matrix_params", nn.Linear(self.hidden_size, d_k, bias=False))
        self.c_v = set_label("matrix_params", nn.Linear(self.hidden_size, d_v, bias=False))
        self.ln_q = set_label("scalars", nn.LayerNorm(self.d_qk_head))
        self.ln_k = set_label("scalars", nn.LayerNorm(self.d_qk_head))
        self.c_proj = set_label("matrix_params", nn.Linear(d_out, self.hidden_size, bias=False))
        with torch.no_grad():
            self.c_proj.weight.zero_()
        self.lamb = None
        self.value_residual_mode = "none"
        if config.use_value_residual:
            mode = config.kvm_value_residual_mode
            if mode not in ("linear", "rwkv", "rwkv_post_tokenshift"):
                raise AssertionError(f"Unsupported value residual mode: {mode!r}")
            self.value_residual_mode = mode
            if mode == "linear":
                self.lamb = set_label("scalars", nn.Parameter(torch.tensor(0.5)))
            else:
                if not hasattr(self, "x_v"):
                    self.x_v = set_label("scalars", nn.Parameter(torch.zeros(d_v)))

                def lora_dim(c, mult, power):
                    return max(32, int(round((mult * (c ** power)) / 32) * 32))

                r = lora_dim(self.hidden_size, 1.3, 0.5)
                r_base = lora_dim(config.mup_base_dim, 1.3, 0.5)
                self.v_gate1 = set_label("matrix_params", nn.Linear(self.hidden_size, r, bias=False))
                self.v_gate2 = set_label("matrix_params", nn.Linear(r, d_v, bias=False), mup_d_in_ratio=r / r_base)
                with torch.no_grad():
                    self.v_gate1.weight.zero_()
                    w = torch.empty(r, d_v)
                    nn.init.orthogonal_(w, gain=0.1)
                    self.v_gate2.weight.copy_(w.T)
                linear = torch.arange(d_v, dtype=torch.float32) / (d_v - 1) - 0.5
                self.v_gate0 = set_label("scalars", nn.Parameter(torch.zeros(1, 1, d_v) + 0.73 - linear.view(1, 1, d_v) * 0.4))
                if mode == "rwkv_post_tokenshift" and d_v != self.hidden_size:
                    self.x_v_hidden = set_label("scalars", nn.Parameter(torch.zeros(self.hidden_size)))

        # --- KVM attributes (model/kvm_mixer.py:79-118) ---
        self.rope_partial_dim = config.rope_partial_dim if config.rope_partial_dim > 0 else self.d_qk_head
        self.ln_s_k = set_label("scalars", nn.LayerNorm(self.d_qk_head))
        self.sink_len = config.sink_len
        self.chunk_len = config.chunk_len
        self.n_max_d_chunks = config.n_max_d_chunks
        self.n_bswa_chunks = config.n_bswa_chunks
        self.max_state_len = self.chunk_len * self.n_max_d_chunks
        self.state_budget_mode = config.state_budget_mode
        self.state_growth_factor = config.state_growth_factor
        self.state_growth_exponent = config.state_growth_exponent
        self.state_round_down = config.state_round_down
        self.state_min_len = config.state_min_len
        self.state_saturation_n = config.state_saturation_n
        if config.kvm_use_merge_gate_keys or config.kvm_use_merge_gate_values:
            self.key_weighting = set_label(
                "matrix_params", nn.Linear(config.hidden_size, self.num_key_value_heads, bias=False))
        if config.kvm_use_head_temps:
            self.front_head_temp = set_label("scalars", nn.Parameter(torch.ones(config.num_attention_heads)))
            self.state_head_temp = set_label("scalars", nn.Parameter(torch.ones(config.num_attention_heads)))
        # --- constraints of the HIP path (model/kvm_triton_mixer.py:216-219) ---
        if not config.kvm_use_vlens:
            raise ValueError("the HIP KVM mixer requires kvm_use_vlens=1")
        if self.d_qk_head != self.d_v_head or self.d_qk_head not in (64, 128):
            raise ValueError("the HIP KVM mixer supports d_qk_head == d_v_head in {64, 128}")
        if not 1 <= self.chunk_len <= 4096:
            raise ValueError("the HIP KVM mixer needs chunk_len in [1, 4096]")

    # ------------------------------------------------------------------ helpers
    @property
    def state_budget(self) -> StateBudget:
        return StateBudget(
            mode=self.state_budget_mode, growth_factor=float(self.state_growth_factor),
            growth_exponent=float(self.state_growth_exponent), round_down=int(self.state_round_down),
            min_len=int(self.state_min_len),
            saturation_n=None if self.state_saturation_n is None else int(self.state_saturation_n),
            max_state_len=int(self.max_state_len),
        )

    def _bswa_begin_for_total_len(self, total_len: int) -> int:
        return bswa_begin_for_total_len(total_len, self.chunk_len, self.n_bswa_chunks)

    def _desired_state_len(self, ctx_len: int, available_context: int, current_state_len: int) -> int:
        return self.state_budget.desired(ctx_len, available_context, current_state_len)

    def make_plan(self, q_len: int) -> PrefillPlan:
        """Host schedule of a prefill (model/kvm_triton_mixer.py:257-343 make_schedule)."""
        return prefill_plan(q_len, self.chunk_len, self.n_bswa_chunks, self.state_budget)

    def _make_triton_args(self, batch_size: int, q_len: int) -> argparse.Namespace:
        """Schedule arguments of a prefill, the fields of
        model/kvm_triton_mixer.py:257-338 that the schedule reads (benchmark
        harnesses call it, scripts/kvm_benchmark/common.py:153-155)."""
        b = self.state_budget
        return argparse.Namespace(
            batch=int(batch_size), q_heads=self.num_attention_heads, kv_heads=self.num_key_value_heads,
            q_len=int(math.ceil(q_len / self.chunk_len) * self.chunk_len), logical_q_len=int(q_len),
            initial_state_len=min(int(q_len), self.chunk_len), state_capacity=self.max_state_len,
            macro_block=self.chunk_len, bswa_chunks=self.n_bswa_chunks, state_budget_mode=b.mode,
            schedule_factor=b.growth_factor, schedule_exponent=b.growth_exponent, state_min_len=b.min_len,
            state_saturation_n=b.saturation_n, state_round_down=b.round_down, dim=self.d_qk_head,
            value_dim=self.d_v_head, sink_len=self.sink_len, ln_eps=float(self.ln_s_k.eps),
        )

    def _make_schedule(self, triton_args: argparse.Namespace) -> PrefillPlan:
        """Host schedule for `_make_triton_args` output
        (model/kernels/kvm_triton_training_kernels.py:1457-1473); the result
        carries ``final_state_len`` like the reference's schedule."""
        return self.make_plan(int(getattr(triton_args, "logical_q_len", triton_args.q_len)))

    def _head_temperatures(self, device):
        if self.config.kvm_use_head_temps:
            return self.state_head_temp.detach().float().contiguous(), self.front_head_temp.detach().float().contiguous()
        ones = torch.ones(self.num_attention_heads, device=device, dtype=torch.float32)
        return ones, ones

    def _fp32_params(self, device):
        """fp32 copies of ln_s_k and the head temperatures (the kernels read
        fp32), cached until one of the parameters is replaced or modified in
        place (data pointer or version counter)."""
        src = [self.ln_s_k.weight, self.ln_s_k.bias]
        if self.config.kvm_use_head_temps:
            src += [self.state_head_temp, self.front_head_temp]
        key = tuple((p.data_ptr(), p._version, p.device) for p in src) + (str(device),)
        cached = self.__dict__.get("_f32_cache")
        if cached is None or cached[0] != key:
            w = self.ln_s_k.weight.detach().float().contiguous()
            b = self.ln_s_k.bias.detach().float().contiguous()
            ts, tf = self._head_temperatures(device)
            cached = (key, (w, b, ts, tf))
            self.__dict__["_f32_cache"] = cached
        return cached[1]

    def _layer_struct(self, batch: int, device, gate_initial: bool | None = None) -> _LayerHandle:
        w, b, ts, tf = self._fp32_params(device)
        cfg = self.config
        gi = bool(cfg.kvm_apply_merge_gate_to_initial_state) if gate_initial is None else bool(gate_initial)
        s = _lib.KvmLayer(
            batch=int(batch), q_heads=self.num_attention_heads, kv_heads=self.num_key_value_heads,
            head_dim=self.d_qk_head, value_dim=self.d_v_head, chunk_len=self.chunk_len,
            n_bswa_chunks=self.n_bswa_chunks, sink_len=self.sink_len,
            rope_partial_dim=self.rope_partial_dim,
            gate_keys=int(bool(cfg.kvm_use_merge_gate_keys)), gate_values=int(bool(cfg.kvm_use_merge_gate_values)),
            gate_appends=int(bool(cfg.kvm_apply_merge_gate_to_appends)), gate_initial=int(gi),
            ln_eps=float(self.ln_s_k.eps),
            ln_weight=w.data_ptr(), ln_bias=b.data_ptr(), state_temp=ts.data_ptr(), front_temp=tf.data_ptr(),
        )
        return _LayerHandle(s, (w, b, ts, tf))

    def _repeat_kv_for_query_heads(self, x: torch.Tensor) -> torch.Tensor:
        return x if self.kv_group_size == 1 else x.repeat_interleave(self.kv_group_size, dim=1)

    # -------------------------------------------------------- pre-boundary part
    def get_first_layer_kwargs(self, x0, x, x_prior_token=None, **kwargs):
        """model/value_residual_mixin.py:239-246."""
        if self.value_residual_mode == "none":
            return {"v_first": None}
        return {"v_first": module_linear(self.c_v, x)}

    def _value_gate(self, x):
        return torch.sigmoid(self.v_gate0 + module_linear(self.v_gate2, module_linear(self.v_gate1, x)))

    def calc_qkv(self, x, v_first, past_key_values):
        """Projections, value residual, token shift, ln_q/ln_k (model/value_residual_mixin.py:173-237)."""
        B, T, _ = x.size()
        states = past_key_values.get_states(self.layer_idx) if past_key_values is not None else {}
        past = past_key_values.get_seq_length(self.layer_idx) if past_key_values is not None else 0
        if past > 0 and T != 1:
            raise AssertionError("cached decode expects single-token inputs.")
        q, k, v = self.c_q(x), self.c_k(x), self.c_v(x)
        if self.value_residual_mode == "linear":
            v = (1 - self.lamb) * v + self.lamb * v_first.view_as(v)
        elif self.value_residual_mode == "rwkv":
            g = self._value_gate(x)
            v = v + (v_first.to(v.dtype) - v) * g.to(v.dtype)
        qp = kp = vp = xp = None
        if past_key_values is not None:
            qp, kp = states.get(self._CACHE_Q_FINAL), states.get(self._CACHE_K_FINAL)
            vp, xp = states.get(self._CACHE_V_FINAL), states.get(self._CACHE_X_FINAL)
            # Copies, not views: a view would keep the whole [B, T, d] tensors alive.
            past_key_values.update(self.layer_idx, offset=0, states_dict={
                self._CACHE_Q_FINAL: q[:, -1:].detach().clone(), self._CACHE_K_FINAL: k[:, -1:].detach().clone(),
                self._CACHE_V_FINAL: v[:, -1:].detach().clone(), self._CACHE_X_FINAL: x[:, -1:].detach().clone(),
            })
        if self.tokenshift_mode == "rwkv":
            q = _token_shift(q, self.x_q, qp)
            k = _token_shift(k, self.x_k, kp)
            v = _token_shift(v, self.x_v, vp)
        if self.value_residual_mode == "rwkv_post_tokenshift":
            shift = self.x_v if self.value_projection_size == self.hidden_size else self.x_v_hidden
            xv = _token_shift(x, shift.view(1, 1, self.hidden_size), xp)
            g = self._value_gate(xv)
            v = v + (v_first.to(v.dtype) - v) * g.to(v.dtype)
        q = self.ln_q(q.reshape(B, T, self.num_attention_heads, -1))
        k = self.ln_k(k.reshape(B, T, self.num_key_value_heads, -1))
        v = v.reshape(B, T, self.num_key_value_heads, -1)
        return q, k, v

    def forward_prefix(self, x, v_first, position_embeddings, attention_mask, past_key_values=None, **kwargs):
        """q/k/v/merge gate at the post-QKV boundary (model/kvm_mixer.py:367-401).

        bf16 inference on the GPU runs the projections as torch GEMMs and
        everything after them in one ``kvm_prefix`` launch; CPU tensors and
        autograd take the torch op sequence, which is the reference's."""
        if self._use_fused_prefix(x, position_embeddings):
            return self._fused_prefix(x, v_first, position_embeddings, past_key_values,
                                      x_final_stored=bool(kwargs.get("x_final_stored", False)))
        return self._torch_prefix(x, v_first, position_embeddings, past_key_values)

    _VR_MODES = {"none": 0, "linear": 1, "rwkv": 2, "rwkv_post_tokenshift": 3}

    def _use_fused_prefix(self, x, position_embeddings) -> bool:
        if not x.is_cuda or x.dtype != torch.bfloat16 or position_embeddings is None:
            return False
        # The kernel reads every parameter it uses as raw bf16.
        used = [self.c_q.weight, self.ln_q.weight, self.ln_q.bias, self.ln_k.weight, self.ln_k.bias]
        used += [getattr(self, n) for n in ("x_q", "x_k", "x_v", "v_gate0") if hasattr(self, n)]
        if self.lamb is not None:
            used.append(self.lamb)
        if any(p.dtype != torch.bfloat16 for p in used):
            return False
        if torch.is_grad_enabled() and (x.requires_grad or any(p.requires_grad for p in self.parameters())):
            return False
        return self.d_qk_head == self.d_v_head and self.d_qk_head in (64, 128)

    def _fused_prefix(self, x, v_first, position_embeddings, past_key_values, x_final_stored=False):
        """Projections (torch GEMMs), then value residual, token shift,
        ln_q/ln_k, RoPE and merge gate in one HIP launch (include/kvm_amd.h
        kvm_prefix).  Same outputs and cache entries as ``_torch_prefix``.
        ``x_final_stored``: the caller already wrote x's last row over the
        carried ``att_x_final_token`` (the block kernel that produced x)."""
        B, T, _ = x.size()
        states = past_key_values.get_states(self.layer_idx) if past_key_values is not None else {}
        past = past_key_values.get_seq_length(self.layer_idx) if past_key_values is not None else 0
        if past > 0 and T != 1:
            raise AssertionError("cached decode expects single-token inputs.")
        mode = self._VR_MODES[self.value_residual_mode]
        Hq, Hkv, D = self.num_attention_heads, self.num_key_value_heads, self.d_qk_head
        use_gate = bool(self.config.kvm_use_merge_gate_keys or self.config.kvm_use_merge_gate_values)
        xp = states.get(self._CACHE_X_FINAL) if past_key_values is not None else None
        # Every projection of x in one GEMM (c_q, c_k, c_v, key_weighting and,
        # for the rwkv value residual, v_gate1); the kernel reads the column
        # ranges of its output in place.
        mods = [self.c_q, self.c_k, self.c_v]
        if use_gate:
            mods.append(self.key_weighting)
        if mode == 2:
            mods.append(self.v_gate1)
        if self._CONCAT_PROJ:
            y = linear(x, self._projection_weight(mods))
            sizes = [m.out_features for m in mods]
            parts = torch.split(y, sizes + [y.size(-1) - sum(sizes)], dim=-1)[:len(mods)]
        else:
            parts = [m(x) for m in mods]
            # the kernel reads q/k/v with one token stride
            parts[:3] = torch.split(torch.cat(parts[:3], dim=-1), [m.out_features for m in mods[:3]], dim=-1)
        q_lin, k_lin, v_lin = parts[:3]
        kw = parts[3] if use_gate else None
        gate_lin = None
        if mode == 2:
            gate_lin = module_linear(self.v_gate2, parts[-1])
        elif mode == 3:
            shift = self.x_v if self.value_projection_size == self.hidden_size else self.x_v_hidden
            gate_lin = module_linear(self.v_gate2, module_linear(
                self.v_gate1, _token_shift(x, shift.view(1, 1, self.hidden_size), xp)))
        shift_on = self.tokenshift_mode == "rwkv"
        prev = [states.get(k) for k in (self._CACHE_Q_FINAL, self._CACHE_K_FINAL, self._CACHE_V_FINAL)]
        bf = dict(device=x.device, dtype=torch.bfloat16)
        q = torch.empty(B, T, Hq, D, **bf)
        k = torch.empty(B, T, Hkv, D, **bf)
        v = torch.empty(B, T, Hkv, D, **bf)
        gate = torch.empty(B, T, Hkv, **bf) if use_gate else None
        # The carried last rows (q_lin, k_lin, v after a pre-shift value
        # residual) come from the kernel: into the previous step's tensors
        # when the cache keeps fixed addresses (a single token reads them
        # before it writes them), else into new ones.
        last = [None, None, None]
        if past_key_values is not None:
            in_place = getattr(past_key_values, "static_states", False) and T == 1
            for i, width in enumerate((Hq * D, Hkv * D, Hkv * D)):
                p = prev[i]
                if (in_place and p is not None and p.shape == (B, 1, width) and p.dtype == torch.bfloat16
                        and p.is_contiguous()):
                    last[i] = p
                else:
                    last[i] = torch.empty(B, 1, width, **bf)
        cos, sin = position_embeddings
        if cos.dtype != torch.bfloat16 or sin.dtype != torch.bfloat16:
            cos, sin = cos.bfloat16(), sin.bfloat16()
        if cos.stride(-1) != 1 or cos.stride() != sin.stride():
            cos, sin = cos.contiguous(), sin.contiguous()
        rope_sb = cos.stride(0) if cos.size(0) > 1 else 0
        keep = []

        def ptr(t):
            if t is None:
                return None
            t = t.contiguous()
            keep.append(t)
            return t.data_ptr()

        d = _lib.KvmPrefixDesc()
        d.batch, d.seq_len, d.q_heads, d.kv_heads, d.head_dim, d.value_dim = B, T, Hq, Hkv, D, D
        d.value_residual_mode, d.token_shift, d.ln_eps = mode, int(shift_on), float(self.ln_q.eps)
        st = q_lin.stride(1)
        if not (all(t.stride(-1) == 1 and t.stride(1) == st and t.stride(0) == T * st for t in (q_lin, k_lin, v_lin))
                and st % 8 == 0 and all(t.data_ptr() % 16 == 0 for t in (q_lin, k_lin, v_lin))):
            raise AssertionError("q/k/v projections must share one token stride (a multiple of 8 elements)")
        keep.extend((q_lin, k_lin, v_lin))
        d.q_lin, d.k_lin, d.v_lin = q_lin.data_ptr(), k_lin.data_ptr(), v_lin.data_ptr()
        d.qkv_st = q_lin.stride(1)
        d.v_first = ptr(v_first.to(torch.bfloat16).reshape(B, T, -1)) if mode else None
        d.gate_lin = ptr(gate_lin)
        if kw is not None:
            if kw.stride(-1) != 1 or kw.stride(0) != T * kw.stride(1):
                kw = kw.contiguous()
            keep.append(kw)
            d.key_weight, d.kw_st = kw.data_ptr(), kw.stride(1)
        if shift_on:
            d.q_prev, d.k_prev, d.v_prev = (ptr(p.to(torch.bfloat16)) if p is not None else None for p in prev)
            d.x_q, d.x_k, d.x_v = ptr(self.x_q), ptr(self.x_k), ptr(self.x_v)
        if mode >= 2:
            d.v_gate0 = ptr(self.v_gate0)
        if mode == 1:
            d.lamb = ptr(self.lamb.reshape(1))
        d.ln_q_w, d.ln_q_b, d.ln_k_w, d.ln_k_b = (ptr(t) for t in (self.ln_q.weight, self.ln_q.bias,
                                                                   self.ln_k.weight, self.ln_k.bias))
        d.cos, d.sin = ptr(cos), ptr(sin)
        d.rope_sb, d.rope_st = rope_sb, cos.stride(1)
        d.q_out, d.k_out, d.v_out = q.data_ptr(), k.data_ptr(), v.data_ptr()
        d.gate_out = gate.data_ptr() if gate is not None else None
        d.q_last_out, d.k_last_out, d.v_last_out = (t.data_ptr() if t is not None else None for t in last)
        # A captured decode step (device ring counters) writes the token's
        # window-ring row here instead of in a launch of its own.
        dc = states.get(self._CACHE_TRITON_DECODE) if past_key_values is not None else None
        if (T == 1 and isinstance(dc, KVMDecodeCache) and dc.graph_ctl is not None
                and dc.recent_k.dtype == torch.bfloat16 and dc.recent_gate.dtype == torch.bfloat16):
            d.ring_k, d.ring_v, d.ring_gate = dc.recent_k.data_ptr(), dc.recent_v.data_ptr(), dc.recent_gate.data_ptr()
            d.ring_cap, d.ring_ctl = dc.ring_capacity, dc.graph_ctl
            dc.ring_row_written = True
        lib = _lib.load()
        _lib.check(lib.kvm_prefix(ctypes.byref(d), _lib.stream_handle(x.device)), "kvm_prefix")
        del keep
        if past_key_values is not None:
            fresh = {key: t for key, t, p in zip((self._CACHE_Q_FINAL, self._CACHE_K_FINAL, self._CACHE_V_FINAL),
                                                 last, prev) if t is not p}
            if fresh:
                past_key_values.update(self.layer_idx, offset=0, states_dict=fresh)
            if not x_final_stored:
                _store_states(past_key_values, self.layer_idx, states, {self._CACHE_X_FINAL: x[:, -1:].detach()})
        if use_gate:
            merge_gate = gate.view(B, T, Hkv, 1).transpose(1, 2)
        else:
            merge_gate = torch.ones((B, Hkv, T, 1), device=x.device, dtype=torch.float)
        return q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2), merge_gate

    # One concatenated projection GEMM in the fused path (fewer launches;
    # same products, rounded by a different GEMM kernel than separate ones).
    _CONCAT_PROJ = True

    def _projection_weight(self, mods):
        """torch.cat of the modules' weights, padded with zero rows to a
        multiple of 64 outputs (128-byte aligned output rows, so that each
        head's piece of a row is whole cache lines for the prefix kernel),
        rebuilt whenever one of them is replaced or modified in place (data
        pointer or version counter)."""
        key = tuple((m.weight.data_ptr(), m.weight._version, m.weight.device) for m in mods)
        cached = self.__dict__.get("_proj_cat")
        if cached is None or cached[0] != key:
            w0 = mods[0].weight
            pad = -sum(m.out_features for m in mods) % 64
            with torch.no_grad():
                cached = (key, torch.cat([m.weight for m in mods] + [w0.new_zeros(pad, w0.size(1))], dim=0))
            self.__dict__["_proj_cat"] = cached
        return cached[1]

    def _torch_prefix(self, x, v_first, position_embeddings, past_key_values):
        B, T, _ = x.size()
        q, k, v = self.calc_qkv(x, v_first, past_key_values)
        q = apply_rotary_embeddings(q, position_embeddings)
        k = apply_rotary_embeddings(k, position_embeddings)
        if self.config.kvm_use_merge_gate_keys or self.config.kvm_use_merge_gate_values:
            merge_gate = 1.0 + F.elu(self.key_weighting(x).view(B, T, self.num_key_value_heads, 1)).transpose(1, 2)
        else:
            merge_gate = torch.ones((B, self.num_key_value_heads, T, 1), device=x.device, dtype=torch.float)
        return q.transpose(1, 2), k.transpose(1, 2), v.transpose(1, 2), merge_gate

    # ------------------------------------------------------------ entry points
    def forward(self, x, v_first, position_embeddings, attention_mask, past_key_values=None, **kwargs):
        q, k, v, g = self.forward_prefix(x, v_first, position_embeddings, attention_mask, past_key_values, **kwargs)
        return self.forward_prefill(q, k, v, g, v_first, position_embeddings, attention_mask, past_key_values, **kwargs)

    def forward_inference(self, x, v_first, position_embeddings, attention_mask, past_key_values=None, **kwargs):
        """Prefill on an empty cache, single-token decode otherwise (model/kvm_mixer.py:527-570)."""
        past = past_key_values.get_seq_length(self.layer_idx) if past_key_values is not None else 0
        q, k, v, g = self.forward_prefix(x, v_first, position_embeddings, attention_mask, past_key_values, **kwargs)
        if past == 0:
            return self.forward_prefill(q, k, v, g, v_first, position_embeddings, attention_mask, past_key_values, **kwargs)
        return self.forward_single(q, k, v, g, v_first, position_embeddings, attention_mask, past_key_values, **kwargs)

    def _needs_grad(self, *tensors) -> bool:
        return torch.is_grad_enabled() and any(
            t.requires_grad for t in (*tensors, self.ln_s_k.weight, self.ln_s_k.bias,
                                      getattr(self, "state_head_temp", tensors[0]),
                                      getattr(self, "front_head_temp", tensors[0])))

    def _check_no_grad(self, *tensors):
        if self._needs_grad(*tensors):
            raise ValueError("the HIP KVM mixer's cached decode is inference only; run it under torch.no_grad()")

    def _status_word(self, device) -> torch.Tensor:
        """This mixer's sticky device status word (int32[1]) on ``device``:
        the library ORs failure bits into it and never clears it."""
        words = self.__dict__.setdefault("_status_words", {})
        key = str(device)
        if key not in words:
            words[key] = torch.zeros(1, device=device, dtype=torch.int32)
        return words[key]

    def check_prefill_status(self, device=None) -> None:
        """Raise RuntimeError if a prefill on ``device`` (all devices when
        None) reported a device-side failure since the last check.  Waits for
        the work already queued, so call it where a synchronisation is
        acceptable."""
        for key in list(self.__dict__.get("_status_words", {})):
            if device is not None and key != str(device):
                continue
            self._raise_status(self._take_status(key))

    def _take_status(self, device) -> int:
        """The status word's bits for ``device`` (one synchronisation), cleared."""
        word = self.__dict__.get("_status_words", {}).get(str(device))
        if word is None:
            return 0
        bits = int(word.item())
        if bits:
            word.zero_()
        return bits

    def _status_pending(self, device):
        """Queue a copy of the status word into pinned host memory behind the
        work already on the stream; returns a function that waits for that
        copy only (not for work queued after it) and returns the word's bits,
        clearing the word when any is set."""
        word = self._status_word(device)
        host = torch.empty(1, dtype=torch.int32, pin_memory=True)  # one per read: reads may overlap
        host.copy_(word, non_blocking=True)
        done = torch.cuda.Event()
        done.record()

        def wait() -> int:
            done.synchronize()
            bits = int(host[0])
            if bits:
                word.zero_()
            return bits

        return wait

    @staticmethod
    def _raise_status(bits: int) -> None:
        if bits & _lib.KVM_STATUS_CHAIN_TIMEOUT:
            raise _lib.KvmLibraryError(
                "kvm_prefill: the persistent update chain timed out waiting for its row group "
                "(another workload held compute units); the prefill's outputs and state are incomplete")
        if bits:
            raise _lib.KvmLibraryError(f"kvm_prefill: device status word {bits:#x}")

    def prefill_raw(self, q, k, v, merge_gate, *, plan: PrefillPlan | None = None, state_capacity: int | None = None,
                    route_log: bool = False, snapshot_budget: int | None = None,
                    events=None, check_status: bool | None = True, keep_snapshots: bool = False,
                    want_lse: bool = False, chain: bool = True) -> dict:
        """Post-QKV prefill on the HIP library; returns the raw outputs.

        q [B,Hq,T,D], k [B,Hkv,T,D], v [B,Hkv,T,Dv] bf16 (any strides with a
        contiguous last axis), merge_gate [B,Hkv,T,1].  Returns a dict with
        ``out`` [B,T,Hq,Dv], the final state tensors ``state_k``, ``state_v``,
        ``state_vlen``, ``state_k_attn``, ``state_v_attn`` ([B*Hkv, cap, D]),
        ``plan`` and, when requested, ``route_log`` / ``append_log``
        [n_updates, B*Hkv, C] int32.  ``events``: optional four recorded
        torch.cuda.Event objects bracketing the update chain and the
        attention launches (timing).

        ``check_status``: read the device status word after the call (one
        synchronisation).  If the persistent update chain gave up (another
        workload held compute units, so its row groups could not all be
        resident), the call is repeated on the per-update kernels, which give
        bit-identical results without that requirement, and a RuntimeWarning
        is issued; a failure there raises RuntimeError.
        Callers that issue many prefills back to back pass False and call
        ``check_prefill_status()`` once afterwards; the word is sticky.
        With ``check_status=None`` no status word is passed: the library then
        waits for the stream itself and reports a failure as its return code
        (the C ABI's synchronous mode).

        ``chain=False`` runs the memory updates as per-update kernels from the
        start (``KVM_PREFILL_NO_CHAIN``).

        Training (``kvm_amd.training``): ``keep_snapshots`` returns every
        memory snapshot the query chunks read (``snap_k`` / ``snap_v``, bf16
        [n_updates + 1, B*Hkv, max_state_len, D]); ``want_lse`` returns the
        log2-domain log-sum-exp of every query (``lse``, fp32 [B, Hq, T]).
        """
        if q.dtype != torch.bfloat16:
            raise ValueError("the HIP KVM mixer computes in bfloat16; got " + str(q.dtype))
        B, Hq, T, D = q.shape
        if Hq != self.num_attention_heads:
            raise AssertionError("KVM query head count mismatch.")
        if int(k.size(1)) != self.num_key_value_heads:
            raise AssertionError("KVM key/value head count mismatch.")
        dev = q.device
        if plan is None:
            plan = self.make_plan(int(T))
        cap = max(plan.final_state_len, int(state_capacity or 0))
        rows = B * self.num_key_value_heads
        bf = dict(device=dev, dtype=torch.bfloat16)
        out = torch.empty(B, T, Hq, self.d_v_head, **bf)
        st = {
            "state_k": torch.empty(rows, cap, D, **bf), "state_v": torch.empty(rows, cap, D, **bf),
            "state_vlen": torch.empty(rows, cap, device=dev, dtype=torch.float32),
            "state_k_attn": torch.empty(rows, cap, D, **bf), "state_v_attn": torch.empty(rows, cap, D, **bf),
        }
        qv = _lib._bf16_view(q, "q")
        kv, vv = _lib._bf16_view(k, "k"), _lib._bf16_view(v, "v")
        gv = merge_gate if merge_gate.dtype == torch.bfloat16 else merge_gate.to(torch.bfloat16)
        cfg, eps, w, b, ts, tf = self._layer_struct(B, dev).op_args()
        n_snaps = plan.n_updates + 1
        per_snap = 2 * rows * plan.max_state_len * D * 2
        budget = _SNAPSHOT_BUDGET if snapshot_budget is None else int(snapshot_budget)
        ring = max(2, min(n_snaps, budget // max(per_snap, 1)))
        extra = {}
        if keep_snapshots:
            ring = max(2, n_snaps)
            shape = (n_snaps, rows, plan.max_state_len, D)
            extra["snap_k"] = torch.empty(shape, **bf)
            extra["snap_v"] = torch.empty(shape, **bf)
        if want_lse:
            extra["lse"] = torch.empty(B, Hq, T, device=dev, dtype=torch.float32)
        logs = {}
        if route_log:
            n = max(plan.n_updates, 1)
            logs["route_log"] = torch.full((n, rows, self.chunk_len), -1, device=dev, dtype=torch.int32)
            logs["append_log"] = torch.zeros((n, rows, self.chunk_len), device=dev, dtype=torch.int32)
        ev = [] if events is None else [int(e.cuda_event) if e is not None else 0 for e in events]
        status = None if check_status is None else self._status_word(dev)
        # One torch operator (csrc/kvm_torch_ops.cpp) over kvm_prefill, on the
        # current stream; it sizes and allocates the workspace itself.
        def call(flags):
            _lib.call_op(_lib.ops().prefill, qv, kv, vv, gv, w, b, ts, tf, cfg, eps, _plan_arrays(plan)[5],
                         plan.n_chunks, plan.n_updates, plan.max_state_len, ring, out, st["state_k"],
                         st["state_v"], st["state_vlen"], st["state_k_attn"], st["state_v_attn"], status,
                         logs.get("route_log"), logs.get("append_log"), extra.get("snap_k"), extra.get("snap_v"),
                         extra.get("lse"), ev, flags)

        call(0 if chain else _lib.KVM_PREFILL_NO_CHAIN)
        if check_status:
            bits = self._take_status(dev)
            if bits & _lib.KVM_STATUS_CHAIN_TIMEOUT and chain:
                warnings.warn("kvm_prefill: the persistent update chain timed out waiting for its row group "
                              "(another workload held compute units); repeating the prefill on the per-update "
                              "kernels", RuntimeWarning, stacklevel=2)
                if "route_log" in logs:
                    logs["route_log"].fill_(-1)
                    logs["append_log"].zero_()
                call(_lib.KVM_PREFILL_NO_CHAIN)
                bits = self._take_status(dev)
            self._raise_status(bits)
        res = {"out": out, "plan": plan, "capacity": cap, **st, **logs, **extra}
        return res

    def forward_prefill(self, q, k, v, merge_gate, v_first, position_embeddings, attention_mask,
                        past_key_values=None, **kwargs):
        """Prefill at the post-QKV boundary (model/kvm_triton_mixer.py:560-666)."""
        if attention_mask is not None:
            raise ValueError("the HIP KVM mixer does not support attention_mask")
        B, _, T, _ = q.size()
        if self._needs_grad(q, k, v, merge_gate):
            # Training (model/kvm_triton_mixer.py:24-195): the differentiable prefill with
            # the forward's routes as fixed metadata; no decode cache is built.
            if past_key_values is not None:
                raise ValueError("the HIP KVM mixer's training path does not build a decode cache")
            from .training import prefill_with_grad

            y = prefill_with_grad(self, q, k, v, merge_gate)
            return self.c_proj(y.reshape(B, T, -1))
        plan = self.make_plan(int(T))
        cap = None
        if past_key_values is not None:
            cap = max(plan.final_state_len, min(self.chunk_len, self.max_state_len),
                      state_length_after_cycle(self.state_budget, self.chunk_len, self.n_bswa_chunks,
                                               int(T), plan.final_state_len, self.n_bswa_chunks * self.chunk_len))
        # The status word is read without stalling the GPU: the output
        # projection is queued behind the prefill before the host waits for
        # the word's copy.  A timed-out chain is repeated on the per-update
        # kernels (bit-identical results), as prefill_raw does.
        res = self.prefill_raw(q, k, v, merge_gate, plan=plan, state_capacity=cap, check_status=False)
        status = self._status_pending(q.device)
        y = self.c_proj(res["out"].view(B, T, -1))
        bits = status()
        if bits & _lib.KVM_STATUS_CHAIN_TIMEOUT:
            warnings.warn("kvm_prefill: the persistent update chain timed out waiting for its row group "
                          "(another workload held compute units); repeating the prefill on the per-update "
                          "kernels", RuntimeWarning, stacklevel=2)
            res = self.prefill_raw(q, k, v, merge_gate, plan=plan, state_capacity=cap, chain=False)
            y = self.c_proj(res["out"].view(B, T, -1))
        else:
            self._raise_status(bits)
        if past_key_values is not None:
            begin = self._bswa_begin_for_total_len(int(T))
            if plan.final_coverage != max(plan.initial_state_len, begin):
                raise AssertionError("KVM prefill state progression drifted from cache bookkeeping.")
            cache = self._cache_from_prefill(res, k, v, merge_gate, int(T), begin)
            past_key_values.update(self.layer_idx, offset=int(T), states_dict={self._CACHE_TRITON_DECODE: cache})
        return y

    def _cache_from_prefill(self, res, k, v, gate, T, begin) -> KVMDecodeCache:
        """Decode cache adopting the prefill's state buffers (no copy, no refresh)."""
        B = int(k.size(0))
        cache = KVMDecodeCache(self, None, state_capacity=res["capacity"], _device=k.device, _batch=B)
        cache.state_k, cache.state_v, cache.state_vlen = res["state_k"], res["state_v"], res["state_vlen"]
        cache.state_k_attn, cache.state_v_attn = res["state_k_attn"], res["state_v_attn"]
        R = T - begin
        rows = cache.kv_rows
        cache.recent_k[:, :R].copy_(k[:, :, begin:].reshape(rows, R, self.d_qk_head))
        cache.recent_v[:, :R].copy_(v[:, :, begin:].reshape(rows, R, self.d_v_head))
        cache.recent_gate[:, :R].copy_(gate[:, :, begin:].reshape(rows, R))
        cache.total_len = T
        cache.state_len = res["plan"].final_state_len
        cache.state_coverage_len = res["plan"].final_coverage
        cache.recent_begin = begin
        cache.recent_start = 0
        cache.recent_len = R
        return cache

    def forward_single(self, q, k, v, merge_gate, v_first, position_embeddings, attention_mask,
                       past_key_values=None, **kwargs):
        """Decode one token through the cache (model/kvm_triton_mixer.py:668-715)."""
        if attention_mask is not None:
            raise ValueError("the HIP KVM mixer does not support attention_mask")
        if past_key_values is None:
            raise ValueError("HIP KVM cached decode requires past_key_values")
        if int(q.size(2)) != 1:
            raise AssertionError("HIP KVM cached decode expects a single-token input")
        cache = past_key_values.get_states(self.layer_idx).get(self._CACHE_TRITON_DECODE)
        if not isinstance(cache, KVMDecodeCache):
            raise RuntimeError("HIP KVM cache is missing its decode state; run a prefill with this cache first")
        if cache.mixer is not self:
            raise RuntimeError("HIP KVM decode cache belongs to another mixer")
        past = past_key_values.get_seq_length(self.layer_idx)
        if cache.total_len != past:
            raise AssertionError(f"HIP KVM decode cache length disagrees with the layer cache: {cache.total_len} != {past}")
        out = self._decode_one_token(q, k, v, merge_gate, cache)
        past_key_values.update(self.layer_idx, offset=1, states_dict={self._CACHE_TRITON_DECODE: cache})
        return module_linear(self.c_proj, out.transpose(1, 2).contiguous().view(int(q.size(0)), 1, -1))

    def _decode_one_token(self, q, k, v, merge_gate, decode_cache: KVMDecodeCache) -> torch.Tensor:
        """Advance ``decode_cache`` by one post-QKV token and attend (model/kvm_triton_mixer.py:717-757)."""
        fresh = self._decode_advance(k, v, merge_gate, decode_cache, defer_ring_write=True)
        return self._decode_attention(q, decode_cache, fresh)

    def _decode_advance(self, k, v, merge_gate, decode_cache: KVMDecodeCache, *,
                        defer_ring_write: bool = False):
        """Cache bookkeeping of one decode token: direct-state append while the
        prompt is shorter than a chunk, the state update when the window
        crosses a chunk boundary, and the ring write.  With
        ``defer_ring_write`` (and KVM_AMD_FUSED_RING_WRITE not 0) the ring
        write may be left to the attention launch: the return value is then
        the token's (k, v, gate) to hand to :meth:`_decode_attention`, which
        must come next; None when the row was written here."""
        if int(k.size(2)) != 1:
            raise ValueError("HIP KVM decode cache update accepts one token")
        c = decode_cache
        new_total = c.total_len + 1
        new_begin = self._bswa_begin_for_total_len(new_total)
        direct_target = min(new_total, c.chunk_len)
        new_cov = max(direct_target, new_begin)
        if new_cov < c.state_coverage_len:
            raise AssertionError("KVM decode state coverage cannot shrink")
        lib = _lib.load()
        stream = _lib.stream_handle(c.device)
        if direct_target > c.state_coverage_len:
            if direct_target - c.state_coverage_len != 1:
                raise AssertionError("decode crossed more than one direct-state token")
            c._reserve_state_capacity(c.state_len + 1)
            seq, keep = _lib.seq4(k, v, merge_gate)
            # Eager decode appends the ungated prepared key (model/kvm_mixer.py:627-642).
            _lib.check(lib.kvm_state_append_direct(c.direct_layer.ref(), seq, 0, 1, c.state_struct(),
                                                   c.state_len, stream), "kvm_state_append_direct")
            del keep
            c.state_len += 1
            c.state_coverage_len = direct_target
        if new_cov > c.state_coverage_len:
            if new_cov - c.state_coverage_len != self.chunk_len:
                raise AssertionError("decode crossed more than one state boundary")
            self._run_decode_state_update(c)
            c.state_coverage_len = new_cov
        defer = defer_ring_write and os.environ.get("KVM_AMD_FUSED_RING_WRITE", "1") != "0"
        if c.append_recent_(k, v, merge_gate, total_len=new_total, recent_begin=new_begin, defer_write=defer):
            return (k, v, merge_gate)
        return None

    def _run_decode_state_update(self, c: KVMDecodeCache) -> None:
        """Fold the oldest window chunk into the state (model/kvm_triton_mixer.py:759-864;
        eager model/kvm_mixer.py:646-669)."""
        cur = c.state_len
        want = self._desired_state_len(self.n_bswa_chunks * c.chunk_len + c.state_coverage_len,
                                       c.state_coverage_len + c.chunk_len, cur)
        n_app = min(max(want - cur, 0), c.chunk_len)
        c._reserve_state_capacity(cur + n_app)
        seq, keep = _lib.seq_rows(c.recent_k, c.recent_v, c.recent_gate, c.kv_heads, ring=c.ring_capacity)
        lib = _lib.load()
        _lib.check(lib.kvm_state_update(
            c.layer.ref(), seq, c.recent_start, c.chunk_len, cur, n_app, c.state_struct(),
            c.state_k_attn.data_ptr(), c.state_v_attn.data_ptr(), c.update_workspace.data_ptr(),
            c.update_workspace.numel(), c.route_by_token.data_ptr(), c.append_by_token.data_ptr(),
            _lib.stream_handle(c.device)), "kvm_state_update")
        del keep
        c.state_len = cur + n_app
        c.update_count += 1

    def _decode_attention(self, q: torch.Tensor, c: KVMDecodeCache, fresh=None) -> torch.Tensor:
        """Attention of one query over the state and the window ring
        (model/kvm_triton_mixer.py:902-929); ``fresh`` is the deferred ring
        row of :meth:`_decode_advance`, written by this launch (kvm_decode_step)."""
        active = c.state_len if c.total_len > c.ring_capacity else 0
        qv = _lib._bf16_view(q, "q")
        lib = _lib.load()
        if fresh is not None:
            if c.graph_ctl is not None:
                raise AssertionError("a deferred ring row cannot be written under graph capture")
            k1, v1, g1 = fresh
            g1 = g1 if g1.dtype == torch.bfloat16 else g1.to(torch.bfloat16)
            cfg, eps, w, b, ts, tf = c.layer.op_args()
            # The torch operator over kvm_decode_step (csrc/kvm_torch_ops.cpp), on the current stream.
            _lib.call_op(_lib.ops().decode_step, qv, _lib._bf16_view(k1, "k"), _lib._bf16_view(v1, "v"), g1, w, b,
                         ts, tf, cfg, eps, c.state_k, c.state_v, c.state_vlen, c.state_k_attn, c.state_v_attn,
                         active, c.recent_k, c.recent_v, c.recent_gate, c.recent_start, c.recent_len, c.out,
                         c.decode_workspace)
            return c.out
        if c.graph_ctl is not None:  # capture of a graph step: counters from device memory
            _lib.check(lib.kvm_decode_attention_dev(
                c.layer.ref(), qv.data_ptr(), qv.stride(0), qv.stride(1), c.state_struct(), c.graph_ctl, 1,
                c.recent_k.data_ptr(), c.recent_v.data_ptr(), c.ring_capacity, c.out.data_ptr(), c.out.stride(0),
                c.out.stride(1), c.decode_workspace.data_ptr(), c.decode_workspace.numel(),
                _lib.stream_handle(c.device)), "kvm_decode_attention_dev")
            return c.out
        _lib.check(lib.kvm_decode_attention(
            c.layer.ref(), qv.data_ptr(), qv.stride(0), qv.stride(1), c.state_struct(), active,
            c.recent_k.data_ptr(), c.recent_v.data_ptr(), c.ring_capacity, c.recent_start, c.recent_len,
            c.out.data_ptr(), c.out.stride(0), c.out.stride(1), c.decode_workspace.data_ptr(),
            c.decode_workspace.numel(), _lib.stream_handle(c.device)), "kvm_decode_attention")
        return c.out

    def make_decode_cache(self, snapshot: DecodeCacheSnapshot, state_capacity: int | None = None) -> KVMDecodeCache:
        """Decode cache from a carried-state snapshot (model/kvm_triton_decode.py:47-186)."""
        S = int(snapshot.state_k.size(2))
        cap = max(S, int(state_capacity or 0))
        return KVMDecodeCache(self, snapshot, state_capacity=cap)


__all__ = ["SequenceMixer", "apply_rotary_embeddings", "set_label"]
