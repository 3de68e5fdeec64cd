"""GPTAlpha2-style decoder whose token mixers are the HIP KVM ``SequenceMixer``.

Restates the reference's decoder around the mixer, so a whole model (token
ids -> logits, prefill then cached greedy decode) runs with every KVM layer on
the MI355X kernels:

  * model/rwkv7_backbone.py:34-73     ``RotaryEmbedding`` (partial interleaved RoPE)
  * model/rwkv7_backbone.py:103-177   ``MLP`` (relu^2, optional token shift)
  * model/rwkv7_backbone.py:180-235   ``Block`` (pre-LN, residual scale, lambdas)
  * model/rwkv7_backbone.py:276-405   ``MixerConfig`` fields and defaults
  * model/rwkv7_backbone.py:417-685   ``RWKV7BackboneModel`` (embedding, layers,
                                      U-net skips, head LayerNorm)
  * model/rwkv7_backbone.py:688-775   ``RWKV7BackboneForCausalLM`` (LM head,
                                      logit soft cap, fp32 logits)

Parameter names and shapes equal the reference's, so its ``state_dict``
loads unchanged.  The classes are plain ``nn.Module``s (no HuggingFace
base classes); generation is ``generate_greedy`` (prefill, then one token
per step through the layer caches), the loop HuggingFace's greedy
``generate`` runs on the reference model.

Token-mixer selection follows the reference's ``token_mixer_class_path`` /
``token_mixer`` (model/rwkv7_backbone.py:186-201).  The reference's KVM mixer
paths (``model.kvm_mixer``, ``model.kvm_triton_mixer``,
``model.kvm_fp32_routing_reference``) and ``token_mixer: kvm`` resolve to
``kvm_amd.mixer.SequenceMixer``; other reference mixers are not part of this
build and raise ``ValueError``.  Any other importable class path is loaded
as given.
"""

from __future__ import annotations

import ctypes
import importlib
import math
from dataclasses import dataclass
from typing import Any

import torch
import torch.nn.functional as F
from torch import nn

from . import _lib
from .linear import linear, module_linear
from .mixer import SequenceMixer, set_label
from .states_cache import StatesDictCache

_KVM_PATH = "kvm_amd.mixer.SequenceMixer"
_KVM_ALIASES = {
    "model.kvm_mixer.SequenceMixer",
    "model.kvm_triton_mixer.SequenceMixer",
    "model.kvm_fp32_routing_reference.SequenceMixer",
}

# MixerConfigDataclass defaults (model/rwkv7_backbone.py:276-405) of every
# field this decoder or the KVM mixer reads.
_DEFAULTS: dict[str, Any] = dict(
    model_class_path="kvm_amd.backbone.RWKV7BackboneForCausalLM",
    vocab_size=50304, num_hidden_layers=12, num_attention_heads=6, num_key_value_heads=None,
    d_qk_head=None, d_v_head=None, d_head=None, hidden_size=768, mup_base_dim=768,
    rope_theta=10_000.0, rope_partial_dim=64, ffn_expansion=4.0, token_mixer="kvm",
    token_mixer_class_path=None, alt_token_mixer="swa", alt_token_mixer_class_path=None,
    alt_layer_every=-1, use_tokenshift_ffn=False, use_block_lambdas=False, use_skip_connections=False,
    use_l2wrap=False, logit_softcap=0.0, residual_scale=None,
    use_value_residual=1, kvm_value_residual_mode="rwkv", kvm_token_shift_mode="rwkv",
    kvm_apply_merge_gate_to_initial_state=0, kvm_apply_merge_gate_to_appends=0,
    kvm_use_merge_gate_keys=1, kvm_use_merge_gate_values=1, kvm_use_head_temps=1, kvm_use_vlens=1,
    kvm_aotriton_forward_attention=1, kvm_aotriton_precompiled_forward=0, use_tokenshift_att=0,
    sink_len=1, chunk_len=256, n_max_d_chunks=1, n_bswa_chunks=2, state_budget_mode="fixed",
    state_growth_factor=1.0, state_growth_exponent=0.5, state_round_down=1, state_min_len=-1,
    state_saturation_n=None, param_dtype="bfloat16", pad_token_id=None, bos_token_id=None,
    eos_token_id=None,
)


class MixerConfig:
    """Model config with the reference's field names and defaults
    (model/rwkv7_backbone.py:276-405).  Unknown keyword arguments are kept as
    attributes, as the reference's ``PretrainedConfig`` base does."""

    def __init__(self, **kwargs: Any):
        for k, v in _DEFAULTS.items():
            setattr(self, k, v)
        for k, v in kwargs.items():
            setattr(self, k, v)

    def to_dict(self) -> dict[str, Any]:
        return dict(vars(self))


@dataclass
class BaseModelOutput:
    """The decoder's final hidden states and the cache the step used (the
    fields of transformers' BaseModelOutputWithPast the reference returns)."""

    last_hidden_state: torch.Tensor
    past_key_values: StatesDictCache | None = None


@dataclass
class CausalLMOutput:
    """Logits (fp32) and the cache the step used (the fields of the
    reference's CausalLMOutputWithPastAndAccuracy this build fills; no loss)."""

    logits: torch.Tensor
    past_key_values: StatesDictCache | None = None
    loss: torch.Tensor | None = None


def token_shift_delta(x: torch.Tensor, prev_token: torch.Tensor | None = None, *,
                      fallback: str = "first") -> torch.Tensor:
    """``shift(x) - x`` with the previous token carried across calls (model/tokenshift.py:11-28)."""
    if prev_token is None:
        if fallback == "first":
            prev_token = x[:, :1]
        elif fallback == "zero":
            prev_token = torch.zeros_like(x[:, :1])
        else:
            raise ValueError(f"Unsupported token-shift fallback: {fallback!r}")
    elif prev_token.dtype != x.dtype or prev_token.device != x.device:
        prev_token = prev_token.to(device=x.device, dtype=x.dtype)
    return torch.cat([prev_token, x[:, :-1]], dim=1) - x


def _orthogonal_(weight: torch.Tensor, gain: float) -> None:
    """utils/init.py:4-8: fp32 orthogonal init copied into the parameter."""
    with torch.no_grad():
        weight.copy_(torch.nn.init.orthogonal_(torch.empty_like(weight, dtype=torch.float), gain))


class RotaryEmbedding(nn.Module):
    """Partial RoPE over interleaved pairs (model/rwkv7_backbone.py:34-73).

    Frequencies ``base^-linspace(0, 1, partial_dim/2)``, each repeated for
    its pair, zero past ``partial_dim``; cos/sin rounded to bf16 with the odd
    sine entries negated (the pair swap in ``apply_rotary_embeddings``)."""

    def __init__(self, full_dim: int, partial_dim: int, base: float = 10000.0):
        super().__init__()
        self.full_dim, self.partial_dim, self.base = full_dim, partial_dim, base
        self._freq: torch.Tensor | None = None

    def forward(self, position_ids: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
        dev = position_ids.device
        if self._freq is None or self._freq.device != dev:
            f = (1 / self.base) ** torch.linspace(0.0, 1.0, steps=self.partial_dim // 2,
                                                  dtype=torch.float32, device=dev)
            f = f.repeat_interleave(2)
            self._freq = torch.cat([f, f.new_zeros(self.full_dim - self.partial_dim)])
        B, T = position_ids.shape
        # A K=1 product: one fp32 multiply per element, as the reference's matmul.
        theta = position_ids.float().view(B, T, 1, 1) * self._freq.view(1, 1, 1, -1)
        cos = theta.cos().bfloat16()
        sin = theta.sin().bfloat16()
        sin[..., 1::2] *= -1
        return cos, sin


class MLP(nn.Module):
    """relu(x W_fc)^2 W_proj with an optional RWKV token shift (model/rwkv7_backbone.py:103-177)."""

    _CACHE_FINAL = "mlp_final_token"

    def __init__(self, config, layer_idx: int):
        super().__init__()
        self.config, self.layer_idx = config, layer_idx
        d_hidden = int(config.ffn_expansion * config.hidden_size) // 32 * 32
        self.c_fc = set_label("matrix_params", nn.Linear(config.hidden_size, d_hidden, bias=False))
        _orthogonal_(self.c_fc.weight, gain=1)
        self.c_proj = set_label("matrix_params", nn.Linear(d_hidden, config.hidden_size, bias=False))
        self.c_proj.weight.data.zero_()
        if config.use_tokenshift_ffn:
            with torch.no_grad():
                ratio = 1.0 - (layer_idx / config.num_hidden_layers)
                ddd = torch.arange(config.hidden_size, dtype=torch.float32).div_(config.hidden_size).view(1, 1, -1)
                self.x_k = set_label("scalars", nn.Parameter(1.0 - torch.pow(ddd, ratio ** 4)))

    def forward(self, x, past_key_values=None, **kwargs):
        if self.config.use_tokenshift_ffn:
            prev = self.carried_row(x, past_key_values)
            if self._use_kernels(x):
                xk = _kernel_token_shift(x, prev, self.x_k)
            else:
                xk = x + self.x_k * token_shift_delta(x, prev, fallback="zero")
            if past_key_values is not None:
                self.store_carried_row(x[:, -1:], prev, past_key_values)
        else:
            xk = x
        return self.ffn(xk)

    def carried_row(self, x, past_key_values):
        """The previous step's last input row [B, 1, d] from the cache (None
        on an empty cache), with the cache invariants the reference asserts."""
        if past_key_values is None:
            return None
        layer_len = past_key_values.get_seq_length(self.layer_idx)
        cur = int(x.size(1))
        if layer_len < cur:
            raise AssertionError("MLP cache invariant violated: the layer cache must already include "
                                 "the current attention pass before the MLP runs.")
        prev = past_key_values.get_states(self.layer_idx).get(self._CACHE_FINAL)
        prior = layer_len - cur
        if prior > 0 and prev is None:
            raise AssertionError("cached MLP decode requires 'mlp_final_token' from a prior MLP pass.")
        if prior == 0 and prev is not None:
            raise AssertionError("MLP cache invariant violated: found 'mlp_final_token' although no "
                                 "prior MLP tokens exist for this layer.")
        if prev is not None and prev.shape != (x.shape[0], 1, x.shape[2]):
            raise AssertionError(f"cached MLP decode requires 'mlp_final_token' of shape "
                                 f"{(x.shape[0], 1, x.shape[2])}, got {tuple(prev.shape)}.")
        return prev

    def store_carried_row(self, last, prev, past_key_values):
        """Carry ``last`` [B, 1, d] to the next step: a copy, not a view (a
        view would keep the whole [B, T, d] input alive), written in place,
        after its last read, when the cache keeps fixed addresses for a
        captured decode step."""
        if self.in_place_carry(prev, last, past_key_values):
            prev.copy_(last)
        else:
            past_key_values.update(self.layer_idx, offset=0, states_dict={self._CACHE_FINAL: last.clone()})

    @staticmethod
    def in_place_carry(prev, last, past_key_values) -> bool:
        return (getattr(past_key_values, "static_states", False) and prev is not None
                and prev.shape == last.shape and prev.dtype == last.dtype)

    # Rows per chunk of a long input: the chunk's hidden activations
    # (8192 x 4d bf16, 134 MB at d = 2048) stay in the last-level cache
    # between the first GEMM, the activation and the second GEMM.
    _FFN_CHUNK = 8192

    def ffn(self, xk):
        """c_proj(relu(c_fc(xk))^2); every row is independent, so long inputs
        run in row chunks (the same GEMMs per row, the same results)."""
        if self._use_kernels(xk) and type(self.c_fc) is nn.Linear and self.c_fc.bias is None:
            rows = xk.numel() // xk.size(-1)
            if rows <= self._FFN_CHUNK or type(self.c_proj) is not nn.Linear or self.c_proj.bias is not None:
                return module_linear(self.c_proj, linear(xk, self.c_fc.weight, relu_square=True))
            x2 = xk.reshape(rows, xk.size(-1))
            out = x2.new_empty(rows, self.c_proj.out_features)
            w_proj_t = self.c_proj.weight.t()
            for r in range(0, rows, self._FFN_CHUNK):
                h = linear(x2[r:r + self._FFN_CHUNK], self.c_fc.weight, relu_square=True)
                torch.matmul(h, w_proj_t, out=out[r:r + self._FFN_CHUNK])
            return out.view(*xk.shape[:-1], self.c_proj.out_features)
        return module_linear(self.c_proj, F.relu(module_linear(self.c_fc, xk)).square())

    def _use_kernels(self, t: torch.Tensor) -> bool:
        """bf16 inference on the GPU takes the HIP elementwise kernels (same
        bf16 rounding points as the torch ops); CPU tensors and autograd take
        the torch ops."""
        if not t.is_cuda or t.dtype != torch.bfloat16 or t.size(-1) % 8:
            return False
        if self.config.use_tokenshift_ffn and self.x_k.dtype != torch.bfloat16:
            return False
        return not (torch.is_grad_enabled() and (t.requires_grad or any(p.requires_grad for p in self.parameters())))


def _kernel_token_shift(x: torch.Tensor, prev: torch.Tensor | None, mix: torch.Tensor) -> torch.Tensor:
    """x + mix * (shift(x) - x), fallback "zero", in one HIP launch (kvm_token_shift)."""
    from . import _lib

    x = x.contiguous()
    B, T, d = x.shape
    out = torch.empty_like(x)
    if prev is not None:
        prev = prev.to(device=x.device, dtype=x.dtype).reshape(B, d).contiguous()
    mix = mix.reshape(d).contiguous()
    _lib.check(_lib.load().kvm_token_shift(x.data_ptr(), prev.data_ptr() if prev is not None else None,
                                           mix.data_ptr(), out.data_ptr(), B, T, d, 1,
                                           _lib.stream_handle(x.device)), "kvm_token_shift")
    return out


def _resolve_mixer_path(config, layer_idx: int) -> str:
    """model/rwkv7_backbone.py:186-201, with the KVM paths mapped onto this build."""
    alt = config.alt_layer_every > 1 and layer_idx % config.alt_layer_every == 0
    if alt:
        path = config.alt_token_mixer_class_path or f"model.{config.alt_token_mixer}_mixer.SequenceMixer"
    else:
        path = config.token_mixer_class_path or f"model.{config.token_mixer}_mixer.SequenceMixer"
    if path in _KVM_ALIASES:
        return _KVM_PATH
    if path.startswith("model."):
        raise ValueError(f"token mixer {path!r} is not part of this build; only the KVM mixer "
                         f"({_KVM_PATH}) is provided")
    return path


def _load_class(class_path: str):
    module_path, class_name = class_path.rsplit(".", 1)
    return getattr(importlib.import_module(module_path), class_name)


class Block(nn.Module):
    """Pre-LN block: x + scale*mixer(LN(x)), then x + scale*MLP(LN(x)) (model/rwkv7_backbone.py:180-235)."""

    def __init__(self, config, layer_idx: int):
        super().__init__()
        self.config, self.layer_idx = config, layer_idx
        self.residual_scale = config.residual_scale or 1.0
        mixer_cls = _load_class(_resolve_mixer_path(config, layer_idx))
        self.ln_attn = set_label("scalars", nn.LayerNorm(config.hidden_size))
        self.attn = mixer_cls(config, layer_idx)
        self.ln_mlp = set_label("scalars", nn.LayerNorm(config.hidden_size))
        self.mlp = MLP(config, layer_idx)
        if config.use_block_lambdas:
            self.lambdas = set_label("scalars", nn.Parameter(torch.tensor([1.0, 0.0])))

    def _residual(self, x, y):
        """x + y * residual_scale.  For a power-of-two scale the product is
        exact, so one fused add (alpha) gives the same bf16 result as the
        reference's two ops."""
        sc = float(self.residual_scale)
        if sc > 0 and math.frexp(sc)[0] == 0.5:
            return torch.add(x, y, alpha=sc)
        return x + y * self.residual_scale

    def forward(self, x, x0, **kwargs):
        if self.config.use_block_lambdas:
            x = self.lambdas[0] * x + self.lambdas[1] * x0
        cached = not self.training and kwargs.get("past_key_values") is not None
        attn_fn = getattr(self.attn, "forward_inference", self.attn.forward) if cached else self.attn.forward
        x = self._residual(x, attn_fn(self.ln_attn(x), x0=x0, **kwargs))
        return self._residual(x, self.mlp(self.ln_mlp(x), x0=x0, **kwargs))


class RWKV7BackboneModel(nn.Module):
    """Embedding -> LayerNorm -> blocks (with optional U-net skips) -> LayerNorm
    (model/rwkv7_backbone.py:417-685)."""

    def __init__(self, config):
        super().__init__()
        if config.alt_layer_every > 0:
            raise ValueError("alternating token mixers are not part of this build (alt_layer_every must be <= 0)")
        self.config = config
        self.padding_idx = config.pad_token_id
        self.vocab_size = config.vocab_size
        self.d_qk_head = config.d_qk_head or config.d_head or (config.hidden_size // config.num_attention_heads)
        self.d_v_head = config.d_v_head or config.d_head or (config.hidden_size // config.num_attention_heads)
        self.wte = set_label("wte_embed", nn.Embedding(config.vocab_size, config.hidden_size, self.padding_idx),
                             mup_d_in_ratio=1.0)
        self.h = nn.ModuleList([Block(config, i) for i in range(config.num_hidden_layers)])
        with torch.no_grad():
            nn.init.uniform_(self.wte.weight, a=-1e-4, b=1e-4)
        if config.use_skip_connections:
            self.encoder_layers = config.num_hidden_layers // 2
            self.decoder_layers = config.num_hidden_layers - self.encoder_layers
            self.skip_weights = set_label("scalars", nn.Parameter(torch.ones(self.decoder_layers)))
        else:
            self.encoder_layers, self.decoder_layers = config.num_hidden_layers, 0
        self.ln_emb = set_label("scalars", nn.LayerNorm(config.hidden_size))
        self.ln_head = set_label("scalars", nn.LayerNorm(config.hidden_size))
        self.rotary = RotaryEmbedding(self.d_qk_head, config.rope_partial_dim, config.rope_theta)

    def embed(self, input_ids):
        return self.ln_emb(self.wte(input_ids))

    def forward(self, input_ids=None, attention_mask=None, position_ids=None, past_key_values=None,
                inputs_embeds=None, use_cache=None, cache_position=None, **kwargs):
        """BaseModelOutput(last_hidden_state, past_key_values or None) (model/rwkv7_backbone.py:468-570)."""
        if (input_ids is None) ^ (inputs_embeds is not None):
            raise ValueError("You must specify exactly one of input_ids or inputs_embeds")
        if inputs_embeds is None:
            inputs_embeds = self.embed(input_ids)
        if (cache_position is not None and cache_position.numel() > 0 and cache_position.is_cuda
                and isinstance(past_key_values, StatesDictCache)):
            # The cache's own token count is what cache_position[0] must equal (each
            # layer's cache asserts it); reading the GPU tensor back would stall the
            # host on every decode step.
            past_seen = past_key_values.get_seq_length(0)
        elif cache_position is not None and cache_position.numel() > 0:
            past_seen = int(cache_position.reshape(-1)[0].item())
        elif position_ids is not None and position_ids.numel() > 0:
            past_seen = int(position_ids.reshape(-1)[0].item())
        elif (attention_mask is not None and past_key_values is not None
              and attention_mask.shape[-1] > inputs_embeds.shape[1]):
            past_seen = int(attention_mask.shape[-1] - inputs_embeds.shape[1])
        elif past_key_values is None:
            past_seen = 0
        else:
            raise ValueError("Cannot infer cached token count from past_key_values alone. "
                             "Pass cache_position or position_ids when using a layer-indexed cache.")
        if use_cache and not isinstance(past_key_values, StatesDictCache):
            past_key_values = StatesDictCache()
        if position_ids is None:
            position_ids = (torch.arange(inputs_embeds.shape[1], device=inputs_embeds.device) + past_seen).unsqueeze(0)
        if attention_mask is not None:
            if bool(torch.all(attention_mask.sum(dim=-1) == attention_mask.shape[-1]).item()):
                attention_mask = None
            else:
                raise NotImplementedError("left or right padding attention_masks are not supported by the model code")
        if past_seen > 0 and inputs_embeds.shape[1] > 1:
            raise AssertionError("multi-token inputs with past_key_values are not supported; "
                                 "decode one token per step")
        x = self._forward_model(input_ids, inputs_embeds, position_ids=position_ids, attention_mask=attention_mask,
                                past_key_values=past_key_values, use_cache=use_cache, **kwargs)
        return BaseModelOutput(last_hidden_state=x, past_key_values=past_key_values if use_cache else None)

    def _forward_model(self, input_ids, x, position_ids, **kwargs):
        """model/rwkv7_backbone.py:585-685 (no alternating layers)."""
        x0 = x
        position_embeddings = self.rotary(position_ids)
        if self._fused_blocks_ok(x):
            return self._forward_fused(input_ids, x0, position_embeddings, kwargs)
        first = self.h[0]
        first_kwargs_fn = getattr(first.attn, "get_first_layer_kwargs", lambda x0, x, **kw: {})
        first_kwargs = first_kwargs_fn(x0=x0, x=first.ln_attn(x0), input_ids=input_ids, **kwargs)
        layer_kwargs = dict(x0=x0, **first_kwargs, **kwargs)
        layer_kwargs["position_embeddings"] = position_embeddings
        skips = []
        for i in range(self.encoder_layers):
            x = self.h[i](x, **layer_kwargs)
            if self.config.use_skip_connections:
                skips.append(x)
        for i in range(self.decoder_layers):
            # An odd layer count pops an empty list, as the reference does.
            x = self.h[self.encoder_layers + i](x + self.skip_weights[i] * skips.pop(), **layer_kwargs)
        return self.ln_head(x)


    def _fused_blocks_ok(self, x) -> bool:
        """bf16 GPU inference of blocks without lambdas or U-net skips runs
        each residual add with the LayerNorm after it (and the MLP's token
        shift) in one kvm_add_norm launch."""
        c = self.config
        if (not x.is_cuda or x.dtype != torch.bfloat16 or c.use_block_lambdas or c.use_skip_connections
                or x.size(-1) % 8 or x.size(-1) > 4096):
            return False
        if torch.is_grad_enabled() and (x.requires_grad or any(p.requires_grad for p in self.parameters())):
            return False
        lns = [self.ln_head] + [ln for b in self.h for ln in (b.ln_attn, b.ln_mlp)]
        if any(ln.weight is None or ln.bias is None or ln.weight.dtype != torch.bfloat16
               or ln.bias.dtype != torch.bfloat16 for ln in lns):
            return False
        return not (c.use_tokenshift_ffn and any(b.mlp.x_k.dtype != torch.bfloat16 for b in self.h))

    def _forward_fused(self, input_ids, x0, position_embeddings, kwargs):
        """The block loop of _forward_model with each residual add fused to
        the LayerNorm that reads its result (the next block's ln_attn, or
        ln_head after the last block) and the MLP's token shift fused to
        ln_mlp: x + s * f(h) and LN(x + s * f(h)) from one read of each."""
        blocks = self.h
        first = blocks[0]
        pkv = kwargs.get("past_key_values")
        xf = self._carried_mixer_row(first, x0, pkv)
        _, h = _add_norm(x0, None, 1.0, first.ln_attn, state_out=xf)
        first_kwargs_fn = getattr(first.attn, "get_first_layer_kwargs", lambda x0, x, **kw: {})
        first_kwargs = first_kwargs_fn(x0=x0, x=h, input_ids=input_ids, **kwargs)
        layer_kwargs = dict(x0=x0, **first_kwargs, **kwargs)
        layer_kwargs["position_embeddings"] = position_embeddings
        x = x0
        for i, blk in enumerate(blocks):
            attn_fn = (getattr(blk.attn, "forward_inference", blk.attn.forward)
                       if not blk.training and pkv is not None else blk.attn.forward)
            a = attn_fn(h, **layer_kwargs) if xf is None else attn_fn(h, x_final_stored=True, **layer_kwargs)
            mlp = blk.mlp
            if self.config.use_tokenshift_ffn:
                prev = mlp.carried_row(a, pkv)
                state = None
                if pkv is not None:
                    last_shape = (a.shape[0], 1, a.shape[2])
                    in_place = a.size(1) == 1 and mlp.in_place_carry(prev, a[:, -1:], pkv) and prev.is_contiguous()
                    state = prev if in_place else torch.empty(last_shape, device=a.device, dtype=a.dtype)
                x, xk = _add_norm(x, a, blk.residual_scale, blk.ln_mlp, mix=mlp.x_k, prev=prev, state_out=state)
                if pkv is not None and state is not prev:
                    pkv.update(mlp.layer_idx, offset=0, states_dict={mlp._CACHE_FINAL: state})
            else:
                x, xk = _add_norm(x, a, blk.residual_scale, blk.ln_mlp)
            m = mlp.ffn(xk)
            last = i + 1 == len(blocks)
            xf = None if last else self._carried_mixer_row(blocks[i + 1], x, pkv)
            x, h = _add_norm(x, m, blk.residual_scale, self.ln_head if last else blocks[i + 1].ln_attn,
                             want_x=not last, state_out=xf)
        return h

    @staticmethod
    def _carried_mixer_row(blk, x, pkv):
        """The mixer's carried input row (``att_x_final_token``) of ``blk``
        when the block kernel can write the new one in place: a single token,
        a cache with fixed addresses, an existing bf16 [B, 1, d] row, and a
        mixer that does not read the old row during the step (every value
        residual mode but rwkv_post_tokenshift, whose value-gate token shift
        reads it)."""
        if pkv is None or x.size(1) != 1 or not getattr(pkv, "static_states", False):
            return None
        mixer = blk.attn
        key = getattr(mixer, "_CACHE_X_FINAL", None)
        if key is None or getattr(mixer, "value_residual_mode", None) == "rwkv_post_tokenshift":
            return None
        prev = pkv.get_states(mixer.layer_idx).get(key)
        if (prev is None or prev.shape != (x.shape[0], 1, x.shape[2]) or prev.dtype != torch.bfloat16
                or not prev.is_contiguous()):
            return None
        return prev


def _add_norm(x, y, scale, ln, *, mix=None, prev=None, state_out=None, want_x=True):
    """(x + scale * y, LN(x + scale * y)) in one kvm_add_norm launch; with
    ``mix`` the second output is the token-shifted LN (fallback "zero", the
    carried row ``prev`` before token 0) and ``state_out`` [B, 1, d] receives
    the last token's LN row.  ``y`` None: (x, LN(x)).  The residual rounds as
    Block._residual does."""
    B, T, d = x.shape
    x = x.contiguous()
    desc = _lib.KvmAddNormDesc()
    desc.x, desc.batch, desc.seq_len, desc.width = x.data_ptr(), B, T, d
    out_x = x
    keep = [x]
    if y is not None:
        y = y.contiguous()
        keep.append(y)
        sc = float(scale)
        desc.y, desc.alpha = y.data_ptr(), sc
        desc.round_product = 0 if sc > 0 and math.frexp(sc)[0] == 0.5 else 1
        if want_x:
            out_x = torch.empty_like(x)
            desc.out_x = out_x.data_ptr()
        else:
            out_x = None
    desc.ln_w, desc.ln_b, desc.eps = ln.weight.data_ptr(), ln.bias.data_ptr(), float(ln.eps)
    out = torch.empty_like(x)
    if mix is not None:
        mix = mix.reshape(d).contiguous()
        keep.append(mix)
        desc.mix, desc.out_shift = mix.data_ptr(), out.data_ptr()
        if prev is not None:
            prev_c = prev.reshape(B, d)
            if prev_c.data_ptr() != prev.data_ptr() or not prev.is_contiguous():
                raise ValueError("add_norm: the carried row must be a contiguous [B, 1, d] tensor")
            desc.prev = prev.data_ptr()
    else:
        desc.out_h = out.data_ptr()
    if state_out is not None:
        if not state_out.is_contiguous() or state_out.numel() != B * d:
            raise ValueError("add_norm: state_out must be a contiguous [B, 1, d] tensor")
        desc.state_out = state_out.data_ptr()
    _lib.check(_lib.load().kvm_add_norm(ctypes.byref(desc), _lib.stream_handle(x.device)), "kvm_add_norm")
    del keep
    return out_x, out


class RWKV7BackboneForCausalLM(nn.Module):
    """Decoder + LM head (model/rwkv7_backbone.py:688-775)."""

    def __init__(self, config):
        super().__init__()
        self.config = config
        self.transformer = RWKV7BackboneModel(config)
        self.lm_head = set_label("lm_head", nn.Linear(config.hidden_size, config.vocab_size, bias=False))
        _orthogonal_(self.lm_head.weight, gain=0.5 * (config.vocab_size / config.hidden_size) ** 0.5)

    def get_input_embeddings(self):
        return self.transformer.wte

    def get_output_embeddings(self):
        return self.lm_head

    def forward(self, input_ids=None, attention_mask=None, position_ids=None, past_key_values=None,
                inputs_embeds=None, labels=None, use_cache=None, logits_to_keep: int | torch.Tensor = 0,
                **kwargs) -> CausalLMOutput:
        if labels is not None:
            raise ValueError("this build runs the inference forward path only (no loss)")
        base = self.transformer(input_ids=input_ids, attention_mask=attention_mask, position_ids=position_ids,
                                past_key_values=past_key_values, inputs_embeds=inputs_embeds, use_cache=use_cache,
                                **kwargs)
        hidden, cache = base.last_hidden_state, base.past_key_values
        keep = slice(-logits_to_keep, None) if isinstance(logits_to_keep, int) else logits_to_keep
        logits = module_linear(self.lm_head, hidden[:, keep, :])
        if self.config.logit_softcap != 0:
            logits = self.config.logit_softcap * torch.tanh(logits / self.config.logit_softcap)
        return CausalLMOutput(logits=logits.float(), past_key_values=cache)

    @torch.no_grad()
    def generate_greedy(self, input_ids: torch.Tensor, max_new_tokens: int,
                        cache: StatesDictCache | None = None, on_step=None) -> torch.Tensor:
        """Prefill ``input_ids`` [B, T], then append ``max_new_tokens`` argmax
        tokens, one cached single-token step each.  Returns [B, max_new_tokens].
        ``on_step(step, logits)`` (optional) sees each step's fp32 logits
        [B, vocab]; step 0 is the prefill's last position."""
        B, T = input_ids.shape
        cache = StatesDictCache() if cache is None else cache
        out = self(input_ids=input_ids, past_key_values=cache, use_cache=True,
                   cache_position=torch.arange(T, device=input_ids.device), logits_to_keep=1)
        logits = out.logits[:, -1]
        tokens = torch.empty(B, max_new_tokens, dtype=torch.long, device=input_ids.device)
        for s in range(max_new_tokens):
            if on_step is not None:
                on_step(s, logits)
            tok = logits.argmax(-1)
            tokens[:, s] = tok
            if s + 1 == max_new_tokens:
                break
            pos = torch.tensor([T + s], device=input_ids.device)
            logits = self(input_ids=tok[:, None], past_key_values=cache, use_cache=True,
                          cache_position=pos, logits_to_keep=1).logits[:, -1]
        return tokens


class DecodeGraph:
    """Cached single-token decode of ``model`` with the steady-state step
    captured once in a HIP graph (torch.cuda.CUDAGraph) and replayed.

    A step that only appends the new token to every KVM layer's window ring
    (the common case: no direct-state append, no state update, no window
    slide) is replayed; the KVM kernels of the replay read their per-layer
    counters {active state, ring start, window length} from device memory
    (``kvm_ring_write_dev`` / ``kvm_decode_attention_dev``), one
    ``kvm_decode_advance`` per step moves them on, and the host bookkeeping a
    step does (cache token counts, window length) is mirrored in Python.
    The other steps (one per chunk_len tokens) run eagerly and resynchronise
    the device counters.  The layer cache keeps its per-token states at fixed
    addresses (``static_states``) so that every replay reads the previous
    step's.  No counterpart in the reference, which decodes eagerly
    (model/kvm_triton_mixer.py:717-757): it removes the host cost of the
    ~20 launches per layer of an eager step.  The graph is captured again
    when a buffer it uses has been reallocated (a growing state budget) or a
    parameter has changed (new storage, or an in-place update seen by its
    version counter): a replay would otherwise keep reading the weight copies
    packed for kvm_gemm_small_packed at capture time."""

    def __init__(self, model: "RWKV7BackboneForCausalLM", cache: StatesDictCache):
        self.model, self.cache = model, cache
        cache.static_states = True
        self.graph: torch.cuda.CUDAGraph | None = None
        self.signature = None
        self.ids = self.pos = self.ctl = self.logits = None
        self.ctl_synced = False
        self.replays = self.eager_steps = 0
        self.warmed = False  # the first plain step runs eagerly (lazy allocations, packed weights)
        self._params = list(model.parameters())

    def _weights_signature(self):
        return tuple((p.data_ptr(), p._version) for p in self._params)

    def close(self) -> None:
        """Release the captured graph and its memory pool now.  Their teardown
        waits for the device, so a caller chooses where it happens instead of
        a garbage collection (possibly inside timed or latency-critical
        work).  A later step captures the graph again."""
        if self.graph is not None:
            self.graph.reset()
        self.graph = self.signature = None

    def _kvm_caches(self):
        from .decode_cache import KVMDecodeCache
        out = []
        for i in range(len(self.cache.layers)):
            c = self.cache.layers[i].get(SequenceMixer._CACHE_TRITON_DECODE)
            if isinstance(c, KVMDecodeCache):
                out.append(c)
        return out

    def _sync_ctl(self, kv) -> None:
        vals = torch.tensor([c.graph_counters() for c in kv], dtype=torch.int32)
        self.ctl.copy_(vals)  # host to device, outside the graph
        self.ctl_synced = True

    @torch.no_grad()
    def step(self, tok: torch.Tensor) -> torch.Tensor:
        """Decode one token per sequence (``tok`` [B] ids on the GPU); returns
        the fp32 logits [B, vocab] of the next position (for a replayed step, a
        buffer the next step overwrites)."""
        pos = self.cache.get_seq_length(0)
        kv = self._kvm_caches()
        plain = bool(kv) and len(kv) == len(self.cache.layers) and all(c.graph_step_is_plain() for c in kv)
        if plain and self.graph is None and not self.warmed:
            self.warmed = True
            plain = False
        if not plain:
            self.ctl_synced = False
            self.eager_steps += 1
            out = self.model(input_ids=tok[:, None], past_key_values=self.cache, use_cache=True,
                             cache_position=torch.tensor([pos]), logits_to_keep=1)
            return out.logits[:, -1]
        sig = (tuple(c.graph_buffers() for c in kv), self._weights_signature())
        if self.graph is None or sig != self.signature:
            if self.graph is not None and sig[1] != self.signature[1]:
                self.warmed = False  # repack the changed weights in an eager step first
                self.graph = None
                return self.step(tok)
            return self._capture(tok, pos, kv, sig)
        if not self.ctl_synced:
            self._sync_ctl(kv)
        self.ids.copy_(tok[:, None])
        self.pos.fill_(pos)
        for i in range(len(self.cache.layers)):
            self.cache.seen[i] += 1
        for c in kv:
            c.graph_advance_host_()
        self.graph.replay()
        self.replays += 1
        return self.logits[:, -1]

    def _capture(self, tok, pos, kv, sig):
        dev = tok.device
        if self.ids is None or self.ids.shape[0] != tok.shape[0]:
            self.ids = torch.zeros(tok.shape[0], 1, dtype=torch.long, device=dev)
            self.pos = torch.zeros(1, 1, dtype=torch.long, device=dev)
        self.ctl = torch.zeros(len(kv), 4, dtype=torch.int32, device=dev)
        self._sync_ctl(kv)
        self.ids.copy_(tok[:, None])
        self.pos.fill_(pos)
        for i, c in enumerate(kv):
            c.graph_ctl = self.ctl[i].data_ptr()
        torch.cuda.synchronize(dev)
        graph = torch.cuda.CUDAGraph()
        try:
            # The step's host bookkeeping runs here, once; the capture records
            # its device work, which the replay below then performs.
            with torch.cuda.graph(graph):
                out = self.model(input_ids=self.ids, past_key_values=self.cache, use_cache=True,
                                 cache_position=torch.tensor([pos]), position_ids=self.pos, logits_to_keep=1)
                self.logits = out.logits
                _lib.check(_lib.load().kvm_decode_advance(self.ctl.data_ptr(), len(kv), _lib.stream_handle(dev)),
                           "kvm_decode_advance")
        finally:
            for c in kv:
                c.graph_ctl = None
                c.ring_row_written = False
        self.graph, self.signature = graph, sig
        graph.replay()
        self.replays += 1
        return self.logits[:, -1]

    @torch.no_grad()
    def generate_greedy(self, input_ids: torch.Tensor, max_new_tokens: int) -> torch.Tensor:
        """``RWKV7BackboneForCausalLM.generate_greedy`` through this runner:
        prefill eagerly, then decode step by step.  Returns [B, max_new_tokens]."""
        B, T = input_ids.shape
        out = self.model(input_ids=input_ids, past_key_values=self.cache, use_cache=True,
                         cache_position=torch.arange(T, device=input_ids.device), logits_to_keep=1)
        logits = out.logits[:, -1]
        tokens = torch.empty(B, max_new_tokens, dtype=torch.long, device=input_ids.device)
        for s in range(max_new_tokens):
            tok = logits.argmax(-1)
            tokens[:, s] = tok
            if s + 1 == max_new_tokens:
                break
            logits = self.step(tok)
        return tokens


@torch.no_grad()
def init_random_(model: nn.Module, seed: int = 0) -> nn.Module:
    """Seeded random weights for benchmarks and tests, generated on the
    device the parameters live on (a model built under ``torch.device("meta")``
    and materialised with ``to_empty`` gets every value here).

    Linear / embedding matrices ~ N(0, 1/fan_in) (embedding N(0, 1)); LayerNorm
    weight 1 + 0.1 N, bias 0.1 N; token-shift mixing coefficients U(0, 1);
    every other parameter 1 + 0.1 N for scales (temperatures, lambdas, skip
    weights) and 0.1 N otherwise.  Unlike the reference's initialisation, no
    output projection is zero, so every layer contributes."""
    p0 = next(model.parameters())
    gen = torch.Generator(device=p0.device).manual_seed(seed)

    def normal_(t, mean=0.0, std=1.0):
        t.copy_(torch.randn(t.shape, generator=gen, device=t.device, dtype=torch.float32) * std + mean)

    done = set()
    for mod in model.modules():
        if isinstance(mod, nn.LayerNorm):
            normal_(mod.weight, 1.0, 0.1)
            normal_(mod.bias, 0.0, 0.1)
            done.update((id(mod.weight), id(mod.bias)))
        elif isinstance(mod, (nn.Linear, nn.Embedding)):
            normal_(mod.weight, 0.0, 1.0 if isinstance(mod, nn.Embedding) else mod.weight.shape[1] ** -0.5)
            done.add(id(mod.weight))
    for name, p in model.named_parameters():
        if id(p) in done:
            continue
        leaf = name.rsplit(".", 1)[-1]
        if leaf in ("x_q", "x_k", "x_v", "x_v_hidden"):
            p.copy_(torch.rand(p.shape, generator=gen, device=p.device, dtype=torch.float32))
        elif leaf in ("front_head_temp", "state_head_temp", "lambdas", "skip_weights", "lamb"):
            normal_(p, 1.0, 0.1)
        else:
            normal_(p, 0.0, 0.1)
    return model


__all__ = ["MixerConfig", "RotaryEmbedding", "MLP", "Block", "RWKV7BackboneModel", "RWKV7BackboneForCausalLM",
           "BaseModelOutput", "CausalLMOutput", "StatesDictCache", "DecodeGraph", "init_random_", "token_shift_delta"]
