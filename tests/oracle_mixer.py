"""Test-only KVM mixer whose post-QKV part is the CPU oracle.

``OracleSequenceMixer`` keeps everything of ``kvm_amd.mixer.SequenceMixer``
before the QKV boundary (projections, value residual, token shift, ln_q/ln_k,
RoPE, merge gate) and replaces the HIP prefill / decode with
``oracle.kvm_oracle.prefill`` / ``decode_step``.  Plugged into the decoder
through ``token_mixer_class_path``, it lets the CPU tests check the decoder's
host code (``kvm_amd.backbone``) and the mixer's pre-boundary code against the
reference's whole-model golden fixtures without a GPU.  It is a checker: the
product never loads it.
"""

from __future__ import annotations

from kvm_amd.mixer import SequenceMixer
from oracle import kvm_oracle as O

_STATE = "oracle_kvm_state"


class OracleSequenceMixer(SequenceMixer):
    def _oracle(self):
        c = self.config
        cfg = O.OracleConfig(
            q_heads=self.num_attention_heads, kv_heads=self.num_key_value_heads, head_dim=self.d_qk_head,
            value_dim=self.d_v_head, chunk_len=self.chunk_len, n_bswa_chunks=self.n_bswa_chunks,
            n_max_d_chunks=self.n_max_d_chunks, sink_len=self.sink_len, rope_partial_dim=self.rope_partial_dim,
            state_budget_mode=self.state_budget_mode, state_growth_factor=self.state_growth_factor,
            state_growth_exponent=self.state_growth_exponent, state_round_down=self.state_round_down,
            state_min_len=self.state_min_len, state_saturation_n=self.state_saturation_n,
            gate_keys=bool(c.kvm_use_merge_gate_keys), gate_values=bool(c.kvm_use_merge_gate_values),
            gate_appends=bool(c.kvm_apply_merge_gate_to_appends),
            gate_initial=bool(c.kvm_apply_merge_gate_to_initial_state),
            use_head_temps=bool(c.kvm_use_head_temps), use_vlens=True, fp32_routing=True,
        )
        p = O.OracleParams(
            ln_weight=self.ln_s_k.weight, ln_bias=self.ln_s_k.bias,
            front_temp=getattr(self, "front_head_temp", None), state_temp=getattr(self, "state_head_temp", None),
            ln_eps=self.ln_s_k.eps,
        )
        return cfg, p

    def forward_prefill(self, q, k, v, merge_gate, v_first, position_embeddings, attention_mask,
                        past_key_values=None, **kwargs):
        B, _, T, _ = q.shape
        cfg, p = self._oracle()
        y, state = O.prefill(q, k, v, merge_gate, p, cfg)
        if past_key_values is not None:
            past_key_values.update(self.layer_idx, offset=int(T), states_dict={_STATE: state})
        return self.c_proj(y.transpose(1, 2).reshape(B, T, -1))

    def forward_single(self, q, k, v, merge_gate, v_first, position_embeddings, attention_mask,
                       past_key_values=None, **kwargs):
        B = int(q.size(0))
        cfg, p = self._oracle()
        state = past_key_values.get_states(self.layer_idx)[_STATE]
        total = past_key_values.get_seq_length(self.layer_idx)
        y, new = O.decode_step(state, total, q, k, v, merge_gate, p, cfg)
        past_key_values.update(self.layer_idx, offset=1, states_dict={_STATE: new})
        return self.c_proj(y.transpose(1, 2).reshape(B, 1, -1))
