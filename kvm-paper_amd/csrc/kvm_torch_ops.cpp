// torch operator library over the C ABI of libkvm_amd.so (include/kvm_amd.h).
//
// The two calls of the north-star path that a mixer makes per layer and step
// are registered as torch operators, so that they run on torch's current HIP
// stream, take tensors instead of raw pointers, and are visible to torch's
// tooling (profiler, op registry):
//   kvm_amd::prefill      one prefill at the post-QKV boundary: the memory
//                         state updates and the fused window + memory
//                         attention (kvm_prefill; replaces
//                         model/kvm_triton_mixer.py:560-666 below the
//                         projections);
//   kvm_amd::decode_step  one decode token: ring write + split-K attention
//                         (kvm_decode_step; replaces
//                         model/kvm_triton_mixer.py:717-757, the write and
//                         attention of model/kernels/kvm_triton_decode.py).
// Each operator fills the C descriptor from its tensors and calls the C ABI;
// no computation happens here.  Errors of the C ABI are raised as the
// reference's exception types: invalid arguments as ValueError, any other
// failure as RuntimeError.
//
// The configuration integers `cfg` are the kvm_layer fields in order:
//   batch, q_heads, kv_heads, head_dim, value_dim, chunk_len, n_bswa_chunks,
//   sink_len, rope_partial_dim, gate_keys, gate_values, gate_appends,
//   gate_initial.

#include <ATen/core/Tensor.h>
#include <ATen/ops/empty.h>
#include <c10/hip/HIPStream.h>
#include <torch/library.h>

#include <vector>

#include "../../include/kvm_amd.h"

namespace {

constexpr int kCfgFields = 13;

void check(int rc, const char *what) {
  if (rc == KVM_OK) return;
  if (rc == KVM_EINVAL) TORCH_CHECK_VALUE(false, what, ": ", kvm_last_error());
  TORCH_CHECK(false, what, ": ", kvm_last_error());
}

const void *ptr(const c10::optional<at::Tensor> &t) { return t.has_value() ? t->data_ptr() : nullptr; }

kvm_layer make_layer(const std::vector<int64_t> &cfg, double ln_eps, const at::Tensor &ln_w,
                     const at::Tensor &ln_b, const at::Tensor &state_temp, const at::Tensor &front_temp) {
  TORCH_CHECK_VALUE(int(cfg.size()) == kCfgFields, "kvm_amd: cfg needs ", kCfgFields, " integers, got ",
                    cfg.size());
  for (const at::Tensor *t : {&ln_w, &ln_b, &state_temp, &front_temp})
    TORCH_CHECK_VALUE(t->scalar_type() == at::kFloat && t->is_contiguous() && t->is_cuda(),
                      "kvm_amd: LayerNorm parameters and head temperatures are contiguous fp32 device tensors");
  kvm_layer L{};
  L.batch = cfg[0];
  L.q_heads = cfg[1];
  L.kv_heads = cfg[2];
  L.head_dim = cfg[3];
  L.value_dim = cfg[4];
  L.chunk_len = cfg[5];
  L.n_bswa_chunks = cfg[6];
  L.sink_len = cfg[7];
  L.rope_partial_dim = cfg[8];
  L.gate_keys = cfg[9];
  L.gate_values = cfg[10];
  L.gate_appends = cfg[11];
  L.gate_initial = cfg[12];
  L.ln_eps = ln_eps;
  L.ln_weight = ln_w.data_ptr();
  L.ln_bias = ln_b.data_ptr();
  L.state_temp = state_temp.data_ptr();
  L.front_temp = front_temp.data_ptr();
  return L;
}

// Element strides of a [B, H, T, *] bf16 view (last axis contiguous).
void check_bf16_rows(const at::Tensor &t, const char *name) {
  TORCH_CHECK_VALUE(t.scalar_type() == at::kBFloat16, "kvm_amd: ", name, " must be bfloat16");
  TORCH_CHECK(t.is_cuda(), "kvm_amd: ", name, " must be a ROCm device tensor");
  TORCH_CHECK_VALUE(t.dim() == 4 && (t.size(3) == 1 || t.stride(3) == 1),
                    "kvm_amd: ", name, " must be a 4-D view with a contiguous last axis");
}

kvm_seq make_seq(const at::Tensor &k, const at::Tensor &v, const at::Tensor &gate, int64_t ring) {
  check_bf16_rows(k, "k");
  check_bf16_rows(v, "v");
  check_bf16_rows(gate, "gate");
  kvm_seq s{};
  s.k = k.data_ptr();
  s.v = v.data_ptr();
  s.gate = gate.data_ptr();
  s.k_sb = k.stride(0);
  s.k_sh = k.stride(1);
  s.k_st = k.stride(2);
  s.v_sb = v.stride(0);
  s.v_sh = v.stride(1);
  s.v_st = v.stride(2);
  s.g_sb = gate.stride(0);
  s.g_sh = gate.stride(1);
  s.g_st = gate.stride(2);
  s.ring = ring;
  return s;
}

kvm_state make_state(const at::Tensor &s_k, const at::Tensor &s_v, const at::Tensor &s_vlen,
                     const at::Tensor &s_k_attn, const at::Tensor &s_v_attn) {
  kvm_state st{};
  st.s_k = s_k.data_ptr();
  st.s_v = s_v.data_ptr();
  st.s_vlen = s_vlen.data_ptr();
  st.s_k_attn = s_k_attn.data_ptr();
  st.s_v_attn = s_v_attn.data_ptr();
  st.capacity = s_k.size(1);
  return st;
}

void *current_stream(const at::Tensor &like) {
  return c10::hip::getCurrentHIPStream(like.device().index()).stream();
}

// plan: host int32 [2 * n_chunks + 3 * n_updates]: chunk_state_len,
// chunk_snapshot, upd_token_begin, upd_state_before, upd_n_append.
// Returns the workspace tensor the call used (the caller may drop it).
void prefill(const at::Tensor &q, const at::Tensor &k, const at::Tensor &v, const at::Tensor &gate,
             const at::Tensor &ln_w, const at::Tensor &ln_b, const at::Tensor &state_temp,
             const at::Tensor &front_temp, std::vector<int64_t> cfg, double ln_eps, const at::Tensor &plan,
             int64_t n_chunks, int64_t n_updates, int64_t max_state_len, int64_t snapshot_ring,
             const at::Tensor &out, const at::Tensor &state_k, const at::Tensor &state_v,
             const at::Tensor &state_vlen, const at::Tensor &state_k_attn, const at::Tensor &state_v_attn,
             const c10::optional<at::Tensor> &status, const c10::optional<at::Tensor> &route_log,
             const c10::optional<at::Tensor> &append_log, const c10::optional<at::Tensor> &snap_k,
             const c10::optional<at::Tensor> &snap_v, const c10::optional<at::Tensor> &lse,
             std::vector<int64_t> events, int64_t flags) {
  check_bf16_rows(q, "q");
  TORCH_CHECK_VALUE(plan.device().is_cpu() && plan.scalar_type() == at::kInt && plan.is_contiguous() &&
                        plan.numel() == 2 * n_chunks + 3 * n_updates,
                    "kvm_amd.prefill: plan must be a contiguous host int32 tensor of 2 * n_chunks + "
                    "3 * n_updates entries");
  TORCH_CHECK_VALUE(events.empty() || events.size() == 4, "kvm_amd.prefill: events holds 0 or 4 handles");
  kvm_prefill_desc d{};
  d.layer = make_layer(cfg, ln_eps, ln_w, ln_b, state_temp, front_temp);
  d.q = q.data_ptr();
  d.q_sb = q.stride(0);
  d.q_sh = q.stride(1);
  d.q_st = q.stride(2);
  d.kv = make_seq(k, v, gate, 0);
  d.seq_len = q.size(2);
  d.out = out.data_ptr();
  d.o_sb = out.stride(0);
  d.o_st = out.stride(1);
  d.o_sh = out.stride(2);
  d.state = make_state(state_k, state_v, state_vlen, state_k_attn, state_v_attn);
  const int32_t *pl = plan.data_ptr<int32_t>();
  d.n_chunks = n_chunks;
  d.chunk_state_len = pl;
  d.chunk_snapshot = pl + n_chunks;
  d.n_updates = n_updates;
  d.upd_token_begin = pl + 2 * n_chunks;
  d.upd_state_before = pl + 2 * n_chunks + n_updates;
  d.upd_n_append = pl + 2 * n_chunks + 2 * n_updates;
  d.max_state_len = max_state_len;
  d.snapshot_ring = snapshot_ring;
  d.route_log = static_cast<int32_t *>(const_cast<void *>(ptr(route_log)));
  d.append_log = static_cast<int32_t *>(const_cast<void *>(ptr(append_log)));
  d.status = static_cast<int32_t *>(const_cast<void *>(ptr(status)));
  d.lse = static_cast<float *>(const_cast<void *>(ptr(lse)));
  d.snap_k = const_cast<void *>(ptr(snap_k));
  d.snap_v = const_cast<void *>(ptr(snap_v));
  d.flags = flags;
  void *ev[4] = {nullptr, nullptr, nullptr, nullptr};
  for (size_t i = 0; i < events.size(); ++i) ev[i] = reinterpret_cast<void *>(events[i]);
  if (!events.empty()) d.events = ev;
  const int64_t nbytes = kvm_prefill_workspace_bytes(&d);
  check(nbytes < 0 ? int(nbytes) : KVM_OK, "kvm_prefill_workspace_bytes");
  // Work buffers from torch's caching allocator, for this call only (the
  // stream keeps them alive until the work queued on it has used them).
  at::Tensor ws = at::empty({std::max<int64_t>(nbytes, 1)}, q.options().dtype(at::kByte));
  d.workspace = ws.data_ptr();
  d.workspace_bytes = nbytes;
  check(kvm_prefill(&d, current_stream(q)), "kvm_prefill");
}

void decode_step(const at::Tensor &q, const at::Tensor &k_new, const at::Tensor &v_new,
                 const at::Tensor &gate_new, const at::Tensor &ln_w, const at::Tensor &ln_b,
                 const at::Tensor &state_temp, const at::Tensor &front_temp, std::vector<int64_t> cfg,
                 double ln_eps, const at::Tensor &state_k, const at::Tensor &state_v,
                 const at::Tensor &state_vlen, const at::Tensor &state_k_attn, const at::Tensor &state_v_attn,
                 int64_t active_state_len, const at::Tensor &ring_k, const at::Tensor &ring_v,
                 const at::Tensor &ring_gate, int64_t ring_start, int64_t recent_len, const at::Tensor &out,
                 const at::Tensor &workspace) {
  check_bf16_rows(q, "q");
  const kvm_layer L = make_layer(cfg, ln_eps, ln_w, ln_b, state_temp, front_temp);
  const kvm_seq src = make_seq(k_new, v_new, gate_new, 0);
  const kvm_state st = make_state(state_k, state_v, state_vlen, state_k_attn, state_v_attn);
  check(kvm_decode_step(&L, q.data_ptr(), q.stride(0), q.stride(1), &st, active_state_len, &src,
                        ring_k.data_ptr(), ring_v.data_ptr(), ring_gate.data_ptr(), ring_k.size(1), ring_start,
                        recent_len, out.data_ptr(), out.stride(0), out.stride(1), workspace.data_ptr(),
                        workspace.numel(), current_stream(q)),
        "kvm_decode_step");
}

}  // namespace

TORCH_LIBRARY(kvm_amd, m) {
  m.def(
      "prefill(Tensor q, Tensor k, Tensor v, Tensor gate, Tensor ln_w, Tensor ln_b, Tensor state_temp, "
      "Tensor front_temp, int[] cfg, float ln_eps, Tensor plan, int n_chunks, int n_updates, "
      "int max_state_len, int snapshot_ring, Tensor(a!) out, Tensor(b!) state_k, Tensor(c!) state_v, "
      "Tensor(d!) state_vlen, Tensor(e!) state_k_attn, Tensor(f!) state_v_attn, Tensor(g!)? status, "
      "Tensor(h!)? route_log, Tensor(i!)? append_log, Tensor(j!)? snap_k, Tensor(k!)? snap_v, "
      "Tensor(l!)? lse, int[] events, int flags) -> ()",
      prefill);
  m.def(
      "decode_step(Tensor q, Tensor k_new, Tensor v_new, Tensor gate_new, Tensor ln_w, Tensor ln_b, "
      "Tensor state_temp, Tensor front_temp, int[] cfg, float ln_eps, Tensor state_k, Tensor state_v, "
      "Tensor state_vlen, Tensor state_k_attn, Tensor state_v_attn, int active_state_len, "
      "Tensor(a!) ring_k, Tensor(b!) ring_v, Tensor(c!) ring_gate, int ring_start, int recent_len, "
      "Tensor(d!) out, Tensor(e!) workspace) -> ()",
      decode_step);
}
