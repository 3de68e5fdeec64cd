// extern "C" entry points of libkvm_amd.so (declared in include/kvm_amd.h):
// argument validation, workspace layout and the prefill launch schedule.

#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>

#include <algorithm>
#include <string>

#include "kvm_internal.hpp"

namespace {

thread_local std::string g_error;

int fail(int code, const char *fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_error = buf;
  return code;
}

int hip_fail(hipError_t e, const char *what) {
  return fail(KVM_EHIP, "%s: %s", what, hipGetErrorString(e));
}

#define KVM_HIP(expr, what)                     \
  do {                                          \
    hipError_t e_ = (expr);                     \
    if (e_ != hipSuccess) return hip_fail(e_, what); \
  } while (0)

bool aligned16(const void *p) {
  return (reinterpret_cast<uintptr_t>(p) & 15u) == 0;
}

int check_layer(const kvm_layer *L) {
  if (!L) return fail(KVM_EINVAL, "layer descriptor is NULL");
  if (L->batch < 1 || L->q_heads < 1 || L->kv_heads < 1)
    return fail(KVM_EINVAL, "batch and head counts must be positive");
  if (L->q_heads % L->kv_heads)
    return fail(KVM_EINVAL, "q_heads (%lld) must be a multiple of kv_heads (%lld)",
                (long long)L->q_heads, (long long)L->kv_heads);
  if (L->head_dim != 64 && L->head_dim != 128)
    return fail(KVM_EINVAL, "head_dim must be 64 or 128, got %lld",
                (long long)L->head_dim);
  if (L->value_dim != L->head_dim)
    return fail(KVM_EINVAL, "value_dim must equal head_dim");
  if (L->chunk_len < 1 || L->chunk_len > 4096)
    return fail(KVM_EINVAL, "chunk_len must be in [1, 4096], got %lld",
                (long long)L->chunk_len);
  if (L->n_bswa_chunks < 1) return fail(KVM_EINVAL, "n_bswa_chunks must be >= 1");
  if (L->sink_len < 0) return fail(KVM_EINVAL, "sink_len must be >= 0");
  if (L->rope_partial_dim < 0 || L->rope_partial_dim > L->head_dim)
    return fail(KVM_EINVAL, "rope_partial_dim must be in [0, head_dim]");
  if (!L->ln_weight || !L->ln_bias || !L->state_temp || !L->front_temp)
    return fail(KVM_EINVAL, "layer parameter pointers must be set");
  if (!(L->ln_eps > 0.0)) return fail(KVM_EINVAL, "ln_eps must be positive");
  return KVM_OK;
}

int check_seq(const kvm_seq *s, const char *what) {
  if (!s || !s->k || !s->v || !s->gate)
    return fail(KVM_EINVAL, "%s: k, v and gate pointers must be set", what);
  if (!aligned16(s->k) || !aligned16(s->v))
    return fail(KVM_EINVAL, "%s: k and v must be 16-byte aligned", what);
  const int64_t st[6] = {s->k_sb, s->k_sh, s->k_st, s->v_sb, s->v_sh, s->v_st};
  for (int i = 0; i < 6; ++i)
    if (st[i] % 8)
      return fail(KVM_EINVAL, "%s: k/v strides must be multiples of 8 elements", what);
  if (s->ring < 0) return fail(KVM_EINVAL, "%s: ring must be >= 0", what);
  return KVM_OK;
}

int check_state(const kvm_state *st, bool need_attn) {
  if (!st || !st->s_k || !st->s_v || !st->s_vlen)
    return fail(KVM_EINVAL, "state: s_k, s_v and s_vlen must be set");
  if (need_attn && (!st->s_k_attn || !st->s_v_attn))
    return fail(KVM_EINVAL, "state: s_k_attn and s_v_attn must be set");
  if (!aligned16(st->s_k) || !aligned16(st->s_v) ||
      (st->s_k_attn && !aligned16(st->s_k_attn)) ||
      (st->s_v_attn && !aligned16(st->s_v_attn)))
    return fail(KVM_EINVAL, "state tensors must be 16-byte aligned");
  if (st->capacity < 1) return fail(KVM_EINVAL, "state capacity must be positive");
  return KVM_OK;
}

hipStream_t as_stream(void *s) { return static_cast<hipStream_t>(s); }

size_t align256(size_t x) { return (x + 255) & ~size_t(255); }

struct PrefillLayout {
  size_t slices;       // per-update scratch slices (one prep batch)
  size_t slice_bytes;
  size_t update_bytes;
  size_t snap_elems;  // elements of one snapshot array (keys or values)
  size_t status_off;  // the status word used when the caller passes none
  size_t total;
};

PrefillLayout prefill_layout(const kvm_prefill_desc *d) {
  PrefillLayout p;
  const kvm_layer &L = d->layer;
  p.slices = size_t(std::max<int64_t>(1, std::min<int64_t>(d->n_updates, kvm::kMaxPrep)));
  p.slice_bytes = size_t(kvm::update_slice_bytes(L, L.chunk_len));
  // The per-update scratch (prep slices + reduction keys) and the chain's
  // scratch share one region: a prefill uses one or the other.
  p.update_bytes = align256(std::max(p.slices * p.slice_bytes +
                                         size_t(kvm::update_keys_bytes(L, L.chunk_len)),
                                     size_t(kvm::chain_scratch_bytes(L, L.chunk_len))));
  p.snap_elems = size_t(L.batch * L.kv_heads) * size_t(d->max_state_len) *
                 size_t(L.head_dim);
  // Caller-held snapshots (d->snap_k / snap_v) replace the workspace ring.
  const size_t ring = d->snap_k ? 0 : size_t(d->snapshot_ring);
  p.status_off = p.update_bytes + 2 * ring * align256(p.snap_elems * 2);
  p.total = p.status_off + 256;
  return p;
}

}  // namespace

extern "C" {

int kvm_abi_version(void) { return KVM_ABI_VERSION; }

int64_t kvm_struct_size(int which) {
  switch (which) {
    case 0: return sizeof(kvm_layer);
    case 1: return sizeof(kvm_seq);
    case 2: return sizeof(kvm_state);
    case 3: return sizeof(kvm_prefill_desc);
    case 4: return sizeof(kvm_prefix_desc);
    case 5: return sizeof(kvm_prefill_bwd_desc);
    case 6: return sizeof(kvm_state_bwd_desc);
    case 7: return sizeof(kvm_add_norm_desc);
    default: return -1;
  }
}

const char *kvm_last_error(void) { return g_error.c_str(); }

int kvm_token_shift(const void *x, const void *prev, const void *mix, void *out, int64_t batch,
                    int64_t seq_len, int64_t width, int zero_fallback, void *stream) {
  if (batch < 1 || seq_len < 1 || width < 8 || width % 8)
    return fail(KVM_EINVAL, "token shift needs positive batch / seq_len and a width that is a multiple of 8");
  if (!x || !mix || !out || !aligned16(x) || !aligned16(mix) || !aligned16(out) || (prev && !aligned16(prev)))
    return fail(KVM_EINVAL, "token shift pointers must be non-NULL (prev may be NULL) and 16-byte aligned");
  KVM_HIP(kvm::launch_token_shift(x, prev, mix, out, batch, seq_len, width, zero_fallback, as_stream(stream)),
          "token shift");
  return KVM_OK;
}

int kvm_add_norm(const kvm_add_norm_desc *d, void *stream) {
  if (!d) return fail(KVM_EINVAL, "add_norm: NULL descriptor");
  const kvm_add_norm_desc &P = *d;
  if (P.batch < 1 || P.seq_len < 1 || P.width < 8 || P.width % 8 || P.width > 4096)
    return fail(KVM_EINVAL, "add_norm needs batch, seq_len >= 1 and width a multiple of 8 in [8, 4096]");
  if (!P.x || !P.ln_w || !P.ln_b)
    return fail(KVM_EINVAL, "add_norm needs x and the LayerNorm parameters");
  if (P.out_shift && !P.mix) return fail(KVM_EINVAL, "add_norm: out_shift needs mix");
  if (P.state_out && P.state_out == P.prev && P.seq_len != 1)
    return fail(KVM_EINVAL, "add_norm: state_out may alias prev only when seq_len == 1");
  // With token shift, a run of rows starts from the previous run's last row
  // of x and y, which that run's wave may already have overwritten through
  // an aliased output.
  if (P.seq_len != 1)
    for (const void *o : {static_cast<const void *>(P.out_x), static_cast<const void *>(P.out_h),
                          static_cast<const void *>(P.out_shift)})
      if (o && (o == P.x || (P.y && o == P.y)))
        return fail(KVM_EINVAL, "add_norm: an output may alias x or y only when seq_len == 1");
  const void *ptrs[] = {P.x, P.y, P.ln_w, P.ln_b, P.mix, P.prev, P.out_x, P.out_h, P.out_shift, P.state_out};
  for (const void *p : ptrs)
    if (p && !aligned16(p)) return fail(KVM_EINVAL, "add_norm pointers must be 16-byte aligned");
  if (!(P.eps >= 0.0)) return fail(KVM_EINVAL, "add_norm: eps must be >= 0");
  KVM_HIP(kvm::launch_add_norm(P, as_stream(stream)), "add_norm");
  return KVM_OK;
}

int kvm_gemm_small(const void *x, int64_t x_st, const void *w, int64_t w_st, void *y, int64_t y_st, int64_t M,
                   int64_t N, int64_t K, int epilogue, void *stream) {
  if (M < 1 || M > 16 || N < 1 || K < 32 || K % 32)
    return fail(KVM_EINVAL, "gemm_small needs 1 <= M <= 16, N >= 1 and K a positive multiple of 32");
  if (!x || !w || !y || !aligned16(x) || !aligned16(w) || x_st % 8 || w_st % 8 || x_st < K || w_st < K ||
      y_st < N)
    return fail(KVM_EINVAL, "gemm_small operands must be 16-byte aligned rows (strides multiples of 8)");
  if (epilogue != 0 && epilogue != 1) return fail(KVM_EINVAL, "gemm_small: epilogue must be 0 or 1");
  KVM_HIP(kvm::launch_gemm_small(x, x_st, w, w_st, y, y_st, M, N, K, epilogue, false, as_stream(stream)),
          "gemm_small");
  return KVM_OK;
}

int kvm_gemm_small_tile_rows(int64_t M, int64_t N) {
  if (M < 1 || M > 16 || N < 1) return fail(KVM_EINVAL, "gemm_small_tile_rows needs 1 <= M <= 16 and N >= 1");
  return kvm::gemm_small_tile_rows(M, N);
}

int kvm_gemm_small_packed(const void *x, int64_t x_st, const void *wp, void *y, int64_t y_st, int64_t M,
                          int64_t N, int64_t K, int tile_rows, int epilogue, void *stream) {
  if (M < 1 || M > 16 || N < 1 || K < 32 || K % 32)
    return fail(KVM_EINVAL, "gemm_small_packed needs 1 <= M <= 16, N >= 1 and K a positive multiple of 32");
  const int rows = kvm::gemm_small_tile_rows(M, N);
  if (tile_rows != rows)
    return fail(KVM_EINVAL, "gemm_small_packed: W packed for %d-row tiles, this shape takes %d-row tiles",
                tile_rows, rows);
  if (rows == 8 && K % 64)
    return fail(KVM_EINVAL, "gemm_small_packed: 8-row tiles need K a multiple of 64");
  if (!x || !wp || !y || !aligned16(x) || !aligned16(wp) || x_st % 8 || x_st < K || y_st < N)
    return fail(KVM_EINVAL, "gemm_small_packed operands must be 16-byte aligned rows (strides multiples of 8)");
  if (epilogue != 0 && epilogue != 1) return fail(KVM_EINVAL, "gemm_small_packed: epilogue must be 0 or 1");
  KVM_HIP(kvm::launch_gemm_small(x, x_st, wp, 0, y, y_st, M, N, K, epilogue, true, as_stream(stream)),
          "gemm_small_packed");
  return KVM_OK;
}

int kvm_relu_square(const void *x, void *out, int64_t n, void *stream) {
  if (n < 8 || n % 8) return fail(KVM_EINVAL, "relu_square needs a positive element count that is a multiple of 8");
  if (!x || !out || !aligned16(x) || !aligned16(out))
    return fail(KVM_EINVAL, "relu_square pointers must be non-NULL and 16-byte aligned");
  KVM_HIP(kvm::launch_relu_square(x, out, n, as_stream(stream)), "relu square");
  return KVM_OK;
}

int kvm_prefix(const kvm_prefix_desc *d, void *stream) {
  if (!d) return fail(KVM_EINVAL, "prefix descriptor is NULL");
  if (d->batch < 1 || d->seq_len < 1 || d->q_heads < 1 || d->kv_heads < 1)
    return fail(KVM_EINVAL, "batch, seq_len and head counts must be positive");
  if (d->head_dim != 64 && d->head_dim != 128)
    return fail(KVM_EINVAL, "head_dim must be 64 or 128, got %lld", (long long)d->head_dim);
  if (d->value_dim != d->head_dim) return fail(KVM_EINVAL, "value_dim must equal head_dim");
  if (d->value_residual_mode < 0 || d->value_residual_mode > 3)
    return fail(KVM_EINVAL, "value_residual_mode must be 0..3, got %lld", (long long)d->value_residual_mode);
  if (d->token_shift != 0 && d->token_shift != 1) return fail(KVM_EINVAL, "token_shift must be 0 or 1");
  if (!(d->ln_eps > 0.0)) return fail(KVM_EINVAL, "ln_eps must be positive");
  const void *rows[] = {d->q_lin, d->k_lin, d->v_lin, d->q_out, d->k_out, d->v_out, d->cos, d->sin,
                        d->ln_q_w, d->ln_q_b, d->ln_k_w, d->ln_k_b};
  for (const void *p : rows)
    if (!p || !aligned16(p)) return fail(KVM_EINVAL, "projection, output, RoPE and LayerNorm pointers must be non-NULL and 16-byte aligned");
  const int64_t mode = d->value_residual_mode;
  if (mode >= 1 && (!d->v_first || !aligned16(d->v_first)))
    return fail(KVM_EINVAL, "value residual needs a 16-byte aligned v_first");
  if (mode == 1 && !d->lamb) return fail(KVM_EINVAL, "linear value residual needs lamb");
  if (mode >= 2 && (!d->gate_lin || !d->v_gate0 || !aligned16(d->gate_lin) || !aligned16(d->v_gate0)))
    return fail(KVM_EINVAL, "rwkv value residual needs 16-byte aligned gate_lin and v_gate0");
  if (d->token_shift) {
    const void *mix[] = {d->x_q, d->x_k, d->x_v};
    for (const void *p : mix)
      if (!p || !aligned16(p)) return fail(KVM_EINVAL, "token shift needs 16-byte aligned x_q, x_k, x_v");
    const void *prev[] = {d->q_prev, d->k_prev, d->v_prev};
    for (const void *p : prev)
      if (p && !aligned16(p)) return fail(KVM_EINVAL, "previous-token rows must be 16-byte aligned");
  }
  if (d->v_last_out && !aligned16(d->v_last_out)) return fail(KVM_EINVAL, "v_last_out must be 16-byte aligned");
  if ((d->q_last_out && !aligned16(d->q_last_out)) || (d->k_last_out && !aligned16(d->k_last_out)))
    return fail(KVM_EINVAL, "q_last_out / k_last_out must be 16-byte aligned");
  if (d->ring_k) {
    if (d->seq_len != 1) return fail(KVM_EINVAL, "the prefix's ring write is for a single token (seq_len 1)");
    if (!d->ring_v || !d->ring_gate || !aligned16(d->ring_k) || !aligned16(d->ring_v) || d->ring_cap < 1)
      return fail(KVM_EINVAL, "ring write needs 16-byte aligned ring_k / ring_v, ring_gate and ring_cap >= 1");
    if (!d->ring_ctl && (d->ring_pos < 0 || d->ring_pos >= d->ring_cap))
      return fail(KVM_EINVAL, "ring_pos %lld outside the ring of %lld rows", (long long)d->ring_pos,
                  (long long)d->ring_cap);
  }
  if (d->rope_sb % 8 || d->rope_st % 8 || d->rope_st < d->head_dim)
    return fail(KVM_EINVAL, "cos/sin strides must be multiples of 8 elements covering head_dim");
  if (d->key_weight && !d->gate_out) return fail(KVM_EINVAL, "key_weight needs gate_out");
  const int64_t widest = std::max(d->q_heads, d->kv_heads) * d->head_dim;
  if (d->qkv_st % 8 || d->qkv_st < widest)
    return fail(KVM_EINVAL, "qkv_st must be a multiple of 8 elements covering the widest projection");
  if (d->key_weight && d->kw_st < d->kv_heads) return fail(KVM_EINVAL, "kw_st must cover kv_heads");
  KVM_HIP(kvm::launch_prefix(*d, as_stream(stream)), "prefix");
  return KVM_OK;
}

int64_t kvm_update_workspace_bytes(const kvm_layer *layer, int64_t n_tok) {
  if (check_layer(layer) != KVM_OK || n_tok < 1) return -1;
  return kvm::update_scratch_bytes(*layer, n_tok);
}

int64_t kvm_decode_workspace_bytes(const kvm_layer *layer, int64_t max_rows) {
  if (check_layer(layer) != KVM_OK) return -1;
  return kvm::decode_workspace_bytes(*layer, max_rows);
}

int64_t kvm_prefill_workspace_bytes(const kvm_prefill_desc *d) {
  if (!d || check_layer(&d->layer) != KVM_OK) return -1;
  if (d->max_state_len < 1 || d->snapshot_ring < 2) return -1;
  return int64_t(prefill_layout(d).total);
}

int kvm_state_append_direct(const kvm_layer *layer, const kvm_seq *src,
                            int64_t tok_begin, int64_t n_tok,
                            const kvm_state *st, int64_t slot_begin,
                            void *stream) {
  int rc;
  if ((rc = check_layer(layer)) || (rc = check_seq(src, "src")) ||
      (rc = check_state(st, true)))
    return rc;
  if (n_tok < 0 || tok_begin < 0 || slot_begin < 0 ||
      slot_begin + n_tok > st->capacity)
    return fail(KVM_ESPACE, "direct append of %lld tokens at slot %lld exceeds capacity %lld",
                (long long)n_tok, (long long)slot_begin, (long long)st->capacity);
  kvm::AttnRows attn{static_cast<uint16_t *>(st->s_k_attn),
                     static_cast<uint16_t *>(st->s_v_attn), st->capacity};
  KVM_HIP(kvm::launch_append_direct(*layer, *src, tok_begin, n_tok, *st,
                                    slot_begin, attn, layer->gate_initial != 0,
                                    as_stream(stream)),
          "kvm_state_append_direct");
  return KVM_OK;
}

int kvm_state_refresh(const kvm_layer *layer, const kvm_state *st,
                      int64_t slot_begin, int64_t n_slots, void *stream) {
  int rc;
  if ((rc = check_layer(layer)) || (rc = check_state(st, true))) return rc;
  if (slot_begin < 0 || n_slots < 0 || slot_begin + n_slots > st->capacity)
    return fail(KVM_EINVAL, "refresh range exceeds the state capacity");
  kvm::AttnRows attn{static_cast<uint16_t *>(st->s_k_attn),
                     static_cast<uint16_t *>(st->s_v_attn), st->capacity};
  KVM_HIP(kvm::launch_refresh(*layer, *st, slot_begin, n_slots, attn,
                              as_stream(stream)),
          "kvm_state_refresh");
  return KVM_OK;
}

int kvm_state_update(const kvm_layer *layer, const kvm_seq *src,
                     int64_t tok_begin, int64_t n_tok, int64_t state_before,
                     int64_t n_append, const kvm_state *st, void *attn_k_out,
                     void *attn_v_out, void *workspace, int64_t workspace_bytes,
                     int32_t *route_out, int32_t *append_out, void *stream) {
  int rc;
  if ((rc = check_layer(layer)) || (rc = check_seq(src, "src")) ||
      (rc = check_state(st, true)))
    return rc;
  if (n_tok < 1 || n_tok > 4096)
    return fail(KVM_EINVAL, "update token count must be in [1, 4096]");
  if (n_append < 0 || n_append > n_tok)
    return fail(KVM_EINVAL, "n_append must be in [0, n_tok]");
  if (state_before < 1)
    return fail(KVM_EINVAL, "a state update needs a non-empty state");
  const int64_t after = state_before + n_append;
  if (after > st->capacity)
    return fail(KVM_ESPACE, "state of %lld slots exceeds capacity %lld",
                (long long)after, (long long)st->capacity);
  if (n_append < n_tok && after <= std::min(layer->sink_len, after))
    return fail(KVM_EINVAL,
                "KVM state update requires at least one non-sink slot before merging.");
  if (!attn_k_out || !attn_v_out || !aligned16(attn_k_out) || !aligned16(attn_v_out))
    return fail(KVM_EINVAL, "attention output rows must be set and 16-byte aligned");
  const int64_t need = kvm::update_scratch_bytes(*layer, n_tok);
  if (!workspace || workspace_bytes < need)
    return fail(KVM_ESPACE, "update workspace of %lld bytes is smaller than %lld",
                (long long)workspace_bytes, (long long)need);
  kvm::UpdateScratch sc = kvm::carve_update_scratch(
      workspace, static_cast<unsigned char *>(workspace) + kvm::update_slice_bytes(*layer, n_tok),
      *layer, n_tok);
  kvm::AttnRows in{static_cast<uint16_t *>(st->s_k_attn),
                   static_cast<uint16_t *>(st->s_v_attn), st->capacity};
  kvm::AttnRows out{static_cast<uint16_t *>(attn_k_out),
                    static_cast<uint16_t *>(attn_v_out), st->capacity};
  hipStream_t s = as_stream(stream);
  kvm::PrepList pl;
  pl.count = 1;
  pl.tok_begin[0] = int32_t(tok_begin);
  KVM_HIP(kvm::launch_prep(*layer, *src, pl, n_tok, sc, 0, s), "kvm_state_update");
  KVM_HIP(kvm::launch_zero_keys(*layer, n_tok, sc, s), "kvm_state_update");
  KVM_HIP(kvm::launch_update(*layer, *src, tok_begin, n_tok, state_before, n_append, *st, in,
                             out, sc, 0, route_out, append_out, s),
          "kvm_state_update");
  return KVM_OK;
}

int kvm_ring_write(const kvm_layer *layer, const kvm_seq *src, void *ring_k,
                   void *ring_v, void *ring_gate, int64_t ring_cap, int64_t pos,
                   void *stream) {
  int rc;
  if ((rc = check_layer(layer)) || (rc = check_seq(src, "src"))) return rc;
  if (!ring_k || !ring_v || !ring_gate || !aligned16(ring_k) || !aligned16(ring_v))
    return fail(KVM_EINVAL, "ring buffers must be set and 16-byte aligned");
  if (ring_cap < 1 || pos < 0 || pos >= ring_cap)
    return fail(KVM_EINVAL, "ring position %lld outside [0, %lld)", (long long)pos,
                (long long)ring_cap);
  KVM_HIP(kvm::launch_ring_write(*layer, *src, ring_k, ring_v, ring_gate, ring_cap,
                                 pos, as_stream(stream)),
          "kvm_ring_write");
  return KVM_OK;
}

int kvm_ring_write_dev(const kvm_layer *layer, const kvm_seq *src, void *ring_k, void *ring_v,
                       void *ring_gate, int64_t ring_cap, const int32_t *ctl, void *stream) {
  int rc;
  if ((rc = check_layer(layer)) || (rc = check_seq(src, "src"))) return rc;
  if (!ring_k || !ring_v || !ring_gate || !aligned16(ring_k) || !aligned16(ring_v) || ring_cap < 1)
    return fail(KVM_EINVAL, "ring buffers must be set and 16-byte aligned");
  if (!ctl) return fail(KVM_EINVAL, "ctl must point to the device counters");
  KVM_HIP(kvm::launch_ring_write(*layer, *src, ring_k, ring_v, ring_gate, ring_cap, 0, as_stream(stream), ctl),
          "kvm_ring_write_dev");
  return KVM_OK;
}

int kvm_decode_advance(int32_t *ctl, int64_t n, void *stream) {
  if (!ctl || n < 1) return fail(KVM_EINVAL, "decode advance needs counters");
  KVM_HIP(kvm::launch_decode_advance(ctl, n, as_stream(stream)), "kvm_decode_advance");
  return KVM_OK;
}

int64_t kvm_prefill_backward_workspace_bytes(const kvm_prefill_bwd_desc *d) {
  if (!d || check_layer(&d->layer) != KVM_OK || d->n_chunks < 1) return -1;
  return kvm::attn_bwd_workspace_bytes(d->layer, d->n_chunks);
}

int kvm_prefill_backward(const kvm_prefill_bwd_desc *d, void *stream) {
  if (!d) return fail(KVM_EINVAL, "backward descriptor is NULL");
  int rc;
  const kvm_layer &L = d->layer;
  if ((rc = check_layer(&L)) || (rc = check_seq(&d->kv, "kv"))) return rc;
  const int64_t T = d->seq_len, C = L.chunk_len, n = L.n_bswa_chunks;
  if (T < 1) return fail(KVM_EINVAL, "seq_len must be positive");
  const int64_t n_chunks = (T + C - 1) / C;
  if (d->n_chunks != n_chunks)
    return fail(KVM_EINVAL, "n_chunks %lld != ceil(T / C) = %lld", (long long)d->n_chunks,
                (long long)n_chunks);
  if (n_chunks > kvm::kMaxChunksPerLaunch)
    return fail(KVM_EINVAL, "the backward handles at most %d query chunks", kvm::kMaxChunksPerLaunch);
  const void *need[] = {d->q, d->dout, d->lse, d->delta, d->dq, d->dk, d->dv, d->d_state_temp,
                        d->d_front_temp, d->chunk_state_len, d->chunk_snapshot};
  for (const void *p : need)
    if (!p) return fail(KVM_EINVAL, "backward: a required pointer is NULL");
  if (!aligned16(d->q) || !aligned16(d->dout) || d->q_sb % 8 || d->q_sh % 8 || d->q_st % 8 ||
      d->do_sb % 8 || d->do_sh % 8 || d->do_st % 8)
    return fail(KVM_EINVAL, "q and dout must be 16-byte aligned with strides multiple of 8");
  if (d->out && (!aligned16(d->out) || d->o_sb % 8 || d->o_sh % 8 || d->o_st % 8))
    return fail(KVM_EINVAL, "out must be 16-byte aligned with strides multiple of 8");
  const bool has_state = n_chunks > n;
  if (has_state && (!d->snap_k || !d->snap_v || !d->d_snap_k || !d->d_snap_v ||
                    !aligned16(d->snap_k) || !aligned16(d->snap_v)))
    return fail(KVM_EINVAL, "backward: snapshot arrays (and their gradients) must be set and aligned");
  if (d->max_state_len < 1) return fail(KVM_EINVAL, "max_state_len must be positive");
  kvm::ChunkTable table;
  int64_t first_snap = -1;
  for (int64_t m = 0; m < n_chunks; ++m) {
    const int32_t s = d->chunk_state_len[m], snap = d->chunk_snapshot[m];
    if (m < n) {
      table.state_len[m] = 0;
      table.snap_slot[m] = 0;
      continue;
    }
    if (snap < 0 || s < 1 || s > d->max_state_len)
      return fail(KVM_EINVAL, "chunk %lld schedule (state %d, snapshot %d) is invalid", (long long)m, s, snap);
    // Each snapshot's gradient has one writer: the chunk that reads it.
    if (m > n && snap != table.snap_slot[m - 1] + 1)
      return fail(KVM_EINVAL, "chunk %lld reads snapshot %d: snapshots must be read once each, in order",
                  (long long)m, snap);
    if (m == n) first_snap = snap;
    table.state_len[m] = s;
    table.snap_slot[m] = snap;
  }
  const int64_t need_ws = kvm::attn_bwd_workspace_bytes(L, n_chunks);
  if (!d->workspace || d->workspace_bytes < need_ws)
    return fail(KVM_ESPACE, "backward workspace of %lld bytes is smaller than %lld",
                (long long)d->workspace_bytes, (long long)need_ws);
  kvm::BwdArgs a;
  a.q = d->q;
  a.q_sb = d->q_sb; a.q_sh = d->q_sh; a.q_st = d->q_st;
  a.kv = d->kv;
  a.T = T;
  a.dout = d->dout;
  a.do_sb = d->do_sb; a.do_st = d->do_st; a.do_sh = d->do_sh;
  a.lse = d->lse;
  a.delta = d->delta;
  a.snap_k = static_cast<const uint16_t *>(d->snap_k);
  a.snap_v = static_cast<const uint16_t *>(d->snap_v);
  const int64_t rows = L.batch * L.kv_heads;
  a.snap_stride = rows * d->max_state_len * L.head_dim;
  a.snap_cap = d->max_state_len;
  a.n_chunks = n_chunks;
  a.dq = d->dq;
  a.dq_sb = d->dq_sb; a.dq_sh = d->dq_sh; a.dq_st = d->dq_st;
  a.dk = d->dk;
  a.dv = d->dv;
  a.d_snap_k = d->d_snap_k;
  a.d_snap_v = d->d_snap_v;
  a.dsnap_stride = a.snap_stride;
  a.d_state_temp = d->d_state_temp;
  a.d_front_temp = d->d_front_temp;
  hipStream_t s = as_stream(stream);
  // Snapshots below the first one read keep a zero gradient (the snapshot
  // kernel writes every row of the ones read, zeros past their length).
  if (has_state && first_snap > 0) {
    const int64_t words = first_snap * a.snap_stride;
    KVM_HIP(kvm::launch_fill_u32(reinterpret_cast<unsigned *>(d->d_snap_k), words, 0u, s), "d_snap_k clear");
    KVM_HIP(kvm::launch_fill_u32(reinterpret_cast<unsigned *>(d->d_snap_v), words, 0u, s), "d_snap_v clear");
  }
  if (d->out)
    KVM_HIP(kvm::launch_attn_delta(L, d->dout, d->do_sb, d->do_st, d->do_sh, d->out, d->o_sb, d->o_st, d->o_sh, T,
                                   d->delta, s),
            "delta");
  KVM_HIP(kvm::launch_attn_backward(L, a, table, static_cast<float *>(d->workspace), s), "attention backward");
  return KVM_OK;
}

int64_t kvm_state_backward_workspace_bytes(const kvm_state_bwd_desc *d) {
  if (!d || check_layer(&d->layer) != KVM_OK || d->max_state_len < 1) return -1;
  return kvm::state_bwd_workspace_bytes(d->layer.head_dim, d->layer.batch * d->layer.kv_heads, d->max_state_len);
}

int kvm_state_backward(const kvm_state_bwd_desc *d, void *stream) {
  if (!d) return fail(KVM_EINVAL, "state backward descriptor is NULL");
  int rc;
  const kvm_layer &L = d->layer;
  if ((rc = check_layer(&L)) || (rc = check_seq(&d->kv, "kv"))) return rc;
  if (d->kv.ring) return fail(KVM_EINVAL, "state backward: the token source cannot be a ring");
  const int64_t D = L.head_dim, T = d->seq_len, C = L.chunk_len, L0 = d->initial_state_len,
                nu = d->n_updates, S = d->max_state_len, rows = L.batch * L.kv_heads;
  if (T < 1 || L0 != std::min(T, C) || S < L0 || nu < 0)
    return fail(KVM_EINVAL, "state backward: sizes out of range (initial_state_len must be min(T, chunk_len))");
  if (C > kvm::state_bwd_max_chunk())
    return fail(KVM_EINVAL, "state backward: chunk_len above %lld", (long long)kvm::state_bwd_max_chunk());
  if (nu >= kvm::kMaxChunksPerLaunch)
    return fail(KVM_EINVAL, "state backward handles at most %d updates", kvm::kMaxChunksPerLaunch - 1);
  const void *need[] = {d->d_snap_k, d->d_snap_v, d->dk, d->dv, d->dgate, d->d_ln};
  for (const void *p : need)
    if (!p || !aligned16(p)) return fail(KVM_EINVAL, "state backward: a required pointer is NULL or unaligned");
  kvm::UpdTable U;
  int64_t len = L0, prev_end = L0;
  for (int64_t u = 0; u < nu; ++u) {
    if (!d->upd_token_begin || !d->upd_state_before || !d->upd_n_append)
      return fail(KVM_EINVAL, "state backward: the update schedule is NULL");
    const int32_t tb = d->upd_token_begin[u], before = d->upd_state_before[u], na = d->upd_n_append[u];
    // Update chunks are disjoint, follow the initial tokens and hold C tokens each.
    if (tb < prev_end || tb + C > T || before != len || na < 0 || na > C || before + na > S)
      return fail(KVM_EINVAL, "update %lld schedule (token %d, state %d + %d) is invalid", (long long)u, tb,
                  before, na);
    U.token_begin[u] = tb;
    U.state_before[u] = before;
    U.n_append[u] = na;
    len = before + na;
    prev_end = tb + C;
  }
  if (nu > 0 && (!d->route_log || !d->append_log))
    return fail(KVM_EINVAL, "state backward: route_log and append_log are required");
  const int64_t need_ws = kvm::state_bwd_workspace_bytes(D, rows, S);
  if (!d->workspace || d->workspace_bytes < need_ws || !aligned16(d->workspace))
    return fail(KVM_ESPACE, "state backward workspace of %lld bytes is smaller than %lld",
                (long long)d->workspace_bytes, (long long)need_ws);
  kvm::StateBwdArgs a;
  a.L = L;
  a.kv = d->kv;
  a.rows = rows; a.T = T; a.L0 = L0; a.n_updates = nu; a.max_state_len = S;
  a.route_log = d->route_log; a.append_log = d->append_log;
  a.d_snap_k = d->d_snap_k; a.d_snap_v = d->d_snap_v;
  a.dk = d->dk; a.dv = d->dv; a.dgate = d->dgate;
  a.d_ln = d->d_ln;
  KVM_HIP(kvm::launch_state_backward(a, U, static_cast<float *>(d->workspace), as_stream(stream)),
          "state backward");
  return KVM_OK;
}

int kvm_decode_attention_dev(const kvm_layer *layer, const void *q, int64_t q_sb, int64_t q_sh,
                             const kvm_state *st, const int32_t *ctl, int32_t pending, const void *ring_k,
                             const void *ring_v, int64_t ring_cap, void *out, int64_t o_sb, int64_t o_sh,
                             void *workspace, int64_t workspace_bytes, void *stream) {
  int rc;
  if ((rc = check_layer(layer)) || (rc = check_state(st, true))) return rc;
  if (!q || !aligned16(q) || q_sb % 8 || q_sh % 8)
    return fail(KVM_EINVAL, "q must be 16-byte aligned with strides multiple of 8");
  if (!out) return fail(KVM_EINVAL, "out must be set");
  if (!ring_k || !ring_v || !aligned16(ring_k) || !aligned16(ring_v) || ring_cap < 1)
    return fail(KVM_EINVAL, "ring buffers must be set and 16-byte aligned");
  if (!ctl) return fail(KVM_EINVAL, "ctl must point to the device counters");
  if (pending < 0 || pending > 1) return fail(KVM_EINVAL, "pending must be 0 or 1");
  const int64_t max_rows = st->capacity + ring_cap;
  const int64_t need = kvm::decode_workspace_bytes(*layer, max_rows);
  if (!workspace || workspace_bytes < need)
    return fail(KVM_ESPACE, "decode workspace of %lld bytes is smaller than %lld",
                (long long)workspace_bytes, (long long)need);
  KVM_HIP(kvm::launch_decode(*layer, q, q_sb, q_sh, *st, 0, ring_k, ring_v, ring_cap, 0, 0, out, o_sb, o_sh,
                             workspace, as_stream(stream), ctl, int(pending), max_rows),
          "kvm_decode_attention_dev");
  return KVM_OK;
}

int kvm_decode_attention_noalloc(const kvm_layer *layer, const void *q, int64_t q_sb,
                                 int64_t q_sh, const kvm_state *st,
                                 int64_t active_state_len, const void *ring_k,
                                 const void *ring_v, int64_t ring_cap,
                                 int64_t ring_start, int64_t recent_len, void *out,
                                 int64_t o_sb, int64_t o_sh, void *stream) {
  if (check_layer(layer) != KVM_OK) return KVM_EINVAL;
  const int64_t need = kvm::decode_workspace_bytes(*layer, active_state_len + recent_len);
  if (need > int64_t(KVM_DECODE_SCRATCH_BYTES))
    return fail(KVM_ESPACE,
                "decode needs %lld bytes of scratch; the allocation-free entry point holds %lld "
                "(use kvm_decode_attention with a workspace)",
                (long long)need, (long long)KVM_DECODE_SCRATCH_BYTES);
  void *scratch = nullptr;
  KVM_HIP(kvm::decode_scratch(&scratch), "decode scratch address");
  return kvm_decode_attention(layer, q, q_sb, q_sh, st, active_state_len, ring_k, ring_v,
                              ring_cap, ring_start, recent_len, out, o_sb, o_sh, scratch,
                              int64_t(KVM_DECODE_SCRATCH_BYTES), stream);
}

int kvm_decode_attention(const kvm_layer *layer, const void *q, int64_t q_sb,
                         int64_t q_sh, const kvm_state *st,
                         int64_t active_state_len, const void *ring_k,
                         const void *ring_v, int64_t ring_cap,
                         int64_t ring_start, int64_t recent_len, void *out,
                         int64_t o_sb, int64_t o_sh, void *workspace,
                         int64_t workspace_bytes, void *stream) {
  int rc;
  if ((rc = check_layer(layer)) || (rc = check_state(st, true))) return rc;
  if (!q || !aligned16(q) || q_sb % 8 || q_sh % 8)
    return fail(KVM_EINVAL, "q must be 16-byte aligned with strides multiple of 8");
  if (!out) return fail(KVM_EINVAL, "out must be set");
  if (!ring_k || !ring_v || !aligned16(ring_k) || !aligned16(ring_v) || ring_cap < 1)
    return fail(KVM_EINVAL, "ring buffers must be set and 16-byte aligned");
  if (active_state_len < 0 || active_state_len > st->capacity)
    return fail(KVM_EINVAL, "active state length outside the state capacity");
  if (recent_len < 0 || recent_len > ring_cap || ring_start < 0 || ring_start >= ring_cap)
    return fail(KVM_EINVAL, "recent window outside the ring");
  if (active_state_len + recent_len < 1)
    return fail(KVM_EINVAL, "decode attention needs at least one key row");
  const int64_t need = kvm::decode_workspace_bytes(*layer, active_state_len + recent_len);
  if (!workspace || workspace_bytes < need)
    return fail(KVM_ESPACE, "decode workspace of %lld bytes is smaller than %lld",
                (long long)workspace_bytes, (long long)need);
  KVM_HIP(kvm::launch_decode(*layer, q, q_sb, q_sh, *st, active_state_len, ring_k,
                             ring_v, ring_cap, ring_start, recent_len, out, o_sb,
                             o_sh, workspace, as_stream(stream)),
          "kvm_decode_attention");
  return KVM_OK;
}

int kvm_decode_step(const kvm_layer *layer, const void *q, int64_t q_sb, int64_t q_sh,
                    const kvm_state *st, int64_t active_state_len, const kvm_seq *src,
                    void *ring_k, void *ring_v, void *ring_gate, int64_t ring_cap,
                    int64_t ring_start, int64_t recent_len, void *out, int64_t o_sb,
                    int64_t o_sh, void *workspace, int64_t workspace_bytes, void *stream) {
  int rc;
  if ((rc = check_seq(src, "src"))) return rc;
  if (src->ring != 0) return fail(KVM_EINVAL, "the step's token cannot come from a ring");
  if (!ring_gate) return fail(KVM_EINVAL, "ring_gate must be set");
  if (recent_len < 1) return fail(KVM_EINVAL, "the step's token must be the last window row");
  if ((rc = check_layer(layer)) || (rc = check_state(st, true))) return rc;
  if (!q || !aligned16(q) || q_sb % 8 || q_sh % 8)
    return fail(KVM_EINVAL, "q must be 16-byte aligned with strides multiple of 8");
  if (!out) return fail(KVM_EINVAL, "out must be set");
  if (!ring_k || !ring_v || !aligned16(ring_k) || !aligned16(ring_v) || ring_cap < 1)
    return fail(KVM_EINVAL, "ring buffers must be set and 16-byte aligned");
  if (active_state_len < 0 || active_state_len > st->capacity)
    return fail(KVM_EINVAL, "active state length outside the state capacity");
  if (recent_len > ring_cap || ring_start < 0 || ring_start >= ring_cap)
    return fail(KVM_EINVAL, "recent window outside the ring");
  const int64_t need = kvm::decode_workspace_bytes(*layer, active_state_len + recent_len);
  if (!workspace || workspace_bytes < need)
    return fail(KVM_ESPACE, "decode workspace of %lld bytes is smaller than %lld",
                (long long)workspace_bytes, (long long)need);
  KVM_HIP(kvm::launch_decode(*layer, q, q_sb, q_sh, *st, active_state_len, ring_k, ring_v,
                             ring_cap, ring_start, recent_len, out, o_sb, o_sh, workspace,
                             as_stream(stream), nullptr, 0, 0, src, ring_gate),
          "kvm_decode_step");
  return KVM_OK;
}

int kvm_prefill(const kvm_prefill_desc *d, void *stream) {
  if (!d) return fail(KVM_EINVAL, "prefill descriptor is NULL");
  int rc;
  const kvm_layer &L = d->layer;
  if ((rc = check_layer(&L)) || (rc = check_seq(&d->kv, "kv")) ||
      (rc = check_state(&d->state, false)))
    return rc;
  if (d->kv.ring != 0) return fail(KVM_EINVAL, "prefill tokens cannot come from a ring");
  if (!d->q || !aligned16(d->q) || d->q_sb % 8 || d->q_sh % 8 || d->q_st % 8)
    return fail(KVM_EINVAL, "q must be 16-byte aligned with strides multiple of 8");
  if (!d->out || !aligned16(d->out) || d->o_sb % 4 || d->o_st % 4 || d->o_sh % 4)
    return fail(KVM_EINVAL, "out must be 16-byte aligned with strides multiple of 4");
  const int64_t T = d->seq_len, C = L.chunk_len, n = L.n_bswa_chunks;
  if (T < 1) return fail(KVM_EINVAL, "seq_len must be positive");
  const int64_t n_chunks = (T + C - 1) / C;
  if (d->n_chunks != n_chunks)
    return fail(KVM_EINVAL, "n_chunks %lld != ceil(T / C) = %lld",
                (long long)d->n_chunks, (long long)n_chunks);
  if (!d->chunk_state_len || !d->chunk_snapshot)
    return fail(KVM_EINVAL, "chunk schedule arrays must be set");
  if (d->n_updates < 0 || (d->n_updates > 0 && (!d->upd_token_begin ||
                                                !d->upd_state_before ||
                                                !d->upd_n_append)))
    return fail(KVM_EINVAL, "update schedule arrays must be set");
  if (d->snapshot_ring < 2) return fail(KVM_EINVAL, "snapshot_ring must be >= 2");
  if (!d->snap_k != !d->snap_v) return fail(KVM_EINVAL, "snap_k and snap_v must be set together");
  if (d->snap_k) {
    if (d->snapshot_ring != std::max<int64_t>(2, d->n_updates + 1))
      return fail(KVM_EINVAL, "caller-held snapshots need snapshot_ring = max(2, n_updates + 1)");
    if (!aligned16(d->snap_k) || !aligned16(d->snap_v))
      return fail(KVM_EINVAL, "snapshot arrays must be 16-byte aligned");
  }
  if (d->lse && (reinterpret_cast<uintptr_t>(d->lse) & 3u))
    return fail(KVM_EINVAL, "lse must be 4-byte aligned");
  const int64_t L0 = std::min(T, C);
  if (d->max_state_len < L0 || d->max_state_len > d->state.capacity)
    return fail(KVM_ESPACE, "max_state_len %lld must be in [%lld, capacity %lld]",
                (long long)d->max_state_len, (long long)L0,
                (long long)d->state.capacity);
  // Schedule sanity: chunk m >= n sees the snapshot after m - n updates.
  for (int64_t m = 0; m < n_chunks; ++m) {
    const int32_t s = d->chunk_state_len[m], snap = d->chunk_snapshot[m];
    if (m < n) {
      if (s != 0) return fail(KVM_EINVAL, "front chunk %lld must see no memory slots", (long long)m);
      continue;
    }
    if (snap < 0 || snap > d->n_updates || s < 1 || s > d->max_state_len)
      return fail(KVM_EINVAL, "chunk %lld schedule (state %d, snapshot %d) is invalid",
                  (long long)m, s, snap);
    if (m > n && snap < d->chunk_snapshot[m - 1])
      return fail(KVM_EINVAL, "chunk snapshots must be nondecreasing");
  }
  int64_t cur = L0;
  for (int64_t u = 0; u < d->n_updates; ++u) {
    const int64_t tb = d->upd_token_begin[u];
    if (d->upd_state_before[u] != cur)
      return fail(KVM_EINVAL, "update %lld starts from %d slots, schedule has %lld",
                  (long long)u, d->upd_state_before[u], (long long)cur);
    if (tb < 0 || tb % C || tb + C > T)
      return fail(KVM_EINVAL, "update %lld overflow chunk at token %lld is invalid",
                  (long long)u, (long long)tb);
    const int64_t na = d->upd_n_append[u];
    if (na < 0 || na > C) return fail(KVM_EINVAL, "update %lld append count invalid", (long long)u);
    if (na < C && cur + na <= std::min(L.sink_len, cur + na))
      return fail(KVM_EINVAL,
                  "KVM state update requires at least one non-sink slot before merging.");
    cur += na;
    if (cur > d->max_state_len)
      return fail(KVM_ESPACE, "state grows past max_state_len");
  }
  const PrefillLayout lay = prefill_layout(d);
  if (!d->workspace || d->workspace_bytes < int64_t(lay.total))
    return fail(KVM_ESPACE, "prefill workspace of %lld bytes is smaller than %lld",
                (long long)d->workspace_bytes, (long long)lay.total);
  if (reinterpret_cast<uintptr_t>(d->status) & 3u)
    return fail(KVM_EINVAL, "status word must be 4-byte aligned");

  hipStream_t s = as_stream(stream);
  auto mark = [&](int i) -> int {
    if (d->events && d->events[i])
      KVM_HIP(hipEventRecord(static_cast<hipEvent_t>(d->events[i]), s), "event record");
    return KVM_OK;
  };
  unsigned char *ws = static_cast<unsigned char *>(d->workspace);
  kvm::UpdateScratch sc = kvm::carve_update_scratch(ws, ws + lay.slices * lay.slice_bytes, L, C);
  uint16_t *snap_k = reinterpret_cast<uint16_t *>(ws + lay.update_bytes);
  size_t snap_bytes = align256(lay.snap_elems * 2);
  uint16_t *snap_v = reinterpret_cast<uint16_t *>(
      ws + lay.update_bytes + size_t(d->snapshot_ring) * snap_bytes);
  if (d->snap_k) {  // the caller's dense [n_updates + 1, rows, max_state_len, D] arrays
    snap_k = static_cast<uint16_t *>(d->snap_k);
    snap_v = static_cast<uint16_t *>(d->snap_v);
    snap_bytes = lay.snap_elems * 2;
  }
  const int64_t snap_stride = int64_t(snap_bytes / 2);
  const int64_t R = d->snapshot_ring;
  auto snap_rows = [&](int64_t idx) {
    return kvm::AttnRows{snap_k + (idx % R) * snap_stride,
                         snap_v + (idx % R) * snap_stride, d->max_state_len};
  };

  // Updates run as persistent chains when the shape fits (one launch per
  // batch of updates), else as per-update kernels.  KVM_PREFILL_NO_CHAIN in
  // the call's flags, or KVM_AMD_CHAIN=0, forces the per-update kernels.
  kvm::ChainPlan cp;
  const char *chain_env = getenv("KVM_AMD_CHAIN");
  const bool use_chain = !(d->flags & KVM_PREFILL_NO_CHAIN) && !(chain_env && chain_env[0] == '0') &&
                         kvm::chain_plan(L, C, d->max_state_len, &cp);

  // Status word of the chain: the caller's (sticky, never cleared here), or
  // one in the workspace, cleared now and checked at the end of the call.
  const bool own_status = d->status == nullptr;
  unsigned *status = own_status ? reinterpret_cast<unsigned *>(ws + lay.status_off)
                                : reinterpret_cast<unsigned *>(d->status);
  if (own_status && use_chain) KVM_HIP(kvm::launch_fill_u32(status, 1, 0u, s), "status reset");

  // Initial state: the first min(T, C) tokens (model/kvm_mixer.py:434-447).
  if ((rc = mark(0)) != KVM_OK) return rc;
  if (!use_chain) KVM_HIP(kvm::launch_zero_keys(L, C, sc, s), "key reset");
  KVM_HIP(kvm::launch_append_direct(L, d->kv, 0, L0, d->state, 0, snap_rows(0),
                                    L.gate_initial != 0, s),
          "initial state");

  kvm::PrefillAttnArgs a;
  a.q = d->q;
  a.q_sb = d->q_sb; a.q_sh = d->q_sh; a.q_st = d->q_st;
  a.kv = d->kv;
  a.T = T;
  a.out = d->out;
  a.o_sb = d->o_sb; a.o_st = d->o_st; a.o_sh = d->o_sh;
  a.snap_k = snap_k;
  a.snap_v = snap_v;
  a.snap_stride = snap_stride;
  a.snap_cap = d->max_state_len;
  a.lse = d->lse;

  int64_t next_chunk = 0;
  bool attn_marked = false;
  // Launch attention for every chunk whose snapshot index is < ready.
  auto flush = [&](int64_t ready) -> int {
    if (!attn_marked && next_chunk < n_chunks) {
      int r = mark(2);
      if (r != KVM_OK) return r;
      attn_marked = true;
    }
    while (next_chunk < n_chunks &&
           (next_chunk < n || d->chunk_snapshot[next_chunk] < ready)) {
      kvm::ChunkTable table;
      int64_t cnt = 0;
      while (next_chunk + cnt < n_chunks && cnt < kvm::kMaxChunksPerLaunch) {
        const int64_t m = next_chunk + cnt;
        if (m >= n && d->chunk_snapshot[m] >= ready) break;
        table.state_len[cnt] = m >= n ? d->chunk_state_len[m] : 0;
        table.snap_slot[cnt] = m >= n ? int32_t(d->chunk_snapshot[m] % R) : 0;
        ++cnt;
      }
      KVM_HIP(kvm::launch_prefill_attention(L, a, next_chunk, cnt, table, s),
              "prefill attention");
      next_chunk += cnt;
    }
    return KVM_OK;
  };

  const size_t log_stride = size_t(L.batch * L.kv_heads) * size_t(C);
  bool attn_rows_written = false;
  if (use_chain) {
    // Batches of consecutive updates, one persistent launch each.  A batch
    // [u, e) writes snapshots u+1..e into ring slots: every chunk reading a
    // snapshot <= e - R is launched first, which needs e <= u + R.
    kvm::ChainScratch cs = kvm::carve_chain_scratch(ws, L, C);
    cs.status = status;
    // KVM_AMD_CHAIN_POLLS overrides the poll budget of a group wait (0 makes
    // every wait give up at once: the error path, with every workgroup
    // leaving normally).
    if (const char *polls = getenv("KVM_AMD_CHAIN_POLLS"))
      cs.max_polls = unsigned(strtoul(polls, nullptr, 10));
    // KVM_AMD_CHAIN_FIXED=0 keeps batches without appends on the token-split kernel.
    const char *fixed_env = getenv("KVM_AMD_CHAIN_FIXED");
    const kvm::SnapRing ring{snap_k, snap_v, snap_stride, R, d->max_state_len};
    for (int64_t u = 0; u < d->n_updates;) {
      int64_t e = std::min({d->n_updates, u + int64_t(kvm::kChainMax), u + R});
      // A batch whose updates stop appending part-way (a growing budget that
      // reaches its cap) ends where they stop: the tail, whose state length
      // no longer changes, runs on the slot-owner kernel in the next launch.
      {
        int64_t tail = e;
        while (tail > u + 1 && d->upd_n_append[tail - 1] == 0 &&
               d->upd_state_before[tail - 1] == d->upd_state_before[e - 1])
          --tail;
        if (tail > u && tail < e && (d->upd_n_append[tail - 1] != 0 ||
                                     d->upd_state_before[tail - 1] != d->upd_state_before[e - 1]))
          e = tail;
      }
      if (e - R >= 0) {
        if ((rc = flush(u + 1)) != KVM_OK) return rc;
        if (next_chunk < n_chunks && next_chunk >= n && d->chunk_snapshot[next_chunk] <= e - R)
          return fail(KVM_EINVAL, "snapshot ring too small for the schedule");
      }
      kvm::ChainList cl;
      cl.u0 = int32_t(u);
      cl.count = int32_t(e - u);
      for (int64_t i = u; i < e; ++i) {
        cl.tok_begin[i - u] = d->upd_token_begin[i];
        cl.state_before[i - u] = d->upd_state_before[i];
        cl.n_append[i - u] = d->upd_n_append[i];
      }
      kvm::ChainPlan bp = cp;
      bp.fixed = !(fixed_env && fixed_env[0] == '0') && kvm::chain_fixed_ok(cp, cl, C);
      // The fixed chain's last batch writes the final attention rows itself.
      cl.final_rows = int32_t(bp.fixed && e == d->n_updates && d->state.s_k_attn && d->state.s_v_attn);
      attn_rows_written = cl.final_rows != 0;
      KVM_HIP(kvm::launch_chain(L, d->kv, C, d->state, ring, cl, cs, bp, d->route_log,
                                d->append_log, s),
              "state update chain");
      u = e;
    }
  }
  for (int64_t u = 0; !use_chain && u < d->n_updates; ++u) {
    // Snapshot u + 1 overwrites ring slot (u + 1) % R: every chunk reading
    // snapshot u + 1 - R must have been launched (stream order does the rest).
    if (u + 1 - R >= 0) {
      if ((rc = flush(u + 1)) != KVM_OK) return rc;
      if (next_chunk < n_chunks && next_chunk >= n &&
          d->chunk_snapshot[next_chunk] <= u + 1 - R)
        return fail(KVM_EINVAL, "snapshot ring too small for the schedule");
    }
    // Overflow-token streams of the next batch of updates, ahead of the chain.
    if (u % int64_t(lay.slices) == 0) {
      kvm::PrepList pl;
      pl.count = int32_t(std::min<int64_t>(int64_t(lay.slices), d->n_updates - u));
      for (int i = 0; i < pl.count; ++i) pl.tok_begin[i] = d->upd_token_begin[u + i];
      KVM_HIP(kvm::launch_prep(L, d->kv, pl, C, sc, int64_t(lay.slice_bytes), s), "prep");
    }
    const kvm::UpdateScratch su =
        kvm::scratch_slice(sc, int64_t(lay.slice_bytes), int(u % int64_t(lay.slices)));
    KVM_HIP(kvm::launch_update(L, d->kv, d->upd_token_begin[u], C, d->upd_state_before[u],
                               d->upd_n_append[u], d->state, snap_rows(u), snap_rows(u + 1), su,
                               int(u & 1), d->route_log ? d->route_log + u * log_stride : nullptr,
                               d->append_log ? d->append_log + u * log_stride : nullptr, s),
            "state update");
  }
  if ((rc = mark(1)) != KVM_OK) return rc;
  if ((rc = flush(d->n_updates + 1)) != KVM_OK) return rc;
  if ((rc = mark(3)) != KVM_OK) return rc;

  // Final attention rows into the caller's state (unless the chain wrote them).
  if (d->state.s_k_attn && d->state.s_v_attn && !attn_rows_written) {
    const kvm::AttnRows last = snap_rows(d->n_updates);
    const size_t row_bytes = size_t(cur) * size_t(L.head_dim) * 2;
    const size_t dpitch = size_t(d->state.capacity) * size_t(L.head_dim) * 2;
    const size_t spitch = size_t(d->max_state_len) * size_t(L.head_dim) * 2;
    const size_t rows = size_t(L.batch * L.kv_heads);
    KVM_HIP(hipMemcpy2DAsync(d->state.s_k_attn, dpitch, last.k, spitch, row_bytes,
                             rows, hipMemcpyDeviceToDevice, s),
            "final key rows");
    KVM_HIP(hipMemcpy2DAsync(d->state.s_v_attn, dpitch, last.v, spitch, row_bytes,
                             rows, hipMemcpyDeviceToDevice, s),
            "final value rows");
  }
  if (own_status && use_chain) {
    unsigned word = 0;
    KVM_HIP(hipMemcpyAsync(&word, status, sizeof(word), hipMemcpyDeviceToHost, s), "status read");
    KVM_HIP(hipStreamSynchronize(s), "status read");
    if (word & KVM_STATUS_CHAIN_TIMEOUT)
      return fail(KVM_EABORT,
                  "the persistent update chain timed out waiting for its row group (another "
                  "workload held compute units); state and outputs of this prefill are incomplete");
  }
  return KVM_OK;
}

}  // extern "C"
