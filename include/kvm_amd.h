/*
 * kvm_amd.h - C ABI of the MI355X (gfx950) Key-Value Means forward path.
 *
 * The library (libkvm_amd.so, built from kvm-paper_amd/csrc) implements the
 * forward path of the KVM token mixer at the post-QKV boundary: prefill
 * (block-sliding-window attention plus attention over compressed memory
 * slots), the block-boundary memory update (routing, append, merge) and
 * single-token decode.  Every entry point takes plain device pointers,
 * element strides and sizes; nothing here names a torch type.  All work is
 * enqueued on the caller's HIP stream (`stream`, a hipStream_t; NULL is the
 * legacy default stream).  No entry point allocates device memory: scratch
 * space is passed in as `workspace`, sized by the matching
 * *_workspace_bytes() query.  No entry point synchronises, except
 * kvm_prefill when the caller passes no status word (see kvm_prefill_desc).
 *
 * Tensors
 *   bf16 tensors are stored as raw 16-bit bfloat16; the last (feature) axis
 *   is always contiguous and every other axis is described by an element
 *   stride.  "rows" are (batch, kv_head) pairs, row = b * kv_heads + h.
 *   State tensors are dense [rows, capacity, dim] (bf16) and
 *   [rows, capacity] (fp32 vlen), the layout of the reference decode cache
 *   (model/kvm_triton_decode.py:73-105).
 *
 * Errors
 *   Entry points return KVM_OK (0) or a negative code; kvm_last_error()
 *   returns a thread-local message describing the last failure.
 *   KVM_EINVAL marks an argument the reference would reject with ValueError
 *   or AssertionError, KVM_EHIP a HIP runtime failure, KVM_ESPACE a
 *   workspace or capacity that is too small (RuntimeError in the reference,
 *   model/kvm_triton_decode.py:207-211), KVM_EABORT a device-side failure
 *   reported through a status word (RuntimeError in the Python binding).
 *
 * Numeric contract (the reference's Triton path, model/kvm_triton_mixer.py:199-211,
 * evaluated against the eager golden model/kvm_mixer.py with the FP32
 * routing of model/kvm_fp32_routing_reference.py:24-49):
 *   - routing keys  prep(k) = LayerNorm_s(k with dims < rope_partial_dim
 *     zeroed), rounded to bf16; gated streams bf16(prep(k) * g), bf16(v * g);
 *   - append novelty scores bf16-rounded dot products, lowest first, ties to
 *     the lower token index;
 *   - merge routing fp32 dot products of bf16 operands, first maximum wins,
 *     the first sink_len slots never receive merges;
 *   - merge sums accumulated in fp32 in token order (deterministic), then
 *     state = bf16(state + bf16(sum)) as the eager bf16 arithmetic does;
 *   - attention keys bf16(key * temperature), fp32 scores and softmax,
 *     probabilities rounded to bf16 for the PV product, fp32 accumulation.
 */
#ifndef KVM_AMD_H
#define KVM_AMD_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define KVM_ABI_VERSION 12

#define KVM_OK 0
#define KVM_EINVAL (-1)
#define KVM_EHIP (-2)
#define KVM_ESPACE (-3)
#define KVM_EABORT (-4) /* the device reported an incomplete result (see status words) */

/* Bits of a device status word (kvm_prefill_desc.status). */
#define KVM_STATUS_CHAIN_TIMEOUT 1 /* a persistent update chain gave up waiting for its
                                      row group: state, snapshots and outputs of that
                                      prefill are incomplete */

/* Bits of kvm_prefill_desc.flags. */
#define KVM_PREFILL_NO_CHAIN 1 /* run the memory updates as per-update kernels instead of a
                                  persistent chain (bit-identical results; no requirement
                                  that every workgroup of the chain be resident at once, so
                                  it completes on a GPU shared with other work) */

/* Static description of one KVM layer (the mixer attributes the forward
 * path reads: model/kvm_mixer.py:79-118, model/rwkv7_backbone.py:319-373).
 * All fields are 8 bytes wide so the struct has no padding. */
typedef struct kvm_layer {
  int64_t batch;
  int64_t q_heads;          /* num_attention_heads */
  int64_t kv_heads;         /* num_key_value_heads (q_heads % kv_heads == 0) */
  int64_t head_dim;         /* d_qk_head: 64 or 128 */
  int64_t value_dim;        /* d_v_head: must equal head_dim */
  int64_t chunk_len;        /* C: 1..4096 */
  int64_t n_bswa_chunks;    /* n: window = n * C tokens */
  int64_t sink_len;         /* slots never merged into */
  int64_t rope_partial_dim; /* dims zeroed before LayerNorm_s (already mapped from <=0 to head_dim) */
  int64_t gate_keys;        /* kvm_use_merge_gate_keys */
  int64_t gate_values;      /* kvm_use_merge_gate_values */
  int64_t gate_appends;     /* kvm_apply_merge_gate_to_appends */
  int64_t gate_initial;     /* kvm_apply_merge_gate_to_initial_state */
  double ln_eps;            /* ln_s_k.eps */
  const void *ln_weight;    /* fp32 [head_dim] (ln_s_k.weight) */
  const void *ln_bias;      /* fp32 [head_dim] (ln_s_k.bias) */
  const void *state_temp;   /* fp32 [q_heads] (state_head_temp, ones when disabled) */
  const void *front_temp;   /* fp32 [q_heads] (front_head_temp, ones when disabled) */
} kvm_layer;

/* A token source: keys, values and merge gates of every (batch, kv_head).
 * Element (b, h, t, :) of k lives at k + b*k_sb + h*k_sh + t*k_st.  When
 * ring > 0 the token index is taken modulo ring (the decode window ring). */
typedef struct kvm_seq {
  const void *k;            /* bf16 [B, Hkv, *, head_dim] */
  const void *v;            /* bf16 [B, Hkv, *, value_dim] */
  const void *gate;         /* bf16 [B, Hkv, *, 1] */
  int64_t k_sb, k_sh, k_st;
  int64_t v_sb, v_sh, v_st;
  int64_t g_sb, g_sh, g_st;
  int64_t ring;
} kvm_seq;

/* Carried memory state (model/kvm_triton_decode.py:73-105):
 * s_k, s_v         bf16 [rows, capacity, dim] running key / value sums
 * s_vlen           fp32 [rows, capacity]      value norms (kvm_use_vlens=1)
 * s_k_attn         bf16 [rows, capacity, dim] LayerNorm_s(s_k)
 * s_v_attn         bf16 [rows, capacity, dim] bf16(normalize(s_v) * s_vlen) */
typedef struct kvm_state {
  void *s_k;
  void *s_v;
  void *s_vlen;
  void *s_k_attn;
  void *s_v_attn;
  int64_t capacity;
} kvm_state;

/* One prefill (model/kvm_triton_mixer.py:560-666 forward_prefill, eager
 * semantics model/kvm_mixer.py:403-516).  The schedule arrays are HOST
 * int32 arrays computed by the caller from the state budget
 * (model/kernels/kvm_triton_training_kernels.py:85-171). */
typedef struct kvm_prefill_desc {
  kvm_layer layer;
  const void *q;                 /* bf16 [B, Hq, T, head_dim] */
  int64_t q_sb, q_sh, q_st;
  kvm_seq kv;                    /* k, v, gate of the prompt (ring = 0) */
  int64_t seq_len;               /* T */
  void *out;                     /* bf16 out[b, t, hq, :] at out + b*o_sb + t*o_st + hq*o_sh */
  int64_t o_sb, o_st, o_sh;
  kvm_state state;               /* receives the final state; capacity >= final length */
  int64_t n_chunks;              /* ceil(T / C) */
  const int32_t *chunk_state_len;/* host [n_chunks]: memory slots visible to query chunk m */
  const int32_t *chunk_snapshot; /* host [n_chunks]: updates applied before chunk m */
  int64_t n_updates;
  const int32_t *upd_token_begin;/* host [n_updates]: first token of the overflow chunk */
  const int32_t *upd_state_before;/* host [n_updates] */
  const int32_t *upd_n_append;   /* host [n_updates] */
  int64_t max_state_len;         /* largest state length reached (snapshot row count) */
  int64_t snapshot_ring;         /* snapshots kept in the workspace (>= 2) */
  void *workspace;
  int64_t workspace_bytes;
  int32_t *route_log;            /* optional device int32 [n_updates, rows, C]: slot per overflow token */
  int32_t *append_log;           /* optional device int32 [n_updates, rows, C]: 1 if appended */
  void *const *events;           /* optional hipEvent_t[4] recorded on `stream`: before the first
                                    and after the last memory update, before the first and
                                    after the last attention launch (for timing) */
  int32_t *status;               /* optional device int32 status word.  Set: the call stays
                                    asynchronous; failure bits (KVM_STATUS_*) are ORed into
                                    the word on the device and never cleared, so the caller
                                    zeroes it once and reads it at a point where it
                                    synchronises anyway.  NULL: the library keeps the word in
                                    the workspace, waits for `stream` at the end of the call
                                    and returns KVM_EABORT when a failure bit is set. */
  float *lse;                    /* optional fp32 [B, Hq, T] (contiguous): log2-domain
                                    log-sum-exp of every query's scaled scores,
                                    log2(sum_j exp2(s_j)) with s = (q.k) * tau * log2(e) / sqrt(D);
                                    the backward recomputes the probabilities from it */
  void *snap_k;                  /* optional caller-held snapshots of the memory rows every query
                                    chunk attends to: bf16 [n_updates + 1, rows, max_state_len,
                                    head_dim] keys (LayerNorm_s(s_k)) and values; when set, they
                                    replace the workspace's snapshot ring (snapshot_ring must be
                                    n_updates + 1) and keep every snapshot for the backward */
  void *snap_v;
  int64_t flags;                 /* KVM_PREFILL_* bits (0: defaults) */
} kvm_prefill_desc;

/* One prefill's attention backward (the gradient of
 * model/kernels/kvm_triton_training_kernels.py:1803-1948; the reference's
 * _kvm_attn_live_state_dq_kernel :1950-2090, _live_state_dkdv_to_raw_grad_kernel
 * :2093-2305 and _kvm_attn_snapshot_bswa_dkdv_kernel :668-830), with the
 * memory snapshots held fixed: gradients w.r.t. the queries, the window keys
 * and values, every snapshot's key and value rows, and the two head
 * temperatures.  The chain rule from the snapshot rows back to the tokens
 * (LayerNorm_s, the value normalisation, the merge sums under the forward's
 * routes) is the caller's. */
typedef struct kvm_prefill_bwd_desc {
  kvm_layer layer;
  const void *q;                 /* bf16 [B, Hq, T, head_dim], strides as in kvm_prefill_desc */
  int64_t q_sb, q_sh, q_st;
  kvm_seq kv;                    /* window keys and values of the prompt (gate unused) */
  int64_t seq_len;
  const void *dout;              /* bf16 dL/d(out), out's layout: dout + b*do_sb + t*do_st + hq*do_sh */
  int64_t do_sb, do_st, do_sh;
  const float *lse;              /* fp32 [B, Hq, T] from the forward */
  float *delta;                  /* fp32 [B, Hq, T]: sum over features of dout * out; filled by the
                                    library when `out` is set, else read */
  const void *out;               /* bf16 forward output (dout's layout) or NULL */
  int64_t o_sb, o_st, o_sh;
  const void *snap_k, *snap_v;   /* bf16 [n_snap, rows, max_state_len, head_dim] from the forward */
  int64_t max_state_len;
  int64_t n_chunks;
  const int32_t *chunk_state_len;/* host [n_chunks], as in kvm_prefill_desc */
  const int32_t *chunk_snapshot; /* host [n_chunks] */
  void *dq;                      /* bf16 out [B, Hq, T, head_dim] at dq + b*dq_sb + h*dq_sh + t*dq_st */
  int64_t dq_sb, dq_sh, dq_st;
  float *dk, *dv;                /* fp32 out [B, Hkv, T, head_dim] contiguous: window keys / values */
  float *d_snap_k, *d_snap_v;    /* fp32 out [n_snap, rows, max_state_len, head_dim]: rows no
                                    query chunk reads are zero (each snapshot is read by one chunk:
                                    chunk_snapshot strictly increases over the chunks >= n_bswa) */
  float *d_state_temp;           /* fp32 out [q_heads] (summed over the batch) */
  float *d_front_temp;           /* fp32 out [q_heads] */
  void *workspace;               /* kvm_prefill_backward_workspace_bytes() */
  int64_t workspace_bytes;
} kvm_prefill_bwd_desc;

int64_t kvm_prefill_backward_workspace_bytes(const kvm_prefill_bwd_desc *d);
int kvm_prefill_backward(const kvm_prefill_bwd_desc *d, void *stream);

/* The memory state's part of the backward (the reference's
 * _live_state_dkdv_to_raw_grad_kernel, _reverse_route_scatter_grad_split_kernel,
 * _restore_refresh_from_undo_routes_kernel and _initial_state_grad_kernel,
 * model/kernels/kvm_triton_training_kernels.py:2093-2745), under the forward's
 * routes.  Snapshot s (s = 0 .. n_updates) holds slot rows
 * LayerNorm_s(s_k) and normalize(s_v) * vlen of the state after s updates;
 * the state starts from the initial token rows (slots < initial_state_len),
 * update u appends the tokens marked in append_log to slots
 * upd_state_before[u] .. + upd_n_append[u] - 1 (in token order, vlen =
 * |appended value row|) and then adds every other token's merge rows to the
 * slot route_log names.  Token rows are prep = LayerNorm_s(k with dims <
 * rope_partial_dim zeroed) and v, times the merge gate as the layer's gate
 * flags say.  Given the gradients of every snapshot's rows (d_snap_k /
 * d_snap_v, as kvm_prefill_backward writes them), this adds the state's
 * share of the gradient to dk and dv (the attention backward's window
 * gradients), writes dgate for the tokens the state holds, and writes the
 * LayerNorm parameters' gradient (both uses of ln_s_k).  The sums are taken
 * in fp32 and the forward's bf16 roundings as the identity. */
typedef struct kvm_state_bwd_desc {
  kvm_layer layer;               /* shapes, ln_s_k (fp32), rope_partial_dim, gate flags, chunk_len */
  kvm_seq kv;                    /* the prefill's keys, values and merge gates (bf16) */
  int64_t seq_len;
  int64_t initial_state_len;     /* L0 = min(seq_len, chunk_len) */
  int64_t n_updates;             /* < 256 */
  const int32_t *upd_token_begin, *upd_state_before, *upd_n_append;  /* host [n_updates] */
  const int32_t *route_log, *append_log;   /* device [n_updates, rows, chunk_len] (kvm_prefill's logs) */
  int64_t max_state_len;
  const float *d_snap_k, *d_snap_v;        /* fp32 [n_updates + 1, rows, max_state_len, head_dim] */
  float *dk, *dv;                          /* fp32 [B, Hkv, seq_len, head_dim], in/out: the state's share is added */
  float *dgate;                            /* fp32 out [B, Hkv, seq_len]: written for the tokens the state
                                              holds (others are left as they are: zero them first) */
  float *d_ln;                             /* fp32 out [2, head_dim]: d ln_w, d ln_b */
  void *workspace;                         /* kvm_state_backward_workspace_bytes() */
  int64_t workspace_bytes;
} kvm_state_bwd_desc;

int64_t kvm_state_backward_workspace_bytes(const kvm_state_bwd_desc *d);
int kvm_state_backward(const kvm_state_bwd_desc *d, void *stream);

/* The mixer's pre-boundary elementwise work on the q/k/v projections, for
 * one layer (model/value_residual_mixin.py:173-237 calc_qkv and
 * model/kvm_mixer.py:367-401 forward_prefix after the GEMMs):
 *   value residual (value_residual_mode 1 linear: (1-lamb) v + lamb v_first;
 *     2 rwkv: v + (v_first - v) * sigmoid(v_gate0 + gate_lin), before the
 *     token shift; 3 rwkv_post_tokenshift: the same after it);
 *   RWKV token shift (token_shift 1): x + x_mix * (prev - x), prev = the
 *     previous token, or q_prev/k_prev/v_prev for token 0, or token 0 itself
 *     when those are NULL (fallback "first", model/tokenshift.py:11-28);
 *   ln_q / ln_k (LayerNorm over head_dim), then interleaved-pair RoPE with
 *     the caller's bf16 cos/sin [B, T, 1, head_dim] (model/rwkv7_backbone.py:76-88);
 *   merge gate 1 + elu(key_weight).
 * Every step rounds to bf16 where the reference's torch ops do.
 * Inputs q_lin [B,T,Hq*D], k_lin [B,T,Hkv*D], v_lin [B,T,Hkv*Dv] are bf16
 * rows qkv_st elements apart (the three may be column ranges of one
 * concatenated projection), key_weight [B,T,Hkv] rows kw_st apart;
 * v_first / gate_lin [B,T,Hkv*Dv] are contiguous; the per-channel
 * parameters are bf16.  Outputs q_out [B,T,Hq,D], k_out [B,T,Hkv,D], v_out
 * [B,T,Hkv,Dv], gate_out [B,T,Hkv] (bf16, contiguous); v_last_out
 * (optional, [B,1,Hkv*Dv]) receives the last token's value after a value
 * residual applied before the shift (the decode cache's carried value);
 * q_last_out / k_last_out (optional, [B,1,Hq*D] / [B,1,Hkv*D]) receive the
 * last token's q_lin / k_lin rows (the carried rows of the next step's token
 * shift).  With seq_len == 1 each of the three may be the corresponding
 * q_prev / k_prev / v_prev itself (read before it is written).
 * Optional window-ring write (seq_len == 1 only; model/kvm_triton_decode.py
 * write_recent_ring, the row kvm_ring_write would write): with ring_k set,
 * the token's k_out and v_out rows and its merge gate (1 when gate_out is
 * NULL) of every (batch, kv head) row r = b * Hkv + h also go to ring_k /
 * ring_v [r, ring_cap, D] and ring_gate [r, ring_cap] at position ring_pos,
 * or, with ring_ctl (the int32[4] counters of kvm_ring_write_dev), at
 * (ctl[1] + ctl[2]) mod ring_cap. */
typedef struct kvm_prefix_desc {
  int64_t batch, seq_len, q_heads, kv_heads, head_dim, value_dim;
  int64_t value_residual_mode; /* 0 none, 1 linear, 2 rwkv, 3 rwkv_post_tokenshift */
  int64_t token_shift;         /* 0 none, 1 rwkv */
  double ln_eps;
  const void *q_lin, *k_lin, *v_lin, *v_first, *gate_lin, *key_weight;
  const void *q_prev, *k_prev, *v_prev; /* [B, 1, width] or NULL */
  const void *x_q, *x_k, *x_v, *v_gate0, *lamb;
  const void *ln_q_w, *ln_q_b, *ln_k_w, *ln_k_b;
  const void *cos, *sin;
  int64_t rope_sb, rope_st; /* element strides of cos/sin over batch and tokens */
  int64_t qkv_st, kw_st;     /* token strides (elements) of q/k/v_lin and key_weight */
  void *q_out, *k_out, *v_out, *gate_out, *v_last_out;
  void *q_last_out, *k_last_out; /* optional [B, 1, width]: the last token's q_lin / k_lin rows */
  void *ring_k, *ring_v, *ring_gate; /* optional window-ring write, above */
  int64_t ring_cap, ring_pos;
  const int32_t *ring_ctl;
} kvm_prefix_desc;

/* Run the pre-boundary elementwise work described above.  Replaces the
 * torch op sequence of calc_qkv + forward_prefix after the projections
 * (model/value_residual_mixin.py:173-237, model/kvm_mixer.py:367-401). */
int kvm_prefix(const kvm_prefix_desc *d, void *stream);

/* RWKV token shift out = x + mix * (shift(x) - x) over x [B, T, width]
 * (bf16, contiguous, width a multiple of 8): shift(x) is the previous token,
 * prev [B, width] for token 0, or when prev is NULL zeros (zero_fallback != 0)
 * or token 0 itself.  Replaces model/tokenshift.py:11-37 as the decoder's MLP
 * calls it (model/rwkv7_backbone.py:163-170, fallback "zero"). */
int kvm_token_shift(const void *x, const void *prev, const void *mix, void *out, int64_t batch,
                    int64_t seq_len, int64_t width, int zero_fallback, void *stream);

/* out = relu(x)^2 over n bf16 elements (n a multiple of 8): the decoder MLP's
 * activation, F.relu(x).square() (model/rwkv7_backbone.py:174-175). */
int kvm_relu_square(const void *x, void *out, int64_t n, void *stream);

/* Residual add, LayerNorm and token shift of the decoder block
 * (model/rwkv7_backbone.py:180-235: x + s * f(ln(x)) around the mixer and
 * the MLP, the final LayerNorm; :163-177 with model/tokenshift.py:11-37: the
 * MLP's token shift, fallback "zero").  Over rows of x [batch, seq_len, width]
 * (bf16, contiguous, width a multiple of 8 and at most 4096):
 *   r = x + alpha * y   (y NULL: r = x; round_product != 0: bf16(y * alpha)
 *                        is rounded before the add, as torch's x + y * s)
 *   h = LayerNorm(r) * ln_w + ln_b   (eps; fp32, rounded once to bf16)
 *   shifted = h + mix * (h_prev - h)  (h_prev: the previous token's h; for
 *                        token 0 the carried row prev [batch, width], or
 *                        zeros when prev is NULL)
 * Every output is optional (NULL): out_x = r, out_h = h, out_shift = shifted
 * (needs mix), state_out [batch, width] = h of the last token.  state_out may
 * be prev itself, and out_x / out_h / out_shift may be x or y, only when
 * seq_len == 1 (KVM_EINVAL otherwise: the token shift reads the row before
 * each run of rows, which another run may already have overwritten). */
typedef struct kvm_add_norm_desc {
  const void *x, *y;
  double alpha;
  int64_t round_product;
  const void *ln_w, *ln_b; /* bf16 [width] */
  double eps;
  const void *mix, *prev; /* bf16 [width], bf16 [batch, width] */
  void *out_x, *out_h, *out_shift, *state_out;
  int64_t batch, seq_len, width;
} kvm_add_norm_desc;

int kvm_add_norm(const kvm_add_norm_desc *d, void *stream);

/* Y = X W^T for a few token rows: X bf16 [M, K] (row stride x_st), W bf16
 * [N, K] (an nn.Linear weight, row stride w_st), Y bf16 [M, N] (row stride
 * y_st), fp32 accumulation; 1 <= M <= 16, K a multiple of 32.  The linear
 * layers of the decoder's single-token decode step (model/rwkv7_backbone.py
 * MLP and attention projections, the LM head), which stream their weights
 * once per step.  epilogue 1 writes relu(y)^2 instead of y (the MLP's
 * activation, rounded as kvm_relu_square of the bf16 product). */
int kvm_gemm_small(const void *x, int64_t x_st, const void *w, int64_t w_st, void *y, int64_t y_st, int64_t M,
                   int64_t N, int64_t K, int epilogue, void *stream);

/* Rows of W per workgroup (8 or 16) kvm_gemm_small takes for M tokens and N
 * outputs: the tile a packed W must be arranged for. */
int kvm_gemm_small_tile_rows(int64_t M, int64_t N);

/* kvm_gemm_small with W pre-arranged (once, by the caller) into 1 KiB chunks
 * that each load instruction reads whole.  For tile_rows R = 16: chunk
 * (b, s) = W rows 16b..16b+15, k 32s..32s+31, at element offset
 * (b * K/32 + s) * 512, element (g * 16 + i) * 8 + e = W[16b + i][32s + 8g + e]
 * (i < 16, g < 4, e < 8).  For R = 8 (K a multiple of 64): chunk (b, c) = rows
 * 8b..8b+7, k 64c..64c+63, at (b * K/64 + c) * 512, element
 * (g * 16 + h * 8 + j) * 8 + e = W[8b + j][64c + 32h + 8g + e] (j < 8, h < 2).
 * Rows past N are zeros; wp holds ceil(N / R) * R * K elements.  tile_rows
 * must be kvm_gemm_small_tile_rows(M, N).  Results are bit-identical to
 * kvm_gemm_small's. */
int kvm_gemm_small_packed(const void *x, int64_t x_st, const void *wp, void *y, int64_t y_st, int64_t M,
                          int64_t N, int64_t K, int tile_rows, int epilogue, void *stream);

/* ABI self-description, checked by the host binding at load time. */
int kvm_abi_version(void);
int64_t kvm_struct_size(int which); /* 0 layer, 1 seq, 2 state, 3 prefill_desc, 4 prefix_desc,
                                        5 prefill_bwd_desc, 6 state_bwd_desc, 7 add_norm_desc */
const char *kvm_last_error(void);

/* Workspace of kvm_prefill for the given descriptor (snapshot_ring and
 * max_state_len set). */
int64_t kvm_prefill_workspace_bytes(const kvm_prefill_desc *d);

/* Whole prefill: initial state from the first chunk, every block-boundary
 * update of the schedule, and the attention of every query chunk.
 * Replaces build_prefill_forward (model/kernels/kvm_triton_training_kernels.py:3386-3619)
 * as called from model/kvm_triton_mixer.py:470-536. */
int kvm_prefill(const kvm_prefill_desc *d, void *stream);

/* Write prep(k) (gated when layer->gate_initial), v (gated likewise) and
 * |v| of tokens [tok_begin, tok_begin + n_tok) of src into memory slots
 * [slot_begin, slot_begin + n_tok), with their attention rows.  The initial
 * state of a prefill (model/kvm_mixer.py:434-447) and the decode-time
 * direct-state append (model/kvm_triton_mixer.py:866-900). */
int kvm_state_append_direct(const kvm_layer *layer, const kvm_seq *src,
                            int64_t tok_begin, int64_t n_tok,
                            const kvm_state *st, int64_t slot_begin,
                            void *stream);

/* Recompute s_k_attn / s_v_attn of slots [slot_begin, slot_begin + n_slots)
 * from s_k, s_v, s_vlen (model/kvm_triton_decode.py:264-291 reset_). */
int kvm_state_refresh(const kvm_layer *layer, const kvm_state *st,
                      int64_t slot_begin, int64_t n_slots, void *stream);

/* Scratch of one kvm_state_update over n_tok overflow tokens.  Its first
 * three arrays hold, after the call, the streams of the overflow tokens
 * (bf16 [rows, n_tok, head_dim] each, at byte offsets 0, A and 2A with
 * A = rows * n_tok * head_dim * 2 rounded up to a multiple of 256):
 * prep(k), the merge key and the merge value. */
int64_t kvm_update_workspace_bytes(const kvm_layer *layer, int64_t n_tok);

/* One block-boundary memory update from overflow tokens
 * [tok_begin, tok_begin + n_tok) of src: append the n_append least novel
 * tokens, route the rest to their most similar non-sink slot and add them
 * in.  state_before is the current state length.  The attention rows of the
 * updated state are written to (attn_k_out, attn_v_out), which may alias
 * st->s_k_attn / st->s_v_attn; routing reads st->s_k_attn.
 * route_out / append_out (optional, device int32 [rows, n_tok]) receive the
 * slot of every token and whether it was appended.
 * Replaces run_forward_state_update (model/kernels/kvm_triton_training_kernels.py:1530-1800);
 * eager model/kvm_mixer.py:250-340 with model/kvm_fp32_routing_reference.py:24-49. */
int kvm_state_update(const kvm_layer *layer, const kvm_seq *src,
                     int64_t tok_begin, int64_t n_tok, int64_t state_before,
                     int64_t n_append, const kvm_state *st, void *attn_k_out,
                     void *attn_v_out, void *workspace, int64_t workspace_bytes,
                     int32_t *route_out, int32_t *append_out, void *stream);

/* Write one token (src token 0) into slot `pos` of the window ring
 * ring_k/ring_v [rows, ring_cap, dim], ring_gate [rows, ring_cap].
 * Replaces write_recent_ring (model/kernels/kvm_triton_decode.py:18-70, 287-322). */
int kvm_ring_write(const kvm_layer *layer, const kvm_seq *src, void *ring_k,
                   void *ring_v, void *ring_gate, int64_t ring_cap,
                   int64_t pos, void *stream);

/* Scratch of kvm_decode_attention for a window of up to max_rows
 * (state + ring) key rows. */
int64_t kvm_decode_workspace_bytes(const kvm_layer *layer, int64_t max_rows);

/* Single-token attention over active_state_len memory slots and recent_len
 * window rows stored in the ring from ring_start (modulo ring_cap).
 * q: bf16 [B, Hq, 1, head_dim] at q + b*q_sb + h*q_sh;
 * out: bf16 [B, Hq, value_dim] at out + b*o_sb + h*o_sh.
 * Split over key rows, combined deterministically.
 * Replaces kvm_decode_attention (model/kernels/kvm_triton_decode.py:175-284, 409-467). */
int kvm_decode_attention(const kvm_layer *layer, const void *q, int64_t q_sb,
                         int64_t q_sh, const kvm_state *st,
                         int64_t active_state_len, const void *ring_k,
                         const void *ring_v, int64_t ring_cap,
                         int64_t ring_start, int64_t recent_len, void *out,
                         int64_t o_sb, int64_t o_sh, void *workspace,
                         int64_t workspace_bytes, void *stream);

/* One decode step's ring write and attention in the launches of
 * kvm_decode_attention: the same result as kvm_ring_write(layer, src, ring_k,
 * ring_v, ring_gate, ring_cap, (ring_start + recent_len - 1) % ring_cap)
 * followed by kvm_decode_attention with these arguments.  recent_len counts
 * the step's token (src, one token, not a ring) as the last window row; the
 * attention reads it from src and stores its k, v and merge gate in the ring
 * slot, which no other read of the step touches.
 * Replaces the ring write + attention of one decode token
 * (write_recent_ring + kvm_decode_attention, model/kernels/kvm_triton_decode.py:18-70,
 * 287-322, 175-284, 409-467). */
int kvm_decode_step(const kvm_layer *layer, const void *q, int64_t q_sb, int64_t q_sh,
                    const kvm_state *st, int64_t active_state_len, const kvm_seq *src,
                    void *ring_k, void *ring_v, void *ring_gate, int64_t ring_cap,
                    int64_t ring_start, int64_t recent_len, void *out, int64_t o_sb,
                    int64_t o_sh, void *workspace, int64_t workspace_bytes, void *stream);

/* Decode with the step counters in device memory, so that a decode step can
 * be captured once in a HIP graph and replayed (the kernels read the counters
 * when they run; the arguments of a replayed launch never change).  ctl is
 * an int32 record {active_state_len, ring_start, recent_len, reserved} per
 * layer, holding the values BEFORE the step's token is written: the ring
 * write stores it at row (ring_start + recent_len) % ring_cap, the attention
 * reads recent_len + pending window rows (pending = 1 after that write), and
 * kvm_decode_advance moves recent_len past it.  Kernels clamp the counters to
 * the ring and state capacities.  The same operations as kvm_ring_write and
 * kvm_decode_attention (model/kvm_triton_mixer.py:717-757, whose counters are
 * host values); the attention's grid covers st->capacity + ring_cap rows
 * (workspace: kvm_decode_workspace_bytes of that many rows), and its result
 * is bit-identical to kvm_decode_attention's for the same counters. */
int kvm_ring_write_dev(const kvm_layer *layer, const kvm_seq *src, void *ring_k,
                       void *ring_v, void *ring_gate, int64_t ring_cap,
                       const int32_t *ctl, void *stream);
int kvm_decode_attention_dev(const kvm_layer *layer, const void *q, int64_t q_sb,
                             int64_t q_sh, const kvm_state *st, const int32_t *ctl,
                             int32_t pending, const void *ring_k, const void *ring_v,
                             int64_t ring_cap, void *out, int64_t o_sb, int64_t o_sh,
                             void *workspace, int64_t workspace_bytes, void *stream);
/* recent_len += 1 in the n records at ctl (record i at ctl + 4 i). */
int kvm_decode_advance(int32_t *ctl, int64_t n, void *stream);

/* Size of the library-owned scratch of kvm_decode_attention_noalloc, per GPU. */
#define KVM_DECODE_SCRATCH_BYTES (16 << 20)

/* kvm_decode_attention without a workspace argument: the split-K partials go
 * to a scratch array the library holds on each GPU (KVM_DECODE_SCRATCH_BYTES,
 * kept until the process ends), so the call performs no device allocation.
 * No counterpart in the reference: it is for callers that cannot allocate
 * (code under HIP graph capture, serving loops, harnesses that forbid
 * hipMalloc).  The scratch must hold B * q_heads * ceil((active_state_len +
 * recent_len) / 256) * (head_dim + 2) * 4 bytes (kvm_decode_workspace_bytes);
 * larger calls return KVM_ESPACE.  All calls on one GPU share its array and
 * keep no state in it between calls, so calls that overlap on one GPU (two
 * streams, two threads) race.  Arguments and results are those of
 * kvm_decode_attention. */
int kvm_decode_attention_noalloc(const kvm_layer *layer, const void *q, int64_t q_sb,
                                 int64_t q_sh, const kvm_state *st,
                                 int64_t active_state_len, const void *ring_k,
                                 const void *ring_v, int64_t ring_cap,
                                 int64_t ring_start, int64_t recent_len, void *out,
                                 int64_t o_sb, int64_t o_sh, void *stream);

#ifdef __cplusplus
}
#endif

#endif /* KVM_AMD_H */
