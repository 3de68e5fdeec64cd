// Internal launcher interface shared by the KVM translation units.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/kvm_amd.h"

namespace kvm {

// Scratch of one block-boundary update over n_tok overflow tokens
// (all arrays [rows, n_tok, ...], row-major).
struct UpdateScratch {
  uint16_t *pk;       // prep(k)                      bf16 [rows, n_tok, D]
  uint16_t *gk;       // merge key  (gated or not)    bf16 [rows, n_tok, D]
  uint16_t *gv;       // merge value (gated or not)   bf16 [rows, n_tok, D]
  uint64_t *rkey[2];  // route max-reduction keys, alternating per update [rows, n_tok]
  uint32_t *nkey;     // novelty max-reduction keys   [rows, n_tok]
  int32_t *route;     // slot of appended tokens      int32 [rows, n_tok]
  int32_t *is_append; // 1 if appended                int32 [rows, n_tok]
};

// Scratch of updates: a slice per update (pk, gk, gv, route, is_append; the
// first three at byte offsets 0, A, 2A) and one shared region of reduction
// keys.
int64_t update_slice_bytes(const kvm_layer &L, int64_t n_tok);
int64_t update_keys_bytes(const kvm_layer &L, int64_t n_tok);
int64_t update_scratch_bytes(const kvm_layer &L, int64_t n_tok);  // one slice + keys
UpdateScratch carve_update_scratch(void *slice, void *keys, const kvm_layer &L,
                                   int64_t n_tok);
// The per-update pointers of slice u (slices are slice_bytes apart).
__host__ __device__ inline UpdateScratch scratch_slice(UpdateScratch s0, int64_t slice_bytes,
                                                       int u) {
  const int64_t o = slice_bytes * u;
  s0.pk = reinterpret_cast<uint16_t *>(reinterpret_cast<unsigned char *>(s0.pk) + o);
  s0.gk = reinterpret_cast<uint16_t *>(reinterpret_cast<unsigned char *>(s0.gk) + o);
  s0.gv = reinterpret_cast<uint16_t *>(reinterpret_cast<unsigned char *>(s0.gv) + o);
  s0.route = reinterpret_cast<int32_t *>(reinterpret_cast<unsigned char *>(s0.route) + o);
  s0.is_append = reinterpret_cast<int32_t *>(reinterpret_cast<unsigned char *>(s0.is_append) + o);
  return s0;
}
constexpr int kMaxPrep = 64;
struct PrepList {
  int32_t count;
  int32_t tok_begin[kMaxPrep];  // first overflow token of each update (ring index for rings)
};
// Overflow-token streams of P.count updates into slices 0..count-1.
hipError_t launch_prep(const kvm_layer &L, const kvm_seq &src, const PrepList &P,
                       int64_t n_tok, const UpdateScratch &s0, int64_t slice_bytes,
                       hipStream_t stream);

// Attention-row arrays of a state: bf16 [rows, cap, D] each.
struct AttnRows {
  uint16_t *k;
  uint16_t *v;
  int64_t cap;
};

hipError_t launch_append_direct(const kvm_layer &L, const kvm_seq &src,
                                int64_t tok_begin, int64_t n_tok,
                                const kvm_state &st, int64_t slot_begin,
                                AttnRows attn, bool apply_gate,
                                hipStream_t stream);

hipError_t launch_refresh(const kvm_layer &L, const kvm_state &st,
                          int64_t slot_begin, int64_t n_slots, AttnRows attn,
                          hipStream_t stream);

// One update.  Routing reads attn_in (the attention rows of the state before
// the update; appended rows are added to it), the refreshed rows of every
// slot < state_before + n_append are written to attn_out.
// The key buffers must be zero before the first update on a workspace
// (launch_zero_keys); each update then clears the buffer of the next one.
// `parity` alternates between consecutive updates on the same workspace.
hipError_t launch_zero_keys(const kvm_layer &L, int64_t n_tok,
                            const UpdateScratch &sc, hipStream_t stream);
hipError_t launch_update(const kvm_layer &L, const kvm_seq &src,
                         int64_t tok_begin, int64_t n_tok, int64_t state_before,
                         int64_t n_append, const kvm_state &st, AttnRows attn_in,
                         AttnRows attn_out, const UpdateScratch &sc, int parity,
                         int32_t *route_out, int32_t *append_out,
                         hipStream_t stream);

// Persistent update chain (kvm_chain.hip): a batch of consecutive updates
// of every row in one launch.
constexpr int kChainMax = 128;             // updates per launch
constexpr int kChainMaxWorkgroups = 256;   // one 512-thread workgroup per CU
struct ChainList {
  int32_t u0;     // update index of entry 0 (snapshot u0 -> u0 + 1, log offset)
  int32_t count;
  int32_t final_rows;  // k_chain_fixed: also write the last snapshot's rows to the state's s_k_attn / s_v_attn
  int32_t tok_begin[kChainMax];
  int32_t state_before[kChainMax];
  int32_t n_append[kChainMax];
};
// Snapshot ring of attention rows: snapshot i at k + (i % ring) * stride.
struct SnapRing {
  uint16_t *k;
  uint16_t *v;
  int64_t stride;  // elements between ring entries
  int64_t ring;
  int64_t cap;     // slots per row
};
struct ChainScratch {
  uint16_t *gk;          // merge keys   bf16 [3][rows, n_tok, D] (rotating over updates)
  uint16_t *gv;          // merge values bf16 [3][rows, n_tok, D]
  int32_t *route;        // merge slot of each token, -1 if appended [rows, n_tok]
  float *nov;            // novelty of each token [rows, n_tok]
  uint2 *part;           // per-member route maxima as route keys {mono(score), tag << 16 | (0xffff - slot)} [2][rows, n_tok, G]
  unsigned *bar;         // group barrier counters
  unsigned *abort_flag;  // set when a group wait timed out (cleared per launch)
  unsigned *status;      // sticky: KVM_STATUS_CHAIN_TIMEOUT is ORed in on a time-out
  unsigned max_polls;    // L2 polls a group wait makes before giving up
};
struct ChainPlan {
  bool fixed;     // slot-owner routing (no appends in the batch)
  int G;          // workgroups per row
  int tpw;        // tokens per workgroup (multiple of 16, <= 64)
  int spm_max;    // slots per workgroup at max_slots
  int row_batch;  // rows per launch (all rows, or batches of them when they do not fit at once)
  int workgroups; // per launch
  size_t dyn_lds;
};
// False when the shape does not fit the chain (the per-update kernels then run).
bool chain_plan(const kvm_layer &L, int64_t n_tok, int64_t max_slots, ChainPlan *p);
// Whether a batch may use the slot-owner kernel: no appends, one state
// length, at most 64 slots per member and 512 tokens per update.
bool chain_fixed_ok(const ChainPlan &p, const ChainList &list, int64_t n_tok);
int64_t chain_scratch_bytes(const kvm_layer &L, int64_t n_tok);
ChainScratch carve_chain_scratch(void *base, const kvm_layer &L, int64_t n_tok);
hipError_t launch_chain(const kvm_layer &L, const kvm_seq &src, int64_t n_tok,
                        const kvm_state &st, const SnapRing &snaps, const ChainList &list,
                        const ChainScratch &cs, const ChainPlan &p, int32_t *route_log,
                        int32_t *append_log, hipStream_t stream);

// Default poll budget of a group wait (about a second of polling).
constexpr unsigned kChainDefaultPolls = 1u << 22;
// Fill n words at p with v (a kernel, so the work may be graph-captured).
hipError_t launch_fill_u32(unsigned *p, int64_t n, unsigned v, hipStream_t stream);

// ctl (optional): device counters {.., ring_start, recent_len, ..}; the row is
// then (ring_start + recent_len) % ring_cap, read when the kernel runs.
hipError_t launch_ring_write(const kvm_layer &L, const kvm_seq &src,
                             void *ring_k, void *ring_v, void *ring_gate,
                             int64_t ring_cap, int64_t pos, hipStream_t stream,
                             const int32_t *ctl = nullptr);

int64_t decode_segments(int64_t rows_total);
// Address of this device's library-owned decode scratch
// (KVM_DECODE_SCRATCH_BYTES, resolved once per device).
hipError_t decode_scratch(void **ptr);
int64_t decode_workspace_bytes(const kvm_layer &L, int64_t max_rows);
hipError_t launch_decode(const kvm_layer &L, const void *q, int64_t q_sb,
                         int64_t q_sh, const kvm_state &st, int64_t active,
                         const void *ring_k, const void *ring_v,
                         int64_t ring_cap, int64_t ring_start,
                         int64_t recent_len, void *out, int64_t o_sb,
                         int64_t o_sh, void *workspace, hipStream_t stream,
                         const int32_t *ctl = nullptr, int pending = 0, int64_t max_rows = 0,
                         const kvm_seq *fresh = nullptr, void *ring_gate = nullptr);
hipError_t launch_decode_advance(int32_t *ctl, int64_t n, hipStream_t stream);

// Per-launch table of the query chunks an attention launch covers.
constexpr int kMaxChunksPerLaunch = 256;
struct ChunkTable {
  int32_t state_len[kMaxChunksPerLaunch];  // memory slots visible to the chunk
  int32_t snap_slot[kMaxChunksPerLaunch];  // ring slot of its snapshot
};

struct PrefillAttnArgs {
  const void *q;
  int64_t q_sb, q_sh, q_st;
  kvm_seq kv;
  int64_t T;
  void *out;
  int64_t o_sb, o_st, o_sh;
  const uint16_t *snap_k;  // snapshot ring base (keys)
  const uint16_t *snap_v;  // snapshot ring base (values)
  int64_t snap_stride;     // elements between consecutive snapshots
  int64_t snap_cap;        // slots per row in a snapshot
  float *lse;              // optional fp32 [B, Hq, T]: log2-domain log-sum-exp per query
};

// Attention backward (kvm_attn_bwd.hip).
struct BwdArgs {
  const void *q;
  int64_t q_sb, q_sh, q_st;
  kvm_seq kv;
  int64_t T;
  const void *dout;
  int64_t do_sb, do_st, do_sh;
  const float *lse, *delta;  // [B, Hq, T]
  const uint16_t *snap_k, *snap_v;
  int64_t snap_stride;       // elements between snapshots
  int64_t snap_cap;          // slots per row in a snapshot
  int64_t n_chunks;
  void *dq;
  int64_t dq_sb, dq_sh, dq_st;
  float *dk, *dv;            // [B*Hkv, T, D]
  float *d_snap_k, *d_snap_v;
  int64_t dsnap_stride;
  float *d_state_temp, *d_front_temp;
};
int64_t attn_bwd_workspace_bytes(const kvm_layer &L, int64_t n_chunks);
hipError_t launch_attn_backward(const kvm_layer &L, const BwdArgs &a, const ChunkTable &table,
                                float *tpart, hipStream_t stream);
// delta = rowsum(dout * out) over [B, Hq, T] rows (bf16 inputs, fp32 out).
hipError_t launch_attn_delta(const kvm_layer &L, const void *dout, int64_t do_sb, int64_t do_st, int64_t do_sh,
                             const void *out, int64_t o_sb, int64_t o_st, int64_t o_sh, int64_t T, float *delta,
                             hipStream_t stream);

// Memory-state backward (kvm_state_bwd.hip).  dk / dv are [rows, T, D]
// fp32 (added to), dgate [rows, T]; snapshot gradients
// [n_updates + 1, rows, max_state_len, D].
struct StateBwdArgs {
  kvm_layer L;
  kvm_seq kv;
  int64_t rows, T, L0, n_updates, max_state_len;
  const int32_t *route_log, *append_log;  // [n_updates, rows, chunk_len]
  const float *d_snap_k, *d_snap_v;
  float *dk, *dv, *dgate;
  float *d_ln;                            // [2, D]
};
// Per-update schedule, passed by value as a kernel argument (3 KiB).
struct UpdTable {
  int32_t token_begin[kMaxChunksPerLaunch];
  int32_t state_before[kMaxChunksPerLaunch];
  int32_t n_append[kMaxChunksPerLaunch];
};
int64_t state_bwd_workspace_bytes(int64_t head_dim, int64_t rows, int64_t max_state_len);
int64_t state_bwd_max_chunk();
// part: the per-workgroup LayerNorm partials (the workspace).
hipError_t launch_state_backward(const StateBwdArgs &a, const UpdTable &sched, float *part,
                                 hipStream_t stream);

// Y[M, N] = X[M, K] W[N, K]^T, bf16, M <= 16, epilogue 1 = relu^2 (kvm_gemm.hip).
// packed: w in the chunked layout of kvm_gemm_small_packed (w_st unused).
hipError_t launch_gemm_small(const void *x, int64_t x_st, const void *w, int64_t w_st, void *y, int64_t y_st,
                             int64_t M, int64_t N, int64_t K, int epilogue, bool packed, hipStream_t stream);
int gemm_small_tile_rows(int64_t M, int64_t N);
// Residual add + LayerNorm + token shift of the decoder block (kvm_block.hip).
hipError_t launch_add_norm(const kvm_add_norm_desc &P, hipStream_t stream);
hipError_t launch_prefix(const kvm_prefix_desc &P, hipStream_t stream);
hipError_t launch_token_shift(const void *x, const void *prev, const void *mix, void *out, int64_t B,
                              int64_t T, int64_t width, int zero_fallback, hipStream_t stream);
hipError_t launch_relu_square(const void *x, void *out, int64_t n, hipStream_t stream);

hipError_t launch_prefill_attention(const kvm_layer &L,
                                    const PrefillAttnArgs &a,
                                    int64_t chunk_begin, int64_t n_chunks,
                                    const ChunkTable &table,
                                    hipStream_t stream);

}  // namespace kvm
