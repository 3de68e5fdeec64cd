// Block-boundary memory update of the KVM mixer on gfx950.
//
// Reference semantics: model/kvm_mixer.py:250-340 (append + merge),
// model/kvm_fp32_routing_reference.py:24-49 (fp32 merge routing),
// model/kvm_mixer.py:434-447 (initial state), and the Triton contract of
// model/kvm_triton_mixer.py:199-211 (one rounded state write, cached
// normalized state rows).
//
// An update is a prep pass (batched ahead over many updates) and then up
// to four launches over rows = batch * kv_heads:
//   k_route<NOVELTY>      (growable memory) bf16-rounded max similarity of
//       every overflow token to the current slots, 64 tokens x 128 slots
//       per workgroup on MFMA, combined by an order-independent atomicMax;
//   k_rank_append         (growable) one workgroup per row ranks novelty in
//       LDS and appends the least novel tokens as new slots;
//   k_route<ROUTE>        fp32 similarity of the merge keys to the slots,
//       first argmax (same split and combination);
//   k_merge_refresh       16 slots per workgroup: each slot sums the tokens
//       routed to it in token order (fp32, deterministic, no global
//       atomics), writes bf16(state + bf16(sum)) and its LayerNorm /
//       normalized-value attention rows.  When the attention rows are
//       updated in place, a slot no token merges into is left untouched.

#include "kvm_device.hpp"
#include "kvm_internal.hpp"
#include "kvm_seq.hpp"

namespace kvm {
namespace {

constexpr int kThreads = 256;

// ---------------------------------------------------------------------------
// Direct append: tokens [tok_begin, +n_tok) -> slots [slot_begin, +n_tok).
// grid (rows, ceil(n_tok / (256 / (D/8)))), 256 threads, D/8 lanes per token.
template <int D>
__global__ __launch_bounds__(kThreads) void k_append_direct(
    kvm_layer L, kvm_seq src, int64_t tok_begin, int n_tok, kvm_state st,
    int64_t slot_begin, AttnRows attn, int apply_gate) {
  constexpr int G = D / 8;
  constexpr int TPW = kThreads / G;
  const int row = blockIdx.x;
  const int b = row / int(L.kv_heads), h = row % int(L.kv_heads);
  const int part = threadIdx.x % G;
  const int i_tok = blockIdx.y * TPW + threadIdx.x / G;
  const bool valid = i_tok < n_tok;
  const int64_t t = tok_begin + (valid ? i_tok : 0);

  float k[8], v[8];
  load8(seq_k(src, b, h, t) + part * 8, k);
  load8(seq_v(src, b, h, t) + part * 8, v);
  const float g = seq_g(src, b, h, t);
  prep_key<D>(k, part, L);
  const float vlen = row_norm8<D>(v);  // |v| of the raw value
  if (apply_gate) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      k[i] = rbf(k[i] * g);
      v[i] = rbf(v[i] * g);
    }
  }
  float ka[8], va[8];
  attn_rows<D>(k, v, vlen, part, L, ka, va);
  if (!valid) return;
  const int64_t slot = slot_begin + i_tok;
  const int64_t off = (int64_t(row) * st.capacity + slot) * D + part * 8;
  store8(static_cast<uint16_t *>(st.s_k) + off, k);
  store8(static_cast<uint16_t *>(st.s_v) + off, v);
  if (part == 0)
    static_cast<float *>(st.s_vlen)[int64_t(row) * st.capacity + slot] = vlen;
  const int64_t aoff = (int64_t(row) * attn.cap + slot) * D + part * 8;
  store8(attn.k + aoff, ka);
  store8(attn.v + aoff, va);
}

// Attention rows of slots [slot_begin, +n_slots) from s_k, s_v, s_vlen.
template <int D>
__global__ __launch_bounds__(kThreads) void k_refresh(kvm_layer L,
                                                      kvm_state st,
                                                      int64_t slot_begin,
                                                      int n_slots,
                                                      AttnRows attn) {
  constexpr int G = D / 8;
  constexpr int SPW = kThreads / G;
  const int row = blockIdx.x;
  const int part = threadIdx.x % G;
  const int i_slot = blockIdx.y * SPW + threadIdx.x / G;
  const bool valid = i_slot < n_slots;
  const int64_t slot = slot_begin + (valid ? i_slot : 0);
  const int64_t off = (int64_t(row) * st.capacity + slot) * D + part * 8;
  float k[8], v[8], ka[8], va[8];
  load8(static_cast<const uint16_t *>(st.s_k) + off, k);
  load8(static_cast<const uint16_t *>(st.s_v) + off, v);
  const float vlen =
      static_cast<const float *>(st.s_vlen)[int64_t(row) * st.capacity + slot];
  attn_rows<D>(k, v, vlen, part, L, ka, va);
  if (!valid) return;
  const int64_t aoff = (int64_t(row) * attn.cap + slot) * D + part * 8;
  store8(attn.k + aoff, ka);
  store8(attn.v + aoff, va);
}

// ---------------------------------------------------------------------------
// Reduction keys.  The per-token maximum over slots is combined across
// workgroups with integer atomicMax on order-preserving encodings, which
// is exact and independent of arrival order:
//   novelty  u32  mono(bf16-rounded similarity)
//   route    u64  mono(fp32 similarity) << 32 | (0xffffffff - slot)
// so the largest similarity wins and, among equal similarities, the lowest
// slot (torch.max returns the first maximum).  0 means "no candidate".
__device__ __forceinline__ uint32_t mono(float f) {
  const uint32_t u = __float_as_uint(f);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__device__ __forceinline__ float unmono(uint32_t m) {
  return __uint_as_float((m & 0x80000000u) ? (m & 0x7fffffffu) : ~m);
}

// ---------------------------------------------------------------------------
// Overflow-token streams of a batch of updates (independent of the state,
// so computed ahead of the update chain): prep(k) = LayerNorm_s(k with dims
// < rope_partial_dim zeroed) (model/kvm_mixer.py:120-129), the merge key
// bf16(prep(k) * g) and value bf16(v * g) when gated (:264-281), and the
// append flags cleared.  grid (rows, token tiles of 64, updates).
template <int D>
__global__ __launch_bounds__(kThreads) void k_prep(kvm_layer L, kvm_seq src, PrepList P,
                                                   int n_tok, UpdateScratch s0,
                                                   int64_t slice_bytes) {
  constexpr int G = D / 8;
  constexpr int IT = 64 * G / kThreads;
  const int row = blockIdx.x;
  const int b = row / int(L.kv_heads), h = row % int(L.kv_heads);
  const int tok0 = blockIdx.y * 64;
  const UpdateScratch sc = scratch_slice(s0, slice_bytes, blockIdx.z);
  const int64_t tok_begin = P.tok_begin[blockIdx.z];
  const int tid = threadIdx.x;
  const int64_t rbase = int64_t(row) * n_tok;
  uint4 kr[IT], vr[IT];
  float gr[IT];
#pragma unroll
  for (int it = 0; it < IT; ++it) {
    const int p = tid + it * kThreads;
    const int i_tok = tok0 + p / G;
    const int64_t t = tok_begin + (i_tok < n_tok ? i_tok : 0);
    kr[it] = *reinterpret_cast<const uint4 *>(seq_k(src, b, h, t) + (p % G) * 8);
    vr[it] = *reinterpret_cast<const uint4 *>(seq_v(src, b, h, t) + (p % G) * 8);
    gr[it] = seq_g(src, b, h, t);
  }
#pragma unroll
  for (int it = 0; it < IT; ++it) {
    const int p = tid + it * kThreads;
    const int i_tok = tok0 + p / G, part = p % G;
    float k[8], v[8];
    unpack8(kr[it], k);
    unpack8(vr[it], v);
    const float g = gr[it];
    prep_key<D>(k, part, L);
    float gk[8], gv[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      gk[i] = L.gate_keys ? rbf(k[i] * g) : k[i];
      gv[i] = L.gate_values ? rbf(v[i] * g) : v[i];
    }
    if (i_tok < n_tok) {
      const int64_t off = (rbase + i_tok) * D + part * 8;
      store8(sc.pk + off, k);
      store8(sc.gk + off, gk);
      store8(sc.gv + off, gv);
      if (part == 0) sc.is_append[rbase + i_tok] = 0;
    }
  }
}

// ---------------------------------------------------------------------------
// Token x slot similarity on MFMA 16x16x32 bf16.
//
// Workgroup: kRouteTok overflow tokens x one split of at most kSplit slots of one
// row (1-D grid of rows x token tiles x slot splits).  The similarity is computed
// transposed, D^T[slot][token] = S_attn . X^T, so the accumulator lane
// layout (lane l holds slots 4*(l/16)+i of token l%16) reduces over slots
// within a lane, then across the 4 lane groups and the 4 waves (LDS); one
// atomicMax per token and workgroup publishes the split's result.  Each wave
// loads its two 16-slot tiles straight into A-operand registers at kernel
// start, so the slot rows are in flight while the tokens are prepared.
//
// The operand comes from the update's scratch slice (written by k_prep):
// NOVELTY: prep(k), value max_j bf16(prep(k).s_attn_j) over all s_lim slots
//       (model/kvm_mixer.py:66-68); otherwise the merge key, value = first
//       argmax over slots [protect, s_lim) of the fp32 dot
//       (model/kvm_fp32_routing_reference.py:30-34).
constexpr int kSplit = 128;  // slots per workgroup
constexpr int kRouteTok = 128;  // tokens per workgroup (8 tiles of 16)

template <int D, bool NOVELTY>
__global__ __launch_bounds__(kThreads) void k_route(
    kvm_layer L, int n_tok, AttnRows sref, int s_lim, int protect, UpdateScratch sc,
    int parity, int tiles, int splits) {
  constexpr int G = D / 8;
  constexpr int STR = D + 8;  // LDS row stride (elements), 16 B pad
  constexpr int KS = D / 32;
  constexpr int TT = kRouteTok / 16;  // token tiles
  __shared__ __attribute__((aligned(16))) uint16_t tok_lds[kRouteTok * STR];
  __shared__ uint32_t hi_lds[4][kRouteTok];
  __shared__ int idx_lds[4][kRouteTok];

  // Logical order (row, token tile, slot split), contiguous per XCD: the
  // workgroups of a row share its slot rows and tokens through one L2.
  const int wg = xcd_contiguous(int(blockIdx.x), int(gridDim.x));
  const int split = wg % splits;
  const int tok0 = (wg / splits) % tiles * kRouteTok;
  const int row = wg / (splits * tiles);
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t rbase = int64_t(row) * n_tok;

  // Slot rows of this wave (two 16-slot tiles) and the kRouteTok token operands,
  // all issued before any is used.
  const uint16_t *sbase = sref.k + int64_t(row) * sref.cap * D;
  const int jw = split * kSplit + wave * 32;
  uint4 a_reg[2][KS];
#pragma unroll
  for (int st = 0; st < 2; ++st) {
    const int j = jw + st * 16 + (lane & 15);
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)
      a_reg[st][ks] = j < s_lim ? *reinterpret_cast<const uint4 *>(sbase + int64_t(j) * D + ks * 32 +
                                                                   (lane >> 4) * 8)
                                : make_uint4(0, 0, 0, 0);
  }
  constexpr int IT = kRouteTok * G / kThreads;
  const uint16_t *opnd = NOVELTY ? sc.pk : sc.gk;
  uint4 xr[IT];
#pragma unroll
  for (int it = 0; it < IT; ++it) {
    const int p = tid + it * kThreads;
    const int i_tok = tok0 + p / G;
    xr[it] = i_tok < n_tok ? *reinterpret_cast<const uint4 *>(opnd + (rbase + i_tok) * D + (p % G) * 8)
                           : make_uint4(0, 0, 0, 0);
  }
#pragma unroll
  for (int it = 0; it < IT; ++it) {
    const int p = tid + it * kThreads;
    *reinterpret_cast<uint4 *>(&tok_lds[(p / G) * STR + (p % G) * 8]) = xr[it];
  }
  __syncthreads();

  // (2) similarity of the TT token tiles against the wave's 32 slots.
  float best[TT];
  int bidx[TT];
#pragma unroll
  for (int tt = 0; tt < TT; ++tt) {
    best[tt] = -INFINITY;
    bidx[tt] = -1;
    bf16x8 bx[KS];
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)
      bx[ks] = as_bf16x8(*reinterpret_cast<const uint4 *>(
          &tok_lds[(tt * 16 + (lane & 15)) * STR + ks * 32 + (lane >> 4) * 8]));
    // Both 16-slot tiles' accumulations interleave (each sums its k-steps
    // in order); the tiles are then scanned in slot order.
    f32x4 accs[2] = {f32x4{0.f, 0.f, 0.f, 0.f}, f32x4{0.f, 0.f, 0.f, 0.f}};
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)
#pragma unroll
      for (int st = 0; st < 2; ++st)
        accs[st] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(a_reg[st][ks]), bx[ks], accs[st], 0, 0, 0);
#pragma unroll
    for (int st = 0; st < 2; ++st) {
      const f32x4 acc = accs[st];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int j = jw + st * 16 + (lane >> 4) * 4 + i;
        if constexpr (NOVELTY) {
          if (j < s_lim) best[tt] = fmaxf(best[tt], rbf(acc[i]));
        } else {
          if (j >= protect && j < s_lim && acc[i] > best[tt]) {
            best[tt] = acc[i];
            bidx[tt] = j;
          }
        }
      }
    }
  }

  // (3) lane groups, then waves (slot order: lower wave = lower slots).
#pragma unroll
  for (int tt = 0; tt < TT; ++tt) {
#pragma unroll
    for (int o = 16; o <= 32; o <<= 1) {
      const float ob = __shfl_xor(best[tt], o);
      const int oi = __shfl_xor(bidx[tt], o);
      if constexpr (NOVELTY) {
        best[tt] = fmaxf(best[tt], ob);
      } else if (oi >= 0 && (bidx[tt] < 0 || ob > best[tt] || (ob == best[tt] && oi < bidx[tt]))) {
        best[tt] = ob;
        bidx[tt] = oi;
      }
    }
    if (lane < 16) {
      hi_lds[wave][tt * 16 + lane] = (NOVELTY || bidx[tt] >= 0) ? mono(best[tt]) : 0u;
      idx_lds[wave][tt * 16 + lane] = bidx[tt];
    }
  }
  __syncthreads();
  if (tid < kRouteTok) {
    const int i_tok = tok0 + tid;
    if (i_tok < n_tok) {
      const int64_t o = rbase + i_tok;
      if constexpr (NOVELTY) {
        uint32_t m = hi_lds[0][tid];
#pragma unroll
        for (int w = 1; w < 4; ++w) m = max(m, hi_lds[w][tid]);
        atomicMax(sc.nkey + o, m);
      } else {
        uint64_t key = 0;
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          const int oi = idx_lds[w][tid];
          if (oi >= 0) {
            const uint64_t kk = (uint64_t(hi_lds[w][tid]) << 32) | uint64_t(0xffffffffu - uint32_t(oi));
            key = kk > key ? kk : key;
          }
        }
        if (key) atomicMax(reinterpret_cast<unsigned long long *>(sc.rkey[parity]) + o,
                           (unsigned long long)key);
        // The other key buffer serves the next update: clear it.
        if (split == 0) sc.rkey[parity ^ 1][o] = 0;
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Append ranking (model/kvm_mixer.py:44-75, 231-248): the n_append tokens
// with the lowest novelty, ties to the lower token index, become slots
// state_before.. in token order.  One workgroup per row; dynamic LDS holds
// novelty, flags and positions of the n_tok tokens.  The novelty keys are
// cleared after use (this workgroup is their only reader).
template <int D>
__global__ __launch_bounds__(512) void k_rank_append(
    kvm_layer L, kvm_seq src, int64_t tok_begin, int n_tok, int n_append,
    int state_before, kvm_state st, AttnRows attn_cur, UpdateScratch sc) {
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  float *nov = reinterpret_cast<float *>(smem);
  int *flag = reinterpret_cast<int *>(nov + n_tok);
  int *pos = flag + n_tok;
  const int row = blockIdx.x;
  const int b = row / int(L.kv_heads), h = row % int(L.kv_heads);
  const int tid = threadIdx.x, nt = blockDim.x;
  const int64_t base = int64_t(row) * n_tok;

  for (int t = tid; t < n_tok; t += nt) {
    nov[t] = unmono(sc.nkey[base + t]);
    sc.nkey[base + t] = 0;
  }
  __syncthreads();
  for (int t = tid; t < n_tok; t += nt) {
    const float x = nov[t];
    int r = 0;
    for (int u = 0; u < n_tok; ++u) {
      const float y = nov[u];
      r += (y < x) || (y == x && u < t);
    }
    flag[t] = r < n_append ? 1 : 0;
  }
  __syncthreads();
  for (int t = tid; t < n_tok; t += nt) {
    int p = 0;
    for (int u = 0; u < t; ++u) p += flag[u];
    pos[t] = p;
    sc.is_append[base + t] = flag[t];
    sc.route[base + t] = flag[t] ? state_before + p : -1;
  }
  __syncthreads();

  // Appended rows: D/8 lanes per token, uniform trip count for the shuffles.
  constexpr int G = D / 8;
  const int tpp = nt / G;
  const int passes = (n_tok + tpp - 1) / tpp;
  const int part = tid % G;
  for (int ps = 0; ps < passes; ++ps) {
    const int t = ps * tpp + tid / G;
    const bool valid = t < n_tok && flag[t] != 0;
    const int tt = t < n_tok ? t : 0;
    const int64_t off = (base + tt) * D + part * 8;
    float k[8], v[8];
    if (L.gate_appends) {
      load8(sc.gk + off, k);
      load8(sc.gv + off, v);
    } else {
      load8(sc.pk + off, k);
      load8(seq_v(src, b, h, tok_begin + tt) + part * 8, v);
    }
    const float vlen = row_norm8<D>(v);
    float ka[8], va[8];
    attn_rows<D>(k, v, vlen, part, L, ka, va);
    if (valid) {
      const int64_t slot = state_before + pos[t];
      const int64_t so = (int64_t(row) * st.capacity + slot) * D + part * 8;
      store8(static_cast<uint16_t *>(st.s_k) + so, k);
      store8(static_cast<uint16_t *>(st.s_v) + so, v);
      if (part == 0)
        static_cast<float *>(st.s_vlen)[int64_t(row) * st.capacity + slot] =
            vlen;
      const int64_t ao = (int64_t(row) * attn_cur.cap + slot) * D + part * 8;
      store8(attn_cur.k + ao, ka);
      store8(attn_cur.v + ao, va);
    }
  }
}

// ---------------------------------------------------------------------------
// Merge + refresh (model/kvm_mixer.py:329-335): slot j gains
// bf16(sum of merge keys / values routed to it), summed in fp32 in token
// order; every slot < s_after gets fresh attention rows in attn_out.
// Workgroup: 4 waves x (64 / (D/8)) slots, D/8 lanes per slot.  The tokens
// routed to the workgroup's slots are counted and placed with LDS atomics,
// then each slot's list is sorted by token index (rank sort), so the fp32
// sums run in token order whatever the arrival order; the gathers are
// issued four rows at a time.
template <int D>
__global__ __launch_bounds__(kThreads) void k_merge_refresh(
    kvm_layer L, int n_tok, int s_after, kvm_state st, AttnRows attn_out,
    UpdateScratch sc, int parity, int in_place) {
  constexpr int G = D / 8;
  constexpr int SPW = 64 / G;   // slots per wave
  constexpr int SPB = 4 * SPW;  // slots per workgroup
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  int *mr = reinterpret_cast<int *>(smem);  // [n_tok] local slot of each token, -1 otherwise
  int *list = mr + n_tok;                   // [n_tok] placed tokens
  int *sorted = list + n_tok;               // [n_tok] lists in token order
  __shared__ int cnt[SPB], off[SPB], fill[SPB];
  const int row = blockIdx.x;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t base = int64_t(row) * n_tok;
  const int part = lane % G;
  const int local = wave * SPW + lane / G;
  const int j0 = blockIdx.y * SPB;
  const int j = j0 + local;
  const bool valid = j < s_after;
  const int jj = valid ? j : 0;

  // The slot's current sums and vlen, in flight during the listing (in
  // place: loaded after it, for the slots that change).
  const int64_t so = (int64_t(row) * st.capacity + jj) * D + part * 8;
  auto load_k = [&]() { return *reinterpret_cast<const uint4 *>(static_cast<const uint16_t *>(st.s_k) + so); };
  auto load_v = [&]() { return *reinterpret_cast<const uint4 *>(static_cast<const uint16_t *>(st.s_v) + so); };
  auto load_vlen = [&]() { return static_cast<const float *>(st.s_vlen)[int64_t(row) * st.capacity + jj]; };
  uint4 k_raw = make_uint4(0, 0, 0, 0), v_raw = make_uint4(0, 0, 0, 0);
  float vlen = 0.f;
  if (!in_place) {
    k_raw = load_k();
    v_raw = load_v();
    vlen = load_vlen();
  }

  if (tid < SPB) {
    cnt[tid] = 0;
    fill[tid] = 0;
  }
  __syncthreads();
  for (int t = tid; t < n_tok; t += kThreads) {
    int r = -1;
    if (!sc.is_append[base + t]) {
      const uint64_t key = sc.rkey[parity][base + t];
      if (key) r = int(0xffffffffu - uint32_t(key & 0xffffffffu));
    }
    const int lr = (r >= j0 && r < j0 + SPB && r < s_after) ? r - j0 : -1;
    mr[t] = lr;
    if (lr >= 0) atomicAdd(&cnt[lr], 1);
  }
  __syncthreads();
  if (tid == 0) {
    int run = 0;
    for (int i = 0; i < SPB; ++i) {
      off[i] = run;
      run += cnt[i];
    }
  }
  __syncthreads();
  for (int t = tid; t < n_tok; t += kThreads) {
    const int lr = mr[t];
    if (lr >= 0) list[off[lr] + atomicAdd(&fill[lr], 1)] = t;
  }
  __syncthreads();
  const int n = valid ? cnt[local] : 0;
  const int o = off[local];
  for (int e = part; e < n; e += G) {
    const int x = list[o + e];
    int r = 0;
    for (int f = 0; f < n; ++f) r += list[o + f] < x;
    sorted[o + r] = x;
  }
  __syncthreads();
  if (in_place) {
    // Unchanged slots keep their state and attention rows (appended slots
    // got theirs from k_rank_append); no barrier follows.
    if (n == 0) return;
    k_raw = load_k();
    v_raw = load_v();
    vlen = load_vlen();
  }

  float sk[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  float sv[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  for (int i0 = 0; i0 < n; i0 += 4) {
    uint4 xk[4], xv[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      if (i0 + u < n) {
        const int64_t to = (base + sorted[o + i0 + u]) * D + part * 8;
        xk[u] = *reinterpret_cast<const uint4 *>(sc.gk + to);
        xv[u] = *reinterpret_cast<const uint4 *>(sc.gv + to);
      }
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      if (i0 + u < n) {
        float fk[8], fv[8];
        unpack8(xk[u], fk);
        unpack8(xv[u], fv);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
          sk[i] += fk[i];
          sv[i] += fv[i];
        }
      }
    }
  }
  float k[8], v[8];
  unpack8(k_raw, k);
  unpack8(v_raw, v);
  if (n > 0) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      k[i] = rbf(k[i] + rbf(sk[i]));
      v[i] = rbf(v[i] + rbf(sv[i]));
    }
    if (valid) {
      store8(static_cast<uint16_t *>(st.s_k) + so, k);
      store8(static_cast<uint16_t *>(st.s_v) + so, v);
    }
  }
  float ka[8], va[8];
  attn_rows<D>(k, v, vlen, part, L, ka, va);
  if (valid) {
    const int64_t ao = (int64_t(row) * attn_out.cap + j) * D + part * 8;
    store8(attn_out.k + ao, ka);
    store8(attn_out.v + ao, va);
  }
}

// Route of every overflow token (appended tokens: their new slot), for logs.
__global__ __launch_bounds__(256) void k_route_out(int n, UpdateScratch sc, int parity,
                                                   int32_t *route_out, int32_t *append_out) {
  const int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x;
  if (i >= n) return;
  const int app = sc.is_append[i];
  int r = -1;
  if (app) {
    r = sc.route[i];
  } else {
    const uint64_t key = sc.rkey[parity][i];
    if (key) r = int(0xffffffffu - uint32_t(key & 0xffffffffu));
  }
  if (route_out) route_out[i] = r;
  if (append_out) append_out[i] = app;
}

// Clear both route-key buffers and the novelty keys of a fresh workspace.
__global__ __launch_bounds__(256) void k_zero_keys(int64_t n, UpdateScratch sc) {
  const int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x;
  if (i >= n) return;
  sc.rkey[0][i] = 0;
  sc.rkey[1][i] = 0;
  sc.nkey[i] = 0;
}

// Window ring write: token 0 of src -> ring slot pos of every row.
template <int D>
__global__ __launch_bounds__(64) void k_ring_write(kvm_layer L, kvm_seq src,
                                                   uint16_t *rk, uint16_t *rv,
                                                   uint16_t *rg,
                                                   int64_t ring_cap,
                                                   int64_t pos, const int32_t *ctl) {
  if (ctl) {  // row after the window held in device counters (clamped to the ring)
    const int64_t start = ((int64_t(ctl[1]) % ring_cap) + ring_cap) % ring_cap;
    const int64_t len = min(max(int64_t(ctl[2]), int64_t(0)), ring_cap);
    pos = (start + len) % ring_cap;
  }
  const int row = blockIdx.x;
  const int b = row / int(L.kv_heads), h = row % int(L.kv_heads);
  const int lane = threadIdx.x;
  constexpr int G = D / 8;
  const int64_t o = (int64_t(row) * ring_cap + pos) * D;
  if (lane < G) {
    *reinterpret_cast<uint4 *>(rk + o + lane * 8) =
        *reinterpret_cast<const uint4 *>(seq_k(src, b, h, 0) + lane * 8);
  } else if (lane >= 32 && lane < 32 + G) {
    const int p = lane - 32;
    *reinterpret_cast<uint4 *>(rv + o + p * 8) =
        *reinterpret_cast<const uint4 *>(seq_v(src, b, h, 0) + p * 8);
  } else if (lane == 63) {
    const uint16_t *g = static_cast<const uint16_t *>(src.gate) + b * src.g_sb +
                        h * src.g_sh;
    rg[int64_t(row) * ring_cap + pos] = *g;
  }
}

inline int64_t rows_of(const kvm_layer &L) { return L.batch * L.kv_heads; }
inline size_t align256(size_t x) { return (x + 255) & ~size_t(255); }

}  // namespace

int64_t update_slice_bytes(const kvm_layer &L, int64_t n_tok) {
  const size_t tok = size_t(rows_of(L)) * size_t(n_tok);
  return int64_t(3 * align256(tok * size_t(L.head_dim) * 2) + 2 * align256(tok * 4));
}

int64_t update_keys_bytes(const kvm_layer &L, int64_t n_tok) {
  const size_t tok = size_t(rows_of(L)) * size_t(n_tok);
  return int64_t(2 * align256(tok * 8) + align256(tok * 4));
}

int64_t update_scratch_bytes(const kvm_layer &L, int64_t n_tok) {
  return update_slice_bytes(L, n_tok) + update_keys_bytes(L, n_tok);
}

UpdateScratch carve_update_scratch(void *slice, void *keys, const kvm_layer &L,
                                   int64_t n_tok) {
  const size_t tok = size_t(rows_of(L)) * size_t(n_tok);
  const size_t kb = align256(tok * size_t(L.head_dim) * 2);
  const size_t qb = align256(tok * 8);
  const size_t ib = align256(tok * 4);
  unsigned char *p = static_cast<unsigned char *>(slice);
  unsigned char *k = static_cast<unsigned char *>(keys);
  UpdateScratch s;
  s.pk = reinterpret_cast<uint16_t *>(p);
  s.gk = reinterpret_cast<uint16_t *>(p + kb);
  s.gv = reinterpret_cast<uint16_t *>(p + 2 * kb);
  s.route = reinterpret_cast<int32_t *>(p + 3 * kb);
  s.is_append = reinterpret_cast<int32_t *>(p + 3 * kb + ib);
  s.rkey[0] = reinterpret_cast<uint64_t *>(k);
  s.rkey[1] = reinterpret_cast<uint64_t *>(k + qb);
  s.nkey = reinterpret_cast<uint32_t *>(k + 2 * qb);
  return s;
}

hipError_t launch_append_direct(const kvm_layer &L, const kvm_seq &src,
                                int64_t tok_begin, int64_t n_tok,
                                const kvm_state &st, int64_t slot_begin,
                                AttnRows attn, bool apply_gate,
                                hipStream_t stream) {
  if (n_tok <= 0) return hipSuccess;
  const int tpw = kThreads / int(L.head_dim / 8);
  dim3 grid(unsigned(rows_of(L)), unsigned((n_tok + tpw - 1) / tpw));
  if (L.head_dim == 128)
    hipLaunchKernelGGL(k_append_direct<128>, grid, dim3(kThreads), 0, stream,
                       L, src, tok_begin, int(n_tok), st, slot_begin, attn,
                       int(apply_gate));
  else
    hipLaunchKernelGGL(k_append_direct<64>, grid, dim3(kThreads), 0, stream,
                       L, src, tok_begin, int(n_tok), st, slot_begin, attn,
                       int(apply_gate));
  return hipGetLastError();
}

hipError_t launch_refresh(const kvm_layer &L, const kvm_state &st,
                          int64_t slot_begin, int64_t n_slots, AttnRows attn,
                          hipStream_t stream) {
  if (n_slots <= 0) return hipSuccess;
  const int spw = kThreads / int(L.head_dim / 8);
  dim3 grid(unsigned(rows_of(L)), unsigned((n_slots + spw - 1) / spw));
  if (L.head_dim == 128)
    hipLaunchKernelGGL(k_refresh<128>, grid, dim3(kThreads), 0, stream, L, st,
                       slot_begin, int(n_slots), attn);
  else
    hipLaunchKernelGGL(k_refresh<64>, grid, dim3(kThreads), 0, stream, L, st,
                       slot_begin, int(n_slots), attn);
  return hipGetLastError();
}

hipError_t launch_zero_keys(const kvm_layer &L, int64_t n_tok,
                            const UpdateScratch &sc, hipStream_t stream) {
  const int64_t n = rows_of(L) * n_tok;
  hipLaunchKernelGGL(k_zero_keys, dim3(unsigned((n + 255) / 256)), dim3(256), 0, stream, n, sc);
  return hipGetLastError();
}

hipError_t launch_prep(const kvm_layer &L, const kvm_seq &src, const PrepList &P,
                       int64_t n_tok, const UpdateScratch &s0, int64_t slice_bytes,
                       hipStream_t stream) {
  if (P.count <= 0) return hipSuccess;
  const dim3 grid{unsigned(rows_of(L)), unsigned((n_tok + 63) / 64), unsigned(P.count)};
  if (L.head_dim == 128)
    hipLaunchKernelGGL(k_prep<128>, grid, dim3(kThreads), 0, stream, L, src, P, int(n_tok), s0,
                       slice_bytes);
  else
    hipLaunchKernelGGL(k_prep<64>, grid, dim3(kThreads), 0, stream, L, src, P, int(n_tok), s0,
                       slice_bytes);
  return hipGetLastError();
}

template <int D>
static hipError_t launch_update_d(const kvm_layer &L, const kvm_seq &src,
                                  int64_t tok_begin, int64_t n_tok,
                                  int64_t state_before, int64_t n_append,
                                  const kvm_state &st, AttnRows attn_in,
                                  AttnRows attn_out, const UpdateScratch &sc,
                                  int parity, int32_t *route_out,
                                  int32_t *append_out, hipStream_t stream) {
  const unsigned rows = unsigned(rows_of(L));
  const int s_after = int(state_before + n_append);
  const int protect = int(L.sink_len < s_after ? L.sink_len : s_after);
  const unsigned tiles = unsigned((n_tok + kRouteTok - 1) / kRouteTok);
  hipError_t e;
  if (n_append > 0) {
    const unsigned nsplit = unsigned((state_before + kSplit - 1) / kSplit);
    hipLaunchKernelGGL((k_route<D, true>), dim3(rows * tiles * nsplit), dim3(kThreads), 0, stream, L,
                       int(n_tok), attn_in, int(state_before), 0, sc, parity, int(tiles), int(nsplit));
    if ((e = hipGetLastError()) != hipSuccess) return e;
    const size_t lds = size_t(n_tok) * 12;
    hipLaunchKernelGGL(k_rank_append<D>, dim3(rows), dim3(512), lds, stream, L,
                       src, tok_begin, int(n_tok), int(n_append),
                       int(state_before), st, attn_in, sc);
    if ((e = hipGetLastError()) != hipSuccess) return e;
  }
  const unsigned rsplit = unsigned((s_after + kSplit - 1) / kSplit);
  hipLaunchKernelGGL((k_route<D, false>), dim3(rows * tiles * rsplit), dim3(kThreads), 0, stream, L,
                     int(n_tok), attn_in, s_after, protect, sc, parity, int(tiles), int(rsplit));
  if ((e = hipGetLastError()) != hipSuccess) return e;
  if (route_out || append_out) {
    const int64_t n = int64_t(rows) * n_tok;
    hipLaunchKernelGGL(k_route_out, dim3(unsigned((n + 255) / 256)), dim3(256), 0, stream,
                       int(n), sc, parity, route_out, append_out);
    if ((e = hipGetLastError()) != hipSuccess) return e;
  }
  constexpr int spb = 4 * (64 / (D / 8));
  const dim3 mgrid{rows, unsigned((s_after + spb - 1) / spb), 1u};
  const int in_place = attn_out.k == attn_in.k && attn_out.v == attn_in.v && attn_out.cap == attn_in.cap;
  hipLaunchKernelGGL(k_merge_refresh<D>, mgrid, dim3(kThreads), size_t(n_tok) * 12, stream, L,
                     int(n_tok), s_after, st, attn_out, sc, parity, in_place);
  return hipGetLastError();
}

hipError_t launch_update(const kvm_layer &L, const kvm_seq &src,
                         int64_t tok_begin, int64_t n_tok, int64_t state_before,
                         int64_t n_append, const kvm_state &st, AttnRows attn_in,
                         AttnRows attn_out, const UpdateScratch &sc, int parity,
                         int32_t *route_out, int32_t *append_out,
                         hipStream_t stream) {
  if (L.head_dim == 128)
    return launch_update_d<128>(L, src, tok_begin, n_tok, state_before, n_append, st, attn_in,
                                attn_out, sc, parity, route_out, append_out, stream);
  return launch_update_d<64>(L, src, tok_begin, n_tok, state_before, n_append, st, attn_in,
                             attn_out, sc, parity, route_out, append_out, stream);
}

hipError_t launch_ring_write(const kvm_layer &L, const kvm_seq &src,
                             void *ring_k, void *ring_v, void *ring_gate,
                             int64_t ring_cap, int64_t pos,
                             hipStream_t stream, const int32_t *ctl) {
  dim3 grid(unsigned(rows_of(L)));
  if (L.head_dim == 128)
    hipLaunchKernelGGL(k_ring_write<128>, grid, dim3(64), 0, stream, L, src,
                       static_cast<uint16_t *>(ring_k),
                       static_cast<uint16_t *>(ring_v),
                       static_cast<uint16_t *>(ring_gate), ring_cap, pos, ctl);
  else
    hipLaunchKernelGGL(k_ring_write<64>, grid, dim3(64), 0, stream, L, src,
                       static_cast<uint16_t *>(ring_k),
                       static_cast<uint16_t *>(ring_v),
                       static_cast<uint16_t *>(ring_gate), ring_cap, pos, ctl);
  return hipGetLastError();
}

}  // namespace kvm
