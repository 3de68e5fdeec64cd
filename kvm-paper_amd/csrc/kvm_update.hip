// Block-boundary memory update of the KVM mixer on gfx950.
//
// Reference semantics: model/kvm_mixer.py:250-340 (append + merge),
// model/kvm_fp32_routing_reference.py:24-49 (fp32 merge routing),
// model/kvm_mixer.py:434-447 (initial state), and the Triton contract of
// model/kvm_triton_mixer.py:199-211 (one rounded state write, cached
// normalized state rows).
//
// One update is up to four launches over rows = batch * kv_heads:
//   k_route<PREP=1, NOVELTY>  64 tokens per workgroup: LayerNorm_s of the
//       overflow keys, gated streams to scratch, then the token x slot
//       similarity on bf16 MFMA (fp32 accumulate) and a per-token reduction
//       (argmax for merges, bf16-rounded max for append novelty);
//   k_rank_append             (growable memory only) one workgroup per row
//       ranks novelty in LDS, appends the least novel tokens as new slots;
//   k_route<PREP=0, ROUTE>    (growable only) merge routing against the
//       post-append state;
//   k_merge_refresh           16 slots per workgroup: each slot gathers the
//       tokens routed to it in token order (an LDS list built by a ballot
//       scan; fp32 sum, deterministic, no atomics), writes
//       bf16(state + bf16(sum)) and its LayerNorm / normalized-value
//       attention rows.

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
// Token x slot similarity on MFMA 16x16x32 bf16.
//
// Workgroup: 64 overflow tokens of one row.  The similarity is computed
// transposed, D^T[slot][token] = S_attn . X^T, so the accumulator lane layout
// (lane l holds slots 4*(l/16)+i of token l%16) reduces over slots within a
// lane, then across the 4 lane groups.  Each of the 4 waves takes a
// contiguous quarter of the slots for all 64 tokens (the 4 token tiles stay
// in registers as B operands); slot rows are read straight from global
// memory into A-operand registers, the next 16-slot tile being fetched while
// the current one is multiplied.  The per-wave results are combined in slot
// order, so the first maximum wins as in torch.max.
//
// PREP: compute prep(k), gated streams from the raw tokens (written to
//       scratch); otherwise read the routing operand from scratch.
// NOVELTY: operand prep(k) and value max_j bf16(prep(k).s_attn_j) over all
//       s_lim slots (model/kvm_mixer.py:66-68); otherwise operand = merge key
//       and value = first argmax over slots [protect, s_lim) of the fp32 dot
//       (model/kvm_fp32_routing_reference.py:30-34).
template <int D, bool PREP, bool NOVELTY>
__global__ __launch_bounds__(kThreads) void k_route(
    kvm_layer L, kvm_seq src, int64_t tok_begin, int n_tok, AttnRows sref,
    int s_lim, int protect, UpdateScratch sc) {
  constexpr int G = D / 8;
  constexpr int STR = D + 8;  // LDS row stride (elements), 16 B pad
  constexpr int KS = D / 32;
  __shared__ __attribute__((aligned(16))) uint16_t tok_lds[64 * STR];
  __shared__ float best_lds[4][64];
  __shared__ int idx_lds[4][64];

  const int row = blockIdx.x;
  const int b = row / int(L.kv_heads), h = row % int(L.kv_heads);
  const int tok0 = blockIdx.y * 64;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;

  // (1) routing operand of the 64 tokens -> LDS (zeros past n_tok).  All
  //     token loads are issued before any is consumed.
  constexpr int IT = 64 * G / kThreads;
  uint4 kr[IT], vr[IT];
  float gr[IT];
  if constexpr (PREP) {
#pragma unroll
    for (int it = 0; it < IT; ++it) {
      const int p = tid + it * kThreads;
      const int i_tok = tok0 + p / G;
      const int64_t t = tok_begin + (i_tok < n_tok ? i_tok : 0);
      kr[it] = *reinterpret_cast<const uint4 *>(seq_k(src, b, h, t) + (p % G) * 8);
      vr[it] = *reinterpret_cast<const uint4 *>(seq_v(src, b, h, t) + (p % G) * 8);
      gr[it] = seq_g(src, b, h, t);
    }
  }
#pragma unroll
  for (int it = 0; it < IT; ++it) {
    const int p = tid + it * kThreads;
    const int lt = p / G, part = p % G;
    const int i_tok = tok0 + lt;
    const bool valid = i_tok < n_tok;
    float x[8];
    if constexpr (PREP) {
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
      if (valid) {
        const int64_t off = (int64_t(row) * n_tok + i_tok) * D + part * 8;
        store8(sc.pk + off, k);
        store8(sc.gk + off, gk);
        store8(sc.gv + off, gv);
      }
#pragma unroll
      for (int i = 0; i < 8; ++i) x[i] = valid ? (NOVELTY ? k[i] : gk[i]) : 0.f;
    } else {
      if (valid) {
        const int64_t off = (int64_t(row) * n_tok + i_tok) * D + part * 8;
        load8((NOVELTY ? sc.pk : sc.gk) + off, x);
      } else {
#pragma unroll
        for (int i = 0; i < 8; ++i) x[i] = 0.f;
      }
    }
    store8(&tok_lds[lt * STR + part * 8], x);
  }
  __syncthreads();

  // (2) B operands (X^T) of the 4 token tiles: token tt*16 + lane%16,
  //     dims ks*32 + 8*(lane/16).
  bf16x8 bx[4][KS];
#pragma unroll
  for (int tt = 0; tt < 4; ++tt)
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)
      bx[tt][ks] = as_bf16x8(*reinterpret_cast<const uint4 *>(
          &tok_lds[(tt * 16 + (lane & 15)) * STR + ks * 32 + (lane >> 4) * 8]));

  float best[4] = {-INFINITY, -INFINITY, -INFINITY, -INFINITY};
  int bidx[4] = {-1, -1, -1, -1};
  const uint16_t *sbase = sref.k + int64_t(row) * sref.cap * D;

  // (3) this wave's 16-slot tiles [t_lo, t_hi), fetched NB tiles at a time
  //     with the next batch in flight while the current one is multiplied.
  constexpr int NB = 4;
  const int ntiles = (s_lim + 15) / 16;
  const int tw = (ntiles + 3) / 4;
  const int t_lo = min(wave * tw, ntiles), t_hi = min(t_lo + tw, ntiles);
  auto fetch = [&](int tile0, uint4 (&a)[NB][KS]) {
#pragma unroll
    for (int bt = 0; bt < NB; ++bt) {
      const int j = (tile0 + bt) * 16 + (lane & 15);
      const bool ok = tile0 + bt < t_hi && j < s_lim;
#pragma unroll
      for (int ks = 0; ks < KS; ++ks)
        a[bt][ks] = ok ? *reinterpret_cast<const uint4 *>(sbase + int64_t(j) * D + ks * 32 +
                                                          (lane >> 4) * 8)
                       : make_uint4(0, 0, 0, 0);
    }
  };
  uint4 a_cur[NB][KS], a_nxt[NB][KS];
  if (t_lo < t_hi) fetch(t_lo, a_cur);
  for (int tile0 = t_lo; tile0 < t_hi; tile0 += NB) {
    if (tile0 + NB < t_hi) fetch(tile0 + NB, a_nxt);
#pragma unroll
    for (int bt = 0; bt < NB; ++bt) {
      const int tile = tile0 + bt;
      if (tile >= t_hi) break;
      f32x4 acc[4];
#pragma unroll
      for (int tt = 0; tt < 4; ++tt) {
        acc[tt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ks = 0; ks < KS; ++ks)
          acc[tt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(a_cur[bt][ks]), bx[tt][ks],
                                                            acc[tt], 0, 0, 0);
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int j = tile * 16 + (lane >> 4) * 4 + i;
#pragma unroll
        for (int tt = 0; tt < 4; ++tt) {
          if constexpr (NOVELTY) {
            if (j < s_lim) best[tt] = fmaxf(best[tt], rbf(acc[tt][i]));
          } else {
            if (j >= protect && j < s_lim && acc[tt][i] > best[tt]) {
              best[tt] = acc[tt][i];
              bidx[tt] = j;
            }
          }
        }
      }
    }
#pragma unroll
    for (int bt = 0; bt < NB; ++bt)
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) a_cur[bt][ks] = a_nxt[bt][ks];
  }

  // (4) combine the 4 lane groups holding the same token, then the waves.
#pragma unroll
  for (int tt = 0; tt < 4; ++tt) {
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
      best_lds[wave][tt * 16 + lane] = best[tt];
      idx_lds[wave][tt * 16 + lane] = bidx[tt];
    }
  }
  __syncthreads();
  if (tid < 64) {
    const int i_tok = tok0 + tid;
    float bv = best_lds[0][tid];
    int bi = idx_lds[0][tid];
#pragma unroll
    for (int w = 1; w < 4; ++w) {
      const float ov = best_lds[w][tid];
      const int oi = idx_lds[w][tid];
      if constexpr (NOVELTY) {
        bv = fmaxf(bv, ov);
      } else if (oi >= 0 && (bi < 0 || ov > bv)) {  // waves hold increasing slots
        bv = ov;
        bi = oi;
      }
    }
    if (i_tok < n_tok) {
      const int64_t o = int64_t(row) * n_tok + i_tok;
      if constexpr (NOVELTY) {
        sc.novelty[o] = bv;
      } else if constexpr (PREP) {
        // No appends in this update: every token merges.
        sc.is_append[o] = 0;
        sc.route[o] = bi;
      } else {
        if (sc.is_append[o] == 0) sc.route[o] = bi;
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Append ranking (model/kvm_mixer.py:44-75, 231-248): the n_append tokens
// with the lowest novelty, ties to the lower token index, become slots
// state_before.. in token order.  One workgroup per row; dynamic LDS holds
// novelty, flags and positions of the n_tok tokens.
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

  for (int t = tid; t < n_tok; t += nt) nov[t] = sc.novelty[base + t];
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
// routed to the workgroup's slots are first listed in LDS in token order
// (a ballot scan, no global traffic), then each slot gathers its list four
// rows at a time so the loads overlap.
template <int D>
__global__ __launch_bounds__(kThreads) void k_merge_refresh(
    kvm_layer L, int n_tok, int s_after, kvm_state st, AttnRows attn_out,
    UpdateScratch sc) {
  constexpr int G = D / 8;
  constexpr int SPW = 64 / G;  // slots per wave
  constexpr int SPB = 4 * SPW; // slots per workgroup
  extern __shared__ __attribute__((aligned(16))) unsigned char smem[];
  int *rt = reinterpret_cast<int *>(smem);  // [n_tok] slot of each token (-1: appended)
  int *list = rt + n_tok;                   // [n_tok] tokens grouped by slot
  __shared__ int counts[SPB];
  const int row = blockIdx.x;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t base = int64_t(row) * n_tok;
  const int part = lane % G;
  const int grp = lane / G;
  const int local = wave * SPW + grp;
  const int j = blockIdx.y * SPB + local;
  const bool valid = j < s_after;
  const int jj = valid ? j : 0;

  // The slot's current sums and vlen (in flight during the scans).
  const int64_t so = (int64_t(row) * st.capacity + jj) * D + part * 8;
  const uint4 k_raw = *reinterpret_cast<const uint4 *>(static_cast<const uint16_t *>(st.s_k) + so);
  const uint4 v_raw = *reinterpret_cast<const uint4 *>(static_cast<const uint16_t *>(st.s_v) + so);
  const float vlen = static_cast<const float *>(st.s_vlen)[int64_t(row) * st.capacity + jj];

  for (int t = tid; t < n_tok; t += kThreads)
    rt[t] = sc.is_append[base + t] ? -1 : sc.route[base + t];
  __syncthreads();

  const uint64_t gmask = (G == 64) ? ~0ull : ((1ull << G) - 1ull);
  int cnt = 0;
  for (int g0 = 0; g0 < n_tok; g0 += G) {
    const int t = g0 + part;
    const bool hit = valid && t < n_tok && rt[t] == j;
    cnt += __popcll((__ballot(hit) >> (grp * G)) & gmask);
  }
  if (part == 0) counts[local] = cnt;
  __syncthreads();
  int off = 0;
  for (int i = 0; i < local; ++i) off += counts[i];
  if (cnt > 0) {
    int w = off;
    for (int g0 = 0; g0 < n_tok; g0 += G) {
      const int t = g0 + part;
      const bool hit = valid && t < n_tok && rt[t] == j;
      uint64_t m = (__ballot(hit) >> (grp * G)) & gmask;
      while (m) {
        const int p = __ffsll((unsigned long long)m) - 1;
        m &= m - 1;
        if (part == 0) list[w] = g0 + p;
        ++w;
      }
    }
  }
  __syncthreads();

  float sk[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  float sv[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  for (int i0 = 0; i0 < cnt; i0 += 4) {
    uint4 xk[4], xv[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      if (i0 + u < cnt) {
        const int64_t o = (base + list[off + i0 + u]) * D + part * 8;
        xk[u] = *reinterpret_cast<const uint4 *>(sc.gk + o);
        xv[u] = *reinterpret_cast<const uint4 *>(sc.gv + o);
      }
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      if (i0 + u < cnt) {
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
  if (cnt > 0) {
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

// Window ring write: token 0 of src -> ring slot pos of every row.
template <int D>
__global__ __launch_bounds__(64) void k_ring_write(kvm_layer L, kvm_seq src,
                                                   uint16_t *rk, uint16_t *rv,
                                                   uint16_t *rg,
                                                   int64_t ring_cap,
                                                   int64_t pos) {
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

int64_t update_scratch_bytes(const kvm_layer &L, int64_t n_tok) {
  const size_t rows = size_t(rows_of(L));
  const size_t tok = rows * size_t(n_tok);
  return int64_t(3 * align256(tok * size_t(L.head_dim) * 2) +
                 3 * align256(tok * 4));
}

UpdateScratch carve_update_scratch(void *ws, const kvm_layer &L,
                                   int64_t n_tok) {
  const size_t tok = size_t(rows_of(L)) * size_t(n_tok);
  const size_t kb = align256(tok * size_t(L.head_dim) * 2);
  const size_t ib = align256(tok * 4);
  unsigned char *p = static_cast<unsigned char *>(ws);
  UpdateScratch s;
  s.pk = reinterpret_cast<uint16_t *>(p);
  s.gk = reinterpret_cast<uint16_t *>(p + kb);
  s.gv = reinterpret_cast<uint16_t *>(p + 2 * kb);
  s.novelty = reinterpret_cast<float *>(p + 3 * kb);
  s.route = reinterpret_cast<int32_t *>(p + 3 * kb + ib);
  s.is_append = reinterpret_cast<int32_t *>(p + 3 * kb + 2 * ib);
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

template <int D>
static hipError_t launch_update_d(const kvm_layer &L, const kvm_seq &src,
                                  int64_t tok_begin, int64_t n_tok,
                                  int64_t state_before, int64_t n_append,
                                  const kvm_state &st, AttnRows attn_in,
                                  AttnRows attn_out, const UpdateScratch &sc,
                                  hipStream_t stream) {
  const unsigned rows = unsigned(rows_of(L));
  const int s_after = int(state_before + n_append);
  const int protect = int(L.sink_len < s_after ? L.sink_len : s_after);
  dim3 rgrid(rows, unsigned((n_tok + 63) / 64));
  hipError_t e;
  if (n_append > 0) {
    hipLaunchKernelGGL((k_route<D, true, true>), rgrid, dim3(kThreads), 0,
                       stream, L, src, tok_begin, int(n_tok), attn_in,
                       int(state_before), 0, sc);
    if ((e = hipGetLastError()) != hipSuccess) return e;
    const size_t lds = size_t(n_tok) * 12;
    hipLaunchKernelGGL(k_rank_append<D>, dim3(rows), dim3(512), lds, stream, L,
                       src, tok_begin, int(n_tok), int(n_append),
                       int(state_before), st, attn_in, sc);
    if ((e = hipGetLastError()) != hipSuccess) return e;
    if (n_append < n_tok) {
      hipLaunchKernelGGL((k_route<D, false, false>), rgrid, dim3(kThreads), 0,
                         stream, L, src, tok_begin, int(n_tok), attn_in,
                         s_after, protect, sc);
      if ((e = hipGetLastError()) != hipSuccess) return e;
    }
  } else {
    // No appends: every token merges (the kernel clears the append flags).
    hipLaunchKernelGGL((k_route<D, true, false>), rgrid, dim3(kThreads), 0,
                       stream, L, src, tok_begin, int(n_tok), attn_in, s_after,
                       protect, sc);
    if ((e = hipGetLastError()) != hipSuccess) return e;
  }
  constexpr int spb = 4 * (64 / (D / 8));
  dim3 mgrid(rows, unsigned((s_after + spb - 1) / spb));
  hipLaunchKernelGGL(k_merge_refresh<D>, mgrid, dim3(kThreads),
                     size_t(n_tok) * 8, stream, L, int(n_tok), s_after, st,
                     attn_out, sc);
  return hipGetLastError();
}

hipError_t launch_update(const kvm_layer &L, const kvm_seq &src,
                         int64_t tok_begin, int64_t n_tok, int64_t state_before,
                         int64_t n_append, const kvm_state &st, AttnRows attn_in,
                         AttnRows attn_out, const UpdateScratch &sc,
                         hipStream_t stream) {
  if (L.head_dim == 128)
    return launch_update_d<128>(L, src, tok_begin, n_tok, state_before,
                                n_append, st, attn_in, attn_out, sc, stream);
  return launch_update_d<64>(L, src, tok_begin, n_tok, state_before, n_append,
                             st, attn_in, attn_out, sc, stream);
}

hipError_t launch_ring_write(const kvm_layer &L, const kvm_seq &src,
                             void *ring_k, void *ring_v, void *ring_gate,
                             int64_t ring_cap, int64_t pos,
                             hipStream_t stream) {
  dim3 grid(unsigned(rows_of(L)));
  if (L.head_dim == 128)
    hipLaunchKernelGGL(k_ring_write<128>, grid, dim3(64), 0, stream, L, src,
                       static_cast<uint16_t *>(ring_k),
                       static_cast<uint16_t *>(ring_v),
                       static_cast<uint16_t *>(ring_gate), ring_cap, pos);
  else
    hipLaunchKernelGGL(k_ring_write<64>, grid, dim3(64), 0, stream, L, src,
                       static_cast<uint16_t *>(ring_k),
                       static_cast<uint16_t *>(ring_v),
                       static_cast<uint16_t *>(ring_gate), ring_cap, pos);
  return hipGetLastError();
}

}  // namespace kvm
