// Backward of the KVM memory state under the forward's routes, on gfx950.
//
// The state of one row (batch, kv head) is a set of slots whose key / value
// sums s_k, s_v evolve over the prefill's updates: slot j starts as an
// initial token row (j < L0) or as the token row appended into it by some
// update, and every later merge routed to it adds a token row.  Snapshot s
// (the state after s updates) contributes attention rows
//   ka = LayerNorm_s(s_k) = ((s_k - mean) / sqrt(var + eps)) w + b,
//   va = normalize(s_v) * vlen,
// whose gradients (G_k, G_v) the attention backward produced.  With sums in
// fp32 and the forward's bf16 roundings taken as the identity (as the
// reference's training kernels do, model/kernels/kvm_triton_training_kernels.py:2093-2745):
//   dL/ds(s) = sum over snapshots s' >= s that hold the slot of the local
//              LayerNorm / normalisation backward H(s') (identity carry),
//   a token merged by update u into slot j gets dL/ds(u + 1)[j];
//   an appended token gets the same for the slot's base row, plus the vlen
//   gradient sum_{s'} G_v . normalize(s_v) of the snapshots holding it;
//   the initial rows get dL/ds(0).
// The token rows themselves are functions of the raw tokens
// (model/kvm_mixer.py:120-129, 231-248, 321-340, 434-447):
//   prep = LayerNorm_s(k with dims < rope_partial_dim zeroed),
//   merge rows   (prep * g if gate_keys, v * g if gate_values),
//   append rows  (the merge rows if gate_appends, else prep, v), vlen = |append value row|,
//   initial rows (prep * g, v * g if gate_initial, else prep, v), vlen = |v|,
// and this kernel recomputes them from the bf16 tokens and carries the chain
// rule down to dk, dv (added to the attention backward's window gradients),
// the merge gate and the LayerNorm parameters (both uses of ln_s_k).
// One single-wave workgroup owns RPW slots of one row (a lane group of D/8
// lanes per slot) and holds their sums and gradient accumulators in
// registers: a forward scan over the updates rebuilds the final sums, a
// reverse scan accumulates H and undoes each update's merges.  The tokens
// routed to the workgroup's slots in one update are processed RPW at a time,
// one per lane group whatever slot they belong to (the per-token LayerNorm
// and chain rule keep every lane busy); their rows and the slots' gradients
// cross between lane groups through LDS, and each owner folds its tokens in
// list (token) order.  Every state token is routed to exactly one slot, so
// each token row of dk / dv / dgate has exactly one writer (no atomics).

#include "kvm_device.hpp"
#include "kvm_internal.hpp"
#include "kvm_seq.hpp"

namespace kvm {
namespace {

constexpr int kThreads = 64;  // one wave per workgroup: the per-update compaction needs no barrier
constexpr int kMaxChunk = 4096;
constexpr float kNormEps = 1e-12f;  // torch.nn.functional.normalize
constexpr int kPf = 8;              // route entries per lane loaded one update ahead

__device__ __forceinline__ void load8f(const float *p, float (&x)[8]) {
  const float4 a = *reinterpret_cast<const float4 *>(p), b = *reinterpret_cast<const float4 *>(p + 4);
  x[0] = a.x; x[1] = a.y; x[2] = a.z; x[3] = a.w;
  x[4] = b.x; x[5] = b.y; x[6] = b.z; x[7] = b.w;
}
__device__ __forceinline__ void store8f(float *p, const float (&x)[8]) {
  *reinterpret_cast<float4 *>(p) = make_float4(x[0], x[1], x[2], x[3]);
  *reinterpret_cast<float4 *>(p + 4) = make_float4(x[4], x[5], x[6], x[7]);
}

enum TokKind { kMerged = 0, kAppended = 1, kInitial = 2 };

// One raw token of the row, recomputed in fp32: xh = normalised rope-zeroed
// key, prep = xh * w + b, the value row and the gate.
struct Tok {
  float xh[8], prep[8], v[8];
  float r, g;
};

// Raw bf16 loads of one token (issued early, used later).
struct RawTok {
  uint4 k, v;
  uint32_t g;
};
// Token rows of one (batch, kv head): the prefill's k / v / gate views (no ring).
struct RowSrc {
  const uint16_t *k, *v, *g;
  int64_t k_st, v_st, g_st;
};
__device__ __forceinline__ RawTok fetch_tok(const RowSrc &R, int64_t t, int part) {
  RawTok r;
  r.k = *reinterpret_cast<const uint4 *>(R.k + t * R.k_st + part * 8);
  r.v = *reinterpret_cast<const uint4 *>(R.v + t * R.v_st + part * 8);
  r.g = R.g[t * R.g_st];
  return r;
}

template <int D>
__device__ __forceinline__ void make_tok(const StateBwdArgs &A, const RawTok &r, int part, const float (&w)[8],
                                         const float (&bb)[8], Tok &x) {
  float k[8];
  unpack8(r.k, k);
  unpack8(r.v, x.v);
  x.g = bf2f(r.g);
#pragma unroll
  for (int e = 0; e < 8; ++e)
    if (part * 8 + e < A.L.rope_partial_dim) k[e] = 0.f;
  float s = 0.f;
#pragma unroll
  for (int e = 0; e < 8; ++e) s += k[e];
  const float mean = group_sum<D / 8>(s) / float(D);
  float q = 0.f;
#pragma unroll
  for (int e = 0; e < 8; ++e) q += (k[e] - mean) * (k[e] - mean);
  x.r = 1.0f / sqrtf(group_sum<D / 8>(q) / float(D) + float(A.L.ln_eps));
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    x.xh[e] = (k[e] - mean) * x.r;
    x.prep[e] = x.xh[e] * w[e] + bb[e];
  }
}

// Whether the gate multiplies a token's key / value row: merge rows follow
// gate_keys / gate_values, appended rows are the merge rows when
// gate_appends is set (else ungated), initial rows follow gate_initial
// (model/kvm_mixer.py:264-281, 434-441).
__device__ __forceinline__ bool gate_k(const kvm_layer &L, int kind) {
  return kind == kMerged ? L.gate_keys != 0
         : kind == kAppended ? (L.gate_appends != 0 && L.gate_keys != 0)
                             : L.gate_initial != 0;
}
__device__ __forceinline__ bool gate_v(const kvm_layer &L, int kind) {
  return kind == kMerged ? L.gate_values != 0
         : kind == kAppended ? (L.gate_appends != 0 && L.gate_values != 0)
                             : L.gate_initial != 0;
}

// The key / value rows a token contributes to the state.
__device__ __forceinline__ void tok_rows(const kvm_layer &L, const Tok &x, int kind, float (&rk)[8],
                                         float (&rv)[8]) {
  const bool gk = gate_k(L, kind), gv = gate_v(L, kind);
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    rk[e] = gk ? x.prep[e] * x.g : x.prep[e];
    rv[e] = gv ? x.v[e] * x.g : x.v[e];
  }
}

// Chain rule from the gradients of a token's state rows (dk_row, dv_row and
// the vlen gradient dl) to dk, dv, dgate of the token and the LayerNorm
// parameters.  dk / dv hold the token's current rows of A.dk / A.dv (loaded
// by the caller ahead of time); the sums are stored back (one writer per
// token row).
template <int D>
__device__ __forceinline__ void tok_backward(const StateBwdArgs &A, const Tok &x, int kind, int64_t tok_row,
                                             int part, const float (&w)[8], const float (&dk_row)[8],
                                             const float (&dv_row)[8], float dl, float (&dlw)[8],
                                             float (&dlb)[8], float (&dk)[8], float (&dv)[8]) {
  const bool gk = gate_k(A.L, kind), gv = gate_v(A.L, kind);
  float dxv[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) dxv[e] = dv_row[e];
  float dvl[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};  // vlen gradient on the raw value (initial)
  if (kind != kMerged) {
    // vlen = |append value row| (appended) or |v| (initial)
    float rv[8], n2 = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      rv[e] = (kind == kAppended && gv) ? x.v[e] * x.g : x.v[e];
      n2 += rv[e] * rv[e];
    }
    const float n = sqrtf(group_sum<D / 8>(n2));
    const float c = n > 0.f ? dl / n : 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      if (kind == kAppended)
        dxv[e] += c * rv[e];
      else
        dvl[e] = c * rv[e];
    }
  }
  float dg = 0.f, dprep[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    dprep[e] = gk ? dk_row[e] * x.g : dk_row[e];
    if (gk) dg += dk_row[e] * x.prep[e];
    if (gv) dg += dxv[e] * x.v[e];
  }
  dg = group_sum<D / 8>(dg);
  float m1 = 0.f, m2 = 0.f, dxh[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    dxh[e] = dprep[e] * w[e];
    m1 += dxh[e];
    m2 += dxh[e] * x.xh[e];
    dlw[e] += dprep[e] * x.xh[e];
    dlb[e] += dprep[e];
  }
  m1 = group_sum<D / 8>(m1) / float(D);
  m2 = group_sum<D / 8>(m2) / float(D);
  const int64_t o = tok_row * D + part * 8;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    if (part * 8 + e >= A.L.rope_partial_dim) dk[e] += x.r * (dxh[e] - m1 - x.xh[e] * m2);
    dv[e] += (gv ? dxv[e] * x.g : dxv[e]) + dvl[e];
  }
  store8f(A.dk + o, dk);
  store8f(A.dv + o, dv);
  if (part == 0) A.dgate[tok_row] = dg;
}

template <int D>
__global__ __launch_bounds__(kThreads) void k_state_bwd(StateBwdArgs A, UpdTable U, float *__restrict__ dln_part) {
  constexpr int GL = D / 8;            // lanes per slot row (a lane group)
  constexpr int RPW = kThreads / GL;   // slot rows per workgroup = lane groups
  // Tokens of the current update routed to this workgroup's slots, in token
  // order: (token << 8) | (local slot << 1) | appended (dynamic LDS, chunk_len entries).
  extern __shared__ int32_t lst[];
  __shared__ __attribute__((aligned(16))) float rows[RPW][2][D];  // token rows, one per lane group
  __shared__ __attribute__((aligned(16))) float accb[RPW][2][D];  // slot gradients (reverse scan)
  __shared__ float accl_s[RPW];
  __shared__ float red[2][D];
  const int tid = threadIdx.x, part = tid % GL, lane = tid & 63;
  const int row = blockIdx.y;
  const int hb = row / int(A.L.kv_heads), hh = row % int(A.L.kv_heads);
  const int j0 = blockIdx.x * RPW, my = tid / GL;
  const int j = j0 + my;  // this lane group's slot
  const int C = int(A.L.chunk_len), L0 = int(A.L0), nu = int(A.n_updates);
  const int64_t rowT = int64_t(row) * A.T;
  const float eps = float(A.L.ln_eps);
  RowSrc R;
  R.k = static_cast<const uint16_t *>(A.kv.k) + hb * A.kv.k_sb + hh * A.kv.k_sh;
  R.v = static_cast<const uint16_t *>(A.kv.v) + hb * A.kv.v_sb + hh * A.kv.v_sh;
  R.g = static_cast<const uint16_t *>(A.kv.gate) + hb * A.kv.g_sb + hh * A.kv.g_sh;
  R.k_st = A.kv.k_st;
  R.v_st = A.kv.v_st;
  R.g_st = A.kv.g_st;
  float w[8], bb[8];
  load8f(static_cast<const float *>(A.L.ln_weight) + part * 8, w);
  load8f(static_cast<const float *>(A.L.ln_bias) + part * 8, bb);
  auto tb_of = [&](int u) { return U.token_begin[u]; };
  auto before_of = [&](int u) { return U.state_before[u]; };
  auto napp_of = [&](int u) { return U.n_append[u]; };
  // Route / append entries of the first kPf * 64 tokens of an update are
  // loaded one update ahead (in registers); the rest, if any, when used.
  int pr[kPf], pa[kPf];
  auto prefetch = [&](int u) {
    if (u < 0 || u >= nu) return;
    const int64_t o = (int64_t(u) * A.rows + row) * C;
#pragma unroll
    for (int it = 0; it < kPf; ++it) {
      const int t = it * kThreads + tid;
      pr[it] = t < C ? A.route_log[o + t] : -1;
      pa[it] = t < C ? A.append_log[o + t] : 0;
    }
  };
  // Ordered compaction of update u's routes onto [j0, j0 + RPW) (the first
  // part from the prefetched registers); returns the list length (the same
  // in every lane).
  auto stage = [&](int u) {
    const int64_t o = (int64_t(u) * A.rows + row) * C;
    int n = 0;
    __syncthreads();  // the previous list has been read
    auto add = [&](int t, int r, int a) {
      const bool hit = r >= j0 && r < j0 + RPW;
      const uint64_t m = __ballot(hit);
      if (hit) lst[n + __popcll(m & ((uint64_t(1) << lane) - 1))] = (t << 8) | ((r - j0) << 1) | (a ? 1 : 0);
      n += __popcll(m);
    };
#pragma unroll
    for (int it = 0; it < kPf; ++it) add(it * kThreads + tid, pr[it], pa[it]);
    for (int t0 = kPf * kThreads; t0 < C; t0 += kThreads) {
      const int t = t0 + tid;
      add(t, t < C ? A.route_log[o + t] : -1, t < C ? A.append_log[o + t] : 0);
    }
    __syncthreads();  // the list is complete
    return n;
  };
  auto put_rows = [&](const float (&rk)[8], const float (&rv)[8]) {
    store8f(&rows[my][0][part * 8], rk);
    store8f(&rows[my][1][part * 8], rv);
  };

  // ---- forward scan: final fp32 sums of my slot, and its vlen.  Lane group
  // g prepares the rows of list entry i0 + g; the owning group then folds
  // them in list order.
  float sk[8], sv[8];
  float vlen = 0.f;
  if (j < L0) {
    Tok x;
    make_tok<D>(A, fetch_tok(R, j, part), part, w, bb, x);
    tok_rows(A.L, x, kInitial, sk, sv);
    vlen = row_norm8<D>(x.v);
  } else {
#pragma unroll
    for (int e = 0; e < 8; ++e) sk[e] = sv[e] = 0.f;
  }
  prefetch(0);
  for (int u = 0; u < nu; ++u) {
    const int n = stage(u);
    prefetch(u + 1);
    const int tb = tb_of(u);
    float dk[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f}, dv[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    for (int i0 = 0; i0 < n; i0 += RPW) {
      const int i = i0 + my;
      const int e = i < n ? lst[i] : 0;
      Tok x;
      make_tok<D>(A, fetch_tok(R, tb + (e >> 8), part), part, w, bb, x);
      float rk[8], rv[8];
      tok_rows(A.L, x, (e & 1) ? kAppended : kMerged, rk, rv);
      put_rows(rk, rv);
      __syncthreads();
      for (int g = 0; g < RPW && i0 + g < n; ++g) {
        const int eg = lst[i0 + g];
        if (((eg >> 1) & 127) != my) continue;
        float xk[8], xv[8];
        load8f(&rows[g][0][part * 8], xk);
        load8f(&rows[g][1][part * 8], xv);
        if (eg & 1) {  // the slot's base row (appended before this update's merges)
#pragma unroll
          for (int c = 0; c < 8; ++c) {
            sk[c] = xk[c];
            sv[c] = xv[c];
          }
          vlen = row_norm8<D>(sv);
        } else {
#pragma unroll
          for (int c = 0; c < 8; ++c) {
            dk[c] += xk[c];
            dv[c] += xv[c];
          }
        }
      }
      __syncthreads();  // rows is rewritten by the next batch
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      sk[e] += dk[e];
      sv[e] += dv[e];
    }
  }

  // ---- reverse scan.
  float gk[8], gv[8], acck[8], accv[8], dlw[8], dlb[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) acck[e] = accv[e] = dlw[e] = dlb[e] = 0.f;
  float accl = 0.f;  // d vlen of my slot (row-reduced, replicated over the group's lanes)
  auto snap_len = [&](int s) { return s == 0 ? L0 : before_of(s - 1) + napp_of(s - 1); };
  // Snapshot-row gradients of snapshot s at my slot (issued one step ahead).
  auto load_snap = [&](int s) {
    if (j < snap_len(s)) {
      const int64_t so = ((int64_t(s) * A.rows + row) * A.max_state_len + j) * D + part * 8;
      load8f(A.d_snap_k + so, gk);
      load8f(A.d_snap_v + so, gv);
    }
  };
  prefetch(nu - 1);
  load_snap(nu);
  for (int s = nu; s >= 0; --s) {
    const int len = snap_len(s);
    if (j < len) {
      // Local backward of snapshot s at my slot.
      float mean = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) mean += sk[e];
      mean = group_sum<GL>(mean) / float(D);
      float var = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) var += (sk[e] - mean) * (sk[e] - mean);
      var = group_sum<GL>(var) / float(D);
      const float r = 1.0f / sqrtf(var + eps);
      float xh[8], dxh[8], m1 = 0.f, m2 = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        xh[e] = (sk[e] - mean) * r;
        dxh[e] = gk[e] * w[e];
        m1 += dxh[e];
        m2 += dxh[e] * xh[e];
        dlw[e] += gk[e] * xh[e];
        dlb[e] += gk[e];
      }
      m1 = group_sum<GL>(m1) / float(D);
      m2 = group_sum<GL>(m2) / float(D);
#pragma unroll
      for (int e = 0; e < 8; ++e) acck[e] += r * (dxh[e] - m1 - xh[e] * m2);
      // va = sv / max(|sv|, eps) * vlen
      float nn = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) nn += sv[e] * sv[e];
      const float nrm = sqrtf(group_sum<GL>(nn));
      const float inv = 1.0f / fmaxf(nrm, kNormEps);
      float gs = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) gs += gv[e] * sv[e] * inv;
      gs = group_sum<GL>(gs);
      accl += gs;
      const float proj = nrm > kNormEps ? gs * inv : 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) accv[e] += vlen * inv * (gv[e] - proj * sv[e]);
    }
    if (s == 0) break;
    // Undo update s - 1, which built snapshot s from snapshot s - 1: lane
    // group g runs the token-side chain rule of list entry i0 + g with the
    // owning slot's gradient (published in accb), the owner subtracts the
    // merged rows in list order.
    const int u = s - 1;
    const int n = stage(u);
    prefetch(u - 1);
    load_snap(s - 1);  // used at the next step
    const int tb = tb_of(u);
    store8f(&accb[my][0][part * 8], acck);
    store8f(&accb[my][1][part * 8], accv);
    if (part == 0) accl_s[my] = accl;
    __syncthreads();
    for (int i0 = 0; i0 < n; i0 += RPW) {
      const int i = i0 + my;
      const bool valid = i < n;
      const int e = valid ? lst[i] : 0;
      const int64_t t = tb + (e >> 8);
      const int ls = (e >> 1) & 127;
      const RawTok raw = fetch_tok(R, t, part);
      float cdk[8], cdv[8];  // the token's rows of A.dk / A.dv, loaded with its k / v
      const int64_t o = (rowT + t) * D + part * 8;
      load8f(A.dk + o, cdk);
      load8f(A.dv + o, cdv);
      Tok x;
      make_tok<D>(A, raw, part, w, bb, x);
      float ak[8], av[8];
      load8f(&accb[ls][0][part * 8], ak);
      load8f(&accb[ls][1][part * 8], av);
      const bool app = (e & 1) != 0;
      if (valid) tok_backward<D>(A, x, app ? kAppended : kMerged, rowT + t, part, w, ak, av,
                                 app ? accl_s[ls] : 0.f, dlw, dlb, cdk, cdv);
      float rk[8], rv[8];
      tok_rows(A.L, x, kMerged, rk, rv);
      put_rows(rk, rv);
      __syncthreads();
      for (int g = 0; g < RPW && i0 + g < n; ++g) {
        const int eg = lst[i0 + g];
        if (((eg >> 1) & 127) != my || (eg & 1)) continue;
        float xk[8], xv[8];
        load8f(&rows[g][0][part * 8], xk);
        load8f(&rows[g][1][part * 8], xv);
#pragma unroll
        for (int c = 0; c < 8; ++c) {
          sk[c] -= xk[c];
          sv[c] -= xv[c];
        }
      }
      __syncthreads();  // rows is rewritten by the next batch
    }
    if (j >= before_of(u) && j < before_of(u) + napp_of(u)) {  // the slot did not exist before
#pragma unroll
      for (int e = 0; e < 8; ++e) acck[e] = accv[e] = sk[e] = sv[e] = 0.f;
      accl = 0.f;
    }
  }
  if (j < L0) {
    Tok x;
    make_tok<D>(A, fetch_tok(R, j, part), part, w, bb, x);
    float cdk[8], cdv[8];
    const int64_t o = (rowT + j) * D + part * 8;
    load8f(A.dk + o, cdk);
    load8f(A.dv + o, cdv);
    tok_backward<D>(A, x, kInitial, rowT + j, part, w, acck, accv, accl, dlw, dlb, cdk, cdv);
  }
  // LayerNorm parameter gradients: sum over the wave, then this workgroup's partial.
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    float x = dlw[e], y = dlb[e];
    // lanes part, part + GL, ... of the wave hold the same features
#pragma unroll
    for (int o = GL; o < 64; o <<= 1) {
      x += __shfl_xor(x, o);
      y += __shfl_xor(y, o);
    }
    if (lane < GL) {
      red[0][part * 8 + e] = x;
      red[1][part * 8 + e] = y;
    }
  }
  __syncthreads();
  for (int i = tid; i < 2 * D; i += kThreads)
    dln_part[(int64_t(blockIdx.y) * gridDim.x + blockIdx.x) * 2 * D + i] = red[i / D][i % D];
}

// d ln_w / d ln_b: feature blockIdx.x of the 2D outputs summed over the
// workgroups' partials (fixed order: strided per thread, then a tree).
__global__ __launch_bounds__(256) void k_state_bwd_ln(const float *part, int nwg, int width, float *out) {
  __shared__ float wred[4];
  const int f = blockIdx.x, tid = threadIdx.x;
  float a = 0.f;
  for (int w = tid; w < nwg; w += 256) a += part[int64_t(w) * width + f];
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) a += __shfl_xor(a, o);
  if ((tid & 63) == 0) wred[tid >> 6] = a;
  __syncthreads();
  if (tid == 0) out[f] = (wred[0] + wred[1]) + (wred[2] + wred[3]);
}

template <int D>
hipError_t launch_d(const StateBwdArgs &a, const UpdTable &sched, float *part, hipStream_t s) {
  constexpr int RPW = kThreads / (D / 8);
  const dim3 grid(unsigned((a.max_state_len + RPW - 1) / RPW), unsigned(a.rows));
  hipLaunchKernelGGL((k_state_bwd<D>), grid, dim3(kThreads), size_t(a.L.chunk_len) * 4, s, a, sched, part);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(k_state_bwd_ln, dim3(2 * D), dim3(256), 0, s, part, int(grid.x * grid.y), 2 * D,
                     a.d_ln);
  return hipGetLastError();
}

}  // namespace

int64_t state_bwd_workspace_bytes(int64_t head_dim, int64_t rows, int64_t max_state_len) {
  const int64_t rpw = kThreads / (head_dim / 8);
  const int64_t nwg = (max_state_len + rpw - 1) / rpw * rows;
  return nwg * 2 * head_dim * 4;
}

int64_t state_bwd_max_chunk() { return kMaxChunk; }

hipError_t launch_state_backward(const StateBwdArgs &a, const UpdTable &sched, float *part,
                                 hipStream_t stream) {
  if (a.L.head_dim == 128) return launch_d<128>(a, sched, part, stream);
  return launch_d<64>(a, sched, part, stream);
}

}  // namespace kvm
