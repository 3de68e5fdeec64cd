// The KVM mixer's pre-boundary elementwise work in one kernel on gfx950.
//
// Reference: model/value_residual_mixin.py:173-237 (calc_qkv: value
// residual, RWKV token shift, ln_q / ln_k) and model/kvm_mixer.py:367-401
// (forward_prefix: RoPE, merge gate), after the projection GEMMs.  In the
// reference every step is one torch op over the whole [B, T, H*D] tensor
// (about twenty launches per layer, each reading and writing the tensor);
// here every element is read once and written once.
//
// Work split: a wave covers 32 consecutive tokens of one (batch, head) and
// one row kind: q, k or v.  A row of D features is held by D/8
// consecutive lanes, 8 features per lane (one 16-byte access), so a pass
// works on 64/(D/8) tokens.  The token shift takes the previous token's row
// from the neighbouring lane group (or the pass before): every input row is
// loaded once, and only a wave's first token loads its predecessor.
//
// Rounding: each reference op computes in fp32 and rounds to bf16 (torch's
// opmath for bf16 tensors); the same rounding points are kept here, so the
// outputs match the torch sequence except where an fp32 result of a
// transcendental, of the sigmoid's quotient or of the LayerNorm's reductions
// differs in its last bit.

#include "kvm_device.hpp"
#include "kvm_internal.hpp"

namespace kvm {
namespace {

constexpr int kThreads = 256;

// The rows a value residual reads besides v: v_first and (modes 2 and 3)
// gate_lin, both contiguous [B, T, width].
struct VRes {
  float vf[8], gl[8];
};

// rbf of 8 values, two per conversion instruction.
__device__ __forceinline__ void rbf8(float (&x)[8]) { (void)round_pack8(x); }

// 1 / (1 + exp(-t)) in fp32: the reciprocal from v_rcp_f32 refined by one
// Newton step, which gives the correctly rounded quotient of the division
// except in rare cases one ulp off (and 0 where exp(-t) overflows).
__device__ __forceinline__ float sigmoid_f32(float t) {
  const float d = 1.f + expf(-t);
  const float r = __builtin_amdgcn_rcpf(d);
  return d == INFINITY ? 0.f : __builtin_fmaf(__builtin_fmaf(-d, r, 1.f), r, r);
}

// value residual applied to one row (v in place).  g0: v_gate0 of the lane's
// channels (modes 2, 3); lamb: the mixing weight (mode 1).
__device__ __forceinline__ void value_residual(int mode, float (&v)[8], const VRes &r, const float (&g0)[8],
                                               float lamb) {
  float a[8], b[8];
  if (mode == 1) {  // (1 - lamb) * v + lamb * v_first
    const float c1 = rbf(1.f - lamb);
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      a[i] = c1 * v[i];
      b[i] = lamb * r.vf[i];
    }
    rbf8(a);
    rbf8(b);
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = a[i] + b[i];
  } else {  // v + (v_first - v) * sigmoid(v_gate0 + gate_lin)
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      a[i] = g0[i] + r.gl[i];
      b[i] = r.vf[i] - v[i];
    }
    rbf8(a);
    rbf8(b);
#pragma unroll
    for (int i = 0; i < 8; ++i) a[i] = sigmoid_f32(a[i]);
    rbf8(a);
#pragma unroll
    for (int i = 0; i < 8; ++i) b[i] *= a[i];
    rbf8(b);
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] += b[i];
  }
  rbf8(v);
}

// x + x_mix * (prev - x)
__device__ __forceinline__ void token_shift(float (&x)[8], const float (&prev)[8], const float (&mix)[8]) {
  float d[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) d[i] = prev[i] - x[i];
  rbf8(d);
#pragma unroll
  for (int i = 0; i < 8; ++i) d[i] *= mix[i];
  rbf8(d);
#pragma unroll
  for (int i = 0; i < 8; ++i) x[i] += d[i];
  rbf8(x);
}

// LayerNorm over the row (bf16 output; w, b: the lane's 8 parameters),
// then interleaved-pair RoPE with the row's cos / sin:
// bf16(bf16(cos * x) + bf16(sin * x_pair)).
template <int D>
__device__ __forceinline__ void norm_rope(float (&x)[8], const float (&wf)[8], const float (&bfv)[8], float eps,
                                          const float (&c)[8], const float (&s)[8]) {
  float sum = 0.f;
#pragma unroll
  for (int i = 0; i < 8; ++i) sum += x[i];
  sum = group_sum<D / 8>(sum);
  const float mean = sum / float(D);
  float q = 0.f;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const float d = x[i] - mean;
    q += d * d;
  }
  q = group_sum<D / 8>(q);
  const float rstd = 1.0f / sqrtf(q / float(D) + eps);
#pragma unroll
  for (int i = 0; i < 8; ++i) x[i] = (x[i] - mean) * rstd * wf[i] + bfv[i];
  rbf8(x);
  float a[8], b[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    a[i] = c[i] * x[i];
    b[i] = s[i] * x[i ^ 1];
  }
  rbf8(a);
  rbf8(b);
#pragma unroll
  for (int i = 0; i < 8; ++i) x[i] = a[i] + b[i];
  rbf8(x);
}

// One wave covers kTokWave consecutive tokens of one (batch, head), RPW rows
// (tokens) at a time.  The previous token of a row is the row below it in
// the same pass (a lane move by D/8 lanes) or, for the first row of a pass,
// the last row of the previous pass (carried): only a wave's first token
// loads its predecessor from memory.
constexpr int kTokWave = 32;

// Value `x` of lane (lane - LPR) for lanes of row sub > 0; for sub == 0 the
// value of the last row of the previous pass (`carry`).
template <int LPR>
__device__ __forceinline__ void prev_rows(const float (&x)[8], const float (&carry)[8], int lane,
                                          float (&pv)[8]) {
  const int src = lane >= LPR ? lane - LPR : lane;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const float up = __shfl(x[i], src);
    pv[i] = lane >= LPR ? up : carry[i];
  }
}
// The last row's values (lanes 64 - LPR .. 63) into every lane of the same part.
template <int LPR>
__device__ __forceinline__ void last_row(const float (&x)[8], int part, float (&c)[8]) {
#pragma unroll
  for (int i = 0; i < 8; ++i) c[i] = __shfl(x[i], 64 - LPR + part);
}

// The raw rows one pass of a wave reads (packed bf16, 16 bytes per lane),
// fetched a pass ahead so that their latency overlaps the previous pass: x,
// cos and sin for a q or k row; v, v_first, gate_lin and the key weight for
// a v row.
struct PassRaw {
  uint4 a, b, c;
  uint16_t kw;
};

// The value of a load, pinned where this is called: the compiler cannot sink
// the load past this point (the wave waits here for it).
__device__ __forceinline__ uint4 pinned(uint4 v) {
  typedef unsigned u32x4_t __attribute__((ext_vector_type(4)));
  u32x4_t t = __builtin_bit_cast(u32x4_t, v);
  asm volatile("" : "+v"(t));
  return __builtin_bit_cast(uint4, t);
}

__device__ __forceinline__ uint4 raw8(const void *base, int64_t elem) {
  return *reinterpret_cast<const uint4 *>(static_cast<const uint16_t *>(base) + elem);
}

// What one wave works on: kTokWave tokens from t0 of one (batch, head) row
// kind, channels chan.. of a row of `width` elements.
struct PrefixTile {
  int64_t bi, t0, hk, chan, width;
  int npass, lane, part, sub;
};

// Window-ring row of a single decode token (kv heads): ring_pos, or with
// device counters (start, length) the row after the live ones.
__device__ __forceinline__ int64_t ring_row(const kvm_prefix_desc &P, const PrefixTile &w, int32_t ctl_start,
                                            int32_t ctl_len) {
  int64_t pos = P.ring_pos;
  if (P.ring_ctl) {
    const int64_t cap = P.ring_cap;
    const int64_t start = ((int64_t(ctl_start) % cap) + cap) % cap;
    const int64_t len = min(max(int64_t(ctl_len), int64_t(0)), cap);
    pos = (start + len) % cap;
  }
  return (w.bi * P.kv_heads + w.hk) * P.ring_cap + pos;
}

// q or k rows: carried raw row, token shift, LayerNorm, RoPE.
//
// Prologue (both row kinds): the first pass's rows, then every parameter and
// predecessor row, all loaded before any of them is used and without
// branches around the loads (an unused or NULL operand reads a valid
// stand-in that is never used): a load whose value is consumed inside a
// branch makes the wave wait there, which would give every prologue load a
// round trip of its own.
template <int D>
__device__ __forceinline__ void qk_rows(const kvm_prefix_desc &P, const PrefixTile &w, bool is_q) {
  constexpr int LPR = D / 8, RPW = 64 / LPR;
  const int64_t T = P.seq_len;
  const bool shift = P.token_shift != 0;
  const void *src = is_q ? P.q_lin : P.k_lin;
  auto fetch = [&](int ps, PassRaw &r) {
    const int64_t t = w.t0 + ps * RPW + w.sub;
    const int64_t tt = t < T ? t : T - 1;  // lanes past the end read the last token
    const int64_t ro = w.bi * P.rope_sb + tt * P.rope_st + w.part * 8;
    r.a = raw8(src, (w.bi * T + tt) * P.qkv_st + w.chan);
    r.b = raw8(P.cos, ro);
    r.c = raw8(P.sin, ro);
  };
  PassRaw next;
  fetch(0, next);
  const void *ln_w = is_q ? P.ln_q_w : P.ln_k_w;
  const int64_t own = w.part * 8;  // stand-in index: the lane's LayerNorm weights
  uint4 r_w = raw8(ln_w, own);
  uint4 r_b = raw8(is_q ? P.ln_q_b : P.ln_k_b, own);
  uint4 r_mix = raw8(shift ? (is_q ? P.x_q : P.x_k) : ln_w, shift ? w.chan : own);
  // Predecessor of the tile's first token: the row before it (t0 > 0) or
  // the carried row.
  const void *x_prev = is_q ? P.q_prev : P.k_prev;
  const bool lin_pred = shift && w.t0 > 0;
  const bool c_on = lin_pred || (shift && x_prev);
  uint4 r_c = raw8(!c_on ? ln_w : lin_pred ? src : x_prev,
                   !c_on ? own : lin_pred ? (w.bi * T + w.t0 - 1) * P.qkv_st + w.chan : w.bi * w.width + w.chan);
  // ring counters of a graph-replayed decode step (start, length)
  const int32_t *ctl = P.ring_ctl ? P.ring_ctl : static_cast<const int32_t *>(ln_w);
  int32_t ctl_start = ctl[1], ctl_len = ctl[2];
  for (uint4 *r : {&r_w, &r_b, &r_mix, &r_c}) *r = pinned(*r);
  asm volatile("" : "+v"(ctl_start), "+v"(ctl_len));

  float wf[8], bfv[8], mix[8], carry[8];
  unpack8(r_w, wf);
  unpack8(r_b, bfv);
  if (shift) {
    unpack8(r_mix, mix);
    unpack8(r_c, carry);  // (no carried row at t0 == 0: the "first" fallback in the first pass)
  }
  const bool ring = !is_q && P.ring_k && T == 1;
  const int64_t ring_o = ring ? ring_row(P, w, ctl_start, ctl_len) : 0;
  uint16_t *x_out = static_cast<uint16_t *>(is_q ? P.q_out : P.k_out);
  uint16_t *x_last = static_cast<uint16_t *>(is_q ? P.q_last_out : P.k_last_out);
  const float eps = float(P.ln_eps);
#pragma unroll 1
  for (int ps = 0; ps < w.npass; ++ps) {
    const PassRaw cur = next;
    if (ps + 1 < w.npass) fetch(ps + 1, next);
    const int64_t t = w.t0 + ps * RPW + w.sub;
    const bool live = t < T;
    const int64_t e = (w.bi * T + (live ? t : T - 1)) * w.width + w.chan;
    float x[8], c[8], sn[8];
    unpack8(cur.a, x);
    unpack8(cur.b, c);
    unpack8(cur.c, sn);
    if (live && x_last && t == T - 1) store8(x_last + w.bi * w.width + w.chan, x);
    if (shift) {
      float pv[8];
      if (ps == 0 && w.t0 == 0 && !x_prev)  // fallback "first": token 0 is its own predecessor
        for (int i = 0; i < 8; ++i) carry[i] = __shfl(x[i], w.part);
      prev_rows<LPR>(x, carry, w.lane, pv);
      last_row<LPR>(x, w.part, carry);
      token_shift(x, pv, mix);
    }
    norm_rope<D>(x, wf, bfv, eps, c, sn);
    if (live) store8(x_out + e, x);
    if (ring && live) store8(static_cast<uint16_t *>(P.ring_k) + ring_o * D + w.part * 8, x);
  }
}

// v rows: value residual before / after the token shift, and the merge gate
// 1 + elu(key_weight), one value per (b, t, kv head).
template <int D>
__device__ __forceinline__ void v_rows(const kvm_prefix_desc &P, const PrefixTile &w) {
  constexpr int LPR = D / 8, RPW = 64 / LPR;
  const int64_t T = P.seq_len;
  const int mode = int(P.value_residual_mode);
  const bool shift = P.token_shift != 0;
  const bool pre = mode == 1 || mode == 2;
  auto fetch = [&](int ps, PassRaw &r) {
    const int64_t t = w.t0 + ps * RPW + w.sub;
    const int64_t row = w.bi * T + (t < T ? t : T - 1);
    r.a = raw8(P.v_lin, row * P.qkv_st + w.chan);
    r.b = r.c = make_uint4(0, 0, 0, 0);
    if (mode != 0) r.b = raw8(P.v_first, row * w.width + w.chan);
    if (mode >= 2) r.c = raw8(P.gate_lin, row * w.width + w.chan);
    // every lane loads the (b, t, kv head) weight; lane part 0 uses it
    r.kw = static_cast<const uint16_t *>(P.key_weight ? P.key_weight : P.v_lin)[P.key_weight ? row * P.kw_st + w.hk : 0];
  };
  PassRaw next;
  fetch(0, next);
  const void *stand = P.ln_k_w;  // a valid operand for the loads a mode does not use
  const int64_t own = w.part * 8;
  const bool use_g0 = mode >= 2, use_lamb = mode == 1;
  uint4 r_g0 = raw8(use_g0 ? P.v_gate0 : stand, use_g0 ? w.chan : own);
  uint32_t r_lamb = static_cast<const uint16_t *>(use_lamb ? P.lamb : stand)[0];
  uint4 r_mix = raw8(shift ? P.x_v : stand, shift ? w.chan : own);
  // Predecessor of the tile's first token: the row before it (with the
  // inputs of a pre-shift value residual) or the carried row.
  const bool lin_pred = shift && w.t0 > 0;
  const int64_t rp = w.bi * T + w.t0 - 1;
  const bool c_on = lin_pred || (shift && P.v_prev);
  const bool vres_on = lin_pred && pre;
  uint4 r_c = raw8(!c_on ? stand : lin_pred ? P.v_lin : P.v_prev,
                   !c_on ? own : lin_pred ? rp * P.qkv_st + w.chan : w.bi * w.width + w.chan);
  uint4 r_vf = raw8(vres_on ? P.v_first : stand, vres_on ? rp * w.width + w.chan : own);
  uint4 r_gl = raw8(vres_on && mode >= 2 ? P.gate_lin : stand, vres_on && mode >= 2 ? rp * w.width + w.chan : own);
  const int32_t *ctl = P.ring_ctl ? P.ring_ctl : static_cast<const int32_t *>(stand);
  int32_t ctl_start = ctl[1], ctl_len = ctl[2];
  for (uint4 *r : {&r_g0, &r_mix, &r_c, &r_vf, &r_gl}) *r = pinned(*r);
  asm volatile("" : "+v"(r_lamb), "+v"(ctl_start), "+v"(ctl_len));

  float g0[8], mix[8], carry[8];
  unpack8(r_g0, g0);
  const float lamb = use_lamb ? bf2f(r_lamb) : 0.f;
  if (shift) {
    unpack8(r_mix, mix);
    unpack8(r_c, carry);
    if (vres_on) {
      VRes vr;
      unpack8(r_vf, vr.vf);
      unpack8(r_gl, vr.gl);
      value_residual(mode, carry, vr, g0, lamb);
    }
  }
  const bool ring = P.ring_k && T == 1;
  const int64_t ring_o = ring ? ring_row(P, w, ctl_start, ctl_len) : 0;
#pragma unroll 1
  for (int ps = 0; ps < w.npass; ++ps) {
    const PassRaw cur = next;
    if (ps + 1 < w.npass) fetch(ps + 1, next);
    const int64_t t = w.t0 + ps * RPW + w.sub;
    const bool live = t < T;
    const int64_t e = (w.bi * T + (live ? t : T - 1)) * w.width + w.chan;
    float v[8];
    VRes vr;
    unpack8(cur.a, v);
    unpack8(cur.b, vr.vf);
    unpack8(cur.c, vr.gl);
    if (pre) value_residual(mode, v, vr, g0, lamb);
    if (live && P.v_last_out && t == T - 1)
      store8(static_cast<uint16_t *>(P.v_last_out) + w.bi * w.width + w.chan, v);
    if (shift) {
      float pv[8];
      if (ps == 0 && w.t0 == 0 && !P.v_prev)
        for (int i = 0; i < 8; ++i) carry[i] = __shfl(v[i], w.part);
      prev_rows<LPR>(v, carry, w.lane, pv);
      last_row<LPR>(v, w.part, carry);
      token_shift(v, pv, mix);
    }
    if (mode == 3) value_residual(2, v, vr, g0, lamb);
    if (live) store8(static_cast<uint16_t *>(P.v_out) + e, v);
    if (ring && live) store8(static_cast<uint16_t *>(P.ring_v) + ring_o * D + w.part * 8, v);
    uint16_t gbits = 0x3f80;  // 1.0: no key weighting
    if (live && w.part == 0 && P.key_weight && P.gate_out) {
      const int64_t ge = (w.bi * T + t) * P.kv_heads + w.hk;
      const float kw = bf2f(cur.kw);
      const float el = rbf(kw > 0.f ? kw : expm1f(kw));
      gbits = uint16_t(f2bf(1.f + el));
      static_cast<uint16_t *>(P.gate_out)[ge] = gbits;
    }
    if (ring && live && w.part == 0) static_cast<uint16_t *>(P.ring_gate)[ring_o] = gbits;
  }
}

// One wave per (batch, row kind, token tile); row kinds: the q heads, the k
// heads, then the v heads.  A wave holds only its own kind's parameters and
// rows, so the kernel keeps few enough registers for four waves per SIMD.
template <int D>
__global__ __launch_bounds__(kThreads) void k_prefix(kvm_prefix_desc P) {
  constexpr int LPR = D / 8, RPW = 64 / LPR, PASSES = kTokWave / RPW;
  const int64_t T = P.seq_len, Hq = P.q_heads, Hkv = P.kv_heads;
  const int64_t tiles = (T + kTokWave - 1) / kTokWave;
  const int64_t wv = int64_t(blockIdx.x) * (kThreads / 64) + (threadIdx.x >> 6);
  const int64_t tile = wv % tiles;
  const int64_t kind = (wv / tiles) % (Hq + 2 * Hkv);
  PrefixTile w;
  w.bi = wv / tiles / (Hq + 2 * Hkv);
  if (w.bi >= P.batch) return;  // wave-uniform
  w.lane = threadIdx.x & 63;
  w.part = w.lane % LPR;
  w.sub = w.lane / LPR;
  w.t0 = tile * kTokWave;
  w.npass = int(min(int64_t(PASSES), (T - w.t0 + RPW - 1) / RPW));  // passes with a live token
  const bool is_q = kind < Hq;
  w.hk = is_q ? 0 : (kind - Hq) % Hkv;
  w.width = is_q ? Hq * D : Hkv * D;
  w.chan = (is_q ? kind : w.hk) * D + w.part * 8;
  if (kind < Hq + Hkv)
    qk_rows<D>(P, w, is_q);
  else
    v_rows<D>(P, w);
}

}  // namespace

hipError_t launch_prefix(const kvm_prefix_desc &P, hipStream_t stream) {
  const int64_t tiles = (P.seq_len + kTokWave - 1) / kTokWave;
  const int64_t waves = P.batch * (P.q_heads + 2 * P.kv_heads) * tiles;
  const dim3 grid{unsigned((waves + kThreads / 64 - 1) / (kThreads / 64)), 1u, 1u};
  if (P.head_dim == 128)
    hipLaunchKernelGGL(k_prefix<128>, grid, dim3(kThreads), 0, stream, P);
  else
    hipLaunchKernelGGL(k_prefix<64>, grid, dim3(kThreads), 0, stream, P);
  return hipGetLastError();
}

}  // namespace kvm

// ---------------------------------------------------------------------------
// Elementwise ops of the decoder's MLP (model/rwkv7_backbone.py:163-177):
// the RWKV token shift x + mix * (shift(x) - x) (model/tokenshift.py:11-37)
// and relu(x)^2, one read and one write per element, with the reference's
// bf16 rounding points.

namespace kvm {
namespace {

// One thread per 8 channels of one token row.  prev: the row before token 0
// ([B, width]), or NULL for the fallback: zeros (zero_fallback) or token 0
// itself ("first").
__global__ __launch_bounds__(256) void k_token_shift(const uint16_t *__restrict__ x,
                                                     const uint16_t *__restrict__ prev,
                                                     const uint16_t *__restrict__ mix,
                                                     uint16_t *__restrict__ out, int64_t B, int64_t T,
                                                     int64_t width, int zero_fallback) {
  const int64_t per_row = width / 8;
  const int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= B * T * per_row) return;
  const int64_t c = (i % per_row) * 8, r = i / per_row, t = r % T, b = r / T;
  float xv[8], pv[8], mv[8];
  load8(x + r * width + c, xv);
  load8(mix + c, mv);
  if (t > 0) {
    load8(x + (r - 1) * width + c, pv);
  } else if (prev) {
    load8(prev + b * width + c, pv);
  } else {
#pragma unroll
    for (int e = 0; e < 8; ++e) pv[e] = zero_fallback ? 0.f : xv[e];
  }
#pragma unroll
  for (int e = 0; e < 8; ++e) xv[e] = rbf(xv[e] + rbf(mv[e] * rbf(pv[e] - xv[e])));
  store8(out + r * width + c, xv);
}

// relu(x)^2: the relu is exact, the square rounds once (as torch's two ops).
__global__ __launch_bounds__(256) void k_relu_square(const uint16_t *__restrict__ x, uint16_t *__restrict__ out,
                                                     int64_t n8) {
  const int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i >= n8) return;
  float v[8];
  load8(x + i * 8, v);
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float r = fmaxf(v[e], 0.f);
    v[e] = rbf(r * r);
  }
  store8(out + i * 8, v);
}

}  // namespace

hipError_t launch_token_shift(const void *x, const void *prev, const void *mix, void *out, int64_t B,
                              int64_t T, int64_t width, int zero_fallback, hipStream_t stream) {
  const int64_t n = B * T * (width / 8);
  hipLaunchKernelGGL(k_token_shift, dim3(unsigned((n + 255) / 256)), dim3(256), 0, stream,
                     static_cast<const uint16_t *>(x), static_cast<const uint16_t *>(prev),
                     static_cast<const uint16_t *>(mix), static_cast<uint16_t *>(out), B, T, width, zero_fallback);
  return hipGetLastError();
}

hipError_t launch_relu_square(const void *x, void *out, int64_t n, hipStream_t stream) {
  const int64_t n8 = n / 8;
  hipLaunchKernelGGL(k_relu_square, dim3(unsigned((n8 + 255) / 256)), dim3(256), 0, stream,
                     static_cast<const uint16_t *>(x), static_cast<uint16_t *>(out), n8);
  return hipGetLastError();
}

}  // namespace kvm
