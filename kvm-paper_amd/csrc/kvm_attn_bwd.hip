// Backward of the fused KVM prefill attention on gfx950, with the memory
// snapshots held fixed.
//
// Forward (kvm_attn.hip): query t of chunk m attends to the S_m rows of
// snapshot m - n (keys k_attn * tau_state) and to the window tokens
// [wb(m), t] (keys k * tau_front), wb(m) = max(0, (m - n + 1) C), with
// s = (q . k) tau / sqrt(D), p = softmax(s), out = sum p v.  Given lse (the
// log2-domain log-sum-exp the forward stores) and delta = dout . out, the
// gradients are, with dS = p (dout . v - delta) (the gradient of s):
//   dq   = sum_k dS k tau / sqrt(D)
//   dk   = sum_q dS q tau / sqrt(D),   dv = sum_q p dout
//   dtau = sum_{q,k} dS (q . k) / sqrt(D)   (per head, per key segment)
// Reference: the Triton training kernels
// model/kernels/kvm_triton_training_kernels.py:1950-2090 (dq),
// :668-830 (window dk/dv) and :2093-2305 (snapshot rows).
//
// Two kernels, each owning what it writes (no atomics, deterministic):
//   k_attn_bwd_dq    one 64-query tile of one (batch, q head): loops over
//                    its memory rows and window keys; writes dq and a
//                    per-workgroup temperature partial;
//   k_attn_bwd_dkdv  one 64-key block of one (batch, kv head), either rows of
//                    one snapshot or window tokens: loops over every query
//                    of every head of its GQA group that sees them; writes
//                    dk and dv.
// MFMA (v_mfma_f32_16x16x32_bf16) operands are arranged so that the
// reduction axis is contiguous: S = Q K^T and dP = dO V^T read K / V / Q /
// dO rows straight from row-major LDS tiles; the products over keys (dq) or
// over queries (dk, dv) take their bf16 P / dS operand from a per-wave LDS
// transpose tile and the second operand as 8 column reads.

#include "kvm_device.hpp"
#include "kvm_internal.hpp"

namespace kvm {
namespace {

constexpr int BQ = 64;   // queries per dq workgroup / query block of dkdv
constexpr int BK = 64;   // keys per key block
constexpr int NWB = 4;   // waves per workgroup
constexpr float kLog2e = 1.4426950408889634f;

__device__ __forceinline__ uint4 ld16_or_zero(const uint16_t *p, bool ok) {
  return ok ? *reinterpret_cast<const uint4 *>(p) : make_uint4(0, 0, 0, 0);
}

// Row-major tile [rows x D] bf16 in LDS from global rows r0.. (row stride
// `st` elements), rows >= nvalid zero-filled.
template <int D, int ROWS>
__device__ __forceinline__ void stage_rows(uint16_t *lds, const uint16_t *g, int64_t st, int nvalid) {
  constexpr int PER_ROW = D / 8;
  for (int i = threadIdx.x; i < ROWS * PER_ROW; i += NWB * 64) {
    const int r = i / PER_ROW, c = i % PER_ROW;
    *reinterpret_cast<uint4 *>(lds + r * D + c * 8) = ld16_or_zero(g + int64_t(r) * st + c * 8, r < nvalid);
  }
}

// B operand (K x N = 32 x 16) whose K rows are 8 consecutive rows of a
// row-major LDS tile `t` ([.. x D]) and whose N column is feature `col`:
// lane l supplies rows k0 + 8 (l / 16) .. + 7 of column col.
template <int D>
__device__ __forceinline__ bf16x8 col_frag(const uint16_t *t, int k0, int col) {
  const int lane = threadIdx.x & 63;
  const int r = k0 + 8 * (lane >> 4);
  uint16_t v[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) v[j] = t[(r + j) * D + col];
  return as_bf16x8(make_uint4(v[0] | (uint32_t(v[1]) << 16), v[2] | (uint32_t(v[3]) << 16),
                              v[4] | (uint32_t(v[5]) << 16), v[6] | (uint32_t(v[7]) << 16)));
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o);
  return v;
}

struct BwdKeySeg {
  const uint16_t *k, *v;  // row 0 of the segment
  int64_t kst, vst;       // row strides (elements)
  int nkeys;
  int64_t pos0;           // sequence position of row 0 (window); unused for memory rows
  bool causal;
  float tau;
};

// ---------------------------------------------------------------------------
// dq: workgroup = 64 queries of one (batch, q head) in chunk m.
template <int D>
__global__ __launch_bounds__(NWB * 64) void k_attn_bwd_dq(kvm_layer L, BwdArgs A, int qtiles,
                                                          ChunkTable table, float *tpart) {
  constexpr int KS = D / 32, DT = D / 16;
  __shared__ __attribute__((aligned(16))) uint16_t kt[BK * D];
  __shared__ __attribute__((aligned(16))) uint16_t vt[BK * D];
  __shared__ __attribute__((aligned(16))) uint16_t dst[NWB][16 * BK];
  __shared__ float red[NWB][2];
  const int C = int(L.chunk_len), n = int(L.n_bswa_chunks);
  const int Hq = int(L.q_heads), Hkv = int(L.kv_heads);
  const int wg = blockIdx.x;
  const int qt = wg % qtiles, m = (wg / qtiles) % int(A.n_chunks), qrow = wg / (qtiles * int(A.n_chunks));
  const int b = qrow / Hq, hq = qrow % Hq, hk = hq / (Hq / Hkv), kvrow = b * Hkv + hk;
  const int64_t T = A.T;
  const int64_t q0 = int64_t(m) * C + int64_t(qt) * BQ;
  const int64_t q_hi = min(int64_t(m + 1) * C, T);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, g = lane >> 4;
  const float scale_nat = 1.0f / sqrtf(float(D));
  float tacc[2] = {0.f, 0.f};
  if (q0 < q_hi) {
    // A operands: Q and dO rows of this wave's 16 queries.
    const int64_t tr = q0 + wave * 16 + (lane & 15);
    const bool rok = tr < q_hi;
    const uint16_t *qp = static_cast<const uint16_t *>(A.q) + b * A.q_sb + hq * A.q_sh + tr * A.q_st;
    const uint16_t *dop = static_cast<const uint16_t *>(A.dout) + b * A.do_sb + hq * A.do_sh + tr * A.do_st;
    bf16x8 qa[KS], da[KS];
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      qa[ks] = as_bf16x8(ld16_or_zero(qp + ks * 32 + g * 8, rok));
      da[ks] = as_bf16x8(ld16_or_zero(dop + ks * 32 + g * 8, rok));
    }
    // The lane's C-layout rows: queries q0 + 16 wave + 4 g + i.
    float lse[4], dl[4];
    int64_t tq[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      tq[i] = q0 + wave * 16 + 4 * g + i;
      const bool ok = tq[i] < q_hi;
      const int64_t o = (int64_t(b) * Hq + hq) * T + (ok ? tq[i] : 0);
      lse[i] = ok ? A.lse[o] : INFINITY;
      dl[i] = ok ? A.delta[o] : 0.f;
    }
    f32x4 dq[DT];
#pragma unroll
    for (int t = 0; t < DT; ++t) dq[t] = f32x4{0.f, 0.f, 0.f, 0.f};

    const float tau_s = static_cast<const float *>(L.state_temp)[hq];
    const float tau_f = static_cast<const float *>(L.front_temp)[hq];
    const int64_t wb = max(int64_t(0), int64_t(m - n + 1) * C);
    BwdKeySeg segs[2];
    const int S = m >= n ? table.state_len[m] : 0;
    const int64_t soff = int64_t(table.snap_slot[m]) * A.snap_stride + int64_t(kvrow) * A.snap_cap * D;
    segs[0] = {A.snap_k + soff, A.snap_v + soff, D, D, S, 0, false, tau_s};
    const uint16_t *kw = static_cast<const uint16_t *>(A.kv.k) + b * A.kv.k_sb + hk * A.kv.k_sh;
    const uint16_t *vw = static_cast<const uint16_t *>(A.kv.v) + b * A.kv.v_sb + hk * A.kv.v_sh;
    segs[1] = {kw + wb * A.kv.k_st, vw + wb * A.kv.v_st, A.kv.k_st, A.kv.v_st, int(q_hi - wb), wb, true, tau_f};
#pragma unroll 1
    for (int sg = 0; sg < 2; ++sg) {
      const BwdKeySeg &sgm = segs[sg];
      const float sc = kLog2e * scale_nat * sgm.tau;
      const float dsc = scale_nat * sgm.tau;
      // Causal window: keys past the tile's last query are never visible.
      const int nk = sgm.causal ? int(min(int64_t(sgm.nkeys), q0 + BQ - sgm.pos0)) : sgm.nkeys;
#pragma unroll 1
      for (int j0 = 0; j0 < nk; j0 += BK) {
        const int nv = min(BK, nk - j0);
        __syncthreads();
        stage_rows<D, BK>(kt, sgm.k + int64_t(j0) * sgm.kst, sgm.kst, nv);
        stage_rows<D, BK>(vt, sgm.v + int64_t(j0) * sgm.vst, sgm.vst, nv);
        __syncthreads();
#pragma unroll
        for (int nt = 0; nt < BK / 16; ++nt) {
          f32x4 s = {0.f, 0.f, 0.f, 0.f}, dp = {0.f, 0.f, 0.f, 0.f};
          const int key = nt * 16 + (lane & 15);
#pragma unroll
          for (int ks = 0; ks < KS; ++ks) {
            const bf16x8 kb = as_bf16x8(*reinterpret_cast<const uint4 *>(kt + key * D + ks * 32 + g * 8));
            const bf16x8 vb = as_bf16x8(*reinterpret_cast<const uint4 *>(vt + key * D + ks * 32 + g * 8));
            s = __builtin_amdgcn_mfma_f32_16x16x32_bf16(qa[ks], kb, s, 0, 0, 0);
            dp = __builtin_amdgcn_mfma_f32_16x16x32_bf16(da[ks], vb, dp, 0, 0, 0);
          }
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int kj = j0 + key;
            const bool vis = kj < nk && (!sgm.causal || sgm.pos0 + kj <= tq[i]);
            const float p = vis ? exp2f(s[i] * sc - lse[i]) : 0.f;
            const float ds = p * (dp[i] - dl[i]);
            tacc[sg] += ds * s[i];
            dst[wave][(4 * g + i) * BK + key] = uint16_t(f2bf(ds * dsc));
          }
        }
        __syncthreads();
        // dq += dS K over the block's 64 keys (two 32-key steps).
#pragma unroll
        for (int kk = 0; kk < BK / 32; ++kk) {
          const bf16x8 a = as_bf16x8(*reinterpret_cast<const uint4 *>(
              &dst[wave][(lane & 15) * BK + kk * 32 + g * 8]));
#pragma unroll
          for (int t = 0; t < DT; ++t)
            dq[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, col_frag<D>(kt, kk * 32, t * 16 + (lane & 15)),
                                                            dq[t], 0, 0, 0);
        }
      }
    }
    uint16_t *dqp = static_cast<uint16_t *>(A.dq) + b * A.dq_sb + hq * A.dq_sh;
#pragma unroll
    for (int i = 0; i < 4; ++i)
      if (tq[i] < q_hi)
#pragma unroll
        for (int t = 0; t < DT; ++t) dqp[tq[i] * A.dq_st + t * 16 + (lane & 15)] = uint16_t(f2bf(dq[t][i]));
  }
  // Temperature partials of this workgroup: sum of dS (q . k) / sqrt(D).
  const float t0 = wave_sum(tacc[0]) * scale_nat, t1 = wave_sum(tacc[1]) * scale_nat;
  if (lane == 0) {
    red[wave][0] = t0;
    red[wave][1] = t1;
  }
  __syncthreads();
  if (threadIdx.x < 2) {
    float a = 0.f;
    for (int w = 0; w < NWB; ++w) a += red[w][threadIdx.x];
    tpart[int64_t(wg) * 2 + threadIdx.x] = a;
  }
}

// Per-head temperature gradients: partials summed in a fixed order
// (batch, chunk, tile).
__global__ void k_attn_bwd_temps(const float *tpart, int B, int Hq, int n_chunks, int qtiles,
                                 float *d_state, float *d_front) {
  const int hq = blockIdx.x * blockDim.x + threadIdx.x;
  if (hq >= Hq) return;
  float a = 0.f, f = 0.f;
  for (int b = 0; b < B; ++b)
    for (int w = 0; w < n_chunks * qtiles; ++w) {
      const int64_t wg = int64_t(b * Hq + hq) * n_chunks * qtiles + w;
      a += tpart[wg * 2];
      f += tpart[wg * 2 + 1];
    }
  d_state[hq] = a;
  d_front[hq] = f;
}

// ---------------------------------------------------------------------------
// dk / dv: workgroup = 64 keys of one (batch, kv head).
//   snapshot mode: rows [kb*64, +64) of the snapshot chunk m = n + blockIdx.x / kblocks
//                  reads (all its queries, no causal mask, state temperature);
//   window mode:   tokens [kb*64, +64): query t sees token p iff
//                  wb(chunk(t)) <= p <= t (front temperature).
template <int D, bool SNAP>
__global__ __launch_bounds__(NWB * 64) void k_attn_bwd_dkdv(kvm_layer L, BwdArgs A, int kblocks,
                                                            ChunkTable table) {
  constexpr int KS = D / 32, DT = D / 16;
  __shared__ __attribute__((aligned(16))) uint16_t qt[BQ * D];
  __shared__ __attribute__((aligned(16))) uint16_t dot[BQ * D];
  __shared__ __attribute__((aligned(16))) uint16_t pt[NWB][16 * BQ];
  __shared__ __attribute__((aligned(16))) uint16_t dt[NWB][16 * BQ];
  __shared__ float lse_s[BQ], dl_s[BQ];
  const int C = int(L.chunk_len), n = int(L.n_bswa_chunks);
  const int Hq = int(L.q_heads), Hkv = int(L.kv_heads), grp = Hq / Hkv;
  const int kvrow = blockIdx.y, b = kvrow / Hkv, hk = kvrow % Hkv;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, g = lane >> 4;
  const int64_t T = A.T;
  const float scale_nat = 1.0f / sqrtf(float(D));

  int m_snap = 0, nkeys;
  int64_t kb0;
  const uint16_t *kbase, *vbase;
  int64_t kst, vst;
  if (SNAP) {
    m_snap = n + int(blockIdx.x) / kblocks;
    kb0 = int64_t(blockIdx.x % kblocks) * BK;
    if (m_snap >= int(A.n_chunks)) return;
    nkeys = table.state_len[m_snap];
    const int64_t soff = int64_t(table.snap_slot[m_snap]) * A.snap_stride + int64_t(kvrow) * A.snap_cap * D;
    kbase = A.snap_k + soff;
    vbase = A.snap_v + soff;
    kst = vst = D;
  } else {
    kb0 = int64_t(blockIdx.x) * BK;
    nkeys = int(T);
    kbase = static_cast<const uint16_t *>(A.kv.k) + b * A.kv.k_sb + hk * A.kv.k_sh;
    vbase = static_cast<const uint16_t *>(A.kv.v) + b * A.kv.v_sb + hk * A.kv.v_sh;
    kst = A.kv.k_st;
    vst = A.kv.v_st;
  }
  if (kb0 >= nkeys) return;
  // A operands: this wave's 16 keys (K for S^T = K Q^T, V for dP^T = V dO^T).
  const int64_t kr = kb0 + wave * 16 + (lane & 15);
  const bool kok = kr < nkeys;
  bf16x8 ka[KS], va[KS];
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) {
    ka[ks] = as_bf16x8(ld16_or_zero(kbase + kr * kst + ks * 32 + g * 8, kok));
    va[ks] = as_bf16x8(ld16_or_zero(vbase + kr * vst + ks * 32 + g * 8, kok));
  }
  int64_t kp[4];  // the lane's C-layout keys: kb0 + 16 wave + 4 g + i
#pragma unroll
  for (int i = 0; i < 4; ++i) kp[i] = kb0 + wave * 16 + 4 * g + i;
  f32x4 dk[DT], dv[DT];
#pragma unroll
  for (int t = 0; t < DT; ++t) {
    dk[t] = f32x4{0.f, 0.f, 0.f, 0.f};
    dv[t] = f32x4{0.f, 0.f, 0.f, 0.f};
  }
  // Query range that sees the block.
  int64_t tq_lo, tq_hi;
  if (SNAP) {
    tq_lo = int64_t(m_snap) * C;
    tq_hi = min(int64_t(m_snap + 1) * C, T);
  } else {
    tq_lo = kb0 / BQ * BQ;
    const int64_t last_key = min(kb0 + BK, T) - 1;
    tq_hi = min(T, (last_key / C + n) * int64_t(C));
  }
#pragma unroll 1
  for (int h = 0; h < grp; ++h) {
    const int hq = hk * grp + h;
    const float tau = static_cast<const float *>(SNAP ? L.state_temp : L.front_temp)[hq];
    const float sc = kLog2e * scale_nat * tau, dsc = scale_nat * tau;
    const uint16_t *qrow = static_cast<const uint16_t *>(A.q) + b * A.q_sb + hq * A.q_sh;
    const uint16_t *dorow = static_cast<const uint16_t *>(A.dout) + b * A.do_sb + hq * A.do_sh;
    const float *lse_row = A.lse + (int64_t(b) * Hq + hq) * T;
    const float *dl_row = A.delta + (int64_t(b) * Hq + hq) * T;
#pragma unroll 1
    for (int64_t t0 = tq_lo; t0 < tq_hi; t0 += BQ) {
      const int nq = int(min(int64_t(BQ), tq_hi - t0));
      __syncthreads();
      stage_rows<D, BQ>(qt, qrow + t0 * A.q_st, A.q_st, nq);
      stage_rows<D, BQ>(dot, dorow + t0 * A.do_st, A.do_st, nq);
      if (threadIdx.x < BQ) {
        const bool ok = threadIdx.x < nq;
        lse_s[threadIdx.x] = ok ? lse_row[t0 + threadIdx.x] : INFINITY;
        dl_s[threadIdx.x] = ok ? dl_row[t0 + threadIdx.x] : 0.f;
      }
      __syncthreads();
#pragma unroll
      for (int nt = 0; nt < BQ / 16; ++nt) {
        f32x4 s = {0.f, 0.f, 0.f, 0.f}, dp = {0.f, 0.f, 0.f, 0.f};
        const int qi = nt * 16 + (lane & 15);
#pragma unroll
        for (int ks = 0; ks < KS; ++ks) {
          const bf16x8 qb = as_bf16x8(*reinterpret_cast<const uint4 *>(qt + qi * D + ks * 32 + g * 8));
          const bf16x8 db = as_bf16x8(*reinterpret_cast<const uint4 *>(dot + qi * D + ks * 32 + g * 8));
          s = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ka[ks], qb, s, 0, 0, 0);
          dp = __builtin_amdgcn_mfma_f32_16x16x32_bf16(va[ks], db, dp, 0, 0, 0);
        }
        const int64_t t = t0 + qi;
        const int64_t wbt = max(int64_t(0), (t / C - n + 1) * int64_t(C));
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          bool vis = t < tq_hi && kp[i] < nkeys;
          if (!SNAP) vis = vis && kp[i] <= t && wbt <= kp[i];
          const float p = vis ? exp2f(s[i] * sc - lse_s[qi]) : 0.f;
          const float ds = p * (dp[i] - dl_s[qi]);
          pt[wave][(4 * g + i) * BQ + qi] = uint16_t(f2bf(p));
          dt[wave][(4 * g + i) * BQ + qi] = uint16_t(f2bf(ds * dsc));
        }
      }
      __syncthreads();
      // dv += P^T dO, dk += dS^T Q over the block's 64 queries.
#pragma unroll
      for (int kk = 0; kk < BQ / 32; ++kk) {
        const bf16x8 pa = as_bf16x8(*reinterpret_cast<const uint4 *>(&pt[wave][(lane & 15) * BQ + kk * 32 + g * 8]));
        const bf16x8 sa = as_bf16x8(*reinterpret_cast<const uint4 *>(&dt[wave][(lane & 15) * BQ + kk * 32 + g * 8]));
#pragma unroll
        for (int t = 0; t < DT; ++t) {
          const int col = t * 16 + (lane & 15);
          dv[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(pa, col_frag<D>(dot, kk * 32, col), dv[t], 0, 0, 0);
          dk[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(sa, col_frag<D>(qt, kk * 32, col), dk[t], 0, 0, 0);
        }
      }
    }
  }
  // Owner writes (fp32).
  float *dkp, *dvp;
  int64_t rowst = D;
  if (SNAP) {
    const int64_t off = int64_t(table.snap_slot[m_snap]) * A.dsnap_stride + int64_t(kvrow) * A.snap_cap * D;
    dkp = A.d_snap_k + off;
    dvp = A.d_snap_v + off;
  } else {
    const int64_t off = int64_t(kvrow) * T * D;
    dkp = A.dk + off;
    dvp = A.dv + off;
  }
#pragma unroll
  for (int i = 0; i < 4; ++i)
    if (kp[i] < nkeys)
#pragma unroll
      for (int t = 0; t < DT; ++t) {
        dkp[kp[i] * rowst + t * 16 + (lane & 15)] = dk[t][i];
        dvp[kp[i] * rowst + t * 16 + (lane & 15)] = dv[t][i];
      }
}

template <int D>
hipError_t launch_bwd_d(const kvm_layer &L, const BwdArgs &a, const ChunkTable &table, float *tpart,
                        hipStream_t stream) {
  const int n_chunks = int(a.n_chunks);
  const int qtiles = int((L.chunk_len + BQ - 1) / BQ);
  const int64_t rows = L.batch * L.kv_heads;
  hipLaunchKernelGGL((k_attn_bwd_dq<D>), dim3(unsigned(L.batch * L.q_heads * n_chunks * qtiles)),
                     dim3(NWB * 64), 0, stream, L, a, qtiles, table, tpart);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(k_attn_bwd_temps, dim3(unsigned((L.q_heads + 63) / 64)), dim3(64), 0, stream, tpart,
                     int(L.batch), int(L.q_heads), n_chunks, qtiles, a.d_state_temp, a.d_front_temp);
  if ((e = hipGetLastError()) != hipSuccess) return e;
  const int wblocks = int((a.T + BK - 1) / BK);
  hipLaunchKernelGGL((k_attn_bwd_dkdv<D, false>), dim3(unsigned(wblocks), unsigned(rows)), dim3(NWB * 64), 0,
                     stream, L, a, 0, table);
  if ((e = hipGetLastError()) != hipSuccess) return e;
  const int n = int(L.n_bswa_chunks);
  if (n_chunks > n) {
    const int kblocks = int((a.snap_cap + BK - 1) / BK);
    hipLaunchKernelGGL((k_attn_bwd_dkdv<D, true>), dim3(unsigned((n_chunks - n) * kblocks), unsigned(rows)),
                       dim3(NWB * 64), 0, stream, L, a, kblocks, table);
    e = hipGetLastError();
  }
  return e;
}

}  // namespace

int64_t attn_bwd_workspace_bytes(const kvm_layer &L, int64_t n_chunks) {
  const int64_t qtiles = (L.chunk_len + BQ - 1) / BQ;
  return L.batch * L.q_heads * n_chunks * qtiles * 2 * 4;
}

hipError_t launch_attn_backward(const kvm_layer &L, const BwdArgs &a, const ChunkTable &table,
                                float *tpart, hipStream_t stream) {
  if (L.head_dim == 128) return launch_bwd_d<128>(L, a, table, tpart, stream);
  return launch_bwd_d<64>(L, a, table, tpart, stream);
}

}  // namespace kvm
