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
//   k_attn_bwd_dq    128 queries (4 waves x 32) of one (batch, q head) in
//                    chunk m: streams the chunk's memory rows and window keys
//                    as 64-row K / V blocks; writes dq and a per-workgroup
//                    temperature partial;
//   k_attn_bwd_dkdv  64 keys (4 waves x 16) of one (batch, kv head), either
//                    rows of one snapshot or window tokens: streams every
//                    query of every head of its GQA group that sees them as
//                    64-row Q / dO blocks; writes dk and dv.
// Both stream their blocks the way the forward does (kvm_attn_tile.hpp):
// LDS-DMA into a swizzled double-buffered image, row fragments with
// ds_read_b128, transposed fragments with ds_read_b64_tr_b16.  The score-like
// products put the streamed rows in the A operand, so their C layout (4
// consecutive rows per lane) is already the B operand of the next product:
//   dq kernel:   S^T = K Q^T, dP^T = V dO^T, dq^T += K^T dS^T;
//   dkdv kernel: S = Q K^T, dP = dO V^T, dv^T += dO^T P, dk^T += Q^T dS;
// P and dS never leave registers.  Each 64-row block is consumed as two
// 32-row halves (fewer live score registers).

#include "kvm_attn_tile.hpp"
#include "kvm_device.hpp"
#include "kvm_internal.hpp"

namespace kvm {
namespace {

using namespace tile;

constexpr int NWB = 4;            // waves per workgroup
constexpr int NTB = NWB * 64;     // threads per workgroup
constexpr int BQ = NWB * 32;      // queries per dq workgroup (32 per wave)
constexpr int BKW = NWB * 16;     // keys per dk/dv workgroup (16 per wave)

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o);
  return v;
}

// XCD-contiguous renumbering of a 1-D grid (dispatch is round-robin over the
// 8 XCDs): each XCD runs a contiguous range of logical tiles, so tiles that
// share streamed rows share that XCD's L2.
__device__ __forceinline__ int xcd_logical(int bid, int N) {
  const int x = bid % kXcds, jx = bid / kXcds;
  const int q8 = N / kXcds, r8 = N % kXcds;
  return x * q8 + min(x, r8) + jx;
}

// ---------------------------------------------------------------------------
// dq.  Logical tile order (b, hq, chunk, query tile); the temperature partial
// of tile w goes to tpart[2 w + segment].
template <int D>
__global__ __launch_bounds__(NTB) __attribute__((amdgpu_waves_per_eu(2)))
void k_attn_bwd_dq(kvm_layer L, BwdArgs A, int qtiles, ChunkTable table, float *tpart) {
  constexpr int KS = D / 32, DT = D / 16;
  constexpr int BUF = Lay<D>::BUF, BLK = Lay<D>::BLK;
  __shared__ __attribute__((aligned(1024))) unsigned char lds[2 * BUF];
  __shared__ float red[NWB][2];
  const int C = int(L.chunk_len), n = int(L.n_bswa_chunks);
  const int Hq = int(L.q_heads), Hkv = int(L.kv_heads);
  const int n_chunks = int(A.n_chunks);
  const int wg = xcd_logical(blockIdx.x, gridDim.x);
  const int qt = wg % qtiles, m = (wg / qtiles) % n_chunks, qrow = wg / (qtiles * n_chunks);
  const int b = qrow / Hq, hq = qrow % Hq, hk = hq / (Hq / Hkv), kvrow = b * Hkv + hk;
  const int64_t T = A.T;
  const int64_t q0 = int64_t(m) * C + int64_t(qt) * BQ;
  const int64_t q_hi = min(int64_t(m + 1) * C, T);
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(int(threadIdx.x >> 6));
  const int64_t qpos0 = q0 + wave * 32;
  const float scale_nat = 1.0f / sqrtf(float(D));
  float t_state = 0.f, t_front = 0.f;  // temperature partials of the two key segments

  // Zero both buffers once: rows past a short block are then zeros or
  // earlier rows, never uninitialised bytes.
  for (int i = threadIdx.x; i < 2 * BUF / 16; i += NTB)
    reinterpret_cast<uint4 *>(lds)[i] = make_uint4(0, 0, 0, 0);

  if (q0 < q_hi) {  // workgroup-uniform
    // B operands: Q and dO rows rt*16 + lane%16, dims ks*32 + 8*(lane/16).
    bf16x8 qf[2][KS], dof[2][KS];
    float lse[2], dl[2];
    const uint16_t *qb = static_cast<const uint16_t *>(A.q) + b * A.q_sb + hq * A.q_sh;
    const uint16_t *db = static_cast<const uint16_t *>(A.dout) + b * A.do_sb + hq * A.do_sh;
#pragma unroll
    for (int rt = 0; rt < 2; ++rt) {
      const int64_t t = qpos0 + rt * 16 + (lane & 15);
      const bool ok = t < q_hi;
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        uint4 u = make_uint4(0, 0, 0, 0), w = make_uint4(0, 0, 0, 0);
        if (ok) {
          u = *reinterpret_cast<const uint4 *>(qb + t * A.q_st + ks * 32 + (lane >> 4) * 8);
          w = *reinterpret_cast<const uint4 *>(db + t * A.do_st + ks * 32 + (lane >> 4) * 8);
        }
        qf[rt][ks] = as_bf16x8(u);
        dof[rt][ks] = as_bf16x8(w);
      }
      const int64_t o = (int64_t(b) * Hq + hq) * T + (ok ? t : 0);
      lse[rt] = ok ? A.lse[o] : INFINITY;  // p = 0 for rows past the chunk
      dl[rt] = ok ? A.delta[o] : 0.f;
    }
    // Complete these loads and hide them from the compiler's wait tracking:
    // inside the block loop the only vector-memory operations are the DMAs.
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
#pragma unroll
    for (int rt = 0; rt < 2; ++rt) {
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        asm volatile("" : "+v"(qf[rt][ks]));
        asm volatile("" : "+v"(dof[rt][ks]));
      }
      asm volatile("" : "+v"(lse[rt]));
      asm volatile("" : "+v"(dl[rt]));
    }
    f32x4 dq[2][DT];
#pragma unroll
    for (int rt = 0; rt < 2; ++rt)
#pragma unroll
      for (int t = 0; t < DT; ++t) dq[rt][t] = f32x4{0.f, 0.f, 0.f, 0.f};

    const Lanes lo = lane_offsets(lane);
    const uint32_t lds_base = uint32_t(uintptr_t((lds_void *)lds));
    const float tau_s = static_cast<const float *>(L.state_temp)[hq];
    const float tau_f = static_cast<const float *>(L.front_temp)[hq];
    const int S = m >= n ? table.state_len[m] : 0;
    const int64_t wb = max(int64_t(0), int64_t(m - n + 1) * C);
    const int64_t soff = int64_t(table.snap_slot[m]) * A.snap_stride + int64_t(kvrow) * A.snap_cap * D;
    const uint16_t *kwin = static_cast<const uint16_t *>(A.kv.k) + b * A.kv.k_sb + hk * A.kv.k_sh;
    const uint16_t *vwin = static_cast<const uint16_t *>(A.kv.v) + b * A.kv.v_sb + hk * A.kv.v_sh;
#pragma unroll 1
    for (int seg = 0; seg < 2; ++seg) {
      const bool st = seg == 0;
      // Causal window: keys past the tile's last query are never visible.
      const int nkeys = st ? S : int(min(q_hi, q0 + BQ) - wb);
      if (nkeys <= 0) continue;
      const uint16_t *kp = st ? A.snap_k + soff : kwin + wb * A.kv.k_st;
      const uint16_t *vp = st ? A.snap_v + soff : vwin + wb * A.kv.v_st;
      const int64_t kstride = st ? D : A.kv.k_st, vstride = st ? D : A.kv.v_st;
      const uint32_t kstride_b = uint32_t(kstride * 2), vstride_b = uint32_t(vstride * 2);
      const uint32_t ko = lo.drow * kstride_b + lo.dcol, vo = lo.drow * vstride_b + lo.dcol;
      const float tau = st ? tau_s : tau_f;
      const float sc = kLog2e * scale_nat * tau, dsc = scale_nat * tau;
      const bool causal = !st;
      const int nb = (nkeys + BN - 1) / BN;
      float tacc = 0.f;
      auto issue = [&](int jj) {
        const int jn = jj * BN;
        const int nv = min(BN, nkeys - jn);
        unsigned char *img = lds + (jj & 1) * BUF;
        if (nv < BN) {  // both halves meet zero weights there
          zero_v_tail<D, NTB>(img, nv);
          zero_v_tail<D, NTB>(img + BLK, nv);
        }
        issue_block<D, NWB>(lds_base + uint32_t((jj & 1) * BUF), key_rsrc(kp + int64_t(jn) * kstride, kstride, nv),
                            key_rsrc(vp + int64_t(jn) * vstride, vstride, nv), ko, vo, kstride_b, vstride_b,
                            wave);
      };
      __syncthreads();  // both buffers are free (and zeroed, the first time)
      issue(0);
#pragma unroll 1
      for (int j = 0; j < nb; ++j) {
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
        if (j + 1 < nb) issue(j + 1);
        // qrel: the wave's first query minus the block's first key (clamped).
        const int qrel = causal ? int(min(max(qpos0 - (wb + int64_t(j) * BN), int64_t(-64)), int64_t(BN))) : BN;
        const int nvalid = min(BN, nkeys - j * BN);
        const bool masked = nvalid < BN || qrel < BN - 1;
        const unsigned char *kimg = lds + (j & 1) * BUF, *vimg = kimg + BLK;
#pragma unroll
        for (int hb = 0; hb < 2; ++hb) {
          if (nvalid <= 32 * hb || qrel + 31 < 32 * hb) continue;  // wave-uniform: nothing visible
          // One 16-key tile at a time: S^T and dP^T, then its dS^T pairs.
          uint32_t pk[2][2][2];  // [rt][k2][pair]
#pragma unroll
          for (int k2 = 0; k2 < 2; ++k2) {
            const int kt = 2 * hb + k2;
            f32x4 s[2], dp[2];
#pragma unroll
            for (int rt = 0; rt < 2; ++rt) {
              s[rt] = f32x4{0.f, 0.f, 0.f, 0.f};
              dp[rt] = f32x4{0.f, 0.f, 0.f, 0.f};
            }
#pragma unroll
            for (int ks = 0; ks < KS; ++ks) {
              const bf16x8 kf = row_frag(kimg, lo, kt, ks), vf = row_frag(vimg, lo, kt, ks);
#pragma unroll
              for (int rt = 0; rt < 2; ++rt) {
                s[rt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kf, qf[rt][ks], s[rt], 0, 0, 0);
                dp[rt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vf, dof[rt][ks], dp[rt], 0, 0, 0);
              }
            }
#pragma unroll
            for (int rt = 0; rt < 2; ++rt) {
              const int lim = qrel + rt * 16 + (lane & 15);
              float d[4];
#pragma unroll
              for (int i = 0; i < 4; ++i) {
                const int key = kt * 16 + (lane >> 4) * 4 + i;
                const bool vis = !masked || (key < nvalid && (!causal || key <= lim));
                const float p = vis ? __builtin_amdgcn_exp2f(__builtin_fmaf(s[rt][i], sc, -lse[rt])) : 0.f;
                const float ds = p * (dp[rt][i] - dl[rt]);
                tacc += ds * s[rt][i];
                d[i] = ds * dsc;
              }
              pk[rt][k2][0] = pack_bf16x2(d[0], d[1]);
              pk[rt][k2][1] = pack_bf16x2(d[2], d[3]);
            }
          }
          // dS^T (scaled by tau / sqrt(D)) in the B-operand layout of step hb.
          bf16x8 dsb[2];
#pragma unroll
          for (int rt = 0; rt < 2; ++rt)
            dsb[rt] = as_bf16x8(make_uint4(pk[rt][0][0], pk[rt][0][1], pk[rt][1][0], pk[rt][1][1]));
          // dq^T += K^T dS^T over the 32 keys of step hb.
#pragma unroll
          for (int dt = 0; dt < DT; ++dt) {
            const bf16x8 kt_f = tr_frag(kimg, lo, hb, dt);
#pragma unroll
            for (int rt = 0; rt < 2; ++rt)
              dq[rt][dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kt_f, dsb[rt], dq[rt][dt], 0, 0, 0);
          }
        }
      }
      if (st)
        t_state = tacc;
      else
        t_front = tacc;
    }
    // dq rows: lane holds dims dt*16 + 4*(lane/16) + i of query rt*16 + lane%16.
    uint16_t *dqp = static_cast<uint16_t *>(A.dq) + b * A.dq_sb + hq * A.dq_sh;
#pragma unroll
    for (int rt = 0; rt < 2; ++rt) {
      const int64_t t = qpos0 + rt * 16 + (lane & 15);
      if (t < q_hi) {
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) {
          uint2 w;
          w.x = pack_bf16x2(dq[rt][dt][0], dq[rt][dt][1]);
          w.y = pack_bf16x2(dq[rt][dt][2], dq[rt][dt][3]);
          *reinterpret_cast<uint2 *>(dqp + t * A.dq_st + dt * 16 + (lane >> 4) * 4) = w;
        }
      }
    }
  }
  // Temperature partials of this workgroup: sum of dS (q . k) / sqrt(D).
  const float t0 = wave_sum(t_state) * scale_nat, t1 = wave_sum(t_front) * scale_nat;
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

// delta[b, hq, t] = sum over features of dout * out (fp32 sum of the bf16
// products), the row term of dS = p (dP - delta).  D/8 lanes per row, each
// with 8 features (16-byte loads of both bf16 rows).
template <int D>
__global__ __launch_bounds__(256) void k_attn_bwd_delta(const uint16_t *dout, int64_t do_sb, int64_t do_st,
                                                        int64_t do_sh, const uint16_t *out, int64_t o_sb,
                                                        int64_t o_st, int64_t o_sh, int Hq, int64_t T,
                                                        int64_t n_rows, float *delta) {
  constexpr int GL = D / 8;
  const int64_t r = int64_t(blockIdx.x) * (256 / GL) + threadIdx.x / GL;  // row (b, hq, t)
  const int part = threadIdx.x % GL;
  const bool ok = r < n_rows;
  const int64_t rr = ok ? r : 0;
  const int64_t t = rr % T, bh = rr / T;
  const int hq = int(bh % Hq), b = int(bh / Hq);
  float x[8], y[8];
  load8(dout + b * do_sb + t * do_st + hq * do_sh + part * 8, x);
  load8(out + b * o_sb + t * o_st + hq * o_sh + part * 8, y);
  float a = 0.f;
#pragma unroll
  for (int e = 0; e < 8; ++e) a += x[e] * y[e];
  a = group_sum<GL>(a);
  if (ok && part == 0) delta[r] = a;
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
// dk / dv: workgroup = 64 keys of one (batch, kv head); logical tile order
// (kv row, key block).
//   snapshot mode: rows [kb*64, +64) of the snapshot chunk m = n + kblock / kblocks
//                  reads (all its queries, no causal mask, state temperature);
//   window mode:   tokens [kb*64, +64): query t sees token p iff
//                  wb(chunk(t)) <= p <= t (front temperature).
// Q and dO of 64 queries stream as blocks; the block's lse and delta go into
// LDS with the same DMA (wave 0, one float per lane).
template <int D, bool SNAP>
__global__ __launch_bounds__(NTB) __attribute__((amdgpu_waves_per_eu(2)))
void k_attn_bwd_dkdv(kvm_layer L, BwdArgs A, int kblocks, ChunkTable table) {
  constexpr int KS = D / 32, DT = D / 16;
  constexpr int BUF = Lay<D>::BUF, BLK = Lay<D>::BLK;
  __shared__ __attribute__((aligned(1024))) unsigned char lds[2 * BUF];
  __shared__ __attribute__((aligned(1024))) float stat[2][2][BN];  // [buffer][lse, delta][query]
  const int C = int(L.chunk_len), n = int(L.n_bswa_chunks);
  const int Hq = int(L.q_heads), Hkv = int(L.kv_heads), grp = Hq / Hkv;
  const int wg = xcd_logical(blockIdx.x, gridDim.x);
  const int kvrow = wg / kblocks, kblk = wg % kblocks;
  const int b = kvrow / Hkv, hk = kvrow % Hkv;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(int(threadIdx.x >> 6));
  const int64_t T = A.T;
  const float scale_nat = 1.0f / sqrtf(float(D));

  int m_snap = 0, nkeys;
  int64_t kb0;
  const uint16_t *kbase, *vbase;
  int64_t kst, vst;
  if (SNAP) {
    const int per = (int(A.snap_cap) + BKW - 1) / BKW;  // key blocks per snapshot
    m_snap = n + kblk / per;
    kb0 = int64_t(kblk % per) * BKW;
    nkeys = table.state_len[m_snap];
    const int64_t soff = int64_t(table.snap_slot[m_snap]) * A.snap_stride + int64_t(kvrow) * A.snap_cap * D;
    kbase = A.snap_k + soff;
    vbase = A.snap_v + soff;
    kst = vst = D;
  } else {
    kb0 = int64_t(kblk) * BKW;
    nkeys = int(T);
    kbase = static_cast<const uint16_t *>(A.kv.k) + b * A.kv.k_sb + hk * A.kv.k_sh;
    vbase = static_cast<const uint16_t *>(A.kv.v) + b * A.kv.v_sb + hk * A.kv.v_sh;
    kst = A.kv.k_st;
    vst = A.kv.v_st;
  }
  if (kb0 >= nkeys) {  // workgroup-uniform, before any barrier
    if (SNAP) {  // rows past the snapshot's length get a zero gradient
      const int64_t off = int64_t(table.snap_slot[m_snap]) * A.dsnap_stride + int64_t(kvrow) * A.snap_cap * D;
      const int64_t nrow = min(int64_t(BKW), A.snap_cap - kb0);
      for (int64_t i = threadIdx.x; i < nrow * D / 4; i += NTB) {
        reinterpret_cast<float4 *>(A.d_snap_k + off + kb0 * D)[i] = make_float4(0.f, 0.f, 0.f, 0.f);
        reinterpret_cast<float4 *>(A.d_snap_v + off + kb0 * D)[i] = make_float4(0.f, 0.f, 0.f, 0.f);
      }
    }
    return;
  }

  for (int i = threadIdx.x; i < 2 * BUF / 16; i += NTB)
    reinterpret_cast<uint4 *>(lds)[i] = make_uint4(0, 0, 0, 0);

  // B operands: K and V rows of this wave's 16 keys (row lane%16, dims ks*32 + 8*(lane/16)).
  const int64_t kr = kb0 + wave * 16 + (lane & 15);
  const bool kok = kr < nkeys;
  bf16x8 kf[KS], vf[KS];
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) {
    uint4 u = make_uint4(0, 0, 0, 0), w = make_uint4(0, 0, 0, 0);
    if (kok) {
      u = *reinterpret_cast<const uint4 *>(kbase + kr * kst + ks * 32 + (lane >> 4) * 8);
      w = *reinterpret_cast<const uint4 *>(vbase + kr * vst + ks * 32 + (lane >> 4) * 8);
    }
    kf[ks] = as_bf16x8(u);
    vf[ks] = as_bf16x8(w);
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
#pragma unroll
  for (int ks = 0; ks < KS; ++ks) {
    asm volatile("" : "+v"(kf[ks]));
    asm volatile("" : "+v"(vf[ks]));
  }
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
    tq_lo = kb0;
    const int64_t last_key = min(kb0 + BKW, T) - 1;
    tq_hi = min(T, (last_key / C + n) * int64_t(C));
  }
  const Lanes lo = lane_offsets(lane);
  const uint32_t lds_base = uint32_t(uintptr_t((lds_void *)lds));
  const uint32_t stat_base = uint32_t(uintptr_t((lds_void *)&stat[0][0][0]));
  const uint32_t qstride_b = uint32_t(A.q_st * 2), dstride_b = uint32_t(A.do_st * 2);
  const uint32_t qo = lo.drow * qstride_b + lo.dcol, doo = lo.drow * dstride_b + lo.dcol;
  const int nqb = int((tq_hi - tq_lo + BN - 1) / BN);
  const int64_t kp = kr;  // the lane's key (column lane%16 of every C tile)
#pragma unroll 1
  for (int h = 0; h < grp; ++h) {
    const int hq = hk * grp + h;
    const float tau = static_cast<const float *>(SNAP ? L.state_temp : L.front_temp)[hq];
    const float sc = kLog2e * scale_nat * tau, dsc = scale_nat * tau;
    const uint16_t *qrow = static_cast<const uint16_t *>(A.q) + b * A.q_sb + hq * A.q_sh;
    const uint16_t *dorow = static_cast<const uint16_t *>(A.dout) + b * A.do_sb + hq * A.do_sh;
    const float *lse_row = A.lse + (int64_t(b) * Hq + hq) * T;
    const float *dl_row = A.delta + (int64_t(b) * Hq + hq) * T;
    auto issue = [&](int jj) {
      const int64_t t0 = tq_lo + int64_t(jj) * BN;
      const int nv = int(min(int64_t(BN), tq_hi - t0));
      unsigned char *img = lds + (jj & 1) * BUF;
      if (nv < BN) {
        zero_v_tail<D, NTB>(img, nv);
        zero_v_tail<D, NTB>(img + BLK, nv);
      }
      issue_block<D, NWB>(lds_base + uint32_t((jj & 1) * BUF), key_rsrc(qrow + t0 * A.q_st, A.q_st, nv),
                          key_rsrc(dorow + t0 * A.do_st, A.do_st, nv), qo, doo, qstride_b, dstride_b, wave);
      if (wave == 0) {  // lse and delta of the block: one float per lane, rows >= nv not written
        const __amdgpu_buffer_rsrc_t lr = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<float *>(lse_row + t0), (short)0, nv * 4, kBufWord3);
        const __amdgpu_buffer_rsrc_t dr = __builtin_amdgcn_make_buffer_rsrc(
            const_cast<float *>(dl_row + t0), (short)0, nv * 4, kBufWord3);
        dma4(lr, stat_base + uint32_t(((jj & 1) * 2 + 0) * BN * 4), uint32_t(lane * 4));
        dma4(dr, stat_base + uint32_t(((jj & 1) * 2 + 1) * BN * 4), uint32_t(lane * 4));
      }
    };
    __syncthreads();  // both buffers are free (and zeroed, the first time)
    issue(0);
#pragma unroll 1
    for (int j = 0; j < nqb; ++j) {
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      __syncthreads();
      if (j + 1 < nqb) issue(j + 1);
      const int64_t t0 = tq_lo + int64_t(j) * BN;
      const int nq = int(min(int64_t(BN), tq_hi - t0));
      const unsigned char *qimg = lds + (j & 1) * BUF, *dimg = qimg + BLK;
      // Window start of the chunks the block's queries lie in: with C >= 64
      // a 64-query block spans at most two chunks, c0 and c0 + 1 (first
      // query of c0 + 1 at `bnd`); shorter chunks take the division per query.
      const int64_t c0 = t0 / C, bnd = (c0 + 1) * C;
      const int64_t wb0 = max(int64_t(0), (c0 - n + 1) * int64_t(C)), wb1 = max(int64_t(0), (c0 - n + 2) * int64_t(C));
      const bool two_chunks = C >= BN;
      const float *lse_s = &stat[j & 1][0][0], *dl_s = &stat[j & 1][1][0];
#pragma unroll
      for (int hb = 0; hb < 2; ++hb) {
        // wave-uniform: no valid query in the half, or (window) all of its
        // queries before the wave's first key
        if (nq <= 32 * hb) continue;
        if (!SNAP && t0 + 32 * hb + 31 < kb0 + wave * 16) continue;
        f32x4 s[2], dp[2];
#pragma unroll
        for (int q2 = 0; q2 < 2; ++q2) {
          const int qt = 2 * hb + q2;
          s[q2] = f32x4{0.f, 0.f, 0.f, 0.f};
          dp[q2] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int ks = 0; ks < KS; ++ks) {
            s[q2] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(row_frag(qimg, lo, qt, ks), kf[ks], s[q2], 0, 0, 0);
            dp[q2] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(row_frag(dimg, lo, qt, ks), vf[ks], dp[q2], 0, 0, 0);
          }
        }
        // P and dS (scaled by tau / sqrt(D)) in the B-operand layout of step hb:
        // lane holds queries qt*16 + 4*(lane/16) + i of key lane%16.
        // Wave-uniform: every (query, key) pair of the step is visible (all 32
        // queries valid, the wave's 16 keys valid and, in the window, at or
        // before the first query and at or after the last query's window
        // start), so no per-pair test is needed.
        const int64_t kw = kb0 + wave * 16;
        bool all_vis = 32 * hb + 32 <= nq && kw + 16 <= nkeys;
        if (!SNAP) {
          const int64_t qa = t0 + 32 * hb, qz = qa + 31;
          all_vis = all_vis && kw + 15 <= qa && max(int64_t(0), (qz / C - n + 1) * int64_t(C)) <= kw;
        }
        uint32_t pp[2][2], pd[2][2];
#pragma unroll
        for (int q2 = 0; q2 < 2; ++q2) {
          const int qr = (2 * hb + q2) * 16 + (lane >> 4) * 4;  // block-relative query of i = 0
          const float4 l4 = *reinterpret_cast<const float4 *>(lse_s + qr);
          const float4 d4 = *reinterpret_cast<const float4 *>(dl_s + qr);
          const float lv[4] = {l4.x, l4.y, l4.z, l4.w}, dv4[4] = {d4.x, d4.y, d4.z, d4.w};
          float p[4], d[4];
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            bool vis = true;
            if (!all_vis) {
              const int64_t t = t0 + qr + i;
              vis = qr + i < nq && kp < nkeys;
              if (!SNAP) {
                const int64_t wbt =
                    two_chunks ? (t < bnd ? wb0 : wb1) : max(int64_t(0), (t / C - n + 1) * int64_t(C));
                vis = vis && kp <= t && wbt <= kp;
              }
            }
            p[i] = vis ? __builtin_amdgcn_exp2f(__builtin_fmaf(s[q2][i], sc, -lv[i])) : 0.f;
            d[i] = p[i] * (dp[q2][i] - dv4[i]) * dsc;
          }
          pp[q2][0] = pack_bf16x2(p[0], p[1]);
          pp[q2][1] = pack_bf16x2(p[2], p[3]);
          pd[q2][0] = pack_bf16x2(d[0], d[1]);
          pd[q2][1] = pack_bf16x2(d[2], d[3]);
        }
        const bf16x8 pb = as_bf16x8(make_uint4(pp[0][0], pp[0][1], pp[1][0], pp[1][1]));
        const bf16x8 db = as_bf16x8(make_uint4(pd[0][0], pd[0][1], pd[1][0], pd[1][1]));
        // dv^T += dO^T P, dk^T += Q^T dS over the 32 queries of step hb.
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) {
          dv[dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(tr_frag(dimg, lo, hb, dt), pb, dv[dt], 0, 0, 0);
          dk[dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(tr_frag(qimg, lo, hb, dt), db, dk[dt], 0, 0, 0);
        }
      }
    }
  }
  // Owner writes (fp32): lane holds dims dt*16 + 4*(lane/16) + i of key kp;
  // snapshot rows past the snapshot's length are written as zeros.
  if (SNAP && kp >= nkeys) {
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) dk[dt] = dv[dt] = f32x4{0.f, 0.f, 0.f, 0.f};
  }
  if (kp < nkeys || (SNAP && kp < A.snap_cap)) {
    float *dkp, *dvp;
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
    for (int dt = 0; dt < DT; ++dt) {
      const int64_t o = kp * D + dt * 16 + (lane >> 4) * 4;
      *reinterpret_cast<float4 *>(dkp + o) = make_float4(dk[dt][0], dk[dt][1], dk[dt][2], dk[dt][3]);
      *reinterpret_cast<float4 *>(dvp + o) = make_float4(dv[dt][0], dv[dt][1], dv[dt][2], dv[dt][3]);
    }
  }
}

template <int D>
hipError_t launch_bwd_d(const kvm_layer &L, const BwdArgs &a, const ChunkTable &table, float *tpart,
                        hipStream_t stream) {
  const int n_chunks = int(a.n_chunks);
  const int qtiles = int((L.chunk_len + BQ - 1) / BQ);
  const int64_t rows = L.batch * L.kv_heads;
  hipLaunchKernelGGL((k_attn_bwd_dq<D>), dim3(unsigned(L.batch * L.q_heads * n_chunks * qtiles)), dim3(NTB), 0,
                     stream, L, a, qtiles, table, tpart);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(k_attn_bwd_temps, dim3(unsigned((L.q_heads + 63) / 64)), dim3(64), 0, stream, tpart,
                     int(L.batch), int(L.q_heads), n_chunks, qtiles, a.d_state_temp, a.d_front_temp);
  if ((e = hipGetLastError()) != hipSuccess) return e;
  const int wblocks = int((a.T + BKW - 1) / BKW);
  hipLaunchKernelGGL((k_attn_bwd_dkdv<D, false>), dim3(unsigned(wblocks * rows)), dim3(NTB), 0, stream, L, a,
                     wblocks, table);
  if ((e = hipGetLastError()) != hipSuccess) return e;
  const int n = int(L.n_bswa_chunks);
  if (n_chunks > n) {
    const int per = int((a.snap_cap + BKW - 1) / BKW);
    const int kblocks = (n_chunks - n) * per;
    hipLaunchKernelGGL((k_attn_bwd_dkdv<D, true>), dim3(unsigned(kblocks * rows)), dim3(NTB), 0, stream, L, a,
                       kblocks, table);
    e = hipGetLastError();
  }
  return e;
}

}  // namespace

int64_t attn_bwd_workspace_bytes(const kvm_layer &L, int64_t n_chunks) {
  const int64_t qtiles = (L.chunk_len + BQ - 1) / BQ;
  return L.batch * L.q_heads * n_chunks * qtiles * 2 * 4;
}

hipError_t launch_attn_delta(const kvm_layer &L, const void *dout, int64_t do_sb, int64_t do_st, int64_t do_sh,
                             const void *out, int64_t o_sb, int64_t o_st, int64_t o_sh, int64_t T, float *delta,
                             hipStream_t stream) {
  const int64_t n_rows = L.batch * L.q_heads * T;
  const int gl = int(L.head_dim / 8);
  const unsigned grid = unsigned((n_rows + (256 / gl) - 1) / (256 / gl));
  const uint16_t *dp = static_cast<const uint16_t *>(dout), *op = static_cast<const uint16_t *>(out);
  if (L.head_dim == 128)
    hipLaunchKernelGGL((k_attn_bwd_delta<128>), dim3(grid), dim3(256), 0, stream, dp, do_sb, do_st, do_sh, op,
                       o_sb, o_st, o_sh, int(L.q_heads), T, n_rows, delta);
  else
    hipLaunchKernelGGL((k_attn_bwd_delta<64>), dim3(grid), dim3(256), 0, stream, dp, do_sb, do_st, do_sh, op,
                       o_sb, o_st, o_sh, int(L.q_heads), T, n_rows, delta);
  return hipGetLastError();
}

hipError_t launch_attn_backward(const kvm_layer &L, const BwdArgs &a, const ChunkTable &table,
                                float *tpart, hipStream_t stream) {
  if (L.head_dim == 128) return launch_bwd_d<128>(L, a, table, tpart, stream);
  return launch_bwd_d<64>(L, a, table, tpart, stream);
}

}  // namespace kvm
