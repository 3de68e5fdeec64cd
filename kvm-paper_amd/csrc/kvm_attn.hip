// Fused KVM prefill attention on gfx950: memory slots + block-sliding window.
//
// Reference semantics: model/kvm_mixer.py:194-229 (_attend_with_state_and_bswa,
// lower-right causal mask :16-22) and the front causal attention :419-432;
// the Triton kernel it replaces is _kvm_attn_live_state_fwd_kernel
// (model/kernels/kvm_triton_training_kernels.py:1803-1948), which runs one
// launch per query chunk.
//
// Here one launch covers many query chunks.  Chunk m (queries [mC, mC+C))
// attends to
//   * the S_m memory slots of the state after the updates that precede it
//     (a snapshot: LayerNorm_s(s_k) and bf16(normalize(s_v) * vlen) rows),
//     keys scaled by the state temperature;
//   * window tokens [max(0, (m-n+1)C), query] causally, keys scaled by the
//     front temperature.
// Workgroup = NW waves = 32*NW queries of one (batch, q_head); each wave owns
// 32 queries (two 16-row MFMA tiles).  Scores are computed transposed,
// S^T = K Q^T, with v_mfma_f32_16x16x32_bf16, so that each lane holds 4
// consecutive keys of one query row: the P^T tiles feed the O^T = V^T P^T
// product directly as the B operand (the key order inside a 32-key step is
// permuted identically in the A operand, which leaves the sum unchanged).
// Online softmax in fp32 registers with exp2; P rounded to bf16 for the PV
// product.
//
// Numerics against the Triton kernel: the temperature multiplies the fp32
// score (scale * tau) instead of being rounded into a bf16 copy of K
// (:1868, :1900); the row sums are fp32 sums of the unrounded weights, as
// there (:1884).
//
// Data movement: key blocks of 64 go from HBM/L2 straight into LDS with
// buffer_load_dwordx4 ... lds (no register staging, no VALU or ds_write
// work).  The LDS image of a block keeps keys row-major in 64-byte column
// groups with a per-key swap of 32-byte halves, so that the K fragment reads
// (ds_read_b128) and the V^T fragment reads (ds_read_b64_tr_b16, the gfx950
// transposing LDS read) are free of bank conflicts while each 1 KiB DMA
// instruction still reads whole 64-byte runs of 16 keys.  Key images are
// triple-buffered and value images double-buffered: while block j is
// consumed, the values of block j+1 and the keys of blocks j+1 and j+2 are in
// flight (the loop is bound by how many bytes each CU has in flight from
// L2).  One barrier per block.  A workgroup of 4 waves (one per SIMD) uses
// 80 KiB of LDS (D = 128), so two independent workgroups share a CU (160 KiB)
// and fill each other's stalls.
// Workgroups are renumbered so that each XCD (dispatch is round-robin over
// the 8 XCDs) runs a contiguous range of (head, chunk) tiles: the window keys
// shared by neighbouring chunks stay in that XCD's L2.

#include "kvm_attn_tile.hpp"
#include "kvm_device.hpp"
#include "kvm_internal.hpp"

namespace kvm {
namespace {

constexpr int NW = 4;  // waves per workgroup
using namespace tile;

template <int D>
struct AttnState {
  f32x4 o[2][D / 16];  // O^T tiles [row tile][dv tile]
  float m[2];          // reference maximum of each row (log2 domain), -inf before any key
  float l[2];          // lane-partial running row sums (fp32, unrounded weights)
};

// A row's reference maximum moves only when a block's maximum exceeds it by
// more than this (log2 units): probabilities stay <= 2^8, exactly
// representable range for fp32 sums and bf16 P, and the O rescale (64
// multiplies per lane) is skipped in almost every block.
constexpr float kRescaleSlack = 8.0f;
// A block's weights are first computed against the current reference
// maxima; the block maxima are needed only when some lane's sum of its
// weights of a row exceeds 2^kRescaleSlack (no weight exceeds that when no
// sum does) or a row has no reference yet.
constexpr float kSumLimit = 256.0f;

// Maxima of scores without the quieting copies (v_max_f32 x, x) the compiler
// adds around fmaxf in IEEE mode: scores are MFMA sums of finite products or
// the -inf of a mask, never NaN, so the plain instructions give the same
// result.
__device__ __forceinline__ float max2_raw(float a, float b) {
  float r;
  asm("v_max_f32 %0, %1, %2" : "=v"(r) : "v"(a), "v"(b));
  return r;
}
__device__ __forceinline__ float max3_raw(float a, float b, float c) {
  float r;
  asm("v_max3_f32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "v"(c));
  return r;
}

// S^T tiles of the 64 keys of a buffered block: s[kt][rt], kt = 16-key
// tile, rt = 16-query tile.  kbuf + kb addresses key lane&15, dims
// 8*(lane>>4).. of column group 0.  The k-step loop is outermost, so eight
// independent accumulations are in flight between dependent MFMAs (each
// tile still sums its k-steps in order 0, 1, ...).
template <int D>
__device__ __forceinline__ void score_block(const unsigned char *kbuf, const bf16x8 (&qf)[2][D / 32],
                                            f32x4 (&s)[4][2]) {
#pragma unroll
  for (int kt = 0; kt < 4; ++kt) {
    s[kt][0] = f32x4{0.f, 0.f, 0.f, 0.f};
    s[kt][1] = f32x4{0.f, 0.f, 0.f, 0.f};
  }
#pragma unroll
  for (int ks = 0; ks < D / 32; ++ks) {
    bf16x8 kf[4];
#pragma unroll
    for (int kt = 0; kt < 4; ++kt)
      kf[kt] = as_bf16x8(*reinterpret_cast<const uint4 *>(kbuf + ks * 4096 + kt * 1024));
#pragma unroll
    for (int kt = 0; kt < 4; ++kt) {
      s[kt][0] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kf[kt], qf[0][ks], s[kt][0], 0, 0, 0);
      s[kt][1] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kf[kt], qf[1][ks], s[kt][1], 0, 0, 0);
    }
  }
}

// Masking: keys >= nvalid, or causal keys > qrel + row, where qrel is the
// wave's first query minus the position of the block's first key.
__device__ __forceinline__ void block_mask(f32x4 (&s)[4][2], int nvalid, bool causal, int qrel) {
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int rt = 0; rt < 2; ++rt) {
    const int lim = qrel + rt * 16 + (lane & 15);
#pragma unroll
    for (int kt = 0; kt < 4; ++kt)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int key = kt * 16 + (lane >> 4) * 4 + i;
        if (key >= nvalid || (causal && key > lim)) s[kt][rt][i] = -INFINITY;
      }
  }
}

// Row maxima (v_permlane swaps across the 16-lane groups) and the lazy move
// of the reference maximum with its O rescale.
template <int D>
__device__ __forceinline__ void block_max(const f32x4 (&s)[4][2], AttnState<D> &as, float scale) {
  bool need = false;
  float m_new[2];
#pragma unroll
  for (int rt = 0; rt < 2; ++rt) {
    float mx = max3_raw(s[0][rt][0], s[0][rt][1], s[0][rt][2]);
    mx = max3_raw(mx, s[0][rt][3], s[1][rt][0]);
    mx = max3_raw(mx, s[1][rt][1], s[1][rt][2]);
    mx = max3_raw(mx, s[1][rt][3], s[2][rt][0]);
    mx = max3_raw(mx, s[2][rt][1], s[2][rt][2]);
    mx = max3_raw(mx, s[2][rt][3], s[3][rt][0]);
    mx = max3_raw(mx, s[3][rt][1], s[3][rt][2]);
    mx = max2_raw(mx, s[3][rt][3]);
    // max with lane ^ 16, then lane ^ 32 (each swap returns both values)
    const auto r16 = __builtin_amdgcn_permlane16_swap(__float_as_uint(mx), __float_as_uint(mx), false, false);
    mx = max2_raw(__uint_as_float(r16[0]), __uint_as_float(r16[1]));
    const auto r32 = __builtin_amdgcn_permlane32_swap(__float_as_uint(mx), __float_as_uint(mx), false, false);
    mx = max2_raw(__uint_as_float(r32[0]), __uint_as_float(r32[1]));
    m_new[rt] = mx * scale;
    need |= m_new[rt] > as.m[rt] + kRescaleSlack;
  }
  if (__ballot(need)) {
#pragma unroll
    for (int rt = 0; rt < 2; ++rt) {
      const bool mv = m_new[rt] > as.m[rt] + kRescaleSlack;
      const float alpha = mv ? (as.m[rt] == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(as.m[rt] - m_new[rt])) : 1.f;
      if (mv) as.m[rt] = m_new[rt];
      as.l[rt] *= alpha;
#pragma unroll
      for (int dt = 0; dt < D / 16; ++dt) as.o[rt][dt] *= alpha;
    }
  }
}

// P^T = exp2(S^T * scale - m) in the B-operand layout (two 32-key steps,
// each lane 8 keys, 4 per kt) and the lane-partial row sums of the block.
template <int D>
__device__ __forceinline__ void block_probs(const f32x4 (&s)[4][2], const AttnState<D> &as,
                                            float scale, bf16x8 (&pb)[2][2], float (&bsum)[2]) {
#pragma unroll
  for (int rt = 0; rt < 2; ++rt) {
    const float base = as.m[rt] == -INFINITY ? 0.f : as.m[rt];
    float psum;
    uint32_t pk[4][2];
#pragma unroll
    for (int kt = 0; kt < 4; ++kt) {
      float p[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        p[i] = __builtin_amdgcn_exp2f(__builtin_fmaf(s[kt][rt][i], scale, -base));
        // The block's sum starts at its first weight (p >= +0, so 0 + p == p).
        psum = (kt == 0 && i == 0) ? p[i] : psum + p[i];
      }
      pk[kt][0] = pack_bf16x2(p[0], p[1]);
      pk[kt][1] = pack_bf16x2(p[2], p[3]);
    }
    bsum[rt] = psum;
    pb[0][rt] = as_bf16x8(make_uint4(pk[0][0], pk[0][1], pk[1][0], pk[1][1]));
    pb[1][rt] = as_bf16x8(make_uint4(pk[2][0], pk[2][1], pk[3][0], pk[3][1]));
  }
}

// O^T += V^T P^T over the 64 keys (two 32-key steps).  The
// V^T fragment (dims dt*16 + lane%16, the 8 keys of the lane's B slots) is
// two ds_read_b64_tr_b16 reads of the key-major block: within each 16-lane
// group, source lane s reads 4 dims of key 4*(lane/16) + s/4 and the
// transpose hands lane l the 4 keys of dim l.  vbuf + vb0 / vb1: lane
// offsets for even / odd dim tiles.
template <int D>
__device__ __forceinline__ void block_pv(const unsigned char *vbuf, uint32_t vb0, uint32_t vb1,
                                         const bf16x8 (&pb)[2][2], AttnState<D> &as) {
#pragma unroll
  for (int h = 0; h < 2; ++h) {
#pragma unroll
    for (int dt = 0; dt < D / 16; ++dt) {
      const unsigned char *p = vbuf + ((dt & 1) ? vb1 : vb0) + (dt >> 1) * 4096 + h * 2048;
      const v4i16 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16 *)(p));
      const v4i16 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16 *)(p + 1024));
      const uint2 l2 = __builtin_bit_cast(uint2, lo), h2 = __builtin_bit_cast(uint2, hi);
      const bf16x8 vf = as_bf16x8(make_uint4(l2.x, l2.y, h2.x, h2.y));
      as.o[0][dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vf, pb[h][0], as.o[0][dt], 0, 0, 0);
      as.o[1][dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vf, pb[h][1], as.o[1][dt], 0, 0, 0);
    }
  }
}

template <int D>
__global__ __launch_bounds__(NW * 64) __attribute__((amdgpu_waves_per_eu(2)))
void k_attn_prefill(kvm_layer L, PrefillAttnArgs A, int chunk_begin, int qtiles, int n_chunks,
                    ChunkTable table) {
  constexpr int NT = NW * 64, BM = NW * 32;
  constexpr int BLK = Lay<D>::BLK;
  constexpr int KBUFS = 3, VBUFS = 2;
  constexpr int PER = Lay<D>::CHUNKS / NW;  // DMA instructions per wave and image
  __shared__ __attribute__((aligned(1024))) unsigned char lds[(KBUFS + VBUFS) * BLK];
  const int C = int(L.chunk_len), n = int(L.n_bswa_chunks);
  const int Hq = int(L.q_heads), Hkv = int(L.kv_heads);
  // XCD-contiguous renumbering of the 1-D grid: logical order (q row, chunk, q tile).
  const int N = gridDim.x;
  const int x = blockIdx.x % kXcds, jx = blockIdx.x / kXcds;
  const int q8 = N / kXcds, r8 = N % kXcds;
  const int logical = x * q8 + min(x, r8) + jx;
  const int per_row = n_chunks * qtiles;
  const int qrow = logical / per_row;
  const int rem = logical % per_row;
  const int c_local = rem / qtiles, qt = rem % qtiles;
  const int b = qrow / Hq, hq = qrow % Hq;
  const int hk = hq / (Hq / Hkv);
  const int kvrow = b * Hkv + hk;
  const int m = chunk_begin + c_local;
  const int64_t T = A.T;
  const int64_t q0 = int64_t(m) * C + int64_t(qt) * BM;
  if (q0 >= T) return;
  const int64_t q_hi = min(min(q0 + BM, int64_t(m + 1) * C), T);  // exclusive
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(int(threadIdx.x >> 6));
  const int64_t qpos0 = q0 + wave * 32;

  // LDS is not cleared: key rows past a short block are masked (their
  // scores are replaced, whatever the stale bytes), and the value rows past
  // it are zeroed before each such block's DMA (zero_v_tail).

  // Q fragments (B operand of S^T): row rt*16 + lane%16, dims ks*32 + 8*(lane/16).
  bf16x8 qf[2][D / 32];
  const uint16_t *qbase = static_cast<const uint16_t *>(A.q) + b * A.q_sb + hq * A.q_sh;
#pragma unroll
  for (int rt = 0; rt < 2; ++rt) {
    const int64_t t = qpos0 + rt * 16 + (lane & 15);
#pragma unroll
    for (int ks = 0; ks < D / 32; ++ks) {
      uint4 u = make_uint4(0, 0, 0, 0);
      if (t < q_hi)
        u = *reinterpret_cast<const uint4 *>(qbase + t * A.q_st + ks * 32 + (lane >> 4) * 8);
      qf[rt][ks] = as_bf16x8(u);
    }
  }
  // Complete the Q loads here and hide them from the compiler's wait
  // tracking: inside the key loop the only outstanding vector-memory
  // operations are then the block DMAs, awaited explicitly.
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
#pragma unroll
  for (int rt = 0; rt < 2; ++rt)
#pragma unroll
    for (int ks = 0; ks < D / 32; ++ks) asm volatile("" : "+v"(qf[rt][ks]));

  AttnState<D> as;
#pragma unroll
  for (int rt = 0; rt < 2; ++rt) {
    as.m[rt] = -INFINITY;
    as.l[rt] = 0.f;
#pragma unroll
    for (int dt = 0; dt < D / 16; ++dt) as.o[rt][dt] = f32x4{0.f, 0.f, 0.f, 0.f};
  }
  const float scale = kLog2e / sqrtf(float(D));
  const float tau_s = static_cast<const float *>(L.state_temp)[hq];
  const float tau_f = static_cast<const float *>(L.front_temp)[hq];

  // Lane offsets in a block image.  K fragments: key lane&15, unit
  // (lane>>4) ^ swap(key).  V^T transpose reads: key 4*(lane/16) +
  // (lane%16)/4, 8-byte piece lane&3 of the 32-byte half (dt&1) ^ swap(key)
  // (bit 2 of the key is bit 0 of lane/16).  DMA: key lane/4 of the
  // instruction's 16, unit (lane&3) ^ swap(key).
  const uint32_t kb = uint32_t((lane & 15) * 64 + (((lane >> 4) ^ (((lane >> 2) & 1) << 1)) * 16));
  const int g = lane >> 4, s4 = lane & 15;
  const uint32_t vrow = uint32_t((4 * g + (s4 >> 2)) * 64 + 8 * (s4 & 3));
  const uint32_t vb0 = vrow + uint32_t(32 * (g & 1));
  const uint32_t vb1 = vrow + uint32_t(32 * ((g & 1) ^ 1));
  const uint32_t dcol = uint32_t(((lane & 3) ^ (((lane >> 4) & 1) << 1)) * 16);
  const uint32_t drow = uint32_t(lane >> 2);
  const uint32_t lds_base = uint32_t(uintptr_t((lds_void *)lds));

  // Key ranges: the memory slots (state temperature, never causal), then
  // the window tokens [wb, q_hi) (front temperature, causal).  One copy of
  // the pipeline serves both.
  const int S = table.state_len[c_local];
  const int64_t wb = max(int64_t(0), int64_t(m - n + 1) * C);
  const int64_t soff = int64_t(table.snap_slot[c_local]) * A.snap_stride +
                       int64_t(kvrow) * A.snap_cap * D;
  const uint16_t *kwin = static_cast<const uint16_t *>(A.kv.k) + b * A.kv.k_sb + hk * A.kv.k_sh;
  const uint16_t *vwin = static_cast<const uint16_t *>(A.kv.v) + b * A.kv.v_sb + hk * A.kv.v_sh;
#pragma unroll 1
  for (int seg = 0; seg < 2; ++seg) {
    const bool st = seg == 0;
    const int nkeys = st ? ((m >= n) ? S : 0) : int(q_hi - wb);
    if (nkeys <= 0) continue;
    const uint16_t *kp = st ? A.snap_k + soff : kwin + wb * A.kv.k_st;
    const uint16_t *vp = st ? A.snap_v + soff : vwin + wb * A.kv.v_st;
    const int64_t kstride = st ? D : A.kv.k_st;
    const int64_t vstride = st ? D : A.kv.v_st;
    const uint32_t kstride_b = uint32_t(kstride * 2), vstride_b = uint32_t(vstride * 2);
    const uint32_t ko = drow * kstride_b + dcol, vo = drow * vstride_b + dcol;
    const float sc = scale * (st ? tau_s : tau_f);
    const bool causal = !st;
    const int nb = (nkeys + BN - 1) / BN;
    // Causal ranges: block jj's first key is at wb + jj * BN.
    auto qrel_of = [&](int jj) -> int {
      const int64_t q = causal ? qpos0 - (wb + int64_t(jj) * BN) : int64_t(BN);
      return int(min(max(q, int64_t(-64)), int64_t(BN)));
    };
    // Keys of block jj into image jj % 3, values into image 3 + jj % 2.
    auto issue_k = [&](int jj) {
      const int jn = jj * BN;
      const int nv = min(BN, nkeys - jn);
      issue_image<D, NW>(lds_base + uint32_t((jj % KBUFS) * BLK),
                         key_rsrc(kp + int64_t(jn) * kstride, kstride, nv), ko, kstride_b, wave);
    };
    auto issue_v = [&](int jj) {
      const int jn = jj * BN;
      const int nv = min(BN, nkeys - jn);
      if (nv < BN) zero_v_tail<D, NT>(lds + (KBUFS + (jj & 1)) * BLK, nv);
      issue_image<D, NW>(lds_base + uint32_t((KBUFS + (jj & 1)) * BLK),
                         key_rsrc(vp + int64_t(jn) * vstride, vstride, nv), vo, vstride_b, wave);
    };
    __syncthreads();  // every image is free
    issue_k(0);
    issue_v(0);
    if (nb > 1) issue_k(1);
    // Step j: this wave's DMAs were issued in the order ..., keys j, values
    // j, keys j + 1; wait until only the keys of block j + 1 may be in
    // flight, barrier (block j complete in LDS; every wave is past block
    // j - 1, whose images are reused now), DMA of the values of block j + 1
    // and the keys of block j + 2, then consume block j.
#pragma unroll 1
    for (int j = 0; j < nb; ++j) {
      if (j + 1 < nb)
        asm volatile("s_waitcnt vmcnt(%0)" :: "n"(PER) : "memory");
      else
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      __syncthreads();
      if (j + 1 < nb) issue_v(j + 1);
      if (j + 2 < nb) issue_k(j + 2);
      const int qrel = qrel_of(j);
      if (qrel + 31 < 0) continue;  // wave-uniform: block above the wave's causal diagonal
      const int nvalid = min(BN, nkeys - j * BN);
      const bool masked = nvalid < BN || qrel < BN - 1;
      f32x4 s[4][2];
      score_block<D>(lds + (j % KBUFS) * BLK + kb, qf, s);
      if (masked) block_mask(s, nvalid, causal, qrel);
      // Weights against the current references; the maxima (and a second
      // pass over the weights) only where a reference must be set or may
      // move (a weight above 2^kRescaleSlack: the block maximum exceeds the
      // reference by more than the slack).  Outside rounding ties at that
      // boundary the references move in the same blocks as when the maxima
      // come first.
      bf16x8 pb[2][2];
      float bsum[2];
      bool slow = __ballot(as.m[0] == -INFINITY || as.m[1] == -INFINITY) != 0;
      if (!slow) {
        block_probs<D>(s, as, sc, pb, bsum);
        slow = __ballot(bsum[0] > kSumLimit || bsum[1] > kSumLimit) != 0;
      }
      if (slow) {
        block_max<D>(s, as, sc);
        block_probs<D>(s, as, sc, pb, bsum);
      }
      as.l[0] += bsum[0];
      as.l[1] += bsum[1];
      block_pv<D>(lds + (KBUFS + (j & 1)) * BLK, vb0, vb1, pb, as);
    }
  }

  // Normalise and store: lane holds dv = dt*16 + 4*(lane/16) + i of row lane%16.
  uint16_t *obase = static_cast<uint16_t *>(A.out) + b * A.o_sb + hq * A.o_sh;
#pragma unroll
  for (int rt = 0; rt < 2; ++rt) {
    // row sum over the 4 lanes of the row (lane ^ 16, lane ^ 32)
    float l = as.l[rt];
    const auto r16 = __builtin_amdgcn_permlane16_swap(__float_as_uint(l), __float_as_uint(l), false, false);
    l = __uint_as_float(r16[0]) + __uint_as_float(r16[1]);
    const auto r32 = __builtin_amdgcn_permlane32_swap(__float_as_uint(l), __float_as_uint(l), false, false);
    l = __uint_as_float(r32[0]) + __uint_as_float(r32[1]);
    const float inv = 1.0f / l;
    const int64_t t = qpos0 + rt * 16 + (lane & 15);
    // log2-domain log-sum-exp of the row: the probabilities are exp2(s - m) / l.
    if (A.lse && lane < 16 && t < q_hi)
      A.lse[(int64_t(b) * Hq + hq) * T + t] = as.m[rt] + log2f(l);
    if (t < q_hi) {
#pragma unroll
      for (int dt = 0; dt < D / 16; ++dt) {
        uint2 w;
        w.x = pack_bf16x2(as.o[rt][dt][0] * inv, as.o[rt][dt][1] * inv);
        w.y = pack_bf16x2(as.o[rt][dt][2] * inv, as.o[rt][dt][3] * inv);
        *reinterpret_cast<uint2 *>(obase + t * A.o_st + dt * 16 + (lane >> 4) * 4) = w;
      }
    }
  }
}

template <int D>
hipError_t launch_d(const kvm_layer &L, const PrefillAttnArgs &a, int64_t chunk_begin,
                    int64_t n_chunks, const ChunkTable &table, hipStream_t stream) {
  const int qtiles = int((L.chunk_len + NW * 32 - 1) / (NW * 32));
  const int64_t n_wg = n_chunks * qtiles * L.batch * L.q_heads;
  const dim3 grid{unsigned(n_wg), 1u, 1u};
  hipLaunchKernelGGL((k_attn_prefill<D>), grid, dim3(NW * 64), 0, stream, L, a,
                     int(chunk_begin), qtiles, int(n_chunks), table);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_prefill_attention(const kvm_layer &L, const PrefillAttnArgs &a,
                                    int64_t chunk_begin, int64_t n_chunks,
                                    const ChunkTable &table, hipStream_t stream) {
  if (n_chunks <= 0) return hipSuccess;
  if (L.head_dim == 128) return launch_d<128>(L, a, chunk_begin, n_chunks, table, stream);
  return launch_d<64>(L, a, chunk_begin, n_chunks, table, stream);
}

}  // namespace kvm
