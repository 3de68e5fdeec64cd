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
// 32 queries (two 16-row MFMA tiles).  Keys stream through LDS in blocks of
// 64: K row-major (times temperature, rounded to bf16, as the reference
// does), V transposed.  Scores are computed transposed, S^T = K Q^T, with
// v_mfma_f32_16x16x32_bf16, so that each lane holds 4 consecutive keys of one
// query row: the P^T tiles feed the O^T = V^T P^T product directly as the B
// operand (the key order inside a 32-key step is permuted identically in the
// A operand, which leaves the sum unchanged).  Online softmax in fp32
// registers with exp2; P rounded to bf16 for the PV product.
//
// Latency structure: a workgroup of 8 waves (256 queries) shares each staged
// key block, so a block load feeds twice the MFMA work of a 4-wave tile and
// each thread stages half as much.  A wave consumes a whole 64-key block per
// step (8 independent MFMA chains, one max reduction per 64 keys) and keeps
// a lazily moved reference maximum per row, so the O rescale is rare.  Global loads are buffer loads whose
// range check zero-fills keys past the end of a range (no per-load
// branches, 32-bit offsets).  Every 32-key step reads all of its K fragments
// from LDS before the score MFMAs and all of its V fragments before the
// softmax arithmetic, so LDS latency overlaps MFMA and VALU work instead of
// serialising with it.  Two LDS buffers, one barrier per block.  Workgroups
// are renumbered so that each XCD (dispatch is round-robin over the 8 XCDs)
// runs a contiguous range of (head, chunk) tiles: the window keys shared by
// neighbouring chunks stay in that XCD's L2.

#include "kvm_device.hpp"
#include "kvm_internal.hpp"

namespace kvm {
namespace {

constexpr int BN = 64;   // keys per block
constexpr float kLog2e = 1.4426950408889634f;
constexpr int kXcds = 8;
// Buffer resource word 3 for raw (unformatted, unswizzled) dword access with
// range checking: out-of-range loads return zero.
constexpr int kBufWord3 = 0x00020000;

typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
  const f32x2 v = {a, b};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2));
}

template <int D>
struct AttnSmem {
  static constexpr int KSTR = D + 8;   // K row stride (elements)
  static constexpr int VSTR = BN + 8;  // V^T row stride (elements)
  uint16_t k[BN * KSTR];
  uint16_t vt[D * VSTR];
};

// Register staging of one K/V block over NT threads: K in 16-byte pieces
// (key p / (D/8), dims 8 * (p % (D/8))), V in units of 2 keys x 8 dims.
template <int D, int NT>
struct Stage {
  static constexpr int KPIECES = BN * (D / 8);
  static constexpr int KPT = (KPIECES + NT - 1) / NT;
  static constexpr int VUNITS = (BN / 2) * (D / 8);
  static constexpr int VPT = (VUNITS + NT - 1) / NT;
  uint4 k[KPT];
  uint4 v[VPT][2];
};

__device__ __forceinline__ uint4 buf_load16(__amdgpu_buffer_rsrc_t r, uint32_t off) {
  const u32x4 x = __builtin_amdgcn_raw_buffer_load_b128(r, int(off), 0, 0);
  return make_uint4(x[0], x[1], x[2], x[3]);
}

// Resource over keys [0, nvalid) of a range starting at p with row stride
// `stride` elements: byte offsets key * stride * 2 + 16 * part of keys past
// nvalid fall outside it and read as zero.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t key_rsrc(const uint16_t *p, int64_t stride,
                                                          int nvalid) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t *>(p), (short)0,
                                           int(nvalid * stride * 2), kBufWord3);
}

template <int D, int NT>
__device__ __forceinline__ void stage_load(Stage<D, NT> &sg, __amdgpu_buffer_rsrc_t kr,
                                           uint32_t kstride_b, __amdgpu_buffer_rsrc_t vr,
                                           uint32_t vstride_b) {
  using S = Stage<D, NT>;
  const int tid = threadIdx.x;
#pragma unroll
  for (int i = 0; i < S::KPT; ++i) {
    const int p = tid + i * NT;
    if (S::KPIECES % NT == 0 || p < S::KPIECES) {
      const int key = p / (D / 8), part = p % (D / 8);
      sg.k[i] = buf_load16(kr, uint32_t(key) * kstride_b + uint32_t(part) * 16u);
    }
  }
#pragma unroll
  for (int i = 0; i < S::VPT; ++i) {
    const int u = tid + i * NT;
    if (S::VUNITS % NT == 0 || u < S::VUNITS) {
      const int kp = u % (BN / 2), dg = u / (BN / 2);
      const uint32_t off = uint32_t(2 * kp) * vstride_b + uint32_t(dg) * 16u;
      sg.v[i][0] = buf_load16(vr, off);
      sg.v[i][1] = buf_load16(vr, off + vstride_b);
    }
  }
}

// bf16 pair (lo half of a, lo half of b) -> one word, etc.
__device__ __forceinline__ uint32_t lo_lo(uint32_t a, uint32_t b) {
  return __builtin_amdgcn_perm(b, a, 0x05040100u);
}
__device__ __forceinline__ uint32_t hi_hi(uint32_t a, uint32_t b) {
  return __builtin_amdgcn_perm(b, a, 0x07060302u);
}

template <int D, int NT>
__device__ __forceinline__ void stage_store(AttnSmem<D> &sm, const Stage<D, NT> &sg,
                                            float tau, bool scale) {
  using S = Stage<D, NT>;
  constexpr int KSTR = AttnSmem<D>::KSTR, VSTR = AttnSmem<D>::VSTR;
  const int tid = threadIdx.x;
#pragma unroll
  for (int i = 0; i < S::KPT; ++i) {
    const int p = tid + i * NT;
    if (S::KPIECES % NT == 0 || p < S::KPIECES) {
      const int key = p / (D / 8), part = p % (D / 8);
      uint4 w = sg.k[i];
      if (scale) {
        float x[8];
        unpack8(w, x);
        w.x = pack_bf16x2(x[0] * tau, x[1] * tau);
        w.y = pack_bf16x2(x[2] * tau, x[3] * tau);
        w.z = pack_bf16x2(x[4] * tau, x[5] * tau);
        w.w = pack_bf16x2(x[6] * tau, x[7] * tau);
      }
      *reinterpret_cast<uint4 *>(&sm.k[key * KSTR + part * 8]) = w;
    }
  }
#pragma unroll
  for (int i = 0; i < S::VPT; ++i) {
    const int u = tid + i * NT;
    if (S::VUNITS % NT == 0 || u < S::VUNITS) {
      const int kp = u % (BN / 2), dg = u / (BN / 2);
      const uint32_t a0[4] = {sg.v[i][0].x, sg.v[i][0].y, sg.v[i][0].z, sg.v[i][0].w};
      const uint32_t a1[4] = {sg.v[i][1].x, sg.v[i][1].y, sg.v[i][1].z, sg.v[i][1].w};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        // dims 2j (low halves) and 2j+1 (high halves) of keys 2kp, 2kp+1
        *reinterpret_cast<uint32_t *>(&sm.vt[(dg * 8 + 2 * j) * VSTR + 2 * kp]) = lo_lo(a0[j], a1[j]);
        *reinterpret_cast<uint32_t *>(&sm.vt[(dg * 8 + 2 * j + 1) * VSTR + 2 * kp]) = hi_hi(a0[j], a1[j]);
      }
    }
  }
}

template <int D>
struct AttnState {
  f32x4 o[2][D / 16];  // O^T tiles [row tile][dv tile]
  float m[2];          // reference maximum of each row (log2 domain), -inf before any key
  float l[2];          // lane-partial running sum
};

// A row's reference maximum moves only when a block's maximum exceeds it by
// more than this (log2 units): probabilities stay <= 2^8, exactly
// representable range for fp32 sums and bf16 P, and the O rescale (64
// multiplies per lane) is skipped in almost every block.
constexpr float kRescaleSlack = 8.0f;

// Online-softmax update with the 64 keys of a staged block.  Masked path:
// keys >= nvalid, or (causal ranges) keys past the query: key > qrel + row,
// where qrel is the wave's first query minus the position of the block's
// first key.
template <int D>
__device__ __forceinline__ void consume_block(const AttnSmem<D> &sm, AttnState<D> &as,
                                              const bf16x8 (&qf)[2][D / 32], bool masked,
                                              int nvalid, bool causal, int qrel, float scale) {
  constexpr int KSTR = AttnSmem<D>::KSTR, VSTR = AttnSmem<D>::VSTR;
  const int lane = threadIdx.x & 63;
  // S^T tiles for 64 keys: s[kt][rt], kt = 16-key tile, rt = 16-query tile.
  f32x4 s[4][2];
#pragma unroll
  for (int kt = 0; kt < 4; ++kt) {
    bf16x8 kf[D / 32];
#pragma unroll
    for (int ks = 0; ks < D / 32; ++ks)
      kf[ks] = as_bf16x8(*reinterpret_cast<const uint4 *>(
          &sm.k[(kt * 16 + (lane & 15)) * KSTR + ks * 32 + (lane >> 4) * 8]));
    s[kt][0] = f32x4{0.f, 0.f, 0.f, 0.f};
    s[kt][1] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < D / 32; ++ks) {
      s[kt][0] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kf[ks], qf[0][ks], s[kt][0], 0, 0, 0);
      s[kt][1] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kf[ks], qf[1][ks], s[kt][1], 0, 0, 0);
    }
  }
  if (masked) {
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
  bool need = false;
  float m_new[2];
#pragma unroll
  for (int rt = 0; rt < 2; ++rt) {
    float mx = fmaxf(fmaxf(s[0][rt][0], s[0][rt][1]), s[0][rt][2]);
    mx = fmaxf(fmaxf(mx, s[0][rt][3]), s[1][rt][0]);
    mx = fmaxf(fmaxf(mx, s[1][rt][1]), s[1][rt][2]);
    mx = fmaxf(fmaxf(mx, s[1][rt][3]), s[2][rt][0]);
    mx = fmaxf(fmaxf(mx, s[2][rt][1]), s[2][rt][2]);
    mx = fmaxf(fmaxf(mx, s[2][rt][3]), s[3][rt][0]);
    mx = fmaxf(fmaxf(mx, s[3][rt][1]), s[3][rt][2]);
    mx = fmaxf(mx, s[3][rt][3]);
    mx = fmaxf(mx, __shfl_xor(mx, 16));
    mx = fmaxf(mx, __shfl_xor(mx, 32));
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
  // P^T in the B-operand layout: two 32-key steps, each lane 8 keys (4 per kt).
  bf16x8 pb[2][2];  // [32-key step][rt]
#pragma unroll
  for (int rt = 0; rt < 2; ++rt) {
    const float base = as.m[rt] == -INFINITY ? 0.f : as.m[rt];
    float psum = 0.f;
    uint32_t pk[4][2];
#pragma unroll
    for (int kt = 0; kt < 4; ++kt) {
      float p[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        p[i] = __builtin_amdgcn_exp2f(__builtin_fmaf(s[kt][rt][i], scale, -base));
        psum += p[i];
      }
      pk[kt][0] = pack_bf16x2(p[0], p[1]);
      pk[kt][1] = pack_bf16x2(p[2], p[3]);
    }
    pb[0][rt] = as_bf16x8(make_uint4(pk[0][0], pk[0][1], pk[1][0], pk[1][1]));
    pb[1][rt] = as_bf16x8(make_uint4(pk[2][0], pk[2][1], pk[3][0], pk[3][1]));
    as.l[rt] += psum;
  }
  // O^T += V^T P^T over the 64 keys (two 32-key steps).
#pragma unroll
  for (int h = 0; h < 2; ++h) {
#pragma unroll
    for (int dt = 0; dt < D / 16; ++dt) {
      const uint16_t *vrow = &sm.vt[(dt * 16 + (lane & 15)) * VSTR + h * 32 + (lane >> 4) * 4];
      const uint2 lo = *reinterpret_cast<const uint2 *>(vrow);
      const uint2 hi = *reinterpret_cast<const uint2 *>(vrow + 16);
      const bf16x8 vf = as_bf16x8(make_uint4(lo.x, lo.y, hi.x, hi.y));
      as.o[0][dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vf, pb[h][0], as.o[0][dt], 0, 0, 0);
      as.o[1][dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vf, pb[h][1], as.o[1][dt], 0, 0, 0);
    }
  }
}

template <int D, int NW>
__global__ __launch_bounds__(NW * 64) __attribute__((amdgpu_waves_per_eu(2)))
void k_attn_prefill(kvm_layer L, PrefillAttnArgs A, int chunk_begin, int qtiles, int n_chunks,
                    ChunkTable table) {
  constexpr int NT = NW * 64, BM = NW * 32;
  __shared__ __attribute__((aligned(16))) AttnSmem<D> sm[2];
  const int C = int(L.chunk_len), n = int(L.n_bswa_chunks);
  const int Hq = int(L.q_heads), Hkv = int(L.kv_heads);
  // XCD-contiguous renumbering of the 1-D grid: logical order (q row, chunk, q tile).
  const int N = gridDim.x;
  const int x = blockIdx.x % kXcds, j = blockIdx.x / kXcds;
  const int q8 = N / kXcds, r8 = N % kXcds;
  const int logical = x * q8 + min(x, r8) + j;
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
    const float tau = st ? tau_s : tau_f;
    const bool do_scale = tau != 1.0f;
    const bool causal = !st;
    const int nb = (nkeys + BN - 1) / BN;
    __syncthreads();  // both buffers are free
    {
      Stage<D, NT> sg;
      const int nv = min(BN, nkeys);
      stage_load<D, NT>(sg, key_rsrc(kp, kstride, nv), kstride_b, key_rsrc(vp, vstride, nv), vstride_b);
      stage_store<D, NT>(sm[0], sg, tau, do_scale);
    }
    __syncthreads();
#pragma unroll 1
    for (int j = 0; j < nb; ++j) {
      const int j0 = j * BN;
      const int nvalid = min(BN, nkeys - j0);
      const bool more = j + 1 < nb;
      Stage<D, NT> sg;
      if (more) {
        const int jn = (j + 1) * BN;
        const int nv = min(BN, nkeys - jn);
        stage_load<D, NT>(sg, key_rsrc(kp + int64_t(jn) * kstride, kstride, nv), kstride_b,
                          key_rsrc(vp + int64_t(jn) * vstride, vstride, nv), vstride_b);
      }
      // Causal ranges: position of the block's first key is wb + j0.
      const int64_t qrel64 = causal ? qpos0 - (wb + j0) : int64_t(BN);
      const int qrel = int(min(max(qrel64, int64_t(-64)), int64_t(BN)));
      const bool masked = nvalid < BN || qrel < BN - 1;
      // wave-uniform: skip blocks entirely above the wave's causal diagonal
      if (qrel + 31 >= 0)
        consume_block<D>(sm[j & 1], as, qf, masked, nvalid, causal, qrel, scale);
      if (more) stage_store<D, NT>(sm[(j + 1) & 1], sg, tau, do_scale);
      __syncthreads();
    }
  }

  // Normalise and store: lane holds dv = dt*16 + 4*(lane/16) + i of row lane%16.
  uint16_t *obase = static_cast<uint16_t *>(A.out) + b * A.o_sb + hq * A.o_sh;
#pragma unroll
  for (int rt = 0; rt < 2; ++rt) {
    float l = as.l[rt];
    l += __shfl_xor(l, 16);
    l += __shfl_xor(l, 32);
    const float inv = 1.0f / l;
    const int64_t t = qpos0 + rt * 16 + (lane & 15);
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

template <int D, int NW>
hipError_t launch_nw(const kvm_layer &L, const PrefillAttnArgs &a, int64_t chunk_begin,
                     int64_t n_chunks, const ChunkTable &table, hipStream_t stream) {
  const int qtiles = int((L.chunk_len + NW * 32 - 1) / (NW * 32));
  const int64_t n_wg = n_chunks * qtiles * L.batch * L.q_heads;
  const dim3 grid{unsigned(n_wg), 1u, 1u};
  hipLaunchKernelGGL((k_attn_prefill<D, NW>), grid, dim3(NW * 64), 0, stream, L, a,
                     int(chunk_begin), qtiles, int(n_chunks), table);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_prefill_attention(const kvm_layer &L, const PrefillAttnArgs &a,
                                    int64_t chunk_begin, int64_t n_chunks,
                                    const ChunkTable &table, hipStream_t stream) {
  if (n_chunks <= 0) return hipSuccess;
  const bool wide = L.chunk_len >= 256;
  if (L.head_dim == 128)
    return wide ? launch_nw<128, 8>(L, a, chunk_begin, n_chunks, table, stream)
                : launch_nw<128, 4>(L, a, chunk_begin, n_chunks, table, stream);
  return wide ? launch_nw<64, 8>(L, a, chunk_begin, n_chunks, table, stream)
              : launch_nw<64, 4>(L, a, chunk_begin, n_chunks, table, stream);
}

}  // namespace kvm
