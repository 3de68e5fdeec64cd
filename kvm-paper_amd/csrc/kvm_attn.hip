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
// Workgroup = 4 waves = 128 queries of one (batch, q_head); each wave owns
// 32 queries (two 16-row MFMA tiles).  Keys stream through LDS in blocks of
// 64: K row-major (times temperature, rounded to bf16, as the reference
// does), V transposed.  Scores are computed transposed, S^T = K Q^T, with
// v_mfma_f32_16x16x32_bf16, so that each lane holds 4 consecutive keys of one
// query row: the P^T tiles feed the O^T = V^T P^T product directly as the B
// operand (the key order inside a 32-key step is permuted identically in the
// A operand, which leaves the sum unchanged).  Online softmax in fp32
// registers with exp2; P rounded to bf16 for the PV product.
//
// VALU budget (the limiter next to MFMA on CDNA): bf16 packing uses the
// hardware v_cvt_pk_bf16_f32, exp2 the raw v_exp_f32, the softmax scale is
// folded into one fma per score, masks are applied only on tail / diagonal
// blocks, the O rescale is skipped when no row maximum of the wave moved,
// and a wave skips 32-key halves that lie entirely above its causal
// diagonal.  Latency: two LDS buffers (one barrier per block; the next
// block is fetched while the current one is multiplied) and a single
// inlined copy of the pipeline for both key ranges keep the kernel under
// 256 VGPRs, so two workgroups share a CU and cover each other's waits.
// Workgroups are renumbered so that each XCD (dispatch is round-robin over
// the 8 XCDs) runs a contiguous range of (head, chunk) tiles: the window
// keys shared by neighbouring chunks stay in that XCD's L2.

#include "kvm_device.hpp"
#include "kvm_internal.hpp"

namespace kvm {
namespace {

constexpr int BM = 128;  // queries per workgroup
constexpr int BN = 64;   // keys per block
constexpr float kLog2e = 1.4426950408889634f;
constexpr int kXcds = 8;

typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));

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

// Register staging of one K/V block: each thread owns KPT 16-byte pieces of
// K (key p / (D/8), dims 8 * (p % (D/8))) and one 4-key x 8-dim piece of V.
template <int D>
struct Stage {
  static constexpr int KPT = BN * (D / 8) / 256;  // K pieces per thread
  static constexpr int VUNITS = (BN / 4) * (D / 8);
  uint4 k[KPT];
  uint4 v[4];
};

template <int D>
__device__ __forceinline__ void stage_load(Stage<D> &sg,
                                           const uint16_t *__restrict__ kp,
                                           int64_t kstride,
                                           const uint16_t *__restrict__ vp,
                                           int64_t vstride, int nvalid) {
  const int tid = threadIdx.x;
#pragma unroll
  for (int i = 0; i < Stage<D>::KPT; ++i) {
    const int p = tid + i * 256;
    const int key = p / (D / 8), part = p % (D / 8);
    sg.k[i] = key < nvalid
                  ? *reinterpret_cast<const uint4 *>(kp + key * kstride + part * 8)
                  : make_uint4(0, 0, 0, 0);
  }
  if (tid < Stage<D>::VUNITS) {
    const int kg = tid % (BN / 4), dg = tid / (BN / 4);
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int key = kg * 4 + r;
      sg.v[r] = key < nvalid ? *reinterpret_cast<const uint4 *>(
                                   vp + key * vstride + dg * 8)
                             : make_uint4(0, 0, 0, 0);
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

template <int D>
__device__ __forceinline__ void stage_store(AttnSmem<D> &sm,
                                            const Stage<D> &sg, float tau) {
  constexpr int KSTR = AttnSmem<D>::KSTR, VSTR = AttnSmem<D>::VSTR;
  const int tid = threadIdx.x;
#pragma unroll
  for (int i = 0; i < Stage<D>::KPT; ++i) {
    const int p = tid + i * 256;
    const int key = p / (D / 8), part = p % (D / 8);
    float x[8];
    unpack8(sg.k[i], x);
    uint4 w;
    w.x = pack_bf16x2(x[0] * tau, x[1] * tau);
    w.y = pack_bf16x2(x[2] * tau, x[3] * tau);
    w.z = pack_bf16x2(x[4] * tau, x[5] * tau);
    w.w = pack_bf16x2(x[6] * tau, x[7] * tau);
    *reinterpret_cast<uint4 *>(&sm.k[key * KSTR + part * 8]) = w;
  }
  if (tid < Stage<D>::VUNITS) {
    const int kg = tid % (BN / 4), dg = tid / (BN / 4);
    const uint32_t a[4][4] = {{sg.v[0].x, sg.v[0].y, sg.v[0].z, sg.v[0].w},
                              {sg.v[1].x, sg.v[1].y, sg.v[1].z, sg.v[1].w},
                              {sg.v[2].x, sg.v[2].y, sg.v[2].z, sg.v[2].w},
                              {sg.v[3].x, sg.v[3].y, sg.v[3].z, sg.v[3].w}};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      // dims 2j (low halves) and 2j+1 (high halves) of keys kg*4 .. kg*4+3
      uint2 lo, hi;
      lo.x = lo_lo(a[0][j], a[1][j]);
      lo.y = lo_lo(a[2][j], a[3][j]);
      hi.x = hi_hi(a[0][j], a[1][j]);
      hi.y = hi_hi(a[2][j], a[3][j]);
      *reinterpret_cast<uint2 *>(&sm.vt[(dg * 8 + 2 * j) * VSTR + kg * 4]) = lo;
      *reinterpret_cast<uint2 *>(&sm.vt[(dg * 8 + 2 * j + 1) * VSTR + kg * 4]) = hi;
    }
  }
}

template <int D>
struct AttnState {
  f32x4 o[2][D / 16];  // O^T tiles [row tile][dv tile]
  float m[2];          // running max of scaled scores (log2 domain)
  float l[2];          // lane-partial running sum
};

// Online-softmax update with 32 keys (half of a staged block, key offset
// k0 in the block).  Masked path: keys >= nvalid, or causal keys
// kpos0 + key > row (kpos0 < 0: memory slots, never causal).
template <int D>
__device__ __forceinline__ void consume_half(const AttnSmem<D> &sm, int k0,
                                             AttnState<D> &as,
                                             const bf16x8 (&qf)[2][D / 32],
                                             bool masked, int nvalid,
                                             int64_t kpos0, int64_t qpos0,
                                             float scale) {
  constexpr int KSTR = AttnSmem<D>::KSTR, VSTR = AttnSmem<D>::VSTR;
  const int lane = threadIdx.x & 63;
  f32x4 s[2][2];
#pragma unroll
  for (int kt = 0; kt < 2; ++kt) {
    s[kt][0] = f32x4{0.f, 0.f, 0.f, 0.f};
    s[kt][1] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < D / 32; ++ks) {
      const bf16x8 a = as_bf16x8(*reinterpret_cast<const uint4 *>(
          &sm.k[(k0 + kt * 16 + (lane & 15)) * KSTR + ks * 32 + (lane >> 4) * 8]));
      s[kt][0] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, qf[0][ks], s[kt][0], 0, 0, 0);
      s[kt][1] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, qf[1][ks], s[kt][1], 0, 0, 0);
    }
  }
  bf16x8 pb[2];
  bool moved = false;
  float alpha[2];
#pragma unroll
  for (int rt = 0; rt < 2; ++rt) {
    if (masked) {
      const int64_t qpos = qpos0 + rt * 16 + (lane & 15);
#pragma unroll
      for (int kt = 0; kt < 2; ++kt)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int key = k0 + kt * 16 + (lane >> 4) * 4 + i;
          if (key >= nvalid || (kpos0 >= 0 && kpos0 + key > qpos)) s[kt][rt][i] = -INFINITY;
        }
    }
    float mx = fmaxf(fmaxf(fmaxf(s[0][rt][0], s[0][rt][1]), fmaxf(s[0][rt][2], s[0][rt][3])),
                     fmaxf(fmaxf(s[1][rt][0], s[1][rt][1]), fmaxf(s[1][rt][2], s[1][rt][3])));
    mx = fmaxf(mx, __shfl_xor(mx, 16));
    mx = fmaxf(mx, __shfl_xor(mx, 32));
    const float m_new = fmaxf(as.m[rt], mx * scale);
    moved |= m_new != as.m[rt];
    const float base = (m_new == -INFINITY) ? 0.f : m_new;
    alpha[rt] = (as.m[rt] == -INFINITY) ? 0.f : __builtin_amdgcn_exp2f(as.m[rt] - base);
    float psum = 0.f;
    uint32_t pk[2][2];
#pragma unroll
    for (int kt = 0; kt < 2; ++kt) {
      float p[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        p[i] = __builtin_amdgcn_exp2f(__builtin_fmaf(s[kt][rt][i], scale, -base));
        psum += p[i];
      }
      pk[kt][0] = pack_bf16x2(p[0], p[1]);
      pk[kt][1] = pack_bf16x2(p[2], p[3]);
    }
    pb[rt] = as_bf16x8(make_uint4(pk[0][0], pk[0][1], pk[1][0], pk[1][1]));
    as.l[rt] = as.l[rt] * alpha[rt] + psum;
    as.m[rt] = m_new;
  }
  // Rescale O only when some row maximum of the wave moved.
  if (__ballot(moved)) {
#pragma unroll
    for (int rt = 0; rt < 2; ++rt)
#pragma unroll
      for (int dt = 0; dt < D / 16; ++dt) as.o[rt][dt] *= alpha[rt];
  }
  // O^T += V^T P^T over these 32 keys.
#pragma unroll
  for (int dt = 0; dt < D / 16; ++dt) {
    const uint16_t *vrow = &sm.vt[(dt * 16 + (lane & 15)) * VSTR + k0 + (lane >> 4) * 4];
    const uint2 lo = *reinterpret_cast<const uint2 *>(vrow);
    const uint2 hi = *reinterpret_cast<const uint2 *>(vrow + 16);
    const bf16x8 a = as_bf16x8(make_uint4(lo.x, lo.y, hi.x, hi.y));
    as.o[0][dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, pb[0], as.o[0][dt], 0, 0, 0);
    as.o[1][dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, pb[1], as.o[1][dt], 0, 0, 0);
  }
}

template <int D>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2)))
void k_attn_prefill(kvm_layer L, PrefillAttnArgs A, int chunk_begin,
                    int qtiles, int n_chunks, ChunkTable table) {
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
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
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
    const float tau = st ? tau_s : tau_f;
    const int64_t kpos0 = st ? -1 : wb;
    const int nb = (nkeys + BN - 1) / BN;
    __syncthreads();  // both buffers are free
    {
      Stage<D> sg;
      stage_load<D>(sg, kp, kstride, vp, vstride, min(BN, nkeys));
      stage_store<D>(sm[0], sg, tau);
    }
    __syncthreads();
#pragma unroll 1
    for (int j = 0; j < nb; ++j) {
      const int j0 = j * BN;
      const int nvalid = min(BN, nkeys - j0);
      const int64_t kb = kpos0 >= 0 ? kpos0 + j0 : -1;
      const bool more = j + 1 < nb;
      Stage<D> sg;
      if (more) {
        const int jn = (j + 1) * BN;
        stage_load<D>(sg, kp + int64_t(jn) * kstride, kstride, vp + int64_t(jn) * vstride,
                      vstride, min(BN, nkeys - jn));
      }
      const bool masked = nvalid < BN || (kb >= 0 && kb + BN - 1 > qpos0);
#pragma unroll 1
      for (int h = 0; h < 2; ++h) {
        // wave-uniform: skip halves above the wave's causal diagonal / past the tail
        const bool live = h * 32 < nvalid && !(kb >= 0 && kb + h * 32 > qpos0 + 31);
        if (live) consume_half<D>(sm[j & 1], h * 32, as, qf, masked, nvalid, kb, qpos0, scale);
      }
      if (more) stage_store<D>(sm[(j + 1) & 1], sg, tau);
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

}  // namespace

hipError_t launch_prefill_attention(const kvm_layer &L,
                                    const PrefillAttnArgs &a,
                                    int64_t chunk_begin, int64_t n_chunks,
                                    const ChunkTable &table,
                                    hipStream_t stream) {
  if (n_chunks <= 0) return hipSuccess;
  const int qtiles = int((L.chunk_len + BM - 1) / BM);
  const int64_t n_wg = n_chunks * qtiles * L.batch * L.q_heads;
  const dim3 grid{unsigned(n_wg), 1u, 1u};
  if (L.head_dim == 128)
    hipLaunchKernelGGL(k_attn_prefill<128>, grid, dim3(256), 0, stream, L, a,
                       int(chunk_begin), qtiles, int(n_chunks), table);
  else
    hipLaunchKernelGGL(k_attn_prefill<64>, grid, dim3(256), 0, stream, L, a,
                       int(chunk_begin), qtiles, int(n_chunks), table);
  return hipGetLastError();
}

}  // namespace kvm
