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

#include "kvm_device.hpp"
#include "kvm_internal.hpp"

namespace kvm {
namespace {

constexpr int BM = 128;  // queries per workgroup
constexpr int BN = 64;   // keys per block
constexpr float kLog2e = 1.4426950408889634f;

template <int D>
struct AttnSmem {
  static constexpr int KSTR = D + 8;   // K row stride (elements)
  static constexpr int VSTR = BN + 8;  // V^T row stride (elements)
  uint16_t k[BN * KSTR];
  uint16_t vt[D * VSTR];
};

template <int D>
struct AttnState {
  f32x4 o[2][D / 16];  // O^T tiles [row tile][dv tile]
  float m[2];          // running max (log2 domain) of row rt*16 + lane%16
  float l[2];          // lane-partial running sum
};

// One block of up to BN keys: stage K (x tau, bf16) and V^T in LDS, then
// update the online softmax of the wave's 32 query rows.
// kpos0: absolute position of key 0 (window keys) or -1 (memory slots,
// never masked causally).  qpos0: position of the wave's first query row.
template <int D>
__device__ __forceinline__ void attend_block(
    AttnSmem<D> &sm, AttnState<D> &as, const bf16x8 (&qf)[2][D / 32],
    const uint16_t *__restrict__ kp, int64_t kstride,
    const uint16_t *__restrict__ vp, int64_t vstride, int nvalid, float tau,
    int64_t kpos0, int64_t qpos0, float scale) {
  constexpr int KSTR = AttnSmem<D>::KSTR, VSTR = AttnSmem<D>::VSTR;
  const int tid = threadIdx.x, lane = tid & 63;
  __syncthreads();
  for (int p = tid; p < BN * (D / 8); p += 256) {
    const int key = p / (D / 8), part = p % (D / 8);
    float x[8];
    if (key < nvalid) {
      load8(kp + key * kstride + part * 8, x);
#pragma unroll
      for (int i = 0; i < 8; ++i) x[i] = rbf(x[i] * tau);
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i) x[i] = 0.f;
    }
    store8(&sm.k[key * KSTR + part * 8], x);
  }
  for (int p = tid; p < (BN / 4) * (D / 8); p += 256) {
    const int kg = p % (BN / 4), dg = p / (BN / 4);
    uint16_t e[4][8];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int key = kg * 4 + r;
      uint4 u = make_uint4(0, 0, 0, 0);
      if (key < nvalid)
        u = *reinterpret_cast<const uint4 *>(vp + key * vstride + dg * 8);
      e[r][0] = u.x & 0xffff; e[r][1] = u.x >> 16;
      e[r][2] = u.y & 0xffff; e[r][3] = u.y >> 16;
      e[r][4] = u.z & 0xffff; e[r][5] = u.z >> 16;
      e[r][6] = u.w & 0xffff; e[r][7] = u.w >> 16;
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      uint2 w;
      w.x = uint32_t(e[0][i]) | (uint32_t(e[1][i]) << 16);
      w.y = uint32_t(e[2][i]) | (uint32_t(e[3][i]) << 16);
      *reinterpret_cast<uint2 *>(&sm.vt[(dg * 8 + i) * VSTR + kg * 4]) = w;
    }
  }
  __syncthreads();

  // S^T = K Q^T: s[kt][rt][i] = score(key kt*16 + 4*(lane/16) + i,
  //                                   row  rt*16 + lane%16)
  f32x4 s[4][2];
#pragma unroll
  for (int kt = 0; kt < 4; ++kt) {
    s[kt][0] = f32x4{0.f, 0.f, 0.f, 0.f};
    s[kt][1] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < D / 32; ++ks) {
      const bf16x8 a = as_bf16x8(*reinterpret_cast<const uint4 *>(
          &sm.k[(kt * 16 + (lane & 15)) * KSTR + ks * 32 + (lane >> 4) * 8]));
      s[kt][0] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, qf[0][ks], s[kt][0], 0, 0, 0);
      s[kt][1] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, qf[1][ks], s[kt][1], 0, 0, 0);
    }
  }

  bf16x8 pb[2][BN / 32];
#pragma unroll
  for (int rt = 0; rt < 2; ++rt) {
    const int64_t qpos = qpos0 + rt * 16 + (lane & 15);
    float mx = -INFINITY;
#pragma unroll
    for (int kt = 0; kt < 4; ++kt) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int key = kt * 16 + (lane >> 4) * 4 + i;
        float x = s[kt][rt][i] * scale;
        if (key >= nvalid || (kpos0 >= 0 && kpos0 + key > qpos)) x = -INFINITY;
        s[kt][rt][i] = x;
        mx = fmaxf(mx, x);
      }
    }
    mx = fmaxf(mx, __shfl_xor(mx, 16));
    mx = fmaxf(mx, __shfl_xor(mx, 32));
    const float m_new = fmaxf(as.m[rt], mx);
    const float base = (m_new == -INFINITY) ? 0.f : m_new;
    const float alpha = (as.m[rt] == -INFINITY) ? 0.f : exp2f(as.m[rt] - base);
    float psum = 0.f;
    uint32_t pk[4][2];
#pragma unroll
    for (int kt = 0; kt < 4; ++kt) {
      float p[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        p[i] = exp2f(s[kt][rt][i] - base);
        psum += p[i];
      }
      pk[kt][0] = f2bf(p[0]) | (f2bf(p[1]) << 16);
      pk[kt][1] = f2bf(p[2]) | (f2bf(p[3]) << 16);
    }
#pragma unroll
    for (int ks = 0; ks < BN / 32; ++ks)
      pb[rt][ks] = as_bf16x8(make_uint4(pk[2 * ks][0], pk[2 * ks][1],
                                        pk[2 * ks + 1][0], pk[2 * ks + 1][1]));
    as.l[rt] = as.l[rt] * alpha + psum;
    as.m[rt] = m_new;
#pragma unroll
    for (int dt = 0; dt < D / 16; ++dt) as.o[rt][dt] *= alpha;
  }

  // O^T += V^T P^T
#pragma unroll
  for (int dt = 0; dt < D / 16; ++dt) {
#pragma unroll
    for (int ks = 0; ks < BN / 32; ++ks) {
      const uint16_t *vrow = &sm.vt[(dt * 16 + (lane & 15)) * VSTR + ks * 32 + (lane >> 4) * 4];
      const uint2 lo = *reinterpret_cast<const uint2 *>(vrow);
      const uint2 hi = *reinterpret_cast<const uint2 *>(vrow + 16);
      const bf16x8 a = as_bf16x8(make_uint4(lo.x, lo.y, hi.x, hi.y));
      as.o[0][dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, pb[0][ks], as.o[0][dt], 0, 0, 0);
      as.o[1][dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, pb[1][ks], as.o[1][dt], 0, 0, 0);
    }
  }
}

template <int D>
__global__ __launch_bounds__(256) void k_attn_prefill(
    kvm_layer L, PrefillAttnArgs A, int chunk_begin, int qtiles,
    ChunkTable table) {
  __shared__ __attribute__((aligned(16))) AttnSmem<D> sm;
  const int C = int(L.chunk_len), n = int(L.n_bswa_chunks);
  const int Hq = int(L.q_heads), Hkv = int(L.kv_heads);
  const int qrow = blockIdx.y;
  const int b = qrow / Hq, hq = qrow % Hq;
  const int hk = hq / (Hq / Hkv);
  const int kvrow = b * Hkv + hk;
  const int c_local = blockIdx.x / qtiles, qt = blockIdx.x % qtiles;
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

  // Memory slots.
  const int S = table.state_len[c_local];
  if (m >= n && S > 0) {
    const int64_t soff = int64_t(table.snap_slot[c_local]) * A.snap_stride +
                         int64_t(kvrow) * A.snap_cap * D;
    const uint16_t *sk = A.snap_k + soff;
    const uint16_t *sv = A.snap_v + soff;
    for (int j0 = 0; j0 < S; j0 += BN)
      attend_block<D>(sm, as, qf, sk + int64_t(j0) * D, D, sv + int64_t(j0) * D, D,
                      min(BN, S - j0), tau_s, -1, qpos0, scale);
  }
  // Window tokens [wb, q_hi), causal.
  const int64_t wb = max(int64_t(0), int64_t(m - n + 1) * C);
  const uint16_t *kb = static_cast<const uint16_t *>(A.kv.k) + b * A.kv.k_sb + hk * A.kv.k_sh;
  const uint16_t *vb = static_cast<const uint16_t *>(A.kv.v) + b * A.kv.v_sb + hk * A.kv.v_sh;
  for (int64_t k0 = wb; k0 < q_hi; k0 += BN)
    attend_block<D>(sm, as, qf, kb + k0 * A.kv.k_st, A.kv.k_st, vb + k0 * A.kv.v_st,
                    A.kv.v_st, int(min(int64_t(BN), q_hi - k0)), tau_f, k0, qpos0,
                    scale);

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
        w.x = f2bf(as.o[rt][dt][0] * inv) | (f2bf(as.o[rt][dt][1] * inv) << 16);
        w.y = f2bf(as.o[rt][dt][2] * inv) | (f2bf(as.o[rt][dt][3] * inv) << 16);
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
  dim3 grid(unsigned(n_chunks * qtiles), unsigned(L.batch * L.q_heads));
  if (L.head_dim == 128)
    hipLaunchKernelGGL(k_attn_prefill<128>, grid, dim3(256), 0, stream, L, a,
                       int(chunk_begin), qtiles, table);
  else
    hipLaunchKernelGGL(k_attn_prefill<64>, grid, dim3(256), 0, stream, L, a,
                       int(chunk_begin), qtiles, table);
  return hipGetLastError();
}

}  // namespace kvm
