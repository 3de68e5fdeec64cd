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
// One workgroup owns RPW slots of one row and holds their sums and gradient
// accumulators in registers (D/8 lanes per slot row): a forward scan over the
// updates rebuilds the final sums, a reverse scan accumulates H and undoes
// each update's merges.  Every token is routed to exactly one slot, so each
// output row has exactly one writer (no atomics).

#include "kvm_device.hpp"
#include "kvm_internal.hpp"

namespace kvm {
namespace {

constexpr int kThreads = 256;
constexpr int kMaxChunk = 4096;

__device__ __forceinline__ void load8f(const float *p, float (&x)[8]) {
  const float4 a = *reinterpret_cast<const float4 *>(p), b = *reinterpret_cast<const float4 *>(p + 4);
  x[0] = a.x; x[1] = a.y; x[2] = a.z; x[3] = a.w;
  x[4] = b.x; x[5] = b.y; x[6] = b.z; x[7] = b.w;
}
__device__ __forceinline__ void store8f(float *p, const float (&x)[8]) {
  *reinterpret_cast<float4 *>(p) = make_float4(x[0], x[1], x[2], x[3]);
  *reinterpret_cast<float4 *>(p + 4) = make_float4(x[4], x[5], x[6], x[7]);
}

template <int D>
__global__ __launch_bounds__(kThreads) void k_state_bwd(StateBwdArgs A, UpdTable U, float *__restrict__ dln_part) {
  constexpr int GL = D / 8;            // lanes per slot row
  constexpr int RPW = kThreads / GL;   // slot rows per workgroup
  __shared__ int32_t rt[kMaxChunk];    // route_log of the current update
  __shared__ int32_t ap[kMaxChunk];    // append_log of the current update
  __shared__ float red[kThreads / 64][2][D];
  const int tid = threadIdx.x, part = tid % GL, lane = tid & 63, wave = tid >> 6;
  const int row = blockIdx.y;
  const int j = blockIdx.x * RPW + tid / GL;  // this thread's slot
  const int C = int(A.chunk_len), T = int(A.T), L0 = int(A.L0), nu = int(A.n_updates);
  const int64_t rowT = int64_t(row) * T;
  const float eps = float(A.ln_eps);
  float w[8];
  load8f(A.ln_w + part * 8, w);
  auto tb_of = [&](int u) { return U.token_begin[u]; };
  auto before_of = [&](int u) { return U.state_before[u]; };
  auto napp_of = [&](int u) { return U.n_append[u]; };
  auto stage = [&](int u) {
    const int64_t o = (int64_t(u) * A.rows + row) * C;
    __syncthreads();
    for (int t = tid; t < C; t += kThreads) {
      rt[t] = A.route_log[o + t];
      ap[t] = A.append_log[o + t];
    }
    __syncthreads();
  };
  auto ld_row = [&](const float *base, int64_t r, float (&x)[8]) { load8f(base + r * D + part * 8, x); };

  // ---- forward scan: final fp32 sums of my slot, and its vlen.
  float sk[8], sv[8];
  float vlen = 0.f;
  if (j < L0) {
    ld_row(A.ik, int64_t(row) * L0 + j, sk);
    ld_row(A.iv, int64_t(row) * L0 + j, sv);
    vlen = A.ivl[int64_t(row) * L0 + j];
  } else {
#pragma unroll
    for (int e = 0; e < 8; ++e) sk[e] = sv[e] = 0.f;
  }
  for (int u = 0; u < nu; ++u) {
    stage(u);
    const int tb = tb_of(u);
    float dk[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f}, dv[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    for (int t = 0; t < C; ++t) {
      if (rt[t] != j) continue;
      float xk[8], xv[8];
      if (ap[t]) {  // the slot's base row (appended before this update's merges)
        ld_row(A.ak, rowT + tb + t, sk);
        ld_row(A.av, rowT + tb + t, sv);
        vlen = A.avl[rowT + tb + t];
      } else {
        ld_row(A.mk, rowT + tb + t, xk);
        ld_row(A.mv, rowT + tb + t, xv);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          dk[e] += xk[e];
          dv[e] += xv[e];
        }
      }
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
  float accl = 0.f;  // d vlen of my slot (row-reduced, replicated over the row's lanes)
  for (int s = nu; s >= 0; --s) {
    const int len = s == 0 ? L0 : before_of(s - 1) + napp_of(s - 1);
    if (j < len) {
      // Local backward of snapshot s at my slot.
      const int64_t so = ((int64_t(s) * A.rows + row) * A.max_state_len + j) * D + part * 8;
      load8f(A.d_snap_k + so, gk);
      load8f(A.d_snap_v + so, gv);
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
      float nn = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) nn += sv[e] * sv[e];
      const float nrm = sqrtf(group_sum<GL>(nn));
      const float inv = nrm > 0.f ? 1.0f / nrm : 0.f;
      float gs = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) gs += gv[e] * sv[e] * inv;
      gs = group_sum<GL>(gs);
      accl += gs;
#pragma unroll
      for (int e = 0; e < 8; ++e) accv[e] += vlen * inv * (gv[e] - gs * sv[e] * inv);
    }
    if (s == 0) break;
    // Undo update s - 1, which built snapshot s from snapshot s - 1.
    const int u = s - 1;
    stage(u);
    const int tb = tb_of(u);
    for (int t = 0; t < C; ++t) {
      if (rt[t] != j) continue;
      const int64_t o = (rowT + tb + t) * D + part * 8;
      if (ap[t]) {
        store8f(A.d_ak + o, acck);
        store8f(A.d_av + o, accv);
        if (part == 0) A.d_avl[rowT + tb + t] = accl;
      } else {
        store8f(A.d_mk + o, acck);
        store8f(A.d_mv + o, accv);
        float xk[8], xv[8];
        ld_row(A.mk, rowT + tb + t, xk);
        ld_row(A.mv, rowT + tb + t, xv);
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          sk[e] -= xk[e];
          sv[e] -= xv[e];
        }
      }
    }
    if (j >= before_of(u) && j < before_of(u) + napp_of(u)) {  // the slot did not exist before
#pragma unroll
      for (int e = 0; e < 8; ++e) acck[e] = accv[e] = sk[e] = sv[e] = 0.f;
      accl = 0.f;
    }
  }
  if (j < L0) {
    const int64_t o = (int64_t(row) * L0 + j) * D + part * 8;
    store8f(A.d_ik + o, acck);
    store8f(A.d_iv + o, accv);
    if (part == 0) A.d_ivl[int64_t(row) * L0 + j] = accl;
  }
  // LayerNorm parameter gradients: sum over my slots, then this workgroup's partial.
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
      red[wave][0][part * 8 + e] = x;
      red[wave][1][part * 8 + e] = y;
    }
  }
  __syncthreads();
  for (int i = tid; i < 2 * D; i += kThreads) {
    const int which = i / D, f = i % D;
    float a = 0.f;
    for (int w2 = 0; w2 < kThreads / 64; ++w2) a += red[w2][which][f];
    dln_part[(int64_t(blockIdx.y) * gridDim.x + blockIdx.x) * 2 * D + i] = a;
  }
}

template <int D>
__global__ void k_state_bwd_ln(const float *part, int nwg, float *out) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= 2 * D) return;
  float a = 0.f;
  for (int w = 0; w < nwg; ++w) a += part[int64_t(w) * 2 * D + i];
  out[i] = a;
}

template <int D>
hipError_t launch_d(const StateBwdArgs &a, const UpdTable &sched, float *part, hipStream_t s) {
  constexpr int RPW = kThreads / (D / 8);
  const dim3 grid(unsigned((a.max_state_len + RPW - 1) / RPW), unsigned(a.rows));
  hipLaunchKernelGGL((k_state_bwd<D>), grid, dim3(kThreads), 0, s, a, sched, part);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL((k_state_bwd_ln<D>), dim3((2 * D + 127) / 128), dim3(128), 0, s, part,
                     int(grid.x * grid.y), a.d_ln);
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
  if (a.head_dim == 128) return launch_d<128>(a, sched, part, stream);
  return launch_d<64>(a, sched, part, stream);
}

}  // namespace kvm
