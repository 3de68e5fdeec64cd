// Single-token KVM decode attention on gfx950.
//
// Reference semantics: model/kvm_mixer.py:572-713 (forward_single, attention
// through _attend_with_state_and_bswa :194-229 with q_len = 1) and the
// Triton kernel it replaces, model/kernels/kvm_triton_decode.py:175-284
// (one program per (batch, q_head), serial scan).
//
// Here the key rows [memory slots ; window ring rows] of every
// (batch, kv_head) are split into segments of 256 rows.  A workgroup (4
// waves) owns one segment of one kv row and serves every query head of that
// kv head it is launched for (the GQA group shares each K/V read).  A wave
// reads 64 rows with D/8 lanes per row, i.e. 4 (D=128) or 8 (D=64) whole
// rows per 16-byte-per-lane load: each load instruction covers 1 KiB of
// contiguous HBM.  Scores, the wave softmax and the PV accumulation are in
// fp32; the 4 waves merge (max, sum, acc) through LDS, and a second kernel
// merges the segments in a fixed order (deterministic split-K).

#include <mutex>

#include "kvm_device.hpp"
#include "kvm_internal.hpp"
#include "kvm_seq.hpp"

namespace kvm {
namespace {

constexpr int kRowsPerWave = 64;
constexpr int kWaves = 4;
constexpr int kSegRows = kRowsPerWave * kWaves;
constexpr float kLog2e = 1.4426950408889634f;

// Non-temporal 16-byte load: every K/V row is read once per step, and the
// streaming path sustains ~7.2 TB/s on MI355X against ~6.4 TB/s for plain
// loads of the same 1.5 GB.
__device__ __forceinline__ uint4 ld_stream16(const uint16_t *p) {
  typedef unsigned u4 __attribute__((ext_vector_type(4)));
  const u4 x = __builtin_nontemporal_load(reinterpret_cast<const u4 *>(p));
  return make_uint4(x[0], x[1], x[2], x[3]);
}

template <int D, int GQ>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(GQ == 1 ? 3 : 2))) void k_decode_partial(
    kvm_layer L, const uint16_t *__restrict__ q, int64_t q_sb, int64_t q_sh,
    const uint16_t *__restrict__ sk, const uint16_t *__restrict__ sv,
    int64_t cap, int active, const uint16_t *__restrict__ rk,
    const uint16_t *__restrict__ rv, int64_t ring_cap, int64_t ring_start,
    int recent_len, int nseg, float *__restrict__ part_acc,
    float *__restrict__ part_ml, const int32_t *__restrict__ ctl, int pending, kvm_seq fresh,
    uint16_t *ring_k_out, uint16_t *ring_v_out, uint16_t *ring_g_out) {
  constexpr int G = D / 8;             // lanes per key row
  constexpr int RPS = 64 / G;          // rows per wave step
  constexpr int STEPS = kRowsPerWave / RPS;
  __shared__ float sm_m[kWaves][GQ], sm_l[kWaves][GQ];
  __shared__ float sm_acc[kWaves][GQ][D];

  const int seg = blockIdx.x;
  const int row = blockIdx.y;
  const int Hq = int(L.q_heads), Hkv = int(L.kv_heads);
  const int group = Hq / Hkv;
  const int b = row / Hkv, hk = row % Hkv;
  const int hq0 = hk * group + blockIdx.z * GQ;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int sub = lane / G, part = lane % G;
  if (ctl) {  // counters in device memory (graph-captured decode), clamped to the buffers
    active = min(max(ctl[0], 0), int(cap));
    ring_start = ((int64_t(ctl[1]) % ring_cap) + ring_cap) % ring_cap;
    recent_len = min(max(ctl[2] + pending, 0), int(ring_cap));
  }
  const int total = min(active + recent_len, nseg * kSegRows);
  const float scale = kLog2e / sqrtf(float(D));

  float qv[GQ][8], ts[GQ], tf[GQ];
#pragma unroll
  for (int j = 0; j < GQ; ++j) {
    load8(q + b * q_sb + (hq0 + j) * q_sh + part * 8, qv[j]);
    ts[j] = static_cast<const float *>(L.state_temp)[hq0 + j];
    tf[j] = static_cast<const float *>(L.front_temp)[hq0 + j];
  }

  const int r0 = seg * kSegRows + wave * kRowsPerWave;
  const uint16_t *skrow = sk + int64_t(row) * cap * D;
  const uint16_t *svrow = sv + int64_t(row) * cap * D;
  const uint16_t *rkrow = rk + int64_t(row) * ring_cap * D;
  const uint16_t *rvrow = rv + int64_t(row) * ring_cap * D;
  // The newest window row straight from the step's token.  Its ring slot is
  // read by no workgroup of this launch, so the first query-head group of
  // the segment holding it stores the row there from the loaded registers.
  const bool from_fresh = fresh.k != nullptr;  // uniform
  const int fresh_row = active + recent_len - 1;
  const uint16_t *fkrow = from_fresh ? seq_k(fresh, b, hk, 0) : rkrow;
  const uint16_t *fvrow = from_fresh ? seq_v(fresh, b, hk, 0) : rvrow;
  const bool store_fresh = from_fresh && blockIdx.z == 0 && seg == fresh_row / kSegRows;  // uniform
  const int64_t fresh_slot = int64_t(row) * ring_cap + (ring_start + recent_len - 1) % ring_cap;
  uint16_t gate_val = 0;
  if (store_fresh && threadIdx.x == 0)
    gate_val = *(static_cast<const uint16_t *>(fresh.gate) + b * fresh.g_sb + hk * fresh.g_sh);

  // Issue every K and V load of the wave first (2 x STEPS x 16 B per lane).
  uint4 kraw[STEPS], vraw[STEPS];
#pragma unroll
  for (int s = 0; s < STEPS; ++s) {
    const int r = r0 + s * RPS + sub;
    kraw[s] = make_uint4(0, 0, 0, 0);
    vraw[s] = make_uint4(0, 0, 0, 0);
    if (r < total) {
      int64_t o;
      const uint16_t *kb, *vb;
      if (r < active) {
        o = int64_t(r) * D;
        kb = skrow;
        vb = svrow;
      } else if (from_fresh && r == fresh_row) {
        o = 0;
        kb = fkrow;
        vb = fvrow;
      } else {
        o = ((ring_start + (r - active)) % ring_cap) * D;
        kb = rkrow;
        vb = rvrow;
      }
      kraw[s] = ld_stream16(kb + o + part * 8);
      vraw[s] = ld_stream16(vb + o + part * 8);
    }
  }

  // Scores: (key . q) * temperature * scale in fp32, the prefill kernel's form
  // (k_attn_prefill multiplies the head temperature into the fp32 score), so
  // that a decode step after a prefill of T tokens gives the prefill of T + 1
  // tokens' last row.  The reference's Triton kernels round bf16(key *
  // temperature) first (model/kernels/kvm_triton_decode.py:225-228); both
  // forms are the same at temperature 1.
  float sc[GQ][STEPS];
#pragma unroll
  for (int s = 0; s < STEPS; ++s) {
    const int r = r0 + s * RPS + sub;
    float kx[8];
    unpack8(kraw[s], kx);
    if (store_fresh && r == fresh_row)
      *reinterpret_cast<uint4 *>(ring_k_out + fresh_slot * D + part * 8) = kraw[s];
#pragma unroll
    for (int j = 0; j < GQ; ++j) {
      const float tau = r < active ? ts[j] : tf[j];
      float d = 0.f;
#pragma unroll
      for (int i = 0; i < 8; ++i) d += kx[i] * qv[j][i];
      d = group_sum<G>(d);
      sc[j][s] = r < total ? d * (scale * tau) : -INFINITY;
    }
  }

  float m[GQ], l[GQ], acc[GQ][8];
#pragma unroll
  for (int j = 0; j < GQ; ++j) {
    float mx = -INFINITY;
#pragma unroll
    for (int s = 0; s < STEPS; ++s) mx = fmaxf(mx, sc[j][s]);
#pragma unroll
    for (int o = G; o < 64; o <<= 1) mx = fmaxf(mx, __shfl_xor(mx, o));
    m[j] = mx;
    l[j] = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) acc[j][i] = 0.f;
  }
#pragma unroll
  for (int s = 0; s < STEPS; ++s) {
    float vx[8];
    unpack8(vraw[s], vx);
    if (store_fresh && r0 + s * RPS + sub == fresh_row)
      *reinterpret_cast<uint4 *>(ring_v_out + fresh_slot * D + part * 8) = vraw[s];
#pragma unroll
    for (int j = 0; j < GQ; ++j) {
      const float p = (m[j] == -INFINITY) ? 0.f : exp2f(sc[j][s] - m[j]);
      l[j] += p;
#pragma unroll
      for (int i = 0; i < 8; ++i) acc[j][i] += p * vx[i];
    }
  }
  // Reduce over the RPS rows a step holds (lanes with equal `part`).
#pragma unroll
  for (int j = 0; j < GQ; ++j) {
#pragma unroll
    for (int o = G; o < 64; o <<= 1) {
      l[j] += __shfl_xor(l[j], o);
#pragma unroll
      for (int i = 0; i < 8; ++i) acc[j][i] += __shfl_xor(acc[j][i], o);
    }
  }
  if (sub == 0) {
#pragma unroll
    for (int j = 0; j < GQ; ++j) {
#pragma unroll
      for (int i = 0; i < 8; ++i) sm_acc[wave][j][part * 8 + i] = acc[j][i];
      if (part == 0) {
        sm_m[wave][j] = m[j];
        sm_l[wave][j] = l[j];
      }
    }
  }
  __syncthreads();
  if (store_fresh && threadIdx.x == 0) ring_g_out[fresh_slot] = gate_val;
  for (int e = threadIdx.x; e < GQ * D; e += 256) {
    const int j = e / D, d = e % D;
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) M = fmaxf(M, sm_m[w][j]);
    float a = 0.f, s = 0.f;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) {
      const float f = (sm_m[w][j] == -INFINITY) ? 0.f : exp2f(sm_m[w][j] - M);
      a += sm_acc[w][j][d] * f;
      s += sm_l[w][j] * f;
    }
    const int64_t pid = int64_t(b) * Hq + hq0 + j;
    part_acc[(pid * nseg + seg) * D + d] = a;
    if (d == 0) {
      part_ml[(pid * nseg + seg) * 2 + 0] = M;
      part_ml[(pid * nseg + seg) * 2 + 1] = s;
    }
  }
}

// Merge the segments of one (batch, q_head) in segment order.
template <int D>
__global__ __launch_bounds__(D) void k_decode_combine(
    int Hq, int nseg, const float *__restrict__ part_acc,
    const float *__restrict__ part_ml, uint16_t *__restrict__ out,
    int64_t o_sb, int64_t o_sh) {
  const int pid = blockIdx.x;
  const int b = pid / Hq, h = pid % Hq;
  const int d = threadIdx.x;
  const float *ml = part_ml + int64_t(pid) * nseg * 2;
  const float *acc = part_acc + int64_t(pid) * nseg * D + d;
  float M = -INFINITY, a = 0.f, l = 0.f;
  constexpr int kMaxSeg = 16;
  if (nseg <= kMaxSeg) {
    // Every partial loaded at once (one memory round trip), then the same
    // arithmetic in the same segment order as the loop below.
    float m[kMaxSeg], sl[kMaxSeg], x[kMaxSeg];
#pragma unroll
    for (int s = 0; s < kMaxSeg; ++s) {
      m[s] = s < nseg ? ml[2 * s] : -INFINITY;
      sl[s] = s < nseg ? ml[2 * s + 1] : 0.f;
      x[s] = s < nseg ? acc[s * D] : 0.f;
    }
#pragma unroll
    for (int s = 0; s < kMaxSeg; ++s) M = fmaxf(M, m[s]);
#pragma unroll
    for (int s = 0; s < kMaxSeg; ++s) {
      if (s < nseg) {
        const float f = (m[s] == -INFINITY) ? 0.f : exp2f(m[s] - M);
        a += x[s] * f;
        l += sl[s] * f;
      }
    }
  } else {
    for (int s = 0; s < nseg; ++s) M = fmaxf(M, ml[2 * s]);
    for (int s = 0; s < nseg; ++s) {
      const float ms = ml[2 * s];
      const float f = (ms == -INFINITY) ? 0.f : exp2f(ms - M);
      a += acc[s * D] * f;
      l += ml[2 * s + 1] * f;
    }
  }
  out[b * o_sb + h * o_sh + d] = uint16_t(f2bf(a / l));
}

template <int D, int GQ>
hipError_t launch_partial(const kvm_layer &L, const void *q, int64_t q_sb,
                          int64_t q_sh, const kvm_state &st, int64_t active,
                          const void *ring_k, const void *ring_v,
                          int64_t ring_cap, int64_t ring_start,
                          int64_t recent_len, int nseg, float *pacc,
                          float *pml, const int32_t *ctl, int pending, const kvm_seq &fresh,
                          uint16_t *rkw, uint16_t *rvw, uint16_t *rgw, hipStream_t stream) {
  const int group = int(L.q_heads / L.kv_heads);
  dim3 grid(unsigned(nseg), unsigned(L.batch * L.kv_heads),
            unsigned(group / GQ));
  hipLaunchKernelGGL((k_decode_partial<D, GQ>), grid, dim3(256), 0, stream, L,
                     static_cast<const uint16_t *>(q), q_sb, q_sh,
                     static_cast<const uint16_t *>(st.s_k_attn),
                     static_cast<const uint16_t *>(st.s_v_attn), st.capacity,
                     int(active), static_cast<const uint16_t *>(ring_k),
                     static_cast<const uint16_t *>(ring_v), ring_cap,
                     ring_start, int(recent_len), nseg, pacc, pml, ctl, pending, fresh, rkw, rvw,
                     rgw);
  return hipGetLastError();
}

template <int D>
hipError_t launch_partial_d(const kvm_layer &L, const void *q, int64_t q_sb,
                            int64_t q_sh, const kvm_state &st, int64_t active,
                            const void *ring_k, const void *ring_v,
                            int64_t ring_cap, int64_t ring_start,
                            int64_t recent_len, int nseg, float *pacc,
                            float *pml, const int32_t *ctl, int pending, const kvm_seq &fresh,
                            uint16_t *rkw, uint16_t *rvw, uint16_t *rgw, hipStream_t stream) {
  const int64_t group = L.q_heads / L.kv_heads;
#define KVM_PARTIAL(GQ)                                                      \
  launch_partial<D, GQ>(L, q, q_sb, q_sh, st, active, ring_k, ring_v,       \
                        ring_cap, ring_start, recent_len, nseg, pacc, pml, \
                        ctl, pending, fresh, rkw, rvw, rgw, stream)
  if (group % 4 == 0) return KVM_PARTIAL(4);
  if (group % 2 == 0) return KVM_PARTIAL(2);
  return KVM_PARTIAL(1);
#undef KVM_PARTIAL
}

}  // namespace

int64_t decode_segments(int64_t rows_total) {
  return (rows_total + kSegRows - 1) / kSegRows;
}

int64_t decode_workspace_bytes(const kvm_layer &L, int64_t max_rows) {
  const int64_t nseg = decode_segments(max_rows < 1 ? 1 : max_rows);
  return L.batch * L.q_heads * nseg * (L.head_dim + 2) * 4;
}

// ---------------------------------------------------------------------------
// Library-owned scratch of the allocation-free decode entry point
// (kvm_decode_attention_noalloc): the split-K partials live in this
// file-scope device array instead of a caller workspace.  Each GPU holds its
// own copy at its own address, resolved once per device with
// hipGetSymbolAddress; host code uses only that address, never the array's
// name.  Every call on a device shares the array, so calls that overlap on
// one device race.  The partial kernel writes every (query head, segment)
// entry the combine kernel reads, so nothing needs clearing between calls.
namespace {
constexpr int kMaxScratchDevices = 64;
__device__ __align__(256) unsigned char scratch[KVM_DECODE_SCRATCH_BYTES];
std::mutex g_scratch_mu;
void *g_scratch_ptr[kMaxScratchDevices] = {};
}  // namespace

hipError_t decode_scratch(void **ptr) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  if (dev < 0 || dev >= kMaxScratchDevices) return hipErrorInvalidDevice;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void *p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return e;
    g_scratch_ptr[dev] = p;
  }
  *ptr = g_scratch_ptr[dev];
  return hipSuccess;
}

hipError_t launch_decode(const kvm_layer &L, const void *q, int64_t q_sb,
                         int64_t q_sh, const kvm_state &st, int64_t active,
                         const void *ring_k, const void *ring_v,
                         int64_t ring_cap, int64_t ring_start,
                         int64_t recent_len, void *out, int64_t o_sb,
                         int64_t o_sh, void *workspace, hipStream_t stream,
                         const int32_t *ctl, int pending, int64_t max_rows,
                         const kvm_seq *fresh, void *ring_gate) {
  // Host counters: segments for the rows present; device counters: for
  // max_rows (segments past the live rows contribute nothing).
  // fresh (host counters only): the step's token, the last of the recent_len
  // window rows, read from fresh by the partial kernel, which also stores it
  // (with its merge gate) in its ring slot.
  kvm_seq fr{};
  if (fresh && !ctl) fr = *fresh;
  uint16_t *rk = static_cast<uint16_t *>(const_cast<void *>(ring_k));
  uint16_t *rv = static_cast<uint16_t *>(const_cast<void *>(ring_v));
  uint16_t *rg = static_cast<uint16_t *>(ring_gate);
  const int nseg = int(decode_segments(ctl ? max_rows : active + recent_len));
  const int64_t npid = L.batch * L.q_heads;
  float *pacc = static_cast<float *>(workspace);
  float *pml = pacc + npid * nseg * L.head_dim;
  hipError_t e;
  if (L.head_dim == 128)
    e = launch_partial_d<128>(L, q, q_sb, q_sh, st, active, ring_k, ring_v,
                              ring_cap, ring_start, recent_len, nseg, pacc,
                              pml, ctl, pending, fr, rk, rv, rg, stream);
  else
    e = launch_partial_d<64>(L, q, q_sb, q_sh, st, active, ring_k, ring_v,
                             ring_cap, ring_start, recent_len, nseg, pacc, pml,
                             ctl, pending, fr, rk, rv, rg, stream);
  if (e != hipSuccess) return e;
  if (L.head_dim == 128)
    hipLaunchKernelGGL(k_decode_combine<128>, dim3(unsigned(npid)), dim3(128),
                       0, stream, int(L.q_heads), nseg, pacc, pml,
                       static_cast<uint16_t *>(out), o_sb, o_sh);
  else
    hipLaunchKernelGGL(k_decode_combine<64>, dim3(unsigned(npid)), dim3(64), 0,
                       stream, int(L.q_heads), nseg, pacc, pml,
                       static_cast<uint16_t *>(out), o_sb, o_sh);
  return hipGetLastError();
}

namespace {
// recent_len += 1 in n counter records (vector stores: one lane per record).
__global__ __launch_bounds__(256) void k_decode_advance(int32_t *ctl, int64_t n) {
  const int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x;
  if (i < n) ctl[i * 4 + 2] += 1;
}
}  // namespace

hipError_t launch_decode_advance(int32_t *ctl, int64_t n, hipStream_t stream) {
  hipLaunchKernelGGL(k_decode_advance, dim3(unsigned((n + 255) / 256)), dim3(256), 0, stream, ctl, n);
  return hipGetLastError();
}

}  // namespace kvm
