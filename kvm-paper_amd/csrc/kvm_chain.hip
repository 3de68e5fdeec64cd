// Persistent chain of block-boundary memory updates on gfx950.
//
// Reference semantics are those of the per-update kernels: the update of
// model/kvm_mixer.py:250-340 (append + merge) with the fp32 routing of
// model/kvm_fp32_routing_reference.py:24-49, the overflow-token streams of
// model/kvm_triton_mixer.py:429-446 and the Triton numeric contract of
// model/kvm_triton_mixer.py:199-211.  This kernel runs a whole batch of
// consecutive updates in one launch instead of two to four launches per
// update, because a single update of a prefill is small (one row: 512
// tokens x 512 slots) and a kernel boundary costs more than its work.
//
// Row groups.  Every row (b, kv_head) is served by a group of G workgroups
// ("members") that sit on ONE XCD.  Workgroups are dispatched round-robin
// over the XCDs (workgroup i runs on XCD i mod n, n | 8), so the members of
// group g are the workgroups x + 8 * (q * G + m), x = g mod 8, q = g / 8.
// Members share that XCD's L2, so one member's stores are visible to the
// others once they have reached L2 (s_waitcnt) if the readers load them
// with device-scope loads (sc1), which miss in the reader's L1 (a CU's L1
// is not kept coherent with other CUs' stores; group-scope sc0 loads still
// hit it).  No device-wide L2 writeback or invalidation is needed.
// A group barrier is an L2 atomic counter; every wait is bounded and sets
// an abort flag (all members then leave) instead of spinning forever.  A
// member that gives up also ORs KVM_STATUS_CHAIN_TIMEOUT into the caller's
// sticky status word, which is how the host learns that the state and the
// snapshots of this launch are incomplete.
//
// Co-residency.  A group's members wait for each other, so all of them must
// run at the same time: the launch has at most one 512-thread workgroup per
// compute unit (chain_plan), and it relies on the GPU being otherwise idle
// enough to place all of them.  Work of another stream or process that holds
// compute units for longer than the poll budget makes the waits time out;
// the result is then reported, never silently used.
//
// Work split of one update of a row:
//   member m owns tokens [m * tpw, (m + 1) * tpw)  (prep, novelty, append,
//                routing; tpw <= 64, the token operands stay in LDS)
//   member m owns slots  [m * spm, (m + 1) * spm)  (merge sums, refreshed
//                attention rows), spm = ceil(slots / G)
// Phases, separated by group barriers (|):
//   [novelty -> | -> rank, append my tokens -> |] -> route(my tokens) -> |
//   -> merge(my slots) -> arrive, prep(my tokens of the next update), wait
// The raw keys / values of the next update's tokens are loaded while the
// routing scan runs, and the merge keys / values alternate between two
// buffers, so the next update's prep overlaps the barrier that ends this
// update.
// The state (s_k, s_v, s_vlen) lives in the caller's arrays; snapshot u
// holds the attention rows routing reads and snapshot u + 1 receives the
// refreshed rows of every slot, as in the per-update path.

#include "kvm_device.hpp"
#include "kvm_internal.hpp"
#include "kvm_seq.hpp"

#include <algorithm>

namespace kvm {

// Optional per-phase timestamps of k_chain_fixed (build with
// -DKVM_CHAIN_TIMING): member 0 and member G-1 of group 0 record the wall
// clock (100 MHz) at marks 0..15 of each of the first 128 phases; the host
// reads them with kvm_chain_timing_read.  Without the define the marks
// compile to nothing.
#ifdef KVM_CHAIN_TIMING
__device__ unsigned long long g_chain_ts[2][128][16];
#define KVM_TS(k)                                                                        \
  do {                                                                                   \
    if (threadIdx.x == 0 && p < 128) {                                                   \
      if (blockIdx.x == 0) g_chain_ts[0][p][k] = wall_clock64();                         \
      else if (blockIdx.x == 8 * (GM - 1)) g_chain_ts[1][p][k] = wall_clock64();          \
    }                                                                                    \
  } while (0)
// The appending chain's marks: member 0 of group 0, update i of the launch.
#define KVM_TS_A(k)                                                                      \
  do {                                                                                   \
    if (threadIdx.x == 0 && blockIdx.x == 0 && i < 128) g_chain_ts[0][i][k] = wall_clock64(); \
  } while (0)
#else
#define KVM_TS(k) ((void)0)
#define KVM_TS_A(k) ((void)0)
#endif

namespace {

constexpr int kChainThreads = 512;
constexpr int kChainWaves = kChainThreads / 64;
constexpr int kChainTok = 64;        // tokens per member at most
constexpr int kTilesInFlight = 4;    // 16-slot tiles a wave loads at once
constexpr int kCounterStride = 32;   // words between group counters (128 B)

// Group barrier, split so that independent work can run between arriving
// and waiting.  arrive: this workgroup's global stores have reached L2,
// then one L2 atomic increment.
__device__ __forceinline__ void group_arrive(unsigned *ctr) {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  if (threadIdx.x == 0) __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// Scalar load that misses in the scalar cache (glc) and reads L2, where the
// members' atomic increments land.  It is counted by lgkmcnt, not vmcnt, so
// a poll does not wait behind the wave's outstanding vector loads (which
// return in order): the barrier is seen as soon as the last member arrives.
__device__ __forceinline__ unsigned l2_scalar_load(const unsigned *p) {
  unsigned v;
  asm volatile("s_load_dword %0, %1, 0x0 glc\n\ts_waitcnt lgkmcnt(0)" : "=s"(v) : "s"(p) : "memory");
  return v;
}
// wait: until `target` arrivals (G per barrier), polled by wave 0.  False
// when the wait timed out or another group aborted.
__device__ __forceinline__ bool group_wait(unsigned *ctr, unsigned target, const ChainScratch &cs,
                                           int *ok_lds) {
  if (threadIdx.x < 64) {  // wave 0, wave-uniform
    int ok = 0;
    for (unsigned p = 0; p < cs.max_polls; ++p) {
      if (l2_scalar_load(ctr) >= target) {
        ok = 1;
        break;
      }
      if ((p & 255u) == 255u && l2_scalar_load(cs.abort_flag)) break;
      __builtin_amdgcn_s_sleep(1);
    }
    if (threadIdx.x == 0) {
      if (!ok) {
        __hip_atomic_store(cs.abort_flag, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_fetch_or(cs.status, unsigned(KVM_STATUS_CHAIN_TIMEOUT), __ATOMIC_RELAXED,
                              __HIP_MEMORY_SCOPE_AGENT);
      }
      *ok_lds = ok;
    }
  }
  __syncthreads();
  return *ok_lds != 0;
}

// Loads of data that other members wrote during this launch: buffer loads
// with device scope (sc1), served by the XCD's L2.  Offsets at or past the
// resource's byte count read zero.
constexpr int kBufWord3 = 0x00020000;
constexpr int kScopeDevice = 16;  // cache-policy bits: sc1
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ __amdgpu_buffer_rsrc_t l2_rsrc(const void *base, int64_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0,
                                           int(bytes < 0x7fffffff ? bytes : 0x7fffffff), kBufWord3);
}
__device__ __forceinline__ uint4 l2_ld16(__amdgpu_buffer_rsrc_t r, int off) {
  const u32x4 v = __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, kScopeDevice);
  return make_uint4(v[0], v[1], v[2], v[3]);
}
__device__ __forceinline__ uint32_t l2_ld4(__amdgpu_buffer_rsrc_t r, int off) {
  return __builtin_amdgcn_raw_buffer_load_b32(r, off, 0, kScopeDevice);
}
__device__ __forceinline__ uint64_t l2_ld8(__amdgpu_buffer_rsrc_t r, int off) {
  const auto v = __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, kScopeDevice);
  return uint64_t(v[0]) | (uint64_t(v[1]) << 32);
}

// Route key of a (score, slot) candidate: the per-update routing kernel's
// order-preserving encoding mono(fp32 score) << 32 | (0xffffffff - slot), so
// an integer maximum picks the largest score and, among equal scores, the
// lowest slot (torch.max returns the first maximum).  0 means no candidate.
__device__ __forceinline__ uint64_t route_key(float score, int slot) {
  const uint32_t u = __float_as_uint(score);
  const uint32_t m = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
  return (uint64_t(m) << 32) | uint64_t(0xffffffffu - uint32_t(slot));
}
__device__ __forceinline__ int route_key_slot(uint64_t key) {
  return key ? int(0xffffffffu - uint32_t(key)) : -1;
}

// LDS byte address of a __shared__ object (wave-uniform).
typedef __attribute__((address_space(3))) void lds_void;
template <typename T>
__device__ __forceinline__ uint32_t lds_addr(T *p) {
  return __builtin_amdgcn_readfirstlane(uint32_t(uintptr_t((lds_void *)(p))));
}
// 16-byte-per-lane device-scope (sc1) buffer load from L2 straight into LDS
// at M0 + 16 * lane.  Issued from inline assembly so that the compiler does
// not order later LDS reads behind it; the caller waits with s_waitcnt vmcnt.
// M0 is written inside the statement and not declared clobbered (the compiler
// rejects M0 as a clobber): this is sound only while no compiled code of the
// kernel keeps a value of its own in M0, which holds for these kernels (their
// only M0 writes are these statements; checked in the generated assembly).
__device__ __forceinline__ void dma16_l2(__amdgpu_buffer_rsrc_t r, uint32_t lds, uint32_t voff) {
  asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, 0 offen sc1 lds"
               :: "s"(__builtin_amdgcn_readfirstlane(lds)), "v"(voff), "s"(r) : "memory");
}

// The same from device memory with the non-temporal policy: raw token rows
// are read once, and streaming them keeps them from evicting the merge
// buffers the group reads back from L2 one and two updates later.
__device__ __forceinline__ void dma16_nt(__amdgpu_buffer_rsrc_t r, uint32_t lds, uint32_t voff) {
  asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, 0 offen nt lds"
               :: "s"(__builtin_amdgcn_readfirstlane(lds)), "v"(voff), "s"(r) : "memory");
}

// 16-byte buffer store at a 32-bit byte offset from the resource's base
// (aux: cache policy bits; kPolicyNT streams the line to memory).
constexpr int kPolicyNT = 2;
template <int AUX>
__device__ __forceinline__ void st16(__amdgpu_buffer_rsrc_t r, uint32_t off, const uint4 &v) {
  __builtin_amdgcn_raw_buffer_store_b128(u32x4{v.x, v.y, v.z, v.w}, r, int(off), 0, AUX);
}

// Waits until at most N vector memory operations of the wave are in flight.
template <int N>
__device__ __forceinline__ void wait_vm() {
  asm volatile("s_waitcnt vmcnt(%0)" :: "n"(N) : "memory");
}

// Raw token rows are read once: non-temporal loads keep them from evicting
// the merge buffers the group reads back from L2 one and two updates later.
__device__ __forceinline__ uint4 ld_stream16(const uint16_t *p) {
  const u32x4 x = __builtin_nontemporal_load(reinterpret_cast<const u32x4 *>(p));
  return make_uint4(x[0], x[1], x[2], x[3]);
}

// Lane exchanges across 16 / 32 lanes with v_permlane{16,32}_swap (VALU,
// no LDS round trip): the value of lane l ^ 16 (l ^ 32).
__device__ __forceinline__ uint32_t xor16_lane(uint32_t x, int lane) {
  const auto r = __builtin_amdgcn_permlane16_swap(x, x, false, false);
  return (lane & 16) ? r[0] : r[1];
}
__device__ __forceinline__ uint32_t xor32_lane(uint32_t x, int lane) {
  const auto r = __builtin_amdgcn_permlane32_swap(x, x, false, false);
  return (lane & 32) ? r[0] : r[1];
}

__device__ __forceinline__ AttnRows snap_at(const SnapRing &r, int64_t idx) {
  const int64_t o = (idx % r.ring) * r.stride;
  return AttnRows{r.k + o, r.v + o, r.cap};
}

// Scan of the member's tokens (operand rows in LDS, ntk <= 64 of them)
// against slots [0, hi) of one row's attention keys (written by other
// members) on MFMA 16x16x32 bf16, computed transposed (slot x token) with
// the same operand roles and k-step order as the per-update routing kernel,
// so the fp32 scores are bit-identical.  Wave w takes the 16-slot tiles
// w + 8 * (4p + s), s < 4, in pass p and loads a pass's four tiles at once;
// `hook` runs once, right after the first pass's loads are issued.
//   NOVELTY: max over slots of the bf16-rounded score
//            (model/kvm_mixer.py:66-68);
//   route:   first argmax of the fp32 score over slots [lo, hi)
//            (model/kvm_fp32_routing_reference.py:30-34).
// Result of local token lt: best_v[lt] (and best_i[lt]).
template <int D, bool NOVELTY, typename Hook>
__device__ __forceinline__ void scan_slots(const uint16_t *op, const uint16_t *keys, int lo,
                                           int hi, int ntk, float (*red_v)[kChainTok],
                                           int (*red_i)[kChainTok], float *best_v, int *best_i,
                                           Hook &&hook) {
  constexpr int STR = D + 8;
  constexpr int KS = D / 32;
  constexpr int TF = kTilesInFlight;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int n_tt = (ntk + 15) >> 4;
  const int n_st = (hi + 15) >> 4;
  // Rows j >= hi lie past the resource and read zero (and are masked).
  const __amdgpu_buffer_rsrc_t kr = l2_rsrc(keys, int64_t(hi) * D * 2);

  float best[4];
  int bidx[4];
#pragma unroll
  for (int tt = 0; tt < 4; ++tt) {
    best[tt] = -INFINITY;
    bidx[tt] = -1;
  }
  for (int p0 = 0; p0 < n_st; p0 += kChainWaves * TF) {
    uint4 a[TF][KS];
#pragma unroll
    for (int s = 0; s < TF; ++s) {
      const int j = (p0 + wave + kChainWaves * s) * 16 + (lane & 15);
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) a[s][ks] = l2_ld16(kr, (j * D + ks * 32 + (lane >> 4) * 8) * 2);
    }
    if (p0 == 0) hook();
#pragma unroll
    for (int tt = 0; tt < 4; ++tt) {
      if (tt < n_tt) {
        bf16x8 bx[KS];
#pragma unroll
        for (int ks = 0; ks < KS; ++ks)
          bx[ks] = as_bf16x8(*reinterpret_cast<const uint4 *>(
              &op[(tt * 16 + (lane & 15)) * STR + ks * 32 + (lane >> 4) * 8]));
        f32x4 acc[TF];
#pragma unroll
        for (int s = 0; s < TF; ++s) acc[s] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ks = 0; ks < KS; ++ks)
#pragma unroll
          for (int s = 0; s < TF; ++s)
            acc[s] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(a[s][ks]), bx[ks], acc[s], 0,
                                                             0, 0);
        // Slots in increasing order within the lane: a strict > keeps the
        // first maximum.
#pragma unroll
        for (int s = 0; s < TF; ++s) {
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int j = (p0 + wave + kChainWaves * s) * 16 + (lane >> 4) * 4 + i;
            // Selects, not branches: slots outside [lo, hi) score -inf.
            if constexpr (NOVELTY) {
              best[tt] = fmaxf(best[tt], j < hi ? rbf(acc[s][i]) : -INFINITY);
            } else {
              const float sc = (j >= lo) & (j < hi) ? acc[s][i] : -INFINITY;
              const bool take = sc > best[tt];
              best[tt] = take ? sc : best[tt];
              bidx[tt] = take ? j : bidx[tt];
            }
          }
        }
      }
    }
  }
  if (n_st == 0) hook();

  // Lane groups (slots 4q..4q+3 of every tile), then waves (interleaved
  // tiles): larger score wins, equal scores go to the lower slot.
#pragma unroll
  for (int tt = 0; tt < 4; ++tt) {
    float bv = best[tt];
    int bi = bidx[tt];
#pragma unroll
    for (int r = 0; r < 2; ++r) {
      const uint32_t vb = __float_as_uint(bv), ib = uint32_t(bi);
      const float ob = __uint_as_float(r == 0 ? xor16_lane(vb, lane) : xor32_lane(vb, lane));
      const int oi = int(r == 0 ? xor16_lane(ib, lane) : xor32_lane(ib, lane));
      if constexpr (NOVELTY) {
        bv = fmaxf(bv, ob);
      } else if (oi >= 0 && (bi < 0 || ob > bv || (ob == bv && oi < bi))) {
        bv = ob;
        bi = oi;
      }
    }
    if (lane < 16) {
      red_v[wave][tt * 16 + lane] = bv;
      red_i[wave][tt * 16 + lane] = bi;
    }
  }
  __syncthreads();
  if (tid < kChainTok) {
    float vv[kChainWaves];
    int ii[kChainWaves];
#pragma unroll
    for (int w = 0; w < kChainWaves; ++w) {
      vv[w] = red_v[w][tid];
      ii[w] = red_i[w][tid];
    }
    float bv = vv[0];
    int bi = ii[0];
#pragma unroll
    for (int w = 1; w < kChainWaves; ++w) {
      if constexpr (NOVELTY) {
        bv = fmaxf(bv, vv[w]);
      } else if (ii[w] >= 0 && (bi < 0 || vv[w] > bv || (vv[w] == bv && ii[w] < bi))) {
        bv = vv[w];
        bi = ii[w];
      }
    }
    best_v[tid] = bv;
    if (best_i) best_i[tid] = bi;
  }
  __syncthreads();
}

// Raw key / value / gate of the member's tokens, D/8 lanes per token.
template <int D>
struct RawTok {
  static constexpr int IT = kChainTok * (D / 8) / kChainThreads;
  uint4 k[IT], v[IT];
  uint16_t g[IT];  // bf16 bits, converted where used (no wait at the load)
};

template <int D>
__global__ __launch_bounds__(kChainThreads) void k_chain(
    kvm_layer L, kvm_seq src, int n_tok, kvm_state st, SnapRing snaps, ChainList list,
    ChainScratch cs, int rows, int row0, int nrows, int G, int tpw, int spm_max, int32_t *route_log,
    int32_t *append_log, int64_t log_stride) {
  constexpr int GL = D / 8;                 // lanes per D-wide row
  constexpr int STR = D + 8;                // LDS row stride (elements)
  constexpr int RPP = kChainThreads / GL;   // rows per pass
  constexpr int IT = RawTok<D>::IT;         // passes over the member's tokens
  static_assert(IT * RPP == kChainTok, "token passes");
  __shared__ __attribute__((aligned(16))) uint16_t op_r[kChainTok * STR];  // merge keys
  __shared__ __attribute__((aligned(16))) uint16_t op_n[kChainTok * STR];  // prep(k)
  __shared__ float red_v[kChainWaves][kChainTok];
  __shared__ int red_i[kChainWaves][kChainTok];
  __shared__ float res_v[kChainTok];
  __shared__ int res_i[kChainTok];
  __shared__ int ok_lds;
  __shared__ float ln_w[D], ln_b[D];  // ln_s_k parameters (LDS: no wait on global loads)
  extern __shared__ __attribute__((aligned(16))) int dyn[];
  int *tok_a = dyn;               // [n_tok] novelty rank flag
  int *mr = tok_a + n_tok;        // [n_tok] local slot of each token or -1
  int *lst = mr + n_tok;          // [n_tok] tokens placed per slot
  int *sorted = lst + n_tok;      // [n_tok] per-slot lists in token order
  int *cnt = sorted + n_tok;      // [spm_max]
  int *off = cnt + spm_max;       // [spm_max]
  int *fill = off + spm_max;      // [spm_max]
  int *apos = sorted;             // [n_tok] append position of each token (append phase)
  // [npow] sort keys of the append selection, 8-byte aligned after fill
  const int npow = n_tok <= 1 ? 1 : 1 << (32 - __builtin_clz(unsigned(n_tok - 1)));
  uint64_t *skey = reinterpret_cast<uint64_t *>(fill + spm_max + (spm_max & 1));

  const int tid = threadIdx.x, part = tid % GL;
  const int xcd = blockIdx.x & 7, q = blockIdx.x >> 3;
  const int member = q % G, group = (q / G) * 8 + xcd;
  if (group >= nrows) return;
  for (int d = tid; d < D; d += kChainThreads) {
    ln_w[d] = static_cast<const float *>(L.ln_weight)[d];
    ln_b[d] = static_cast<const float *>(L.ln_bias)[d];
  }
  __syncthreads();
  const int row = row0 + group;  // this launch serves rows row0 .. row0 + nrows - 1
  const int b = row / int(L.kv_heads), h = row % int(L.kv_heads);
  const int t0 = member * tpw;
  const int ntk = max(0, min(n_tok, t0 + tpw) - t0);
  const int64_t rb = int64_t(row) * n_tok;
  const int64_t par_stride = int64_t(rows) * n_tok * D;  // elements between the two merge buffers
  unsigned *ctr = cs.bar + group * kCounterStride;
  unsigned target = 0;
  auto arrive = [&]() __attribute__((always_inline)) {
    target += unsigned(G);
    group_arrive(ctr);
  };
  auto wait = [&]() __attribute__((always_inline)) {
    return group_wait(ctr, target, cs, &ok_lds);
  };
  uint16_t *s_k = static_cast<uint16_t *>(st.s_k);
  uint16_t *s_v = static_cast<uint16_t *>(st.s_v);
  float *s_vlen = static_cast<float *>(st.s_vlen);
  const int64_t srow = int64_t(row) * st.capacity;

  // Raw tokens of update i (token 0 of the chunk for idle lanes).  Prefill
  // tokens never come from a ring (src.ring == 0, checked by the host).
  const uint16_t *k_row = static_cast<const uint16_t *>(src.k) + b * src.k_sb + h * src.k_sh;
  const uint16_t *v_row = static_cast<const uint16_t *>(src.v) + b * src.v_sb + h * src.v_sh;
  const uint16_t *g_row = static_cast<const uint16_t *>(src.gate) + b * src.g_sb + h * src.g_sh;
  auto load_raw = [&](int i, RawTok<D> &rt) __attribute__((always_inline)) {
    const int64_t tb = list.tok_begin[i];
#pragma unroll
    for (int it = 0; it < IT; ++it) {
      const int lt = (tid + it * kChainThreads) / GL;
      const int64_t t = tb + (lt < ntk ? t0 + lt : 0);
      rt.k[it] = ld_stream16(k_row + t * src.k_st + part * 8);
      rt.v[it] = ld_stream16(v_row + t * src.v_st + part * 8);
      rt.g[it] = g_row[t * src.g_st];
    }
  };
  // prep (model/kvm_mixer.py:120-129, model/kvm_triton_mixer.py:429-446):
  // merge key / value of my tokens into LDS (routing operand) and into the
  // update's merge buffer; prep(k) into LDS when the update appends.
  auto prep = [&](int i, const RawTok<D> &rt) __attribute__((always_inline)) {
    const bool nov = list.n_append[i] > 0;
    uint16_t *gkb = cs.gk + (i & 1) * par_stride;
    uint16_t *gvb = cs.gv + (i & 1) * par_stride;
#pragma unroll
    for (int it = 0; it < IT; ++it) {
      const int lt = (tid + it * kChainThreads) / GL;
      const bool valid = lt < ntk;
      float k[8], v[8];
      unpack8(rt.k[it], k);
      unpack8(rt.v[it], v);
      const float g = bf2f(rt.g[it]);
      prep_key<D>(k, part, L, ln_w, ln_b);
      float gk[8], gv[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        gk[e] = L.gate_keys ? rbf(k[e] * g) : k[e];
        gv[e] = L.gate_values ? rbf(v[e] * g) : v[e];
      }
      const uint4 z = make_uint4(0, 0, 0, 0);
      *reinterpret_cast<uint4 *>(&op_r[lt * STR + part * 8]) = valid ? pack8(gk) : z;
      if (nov) *reinterpret_cast<uint4 *>(&op_n[lt * STR + part * 8]) = valid ? pack8(k) : z;
      if (valid) {
        const int64_t o = (rb + t0 + lt) * D + part * 8;
        store8(gkb + o, gk);
        store8(gvb + o, gv);
      }
    }
  };

  RawTok<D> rt;
  load_raw(0, rt);
  prep(0, rt);
  __syncthreads();

  for (int i = 0; i < list.count; ++i) {
    const int64_t u = int64_t(list.u0) + i;
    const int64_t tb = list.tok_begin[i];
    const int sb = list.state_before[i], na = list.n_append[i];
    const int s_after = sb + na;
    const int protect = min(int(L.sink_len), s_after);
    const AttnRows cur = snap_at(snaps, u), nxt = snap_at(snaps, u + 1);
    const uint16_t *gkb = cs.gk + (i & 1) * par_stride;
    const uint16_t *gvb = cs.gv + (i & 1) * par_stride;
    int32_t *rlog = route_log ? route_log + u * log_stride + rb : nullptr;
    int32_t *alog = append_log ? append_log + u * log_stride + rb : nullptr;
    const uint16_t *cur_k = cur.k + int64_t(row) * cur.cap * D;
    KVM_TS_A(0);

    // ---- append (model/kvm_mixer.py:44-75, 231-248): the n_append least
    // novel tokens, ties to the lower index, become slots sb.. in token order.
    if (na > 0) {
      scan_slots<D, true>(op_n, cur_k, 0, sb, ntk, red_v, red_i, res_v, nullptr, [] {});
      if (tid < ntk) cs.nov[rb + t0 + tid] = res_v[tid];
      KVM_TS_A(1);
      arrive();
      if (!wait()) return;
      KVM_TS_A(2);
      // The na smallest (novelty, token) pairs: a bitonic sort of the unique
      // keys mono(novelty) << 32 | token (the same order as comparing the
      // novelty, then the index; -0 is read as +0 so that it ties with it),
      // padded with the largest key to a power of two.
      const __amdgpu_buffer_rsrc_t nr = l2_rsrc(cs.nov + rb, int64_t(n_tok) * 4);
      for (int t = tid; t < npow; t += kChainThreads) {
        uint64_t key = ~uint64_t(0);
        if (t < n_tok) {
          const float x = __uint_as_float(l2_ld4(nr, t * 4)) + 0.0f;
          const uint32_t bits = __float_as_uint(x);
          const uint32_t m = (bits & 0x80000000u) ? ~bits : (bits | 0x80000000u);
          key = (uint64_t(m) << 32) | uint32_t(t);
        }
        skey[t] = key;
        if (t < n_tok) tok_a[t] = 0;
      }
      __syncthreads();
      // Keys tid and tid + 512 in registers: a compare-exchange stage whose
      // partner distance j is below 64 pairs keys of one wave (e ^ j is in
      // e's 64-key block) and runs on lane shuffles; the others go through
      // LDS, a barrier each.
      constexpr int KPT = 2;  // keys per thread (n_tok <= 1024)
      uint64_t rk[KPT];
      auto load_keys = [&]() __attribute__((always_inline)) {
#pragma unroll
        for (int x = 0; x < KPT; ++x) {
          const int e = tid + x * kChainThreads;
          rk[x] = e < npow ? skey[e] : ~uint64_t(0);
        }
      };
      auto store_keys = [&]() __attribute__((always_inline)) {
#pragma unroll
        for (int x = 0; x < KPT; ++x) {
          const int e = tid + x * kChainThreads;
          if (e < npow) skey[e] = rk[x];
        }
      };
      load_keys();
      for (int k2 = 2; k2 <= npow; k2 <<= 1) {
        int j = k2 >> 1;
        if (j >= 64) {
          store_keys();
          __syncthreads();
          for (; j >= 64; j >>= 1) {
            for (int e = tid; e < npow; e += kChainThreads) {
              const int f = e ^ j;
              if (f > e) {
                const uint64_t a = skey[e], c = skey[f];
                if ((a > c) == ((e & k2) == 0)) {
                  skey[e] = c;
                  skey[f] = a;
                }
              }
            }
            __syncthreads();
          }
          load_keys();
        }
        for (; j > 0; j >>= 1) {
#pragma unroll
          for (int x = 0; x < KPT; ++x) {
            const int e = tid + x * kChainThreads;
            const uint32_t lo = uint32_t(__shfl_xor(int(uint32_t(rk[x])), j));
            const uint32_t hi = uint32_t(__shfl_xor(int(uint32_t(rk[x] >> 32)), j));
            const uint64_t o = (uint64_t(hi) << 32) | lo;
            // The lower index of an ascending pair keeps the smaller key.
            const bool take_min = ((e & k2) == 0) == ((e & j) == 0);
            const uint64_t mn = rk[x] < o ? rk[x] : o, mx = rk[x] < o ? o : rk[x];
            if (e < npow) rk[x] = take_min ? mn : mx;
          }
        }
      }
      store_keys();
      __syncthreads();
      for (int r = tid; r < na; r += kChainThreads) tok_a[int(uint32_t(skey[r]))] = 1;
      __syncthreads();
      KVM_TS_A(3);
      // Append position of every appended token: the appended tokens before
      // it, by wave ballots in token order (wave totals in res_v).
      {
        int base = 0;
        for (int c0 = 0; c0 < n_tok; c0 += kChainThreads) {
          const int t = c0 + tid;
          const bool ap = t < n_tok && tok_a[t] != 0;
          const uint64_t bal = __ballot(ap);
          const int before = int(__builtin_amdgcn_mbcnt_hi(uint32_t(bal >> 32),
                                                           __builtin_amdgcn_mbcnt_lo(uint32_t(bal), 0u)));
          if ((tid & 63) == 0) res_v[tid >> 6] = __int_as_float(__popcll(bal));
          __syncthreads();
          int wb = base;
          for (int w = 0; w < (tid >> 6); ++w) wb += __float_as_int(res_v[w]);
          if (t < n_tok) apos[t] = ap ? wb + before : -1;
          for (int w = 0; w < kChainWaves; ++w) base += __float_as_int(res_v[w]);
          __syncthreads();
        }
      }
      if (tid < ntk) res_i[tid] = apos[t0 + tid];
      __syncthreads();
#pragma unroll
      for (int it = 0; it < IT; ++it) {
        const int lt = (tid + it * kChainThreads) / GL;
        const bool valid = lt < ntk && res_i[lt] >= 0;
        const int tl = lt < ntk ? t0 + lt : 0;  // token of this lane (token 0 when idle)
        float k[8], v[8];
        if (L.gate_appends) {
          unpack8(*reinterpret_cast<const uint4 *>(&op_r[lt * STR + part * 8]), k);
          unpack8(l2_ld16(l2_rsrc(gvb + rb * D, int64_t(n_tok) * D * 2), (tl * D + part * 8) * 2), v);
        } else {
          unpack8(*reinterpret_cast<const uint4 *>(&op_n[lt * STR + part * 8]), k);
          load8(v_row + (tb + tl) * src.v_st + part * 8, v);
        }
        const float vlen = row_norm8<D>(v);
        float ka[8], va[8];
        attn_rows<D>(k, v, vlen, part, L, ln_w, ln_b, ka, va);
        if (valid) {
          const int64_t slot = sb + res_i[lt];
          const int64_t so = (srow + slot) * D + part * 8;
          store8(s_k + so, k);
          store8(s_v + so, v);
          if (part == 0) s_vlen[srow + slot] = vlen;
          const int64_t ao = (int64_t(row) * cur.cap + slot) * D + part * 8;
          store8(cur.k + ao, ka);
          store8(cur.v + ao, va);
        }
      }
      KVM_TS_A(4);
      arrive();
      if (!wait()) return;
      KVM_TS_A(5);
    }

    // ---- route (model/kvm_fp32_routing_reference.py:30-34); the next
    // update's raw tokens are loaded behind the scan's slot rows.
    const bool more = i + 1 < list.count;
    scan_slots<D, false>(op_r, cur_k, protect, s_after, ntk, red_v, red_i, res_v, res_i,
                         [&]() __attribute__((always_inline)) {
                           if (more) load_raw(i + 1, rt);
                         });
    KVM_TS_A(6);
    if (tid < ntk) {
      const int t = t0 + tid;
      const bool app = na > 0 && tok_a[t] != 0;
      cs.route[rb + t] = app ? -1 : res_i[tid];
      if (alog) alog[t] = app ? 1 : 0;
      if (rlog) rlog[t] = app ? sb + apos[t] : res_i[tid];
    }
    KVM_TS_A(7);
    arrive();
    if (!wait()) return;
    KVM_TS_A(8);

    // ---- merge + refresh (model/kvm_mixer.py:329-335) of my slots
    const int spm = (s_after + G - 1) / G;
    const int j0 = member * spm;
    const int nsl = max(0, min(s_after, j0 + spm) - j0);
    const __amdgpu_buffer_rsrc_t skr = l2_rsrc(s_k + srow * D, st.capacity * D * 2);
    const __amdgpu_buffer_rsrc_t svr = l2_rsrc(s_v + srow * D, st.capacity * D * 2);
    const __amdgpu_buffer_rsrc_t slr = l2_rsrc(s_vlen + srow, st.capacity * 4);
    const __amdgpu_buffer_rsrc_t gkr = l2_rsrc(gkb + rb * D, int64_t(n_tok) * D * 2);
    const __amdgpu_buffer_rsrc_t gvr = l2_rsrc(gvb + rb * D, int64_t(n_tok) * D * 2);
    const __amdgpu_buffer_rsrc_t rr = l2_rsrc(cs.route + rb, int64_t(n_tok) * 4);
    // Current sums and vlen of the first two slot passes (independent of the
    // routes; rows past the state read zero and are not stored).
    auto ld_state = [&](int local, uint4 &kk, uint4 &vv, float &ll) __attribute__((always_inline)) {
      const int j = j0 + local;
      kk = l2_ld16(skr, (j * D + part * 8) * 2);
      vv = l2_ld16(svr, (j * D + part * 8) * 2);
      ll = __uint_as_float(l2_ld4(slr, j * 4));
    };
    uint4 k0, v0, k1, v1;
    float l0, l1;
    ld_state(tid / GL, k0, v0, l0);
    ld_state(RPP + tid / GL, k1, v1, l1);

    for (int e = tid; e < nsl; e += kChainThreads) {
      cnt[e] = 0;
      fill[e] = 0;
    }
    __syncthreads();
    for (int t = tid; t < n_tok; t += kChainThreads) {
      const int r = int(l2_ld4(rr, t * 4));
      const int lr = (r >= j0 && r < j0 + nsl) ? r - j0 : -1;
      mr[t] = lr;
      if (lr >= 0) atomicAdd(&cnt[lr], 1);
    }
    __syncthreads();
    // Exclusive prefix of the slot counts on one wave.
    if (tid < 64) {
      const int per = (nsl + 63) >> 6;
      const int e0 = tid * per;
      int sum = 0;
      for (int e = 0; e < per; ++e)
        if (e0 + e < nsl) sum += cnt[e0 + e];
      int incl = sum;
#pragma unroll
      for (int o = 1; o < 64; o <<= 1) {
        const int y = __shfl_up(incl, o);
        if (tid >= o) incl += y;
      }
      int run = incl - sum;
      for (int e = 0; e < per; ++e)
        if (e0 + e < nsl) {
          off[e0 + e] = run;
          run += cnt[e0 + e];
        }
    }
    __syncthreads();
    for (int t = tid; t < n_tok; t += kChainThreads) {
      const int lr = mr[t];
      if (lr >= 0) lst[off[lr] + atomicAdd(&fill[lr], 1)] = t;
    }
    __syncthreads();
    // Each slot's list in token order (rank sort), so the fp32 sums run in
    // token order whatever order the LDS atomics placed them in.
    for (int base = 0; base < nsl; base += RPP) {
      const int local = base + tid / GL;
      if (local < nsl) {
        const int n = cnt[local], o = off[local];
        for (int e = part; e < n; e += GL) {
          const int x = lst[o + e];
          int r = 0;
          for (int f = 0; f < n; ++f) r += lst[o + f] < x;
          sorted[o + r] = x;
        }
      }
    }
    __syncthreads();
    KVM_TS_A(9);
    auto merge_slot = [&](int local, const uint4 &k_raw, const uint4 &v_raw,
                          float vlen) __attribute__((always_inline)) {
      const bool valid = local < nsl;
      const int j = j0 + (valid ? local : 0);
      const int n = valid ? cnt[local] : 0;
      const int o = valid ? off[local] : 0;
      float sk[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
      float sv[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
      for (int i0 = 0; i0 < n; i0 += 4) {
        uint4 xk[4], xv[4];
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          if (i0 + w < n) {
            const int to = (sorted[o + i0 + w] * D + part * 8) * 2;
            xk[w] = l2_ld16(gkr, to);
            xv[w] = l2_ld16(gvr, to);
          }
        }
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          if (i0 + w < n) {
            float fk[8], fv[8];
            unpack8(xk[w], fk);
            unpack8(xv[w], fv);
#pragma unroll
            for (int e = 0; e < 8; ++e) {
              sk[e] += fk[e];
              sv[e] += fv[e];
            }
          }
        }
      }
      float k[8], v[8];
      unpack8(k_raw, k);
      unpack8(v_raw, v);
      const int64_t so = (srow + j) * D + part * 8;
      if (n > 0) {
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          k[e] = rbf(k[e] + rbf(sk[e]));
          v[e] = rbf(v[e] + rbf(sv[e]));
        }
        if (valid) {
          store8(s_k + so, k);
          store8(s_v + so, v);
        }
      }
      float ka[8], va[8];
      attn_rows<D>(k, v, vlen, part, L, ln_w, ln_b, ka, va);
      if (valid) {
        const int64_t ao = (int64_t(row) * nxt.cap + j) * D + part * 8;
        store8(nxt.k + ao, ka);
        store8(nxt.v + ao, va);
      }
    };
    for (int base = 0; base < nsl; base += 2 * RPP) {
      if (base > 0) {
        ld_state(base + tid / GL, k0, v0, l0);
        ld_state(base + RPP + tid / GL, k1, v1, l1);
      }
      merge_slot(base + tid / GL, k0, v0, l0);
      if (base + RPP < nsl) merge_slot(base + RPP + tid / GL, k1, v1, l1);
    }
    KVM_TS_A(10);

    // ---- next update's prep while the other members finish this merge.
    if (more) {
      arrive();
      prep(i + 1, rt);
      KVM_TS_A(11);
      if (!wait()) return;
      KVM_TS_A(12);
    }
  }
}

// ---------------------------------------------------------------------------
// Chain of updates that append nothing (a fixed budget, or a batch in which
// the budget does not grow): routing is split by SLOT instead of by token.
//
// Member m owns the 16-slot blocks m, m + G, m + 2G, ... of its row for the
// whole launch: their sums (s_k, s_v, vlen) and attention key rows live in
// the member's LDS.  Phase p of the launch:
//   prep(p + 1)     merge keys / values of my share of update p + 1's tokens
//                   (while the route keys of update p - 1 are in flight);
//   combine(p - 1)  every member's best slot for every token of update
//                   p - 1 (largest score, then lowest slot);
//   lists(p - 1)    the tokens routed to each of my slots, in token order
//                   (wave ballots: rank within the wave, per-wave counts);
//   merge(p - 1)    sums of the tokens routed to my slots (token order),
//                   refreshed attention rows into LDS and, straight from
//                   registers, into snapshot u0 + p;
//   route(p)        the merge keys of ALL tokens of update p against MY
//                   slots (MFMA 16x16x32 bf16, the per-update kernel's
//                   operand roles and k-step order, so the fp32 scores are
//                   bit-identical) -> per-token maximum over my slots,
//                   published as a tagged partial.
// There is no group barrier per update.  A member publishes its partials
// (score, slot, tag of the update) only after its earlier stores (the
// merge keys / values it prepared) have reached L2 and every wave of the
// workgroup has got there; a reader polls the tags of the partials it
// needs.  Seeing member m's partials of update p therefore also shows that
// m's prepared rows of update p + 1 are readable, and that m has finished
// reading every buffer of update p - 1 (so they may be overwritten).
// Merge keys / values rotate through four buffers (prepared one phase
// ahead, read by route and, a phase later, by the merge); partials
// alternate between two.  Four, not three: a member starts the prep of
// update p + 1 (into buffer (p + 1) % 4) before it has seen the partials of
// update p - 1, so another member may still be in phase p - 1, gathering
// the rows of update p - 2 and loading route operands of update p - 1,
// while a member already in phase p + 1 may be preparing update p + 2; with
// three buffers update p + 1 would share the buffer of update p - 2.  The
// two partial buffers suffice: a member publishes update p only after it
// has seen every member's partials of update p - 1, by which time every
// member has stopped polling those of update p - 2.  The raw tokens a prep needs are loaded at the
// end of the phase before; the route operands of update p are loaded once
// the merge's gathered rows have arrived, so they never queue in L2 ahead
// of the gathers.
constexpr int kOwnMax = 128;      // owned slots per member at most (8 blocks of 16)
constexpr int kTokWave = 64;      // tokens per wave in route(p)
constexpr int kFixedMaxTok = kChainWaves * kTokWave;  // == kChainThreads: one token per thread

__device__ __forceinline__ int own_local_to_slot(int l, int G, int m) {
  return (((l >> 4) * G + m) << 4) | (l & 15);
}

// GM: the group size G (8 or 16); OWN: owned slots per member the LDS holds
// (64, or 128 for states of up to 1024 slots at G = 8).
template <int D, int GM, int OWN>
__global__ __launch_bounds__(kChainThreads) void k_chain_fixed(
    kvm_layer L, kvm_seq src, int n_tok, kvm_state st, SnapRing snaps, ChainList list,
    ChainScratch cs, int rows, int row0, int nrows, int32_t *route_log, int32_t *append_log,
    int64_t log_stride) {
  constexpr int GL = D / 8;                 // lanes per D-wide row
  constexpr int STR = D + 8;                // LDS row stride of key rows (elements)
  constexpr int KS = D / 32;
  constexpr int RPP = kChainThreads / GL;   // rows per pass
  constexpr int SP = OWN / RPP;             // passes over the owned slots
  constexpr int HP = SP < 2 ? SP : 2;       // passes per half (the sums of one half live in registers)
  constexpr int NH = SP / HP;               // halves of the owned slots
  // Routed token rows staged in LDS at once (96 at OWN 128 and D 128, where
  // the owned rows need the room).
  constexpr int STAGE = (OWN == 128 && D == 128) ? 96 : 128;
  constexpr int RPI = 1024 / (2 * D);        // token rows per 1 KiB DMA instruction
  constexpr int KI = STAGE / RPI;            // DMA instructions per staged chunk (keys or values)
  constexpr int LOG2_OWN = OWN == 128 ? 7 : 6;
  static_assert(OWN == 64 || OWN == 128, "owned slots");
  static_assert(SP == NH * HP, "refresh halves");
  static_assert(kChainTok <= STAGE, "raw rows alias the staging buffers");
  constexpr int IT = RawTok<D>::IT;         // passes over the member's prep tokens
  constexpr int NRAW = 2 * (kChainTok / RPI) / kChainWaves;  // raw-row DMA instructions per wave
  static_assert(NRAW * kChainWaves == 2 * (kChainTok / RPI), "raw DMA split");
  __shared__ __attribute__((aligned(16))) uint16_t own_k[OWN * STR];  // attention keys
  __shared__ __attribute__((aligned(16))) uint16_t own_sk[OWN * D];   // key sums
  __shared__ __attribute__((aligned(16))) uint16_t own_sv[OWN * D];   // value sums
  // Routed token rows of the merge.  The raw key / value rows of my prep
  // share of an update share these buffers: they are DMA'd during a phase's
  // route, after that phase's sums have read the staged rows, and read by
  // the next phase's prep, before that phase's gathers are issued.
  __shared__ __attribute__((aligned(16))) uint16_t stage_k[STAGE * D];
  __shared__ __attribute__((aligned(16))) uint16_t stage_v[STAGE * D];
  uint16_t *const raw_k = stage_k;
  uint16_t *const raw_v = stage_v;
  __shared__ float own_vl[OWN];
  __shared__ int tok_lds[kChainMax];  // first token of each update (list.tok_begin)
  __shared__ int sorted[kFixedMaxTok];
  __shared__ int wsc[kChainWaves][OWN];  // per-wave slot counts
  __shared__ int cnt[OWN], off[OWN];
  __shared__ int ok_lds;
  __shared__ float ln_w[D], ln_b[D];  // ln_s_k parameters (LDS: no wait on global loads)

  constexpr int G = GM;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, part = tid % GL;
  const int xcd = blockIdx.x & 7, q = blockIdx.x >> 3;
  const int member = q % G, group = (q / G) * 8 + xcd;
  if (group >= nrows) return;
  const int row = row0 + group;  // this launch serves rows row0 .. row0 + nrows - 1
  const int b = row / int(L.kv_heads), h = row % int(L.kv_heads);
  const int64_t rb = int64_t(row) * n_tok;
  // Per-row bases; the buffers of one kind lie a 32-bit stride apart (the host
  // launches the chain only when they fit).
  const int buf_stride = rows * n_tok * D;   // elements between merge buffers
  const int part_stride = rows * n_tok * G;  // partials between the two buffers
  uint16_t *const gk_row = cs.gk + rb * D;
  uint16_t *const gv_row = cs.gv + rb * D;
  uint2 *const part_row = cs.part + rb * G;
  uint16_t *const snk_row = snaps.k + int64_t(row) * snaps.cap * D;
  uint16_t *const snv_row = snaps.v + int64_t(row) * snaps.cap * D;
  const int snap_stride = int(snaps.stride);
  const int snap_bytes = int(snaps.cap) * D * 2;
  const int k_st = int(src.k_st), v_st = int(src.v_st), g_st = int(src.g_st);
  const int tpm = (n_tok + G - 1) / G;                   // prep tokens per member (<= 64)
  const int pt0 = member * tpm;
  const int pnt = max(0, min(n_tok, pt0 + tpm) - pt0);
  unsigned *ctr = cs.bar + group * kCounterStride;
  unsigned target = 0;
  auto arrive = [&]() __attribute__((always_inline)) {
    target += unsigned(G);
    group_arrive(ctr);
  };
  auto wait = [&]() __attribute__((always_inline)) {
    return group_wait(ctr, target, cs, &ok_lds);
  };
  uint16_t *s_k = static_cast<uint16_t *>(st.s_k);
  uint16_t *s_v = static_cast<uint16_t *>(st.s_v);
  float *s_vlen = static_cast<float *>(st.s_vlen);
  const int64_t srow = int64_t(row) * st.capacity;
  const int S = list.state_before[0];  // no appends: constant over the batch
  const int protect = min(int(L.sink_len), S);
  // Owned local slots: 16 per owned block below S.
  const int nblk = (S + 15) >> 4;
  const int nown = member < nblk ? ((nblk - 1 - member) / G + 1) * 16 : 0;
  const uint16_t *k_row = static_cast<const uint16_t *>(src.k) + b * src.k_sb + h * src.k_sh;
  const uint16_t *v_row = static_cast<const uint16_t *>(src.v) + b * src.v_sb + h * src.v_sh;
  const uint16_t *g_row = static_cast<const uint16_t *>(src.gate) + b * src.g_sb + h * src.g_sh;

  for (int d = tid; d < D; d += kChainThreads) {
    ln_w[d] = static_cast<const float *>(L.ln_weight)[d];
    ln_b[d] = static_cast<const float *>(L.ln_bias)[d];
  }
  // The first token of every update, read from LDS where the raw rows are
  // fetched (a scalar load of the kernel argument would wait for memory).
  for (int i = tid; i < list.count; i += kChainThreads) tok_lds[i] = list.tok_begin[i];
  // ---- owned state and attention keys into LDS (slots >= S stay zero).
  {
    const AttnRows a0 = snap_at(snaps, list.u0);
    for (int base = 0; base < OWN; base += RPP) {
      const int l = base + tid / GL;
      const int j = own_local_to_slot(l, G, member);
      const bool valid = l < nown && j < S;
      const uint4 z = make_uint4(0, 0, 0, 0);
      const int64_t so = (srow + j) * D + part * 8;
      *reinterpret_cast<uint4 *>(&own_sk[l * D + part * 8]) =
          valid ? *reinterpret_cast<const uint4 *>(s_k + so) : z;
      *reinterpret_cast<uint4 *>(&own_sv[l * D + part * 8]) =
          valid ? *reinterpret_cast<const uint4 *>(s_v + so) : z;
      *reinterpret_cast<uint4 *>(&own_k[l * STR + part * 8]) =
          valid ? *reinterpret_cast<const uint4 *>(a0.k + (int64_t(row) * a0.cap + j) * D + part * 8)
                : z;
      if (part == 0) own_vl[l] = valid ? s_vlen[srow + j] : 0.f;
    }
  }

  // Raw key / value rows of my prep share of update i go from device memory
  // straight into LDS (non-temporal DMA, no registers): wave w issues
  // instructions w, w + 8, ... of the keys, then of the values, each filling
  // RPI consecutive rows; rows past my share lie past the resource and read
  // zero.  The gates go into registers.  Issued a whole phase before the prep
  // that reads them, so the prep never waits for device memory.  Prefill
  // tokens never come from a ring (src.ring == 0, checked by the host).
  uint16_t rg[IT];
  auto raw_dma = [&](int i) __attribute__((always_inline)) {
    const int64_t tb = int64_t(__builtin_amdgcn_readfirstlane(tok_lds[i])) + pt0;
    const int kb = pnt > 0 ? ((pnt - 1) * k_st + D) * 2 : 0;
    const int vb = pnt > 0 ? ((pnt - 1) * v_st + D) * 2 : 0;
    const __amdgpu_buffer_rsrc_t kr = l2_rsrc(k_row + tb * k_st, kb);
    const __amdgpu_buffer_rsrc_t vr = l2_rsrc(v_row + tb * v_st, vb);
    const uint32_t kbase = lds_addr(raw_k), vbase = lds_addr(raw_v);
#pragma unroll
    for (int t = 0; t < NRAW; ++t) {
      const int c = __builtin_amdgcn_readfirstlane(wave) + kChainWaves * t;
      constexpr int KIR = kChainTok / RPI;
      const int ci = c < KIR ? c : c - KIR;
      const int r = ci * RPI + lane / GL;
      if (c < KIR)
        dma16_nt(kr, kbase + uint32_t(ci * 1024), uint32_t((r * k_st + part * 8) * 2));
      else
        dma16_nt(vr, vbase + uint32_t(ci * 1024), uint32_t((r * v_st + part * 8) * 2));
    }
#pragma unroll
    for (int it = 0; it < IT; ++it) {
      const int lt = (tid + it * kChainThreads) / GL;
      rg[it] = g_row[tb * g_st + (lt < pnt ? lt : 0) * g_st];
    }
  };
  // prep (model/kvm_mixer.py:120-129, model/kvm_triton_mixer.py:429-446):
  // merge key / value rows of my share of update i (from the raw rows in
  // LDS), packed bf16, stored into merge buffer i % 4.
  auto prep = [&](int i) __attribute__((always_inline)) {
#pragma unroll
    for (int it = 0; it < IT; ++it) {
      const int lt = (tid + it * kChainThreads) / GL;
      float k[8], v[8];
      unpack8(*reinterpret_cast<const uint4 *>(&raw_k[lt * D + part * 8]), k);
      unpack8(*reinterpret_cast<const uint4 *>(&raw_v[lt * D + part * 8]), v);
      const float g = bf2f(rg[it]);
      prep_key<D>(k, part, L, ln_w, ln_b);
      float gk[8], gv[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        gk[e] = L.gate_keys ? k[e] * g : k[e];
        gv[e] = L.gate_values ? v[e] * g : v[e];
      }
      if (lt < pnt) {
        const uint32_t o = uint32_t(((pt0 + lt) * D + part * 8) * 2);
        st16<0>(l2_rsrc(gk_row + (i % 4) * buf_stride, n_tok * D * 2), o, pack8(gk));
        st16<0>(l2_rsrc(gv_row + (i % 4) * buf_stride, n_tok * D * 2), o, pack8(gv));
      }
    }
  };
  // Tag of the partials of update i (never 0: the entries are cleared to 0
  // at the start of a launch, so a workspace's old contents never match).
  auto tag_of = [](int i) __attribute__((always_inline)) { return uint32_t(0x8000u | uint32_t(i)); };
  __shared__ int fail_lds;

  // Prologue: prep(0), then the raw rows of update 1; the group barrier's
  // store wait (vmcnt(0)) also completes that DMA, and its workgroup barrier
  // makes the rows visible to every wave.
  __syncthreads();  // tok_lds, ln_w / ln_b and the owned rows are in LDS
  raw_dma(0);
  if (tid == 0) fail_lds = 0;
  // My partials in both buffers start cleared.
  for (int t = tid; t < n_tok; t += kChainThreads) {
    cs.part[rb * G + int64_t(t) * G + member] = make_uint2(0u, 0u);
    cs.part[part_stride + rb * G + int64_t(t) * G + member] = make_uint2(0u, 0u);
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  prep(0);
  __syncthreads();  // every wave has read the raw rows of update 0
  if (list.count > 1) raw_dma(1);
  arrive();
  if (!wait()) return;

  int snap_i = int(int64_t(list.u0) % snaps.ring);  // ring entry of snapshot u0 + p
  for (int p = 0; p <= list.count; ++p) {
    KVM_TS(0);
    const bool do_route = p < list.count;
    const bool do_prep = p + 1 < list.count;
    // Route operands of update p: my wave's 64 tokens (tokens >= n_tok read zero).
    uint4 bx[4][KS];
    auto load_bx = [&](int tt0, int tt1, int ks0, int ks1) __attribute__((always_inline)) {
      const __amdgpu_buffer_rsrc_t gr =
          l2_rsrc(gk_row + (p % 4) * buf_stride, n_tok * D * 2);
#pragma unroll
      for (int tt = tt0; tt < tt1; ++tt)
#pragma unroll
        for (int ks = ks0; ks < ks1; ++ks)
          bx[tt][ks] = l2_ld16(gr, ((wave * kTokWave + tt * 16 + (lane & 15)) * D + ks * 32 +
                                    (lane >> 4) * 8) * 2);
    };
    // Partials of update p - 1 for my token (tokens >= n_tok read zero and
    // are not waited for).
    uint4 pw[GM / 2];
    const __amdgpu_buffer_rsrc_t pr =
        l2_rsrc(part_row + ((p - 1) & 1) * part_stride, n_tok * G * 8);
    if (p >= 1) {
#pragma unroll
      for (int i = 0; i < GM / 2; ++i) pw[i] = l2_ld16(pr, (tid * GM + 2 * i) * 8);
    }
    // The next update's prep (raw rows already in LDS) while that load is
    // in flight.
    if (do_prep) prep(p + 1);
    if (p == 0) {
      load_bx(0, 4, 0, KS);
      __syncthreads();  // every wave has read the raw rows of update 1
    }
    KVM_TS(1);

    if (p >= 1) {
      // ---- combine(p - 1) and the lists of my slots.
      const int pi = p - 1;
      const int64_t u = int64_t(list.u0) + pi;
      // Wait (bounded) until every member's partial of my token carries the
      // tag of update p - 1, then keep the first argmax: larger score, then
      // lower slot (scores are MFMA sums started at +0, never -0 or NaN).
      bool ok_tok = false;
      {
        const uint32_t want = tag_of(pi);
        bool ok = tid >= n_tok;
        unsigned polls = 0;
        for (;;) {
          bool fresh = true;
#pragma unroll
          for (int i = 0; i < GM / 2; ++i) fresh &= (pw[i].y >> 16) == want && (pw[i].w >> 16) == want;
          ok |= fresh;
          if (__all(ok) || polls >= cs.max_polls) break;
          if ((polls & 255u) == 255u &&
              __hip_atomic_load(cs.abort_flag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT))
            break;
          __builtin_amdgcn_s_sleep(1);
          ++polls;
          if (!ok) {
#pragma unroll
            for (int i = 0; i < GM / 2; ++i) pw[i] = l2_ld16(pr, (tid * GM + 2 * i) * 8);
          }
        }
        ok_tok = ok && tid < n_tok;
        KVM_TS(7);
        if (!__all(ok)) {
          if ((tid & 63) == 0) {
            __hip_atomic_store(cs.abort_flag, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_fetch_or(cs.status, unsigned(KVM_STATUS_CHAIN_TIMEOUT), __ATOMIC_RELAXED,
                                  __HIP_MEMORY_SCOPE_AGENT);
            fail_lds = 1;
          }
        }
      }
      // The route operands of update p: every member stores its prepared
      // rows of update p before it publishes any partial of update p - 1,
      // so they are in L2 now.  Issued here, while the memory pipeline is
      // otherwise idle during the lists, they have landed long before the
      // gathers behind them are waited for.
      // The first half of the k-steps here, the rest in two quarters at the
      // refresh passes: a CU's vector memory pipeline moves about 64 bytes
      // per clock, so a burst of all of them would stall the issuing waves
      // and delay the gathers queued behind them.
      if (do_route) load_bx(0, 4, 0, KS / 2);
      KVM_TS(14);
      // Partials are route keys (see route(p)): the largest wins.
      uint64_t best = 0;
#pragma unroll
      for (int i = 0; i < GM / 2; ++i) {
        const uint64_t k0 = (uint64_t(pw[i].x) << 32) | (pw[i].y & 0xffffu);
        const uint64_t k1 = (uint64_t(pw[i].z) << 32) | (pw[i].w & 0xffffu);
        best = k0 > best ? k0 : best;
        best = k1 > best ? k1 : best;
      }
      int bi = (best >> 32) != 0 ? int(0xffffu - uint32_t(best & 0xffffu)) : -1;
      if (!ok_tok) bi = -1;  // past n_tok, or a partial that never arrived
      const bool mine = bi >= 0 && ((bi >> 4) % G) == member;
      const int my_loc = mine ? ((((bi >> 4) / G) << 4) | (bi & 15)) : -1;
      if (tid >= pt0 && tid < pt0 + pnt) {  // each member logs its prep share
        if (route_log) route_log[u * log_stride + rb + tid] = bi;
        if (append_log) append_log[u * log_stride + rb + tid] = 0;
      }
      // Tokens of my wave with the same local slot (ballots over its bits):
      // rank among them, and their count from the group's first lane.  A
      // wave's LDS stores complete in order, so the clear of its own row of
      // wsc precedes the counts it writes.
#pragma unroll
      for (int c = 0; c < OWN; c += 64) wsc[wave][c + lane] = 0;
      uint64_t eq = __ballot(mine);
#pragma unroll
      for (int bit = 0; bit < LOG2_OWN; ++bit) {
        const uint64_t m = __ballot(mine && ((my_loc >> bit) & 1));
        eq &= ((my_loc >> bit) & 1) ? m : ~m;
      }
      const int rank = int(__builtin_amdgcn_mbcnt_hi(uint32_t(eq >> 32),
                                                     __builtin_amdgcn_mbcnt_lo(uint32_t(eq), 0u)));
      if (mine && rank == 0) wsc[wave][my_loc] = __popcll(eq);
      __syncthreads();
      if (fail_lds) return;  // a partial never arrived: the launch is abandoned
      KVM_TS(15);
      // Every wave computes the exclusive prefix over slots (slot e's first
      // list position, and its position after the tokens of lower waves)
      // itself, so that each places its own tokens without another barrier;
      // wave 0 also keeps off / cnt for the sums.
      int ntot;  // tokens routed to my slots
      {
        constexpr int PER = OWN / 64;  // consecutive slots per lane
        int run[PER], mine_pre[PER], tot = 0;
#pragma unroll
        for (int x = 0; x < PER; ++x) {
          const int e = lane * PER + x;
          run[x] = 0;
          mine_pre[x] = 0;
#pragma unroll
          for (int w = 0; w < kChainWaves; ++w) {
            if (w == wave) mine_pre[x] = run[x];
            run[x] += wsc[w][e];
          }
          tot += run[x];
        }
        int incl = tot;
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
          const int y = __shfl_up(incl, o);
          if (lane >= o) incl += y;
        }
        int base = incl - tot;
        int pos[PER];
#pragma unroll
        for (int x = 0; x < PER; ++x) {
          if (wave == 0) {
            off[lane * PER + x] = base;
            cnt[lane * PER + x] = run[x];
          }
          pos[x] = base + mine_pre[x];
          base += run[x];
        }
        ntot = __shfl(incl, 63);
        int at = 0;
#pragma unroll
        for (int x = 0; x < PER; ++x) {
          const int v = __shfl(pos[x], (mine ? my_loc : 0) / PER);
          if ((mine ? my_loc : 0) % PER == x) at = v;
        }
        if (mine) sorted[at + rank] = tid;
      }
      __syncthreads();
      KVM_TS(2);

      // ---- merge(p - 1) (model/kvm_mixer.py:329-335).  The routed token
      // rows are staged in LDS (all loads of a chunk in flight together),
      // then each slot sums its rows in token order.
      const __amdgpu_buffer_rsrc_t gkr =
          l2_rsrc(gk_row + (pi % 4) * buf_stride, n_tok * D * 2);
      const __amdgpu_buffer_rsrc_t gvr =
          l2_rsrc(gv_row + (pi % 4) * buf_stride, n_tok * D * 2);
      // Sums of the half of my slots being merged (registers for HP passes).
      float sk[HP][8], sv[HP][8];
      // Routed rows are staged STAGE at a time, straight from L2 into LDS
      // (device-scope LDS-DMA loads, no registers).  Wave w fills staged rows
      // RPI*ci .. RPI*ci + RPI - 1 for ci = w, w + 8, ...: the token indices
      // of all its instructions are read from LDS first (one wait), then the
      // key and the value row of each are issued.  Rows past ntot point past
      // the resource and are not written.
      auto gather = [&](int c0) __attribute__((always_inline)) {
        const uint32_t kbase = lds_addr(stage_k), vbase = lds_addr(stage_v);
        const int w0 = __builtin_amdgcn_readfirstlane(wave);
        constexpr int NG = KI / kChainWaves;
        static_assert(NG * kChainWaves == KI, "gather split");
        uint32_t to[NG];
#pragma unroll
        for (int t = 0; t < NG; ++t) {
          const int pos = c0 + (w0 + kChainWaves * t) * RPI + lane / GL;
          const int tok = sorted[min(pos, kFixedMaxTok - 1)];
          // Rows past ntot point past the resource (n_tok) and are not written.
          to[t] = uint32_t(((pos < ntot ? tok : n_tok) * D + part * 8) * 2);
        }
#pragma unroll
        for (int t = 0; t < NG; ++t) {
          const int ci = w0 + kChainWaves * t;
          if (c0 + ci * RPI < ntot) {  // instructions wholly past ntot are not issued
            dma16_l2(gkr, kbase + uint32_t(ci * 1024), to[t]);
            dma16_l2(gvr, vbase + uint32_t(ci * 1024), to[t]);
          }
        }
      };
      // Adds the staged rows c0 .. of the slots of half h to the sums, in
      // token order; `arrived`: wait for this wave's gathers, then for every
      // wave's (not needed when the rows were staged for an earlier half);
      // `release`: a barrier after the reads, before another gather reuses
      // the staging buffers (the merge's final barrier covers the last use).
      auto stage_sum = [&](int c0, int h, bool arrived, bool release) __attribute__((always_inline)) {
        const int nrow = min(STAGE, ntot - c0);
        if (arrived) {
          wait_vm<0>();
          __syncthreads();
        }
#pragma unroll
        for (int sp = 0; sp < HP; ++sp) {
          const int l = (h * HP + sp) * RPP + tid / GL;
          if (l < nown) {
            const int e0 = max(off[l], c0), e1 = min(off[l] + cnt[l], c0 + nrow);
            auto add_row = [&](uint4 rk, uint4 rv) __attribute__((always_inline)) {
              float fk[8], fv[8];
              unpack8(rk, fk);
              unpack8(rv, fv);
#pragma unroll
              for (int x = 0; x < 8; ++x) {
                sk[sp][x] += fk[x];
                sv[sp][x] += fv[x];
              }
            };
            auto row_k = [&](int e) { return *reinterpret_cast<const uint4 *>(&stage_k[(e - c0) * D + part * 8]); };
            auto row_v = [&](int e) { return *reinterpret_cast<const uint4 *>(&stage_v[(e - c0) * D + part * 8]); };
            int e = e0;
            if constexpr (OWN == 128) {
              // Four rows' LDS reads in flight at once: at 1024 slots the
              // routes are uneven enough that some slots sum tens of rows.
              // Still added in token order.
              for (; e + 4 <= e1; e += 4) {
                uint4 rk[4], rv[4];
#pragma unroll
                for (int u = 0; u < 4; ++u) {
                  rk[u] = row_k(e + u);
                  rv[u] = row_v(e + u);
                }
#pragma unroll
                for (int u = 0; u < 4; ++u) add_row(rk[u], rv[u]);
              }
            }
            for (; e < e1; ++e) add_row(row_k(e), row_v(e));
          }
        }
        if (release) __syncthreads();
      };
      // Refreshed attention rows: keys into LDS (route operands), keys and
      // values into snapshot u0 + p straight from registers (non-temporal:
      // the attention kernel reads them much later), and after the batch's
      // last update also into the state's attention rows.
      // Snapshot u0 + p: ring entry snap_i (advanced by one per phase).
      const __amdgpu_buffer_rsrc_t nk =
          l2_rsrc(snk_row + int64_t(snap_i) * snap_stride, snap_bytes);
      const __amdgpu_buffer_rsrc_t nv =
          l2_rsrc(snv_row + int64_t(snap_i) * snap_stride, snap_bytes);
      const bool fin = !do_route && list.final_rows != 0;
      uint16_t *s_ka = static_cast<uint16_t *>(st.s_k_attn);
      uint16_t *s_va = static_cast<uint16_t *>(st.s_v_attn);
      auto refresh = [&](int h) __attribute__((always_inline)) {
#pragma unroll
        for (int sp = 0; sp < HP; ++sp) {
          const int l = (h * HP + sp) * RPP + tid / GL;
          const int j = own_local_to_slot(l, G, member);
          const bool valid = l < nown && j < S;
          float k[8], v[8];
          unpack8(*reinterpret_cast<const uint4 *>(&own_sk[l * D + part * 8]), k);
          unpack8(*reinterpret_cast<const uint4 *>(&own_sv[l * D + part * 8]), v);
          if (valid && cnt[l] > 0) {  // state = bf16(state + bf16(sum))
            round_pack8(sk[sp]);
            round_pack8(sv[sp]);
#pragma unroll
            for (int e = 0; e < 8; ++e) {
              k[e] += sk[sp][e];
              v[e] += sv[sp][e];
            }
            *reinterpret_cast<uint4 *>(&own_sk[l * D + part * 8]) = round_pack8(k);
            *reinterpret_cast<uint4 *>(&own_sv[l * D + part * 8]) = round_pack8(v);
          }
          // Attention rows of the slot (kvm_seq.hpp attn_rows, in two steps;
          // the rows are only stored, so they are rounded by the packing).
          float ka[8];
#pragma unroll
          for (int e = 0; e < 8; ++e) ka[e] = k[e];
          layer_norm8<D>(ka, part, ln_w, ln_b, float(L.ln_eps));
          const uint4 kk = pack8(ka);
          const uint4 vv = attn_value8_packed<D>(v, own_vl[l]);
          if (valid) {
            *reinterpret_cast<uint4 *>(&own_k[l * STR + part * 8]) = kk;
            const uint32_t ao = uint32_t((j * D + part * 8) * 2);
            st16<kPolicyNT>(nk, ao, kk);
            st16<kPolicyNT>(nv, ao, vv);
            if (fin) {
              const int64_t so = (srow + j) * D + part * 8;
              *reinterpret_cast<uint4 *>(s_ka + so) = kk;
              *reinterpret_cast<uint4 *>(s_va + so) = vv;
            }
          }
          __builtin_amdgcn_sched_barrier(0);  // one slot pass at a time (register pressure)
          if (h == NH - 1 && sp == 0) {
            KVM_TS(11);
            if (do_route) load_bx(0, 4, KS * 3 / 4, KS);  // the last quarter of the route operands
          }
        }
      };
      auto zero_sums = [&]() __attribute__((always_inline)) {
#pragma unroll
        for (int sp = 0; sp < HP; ++sp)
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            sk[sp][e] = 0.f;
            sv[sp][e] = 0.f;
          }
      };
      gather(0);
      KVM_TS(8);
      if (ntot <= STAGE) {  // one staged round serves every half
#pragma unroll 1
        for (int h = 0; h < NH; ++h) {
          zero_sums();
          stage_sum(0, h, h == 0, false);
          if (h == 0) {
            KVM_TS(9);
            KVM_TS(10);
          }
          // The third quarter of the route operands with the last half (not
          // earlier: with them resident the earlier halves' sums would spill).
          if (h == NH - 1 && do_route) load_bx(0, 4, KS / 2, KS * 3 / 4);
          refresh(h);
        }
      } else {  // several rounds: each half gathers them again
#pragma unroll 1
        for (int h = 0; h < NH; ++h) {
          zero_sums();
          for (int c0 = 0; c0 < ntot; c0 += STAGE) {
            if (h > 0 || c0 > 0) gather(c0);
            stage_sum(c0, h, true, true);
          }
          if (h == NH - 1 && do_route) load_bx(0, 4, KS / 2, KS * 3 / 4);
          refresh(h);
          __syncthreads();  // every wave has read the staged rows before the next gather
        }
      }
      __syncthreads();
    }
    KVM_TS(3);

    if (do_route) {
      // ---- route(p) (model/kvm_fp32_routing_reference.py:30-34) against my
      // slots: per-lane maximum in increasing slot order (strict >), then
      // across the lane groups; larger score wins, ties go to the lower slot.
      float best[4];
      int bidx[4];
#pragma unroll
      for (int tt = 0; tt < 4; ++tt) {
        best[tt] = -INFINITY;
        bidx[tt] = -1;
      }
      for (int lt = 0; lt < nown; lt += 16) {
        const int jb = own_local_to_slot(lt, G, member);  // first slot of the block
        uint4 a[KS];
#pragma unroll
        for (int ks = 0; ks < KS; ++ks)
          a[ks] = *reinterpret_cast<const uint4 *>(
              &own_k[(lt + (lane & 15)) * STR + ks * 32 + (lane >> 4) * 8]);
        // Only a block holding sink slots or slots >= S needs the mask.
        const bool masked = jb < protect || jb + 16 > S;
        // k-steps outermost: the four token tiles' accumulations interleave
        // (each still sums its k-steps in order).
        f32x4 accs[4];
#pragma unroll
        for (int tt = 0; tt < 4; ++tt) accs[tt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ks = 0; ks < KS; ++ks)
#pragma unroll
          for (int tt = 0; tt < 4; ++tt)
            accs[tt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(a[ks]), as_bf16x8(bx[tt][ks]),
                                                               accs[tt], 0, 0, 0);
        // The raw rows of update p + 2 once the first block's products have
        // been issued: every route operand has arrived by then, so the DMA
        // queues behind nothing the route waits for, and the release wait
        // below completes it (every wave read the raw rows of update p + 1
        // at the start of this phase, before the lists' barriers).
        if (lt == 0 && p + 2 < list.count) {
          __builtin_amdgcn_sched_barrier(0);
          raw_dma(p + 2);
          __builtin_amdgcn_sched_barrier(0);
        }
        const int j0 = jb + (lane >> 4) * 4;  // slot of acc[0]
        if (masked) {
#pragma unroll
          for (int tt = 0; tt < 4; ++tt) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              const int j = j0 + i;
              const float sc = ((j >= protect) && (j < S)) ? accs[tt][i] : -INFINITY;
              const bool take = sc > best[tt];
              best[tt] = take ? sc : best[tt];
              bidx[tt] = take ? j : bidx[tt];
            }
          }
        } else {
          // The lane's four slots as a tree (the earlier slot keeps ties),
          // then against the running maximum: the same first maximum as a
          // scan in slot order, with independent chains per token tile.
#pragma unroll
          for (int tt = 0; tt < 4; ++tt) {
            const f32x4 acc = accs[tt];
            const bool t1 = acc[1] > acc[0], t3 = acc[3] > acc[2];
            const float v01 = t1 ? acc[1] : acc[0], v23 = t3 ? acc[3] : acc[2];
            const int i01 = t1 ? 1 : 0, i23 = t3 ? 3 : 2;
            const bool th = v23 > v01;
            const float vh = th ? v23 : v01;
            const int ih = th ? i23 : i01;
            const bool take = vh > best[tt];
            best[tt] = take ? vh : best[tt];
            bidx[tt] = take ? j0 + ih : bidx[tt];
          }
        }
      }
      KVM_TS(12);
      if (nown == 0 && p + 2 < list.count) raw_dma(p + 2);  // a member without slots
      // Release: this member's earlier stores (its prepared rows of update
      // p + 1) are in L2 before any of its partials of update p is.
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
      __syncthreads();
      KVM_TS(13);
      // Partials are route keys: {mono(score), tag << 16 | (0xffff - slot)},
      // compared as 64-bit integers (the tags are equal), so the maximum is
      // the largest score and, among equal scores, the lowest slot; no
      // candidate is {0, tag << 16}, below every real key.
      const uint32_t tg = tag_of(p) << 16;
#pragma unroll
      for (int tt = 0; tt < 4; ++tt) {
        const uint32_t bu = __float_as_uint(best[tt]);
        uint32_t khi = bidx[tt] >= 0 ? ((bu & 0x80000000u) ? ~bu : (bu | 0x80000000u)) : 0u;
        uint32_t klo = bidx[tt] >= 0 ? 0xffffu - uint32_t(bidx[tt]) : 0u;
#pragma unroll
        for (int r = 0; r < 2; ++r) {
          const uint32_t ohi = r == 0 ? xor16_lane(khi, lane) : xor32_lane(khi, lane);
          const uint32_t olo = r == 0 ? xor16_lane(klo, lane) : xor32_lane(klo, lane);
          const uint64_t mine = (uint64_t(khi) << 32) | klo, other = (uint64_t(ohi) << 32) | olo;
          const bool take = other > mine;
          khi = take ? ohi : khi;
          klo = take ? olo : klo;
        }
        const int t = wave * kTokWave + tt * 16 + lane;
        if (lane < 16 && t < n_tok)
          __builtin_amdgcn_raw_buffer_store_b64(
              __builtin_bit_cast(__attribute__((ext_vector_type(2))) unsigned, make_uint2(khi, tg | klo)),
              l2_rsrc(part_row + (p & 1) * part_stride, n_tok * G * 8), (t * G + member) * 8, 0, 0);
      }
      KVM_TS(4);
      KVM_TS(5);
      KVM_TS(6);
    }
    snap_i = snap_i + 1 == int(snaps.ring) ? 0 : snap_i + 1;
  }

  // ---- owned state back to the caller's arrays.
  for (int base = 0; base < nown; base += RPP) {
    const int l = base + tid / GL;
    if (l < nown) {
      const int j = own_local_to_slot(l, G, member);
      if (j < S) {
        const int64_t so = (srow + j) * D + part * 8;
        *reinterpret_cast<uint4 *>(s_k + so) = *reinterpret_cast<const uint4 *>(&own_sk[l * D + part * 8]);
        *reinterpret_cast<uint4 *>(s_v + so) = *reinterpret_cast<const uint4 *>(&own_sv[l * D + part * 8]);
      }
    }
  }
}

__global__ __launch_bounds__(256) void k_fill_u32(unsigned *p, int64_t n, unsigned v) {
  const int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x;
  if (i < n) p[i] = v;
}

}  // namespace

bool chain_plan(const kvm_layer &L, int64_t n_tok, int64_t max_slots, ChainPlan *p) {
  // Every member of a group must be resident at once: at most one
  // workgroup per compute unit of the current device.
  int dev = 0, cus = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
    return false;
  const int64_t limit = std::min<int64_t>(kChainMaxWorkgroups, cus);
  const int64_t rows = L.batch * L.kv_heads;
  const int64_t groups = (rows + 7) / 8 * 8;
  int G = groups * 16 <= limit ? 16 : 8;
  // More rows than one launch keeps resident: consecutive launches over
  // batches of rows (a multiple of 8, one group per XCD each).
  const int64_t batch_groups = std::min<int64_t>(groups, limit / G / 8 * 8);
  const int64_t tpw = ((n_tok + G - 1) / G + 15) / 16 * 16;
  if (tpw > kChainTok || batch_groups < 8 || n_tok < 1) return false;
  p->fixed = false;
  p->G = G;
  p->tpw = int(tpw);
  p->spm_max = int((max_slots + G - 1) / G);
  p->row_batch = int(batch_groups);
  p->workgroups = int(batch_groups * G);
  // ints of the lists, then the append selection's 8-byte keys (a power of
  // two of them) after one int of alignment padding.
  int64_t npow = 1;
  while (npow < n_tok) npow <<= 1;
  const int64_t dyn = (4 * n_tok + 3 * int64_t(p->spm_max) + 1) * 4 + npow * 8;
  if (dyn > 48 * 1024) return false;
  p->dyn_lds = size_t(dyn);
  return true;
}

bool chain_fixed_ok(const ChainPlan &p, const ChainList &list, int64_t n_tok) {
  if (n_tok > kFixedMaxTok || list.count < 1 || (p.G != 8 && p.G != 16)) return false;
  const int S = list.state_before[0];
  for (int i = 0; i < list.count; ++i)
    if (list.n_append[i] != 0 || list.state_before[i] != S) return false;
  // Owned slots per member: up to 64 at G = 16, up to 128 at G = 8.
  const int nblk = (S + 15) / 16;
  return (nblk + p.G - 1) / p.G * 16 <= (p.G == 8 ? kOwnMax : 64);
}

int64_t chain_scratch_bytes(const kvm_layer &L, int64_t n_tok) {
  const size_t tok = size_t(L.batch * L.kv_heads) * size_t(n_tok);
  auto a256 = [](size_t x) { return (x + 255) & ~size_t(255); };
  // four merge buffers of keys, four of values (buffer b at gk + b * rows * n_tok * D),
  // routes, novelty, two sets of per-member maxima (up to 16 members), counters
  return int64_t(2 * a256(4 * tok * size_t(L.head_dim) * 2) + 2 * a256(tok * 4) +
                 a256(2 * tok * 16 * 8) +
                 a256(size_t(kChainMaxWorkgroups) * kCounterStride * 4 + 256));
}

ChainScratch carve_chain_scratch(void *base, const kvm_layer &L, int64_t n_tok) {
  const size_t tok = size_t(L.batch * L.kv_heads) * size_t(n_tok);
  auto a256 = [](size_t x) { return (x + 255) & ~size_t(255); };
  unsigned char *p = static_cast<unsigned char *>(base);
  ChainScratch c;
  const size_t kb = tok * size_t(L.head_dim) * 2, ib = a256(tok * 4);
  const size_t kb4 = a256(4 * kb), pb = a256(2 * tok * 16 * 8);
  c.gk = reinterpret_cast<uint16_t *>(p);
  c.gv = reinterpret_cast<uint16_t *>(p + kb4);
  c.route = reinterpret_cast<int32_t *>(p + 2 * kb4);
  c.nov = reinterpret_cast<float *>(p + 2 * kb4 + ib);
  c.part = reinterpret_cast<uint2 *>(p + 2 * kb4 + 2 * ib);
  c.bar = reinterpret_cast<unsigned *>(p + 2 * kb4 + 2 * ib + pb);
  c.abort_flag = c.bar + size_t(kChainMaxWorkgroups) * kCounterStride;
  c.status = nullptr;  // set by the caller
  c.max_polls = kChainDefaultPolls;
  return c;
}

hipError_t launch_fill_u32(unsigned *p, int64_t n, unsigned v, hipStream_t stream) {
  if (n <= 0) return hipSuccess;
  hipLaunchKernelGGL(k_fill_u32, dim3(unsigned((n + 255) / 256)), dim3(256), 0, stream, p, n, v);
  return hipGetLastError();
}

hipError_t launch_chain(const kvm_layer &L, const kvm_seq &src, int64_t n_tok,
                        const kvm_state &st, const SnapRing &snaps, const ChainList &list,
                        const ChainScratch &cs, const ChainPlan &p, int32_t *route_log,
                        int32_t *append_log, hipStream_t stream) {
  if (list.count <= 0) return hipSuccess;
  const int rows = int(L.batch * L.kv_heads);
  const int64_t log_stride = int64_t(rows) * n_tok;
  const bool fixed = p.fixed && chain_fixed_ok(p, list, n_tok);
  for (int row0 = 0; row0 < rows; row0 += p.row_batch) {
    const int nrows = std::min(p.row_batch, rows - row0);
    // Barrier counters and the abort flag start at zero in every launch.
    hipError_t e = launch_fill_u32(cs.bar, kChainMaxWorkgroups * kCounterStride + 64, 0u, stream);
    if (e != hipSuccess) return e;
    const dim3 grid(unsigned((nrows + 7) / 8 * 8 * p.G)), blk(kChainThreads);
    if (fixed) {
      const int nt = int(n_tok);
      const bool own128 = ((list.state_before[0] + 15) / 16 + p.G - 1) / p.G * 16 > 64;  // G == 8 then
#define KVM_FIXED(DD, GG, OO)                                                                               \
  hipLaunchKernelGGL((k_chain_fixed<DD, GG, OO>), grid, blk, 0, stream, L, src, nt, st, snaps, list, cs, rows, \
                     row0, nrows, route_log, append_log, log_stride)
      if (L.head_dim == 128 && p.G == 8 && own128)
        KVM_FIXED(128, 8, 128);
      else if (L.head_dim == 128 && p.G == 8)
        KVM_FIXED(128, 8, 64);
      else if (L.head_dim == 128)
        KVM_FIXED(128, 16, 64);
      else if (p.G == 8 && own128)
        KVM_FIXED(64, 8, 128);
      else if (p.G == 8)
        KVM_FIXED(64, 8, 64);
      else
        KVM_FIXED(64, 16, 64);
#undef KVM_FIXED
    } else if (L.head_dim == 128) {
      hipLaunchKernelGGL(k_chain<128>, grid, blk, p.dyn_lds, stream, L, src, int(n_tok), st, snaps, list, cs,
                         rows, row0, nrows, p.G, p.tpw, p.spm_max, route_log, append_log, log_stride);
    } else {
      hipLaunchKernelGGL(k_chain<64>, grid, blk, p.dyn_lds, stream, L, src, int(n_tok), st, snaps, list, cs,
                         rows, row0, nrows, p.G, p.tpw, p.spm_max, route_log, append_log, log_stride);
    }
    e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

}  // namespace kvm

#ifdef KVM_CHAIN_TIMING
// Copies the phase timestamps (2 x 128 x 16 words) of the last timed launch.
extern "C" int kvm_chain_timing_read(void *dst, long words) {
  return int(hipMemcpyFromSymbol(dst, HIP_SYMBOL(kvm::g_chain_ts), size_t(words) * 8));
}
#endif
