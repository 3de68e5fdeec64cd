// Skinny GEMM of the decoder's decode step on gfx950: Y = X W^T for a few
// rows of X (M <= 16 tokens) against a bf16 weight W [N, K] (nn.Linear
// layout), fp32 accumulation, bf16 output (or relu(Y)^2, the MLP's
// activation).  The step is bound by streaming W from HBM once (2.7 GB per
// config-5 decode step); a vendor GEMM tuned for square shapes reads it at
// ~1.9 TB/s.
//
// A workgroup owns 16 rows of W (16 outputs per token; 8 in the half tiles
// described below, for narrow W and M <= 8) and its NW waves split
// K evenly; NW (1 to 16) is the largest power of two leaving each wave at
// least 256 of K.  A wave issues the loads of 256 of K before their MFMAs:
// 16 bytes per lane, lanes 0-15 / 16-31 / ... covering 64 contiguous bytes
// of each row; v_mfma_f32_16x16x32_bf16 takes W rows as the A
// operand and the tokens' X rows as the B operand (columns >= M read zero).
// The per-wave partial tiles are summed in wave order through LDS, so the
// result does not depend on timing.

#include "kvm_device.hpp"
#include "kvm_internal.hpp"

namespace kvm {
namespace {

// Load steps per lane in flight together: 256 of K per wave (8 full-tile
// steps of 32, 4 half-tile steps of 64), the share of K a wave gets in the
// usual shapes (NW is chosen to leave each wave at least 256), so that no
// MFMA of a dead step sits in the wave's dependent accumulation chain.
template <bool HALF>
constexpr int kSteps = HALF ? 4 : 8;

constexpr int kGemmHalfBelow = 256;  // full 16-row tiles from this many on

// Rotate within rows of 16 lanes by 8: lane l gets lane l ^ 8's value.
__device__ __forceinline__ uint4 swap_half_rows(uint4 u) {
  uint4 o;
  o.x = uint32_t(__builtin_amdgcn_mov_dpp(int(u.x), 0x128, 0xf, 0xf, false));
  o.y = uint32_t(__builtin_amdgcn_mov_dpp(int(u.y), 0x128, 0xf, 0xf, false));
  o.z = uint32_t(__builtin_amdgcn_mov_dpp(int(u.z), 0x128, 0xf, 0xf, false));
  o.w = uint32_t(__builtin_amdgcn_mov_dpp(int(u.w), 0x128, 0xf, 0xf, false));
  return o;
}

// HALF (M <= 8): a workgroup owns 8 rows of W, twice as many workgroups as
// full tiles, for matrices too narrow to fill the GPU with 16-row tiles.
// Lanes r = lane % 16 < 8 load k-step 2c of W row / token r, lanes r >= 8
// k-step 2c + 1 of row / token r - 8, so every lane's 16-byte load is used;
// the MFMA of step 2c reads the operands as loaded, that of step 2c + 1
// after a swap of the two half rows.  Output rows and tokens 0-7 of the
// 16 x 16 product then take only the wanted halves (rows >= 8 and columns
// >= 8 hold cross terms and are not written).
// PACKED: W comes pre-arranged in 1 KiB chunks, one per (tile of R rows,
// load step of KC k), each holding the 64 lanes' 16-byte A-operand pieces in
// lane order (see kvm_gemm_small_packed): every load instruction then reads
// one contiguous KiB instead of 16 (or 8) row pieces 2*K bytes apart.
template <int NW, bool HALF, bool PACKED>
__global__ __launch_bounds__(NW * 64) void k_gemm_small(const uint16_t *__restrict__ X, int64_t x_st,
                                                        const uint16_t *__restrict__ W, int64_t w_st,
                                                        uint16_t *__restrict__ Y, int64_t y_st, int M, int N,
                                                        int K, int epilogue) {
  constexpr int R = HALF ? 8 : 16;   // W rows (outputs) per workgroup
  constexpr int KC = HALF ? 64 : 32;  // k covered by one load of every lane
  __shared__ float red[NW][16][16];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int r = lane & 15, g = lane >> 4;
  const int jr = HALF ? (r & 7) : r;            // W row / token this lane loads
  const int kk = HALF ? (r >> 3) * 32 : 0;      // its k offset within a load step
  const int n0 = blockIdx.x * R;
  const int kq = K / NW;  // a multiple of 32
  const int kb = wave * kq, ke = kb + kq;
  const bool row_ok = n0 + jr < N, col_ok = jr < M;
  const uint16_t *wrow = W + int64_t(row_ok ? n0 + jr : 0) * w_st + g * 8;
  const uint16_t *xrow = X + int64_t(col_ok ? jr : 0) * x_st + g * 8;
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  for (int k0 = kb; k0 < ke; k0 += KC * kSteps<HALF>) {
    uint4 a[kSteps<HALF>], b[kSteps<HALF>];
#pragma unroll
    for (int c = 0; c < kSteps<HALF>; ++c) {
      const int k = k0 + KC * c + kk;
      const bool in = k < ke;
      if constexpr (PACKED) {
        const int64_t chunk = int64_t(blockIdx.x) * (K / KC) + (k0 + KC * c) / KC;
        a[c] = in ? *reinterpret_cast<const uint4 *>(W + (chunk * 64 + lane) * 8) : make_uint4(0, 0, 0, 0);
      } else {
        a[c] = (in && row_ok) ? *reinterpret_cast<const uint4 *>(wrow + k) : make_uint4(0, 0, 0, 0);
      }
      b[c] = (in && col_ok) ? *reinterpret_cast<const uint4 *>(xrow + k) : make_uint4(0, 0, 0, 0);
    }
#pragma unroll
    for (int c = 0; c < kSteps<HALF>; ++c) {
      acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(a[c]), as_bf16x8(b[c]), acc, 0, 0, 0);
      if constexpr (HALF)
        acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(swap_half_rows(a[c])),
                                                      as_bf16x8(swap_half_rows(b[c])), acc, 0, 0, 0);
    }
  }
  // C layout: lane holds rows n0 + 4g + i (outputs) of column r (token).
#pragma unroll
  for (int i = 0; i < 4; ++i) red[wave][4 * g + i][r] = acc[i];
  __syncthreads();
  for (int i = threadIdx.x; i < R * 16; i += NW * 64) {  // one (output, token) per thread
    const int n = i / 16, m = i % 16;
    if (m < M && n0 + n < N) {
      float s = 0.f;
#pragma unroll
      for (int w = 0; w < NW; ++w) s += red[w][n][m];
      if (epilogue == 1) {  // relu(y)^2 of the bf16 product, rounded once more
        const float q = fmaxf(rbf(s), 0.f);
        s = q * q;
      }
      Y[int64_t(m) * y_st + n0 + n] = uint16_t(f2bf(s));
    }
  }
}

}  // namespace

int gemm_small_tile_rows(int64_t M, int64_t N) {
  // Half tiles where full ones would leave some of the GPU's 256 CUs idle
  // (measured: N = 2048 at K = 2048 / 8192 runs 1.2x / 1.6x faster in half
  // tiles, N = 6224 and 8192 at K = 2048 run slower).
  return M <= 8 && (N + 15) / 16 < kGemmHalfBelow ? 8 : 16;
}

hipError_t launch_gemm_small(const void *x, int64_t x_st, const void *w, int64_t w_st, void *y, int64_t y_st,
                             int64_t M, int64_t N, int64_t K, int epilogue, bool packed, hipStream_t stream) {
  const bool half = gemm_small_tile_rows(M, N) == 8;
  // Waves per workgroup: up to K / 256 (a power of two <= 16 dividing K / 32;
  // K / 64 for packed half tiles, whose chunks span 64 of K).
  const int64_t kc = packed && half ? 64 : 32;
  int nw = 1;
  while (nw < 16 && K / (2 * nw) >= 256 && K % (kc * 2 * nw) == 0) nw *= 2;
  const dim3 grid(unsigned(half ? (N + 7) / 8 : (N + 15) / 16));
  const uint16_t *xp = static_cast<const uint16_t *>(x), *wp = static_cast<const uint16_t *>(w);
  uint16_t *yp = static_cast<uint16_t *>(y);
#define KVM_GEMM(NWV, H, P)                                                                                 \
  hipLaunchKernelGGL((k_gemm_small<NWV, H, P>), grid, dim3(NWV * 64), 0, stream, xp, x_st, wp, w_st, yp, y_st, \
                     int(M), int(N), int(K), epilogue)
#define KVM_GEMM_NW(H, P)            \
  switch (nw) {                      \
    case 1: KVM_GEMM(1, H, P); break;  \
    case 2: KVM_GEMM(2, H, P); break;  \
    case 4: KVM_GEMM(4, H, P); break;  \
    case 8: KVM_GEMM(8, H, P); break;  \
    default: KVM_GEMM(16, H, P); break; \
  }
  if (half) {
    if (packed) {
      KVM_GEMM_NW(true, true)
    } else {
      KVM_GEMM_NW(true, false)
    }
  } else {
    if (packed) {
      KVM_GEMM_NW(false, true)
    } else {
      KVM_GEMM_NW(false, false)
    }
  }
#undef KVM_GEMM_NW
#undef KVM_GEMM
  return hipGetLastError();
}

}  // namespace kvm
