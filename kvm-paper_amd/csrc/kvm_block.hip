// The decoder block's elementwise work around its mixer and MLP on gfx950:
// residual add, LayerNorm and the MLP's token shift in one pass.
//
// Reference: model/rwkv7_backbone.py:180-235 (Block.forward: x + s * f(ln(x))
// for the mixer and the MLP, the final ln after the last block) and
// :163-177 with model/tokenshift.py:11-37 (the MLP's token shift, fallback
// "zero", and its carried last row).  In the reference these are separate
// torch ops (add, layer_norm, sub / mul / add, copy), each reading and
// writing the [B, T, W] tensor; here a row is read once (plus the first row
// of a run once more, below) and each output written once.
//
// One wave per token row, kRun consecutive tokens of one sequence per wave:
// lane l holds the 16-byte chunks l, l + 64, ... of the row (8 bf16 each).
// The token shift takes the previous token's normalised row from registers;
// the first row of a run recomputes its predecessor's (or, at t = 0, takes
// the carried row, or zeros).
//
// Rounding follows the torch ops: the residual is bf16(x + s * y) when s is a
// power of two (one fused add) and bf16(x + bf16(y * s)) otherwise; the
// LayerNorm computes in fp32 (two-pass mean and biased variance) and rounds
// once; the shift rounds after each of its three ops.  Only the LayerNorm's
// fp32 reduction order differs from torch's, which can move a normalised
// value by one bf16 ulp.

#include "kvm_device.hpp"
#include "kvm_internal.hpp"

namespace kvm {
namespace {

constexpr int kRun = 8;  // tokens per wave for seq_len > 1

template <int NC>
struct Row {
  float v[NC][8];
};

// Every load of this file is issued without a branch around it (chunk
// indices past the row's end are clamped, a NULL operand is replaced by a
// valid one) and its value is selected where it is first used: a load whose
// value is selected at a branch join makes the wave wait for it there, which
// turns independent loads into one round trip each.
__device__ __forceinline__ uint4 ld16(const void *base, int64_t chunk) {
  return reinterpret_cast<const uint4 *>(base)[chunk];
}
__device__ __forceinline__ uint4 keep_if(bool in, uint4 v) {
  return in ? v : make_uint4(0, 0, 0, 0);
}

// The per-channel parameters of a lane's chunks (packed bf16), loaded once
// per wave before the first row so that their latency overlaps the rows'.
// Chunks past the row's end hold a clamped chunk's values (never used).
template <int NC>
struct Params {
  uint4 w[NC], b[NC], mix[NC];
};

template <int NC>
__device__ __forceinline__ void load_params(const kvm_add_norm_desc &P, int lane, bool shift, Params<NC> &p) {
  const int nch = int(P.width / 8);
  const void *mix = shift ? P.mix : P.ln_w;
#pragma unroll
  for (int j = 0; j < NC; ++j) {
    const int c = min(lane + 64 * j, nch - 1);
    p.w[j] = ld16(P.ln_w, c);
    p.b[j] = ld16(P.ln_b, c);
    p.mix[j] = ld16(mix, c);
  }
}

// The raw 16-byte chunks of row `r` (flat token index) of x and y (y: x's
// when there is none); chunks past the row's end hold a clamped chunk.
template <int NC>
struct Raw {
  uint4 x[NC], y[NC];
};

template <int NC>
__device__ __forceinline__ void fetch_row(const kvm_add_norm_desc &P, int64_t r, int lane, Raw<NC> &raw) {
  const int nch = int(P.width / 8);
  const void *y = P.y ? P.y : P.x;
#pragma unroll
  for (int j = 0; j < NC; ++j) {
    const int64_t e = r * nch + min(lane + 64 * j, nch - 1);
    raw.x[j] = ld16(P.x, e);
    raw.y[j] = ld16(y, e);
  }
}

// Residual sum x + s * y of a fetched row (zeros past the row's end).
template <int NC>
__device__ __forceinline__ void residual_row(const kvm_add_norm_desc &P, int lane, const Raw<NC> &raw,
                                             Row<NC> &out) {
  const float s = float(P.alpha);
  const int nch = int(P.width / 8);
#pragma unroll
  for (int j = 0; j < NC; ++j) {
    const bool in = lane + 64 * j < nch;
    float x[8];
    unpack8(keep_if(in, raw.x[j]), x);
    if (P.y) {
      float y[8];
      unpack8(keep_if(in, raw.y[j]), y);
#pragma unroll
      for (int i = 0; i < 8; ++i) x[i] = P.round_product ? rbf(x[i] + rbf(y[i] * s)) : rbf(x[i] + s * y[i]);
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) out.v[j][i] = x[i];
  }
}

// Sum over the wave, the same value in every lane: DPP sums within each row
// of 16 lanes, then the four row sums read from lanes 0, 16, 32, 48 and
// added in a fixed order (no LDS round trips).
__device__ __forceinline__ float wave_sum(float v) {
  v = group_sum<16>(v);
  const int b = __builtin_bit_cast(int, v);
  const float r0 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 0));
  const float r1 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 16));
  const float r2 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 32));
  const float r3 = __builtin_bit_cast(float, __builtin_amdgcn_readlane(b, 48));
  return (r0 + r1) + (r2 + r3);
}

// bf16 LayerNorm of `x` into `h` (whole-wave reductions).
template <int NC>
__device__ __forceinline__ void norm_row(const kvm_add_norm_desc &P, int lane, const Params<NC> &p,
                                         const Row<NC> &x, Row<NC> &h) {
  const int nch = int(P.width / 8);
  const float inv_w = 1.0f / float(P.width);
  float s = 0.f;
#pragma unroll
  for (int j = 0; j < NC; ++j)
#pragma unroll
    for (int i = 0; i < 8; ++i) s += x.v[j][i];
  const float mean = wave_sum(s) * inv_w;
  float q = 0.f;
#pragma unroll
  for (int j = 0; j < NC; ++j) {
    if (lane + 64 * j < nch) {
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const float d = x.v[j][i] - mean;
        q += d * d;
      }
    }
  }
  const float rstd = 1.0f / sqrtf(wave_sum(q) * inv_w + float(P.eps));
#pragma unroll
  for (int j = 0; j < NC; ++j) {
    const int c = lane + 64 * j;
    if (c < nch) {
      float w[8], b[8];
      unpack8(p.w[j], w);
      unpack8(p.b[j], b);
#pragma unroll
      for (int i = 0; i < 8; ++i) h.v[j][i] = rbf((x.v[j][i] - mean) * rstd * w[i] + b[i]);
    } else {
#pragma unroll
      for (int i = 0; i < 8; ++i) h.v[j][i] = 0.f;
    }
  }
}

template <int NC>
__device__ __forceinline__ void store_row(void *dst, int64_t r, int64_t width, int lane, const Row<NC> &x) {
  const int nch = int(width / 8);
#pragma unroll
  for (int j = 0; j < NC; ++j) {
    const int c = lane + 64 * j;
    if (c < nch) store8(static_cast<uint16_t *>(dst) + r * width + int64_t(c) * 8, x.v[j]);
  }
}

template <int NC>
__global__ __launch_bounds__(256) void k_add_norm(kvm_add_norm_desc P, int run) {
  const int lane = threadIdx.x & 63;
  const int64_t T = P.seq_len;
  const int64_t runs = (T + run - 1) / run;
  const int64_t wv = int64_t(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (wv >= P.batch * runs) return;  // wave-uniform
  const int64_t b = wv / runs, t0 = (wv % runs) * run;
  const int nch = int(P.width / 8);
  const bool shift = P.mix && P.out_shift;
  Params<NC> prm;
  load_params<NC>(P, lane, shift, prm);
  const int64_t t_end = t0 + run < T ? t0 + run : T;
  Raw<NC> next;  // the next row's loads are in flight while a row is processed
  fetch_row<NC>(P, b * T + t0, lane, next);
  // Normalised row of the token before the current one, packed (its values
  // are bf16 already): half the registers of the float row.
  uint4 carry[NC];
  if (shift) {
    if (t0 > 0) {
      Raw<NC> raw;
      fetch_row<NC>(P, b * T + t0 - 1, lane, raw);
      Row<NC> x, h;
      residual_row<NC>(P, lane, raw, x);
      norm_row<NC>(P, lane, prm, x, h);
#pragma unroll
      for (int j = 0; j < NC; ++j) carry[j] = pack8(h.v[j]);
    } else {
      const void *prev = P.prev ? P.prev : P.x;
#pragma unroll
      for (int j = 0; j < NC; ++j) carry[j] = ld16(prev, b * nch + min(lane + 64 * j, nch - 1));
#pragma unroll
      for (int j = 0; j < NC; ++j) carry[j] = keep_if(P.prev && lane + 64 * j < nch, carry[j]);
    }
  }
#pragma unroll 1
  for (int64_t t = t0; t < t_end; ++t) {
    const int64_t r = b * T + t;
    const Raw<NC> cur = next;
    if (t + 1 < t_end) fetch_row<NC>(P, r + 1, lane, next);
    Row<NC> x, h;
    residual_row<NC>(P, lane, cur, x);
    if (P.out_x) store_row<NC>(P.out_x, r, P.width, lane, x);
    norm_row<NC>(P, lane, prm, x, h);
    if (P.out_h) store_row<NC>(P.out_h, r, P.width, lane, h);
    if (P.state_out && t == T - 1) store_row<NC>(P.state_out, b, P.width, lane, h);
    if (shift) {
#pragma unroll
      for (int j = 0; j < NC; ++j) {
        const int c = lane + 64 * j;
        if (c < nch) {
          float m[8], cv[8], o[8];
          unpack8(prm.mix[j], m);
          unpack8(carry[j], cv);
#pragma unroll
          for (int i = 0; i < 8; ++i) o[i] = rbf(h.v[j][i] + rbf(m[i] * rbf(cv[i] - h.v[j][i])));
          store8(static_cast<uint16_t *>(P.out_shift) + r * P.width + int64_t(c) * 8, o);
        }
        carry[j] = pack8(h.v[j]);
      }
    }
  }
}

}  // namespace

hipError_t launch_add_norm(const kvm_add_norm_desc &P, hipStream_t stream) {
  const int run = P.seq_len > 1 ? kRun : 1;
  const int64_t waves = P.batch * ((P.seq_len + run - 1) / run);
  const dim3 grid(unsigned((waves + 3) / 4));
  const int64_t nch = P.width / 8;
  if (nch <= 64)
    hipLaunchKernelGGL(k_add_norm<1>, grid, dim3(256), 0, stream, P, run);
  else if (nch <= 128)
    hipLaunchKernelGGL(k_add_norm<2>, grid, dim3(256), 0, stream, P, run);
  else if (nch <= 256)
    hipLaunchKernelGGL(k_add_norm<4>, grid, dim3(256), 0, stream, P, run);
  else
    hipLaunchKernelGGL(k_add_norm<8>, grid, dim3(256), 0, stream, P, run);
  return hipGetLastError();
}

}  // namespace kvm
