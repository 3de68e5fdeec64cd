// Device-side helpers shared by the KVM kernels (gfx950, wave64).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace kvm {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kWave = 64;

// Workgroups of a 1-D grid are dispatched round-robin over the 8 XCDs (each
// with its own L2).  This renumbering gives each XCD a contiguous range of
// logical workgroup ids, so neighbouring logical ids (which share operands)
// run on one XCD close together in time.
__device__ __forceinline__ int xcd_contiguous(int bid, int n) {
  constexpr int kXcd = 8;
  const int x = bid % kXcd, jx = bid / kXcd;
  const int q = n / kXcd, r = n % kXcd;
  return x * q + min(x, r) + jx;
}

// bfloat16 <-> float.  float -> bfloat16 rounds to nearest even (the
// rounding torch uses for every float -> bfloat16 conversion), done by the
// gfx950 instruction v_cvt_pk_bf16_f32.
__device__ __forceinline__ float bf2f(uint32_t bits16) {
  return __uint_as_float(bits16 << 16);
}
__device__ __forceinline__ uint32_t pack2bf(float a, float b) {
  const f32x2_t v = {a, b};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_t));
}
__device__ __forceinline__ uint32_t f2bf(float f) {
  return pack2bf(f, 0.f) & 0xffffu;
}
// Round a float to the nearest bfloat16 value, kept as float.
__device__ __forceinline__ float rbf(float f) { return bf2f(f2bf(f)); }

// 8 consecutive bf16 <-> 8 floats (one 16-byte access).
__device__ __forceinline__ void unpack8(const uint4 u, float (&x)[8]) {
  x[0] = __uint_as_float(u.x << 16);
  x[1] = __uint_as_float(u.x & 0xffff0000u);
  x[2] = __uint_as_float(u.y << 16);
  x[3] = __uint_as_float(u.y & 0xffff0000u);
  x[4] = __uint_as_float(u.z << 16);
  x[5] = __uint_as_float(u.z & 0xffff0000u);
  x[6] = __uint_as_float(u.w << 16);
  x[7] = __uint_as_float(u.w & 0xffff0000u);
}
__device__ __forceinline__ uint4 pack8(const float (&x)[8]) {
  uint4 u;
  u.x = pack2bf(x[0], x[1]);
  u.y = pack2bf(x[2], x[3]);
  u.z = pack2bf(x[4], x[5]);
  u.w = pack2bf(x[6], x[7]);
  return u;
}
__device__ __forceinline__ void load8(const uint16_t *p, float (&x)[8]) {
  unpack8(*reinterpret_cast<const uint4 *>(p), x);
}
__device__ __forceinline__ void store8(uint16_t *p, const float (&x)[8]) {
  *reinterpret_cast<uint4 *>(p) = pack8(x);
}
// Rounds 8 floats to bfloat16 in place (rbf of each, two per conversion)
// and returns them packed.
__device__ __forceinline__ uint4 round_pack8(float (&x)[8]) {
  const uint4 u = pack8(x);
  unpack8(u, x);
  return u;
}

__device__ __forceinline__ bf16x8 as_bf16x8(const uint4 u) {
  return __builtin_bit_cast(bf16x8, u);
}

// DPP lane moves within rows of 16 lanes (VALU, no LDS round trip).  Every
// pattern below reads a valid lane, so the `old` operand (0) is never used;
// being the identity of addition, it lets the compiler fold the move into
// the consuming v_add_f32 (v_add_f32_dpp: one instruction per step).
template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
  return __builtin_bit_cast(float,
                            __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xf, 0xf, false));
}
constexpr int kDppQuadXor1 = 0xB1;      // quad_perm [1,0,3,2]
constexpr int kDppQuadXor2 = 0x4E;      // quad_perm [2,3,0,1]
constexpr int kDppRowRor4 = 0x124;      // rotate right by 4 within 16 lanes
constexpr int kDppRowRor8 = 0x128;      // rotate right by 8 within 16 lanes
constexpr int kDppRowHalfMirror = 0x141;  // lane i -> 7 - i within 8 lanes

// Sum over aligned groups of G consecutive lanes (G a power of two <= 64);
// every lane of a group gets the same value.  Groups of 8 and 16 use DPP.
template <int G>
__device__ __forceinline__ float group_sum(float v) {
  if constexpr (G == 16) {
    v += dpp<kDppRowRor8>(v);
    v += dpp<kDppRowRor4>(v);
    v += dpp<kDppQuadXor2>(v);
    v += dpp<kDppQuadXor1>(v);
  } else if constexpr (G == 8) {
    v += dpp<kDppRowHalfMirror>(v);
    v += dpp<kDppQuadXor2>(v);
    v += dpp<kDppQuadXor1>(v);
  } else {
#pragma unroll
    for (int o = G / 2; o >= 1; o >>= 1) v += __shfl_xor(v, o);
  }
  return v;
}
template <int G>
__device__ __forceinline__ float group_max(float v) {
#pragma unroll
  for (int o = G / 2; o >= 1; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
  return v;
}

// LayerNorm of one D-wide row held as 8 floats in each of D/8 consecutive
// lanes (lane part p holds dims 8p..8p+7).  Two-pass mean / biased
// variance in fp32, y = (x - mean) * (1 / sqrt(var + eps)) * w + b, the
// formula of torch.nn.functional.layer_norm.
template <int D>
__device__ __forceinline__ void layer_norm8(float (&x)[8], int part,
                                            const float *__restrict__ w,
                                            const float *__restrict__ b,
                                            float eps) {
  constexpr int G = D / 8;
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < 8; ++i) s += x[i];
  s = group_sum<G>(s);
  const float mean = s / float(D);
  float q = 0.f;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const float c = x[i] - mean;
    q += c * c;
  }
  q = group_sum<G>(q);
  const float rstd = 1.0f / sqrtf(q / float(D) + eps);
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int d = part * 8 + i;
    x[i] = (x[i] - mean) * rstd * w[d] + b[d];
  }
}

// Euclidean norm of a D-wide row held as 8 floats per lane in D/8 lanes.
template <int D>
__device__ __forceinline__ float row_norm8(const float (&x)[8]) {
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < 8; ++i) s += x[i] * x[i];
  return sqrtf(group_sum<D / 8>(s));
}

// Value row as the state contributes it to attention:
// bf16(normalize(v) * vlen), normalize(v) = v / max(|v|, 1e-12)
// (torch.nn.functional.normalize; model/kvm_mixer.py:205-206).
// The quotients use one division per row: r = 1/n correctly rounded,
// q0 = v * r, then one correction q = q0 + r * fma(-q0, n, v) (Markstein's
// method), which gives the correctly rounded v / n for normal operands; it
// was checked bit-identical to v / n on gfx950 over 2^31 random operands.
// attn_value8_packed returns the row packed; attn_value8 rounds in place.
template <int D>
__device__ __forceinline__ uint4 attn_value8_packed(const float (&v)[8], float vlen) {
  const float n = fmaxf(row_norm8<D>(v), 1e-12f);
  const float r = 1.0f / n;
  float o[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const float q0 = v[i] * r;
    const float q = __builtin_fmaf(__builtin_fmaf(-q0, n, v[i]), r, q0);
    o[i] = q * vlen;
  }
  return pack8(o);
}
template <int D>
__device__ __forceinline__ void attn_value8(float (&v)[8], float vlen) {
  unpack8(attn_value8_packed<D>(v, vlen), v);
}

}  // namespace kvm
