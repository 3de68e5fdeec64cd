// Token-source addressing and the row transforms shared by the update
// kernels (device code).
#pragma once

#include "kvm_device.hpp"
#include "kvm_internal.hpp"

namespace kvm {

__device__ __forceinline__ int64_t seq_tok(const kvm_seq &s, int64_t t) {
  return s.ring > 0 ? (t % s.ring) : t;
}
__device__ __forceinline__ const uint16_t *seq_k(const kvm_seq &s, int b,
                                                 int h, int64_t t) {
  return static_cast<const uint16_t *>(s.k) + b * s.k_sb + h * s.k_sh +
         seq_tok(s, t) * s.k_st;
}
__device__ __forceinline__ const uint16_t *seq_v(const kvm_seq &s, int b,
                                                 int h, int64_t t) {
  return static_cast<const uint16_t *>(s.v) + b * s.v_sb + h * s.v_sh +
         seq_tok(s, t) * s.v_st;
}
__device__ __forceinline__ float seq_g(const kvm_seq &s, int b, int h,
                                       int64_t t) {
  const uint16_t *g = static_cast<const uint16_t *>(s.gate) + b * s.g_sb +
                      h * s.g_sh + seq_tok(s, t) * s.g_st;
  return bf2f(*g);
}

// prep(k) = LayerNorm_s(k with dims < r zeroed), rounded to bf16
// (model/kvm_mixer.py:120-129).  w / b: ln_s_k weight and bias (global or
// LDS; kernels that keep many loads in flight pass an LDS copy so that
// reading them does not wait for those loads).
template <int D>
__device__ __forceinline__ void prep_key(float (&k)[8], int part, const kvm_layer &L,
                                         const float *w, const float *b) {
  const int r = int(L.rope_partial_dim);
  if ((r & 7) == 0) {  // a lane's 8 dims are zeroed together (one condition per lane)
    const bool z = part * 8 < r;
#pragma unroll
    for (int i = 0; i < 8; ++i) k[i] = z ? 0.f : k[i];
  } else {
#pragma unroll
    for (int i = 0; i < 8; ++i)
      if (part * 8 + i < r) k[i] = 0.f;
  }
  layer_norm8<D>(k, part, w, b, float(L.ln_eps));
  round_pack8(k);
}
template <int D>
__device__ __forceinline__ void prep_key(float (&k)[8], int part, const kvm_layer &L) {
  prep_key<D>(k, part, L, static_cast<const float *>(L.ln_weight),
              static_cast<const float *>(L.ln_bias));
}

// Attention rows of one slot from its (bf16) key / value sums and vlen.
template <int D>
__device__ __forceinline__ void attn_rows(const float (&sk)[8], const float (&sv)[8], float vlen,
                                          int part, const kvm_layer &L, const float *w,
                                          const float *b, float (&ka)[8], float (&va)[8]) {
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    ka[i] = sk[i];
    va[i] = sv[i];
  }
  layer_norm8<D>(ka, part, w, b, float(L.ln_eps));
  round_pack8(ka);
  attn_value8<D>(va, vlen);
}
template <int D>
__device__ __forceinline__ void attn_rows(const float (&sk)[8], const float (&sv)[8], float vlen,
                                          int part, const kvm_layer &L, float (&ka)[8],
                                          float (&va)[8]) {
  attn_rows<D>(sk, sv, vlen, part, L, static_cast<const float *>(L.ln_weight),
               static_cast<const float *>(L.ln_bias), ka, va);
}

}  // namespace kvm
