// LDS tiles of 64 rows x D bf16 shared by the prefill attention kernels
// (forward and backward) on gfx950: the block image, its LDS-DMA fill and the
// per-lane MFMA fragment reads.
#pragma once

#include "kvm_device.hpp"

namespace kvm {
namespace tile {

constexpr int BN = 64;   // rows (keys or queries) per LDS block
constexpr float kLog2e = 1.4426950408889634f;
constexpr int kXcds = 8;
// Buffer resource word 3 for raw (unformatted, unswizzled) dword access with
// range checking: out-of-range loads return zero (and LDS-DMA lanes out of
// range write nothing).
constexpr int kBufWord3 = 0x00020000;

typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef short v4i16 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void lds_void;
typedef __attribute__((address_space(3))) v4i16 lds_v4i16;

__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
  const f32x2 v = {a, b};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2));
}

// LDS image of one K (or V) block of 64 keys: D/32 column groups of 4 KiB,
// each [64 keys][64 bytes]; byte of (key r, 16-byte unit u) =
// (u/4)*4096 + r*64 + ((u%4) ^ (2 * bit2(r)))*16.
template <int D>
struct Lay {
  static constexpr int GROUPS = D / 32;
  static constexpr int BLK = GROUPS * 4096;  // bytes of one K (or V) block
  static constexpr int BUF = 2 * BLK;        // K block then V block
  static constexpr int CHUNKS = BLK / 1024;  // DMA instructions per K (or V) block
};

// Resource over keys [0, nvalid) of a range starting at p with row stride
// `stride` elements.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t key_rsrc(const uint16_t *p, int64_t stride,
                                                          int nvalid) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t *>(p), (short)0,
                                           int(nvalid * stride * 2), kBufWord3);
}

// 16-byte-per-lane buffer load into LDS at M0 + 16 * lane.  Issued from
// inline assembly: the compiler would otherwise order every later LDS read
// behind it (it cannot tell the DMA target from the buffer being read).  Its
// completion is awaited explicitly with s_waitcnt vmcnt(0).
// M0 is written inside the statement and not declared clobbered (the compiler
// rejects M0 as a clobber): this is sound only while no compiled code of the
// kernel keeps a value of its own in M0, which holds for these kernels (their
// only M0 writes are these statements; checked in the generated assembly).
__device__ __forceinline__ void dma16(__amdgpu_buffer_rsrc_t r, uint32_t lds_addr, uint32_t voff) {
  asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds"
               :: "s"(lds_addr), "v"(voff), "s"(r) : "memory");
}

// 4-byte-per-lane buffer load into LDS at M0 + 4 * lane (the same rules as
// dma16; each lane's dword is range-checked on its own).
__device__ __forceinline__ void dma4(__amdgpu_buffer_rsrc_t r, uint32_t lds_addr, uint32_t voff) {
  asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dword %1, %2, 0 offen lds"
               :: "s"(lds_addr), "v"(voff), "s"(r) : "memory");
}

// DMA of one block (keys [0, nvalid) of both ranges, set by the resources)
// into the buffer at LDS byte address `buf`.  Instruction c fills keys
// 16*(c%4) .. +15 of column group c/4; wave w of NW issues c = w, w + NW, ...
// `ko`/`vo`: lane offsets within an instruction, key lane/4, unit
// (lane%4) ^ swap of that key.
template <int D, int NW>
__device__ __forceinline__ void issue_block(uint32_t buf, __amdgpu_buffer_rsrc_t kr,
                                            __amdgpu_buffer_rsrc_t vr, uint32_t ko, uint32_t vo,
                                            uint32_t kstride_b, uint32_t vstride_b, int wave) {
  constexpr int PER = Lay<D>::CHUNKS / NW;
  static_assert(Lay<D>::CHUNKS % NW == 0, "DMA instructions split evenly over the waves");
#pragma unroll
  for (int t = 0; t < PER; ++t) {
    const int c = wave + NW * t;
    const int cg = c >> 2, rq = c & 3;
    dma16(kr, buf + uint32_t(cg * 4096 + rq * 1024),
          ko + uint32_t(16 * rq) * kstride_b + uint32_t(cg * 64));
  }
#pragma unroll
  for (int t = 0; t < PER; ++t) {
    const int c = wave + NW * t;
    const int cg = c >> 2, rq = c & 3;
    dma16(vr, buf + uint32_t(Lay<D>::BLK + cg * 4096 + rq * 1024),
          vo + uint32_t(16 * rq) * vstride_b + uint32_t(cg * 64));
  }
}

// DMA of one K (or V) block image (keys [0, nvalid) set by the resource) into
// LDS byte address `img`: the instructions of issue_block for one half.
template <int D, int NW>
__device__ __forceinline__ void issue_image(uint32_t img, __amdgpu_buffer_rsrc_t r, uint32_t o,
                                            uint32_t stride_b, int wave) {
  constexpr int PER = Lay<D>::CHUNKS / NW;
  static_assert(Lay<D>::CHUNKS % NW == 0, "DMA instructions split evenly over the waves");
#pragma unroll
  for (int t = 0; t < PER; ++t) {
    const int c = wave + NW * t;
    const int cg = c >> 2, rq = c & 3;
    dma16(r, img + uint32_t(cg * 4096 + rq * 1024), o + uint32_t(16 * rq) * stride_b + uint32_t(cg * 64));
  }
}

// Zero the rows [nv, 64) of one half of a buffer (a block shorter than 64
// rows): the DMA leaves them untouched, and the weights that meet them are
// zero, so stale bytes must not be Inf or NaN.  NT: threads of the workgroup.
template <int D, int NT>
__device__ __forceinline__ void zero_v_tail(unsigned char *vbuf, int nv) {
  const int units = (BN - nv) * 4 * Lay<D>::GROUPS;  // 16-byte units
  for (int i = threadIdx.x; i < units; i += NT) {
    const int cg = i / ((BN - nv) * 4), rem = i % ((BN - nv) * 4);
    const int r = nv + (rem >> 2), u = rem & 3;
    *reinterpret_cast<uint4 *>(vbuf + cg * 4096 + r * 64 + u * 16) = make_uint4(0, 0, 0, 0);
  }
}

// Per-lane byte offsets into a block image.
//   row:  A-operand fragment of 16 rows (row lane%16, dims 8*(lane/16)..+7 of
//         column group 0; add ks*4096 for dims ks*32.., kt*1024 for rows
//         kt*16..), read with ds_read_b128;
//   tr0 / tr1: transposing reads (ds_read_b64_tr_b16) for even / odd 16-dim
//         tiles: within each 16-lane group g, source lane s reads 4 dims of
//         row 4*g + s/4 and the transpose hands lane l the 4 rows 4g..4g+3 of
//         dim l;
//   dcol / drow: the DMA lane offsets (row lane/4, unit (lane%4) ^ swap).
struct Lanes {
  uint32_t row, tr0, tr1, dcol, drow;
};
__device__ __forceinline__ Lanes lane_offsets(int lane) {
  Lanes o;
  o.row = uint32_t((lane & 15) * 64 + (((lane >> 4) ^ (((lane >> 2) & 1) << 1)) * 16));
  const int g = lane >> 4, s4 = lane & 15;
  const uint32_t vrow = uint32_t((4 * g + (s4 >> 2)) * 64 + 8 * (s4 & 3));
  o.tr0 = vrow + uint32_t(32 * (g & 1));
  o.tr1 = vrow + uint32_t(32 * ((g & 1) ^ 1));
  o.dcol = uint32_t(((lane & 3) ^ (((lane >> 4) & 1) << 1)) * 16);
  o.drow = uint32_t(lane >> 2);
  return o;
}

// A-operand fragment (16 x 32) of rows kt*16.. and dims ks*32.. of the block
// image at `img` (a K or V half of a buffer).
__device__ __forceinline__ bf16x8 row_frag(const unsigned char *img, const Lanes &o, int kt, int ks) {
  return as_bf16x8(*reinterpret_cast<const uint4 *>(img + o.row + ks * 4096 + kt * 1024));
}

// A-operand fragment (16 x 32) of the transposed image: dims dt*16 + lane%16,
// the 32 rows of step h (rows 32h + 4g..4g+3 and 32h + 16 + 4g..+3 in the
// lane's 8 k-slots: the order the C-layout of two 16-row tiles gives a B
// operand built from them).
__device__ __forceinline__ bf16x8 tr_frag(const unsigned char *img, const Lanes &o, int h, int dt) {
  const unsigned char *p = img + ((dt & 1) ? o.tr1 : o.tr0) + (dt >> 1) * 4096 + h * 2048;
  const v4i16 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16 *)(p));
  const v4i16 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4i16 *)(p + 1024));
  const uint2 l2 = __builtin_bit_cast(uint2, lo), h2 = __builtin_bit_cast(uint2, hi);
  return as_bf16x8(make_uint4(l2.x, l2.y, h2.x, h2.y));
}

}  // namespace tile
}  // namespace kvm
