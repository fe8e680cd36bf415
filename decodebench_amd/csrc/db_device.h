// db_device.h -- wave64 building blocks for the gfx950 decode kernels.
//
// Everything here targets CDNA4 directly: 64-lane wavefronts, DPP lane
// permutations for reductions inside a 16-lane row, v_readlane for the four
// rows of a wave, packed fp16 dot products (v_dot2_f32_f16) and 128-bit
// non-temporal loads for data that is streamed exactly once.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace dbk {

typedef _Float16 h2 __attribute__((ext_vector_type(2)));
typedef _Float16 h8 __attribute__((ext_vector_type(8)));
typedef float f4 __attribute__((ext_vector_type(4)));
typedef unsigned u4 __attribute__((ext_vector_type(4)));

constexpr int kWave = 64;

// ---------------------------------------------------------------- loads
// 16-byte load of streamed data (weights, KV cache): non-temporal so it does
// not displace the small operands every wave re-reads (x, gamma, q).
__device__ __forceinline__ u4 ld_stream(const void* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const u4*>(p));
}
__device__ __forceinline__ u4 ld16(const void* p) {
  return *reinterpret_cast<const u4*>(p);
}

// Raw buffer resource over `bytes` bytes at `base` (stride 0).  A buffer load
// at an offset >= bytes returns zero without a memory access, so a kernel can
// issue the loads of a tile that does not exist (bytes = 0) unconditionally
// and keep one straight-line path through its load/compute pipeline.
// Word 3 is the gfx9 data-format default for raw byte buffers.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, int bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, bytes,
                                           0x00020000);
}
// 16-byte non-temporal buffer load (cache policy bit 1 = nt).
__device__ __forceinline__ u4 ld_buf_stream(__amdgpu_buffer_rsrc_t r, int offset) {
  return __builtin_bit_cast(u4, __builtin_amdgcn_raw_buffer_load_b128(r, offset, 0, 2));
}

__device__ __forceinline__ h2 as_h2(unsigned v) {
  return __builtin_bit_cast(h2, v);
}

// acc + dot(a, b) over four packed fp16 pairs, fp32 accumulation.
__device__ __forceinline__ float dot8(u4 a, u4 b, float acc) {
  acc = __builtin_amdgcn_fdot2(as_h2(a[0]), as_h2(b[0]), acc, false);
  acc = __builtin_amdgcn_fdot2(as_h2(a[1]), as_h2(b[1]), acc, false);
  acc = __builtin_amdgcn_fdot2(as_h2(a[2]), as_h2(b[2]), acc, false);
  acc = __builtin_amdgcn_fdot2(as_h2(a[3]), as_h2(b[3]), acc, false);
  return acc;
}

// ------------------------------------------------------------ DPP moves
// DPP control words (GFX9 encoding).
constexpr int kQuadSwap1 = 0xB1;      // quad_perm [1,0,3,2]
constexpr int kQuadSwap2 = 0x4E;      // quad_perm [2,3,0,1]
constexpr int kRowHalfMirror = 0x141;
constexpr int kRowMirror = 0x140;
constexpr int kRowRor8 = 0x128;      // row_ror:8: lane n of a row <- lane (n + 8) % 16
constexpr int kRowNewBcast0 = 0x150;  // + n: lane n of each row -> whole row

template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL,
                                         0xf, 0xf, true));
}

// Sum over the 16 lanes of each DPP row; every lane of the row gets the sum.
__device__ __forceinline__ float row_sum16(float v) {
  v += dpp<kQuadSwap1>(v);
  v += dpp<kQuadSwap2>(v);
  v += dpp<kRowHalfMirror>(v);
  v += dpp<kRowMirror>(v);
  return v;
}

__device__ __forceinline__ float row_max16(float v) {
  v = fmaxf(v, dpp<kQuadSwap1>(v));
  v = fmaxf(v, dpp<kQuadSwap2>(v));
  v = fmaxf(v, dpp<kRowHalfMirror>(v));
  v = fmaxf(v, dpp<kRowMirror>(v));
  return v;
}

// Broadcast lane N of each 16-lane row to the whole row.
template <int N>
__device__ __forceinline__ float row_bcast(float v) {
  return dpp<kRowNewBcast0 + N>(v);
}

__device__ __forceinline__ float lane_value(float v, int lane) {
  return __builtin_bit_cast(
      float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), lane));
}

// Sum over all 64 lanes, result uniform (held in every lane).
__device__ __forceinline__ float wave_sum(float v) {
  v = row_sum16(v);
  return (lane_value(v, 0) + lane_value(v, 16)) +
         (lane_value(v, 32) + lane_value(v, 48));
}

// ------------------------------------------------------- LDS ordering
// Between a wave's LDS writes and its reads of what other lanes of the same
// wave wrote (or its reads and later overwrites): the wave's LDS accesses
// execute in issue order, so no wait is needed, but the compiler may not
// move a read above a write it cannot prove to touch other addresses (the
// lanes exchange data through swizzled slots).  A wavefront-scope fence
// pair around a wave barrier states that ordering; it emits no
// instruction.
__device__ __forceinline__ void wave_lds_order() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// ---------------------------------------------------------- conversions
__device__ __forceinline__ _Float16 to_h(float f) { return (_Float16)f; }

// Pack two floats into fp16x2 with round-to-nearest-even on each half.
__device__ __forceinline__ unsigned pack_h2(float lo, float hi) {
  h2 r;
  r[0] = (_Float16)lo;
  r[1] = (_Float16)hi;
  return __builtin_bit_cast(unsigned, r);
}

__device__ __forceinline__ float fast_exp2(float x) {
  return __builtin_amdgcn_exp2f(x);
}

}  // namespace dbk
