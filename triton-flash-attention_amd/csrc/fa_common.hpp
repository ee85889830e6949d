// fa_common.hpp — gfx950 building blocks shared by the FlashAttention kernels.
//
// Everything here is CDNA4-specific: 64-lane wavefronts, the
// v_mfma_f32_32x32x16_f16 matrix core instruction, raw buffer loads/stores
// whose hardware range check turns out-of-range rows into zeros (loads) or
// no-ops (stores), and the native base-2 exponential v_exp_f32.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace fa {

typedef _Float16 half_t;
typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half4 __attribute__((ext_vector_type(4)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef float float16v __attribute__((ext_vector_type(16)));
typedef float float4v __attribute__((ext_vector_type(4)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));

typedef __amdgpu_buffer_rsrc_t rsrc_t;

// Buffer descriptor word 3 for gfx9-family raw buffers: 32-bit untyped data,
// no swizzle, offset range checked against num_records.
constexpr int kRsrcWord3 = 0x00020000;

// A raw buffer over [base, base + bytes). Loads at byte offsets >= bytes
// return 0, stores there are dropped: tail rows need no extra masking.
__device__ __forceinline__ rsrc_t make_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes,
                                           kRsrcWord3);
}

__device__ __forceinline__ u32x4 buf_load_b128(rsrc_t r, uint32_t byte_off) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, byte_off, 0, 0);
}
__device__ __forceinline__ float buf_load_f32(rsrc_t r, uint32_t byte_off) {
  return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, byte_off, 0, 0));
}
__device__ __forceinline__ void buf_store_b64(rsrc_t r, uint32_t byte_off, u32x2 v) {
  __builtin_amdgcn_raw_buffer_store_b64(v, r, byte_off, 0, 0);
}
__device__ __forceinline__ void buf_store_f32(rsrc_t r, uint32_t byte_off, float v) {
  __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(unsigned, v), r, byte_off, 0, 0);
}

// D(32x32, fp32) += A(32x16, fp16) * B(16x32, fp16).
// Lane l supplies A row (l % 32) and B column (l % 32), each with 8 k-values
// taken from the k-half (l / 32). Only the pairing of A's and B's k-values
// matters, so any consistent assignment of k inside a lane is valid.
// Result: lane l holds column (l % 32), rows 8*(j/4) + 4*(l/32) + (j%4), j=0..15.
__device__ __forceinline__ float16v mfma32(half8 a, half8 b, float16v c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

// Row permutation applied when a 32-row A operand is read from LDS so that
// the MFMA result rows held by lane half g, values j = 0..7 / 8..15, are the
// CONTIGUOUS operand rows 8g..8g+7 / 16+8g..16+8g+7. That makes a lane's
// result values directly reusable as the 8 k-values of the next MFMA's
// operand (P after QK^T feeds PV with no data movement).
// perm swaps row groups [4,8) and [8,12) inside every 16 rows.
__device__ __forceinline__ int row_perm(int r) {
  return r ^ ((((r >> 2) ^ (r >> 3)) & 1) * 12);
}
// Operand row that result value j of lane half g corresponds to (inverse view).
__device__ __forceinline__ constexpr int result_row(int j, int g) {
  return 16 * (j >> 3) + 8 * g + (j & 7);
}

__device__ __forceinline__ float exp2_fast(float x) { return __builtin_amdgcn_exp2f(x); }
__device__ __forceinline__ float log2_fast(float x) { return __builtin_amdgcn_logf(x); }

// Value of the same register in lane (l ^ 32).
__device__ __forceinline__ float swap_halves(float x) {
  return __shfl_xor(x, 32, 64);
}

__device__ __forceinline__ half8 to_half8(const float* p) {
  half8 h;
#pragma unroll
  for (int i = 0; i < 8; ++i) h[i] = (half_t)p[i];
  return h;
}

// Pack the lo (sel=0) or hi (sel=1) 16-bit halves of two dwords: (a.sel, b.sel).
__device__ __forceinline__ unsigned pack_lo(unsigned a, unsigned b) {
  return (a & 0xffffu) | (b << 16);
}
__device__ __forceinline__ unsigned pack_hi(unsigned a, unsigned b) {
  return (a >> 16) | (b & 0xffff0000u);
}

// Four fp32 -> four fp16 (round to nearest even) packed in 8 bytes.
__device__ __forceinline__ u32x2 pack4_half(float a, float b, float c, float d) {
  half4 h;
  h[0] = (half_t)a;
  h[1] = (half_t)b;
  h[2] = (half_t)c;
  h[3] = (half_t)d;
  return __builtin_bit_cast(u32x2, h);
}

// Work-group order: tile-major, head-minor. With B*H a multiple of 8 every
// tile of head h lands on XCD (h % 8) (work-groups are dealt to the 8 XCDs
// round-robin), so the K/V of a head stays in one XCD's L2.
struct TileHead {
  int tile_rank;
  int head;
};
__device__ __forceinline__ TileHead decode_block(int block, int heads) {
  TileHead t;
  t.tile_rank = block / heads;
  t.head = block - t.tile_rank * heads;
  return t;
}

}  // namespace fa
