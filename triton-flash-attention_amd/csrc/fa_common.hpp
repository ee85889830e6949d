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

// The same MFMA accumulating in place into AGPRs, for accumulators that only
// MFMAs touch until the epilogue (the compiler's MFMA selection keeps every
// accumulator in VGPRs, which a kernel needing more than 256 registers would
// otherwise spill). The leading s_nop 1 gives the two wait states a VALU
// write of an operand needs before an MFMA reads it (the hazard checks do
// not look inside asm); after the last call and before the accumulator is
// read, agpr_acc_drain() waits out the MFMA's passes.
__device__ __forceinline__ void mfma32_agpr(float16v& acc, half8 a, half8 b) {
  asm volatile("s_nop 1\n\tv_mfma_f32_32x32x16_f16 %0, %1, %2, %0" : "+a"(acc) : "v"(a), "v"(b));
}
__device__ __forceinline__ void agpr_acc_drain() {
  asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7" ::: "memory");
}

// ---------------------------------------------------------------------------
// Element types. Tensors are fp16 (F16) or bf16 (BF16); the kernels move and
// stage both as 16-bit containers (half_t, half8) and only the conversions
// and the MFMA opcode depend on the type. Round-to-nearest-even both ways.
// ---------------------------------------------------------------------------
struct F16 {};
struct BF16 {};
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));

template <class E> __device__ __forceinline__ half_t to_elem(float x);
template <> __device__ __forceinline__ half_t to_elem<F16>(float x) { return (half_t)x; }
template <> __device__ __forceinline__ half_t to_elem<BF16>(float x) {
  return __builtin_bit_cast(half_t, (__bf16)x);
}
template <class E> __device__ __forceinline__ float elem_to_f32(half_t h);
template <> __device__ __forceinline__ float elem_to_f32<F16>(half_t h) { return (float)h; }
template <> __device__ __forceinline__ float elem_to_f32<BF16>(half_t h) {
  return (float)__builtin_bit_cast(__bf16, h);
}

// D(32x32, fp32) += A(32x16) * B(16x32) in the element type.
template <class E> __device__ __forceinline__ float16v mma(half8 a, half8 b, float16v c);
template <> __device__ __forceinline__ float16v mma<F16>(half8 a, half8 b, float16v c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}
template <> __device__ __forceinline__ float16v mma<BF16>(half8 a, half8 b, float16v c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a),
                                                 __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}
// mfma32_agpr in the element type.
template <class E> __device__ __forceinline__ void mma_agpr(float16v& acc, half8 a, half8 b);
template <> __device__ __forceinline__ void mma_agpr<F16>(float16v& acc, half8 a, half8 b) {
  mfma32_agpr(acc, a, b);
}
template <> __device__ __forceinline__ void mma_agpr<BF16>(float16v& acc, half8 a, half8 b) {
  asm volatile("s_nop 1\n\tv_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+a"(acc) : "v"(a), "v"(b));
}

// Sign flip of 8 packed 16-bit values (the same bits for fp16 and bf16).
__device__ __forceinline__ half8 neg8(half8 v) {
  const u32x4 m = {0x80008000u, 0x80008000u, 0x80008000u, 0x80008000u};
  return __builtin_bit_cast(half8, __builtin_bit_cast(u32x4, v) ^ m);
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

// ---- 16x16x32 MFMA helpers (fa_bwd_pipe16.hpp, the 16x16x32 forward) ----
// D(16x16, fp32) += A(16x32) * B(32x16) in the element type. Lane l supplies
// A row (l % 16) and B column (l % 16), each with k-values 8 (l / 16) .. +7;
// the result: lane l holds column (l % 16), rows 4 (l / 16) + j, j = 0..3.
template <class E> __device__ __forceinline__ float4v mma16(half8 a, half8 b, float4v c);
template <> __device__ __forceinline__ float4v mma16<F16>(half8 a, half8 b, float4v c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}
template <> __device__ __forceinline__ float4v mma16<BF16>(half8 a, half8 b, float4v c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                 __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
}

// Sum over the four lanes l, l ^ 16, l ^ 32, l ^ 48 (the lanes that hold the
// four 8-wide quarters of a 32-wide d chunk of one query).
__device__ __forceinline__ float quarters_sum(float x) {
  x += __shfl_xor(x, 16, 64);
  return x + __shfl_xor(x, 32, 64);
}
// Maximum over the same four lanes.
__device__ __forceinline__ float quarters_max(float x) {
  x = __builtin_fmaxf(x, __shfl_xor(x, 16, 64));
  return __builtin_fmaxf(x, __shfl_xor(x, 32, 64));
}

// Row order of the 16x16x32 A operands read from LDS (K rows for dQ's S^T
// and dP^T and the forward's S^T, Q and dO rows for dK/dV's S and dP). At
// D = 64 the natural order;
// at D = 32 the quad swap of row_perm (quads 1 and 2 exchanged), without
// which the transposing reads of a result quad (rows 4 G' .. 4 G' + 3 for the
// lanes G = 0, 1 at once) hit the same banks as the quad four rows on under
// the D = 32 swizzle (two-way conflicts, measured). Result row 4 G + j of a
// 16-row block is then operand row 4 quad16<D>(G) + j.
template <int D>
__device__ __forceinline__ int rows16(int r) {
  return D == 32 ? row_perm(r) : r;
}
template <int D>
__device__ __forceinline__ int quad16(int G) {
  return rows16<D>(4 * G) >> 2;
}

// A value the compiler must treat as wave-uniform (lives in an SGPR), so
// branches on it are scalar branches rather than exec-masked regions.
__device__ __forceinline__ int uniform(int x) { return __builtin_amdgcn_readfirstlane(x); }

__device__ __forceinline__ float exp2_fast(float x) { return __builtin_amdgcn_exp2f(x); }
__device__ __forceinline__ float log2_fast(float x) { return __builtin_amdgcn_logf(x); }

// Value of the same register in lane (l ^ 32).
__device__ __forceinline__ float swap_halves(float x) {
  return __shfl_xor(x, 32, 64);
}

// x[l] and x[l ^ 32] via v_permlane32_swap (VALU only, no LDS round trip).
// The swap exchanges the upper half of its first operand with the lower half
// of its second; applied to two copies of x the results are {x[l], x[l^32]}
// in some order per lane, so any symmetric combination is the half-pair
// reduction. Written as assembly because the compiler folds the two results
// of the builtin when both inputs are the same value; the s_nop pairs cover
// the VALU-write -> permlane-read and permlane-write -> VALU-read hazards.
__device__ __forceinline__ void halves_pair(float x, float& a, float& b) {
  a = x;
  asm volatile(
      "v_mov_b32 %1, %0\n\t"
      "s_nop 1\n\t"
      "v_permlane32_swap_b32 %0, %1\n\t"
      "s_nop 1"
      : "+v"(a), "=&v"(b));
}
__device__ __forceinline__ float halves_max(float x) {
  float a, b;
  halves_pair(x, a, b);
  return fmaxf(a, b);
}
__device__ __forceinline__ float halves_sum(float x) {
  float a, b;
  halves_pair(x, a, b);
  return a + b;
}

// Wait for all of this wave's outstanding vector-memory loads, visibly to the
// compiler (so it stops tracking them; asm waits are invisible to it).
__device__ __forceinline__ void wait_all_vm() {
  // vmcnt = 0 (bits 3:0 and 15:14), expcnt = 7 and lgkmcnt = 15 (no wait).
  __builtin_amdgcn_s_waitcnt(0x0F70);
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
// The same for the element type E.
template <class E> __device__ __forceinline__ u32x2 pack4(float a, float b, float c, float d);
template <> __device__ __forceinline__ u32x2 pack4<F16>(float a, float b, float c, float d) {
  return pack4_half(a, b, c, d);
}
template <> __device__ __forceinline__ u32x2 pack4<BF16>(float a, float b, float c, float d) {
  bf16x4 h;
  h[0] = (__bf16)a;
  h[1] = (__bf16)b;
  h[2] = (__bf16)c;
  h[3] = (__bf16)d;
  return __builtin_bit_cast(u32x2, h);
}

// ---------------------------------------------------------------------------
// LDS tiles: [rows][D] fp16, row-major, no padding, with the 16-byte chunks of
// each row XOR-permuted. The permutation is chosen per head_dim so that the
// three access patterns the kernels use are free of LDS bank conflicts
// (64 banks x 4 bytes):
//   * staging writes: 16 consecutive lanes write consecutive 16-byte chunks
//     of consecutive rows;
//   * row reads (ds_read_b128): 16 lanes read one logical chunk of 16
//     consecutive rows (any order inside the 16);
//   * transposed reads (ds_read_b64_tr_b16): 32 lanes read 4 consecutive rows
//     (first row a multiple of 4) x 32 consecutive bytes.
// D=32  (64 B rows):  chunk c of row r at c ^ ((r >> 2) & 3)
// D=64  (128 B rows): chunk c of row r at c ^ bitrev3((r >> 1) & 7)
// D=128 (256 B rows): chunk c of row r at c ^ bitrev4(r & 15)
// ---------------------------------------------------------------------------
template <int D>
__device__ __forceinline__ int swz_chunk(int row, int c) {
  static_assert(D == 32 || D == 64 || D == 128, "head_dim");
  if constexpr (D == 32) {
    return c ^ ((row >> 2) & 3);
  } else if constexpr (D == 64) {
    const int u = (row >> 1) & 7;
    return c ^ (((u & 1) << 2) | (u & 2) | (u >> 2));
  } else {
    const int u = row & 15;
    return c ^ (((u & 1) << 3) | ((u & 2) << 1) | ((u & 4) >> 1) | (u >> 3));
  }
}
// Offset (in halves) of the 8 halves [8c, 8c+8) of row `row`.
template <int D>
__device__ __forceinline__ int swz_offset(int row, int c) {
  return row * D + 8 * swz_chunk<D>(row, c);
}

typedef short short4v __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) short4v lds_short4;

// MFMA operand whose k-axis runs DOWN the rows of an LDS tile:
//   value e (0..7) of lane l = tile[k0 + 8*(l/32) + e][m0 + (l % 32)],
// i.e. the A operand of X with X[m][k] = tile[k][m] (or the B operand with
// n in place of m). Two ds_read_b64_tr_b16: inside each 16-lane group, source
// lane 4r+q addresses row k0 + 8g + r (+4), columns m0 + 16*(group&1) + 4q..+3,
// and lane i receives rows +0..3 of column m0 + 16*(group&1) + i.
template <int D>
__device__ __forceinline__ half8 read_tr(const half_t* tile, int k0, int m0, int lane) {
  const int grp = lane >> 4;
  const int i = lane & 15;
  const int g = lane >> 5;
  const int r = i >> 2, q = i & 3;
  const int col = m0 + 16 * (grp & 1) + 4 * q;  // multiple of 4
  const int c = col >> 3, sub = col & 7;        // chunk, 0 or 4 inside it
  const int row0 = k0 + 8 * g + r;
  const int row1 = row0 + 4;
  const half_t* p0 = tile + row0 * D + 8 * swz_chunk<D>(row0, c) + sub;
  const half_t* p1 = tile + row1 * D + 8 * swz_chunk<D>(row1, c) + sub;
  const half4 lo =
      __builtin_bit_cast(half4, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_short4*)(p0)));
  const half4 hi =
      __builtin_bit_cast(half4, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_short4*)(p1)));
  half8 out;
  out[0] = lo[0];
  out[1] = lo[1];
  out[2] = lo[2];
  out[3] = lo[3];
  out[4] = hi[0];
  out[5] = hi[1];
  out[6] = hi[2];
  out[7] = hi[3];
  return out;
}

// MFMA operand whose k-axis runs ALONG a row: value e of lane l =
// tile[row][k0 + 8*(l/32) + e] with `row` chosen by the caller.
template <int D>
__device__ __forceinline__ half8 read_row(const half_t* tile, int row, int k0, int lane) {
  const int c = (k0 >> 3) + (lane >> 5);
  return *reinterpret_cast<const half8*>(tile + swz_offset<D>(row, c));
}

// Global -> registers -> LDS staging of an R x D tile (16-byte chunks;
// consecutive threads take consecutive chunks of a row, so global reads
// coalesce and LDS writes are conflict-free).
template <int D, int R, int NT>
struct Stager {
  static constexpr int DC = D / 8;
  static constexpr int CHUNKS = R * DC;
  static constexpr int PER_T = (CHUNKS + NT - 1) / NT;
  u32x4 reg[PER_T];

  __device__ __forceinline__ void load(rsrc_t r, int row0, int tid) {
#pragma unroll
    for (int i = 0; i < PER_T; ++i) {
      const int ci = tid + i * NT;
      if (CHUNKS % NT == 0 || ci < CHUNKS) {
        const int row = ci / DC, c = ci - row * DC;
        reg[i] = buf_load_b128(r, (uint32_t)((row0 + row) * D + 8 * c) * 2u);
      }
    }
  }
  __device__ __forceinline__ void store(half_t* tile, int tid) const {
#pragma unroll
    for (int i = 0; i < PER_T; ++i) {
      const int ci = tid + i * NT;
      if (CHUNKS % NT == 0 || ci < CHUNKS) {
        const int row = ci / DC, c = ci - row * DC;
        *reinterpret_cast<u32x4*>(tile + swz_offset<D>(row, c)) = reg[i];
      }
    }
  }
};

// ---------------------------------------------------------------------------
// Global -> LDS direct (DMA) staging with buffer_load_dwordx4 ... lds.
// One wave instruction writes 1 KiB of LDS contiguously (lane l at M0 + 16 l),
// so each lane picks the global chunk that the swizzled layout keeps at its
// LDS slot. No VGPRs and no LDS write instructions are spent on staging.
//
// The load is issued through inline assembly on purpose: the compiler's own
// wait insertion treats every LDS read after an LDS-DMA as dependent on it and
// would drain all outstanding loads (vmcnt(0)), which defeats a multi-tile
// prefetch ring. Completion is instead tracked explicitly: the issuing wave
// waits with vmcnt(n) (loads retire in order), then a work-group barrier
// publishes the tile (wait_vm_and_barrier).
// ---------------------------------------------------------------------------
typedef int int4v __attribute__((ext_vector_type(4)));

// Raw buffer descriptor as four SGPR words (for the inline-assembly loads).
__device__ __forceinline__ int4v make_rsrc_words(const void* base, uint32_t bytes) {
  const uint64_t p = reinterpret_cast<uint64_t>(base);
  int4v r;
  r[0] = (int)(uint32_t)p;
  r[1] = (int)(uint32_t)(p >> 32);  // stride 0
  r[2] = (int)bytes;
  r[3] = kRsrcWord3;
  return r;
}

__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)(p);
}

// 16 bytes per lane from byte offset `voff` of the buffer to LDS[m0 + 16 lane].
// M0 is reserved by the compiler, so the block restores it before returning.
__device__ __forceinline__ void dma_b128(int4v rsrc, uint32_t voff, uint32_t lds_base) {
  uint32_t saved;
  asm volatile(
      "s_mov_b32 %0, m0\n\t"
      "s_mov_b32 m0, %3\n\t"
      "buffer_load_dwordx4 %1, %2, 0 offen lds\n\t"
      "s_mov_b32 m0, %0"
      : "=&s"(saved)
      : "v"(voff), "s"(rsrc), "s"(lds_base)
      : "memory");
}

// 4 bytes per lane from byte offset `voff` to LDS[m0 + 4 lane] (256 B per wave).
__device__ __forceinline__ void dma_b32(int4v rsrc, uint32_t voff, uint32_t lds_base) {
  uint32_t saved;
  asm volatile(
      "s_mov_b32 %0, m0\n\t"
      "s_mov_b32 m0, %3\n\t"
      "buffer_load_dword %1, %2, 0 offen lds\n\t"
      "s_mov_b32 m0, %0"
      : "=&s"(saved)
      : "v"(voff), "s"(rsrc), "s"(lds_base)
      : "memory");
}

// Wait until at most N of this wave's vector-memory operations are in flight,
// then synchronise the work-group. Both are opaque to the compiler (memory
// clobber), so no LDS access moves across them.
template <int N>
__device__ __forceinline__ void wait_vm_and_barrier() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" : : "n"(N) : "memory");
}

// When the tile has fewer 1 KiB pieces than the work-group has waves, wave w
// loads piece w % INSTR: the duplicates write identical bytes, and every wave
// still issues the same number of instructions per tile (uniform vmcnt).
template <int D, int R, int NW>
struct DmaStager {
  static constexpr int BYTES = R * D * 2;
  static constexpr int INSTR = BYTES / 1024;  // wave instructions per tile
  static constexpr int PER_WAVE = INSTR >= NW ? INSTR / NW : 1;
  static_assert(BYTES % 1024 == 0, "tile must be a multiple of 1 KiB");
  static_assert(INSTR % NW == 0 || NW % INSTR == 0,
                "tile instructions must split evenly over the waves");

  // Per-lane byte offsets inside the tile's global rows (loop-invariant).
  uint32_t voff[PER_WAVE];
  int piece0;  // first 1 KiB piece of this wave

  __device__ __forceinline__ void init(int wave, int lane) {
    piece0 = INSTR >= NW ? wave * PER_WAVE : wave % INSTR;
#pragma unroll
    for (int i = 0; i < PER_WAVE; ++i) {
      const int byte = (piece0 + i) * 1024 + lane * 16;
      const int row = byte / (D * 2);
      const int pc = (byte % (D * 2)) / 16;
      const int c = swz_chunk<D>(row, pc);  // XOR swizzle is an involution
      voff[i] = (uint32_t)(row * D + 8 * c) * 2u;
    }
  }
  // Tile rows [row0, row0 + R) of the buffer -> LDS tile at `tile`.
  __device__ __forceinline__ void issue(int4v rsrc, int row0, const half_t* tile, int) const {
    const uint32_t base = lds_addr(tile) + (uint32_t)piece0 * 1024u;
    const uint32_t roff = (uint32_t)row0 * D * 2u;
#pragma unroll
    for (int i = 0; i < PER_WAVE; ++i) dma_b128(rsrc, roff + voff[i], base + 1024u * i);
  }
};

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

// The same order for query-head launches (forward, dQ) with GQA groups: when
// the B * Hkv key/value heads are a multiple of 8, position p of a tile row
// takes query head (p % BHkv) * group + p / BHkv, so every query head of key/
// value head j (and each of its tiles and key splits) lands on XCD j % 8 and
// the group reads its K/V through one L2. A bijection on [0, heads); the
// identity for MHA or other head counts.
__device__ __forceinline__ TileHead decode_block_grouped(int block, int heads, int group) {
  TileHead t = decode_block(block, heads);
  const int bhkv = heads / group;
  if (group > 1 && bhkv % 8 == 0) t.head = (t.head % bhkv) * group + t.head / bhkv;
  return t;
}

}  // namespace fa
