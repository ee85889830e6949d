// fa_bwd_pipe.hpp — bodies of the software-pipelined dK/dV and dQ kernels
// (gfx950). fa_bwd.hip wraps each in its own kernel; fa_bwd_pair.hip runs
// both in one launch. Each body is the work of one work-group, given its
// block index and the LDS ring (a __shared__ array of the wrapping kernel).
#pragma once

#include <type_traits>

#include "fa_common.hpp"
#include "fa_kernels.hpp"

namespace fa {

template <int V>
using ic = std::integral_constant<int, V>;

// f(integral_constant<int, I>) for I = B .. E-1, fully unrolled.
template <int B, int E, typename F>
__device__ __forceinline__ void static_for(F&& f) {
  if constexpr (B < E) {
    f(std::integral_constant<int, B>{});
    static_for<B + 1, E>(f);
  }
}

// dQ epilogue: lane (query qrow, half g) holds d = 32*db + 8*(j/4) + 4*g + j%4
// of dQ / mul: 16-bit through rdq, or in split mode the fp32 partial of split
// `split` (part[split][B*Hq][N][D]).
template <int D, class E>
__device__ __forceinline__ void store_dq(const BwdArgs& a, const rsrc_t& rdq, int split, int head,
                                         int qrow, const float16v (&dq)[D / 32], float mul) {
  const bool split_mode = a.nsplit > 1;
  // The lane's half, recomputed (mbcnt needs no live register).
  const int g = (int)(__builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u)) >> 5);
  const int64_t prow = ((int64_t)split * a.BH + head) * a.N + qrow;
  float* po = split_mode ? a.part + prow * D : nullptr;  // part is null in one-pass mode
#pragma unroll
  for (int db = 0; db < D / 32; ++db)
#pragma unroll
    for (int jq = 0; jq < 4; ++jq) {
      float4v v;
#pragma unroll
      for (int e = 0; e < 4; ++e) v[e] = dq[db][4 * jq + e] * mul;
      if (split_mode) {
        if (qrow < a.N) *reinterpret_cast<float4v*>(po + 32 * db + 8 * jq + 4 * g) = v;
      } else {
        buf_store_b64(rdq, (uint32_t)(qrow * D + 32 * db + 8 * jq + 4 * g) * 2u,
                      pack4<E>(v[0], v[1], v[2], v[3]));
      }
    }
}

template <int I, int N, typename F>
__device__ __forceinline__ void bwd_static_for(F&& f) {
  if constexpr (I < N) {
    f(std::integral_constant<int, I>{});
    bwd_static_for<I + 1, N>(f);
  }
}

// --------------------------------------------------------------------------
// dK / dV, software-pipelined over 32-query units.
//
// Same work decomposition as dkdv_kernel (NW waves x 32 keys, K and V held
// as MFMA B operands, (query head, query tile) units streamed through an LDS
// DMA ring), but the three stages of a unit are spread over consecutive
// units so that each unit's body has matrix and vector work that do not
// depend on each other:
//   body of unit u:  vector work of unit u      P = exp2(-Sl), dS' = P dPd
//                    matrix work of unit u + 1  Sl = LSE' - Q fp16(c K)^T,
//                                               dPd = Delta - dO V^T
//                    matrix work of unit u - 1  dV^T += dO^T P, dK^T += Q^T dS'
// The scores use the reference's scaled key operand fp16(c K) (k_scaled,
// attention.py:435). Both accumulators start from a per-query table (LSE' in
// log2 units, Delta) and multiply -fp16(c K) and -V, so neither the LSE'
// subtraction nor the Delta subtraction costs vector work; dS' = -dS and dK
// is negated once at the end. Causal mask: units a wave sees entirely before
// its keys read LSE' = +inf (P = 0 exactly) from a small table; the diagonal
// unit sets its masked Sl values to +inf. Rows past N need no mask: their Q
// and dO rows load as zeros, so their P (finite) multiplies zero in both
// updates.
// A step is two units and ends with one work-group barrier. The ring has 8
// unit slots: units 2s-1 .. 2s+2 are read in step s, 2s+3 and 2s+4 are in
// flight and 2s+5, 2s+6 are issued. Every work-group runs its unit count
// rounded up to the 8-unit unroll; the extra units stream rows past N
// (zeros) and add nothing.
// --------------------------------------------------------------------------
template <int D, int NW>
struct DkdvPipeTile {
  static constexpr int BKV = 32 * NW;
  static constexpr int NT = 64 * NW;
  static constexpr int QT = 32;
  static constexpr int TILE = QT * D;               // halves of the Q (or dO) unit
  static constexpr int AUX = 128;                   // floats: LSE[64], Delta[64]
  static constexpr int STAGE = 2 * TILE + 2 * AUX;  // halves per ring slot
  static constexpr int NSTAGE = 8;
  static constexpr int AHEAD = 5;                   // units issued before step 0
  static constexpr int LDS_HALVES = NSTAGE * STAGE + 2 * 64;  // + 64 x +inf
  // D <= 64: two work-groups (two waves per SIMD, <= 256 registers each);
  // D = 128: one (one wave per SIMD, up to 512 registers).
  static constexpr int WGS_PER_CU = D <= 64 ? 2 : 1;
};

template <int D, int NW>
constexpr bool dkdv_pipe_tiling_ok() {
  using T = DkdvPipeTile<D, NW>;
  constexpr int instr = T::TILE * 2 / 1024;
  // one or two 1 KiB pieces per wave (duplicates allowed when the tile has
  // fewer pieces than waves), and the ring of every resident work-group in LDS
  return (T::TILE * 2) % 1024 == 0 &&
         ((instr <= NW && NW % instr == 0) || instr == 2 * NW) &&
         T::WGS_PER_CU * T::LDS_HALVES * 2 <= 160 * 1024;
}

// LDS reads of the pipelined dK/dV body are issued this many MFMA tasks
// ahead of their consumer.
#ifndef FA_DKDV_LEAD
#define FA_DKDV_LEAD 3
#endif
// Task order of the pipelined dK/dV body (kinds 0 dV, 1 dK of unit u-1; 2 S,
// 3 dPd of unit u+1; NQ tasks of each kind):
//   0: (dV_q, dK_q, S_q, dPd_q) for q = 0 .. NQ-1;
//   1: dV_0, dK_0, dV_1, dK_1, then (S_j, dPd_j, dV_j+2, dK_j+2) for
//      j = 0 .. NQ-3, then S, dPd of NQ-2 and NQ-1: the first S and dPd tasks,
//      whose accumulators start from the LSE' and Delta table reads issued at
//      the top of the body, run four tasks in instead of two.
// Order 1 measured no faster (MI355X, one box: dK/dV c2 292.4 vs 292.0 us, c3
// 70.0 vs 70.8, B2 H32 N8192 D128 causal 2261 vs 2232), so 0 stays.
#ifndef FA_DKDV_ORDER
#define FA_DKDV_ORDER 0
#endif
// Cross-unit operand prefetch in the pipelined backward bodies (dK/dV and dQ):
// a two-unit step publishes the rows of both of its units at its barrier, so
// the second unit's first FA_*_LEAD operand reads are issued during the first
// unit's last task groups instead of at the top of its own body, where the
// first MFMA would wait out their whole LDS latency. Same results bit for bit;
// MI355X, one box, min of two, us, off / on: dK/dV c2 292.0 / 288.2, c3 70.8 /
// 68.5, c5 359.5 / 357.9, B2 H32 N8192 D128 causal 2232 / 2228; dQ c5 236.0 /
// 233.8, c2, c3 and D = 128 even.
#ifndef FA_BWD_XPREFETCH
#define FA_BWD_XPREFETCH 1
#endif

// (kind, q) of task slot i of the pipelined dK/dV body (see FA_DKDV_ORDER).
template <int NQ>
constexpr int dkdv_task_kind(int i) {
  if (FA_DKDV_ORDER == 0) return i % 4;
  const int p = i / 2, w = i % 2;
  if (p < 2) return w;
  if (p < 2 + 2 * (NQ - 2)) return ((p - 2) % 2 == 0) ? 2 + w : w;
  return 2 + w;
}
template <int NQ>
constexpr int dkdv_task_q(int i) {
  if (FA_DKDV_ORDER == 0) return i / 4;
  const int p = i / 2;
  if (p < 2) return p;
  if (p < 2 + 2 * (NQ - 2)) return ((p - 2) % 2 == 0) ? (p - 2) / 2 : (p - 3) / 2 + 2;
  return NQ - 2 + (p - 2 - 2 * (NQ - 2));
}

template <int D, bool CAUSAL, int NW, class E>
__device__ __forceinline__ void dkdv_pipe_body(const BwdArgs& a, const unsigned block,
                                        half_t* __restrict__ lds) {
  using T = DkdvPipeTile<D, NW>;
  using Dma = DmaStager<D, T::QT, NW>;
  static_assert(Dma::PER_WAVE == 1 || Dma::PER_WAVE == 2, "one or two tile pieces per wave");
  constexpr int NS = T::NSTAGE;
  // this wave's DMA instructions per unit: its Q and dO pieces, LSE or Delta
  constexpr int IPU = 2 * Dma::PER_WAVE + 1;
  constexpr int kInfOff = NS * T::STAGE / 2;  // float offset of the +inf table

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int ql = lane & 31;
  const int g = lane >> 5;

  const int split = block / (a.num_tiles * a.BHkv);
  const TileHead th = decode_block(block - split * a.num_tiles * a.BHkv, a.BHkv);
  const int kvh = th.head;
  const int b = kvh / a.Hkv;
  const int hkv = kvh - b * a.Hkv;
  const int G = a.group;
  const int N = a.N;      // queries
  const int Nkv = a.Nkv;  // keys
  const uint32_t slab = (uint32_t)N * D * 2u;
  const uint32_t kv_slab = (uint32_t)Nkv * D * 2u;
  const uint32_t aux_bytes = (uint32_t)N * 4u;
  const rsrc_t rk = make_rsrc(a.k + (int64_t)kvh * Nkv * D, kv_slab);
  const rsrc_t rv = make_rsrc(a.v + (int64_t)kvh * Nkv * D, kv_slab);

  const int k0 = th.tile_rank * T::BKV;
  const int k0w = k0 + 32 * wave;
  const int krow = k0w + ql;

  // -fp16(c K) and -V as B operands (column = key ql, d = 16*kk + 8*g .. +7).
  // The scaled key operand is the reference's k_scaled (attention.py:435):
  // c K in fp32 rounded to fp16. With the S accumulator started from LSE',
  // the MFMA yields LSE' - s and P = exp2(-acc) needs no multiply-add.
  const float c = a.c;
  half8 kf[D / 16], vn[D / 16];
#pragma unroll
  for (int kk = 0; kk < D / 16; ++kk) {
    const uint32_t off = (uint32_t)(krow * D + 16 * kk + 8 * g) * 2u;
    kf[kk] = __builtin_bit_cast(half8, buf_load_b128(rk, off));
    vn[kk] = neg8(__builtin_bit_cast(half8, buf_load_b128(rv, off)));
  }
  wait_all_vm();
#pragma unroll
  for (int kk = 0; kk < D / 16; ++kk)
#pragma unroll
    for (int e = 0; e < 8; ++e) kf[kk][e] = to_elem<E>(-c * elem_to_f32<E>(kf[kk][e]));
  // Opaque from here on, so that the operands are not recomputed inside the loop.
#pragma unroll
  for (int kk = 0; kk < D / 16; ++kk) asm volatile("" : "+v"(kf[kk]), "+v"(vn[kk]));

  const int q_begin = CAUSAL ? k0 : 0;  // k0 is a multiple of 32
  // Under the causal mask a key tile past the last query (N < Nkv) sees no
  // query: it takes no unit (every chunk gets none, as the chunks past the
  // last unit of a split tile do), the zeroed slot stands in for the last
  // unit, and its dK = dV = 0 are written.
  const int ntq = max(1, (N - q_begin + T::QT - 1) / T::QT);
  const int total_units = CAUSAL && q_begin >= N ? 0 : G * ntq;
  const int chunk = (total_units + a.nsplit - 1) / a.nsplit;
  const int u_lo = min(split * chunk, total_units);
  const int nunits = min(chunk, total_units - u_lo);
  const int npad = (nunits + NS - 1) / NS * NS;
  // The units end in the ring's last slot: the first ring turn starts at step
  // p0 (slot s0), so at most one padding unit runs and the loop over whole
  // turns has no branches between its steps.
  const int p0 = __builtin_amdgcn_readfirstlane((npad - nunits) / 2);
  const int s0 = 2 * p0;

  // Issue cursor: query head gi of the group and first row of the next unit
  // to fetch; after the last unit the row is N (zeros from then on).
  int i_gi = min(u_lo / ntq, G - 1);
  int i_row = q_begin + (u_lo - i_gi * ntq) * T::QT;
  int i_left = nunits;
  int4v r_q, r_do, r_aux;
  const bool is_lse = (wave & 1) == 0;  // even waves fetch LSE, odd waves Delta
  auto set_head = [&]() {
    const int head = b * a.Hq + hkv * G + i_gi;
    r_q = make_rsrc_words(a.q + (int64_t)head * N * D, slab);
    r_do = make_rsrc_words(a.dO + (int64_t)head * N * D, slab);
    r_aux = make_rsrc_words((is_lse ? a.lse : a.delta) + (int64_t)head * N, aux_bytes);
  };
  set_head();

  Dma dma;
  dma.init(wave, lane);
  const uint32_t lds0 = lds_addr(lds);
  const uint32_t aux_lane = (uint32_t)lane * 4u;
  const uint32_t aux_lds = 2u * T::TILE * 2u + (is_lse ? 0u : 64u * 4u);
  auto issue = [&](int slot) __attribute__((always_inline)) {
    const int row0 = i_left > 0 ? i_row : N;
    const uint32_t vt = (uint32_t)row0 * (D * 2u) + dma.voff[0];
    const uint32_t va = (uint32_t)row0 * 4u + aux_lane;
    const uint32_t base = lds0 + (uint32_t)slot * (T::STAGE * 2u);
    const uint32_t piece = (uint32_t)dma.piece0 * 1024u;
    uint32_t saved;
    if constexpr (Dma::PER_WAVE == 1) {
      asm volatile(
          "s_mov_b32 %0, m0\n\t"
          "s_mov_b32 m0, %5\n\t"
          "buffer_load_dwordx4 %1, %3, 0 offen lds\n\t"
          "s_mov_b32 m0, %6\n\t"
          "buffer_load_dwordx4 %1, %4, 0 offen lds\n\t"
          "s_mov_b32 m0, %8\n\t"
          "buffer_load_dword %2, %7, 0 offen lds\n\t"
          "s_mov_b32 m0, %0"
          : "=&s"(saved)
          : "v"(vt), "v"(va), "s"(r_q), "s"(r_do), "s"(base + piece),
            "s"(base + T::TILE * 2u + piece), "s"(r_aux), "s"(base + aux_lds)
          : "memory");
    } else {
      const uint32_t vt1 = (uint32_t)row0 * (D * 2u) + dma.voff[1];
      asm volatile(
          "s_mov_b32 %0, m0\n\t"
          "s_mov_b32 m0, %6\n\t"
          "buffer_load_dwordx4 %1, %4, 0 offen lds\n\t"
          "s_mov_b32 m0, %7\n\t"
          "buffer_load_dwordx4 %2, %4, 0 offen lds\n\t"
          "s_mov_b32 m0, %8\n\t"
          "buffer_load_dwordx4 %1, %5, 0 offen lds\n\t"
          "s_mov_b32 m0, %9\n\t"
          "buffer_load_dwordx4 %2, %5, 0 offen lds\n\t"
          "s_mov_b32 m0, %11\n\t"
          "buffer_load_dword %3, %10, 0 offen lds\n\t"
          "s_mov_b32 m0, %0"
          : "=&s"(saved)
          : "v"(vt), "v"(vt1), "v"(va), "s"(r_q), "s"(r_do), "s"(base + piece),
            "s"(base + piece + 1024u), "s"(base + T::TILE * 2u + piece),
            "s"(base + T::TILE * 2u + piece + 1024u), "s"(r_aux), "s"(base + aux_lds)
          : "memory");
    }
    --i_left;
    i_row += T::QT;
    if (i_row >= N && i_left > 0) {
      ++i_gi;
      i_row = q_begin;
      set_head();
    }
  };
#pragma unroll
  for (int u = 0; u < T::AHEAD; ++u) issue(s0 + u < NS ? s0 + u : s0 + u - NS);

  // The slot read as "unit -1" holds zeros (its P and dS' are zero too);
  // the +inf table of fully masked units.
  {
    half_t* zs = lds + (s0 > 0 ? s0 - 1 : NS - 1) * T::STAGE;
    const u32x4 z = {0u, 0u, 0u, 0u};
    for (int i = tid; i < 2 * T::TILE / 8; i += T::NT) *reinterpret_cast<u32x4*>(zs + 8 * i) = z;
    if (tid < 64) reinterpret_cast<float*>(lds)[kInfOff + tid] = __builtin_inff();
  }
  // Units 0, 1, 2 landed (3, 4 in flight), zeros and table written.
  asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" : : "n"(2 * IPU) : "memory");

  int r_off[D / 16];  // row reads: row row_perm(ql), chunk 2*kk + g
#pragma unroll
  for (int kk = 0; kk < D / 16; ++kk) r_off[kk] = swz_offset<D>(row_perm(ql), 2 * kk + g);
  int t_off[D / 32][2];  // transposed reads (see read_tr)
  {
    const int grp = lane >> 4, i = lane & 15, r = i >> 2, qq = i & 3;
#pragma unroll
    for (int db = 0; db < D / 32; ++db) {
      const int col = 32 * db + 16 * (grp & 1) + 4 * qq;
#pragma unroll
      for (int h2 = 0; h2 < 2; ++h2) {
        const int row = 8 * g + r + 4 * h2;
        t_off[db][h2] = row * D + 8 * swz_chunk<D>(row, col >> 3) + (col & 7);
      }
    }
  }
  auto tr8 = [&](const half_t* base, int db) {
    const half4 lo = __builtin_bit_cast(
        half4, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_short4*)(base + t_off[db][0])));
    const half4 hi = __builtin_bit_cast(
        half4, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_short4*)(base + t_off[db][1])));
    half8 v;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      v[e] = lo[e];
      v[4 + e] = hi[e];
    }
    return v;
  };
  // 16 per-query floats at tab[16h + e] (h = 0, 1; e = 0..7) for a table
  // pointer that already includes the lane's 8g: value j = 8h + e of the
  // lane's S values is query 16h + 8g + e.
  auto table16 = [&](const float* tab) {
    float16v r;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const float4v x0 = *reinterpret_cast<const float4v*>(&tab[16 * h]);
      const float4v x1 = *reinterpret_cast<const float4v*>(&tab[16 * h + 4]);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        r[8 * h + e] = x0[e];
        r[8 * h + 4 + e] = x1[e];
      }
    }
    return r;
  };

  float16v dk[D / 32], dv[D / 32];
#pragma unroll
  for (int db = 0; db < D / 32; ++db)
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      dk[db][j] = 0.f;
      dv[db][j] = 0.f;
    }

  const float* const fl = reinterpret_cast<const float*>(lds);
  int c_row = q_begin + (u_lo - min(u_lo / ntq, G - 1) * ntq) * T::QT;  // compute cursor
  // Float offset (from lds) of the lane's LSE' values for the unit of row qa
  // in ring slot slot: units a wave sees entirely before its keys read +inf.
  auto lse_table = [&](int slot, int qa) {
    if (CAUSAL && qa < k0w) return kInfOff + 8 * g;
    return (slot * T::STAGE + 2 * T::TILE) / 2 + 8 * g;
  };
  // Pipeline registers: LSE' - s, dPd of the current unit; P, dS' of the
  // previous one.
  float16v s_cur, dp_cur;
  {
    const half_t* first = lds + s0 * T::STAGE;
    dp_cur = table16(reinterpret_cast<const float*>(first + 2 * T::TILE) + 64 + 8 * g);
    s_cur = table16(fl + lse_table(s0, c_row));
#pragma unroll
    for (int kk = 0; kk < D / 16; ++kk) {
      s_cur = mma<E>(*reinterpret_cast<const half8*>(first + r_off[kk]), kf[kk], s_cur);
      dp_cur = mma<E>(*reinterpret_cast<const half8*>(first + T::TILE + r_off[kk]), vn[kk], dp_cur);
    }
  }
  half8 pa_prev[2], sa_prev[2];
#pragma unroll
  for (int h = 0; h < 2; ++h)
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      pa_prev[h][e] = (half_t)0.f;
      sa_prev[h][e] = (half_t)0.f;
    }

  // D = 128 holds dK and dV (128 registers) in AGPRs, beside ~250 VGPRs.
  constexpr bool kAgprAcc = D > 64;
  auto acc_mfma = [&](float16v& acc, const half8& a, const half8& b) {
    if constexpr (kAgprAcc) mma_agpr<E>(acc, a, b);
    else acc = mma<E>(a, b, acc);
  };
  auto dvdk = [&](const half_t* slot) {
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int db = 0; db < D / 32; ++db) {
        acc_mfma(dv[db], tr8(slot + T::TILE + 16 * h * D, db), pa_prev[h]);
        acc_mfma(dk[db], tr8(slot + 16 * h * D, db), sa_prev[h]);
      }
  };

  // Body of one unit in ring slot SLOT (see the header comment).
  // Operands of the second unit of a step, read during the first (FA_BWD_XPREFETCH).
  // Step p reads the slots of units 2p-1 .. 2p+2 and its DMA fills those of
  // units 2p+5, 2p+6 (see `step`), which are other slots of the 8-slot ring.
  half8 xpre[FA_DKDV_LEAD];
  static_assert(NS == 8, "the step's DMA targets (units 2p+5, 2p+6) assume an 8-slot ring");
  auto body = [&](auto slot_c) __attribute__((always_inline)) {
    constexpr int SLOT = decltype(slot_c)::value;
    // Steps run units in slots (2p, 2p+1): the even one prefetches for the odd one.
    constexpr bool kMakesPre = FA_BWD_XPREFETCH && SLOT % 2 == 0;
    constexpr bool kTakesPre = FA_BWD_XPREFETCH && SLOT % 2 == 1;
    const half_t* cur = lds + SLOT * T::STAGE;
    const half_t* nxt = lds + ((SLOT + 1) % NS) * T::STAGE;
    const half_t* prv = lds + ((SLOT + NS - 1) % NS) * T::STAGE;
    const int qa = c_row;
    c_row += T::QT;
    if (c_row >= N) c_row = q_begin;  // next query head of the group

    // LSE' offset of the next unit, whose S accumulator starts from it.
    int ltab = lse_table((SLOT + 1) % NS, c_row);
    if constexpr (CAUSAL) {
      if (qa == k0w) {
        // diagonal unit: query 16h + 8g + e is kept iff it is >= key ql
#pragma unroll
        for (int j = 0; j < 16; ++j)
          if (16 * (j >> 3) + 8 * g + (j & 7) < ql) s_cur[j] = __builtin_inff();
      }
    }

    // Hand-ordered body: 16 (D = 64) or 8 (D = 32) MFMA tasks in the order
    // dV, dK (unit u-1), S, dPd (unit u+1), repeated, so that no two
    // adjacent tasks share an accumulator. Group i issues the LDS reads of
    // task i + kLead, runs task i and part of unit u's vector work; fences
    // keep the compiler from regrouping.
    constexpr int NQ = D / 16;  // tasks of each kind
    constexpr int NTASK = 4 * NQ;
    constexpr int kLead = FA_DKDV_LEAD;
    // Operand of task t of the body whose previous unit's rows are at p and
    // next unit's rows at n.
    auto load_op_at = [&](auto t_c, const half_t* p, const half_t* n) -> half8 {
      constexpr int t = decltype(t_c)::value;
      constexpr int kind = dkdv_task_kind<NQ>(t), q = dkdv_task_q<NQ>(t);
      constexpr int h = q / (D / 32), db = q % (D / 32);
      if constexpr (kind == 0) return tr8(p + T::TILE + 16 * h * D, db);
      else if constexpr (kind == 1) return tr8(p + 16 * h * D, db);
      else if constexpr (kind == 2) return *reinterpret_cast<const half8*>(n + r_off[q]);
      else return *reinterpret_cast<const half8*>(n + T::TILE + r_off[q]);
    };
    auto load_op = [&](auto t_c) -> half8 { return load_op_at(t_c, prv, nxt); };
    // The next body (slot SLOT + 1) reads its previous unit from this slot.
    const half_t* nxt2 = lds + ((SLOT + 2) % NS) * T::STAGE;
    float16v s_nx, dp_nx;
    auto run_task = [&](auto t_c, const half8& op) {
      constexpr int t = decltype(t_c)::value;
      constexpr int kind = dkdv_task_kind<NQ>(t), q = dkdv_task_q<NQ>(t);
      constexpr int h = q / (D / 32), db = q % (D / 32);
      if constexpr (kind == 0) acc_mfma(dv[db], op, pa_prev[h]);
      else if constexpr (kind == 1) acc_mfma(dk[db], op, sa_prev[h]);
      else if constexpr (kind == 2) s_nx = mma<E>(op, kf[q], s_nx);
      else dp_nx = mma<E>(op, vn[q], dp_nx);
    };
    half8 pa[2], sa[2];
    // Vector work on value pairs (2pr, 2pr+1) in two stages placed in
    // different groups, so that an MFMA separates each exp from its users:
    //   A: p = exp2(-(LSE' - s))      B: dS' = p dPd, both packed to fp16.
    // The empty asm statements pin each stage to its fenced group (plain
    // arithmetic would otherwise float).
    float pexp[16];
    auto stage_a = [&](int pr) {
      float p2[2];
#pragma unroll
      for (int e = 0; e < 2; ++e) p2[e] = exp2_fast(-s_cur[2 * pr + e]);
      asm volatile("" : "+v"(p2[0]), "+v"(p2[1]));
      pexp[2 * pr] = p2[0];
      pexp[2 * pr + 1] = p2[1];
    };
    // At D = 32 (vector-issue bound) fp16 dS' is the packed product of the
    // fp16 P, which dV needs anyway, and fp16 dPd: one v_pk_mul_f16 and one
    // conversion per pair instead of two multiplies and a conversion (B1 Hq8
    // Hkv2 N16381 fwd+bwd 0.829 -> 0.815 ms; dK rel-L2 4.8e-4 vs 3.9e-4 against
    // the fp32 reference). It rounds Delta - dP to fp16 first, so it assumes
    // |Delta - dP| < 65504 (fp16's largest finite value).
    auto stage_b = [&](int pr) {
      half2v pp, ss;
      if constexpr (D == 32 && std::is_same<E, F16>::value) {
        half2v dd;
#pragma unroll
        for (int e = 0; e < 2; ++e) {
          pp[e] = (_Float16)pexp[2 * pr + e];
          dd[e] = (_Float16)dp_cur[2 * pr + e];
        }
        ss = pp * dd;
      } else {
#pragma unroll
        for (int e = 0; e < 2; ++e) {
          const int j = 2 * pr + e;
          pp[e] = to_elem<E>(pexp[j]);
          ss[e] = to_elem<E>(pexp[j] * dp_cur[j]);
        }
      }
      asm volatile("" : "+v"(pp), "+v"(ss));
      const int j = 2 * pr;
      pa[j >> 3][j & 7] = pp[0];
      pa[j >> 3][(j & 7) + 1] = pp[1];
      sa[j >> 3][j & 7] = ss[0];
      sa[j >> 3][(j & 7) + 1] = ss[1];
    };

    half8 op[NTASK];
    // The LSE' offset as an opaque value, so that its loads stay after the
    // fence instead of being split into the branches above.
    __builtin_amdgcn_sched_barrier(0);
    asm volatile("" : "+v"(ltab));
    static_for<0, kLead>([&](auto t_c) {
      if constexpr (kTakesPre) op[decltype(t_c)::value] = xpre[decltype(t_c)::value];
      else op[decltype(t_c)::value] = load_op(t_c);
    });
    s_nx = table16(fl + ltab);
    dp_nx = table16(reinterpret_cast<const float*>(nxt + 2 * T::TILE) + 64 + 8 * g);
    __builtin_amdgcn_sched_barrier(0);
    static_for<0, NTASK>([&](auto i_c) {
      constexpr int i = decltype(i_c)::value;
      if constexpr (i + kLead < NTASK)
        op[i + kLead] = load_op(std::integral_constant<int, i + kLead>{});
      else if constexpr (kMakesPre)
        xpre[i + kLead - NTASK] =
            load_op_at(std::integral_constant<int, i + kLead - NTASK>{}, cur, nxt2);
      run_task(i_c, op[i]);
      // vector work of unit u: stage A of pair pr in group (2pr NTASK)/16,
      // stage B one group later (B of the last pair shares the last group)
#pragma unroll
      for (int pr = 0; pr < 8; ++pr) {
        constexpr int kSpan = NTASK;
        const int ga = (2 * pr * kSpan) / 16;
        const int gb = ga + 1 < NTASK ? ga + 1 : NTASK - 1;
        if (ga == i) stage_a(pr);
        if (gb == i) stage_b(pr);
      }
      __builtin_amdgcn_sched_barrier(0);
    });

    s_cur = s_nx;
    dp_cur = dp_nx;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      pa_prev[h] = pa[h];
      sa_prev[h] = sa[h];
    }
  };

  // Step p of the unrolled loop: units in slots 2p, 2p+1; issues the units
  // 5 and 6 ahead (slots of the units finished before the last barrier).
  auto step = [&](auto p_c) __attribute__((always_inline)) {
    constexpr int P = decltype(p_c)::value;
    issue((2 * P + 5) % NS);
    issue((2 * P + 6) % NS);
    body(std::integral_constant<int, 2 * P>{});
    body(std::integral_constant<int, 2 * P + 1>{});
    // Units up to 2s+4 landed for this wave, then published.
    wait_vm_and_barrier<2 * IPU>();
  };

  // The first turn from step p0 (its branches run once), then whole turns.
  static_assert(NS % 2 == 0, "whole two-unit steps per ring turn");
  if (npad > 0) {
    bwd_static_for<0, NS / 2>([&](auto p_c) {
      if (decltype(p_c)::value >= p0) step(p_c);
    });
    for (int u = NS; u < npad; u += NS) bwd_static_for<0, NS / 2>([&](auto p_c) { step(p_c); });
  }
  // dV/dK of the last unit run, in the ring's last slot (zeros if it was a
  // padding unit, or the zeroed slot if no unit ran).
  dvdk(lds + (NS - 1) * T::STAGE);
  if constexpr (kAgprAcc) agpr_acc_drain();
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");

  const float nscale = -a.scale;  // dK accumulated -dS
  if (a.nsplit > 1) {
    const int64_t plane = (int64_t)a.BHkv * Nkv * D;
    float* pk = a.part + (int64_t)split * 2 * plane + (int64_t)kvh * Nkv * D;
    float* pv = pk + plane;
    if (krow < Nkv) {
#pragma unroll
      for (int db = 0; db < D / 32; ++db)
#pragma unroll
        for (int jq = 0; jq < 4; ++jq) {
          const int64_t e0 = (int64_t)krow * D + 32 * db + 8 * jq + 4 * g;
          float4v kq, vq;
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            kq[e] = dk[db][4 * jq + e] * nscale;
            vq[e] = dv[db][4 * jq + e];
          }
          *reinterpret_cast<float4v*>(pk + e0) = kq;
          *reinterpret_cast<float4v*>(pv + e0) = vq;
        }
    }
    return;
  }
  const rsrc_t rdk = make_rsrc(a.dk + (int64_t)kvh * Nkv * D, kv_slab);
  const rsrc_t rdv = make_rsrc(a.dv + (int64_t)kvh * Nkv * D, kv_slab);
#pragma unroll
  for (int db = 0; db < D / 32; ++db)
#pragma unroll
    for (int jq = 0; jq < 4; ++jq) {
      const uint32_t off = (uint32_t)(krow * D + 32 * db + 8 * jq + 4 * g) * 2u;
      buf_store_b64(rdk, off,
                    pack4<E>(dk[db][4 * jq] * nscale, dk[db][4 * jq + 1] * nscale,
                               dk[db][4 * jq + 2] * nscale, dk[db][4 * jq + 3] * nscale));
      buf_store_b64(rdv, off,
                    pack4<E>(dv[db][4 * jq], dv[db][4 * jq + 1], dv[db][4 * jq + 2],
                               dv[db][4 * jq + 3]));
    }
}

// --------------------------------------------------------------------------
// dQ, software-pipelined over 32-key units.
//
// Work-group: NW waves x 32 queries (Q, dO as MFMA B operands, LSE and Delta
// one per lane), 32-key units (K, V rows) streamed through an 8-slot LDS DMA
// ring, two units per barrier step. The body of unit u runs
//   vector work of unit u      P^T = exp2(-Sl^T), dS'^T = P^T dPd^T
//   matrix work of unit u + 1  Sl^T = LSE - K fp16(c Q)^T, dPd^T = Delta - V dO^T
//   matrix work of unit u - 1  dQ^T += K^T dS'^T      (K^T via transposing reads)
// The scores use the reference's scaled query operand fp16(c Q) (q_scaled,
// attention.py:515); both accumulators start from per-query values (operands
// -fp16(c Q) and -dO), so dS' = -dS and dQ is negated once at the end. Keys
// past N need no mask: their K and V rows load as zeros, so their P (finite)
// multiplies zero. Causal: units of keys after all of a wave's queries, and
// the masked values of the diagonal unit, get Sl = +inf (P = 0 exactly).
// Each work-group rounds its unit count up to the 8-unit unroll (padding
// units are zeros).
// --------------------------------------------------------------------------
#ifndef FA_DQ_NSTAGE
#define FA_DQ_NSTAGE 8
#endif

template <int D, int NW>
struct DqPipeTile {
  static constexpr int BQ = 32 * NW;
  static constexpr int NT = 64 * NW;
  static constexpr int KT = 32;
  static constexpr int TILE = KT * D;   // halves of the K (or V) unit
  static constexpr int STAGE = 2 * TILE;
  static constexpr int NSTAGE = FA_DQ_NSTAGE;
  // Units issued ahead: the ring less the three a step reads (its two units
  // and the next unit's S operand).
  static constexpr int AHEAD = NSTAGE - 3;
  static_assert(NSTAGE % 2 == 0 && NSTAGE >= 8, "whole two-unit steps per ring turn");
  // D <= 64: two work-groups per CU; D = 128: one (dQ accumulated in AGPRs).
  static constexpr int WGS_PER_CU = D <= 64 ? 2 : 1;
};

template <int D, int NW>
constexpr bool dq_pipe_tiling_ok() {
  using T = DqPipeTile<D, NW>;
  constexpr int instr = T::TILE * 2 / 1024;
  return (T::TILE * 2) % 1024 == 0 &&
         ((instr <= NW && NW % instr == 0) || instr == 2 * NW) &&
         T::WGS_PER_CU * T::NSTAGE * T::STAGE * 2 <= 160 * 1024;
}

#ifndef FA_DQ_LEAD
#define FA_DQ_LEAD 3
#endif

// A dQ launch whose key ranges have no unit reaching past them that its
// queries see: the causal mask hides keys past N_kv when N_q <= N_kv (in one
// pass), and a bidirectional pass over N_kv a multiple of 64 has whole units
// in even number (no padding unit). Those launches skip the tail test.
inline bool dq_tail_free(const BwdArgs& a, bool causal) {
  if (a.nsplit != 1) return false;
  return causal ? a.N <= a.Nkv : a.Nkv % 64 == 0;
}

// TAIL: the launch may have units with keys past its range (see the body);
// dq_tail_free() says when it cannot.
template <int D, bool CAUSAL, int NW, class E, bool TAIL = true>
__device__ __forceinline__ void dq_pipe_body(const BwdArgs& a, const unsigned block,
                                        half_t* __restrict__ lds) {
  using T = DqPipeTile<D, NW>;
  using Dma = DmaStager<D, T::KT, NW>;
  static_assert(Dma::PER_WAVE == 1 || Dma::PER_WAVE == 2, "one or two tile pieces per wave");
  constexpr int NS = T::NSTAGE;
  constexpr int IPU = 2 * Dma::PER_WAVE;  // this wave's DMA instructions per unit: K, V pieces

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int ql = lane & 31;
  const int g = lane >> 5;

  // Split mode: the split index is the slowest-varying part of the block index.
  const int split = block / (a.num_tiles * a.BH);
  const TileHead th =
      decode_block_grouped(block - split * a.num_tiles * a.BH, a.BH, a.group);
  const int qtile = CAUSAL ? (a.num_tiles - 1 - th.tile_rank) : th.tile_rank;
  const int head = th.head;
  const int b = head / a.Hq;
  const int hq = head - b * a.Hq;
  const int kvh = b * a.Hkv + hq / a.group;
  const int N = a.N;      // queries
  const int Nkv = a.Nkv;  // keys
  const uint32_t slab = (uint32_t)N * D * 2u;
  const uint32_t kv_slab = (uint32_t)Nkv * D * 2u;
  const uint32_t aux = (uint32_t)N * 4u;
  const rsrc_t rq = make_rsrc(a.q + (int64_t)head * N * D, slab);
  const rsrc_t rdo = make_rsrc(a.dO + (int64_t)head * N * D, slab);
  const rsrc_t rl = make_rsrc(a.lse + (int64_t)head * N, aux);
  const rsrc_t rd = make_rsrc(a.delta + (int64_t)head * N, aux);
  const int4v r_k = make_rsrc_words(a.k + (int64_t)kvh * Nkv * D, kv_slab);
  const int4v r_v = make_rsrc_words(a.v + (int64_t)kvh * Nkv * D, kv_slab);

  const int q0 = qtile * T::BQ;
  const int q0w = q0 + 32 * wave;
  const int qrow = q0w + ql;

  // -fp16(c Q) and -dO as B operands (column = query ql, d = 16*kk + 8*g .. +7).
  const float c = a.c;
  half8 qf[D / 16], don[D / 16];
#pragma unroll
  for (int kk = 0; kk < D / 16; ++kk) {
    const uint32_t off = (uint32_t)(qrow * D + 16 * kk + 8 * g) * 2u;
    qf[kk] = __builtin_bit_cast(half8, buf_load_b128(rq, off));
    don[kk] = neg8(__builtin_bit_cast(half8, buf_load_b128(rdo, off)));
  }
  const float lse = buf_load_f32(rl, (uint32_t)qrow * 4u);
  float delta;
  if (a.o != nullptr) {
    // Delta = rowsum(O * dO) of this lane's query (the halves g = 0, 1 hold
    // the two 8-wide halves of every 16-wide chunk of the row).
    const rsrc_t ro = make_rsrc(a.o + (int64_t)head * N * D, slab);
    float part = 0.f;
#pragma unroll
    for (int kk = 0; kk < D / 16; ++kk) {
      const half8 ov = __builtin_bit_cast(
          half8, buf_load_b128(ro, (uint32_t)(qrow * D + 16 * kk + 8 * g) * 2u));
#pragma unroll
      for (int e = 0; e < 8; ++e) part = fmaf(elem_to_f32<E>(ov[e]), -elem_to_f32<E>(don[kk][e]), part);
    }
    delta = halves_sum(part);
    if (g == 0 && qrow < N && split == 0) a.delta_out[(int64_t)head * N + qrow] = delta;
  } else {
    delta = buf_load_f32(rd, (uint32_t)qrow * 4u);
  }
  wait_all_vm();
#pragma unroll
  for (int kk = 0; kk < D / 16; ++kk)
#pragma unroll
    for (int e = 0; e < 8; ++e) qf[kk][e] = to_elem<E>(-c * elem_to_f32<E>(qf[kk][e]));
#pragma unroll
  for (int kk = 0; kk < D / 16; ++kk) asm volatile("" : "+v"(qf[kk]), "+v"(don[kk]));

  const int kv_end = CAUSAL ? min(Nkv, q0 + T::BQ) : Nkv;
  // This work-group's keys [kv_lo, kv_hi): all of [0, kv_end) unless split.
  const int kv_lo = split * a.split_keys;
  const int kv_hi = min(kv_end, kv_lo + a.split_keys);
  const int nunits = kv_hi > kv_lo ? (kv_hi - kv_lo + T::KT - 1) / T::KT : 0;
  const int npad = (nunits + NS - 1) / NS * NS;
  // The units end in the ring's last slot: the first ring turn starts at step
  // p0 (slot s0), so at most one padding unit runs and the loop over whole
  // turns has no branches between its steps.
  const int p0 = __builtin_amdgcn_readfirstlane((npad - nunits) / 2);
  const int s0 = 2 * p0;

  Dma dma;
  dma.init(wave, lane);
  const uint32_t lds0 = lds_addr(lds);
  int i_row = kv_lo;  // first key row of the next unit to fetch
  auto issue = [&](int slot) __attribute__((always_inline)) {
    const int row0 = i_row < kv_hi ? i_row : Nkv;  // past the range: zeros
    const uint32_t vt = (uint32_t)row0 * (D * 2u) + dma.voff[0];
    const uint32_t base = lds0 + (uint32_t)slot * (T::STAGE * 2u) + (uint32_t)dma.piece0 * 1024u;
    uint32_t saved;
    if constexpr (Dma::PER_WAVE == 1) {
      asm volatile(
          "s_mov_b32 %0, m0\n\t"
          "s_mov_b32 m0, %4\n\t"
          "buffer_load_dwordx4 %1, %2, 0 offen lds\n\t"
          "s_mov_b32 m0, %5\n\t"
          "buffer_load_dwordx4 %1, %3, 0 offen lds\n\t"
          "s_mov_b32 m0, %0"
          : "=&s"(saved)
          : "v"(vt), "s"(r_k), "s"(r_v), "s"(base), "s"(base + T::TILE * 2u)
          : "memory");
    } else {
      const uint32_t vt1 = (uint32_t)row0 * (D * 2u) + dma.voff[1];
      asm volatile(
          "s_mov_b32 %0, m0\n\t"
          "s_mov_b32 m0, %5\n\t"
          "buffer_load_dwordx4 %1, %3, 0 offen lds\n\t"
          "s_mov_b32 m0, %6\n\t"
          "buffer_load_dwordx4 %2, %3, 0 offen lds\n\t"
          "s_mov_b32 m0, %7\n\t"
          "buffer_load_dwordx4 %1, %4, 0 offen lds\n\t"
          "s_mov_b32 m0, %8\n\t"
          "buffer_load_dwordx4 %2, %4, 0 offen lds\n\t"
          "s_mov_b32 m0, %0"
          : "=&s"(saved)
          : "v"(vt), "v"(vt1), "s"(r_k), "s"(r_v), "s"(base), "s"(base + 1024u),
            "s"(base + T::TILE * 2u), "s"(base + T::TILE * 2u + 1024u)
          : "memory");
    }
    i_row += T::KT;
  };
#pragma unroll
  for (int u = 0; u < T::AHEAD; ++u) issue(s0 + u < NS ? s0 + u : s0 + u - NS);

  // The slot read as "unit -1" holds zeros (its dS' is zero too).
  {
    half_t* zs = lds + (s0 > 0 ? s0 - 1 : NS - 1) * T::STAGE;
    const u32x4 z = {0u, 0u, 0u, 0u};
    for (int i = tid; i < T::TILE / 8; i += T::NT) *reinterpret_cast<u32x4*>(zs + 8 * i) = z;
  }
  // Units 0, 1, 2 landed (the rest in flight), zeros written.
  constexpr int kInFlight = (T::AHEAD - 3) * IPU;
  asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" : : "n"(kInFlight) : "memory");

  // A wave whose 32 queries are all past N (in the last query tile, or in a
  // launch of few queries) has no dQ row to produce. It still issues its
  // share of every unit's loads and meets every barrier, exactly as the steps
  // below do (same slots, same order, same waits), but runs no body and
  // stores nothing: 3 of the 4 waves at 16 queries.
  if (q0w >= N) {
    auto idle_step = [&](auto p_c) __attribute__((always_inline)) {
      constexpr int P = decltype(p_c)::value;
      issue((2 * P + T::AHEAD) % NS);
      issue((2 * P + T::AHEAD + 1) % NS);
      wait_vm_and_barrier<kInFlight>();
    };
    if (npad > 0) {
      bwd_static_for<0, NS / 2>([&](auto p_c) {
        if (decltype(p_c)::value >= p0) idle_step(p_c);
      });
      for (int u = NS; u < npad; u += NS)
        bwd_static_for<0, NS / 2>([&](auto p_c) { idle_step(p_c); });
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    return;
  }

  int r_off[D / 16];  // row reads: row row_perm(ql), chunk 2*kk + g
#pragma unroll
  for (int kk = 0; kk < D / 16; ++kk) r_off[kk] = swz_offset<D>(row_perm(ql), 2 * kk + g);
  int t_off[D / 32][2];  // transposed reads (see read_tr)
  {
    const int grp = lane >> 4, i = lane & 15, r = i >> 2, qq = i & 3;
#pragma unroll
    for (int db = 0; db < D / 32; ++db) {
      const int col = 32 * db + 16 * (grp & 1) + 4 * qq;
#pragma unroll
      for (int h2 = 0; h2 < 2; ++h2) {
        const int row = 8 * g + r + 4 * h2;
        t_off[db][h2] = row * D + 8 * swz_chunk<D>(row, col >> 3) + (col & 7);
      }
    }
  }
  auto tr8 = [&](const half_t* base, int db) {
    const half4 lo = __builtin_bit_cast(
        half4, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_short4*)(base + t_off[db][0])));
    const half4 hi = __builtin_bit_cast(
        half4, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_short4*)(base + t_off[db][1])));
    half8 v;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      v[e] = lo[e];
      v[4 + e] = hi[e];
    }
    return v;
  };

  float16v dq[D / 32];
#pragma unroll
  for (int db = 0; db < D / 32; ++db)
#pragma unroll
    for (int j = 0; j < 16; ++j) dq[db][j] = 0.f;

  const float inf = __builtin_inff();
  // Accumulator starts: LSE and Delta of the lane's query in every value.
  float16v lse16, delta16;
#pragma unroll
  for (int j = 0; j < 16; ++j) {
    lse16[j] = lse;
    delta16[j] = delta;
  }
  // Pipeline registers: Sl^T, dPd^T of the current unit; dS'^T of the previous one.
  float16v s_cur = lse16, dp_cur = delta16;
#pragma unroll
  for (int kk = 0; kk < D / 16; ++kk) {
    s_cur = mma<E>(*reinterpret_cast<const half8*>(lds + s0 * T::STAGE + r_off[kk]), qf[kk], s_cur);
    dp_cur = mma<E>(*reinterpret_cast<const half8*>(lds + s0 * T::STAGE + T::TILE + r_off[kk]),
                    don[kk], dp_cur);
  }
  half8 sa_prev[2];
#pragma unroll
  for (int h = 0; h < 2; ++h)
#pragma unroll
    for (int e = 0; e < 8; ++e) sa_prev[h][e] = (half_t)0.f;

  // D = 128 holds dQ (64 registers) in AGPRs.
  constexpr bool kAgprAcc = D > 64;
  auto acc_mfma = [&](float16v& acc, const half8& a, const half8& b) {
    if constexpr (kAgprAcc) mma_agpr<E>(acc, a, b);
    else acc = mma<E>(a, b, acc);
  };
  auto dq_mm = [&](const half_t* slot) {
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int db = 0; db < D / 32; ++db) acc_mfma(dq[db], tr8(slot + 16 * h * D, db), sa_prev[h]);
  };

  int c_key = kv_lo;  // first key of the unit the body works on

  // Operands of the second unit of a step, read during the first (FA_BWD_XPREFETCH).
  half8 xpre[FA_DQ_LEAD];
  static_assert(T::AHEAD >= 3 && T::AHEAD + 1 <= NS - 1,
                "a step's DMA must not target the slots its two bodies read");
  auto body = [&](auto slot_c) __attribute__((always_inline)) {
    constexpr int SLOT = decltype(slot_c)::value;
    constexpr bool kMakesPre = FA_BWD_XPREFETCH && SLOT % 2 == 0;
    constexpr bool kTakesPre = FA_BWD_XPREFETCH && SLOT % 2 == 1;
    const half_t* cur = lds + SLOT * T::STAGE;
    const half_t* nxt = lds + ((SLOT + 1) % NS) * T::STAGE;
    const half_t* prv = lds + ((SLOT + NS - 1) % NS) * T::STAGE;
    const half_t* nxt2 = lds + ((SLOT + 2) % NS) * T::STAGE;
    const int ka = c_key;
    c_key += T::KT;

    // Keys past the range (past N_kv, or a padding unit) load as zero rows and
    // get P = 0, as the reference's invalid keys do (attention.py:339-340): a
    // zero score against an LSE below -128 would overflow exp2, and inf times
    // the zero key row is NaN. Such keys can only be in the range's last unit
    // or the padding unit after it, which the rotated ring start puts in the
    // ring's last two slots; the other bodies, and launches without such
    // units (TAIL = false), carry no test for them.
    constexpr bool kTailSlot = TAIL && SLOT >= NS - 2;
    if constexpr (CAUSAL) {
      if (ka > q0w) {
        // every key of the unit follows every query of the wave
#pragma unroll
        for (int j = 0; j < 16; ++j) s_cur[j] = inf;
      } else if (ka == q0w || (kTailSlot && ka + T::KT > kv_hi)) {
        // diagonal or tail unit: key ka + 16h + 8g + e (value j = 8h + e) is
        // kept iff it is <= the lane's query (and < kv_hi)
        const int lim = kTailSlot ? min(q0w + ql, kv_hi - 1) - ka : ql;
#pragma unroll
        for (int j = 0; j < 16; ++j)
          if (16 * (j >> 3) + 8 * g + (j & 7) > lim) s_cur[j] = inf;
      }
    } else if constexpr (kTailSlot) {
      if (ka + T::KT > kv_hi) {
        const int lim = kv_hi - 1 - ka;
#pragma unroll
        for (int j = 0; j < 16; ++j)
          if (16 * (j >> 3) + 8 * g + (j & 7) > lim) s_cur[j] = inf;
      }
    }

    // Hand-ordered body: 3 * D/16 MFMA tasks in the order dQ (unit u-1),
    // S^T, dPd^T (unit u+1), repeated; group i issues the LDS reads of task
    // i + kLead, runs task i and part of unit u's vector work.
    constexpr int NQ = D / 16;
    constexpr int NTASK = 3 * NQ;
    constexpr int kLead = FA_DQ_LEAD;
    // Operand of task t of the body whose previous unit's rows are at p and
    // next unit's rows at n.
    auto load_op_at = [&](auto t_c, const half_t* p, const half_t* n) -> half8 {
      constexpr int t = decltype(t_c)::value;
      constexpr int kind = t % 3, q = t / 3;
      constexpr int h = q / (D / 32), db = q % (D / 32);
      if constexpr (kind == 0) return tr8(p + 16 * h * D, db);
      else if constexpr (kind == 1) return *reinterpret_cast<const half8*>(n + r_off[q]);
      else return *reinterpret_cast<const half8*>(n + T::TILE + r_off[q]);
    };
    auto load_op = [&](auto t_c) -> half8 { return load_op_at(t_c, prv, nxt); };
    float16v s_nx = lse16, dp_nx = delta16;
    auto run_task = [&](auto t_c, const half8& op) {
      constexpr int t = decltype(t_c)::value;
      constexpr int kind = t % 3, q = t / 3;
      constexpr int h = q / (D / 32), db = q % (D / 32);
      if constexpr (kind == 0) acc_mfma(dq[db], op, sa_prev[h]);
      else if constexpr (kind == 1) s_nx = mma<E>(op, qf[q], s_nx);
      else dp_nx = mma<E>(op, don[q], dp_nx);
    };
    half8 sa[2];
    float pexp[16];
    // Vector work on value pairs in two stages placed in different groups:
    //   A: p = exp2(-Sl)      B: dS' = p dPd, packed to fp16.
    auto stage_a = [&](int pr) {
      float p2[2];
#pragma unroll
      for (int e = 0; e < 2; ++e) p2[e] = exp2_fast(-s_cur[2 * pr + e]);
      asm volatile("" : "+v"(p2[0]), "+v"(p2[1]));
      pexp[2 * pr] = p2[0];
      pexp[2 * pr + 1] = p2[1];
    };
    auto stage_b = [&](int pr) {
      half2v ss;
#pragma unroll
      for (int e = 0; e < 2; ++e) ss[e] = to_elem<E>(pexp[2 * pr + e] * dp_cur[2 * pr + e]);
      asm volatile("" : "+v"(ss));
      const int j = 2 * pr;
      sa[j >> 3][j & 7] = ss[0];
      sa[j >> 3][(j & 7) + 1] = ss[1];
    };

    half8 op[NTASK];
    __builtin_amdgcn_sched_barrier(0);
    static_for<0, kLead>([&](auto t_c) {
      if constexpr (kTakesPre) op[decltype(t_c)::value] = xpre[decltype(t_c)::value];
      else op[decltype(t_c)::value] = load_op(t_c);
    });
    __builtin_amdgcn_sched_barrier(0);
    static_for<0, NTASK>([&](auto i_c) {
      constexpr int i = decltype(i_c)::value;
      if constexpr (i + kLead < NTASK)
        op[i + kLead] = load_op(std::integral_constant<int, i + kLead>{});
      else if constexpr (kMakesPre)
        xpre[i + kLead - NTASK] =
            load_op_at(std::integral_constant<int, i + kLead - NTASK>{}, cur, nxt2);
      run_task(i_c, op[i]);
#pragma unroll
      for (int pr = 0; pr < 8; ++pr) {
        const int ga = (2 * pr * NTASK) / 16;
        const int gb = ga + 1 < NTASK ? ga + 1 : NTASK - 1;
        if (ga == i) stage_a(pr);
        if (gb == i) stage_b(pr);
      }
      __builtin_amdgcn_sched_barrier(0);
    });

    s_cur = s_nx;
    dp_cur = dp_nx;
#pragma unroll
    for (int h = 0; h < 2; ++h) sa_prev[h] = sa[h];
  };

  auto step = [&](auto p_c) __attribute__((always_inline)) {
    constexpr int P = decltype(p_c)::value;
    issue((2 * P + T::AHEAD) % NS);
    issue((2 * P + T::AHEAD + 1) % NS);
    body(std::integral_constant<int, 2 * P>{});
    body(std::integral_constant<int, 2 * P + 1>{});
    // the next step reads up to unit 2P + 4; later ones may stay in flight
    wait_vm_and_barrier<kInFlight>();
  };

  // The first turn from step p0, then whole turns (as in dK/dV above).
  if (npad > 0) {
    bwd_static_for<0, NS / 2>([&](auto p_c) {
      if (decltype(p_c)::value >= p0) step(p_c);
    });
    for (int u = NS; u < npad; u += NS) bwd_static_for<0, NS / 2>([&](auto p_c) { step(p_c); });
  }
  dq_mm(lds + (NS - 1) * T::STAGE);  // dQ of the last unit run (the ring's last slot)
  if constexpr (kAgprAcc) agpr_acc_drain();
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");

  const rsrc_t rdq = make_rsrc(a.dq + (int64_t)head * N * D, slab);
  store_dq<D, E>(a, rdq, split, head, qrow, dq, -a.scale);  // accumulated -dS
}

}  // namespace fa
