// fa_bwd_pipe16.hpp — the software-pipelined dQ and dK/dV bodies on 16x16x32
// MFMAs (gfx950, D <= 64). fa_bwd.hip wraps them as dQ tiling 5 and dK/dV
// tiling 5.
//
// Same work, ring, DMA and pipeline as dq_pipe_body (fa_bwd_pipe.hpp): a wave
// owns 32 queries, 32-key units stream through the 8-slot LDS ring, and the
// body of unit u runs the vector work of u against the S / dP MFMAs of u + 1
// and the dQ MFMAs of u - 1. What changes is the MFMA shape. Each 32 x 32
// block of scores is four 16 x 16 blocks (key block kb, query block qb), and
// every operand read from LDS feeds two MFMAs (the two query blocks, or the
// two key blocks), so LDS traffic, vector work and FLOP are those of the
// 32x32x16 body. Under random operands the chip sustains more 16x16x32 FLOP
// per second than 32x32x16 at its power limit (16x16x32 moves a quarter of
// the accumulator bytes per instruction).
//
// Layouts (lane l, c16 = l % 16, G = l / 16):
//   S^T, dP^T block (kb, qb): lane holds query 16 qb + c16 of the wave and
//     keys 16 kb + 4 G + j (j = 0..3) of the unit (the 16x16 result layout;
//     4 quad16(G) + j at D = 32, see rows16);
//   value v = 8 kb + 4 qb + j of the lane's 16 score values;
//   dQ^T block (dd, qb): lane holds query 16 qb + c16, d = 16 dd + 4 G + j.
// dQ^T += K^T dS'^T: k-slot 8 G + 4 kb + j of the MFMA is key 16 kb + 4 G + j,
// so the lane's dS' values of blocks (0, qb), (1, qb) are its B operand as
// they stand, and the K^T operand reads keys 4G..4G+3 and 16+4G..16+4G+3 with
// two transposing LDS reads.
#pragma once

#include "fa_bwd_pipe.hpp"

namespace fa {

template <int D, bool CAUSAL, int NW, class E, bool TAIL = true>
__device__ __forceinline__ void dq_pipe16_body(const BwdArgs& a, const unsigned block,
                                               half_t* __restrict__ lds) {
  using T = DqPipeTile<D, NW>;
  using Dma = DmaStager<D, T::KT, NW>;
  static_assert(D == 32 || D == 64, "16x16x32 dQ body: D <= 64");
  static_assert(Dma::PER_WAVE == 1 || Dma::PER_WAVE == 2, "one or two tile pieces per wave");
  constexpr int NS = T::NSTAGE;
  constexpr int IPU = 2 * Dma::PER_WAVE;  // this wave's DMA instructions per unit: K, V pieces
  constexpr int KD = D / 32;              // 32-wide d chunks: k-steps of S and dP
  constexpr int DD = D / 16;              // 16-row d blocks of dQ^T

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int c16 = lane & 15;
  const int G = lane >> 4;
  // k-slots 8 G .. 8 G + 7 of the S and dP MFMAs hold d = 32 kd + 8 sg .. +7:
  // the chunk order sg = -G mod 4 makes the K and V row reads free of LDS bank
  // conflicts (chunk 4 kd + G would be two-way conflicted, measured).
  const int sg = (4 - G) & 3;
  const int gq = quad16<D>(G);  // key quad (of 16) of the lane's result rows

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
  const int qrow0 = q0w + c16;  // query of block qb: qrow0 + 16 qb

  // -fp16(c Q) and -dO as B operands: column = query 16 qb + c16,
  // d = 32 kd + 8 sg .. +7. Rows past N read as zeros (buffer range check).
  const float c = a.c;
  half8 qf[2][KD], don[2][KD];
#pragma unroll
  for (int qb = 0; qb < 2; ++qb)
#pragma unroll
    for (int kd = 0; kd < KD; ++kd) {
      const uint32_t off = (uint32_t)((qrow0 + 16 * qb) * D + 32 * kd + 8 * sg) * 2u;
      qf[qb][kd] = __builtin_bit_cast(half8, buf_load_b128(rq, off));
      don[qb][kd] = neg8(__builtin_bit_cast(half8, buf_load_b128(rdo, off)));
    }
  float lse[2], delta[2];
#pragma unroll
  for (int qb = 0; qb < 2; ++qb) lse[qb] = buf_load_f32(rl, (uint32_t)(qrow0 + 16 * qb) * 4u);
  if (a.o != nullptr) {
    // Delta = rowsum(O * dO) of each of the lane's two queries; the lanes
    // l, l^16, l^32, l^48 hold the four quarters of every 32-wide chunk.
    const rsrc_t ro = make_rsrc(a.o + (int64_t)head * N * D, slab);
#pragma unroll
    for (int qb = 0; qb < 2; ++qb) {
      float part = 0.f;
#pragma unroll
      for (int kd = 0; kd < KD; ++kd) {
        const half8 ov = __builtin_bit_cast(
            half8, buf_load_b128(ro, (uint32_t)((qrow0 + 16 * qb) * D + 32 * kd + 8 * sg) * 2u));
#pragma unroll
        for (int e = 0; e < 8; ++e)
          part = fmaf(elem_to_f32<E>(ov[e]), -elem_to_f32<E>(don[qb][kd][e]), part);
      }
      delta[qb] = quarters_sum(part);
      const int qr = qrow0 + 16 * qb;
      if (G == 0 && qr < N && split == 0) a.delta_out[(int64_t)head * N + qr] = delta[qb];
    }
  } else {
#pragma unroll
    for (int qb = 0; qb < 2; ++qb) delta[qb] = buf_load_f32(rd, (uint32_t)(qrow0 + 16 * qb) * 4u);
  }
  wait_all_vm();
#pragma unroll
  for (int qb = 0; qb < 2; ++qb)
#pragma unroll
    for (int kd = 0; kd < KD; ++kd)
#pragma unroll
      for (int e = 0; e < 8; ++e) qf[qb][kd][e] = to_elem<E>(-c * elem_to_f32<E>(qf[qb][kd][e]));
#pragma unroll
  for (int qb = 0; qb < 2; ++qb)
#pragma unroll
    for (int kd = 0; kd < KD; ++kd) asm volatile("" : "+v"(qf[qb][kd]), "+v"(don[qb][kd]));

  const int kv_end = CAUSAL ? min(Nkv, q0 + T::BQ) : Nkv;
  // This work-group's keys [kv_lo, kv_hi): all of [0, kv_end) unless split.
  const int kv_lo = split * a.split_keys;
  const int kv_hi = min(kv_end, kv_lo + a.split_keys);
  const int nunits = kv_hi > kv_lo ? (kv_hi - kv_lo + T::KT - 1) / T::KT : 0;
  const int npad = (nunits + NS - 1) / NS * NS;
  // The units end in the ring's last slot (rotated start, as in dq_pipe_body).
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

  // A wave whose 32 queries are all past N has no dQ row to produce: it keeps
  // issuing its share of the ring's loads and meets every barrier, exactly as
  // the steps below do, but runs no body and stores nothing (as in
  // dq_pipe_body).
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

  // Row reads of K and V (A operands of S^T and dP^T): key row 16 kb + c16,
  // 16-byte chunk 4 kd + sg.
  int r_off[2][KD];
#pragma unroll
  for (int kb = 0; kb < 2; ++kb)
#pragma unroll
    for (int kd = 0; kd < KD; ++kd)
      r_off[kb][kd] = swz_offset<D>(16 * kb + rows16<D>(c16), 4 * kd + sg);
  // Transposing reads of K (A operand of dQ^T += K^T dS'^T): in 16-lane group
  // G, source lane i addresses key row 16 h + 4 gq + i / 4, columns
  // 16 dd + 4 (i % 4) .. +3, and lane i receives keys 16 h + 4 gq + 0..3 of
  // column (d) 16 dd + i (ds_read_b64_tr_b16).
  int t_off[DD][2];
#pragma unroll
  for (int dd = 0; dd < DD; ++dd)
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int row = 16 * h + 4 * gq + (c16 >> 2);
      const int col = 16 * dd + 4 * (c16 & 3);
      t_off[dd][h] = row * D + 8 * swz_chunk<D>(row, col >> 3) + (col & 7);
    }
  auto trk = [&](const half_t* base, int dd) {
    const half4 lo = __builtin_bit_cast(
        half4, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_short4*)(base + t_off[dd][0])));
    const half4 hi = __builtin_bit_cast(
        half4, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_short4*)(base + t_off[dd][1])));
    half8 v;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      v[e] = lo[e];
      v[4 + e] = hi[e];
    }
    return v;
  };

  float4v dq[DD][2];
#pragma unroll
  for (int dd = 0; dd < DD; ++dd)
#pragma unroll
    for (int qb = 0; qb < 2; ++qb)
#pragma unroll
      for (int j = 0; j < 4; ++j) dq[dd][qb][j] = 0.f;

  const float inf = __builtin_inff();
  // Accumulator starts: LSE and Delta of the block's query in every value.
  float4v lse4[2], delta4[2];
#pragma unroll
  for (int qb = 0; qb < 2; ++qb)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      lse4[qb][j] = lse[qb];
      delta4[qb][j] = delta[qb];
    }
  // Pipeline registers: Sl^T, dPd^T of the current unit ([kb][qb]); dS'^T of
  // the previous one (B operands, [qb]).
  float4v s_cur[2][2], dp_cur[2][2];
#pragma unroll
  for (int kb = 0; kb < 2; ++kb)
#pragma unroll
    for (int qb = 0; qb < 2; ++qb) {
      s_cur[kb][qb] = lse4[qb];
      dp_cur[kb][qb] = delta4[qb];
    }
#pragma unroll
  for (int kb = 0; kb < 2; ++kb)
#pragma unroll
    for (int kd = 0; kd < KD; ++kd) {
      const half_t* first = lds + s0 * T::STAGE;
      const half8 ok = *reinterpret_cast<const half8*>(first + r_off[kb][kd]);
      const half8 ov = *reinterpret_cast<const half8*>(first + T::TILE + r_off[kb][kd]);
#pragma unroll
      for (int qb = 0; qb < 2; ++qb) {
        s_cur[kb][qb] = mma16<E>(ok, qf[qb][kd], s_cur[kb][qb]);
        dp_cur[kb][qb] = mma16<E>(ov, don[qb][kd], dp_cur[kb][qb]);
      }
    }
  half8 sa_prev[2];
#pragma unroll
  for (int qb = 0; qb < 2; ++qb)
#pragma unroll
    for (int e = 0; e < 8; ++e) sa_prev[qb][e] = (half_t)0.f;

  auto dq_mm = [&](const half_t* slot) {
#pragma unroll
    for (int dd = 0; dd < DD; ++dd) {
      const half8 op = trk(slot, dd);
#pragma unroll
      for (int qb = 0; qb < 2; ++qb) dq[dd][qb] = mma16<E>(op, sa_prev[qb], dq[dd][qb]);
    }
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

    // Masks as in dq_pipe_body: keys after every query of the wave, the
    // diagonal unit, and keys past the range (only in the ring's last two
    // slots, see there) get Sl = +inf, so P = 0 exactly. Value (kb, qb, j) is
    // key ka + 16 kb + 4 gq + j against query q0w + 16 qb + c16.
    constexpr bool kTailSlot = TAIL && SLOT >= NS - 2;
    auto mask_from = [&](const int (&lim)[2]) {
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int qb = 0; qb < 2; ++qb)
#pragma unroll
          for (int j = 0; j < 4; ++j)
            if (16 * kb + 4 * gq + j > lim[qb]) s_cur[kb][qb][j] = inf;
    };
    if constexpr (CAUSAL) {
      if (ka > q0w) {
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
          for (int qb = 0; qb < 2; ++qb)
#pragma unroll
            for (int j = 0; j < 4; ++j) s_cur[kb][qb][j] = inf;
      } else if (ka == q0w || (kTailSlot && ka + T::KT > kv_hi)) {
        int lim[2];
#pragma unroll
        for (int qb = 0; qb < 2; ++qb)
          lim[qb] = kTailSlot ? min(q0w + 16 * qb + c16, kv_hi - 1) - ka : 16 * qb + c16;
        mask_from(lim);
      }
    } else if constexpr (kTailSlot) {
      if (ka + T::KT > kv_hi) {
        const int lim[2] = {kv_hi - 1 - ka, kv_hi - 1 - ka};
        mask_from(lim);
      }
    }

    // Hand-ordered body: 3 * D/16 tasks in the order dQ (unit u-1), S^T,
    // dPd^T (unit u+1), repeated; each task is one LDS operand and two MFMAs.
    // Group i issues the LDS reads of task i + kLead, runs task i and part of
    // unit u's vector work.
    constexpr int NQ = D / 16;
    constexpr int NTASK = 3 * NQ;
    constexpr int kLead = FA_DQ_LEAD;
    auto load_op_at = [&](auto t_c, const half_t* p, const half_t* n) -> half8 {
      constexpr int t = decltype(t_c)::value;
      constexpr int kind = t % 3, q = t / 3;
      constexpr int kb = q / KD, kd = q % KD;
      if constexpr (kind == 0) return trk(p, q);
      else if constexpr (kind == 1) return *reinterpret_cast<const half8*>(n + r_off[kb][kd]);
      else return *reinterpret_cast<const half8*>(n + T::TILE + r_off[kb][kd]);
    };
    auto load_op = [&](auto t_c) -> half8 { return load_op_at(t_c, prv, nxt); };
    float4v s_nx[2][2], dp_nx[2][2];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int qb = 0; qb < 2; ++qb) {
        s_nx[kb][qb] = lse4[qb];
        dp_nx[kb][qb] = delta4[qb];
      }
    auto run_task = [&](auto t_c, const half8& op) {
      constexpr int t = decltype(t_c)::value;
      constexpr int kind = t % 3, q = t / 3;
      constexpr int kb = q / KD, kd = q % KD;
#pragma unroll
      for (int qb = 0; qb < 2; ++qb) {
        if constexpr (kind == 0) dq[q][qb] = mma16<E>(op, sa_prev[qb], dq[q][qb]);
        else if constexpr (kind == 1) s_nx[kb][qb] = mma16<E>(op, qf[qb][kd], s_nx[kb][qb]);
        else dp_nx[kb][qb] = mma16<E>(op, don[qb][kd], dp_nx[kb][qb]);
      }
    };
    half8 sa[2];
    float pexp[16];
    // Vector work on value pairs (v = 2 pr, 2 pr + 1: block kb = pr / 4,
    // qb = pr / 2 % 2, j = 2 (pr % 2) + e) in two stages placed in different
    // groups:   A: p = exp2(-Sl)      B: dS' = p dPd, packed to fp16.
    auto stage_a = [&](int pr) {
      const int kb = pr >> 2, qb = (pr >> 1) & 1, j0 = 2 * (pr & 1);
      float p2[2];
#pragma unroll
      for (int e = 0; e < 2; ++e) p2[e] = exp2_fast(-s_cur[kb][qb][j0 + e]);
      asm volatile("" : "+v"(p2[0]), "+v"(p2[1]));
      pexp[2 * pr] = p2[0];
      pexp[2 * pr + 1] = p2[1];
    };
    auto stage_b = [&](int pr) {
      const int kb = pr >> 2, qb = (pr >> 1) & 1, j0 = 2 * (pr & 1);
      half2v ss;
#pragma unroll
      for (int e = 0; e < 2; ++e) ss[e] = to_elem<E>(pexp[2 * pr + e] * dp_cur[kb][qb][j0 + e]);
      asm volatile("" : "+v"(ss));
      sa[qb][4 * kb + j0] = ss[0];
      sa[qb][4 * kb + j0 + 1] = ss[1];
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

#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int qb = 0; qb < 2; ++qb) {
        s_cur[kb][qb] = s_nx[kb][qb];
        dp_cur[kb][qb] = dp_nx[kb][qb];
      }
#pragma unroll
    for (int qb = 0; qb < 2; ++qb) sa_prev[qb] = sa[qb];
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

  // The first turn from step p0, then whole turns (as in dq_pipe_body).
  if (npad > 0) {
    bwd_static_for<0, NS / 2>([&](auto p_c) {
      if (decltype(p_c)::value >= p0) step(p_c);
    });
    for (int u = NS; u < npad; u += NS) bwd_static_for<0, NS / 2>([&](auto p_c) { step(p_c); });
  }
  dq_mm(lds + (NS - 1) * T::STAGE);  // dQ of the last unit run (the ring's last slot)
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");

  // Epilogue: lane holds d = 16 dd + 4 G + j of query 16 qb + c16 (scaled by
  // -scale: the accumulator holds -dS K).
  const float mul = -a.scale;
  const rsrc_t rdq = make_rsrc(a.dq + (int64_t)head * N * D, slab);
  const bool split_mode = a.nsplit > 1;
#pragma unroll
  for (int qb = 0; qb < 2; ++qb) {
    const int qr = qrow0 + 16 * qb;
    const int64_t prow = ((int64_t)split * a.BH + head) * a.N + qr;
    float* po = split_mode ? a.part + prow * D : nullptr;  // part is null in one-pass mode
#pragma unroll
    for (int dd = 0; dd < DD; ++dd) {
      float4v v;
#pragma unroll
      for (int e = 0; e < 4; ++e) v[e] = dq[dd][qb][e] * mul;
      if (split_mode) {
        if (qr < a.N) *reinterpret_cast<float4v*>(po + 16 * dd + 4 * G) = v;
      } else {
        buf_store_b64(rdq, (uint32_t)(qr * D + 16 * dd + 4 * G) * 2u,
                      pack4<E>(v[0], v[1], v[2], v[3]));
      }
    }
  }
}

// --------------------------------------------------------------------------
// dK / dV on 16x16x32 MFMAs: dkdv_pipe_body's work, ring, DMA and pipeline
// (a wave owns 32 keys; 32-query units stream through the 8-slot ring with
// their LSE' and Delta tables), with each 32 x 32 block of scores as four
// 16 x 16 blocks (query block qb, key block kb).
// Layouts (lane l, c16 = l % 16, G = l / 16):
//   S, dP block (qb, kb): lane holds key 16 kb + c16 of the wave and queries
//     16 qb + 4 G + j (j = 0..3) of the unit (4 quad16(G) + j at D = 32);
//     value v = 8 qb + 4 kb + j;
//   dK^T, dV^T block (dd, kb): lane holds key 16 kb + c16, d = 16 dd + 4 G + j.
// dV^T += dO^T P and dK^T += Q^T dS': k-slot 8 G + 4 qb + j is query
// 16 qb + 4 G + j, so the lane's P (dS') values of blocks (0, kb), (1, kb) are
// the B operand as they stand; the dO^T (Q^T) operand reads queries
// 4G..4G+3 and 16+4G..16+4G+3 with two transposing LDS reads.
// --------------------------------------------------------------------------
template <int D, bool CAUSAL, int NW, class E>
__device__ __forceinline__ void dkdv_pipe16_body(const BwdArgs& a, const unsigned block,
                                                 half_t* __restrict__ lds) {
  using T = DkdvPipeTile<D, NW>;
  using Dma = DmaStager<D, T::QT, NW>;
  static_assert(D == 32 || D == 64, "16x16x32 dK/dV body: D <= 64");
  static_assert(Dma::PER_WAVE == 1 || Dma::PER_WAVE == 2, "one or two tile pieces per wave");
  constexpr int NS = T::NSTAGE;
  // this wave's DMA instructions per unit: its Q and dO pieces, LSE or Delta
  constexpr int IPU = 2 * Dma::PER_WAVE + 1;
  constexpr int kInfOff = NS * T::STAGE / 2;  // float offset of the +inf table
  constexpr int KD = D / 32;                  // 32-wide d chunks: k-steps of S and dP
  constexpr int DD = D / 16;                  // 16-row d blocks of dK^T, dV^T

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int c16 = lane & 15;
  const int G = lane >> 4;
  // k-slots 8 G .. +7 of the S and dP MFMAs hold d = 32 kd + 8 sg .. +7 (the
  // conflict-free row-read order of dq_pipe16_body).
  const int sg = (4 - G) & 3;
  const int gq = quad16<D>(G);  // query quad (of 16) of the lane's result rows

  const int split = block / (a.num_tiles * a.BHkv);
  const TileHead th = decode_block(block - split * a.num_tiles * a.BHkv, a.BHkv);
  const int kvh = th.head;
  const int b = kvh / a.Hkv;
  const int hkv = kvh - b * a.Hkv;
  const int QG = a.group;
  const int N = a.N;      // queries
  const int Nkv = a.Nkv;  // keys
  const uint32_t slab = (uint32_t)N * D * 2u;
  const uint32_t kv_slab = (uint32_t)Nkv * D * 2u;
  const uint32_t aux_bytes = (uint32_t)N * 4u;
  const rsrc_t rk = make_rsrc(a.k + (int64_t)kvh * Nkv * D, kv_slab);
  const rsrc_t rv = make_rsrc(a.v + (int64_t)kvh * Nkv * D, kv_slab);

  const int k0 = th.tile_rank * T::BKV;
  const int k0w = k0 + 32 * wave;
  const int krow0 = k0w + c16;  // key of block kb: krow0 + 16 kb

  // -fp16(c K) and -V as B operands (column = key 16 kb + c16, d = 32 kd +
  // 8 sg .. +7); the scaled key operand is the reference's k_scaled
  // (attention.py:435). Rows past N_kv read as zeros.
  const float c = a.c;
  half8 kf[2][KD], vn[2][KD];
#pragma unroll
  for (int kb = 0; kb < 2; ++kb)
#pragma unroll
    for (int kd = 0; kd < KD; ++kd) {
      const uint32_t off = (uint32_t)((krow0 + 16 * kb) * D + 32 * kd + 8 * sg) * 2u;
      kf[kb][kd] = __builtin_bit_cast(half8, buf_load_b128(rk, off));
      vn[kb][kd] = neg8(__builtin_bit_cast(half8, buf_load_b128(rv, off)));
    }
  wait_all_vm();
#pragma unroll
  for (int kb = 0; kb < 2; ++kb)
#pragma unroll
    for (int kd = 0; kd < KD; ++kd)
#pragma unroll
      for (int e = 0; e < 8; ++e) kf[kb][kd][e] = to_elem<E>(-c * elem_to_f32<E>(kf[kb][kd][e]));
#pragma unroll
  for (int kb = 0; kb < 2; ++kb)
#pragma unroll
    for (int kd = 0; kd < KD; ++kd) asm volatile("" : "+v"(kf[kb][kd]), "+v"(vn[kb][kd]));

  const int q_begin = CAUSAL ? k0 : 0;  // k0 is a multiple of 32
  const int ntq = max(1, (N - q_begin + T::QT - 1) / T::QT);
  const int total_units = CAUSAL && q_begin >= N ? 0 : QG * ntq;  // as in dkdv_pipe_body
  const int chunk = (total_units + a.nsplit - 1) / a.nsplit;
  const int u_lo = min(split * chunk, total_units);
  const int nunits = min(chunk, total_units - u_lo);
  const int npad = (nunits + NS - 1) / NS * NS;
  const int p0 = __builtin_amdgcn_readfirstlane((npad - nunits) / 2);
  const int s0 = 2 * p0;

  // Issue cursor (as in dkdv_pipe_body).
  int i_gi = min(u_lo / ntq, QG - 1);
  int i_row = q_begin + (u_lo - i_gi * ntq) * T::QT;
  int i_left = nunits;
  int4v r_q, r_do, r_aux;
  const bool is_lse = (wave & 1) == 0;  // even waves fetch LSE, odd waves Delta
  auto set_head = [&]() {
    const int head = b * a.Hq + hkv * QG + i_gi;
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

  // Row reads of Q and dO (A operands of S and dP): query row 16 qb + c16,
  // 16-byte chunk 4 kd + sg.
  int r_off[2][KD];
#pragma unroll
  for (int qb = 0; qb < 2; ++qb)
#pragma unroll
    for (int kd = 0; kd < KD; ++kd)
      r_off[qb][kd] = swz_offset<D>(16 * qb + rows16<D>(c16), 4 * kd + sg);
  // Transposing reads of dO and Q (A operands of dV^T and dK^T): in 16-lane
  // group G, source lane i addresses query row 16 h + 4 gq + i / 4, columns
  // 16 dd + 4 (i % 4) .. +3; lane i receives queries 16 h + 4 gq + 0..3 of
  // column (d) 16 dd + i.
  int t_off[DD][2];
#pragma unroll
  for (int dd = 0; dd < DD; ++dd)
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int row = 16 * h + 4 * gq + (c16 >> 2);
      const int col = 16 * dd + 4 * (c16 & 3);
      t_off[dd][h] = row * D + 8 * swz_chunk<D>(row, col >> 3) + (col & 7);
    }
  auto trq = [&](const half_t* base, int dd) {
    const half4 lo = __builtin_bit_cast(
        half4, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_short4*)(base + t_off[dd][0])));
    const half4 hi = __builtin_bit_cast(
        half4, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_short4*)(base + t_off[dd][1])));
    half8 v;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      v[e] = lo[e];
      v[4 + e] = hi[e];
    }
    return v;
  };
  // The lane's four per-query floats of query block qb from a table of the
  // unit's 32 queries: queries 16 qb + 4 gq .. +3.
  auto tab4 = [&](const float* tab, int qb) {
    return *reinterpret_cast<const float4v*>(tab + 16 * qb + 4 * gq);
  };

  float4v dk[DD][2], dv[DD][2];
#pragma unroll
  for (int dd = 0; dd < DD; ++dd)
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        dk[dd][kb][j] = 0.f;
        dv[dd][kb][j] = 0.f;
      }

  const float* const fl = reinterpret_cast<const float*>(lds);
  int c_row = q_begin + (u_lo - min(u_lo / ntq, QG - 1) * ntq) * T::QT;  // compute cursor
  // Float offset (from lds) of the LSE' table of the unit of row qa in ring
  // slot `slot`: units a wave sees entirely before its keys read +inf.
  auto lse_table = [&](int slot, int qa) {
    if (CAUSAL && qa < k0w) return kInfOff;
    return (slot * T::STAGE + 2 * T::TILE) / 2;
  };
  // Pipeline registers: LSE' - s, dPd of the current unit ([qb][kb]); P, dS'
  // of the previous one (B operands, [kb]).
  float4v s_cur[2][2], dp_cur[2][2];
  {
    const half_t* first = lds + s0 * T::STAGE;
    const float* lt = fl + lse_table(s0, c_row);
    const float* dt = reinterpret_cast<const float*>(first + 2 * T::TILE) + 64;
#pragma unroll
    for (int qb = 0; qb < 2; ++qb) {
      const float4v l4 = tab4(lt, qb), d4 = tab4(dt, qb);
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
        s_cur[qb][kb] = l4;
        dp_cur[qb][kb] = d4;
      }
    }
#pragma unroll
    for (int qb = 0; qb < 2; ++qb)
#pragma unroll
      for (int kd = 0; kd < KD; ++kd) {
        const half8 oq = *reinterpret_cast<const half8*>(first + r_off[qb][kd]);
        const half8 od = *reinterpret_cast<const half8*>(first + T::TILE + r_off[qb][kd]);
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) {
          s_cur[qb][kb] = mma16<E>(oq, kf[kb][kd], s_cur[qb][kb]);
          dp_cur[qb][kb] = mma16<E>(od, vn[kb][kd], dp_cur[qb][kb]);
        }
      }
  }
  half8 pa_prev[2], sa_prev[2];
#pragma unroll
  for (int kb = 0; kb < 2; ++kb)
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      pa_prev[kb][e] = (half_t)0.f;
      sa_prev[kb][e] = (half_t)0.f;
    }

  auto dvdk = [&](const half_t* slot) {
#pragma unroll
    for (int dd = 0; dd < DD; ++dd) {
      const half8 od = trq(slot + T::TILE, dd);
      const half8 oq = trq(slot, dd);
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
        dv[dd][kb] = mma16<E>(od, pa_prev[kb], dv[dd][kb]);
        dk[dd][kb] = mma16<E>(oq, sa_prev[kb], dk[dd][kb]);
      }
    }
  };

  // Operands of the second unit of a step, read during the first (FA_BWD_XPREFETCH).
  half8 xpre[FA_DKDV_LEAD];
  static_assert(NS == 8, "the step's DMA targets (units 2p+5, 2p+6) assume an 8-slot ring");
  auto body = [&](auto slot_c) __attribute__((always_inline)) {
    constexpr int SLOT = decltype(slot_c)::value;
    constexpr bool kMakesPre = FA_BWD_XPREFETCH && SLOT % 2 == 0;
    constexpr bool kTakesPre = FA_BWD_XPREFETCH && SLOT % 2 == 1;
    const half_t* cur = lds + SLOT * T::STAGE;
    const half_t* nxt = lds + ((SLOT + 1) % NS) * T::STAGE;
    const half_t* prv = lds + ((SLOT + NS - 1) % NS) * T::STAGE;
    const int qa = c_row;
    c_row += T::QT;
    if (c_row >= N) c_row = q_begin;  // next query head of the group

    // LSE' table of the next unit, whose S accumulators start from it.
    int ltab = lse_table((SLOT + 1) % NS, c_row);
    if constexpr (CAUSAL) {
      if (qa == k0w) {
        // diagonal unit: value (qb, kb, j) is kept iff query 16 qb + 4 gq + j
        // is >= key 16 kb + c16
#pragma unroll
        for (int qb = 0; qb < 2; ++qb)
#pragma unroll
          for (int kb = 0; kb < 2; ++kb)
#pragma unroll
            for (int j = 0; j < 4; ++j)
              if (16 * qb + 4 * gq + j < 16 * kb + c16) s_cur[qb][kb][j] = __builtin_inff();
      }
    }

    // Hand-ordered body: 4 * D/16 tasks (dV, dK of unit u-1; S, dPd of unit
    // u+1), each one LDS operand and two MFMAs, in dkdv_pipe_body's order.
    constexpr int NQ = D / 16;
    constexpr int NTASK = 4 * NQ;
    constexpr int kLead = FA_DKDV_LEAD;
    auto load_op_at = [&](auto t_c, const half_t* p, const half_t* n) -> half8 {
      constexpr int t = decltype(t_c)::value;
      constexpr int kind = dkdv_task_kind<NQ>(t), q = dkdv_task_q<NQ>(t);
      constexpr int qb = q / KD, kd = q % KD;
      if constexpr (kind == 0) return trq(p + T::TILE, q);
      else if constexpr (kind == 1) return trq(p, q);
      else if constexpr (kind == 2) return *reinterpret_cast<const half8*>(n + r_off[qb][kd]);
      else return *reinterpret_cast<const half8*>(n + T::TILE + r_off[qb][kd]);
    };
    auto load_op = [&](auto t_c) -> half8 { return load_op_at(t_c, prv, nxt); };
    const half_t* nxt2 = lds + ((SLOT + 2) % NS) * T::STAGE;
    float4v s_nx[2][2], dp_nx[2][2];
    auto run_task = [&](auto t_c, const half8& op) {
      constexpr int t = decltype(t_c)::value;
      constexpr int kind = dkdv_task_kind<NQ>(t), q = dkdv_task_q<NQ>(t);
      constexpr int qb = q / KD, kd = q % KD;
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
        if constexpr (kind == 0) dv[q][kb] = mma16<E>(op, pa_prev[kb], dv[q][kb]);
        else if constexpr (kind == 1) dk[q][kb] = mma16<E>(op, sa_prev[kb], dk[q][kb]);
        else if constexpr (kind == 2) s_nx[qb][kb] = mma16<E>(op, kf[kb][kd], s_nx[qb][kb]);
        else dp_nx[qb][kb] = mma16<E>(op, vn[kb][kd], dp_nx[qb][kb]);
      }
    };
    half8 pa[2], sa[2];
    float pexp[16];
    // Vector work on value pairs (v = 2 pr, 2 pr + 1: block qb = pr / 4,
    // kb = pr / 2 % 2, j = 2 (pr % 2) + e) in two stages placed in different
    // groups:   A: p = exp2(-(LSE' - s))      B: dS' = p dPd, both packed.
    auto stage_a = [&](int pr) {
      const int qb = pr >> 2, kb = (pr >> 1) & 1, j0 = 2 * (pr & 1);
      float p2[2];
#pragma unroll
      for (int e = 0; e < 2; ++e) p2[e] = exp2_fast(-s_cur[qb][kb][j0 + e]);
      asm volatile("" : "+v"(p2[0]), "+v"(p2[1]));
      pexp[2 * pr] = p2[0];
      pexp[2 * pr + 1] = p2[1];
    };
    // At D = 32 fp16 dS' is the packed product of the fp16 P and fp16 dPd, as
    // in dkdv_pipe_body.
    auto stage_b = [&](int pr) {
      const int qb = pr >> 2, kb = (pr >> 1) & 1, j0 = 2 * (pr & 1);
      half2v pp, ss;
      if constexpr (D == 32 && std::is_same<E, F16>::value) {
        half2v dd;
#pragma unroll
        for (int e = 0; e < 2; ++e) {
          pp[e] = (_Float16)pexp[2 * pr + e];
          dd[e] = (_Float16)dp_cur[qb][kb][j0 + e];
        }
        ss = pp * dd;
      } else {
#pragma unroll
        for (int e = 0; e < 2; ++e) {
          pp[e] = to_elem<E>(pexp[2 * pr + e]);
          ss[e] = to_elem<E>(pexp[2 * pr + e] * dp_cur[qb][kb][j0 + e]);
        }
      }
      asm volatile("" : "+v"(pp), "+v"(ss));
      pa[kb][4 * qb + j0] = pp[0];
      pa[kb][4 * qb + j0 + 1] = pp[1];
      sa[kb][4 * qb + j0] = ss[0];
      sa[kb][4 * qb + j0 + 1] = ss[1];
    };

    half8 op[NTASK];
    __builtin_amdgcn_sched_barrier(0);
    asm volatile("" : "+v"(ltab));
    static_for<0, kLead>([&](auto t_c) {
      if constexpr (kTakesPre) op[decltype(t_c)::value] = xpre[decltype(t_c)::value];
      else op[decltype(t_c)::value] = load_op(t_c);
    });
    {
      const float* lt = fl + ltab;
      const float* dt = reinterpret_cast<const float*>(nxt + 2 * T::TILE) + 64;
#pragma unroll
      for (int qb = 0; qb < 2; ++qb) {
        const float4v l4 = tab4(lt, qb), d4 = tab4(dt, qb);
#pragma unroll
        for (int kb = 0; kb < 2; ++kb) {
          s_nx[qb][kb] = l4;
          dp_nx[qb][kb] = d4;
        }
      }
    }
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

#pragma unroll
    for (int qb = 0; qb < 2; ++qb)
#pragma unroll
      for (int kb = 0; kb < 2; ++kb) {
        s_cur[qb][kb] = s_nx[qb][kb];
        dp_cur[qb][kb] = dp_nx[qb][kb];
      }
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      pa_prev[kb] = pa[kb];
      sa_prev[kb] = sa[kb];
    }
  };

  auto step = [&](auto p_c) __attribute__((always_inline)) {
    constexpr int P = decltype(p_c)::value;
    issue((2 * P + 5) % NS);
    issue((2 * P + 6) % NS);
    body(std::integral_constant<int, 2 * P>{});
    body(std::integral_constant<int, 2 * P + 1>{});
    wait_vm_and_barrier<2 * IPU>();
  };

  if (npad > 0) {
    bwd_static_for<0, NS / 2>([&](auto p_c) {
      if (decltype(p_c)::value >= p0) step(p_c);
    });
    for (int u = NS; u < npad; u += NS) bwd_static_for<0, NS / 2>([&](auto p_c) { step(p_c); });
  }
  dvdk(lds + (NS - 1) * T::STAGE);
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");

  // Epilogue: lane holds d = 16 dd + 4 G + j of key 16 kb + c16.
  const float nscale = -a.scale;  // dK accumulated -dS
  if (a.nsplit > 1) {
    const int64_t plane = (int64_t)a.BHkv * Nkv * D;
    float* pk = a.part + (int64_t)split * 2 * plane + (int64_t)kvh * Nkv * D;
    float* pv = pk + plane;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
      const int krow = krow0 + 16 * kb;
      if (krow < Nkv) {
#pragma unroll
        for (int dd = 0; dd < DD; ++dd) {
          const int64_t e0 = (int64_t)krow * D + 16 * dd + 4 * G;
          float4v kq, vq;
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            kq[e] = dk[dd][kb][e] * nscale;
            vq[e] = dv[dd][kb][e];
          }
          *reinterpret_cast<float4v*>(pk + e0) = kq;
          *reinterpret_cast<float4v*>(pv + e0) = vq;
        }
      }
    }
    return;
  }
  const rsrc_t rdk = make_rsrc(a.dk + (int64_t)kvh * Nkv * D, kv_slab);
  const rsrc_t rdv = make_rsrc(a.dv + (int64_t)kvh * Nkv * D, kv_slab);
#pragma unroll
  for (int kb = 0; kb < 2; ++kb)
#pragma unroll
    for (int dd = 0; dd < DD; ++dd) {
      const uint32_t off = (uint32_t)((krow0 + 16 * kb) * D + 16 * dd + 4 * G) * 2u;
      buf_store_b64(rdk, off,
                    pack4<E>(dk[dd][kb][0] * nscale, dk[dd][kb][1] * nscale,
                             dk[dd][kb][2] * nscale, dk[dd][kb][3] * nscale));
      buf_store_b64(rdv, off, pack4<E>(dv[dd][kb][0], dv[dd][kb][1], dv[dd][kb][2], dv[dd][kb][3]));
    }
}

}  // namespace fa
