// fa_fwd.hip — FlashAttention-2 forward for gfx950.
//
// Semantics follow the reference forward (triton_flash_attention/attention.py):
//   scores in the log2 domain  s * scale * log2(e)               (61, 177)
//   invalid keys / causal keys -> -inf before the row max         (63-66)
//   online max / sum, P rounded to fp16 for P.V, fp32 sum          (68-73)
//   O = acc / l, LSE = m + log2(l) (base 2), tail rows not stored  (230-234)
//   causal: key tiles past the query tile are never visited        (43-49, 179-211)
//   GQA: key/value head = query head / (Hq / Hkv)                  (128-131)
//
// MI355X design (not a translation of the Triton program):
//   * one work-group = NW wavefronts x 32 query rows; each wave keeps its
//     32x D query tile in VGPRs as MFMA B-operands for the whole sweep;
//   * K and V tiles are staged row-major (XOR-swizzled, conflict-free) in a
//     3-slot LDS ring, one barrier per key tile; the V^T operand of P.V is
//     read with the transposing LDS read (ds_read_b64_tr_b16);
//   * software pipeline: the next tile's QK^T MFMAs are issued before this
//     tile's softmax so matrix and vector work of one wave overlap;
//   * the running max is moved lazily (threshold 2^8), skipping most O/l
//     rescales;
//   * S^T = K Q^T on v_mfma_f32_32x32x16_f16: each lane owns ONE query
//     column, so the row max needs one cross-half exchange and the per-row
//     rescale of the accumulator is a per-lane scalar;
//   * the K rows are read through row_perm so the fp16 P^T values a lane
//     holds are exactly the B-operand of O^T += V^T P^T (no shuffles);
//   * tails use the buffer range check (zero fill), masks run only on the
//     diagonal / tail tiles.
#include <type_traits>

#include "fa_common.hpp"
#include "fa_kernels.hpp"

namespace fa {

template <int D, int NW, int BN>
struct FwdTile {
  static constexpr int BM = 32 * NW;        // queries per work-group
  static constexpr int NT = 64 * NW;        // threads
  static constexpr int TILE = BN * D;       // halves of one K (or V) tile
  static constexpr int STAGE = 2 * TILE;    // halves per ring slot: K tile, V tile
  static constexpr int NSTAGE = 4;          // ring slots
  static constexpr int AHEAD = NSTAGE - 1;  // tiles in flight ahead of the consumer
  static constexpr int UNROLL = 4;          // lcm(NSTAGE, 2): static slot and score buffer
  static_assert(BN % 32 == 0, "key tile must be a multiple of 32");
  static_assert(NSTAGE * STAGE * 2 <= 160 * 1024, "LDS budget");
};

// Lazy reference max. P = exp2(s c - m) is first computed against the
// current reference max m; a lane's row sum of P over the tile is at least
// each of its P, so while every lane's sum stays <= 2^8 every P is <= 2^8
// (exact in fp16 and fp32) and nothing else is done. Otherwise (and on the
// first tile, where m = -inf gives inf / NaN sums) a rare branch computes the
// tile max, moves m to it, rescales O and l, and recomputes P. The max is
// thus only reduced when it is needed.
constexpr float kSumLimit = 256.0f;

template <int V>
using ic = std::integral_constant<int, V>;

// Epilogue, lane (query qrow, half g) holding d = 32*db + 8*(j/4) + 4*g + j%4
// of O (unnormalised), the reference max m and the row sum lt:
//   unsplit: O / lt as 16-bit through the range-checked resource ro, and the
//            base-2 LSE m + log2(lt);
//   split:   the fp32 partial O / lt and LSE of split `split` (a query that
//            saw no key of the split, lt == 0, writes O = 0 and LSE = -inf,
//            which the combine weighs with 0).
template <int D, class E, bool SPLITS = true>
__device__ __forceinline__ void store_fwd_output(const FwdArgs& a, const rsrc_t& ro, int split,
                                                 int head, int qrow, int g,
                                                 const float16v (&o)[D / 32], float m, float lt) {
  const bool split_mode = SPLITS && a.nsplit > 1;
  const bool seen = lt > 0.f;
  const float inv = seen ? 1.0f / lt : 0.f;
  // The lane's half is recomputed here (mbcnt needs no live register), so
  // no lane value has to stay live, and spill, across the main loop.
  g = (int)(__builtin_amdgcn_mbcnt_hi(~0u, __builtin_amdgcn_mbcnt_lo(~0u, 0u)) >> 5);
  const int64_t prow = ((int64_t)split * a.BH + head) * a.N + qrow;
  float* po = split_mode ? a.part + prow * D : nullptr;  // part is null in one-pass mode
  const bool row_ok = qrow < a.N;
#pragma unroll
  for (int db = 0; db < D / 32; ++db)
#pragma unroll
    for (int jq = 0; jq < 4; ++jq) {
      float4v v;
#pragma unroll
      for (int e = 0; e < 4; ++e) v[e] = o[db][4 * jq + e] * inv;
      if (split_mode) {
        if (row_ok) *reinterpret_cast<float4v*>(po + 32 * db + 8 * jq + 4 * g) = v;
      } else {
        buf_store_b64(ro, (uint32_t)(qrow * D + 32 * db + 8 * jq + 4 * g) * 2u,
                      pack4<E>(v[0], v[1], v[2], v[3]));
      }
    }
  if (g == 0 && row_ok) {
    const float lse = seen ? m + log2_fast(lt) : -INFINITY;
    if (split_mode) a.part[(int64_t)a.nsplit * a.BH * a.N * D + prow] = lse;
    else a.lse[(int64_t)head * a.N + qrow] = lse;
  }
}

// Split-KV is compiled for key tiles of at most 64 (the 128-key tiling is a
// sweep variant whose register allocation the split epilogue upsets).
template <int BN>
constexpr bool fwd_tile_splits_kv() {
  return BN <= 64;
}

template <int D, bool CAUSAL, int NW, int BN, class E = F16>
__global__ __launch_bounds__(64 * NW) void fwd_kernel(FwdArgs a) {
  using T = FwdTile<D, NW, BN>;
  constexpr bool kSplits = fwd_tile_splits_kv<BN>();
  using Dma = DmaStager<D, BN, NW>;
  constexpr int KB = BN / 32;                 // 32-key blocks per tile
  constexpr int IPT = 2 * Dma::PER_WAVE;      // this wave's DMA instructions per tile
  __shared__ __attribute__((aligned(16))) half_t lds[T::NSTAGE * T::STAGE];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform
  const int ql = lane & 31;
  const int g = lane >> 5;

  // Split-KV mode: the split index is the slowest-varying part of the block
  // index. Packed GQA: the work-group serves P query heads, wave w head w % P.
  const int P = a.pack;
  const int row_wgs = a.BH / P;  // work-groups per tile row
  const int split = kSplits ? blockIdx.x / (a.num_tiles * row_wgs) : 0;
  const TileHead th =
      decode_block_grouped(blockIdx.x - split * a.num_tiles * row_wgs, row_wgs, a.group / P);
  const int qtile = CAUSAL ? (a.num_tiles - 1 - th.tile_rank) : th.tile_rank;
  const int head = th.head * P + wave % P;  // wave-uniform
  const int b = head / a.Hq;
  const int hq = head - b * a.Hq;
  const int kvh = b * a.Hkv + hq / a.group;
  const int N = a.N;      // queries
  const int Nkv = a.Nkv;  // keys
  const uint32_t slab = (uint32_t)N * D * 2u;
  const uint32_t kv_slab = (uint32_t)Nkv * D * 2u;
  const rsrc_t rq = make_rsrc(a.q + (int64_t)head * N * D, slab);
  const rsrc_t ro = make_rsrc(a.o + (int64_t)head * N * D, slab);
  const int4v rk = make_rsrc_words(a.k + (int64_t)kvh * Nkv * D, kv_slab);
  const int4v rv = make_rsrc_words(a.v + (int64_t)kvh * Nkv * D, kv_slab);

  const int bm = T::BM / P;  // query rows per head
  const int q0 = qtile * bm;
  const int q0w = q0 + 32 * (wave / P);
  const int qrow = q0w + ql;

  const int kv_end = CAUSAL ? min(Nkv, q0 + bm) : Nkv;
  // This work-group's keys [kv_lo, kv_hi): all of [0, kv_end) unless split.
  const int kv_lo = kSplits ? split * a.split_keys : 0;
  const int kv_hi = kSplits ? min(kv_end, kv_lo + a.split_keys) : kv_end;
  const int ntiles = kv_hi > kv_lo ? (kv_hi - kv_lo + BN - 1) / BN : 0;

  // Q^T operand fragments: lane (query ql, k-half g), d = 16*kk + 8*g .. +7.
  // Completed before the first DMA so no later wait on them drains the ring.
  half8 qf[D / 16];
#pragma unroll
  for (int kk = 0; kk < D / 16; ++kk)
    qf[kk] = __builtin_bit_cast(half8, buf_load_b128(rq, (uint32_t)(qrow * D + 16 * kk + 8 * g) * 2u));
  wait_all_vm();

  // DMA prologue: tiles 0 .. AHEAD-1 into ring slots 0 .. AHEAD-1. Every
  // step then issues exactly one tile (past the end the loads read zeros or
  // unused rows), so the in-flight count is the same at every wait.
  Dma dma;
  dma.init(wave, lane);
  auto issue_tile = [&](int t, int slot) {
    const half_t* base = lds + slot * T::STAGE;
    dma.issue(rk, kv_lo + t * BN, base, wave);
    dma.issue(rv, kv_lo + t * BN, base + T::TILE, wave);
  };
#pragma unroll
  for (int t = 0; t < T::AHEAD; ++t) issue_tile(t, t);

  float16v o[D / 32];
#pragma unroll
  for (int db = 0; db < D / 32; ++db)
#pragma unroll
    for (int j = 0; j < 16; ++j) o[db][j] = 0.f;
  float m = -INFINITY;  // reference max (scaled, log2 units); may lag the true max by <= 8
  float l = 0.f;        // this lane's partial sum of exp2(s*c - m) (its 16 keys per block)
  const float c = a.c;

  // Loop-invariant per-lane LDS offsets (halves). The swizzle of a row does
  // not change when the row moves by a multiple of 16, so key blocks (32 rows)
  // and k-steps (16 rows) only add constants.
  int k_off[D / 16];  // row reads of K: row row_perm(ql), chunk 2*kk + g
#pragma unroll
  for (int kk = 0; kk < D / 16; ++kk) k_off[kk] = swz_offset<D>(row_perm(ql), 2 * kk + g);
  int v_off[D / 32][2];  // transposed reads of V (see read_tr)
  {
    const int grp = lane >> 4, i = lane & 15, r = i >> 2, qq = i & 3;
#pragma unroll
    for (int db = 0; db < D / 32; ++db) {
      const int col = 32 * db + 16 * (grp & 1) + 4 * qq;
#pragma unroll
      for (int h2 = 0; h2 < 2; ++h2) {
        const int row = 8 * g + r + 4 * h2;
        v_off[db][h2] = row * D + 8 * swz_chunk<D>(row, col >> 3) + (col & 7);
      }
    }
  }

  // A wave takes part in tile t unless all its queries are past the end or,
  // causally, before every key of the tile (wave-uniform).
  auto active = [&](int t) {
    return uniform((q0w < N) && !(CAUSAL && kv_lo + t * BN > q0w + 31)) != 0;
  };

  float16v sbuf[2][KB];  // S^T of two consecutive tiles (software pipeline)

  // S^T = K Q^T of the tile in ring slot SLOT into sbuf[SB].
  auto scores = [&](auto slot_c, auto sb_c) {
    constexpr int SLOT = decltype(slot_c)::value;
    constexpr int SB = decltype(sb_c)::value;
    const half_t* Ks = lds + SLOT * T::STAGE;
    half8 ka[KB][D / 16];
#pragma unroll
    for (int kb = 0; kb < KB; ++kb)
#pragma unroll
      for (int kk = 0; kk < D / 16; ++kk)
        ka[kb][kk] = *reinterpret_cast<const half8*>(Ks + 32 * kb * D + k_off[kk]);
#pragma unroll
    for (int kb = 0; kb < KB; ++kb) {
#pragma unroll
      for (int j = 0; j < 16; ++j) sbuf[SB][kb][j] = 0.f;
#pragma unroll
      for (int kk = 0; kk < D / 16; ++kk) sbuf[SB][kb] = mma<E>(ka[kb][kk], qf[kk], sbuf[SB][kb]);
    }
  };

  // One key tile: next DMA, next tile's scores, this tile's softmax + P.V.
  auto step = [&](auto slot_c, auto sb_c, int t_in) {
    constexpr int SLOT = decltype(slot_c)::value;
    constexpr int SB = decltype(sb_c)::value;
    const int t = uniform(t_in);
    const int kv0 = kv_lo + t * BN;
    // (1) tile t+AHEAD -> the slot tile t-1 used (released by the last barrier).
    issue_tile(t + T::AHEAD, (SLOT + T::AHEAD) % T::NSTAGE);
    const bool act = active(t);
    // (2) this tile's V^T fragments, read ahead of the softmax.
    half8 va[KB][2][D / 32];
    const half_t* Vs = lds + SLOT * T::STAGE + T::TILE;
    if (act) {
#pragma unroll
      for (int kb = 0; kb < KB; ++kb)
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
          for (int db = 0; db < D / 32; ++db) {
            const half_t* base = Vs + (32 * kb + 16 * h) * D;
            const half4 lo = __builtin_bit_cast(
                half4, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_short4*)(base + v_off[db][0])));
            const half4 hi = __builtin_bit_cast(
                half4, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_short4*)(base + v_off[db][1])));
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              va[kb][h][db][e] = lo[e];
              va[kb][h][db][4 + e] = hi[e];
            }
          }
    }
    // (3) next tile's scores: these MFMAs overlap the softmax below.
    if (t + 1 < ntiles && active(t + 1)) scores(ic<(SLOT + 1) % T::NSTAGE>{}, ic<1 - SB>{});

    if (act) {
      float16v* sc = sbuf[SB];
      const bool need_mask = uniform((CAUSAL && kv0 + BN - 1 > q0w) || (kv0 + BN > kv_hi)) != 0;
      if (need_mask) {
#pragma unroll
        for (int kb = 0; kb < KB; ++kb)
#pragma unroll
          for (int j = 0; j < 16; ++j) {
            const int key = kv0 + 32 * kb + result_row(j, g);
            const bool ok = key < kv_hi && (!CAUSAL || key <= qrow);
            if (!ok) sc[kb][j] = -INFINITY;
          }
      }
      half8 pk[KB][2];
      // P against the current reference max, and this lane's row sum.
      auto probs = [&](const float16v* s) {
        const float nm = -m;
        float ls4[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int kb = 0; kb < KB; ++kb)
#pragma unroll
          for (int j = 0; j < 16; ++j) {
            const float p = exp2_fast(fmaf(s[kb][j], c, nm));
            ls4[j & 3] += p;
            pk[kb][j >> 3][j & 7] = to_elem<E>(p);
          }
        return (ls4[0] + ls4[1]) + (ls4[2] + ls4[3]);
      };
      float lt = probs(sc);
      if (__builtin_amdgcn_ballot_w64(!(lt <= kSumLimit)) != 0) {
        // Rare: the scores are rebuilt from the K tile (still in this slot)
        // rather than kept alive across the common path.
        float16v s2[KB];
        const half_t* Ks = lds + SLOT * T::STAGE;
#pragma unroll
        for (int kb = 0; kb < KB; ++kb) {
#pragma unroll
          for (int j = 0; j < 16; ++j) s2[kb][j] = 0.f;
#pragma unroll
          for (int kk = 0; kk < D / 16; ++kk)
            s2[kb] = mma<E>(*reinterpret_cast<const half8*>(Ks + 32 * kb * D + k_off[kk]), qf[kk],
                            s2[kb]);
        }
        float mx = -INFINITY;
#pragma unroll
        for (int kb = 0; kb < KB; ++kb)
#pragma unroll
          for (int j = 0; j < 16; ++j) {
            const int key = kv0 + 32 * kb + result_row(j, g);
            if (need_mask && (key >= kv_hi || (CAUSAL && key > qrow))) s2[kb][j] = -INFINITY;
            mx = fmaxf(mx, s2[kb][j]);
          }
        mx = halves_max(mx) * c;
        const float m_new = fmaxf(m, mx);
        const float alpha = exp2_fast(m - m_new);
        l *= alpha;
#pragma unroll
        for (int db = 0; db < D / 32; ++db) o[db] *= alpha;
        m = m_new;
        lt = probs(s2);
      }
      l += lt;
      // O^T += V^T P^T
#pragma unroll
      for (int kb = 0; kb < KB; ++kb)
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
          for (int db = 0; db < D / 32; ++db) o[db] = mma<E>(va[kb][h][db], pk[kb][h], o[db]);
    }
    // (4) tile t+2 complete for this wave (AHEAD-2 newer tiles may still be
    //     in flight), then publish it and release slot t to the next DMA.
    wait_vm_and_barrier<(T::AHEAD - 2) * IPT>();
  };

  // Tiles 0 and 1 complete and visible.
  wait_vm_and_barrier<(T::AHEAD - 2) * IPT>();
  if (ntiles > 0 && active(0)) scores(ic<0>{}, ic<0>{});

  for (int t = 0; t < ntiles; t += T::UNROLL) {
    step(ic<0>{}, ic<0>{}, t);
    if (t + 1 >= ntiles) break;
    step(ic<1>{}, ic<1>{}, t + 1);
    if (t + 2 >= ntiles) break;
    step(ic<2>{}, ic<0>{}, t + 2);
    if (t + 3 >= ntiles) break;
    step(ic<3>{}, ic<1>{}, t + 3);
  }
  // Drain the DMA ring before the work-group's LDS is released.
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");

  // Epilogue: lane (query qrow, half g) holds d = 32*db + 8*(j/4) + 4*g + j%4.
  const float lt = halves_sum(l);
  store_fwd_output<D, E, kSplits>(a, ro, split, head, qrow, g, o, m, lt);
}

// ---------------------------------------------------------------------------
// Software-pipelined forward over 32-key units.
//
// Work-group: NW waves x 32 queries (Q as MFMA B operand), 32-key units (K,
// V rows) streamed through an 8-slot LDS DMA ring, two units per barrier
// step. The body of unit u runs
//   vector work of unit u      P^T = exp2(S^T c - m), its row sums, fp16 P^T
//   matrix work of unit u + 1  S^T = K Q^T
//   matrix work of unit u - 1  O^T += V^T P^T        (V^T via transposing reads)
// P is computed against the current reference max m (see kSumLimit); only
// when a row sum exceeds the limit (rare after the first unit) does a branch
// after the body reduce the tile max, rescale O and l and recompute P of
// unit u against the new max. Causal units whose keys all follow the
// wave's queries use m = +inf (P = 0 exactly); the diagonal and the tail unit
// set their masked S to -inf first. Each work-group rounds its unit count up
// to the 8-unit unroll; padding units are masked the same way.
// ---------------------------------------------------------------------------
// UPS = units per barrier step: 2 (8-slot ring, 64 KiB at D = 64, two
// work-groups per CU) or 1 (6-slot ring, 48 KiB, three work-groups per CU).
// KG = key groups: with KG = 2 the NW waves form two groups of NW/2 that
// serve the same queries, each streaming one half of the work-group's key
// range through a ring of its own with the UPS = 1 pipeline; the two partial
// results are merged through LDS at the end. That halves the longest
// work-group of a causal launch whose end is set by its last query tiles
// (few heads: the tiles reading all keys run alone on the GPU at the end).
template <int D, int NW, int UPS, int KG = 1>
struct FwdPipeTile {
  static constexpr int NWG = NW / KG;  // waves per key group
  static constexpr int BM = 32 * NWG;
  static constexpr int NT = 64 * NW;
  static constexpr int KT = 32;
  static constexpr int TILE = KT * D;  // halves of the K (or V) unit
  static constexpr int STAGE = 2 * TILE;
  static constexpr int NSTAGE = UPS == 2 ? 8 : 6;
  static constexpr int AHEAD = UPS == 2 ? 5 : 4;  // units issued before step 0
  // Work-groups per CU: three 4-wave work-groups with one unit per barrier,
  // two with two; at D = 128 (16 KiB units, a 96 KiB ring) a work-group takes
  // a CU alone; with two key groups (two rings) two at D = 32 and one at D = 64.
  static constexpr int WGS_PER_CU =
      KG == 2 ? (D <= 32 ? 2 : 1) : (NW == 8 || D == 128 ? 1 : (UPS == 2 ? 2 : 3));
  static constexpr int WAVES_PER_SIMD = WGS_PER_CU * NW / 4;
  static_assert(UPS == 1 || UPS == 2, "units per step");
  static_assert(KG == 1 || (KG == 2 && UPS == 1 && NW == 8), "two 4-wave key groups, one unit each");
};

template <int D, int NW, int UPS, int KG = 1>
constexpr bool fwd_pipe_tiling_ok() {
  using T = FwdPipeTile<D, NW, UPS, KG>;
  constexpr int instr = T::TILE * 2 / 1024;
  return (T::TILE * 2) % 1024 == 0 && instr <= T::NWG && T::NWG % instr == 0 &&
         T::WGS_PER_CU * KG * T::NSTAGE * T::STAGE * 2 <= 160 * 1024 &&
         (KG == 1 ? (D <= 64 || NW == 8) : D <= 64);
}

#ifndef FA_FWD_LEAD
#define FA_FWD_LEAD 3
#endif
#ifndef FA_FWD_SKEW
#define FA_FWD_SKEW 1
#endif

template <int V>
using fic = std::integral_constant<int, V>;

// f(integral_constant<int, I>) for I = B .. E-1, fully unrolled.
template <int B, int E, typename F>
__device__ __forceinline__ void fwd_static_for(F&& f) {
  if constexpr (B < E) {
    f(std::integral_constant<int, B>{});
    fwd_static_for<B + 1, E>(f);
  }
}

template <int N, typename F>
__device__ __forceinline__ void static_for_fwd_issue(F&& f) {
  fwd_static_for<0, N>(f);
}

// One job of the pipelined forward: query tile `qtile` of head block
// `head_blk` (the work-group's P = a.pack query heads), keys of split `split`.
// lds_all: the work-group's KG * NSTAGE * STAGE halves of LDS.
template <int D, bool CAUSAL, int NW, int UPS, class E, int KG>
__device__ __forceinline__ void fwd_pipe_body(const FwdArgs& a, int split, int qtile,
                                              int head_blk, half_t* lds_all) {
  using T = FwdPipeTile<D, NW, UPS, KG>;
  using Dma = DmaStager<D, T::KT, T::NWG>;
  static_assert(Dma::PER_WAVE == 1, "one tile piece per wave");
  constexpr int NS = T::NSTAGE;
  constexpr int IPU = 2;  // this wave's DMA instructions per unit: K, V

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave_wg = __builtin_amdgcn_readfirstlane(tid >> 6);
  // Key group of the wave and its place in the group (KG = 1: the work-group).
  const int gk = KG == 1 ? 0 : wave_wg / T::NWG;
  const int wave = wave_wg - gk * T::NWG;
  half_t* const lds = lds_all + gk * (NS * T::STAGE);  // the group's ring
  const int ql = lane & 31;
  const int g = lane >> 5;

  // Packed GQA: the work-group serves P query heads, wave w head w % P.
  const int P = a.pack;
  const int head = head_blk * P + wave % P;  // wave-uniform
  const int b = head / a.Hq;
  const int hq = head - b * a.Hq;
  const int kvh = b * a.Hkv + hq / a.group;
  const int N = a.N;      // queries
  const int Nkv = a.Nkv;  // keys
  const uint32_t slab = (uint32_t)N * D * 2u;
  const uint32_t kv_slab = (uint32_t)Nkv * D * 2u;
  const rsrc_t rq = make_rsrc(a.q + (int64_t)head * N * D, slab);
  const rsrc_t ro = make_rsrc(a.o + (int64_t)head * N * D, slab);
  const int4v r_k = make_rsrc_words(a.k + (int64_t)kvh * Nkv * D, kv_slab);
  const int4v r_v = make_rsrc_words(a.v + (int64_t)kvh * Nkv * D, kv_slab);

  const int bm = T::BM / P;  // query rows per head
  const int q0 = qtile * bm;
  const int q0w = q0 + 32 * (wave / P);
  const int qrow = q0w + ql;

  // Q^T operand fragments: lane (query ql, k-half g), d = 16*kk + 8*g .. +7.
  half8 qf[D / 16];
#pragma unroll
  for (int kk = 0; kk < D / 16; ++kk)
    qf[kk] = __builtin_bit_cast(half8, buf_load_b128(rq, (uint32_t)(qrow * D + 16 * kk + 8 * g) * 2u));
  wait_all_vm();

  const int kv_end = CAUSAL ? min(Nkv, q0 + bm) : Nkv;
  // This work-group's keys: all of [0, kv_end) unless split; with two key
  // groups, the first ceil(units / 2) units go to group 0, the rest to group
  // 1, and both run the same number of steps (group 1's last unit may lie
  // past its keys and then counts as dead).
  const int kv_lo_wg = split * a.split_keys;
  const int kv_hi_wg = min(kv_end, kv_lo_wg + a.split_keys);
  const int n_wg = kv_hi_wg > kv_lo_wg ? (kv_hi_wg - kv_lo_wg + T::KT - 1) / T::KT : 0;
  const int n_grp = (n_wg + KG - 1) / KG;
  const int kv_lo = kv_lo_wg + gk * n_grp * T::KT;
  const int kv_hi = KG == 1 ? kv_hi_wg : min(kv_hi_wg, kv_lo + n_grp * T::KT);
  const int npad = (n_grp + NS - 1) / NS * NS;
  // The group's units end in the ring's last slot: the first ring turn
  // starts at step p0 (slot s0), so no padding unit runs (one at most with
  // two units per step) and the loop over whole turns has no branches.
  const int p0 = __builtin_amdgcn_readfirstlane((npad - n_grp) / UPS);
  const int s0 = UPS * p0;

  Dma dma;
  dma.init(wave, lane);
  const uint32_t lds0 = lds_addr(lds);
  int i_row = kv_lo;  // first key row of the next unit to fetch
  auto issue = [&](int slot) __attribute__((always_inline)) {
    const int row0 = i_row < kv_hi ? i_row : Nkv;  // past the range: zeros
    const uint32_t vt = (uint32_t)row0 * (D * 2u) + dma.voff[0];
    const uint32_t base = lds0 + (uint32_t)slot * (T::STAGE * 2u) + (uint32_t)dma.piece0 * 1024u;
    uint32_t saved;
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
    i_row += T::KT;
  };
#pragma unroll
  for (int u = 0; u < T::AHEAD; ++u) issue(s0 + u < NS ? s0 + u : s0 + u - NS);

  // The V tile read as "unit -1" holds zeros (its P is zero too).
  {
    half_t* zs = lds + (s0 > 0 ? s0 - 1 : NS - 1) * T::STAGE + T::TILE;
    // The zero comes from an asm move, so the persistent form's job loop
    // cannot hoist it and keep (or spill) it across the jobs.
    unsigned zr;
    asm volatile("v_mov_b32 %0, 0" : "=v"(zr));
    const u32x4 z = {zr, zr, zr, zr};
    for (int i = tid - gk * 64 * T::NWG; i < T::TILE / 8; i += 64 * T::NWG)
      *reinterpret_cast<u32x4*>(zs + 8 * i) = z;
  }
  // Units 0 .. AHEAD-3 landed (the last two in flight), zeros written.
  asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" : : "n"(2 * IPU) : "memory");

  int k_off[D / 16];  // row reads of K: row row_perm(ql), chunk 2*kk + g
#pragma unroll
  for (int kk = 0; kk < D / 16; ++kk) k_off[kk] = swz_offset<D>(row_perm(ql), 2 * kk + g);
  int v_off[D / 32][2];  // transposed reads of V (see read_tr)
  {
    const int grp = lane >> 4, i = lane & 15, r = i >> 2, qq = i & 3;
#pragma unroll
    for (int db = 0; db < D / 32; ++db) {
      const int col = 32 * db + 16 * (grp & 1) + 4 * qq;
#pragma unroll
      for (int h2 = 0; h2 < 2; ++h2) {
        const int row = 8 * g + r + 4 * h2;
        v_off[db][h2] = row * D + 8 * swz_chunk<D>(row, col >> 3) + (col & 7);
      }
    }
  }
  auto tr8 = [&](const half_t* base, int db) {
    const half4 lo = __builtin_bit_cast(
        half4, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_short4*)(base + v_off[db][0])));
    const half4 hi = __builtin_bit_cast(
        half4, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_short4*)(base + v_off[db][1])));
    half8 v;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      v[e] = lo[e];
      v[4 + e] = hi[e];
    }
    return v;
  };

  float16v o[D / 32];
#pragma unroll
  for (int db = 0; db < D / 32; ++db)
#pragma unroll
    for (int j = 0; j < 16; ++j) o[db][j] = 0.f;
  float m = -INFINITY;  // reference max (scaled, log2 units); may lag the true max by <= 8
  float l = 0.f;        // this lane's partial sum of exp2(s*c - m) (its half of each unit's keys)
  const float c = a.c;
  const float inf = __builtin_inff();

  // Pipeline registers: S^T of the current unit, P^T of the previous one.
  float16v s_cur;
#pragma unroll
  for (int j = 0; j < 16; ++j) s_cur[j] = 0.f;
#pragma unroll
  for (int kk = 0; kk < D / 16; ++kk)
    s_cur = mma<E>(*reinterpret_cast<const half8*>(lds + s0 * T::STAGE + k_off[kk]), qf[kk], s_cur);
  half8 pa_prev[2];
#pragma unroll
  for (int h = 0; h < 2; ++h)
#pragma unroll
    for (int e = 0; e < 8; ++e) pa_prev[h][e] = (half_t)0.f;

  auto pv = [&](const half_t* slot) __attribute__((always_inline)) {
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int db = 0; db < D / 32; ++db)
        o[db] = mma<E>(tr8(slot + T::TILE + 16 * h * D, db), pa_prev[h], o[db]);
  };

  int c_key = kv_lo;  // first key of the unit the body works on

  auto body = [&](auto slot_c) __attribute__((always_inline)) {
    constexpr int SLOT = decltype(slot_c)::value;
    const half_t* nxt = lds + ((SLOT + 1) % NS) * T::STAGE;
    const half_t* prv = lds + ((SLOT + NS - 1) % NS) * T::STAGE;
    const int ka = c_key;
    c_key += T::KT;

    // Unit modes (wave-uniform): keys all past the queries (or past N), or
    // a diagonal / tail unit whose masked scores become -inf.
    const bool dead = (CAUSAL && ka > q0w) || ka >= kv_hi;
    float m_eff = dead ? inf : m;
    if (!dead && ((CAUSAL && ka == q0w) || ka + T::KT > kv_hi)) {
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        const int key = ka + result_row(j, g);
        if (key >= kv_hi || (CAUSAL && key > qrow)) s_cur[j] = -inf;
      }
    }

    // Hand-ordered body: D/16 S tasks (unit u+1) and D/16 O tasks (unit
    // u-1), alternating; group i issues the LDS reads of task i + kLead,
    // runs task i and part of unit u's vector work; fences keep the order.
    constexpr int NQ = D / 16;
    constexpr int NTASK = 2 * NQ;
    constexpr int kLead = FA_FWD_LEAD;
    auto load_op = [&](auto t_c) -> half8 {
      constexpr int t = decltype(t_c)::value;
      constexpr int q = t / 2;
      constexpr int h = q / (D / 32), db = q % (D / 32);
      if constexpr (t % 2 == 0) return *reinterpret_cast<const half8*>(nxt + k_off[q]);
      else return tr8(prv + T::TILE + 16 * h * D, db);
    };
    float16v s_nx;
#pragma unroll
    for (int j = 0; j < 16; ++j) s_nx[j] = 0.f;
    auto run_task = [&](auto t_c, const half8& op) {
      constexpr int t = decltype(t_c)::value;
      constexpr int q = t / 2;
      constexpr int h = q / (D / 32), db = q % (D / 32);
      if constexpr (t % 2 == 0) s_nx = mma<E>(op, qf[q], s_nx);
      else o[db] = mma<E>(op, pa_prev[h], o[db]);
    };
    half8 pa[2];
    float pexp[16];
    float targ[16];  // s c - m of the pairs whose exp runs in the next group
    float lsum[2];   // set by the first pair
    // Vector work on value pairs in stages placed in different groups:
    //   F: s c - m   A: p = exp2(F)   B: row sums, fp16 P^T.
    // With FA_FWD_SKEW the F stage of a pair runs one group before its A
    // stage, so no exp waits on the fma just issued.
    auto stage_f = [&](int pr) {
#pragma unroll
      for (int e = 0; e < 2; ++e) targ[2 * pr + e] = fmaf(s_cur[2 * pr + e], c, -m_eff);
      asm volatile("" : "+v"(targ[2 * pr]), "+v"(targ[2 * pr + 1]));
    };
    auto stage_a = [&](int pr) {
      float p2[2];
      if constexpr (FA_FWD_SKEW) {
#pragma unroll
        for (int e = 0; e < 2; ++e) p2[e] = exp2_fast(targ[2 * pr + e]);
      } else {
#pragma unroll
        for (int e = 0; e < 2; ++e) p2[e] = exp2_fast(fmaf(s_cur[2 * pr + e], c, -m_eff));
      }
      asm volatile("" : "+v"(p2[0]), "+v"(p2[1]));
      pexp[2 * pr] = p2[0];
      pexp[2 * pr + 1] = p2[1];
    };
    auto stage_b = [&](int pr) {
      half2v pp;
#pragma unroll
      for (int e = 0; e < 2; ++e) {
        lsum[e] = pr == 0 ? pexp[e] : lsum[e] + pexp[2 * pr + e];
        pp[e] = to_elem<E>(pexp[2 * pr + e]);
      }
      asm volatile("" : "+v"(pp));
      const int j = 2 * pr;
      pa[j >> 3][j & 7] = pp[0];
      pa[j >> 3][(j & 7) + 1] = pp[1];
    };

    half8 op[NTASK];
    __builtin_amdgcn_sched_barrier(0);
    asm volatile("" : "+v"(m_eff));
    fwd_static_for<0, (kLead < NTASK ? kLead : NTASK)>(
        [&](auto t_c) { op[decltype(t_c)::value] = load_op(t_c); });
    if constexpr (FA_FWD_SKEW) {
#pragma unroll
      for (int pr = 0; pr < 8; ++pr)
        if ((2 * pr * NTASK) / 16 == 0) stage_f(pr);
    }
    __builtin_amdgcn_sched_barrier(0);
    fwd_static_for<0, NTASK>([&](auto i_c) {
      constexpr int i = decltype(i_c)::value;
      if constexpr (i + kLead < NTASK) op[i + kLead] = load_op(fic<i + kLead>{});
      run_task(i_c, op[i]);
#pragma unroll
      for (int pr = 0; pr < 8; ++pr) {
        const int ga = (2 * pr * NTASK) / 16;
        const int gb = ga + 1 < NTASK ? ga + 1 : NTASK - 1;
        if (ga == i) stage_a(pr);
        if (gb == i) stage_b(pr);
      }
      if constexpr (FA_FWD_SKEW) {
#pragma unroll
        for (int pr = 0; pr < 8; ++pr)
          if ((2 * pr * NTASK) / 16 == i + 1) stage_f(pr);
      }
      __builtin_amdgcn_sched_barrier(0);
    });

    // Row sum of unit u; a rare branch moves the reference max.
    float l_u = lsum[0] + lsum[1];
    if (!dead && __builtin_amdgcn_ballot_w64(!(l_u <= kSumLimit)) != 0) {
      float mt = s_cur[0];
#pragma unroll
      for (int j = 1; j < 16; ++j) mt = __builtin_fmaxf(mt, s_cur[j]);
      mt = halves_max(mt) * c;
      const float m_new = __builtin_fmaxf(m, mt);
      const float alpha = exp2_fast(m - m_new);
      l *= alpha;
#pragma unroll
      for (int db = 0; db < D / 32; ++db) o[db] *= alpha;
      m = m_new;
      l_u = 0.f;
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        const float p = exp2_fast(fmaf(s_cur[j], c, -m));
        l_u += p;
        pa[j >> 3][j & 7] = to_elem<E>(p);
      }
    }
    l += l_u;

    s_cur = s_nx;
#pragma unroll
    for (int h = 0; h < 2; ++h) pa_prev[h] = pa[h];
  };

  // One barrier step: UPS units; issues the units AHEAD.. ahead into the
  // slots of units finished before the last barrier, then waits for all but
  // the two most recent units (the next step reads up to 2 units ahead).
  auto step = [&](auto p_c) __attribute__((always_inline)) {
    constexpr int P = decltype(p_c)::value;
    static_for_fwd_issue<UPS>([&](auto e_c) {
      issue((UPS * P + T::AHEAD + decltype(e_c)::value) % NS);
    });
    static_for_fwd_issue<UPS>([&](auto e_c) { body(fic<UPS * P + decltype(e_c)::value>{}); });
    wait_vm_and_barrier<2 * IPU>();
  };

  static_assert(NS % UPS == 0, "whole steps per ring turn");
  if (npad > 0) {
    // first turn from step p0 (the branches run once), then whole turns
    fwd_static_for<0, NS / UPS>([&](auto p_c) {
      if (decltype(p_c)::value >= p0) step(p_c);
    });
    for (int u = NS; u < npad; u += NS) {
      fwd_static_for<0, NS / UPS>([&](auto p_c) { step(p_c); });
    }
  }
  pv(lds + (NS - 1) * T::STAGE);  // O of the last unit (the ring's last slot)
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");

  if constexpr (KG == 2) {
    // Group 1 hands its O, m and l (per lane) to the group-0 wave serving the
    // same queries through LDS (the rings are drained), [wave][value][lane].
    constexpr int F = D / 32 * 16 + 2;
    __syncthreads();
    float* const xs = reinterpret_cast<float*>(lds_all) + wave * F * 64 + lane;
    if (gk == 1) {
#pragma unroll
      for (int db = 0; db < D / 32; ++db)
#pragma unroll
        for (int j = 0; j < 16; ++j) xs[(16 * db + j) * 64] = o[db][j];
      xs[(F - 2) * 64] = m;
      xs[(F - 1) * 64] = l;
    }
    __syncthreads();
    if (gk == 1) return;
    // O = O0 w0 + O1 w1, l = l0 w0 + l1 w1 against the larger reference max
    // (a group that saw no key has m = -inf, l = 0 and weighs 0).
    const float m1 = xs[(F - 2) * 64];
    const float l1 = xs[(F - 1) * 64];
    const float mt = __builtin_fmaxf(m, m1);
    const float w0 = m == -inf ? 0.f : exp2_fast(m - mt);
    const float w1 = m1 == -inf ? 0.f : exp2_fast(m1 - mt);
#pragma unroll
    for (int db = 0; db < D / 32; ++db)
#pragma unroll
      for (int j = 0; j < 16; ++j) o[db][j] = o[db][j] * w0 + xs[(16 * db + j) * 64] * w1;
    l = l * w0 + l1 * w1;
    m = mt;
  }

  // Epilogue: lane (query qrow, half g) holds d = 32*db + 8*(j/4) + 4*g + j%4.
  const float lt = halves_sum(l);
  store_fwd_output<D, E>(a, ro, split, head, qrow, g, o, m, lt);
}

// --------------------------------------------------------------------------
// The pipelined forward of tiling 6 (4 waves, 32-key units, one unit per
// barrier, a 6-slot ring, three work-groups per CU at D <= 64) on 16x16x32
// MFMAs, with QB 16-row query blocks per wave: QB = 2 is tiling 6's
// 32 queries per wave (tiling 10), QB = 1 halves the work-group to 64
// queries (tiling 11: twice the work-groups and half the work per unit, for
// launches too small to fill the GPU, whose time is their longest key loop,
// and for decoding; at D = 128 too, with two DMA pieces per wave and a 96 KiB
// ring, one work-group per CU).
// Each 32-key unit against a query block is two 16 x 16 score blocks (key
// block kb); each K row read and each transposed V read from LDS feeds QB
// MFMAs, so with QB = 2 LDS traffic, vector work and FLOP are tiling 6's.
// Layouts (lane l, c16 = l % 16, G = l / 16):
//   S^T block (kb, qb): lane holds query 16 qb + c16 of the wave and keys
//     16 kb + 4 gq + j (j = 0..3) of the unit (gq = quad16(G));
//   O^T block (dd, qb): lane holds query 16 qb + c16, d = 16 dd + 4 G + j.
// A lane holds QB queries, so the running max m and the row sums are kept
// per query block, over the lane's 8 keys of each unit; the four lanes
// l, l ^ 16, l ^ 32, l ^ 48 hold one query's keys, share its m (the rare
// max update reduces over them) and add their sums at the end.
// O^T += V^T P^T: k-slot 8 G + 4 kb + j is key 16 kb + 4 gq + j, so the
// lane's P values of blocks (0, qb), (1, qb) are the B operand as they stand.
// --------------------------------------------------------------------------
template <int D, bool CAUSAL, class E, int QB>
__device__ __forceinline__ void fwd_pipe16_body(const FwdArgs& a, int split, int qtile,
                                                int head_blk, half_t* lds) {
  constexpr int NW = 4;
  using T = FwdPipeTile<D, NW, 1, 1>;
  using Dma = DmaStager<D, T::KT, NW>;
  static_assert(Dma::PER_WAVE == 1 || Dma::PER_WAVE == 2, "one or two tile pieces per wave");
  static_assert(D == 32 || D == 64 || (D == 128 && QB == 1),
                "16x16x32 forward: D <= 64, and D = 128 with one query block per wave");
  static_assert(QB == 1 || QB == 2, "one or two 16-row query blocks per wave");
  static_assert(T::WGS_PER_CU * T::NSTAGE * T::STAGE * 2 <= 160 * 1024, "ring fits the LDS");
  constexpr int BM = 4 * 16 * QB;  // query rows per work-group
  constexpr int NPAIR = 4 * QB;    // score value pairs per lane and unit
  constexpr int NS = T::NSTAGE;
  constexpr int IPU = 2 * Dma::PER_WAVE;  // this wave's DMA instructions per unit: K, V
  constexpr int KD = D / 32;  // 32-wide d chunks: k-steps of S^T
  constexpr int DD = D / 16;  // 16-row d blocks of O^T

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int c16 = lane & 15;
  const int G = lane >> 4;
  const int sg = (4 - G) & 3;   // d chunk order of the k-slots (conflict-free row reads)
  const int gq = quad16<D>(G);  // key quad (of 16) of the lane's result rows

  // Packed GQA: the work-group serves P query heads, wave w head w % P.
  const int P = a.pack;
  const int head = head_blk * P + wave % P;  // wave-uniform
  const int b = head / a.Hq;
  const int hq = head - b * a.Hq;
  const int kvh = b * a.Hkv + hq / a.group;
  const int N = a.N;      // queries
  const int Nkv = a.Nkv;  // keys
  const uint32_t slab = (uint32_t)N * D * 2u;
  const uint32_t kv_slab = (uint32_t)Nkv * D * 2u;
  const rsrc_t rq = make_rsrc(a.q + (int64_t)head * N * D, slab);
  const rsrc_t ro = make_rsrc(a.o + (int64_t)head * N * D, slab);
  const int4v r_k = make_rsrc_words(a.k + (int64_t)kvh * Nkv * D, kv_slab);
  const int4v r_v = make_rsrc_words(a.v + (int64_t)kvh * Nkv * D, kv_slab);

  const int bm = BM / P;  // query rows per head
  const int q0 = qtile * bm;
  const int q0w = q0 + 16 * QB * (wave / P);
  const int qrow0 = q0w + c16;  // query of block qb: qrow0 + 16 qb

  // Q^T operand fragments: column = query 16 qb + c16, d = 32 kd + 8 sg .. +7.
  half8 qf[QB][KD];
#pragma unroll
  for (int qb = 0; qb < QB; ++qb)
#pragma unroll
    for (int kd = 0; kd < KD; ++kd)
      qf[qb][kd] = __builtin_bit_cast(
          half8, buf_load_b128(rq, (uint32_t)((qrow0 + 16 * qb) * D + 32 * kd + 8 * sg) * 2u));
  wait_all_vm();

  const int kv_end = CAUSAL ? min(Nkv, q0 + bm) : Nkv;
  const int kv_lo = split * a.split_keys;
  const int kv_hi = min(kv_end, kv_lo + a.split_keys);
  const int n_units = kv_hi > kv_lo ? (kv_hi - kv_lo + T::KT - 1) / T::KT : 0;
  const int npad = (n_units + NS - 1) / NS * NS;
  // Rotated ring start, as in fwd_pipe_body: the units end in the ring's last slot.
  const int p0 = __builtin_amdgcn_readfirstlane(npad - n_units);
  const int s0 = p0;

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
      // D = 128: the wave's two consecutive 1 KiB pieces of the K and the V unit
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

  // The V tile read as "unit -1" holds zeros (its P is zero too).
  {
    half_t* zs = lds + (s0 > 0 ? s0 - 1 : NS - 1) * T::STAGE + T::TILE;
    unsigned zr;
    asm volatile("v_mov_b32 %0, 0" : "=v"(zr));
    const u32x4 z = {zr, zr, zr, zr};
    for (int i = tid; i < T::TILE / 8; i += T::NT) *reinterpret_cast<u32x4*>(zs + 8 * i) = z;
  }
  asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" : : "n"(2 * IPU) : "memory");

  // Row reads of K (A operand of S^T): key row 16 kb + rows16(c16), chunk 4 kd + sg.
  int k_off[2][KD];
#pragma unroll
  for (int kb = 0; kb < 2; ++kb)
#pragma unroll
    for (int kd = 0; kd < KD; ++kd)
      k_off[kb][kd] = swz_offset<D>(16 * kb + rows16<D>(c16), 4 * kd + sg);
  // Transposing reads of V (A operand of O^T += V^T P^T): in 16-lane group G,
  // source lane i addresses key row 16 h + 4 gq + i / 4, columns
  // 16 dd + 4 (i % 4) .. +3; lane i receives keys 16 h + 4 gq + 0..3 of
  // column (d) 16 dd + i.
  int v_off[DD][2];
#pragma unroll
  for (int dd = 0; dd < DD; ++dd)
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int row = 16 * h + 4 * gq + (c16 >> 2);
      const int col = 16 * dd + 4 * (c16 & 3);
      v_off[dd][h] = row * D + 8 * swz_chunk<D>(row, col >> 3) + (col & 7);
    }
  auto trv = [&](const half_t* base, int dd) {
    const half4 lo = __builtin_bit_cast(
        half4, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_short4*)(base + v_off[dd][0])));
    const half4 hi = __builtin_bit_cast(
        half4, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_short4*)(base + v_off[dd][1])));
    half8 v;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      v[e] = lo[e];
      v[4 + e] = hi[e];
    }
    return v;
  };

  float4v o[DD][QB];
#pragma unroll
  for (int dd = 0; dd < DD; ++dd)
#pragma unroll
    for (int qb = 0; qb < QB; ++qb)
#pragma unroll
      for (int j = 0; j < 4; ++j) o[dd][qb][j] = 0.f;
  float m[QB], l[QB];  // reference max per query block (scaled, log2 units); this
                       // lane's partial sums of exp2(s c - m)
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
    m[qb] = -INFINITY;
    l[qb] = 0.f;
  }
  const float c = a.c;
  const float inf = __builtin_inff();

  // Pipeline registers: S^T of the current unit ([kb][qb]), P^T of the previous
  // one (B operands, [qb]).
  float4v s_cur[2][QB];
#pragma unroll
  for (int kb = 0; kb < 2; ++kb)
#pragma unroll
    for (int qb = 0; qb < QB; ++qb)
#pragma unroll
      for (int j = 0; j < 4; ++j) s_cur[kb][qb][j] = 0.f;
#pragma unroll
  for (int kb = 0; kb < 2; ++kb)
#pragma unroll
    for (int kd = 0; kd < KD; ++kd) {
      const half8 ok = *reinterpret_cast<const half8*>(lds + s0 * T::STAGE + k_off[kb][kd]);
#pragma unroll
      for (int qb = 0; qb < QB; ++qb) s_cur[kb][qb] = mma16<E>(ok, qf[qb][kd], s_cur[kb][qb]);
    }
  half8 pa_prev[QB];
#pragma unroll
  for (int qb = 0; qb < QB; ++qb)
#pragma unroll
    for (int e = 0; e < 8; ++e) pa_prev[qb][e] = (half_t)0.f;

  int c_key = kv_lo;  // first key of the unit the body works on

  auto body = [&](auto slot_c) __attribute__((always_inline)) {
    constexpr int SLOT = decltype(slot_c)::value;
    const half_t* nxt = lds + ((SLOT + 1) % NS) * T::STAGE;
    const half_t* prv = lds + ((SLOT + NS - 1) % NS) * T::STAGE;
    const int ka = c_key;
    c_key += T::KT;

    // Unit modes (wave-uniform): keys all past the queries (or past N_kv), or
    // a diagonal / tail unit whose masked scores become -inf. Units start at
    // multiples of 32 keys and the wave's queries at a multiple of 16 QB, so
    // a live unit holds a key past a query exactly when ka + 32 > q0w.
    const bool dead = (CAUSAL && ka > q0w) || ka >= kv_hi;
    float m_eff[QB];
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) m_eff[qb] = dead ? inf : m[qb];
    if (!dead && ((CAUSAL && ka + T::KT > q0w) || ka + T::KT > kv_hi)) {
#pragma unroll
      for (int kb = 0; kb < 2; ++kb)
#pragma unroll
        for (int qb = 0; qb < QB; ++qb)
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const int key = ka + 16 * kb + 4 * gq + j;
            if (key >= kv_hi || (CAUSAL && key > qrow0 + 16 * qb)) s_cur[kb][qb][j] = -inf;
          }
    }

    // Hand-ordered body: D/16 S^T tasks (unit u+1) and D/16 O^T tasks (unit
    // u-1), alternating, each one LDS operand and two MFMAs; group i issues
    // the LDS reads of task i + kLead, runs task i and part of unit u's
    // vector work (as in fwd_pipe_body).
    constexpr int NQ = D / 16;
    constexpr int NTASK = 2 * NQ;
    constexpr int kLead = FA_FWD_LEAD;
    auto load_op = [&](auto t_c) -> half8 {
      constexpr int t = decltype(t_c)::value;
      constexpr int q = t / 2;
      constexpr int kb = q / KD, kd = q % KD;
      if constexpr (t % 2 == 0) return *reinterpret_cast<const half8*>(nxt + k_off[kb][kd]);
      else return trv(prv + T::TILE, q);
    };
    float4v s_nx[2][QB];
#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int qb = 0; qb < QB; ++qb)
#pragma unroll
        for (int j = 0; j < 4; ++j) s_nx[kb][qb][j] = 0.f;
    auto run_task = [&](auto t_c, const half8& op) {
      constexpr int t = decltype(t_c)::value;
      constexpr int q = t / 2;
      constexpr int kb = q / KD, kd = q % KD;
#pragma unroll
      for (int qb = 0; qb < QB; ++qb) {
        if constexpr (t % 2 == 0) s_nx[kb][qb] = mma16<E>(op, qf[qb][kd], s_nx[kb][qb]);
        else o[q][qb] = mma16<E>(op, pa_prev[qb], o[q][qb]);
      }
    };
    half8 pa[QB];
    float pexp[2 * NPAIR];
    float targ[2 * NPAIR];  // s c - m of the pairs whose exp runs in the next group
    float lsum[QB][2];      // per query block, set by its first pair
    // Vector work on value pairs (v = 2 pr, 2 pr + 1: block kb = pr / (2 QB),
    // qb = pr / 2 % QB, j = 2 (pr % 2) + e) in stages placed in different
    // groups:  F: s c - m   A: p = exp2(F)   B: row sums, fp16 P^T.
    auto stage_f = [&](int pr) {
      const int kb = pr / (2 * QB), qb = (pr >> 1) % QB, j0 = 2 * (pr & 1);
#pragma unroll
      for (int e = 0; e < 2; ++e) targ[2 * pr + e] = fmaf(s_cur[kb][qb][j0 + e], c, -m_eff[qb]);
      asm volatile("" : "+v"(targ[2 * pr]), "+v"(targ[2 * pr + 1]));
    };
    auto stage_a = [&](int pr) {
      float p2[2];
#pragma unroll
      for (int e = 0; e < 2; ++e) p2[e] = exp2_fast(targ[2 * pr + e]);
      asm volatile("" : "+v"(p2[0]), "+v"(p2[1]));
      pexp[2 * pr] = p2[0];
      pexp[2 * pr + 1] = p2[1];
    };
    auto stage_b = [&](int pr) {
      const int kb = pr / (2 * QB), qb = (pr >> 1) % QB, j0 = 2 * (pr & 1);
      const bool first = kb == 0 && (pr & 1) == 0;  // the block's first pair
      half2v pp;
#pragma unroll
      for (int e = 0; e < 2; ++e) {
        lsum[qb][e] = first ? pexp[2 * pr + e] : lsum[qb][e] + pexp[2 * pr + e];
        pp[e] = to_elem<E>(pexp[2 * pr + e]);
      }
      asm volatile("" : "+v"(pp));
      pa[qb][4 * kb + j0] = pp[0];
      pa[qb][4 * kb + j0 + 1] = pp[1];
    };

    half8 op[NTASK];
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) asm volatile("" : "+v"(m_eff[qb]));
    fwd_static_for<0, (kLead < NTASK ? kLead : NTASK)>(
        [&](auto t_c) { op[decltype(t_c)::value] = load_op(t_c); });
#pragma unroll
    for (int pr = 0; pr < NPAIR; ++pr)
      if ((pr * NTASK) / NPAIR == 0) stage_f(pr);
    __builtin_amdgcn_sched_barrier(0);
    fwd_static_for<0, NTASK>([&](auto i_c) {
      constexpr int i = decltype(i_c)::value;
      if constexpr (i + kLead < NTASK) op[i + kLead] = load_op(fic<i + kLead>{});
      run_task(i_c, op[i]);
#pragma unroll
      for (int pr = 0; pr < NPAIR; ++pr) {
        const int ga = (pr * NTASK) / NPAIR;
        const int gb = ga + 1 < NTASK ? ga + 1 : NTASK - 1;
        if (ga == i) stage_a(pr);
        if (gb == i) stage_b(pr);
      }
#pragma unroll
      for (int pr = 0; pr < NPAIR; ++pr)
        if ((pr * NTASK) / NPAIR == i + 1) stage_f(pr);
      __builtin_amdgcn_sched_barrier(0);
    });

    // Row sums of unit u; a rare branch moves the reference maxima (for both
    // query blocks: the branch is wave-uniform).
    float l_u[QB];
    bool over = false;
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) {
      l_u[qb] = lsum[qb][0] + lsum[qb][1];
      over = over || !(l_u[qb] <= kSumLimit);
    }
    if (!dead && __builtin_amdgcn_ballot_w64(over) != 0) {
#pragma unroll
      for (int qb = 0; qb < QB; ++qb) {
        float mt = s_cur[0][qb][0];
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
          for (int j = 0; j < 4; ++j) mt = __builtin_fmaxf(mt, s_cur[kb][qb][j]);
        mt = quarters_max(mt) * c;
        const float m_new = __builtin_fmaxf(m[qb], mt);
        const float alpha = exp2_fast(m[qb] - m_new);
        l[qb] *= alpha;
#pragma unroll
        for (int dd = 0; dd < DD; ++dd) o[dd][qb] *= alpha;
        m[qb] = m_new;
        l_u[qb] = 0.f;
#pragma unroll
        for (int kb = 0; kb < 2; ++kb)
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const float p = exp2_fast(fmaf(s_cur[kb][qb][j], c, -m[qb]));
            l_u[qb] += p;
            pa[qb][4 * kb + j] = to_elem<E>(p);
          }
      }
    }
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) l[qb] += l_u[qb];

#pragma unroll
    for (int kb = 0; kb < 2; ++kb)
#pragma unroll
      for (int qb = 0; qb < QB; ++qb) s_cur[kb][qb] = s_nx[kb][qb];
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) pa_prev[qb] = pa[qb];
  };

  // One barrier step per unit (tiling 6's pipeline): issue the unit AHEAD
  // ahead into the slot of the unit finished before the last barrier, run the
  // body, wait for all but the two most recent units.
  auto step = [&](auto p_c) __attribute__((always_inline)) {
    constexpr int Pp = decltype(p_c)::value;
    issue((Pp + T::AHEAD) % NS);
    body(fic<Pp>{});
    wait_vm_and_barrier<2 * IPU>();
  };
  if (npad > 0) {
    fwd_static_for<0, NS>([&](auto p_c) {
      if (decltype(p_c)::value >= p0) step(p_c);
    });
    for (int u = NS; u < npad; u += NS) fwd_static_for<0, NS>([&](auto p_c) { step(p_c); });
  }
  // O of the last unit (the ring's last slot).
#pragma unroll
  for (int dd = 0; dd < DD; ++dd) {
    const half8 op = trv(lds + (NS - 1) * T::STAGE + T::TILE, dd);
#pragma unroll
    for (int qb = 0; qb < QB; ++qb) o[dd][qb] = mma16<E>(op, pa_prev[qb], o[dd][qb]);
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");

  // Epilogue: the four lanes of a query add their sums; lane holds
  // d = 16 dd + 4 G + j of query 16 qb + c16.
  const bool split_mode = a.nsplit > 1;
#pragma unroll
  for (int qb = 0; qb < QB; ++qb) {
    const float lt = quarters_sum(l[qb]);
    const bool seen = lt > 0.f;
    const float inv = seen ? 1.0f / lt : 0.f;
    const int qrow = qrow0 + 16 * qb;
    const bool row_ok = qrow < N;
    const int64_t prow = ((int64_t)split * a.BH + head) * N + qrow;
    float* po = split_mode ? a.part + prow * D : nullptr;  // part is null in one-pass mode
#pragma unroll
    for (int dd = 0; dd < DD; ++dd) {
      float4v v;
#pragma unroll
      for (int e = 0; e < 4; ++e) v[e] = o[dd][qb][e] * inv;
      if (split_mode) {
        if (row_ok) *reinterpret_cast<float4v*>(po + 16 * dd + 4 * G) = v;
      } else {
        buf_store_b64(ro, (uint32_t)(qrow * D + 16 * dd + 4 * G) * 2u,
                      pack4<E>(v[0], v[1], v[2], v[3]));
      }
    }
    if (G == 0 && row_ok) {
      const float lse = seen ? m[qb] + log2_fast(lt) : -INFINITY;
      if (split_mode) a.part[(int64_t)a.nsplit * a.BH * N * D + prow] = lse;
      else a.lse[(int64_t)head * N + qrow] = lse;
    }
  }
}

// The grid form: one job per work-group, tile-major / head-minor (heaviest
// causal tiles first), the split index slowest.
template <int D, bool CAUSAL, int NW, int UPS, class E = F16, int KG = 1>
__global__ __launch_bounds__(64 * NW)
__attribute__((amdgpu_waves_per_eu(FwdPipeTile<D, NW, UPS, KG>::WAVES_PER_SIMD)))
void fwd_pipe_kernel(FwdArgs a) {
  using T = FwdPipeTile<D, NW, UPS, KG>;
  __shared__ __attribute__((aligned(16))) half_t lds_all[KG * T::NSTAGE * T::STAGE];
  const int row_wgs = a.BH / a.pack;  // work-groups per tile row
  const int split = blockIdx.x / (a.num_tiles * row_wgs);
  const TileHead th = decode_block_grouped(blockIdx.x - split * a.num_tiles * row_wgs, row_wgs,
                                           a.group / a.pack);
  const int qtile = CAUSAL ? (a.num_tiles - 1 - th.tile_rank) : th.tile_rank;
  fwd_pipe_body<D, CAUSAL, NW, UPS, E, KG>(a, split, qtile, th.head, lds_all);
}

// The persistent form (causal, one pass, one head per work-group): one
// work-group per slot of the plan, running the jobs of its bin in order.
// Slot s serves head group s % ngroups and bin s / ngroups; job (hoff, qtile)
// of that bin is query tile qtile of head position ngroups * hoff + group,
// mapped to a head as the grid form maps tile-row positions (so with the
// same XCD for all of a key/value head's query heads when ngroups is a
// multiple of 8). The LDS ring is reused from job to job: a barrier between
// jobs keeps the next job's first DMA from overwriting tiles a slower wave
// still reads.
template <int D, int NW, class E = F16>
__global__ __launch_bounds__(64 * NW)
__attribute__((amdgpu_waves_per_eu(FwdPipeTile<D, NW, 1, 1>::WAVES_PER_SIMD)))
void fwd_pipe_jobs_kernel(FwdArgs a, FwdJobs jobs) {
  using T = FwdPipeTile<D, NW, 1, 1>;
  __shared__ __attribute__((aligned(16))) half_t lds_all[T::NSTAGE * T::STAGE];
  const int gi = blockIdx.x % jobs.ngroups;
  const int bin = blockIdx.x / jobs.ngroups;
  const int j0 = jobs.start[bin];
  const int j1 = jobs.start[bin + 1];
  const int bhkv = a.BH / a.group;
  for (int j = j0; j < j1; ++j) {
    const int e = jobs.job[j];
    const int qtile = e & (FwdJobs::kTileLimit - 1);
    const int p = gi + jobs.ngroups * (e / FwdJobs::kTileLimit);
    const int head = (a.group > 1 && bhkv % 8 == 0) ? (p % bhkv) * a.group + p / bhkv : p;
    if (j > j0) __syncthreads();
    fwd_pipe_body<D, true, NW, 1, E, 1>(a, 0, qtile, head, lds_all);
  }
}

template <int D, bool CAUSAL, int NW, int UPS, class E = F16, int KG = 1>
hipError_t fwd_pipe_launch(const FwdArgs& a, hipStream_t stream);

// The plan variants: the persistent form when the host attached a job plan
// (causal, one pass, one head per work-group), else the grid form of the
// same tiling (split-KV and packed GQA included).
template <int D, bool CAUSAL, int NW, class E>
hipError_t fwd_pipe_jobs_launch(const FwdArgs& a, hipStream_t stream) {
  using T = FwdPipeTile<D, NW, 1, 1>;
  if constexpr (!CAUSAL) {
    return fwd_pipe_launch<D, CAUSAL, NW, 1, E, 1>(a, stream);
  } else {
    const FwdJobs* jb = a.jobs;
    if (jb == nullptr) return fwd_pipe_launch<D, CAUSAL, NW, 1, E, 1>(a, stream);
    if (a.pack != 1 || a.nsplit != 1 || jb->ngroups < 1 || jb->nbin < 1 ||
        jb->nbin > FwdJobs::kMaxBins || jb->start[0] != 0 ||
        jb->start[jb->nbin] > FwdJobs::kMaxJobs || a.BH % jb->ngroups != 0)
      return hipErrorInvalidValue;
    FwdArgs b = a;
    b.num_tiles = (a.N + T::BM - 1) / T::BM;
    // Every job must name a query tile and a head of this launch.
    const int per_group = a.BH / jb->ngroups;
    for (int i = 0; i < jb->nbin; ++i)
      if (jb->start[i + 1] < jb->start[i]) return hipErrorInvalidValue;
    for (int j = 0; j < jb->start[jb->nbin]; ++j) {
      const int e = jb->job[j];
      if (e < 0 || (e & (FwdJobs::kTileLimit - 1)) >= b.num_tiles ||
          e / FwdJobs::kTileLimit >= per_group)
        return hipErrorInvalidValue;
    }
    const int64_t blocks = (int64_t)jb->ngroups * jb->nbin;
    if (blocks <= 0 || blocks > 0x7fffffff) return hipErrorInvalidConfiguration;
    hipLaunchKernelGGL((fwd_pipe_jobs_kernel<D, NW, E>), dim3((unsigned)blocks), dim3(T::NT), 0,
                       stream, b, *jb);
    return hipGetLastError();
  }
}

template <int D, bool CAUSAL, int NW, int UPS, class E, int KG>
hipError_t fwd_pipe_launch(const FwdArgs& a, hipStream_t stream) {
  using T = FwdPipeTile<D, NW, UPS, KG>;
  FwdArgs b = a;
  if (b.pack < 1 || NW % b.pack != 0 || a.group % b.pack != 0 || (KG > 1 && b.pack != 1))
    return hipErrorInvalidValue;
  b.num_tiles = (a.N + T::BM / b.pack - 1) / (T::BM / b.pack);
  if (b.nsplit < 1 || (b.nsplit > 1 && b.part == nullptr) || b.split_keys % 128 != 0 ||
      (int64_t)b.nsplit * b.split_keys < visible_kv<CAUSAL>(a))
    return hipErrorInvalidValue;
  const int64_t blocks = (int64_t)b.num_tiles * (a.BH / b.pack) * b.nsplit;
  if (blocks <= 0 || blocks > 0x7fffffff) return hipErrorInvalidConfiguration;
  hipLaunchKernelGGL((fwd_pipe_kernel<D, CAUSAL, NW, UPS, E, KG>), dim3((unsigned)blocks),
                     dim3(T::NT), 0, stream, b);
  return hipGetLastError();
}

// Tiling 6 on 16x16x32 MFMAs (fwd_pipe16_body), grid form; QB query blocks
// of 16 rows per wave (64 QB queries per work-group).
template <int D, bool CAUSAL, class E = F16, int QB = 2>
__global__ __launch_bounds__(256)
__attribute__((amdgpu_waves_per_eu(FwdPipeTile<D, 4, 1, 1>::WAVES_PER_SIMD)))
void fwd_pipe16_kernel(FwdArgs a) {
  using T = FwdPipeTile<D, 4, 1, 1>;
  __shared__ __attribute__((aligned(16))) half_t lds[T::NSTAGE * T::STAGE];
  const int row_wgs = a.BH / a.pack;  // work-groups per tile row
  const int split = blockIdx.x / (a.num_tiles * row_wgs);
  const TileHead th = decode_block_grouped(blockIdx.x - split * a.num_tiles * row_wgs, row_wgs,
                                           a.group / a.pack);
  const int qtile = CAUSAL ? (a.num_tiles - 1 - th.tile_rank) : th.tile_rank;
  fwd_pipe16_body<D, CAUSAL, E, QB>(a, split, qtile, th.head, lds);
}

template <int D, bool CAUSAL, class E, int QB>
hipError_t fwd_pipe16_launch(const FwdArgs& a, hipStream_t stream) {
  using T = FwdPipeTile<D, 4, 1, 1>;
  constexpr int BM = 64 * QB;  // query rows per work-group
  FwdArgs b = a;
  if (b.pack < 1 || 4 % b.pack != 0 || a.group % b.pack != 0) return hipErrorInvalidValue;
  b.num_tiles = (a.N + BM / b.pack - 1) / (BM / b.pack);
  if (b.nsplit < 1 || (b.nsplit > 1 && b.part == nullptr) || b.split_keys % 128 != 0 ||
      (int64_t)b.nsplit * b.split_keys < visible_kv<CAUSAL>(a))
    return hipErrorInvalidValue;
  const int64_t blocks = (int64_t)b.num_tiles * (a.BH / b.pack) * b.nsplit;
  if (blocks <= 0 || blocks > 0x7fffffff) return hipErrorInvalidConfiguration;
  hipLaunchKernelGGL((fwd_pipe16_kernel<D, CAUSAL, E, QB>), dim3((unsigned)blocks), dim3(T::NT),
                     0, stream, b);
  return hipGetLastError();
}

template <int D, bool CAUSAL, int NW, int UPS, class E = F16>
constexpr void* fwd_pipe16_entry() {
  if constexpr (D <= 64 && NW == 4 && UPS == 1 && fwd_pipe_tiling_ok<D, 4, 1>())
    return (void*)&fwd_pipe16_launch<D, CAUSAL, E, 2>;
  else
    return nullptr;
}

// The same with one 16-row query block per wave (64 queries per work-group);
// also at D = 128, where a work-group takes a CU alone (a 96 KiB ring).
template <int D, bool CAUSAL, int NW, int UPS, class E = F16>
constexpr void* fwd_pipe16_half_entry() {
  if constexpr (NW == 4 && UPS == 1 && (D == 128 || fwd_pipe_tiling_ok<D, 4, 1>()))
    return (void*)&fwd_pipe16_launch<D, CAUSAL, E, 1>;
  else
    return nullptr;
}

template <int D, bool CAUSAL, int NW, int UPS, class E = F16>
constexpr void* fwd_pipe_entry() {
  if constexpr (fwd_pipe_tiling_ok<D, NW, UPS>())
    return (void*)&fwd_pipe_launch<D, CAUSAL, NW, UPS, E>;
  else
    return nullptr;
}
// The plan variants (one unit per barrier; grid form without a plan).
template <int D, bool CAUSAL, int NW, int UPS, class E = F16>
constexpr void* fwd_pipe_jobs_entry() {
  if constexpr (fwd_pipe_tiling_ok<D, NW, UPS>() && UPS == 1 && NW == 4 && D <= 64)
    return (void*)&fwd_pipe_jobs_launch<D, CAUSAL, NW, E>;
  else
    return nullptr;
}
// The two-key-group forward (KG = 2).
template <int D, bool CAUSAL, int NW, int UPS, class E = F16>
constexpr void* fwd_pipe_kg_entry() {
  if constexpr (fwd_pipe_tiling_ok<D, NW, UPS, 2>())
    return (void*)&fwd_pipe_launch<D, CAUSAL, NW, UPS, E, 2>;
  else
    return nullptr;
}

template <int D, bool CAUSAL, int NW, int BN, class E = F16>
hipError_t fwd_launch(const FwdArgs& a, hipStream_t stream) {
  using T = FwdTile<D, NW, BN>;
  FwdArgs b = a;
  if (b.pack < 1 || NW % b.pack != 0 || a.group % b.pack != 0) return hipErrorInvalidValue;
  b.num_tiles = (a.N + T::BM / b.pack - 1) / (T::BM / b.pack);
  if (b.nsplit < 1 || (b.nsplit > 1 && (b.part == nullptr || !fwd_tile_splits_kv<BN>())) ||
      b.split_keys % 128 != 0 || (int64_t)b.nsplit * b.split_keys < visible_kv<CAUSAL>(a))
    return hipErrorInvalidValue;
  const int64_t blocks = (int64_t)b.num_tiles * (a.BH / b.pack) * b.nsplit;
  if (blocks <= 0 || blocks > 0x7fffffff) return hipErrorInvalidConfiguration;
  hipLaunchKernelGGL((fwd_kernel<D, CAUSAL, NW, BN, E>), dim3((unsigned)blocks), dim3(T::NT), 0,
                     stream, b);
  return hipGetLastError();
}

// Merge of the split-KV partials: one thread per 4 columns of a query row. All
// of a row's partials (at most kMaxFwdSplitKv) are loaded at once, so the merge
// waits on one round of load latency rather than one per split; the max, the
// weights and the weighted sum then run in split order (the summation order
// is fixed).
template <int D, class E>
__global__ __launch_bounds__(256) void fwd_combine_kernel(const float* __restrict__ part,
                                                          half_t* __restrict__ o,
                                                          float* __restrict__ lse, int64_t rows,
                                                          int nsplit) {
  constexpr int CPR = D / 4;
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= rows * CPR) return;
  const int64_t row = i / CPR;
  const int c = (int)(i - row * CPR);
  const float* plse = part + (int64_t)nsplit * rows * D;
  float ls[kMaxFwdSplitKv];
  float4v v[kMaxFwdSplitKv];
#pragma unroll
  for (int sp = 0; sp < kMaxFwdSplitKv; ++sp) {
    if (sp < nsplit) {
      ls[sp] = plse[(int64_t)sp * rows + row];
      v[sp] = *reinterpret_cast<const float4v*>(part + ((int64_t)sp * rows + row) * D + 4 * c);
    }
  }
  float mx = -INFINITY;
#pragma unroll
  for (int sp = 0; sp < kMaxFwdSplitKv; ++sp)
    if (sp < nsplit) mx = fmaxf(mx, ls[sp]);
  float wsum = 0.f;
  float4v acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int sp = 0; sp < kMaxFwdSplitKv; ++sp) {
    if (sp < nsplit) {
      const float w = ls[sp] == -INFINITY ? 0.f : exp2_fast(ls[sp] - mx);
      wsum += w;
#pragma unroll
      for (int e = 0; e < 4; ++e) acc[e] = fmaf(w, v[sp][e], acc[e]);
    }
  }
  const float inv = 1.0f / wsum;
  half4 h;
#pragma unroll
  for (int e = 0; e < 4; ++e) h[e] = to_elem<E>(acc[e] * inv);
  *reinterpret_cast<half4*>(o + row * D + 4 * c) = h;
  if (c == 0) lse[row] = mx + log2_fast(wsum);
}

template <int D, class E>
hipError_t fwd_combine_launch(const float* part, half_t* o, float* lse, int64_t rows, int nsplit,
                              hipStream_t stream) {
  const int64_t blocks = (rows * (D / 4) + 255) / 256;
  if (nsplit < 2 || nsplit > kMaxFwdSplitKv || blocks <= 0 || blocks > 0x7fffffff)
    return hipErrorInvalidValue;
  hipLaunchKernelGGL((fwd_combine_kernel<D, E>), dim3((unsigned)blocks), dim3(256), 0, stream,
                     part, o, lse, rows, nsplit);
  return hipGetLastError();
}

hipError_t launch_fwd_combine(const float* part, half_t* o, float* lse, int64_t rows, int D,
                              int nsplit, int dtype, hipStream_t stream) {
  const bool bf = dtype == kBF16;
  switch (D) {
    case 32: return bf ? fwd_combine_launch<32, BF16>(part, o, lse, rows, nsplit, stream)
                       : fwd_combine_launch<32, F16>(part, o, lse, rows, nsplit, stream);
    case 64: return bf ? fwd_combine_launch<64, BF16>(part, o, lse, rows, nsplit, stream)
                       : fwd_combine_launch<64, F16>(part, o, lse, rows, nsplit, stream);
    case 128: return bf ? fwd_combine_launch<128, BF16>(part, o, lse, rows, nsplit, stream)
                        : fwd_combine_launch<128, F16>(part, o, lse, rows, nsplit, stream);
    default: return hipErrorInvalidValue;
  }
}

// A tiling is compiled for a head_dim only if its K/V tiles split into whole
// 1 KiB DMA instructions evenly over the waves and the ring fits in LDS.
template <int D, int NW, int BN>
constexpr bool fwd_tiling_ok() {
  return (BN * D * 2) % 1024 == 0 && ((BN * D * 2) / 1024) % NW == 0 &&
         4 * (2 * BN * D) * 2 <= 160 * 1024;  // NSTAGE slots of K + V tiles
}

template <int D, bool CAUSAL, int NW, int BN, class E = F16>
constexpr void* fwd_entry() {
  if constexpr (fwd_tiling_ok<D, NW, BN>())
    return (void*)&fwd_launch<D, CAUSAL, NW, BN, E>;
  else
    return nullptr;
}

// FA_FWD_VARIANT_BF also compiles the tiling for bf16; bf16 is compiled only
// for the tilings the default table uses, to bound the build.
#define FA_FWD_VARIANT(NW, BN)                                        \
  {NW, 32 * NW, BN, {FA_ENTRIES(fwd_entry, F16, NW, BN), FA_NO_ENTRIES}, \
   fwd_tile_splits_kv<BN>() ? kSplitsKv : 0}
#define FA_FWD_VARIANT_BF(NW, BN)                                                          \
  {NW, 32 * NW, BN, {FA_ENTRIES(fwd_entry, F16, NW, BN), FA_ENTRIES(fwd_entry, BF16, NW, BN)}, \
   fwd_tile_splits_kv<BN>() ? kSplitsKv : 0}

static const Variant kFwdVariants[] = {
    FA_FWD_VARIANT(4, 64),
    FA_FWD_VARIANT(8, 64),
    FA_FWD_VARIANT_BF(4, 32),
    FA_FWD_VARIANT(2, 64),
    FA_FWD_VARIANT(4, 128),
    {4, 128, 32, {FA_ENTRIES(fwd_pipe_entry, F16, 4, 2), FA_NO_ENTRIES}, kSplitsKv},
    {4, 128, 32, {FA_ENTRIES(fwd_pipe_entry, F16, 4, 1), FA_ENTRIES(fwd_pipe_entry, BF16, 4, 1)},
     kSplitsKv},
    {8, 256, 32, {FA_ENTRIES(fwd_pipe_entry, F16, 8, 1), FA_ENTRIES(fwd_pipe_entry, BF16, 8, 1)},
     kSplitsKv},
    {8, 128, 32,
     {FA_ENTRIES(fwd_pipe_kg_entry, F16, 8, 1), FA_ENTRIES(fwd_pipe_kg_entry, BF16, 8, 1)},
     kSplitsKv | kKeyGroups},
    // 9: tiling 6 with the persistent job-plan form under the mask (D <= 64;
    // at D = 128 the 8-wave kernel's launches leave no tail to recover)
    {4, 128, 32,
     {FA_ENTRIES(fwd_pipe_jobs_entry, F16, 4, 1), FA_ENTRIES(fwd_pipe_jobs_entry, BF16, 4, 1)},
     kSplitsKv | kJobs, FwdPipeTile<64, 4, 1>::WGS_PER_CU},
    // 10: tiling 6 on 16x16x32 MFMAs (D <= 64)
    {4, 128, 32, {FA_ENTRIES(fwd_pipe16_entry, F16, 4, 1), FA_ENTRIES(fwd_pipe16_entry, BF16, 4, 1)},
     kSplitsKv},
    // 11: tiling 10 with one 16-row query block per wave, 64 queries per work-group
    // (all D; at D = 128 one work-group per CU)
    {4, 64, 32,
     {FA_ENTRIES(fwd_pipe16_half_entry, F16, 4, 1), FA_ENTRIES(fwd_pipe16_half_entry, BF16, 4, 1)},
     kSplitsKv | kFewSplits},
};

const Variant* fwd_variants(int* count) {
  *count = (int)(sizeof(kFwdVariants) / sizeof(kFwdVariants[0]));
  return kFwdVariants;
}

}  // namespace fa
