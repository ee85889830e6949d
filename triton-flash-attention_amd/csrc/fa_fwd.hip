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

// The running max only moves when a tile's max exceeds it by more than this
// (log2 units): p = exp2(s - m) then stays <= 2^8, exact in fp16 and fp32,
// and the O / l rescale is skipped for most tiles.
constexpr float kRescaleThreshold = 8.0f;

template <int V>
using ic = std::integral_constant<int, V>;

template <int D, bool CAUSAL, int NW, int BN>
__global__ __launch_bounds__(64 * NW) void fwd_kernel(FwdArgs a) {
  using T = FwdTile<D, NW, BN>;
  using Dma = DmaStager<D, BN, NW>;
  constexpr int KB = BN / 32;                 // 32-key blocks per tile
  constexpr int IPT = 2 * Dma::PER_WAVE;      // this wave's DMA instructions per tile
  __shared__ __attribute__((aligned(16))) half_t lds[T::NSTAGE * T::STAGE];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform
  const int ql = lane & 31;
  const int g = lane >> 5;

  const TileHead th = decode_block(blockIdx.x, a.BH);
  const int qtile = CAUSAL ? (a.num_tiles - 1 - th.tile_rank) : th.tile_rank;
  const int head = th.head;
  const int b = head / a.Hq;
  const int hq = head - b * a.Hq;
  const int kvh = b * a.Hkv + hq / a.group;
  const int N = a.N;
  const uint32_t slab = (uint32_t)N * D * 2u;
  const rsrc_t rq = make_rsrc(a.q + (int64_t)head * N * D, slab);
  const rsrc_t ro = make_rsrc(a.o + (int64_t)head * N * D, slab);
  const int4v rk = make_rsrc_words(a.k + (int64_t)kvh * N * D, slab);
  const int4v rv = make_rsrc_words(a.v + (int64_t)kvh * N * D, slab);

  const int q0 = qtile * T::BM;
  const int q0w = q0 + 32 * wave;
  const int qrow = q0w + ql;

  const int kv_end = CAUSAL ? min(N, q0 + T::BM) : N;
  const int ntiles = (kv_end + BN - 1) / BN;

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
    dma.issue(rk, t * BN, base, wave);
    dma.issue(rv, t * BN, base + T::TILE, wave);
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
  auto active = [&](int t) { return uniform((q0w < N) && !(CAUSAL && t * BN > q0w + 31)) != 0; };

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
      for (int kk = 0; kk < D / 16; ++kk) sbuf[SB][kb] = mfma32(ka[kb][kk], qf[kk], sbuf[SB][kb]);
    }
  };

  // One key tile: next DMA, next tile's scores, this tile's softmax + P.V.
  auto step = [&](auto slot_c, auto sb_c, int t_in) {
    constexpr int SLOT = decltype(slot_c)::value;
    constexpr int SB = decltype(sb_c)::value;
    const int t = uniform(t_in);
    const int kv0 = t * BN;
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
      const bool need_mask = uniform((CAUSAL && kv0 + BN - 1 > q0w) || (kv0 + BN > N)) != 0;
      if (need_mask) {
#pragma unroll
        for (int kb = 0; kb < KB; ++kb)
#pragma unroll
          for (int j = 0; j < 16; ++j) {
            const int key = kv0 + 32 * kb + result_row(j, g);
            const bool ok = key < N && (!CAUSAL || key <= qrow);
            if (!ok) sc[kb][j] = -INFINITY;
          }
      }
      float mx4[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) mx4[u] = fmaxf(sc[0][4 * u], sc[0][4 * u + 1]);
#pragma unroll
      for (int kb = 0; kb < KB; ++kb)
#pragma unroll
        for (int j = (kb == 0 ? 2 : 0); j < 4; ++j)
#pragma unroll
          for (int u = 0; u < 4; ++u) mx4[u] = fmaxf(mx4[u], sc[kb][4 * u + j]);
      float mx = fmaxf(fmaxf(mx4[0], mx4[1]), fmaxf(mx4[2], mx4[3]));
      mx = halves_max(mx) * c;
      // Move the reference max only when it grew by more than the threshold
      // for some lane of the wave (always on the first active tile).
      if (__builtin_amdgcn_ballot_w64(mx > m + kRescaleThreshold) != 0) {
        const float m_new = fmaxf(m, mx);
        const float alpha = exp2_fast(m - m_new);
        l *= alpha;
#pragma unroll
        for (int db = 0; db < D / 32; ++db) o[db] *= alpha;
        m = m_new;
      }
      const float nm = -m;
      half8 pk[KB][2];
      float ls4[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kb = 0; kb < KB; ++kb)
#pragma unroll
        for (int j = 0; j < 16; ++j) {
          const float p = exp2_fast(fmaf(sc[kb][j], c, nm));
          ls4[j & 3] += p;
          pk[kb][j >> 3][j & 7] = (half_t)p;
        }
      l += (ls4[0] + ls4[1]) + (ls4[2] + ls4[3]);
      // O^T += V^T P^T
#pragma unroll
      for (int kb = 0; kb < KB; ++kb)
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
          for (int db = 0; db < D / 32; ++db) o[db] = mfma32(va[kb][h][db], pk[kb][h], o[db]);
    }
    // (4) tile t+2 complete for this wave (AHEAD-2 newer tiles may still be
    //     in flight), then publish it and release slot t to the next DMA.
    wait_vm_and_barrier<(T::AHEAD - 2) * IPT>();
  };

  // Tiles 0 and 1 complete and visible.
  wait_vm_and_barrier<(T::AHEAD - 2) * IPT>();
  if (active(0)) scores(ic<0>{}, ic<0>{});

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
  const float inv = 1.0f / lt;
#pragma unroll
  for (int db = 0; db < D / 32; ++db)
#pragma unroll
    for (int jq = 0; jq < 4; ++jq) {
      const u32x2 v = pack4_half(o[db][4 * jq] * inv, o[db][4 * jq + 1] * inv,
                                 o[db][4 * jq + 2] * inv, o[db][4 * jq + 3] * inv);
      buf_store_b64(ro, (uint32_t)(qrow * D + 32 * db + 8 * jq + 4 * g) * 2u, v);
    }
  if (g == 0 && qrow < N) a.lse[(int64_t)head * N + qrow] = m + log2_fast(lt);
}

template <int D, bool CAUSAL, int NW, int BN>
hipError_t fwd_launch(const FwdArgs& a, hipStream_t stream) {
  using T = FwdTile<D, NW, BN>;
  FwdArgs b = a;
  b.num_tiles = (a.N + T::BM - 1) / T::BM;
  const int64_t blocks = (int64_t)b.num_tiles * a.BH;
  if (blocks <= 0 || blocks > 0x7fffffff) return hipErrorInvalidConfiguration;
  hipLaunchKernelGGL((fwd_kernel<D, CAUSAL, NW, BN>), dim3((unsigned)blocks), dim3(T::NT), 0,
                     stream, b);
  return hipGetLastError();
}

// A tiling is compiled for a head_dim only if its K/V tiles split into whole
// 1 KiB DMA instructions evenly over the waves and the ring fits in LDS.
template <int D, int NW, int BN>
constexpr bool fwd_tiling_ok() {
  return (BN * D * 2) % 1024 == 0 && ((BN * D * 2) / 1024) % NW == 0 &&
         4 * (2 * BN * D) * 2 <= 160 * 1024;  // NSTAGE slots of K + V tiles
}

template <int D, bool CAUSAL, int NW, int BN>
constexpr void* fwd_entry() {
  if constexpr (fwd_tiling_ok<D, NW, BN>())
    return (void*)&fwd_launch<D, CAUSAL, NW, BN>;
  else
    return nullptr;
}

#define FA_FWD_VARIANT(NW, BN)                                                  \
  {                                                                             \
    NW, 32 * NW, BN,                                                            \
    {                                                                           \
      {fwd_entry<32, false, NW, BN>(), fwd_entry<32, true, NW, BN>()},          \
      {fwd_entry<64, false, NW, BN>(), fwd_entry<64, true, NW, BN>()},          \
      {fwd_entry<128, false, NW, BN>(), fwd_entry<128, true, NW, BN>()},        \
    }                                                                           \
  }

static const Variant kFwdVariants[] = {
    FA_FWD_VARIANT(4, 64),
    FA_FWD_VARIANT(8, 64),
    FA_FWD_VARIANT(4, 32),
    FA_FWD_VARIANT(2, 64),
    FA_FWD_VARIANT(4, 128),
};

const Variant* fwd_variants(int* count) {
  *count = (int)(sizeof(kFwdVariants) / sizeof(kFwdVariants[0]));
  return kFwdVariants;
}

}  // namespace fa
