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
//   * K tiles are staged row-major and V tiles TRANSPOSED in LDS (V^T rows are
//     head-dim rows, keys contiguous), so both MFMAs read 16-byte operands;
//   * S^T = K Q^T on v_mfma_f32_32x32x16_f16: each lane owns ONE query
//     column, so the row max needs one cross-half exchange and the per-row
//     rescale of the accumulator is a per-lane scalar;
//   * the K rows are read through row_perm so the fp16 P^T values a lane
//     holds are exactly the B-operand of O^T += V^T P^T (no shuffles);
//   * tails use the buffer range check (zero fill), masks run only on the
//     diagonal / tail tiles.
#include "fa_common.hpp"
#include "fa_kernels.hpp"

namespace fa {

template <int D, int NW, int BN>
struct FwdTile {
  static constexpr int BM = 32 * NW;    // queries per work-group
  static constexpr int NT = 64 * NW;    // threads
  static constexpr int KS = D + 8;      // K row stride in LDS (halves)
  static constexpr int VS = BN + 8;     // V^T row stride in LDS (halves)
  static constexpr int DC = D / 8;      // 16-byte chunks per row
  static constexpr int K_CHUNKS = BN * DC;
  static constexpr int K_PER_T = (K_CHUNKS + NT - 1) / NT;
  static constexpr int V_UNITS = (BN / 2) * DC;  // (key pair, chunk) units
  static constexpr int V_PER_T = (V_UNITS + NT - 1) / NT;
  static constexpr int LDS_HALVES = BN * KS + D * VS;
  static_assert(BN % 32 == 0, "key tile must be a multiple of 32");
  static_assert(LDS_HALVES * 2 <= 160 * 1024, "LDS budget");
};

template <int D, bool CAUSAL, int NW, int BN>
__global__ __launch_bounds__(64 * NW) void fwd_kernel(FwdArgs a) {
  using T = FwdTile<D, NW, BN>;
  __shared__ __attribute__((aligned(16))) half_t lds[T::LDS_HALVES];
  half_t* Ks = lds;
  half_t* Vt = lds + BN * T::KS;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
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
  const rsrc_t rk = make_rsrc(a.k + (int64_t)kvh * N * D, slab);
  const rsrc_t rv = make_rsrc(a.v + (int64_t)kvh * N * D, slab);
  const rsrc_t ro = make_rsrc(a.o + (int64_t)head * N * D, slab);

  const int q0 = qtile * T::BM;
  const int q0w = q0 + 32 * wave;
  const int qrow = q0w + ql;

  // Q^T operand fragments: lane (query ql, k-half g), d = 16*kk + 8*g .. +7.
  half8 qf[D / 16];
#pragma unroll
  for (int kk = 0; kk < D / 16; ++kk)
    qf[kk] = __builtin_bit_cast(half8, buf_load_b128(rq, (uint32_t)(qrow * D + 16 * kk + 8 * g) * 2u));

  float16v o[D / 32];
#pragma unroll
  for (int db = 0; db < D / 32; ++db)
#pragma unroll
    for (int j = 0; j < 16; ++j) o[db][j] = 0.f;
  float m = -INFINITY;  // running max, already multiplied by c
  float l = 0.f;        // this lane's partial running sum (its 16 keys per block)
  const float c = a.c;

  const int kv_end = CAUSAL ? min(N, q0 + T::BM) : N;
  const int ntiles = (kv_end + BN - 1) / BN;

  u32x4 kreg[T::K_PER_T];
  u32x4 vreg[T::V_PER_T][2];

  auto load_tile = [&](int kv0) {
#pragma unroll
    for (int i = 0; i < T::K_PER_T; ++i) {
      const int ci = tid + i * T::NT;
      if (T::K_CHUNKS % T::NT == 0 || ci < T::K_CHUNKS) {
        const int row = ci / T::DC, cc = ci - row * T::DC;
        kreg[i] = buf_load_b128(rk, (uint32_t)((kv0 + row) * D + 8 * cc) * 2u);
      }
    }
#pragma unroll
    for (int i = 0; i < T::V_PER_T; ++i) {
      const int u = tid + i * T::NT;
      if (T::V_UNITS % T::NT == 0 || u < T::V_UNITS) {
        const int p = u / T::DC, cc = u - p * T::DC;
        vreg[i][0] = buf_load_b128(rv, (uint32_t)((kv0 + 2 * p) * D + 8 * cc) * 2u);
        vreg[i][1] = buf_load_b128(rv, (uint32_t)((kv0 + 2 * p + 1) * D + 8 * cc) * 2u);
      }
    }
  };
  auto store_tile = [&]() {
#pragma unroll
    for (int i = 0; i < T::K_PER_T; ++i) {
      const int ci = tid + i * T::NT;
      if (T::K_CHUNKS % T::NT == 0 || ci < T::K_CHUNKS) {
        const int row = ci / T::DC, cc = ci - row * T::DC;
        *reinterpret_cast<u32x4*>(&Ks[row * T::KS + 8 * cc]) = kreg[i];
      }
    }
#pragma unroll
    for (int i = 0; i < T::V_PER_T; ++i) {
      const int u = tid + i * T::NT;
      if (T::V_UNITS % T::NT == 0 || u < T::V_UNITS) {
        const int p = u / T::DC, cc = u - p * T::DC;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const unsigned r0 = vreg[i][0][e], r1 = vreg[i][1][e];
          *reinterpret_cast<unsigned*>(&Vt[(8 * cc + 2 * e) * T::VS + 2 * p]) = pack_lo(r0, r1);
          *reinterpret_cast<unsigned*>(&Vt[(8 * cc + 2 * e + 1) * T::VS + 2 * p]) = pack_hi(r0, r1);
        }
      }
    }
  };

  load_tile(0);
  store_tile();
  __syncthreads();

  const int prow = row_perm(ql);
  for (int t = 0; t < ntiles; ++t) {
    const int kv0 = t * BN;
    const bool more = t + 1 < ntiles;
    if (more) load_tile(kv0 + BN);

    const bool active = (q0w < N) && !(CAUSAL && kv0 > q0w + 31);
    if (active) {
      float16v s[BN / 32];
#pragma unroll
      for (int kb = 0; kb < BN / 32; ++kb) {
#pragma unroll
        for (int j = 0; j < 16; ++j) s[kb][j] = 0.f;
#pragma unroll
        for (int kk = 0; kk < D / 16; ++kk) {
          const half8 ka =
              *reinterpret_cast<const half8*>(&Ks[(32 * kb + prow) * T::KS + 16 * kk + 8 * g]);
          s[kb] = mfma32(ka, qf[kk], s[kb]);
        }
      }
      const bool need_mask = (CAUSAL && kv0 + BN - 1 > q0w) || (kv0 + BN > N);
      if (need_mask) {
#pragma unroll
        for (int kb = 0; kb < BN / 32; ++kb)
#pragma unroll
          for (int j = 0; j < 16; ++j) {
            const int key = kv0 + 32 * kb + result_row(j, g);
            const bool ok = key < N && (!CAUSAL || key <= qrow);
            if (!ok) s[kb][j] = -INFINITY;
          }
      }
      float mx = -INFINITY;
#pragma unroll
      for (int kb = 0; kb < BN / 32; ++kb)
#pragma unroll
        for (int j = 0; j < 16; ++j) mx = fmaxf(mx, s[kb][j]);
      mx = fmaxf(mx, swap_halves(mx));
      const float m_new = fmaxf(m, mx * c);
      const float alpha = exp2_fast(m - m_new);
      const float nm = -m_new;
      half8 pk[BN / 32][2];
      float ls = 0.f;
#pragma unroll
      for (int kb = 0; kb < BN / 32; ++kb)
#pragma unroll
        for (int j = 0; j < 16; ++j) {
          const float p = exp2_fast(fmaf(s[kb][j], c, nm));
          ls += p;
          pk[kb][j >> 3][j & 7] = (half_t)p;
        }
      l = fmaf(l, alpha, ls);
      m = m_new;
#pragma unroll
      for (int db = 0; db < D / 32; ++db) o[db] *= alpha;
#pragma unroll
      for (int kb = 0; kb < BN / 32; ++kb)
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
          for (int db = 0; db < D / 32; ++db) {
            const half8 va = *reinterpret_cast<const half8*>(
                &Vt[(32 * db + ql) * T::VS + 32 * kb + 16 * h + 8 * g]);
            o[db] = mfma32(va, pk[kb][h], o[db]);
          }
    }

    if (more) {
      __syncthreads();
      store_tile();
      __syncthreads();
    }
  }

  // Epilogue: lane (query qrow, half g) holds d = 32*db + 8*(j/4) + 4*g + j%4.
  const float lt = l + swap_halves(l);
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

#define FA_FWD_VARIANT(NW, BN)                                                           \
  {                                                                                      \
    NW, 32 * NW, BN,                                                                     \
    {                                                                                    \
      {(void*)&fwd_launch<32, false, NW, BN>, (void*)&fwd_launch<32, true, NW, BN>},     \
      {(void*)&fwd_launch<64, false, NW, BN>, (void*)&fwd_launch<64, true, NW, BN>},     \
      {(void*)&fwd_launch<128, false, NW, BN>, (void*)&fwd_launch<128, true, NW, BN>},   \
    }                                                                                    \
  }

static const Variant kFwdVariants[] = {
    FA_FWD_VARIANT(4, 64),
    FA_FWD_VARIANT(8, 64),
    FA_FWD_VARIANT(4, 32),
};

const Variant* fwd_variants(int* count) {
  *count = (int)(sizeof(kFwdVariants) / sizeof(kFwdVariants[0]));
  return kFwdVariants;
}

}  // namespace fa
