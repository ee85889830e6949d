// fa_bwd.hip — FlashAttention-2 backward for gfx950: Delta preprocess,
// dK/dV kernel and dQ kernel.
//
// Semantics follow the reference backward (triton_flash_attention/attention.py):
//   Delta_i = sum_d O_id dO_id in fp32 from the stored fp16 O      (237-255)
//   P = exp2(s * scale * log2(e) - LSE), masked keys/queries -> 0 (296-300, 339-343)
//   dV = P^T dO, dP = dO V^T, dS = P (dP - Delta)                  (302-304, 345-346)
//   dK = scale dS^T Q, dQ = scale dS K                             (305, 347, 499, 572)
//   causal: dK/dV visit query tiles at or below the key tile, dQ visits
//   key tiles at or left of the query tile                         (439-478, 518-552)
//   GQA: dK/dV are sums over the Hq/Hkv query heads of a group     (503-505)
//
// MI355X design:
//   * dK/dV and dQ are separate kernels (no atomics). The dK/dV work-group
//     owns 32*NW keys and loops over the query heads of its GQA group inside
//     the kernel, so the group reduction is an fp32 register accumulation and
//     the result is deterministic;
//   * the scale is applied in fp32 after each MFMA (one FMA with -LSE), so
//     P is rebuilt from unrounded operands;
//   * matrices reduced over the sequence axis are staged TRANSPOSED in LDS
//     (Q^T, dO^T for dK/dV; K^T for dQ) so every MFMA operand is one
//     16-byte LDS read; the transposition is done in registers while storing;
//   * every MFMA result layout is chosen so that the next MFMA consumes the
//     lane's own values (row_perm on the LDS reads), and results are written
//     as 8-byte runs along the head dimension.
#include "fa_common.hpp"
#include "fa_kernels.hpp"

namespace fa {

// --------------------------------------------------------------------------
// Delta = rowsum(O * dO)
// --------------------------------------------------------------------------
template <int D>
__global__ __launch_bounds__(256) void preprocess_kernel(const half_t* __restrict__ o,
                                                         const half_t* __restrict__ dO,
                                                         float* __restrict__ delta,
                                                         int64_t rows) {
  constexpr int TPR = D / 8;  // threads per row, 8 halves each
  const int64_t gid = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t row = gid / TPR;
  const int cc = (int)(gid - row * TPR);
  float acc = 0.f;
  if (row < rows) {
    const int64_t off = row * D + 8 * cc;
    const half8 ov = *reinterpret_cast<const half8*>(o + off);
    const half8 dv = *reinterpret_cast<const half8*>(dO + off);
#pragma unroll
    for (int i = 0; i < 8; ++i) acc = fmaf((float)ov[i], (float)dv[i], acc);
  }
#pragma unroll
  for (int off = TPR / 2; off > 0; off >>= 1) acc += __shfl_xor(acc, off, 64);
  if (cc == 0 && row < rows) delta[row] = acc;
}

hipError_t launch_preprocess(const half_t* o, const half_t* dO, float* delta, int64_t rows,
                             int D, hipStream_t stream) {
  const int64_t threads = rows * (D / 8);
  const int64_t blocks = (threads + 255) / 256;
  if (blocks <= 0 || blocks > 0x7fffffff) return hipErrorInvalidConfiguration;
  switch (D) {
    case 32:
      hipLaunchKernelGGL(preprocess_kernel<32>, dim3((unsigned)blocks), dim3(256), 0, stream, o,
                         dO, delta, rows);
      break;
    case 64:
      hipLaunchKernelGGL(preprocess_kernel<64>, dim3((unsigned)blocks), dim3(256), 0, stream, o,
                         dO, delta, rows);
      break;
    case 128:
      hipLaunchKernelGGL(preprocess_kernel<128>, dim3((unsigned)blocks), dim3(256), 0, stream,
                         o, dO, delta, rows);
      break;
    default:
      return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

// --------------------------------------------------------------------------
// Staging of a [R x D] fp16 tile into LDS, both row-major (stride D+8) and,
// optionally, transposed (d-major, stride R+8). Each thread moves
// (row pair, 16-byte chunk) units; the transposition packs the two rows'
// halves pairwise into dwords.
// --------------------------------------------------------------------------
template <int D, int R, int NT, bool TRANSPOSE>
struct TileStager {
  static constexpr int DC = D / 8;
  static constexpr int RS = D + 8;
  static constexpr int TS = R + 8;
  static constexpr int UNITS = (R / 2) * DC;
  static constexpr int PER_T = (UNITS + NT - 1) / NT;
  u32x4 reg[PER_T][2];

  __device__ __forceinline__ void load(rsrc_t r, int row0, int tid) {
#pragma unroll
    for (int i = 0; i < PER_T; ++i) {
      const int u = tid + i * NT;
      if (UNITS % NT == 0 || u < UNITS) {
        const int p = u / DC, cc = u - p * DC;
        reg[i][0] = buf_load_b128(r, (uint32_t)((row0 + 2 * p) * D + 8 * cc) * 2u);
        reg[i][1] = buf_load_b128(r, (uint32_t)((row0 + 2 * p + 1) * D + 8 * cc) * 2u);
      }
    }
  }
  __device__ __forceinline__ void store(half_t* rowmajor, half_t* transposed, int tid) const {
#pragma unroll
    for (int i = 0; i < PER_T; ++i) {
      const int u = tid + i * NT;
      if (UNITS % NT == 0 || u < UNITS) {
        const int p = u / DC, cc = u - p * DC;
        *reinterpret_cast<u32x4*>(&rowmajor[(2 * p) * RS + 8 * cc]) = reg[i][0];
        *reinterpret_cast<u32x4*>(&rowmajor[(2 * p + 1) * RS + 8 * cc]) = reg[i][1];
        if (TRANSPOSE) {
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const unsigned r0 = reg[i][0][e], r1 = reg[i][1][e];
            *reinterpret_cast<unsigned*>(&transposed[(8 * cc + 2 * e) * TS + 2 * p]) =
                pack_lo(r0, r1);
            *reinterpret_cast<unsigned*>(&transposed[(8 * cc + 2 * e + 1) * TS + 2 * p]) =
                pack_hi(r0, r1);
          }
        }
      }
    }
  }
};

// --------------------------------------------------------------------------
// dK / dV
// --------------------------------------------------------------------------
template <int D, int NW, int QT>
struct DkdvTile {
  static constexpr int BKV = 32 * NW;  // keys per work-group
  static constexpr int NT = 64 * NW;
  static constexpr int RS = D + 8;
  static constexpr int TS = QT + 8;
  static constexpr int MAT = QT * RS + D * TS;  // one tensor, both layouts
  static constexpr int LDS_HALVES = 2 * MAT;
  static constexpr int LDS_BYTES = LDS_HALVES * 2 + 2 * QT * 4;
  static_assert(QT % 32 == 0, "query tile must be a multiple of 32");
  static_assert(LDS_BYTES <= 160 * 1024, "LDS budget");
};

template <int D, bool CAUSAL, int NW, int QT>
__global__ __launch_bounds__(64 * NW) void dkdv_kernel(BwdArgs a) {
  using T = DkdvTile<D, NW, QT>;
  __shared__ __attribute__((aligned(16))) half_t lds[T::LDS_HALVES + 4 * QT];
  half_t* Qs = lds;
  half_t* Qt = lds + QT * T::RS;
  half_t* dOs = lds + T::MAT;
  half_t* dOt = dOs + QT * T::RS;
  float* Ls = reinterpret_cast<float*>(lds + T::LDS_HALVES);
  float* Ds = Ls + QT;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int ql = lane & 31;
  const int g = lane >> 5;

  // Key tiles near the start see the most queries under the causal mask:
  // ascending tile order is heavy-first.
  const TileHead th = decode_block(blockIdx.x, a.BHkv);
  const int kvtile = th.tile_rank;
  const int kvh = th.head;
  const int b = kvh / a.Hkv;
  const int hkv = kvh - b * a.Hkv;
  const int N = a.N;
  const uint32_t slab = (uint32_t)N * D * 2u;
  const uint32_t aux = (uint32_t)N * 4u;
  const rsrc_t rk = make_rsrc(a.k + (int64_t)kvh * N * D, slab);
  const rsrc_t rv = make_rsrc(a.v + (int64_t)kvh * N * D, slab);

  const int k0 = kvtile * T::BKV;
  const int k0w = k0 + 32 * wave;
  const int krow = k0w + ql;

  // K and V as B-operands (column = key ql, d = 16*kk + 8*g .. +7).
  half8 kf[D / 16], vf[D / 16];
#pragma unroll
  for (int kk = 0; kk < D / 16; ++kk) {
    const uint32_t off = (uint32_t)(krow * D + 16 * kk + 8 * g) * 2u;
    kf[kk] = __builtin_bit_cast(half8, buf_load_b128(rk, off));
    vf[kk] = __builtin_bit_cast(half8, buf_load_b128(rv, off));
  }

  // dK^T, dV^T accumulators: lane (key ql), rows d = 32*db + 8*(j/4) + 4*g + j%4.
  float16v dk[D / 32], dv[D / 32];
#pragma unroll
  for (int db = 0; db < D / 32; ++db)
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      dk[db][j] = 0.f;
      dv[db][j] = 0.f;
    }

  const float c = a.c;
  const int prow = row_perm(ql);
  const bool wave_live = k0w < N;
  const int q_begin = CAUSAL ? (k0 / QT) * QT : 0;
  const int ntiles = (N - q_begin + QT - 1) / QT;

  TileStager<D, QT, T::NT, true> sq, sdo;
  // Threads [0, QT) carry the tile's LSE values, [QT, 2 QT) its Delta values
  // (Ls and Ds are adjacent in LDS, so both land at Ls[tid]).
  float aux_reg = 0.f;
  static_assert(2 * QT <= T::NT, "one LSE/Delta value per thread");

  for (int gi = 0; gi < a.group; ++gi) {
    const int head = b * a.Hq + hkv * a.group + gi;
    const rsrc_t rq = make_rsrc(a.q + (int64_t)head * N * D, slab);
    const rsrc_t rdo = make_rsrc(a.dO + (int64_t)head * N * D, slab);
    const rsrc_t rl = make_rsrc(a.lse + (int64_t)head * N, aux);
    const rsrc_t rd = make_rsrc(a.delta + (int64_t)head * N, aux);

    auto load_tile = [&](int qt0) {
      sq.load(rq, qt0, tid);
      sdo.load(rdo, qt0, tid);
      if (tid < 2 * QT) {
        const bool is_lse = tid < QT;
        const int row = qt0 + (is_lse ? tid : tid - QT);
        aux_reg = buf_load_f32(is_lse ? rl : rd, (uint32_t)row * 4u);
      }
    };
    auto store_tile = [&]() {
      sq.store(Qs, Qt, tid);
      sdo.store(dOs, dOt, tid);
      if (tid < 2 * QT) Ls[tid] = aux_reg;
    };

    if (gi > 0) __syncthreads();  // previous head's last tile fully consumed
    load_tile(q_begin);
    store_tile();
    __syncthreads();

    for (int t = 0; t < ntiles; ++t) {
      const int qt0 = q_begin + t * QT;
      const bool more = t + 1 < ntiles;
      if (more) load_tile(qt0 + QT);

#pragma unroll
      for (int qb = 0; qb < QT / 32; ++qb) {
        const int qa = qt0 + 32 * qb;
        const bool active = wave_live && qa < N && !(CAUSAL && qa + 31 < k0w);
        if (!active) continue;
        float16v s, dp;
#pragma unroll
        for (int j = 0; j < 16; ++j) {
          s[j] = 0.f;
          dp[j] = 0.f;
        }
#pragma unroll
        for (int kk = 0; kk < D / 16; ++kk) {
          const int off = (32 * qb + prow) * T::RS + 16 * kk + 8 * g;
          s = mfma32(*reinterpret_cast<const half8*>(&Qs[off]), kf[kk], s);
          dp = mfma32(*reinterpret_cast<const half8*>(&dOs[off]), vf[kk], dp);
        }
        // Lane's queries: local 32*qb + 16*h + 8*g + e, e = 0..7 (value j = 8h + e).
        float lse_v[16], del_v[16];
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const int base = 32 * qb + 16 * h + 8 * g;
          const float4v l0 = *reinterpret_cast<const float4v*>(&Ls[base]);
          const float4v l1 = *reinterpret_cast<const float4v*>(&Ls[base + 4]);
          const float4v d0 = *reinterpret_cast<const float4v*>(&Ds[base]);
          const float4v d1 = *reinterpret_cast<const float4v*>(&Ds[base + 4]);
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            lse_v[8 * h + e] = l0[e];
            lse_v[8 * h + 4 + e] = l1[e];
            del_v[8 * h + e] = d0[e];
            del_v[8 * h + 4 + e] = d1[e];
          }
        }
        const bool need_mask = (CAUSAL && qa < k0w + 31) || (qa + 32 > N);
        float p[16], ds[16];
#pragma unroll
        for (int j = 0; j < 16; ++j) {
          float pj = exp2_fast(fmaf(s[j], c, -lse_v[j]));
          if (need_mask) {
            const int q = qa + result_row(j, g);
            if (q >= N || (CAUSAL && q < krow)) pj = 0.f;
          }
          p[j] = pj;
          ds[j] = pj * (dp[j] - del_v[j]);
        }
        half8 pa[2], sa[2];
        pa[0] = to_half8(p);
        pa[1] = to_half8(p + 8);
        sa[0] = to_half8(ds);
        sa[1] = to_half8(ds + 8);
#pragma unroll
        for (int h = 0; h < 2; ++h)
#pragma unroll
          for (int db = 0; db < D / 32; ++db) {
            const int off = (32 * db + ql) * T::TS + 32 * qb + 16 * h + 8 * g;
            dv[db] = mfma32(*reinterpret_cast<const half8*>(&dOt[off]), pa[h], dv[db]);
            dk[db] = mfma32(*reinterpret_cast<const half8*>(&Qt[off]), sa[h], dk[db]);
          }
      }

      if (more) {
        __syncthreads();
        store_tile();
        __syncthreads();
      }
    }
  }

  const float scale = a.scale;
  const rsrc_t rdk = make_rsrc(a.dk + (int64_t)kvh * N * D, slab);
  const rsrc_t rdv = make_rsrc(a.dv + (int64_t)kvh * N * D, slab);
#pragma unroll
  for (int db = 0; db < D / 32; ++db)
#pragma unroll
    for (int jq = 0; jq < 4; ++jq) {
      const uint32_t off = (uint32_t)(krow * D + 32 * db + 8 * jq + 4 * g) * 2u;
      buf_store_b64(rdk, off,
                    pack4_half(dk[db][4 * jq] * scale, dk[db][4 * jq + 1] * scale,
                               dk[db][4 * jq + 2] * scale, dk[db][4 * jq + 3] * scale));
      buf_store_b64(rdv, off,
                    pack4_half(dv[db][4 * jq], dv[db][4 * jq + 1], dv[db][4 * jq + 2],
                               dv[db][4 * jq + 3]));
    }
}

template <int D, bool CAUSAL, int NW, int QT>
hipError_t dkdv_launch(const BwdArgs& a, hipStream_t stream) {
  using T = DkdvTile<D, NW, QT>;
  BwdArgs b = a;
  b.num_tiles = (a.N + T::BKV - 1) / T::BKV;
  const int64_t blocks = (int64_t)b.num_tiles * a.BHkv;
  if (blocks <= 0 || blocks > 0x7fffffff) return hipErrorInvalidConfiguration;
  hipLaunchKernelGGL((dkdv_kernel<D, CAUSAL, NW, QT>), dim3((unsigned)blocks), dim3(T::NT), 0,
                     stream, b);
  return hipGetLastError();
}

// --------------------------------------------------------------------------
// dQ
// --------------------------------------------------------------------------
template <int D, int NW, int KT>
struct DqTile {
  static constexpr int BQ = 32 * NW;  // queries per work-group
  static constexpr int NT = 64 * NW;
  static constexpr int RS = D + 8;
  static constexpr int TS = KT + 8;
  static constexpr int LDS_HALVES = 2 * KT * RS + D * TS;  // K, V row-major + K^T
  static_assert(KT % 32 == 0, "key tile must be a multiple of 32");
  static_assert(LDS_HALVES * 2 <= 160 * 1024, "LDS budget");
};

template <int D, bool CAUSAL, int NW, int KT>
__global__ __launch_bounds__(64 * NW) void dq_kernel(BwdArgs a) {
  using T = DqTile<D, NW, KT>;
  __shared__ __attribute__((aligned(16))) half_t lds[T::LDS_HALVES];
  half_t* Ks = lds;
  half_t* Kt = lds + KT * T::RS;
  half_t* Vs = Kt + D * T::TS;

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
  const uint32_t aux = (uint32_t)N * 4u;
  const rsrc_t rq = make_rsrc(a.q + (int64_t)head * N * D, slab);
  const rsrc_t rdo = make_rsrc(a.dO + (int64_t)head * N * D, slab);
  const rsrc_t rk = make_rsrc(a.k + (int64_t)kvh * N * D, slab);
  const rsrc_t rv = make_rsrc(a.v + (int64_t)kvh * N * D, slab);
  const rsrc_t rl = make_rsrc(a.lse + (int64_t)head * N, aux);
  const rsrc_t rd = make_rsrc(a.delta + (int64_t)head * N, aux);

  const int q0 = qtile * T::BQ;
  const int q0w = q0 + 32 * wave;
  const int qrow = q0w + ql;

  half8 qf[D / 16], dof[D / 16];
#pragma unroll
  for (int kk = 0; kk < D / 16; ++kk) {
    const uint32_t off = (uint32_t)(qrow * D + 16 * kk + 8 * g) * 2u;
    qf[kk] = __builtin_bit_cast(half8, buf_load_b128(rq, off));
    dof[kk] = __builtin_bit_cast(half8, buf_load_b128(rdo, off));
  }
  const float lse = buf_load_f32(rl, (uint32_t)qrow * 4u);
  const float delta = buf_load_f32(rd, (uint32_t)qrow * 4u);

  // dQ^T accumulator: lane (query ql), rows d = 32*db + 8*(j/4) + 4*g + j%4.
  float16v dq[D / 32];
#pragma unroll
  for (int db = 0; db < D / 32; ++db)
#pragma unroll
    for (int j = 0; j < 16; ++j) dq[db][j] = 0.f;

  const float c = a.c;
  const float nl = -lse;
  const int prow = row_perm(ql);
  const int kv_end = CAUSAL ? min(N, q0 + T::BQ) : N;
  const int ntiles = (kv_end + KT - 1) / KT;

  TileStager<D, KT, T::NT, true> sk;
  TileStager<D, KT, T::NT, false> sv;

  sk.load(rk, 0, tid);
  sv.load(rv, 0, tid);
  sk.store(Ks, Kt, tid);
  sv.store(Vs, nullptr, tid);
  __syncthreads();

  for (int t = 0; t < ntiles; ++t) {
    const int kt0 = t * KT;
    const bool more = t + 1 < ntiles;
    if (more) {
      sk.load(rk, kt0 + KT, tid);
      sv.load(rv, kt0 + KT, tid);
    }
#pragma unroll
    for (int kb = 0; kb < KT / 32; ++kb) {
      const int ka = kt0 + 32 * kb;
      const bool active = q0w < N && ka < N && !(CAUSAL && ka > q0w + 31);
      if (!active) continue;
      float16v s, dp;
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        s[j] = 0.f;
        dp[j] = 0.f;
      }
#pragma unroll
      for (int kk = 0; kk < D / 16; ++kk) {
        const int off = (32 * kb + prow) * T::RS + 16 * kk + 8 * g;
        s = mfma32(*reinterpret_cast<const half8*>(&Ks[off]), qf[kk], s);
        dp = mfma32(*reinterpret_cast<const half8*>(&Vs[off]), dof[kk], dp);
      }
      const bool need_mask = (CAUSAL && ka + 31 > q0w) || (ka + 32 > N);
      float ds[16];
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        float pj = exp2_fast(fmaf(s[j], c, nl));
        if (need_mask) {
          const int key = ka + result_row(j, g);
          if (key >= N || (CAUSAL && key > qrow)) pj = 0.f;
        }
        ds[j] = pj * (dp[j] - delta);
      }
      half8 sa[2];
      sa[0] = to_half8(ds);
      sa[1] = to_half8(ds + 8);
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int db = 0; db < D / 32; ++db) {
          const int off = (32 * db + ql) * T::TS + 32 * kb + 16 * h + 8 * g;
          dq[db] = mfma32(*reinterpret_cast<const half8*>(&Kt[off]), sa[h], dq[db]);
        }
    }
    if (more) {
      __syncthreads();
      sk.store(Ks, Kt, tid);
      sv.store(Vs, nullptr, tid);
      __syncthreads();
    }
  }

  const float scale = a.scale;
  const rsrc_t rdq = make_rsrc(a.dq + (int64_t)head * N * D, slab);
#pragma unroll
  for (int db = 0; db < D / 32; ++db)
#pragma unroll
    for (int jq = 0; jq < 4; ++jq) {
      const uint32_t off = (uint32_t)(qrow * D + 32 * db + 8 * jq + 4 * g) * 2u;
      buf_store_b64(rdq, off,
                    pack4_half(dq[db][4 * jq] * scale, dq[db][4 * jq + 1] * scale,
                               dq[db][4 * jq + 2] * scale, dq[db][4 * jq + 3] * scale));
    }
}

template <int D, bool CAUSAL, int NW, int KT>
hipError_t dq_launch(const BwdArgs& a, hipStream_t stream) {
  using T = DqTile<D, NW, KT>;
  BwdArgs b = a;
  b.num_tiles = (a.N + T::BQ - 1) / T::BQ;
  const int64_t blocks = (int64_t)b.num_tiles * a.BH;
  if (blocks <= 0 || blocks > 0x7fffffff) return hipErrorInvalidConfiguration;
  hipLaunchKernelGGL((dq_kernel<D, CAUSAL, NW, KT>), dim3((unsigned)blocks), dim3(T::NT), 0,
                     stream, b);
  return hipGetLastError();
}

#define FA_BWD_VARIANT(LAUNCH, ROWS_PER_WAVE, NW, TILE)                                   \
  {                                                                                       \
    NW, ROWS_PER_WAVE * NW, TILE,                                                         \
    {                                                                                     \
      {(void*)&LAUNCH<32, false, NW, TILE>, (void*)&LAUNCH<32, true, NW, TILE>},          \
      {(void*)&LAUNCH<64, false, NW, TILE>, (void*)&LAUNCH<64, true, NW, TILE>},          \
      {(void*)&LAUNCH<128, false, NW, TILE>, (void*)&LAUNCH<128, true, NW, TILE>},        \
    }                                                                                     \
  }

static const Variant kDkdvVariants[] = {
    FA_BWD_VARIANT(dkdv_launch, 32, 4, 64),
    FA_BWD_VARIANT(dkdv_launch, 32, 4, 32),
    FA_BWD_VARIANT(dkdv_launch, 32, 2, 64),
};

static const Variant kDqVariants[] = {
    FA_BWD_VARIANT(dq_launch, 32, 4, 64),
    FA_BWD_VARIANT(dq_launch, 32, 4, 32),
    FA_BWD_VARIANT(dq_launch, 32, 2, 64),
};

const Variant* dkdv_variants(int* count) {
  *count = (int)(sizeof(kDkdvVariants) / sizeof(kDkdvVariants[0]));
  return kDkdvVariants;
}

const Variant* dq_variants(int* count) {
  *count = (int)(sizeof(kDqVariants) / sizeof(kDqVariants[0]));
  return kDqVariants;
}

}  // namespace fa
