// fa_bwd.hip — FlashAttention-2 backward for gfx950: Delta preprocess,
// dK/dV kernel and dQ kernel.
//
// Semantics follow the reference backward (triton_flash_attention/attention.py):
//   Delta_i = sum_d O_id dO_id in fp32 from the stored fp16 O      (237-255)
//   P = exp2(s - LSE) with the scores s taken in log2 units from the
//   reference's scaled fp16 operands: s = q . fp16(c k) for dK / dV and
//   s = fp16(c q) . k for dQ, c = fp32(scale * log2(e))       (297, 340, 435, 515)
//   masked keys/queries -> 0                                      (296-300, 339-343)
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
#include <type_traits>

#include "fa_bwd_pipe.hpp"
#include "fa_bwd_pipe16.hpp"
#include "fa_common.hpp"
#include "fa_kernels.hpp"

namespace fa {

// --------------------------------------------------------------------------
// Delta = rowsum(O * dO)
// --------------------------------------------------------------------------
template <int D, class E = F16>
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
    for (int i = 0; i < 8; ++i) acc = fmaf(elem_to_f32<E>(ov[i]), elem_to_f32<E>(dv[i]), acc);
  }
#pragma unroll
  for (int off = TPR / 2; off > 0; off >>= 1) acc += __shfl_xor(acc, off, 64);
  if (cc == 0 && row < rows) delta[row] = acc;
}

template <class E>
hipError_t launch_preprocess_e(const half_t* o, const half_t* dO, float* delta, int64_t rows,
                               int D, hipStream_t stream) {
  const int64_t threads = rows * (D / 8);
  const int64_t blocks = (threads + 255) / 256;
  if (blocks <= 0 || blocks > 0x7fffffff) return hipErrorInvalidConfiguration;
  switch (D) {
    case 32:
      hipLaunchKernelGGL((preprocess_kernel<32, E>), dim3((unsigned)blocks), dim3(256), 0, stream,
                         o, dO, delta, rows);
      break;
    case 64:
      hipLaunchKernelGGL((preprocess_kernel<64, E>), dim3((unsigned)blocks), dim3(256), 0, stream,
                         o, dO, delta, rows);
      break;
    case 128:
      hipLaunchKernelGGL((preprocess_kernel<128, E>), dim3((unsigned)blocks), dim3(256), 0, stream,
                         o, dO, delta, rows);
      break;
    default:
      return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_preprocess(const half_t* o, const half_t* dO, float* delta, int64_t rows,
                             int D, int dtype, hipStream_t stream) {
  return dtype == kBF16 ? launch_preprocess_e<BF16>(o, dO, delta, rows, D, stream)
                        : launch_preprocess_e<F16>(o, dO, delta, rows, D, stream);
}

// --------------------------------------------------------------------------
// dK/dV split reduction: out[i] = E(sum_s part[s][i]) in split order.
// --------------------------------------------------------------------------
template <class E = F16>
__global__ __launch_bounds__(256) void split_reduce_kernel(const float* __restrict__ part,
                                                           half_t* __restrict__ dk,
                                                           half_t* __restrict__ dv,
                                                           int64_t plane4, int nsplit) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;  // float4 index in 2 planes
  if (i >= 2 * plane4) return;
  const bool is_v = i >= plane4;
  const int64_t j = is_v ? i - plane4 : i;
  const float4v* src = reinterpret_cast<const float4v*>(part) + (is_v ? plane4 : 0) + j;
  float4v acc = src[0];
#pragma unroll 8
  for (int sp = 1; sp < nsplit; ++sp) acc += src[(int64_t)sp * 2 * plane4];
  half4 h;
#pragma unroll
  for (int e = 0; e < 4; ++e) h[e] = to_elem<E>(acc[e]);
  *reinterpret_cast<half4*>((is_v ? dv : dk) + 4 * j) = h;
}

template <class E>
__global__ __launch_bounds__(256) void split_sum_kernel(const float* __restrict__ part,
                                                        half_t* __restrict__ out, int64_t elems4,
                                                        int nsplit) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;  // float4 index
  if (i >= elems4) return;
  const float4v* src = reinterpret_cast<const float4v*>(part) + i;
  float4v acc = src[0];
#pragma unroll 8
  for (int sp = 1; sp < nsplit; ++sp) acc += src[(int64_t)sp * elems4];
  half4 h;
#pragma unroll
  for (int e = 0; e < 4; ++e) h[e] = to_elem<E>(acc[e]);
  *reinterpret_cast<half4*>(out + 4 * i) = h;
}

hipError_t launch_split_sum(const float* part, half_t* out, int64_t elems, int nsplit, int dtype,
                            hipStream_t stream) {
  const int64_t elems4 = elems / 4;
  const int64_t blocks = (elems4 + 255) / 256;
  if (elems % 4 != 0 || nsplit < 2 || blocks <= 0 || blocks > 0x7fffffff)
    return hipErrorInvalidValue;
  if (dtype == kBF16)
    hipLaunchKernelGGL(split_sum_kernel<BF16>, dim3((unsigned)blocks), dim3(256), 0, stream, part,
                       out, elems4, nsplit);
  else
    hipLaunchKernelGGL(split_sum_kernel<F16>, dim3((unsigned)blocks), dim3(256), 0, stream, part,
                       out, elems4, nsplit);
  return hipGetLastError();
}


hipError_t launch_split_reduce(const float* part, half_t* dk, half_t* dv, int64_t plane_elems,
                               int nsplit, int dtype, hipStream_t stream) {
  const int64_t plane4 = plane_elems / 4;
  const int64_t blocks = (2 * plane4 + 255) / 256;
  if (plane_elems % 4 != 0 || blocks <= 0 || blocks > 0x7fffffff) return hipErrorInvalidValue;
  if (dtype == kBF16)
    hipLaunchKernelGGL(split_reduce_kernel<BF16>, dim3((unsigned)blocks), dim3(256), 0, stream,
                       part, dk, dv, plane4, nsplit);
  else
    hipLaunchKernelGGL(split_reduce_kernel<F16>, dim3((unsigned)blocks), dim3(256), 0, stream,
                       part, dk, dv, plane4, nsplit);
  return hipGetLastError();
}

// --------------------------------------------------------------------------
// dK / dV
//
// Work-group: NW waves x 32 keys (K, V resident in VGPRs as MFMA B operands).
// Streams (query head of the GQA group, 64-query tile) steps through a
// 3-slot LDS ring filled by DMA: Q tile, dO tile (row-major, swizzled) and
// the tile's LSE / Delta values. Per 32-query block:
//   S = Q fp16(c K)^T, dP = dO V^T          (row reads, result: lane = key)
//   P = exp2(S - LSE), dS = P (dP - Delta)
//   dV^T += dO^T P, dK^T += Q^T dS          (dO^T / Q^T via transposing reads)
// S and dP of every block of the tile are issued before the first block's
// vector work, so matrix and vector work overlap.
// --------------------------------------------------------------------------

template <int D, int NW, int QT>
struct DkdvTile {
  static constexpr int BKV = 32 * NW;  // keys per work-group
  static constexpr int NT = 64 * NW;
  static constexpr int TILE = QT * D;              // halves of the Q (or dO) tile
  static constexpr int AUX = 128;                  // floats: LSE[64], Delta[64]
  static constexpr int STAGE = 2 * TILE + 2 * AUX;  // halves per ring slot
  static constexpr int NSTAGE = 3;
  static constexpr int AHEAD = NSTAGE - 1;
  static_assert(QT == 32 || QT == 64, "query tile");
};

template <int D, int NW, int QT>
constexpr bool dkdv_tiling_ok() {
  return (QT * D * 2) % 1024 == 0 && ((QT * D * 2) / 1024) % NW == 0 &&
         3 * (2 * QT * D + 256) * 2 <= 160 * 1024;
}

// Waves per SIMD the classic dK/dV asks the compiler for.
template <int D, bool CAUSAL, int NW, int QT>
constexpr int dkdv_classic_waves_per_simd() {
  return D == 128 && !CAUSAL && NW == 4 && QT == 32 ? 2 : 1;
}

template <int D, bool CAUSAL, int NW, int QT, class E = F16>
__global__ __launch_bounds__(64 * NW)
__attribute__((amdgpu_waves_per_eu(dkdv_classic_waves_per_simd<D, CAUSAL, NW, QT>())))
void dkdv_kernel(BwdArgs a) {
  using T = DkdvTile<D, NW, QT>;
  using Dma = DmaStager<D, QT, NW>;
  constexpr int NB = QT / 32;                 // 32-query blocks per tile
  constexpr int IPT = 2 * Dma::PER_WAVE + 1;  // this wave's DMA instructions per step
  __shared__ __attribute__((aligned(16))) half_t lds[T::NSTAGE * T::STAGE];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int ql = lane & 31;
  const int g = lane >> 5;

  // Key tiles near the start see the most queries under the causal mask:
  // ascending tile order is heavy-first. Split mode: the split index is the
  // slowest-varying part of the block index.
  const int split = blockIdx.x / (a.num_tiles * a.BHkv);
  const TileHead th = decode_block(blockIdx.x - split * a.num_tiles * a.BHkv, a.BHkv);
  const int kvtile = th.tile_rank;
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

  const int k0 = kvtile * T::BKV;
  const int k0w = k0 + 32 * wave;
  const int krow = k0w + ql;

  // fp16(c K) and V as B-operands (column = key ql, d = 16*kk + 8*g .. +7),
  // completed before the first DMA; fp16(c K) is the reference's k_scaled
  // (attention.py:435), so S comes out in log2 units.
  half8 kf[D / 16], vf[D / 16];
#pragma unroll
  for (int kk = 0; kk < D / 16; ++kk) {
    const uint32_t off = (uint32_t)(krow * D + 16 * kk + 8 * g) * 2u;
    kf[kk] = __builtin_bit_cast(half8, buf_load_b128(rk, off));
    vf[kk] = __builtin_bit_cast(half8, buf_load_b128(rv, off));
  }
  wait_all_vm();
#pragma unroll
  for (int kk = 0; kk < D / 16; ++kk) {
#pragma unroll
    for (int e = 0; e < 8; ++e) kf[kk][e] = to_elem<E>(a.c * elem_to_f32<E>(kf[kk][e]));
    asm volatile("" : "+v"(kf[kk]));
  }

  const int q_begin = CAUSAL ? (k0 / QT) * QT : 0;
  // Under the causal mask a key tile past the last query (N < Nkv) sees no
  // query; it still takes one (empty) step, so its dK = dV = 0 are written.
  const int ntq = max(1, (N - q_begin + QT - 1) / QT);
  // This work-group's chunk [s_lo, s_lo + nsteps) of the tile's G * ntq steps.
  const int total_steps = G * ntq;
  const int chunk = (total_steps + a.nsplit - 1) / a.nsplit;
  const int s_lo = min(split * chunk, total_steps);
  const int nsteps = min(chunk, total_steps - s_lo);

  // Step s streams query tile (s % ntq) of query head (s / ntq) of the group.
  // Steps past the end load harmless data (rows past N read as zeros), so
  // every step issues the same number of DMA instructions.
  Dma dma;
  dma.init(wave, lane);
  auto issue_step = [&](int u, int slot) {
    const int st = s_lo + u;
    const int gi = min(st / ntq, G - 1);
    const int qt0 = q_begin + (st - gi * ntq) * QT;
    const int head = b * a.Hq + hkv * G + gi;
    half_t* base = lds + slot * T::STAGE;
    dma.issue(make_rsrc_words(a.q + (int64_t)head * N * D, slab), qt0, base, wave);
    dma.issue(make_rsrc_words(a.dO + (int64_t)head * N * D, slab), qt0, base + T::TILE, wave);
    // Even waves fetch LSE[qt0 .. qt0+64), odd waves Delta (duplicates of the
    // same bytes are harmless); lane l -> float l of the 64-entry table.
    const bool is_lse = (wave & 1) == 0;
    const float* src = (is_lse ? a.lse : a.delta) + (int64_t)head * N;
    dma_b32(make_rsrc_words(src, aux_bytes), (uint32_t)(qt0 + lane) * 4u,
            lds_addr(base + 2 * T::TILE + (is_lse ? 0 : 2 * 64)));
  };
#pragma unroll
  for (int st = 0; st < T::AHEAD; ++st) issue_step(st, st);

  // Loop-invariant per-lane LDS offsets (halves).
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

  // dK^T, dV^T accumulators: lane (key ql), rows d = 32*db + 8*(j/4) + 4*g + j%4.
  float16v dk[D / 32], dv[D / 32];
#pragma unroll
  for (int db = 0; db < D / 32; ++db)
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      dk[db][j] = 0.f;
      dv[db][j] = 0.f;
    }

  const bool wave_live = k0w < Nkv;

  auto step = [&](auto slot_c, int u) {
    constexpr int SLOT = decltype(slot_c)::value;
    issue_step(u + T::AHEAD, (SLOT + T::AHEAD) % T::NSTAGE);
    const int st = s_lo + u;
    const int gi = st / ntq;
    const int qt0 = q_begin + (st - gi * ntq) * QT;
    const half_t* Qs = lds + SLOT * T::STAGE;
    const half_t* dOs = Qs + T::TILE;
    const float* Ls = reinterpret_cast<const float*>(Qs + 2 * T::TILE);
    const float* Ds = Ls + 64;

    bool act[NB];
    float16v s[NB], dp[NB];
#pragma unroll
    for (int qb = 0; qb < NB; ++qb) {
      const int qa = qt0 + 32 * qb;
      act[qb] = wave_live && qa < N && !(CAUSAL && qa + 31 < k0w);
      if (act[qb]) {
#pragma unroll
        for (int j = 0; j < 16; ++j) {
          s[qb][j] = 0.f;
          dp[qb][j] = 0.f;
        }
#pragma unroll
        for (int kk = 0; kk < D / 16; ++kk) {
          const int off = 32 * qb * D + r_off[kk];
          s[qb] = mma<E>(*reinterpret_cast<const half8*>(Qs + off), kf[kk], s[qb]);
          dp[qb] = mma<E>(*reinterpret_cast<const half8*>(dOs + off), vf[kk], dp[qb]);
        }
      }
    }
#pragma unroll
    for (int qb = 0; qb < NB; ++qb) {
      if (!act[qb]) continue;
      const int qa = qt0 + 32 * qb;
      // The lane's queries: local 32*qb + 16*h + 8*g + e (value j = 8h + e).
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
      // Transposed operands of this block, read ahead of the vector work.
      half8 dot_f[2][D / 32], qt_f[2][D / 32];
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int db = 0; db < D / 32; ++db) {
          dot_f[h][db] = tr8(dOs + (32 * qb + 16 * h) * D, db);
          qt_f[h][db] = tr8(Qs + (32 * qb + 16 * h) * D, db);
        }
      const bool need_mask = (CAUSAL && qa < k0w + 31) || (qa + 32 > N);
      half8 pa[2], sa[2];
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        float pj = exp2_fast(s[qb][j] - lse_v[j]);
        if (need_mask) {
          const int q = qa + result_row(j, g);
          if (q >= N || (CAUSAL && q < krow)) pj = 0.f;
        }
        pa[j >> 3][j & 7] = to_elem<E>(pj);
        sa[j >> 3][j & 7] = to_elem<E>(pj * (dp[qb][j] - del_v[j]));
      }
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int db = 0; db < D / 32; ++db) {
          dv[db] = mma<E>(dot_f[h][db], pa[h], dv[db]);
          dk[db] = mma<E>(qt_f[h][db], sa[h], dk[db]);
        }
    }
    // Step st+1's tile complete for this wave, then published; slot st is free.
    wait_vm_and_barrier<(T::AHEAD - 1) * IPT>();
  };

  wait_vm_and_barrier<(T::AHEAD - 1) * IPT>();  // step 0's tile
  for (int u = 0; u < nsteps; u += T::NSTAGE) {
    step(ic<0>{}, u);
    if (u + 1 >= nsteps) break;
    step(ic<1>{}, u + 1);
    if (u + 2 >= nsteps) break;
    step(ic<2>{}, u + 2);
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");

  const float scale = a.scale;
  if (a.nsplit > 1) {
    // fp32 partials (dK already scaled); an empty chunk writes zeros.
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
            kq[e] = dk[db][4 * jq + e] * scale;
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
                    pack4<E>(dk[db][4 * jq] * scale, dk[db][4 * jq + 1] * scale,
                               dk[db][4 * jq + 2] * scale, dk[db][4 * jq + 3] * scale));
      buf_store_b64(rdv, off,
                    pack4<E>(dv[db][4 * jq], dv[db][4 * jq + 1], dv[db][4 * jq + 2],
                               dv[db][4 * jq + 3]));
    }
}

template <int D, bool CAUSAL, int NW, int QT, class E = F16>
hipError_t dkdv_launch(const BwdArgs& a, hipStream_t stream) {
  using T = DkdvTile<D, NW, QT>;
  BwdArgs b = a;
  b.num_tiles = (a.Nkv + T::BKV - 1) / T::BKV;
  if (b.nsplit < 1 || (b.nsplit > 1 && b.part == nullptr)) return hipErrorInvalidValue;
  const int64_t blocks = (int64_t)b.num_tiles * a.BHkv * b.nsplit;
  if (blocks <= 0 || blocks > 0x7fffffff) return hipErrorInvalidConfiguration;
  hipLaunchKernelGGL((dkdv_kernel<D, CAUSAL, NW, QT, E>), dim3((unsigned)blocks), dim3(T::NT), 0,
                     stream, b);
  return hipGetLastError();
}

// One work-group of dkdv_pipe_body per block.
template <int D, bool CAUSAL, int NW, class E = F16>
__global__ __launch_bounds__(64 * NW)
__attribute__((amdgpu_waves_per_eu(DkdvPipeTile<D, NW>::WGS_PER_CU)))
void dkdv_pipe_kernel(BwdArgs a) {
  __shared__ __attribute__((aligned(16))) half_t lds[DkdvPipeTile<D, NW>::LDS_HALVES];
  dkdv_pipe_body<D, CAUSAL, NW, E>(a, blockIdx.x, lds);
}

template <int D, bool CAUSAL, int NW, class E = F16>
hipError_t dkdv_pipe_launch(const BwdArgs& a, hipStream_t stream) {
  using T = DkdvPipeTile<D, NW>;
  BwdArgs b = a;
  b.num_tiles = (a.Nkv + T::BKV - 1) / T::BKV;
  if (b.nsplit < 1 || (b.nsplit > 1 && b.part == nullptr)) return hipErrorInvalidValue;
  const int64_t blocks = (int64_t)b.num_tiles * a.BHkv * b.nsplit;
  if (blocks <= 0 || blocks > 0x7fffffff) return hipErrorInvalidConfiguration;
  hipLaunchKernelGGL((dkdv_pipe_kernel<D, CAUSAL, NW, E>), dim3((unsigned)blocks), dim3(T::NT), 0,
                     stream, b);
  return hipGetLastError();
}

// --------------------------------------------------------------------------
// dQ
//
// Work-group: NW waves x 32 queries (Q, dO resident in VGPRs as B operands,
// LSE / Delta one per lane). Streams 64-key tiles (K, V row-major, swizzled)
// through a 3-slot DMA ring. Per 32-key block:
//   S^T = K fp16(c Q)^T, dP^T = V dO^T       (row reads, result: lane = query)
//   P^T = exp2(S^T - LSE), dS^T = P^T (dP^T - Delta)
//   dQ^T += K^T dS^T                          (K^T via transposing reads)
// --------------------------------------------------------------------------
template <int D, int NW, int KT>
struct DqTile {
  static constexpr int BQ = 32 * NW;  // queries per work-group
  static constexpr int NT = 64 * NW;
  static constexpr int TILE = KT * D;
  static constexpr int STAGE = 2 * TILE;  // K tile, V tile
  static constexpr int NSTAGE = 3;
  static constexpr int AHEAD = NSTAGE - 1;
  static_assert(KT % 32 == 0, "key tile must be a multiple of 32");
};

template <int D, int NW, int KT>
constexpr bool dq_tiling_ok() {
  return (KT * D * 2) % 1024 == 0 && ((KT * D * 2) / 1024) % NW == 0 &&
         3 * (2 * KT * D) * 2 <= 160 * 1024;
}

template <int D, bool CAUSAL, int NW, int KT, class E = F16>
__global__ __launch_bounds__(64 * NW) void dq_kernel(BwdArgs a) {
  using T = DqTile<D, NW, KT>;
  using Dma = DmaStager<D, KT, NW>;
  constexpr int NB = KT / 32;
  constexpr int IPT = 2 * Dma::PER_WAVE;
  __shared__ __attribute__((aligned(16))) half_t lds[T::NSTAGE * T::STAGE];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int ql = lane & 31;
  const int g = lane >> 5;

  // Split mode: the split index is the slowest-varying part of the block index.
  const int split = blockIdx.x / (a.num_tiles * a.BH);
  const TileHead th =
      decode_block_grouped(blockIdx.x - split * a.num_tiles * a.BH, a.BH, a.group);
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
  const int4v rk = make_rsrc_words(a.k + (int64_t)kvh * Nkv * D, kv_slab);
  const int4v rv = make_rsrc_words(a.v + (int64_t)kvh * Nkv * D, kv_slab);

  const int q0 = qtile * T::BQ;
  const int q0w = q0 + 32 * wave;
  const int qrow = q0w + ql;

  // fp16(c Q) (the reference's q_scaled, attention.py:515) and dO as B operands.
  half8 qf[D / 16], dof[D / 16];
#pragma unroll
  for (int kk = 0; kk < D / 16; ++kk) {
    const uint32_t off = (uint32_t)(qrow * D + 16 * kk + 8 * g) * 2u;
    qf[kk] = __builtin_bit_cast(half8, buf_load_b128(rq, off));
    dof[kk] = __builtin_bit_cast(half8, buf_load_b128(rdo, off));
  }
  const float lse = buf_load_f32(rl, (uint32_t)qrow * 4u);
  const float delta = buf_load_f32(rd, (uint32_t)qrow * 4u);
  wait_all_vm();
#pragma unroll
  for (int kk = 0; kk < D / 16; ++kk) {
#pragma unroll
    for (int e = 0; e < 8; ++e) qf[kk][e] = to_elem<E>(a.c * elem_to_f32<E>(qf[kk][e]));
    asm volatile("" : "+v"(qf[kk]));
  }

  const int kv_end = CAUSAL ? min(Nkv, q0 + T::BQ) : Nkv;
  // This work-group's keys [kv_lo, kv_hi): all of [0, kv_end) unless split.
  const int kv_lo = split * a.split_keys;
  const int kv_hi = min(kv_end, kv_lo + a.split_keys);
  const int ntiles = kv_hi > kv_lo ? (kv_hi - kv_lo + KT - 1) / KT : 0;

  Dma dma;
  dma.init(wave, lane);
  auto issue_tile = [&](int t, int slot) {
    const half_t* base = lds + slot * T::STAGE;
    dma.issue(rk, kv_lo + t * KT, base, wave);
    dma.issue(rv, kv_lo + t * KT, base + T::TILE, wave);
  };
#pragma unroll
  for (int t = 0; t < T::AHEAD; ++t) issue_tile(t, t);

  int r_off[D / 16];
#pragma unroll
  for (int kk = 0; kk < D / 16; ++kk) r_off[kk] = swz_offset<D>(row_perm(ql), 2 * kk + g);
  int t_off[D / 32][2];
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

  // dQ^T accumulator: lane (query ql), rows d = 32*db + 8*(j/4) + 4*g + j%4.
  float16v dq[D / 32];
#pragma unroll
  for (int db = 0; db < D / 32; ++db)
#pragma unroll
    for (int j = 0; j < 16; ++j) dq[db][j] = 0.f;

  const float nl = -lse;

  auto step = [&](auto slot_c, int t) {
    constexpr int SLOT = decltype(slot_c)::value;
    issue_tile(t + T::AHEAD, (SLOT + T::AHEAD) % T::NSTAGE);
    const int kt0 = kv_lo + t * KT;
    const half_t* Ks = lds + SLOT * T::STAGE;
    const half_t* Vs = Ks + T::TILE;
    bool act[NB];
    float16v s[NB], dp[NB];
#pragma unroll
    for (int kb = 0; kb < NB; ++kb) {
      const int ka = kt0 + 32 * kb;
      act[kb] = q0w < N && ka < kv_hi && !(CAUSAL && ka > q0w + 31);
      if (act[kb]) {
#pragma unroll
        for (int j = 0; j < 16; ++j) {
          s[kb][j] = 0.f;
          dp[kb][j] = 0.f;
        }
#pragma unroll
        for (int kk = 0; kk < D / 16; ++kk) {
          const int off = 32 * kb * D + r_off[kk];
          s[kb] = mma<E>(*reinterpret_cast<const half8*>(Ks + off), qf[kk], s[kb]);
          dp[kb] = mma<E>(*reinterpret_cast<const half8*>(Vs + off), dof[kk], dp[kb]);
        }
      }
    }
#pragma unroll
    for (int kb = 0; kb < NB; ++kb) {
      if (!act[kb]) continue;
      const int ka = kt0 + 32 * kb;
      half8 kt_f[2][D / 32];
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int db = 0; db < D / 32; ++db) kt_f[h][db] = tr8(Ks + (32 * kb + 16 * h) * D, db);
      const bool need_mask = (CAUSAL && ka + 31 > q0w) || (ka + 32 > kv_hi);
      half8 sa[2];
#pragma unroll
      for (int j = 0; j < 16; ++j) {
        float pj = exp2_fast(s[kb][j] + nl);
        if (need_mask) {
          const int key = ka + result_row(j, g);
          if (key >= kv_hi || (CAUSAL && key > qrow)) pj = 0.f;
        }
        sa[j >> 3][j & 7] = to_elem<E>(pj * (dp[kb][j] - delta));
      }
#pragma unroll
      for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int db = 0; db < D / 32; ++db) dq[db] = mma<E>(kt_f[h][db], sa[h], dq[db]);
    }
    wait_vm_and_barrier<(T::AHEAD - 1) * IPT>();
  };

  wait_vm_and_barrier<(T::AHEAD - 1) * IPT>();
  for (int t = 0; t < ntiles; t += T::NSTAGE) {
    step(ic<0>{}, t);
    if (t + 1 >= ntiles) break;
    step(ic<1>{}, t + 1);
    if (t + 2 >= ntiles) break;
    step(ic<2>{}, t + 2);
  }
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");

  const rsrc_t rdq = make_rsrc(a.dq + (int64_t)head * N * D, slab);
  store_dq<D, E>(a, rdq, split, head, qrow, dq, a.scale);
}

template <int D, bool CAUSAL, int NW, int KT, class E = F16>
hipError_t dq_launch(const BwdArgs& a, hipStream_t stream) {
  using T = DqTile<D, NW, KT>;
  BwdArgs b = a;
  b.num_tiles = (a.N + T::BQ - 1) / T::BQ;
  if (b.nsplit < 1 || (b.nsplit > 1 && b.part == nullptr) || b.split_keys % 128 != 0 ||
      (int64_t)b.nsplit * b.split_keys < visible_kv<CAUSAL>(a))
    return hipErrorInvalidValue;
  const int64_t blocks = (int64_t)b.num_tiles * a.BH * b.nsplit;
  if (blocks <= 0 || blocks > 0x7fffffff) return hipErrorInvalidConfiguration;
  hipLaunchKernelGGL((dq_kernel<D, CAUSAL, NW, KT, E>), dim3((unsigned)blocks), dim3(T::NT), 0,
                     stream, b);
  return hipGetLastError();
}

// One work-group of dq_pipe_body per block.
template <int D, bool CAUSAL, int NW, class E = F16, bool TAIL = true>
__global__ __launch_bounds__(64 * NW)
__attribute__((amdgpu_waves_per_eu(DqPipeTile<D, NW>::WGS_PER_CU)))
void dq_pipe_kernel(BwdArgs a) {
  using T = DqPipeTile<D, NW>;
  __shared__ __attribute__((aligned(16))) half_t lds[T::NSTAGE * T::STAGE];
  dq_pipe_body<D, CAUSAL, NW, E, TAIL>(a, blockIdx.x, lds);
}

template <int D, bool CAUSAL, int NW, class E = F16>
hipError_t dq_pipe_launch(const BwdArgs& a, hipStream_t stream) {
  using T = DqPipeTile<D, NW>;
  BwdArgs b = a;
  b.num_tiles = (a.N + T::BQ - 1) / T::BQ;
  if (b.nsplit < 1 || (b.nsplit > 1 && b.part == nullptr) || b.split_keys % 128 != 0 ||
      (int64_t)b.nsplit * b.split_keys < visible_kv<CAUSAL>(a))
    return hipErrorInvalidValue;
  const int64_t blocks = (int64_t)b.num_tiles * a.BH * b.nsplit;
  if (blocks <= 0 || blocks > 0x7fffffff) return hipErrorInvalidConfiguration;
  if (dq_tail_free(b, CAUSAL))
    hipLaunchKernelGGL((dq_pipe_kernel<D, CAUSAL, NW, E, false>), dim3((unsigned)blocks),
                       dim3(T::NT), 0, stream, b);
  else
    hipLaunchKernelGGL((dq_pipe_kernel<D, CAUSAL, NW, E, true>), dim3((unsigned)blocks),
                       dim3(T::NT), 0, stream, b);
  return hipGetLastError();
}

// The pipelined dK/dV launch with the 16x16x32 body (fa_bwd_pipe16.hpp, D <= 64).
// At D = 32 without the mask the fp16 body fits three waves per SIMD (164
// VGPRs, no spills; the ring leaves room for three work-groups per CU): B4 H16
// N4000 bidirectional 299.4 -> 286.4 us on MI355X (two vs three, interleaved).
// The bf16 body would spill (20 bytes per lane) and under the mask three would
// spill as well, so those keep two.
template <int D, bool CAUSAL, class E>
constexpr int dkdv16_waves_per_simd() {
  return D == 32 && !CAUSAL && std::is_same_v<E, F16> ? 3 : DkdvPipeTile<D, 4>::WGS_PER_CU;
}
static_assert(3 * DkdvPipeTile<32, 4>::LDS_HALVES * 2 <= 160 * 1024,
              "three D = 32 dK/dV work-groups fit one CU's LDS");

template <int D, bool CAUSAL, int NW, class E = F16>
__global__ __launch_bounds__(64 * NW)
__attribute__((amdgpu_waves_per_eu(NW == 4 ? dkdv16_waves_per_simd<D, CAUSAL, E>()
                                           : DkdvPipeTile<D, NW>::WGS_PER_CU)))
void dkdv_pipe16_kernel(BwdArgs a) {
  __shared__ __attribute__((aligned(16))) half_t lds[DkdvPipeTile<D, NW>::LDS_HALVES];
  dkdv_pipe16_body<D, CAUSAL, NW, E>(a, blockIdx.x, lds);
}

template <int D, bool CAUSAL, int NW, class E = F16>
hipError_t dkdv_pipe16_launch(const BwdArgs& a, hipStream_t stream) {
  using T = DkdvPipeTile<D, NW>;
  BwdArgs b = a;
  b.num_tiles = (a.Nkv + T::BKV - 1) / T::BKV;
  if (b.nsplit < 1 || (b.nsplit > 1 && b.part == nullptr)) return hipErrorInvalidValue;
  const int64_t blocks = (int64_t)b.num_tiles * a.BHkv * b.nsplit;
  if (blocks <= 0 || blocks > 0x7fffffff) return hipErrorInvalidConfiguration;
  hipLaunchKernelGGL((dkdv_pipe16_kernel<D, CAUSAL, NW, E>), dim3((unsigned)blocks), dim3(T::NT),
                     0, stream, b);
  return hipGetLastError();
}

// The same dQ launch with the 16x16x32 body (fa_bwd_pipe16.hpp, D <= 64).
template <int D, bool CAUSAL, int NW, class E = F16, bool TAIL = true>
__global__ __launch_bounds__(64 * NW)
__attribute__((amdgpu_waves_per_eu(DqPipeTile<D, NW>::WGS_PER_CU)))
void dq_pipe16_kernel(BwdArgs a) {
  using T = DqPipeTile<D, NW>;
  __shared__ __attribute__((aligned(16))) half_t lds[T::NSTAGE * T::STAGE];
  dq_pipe16_body<D, CAUSAL, NW, E, TAIL>(a, blockIdx.x, lds);
}

template <int D, bool CAUSAL, int NW, class E = F16>
hipError_t dq_pipe16_launch(const BwdArgs& a, hipStream_t stream) {
  using T = DqPipeTile<D, NW>;
  BwdArgs b = a;
  b.num_tiles = (a.N + T::BQ - 1) / T::BQ;
  if (b.nsplit < 1 || (b.nsplit > 1 && b.part == nullptr) || b.split_keys % 128 != 0 ||
      (int64_t)b.nsplit * b.split_keys < visible_kv<CAUSAL>(a))
    return hipErrorInvalidValue;
  const int64_t blocks = (int64_t)b.num_tiles * a.BH * b.nsplit;
  if (blocks <= 0 || blocks > 0x7fffffff) return hipErrorInvalidConfiguration;
  if (dq_tail_free(b, CAUSAL))
    hipLaunchKernelGGL((dq_pipe16_kernel<D, CAUSAL, NW, E, false>), dim3((unsigned)blocks),
                       dim3(T::NT), 0, stream, b);
  else
    hipLaunchKernelGGL((dq_pipe16_kernel<D, CAUSAL, NW, E, true>), dim3((unsigned)blocks),
                       dim3(T::NT), 0, stream, b);
  return hipGetLastError();
}

template <int D, bool CAUSAL, int NW, int TILE, class E = F16>
constexpr void* dkdv_entry() {
  if constexpr (dkdv_tiling_ok<D, NW, TILE>())
    return (void*)&dkdv_launch<D, CAUSAL, NW, TILE, E>;
  else
    return nullptr;
}
template <int D, bool CAUSAL, int NW, int TILE, class E = F16>
constexpr void* dkdv_pipe_entry() {
  static_assert(TILE == 32, "the pipelined dK/dV kernel streams 32-query units");
  if constexpr (dkdv_pipe_tiling_ok<D, NW>())
    return (void*)&dkdv_pipe_launch<D, CAUSAL, NW, E>;
  else
    return nullptr;
}
template <int D, bool CAUSAL, int NW, int TILE, class E = F16>
constexpr void* dkdv_pipe16_entry() {
  static_assert(TILE == 32, "the pipelined dK/dV kernel streams 32-query units");
  if constexpr (D <= 64 && dkdv_pipe_tiling_ok<D, NW>())
    return (void*)&dkdv_pipe16_launch<D, CAUSAL, NW, E>;
  else
    return nullptr;
}
template <int D, bool CAUSAL, int NW, int TILE, class E = F16>
constexpr void* dq_pipe_entry() {
  static_assert(TILE == 32, "the pipelined dQ kernel streams 32-key units");
  if constexpr (dq_pipe_tiling_ok<D, NW>())
    return (void*)&dq_pipe_launch<D, CAUSAL, NW, E>;
  else
    return nullptr;
}
template <int D, bool CAUSAL, int NW, int TILE, class E = F16>
constexpr void* dq_pipe16_entry() {
  static_assert(TILE == 32, "the pipelined dQ kernel streams 32-key units");
  if constexpr (D <= 64 && dq_pipe_tiling_ok<D, NW>())
    return (void*)&dq_pipe16_launch<D, CAUSAL, NW, E>;
  else
    return nullptr;
}
template <int D, bool CAUSAL, int NW, int TILE, class E = F16>
constexpr void* dq_entry() {
  if constexpr (dq_tiling_ok<D, NW, TILE>())
    return (void*)&dq_launch<D, CAUSAL, NW, TILE, E>;
  else
    return nullptr;
}

// FA_BWD_VARIANT_BF also compiles the tiling for bf16; bf16 is compiled only
// for the tilings the default table uses, to bound the build.
#define FA_BWD_VARIANT(ENTRY, NW, TILE, FLAGS) \
  {NW, 32 * NW, TILE, {FA_ENTRIES(ENTRY, F16, NW, TILE), FA_NO_ENTRIES}, FLAGS}
#define FA_BWD_VARIANT_BF(ENTRY, NW, TILE, FLAGS) \
  {NW, 32 * NW, TILE, {FA_ENTRIES(ENTRY, F16, NW, TILE), FA_ENTRIES(ENTRY, BF16, NW, TILE)}, FLAGS}

static const Variant kDkdvVariants[] = {
    FA_BWD_VARIANT(dkdv_entry, 4, 64, 0),
    FA_BWD_VARIANT_BF(dkdv_entry, 4, 32, 0),
    FA_BWD_VARIANT(dkdv_entry, 2, 64, 0),
    FA_BWD_VARIANT(dkdv_entry, 8, 64, 0),
    FA_BWD_VARIANT_BF(dkdv_pipe_entry, 4, 32, kPairs),
    FA_BWD_VARIANT_BF(dkdv_pipe16_entry, 4, 32, 0),
};

static const Variant kDqVariants[] = {
    FA_BWD_VARIANT(dq_entry, 4, 64, 0),
    FA_BWD_VARIANT_BF(dq_entry, 4, 32, 0),
    FA_BWD_VARIANT(dq_entry, 2, 64, 0),
    FA_BWD_VARIANT(dq_entry, 8, 64, 0),
    FA_BWD_VARIANT_BF(dq_pipe_entry, 4, 32, kFusesDelta | kPairs),
    FA_BWD_VARIANT_BF(dq_pipe16_entry, 4, 32, kFusesDelta),
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
