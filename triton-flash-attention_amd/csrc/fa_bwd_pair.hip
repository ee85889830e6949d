// fa_bwd_pair.hip — the backward's dK/dV and dQ work-groups in one launch
// (gfx950, head_dim 32 and 64).
//
// A backward whose dK/dV launch has too few key tiles to fill the GPU splits
// that launch's query steps into chunks (fp32 partials, summed afterwards by
// launch_split_reduce). Such a shape also gives its dQ launch few
// work-groups, and under the causal mask both launches end in a tail where
// their longest work-groups run on an otherwise idle GPU. bwd_pair_kernel
// runs both sets of work-groups as one grid, so each kind's tail is filled by
// the other's work and one launch boundary disappears. The two lists are dealt
// alternately (dK/dV, dQ, dK/dV, ...), each in its own launch order (longest
// first), and the longer list's remainder follows.
//
// dK/dV reads Delta, which the fused dQ variant would only produce during the
// same launch, so Delta comes from launch_preprocess beforehand and the dQ
// work-groups read it too (BwdArgs::o == nullptr). The bodies are the ones of
// dkdv_pipe_kernel and dq_pipe_kernel (fa_bwd_pipe.hpp); both run four waves
// at two work-groups per CU for D <= 64, so one occupancy serves both, and the
// LDS ring is the larger of the two.
//
// Reference counterpart: TritonAttention.backward launches the Delta
// preprocess and then one _attn_bwd grid (triton_flash_attention/
// attention.py:735-770) in which every program runs phase 1 (dK/dV of key
// block pid, 428-505) and then phase 2 (dQ of query block pid, 507-573).
// Here the phases are separate work-groups of one grid instead, so neither
// waits for the other inside a work-group.
#include "fa_bwd_pipe.hpp"
#include "fa_kernels.hpp"

namespace fa {

constexpr int kPairWaves = 4;

template <int D, bool CAUSAL, int NW, class E, bool TAIL>
__global__ __launch_bounds__(64 * NW)
__attribute__((amdgpu_waves_per_eu(DkdvPipeTile<D, NW>::WGS_PER_CU)))
void bwd_pair_kernel(BwdArgs ad, BwdArgs aq, unsigned n_dkdv, unsigned n_dq) {
  using TK = DkdvPipeTile<D, NW>;
  using TQ = DqPipeTile<D, NW>;
  static_assert(TK::WGS_PER_CU == TQ::WGS_PER_CU && TK::NT == TQ::NT,
                "both kinds run at one occupancy and work-group size");
  constexpr int kDqLds = TQ::NSTAGE * TQ::STAGE;
  constexpr int kLds = TK::LDS_HALVES > kDqLds ? TK::LDS_HALVES : kDqLds;
  __shared__ __attribute__((aligned(16))) half_t lds[kLds];
  const unsigned both = 2u * (n_dkdv < n_dq ? n_dkdv : n_dq);
  const unsigned i = blockIdx.x;
  const bool dq = i < both ? (i & 1u) != 0 : n_dq > n_dkdv;
  const unsigned idx = i < both ? i >> 1 : both / 2 + (i - both);
  if (dq)
    dq_pipe_body<D, CAUSAL, NW, E, TAIL>(aq, idx, lds);
  else
    dkdv_pipe_body<D, CAUSAL, NW, E>(ad, idx, lds);
}

template <int D, bool CAUSAL, class E>
hipError_t bwd_pair_launch(const BwdArgs& dkdv, const BwdArgs& dq, hipStream_t stream) {
  constexpr int NW = kPairWaves;
  using TK = DkdvPipeTile<D, NW>;
  using TQ = DqPipeTile<D, NW>;
  static_assert(dkdv_pipe_tiling_ok<D, NW>() && dq_pipe_tiling_ok<D, NW>(), "pipelined tilings");
  BwdArgs ad = dkdv;
  BwdArgs aq = dq;
  ad.num_tiles = (ad.Nkv + TK::BKV - 1) / TK::BKV;
  aq.num_tiles = (aq.N + TQ::BQ - 1) / TQ::BQ;
  if (ad.nsplit < 1 || (ad.nsplit > 1 && ad.part == nullptr) || ad.delta == nullptr)
    return hipErrorInvalidValue;
  // dQ in one pass over all keys, reading Delta (not computing it)
  if (aq.nsplit != 1 || aq.split_keys % 128 != 0 || aq.split_keys < aq.Nkv || aq.o != nullptr ||
      aq.delta == nullptr)
    return hipErrorInvalidValue;
  const int64_t nk = (int64_t)ad.num_tiles * ad.BHkv * ad.nsplit;
  const int64_t nq = (int64_t)aq.num_tiles * aq.BH;
  if (nk <= 0 || nq <= 0 || nk + nq > 0x7fffffff) return hipErrorInvalidConfiguration;
  if (dq_tail_free(aq, CAUSAL))
    hipLaunchKernelGGL((bwd_pair_kernel<D, CAUSAL, NW, E, false>), dim3((unsigned)(nk + nq)),
                       dim3(TK::NT), 0, stream, ad, aq, (unsigned)nk, (unsigned)nq);
  else
    hipLaunchKernelGGL((bwd_pair_kernel<D, CAUSAL, NW, E, true>), dim3((unsigned)(nk + nq)),
                       dim3(TK::NT), 0, stream, ad, aq, (unsigned)nk, (unsigned)nq);
  return hipGetLastError();
}

bwd_pair_launch_fn bwd_pair_launcher(int dtype, int di, int causal) {
  static const bwd_pair_launch_fn kTable[2][2][2] = {
      // [element type][D = 32, 64][causal]
      {{&bwd_pair_launch<32, false, F16>, &bwd_pair_launch<32, true, F16>},
       {&bwd_pair_launch<64, false, F16>, &bwd_pair_launch<64, true, F16>}},
      {{&bwd_pair_launch<32, false, BF16>, &bwd_pair_launch<32, true, BF16>},
       {&bwd_pair_launch<64, false, BF16>, &bwd_pair_launch<64, true, BF16>}},
  };
  if (dtype < 0 || dtype > 1 || di < 0 || di > 1) return nullptr;
  return kTable[dtype][di][causal ? 1 : 0];
}

int bwd_pair_waves() { return kPairWaves; }

}  // namespace fa
