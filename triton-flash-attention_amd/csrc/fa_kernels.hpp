// fa_kernels.hpp — argument blocks and launcher registry shared by the
// kernel translation units and the C ABI (fa_capi.hip).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace fa {

typedef _Float16 half_t;

// 1 / ln(2): converts natural-log scores to the base-2 domain (attention.py:20).
constexpr float kLog2e = 1.4426950408889634f;

// A persistent causal forward's job plan (the launch takes it by value): the
// grid has ngroups * nbin work-groups; work-group s serves head group
// s % ngroups and runs the jobs job[start[b] .. start[b + 1]) of bin
// b = s / ngroups in order. A job is hoff * kTileLimit + qtile: query tile
// qtile of the head at tile-row position ngroups * hoff + s % ngroups.
struct FwdJobs {
  static constexpr int kMaxBins = 64;
  static constexpr int kMaxJobs = 256;
  static constexpr int kTileLimit = 1 << 16;
  int ngroups;
  int nbin;
  int start[kMaxBins + 1];
  int job[kMaxJobs];
};

// Arguments of one forward launch (the values _attn_fwd receives at
// attention.py:690-718, minus strides: every tensor is contiguous).
struct FwdArgs {
  const half_t* q;
  const half_t* k;
  const half_t* v;
  half_t* o;
  float* lse;
  int N;           // query sequence length
  int Nkv;         // key/value sequence length (== N for self-attention)
  int Hq, Hkv;     // query heads, key/value heads
  int group;       // Hq / Hkv
  int BH;          // B * Hq
  int num_tiles;   // filled in by the launcher
  float c;         // scale * log2(e)
  // Split-KV mode (nsplit > 1): work-group split s covers keys
  // [s * split_keys, (s + 1) * split_keys) and writes its fp32 partial O
  // ([nsplit, BH, N, D], normalised by its own row sums) and base-2 LSE
  // ([nsplit, BH, N], -inf where it saw no key) to `part`;
  // launch_fwd_combine merges them. The ranges together cover the keys some
  // query sees (visible_kv: all Nkv, or min(N, Nkv) under the causal mask).
  // nsplit = 1: split_keys >= Nkv, part unused.
  int nsplit;
  int split_keys;  // a multiple of 128
  float* part;
  // Query heads per work-group. 1: a work-group serves 32 * NW query rows of
  // one head. pack > 1 (GQA, pack dividing both the group and NW): it serves
  // 32 * NW / pack rows of `pack` consecutive query heads of one key/value
  // head, wave w taking head w % pack and rows 32 * (w / pack) onward, so the
  // heads share each K/V tile the work-group streams.
  int pack;
  // Host-side plan of the persistent forward variant (kJobs); its launcher
  // passes *jobs to the kernel by value. Unused by the other variants.
  const FwdJobs* jobs = nullptr;
};

// Arguments of the backward launches (attention.py:736-770).
struct BwdArgs {
  const half_t* q;
  const half_t* k;
  const half_t* v;
  const half_t* dO;
  const float* lse;
  const float* delta;
  half_t* dq;
  half_t* dk;
  half_t* dv;
  int N;           // query sequence length
  int Nkv;         // key/value sequence length (== N for self-attention)
  int Hq, Hkv, group;
  int BH;          // B * Hq
  int BHkv;        // B * Hkv
  int num_tiles;   // filled in by the launcher
  float c;         // scale * log2(e)
  float scale;
  // dK/dV split mode (nsplit > 1): work-group (tile, head, split) covers one
  // contiguous chunk of its key tile's (query head, query tile) steps and
  // writes fp32 partials part[split][B*Hkv][N][D] (dK then dV planes).
  int nsplit;
  float* part;
  // dQ split mode (nsplit > 1 in a dQ launch): work-group split s covers keys
  // [s * split_keys, (s + 1) * split_keys) and writes its fp32 partial dQ
  // (scaled) to part[split][B*Hq][N][D]; launch_split_sum adds them. The
  // ranges cover visible_kv keys; with nsplit = 1, split_keys >= Nkv. Unused
  // by the dK/dV launches.
  int split_keys;
  // Fused Delta (dQ kernels whose variant has kFusesDelta): when o is set the
  // kernel computes Delta = rowsum(O * dO) itself and writes it to delta_out
  // instead of reading delta.
  const half_t* o;
  float* delta_out;
};

// Keys some query can see, which a split launch's key ranges must cover: all
// Nkv, or under the top-left causal mask the first min(N, Nkv) (query i sees
// keys j <= i; the keys after them are masked for every query).
template <bool CAUSAL, class Args>
inline int64_t visible_kv(const Args& a) {
  return CAUSAL && a.N < a.Nkv ? a.N : a.Nkv;
}

enum KernelKind { kFwd = 0, kDkdv = 1, kDq = 2, kNumKinds = 3 };

typedef hipError_t (*fwd_launch_fn)(const FwdArgs&, hipStream_t);
typedef hipError_t (*bwd_launch_fn)(const BwdArgs&, hipStream_t);

// One compiled tiling of a kernel, for every (D, causal).
// rows = rows owned by a work-group (queries for fwd/dq, keys for dkdv),
// tile = length of the streamed tile (keys for fwd/dq, queries for dkdv).
struct Variant {
  int waves;
  int rows;
  int tile;
  void* fn[2][3][2];  // [element type: fp16, bf16][D index: 32, 64, 128][causal]; null = not compiled
  int flags;          // kFusesDelta, kSplitsKv, kPairs, kKeyGroups, kJobs, kFewSplits
  int per_cu = 0;     // kJobs: work-groups resident per CU (the plan's slots per CU)
};

// Element type index of Variant::fn.
enum DType { kF16 = 0, kBF16 = 1 };

// The six launchers (D = 32, 64, 128; bidirectional, causal) of one tiling
// ENTRY<D, causal, args..., E>(), and an empty table.
#define FA_ENTRIES(ENTRY, E, ...)                                              \
  {{ENTRY<32, false, __VA_ARGS__, E>(), ENTRY<32, true, __VA_ARGS__, E>()},    \
   {ENTRY<64, false, __VA_ARGS__, E>(), ENTRY<64, true, __VA_ARGS__, E>()},    \
   {ENTRY<128, false, __VA_ARGS__, E>(), ENTRY<128, true, __VA_ARGS__, E>()}}
#define FA_NO_ENTRIES {{nullptr, nullptr}, {nullptr, nullptr}, {nullptr, nullptr}}

// The dQ variant can compute Delta itself (BwdArgs::o / delta_out).
constexpr int kFusesDelta = 1;
// The forward variant has the split-KV mode (FwdArgs::nsplit > 1).
constexpr int kSplitsKv = 2;
// The backward variant (pipelined dK/dV or dQ, D <= 64) also runs in the
// combined launch of bwd_pair_launcher.
constexpr int kPairs = 4;
// The forward variant splits each work-group's keys over two wave groups
// (one query head per work-group: no packed GQA).
constexpr int kKeyGroups = 8;
// The forward variant runs a causal one-pass launch as a persistent grid when
// the host attaches a job plan (FwdArgs::jobs), else as the grid form.
constexpr int kJobs = 16;
// The forward variant's split-KV launches at D >= 64 aim at one work-group per
// CU (fewer, longer key ranges) instead of three.
constexpr int kFewSplits = 32;

// Most key ranges a split-KV forward uses; its merge holds one partial per
// range in registers.
constexpr int kMaxFwdSplitKv = 32;

// Registries defined in the kernel translation units.
const Variant* fwd_variants(int* count);
const Variant* dkdv_variants(int* count);
const Variant* dq_variants(int* count);

// Combined dK/dV + dQ launch (fa_bwd_pair.hip): `dkdv` as for the pipelined
// dK/dV launch (split mode allowed), `dq` as for the pipelined dQ launch in one
// pass that reads Delta (o == nullptr). Null for head sizes other than 32, 64.
typedef hipError_t (*bwd_pair_launch_fn)(const BwdArgs& dkdv, const BwdArgs& dq, hipStream_t);
bwd_pair_launch_fn bwd_pair_launcher(int dtype, int di, int causal);
// Waves per work-group of the combined launch (both kinds' tiling).
int bwd_pair_waves();

// Sum of the nsplit fp32 partial planes into fp16 dK, dV (fixed order).
// dtype: kF16 or kBF16 (the element type of the 16-bit tensors).
hipError_t launch_split_reduce(const float* part, half_t* dk, half_t* dv, int64_t plane_elems,
                               int nsplit, int dtype, hipStream_t stream);

hipError_t launch_preprocess(const half_t* o, const half_t* dO, float* delta, int64_t rows,
                             int D, int dtype, hipStream_t stream);

// Sum of nsplit fp32 partial planes of `elems` values into 16-bit `out`.
hipError_t launch_split_sum(const float* part, half_t* out, int64_t elems, int nsplit, int dtype,
                            hipStream_t stream);

// Merge of the forward's nsplit partials (FwdArgs::part) into O (16-bit) and
// base-2 LSE, rows = B * Hq * N: O = sum_s w_s O_s / sum_s w_s with
// w_s = exp2(lse_s - max_s lse_s), LSE = max + log2(sum_s w_s).
hipError_t launch_fwd_combine(const float* part, half_t* o, float* lse, int64_t rows, int D,
                              int nsplit, int dtype, hipStream_t stream);

inline int head_dim_index(int64_t D) {
  return D == 32 ? 0 : D == 64 ? 1 : D == 128 ? 2 : -1;
}

}  // namespace fa
