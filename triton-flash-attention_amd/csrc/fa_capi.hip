// fa_capi.hip — extern "C" entry points of libfa_gfx950.so (declared in
// include/fa_gfx950.h). Argument checks happen here, before any HIP call, so
// an unsupported request never reaches the device; a rejected call returns a
// negative FA_ERR_* code and records a message for fa_last_error().
#include <float.h>
#include <math.h>
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <algorithm>
#include <atomic>
#include <initializer_list>
#include <memory>
#include <mutex>
#include <numeric>
#include <vector>

#include "../../include/fa_gfx950.h"
#include "fa_kernels.hpp"

// Device-resident scratch of fa_fwd_noalloc: the split-KV forward's fp32
// partials ([nsplit, B, Hq, N_q, D + 1]) for callers that cannot allocate.
// Every GPU the library runs on holds its own copy for the life of the
// process. This translation unit has no kernels, so with HIP's default
// deferred code-object loading the array is reserved on a GPU only when
// hipGetSymbolAddress first asks for it (the first fa_fwd_noalloc there). In host code `scratch` only names the symbol; its device address
// comes from hipGetSymbolAddress (scratch_address below), once per device.
constexpr int64_t kNoallocScratchBytes = (int64_t)64 << 20;
static __device__ __align__(256) float scratch[kNoallocScratchBytes / 4];

namespace {

thread_local char g_last_error[512] = "";

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_last_error, sizeof(g_last_error), fmt, ap);
  va_end(ap);
  return code;
}

int hip_result(hipError_t e, const char* what) {
  if (e == hipSuccess) {
    g_last_error[0] = '\0';
    return FA_OK;
  }
  return fail((int)e, "%s: %s (hipError %d)", what, hipGetErrorString(e), (int)e);
}

// hip_result for a launch of the entry point `name` ("<name> launch: ...").
int launch_result(hipError_t e, const char* name) {
  if (e == hipSuccess) return hip_result(e, name);
  return fail((int)e, "%s launch: %s (hipError %d)", name, hipGetErrorString(e), (int)e);
}

// Process-wide tiling choice per (kernel, D index, causal); -1 = table default.
// fa_set_tiling may run on one thread while others launch: every entry is an
// atomic, read once per tiling decision (relaxed: each entry is independent and
// every value stored is a valid choice), so a launch sees either the old or the
// new tiling, never a torn value. The array is zero-initialised and holds
// variant + 1, so 0 means "table default".
std::atomic<int> g_override_plus1[fa::kNumKinds][3][2];

int override_of(int kind, int di, int causal) {
  return g_override_plus1[kind][di][causal ? 1 : 0].load(std::memory_order_relaxed) - 1;
}

// Static tiling table (replaces the Triton autotuner). Values are variant
// indices into the registries of fa_fwd.hip / fa_bwd.hip, chosen from
// per-kernel sweeps on MI355X at the BASELINE shapes (D=32: N=16381 GQA;
// D=64: B4 H16 N4096; D=128: B2 H32 N8192):
//   fwd : 0 = 4 waves x 32 queries, 64-key tiles; 1 = 8 waves, 64; 2 = 4 waves, 32;
//         3 = 2 waves, 64; 4 = 4 waves, 128; 5 = 4 waves, 32-key units, software-
//         pipelined, 2 units per barrier (D <= 64); 6 = the same, 1 unit per
//         barrier and a 6-slot ring (three work-groups per CU); 7 = 8 waves, 32-key
//         units, pipelined, one work-group per CU (D = 128); 8 = 8 waves as two
//         4-wave groups that split the keys of 128 queries (D <= 64); 9 = tiling 6
//         run as a persistent grid of bin-packed jobs under the causal mask when
//         its job plan beats the grid's modelled tail (D <= 64; fwd_launch_plan;
//         measured slower than 6 at every shape where a plan forms, so the table
//         does not take it); 10 = tiling 6 on 16x16x32 MFMAs (D <= 64); 11 = 10
//         with 64-query work-groups (all D; select_fwd takes it for small causal
//         launches at D <= 64 and for decoding)
//         (not every variant exists for every D)
//   dkdv: 0 = 4 waves x 32 keys, 64-query tiles; 1 = 4 waves, 32; 2 = 2 waves, 64;
//         3 = 8 waves, 64; 4 = 4 waves, 32-query units, software-pipelined (all D;
//         D = 128 runs one work-group per CU with dK, dV in AGPRs); 5 = tiling 4 on
//         16x16x32 MFMAs (D <= 64; select_dkdv takes it at D = 64, and at D = 32
//         without the mask, when the launch does not split)
//   dq  : 0 = 4 waves x 32 queries, 64-key tiles; 1 = 4 waves, 32; 2 = 2 waves, 64;
//         3 = 8 waves, 64; 4 = 4 waves, 32-key units, software-pipelined (all D;
//         at D = 128 the classic 4 waves x 32 with its separate Delta pass stays
//         faster under the causal mask); 5 = tiling 4 on 16x16x32 MFMAs (D <= 64;
//         select_dq takes it for large launches at D = 64, and at D = 32 without
//         the mask)
const int kDefault[fa::kNumKinds][3][2] = {
    // D=32     D=64     D=128   (each: {bidirectional, causal})
    {{6, 6}, {6, 6}, {7, 7}},  // fwd
    {{4, 4}, {4, 4}, {4, 4}},  // dkdv
    {{4, 4}, {4, 4}, {4, 1}},  // dq
};

const fa::Variant* registry(int kind, int* count) {
  switch (kind) {
    case fa::kFwd:
      return fa::fwd_variants(count);
    case fa::kDkdv:
      return fa::dkdv_variants(count);
    case fa::kDq:
      return fa::dq_variants(count);
    default:
      *count = 0;
      return nullptr;
  }
}

// A variant is usable for (D, causal) when it was compiled for that head_dim.
// (bf16 is compiled for the default tilings only.)
bool usable(const fa::Variant& v, int di, int causal, int dt = fa::kF16) {
  return v.fn[dt][di][causal ? 1 : 0] != nullptr;
}

// The tiling used for (kind, D, causal, element type): the override if set,
// else the default; a bf16 call whose overridden tiling has no bf16 build
// uses the default tiling.
// `ov` is the override as read once by the caller (override_of).
const fa::Variant* select(int kind, int di, int causal, int ov, int* index, int dt = fa::kF16) {
  int count = 0;
  const fa::Variant* vs = registry(kind, &count);
  if (!vs) return nullptr;
  int v = ov;
  if (v < 0 || (v < count && !usable(vs[v], di, causal, dt))) v = kDefault[kind][di][causal ? 1 : 0];
  if (v >= count || !usable(vs[v], di, causal, dt)) return nullptr;
  if (index) *index = v;
  return &vs[v];
}

// select() with the override as it stands now.
const fa::Variant* select_current(int kind, int di, int causal, int* index, int dt = fa::kF16) {
  return select(kind, di, causal, override_of(kind, di, causal), index, dt);
}

// dQ tiling for a launch of N queries. Without the mask at D = 128 the table's
// pipelined kernel (one work-group per CU) is faster once the queries fill its
// 128-row tiles; with fewer (a short-query backward) the classic 4 waves x 32
// tiling, at two work-groups per CU, is (MI355X, B8 Hq32 Hkv8 against 8192
// keys: 16 queries 147 vs 177 us, 128 queries 251 vs 239 us). A tiling set
// with fa_set_tiling is used as set.
constexpr int kDqShortQueryVariant = 1;
// Under the causal mask at D = 128 the table takes that classic tiling: the
// pipelined kernel's single wave per SIMD idles at every diagonal tile, which
// costs more than its fused Delta pass saves once the launch has many
// work-groups (MI355X, one box, tiling sweep, classic vs pipelined: B2 H32
// N8192, 4096 work-groups of 128 queries, 1645 vs 1702 us; B4 H16 N4096, 2048,
// 442 vs 465 us; B4 H16 N2048, 1024, 135 vs 136 us). Smaller launches run the
// pipelined kernel: B1 H16 N4096, 512 work-groups, 147 vs 117 us; B1 H8 N8192,
// 512, 277 vs 218 us; B4 H16 N1024, 512, 50 vs 45 us; B4 H16 N512, 256, 28 vs
// 21 us.
constexpr int kDqPipelinedVariant = 4;
constexpr int64_t kDqPipelinedMaxWorkgroups = 768;
// Launches of more than 768 work-groups (more than the combined dK/dV + dQ
// launch takes, whose dQ body is tiling 4's) run the same pipeline on 16x16x32
// MFMAs (tiling 5) at D = 64, and at D = 32 without the mask. The chip holds a
// higher clock under them at its power limit (2.04 vs 1.70 GHz at B4 H16 N4096
// causal, rocprofv3). MI355X, dQ with Delta, tiling 4 vs 5, us: B4 H16 N4096
// bidirectional 359.8 vs 339.6, 379.3 vs 370.6, 409.4 vs 397.7 on three
// boxes; causal 198.6 vs 192.8 and 223.2 vs 225.8, and the whole causal
// training step with the 16x16x32 dK/dV 0.6567 vs 0.6518 and 0.6556 vs
// 0.6510 ms on two boxes; D = 32, B4 H16 N4096: bidirectional 214.9 vs 207.5,
// causal 119.3 vs 127.4 (B1 Hq8 Hkv2 N16381 causal 230.7 vs 234.6).
constexpr int kDq16Variant = 5;
constexpr int64_t kDq16MinWorkgroups = 769;

const fa::Variant* select_dq(int di, int causal, int64_t N, int64_t BH, int dt) {
  const int ov = override_of(fa::kDq, di, causal);
  const fa::Variant* var = select(fa::kDq, di, causal, ov, nullptr, dt);
  if (!var || ov >= 0) return var;
  int count = 0;
  const fa::Variant* vs = registry(fa::kDq, &count);
  auto pick = [&](int v) { return v < count && usable(vs[v], di, causal, dt) ? &vs[v] : var; };
  if (di != fa::head_dim_index(128)) {
    const bool take = (di == fa::head_dim_index(64) || !causal) &&
                      (N + 127) / 128 * BH >= kDq16MinWorkgroups;
    return take ? pick(kDq16Variant) : var;
  }
  if (!causal) return N < 128 ? pick(kDqShortQueryVariant) : var;
  if (N >= 128 && (N + 127) / 128 * BH <= kDqPipelinedMaxWorkgroups)
    return pick(kDqPipelinedVariant);
  return var;
}

// Forward tiling for a launch of N queries over BH query heads. At D = 128 the
// table's 8-wave pipelined kernel (256 queries per work-group, one per CU) is
// faster once the launch has long query sequences and enough work-groups; for
// short queries or small launches the 4-wave tiling is (MI355X, one box:
// B2 H32 N8192 causal 1091 vs 1181 us, bidirectional 1941 vs 2316 us; 512
// queries x 64 heads against 8192 keys 204 vs 218 us; 128 queries x 256 heads
// 270 vs 223 us; B1 H16 N1024 36 vs 33 us; decoding 2-6 % slower). A tiling
// set with fa_set_tiling is used as set.
constexpr int kFwdWideVariant = 7;
constexpr int kFwdNarrowVariant = 2;
// At D = 32 a causal launch over few heads (B*H * (query tiles + 1) < 1536)
// takes the two-key-group forward: 8 waves per work-group as two groups that
// split its keys, so a CU whose last long tiles run alone keeps twice the
// waves busy (MI355X, one box: B1 H8 N16381 217 vs 225 us, B2 H8 N4096 43.0
// vs 47.5 us; with launches that fill the GPU, B4 H16 N4096, and at D = 64,
// where it runs one work-group per CU, it is slower: 205 vs 164 us, B2 H16
// N2049 41 vs 34 us).
constexpr int kFwdKeyGroupVariant = 8;
// The other causal launches at D = 32 (from 512 queries) take tiling 6 on
// 16x16x32 MFMAs: the chip holds a higher clock under them at its power limit
// (MI355X, one box, tiling 6 vs 10, us: B4 H16 N4096 108.3 vs 102.0, B8 H16
// N2048 60.6 vs 57.8, B2 H16 N8192 200.2 vs 190.1, B16 H16 N1024 38.1 vs 36.5,
// B32 H16 N512 27.5 vs 25.9, B4 H16 N3072 64.4 vs 61.8). At D = 64 and
// without the mask the two are within a few percent either way.
constexpr int kFwd16Variant = 10;
// Causal launches at D <= 64 of 256-512 work-groups of 128 queries (W; 768
// would fill the GPU at three per CU) take tiling 10 with one 16-row query
// block per wave (tiling 11): 64 queries per work-group, so twice the
// work-groups, and half the MFMA and vector work per unit on the longest key
// loops. From W = 384 that fills the GPU; at W = 256 it still wins while the
// key loops are short (N <= 4096). MI355X, interleaved A/B, tiling 6 (D = 64)
// or the two-key-group tiling 8 (D = 32) against 11, us, two boxes: D = 64
// B1 H16 N2048 30.3 / 22.3 and 30.0 / 21.7, B1 H24 N2048 34.5 / 23.9, B1 H8
// N4096 45.7 / 38.6, B1 H12 N4096 49.4 / 43.2, B1 H16 N4096 53.5 / 48.1, B1 H8
// N8192 99.6 / 91.0, B1 H4 N16384 192.8 / 180.3, B1 H32 N2048 30.5 / 29.4;
// D = 32 B1 H16 N2048 24.8 / 18.3, B1 H24 N2048 28.5 / 18.5, B1 H16 N4096
// 43.0 / 38.9, B1 H8 N8192 72.5 / 68.2. Not taken: B1 H4 N8192 (W = 256)
// 72.0 / 78.1 at D = 64 and 46.3 / 61.2 at D = 32; c3 (W = 544) 30.6 / 31.7;
// W = 1024 10-22 % slower. Measured from 2048 queries; shorter launches (and
// decoding, where W counts heads only) keep the other rules.
constexpr int kFwd16HalfVariant = 11;
// Decoding (at most 32 queries; packed GQA: P = gcd(group, 4) heads per
// work-group) takes tiling 11 too while its 64 / P rows per head hold all the
// queries: the same K/V passes as the 128-query tilings with half their
// padding rows (at D = 128 against the 4-wave classic tiling 2, which short
// queries took before, with a 6-unit DMA ring in place of its staging).
// MI355X, interleaved, B8 Hq32 against 8192 keys, library vs 11, us: D = 64
// Hkv8 Nq 1 / 8 / 16 26.0 / 25.2, 27.8 / 26.3, 30.0 / 27.3; Hkv4 Nq 1 / 16
// 24.3 / 19.6, 28.6 / 22.1; Hkv16 Nq 32 52.6 / 51.8; Hkv32 Nq 1 98.6 / 96.9;
// D = 32 Hkv8 Nq 1 / 16 20.5 / 16.7, 23.0 / 18.2; Hkv32 Nq 32 55.9 / 47.1;
// D = 128 Hkv8 Nq 1 / 8 / 16 48.3 / 44.6, 49.8 / 48.2, 54.6 / 52.9, Hkv32
// Nq 1 199.7 / 186.9, Hkv16 Nq 32 124.5 / 117.2, B1 Hkv8 Nq 1 against 32768
// keys 31.4 / 27.2. With more queries than that (Hkv8 Nq 17, 32: two query
// tiles per head, twice the K/V passes) 10-17 % slower at D = 64.
constexpr int64_t kFwdDecodeQueries = 32;
// Without the mask, 33-64 queries (no packing: one 64-query work-group per
// head) take it as well; the 128-query tilings pad half or more of their rows.
// MI355X, interleaved, library (tiling 2 at D = 128, 6 below) vs 11, us:
// D = 128 B8 Hq32 Hkv8 against 8192 keys Nq 33 / 40 / 48 128.4 / 97.9,
// 129.8 / 97.6, 133.4 / 97.2; B1 Hq32 Hkv8 Nq 64 against 32768 keys 74.4 /
// 56.0 (bf16 74.8 / 56.2); B16 Hq32 Hkv8 Nq 64 against 4096 117.3 / 104.5;
// B8 Hq32 Hkv32 Nq 64 221.4 / 184.4; B2 H16 Nq 48 against 16384 52.5 / 47.5;
// D = 64 B16 Hq32 Hkv8 Nq 64 against 4096 70.0 / 50.5, B4 H16 Nq 40 against
// 16384 48.9 / 43.4, B8 Hq32 Hkv8 Nq 64 73.1 / 69.3, Nq 48 73.2 / 75.6;
// D = 32 B8 Hq32 Hkv8 Nq 48 / 64 59.3 / 39.4, 54.7 / 38.4. From 96 queries
// (two work-groups per head) 13-17 % slower; with 128 a tie.
constexpr int64_t kFwdShortQueries = 64;

int fwd_pack(const fa::Variant& var, int64_t group, int64_t N);  // below

const fa::Variant* select_fwd(int di, int causal, int64_t N, int64_t BH, int64_t group, int dt) {
  int index = -1;
  const int ov = override_of(fa::kFwd, di, causal);
  const fa::Variant* var = select(fa::kFwd, di, causal, ov, &index, dt);
  if (!var || ov >= 0) return var;
  int count = 0;
  const fa::Variant* vs = registry(fa::kFwd, &count);
  auto pick = [&](int v) {
    return v < count && usable(vs[v], di, causal, dt) ? &vs[v] : var;
  };
  if (N <= kFwdDecodeQueries || (!causal && N <= kFwdShortQueries)) {
    const fa::Variant* half = pick(kFwd16HalfVariant);
    if (half != var && N <= half->rows / fwd_pack(*half, group, N)) return half;
  }
  if (index == kFwdWideVariant) {
    if (N >= 512 && (N + var->rows - 1) / var->rows * BH >= 128) return var;
    return pick(kFwdNarrowVariant);
  }
  if (causal && di != fa::head_dim_index(128)) {
    const int64_t W = (N + 127) / 128 * BH;
    if (N >= 2048 && W <= 512 && (W >= 384 || (W >= 256 && N <= 4096)))
      return pick(kFwd16HalfVariant);
  }
  if (di == fa::head_dim_index(32) && causal && N > 32) {
    if (BH * ((N + 127) / 128 + 1) < 1536) return pick(kFwdKeyGroupVariant);
    if (N >= 512) return pick(kFwd16Variant);
  }
  return var;
}

int check_common(int64_t B, int64_t Hq, int64_t Hkv, int64_t N, int64_t D) {
  if (B <= 0 || Hq <= 0 || Hkv <= 0 || N <= 0)
    return fail(FA_ERR_BAD_SHAPE, "B, Hq, Hkv and N must be positive (got %lld, %lld, %lld, %lld)",
                (long long)B, (long long)Hq, (long long)Hkv, (long long)N);
  if (Hq % Hkv != 0)
    return fail(FA_ERR_BAD_SHAPE,
                "the number of query heads (%lld) must be divisible by the number of key/value "
                "heads (%lld)",
                (long long)Hq, (long long)Hkv);
  if (fa::head_dim_index(D) < 0)
    return fail(FA_ERR_HEAD_DIM, "head_dim must be one of (32, 64, 128); got %lld", (long long)D);
  // Per-head slabs are addressed with 32-bit byte offsets (buffer range check).
  if (N * D * 2 + 4096 * D * 2 >= ((int64_t)1 << 31))
    return fail(FA_ERR_TOO_LARGE, "sequence length %lld is too large for head_dim %lld",
                (long long)N, (long long)D);
  if (B * Hq >= ((int64_t)1 << 31) / 2)
    return fail(FA_ERR_TOO_LARGE, "batch * heads (%lld) is too large", (long long)(B * Hq));
  return FA_OK;
}

// The key/value length of the *_kv entry points (the same bounds as N).
int check_kv_length(int64_t Nkv, int64_t D) {
  if (Nkv <= 0) return fail(FA_ERR_BAD_SHAPE, "N_kv must be positive (got %lld)", (long long)Nkv);
  if (Nkv * D * 2 + 4096 * D * 2 >= ((int64_t)1 << 31))
    return fail(FA_ERR_TOO_LARGE, "key/value sequence length %lld is too large for head_dim %lld",
                (long long)Nkv, (long long)D);
  return FA_OK;
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

int check_aligned(const char* fn, std::initializer_list<const void*> ptrs) {
  for (const void* p : ptrs)
    if (!aligned16(p))
      return fail(FA_ERR_MISALIGNED, "%s: tensor pointer %p is not 16-byte aligned", fn, p);
  return FA_OK;
}

// The kernels fold c = scale * log2(e) into base-2 exponents and mask by
// setting scores to -inf before multiplying by c, so c must be a positive
// normal float32. Callers serve other finite scales exactly on top of this:
// a negative scale as -q at |scale| (dQ negated back), a zero (or subnormal)
// one as a zero q at scale 1 (dQ = 0).
int check_scale(float scale) {
  const float c = scale * fa::kLog2e;
  if (!isfinite(scale) || !isfinite(c) || !(c >= FLT_MIN))
    return fail(FA_ERR_BAD_SCALE,
                "scale must be finite and > 0 with scale * log2(e) a normal float32 (got %g)",
                (double)scale);
  return FA_OK;
}

fa::BwdArgs bwd_args(const fa_half_t* q, const fa_half_t* k, const fa_half_t* v,
                     const fa_half_t* dO, const float* lse, const float* delta, int64_t B,
                     int64_t Hq, int64_t Hkv, int64_t N, int64_t Nkv, float scale) {
  fa::BwdArgs a;
  a.q = reinterpret_cast<const fa::half_t*>(q);
  a.k = reinterpret_cast<const fa::half_t*>(k);
  a.v = reinterpret_cast<const fa::half_t*>(v);
  a.dO = reinterpret_cast<const fa::half_t*>(dO);
  a.lse = lse;
  a.delta = delta;
  a.dq = nullptr;
  a.dk = nullptr;
  a.dv = nullptr;
  a.N = (int)N;
  a.Nkv = (int)Nkv;
  a.Hq = (int)Hq;
  a.Hkv = (int)Hkv;
  a.group = (int)(Hq / Hkv);
  a.BH = (int)(B * Hq);
  a.BHkv = (int)(B * Hkv);
  a.num_tiles = 0;
  a.c = scale * fa::kLog2e;
  a.scale = scale;
  a.nsplit = 1;
  a.part = nullptr;
  a.split_keys = (int)((Nkv + 127) / 128 * 128);
  a.o = nullptr;
  a.delta_out = nullptr;
  return a;
}

// dK/dV split factor: key tiles x KV heads below ~3 work-groups per CU (GQA
// with few KV heads, or long causal sequences with few heads) split each key
// tile's step sequence (query head of the group x 32-query unit) into up to 16
// chunks that run as separate work-groups. Under the causal mask the first key
// tile carries about twice the mean work, and every tile is split into the
// same number of chunks, so its chunks set the end of the launch: causal
// launches with fewer than 384 work-groups aim at 4x as many (measured on
// MI355X, B1 Hq8 Hkv2 N16381 D32: 471 us at 768, 374 at 1536, 352 at 3072).
// Chunks keep at least 32 units on average, below which the partials and their
// sum cost more than the balance returns (B2 Hq16 Hkv4 N2049 D64: 64 us at 4
// chunks, 83 at 12).
constexpr int64_t kSplitTargetWorkgroups = 768;
constexpr int64_t kSplitTargetWorkgroupsCausal = 3072;
constexpr int64_t kMinSplitUnits = 32;
constexpr int kMaxSplit = 16;

// Chunks per key tile for a launch whose dK/dV work-groups, `wgs` unsplit,
// should number about `target` (at most 16 chunks, each with at least
// `min_units` 32-query units on average).
int64_t chunks_for(int64_t target, int64_t wgs, int64_t units, int64_t min_units) {
  int64_t s = (target + wgs - 1) / wgs;
  s = std::min<int64_t>(s, std::max<int64_t>(1, units / min_units));
  s = std::min<int64_t>(s, kMaxSplit);
  return std::max<int64_t>(s, 1);
}

// mean 32-query units per key tile: every query unit of the group (about
// half under the mask)
int64_t dkdv_tile_units(int64_t Hq, int64_t Hkv, int64_t N, int causal) {
  return (Hq / Hkv) * ((N + 31) / 32) / (causal ? 2 : 1);
}

int dkdv_split(const fa::Variant& var, int64_t B, int64_t Hq, int64_t Hkv, int64_t N,
               int64_t Nkv, int causal) {
  const int64_t tiles = (Nkv + var.rows - 1) / var.rows;
  const int64_t wgs = tiles * B * Hkv;
  if (wgs >= kSplitTargetWorkgroups) return 1;
  const int64_t target =
      causal && 2 * wgs < kSplitTargetWorkgroups ? kSplitTargetWorkgroupsCausal : kSplitTargetWorkgroups;
  return (int)chunks_for(target, wgs, dkdv_tile_units(Hq, Hkv, N, causal), kMinSplitUnits);
}

// dK/dV tiling for a launch. A launch that does not split runs the pipelined
// body on 16x16x32 MFMAs (tiling 5) at D = 64, and at D = 32 without the mask:
// the chip holds a higher clock under them at its power limit (1.99 vs 1.76
// GHz at B4 H16 N4096 causal, rocprofv3). MI355X, one box, dK/dV tiling 4 vs 5,
// us: B4 H16 N4096 causal 258.3 vs 246.1, bidirectional 484.8 vs 446.9; B8 H16
// N2048 causal 144.6 vs 140.6; D = 32 B4 H16 N4096 bidirectional 294.0 vs
// 273.6, causal 154.1 vs 158.7 (B1 Hq8 Hkv2 N16381 344.5 vs 338.1: too close
// to take). Launches that split keep tiling 4, whose body the combined dK/dV +
// dQ launch also runs (B2 Hq16 Hkv4 N2049 causal, split, 61.7 vs 62.7).
constexpr int kDkdv16Variant = 5;
// Short-query launches at D = 128 without the mask (at most 128 queries: each
// 128-key work-group sees only a few 32-query units, so its fixed cost of
// loading K/V and storing dK/dV dominates) run the classic 4 waves x 32
// tiling, which fits two waves per SIMD there (dkdv_classic_waves_per_simd,
// fa_bwd.hip): two work-groups per CU overlap one's loads with the other's
// work, where the pipelined kernel holds one. MI355X, one box, interleaved,
// tiling 4 vs 1, us: B8 Hq32 Hkv8 N_q 16 N_kv 8192 238.4 vs 206.1; B4 Hq32
// Hkv8 N_q 32 N_kv 8192 122.0 vs 103.9; B2 H16 N_q 64 N_kv 16384 214.3 vs
// 185.1; B16 Hq32 Hkv8 N_q 4 N_kv 4096 234.2 vs 204.8; B1 Hq32 Hkv8 N_q 128
// N_kv 32768 200.8 vs 195.3. Longer query loops favour the pipelined kernel:
// B1 Hq32 Hkv8 N_q 512 N_kv 16384 280.0 vs 306.8, B2 H32 N 8192 4186 vs 4692.
constexpr int kDkdvShortQueryVariant = 1;
constexpr int64_t kDkdvShortQueryMax = 128;

const fa::Variant* select_dkdv(int di, int causal, int64_t B, int64_t Hq, int64_t Hkv, int64_t N,
                               int64_t Nkv, int dt) {
  const int ov = override_of(fa::kDkdv, di, causal);
  const fa::Variant* var = select(fa::kDkdv, di, causal, ov, nullptr, dt);
  if (!var || ov >= 0) return var;
  int count = 0;
  const fa::Variant* vs = registry(fa::kDkdv, &count);
  auto pick = [&](int v) { return v < count && usable(vs[v], di, causal, dt) ? &vs[v] : var; };
  if (di == fa::head_dim_index(128))
    return !causal && N <= kDkdvShortQueryMax ? pick(kDkdvShortQueryVariant) : var;
  if (di != fa::head_dim_index(64) && (di != fa::head_dim_index(32) || causal)) return var;
  if (dkdv_split(*var, B, Hq, Hkv, N, Nkv, causal) != 1) return var;
  return pick(kDkdv16Variant);
}

int64_t split_workspace_bytes(int nsplit, int64_t B, int64_t Hkv, int64_t Nkv, int64_t D) {
  return nsplit > 1 ? (int64_t)nsplit * 2 * B * Hkv * Nkv * D * 4 : 0;
}

// Forward split-KV factor: launches with few work-groups (decoding: a few
// queries against a long key sequence, or few heads) split each work-group's
// keys into up to 32 ranges of at least 1024 keys (multiples of 128), run as
// separate work-groups, then merged (launch_fwd_combine). Swept on MI355X
// decoding shapes: ~3 work-groups per CU with long ranges beat more, shorter
// ones (partials and merge cost more than the extra parallelism returns).
constexpr int64_t kFwdSplitBelowWorkgroups = 512;
constexpr int64_t kFwdSplitTargetWorkgroups = 768;
// The 64-query forward (kFewSplits) decodes at D >= 64 faster with one
// work-group per CU than with three: its key ranges run quicker, so partials
// and the merge weigh more, and at D = 128 one work-group fills a CU (MI355X,
// interleaved, targets 768 vs 256, us: B32 Hq32 Hkv8 1 query against 2048
// keys D128 45.4 / 42.3 (no split, no merge), B8 Hq32 Hkv8 16 queries against
// 8192 keys 51.4 / 49.1, B2 Hq32 Hkv32 1 query against 16384 keys 98.6 / 93.7,
// B4 Hq16 Hkv16 1 query against 16384 keys D64 47.9 / 43.1; B8 Hq32 Hkv8 1
// query against 8192 keys D128 45.0 / 46.6; 384 is worse than both: 1.5
// rounds of work-groups). At D = 32 (half the bytes per key) three stay
// faster (16.2 vs 21.4 us at B8 Hq32 Hkv8 against 8192 keys).
constexpr int64_t kFwdSplitTargetFew = 256;
constexpr int64_t kFwdMinSplitKeys = 1024;
constexpr int kMaxFwdSplit = fa::kMaxFwdSplitKv;

struct FwdSplit {
  int nsplit;
  int split_keys;
};

// Query heads per forward work-group: GQA launches of at most 32 queries
// (decoding) pack gcd(group, waves) heads, which then share each K/V tile the
// work-group streams; otherwise 1.
int fwd_pack(const fa::Variant& var, int64_t group, int64_t N) {
  if (N > 32 || group < 2 || (var.flags & fa::kKeyGroups)) return 1;
  return (int)std::gcd<int64_t>(group, var.waves);
}

// Keys some query can see: all N_kv, or under the (top-left) causal mask the
// first min(N, N_kv), as query i sees keys j <= i.
int64_t visible_keys(int64_t N, int64_t Nkv, int causal) {
  return causal ? std::min<int64_t>(N, Nkv) : Nkv;
}

// Key split of a launch of `wgs` work-groups over Nkv keys (forward and dQ),
// aiming at about `target` work-groups. The ranges cover the `visible` keys
// (a multiple of 128 at least that many): under the mask with fewer queries
// than keys the rest are seen by no query, and ranges over them would only
// add empty work-groups and partials (B1 Hq32 Hkv8, 128 queries against 32768
// keys, D128, causal: 24 ranges, of which 23 were empty). A launch that does
// not split keeps the whole key range.
FwdSplit key_split(int64_t wgs, int64_t Nkv, int64_t visible, bool can_split,
                   int64_t target = kFwdSplitTargetWorkgroups) {
  const int whole = (int)((Nkv + 127) / 128 * 128);
  if (wgs >= kFwdSplitBelowWorkgroups || !can_split) return {1, whole};
  int64_t s = (target + wgs - 1) / wgs;
  s = std::min<int64_t>(s, std::max<int64_t>(1, visible / kFwdMinSplitKeys));
  s = std::min<int64_t>(s, kMaxFwdSplit);
  if (s <= 1) return {1, whole};
  const int64_t keys = ((visible + s - 1) / s + 127) / 128 * 128;
  return {(int)((visible + keys - 1) / keys), (int)keys};
}

FwdSplit fwd_split(const fa::Variant& var, int64_t B, int64_t Hq, int64_t N, int64_t Nkv,
                   int64_t D, int pack, int causal) {
  const int64_t rows = var.rows / pack;  // query rows per head and work-group
  const int64_t target = (var.flags & fa::kFewSplits) && D >= 64 ? kFwdSplitTargetFew
                                                                : kFwdSplitTargetWorkgroups;
  return key_split((N + rows - 1) / rows * B * Hq / pack, Nkv, visible_keys(N, Nkv, causal),
                   var.flags & fa::kSplitsKv, target);
}

// dQ: the same split of its key loop; the partials (fp32 dQ) are summed.
FwdSplit dq_split(const fa::Variant& var, int64_t B, int64_t Hq, int64_t N, int64_t Nkv,
                  int causal) {
  return key_split((N + var.rows - 1) / var.rows * B * Hq, Nkv, visible_keys(N, Nkv, causal),
                   true);
}

int64_t dq_workspace_bytes(const FwdSplit& sp, int64_t B, int64_t Hq, int64_t N, int64_t D) {
  return sp.nsplit > 1 ? (int64_t)sp.nsplit * B * Hq * N * D * 4 : 0;
}

int64_t fwd_workspace_bytes(const FwdSplit& sp, int64_t B, int64_t Hq, int64_t N, int64_t D) {
  return sp.nsplit > 1 ? (int64_t)sp.nsplit * B * Hq * N * (D + 1) * 4 : 0;
}

// ---- job plans of the persistent causal forward (variants with kJobs) ----
// Under the causal mask query tile t streams min(N_kv, (t + 1) * rows) keys,
// so the grid's work-groups differ in length. The grid deals them heaviest
// first to the resident slots (list scheduling), and a launch of a few slot
// rounds then ends with a tail: B4 H16 N4096 D64 has 2048 jobs of 4 .. 128
// 32-key units on 768 slots (256 CUs x 3), makespan 196 units against 176 if
// every slot got the same work. A plan instead gives each resident slot one
// bin of jobs, packed to equal sums (there: tile t with tile 42 - t of the
// same head, and the light tiles in groups). The plan is taken when its
// modelled makespan beats the grid's by kPlanMinGain. Measured on MI355X the
// persistent grid is the slower one wherever a plan forms (B4 H16 N4096 D64
// 172 vs 162 us, D32 124 vs 114 us, B1 H16 N16384 D64 616 vs 589 us; job
// overheads of 2, 6 and 12 units in the model change little), while the grid
// form's own tail there is about 5 % (B8 takes 1.90x, not 2x, the time of B4),
// so the table keeps the grid form and the plan variant stays a sweep option.
//
// Job cost model (32-key units): the units it streams plus kJobOverheadUnits
// for its fixed part (query fragments, ring fill, epilogue).
constexpr int kJobOverheadUnits = 2;
constexpr double kPlanMinGain = 0.03;
constexpr size_t kPlanCacheEntries = 64;

int64_t fwd_job_cost(int t, int64_t rows, int64_t Nkv) {
  const int64_t keys = std::min<int64_t>(Nkv, (t + 1) * rows);
  return (keys + 31) / 32 + kJobOverheadUnits;
}

// Makespan of the grid form: jobs in grid order (tile rank r -> query tile
// T - 1 - r, each over BH heads), each taken by the first slot to free up.
int64_t grid_makespan(int64_t T, int64_t BH, int64_t rows, int64_t Nkv, int64_t slots) {
  std::vector<int64_t> heap(std::max<int64_t>(1, slots), 0);  // min-heap of slot end times
  auto cmp = [](int64_t a, int64_t b) { return a > b; };
  for (int64_t r = 0; r < T; ++r) {
    const int64_t c = fwd_job_cost((int)(T - 1 - r), rows, Nkv);
    for (int64_t h = 0; h < BH; ++h) {
      std::pop_heap(heap.begin(), heap.end(), cmp);
      heap.back() += c;
      std::push_heap(heap.begin(), heap.end(), cmp);
    }
  }
  return *std::max_element(heap.begin(), heap.end());
}

// Best-fit decreasing of one head group's jobs (G heads x T tiles) into nbin
// bins of capacity cap: each job, heaviest first, goes to the fullest bin it
// still fits. Returns false when some job fits nowhere.
bool pack_bins(int64_t G, int64_t T, int64_t rows, int64_t Nkv, int nbin, int64_t cap,
               std::vector<std::vector<int>>* bins, int64_t* makespan) {
  std::vector<int64_t> load(nbin, 0);
  bins->assign(nbin, {});
  for (int64_t t = T - 1; t >= 0; --t) {  // costs fall with the tile index
    const int64_t c = fwd_job_cost((int)t, rows, Nkv);
    for (int64_t h = 0; h < G; ++h) {
      int best = -1;
      for (int b = 0; b < nbin; ++b)
        if (load[b] + c <= cap && (best < 0 || load[b] > load[best])) best = b;
      if (best < 0) return false;
      load[best] += c;
      (*bins)[best].push_back((int)(h * fa::FwdJobs::kTileLimit + t));
    }
  }
  *makespan = *std::max_element(load.begin(), load.end());
  return true;
}

struct PlanKey {
  int64_t N, Nkv, BH, rows, slots;  // slots: resident work-groups (CUs x per CU)
  bool operator==(const PlanKey& o) const {
    return N == o.N && Nkv == o.Nkv && BH == o.BH && rows == o.rows && slots == o.slots;
  }
};

// The plan for a causal one-pass launch of BH heads over N queries and N_kv
// keys on `slots` resident work-groups, or null where the grid form is as
// good (one slot round or less, no packing within the plan's size limits, or
// too small a gain). Head groups of G heads: ngroups = BH / G groups, each
// packed into nbin = slots * G / BH bins; G is the smallest that packs.
std::shared_ptr<const fa::FwdJobs> make_fwd_plan(const PlanKey& k) {
  const int64_t T = (k.N + k.rows - 1) / k.rows;
  if (T >= fa::FwdJobs::kTileLimit || T * k.BH <= k.slots) return nullptr;
  const int64_t grid = grid_makespan(T, k.BH, k.rows, k.Nkv, k.slots);
  int64_t head_cost = 0;
  for (int64_t t = 0; t < T; ++t) head_cost += fwd_job_cost((int)t, k.rows, k.Nkv);
  for (int64_t G = 1; G <= k.BH && G * T <= fa::FwdJobs::kMaxJobs; ++G) {
    if (k.BH % G) continue;
    const int64_t ngroups = k.BH / G;
    if (k.BH % 8 == 0 && ngroups % 8 != 0) continue;  // keep heads on their XCD
    const int64_t nbin = k.slots * G / k.BH;
    if (nbin < 1 || nbin > fa::FwdJobs::kMaxBins) continue;
    const int64_t total = G * head_cost;
    std::vector<std::vector<int>> bins;
    int64_t makespan = 0;
    bool packed = false;
    for (int64_t cap = (total + nbin - 1) / nbin; cap <= grid && !packed; ++cap)
      packed = pack_bins(G, T, k.rows, k.Nkv, (int)nbin, cap, &bins, &makespan);
    if (!packed) continue;
    if ((double)makespan > (1.0 - kPlanMinGain) * (double)grid) return nullptr;
    // Every job of the group exactly once.
    std::vector<int> seen(G * T, 0);
    for (const auto& bin : bins)
      for (int e : bin) ++seen[(e / fa::FwdJobs::kTileLimit) * T + e % fa::FwdJobs::kTileLimit];
    if (std::any_of(seen.begin(), seen.end(), [](int c) { return c != 1; })) return nullptr;
    auto plan = std::make_shared<fa::FwdJobs>();
    plan->ngroups = (int)ngroups;
    plan->nbin = (int)nbin;
    int n = 0;
    for (int b = 0; b < nbin; ++b) {
      plan->start[b] = n;
      for (int e : bins[b]) plan->job[n++] = e;
    }
    plan->start[nbin] = n;
    return plan;
  }
  return nullptr;
}

std::mutex g_plan_mu;
std::vector<std::pair<PlanKey, std::shared_ptr<const fa::FwdJobs>>> g_plans;

std::shared_ptr<const fa::FwdJobs> fwd_plan(const PlanKey& k) {
  std::lock_guard<std::mutex> lock(g_plan_mu);
  for (const auto& e : g_plans)
    if (e.first == k) return e.second;
  auto plan = make_fwd_plan(k);
  if (g_plans.size() >= kPlanCacheEntries) g_plans.erase(g_plans.begin());
  g_plans.emplace_back(k, plan);
  return plan;
}

// Compute units of the current device (cached per device).
int current_cu_count() {
  static std::mutex mu;
  static int cached[256] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 256) return 0;
  std::lock_guard<std::mutex> lock(mu);
  if (cached[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) n = 0;
    cached[dev] = n > 0 ? n : -1;
  }
  return cached[dev];
}

// The job plan a forward launch with tiling `var` runs on `cus` compute units
// (0: the current device's), or null for the grid form.
std::shared_ptr<const fa::FwdJobs> fwd_launch_plan(const fa::Variant& var, int causal, int pack,
                                                   int nsplit, int64_t BH, int64_t N,
                                                   int64_t Nkv, int cus = 0) {
  if (!(var.flags & fa::kJobs) || !causal || pack != 1 || nsplit != 1 || var.per_cu < 1)
    return nullptr;
  if (cus < 1) cus = current_cu_count();
  if (cus < 1) return nullptr;
  return fwd_plan({N, Nkv, BH, var.rows, (int64_t)cus * var.per_cu});
}


constexpr int kMaxScratchDevices = 256;
std::mutex g_scratch_mu;
void* g_scratch_addr[kMaxScratchDevices] = {};

// Device address of `scratch` on the current device, looked up on the first
// call on that device (with it current) and kept. The launch stream must
// belong to the current device, whose copy of the array the kernels get.
int scratch_address(const char* name, hipStream_t stream, void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return hip_result(e, name);
  if (stream != nullptr) {
    hipDevice_t sdev = -1;
    if ((e = hipStreamGetDevice(stream, &sdev)) != hipSuccess) return hip_result(e, name);
    if ((int)sdev != dev)
      return fail(FA_ERR_BAD_SHAPE, "%s: the stream belongs to device %d but device %d is "
                  "current; make the stream's device current", name, (int)sdev, dev);
  }
  if (dev < 0 || dev >= kMaxScratchDevices)
    return fail(FA_ERR_BAD_SHAPE, "%s: device index %d out of range", name, dev);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_addr[dev] == nullptr) {
    void* p = nullptr;
    if ((e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch))) != hipSuccess)
      return hip_result(e, name);
    g_scratch_addr[dev] = p;
  }
  *out = g_scratch_addr[dev];
  return FA_OK;
}

}  // namespace

extern "C" {

int fa_abi_version(void) { return FA_ABI_VERSION; }

const char* fa_last_error(void) { return g_last_error; }

// Argument checks of the forward entry points (no HIP call); on success *var
// is the selected tiling and *need the split workspace bytes (0: one pass).
static int fwd_check(int dt, const char* name, const fa_half_t* q, const fa_half_t* k,
                     const fa_half_t* v, fa_half_t* o, float* lse, int64_t B, int64_t Hq,
                     int64_t Hkv, int64_t N, int64_t Nkv, int64_t D, float scale, int causal,
                     const fa::Variant** var, int64_t* need) {
  if (!q || !k || !v || !o || !lse) return fail(FA_ERR_NULL_POINTER, "%s: null pointer", name);
  int rc = check_common(B, Hq, Hkv, N, D);
  if (rc) return rc;
  if ((rc = check_kv_length(Nkv, D))) return rc;
  if ((rc = check_aligned(name, {q, k, v, o, lse}))) return rc;
  if ((rc = check_scale(scale))) return rc;
  *var = select_fwd(fa::head_dim_index(D), causal, N, B * Hq, Hq / Hkv, dt);
  if (!*var) return fail(FA_ERR_BAD_TILING, "%s: no kernel for the selected tiling", name);
  const FwdSplit sp = fwd_split(**var, B, Hq, N, Nkv, D, fwd_pack(**var, Hq / Hkv, N), causal);
  *need = fwd_workspace_bytes(sp, B, Hq, N, D);
  return FA_OK;
}

static int fwd_impl(int dt, const char* name, const fa_half_t* q, const fa_half_t* k,
                    const fa_half_t* v, fa_half_t* o, float* lse, int64_t B, int64_t Hq,
                    int64_t Hkv, int64_t N, int64_t Nkv, int64_t D, float scale, int causal,
                    void* stream, void* workspace = nullptr, int64_t workspace_bytes = 0) {
  const fa::Variant* var = nullptr;
  int64_t need = 0;
  int rc = fwd_check(dt, name, q, k, v, o, lse, B, Hq, Hkv, N, Nkv, D, scale, causal, &var, &need);
  if (rc) return rc;
  fa::FwdArgs a;
  a.q = reinterpret_cast<const fa::half_t*>(q);
  a.k = reinterpret_cast<const fa::half_t*>(k);
  a.v = reinterpret_cast<const fa::half_t*>(v);
  a.o = reinterpret_cast<fa::half_t*>(o);
  a.lse = lse;
  a.N = (int)N;
  a.Nkv = (int)Nkv;
  a.Hq = (int)Hq;
  a.Hkv = (int)Hkv;
  a.group = (int)(Hq / Hkv);
  a.BH = (int)(B * Hq);
  a.num_tiles = 0;
  a.c = scale * fa::kLog2e;
  auto fn = reinterpret_cast<fa::fwd_launch_fn>(var->fn[dt][fa::head_dim_index(D)][causal ? 1 : 0]);
  hipStream_t s = static_cast<hipStream_t>(stream);
  a.pack = fwd_pack(*var, Hq / Hkv, N);
  const FwdSplit sp = fwd_split(*var, B, Hq, N, Nkv, D, a.pack, causal);
  a.nsplit = 1;
  a.split_keys = (int)((Nkv + 127) / 128 * 128);
  a.part = nullptr;
  if (need == 0 || workspace == nullptr) {
    const auto plan = fwd_launch_plan(*var, causal, a.pack, 1, B * Hq, N, Nkv);
    a.jobs = plan.get();
    return launch_result(fn(a, s), name);
  }
  if (workspace_bytes < need)
    return fail(FA_ERR_BAD_SHAPE, "%s: workspace of %lld bytes is smaller than the %lld bytes "
                "fa_fwd_workspace_bytes reports", name, (long long)workspace_bytes, (long long)need);
  if ((rc = check_aligned(name, {workspace}))) return rc;
  a.nsplit = sp.nsplit;
  a.split_keys = sp.split_keys;
  a.part = static_cast<float*>(workspace);
  hipError_t e = fn(a, s);
  if (e != hipSuccess) return launch_result(e, name);
  return launch_result(fa::launch_fwd_combine(a.part, a.o, lse, B * Hq * N, (int)D, sp.nsplit, dt, s),
                       name);
}

int64_t fa_fwd_workspace_bytes(int64_t B, int64_t Hq, int64_t Hkv, int64_t N_q, int64_t N_kv,
                               int64_t D, int causal) {
  int rc = check_common(B, Hq, Hkv, N_q, D);
  if (rc) return rc;
  if ((rc = check_kv_length(N_kv, D))) return rc;
  // Enough for either element type (their tilings can differ when overridden).
  int64_t bytes = 0;
  for (int dt : {fa::kF16, fa::kBF16}) {
    const fa::Variant* var = select_fwd(fa::head_dim_index(D), causal, N_q, B * Hq, Hq / Hkv, dt);
    if (!var) return fail(FA_ERR_BAD_TILING, "fa_fwd_workspace_bytes: no kernel for the selected tiling");
    const FwdSplit sp = fwd_split(*var, B, Hq, N_q, N_kv, D, fwd_pack(*var, Hq / Hkv, N_q), causal);
    bytes = std::max(bytes, fwd_workspace_bytes(sp, B, Hq, N_q, D));
  }
  return bytes;
}

int fa_fwd_plan_info(int64_t B, int64_t Hq, int64_t Hkv, int64_t N_q, int64_t N_kv, int64_t D,
                     int causal, int compute_units, int64_t* out4) {
  if (!out4) return fail(FA_ERR_NULL_POINTER, "fa_fwd_plan_info: null pointer");
  int rc = check_common(B, Hq, Hkv, N_q, D);
  if (rc) return rc;
  if ((rc = check_kv_length(N_kv, D))) return rc;
  const fa::Variant* var = select_fwd(fa::head_dim_index(D), causal, N_q, B * Hq, Hq / Hkv, fa::kF16);
  if (!var) return fail(FA_ERR_BAD_TILING, "fa_fwd_plan_info: no kernel for the selected tiling");
  const int pack = fwd_pack(*var, Hq / Hkv, N_q);
  const FwdSplit sp = fwd_split(*var, B, Hq, N_q, N_kv, D, pack, causal);
  const int64_t grid_wgs = (N_q + var->rows / pack - 1) / (var->rows / pack) * (B * Hq / pack);
  const auto plan = fwd_launch_plan(*var, causal, pack, sp.nsplit, B * Hq, N_q, N_kv,
                                    compute_units);
  out4[0] = plan ? (int64_t)plan->ngroups * plan->nbin : 0;
  out4[1] = grid_wgs * sp.nsplit;
  out4[2] = 0;
  out4[3] = 0;
  if ((var->flags & fa::kJobs) && causal && pack == 1 && sp.nsplit == 1) {
    const int cus = compute_units > 0 ? compute_units : current_cu_count();
    const int64_t slots = (int64_t)std::max(cus, 0) * var->per_cu;
    const int64_t T = (N_q + var->rows - 1) / var->rows;
    if (slots > 0) {
      out4[3] = grid_makespan(T, B * Hq, var->rows, N_kv, slots);
      if (plan) {
        int64_t worst = 0;
        for (int b = 0; b < plan->nbin; ++b) {
          int64_t sum = 0;
          for (int j = plan->start[b]; j < plan->start[b + 1]; ++j)
            sum += fwd_job_cost(plan->job[j] % fa::FwdJobs::kTileLimit, var->rows, N_kv);
          worst = std::max(worst, sum);
        }
        out4[2] = worst;
      }
    }
  }
  return FA_OK;
}

static int preprocess_impl(int dt, const char* name, const fa_half_t* o, const fa_half_t* dO,
                           float* delta, int64_t B, int64_t Hq, int64_t N, int64_t D,
                           void* stream) {
  if (!o || !dO || !delta) return fail(FA_ERR_NULL_POINTER, "%s: null pointer", name);
  int rc = check_common(B, Hq, 1, N, D);
  if (rc) return rc;
  if ((rc = check_aligned(name, {o, dO, delta}))) return rc;
  return launch_result(fa::launch_preprocess(reinterpret_cast<const fa::half_t*>(o),
                                          reinterpret_cast<const fa::half_t*>(dO), delta,
                                          B * Hq * N, (int)D, dt, static_cast<hipStream_t>(stream)),
                    name);
}

static int dkdv_impl(int dt, const char* name, const fa_half_t* q, const fa_half_t* k,
                     const fa_half_t* v, const fa_half_t* dO, const float* lse,
                     const float* delta, fa_half_t* dk, fa_half_t* dv, int64_t B, int64_t Hq,
                     int64_t Hkv, int64_t N, int64_t Nkv, int64_t D, float scale, int causal, void* stream) {
  if (!q || !k || !v || !dO || !lse || !delta || !dk || !dv)
    return fail(FA_ERR_NULL_POINTER, "%s: null pointer", name);
  int rc = check_common(B, Hq, Hkv, N, D);
  if (rc) return rc;
  if ((rc = check_kv_length(Nkv, D))) return rc;
  if ((rc = check_aligned(name, {q, k, v, dO, lse, delta, dk, dv}))) return rc;
  if ((rc = check_scale(scale))) return rc;
  const fa::Variant* var = select_dkdv(fa::head_dim_index(D), causal, B, Hq, Hkv, N, Nkv, dt);
  if (!var) return fail(FA_ERR_BAD_TILING, "%s: no kernel for the selected tiling", name);
  fa::BwdArgs a = bwd_args(q, k, v, dO, lse, delta, B, Hq, Hkv, N, Nkv, scale);
  a.dk = reinterpret_cast<fa::half_t*>(dk);
  a.dv = reinterpret_cast<fa::half_t*>(dv);
  auto fn = reinterpret_cast<fa::bwd_launch_fn>(var->fn[dt][fa::head_dim_index(D)][causal ? 1 : 0]);
  return launch_result(fn(a, static_cast<hipStream_t>(stream)), name);
}

static int64_t dkdv_workspace_impl(const char* name, int64_t B, int64_t Hq, int64_t Hkv,
                                   int64_t N, int64_t Nkv, int64_t D, int causal) {
  int rc = check_common(B, Hq, Hkv, N, D);
  if (rc) return rc;
  if ((rc = check_kv_length(Nkv, D))) return rc;
  // Enough for either element type (an overridden fp16-only tiling leaves
  // bf16 calls on the default tiling, whose split can be larger).
  int64_t bytes = 0;
  for (int dt : {fa::kF16, fa::kBF16}) {
    const fa::Variant* var = select_dkdv(fa::head_dim_index(D), causal, B, Hq, Hkv, N, Nkv, dt);
    if (!var) return fail(FA_ERR_BAD_TILING, "%s: no kernel for the selected tiling", name);
    bytes = std::max(bytes, split_workspace_bytes(dkdv_split(*var, B, Hq, Hkv, N, Nkv, causal),
                                                  B, Hkv, Nkv, D));
  }
  return bytes;
}

int64_t fa_bwd_dkdv_workspace_bytes(int64_t B, int64_t Hq, int64_t Hkv, int64_t N, int64_t D,
                                     int causal) {
  return dkdv_workspace_impl("fa_bwd_dkdv_workspace_bytes", B, Hq, Hkv, N, N, D, causal);
}

static int dkdv_ws_impl(int dt, const char* name, const fa_half_t* q, const fa_half_t* k,
                        const fa_half_t* v, const fa_half_t* dO, const float* lse,
                        const float* delta, fa_half_t* dk, fa_half_t* dv, int64_t B, int64_t Hq,
                        int64_t Hkv, int64_t N, int64_t Nkv, int64_t D, float scale, int causal,
                        void* workspace, int64_t workspace_bytes, void* stream) {
  if (!q || !k || !v || !dO || !lse || !delta || !dk || !dv)
    return fail(FA_ERR_NULL_POINTER, "%s: null pointer", name);
  int rc = check_common(B, Hq, Hkv, N, D);
  if (rc) return rc;
  if ((rc = check_kv_length(Nkv, D))) return rc;
  if ((rc = check_aligned(name, {q, k, v, dO, lse, delta, dk, dv}))) return rc;
  if ((rc = check_scale(scale))) return rc;
  const fa::Variant* var = select_dkdv(fa::head_dim_index(D), causal, B, Hq, Hkv, N, Nkv, dt);
  if (!var) return fail(FA_ERR_BAD_TILING, "%s: no kernel for the selected tiling", name);
  fa::BwdArgs a = bwd_args(q, k, v, dO, lse, delta, B, Hq, Hkv, N, Nkv, scale);
  a.dk = reinterpret_cast<fa::half_t*>(dk);
  a.dv = reinterpret_cast<fa::half_t*>(dv);
  const int nsplit = dkdv_split(*var, B, Hq, Hkv, N, Nkv, causal);
  const int64_t need = split_workspace_bytes(nsplit, B, Hkv, Nkv, D);
  hipStream_t s = static_cast<hipStream_t>(stream);
  auto fn = reinterpret_cast<fa::bwd_launch_fn>(var->fn[dt][fa::head_dim_index(D)][causal ? 1 : 0]);
  if (need == 0 || workspace == nullptr || workspace_bytes < need) {
    if (need > 0 && workspace != nullptr)
      return fail(FA_ERR_BAD_SHAPE, "%s: workspace of %lld bytes is smaller than the "
                  "%lld bytes fa_bwd_dkdv_workspace_bytes reports", name, (long long)workspace_bytes,
                  (long long)need);
    return launch_result(fn(a, s), name);
  }
  if ((rc = check_aligned(name, {workspace}))) return rc;
  a.nsplit = nsplit;
  a.part = static_cast<float*>(workspace);
  hipError_t e = fn(a, s);
  if (e != hipSuccess) return launch_result(e, name);
  return launch_result(fa::launch_split_reduce(a.part, a.dk, a.dv, B * Hkv * Nkv * D, nsplit, dt, s),
                    name);
}

static int dq_impl(int dt, const char* name, const fa_half_t* q, const fa_half_t* k,
                   const fa_half_t* v, const fa_half_t* dO, const float* lse, const float* delta,
                   fa_half_t* dq, int64_t B, int64_t Hq, int64_t Hkv, int64_t N, int64_t Nkv, int64_t D,
                   float scale, int causal, void* stream) {
  if (!q || !k || !v || !dO || !lse || !delta || !dq)
    return fail(FA_ERR_NULL_POINTER, "%s: null pointer", name);
  int rc = check_common(B, Hq, Hkv, N, D);
  if (rc) return rc;
  if ((rc = check_kv_length(Nkv, D))) return rc;
  if ((rc = check_aligned(name, {q, k, v, dO, lse, delta, dq}))) return rc;
  if ((rc = check_scale(scale))) return rc;
  const fa::Variant* var = select_dq(fa::head_dim_index(D), causal, N, B * Hq, dt);
  if (!var) return fail(FA_ERR_BAD_TILING, "%s: no kernel for the selected tiling", name);
  fa::BwdArgs a = bwd_args(q, k, v, dO, lse, delta, B, Hq, Hkv, N, Nkv, scale);
  a.dq = reinterpret_cast<fa::half_t*>(dq);
  auto fn = reinterpret_cast<fa::bwd_launch_fn>(var->fn[dt][fa::head_dim_index(D)][causal ? 1 : 0]);
  return launch_result(fn(a, static_cast<hipStream_t>(stream)), name);
}

static int dq_delta_impl(int dt, const char* name, const fa_half_t* q, const fa_half_t* k,
                         const fa_half_t* v, const fa_half_t* o, const fa_half_t* dO,
                         const float* lse, float* delta, fa_half_t* dq, int64_t B, int64_t Hq,
                         int64_t Hkv, int64_t N, int64_t Nkv, int64_t D, float scale, int causal,
                         void* stream, void* workspace = nullptr, int64_t workspace_bytes = 0) {
  if (!q || !k || !v || !o || !dO || !lse || !delta || !dq)
    return fail(FA_ERR_NULL_POINTER, "%s: null pointer", name);
  int rc = check_common(B, Hq, Hkv, N, D);
  if (rc) return rc;
  if ((rc = check_kv_length(Nkv, D))) return rc;
  if ((rc = check_aligned(name, {q, k, v, o, dO, lse, delta, dq}))) return rc;
  if ((rc = check_scale(scale))) return rc;
  const fa::Variant* var = select_dq(fa::head_dim_index(D), causal, N, B * Hq, dt);
  if (!var) return fail(FA_ERR_BAD_TILING, "%s: no kernel for the selected tiling", name);
  hipStream_t s = static_cast<hipStream_t>(stream);
  fa::BwdArgs a = bwd_args(q, k, v, dO, lse, delta, B, Hq, Hkv, N, Nkv, scale);
  a.dq = reinterpret_cast<fa::half_t*>(dq);
  // Split mode (few work-groups, a workspace given): fp32 partial dQ per key range, then summed.
  const FwdSplit sp = dq_split(*var, B, Hq, N, Nkv, causal);
  const int64_t need = dq_workspace_bytes(sp, B, Hq, N, D);
  const bool split = need > 0 && workspace != nullptr;
  if (split) {
    if (workspace_bytes < need)
      return fail(FA_ERR_BAD_SHAPE, "%s: workspace of %lld bytes is smaller than the %lld bytes "
                  "fa_bwd_dq_workspace_bytes reports", name, (long long)workspace_bytes,
                  (long long)need);
    if ((rc = check_aligned(name, {workspace}))) return rc;
    a.nsplit = sp.nsplit;
    a.split_keys = sp.split_keys;
    a.part = static_cast<float*>(workspace);
  }
  if (var->flags & fa::kFusesDelta) {
    a.o = reinterpret_cast<const fa::half_t*>(o);
    a.delta_out = delta;
  } else {
    hipError_t e = fa::launch_preprocess(reinterpret_cast<const fa::half_t*>(o),
                                         reinterpret_cast<const fa::half_t*>(dO), delta,
                                         B * Hq * N, (int)D, dt, s);
    if (e != hipSuccess) return launch_result(e, name);
  }
  auto fn = reinterpret_cast<fa::bwd_launch_fn>(var->fn[dt][fa::head_dim_index(D)][causal ? 1 : 0]);
  hipError_t e = fn(a, s);
  if (e != hipSuccess || !split) return launch_result(e, name);
  return launch_result(fa::launch_split_sum(a.part, a.dq, B * Hq * N * D, sp.nsplit, dt, s), name);
}

int64_t fa_bwd_dq_workspace_bytes(int64_t B, int64_t Hq, int64_t Hkv, int64_t N_q, int64_t N_kv,
                                  int64_t D, int causal) {
  int rc = check_common(B, Hq, Hkv, N_q, D);
  if (rc) return rc;
  if ((rc = check_kv_length(N_kv, D))) return rc;
  int64_t bytes = 0;  // enough for either element type
  for (int dt : {fa::kF16, fa::kBF16}) {
    const fa::Variant* var = select_dq(fa::head_dim_index(D), causal, N_q, B * Hq, dt);
    if (!var) return fail(FA_ERR_BAD_TILING, "fa_bwd_dq_workspace_bytes: no kernel for the selected tiling");
    bytes = std::max(bytes, dq_workspace_bytes(dq_split(*var, B, Hq, N_q, N_kv, causal), B, Hq, N_q, D));
  }
  return bytes;
}

int fa_bwd_dq_delta_ws(const fa_half_t* q, const fa_half_t* k, const fa_half_t* v,
                       const fa_half_t* o, const fa_half_t* dO, const float* lse, float* delta,
                       fa_half_t* dq, int64_t B, int64_t Hq, int64_t Hkv, int64_t N_q,
                       int64_t N_kv, int64_t D, float scale, int causal, void* workspace,
                       int64_t workspace_bytes, void* stream) {
  return dq_delta_impl(fa::kF16, "fa_bwd_dq_delta_ws", q, k, v, o, dO, lse, delta, dq, B, Hq, Hkv,
                       N_q, N_kv, D, scale, causal, stream, workspace, workspace_bytes);
}
int fa_bwd_dq_delta_ws_bf16(const fa_half_t* q, const fa_half_t* k, const fa_half_t* v,
                            const fa_half_t* o, const fa_half_t* dO, const float* lse,
                            float* delta, fa_half_t* dq, int64_t B, int64_t Hq, int64_t Hkv,
                            int64_t N_q, int64_t N_kv, int64_t D, float scale, int causal,
                            void* workspace, int64_t workspace_bytes, void* stream) {
  return dq_delta_impl(fa::kBF16, "fa_bwd_dq_delta_ws_bf16", q, k, v, o, dO, lse, delta, dq, B,
                       Hq, Hkv, N_q, N_kv, D, scale, causal, stream, workspace, workspace_bytes);
}

// ---- whole backward ---------------------------------------------------------
// Launch plan of one backward call: the dQ and dK/dV tilings, their splits,
// whether they run as one combined launch, and the workspace layout
// [dQ partials | dK/dV partials at a 256-byte boundary].
struct BwdPlan {
  const fa::Variant* dq;
  const fa::Variant* dkdv;
  FwdSplit dq_split;
  int dkdv_nsplit;
  bool pair;
  int64_t dq_bytes;
  int64_t dkdv_offset;
  int64_t dkdv_bytes;
  int64_t total;
};

// A dK/dV launch that splits (too few key tiles) next to a dQ launch that
// does not runs best as one combined launch (fa_bwd_pair.hip): MI355X,
// B2 Hq16 Hkv4 N2049 D64 causal, backward 106 -> 97 us already with the two
// launches on two streams, while with launches that fill the GPU (B4 H16
// N4096) running them together is slower (505 vs 478 us).
// The dQ launch must be short too: the combined plan pays off while dQ has at
// most 768 work-groups (1.5 waves of 2 per CU on 256 CUs). Measured on MI355X,
// whole backward, combined vs separate launches: dQ with 512-544 work-groups
// (B2 Hq16 Hkv4 N2049 D64/D32, B1 Hq4 Hkv1 N16381 D32, B1 Hq8 Hkv2 N8192 D32,
// causal and not) 4-8 % faster; with 1024 (B1 Hq8 Hkv2 N16381 D32, B1 Hq16
// Hkv4 N8192 D64, B1 Hq32 Hkv8 N4096 D64) between 1.5 % faster and 4.6 %
// slower. Work-groups (dK/dV chunks plus dQ) the combined launch aims at, and
// the fewest 32-query units per dK/dV chunk on average.
constexpr int64_t kPairMaxDqWorkgroups = 768;
constexpr int64_t kPairTargetWorkgroups = 3072;
constexpr int64_t kPairMinSplitUnits = 32;

bool plan_bwd(int dt, int64_t B, int64_t Hq, int64_t Hkv, int64_t N, int64_t Nkv, int64_t D,
              int causal, BwdPlan* p) {
  const int di = fa::head_dim_index(D);
  p->dq = select_dq(di, causal, N, B * Hq, dt);
  p->dkdv = select_dkdv(di, causal, B, Hq, Hkv, N, Nkv, dt);
  if (!p->dq || !p->dkdv) return false;
  p->dq_split = dq_split(*p->dq, B, Hq, N, Nkv, causal);
  p->dkdv_nsplit = dkdv_split(*p->dkdv, B, Hq, Hkv, N, Nkv, causal);
  const int64_t dq_wgs = (N + p->dq->rows - 1) / p->dq->rows * B * Hq;
  p->pair = p->dkdv_nsplit > 1 && p->dq_split.nsplit == 1 && dq_wgs <= kPairMaxDqWorkgroups &&
            (p->dq->flags & fa::kPairs) && (p->dkdv->flags & fa::kPairs) &&
            p->dq->waves == fa::bwd_pair_waves() && p->dkdv->waves == fa::bwd_pair_waves() &&
            fa::bwd_pair_launcher(dt, di, causal) != nullptr;
  if (p->pair) {
    // Beside the dQ work-groups the dK/dV chunks need not fill the GPU alone
    // (still split: the plan exists for launches whose key tiles are too few).
    const int64_t dkdv_wgs = (Nkv + p->dkdv->rows - 1) / p->dkdv->rows * B * Hkv;
    p->dkdv_nsplit = (int)std::max<int64_t>(
        2, chunks_for(std::max<int64_t>(kPairTargetWorkgroups - dq_wgs, dkdv_wgs), dkdv_wgs,
                      dkdv_tile_units(Hq, Hkv, N, causal), kPairMinSplitUnits));
  }
  p->dq_bytes = dq_workspace_bytes(p->dq_split, B, Hq, N, D);
  p->dkdv_offset = (p->dq_bytes + 255) / 256 * 256;
  p->dkdv_bytes = split_workspace_bytes(p->dkdv_nsplit, B, Hkv, Nkv, D);
  p->total = p->dkdv_bytes > 0 ? p->dkdv_offset + p->dkdv_bytes : p->dq_bytes;
  return true;
}

int64_t fa_bwd_workspace_bytes(int64_t B, int64_t Hq, int64_t Hkv, int64_t N_q, int64_t N_kv,
                               int64_t D, int causal) {
  int rc = check_common(B, Hq, Hkv, N_q, D);
  if (rc) return rc;
  if ((rc = check_kv_length(N_kv, D))) return rc;
  int64_t bytes = 0;  // enough for either element type
  for (int dt : {fa::kF16, fa::kBF16}) {
    BwdPlan p;
    if (!plan_bwd(dt, B, Hq, Hkv, N_q, N_kv, D, causal, &p))
      return fail(FA_ERR_BAD_TILING, "fa_bwd_workspace_bytes: no kernel for the selected tiling");
    bytes = std::max(bytes, p.total);
  }
  return bytes;
}

static int bwd_impl(int dt, const char* name, const fa_half_t* q, const fa_half_t* k,
                    const fa_half_t* v, const fa_half_t* o, const fa_half_t* dO,
                    const float* lse, float* delta, fa_half_t* dq, fa_half_t* dk, fa_half_t* dv,
                    int64_t B, int64_t Hq, int64_t Hkv, int64_t N, int64_t Nkv, int64_t D,
                    float scale, int causal, void* workspace, int64_t workspace_bytes,
                    void* stream) {
  if (!q || !k || !v || !o || !dO || !lse || !delta || !dq || !dk || !dv)
    return fail(FA_ERR_NULL_POINTER, "%s: null pointer", name);
  int rc = check_common(B, Hq, Hkv, N, D);
  if (rc) return rc;
  if ((rc = check_kv_length(Nkv, D))) return rc;
  if ((rc = check_aligned(name, {q, k, v, o, dO, lse, delta, dq, dk, dv}))) return rc;
  if ((rc = check_scale(scale))) return rc;
  BwdPlan p;
  if (!plan_bwd(dt, B, Hq, Hkv, N, Nkv, D, causal, &p))
    return fail(FA_ERR_BAD_TILING, "%s: no kernel for the selected tiling", name);
  char* ws = static_cast<char*>(workspace);
  if (ws != nullptr && p.total > 0) {
    if (workspace_bytes < p.total)
      return fail(FA_ERR_BAD_SHAPE, "%s: workspace of %lld bytes is smaller than the %lld bytes "
                  "fa_bwd_workspace_bytes reports", name, (long long)workspace_bytes,
                  (long long)p.total);
    if ((rc = check_aligned(name, {workspace}))) return rc;
  }
  if (p.pair && ws != nullptr) {
    hipStream_t s = static_cast<hipStream_t>(stream);
    const auto* o16 = reinterpret_cast<const fa::half_t*>(o);
    const auto* do16 = reinterpret_cast<const fa::half_t*>(dO);
    hipError_t e = fa::launch_preprocess(o16, do16, delta, B * Hq * N, (int)D, dt, s);
    if (e != hipSuccess) return launch_result(e, name);
    fa::BwdArgs ad = bwd_args(q, k, v, dO, lse, delta, B, Hq, Hkv, N, Nkv, scale);
    ad.dk = reinterpret_cast<fa::half_t*>(dk);
    ad.dv = reinterpret_cast<fa::half_t*>(dv);
    ad.nsplit = p.dkdv_nsplit;
    ad.part = reinterpret_cast<float*>(ws + p.dkdv_offset);
    fa::BwdArgs aq = bwd_args(q, k, v, dO, lse, delta, B, Hq, Hkv, N, Nkv, scale);
    aq.dq = reinterpret_cast<fa::half_t*>(dq);
    e = fa::bwd_pair_launcher(dt, fa::head_dim_index(D), causal)(ad, aq, s);
    if (e != hipSuccess) return launch_result(e, name);
    return launch_result(
        fa::launch_split_reduce(ad.part, ad.dk, ad.dv, B * Hkv * Nkv * D, p.dkdv_nsplit, dt, s),
        name);
  }
  rc = dq_delta_impl(dt, name, q, k, v, o, dO, lse, delta, dq, B, Hq, Hkv, N, Nkv, D, scale,
                     causal, stream, p.dq_bytes > 0 ? ws : nullptr, p.dq_bytes);
  if (rc) return rc;
  return dkdv_ws_impl(dt, name, q, k, v, dO, lse, delta, dk, dv, B, Hq, Hkv, N, Nkv, D, scale,
                      causal, p.dkdv_bytes > 0 && ws ? ws + p.dkdv_offset : nullptr,
                      p.dkdv_bytes, stream);
}

int fa_bwd(const fa_half_t* q, const fa_half_t* k, const fa_half_t* v, const fa_half_t* o,
           const fa_half_t* dO, const float* lse, float* delta, fa_half_t* dq, fa_half_t* dk,
           fa_half_t* dv, int64_t B, int64_t Hq, int64_t Hkv, int64_t N_q, int64_t N_kv,
           int64_t D, float scale, int causal, void* workspace, int64_t workspace_bytes,
           void* stream) {
  return bwd_impl(fa::kF16, "fa_bwd", q, k, v, o, dO, lse, delta, dq, dk, dv, B, Hq, Hkv, N_q,
                  N_kv, D, scale, causal, workspace, workspace_bytes, stream);
}
int fa_bwd_bf16(const fa_half_t* q, const fa_half_t* k, const fa_half_t* v, const fa_half_t* o,
                const fa_half_t* dO, const float* lse, float* delta, fa_half_t* dq,
                fa_half_t* dk, fa_half_t* dv, int64_t B, int64_t Hq, int64_t Hkv, int64_t N_q,
                int64_t N_kv, int64_t D, float scale, int causal, void* workspace,
                int64_t workspace_bytes, void* stream) {
  return bwd_impl(fa::kBF16, "fa_bwd_bf16", q, k, v, o, dO, lse, delta, dq, dk, dv, B, Hq, Hkv,
                  N_q, N_kv, D, scale, causal, workspace, workspace_bytes, stream);
}

// ---- exported launches: fp16 (the reference's dtype) and bf16 twins ------
int fa_fwd(const fa_half_t* q, const fa_half_t* k, const fa_half_t* v, fa_half_t* o, float* lse,
           int64_t B, int64_t Hq, int64_t Hkv, int64_t N, int64_t D, float scale, int causal,
           void* stream) {
  return fwd_impl(fa::kF16, "fa_fwd", q, k, v, o, lse, B, Hq, Hkv, N, N, D, scale, causal,
                  stream);
}
int fa_fwd_bf16(const fa_half_t* q, const fa_half_t* k, const fa_half_t* v, fa_half_t* o,
                float* lse, int64_t B, int64_t Hq, int64_t Hkv, int64_t N, int64_t D, float scale,
                int causal, void* stream) {
  return fwd_impl(fa::kBF16, "fa_fwd_bf16", q, k, v, o, lse, B, Hq, Hkv, N, N, D, scale, causal,
                  stream);
}
int fa_bwd_preprocess(const fa_half_t* o, const fa_half_t* dO, float* delta, int64_t B,
                      int64_t Hq, int64_t N, int64_t D, void* stream) {
  return preprocess_impl(fa::kF16, "fa_bwd_preprocess", o, dO, delta, B, Hq, N, D, stream);
}
int fa_bwd_preprocess_bf16(const fa_half_t* o, const fa_half_t* dO, float* delta, int64_t B,
                           int64_t Hq, int64_t N, int64_t D, void* stream) {
  return preprocess_impl(fa::kBF16, "fa_bwd_preprocess_bf16", o, dO, delta, B, Hq, N, D, stream);
}
int fa_bwd_dkdv(const fa_half_t* q, const fa_half_t* k, const fa_half_t* v, const fa_half_t* dO,
                const float* lse, const float* delta, fa_half_t* dk, fa_half_t* dv, int64_t B,
                int64_t Hq, int64_t Hkv, int64_t N, int64_t D, float scale, int causal,
                void* stream) {
  return dkdv_impl(fa::kF16, "fa_bwd_dkdv", q, k, v, dO, lse, delta, dk, dv, B, Hq, Hkv, N, N, D,
                   scale, causal, stream);
}
int fa_bwd_dkdv_bf16(const fa_half_t* q, const fa_half_t* k, const fa_half_t* v,
                     const fa_half_t* dO, const float* lse, const float* delta, fa_half_t* dk,
                     fa_half_t* dv, int64_t B, int64_t Hq, int64_t Hkv, int64_t N, int64_t D,
                     float scale, int causal, void* stream) {
  return dkdv_impl(fa::kBF16, "fa_bwd_dkdv_bf16", q, k, v, dO, lse, delta, dk, dv, B, Hq, Hkv,
                   N, N, D, scale, causal, stream);
}
int fa_bwd_dkdv_ws(const fa_half_t* q, const fa_half_t* k, const fa_half_t* v,
                   const fa_half_t* dO, const float* lse, const float* delta, fa_half_t* dk,
                   fa_half_t* dv, int64_t B, int64_t Hq, int64_t Hkv, int64_t N, int64_t D,
                   float scale, int causal, void* workspace, int64_t workspace_bytes,
                   void* stream) {
  return dkdv_ws_impl(fa::kF16, "fa_bwd_dkdv_ws", q, k, v, dO, lse, delta, dk, dv, B, Hq, Hkv,
                      N, N, D, scale, causal, workspace, workspace_bytes, stream);
}
int fa_bwd_dkdv_ws_bf16(const fa_half_t* q, const fa_half_t* k, const fa_half_t* v,
                        const fa_half_t* dO, const float* lse, const float* delta,
                        fa_half_t* dk, fa_half_t* dv, int64_t B, int64_t Hq, int64_t Hkv,
                        int64_t N, int64_t D, float scale, int causal, void* workspace,
                        int64_t workspace_bytes, void* stream) {
  return dkdv_ws_impl(fa::kBF16, "fa_bwd_dkdv_ws_bf16", q, k, v, dO, lse, delta, dk, dv, B, Hq,
                      Hkv, N, N, D, scale, causal, workspace, workspace_bytes, stream);
}
int fa_bwd_dq(const fa_half_t* q, const fa_half_t* k, const fa_half_t* v, const fa_half_t* dO,
              const float* lse, const float* delta, fa_half_t* dq, int64_t B, int64_t Hq,
              int64_t Hkv, int64_t N, int64_t D, float scale, int causal, void* stream) {
  return dq_impl(fa::kF16, "fa_bwd_dq", q, k, v, dO, lse, delta, dq, B, Hq, Hkv, N, N, D, scale,
                 causal, stream);
}
int fa_bwd_dq_bf16(const fa_half_t* q, const fa_half_t* k, const fa_half_t* v,
                   const fa_half_t* dO, const float* lse, const float* delta, fa_half_t* dq,
                   int64_t B, int64_t Hq, int64_t Hkv, int64_t N, int64_t D, float scale,
                   int causal, void* stream) {
  return dq_impl(fa::kBF16, "fa_bwd_dq_bf16", q, k, v, dO, lse, delta, dq, B, Hq, Hkv, N, N, D,
                 scale, causal, stream);
}
int fa_bwd_dq_delta(const fa_half_t* q, const fa_half_t* k, const fa_half_t* v,
                    const fa_half_t* o, const fa_half_t* dO, const float* lse, float* delta,
                    fa_half_t* dq, int64_t B, int64_t Hq, int64_t Hkv, int64_t N, int64_t D,
                    float scale, int causal, void* stream) {
  return dq_delta_impl(fa::kF16, "fa_bwd_dq_delta", q, k, v, o, dO, lse, delta, dq, B, Hq, Hkv,
                       N, N, D, scale, causal, stream);
}
int fa_bwd_dq_delta_bf16(const fa_half_t* q, const fa_half_t* k, const fa_half_t* v,
                         const fa_half_t* o, const fa_half_t* dO, const float* lse, float* delta,
                         fa_half_t* dq, int64_t B, int64_t Hq, int64_t Hkv, int64_t N, int64_t D,
                         float scale, int causal, void* stream) {
  return dq_delta_impl(fa::kBF16, "fa_bwd_dq_delta_bf16", q, k, v, o, dO, lse, delta, dq, B, Hq,
                       Hkv, N, N, D, scale, causal, stream);
}

// ---- forward without allocation: the split workspace is `scratch` --------
int64_t fa_fwd_noalloc_max_workspace_bytes(void) { return kNoallocScratchBytes; }

int fa_fwd_noalloc(const fa_half_t* q, const fa_half_t* k, const fa_half_t* v, fa_half_t* o,
                   float* lse, int64_t B, int64_t Hq, int64_t Hkv, int64_t N_q, int64_t N_kv,
                   int64_t D, float scale, int causal, void* stream) {
  const char* name = "fa_fwd_noalloc";
  const fa::Variant* var = nullptr;
  int64_t need = 0;
  int rc = fwd_check(fa::kF16, name, q, k, v, o, lse, B, Hq, Hkv, N_q, N_kv, D, scale, causal,
                     &var, &need);
  if (rc) return rc;
  if (need > kNoallocScratchBytes)
    return fail(FA_ERR_TOO_LARGE, "%s: this shape's split-KV partials need %lld bytes, more than "
                "the %lld-byte device scratch; use fa_fwd_ws with a workspace of "
                "fa_fwd_workspace_bytes", name, (long long)need, (long long)kNoallocScratchBytes);
  if (need == 0)
    return fwd_impl(fa::kF16, name, q, k, v, o, lse, B, Hq, Hkv, N_q, N_kv, D, scale, causal,
                    stream);
  void* ws = nullptr;
  if ((rc = scratch_address(name, static_cast<hipStream_t>(stream), &ws))) return rc;
  return fwd_impl(fa::kF16, name, q, k, v, o, lse, B, Hq, Hkv, N_q, N_kv, D, scale, causal,
                  stream, ws, kNoallocScratchBytes);
}

int fa_fwd_ws(const fa_half_t* q, const fa_half_t* k, const fa_half_t* v, fa_half_t* o,
              float* lse, int64_t B, int64_t Hq, int64_t Hkv, int64_t N_q, int64_t N_kv,
              int64_t D, float scale, int causal, void* workspace, int64_t workspace_bytes,
              void* stream) {
  return fwd_impl(fa::kF16, "fa_fwd_ws", q, k, v, o, lse, B, Hq, Hkv, N_q, N_kv, D, scale, causal,
                  stream, workspace, workspace_bytes);
}
int fa_fwd_ws_bf16(const fa_half_t* q, const fa_half_t* k, const fa_half_t* v, fa_half_t* o,
                   float* lse, int64_t B, int64_t Hq, int64_t Hkv, int64_t N_q, int64_t N_kv,
                   int64_t D, float scale, int causal, void* workspace, int64_t workspace_bytes,
                   void* stream) {
  return fwd_impl(fa::kBF16, "fa_fwd_ws_bf16", q, k, v, o, lse, B, Hq, Hkv, N_q, N_kv, D, scale,
                  causal, stream, workspace, workspace_bytes);
}

// ---- exported launches with separate query and key/value lengths --------
int fa_fwd_kv(const fa_half_t* q, const fa_half_t* k, const fa_half_t* v, fa_half_t* o,
              float* lse, int64_t B, int64_t Hq, int64_t Hkv, int64_t N_q, int64_t N_kv,
              int64_t D, float scale, int causal, void* stream) {
  return fwd_impl(fa::kF16, "fa_fwd_kv", q, k, v, o, lse, B, Hq, Hkv, N_q, N_kv, D, scale, causal,
                  stream);
}
int fa_fwd_kv_bf16(const fa_half_t* q, const fa_half_t* k, const fa_half_t* v, fa_half_t* o,
                   float* lse, int64_t B, int64_t Hq, int64_t Hkv, int64_t N_q, int64_t N_kv,
                   int64_t D, float scale, int causal, void* stream) {
  return fwd_impl(fa::kBF16, "fa_fwd_kv_bf16", q, k, v, o, lse, B, Hq, Hkv, N_q, N_kv, D, scale,
                  causal, stream);
}
int64_t fa_bwd_dkdv_workspace_bytes_kv(int64_t B, int64_t Hq, int64_t Hkv, int64_t N_q,
                                        int64_t N_kv, int64_t D, int causal) {
  return dkdv_workspace_impl("fa_bwd_dkdv_workspace_bytes_kv", B, Hq, Hkv, N_q, N_kv, D, causal);
}
int fa_bwd_dkdv_ws_kv(const fa_half_t* q, const fa_half_t* k, const fa_half_t* v,
                      const fa_half_t* dO, const float* lse, const float* delta, fa_half_t* dk,
                      fa_half_t* dv, int64_t B, int64_t Hq, int64_t Hkv, int64_t N_q,
                      int64_t N_kv, int64_t D, float scale, int causal, void* workspace,
                      int64_t workspace_bytes, void* stream) {
  return dkdv_ws_impl(fa::kF16, "fa_bwd_dkdv_ws_kv", q, k, v, dO, lse, delta, dk, dv, B, Hq, Hkv,
                      N_q, N_kv, D, scale, causal, workspace, workspace_bytes, stream);
}
int fa_bwd_dkdv_ws_kv_bf16(const fa_half_t* q, const fa_half_t* k, const fa_half_t* v,
                           const fa_half_t* dO, const float* lse, const float* delta,
                           fa_half_t* dk, fa_half_t* dv, int64_t B, int64_t Hq, int64_t Hkv,
                           int64_t N_q, int64_t N_kv, int64_t D, float scale, int causal,
                           void* workspace, int64_t workspace_bytes, void* stream) {
  return dkdv_ws_impl(fa::kBF16, "fa_bwd_dkdv_ws_kv_bf16", q, k, v, dO, lse, delta, dk, dv, B, Hq,
                      Hkv, N_q, N_kv, D, scale, causal, workspace, workspace_bytes, stream);
}
int fa_bwd_dq_delta_kv(const fa_half_t* q, const fa_half_t* k, const fa_half_t* v,
                       const fa_half_t* o, const fa_half_t* dO, const float* lse, float* delta,
                       fa_half_t* dq, int64_t B, int64_t Hq, int64_t Hkv, int64_t N_q,
                       int64_t N_kv, int64_t D, float scale, int causal, void* stream) {
  return dq_delta_impl(fa::kF16, "fa_bwd_dq_delta_kv", q, k, v, o, dO, lse, delta, dq, B, Hq, Hkv,
                       N_q, N_kv, D, scale, causal, stream);
}
int fa_bwd_dq_delta_kv_bf16(const fa_half_t* q, const fa_half_t* k, const fa_half_t* v,
                            const fa_half_t* o, const fa_half_t* dO, const float* lse,
                            float* delta, fa_half_t* dq, int64_t B, int64_t Hq, int64_t Hkv,
                            int64_t N_q, int64_t N_kv, int64_t D, float scale, int causal,
                            void* stream) {
  return dq_delta_impl(fa::kBF16, "fa_bwd_dq_delta_kv_bf16", q, k, v, o, dO, lse, delta, dq, B,
                       Hq, Hkv, N_q, N_kv, D, scale, causal, stream);
}

int fa_get_tiling(int kernel, int64_t D, int causal, int* out4) {
  if (!out4) return fail(FA_ERR_NULL_POINTER, "fa_get_tiling: null pointer");
  const int di = fa::head_dim_index(D);
  if (di < 0) return fail(FA_ERR_HEAD_DIM, "head_dim must be one of (32, 64, 128)");
  if (kernel < 0 || kernel >= fa::kNumKinds)
    return fail(FA_ERR_BAD_TILING, "unknown kernel %d", kernel);
  int index = -1;
  const fa::Variant* var = select_current(kernel, di, causal, &index);
  if (!var) return fail(FA_ERR_BAD_TILING, "no tiling for kernel %d", kernel);
  out4[0] = var->waves;
  out4[1] = var->rows;
  out4[2] = var->tile;
  out4[3] = index;
  return FA_OK;
}

int fa_num_tiling_variants(int kernel, int64_t D, int causal) {
  (void)causal;
  if (fa::head_dim_index(D) < 0) return fail(FA_ERR_HEAD_DIM, "head_dim must be one of (32, 64, 128)");
  int count = 0;
  if (!registry(kernel, &count)) return fail(FA_ERR_BAD_TILING, "unknown kernel %d", kernel);
  return count;
}

int fa_describe_tiling_variant(int kernel, int64_t D, int causal, int variant, int* out4) {
  if (!out4) return fail(FA_ERR_NULL_POINTER, "fa_describe_tiling_variant: null pointer");
  const int di = fa::head_dim_index(D);
  if (di < 0) return fail(FA_ERR_HEAD_DIM, "head_dim must be one of (32, 64, 128)");
  int count = 0;
  const fa::Variant* vs = registry(kernel, &count);
  if (!vs) return fail(FA_ERR_BAD_TILING, "unknown kernel %d", kernel);
  if (variant < 0 || variant >= count)
    return fail(FA_ERR_BAD_TILING, "variant %d out of range [0, %d)", variant, count);
  if (!usable(vs[variant], di, causal))
    return fail(FA_ERR_BAD_TILING, "variant %d is not compiled for head_dim %lld", variant,
                (long long)D);
  out4[0] = vs[variant].waves;
  out4[1] = vs[variant].rows;
  out4[2] = vs[variant].tile;
  out4[3] = variant;
  return FA_OK;
}

int fa_set_tiling(int kernel, int64_t D, int causal, int variant) {
  const int di = fa::head_dim_index(D);
  if (di < 0) return fail(FA_ERR_HEAD_DIM, "head_dim must be one of (32, 64, 128)");
  int count = 0;
  if (!registry(kernel, &count)) return fail(FA_ERR_BAD_TILING, "unknown kernel %d", kernel);
  if (variant >= count)
    return fail(FA_ERR_BAD_TILING, "variant %d out of range [0, %d)", variant, count);
  if (variant >= 0 && !usable(registry(kernel, &count)[variant], di, causal))
    return fail(FA_ERR_BAD_TILING, "variant %d is not compiled for head_dim %lld", variant,
                (long long)D);
  g_override_plus1[kernel][di][causal ? 1 : 0].store(variant < 0 ? 0 : variant + 1,
                                                      std::memory_order_relaxed);
  return FA_OK;
}

}  // extern "C"
