/*
 * fa_gfx950.h — C ABI of the MI355X (gfx950) FlashAttention-2 library
 * (libfa_gfx950.so).
 *
 * This is the drop-in boundary for the hot path of
 * triton_flash_attention (reference: triton_flash_attention/attention.py).
 * The reference launches three Triton kernels from Python; each entry point
 * below replaces one of those launches (or one half of the fused backward
 * launch) and keeps its argument meaning:
 *
 *   fa_fwd             replaces  _attn_fwd[grid](...)             attention.py:690-718
 *   fa_bwd_preprocess  replaces  _attn_bwd_preprocess[grid](...)  attention.py:736-744
 *   fa_bwd_dkdv        replaces  _attn_bwd[grid](...) phase 1     attention.py:754-770 (kernel 428-505)
 *   fa_bwd_dq          replaces  _attn_bwd[grid](...) phase 2     attention.py:754-770 (kernel 507-573)
 *   fa_bwd_dq_delta    replaces  _attn_bwd_preprocess + phase 2   attention.py:736-744, 754-770
 *   fa_bwd             replaces  all of TritonAttention.backward's launches
 *                                (preprocess, then both phases)   attention.py:720-770
 *
 * Conventions shared by every entry point
 *   - Tensors are caller-owned device memory, contiguous, row-major:
 *       q, o, dO, dq   : [B, Hq,  N, D]  IEEE binary16
 *       k, v, dk, dv   : [B, Hkv, N, D]  IEEE binary16
 *       lse, delta     : [B, Hq,  N]     float32
 *     (the reference forces the same layout with .contiguous(),
 *      attention.py:727, 841-843, and indexes it that way, 251, 412-414).
 *   - lse is the base-2 log-sum-exp of the scaled scores of each query row,
 *     lse = log2(sum_j exp2(scale*log2(e)*q.k_j)), the quantity the reference
 *     stores at attention.py:230.
 *   - Causal masking is top-left: query i sees keys j <= i (attention.py:65).
 *   - GQA: query head h reads key/value head h / (Hq / Hkv) (attention.py:128-131).
 *     dk/dv are the sums over the Hq/Hkv query heads of a group, reduced in
 *     fp32 inside the kernel (no atomics, deterministic).
 *   - Supported head_dim D: 32, 64, 128 (attention.py:21). N >= 1, any value.
 *   - Every tensor pointer must be 16-byte aligned (the kernels move 128-bit
 *     vectors); fresh allocations from any HIP allocator are.
 *   - `stream` is a hipStream_t (NULL = the null stream). Calls are
 *     asynchronous on that stream; nothing allocates, frees or synchronizes.
 *   - Return value: 0 on success; a negative FA_ERR_* code when an argument is
 *     rejected before any HIP call; otherwise the hipError_t of the launch.
 *     fa_last_error() returns a thread-local message describing the last
 *     failure of the calling thread.
 */
#ifndef FA_GFX950_H
#define FA_GFX950_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define FA_ABI_VERSION 7

/* Error codes returned before any HIP call is made. */
#define FA_OK 0
#define FA_ERR_NULL_POINTER (-1)       /* a required pointer is NULL            */
#define FA_ERR_BAD_SHAPE (-2)          /* B, H, N <= 0 or Hq % Hkv != 0          */
#define FA_ERR_HEAD_DIM (-3)           /* D not in {32, 64, 128}                 */
#define FA_ERR_TOO_LARGE (-4)          /* a head slab exceeds 2^31 bytes or the  */
                                       /* launch grid exceeds 2^31 work-groups   */
#define FA_ERR_BAD_SCALE (-5)          /* scale not finite or not > 0            */
#define FA_ERR_BAD_TILING (-6)         /* no compiled kernel for this tiling     */
#define FA_ERR_MISALIGNED (-7)         /* a tensor pointer is not 16-byte aligned */

/* 16-bit storage type of the tensor elements: IEEE binary16 for the entry
 * points without a suffix, bfloat16 for the _bf16 ones. */
typedef uint16_t fa_half_t;

/* Forward: o = softmax(scale * q k^T [+ causal mask]) v, and lse (base 2).
 * Replaces the _attn_fwd launch, attention.py:690-718 (kernel 90-234). */
int fa_fwd(const fa_half_t* q, const fa_half_t* k, const fa_half_t* v,
           fa_half_t* o, float* lse,
           int64_t B, int64_t Hq, int64_t Hkv, int64_t N, int64_t D,
           float scale, int causal, void* stream);

/* delta[b,h,i] = sum_d o[b,h,i,d] * dO[b,h,i,d] in fp32.
 * Replaces the _attn_bwd_preprocess launch, attention.py:736-744 (kernel 237-255). */
int fa_bwd_preprocess(const fa_half_t* o, const fa_half_t* dO, float* delta,
                      int64_t B, int64_t Hq, int64_t N, int64_t D, void* stream);

/* dk, dv (fully overwritten; no zero-fill needed). Recomputes P from lse.
 * Replaces phase 1 of the _attn_bwd launch, attention.py:754-770 (kernel 428-505). */
int fa_bwd_dkdv(const fa_half_t* q, const fa_half_t* k, const fa_half_t* v,
                const fa_half_t* dO, const float* lse, const float* delta,
                fa_half_t* dk, fa_half_t* dv,
                int64_t B, int64_t Hq, int64_t Hkv, int64_t N, int64_t D,
                float scale, int causal, void* stream);

/* Workspace bytes fa_bwd_dkdv_ws needs for this shape (0: it runs as one
 * pass and needs none); negative FA_ERR_* for rejected arguments. No
 * reference counterpart: the reference reduces GQA groups with fp16 atomics. */
int64_t fa_bwd_dkdv_workspace_bytes(int64_t B, int64_t Hq, int64_t Hkv, int64_t N, int64_t D,
                                     int causal);

/* fa_bwd_dkdv with a caller-provided device workspace (16-byte aligned).
 * When the shape has too few (key tile, KV head) work-groups to fill the GPU
 * (GQA with few KV heads, long causal sequences), each key tile's steps are
 * split over several work-groups that write fp32 partials into the workspace,
 * and a second kernel sums them in a fixed order into dk, dv (deterministic).
 * workspace may be NULL when fa_bwd_dkdv_workspace_bytes returned 0; a
 * non-NULL workspace smaller than required is rejected (FA_ERR_BAD_SHAPE).
 * Replaces phase 1 of the _attn_bwd launch, attention.py:754-770 (kernel 428-505). */
int fa_bwd_dkdv_ws(const fa_half_t* q, const fa_half_t* k, const fa_half_t* v,
                   const fa_half_t* dO, const float* lse, const float* delta,
                   fa_half_t* dk, fa_half_t* dv,
                   int64_t B, int64_t Hq, int64_t Hkv, int64_t N, int64_t D,
                   float scale, int causal, void* workspace, int64_t workspace_bytes,
                   void* stream);

/* dq (fully overwritten). Recomputes P from lse.
 * Replaces phase 2 of the _attn_bwd launch, attention.py:754-770 (kernel 507-573). */
int fa_bwd_dq(const fa_half_t* q, const fa_half_t* k, const fa_half_t* v,
              const fa_half_t* dO, const float* lse, const float* delta,
              fa_half_t* dq,
              int64_t B, int64_t Hq, int64_t Hkv, int64_t N, int64_t D,
              float scale, int causal, void* stream);

/* delta = rowsum(o * dO) (as fa_bwd_preprocess) and dq (as fa_bwd_dq with that
 * delta) in one call: the reference's _attn_bwd_preprocess launch
 * (attention.py:736-744) folded into phase 2 of its _attn_bwd launch
 * (attention.py:754-770, kernel 507-573). When the selected dQ tiling computes
 * delta itself this is a single launch; otherwise it is the two launches in
 * order. delta is written before dq is; a dK/dV call that reads delta may
 * follow on the same stream. */
int fa_bwd_dq_delta(const fa_half_t* q, const fa_half_t* k, const fa_half_t* v,
                    const fa_half_t* o, const fa_half_t* dO, const float* lse,
                    float* delta, fa_half_t* dq,
                    int64_t B, int64_t Hq, int64_t Hkv, int64_t N, int64_t D,
                    float scale, int causal, void* stream);

/* bfloat16 twins of the launches above: same arguments, same semantics and
 * checks, q/k/v/o/dO/dq/dk/dv holding bfloat16 (lse and delta stay float32;
 * arithmetic in fp32, P and dS rounded to bfloat16 for the MFMAs, the
 * backward's scaled score operands rounded to bfloat16). No counterpart in
 * the reference, which sends every non-fp16 input to torch SDPA
 * (attention.py:653-655); they widen the dtypes the GPU path serves. Compiled
 * for the default tilings; a bf16 call whose kernel has an overridden tiling
 * without a bf16 build uses the default tiling. */
int fa_fwd_bf16(const fa_half_t* q, const fa_half_t* k, const fa_half_t* v,
                fa_half_t* o, float* lse,
                int64_t B, int64_t Hq, int64_t Hkv, int64_t N, int64_t D,
                float scale, int causal, void* stream);
int fa_bwd_preprocess_bf16(const fa_half_t* o, const fa_half_t* dO, float* delta,
                           int64_t B, int64_t Hq, int64_t N, int64_t D, void* stream);
int fa_bwd_dkdv_bf16(const fa_half_t* q, const fa_half_t* k, const fa_half_t* v,
                     const fa_half_t* dO, const float* lse, const float* delta,
                     fa_half_t* dk, fa_half_t* dv,
                     int64_t B, int64_t Hq, int64_t Hkv, int64_t N, int64_t D,
                     float scale, int causal, void* stream);
int fa_bwd_dkdv_ws_bf16(const fa_half_t* q, const fa_half_t* k, const fa_half_t* v,
                        const fa_half_t* dO, const float* lse, const float* delta,
                        fa_half_t* dk, fa_half_t* dv,
                        int64_t B, int64_t Hq, int64_t Hkv, int64_t N, int64_t D,
                        float scale, int causal, void* workspace, int64_t workspace_bytes,
                        void* stream);
int fa_bwd_dq_bf16(const fa_half_t* q, const fa_half_t* k, const fa_half_t* v,
                   const fa_half_t* dO, const float* lse, const float* delta,
                   fa_half_t* dq,
                   int64_t B, int64_t Hq, int64_t Hkv, int64_t N, int64_t D,
                   float scale, int causal, void* stream);
int fa_bwd_dq_delta_bf16(const fa_half_t* q, const fa_half_t* k, const fa_half_t* v,
                         const fa_half_t* o, const fa_half_t* dO, const float* lse,
                         float* delta, fa_half_t* dq,
                         int64_t B, int64_t Hq, int64_t Hkv, int64_t N, int64_t D,
                         float scale, int causal, void* stream);

/* Cross-attention launches: the query length N_q and the key/value length
 * N_kv differ (q, o, dO, dq, lse, delta are [B, Hq, N_q, ...]; k, v, dk, dv
 * are [B, Hkv, N_kv, D]); otherwise the same arguments, semantics and checks
 * as fa_fwd, fa_bwd_dkdv_workspace_bytes, fa_bwd_dkdv_ws and fa_bwd_dq_delta,
 * with N_kv bounded like N. No counterpart in the reference kernels: the
 * reference sends N_q != N_kv to torch SDPA (attention.py:639-642, 830-838),
 * and these compute what that fallback does. Causal masking stays top-left,
 * query i sees keys j <= i, SDPA's is_causal mask for unequal lengths (the
 * lower triangle of the N_q x N_kv all-ones matrix); no row is fully masked.
 * With N_q < N_kv, keys past the last query get dk = dv = 0 under the causal
 * mask. fa_bwd_preprocess works on the query side and needs no twin. */
int fa_fwd_kv(const fa_half_t* q, const fa_half_t* k, const fa_half_t* v,
              fa_half_t* o, float* lse,
              int64_t B, int64_t Hq, int64_t Hkv, int64_t N_q, int64_t N_kv, int64_t D,
              float scale, int causal, void* stream);
int fa_fwd_kv_bf16(const fa_half_t* q, const fa_half_t* k, const fa_half_t* v,
                   fa_half_t* o, float* lse,
                   int64_t B, int64_t Hq, int64_t Hkv, int64_t N_q, int64_t N_kv, int64_t D,
                   float scale, int causal, void* stream);
int64_t fa_bwd_dkdv_workspace_bytes_kv(int64_t B, int64_t Hq, int64_t Hkv, int64_t N_q,
                                        int64_t N_kv, int64_t D, int causal);
int fa_bwd_dkdv_ws_kv(const fa_half_t* q, const fa_half_t* k, const fa_half_t* v,
                      const fa_half_t* dO, const float* lse, const float* delta,
                      fa_half_t* dk, fa_half_t* dv,
                      int64_t B, int64_t Hq, int64_t Hkv, int64_t N_q, int64_t N_kv, int64_t D,
                      float scale, int causal, void* workspace, int64_t workspace_bytes,
                      void* stream);
int fa_bwd_dkdv_ws_kv_bf16(const fa_half_t* q, const fa_half_t* k, const fa_half_t* v,
                           const fa_half_t* dO, const float* lse, const float* delta,
                           fa_half_t* dk, fa_half_t* dv,
                           int64_t B, int64_t Hq, int64_t Hkv, int64_t N_q, int64_t N_kv,
                           int64_t D, float scale, int causal, void* workspace,
                           int64_t workspace_bytes, void* stream);
int fa_bwd_dq_delta_kv(const fa_half_t* q, const fa_half_t* k, const fa_half_t* v,
                       const fa_half_t* o, const fa_half_t* dO, const float* lse,
                       float* delta, fa_half_t* dq,
                       int64_t B, int64_t Hq, int64_t Hkv, int64_t N_q, int64_t N_kv, int64_t D,
                       float scale, int causal, void* stream);
int fa_bwd_dq_delta_kv_bf16(const fa_half_t* q, const fa_half_t* k, const fa_half_t* v,
                            const fa_half_t* o, const fa_half_t* dO, const float* lse,
                            float* delta, fa_half_t* dq,
                            int64_t B, int64_t Hq, int64_t Hkv, int64_t N_q, int64_t N_kv,
                            int64_t D, float scale, int causal, void* stream);

/* Forward with split-KV for launches with few work-groups (decoding: a few
 * queries against a long key sequence, or few heads): fa_fwd_kv's arguments
 * plus a caller-provided device workspace. fa_fwd_workspace_bytes returns the
 * bytes a call with these sizes needs (0 when it does not split, for either
 * element type). With workspace == NULL, or when no split is needed, the call
 * is fa_fwd_kv; a non-NULL workspace smaller than needed is rejected
 * (FA_ERR_BAD_SHAPE). Splitting, the launch computes fp32 partial O and LSE
 * per key range of at least 1024 keys into the workspace and merges them
 * (O = sum_s w_s O_s / sum_s w_s, w_s = exp2(lse_s - max lse), LSE = max +
 * log2 sum w_s) in a second launch on the same stream; results agree with
 * the unsplit forward up to fp32 summation order. No counterpart in the
 * reference (its forward, attention.py:690-718, is one launch per
 * (query tile, head)); it serves the cross-attention the library takes over
 * from SDPA. The workspace is [nsplit, B, Hq, N_q, D + 1] fp32; concurrent
 * calls need separate workspaces. */
int64_t fa_fwd_workspace_bytes(int64_t B, int64_t Hq, int64_t Hkv, int64_t N_q, int64_t N_kv,
                               int64_t D, int causal);
int fa_fwd_ws(const fa_half_t* q, const fa_half_t* k, const fa_half_t* v,
              fa_half_t* o, float* lse,
              int64_t B, int64_t Hq, int64_t Hkv, int64_t N_q, int64_t N_kv, int64_t D,
              float scale, int causal, void* workspace, int64_t workspace_bytes, void* stream);
int fa_fwd_ws_bf16(const fa_half_t* q, const fa_half_t* k, const fa_half_t* v,
                   fa_half_t* o, float* lse,
                   int64_t B, int64_t Hq, int64_t Hkv, int64_t N_q, int64_t N_kv, int64_t D,
                   float scale, int causal, void* workspace, int64_t workspace_bytes,
                   void* stream);

/* The forward's launch plan for these sizes (fp16; bf16 uses the same
 * tilings): out4[0] = work-groups of the persistent job-plan grid, 0 when the
 * launch runs the grid form (one work-group per (query tile, head) and key
 * range); out4[1] = work-groups of the grid form; out4[2], out4[3] = the
 * modelled makespans, in 32-key units per resident work-group slot, of the
 * plan (0 without one) and of the grid form (0 where no plan is considered).
 * compute_units > 0 plans for that many CUs, else for the current device.
 * No HIP launch; no counterpart in the reference, whose forward grid is
 * (cdiv(N, BLOCK_M), B * Hq) (attention.py:687-688): under the causal mask the
 * library may instead launch one work-group per resident slot, each running a
 * bin of (query tile, head) jobs packed to equal lengths. */
int fa_fwd_plan_info(int64_t B, int64_t Hq, int64_t Hkv, int64_t N_q, int64_t N_kv, int64_t D,
                     int causal, int compute_units, int64_t* out4);

/* dQ (with Delta) with split-KV for launches with few work-groups (a few
 * queries against many keys, or few heads): fa_bwd_dq_delta_kv's arguments
 * plus a caller-provided device workspace, sized by
 * fa_bwd_dq_workspace_bytes (0 when it does not split, for either element
 * type). With workspace == NULL, or when no split is needed, the call is
 * fa_bwd_dq_delta_kv; a non-NULL workspace smaller than needed is rejected
 * (FA_ERR_BAD_SHAPE). Splitting, work-groups over key ranges of at least
 * 1024 keys write fp32 partial dQ ([nsplit, B, Hq, N_q, D]) that a second
 * launch sums in a fixed order (deterministic). No counterpart in the
 * reference, whose backward is one launch per (key block, head) with dQ
 * inside (attention.py:754-770, 507-573). */
int64_t fa_bwd_dq_workspace_bytes(int64_t B, int64_t Hq, int64_t Hkv, int64_t N_q, int64_t N_kv,
                                  int64_t D, int causal);
int fa_bwd_dq_delta_ws(const fa_half_t* q, const fa_half_t* k, const fa_half_t* v,
                       const fa_half_t* o, const fa_half_t* dO, const float* lse,
                       float* delta, fa_half_t* dq,
                       int64_t B, int64_t Hq, int64_t Hkv, int64_t N_q, int64_t N_kv, int64_t D,
                       float scale, int causal, void* workspace, int64_t workspace_bytes,
                       void* stream);
int fa_bwd_dq_delta_ws_bf16(const fa_half_t* q, const fa_half_t* k, const fa_half_t* v,
                            const fa_half_t* o, const fa_half_t* dO, const float* lse,
                            float* delta, fa_half_t* dq,
                            int64_t B, int64_t Hq, int64_t Hkv, int64_t N_q, int64_t N_kv,
                            int64_t D, float scale, int causal, void* workspace,
                            int64_t workspace_bytes, void* stream);

/* Whole backward in one call, as TritonAttention.backward launches it
 * (attention.py:720-770: the Delta preprocess, then one _attn_bwd grid whose
 * programs run phase 1, dK/dV, and phase 2, dQ). Writes Delta ([B, Hq, N_q]
 * fp32, the reference's preprocess output), dq, dk and dv; shapes, element
 * type and key/value length as for fa_bwd_dq_delta_ws and fa_bwd_dkdv_ws_kv
 * (N_q == N_kv for self-attention). fa_bwd_workspace_bytes returns the bytes of
 * device workspace a call with these sizes needs (0 when nothing splits, for
 * either element type): the split partials of dQ and of dK/dV. With
 * workspace == NULL every launch runs in one pass; a non-NULL workspace smaller
 * than needed is rejected (FA_ERR_BAD_SHAPE). Launch plan: dQ with Delta fused,
 * then dK/dV (each split when its launch has few work-groups); except when
 * dK/dV splits and dQ does not and has at most 768 work-groups of 128 queries
 * (head_dim 32 or 64, the default tilings): then Delta runs as its own pass and the dK/dV and dQ work-groups run in one
 * combined launch, each filling the other's tail, before the dK/dV partials
 * are summed. Results are identical for a given plan on every call
 * (deterministic); the two plans differ only in how Delta reaches the dQ
 * kernel, within fp32 rounding. Concurrent calls need separate workspaces. */
int64_t fa_bwd_workspace_bytes(int64_t B, int64_t Hq, int64_t Hkv, int64_t N_q, int64_t N_kv,
                               int64_t D, int causal);
int fa_bwd(const fa_half_t* q, const fa_half_t* k, const fa_half_t* v,
           const fa_half_t* o, const fa_half_t* dO, const float* lse,
           float* delta, fa_half_t* dq, fa_half_t* dk, fa_half_t* dv,
           int64_t B, int64_t Hq, int64_t Hkv, int64_t N_q, int64_t N_kv, int64_t D,
           float scale, int causal, void* workspace, int64_t workspace_bytes, void* stream);
int fa_bwd_bf16(const fa_half_t* q, const fa_half_t* k, const fa_half_t* v,
                const fa_half_t* o, const fa_half_t* dO, const float* lse,
                float* delta, fa_half_t* dq, fa_half_t* dk, fa_half_t* dv,
                int64_t B, int64_t Hq, int64_t Hkv, int64_t N_q, int64_t N_kv, int64_t D,
                float scale, int causal, void* workspace, int64_t workspace_bytes,
                void* stream);

/* Forward that allocates nothing: fa_fwd_ws's computation with the split-KV
 * partials kept in a device array inside the library (64 MiB per GPU, held
 * until the process ends; under HIP's default deferred code-object loading
 * it is reserved at the first fa_fwd_noalloc call on a GPU, since its code
 * object holds no kernel) instead of a caller workspace. No counterpart in
 * the reference; it is for callers that cannot allocate device memory
 * (code under HIP graph capture, tight decoding loops, harnesses that forbid
 * hipMalloc). Same arguments, checks and results as fa_fwd_ws with a large
 * enough workspace; shapes that do not split run as fa_fwd_kv. A shape whose
 * partials need more than fa_fwd_noalloc_max_workspace_bytes() (as reported
 * by fa_fwd_workspace_bytes) is rejected with FA_ERR_TOO_LARGE before any HIP
 * call. The array's device address is looked up once per device, on the
 * first call with that device current; `stream` must belong to the current
 * device. All calls on one GPU share its array: calls that overlap in time on
 * one GPU (different streams or threads) race and must be serialised by the
 * caller. fp16 only. */
int fa_fwd_noalloc(const fa_half_t* q, const fa_half_t* k, const fa_half_t* v,
                   fa_half_t* o, float* lse,
                   int64_t B, int64_t Hq, int64_t Hkv, int64_t N_q, int64_t N_kv, int64_t D,
                   float scale, int causal, void* stream);
/* Bytes of the device array fa_fwd_noalloc uses (the largest workspace it serves). */
int64_t fa_fwd_noalloc_max_workspace_bytes(void);

/* Thread-local description of the last failure on the calling thread
 * ("" if none). The pointer stays valid until the next call on the thread. */
const char* fa_last_error(void);

/* FA_ABI_VERSION of the loaded library. */
int fa_abi_version(void);

/* Tiling table (replaces the Triton autotuner, attention.py:82-90, 353-381).
 * kernel: 0 = fwd, 1 = bwd_dkdv, 2 = bwd_dq.
 * fa_get_tiling writes the entry used for (kernel, D, causal):
 *   out[0] = waves per work-group, out[1] = rows per work-group,
 *   out[2] = streamed tile length (keys for fwd/dq, queries for dkdv),
 *   out[3] = variant index.
 * fa_num_tiling_variants / fa_describe_tiling_variant enumerate the
 * variants of a kernel (describe returns FA_ERR_BAD_TILING for one that is
 * not compiled for this head_dim); fa_set_tiling selects one for the
 * process (variant < 0 restores the default). Used by tuning sweeps.
 * A dK/dV launch that does not split runs the pipelined tiling on 16x16x32
 * MFMAs (variant 5) at D = 64, and at D = 32 without the mask, unless a
 * tiling was set; at D = 128 without the mask, launches of at most 128
 * queries run the classic 4 x 32 tiling (variant 1).
 * Three shape rules refine the dQ entries unless a tiling was set: launches
 * of at least 769 work-groups of 128 queries run the pipelined tiling on
 * 16x16x32 MFMAs (variant 5) at D = 64, and at D = 32 without the mask; at
 * D = 128 without the mask, fewer than 128 queries run the classic 4 x 32
 * tiling (variant 1); at D = 128 under the mask, launches of at least 128
 * queries and at most 768 work-groups of 128 queries run the pipelined
 * tiling (variant 4).
 * The forward's shape rules, unless a tiling was set: at D = 128, fewer than
 * 512 queries or fewer than 128 work-groups of 256 queries run the 4-wave
 * tiling (variant 2) instead of the 8-wave one; at D <= 64 under the mask,
 * launches of at least 2048 queries with W = B * Hq * (query tiles of 128)
 * between 384 and 512, or between 256 and 512 with at most 4096 queries, run
 * the pipelined 16x16x32 tiling with 64-query work-groups (variant 11), and
 * so do launches of at most 32 queries (decoding, any head size) whose queries
 * fit one of its work-groups (at most 64 / P queries, P = gcd(Hq / Hkv, 4)
 * query heads packed per work-group), and launches of 33 to 64 queries
 * without the mask, ahead of the D = 128 rule above;
 * otherwise at D = 32 under the mask,
 * launches over few heads (B * Hq * (query tiles of 128 + 1) < 1536) run the
 * two-key-group tiling (variant 8), and the other launches of at least 512
 * queries the pipelined tiling on 16x16x32 MFMAs (variant 10).
 * fa_set_tiling is safe to call while other threads launch:
 * each (kernel, D, causal) entry is an atomic that a launch reads once, so
 * the launch runs either the previous or the new tiling. */
int fa_get_tiling(int kernel, int64_t D, int causal, int* out4);
int fa_num_tiling_variants(int kernel, int64_t D, int causal);
int fa_describe_tiling_variant(int kernel, int64_t D, int causal, int variant, int* out4);
int fa_set_tiling(int kernel, int64_t D, int causal, int variant);

#ifdef __cplusplus
}
#endif

#endif /* FA_GFX950_H */
