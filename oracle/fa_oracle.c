/*
 * fa_oracle.c — CPU restatement of the reference FlashAttention-2 algorithm,
 * in double precision.
 *
 * TEST INFRASTRUCTURE ONLY. This file is the checker for the gfx950 kernels:
 * only tests/, __graft_entry__.smoke() and bench.py's parity/baseline legs
 * load it. The product path (triton_flash_attention) never calls it and has
 * no CPU fallback through it.
 *
 * Every function cites the reference lines it restates
 * (/root/reference/triton_flash_attention/attention.py, docs/architecture.md).
 * Inputs are the fp16 values of the tensors, widened exactly to double.
 * Layouts: q, dq [B,Hq,N,D]; k, dk [B,Hkv,Nkv,D]; v, dv [B,Hkv,Nkv,Dv];
 * o, dO [B,Hq,N,Dv]; lse2, delta [B,Hq,N]; all contiguous row-major. The
 * reference kernels are self-attention with one head size (Nkv == N,
 * Dv == D); the closed forms also take Nkv != N and Dv != D, inputs the
 * reference hands to torch SDPA (attention.py:639-646, 830-838), with SDPA's
 * causal mask for unequal lengths: query i sees keys j <= i (the lower
 * triangle of the N x Nkv all-ones matrix).
 *
 * Pinning (what checks each function; see tests/test_oracle.py):
 *   oracle_round_half      numpy float16 conversion on 10^5 values incl. ties,
 *                          subnormals and overflow
 *   oracle_fwd_direct      torch fp64 SDPA and logsumexp (Nkv == N and
 *                          Nkv != N, Dv == D and Dv != D); golden fixtures;
 *                          closed forms (causal
 *                          row 0, Q=0 uniform attention, constant V, N=1)
 *   oracle_fwd_online      oracle_fwd_direct (tiling independence at fp64),
 *                          and with round_p=1 the fp16-P rounding bound
 *   oracle_bwd_preprocess  exact dot products of small integers; golden Delta
 *   oracle_bwd             torch fp64 autograd through SDPA (Nkv == N and
 *                          Nkv != N, where keys past the last causal query
 *                          get zero gradients; Dv != D); golden fixtures;
 *                          closed forms (constant V -> dQ = dK = 0, N=1);
 *                          GQA group sum == MHA with repeated K/V
 *   oracle_bwd, fold = 1/2 equal to fold = 0 when c32 is a power of two (the
 *                          rounding of c32 x is then exact); a numpy / torch
 *                          restatement with np.float16 / torch.bfloat16 casts
 *                          of the scaled operands on tiny inputs; differs from
 *                          fold = 0 by no more than a half-ulp relative operand
 *                          perturbation allows, and does differ at a generic
 *                          scale
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define INV_LN2 1.4426950408889634 /* attention.py:20 */

/* Round a double to the nearest IEEE binary16 value (ties to even),
 * including subnormals and overflow to infinity; returned as a double.
 * Restates the fp16 casts of the reference (p.to(tl.float16), attention.py:73;
 * ds_t.to(tl.float16), 305; ds.to(tl.float16), 347; acc.to(Out dtype), 234). */
double oracle_round_half(double x) {
  if (isnan(x) || isinf(x) || x == 0.0) return x;
  double a = fabs(x);
  if (a >= 65520.0) return copysign(INFINITY, x); /* 65504 + half an ulp(65504) */
  int e2;
  frexp(a, &e2);          /* a = m * 2^e2, m in [0.5, 1)  ->  a in [2^(e2-1), 2^e2) */
  int e = e2 - 1;         /* unbiased exponent of a */
  if (e < -14) e = -14;   /* subnormal range shares the quantum 2^-24 */
  double quantum = ldexp(1.0, e - 10);
  double r = nearbyint(a / quantum) * quantum; /* default rounding: nearest, ties to even */
  return copysign(r, x);
}

void oracle_round_half_array(const double* x, double* y, int64_t n) {
  for (int64_t i = 0; i < n; ++i) y[i] = oracle_round_half(x[i]);
}

static double dot(const double* a, const double* b, int64_t d) {
  double s = 0.0;
  for (int64_t i = 0; i < d; ++i) s += a[i] * b[i];
  return s;
}

/* GQA head map, attention.py:128-131: kv_head = q_head // (Hq / Hkv). */
static int64_t kv_head_of(int64_t b, int64_t hq, int64_t Hq, int64_t Hkv) {
  return b * Hkv + hq / (Hq / Hkv);
}

/* Closed form of the forward: per query row i,
 *   s_ij  = (q_i . k_j) * scale * log2(e)      (log2 domain, attention.py:61, 177)
 *   valid = j < Nkv and (not causal or j <= i) (attention.py:57, 63-66)
 *   lse2_i = log2(sum_valid exp2(s_ij))        (attention.py:230)
 *   o_i    = sum_valid exp2(s_ij - lse2_i) v_j (attention.py:231)
 * Two passes over the keys, no tiling, no intermediate rounding. */
void oracle_fwd_direct(const double* q, const double* k, const double* v, int64_t B, int64_t Hq,
                       int64_t Hkv, int64_t N, int64_t Nkv, int64_t D, int64_t Dv, double scale,
                       int causal, double* o, double* lse2) {
  const double c = scale * INV_LN2;
#pragma omp parallel for schedule(dynamic)
  for (int64_t bh = 0; bh < B * Hq; ++bh) {
    const int64_t b = bh / Hq, hq = bh % Hq;
    const int64_t kvh = kv_head_of(b, hq, Hq, Hkv);
    const double* Q = q + bh * N * D;
    const double* K = k + kvh * Nkv * D;
    const double* V = v + kvh * Nkv * Dv;
    double* s = (double*)malloc(sizeof(double) * (size_t)Nkv);
    for (int64_t i = 0; i < N; ++i) {
      const int64_t last = causal && i < Nkv - 1 ? i : Nkv - 1;
      double mx = -INFINITY;
      for (int64_t j = 0; j <= last; ++j) {
        s[j] = dot(Q + i * D, K + j * D, D) * c;
        if (s[j] > mx) mx = s[j];
      }
      double l = 0.0;
      for (int64_t j = 0; j <= last; ++j) l += exp2(s[j] - mx);
      const double lse = mx + log2(l);
      double* out = o + (bh * N + i) * Dv;
      for (int64_t d = 0; d < Dv; ++d) out[d] = 0.0;
      for (int64_t j = 0; j <= last; ++j) {
        const double p = exp2(s[j] - lse);
        const double* vj = V + j * Dv;
        for (int64_t d = 0; d < Dv; ++d) out[d] += p * vj[d];
      }
      lse2[bh * N + i] = lse;
    }
    free(s);
  }
}

/* The reference's online-softmax forward (attention.py:25-79 inner loop,
 * 170-234 program body), one query row at a time but with the reference's
 * tile structure:
 *   causal:       STAGE 1 keys [0, start_m*BM) unmasked, then STAGE 2 keys
 *                 [start_m*BM, (start_m+1)*BM) with the element mask
 *                 (attention.py:43-49, 179-211); start_m = i / BM
 *   bidirectional: STAGE 3 keys [0, N) (attention.py:48-49, 212-228)
 * in tiles of BN keys; state m = -inf, l = 1 (attention.py:173-174); per tile
 *   m_new = max(m, max s); p = exp2(s - m_new); alpha = exp2(m - m_new)
 *   l = l*alpha + sum p; acc = acc*alpha + P V; m = m_new     (attention.py:68-74)
 * with P rounded to fp16 for the P.V product when round_p != 0
 * (p.to(tl.float16), attention.py:73) while l sums the unrounded p (71).
 * Epilogue: lse2 = m + log2(l); o = acc / l (attention.py:230-231). */
void oracle_fwd_online(const double* q, const double* k, const double* v, int64_t B, int64_t Hq,
                       int64_t Hkv, int64_t N, int64_t D, double scale, int causal,
                       int64_t block_m, int64_t block_n, int round_p, double* o, double* lse2) {
  const double c = scale * INV_LN2;
#pragma omp parallel for schedule(dynamic)
  for (int64_t bh = 0; bh < B * Hq; ++bh) {
    const int64_t b = bh / Hq, hq = bh % Hq;
    const int64_t kvh = kv_head_of(b, hq, Hq, Hkv);
    const double* Q = q + bh * N * D;
    const double* K = k + kvh * N * D;
    const double* V = v + kvh * N * D;
    double* s = (double*)malloc(sizeof(double) * (size_t)block_n);
    double* acc = (double*)malloc(sizeof(double) * (size_t)D);
    for (int64_t i = 0; i < N; ++i) {
      double m = -INFINITY, l = 1.0;
      for (int64_t d = 0; d < D; ++d) acc[d] = 0.0;
      const int64_t start_m = i / block_m;
      int64_t ranges[2][3]; /* lo, hi, masked */
      int nranges;
      if (causal) {
        ranges[0][0] = 0;
        ranges[0][1] = start_m * block_m;
        ranges[0][2] = 0;
        ranges[1][0] = start_m * block_m;
        ranges[1][1] = (start_m + 1) * block_m;
        ranges[1][2] = 1;
        nranges = 2;
      } else {
        ranges[0][0] = 0;
        ranges[0][1] = N;
        ranges[0][2] = 0;
        nranges = 1;
      }
      for (int r = 0; r < nranges; ++r) {
        for (int64_t n0 = ranges[r][0]; n0 < ranges[r][1]; n0 += block_n) {
          double mt = -INFINITY;
          for (int64_t t = 0; t < block_n; ++t) {
            const int64_t j = n0 + t;
            int ok = j < N;
            if (ranges[r][2]) ok = ok && (i >= j);
            s[t] = ok ? dot(Q + i * D, K + j * D, D) * c : -INFINITY;
            if (s[t] > mt) mt = s[t];
          }
          const double m_new = m > mt ? m : mt;
          const double alpha = exp2(m - m_new);
          double psum = 0.0;
          for (int64_t d = 0; d < D; ++d) acc[d] *= alpha;
          for (int64_t t = 0; t < block_n; ++t) {
            const double p = exp2(s[t] - m_new);
            psum += p;
            const int64_t j = n0 + t;
            if (j >= N || p == 0.0) continue; /* zero-padded V rows (attention.py:60) */
            const double pv = round_p ? oracle_round_half(p) : p;
            const double* vj = V + j * D;
            for (int64_t d = 0; d < D; ++d) acc[d] += pv * vj[d];
          }
          l = l * alpha + psum;
          m = m_new;
        }
      }
      lse2[bh * N + i] = m + log2(l);
      double* out = o + (bh * N + i) * D;
      for (int64_t d = 0; d < D; ++d) out[d] = acc[d] / l;
    }
    free(s);
    free(acc);
  }
}

/* Delta_i = sum_d O_id * dO_id (attention.py:237-255), O and dO as stored (fp16). */
void oracle_bwd_preprocess(const double* o, const double* dO, int64_t rows, int64_t D,
                           double* delta) {
#pragma omp parallel for schedule(static)
  for (int64_t r = 0; r < rows; ++r) delta[r] = dot(o + r * D, dO + r * D, D);
}

/* Round a float to the nearest bfloat16 value (ties to even), widened back. */
static double round_bf16(float f) {
  uint32_t b;
  memcpy(&b, &f, sizeof b);
  b += 0x7fffu + ((b >> 16) & 1u);
  b &= 0xffff0000u;
  float r;
  memcpy(&r, &b, sizeof r);
  return (double)r;
}

/* rnd(fp32(c32 * x)) for every element, rnd = fp16 (fold = 1) or bf16
 * (fold = 2): the reference backward's scaled score operands,
 * k_scaled = (k * (sm_scale * _INV_LN2)).to(tl.float16) and q_scaled
 * likewise (attention.py:435, 515), an fp32 product rounded to the element
 * type (bf16 is this build's added element type). */
static void scaled_operand(const double* x, int64_t n, float c32, int fold, double* out) {
  for (int64_t i = 0; i < n; ++i) {
    const float p = c32 * (float)x[i];
    out[i] = fold == 2 ? round_bf16(p) : oracle_round_half((double)p);
  }
}

/* Backward from the saved base-2 LSE (attention.py:258-350, 403-573;
 * docs/architecture.md:75-90), closed form per (query row i, key j):
 *   P_ij  = exp2(s_ij - lse2_i) on visible pairs, 0 elsewhere (296-300, 339-343)
 *           with s_ij = c q_i.k_j (fold = 0, exact), or, as the reference
 *           computes it (fold = 1), s_ij = q_i.fp16(c32 k_j) for dK, dV
 *           (297, 435) and s_ij = fp16(c32 q_i).k_j for dQ (340, 515),
 *           c32 = fp32(fp32(scale) * fp32(1/ln 2)); fold = 2 rounds to bf16
 *   dV_j += P_ij dO_i                                          (302)
 *   dP_ij = dO_i . V_j                                         (303, 345)
 *   dS_ij = P_ij (dP_ij - Delta_i)                             (304, 346; the ln2
 *           factor there cancels the 1/ln2 folded into the final scale, 499, 572)
 *   dQ_i += scale dS_ij K_j ;  dK_j += scale dS_ij Q_i         (305, 347, 499, 572)
 * GQA: dK/dV of a key/value head are the sums over the Hq/Hkv query heads that
 * read it (the reference's atomic_add, 503-505). Work is split by key/value
 * head so each output row has one writer. */
void oracle_bwd(const double* q, const double* k, const double* v, const double* dO,
                const double* lse2, const double* delta, int64_t B, int64_t Hq, int64_t Hkv,
                int64_t N, int64_t Nkv, int64_t D, int64_t Dv, double scale, int causal,
                int fold, double* dq, double* dk, double* dv) {
  const double c = scale * INV_LN2;
  const float c32 = (float)scale * (float)INV_LN2;
  const int64_t group = Hq / Hkv;
#pragma omp parallel for schedule(dynamic)
  for (int64_t bkv = 0; bkv < B * Hkv; ++bkv) {
    const int64_t b = bkv / Hkv, hkv = bkv % Hkv;
    const double* K = k + bkv * Nkv * D;
    const double* V = v + bkv * Nkv * Dv;
    double* dK = dk + bkv * Nkv * D;
    double* dV = dv + bkv * Nkv * Dv;
    memset(dK, 0, sizeof(double) * (size_t)(Nkv * D));
    memset(dV, 0, sizeof(double) * (size_t)(Nkv * Dv));
    double* ks = fold ? (double*)malloc(sizeof(double) * (size_t)(Nkv * D)) : NULL;
    double* qs = fold ? (double*)malloc(sizeof(double) * (size_t)(N * D)) : NULL;
    if (fold) scaled_operand(K, Nkv * D, c32, fold, ks);
    for (int64_t gi = 0; gi < group; ++gi) {
      const int64_t bh = b * Hq + hkv * group + gi;
      const double* Q = q + bh * N * D;
      const double* G = dO + bh * N * Dv;
      double* dQ = dq + bh * N * D;
      if (fold) scaled_operand(Q, N * D, c32, fold, qs);
      for (int64_t i = 0; i < N; ++i) {
        const double* qi = Q + i * D;
        const double* gi_row = G + i * Dv;
        double* dqi = dQ + i * D;
        for (int64_t d = 0; d < D; ++d) dqi[d] = 0.0;
        const double lse = lse2[bh * N + i];
        const double dlt = delta[bh * N + i];
        const int64_t last = causal && i < Nkv - 1 ? i : Nkv - 1;
        for (int64_t j = 0; j <= last; ++j) {
          /* p_k feeds dK and dV, p_q feeds dQ; equal unless fold */
          const double p_k = fold ? exp2(dot(qi, ks + j * D, D) - lse)
                                  : exp2(dot(qi, K + j * D, D) * c - lse);
          const double p_q = fold ? exp2(dot(qs + i * D, K + j * D, D) - lse) : p_k;
          const double dp = dot(gi_row, V + j * Dv, Dv);
          const double ds_k = p_k * (dp - dlt);
          const double ds_q = p_q * (dp - dlt);
          double* dvj = dV + j * Dv;
          double* dkj = dK + j * D;
          const double* kj = K + j * D;
          for (int64_t d = 0; d < Dv; ++d) dvj[d] += p_k * gi_row[d];
          for (int64_t d = 0; d < D; ++d) {
            dkj[d] += scale * ds_k * qi[d];
            dqi[d] += scale * ds_q * kj[d];
          }
        }
      }
    }
    free(ks);
    free(qs);
  }
}
