// mfma_shape_power.hip — sustained fp16 MFMA rate of the two gfx950 MFMA
// shapes the kernels can use, v_mfma_f32_32x32x16_f16 (32 cycles, 16
// accumulator registers) and v_mfma_f32_16x16x32_f16 (16 cycles, 4), under
// random operands, i.e. at the chip's power limit. It backs the choice of the
// 16x16x32 dQ tiling (fa_bwd_pipe16.hpp).
//   pure: a stream of independent MFMAs (4 accumulators of 32x32x16 or 8 of
//         16x16x32 per wave), 2 or 3 waves per SIMD, no memory traffic.
//   mix:  the same stream with the vector work of one 32 x 32 score unit of
//         the kernels interleaved: the forward's (16 fma, 16 exp, 16 add, 8
//         fp16 packs per 8 MFMA-equivalents of 32x32x16) or the backward's
//         (16 exp, 16 packs, 8 v_pk_mul_f16 per 16). Inline assembly keeps
//         the instruction counts fixed; results are not checked (timing only).
// Register-only loops; the only loads are in[tid] and in[256 + tid] with
// tid < 256 (in holds 512 half8); each thread writes one float.
//
// Build and run (no other files needed):
//   hipcc --offload-arch=gfx950 -O3 -Xclang -target-feature -Xclang -packed-fp32-ops \
//       -o /tmp/mfma_shape benchmarks/mfma_shape_power.hip && /tmp/mfma_shape
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstdlib>
#include <vector>

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float float16v __attribute__((ext_vector_type(16)));
typedef float float4v __attribute__((ext_vector_type(4)));

// ---- pure MFMA streams ------------------------------------------------------
template <int W>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(W)))
void pure32(const half8* in, float* out, int iters) {
  const int tid = threadIdx.x;
  half8 a0 = in[tid], b0 = in[256 + tid];
  half8 a1 = a0 * (_Float16)0.5f, b1 = b0 * (_Float16)-0.75f;
  float16v c0 = {}, c1 = {}, c2 = {}, c3 = {};
  for (int it = 0; it < iters; ++it) {
    c0 = __builtin_amdgcn_mfma_f32_32x32x16_f16(a0, b0, c0, 0, 0, 0);
    c1 = __builtin_amdgcn_mfma_f32_32x32x16_f16(a1, b0, c1, 0, 0, 0);
    c2 = __builtin_amdgcn_mfma_f32_32x32x16_f16(a0, b1, c2, 0, 0, 0);
    c3 = __builtin_amdgcn_mfma_f32_32x32x16_f16(a1, b1, c3, 0, 0, 0);
  }
  float s = 0.f;
#pragma unroll
  for (int j = 0; j < 16; ++j) s += c0[j] + c1[j] + c2[j] + c3[j];
  out[blockIdx.x * 256 + tid] = s;
}

template <int W>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(W)))
void pure16(const half8* in, float* out, int iters) {
  const int tid = threadIdx.x;
  half8 a0 = in[tid], b0 = in[256 + tid];
  half8 a1 = a0 * (_Float16)0.5f, b1 = b0 * (_Float16)-0.75f;
  half8 a2 = a0 * (_Float16)-1.25f, a3 = a1 * (_Float16)0.625f;
  float4v c[8] = {};
  for (int it = 0; it < iters; ++it) {
    c[0] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a0, b0, c[0], 0, 0, 0);
    c[1] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a1, b0, c[1], 0, 0, 0);
    c[2] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a2, b0, c[2], 0, 0, 0);
    c[3] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a3, b0, c[3], 0, 0, 0);
    c[4] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a0, b1, c[4], 0, 0, 0);
    c[5] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a1, b1, c[5], 0, 0, 0);
    c[6] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a2, b1, c[6], 0, 0, 0);
    c[7] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a3, b1, c[7], 0, 0, 0);
  }
  float s = 0.f;
#pragma unroll
  for (int k = 0; k < 8; ++k)
#pragma unroll
    for (int j = 0; j < 4; ++j) s += c[k][j];
  out[blockIdx.x * 256 + tid] = s;
}

// ---- MFMA streams with the kernels' vector work -------------------------------
#define M32(c, a, b) asm volatile("v_mfma_f32_32x32x16_f16 %0, %1, %2, %0" : "+v"(c) : "v"(a), "v"(b))
#define M16(c, a, b) asm volatile("v_mfma_f32_16x16x32_f16 %0, %1, %2, %0" : "+v"(c) : "v"(a), "v"(b))
#define FMA(d, s) asm volatile("v_fma_f32 %0, %1, %2, %3" : "=v"(d) : "v"(s), "s"(cc), "v"(mm_))
#define EXP(d, s) asm volatile("v_exp_f32 %0, %1" : "=v"(d) : "v"(s))
#define ADD(d, s) asm volatile("v_add_f32 %0, %0, %1" : "+v"(d) : "v"(s))
#define CVT(d, a, b) asm volatile("v_cvt_pk_f16_f32 %0, %1, %2" : "=v"(d) : "v"(a), "v"(b))
#define PKM(d, a) asm volatile("v_pk_mul_f16 %0, %0, %1" : "+v"(d) : "v"(a))
// One pair of scores: forward 2 fma, 2 exp, 2 add, 1 pack; backward 2 exp,
// 2 packs, 1 fp16 multiply.
#define FWD_PAIR() { ADD(l0, f0); ADD(l1, f1); CVT(p, f0, f1); EXP(f0, u0); EXP(f1, u1); FMA(u0, s0); FMA(u1, s1); }
#define BWD_PAIR() { EXP(f0, u0); EXP(f1, u1); CVT(p, f0, f1); CVT(q, u0, u1); PKM(p, q); }

// SHAPE 32 or 16; MIX 0 forward (8 MFMA-equivalents per unit), 1 backward (16).
template <int SHAPE, int MIX, int W>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(W)))
void mixed(const half8* in, float* out, int iters, float cc) {
  const int tid = threadIdx.x;
  half8 a0 = in[tid], b0 = in[256 + tid];
  half8 a1 = a0 * (_Float16)0.5f, b1 = b0 * (_Float16)-0.75f;
  float s0 = (float)a0[0], s1 = (float)a0[1], mm_ = (float)b0[2];
  float u0 = s0, u1 = s1, f0 = s0, f1 = s1, l0 = 0.f, l1 = 0.f;
  unsigned p = 0, q = 0;
  float16v c0 = {}, c1 = {}, c2 = {}, c3 = {};
  float4v d[8] = {};
  constexpr int NM = (MIX == 0 ? 8 : 16) * (SHAPE == 16 ? 2 : 1);
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int k = 0; k < NM; ++k) {
      if constexpr (SHAPE == 32) {
        if (k % 4 == 0) M32(c0, a0, b0);
        if (k % 4 == 1) M32(c1, a1, b0);
        if (k % 4 == 2) M32(c2, a0, b1);
        if (k % 4 == 3) M32(c3, a1, b1);
      } else {
        if (k % 8 == 0) M16(d[0], a0, b0);
        if (k % 8 == 1) M16(d[1], a1, b0);
        if (k % 8 == 2) M16(d[2], a0, b1);
        if (k % 8 == 3) M16(d[3], a1, b1);
        if (k % 8 == 4) M16(d[4], b0, a0);
        if (k % 8 == 5) M16(d[5], b1, a0);
        if (k % 8 == 6) M16(d[6], b0, a1);
        if (k % 8 == 7) M16(d[7], b1, a1);
      }
      // the unit's 8 pairs of scores, spread evenly over its NM MFMAs
      if ((k * 8) % NM == 0) {
        if constexpr (MIX == 0) FWD_PAIR() else BWD_PAIR()
      }
    }
  }
  float s = l0 + l1 + f0 + f1 + u0 + u1 + (float)((p ^ q) & 0xff);
#pragma unroll
  for (int j = 0; j < 16; ++j) s += c0[j] + c1[j] + c2[j] + c3[j];
#pragma unroll
  for (int k = 0; k < 8; ++k)
#pragma unroll
    for (int j = 0; j < 4; ++j) s += d[k][j];
  out[blockIdx.x * 256 + tid] = s;
}

template <class K>
static float best_ms(K kernel, int blocks, int reps, hipEvent_t e0, hipEvent_t e1) {
  float best = 1e30f;
  for (int r = 0; r < reps; ++r) {
    (void)hipEventRecord(e0);
    kernel(blocks);
    (void)hipEventRecord(e1);
    (void)hipEventSynchronize(e1);
    float ms;
    (void)hipEventElapsedTime(&ms, e0, e1);
    if (ms < best) best = ms;
  }
  return best;
}

int main() {
  std::vector<_Float16> h(512 * 8);
  srand(1);
  for (auto& v : h) v = (_Float16)(((rand() / (float)RAND_MAX) * 2.f - 1.f) * 1.7f);
  half8* din;
  float* dout;
  if (hipMalloc(&din, h.size() * 2) != hipSuccess || hipMalloc(&dout, (size_t)768 * 256 * 4) != hipSuccess)
    return 1;
  (void)hipMemcpy(din, h.data(), h.size() * 2, hipMemcpyHostToDevice);
  hipEvent_t e0, e1;
  (void)hipEventCreate(&e0);
  (void)hipEventCreate(&e1);
  struct Case {
    const char* name;
    int wps;        // work-groups (4 waves) per CU = waves per SIMD
    double flop;    // per wave and loop iteration
    int iters;
    void (*launch)(const half8*, float*, int, int);
  };
  const Case cases[] = {
      {"pure 32x32x16, 2 waves/SIMD", 2, 4 * 32768.0, 20000,
       [](const half8* i, float* o, int b, int n) { pure32<2><<<b, 256>>>(i, o, n); }},
      {"pure 16x16x32, 2 waves/SIMD", 2, 8 * 16384.0, 20000,
       [](const half8* i, float* o, int b, int n) { pure16<2><<<b, 256>>>(i, o, n); }},
      {"pure 32x32x16, 3 waves/SIMD", 3, 4 * 32768.0, 20000,
       [](const half8* i, float* o, int b, int n) { pure32<3><<<b, 256>>>(i, o, n); }},
      {"pure 16x16x32, 3 waves/SIMD", 3, 8 * 16384.0, 20000,
       [](const half8* i, float* o, int b, int n) { pure16<3><<<b, 256>>>(i, o, n); }},
      {"forward mix 32x32x16, 3 waves/SIMD", 3, 8 * 32768.0, 3000,
       [](const half8* i, float* o, int b, int n) { mixed<32, 0, 3><<<b, 256>>>(i, o, n, 0.18f); }},
      {"forward mix 16x16x32, 3 waves/SIMD", 3, 8 * 32768.0, 3000,
       [](const half8* i, float* o, int b, int n) { mixed<16, 0, 3><<<b, 256>>>(i, o, n, 0.18f); }},
      {"backward mix 32x32x16, 2 waves/SIMD", 2, 16 * 32768.0, 3000,
       [](const half8* i, float* o, int b, int n) { mixed<32, 1, 2><<<b, 256>>>(i, o, n, 0.18f); }},
      {"backward mix 16x16x32, 2 waves/SIMD", 2, 16 * 32768.0, 3000,
       [](const half8* i, float* o, int b, int n) { mixed<16, 1, 2><<<b, 256>>>(i, o, n, 0.18f); }},
  };
  printf("round,case,ms,TFLOP/s\n");
  for (int round = 0; round < 3; ++round) {
    for (const Case& cs : cases) {
      const int blocks = 256 * cs.wps;
      const float ms = best_ms([&](int b) { cs.launch(din, dout, b, cs.iters); }, blocks, 3, e0, e1);
      const double flop = (double)blocks * 4 * cs.iters * cs.flop;
      printf("%d,%s,%.3f,%.1f\n", round, cs.name, ms, flop / (ms * 1e-3) / 1e12);
      fflush(stdout);
    }
  }
  const hipError_t err = hipGetLastError();
  printf("status %s\n", hipGetErrorString(err));
  return err == hipSuccess ? 0 : 1;
}
