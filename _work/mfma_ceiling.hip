// Sustained fp16 MFMA throughput on one MI355X with random versus zero operands.
//
// A stream of independent v_mfma_f32_32x32x16_f16 (four accumulators per
// wave, two waves per SIMD, no memory traffic inside the loop) is the most an
// attention kernel's matrix work can reach. The chip caps its power: with
// random N(0,1) fp16 operands the engine clock falls well below the nominal
// 2.4 GHz while the same stream on zeros runs near it, so the practical
// ceiling for the attention kernels (whose operands are random-like) is the
// random-operand figure printed here, not the nominal 2516.6 TFLOP/s.
//
// Build and run (prints one line per measurement, three passes):
//   hipcc --offload-arch=gfx950 -O3 -Xclang -target-feature -Xclang -packed-fp32-ops \
//     -o /tmp/mfma_ceiling triton-flash-attention_amd/benchmarks/mfma_ceiling.hip
//   /tmp/mfma_ceiling
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstdlib>

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef float float16v __attribute__((ext_vector_type(16)));

namespace {

constexpr int kAcc = 4;              // independent accumulators per wave
constexpr int kBlocks = 512;         // x 4 waves = 2 waves per SIMD on 256 CUs
constexpr int kIters = 4000;         // x 16 MFMAs per wave
constexpr size_t kPool = 1u << 20;   // half8 operand pool (16 MiB)

__global__ __launch_bounds__(256) void mfma_stream(const half8* __restrict__ src, float* out,
                                                   int iters) {
  const int t = blockIdx.x * 256 + threadIdx.x;
  half8 a[4], b[4];
  for (int i = 0; i < 4; ++i) {
    a[i] = src[(size_t)(t * 8 + i) & (kPool - 1)];
    b[i] = src[(size_t)(t * 8 + 4 + i) & (kPool - 1)];
  }
  float16v c[kAcc];
  for (int j = 0; j < kAcc; ++j)
    for (int i = 0; i < 16; ++i) c[j][i] = 0.f;
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int k = 0; k < 4; ++k)
#pragma unroll
      for (int j = 0; j < kAcc; ++j)
        c[j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(a[k], b[(k + j) & 3], c[j], 0, 0, 0);
  }
  float s = 0.f;
  for (int j = 0; j < kAcc; ++j)
    for (int i = 0; i < 16; ++i) s += c[j][i];
  out[t] = s;  // keeps the stream live
}

bool ok(hipError_t e, const char* what) {
  if (e != hipSuccess) std::fprintf(stderr, "%s: %s\n", what, hipGetErrorString(e));
  return e == hipSuccess;
}

}  // namespace

int main() {
  half8* host = static_cast<half8*>(std::malloc(kPool * sizeof(half8)));
  if (host == nullptr) return 1;
  std::srand(1);
  for (size_t i = 0; i < kPool; ++i)
    for (int e = 0; e < 8; ++e) {
      float u = 0.f;  // Irwin-Hall(4), centred and scaled to unit variance
      for (int r = 0; r < 4; ++r) u += std::rand() / (float)RAND_MAX;
      host[i][e] = (_Float16)((u - 2.0f) * 1.732f);
    }
  half8 *rnd = nullptr, *zero = nullptr;
  float* out = nullptr;
  if (!ok(hipMalloc(&rnd, kPool * sizeof(half8)), "hipMalloc") ||
      !ok(hipMalloc(&zero, kPool * sizeof(half8)), "hipMalloc") ||
      !ok(hipMalloc(&out, kBlocks * 256 * sizeof(float)), "hipMalloc") ||
      !ok(hipMemcpy(rnd, host, kPool * sizeof(half8), hipMemcpyHostToDevice), "hipMemcpy") ||
      !ok(hipMemset(zero, 0, kPool * sizeof(half8)), "hipMemset"))
    return 1;
  hipEvent_t e0, e1;
  if (!ok(hipEventCreate(&e0), "event") || !ok(hipEventCreate(&e1), "event")) return 1;
  const double flops = (double)kBlocks * 4 * kIters * 4 * kAcc * 32768.0;
  for (int pass = 0; pass < 3; ++pass)
    for (int which = 0; which < 2; ++which) {
      const half8* src = which ? zero : rnd;
      hipLaunchKernelGGL(mfma_stream, dim3(kBlocks), dim3(256), 0, 0, src, out, kIters);
      if (!ok(hipDeviceSynchronize(), "warmup")) return 1;
      (void)hipEventRecord(e0);
      for (int r = 0; r < 5; ++r)
        hipLaunchKernelGGL(mfma_stream, dim3(kBlocks), dim3(256), 0, 0, src, out, kIters);
      (void)hipEventRecord(e1);
      if (!ok(hipEventSynchronize(e1), "timing")) return 1;
      float ms = 0.f;
      (void)hipEventElapsedTime(&ms, e0, e1);
      ms /= 5;
      const double tf = flops / (ms * 1e-3) / 1e12;
      std::printf("%-6s operands: %.3f ms per launch, %.1f TFLOP/s = %.1f%% of 2516.6\n",
                  which ? "zero" : "random", ms, tf, 100.0 * tf / 2516.6);
    }
  std::free(host);
  return 0;
}
