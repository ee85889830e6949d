// atomic_dq_throughput.hip — throughput of fp32 atomic adds in the access
// pattern a fused backward would use to accumulate dQ inside the dK/dV kernel
// (FlashAttention-2's one-kernel backward), measured against plain stores to
// the same addresses. It backs the decision to keep a separate dQ kernel.
//
// Pattern: one work-group per (key tile of KT keys, head), tile-major and
// head-minor (so every key tile of a head runs on one XCD, as the library's
// launches place them); each work-group walks the 32-row query units its
// keys see (causal: rows >= its first key) and adds one 32 x 64 fp32 block
// per unit, split over its 4 waves in the lane layout of an MFMA result:
//   16x16: lane l holds column l%16 of rows 4*(l/16)+j  -> 4 x 64 B per instruction
//   32x32: lane l holds column l%32 of rows 4*(l/32)+j%4+8*(j/4) -> 2 x 128 B
// Scopes: agent and work-group scope compile to the same no-return
// global_atomic_add_f32 on gfx950; system scope sets sc1.
// Every address is head*N*64 + q*64 + d with q < N and d < 64 (in bounds); the
// result is checked on the host (each element ends as the number of key tiles
// that see its row).
//
// Build and run (no other files needed):
//   hipcc --offload-arch=gfx950 -O3 -munsafe-fp-atomics -o /tmp/atomic_dq \
//       benchmarks/atomic_dq_throughput.hip && /tmp/atomic_dq
#include <hip/hip_runtime.h>
#include <stdio.h>
#include <stdlib.h>

#include <vector>

#define CHECK(x)                                                                  \
  do {                                                                            \
    hipError_t e_ = (x);                                                          \
    if (e_ != hipSuccess) {                                                       \
      printf("HIP error %s at line %d\n", hipGetErrorString(e_), __LINE__);     \
      exit(1);                                                                    \
    }                                                                             \
  } while (0)

constexpr int D = 64;
constexpr int NW = 4;
constexpr int NI = 32 * D / NW / 64;  // instructions per wave per unit (8)

__device__ __forceinline__ void element(int layout, int gi, int lane, int* row, int* col) {
  if (layout == 0) {  // 16x16 tiles: 8 of them in 32 x 64, 4 instructions each
    const int t = gi / 4, j = gi % 4;
    *row = (t / 4) * 16 + 4 * (lane / 16) + j;
    *col = (t % 4) * 16 + lane % 16;
  } else {  // 32x32 tiles: 2 of them, 16 instructions each
    const int t = gi / 16, j = gi % 16;
    *row = 4 * (lane / 32) + j % 4 + 8 * (j / 4);
    *col = t * 32 + lane % 32;
  }
}

// OP 0: atomic add, agent scope; 1: atomic add, work-group scope; 2: atomic add,
// system scope; 3: plain store.
template <int LAYOUT, int OP>
__global__ __launch_bounds__(NW * 64) void probe(float* __restrict__ dq, int BH, int N, int KT,
                                                 int causal) {
  const int tile = blockIdx.x / BH;
  const int head = blockIdx.x % BH;
  const int lane = threadIdx.x & 63;
  const int w = threadIdx.x >> 6;
  float* base = dq + (size_t)head * N * D;
  for (int qu = causal ? tile * KT : 0; qu < N; qu += 32) {
#pragma unroll
    for (int i = 0; i < NI; ++i) {
      int row, col;
      element(LAYOUT, w * NI + i, lane, &row, &col);
      const int q = qu + row;
      if (q >= N) continue;
      float* p = base + (size_t)q * D + col;
      if constexpr (OP == 0)
        __hip_atomic_fetch_add(p, 1.0f, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      else if constexpr (OP == 1)
        __hip_atomic_fetch_add(p, 1.0f, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
      else if constexpr (OP == 2)
        __hip_atomic_fetch_add(p, 1.0f, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
      else
        *p = 1.0f;
    }
  }
}

using Kernel = void (*)(float*, int, int, int, int);

float time_ms(Kernel k, dim3 grid, float* dq, int BH, int N, int KT, int causal, size_t bytes) {
  hipEvent_t a, b;
  CHECK(hipEventCreate(&a));
  CHECK(hipEventCreate(&b));
  float best = 1e30f;
  for (int r = 0; r < 6; ++r) {  // the first launch warms up
    CHECK(hipMemset(dq, 0, bytes));
    CHECK(hipEventRecord(a));
    k<<<grid, NW * 64>>>(dq, BH, N, KT, causal);
    CHECK(hipGetLastError());
    CHECK(hipEventRecord(b));
    CHECK(hipEventSynchronize(b));
    float ms;
    CHECK(hipEventElapsedTime(&ms, a, b));
    if (r > 0 && ms < best) best = ms;
  }
  CHECK(hipEventDestroy(a));
  CHECK(hipEventDestroy(b));
  return best;
}

// Elements of the last launch (one launch after a memset) that differ from the
// expected count; -1 for the store kernels (expected value 1).
long check(const float* dq, int BH, int N, int KT, int causal, size_t bytes, bool store) {
  std::vector<float> h(bytes / 4);
  CHECK(hipMemcpy(h.data(), dq, bytes, hipMemcpyDeviceToHost));
  const int ntiles = (N + KT - 1) / KT;
  long bad = 0;
  for (int hh = 0; hh < BH; ++hh)
    for (int q = 0; q < N; ++q) {
      const float e = store ? 1.0f : (float)(causal ? q / KT + 1 : ntiles);
      for (int d = 0; d < D; ++d) bad += h[((size_t)hh * N + q) * D + d] != e;
    }
  return bad;
}

int main() {
  const int BH = 64, N = 4096;  // the headline shape: B4 x H16, N 4096, D 64
  const size_t bytes = (size_t)BH * N * D * 4;
  float* dq;
  CHECK(hipMalloc(&dq, bytes));
  struct Case {
    const char* name;
    Kernel k;
    bool store;
  };
  const Case cases[] = {
      {"atomic_agent_16x16", probe<0, 0>, false}, {"atomic_agent_32x32", probe<1, 0>, false},
      {"atomic_wg_16x16", probe<0, 1>, false},    {"atomic_wg_32x32", probe<1, 1>, false},
      {"atomic_system_32x32", probe<1, 2>, false}, {"store_16x16", probe<0, 3>, true},
      {"store_32x32", probe<1, 3>, true},
  };
  printf("op,key_tile,causal,us,payload_GB,TB_per_s,mismatches\n");
  for (int causal = 1; causal >= 0; --causal)
    for (int KT : {128, 256}) {
      const int ntiles = (N + KT - 1) / KT;
      double payload = 0;
      for (int t = 0; t < ntiles; ++t) payload += (double)(N - (causal ? t * KT : 0)) * D * 4;
      payload *= BH;
      const dim3 grid(ntiles * BH);
      for (const Case& c : cases) {
        const float ms = time_ms(c.k, grid, dq, BH, N, KT, causal, bytes);
        CHECK(hipMemset(dq, 0, bytes));
        c.k<<<grid, NW * 64>>>(dq, BH, N, KT, causal);
        CHECK(hipGetLastError());
        CHECK(hipDeviceSynchronize());
        const long bad = check(dq, BH, N, KT, causal, bytes, c.store);
        printf("%s,%d,%d,%.1f,%.3f,%.2f,%ld\n", c.name, KT, causal, ms * 1e3, payload / 1e9,
               payload / (ms * 1e-3) / 1e12, bad);
        fflush(stdout);
      }
    }
  CHECK(hipFree(dq));
  return 0;
}
