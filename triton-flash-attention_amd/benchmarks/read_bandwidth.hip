// read_bandwidth.hip — a plain streaming read of a device buffer, the
// bandwidth reference for the decoding forward (read_bandwidth.py).
//
// read_kernel: every thread reads 16-byte vectors in a grid-stride loop, UNR
// loads in flight, and writes one word (the XOR of what it read) to out, so
// no load is dead. Indices stay below bytes / 16 (the unrolled loop tests its
// last load, the remainder loop each one); out holds one word per thread.
// spin_kernel: one wave that waits `ticks` of the constant-rate wall clock
// (wall_clock64, hipDeviceAttributeWallClockRate kHz; a bounded loop), to keep
// the queue busy while the host enqueues the next measurement.
//
// Built by read_bandwidth.py:
//   hipcc --offload-arch=gfx950 -O3 -shared -fPIC -o libread_bandwidth.so read_bandwidth.hip
#include <hip/hip_runtime.h>

#include <cstdint>

template <int UNR>
__global__ __launch_bounds__(256) void read_kernel(const uint4* __restrict__ src, int64_t n16,
                                                   uint32_t* __restrict__ out) {
  const int64_t tid = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t stride = (int64_t)gridDim.x * 256;
  uint32_t acc = 0;
  int64_t i = tid;
  for (; i + (UNR - 1) * stride < n16; i += UNR * stride) {
    uint4 v[UNR];
#pragma unroll
    for (int u = 0; u < UNR; ++u) v[u] = src[i + u * stride];
#pragma unroll
    for (int u = 0; u < UNR; ++u) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
  }
  for (; i < n16; i += stride) {
    const uint4 v = src[i];
    acc ^= v.x ^ v.y ^ v.z ^ v.w;
  }
  out[tid] = acc;
}

__global__ void spin_kernel(int64_t ticks, uint32_t* out) {
  const int64_t t0 = wall_clock64();
  int64_t n = 0;
  while (wall_clock64() - t0 < ticks) ++n;
  if (threadIdx.x == 0) out[0] = (uint32_t)n;
}

// out: blocks * 256 words. Returns the launch's hipError_t.
extern "C" int launch_read(const void* src, int64_t bytes, void* out, int blocks, int unr,
                           void* stream) {
  const int64_t n16 = bytes / 16;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const uint4* p = static_cast<const uint4*>(src);
  uint32_t* o = static_cast<uint32_t*>(out);
  if (unr == 8)
    hipLaunchKernelGGL(read_kernel<8>, dim3(blocks), dim3(256), 0, s, p, n16, o);
  else if (unr == 4)
    hipLaunchKernelGGL(read_kernel<4>, dim3(blocks), dim3(256), 0, s, p, n16, o);
  else
    hipLaunchKernelGGL(read_kernel<1>, dim3(blocks), dim3(256), 0, s, p, n16, o);
  return (int)hipGetLastError();
}

// out: one word.
extern "C" int launch_spin(int64_t ticks, void* out, void* stream) {
  hipLaunchKernelGGL(spin_kernel, dim3(1), dim3(64), 0, static_cast<hipStream_t>(stream), ticks,
                     static_cast<uint32_t*>(out));
  return (int)hipGetLastError();
}
