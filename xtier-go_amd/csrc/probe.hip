// The device's streaming-read roofline (the reference's readsum probe, tests/gpu_probe.cpp:59-66): every byte of a
// buffer read once in 16-byte loads and XOR-folded, one 32-bit partial per work-group, so the reads cannot be
// dropped. Each thread issues all of its loads before it folds any (kProbeLoads per thread, consecutive threads
// reading consecutive 16-byte blocks per load), nontemporal like the GEMV's weight stream.
#include <hip/hip_runtime.h>

#include "common.hpp"
#include "kernels.hpp"

namespace xtg::hip {

namespace {
constexpr int kProbeThreads = 256, kProbeLoads = 8;
}

__global__ void __launch_bounds__(kProbeThreads) read_probe_kernel(const uint4* __restrict__ src, size_t n16,
                                                                   uint32_t* __restrict__ out) {
  typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
  __shared__ uint32_t red[kProbeThreads / 64];
  const size_t base = size_t(blockIdx.x) * kProbeThreads * kProbeLoads + threadIdx.x;
  u32x4 v[kProbeLoads];
#pragma unroll
  for (int i = 0; i < kProbeLoads; ++i) {
    const size_t at = base + size_t(i) * kProbeThreads;
    v[i] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(src) + (at < n16 ? at : n16 - 1));
  }
  uint32_t acc = 0;
#pragma unroll
  for (int i = 0; i < kProbeLoads; ++i) {
    const size_t at = base + size_t(i) * kProbeThreads;
    if (at < n16) acc ^= v[i][0] ^ v[i][1] ^ v[i][2] ^ v[i][3];
  }
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) acc ^= uint32_t(__shfl_xor(int(acc), off));
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = acc;
  __syncthreads();
  if (threadIdx.x == 0) {
    uint32_t s = 0;
#pragma unroll
    for (int i = 0; i < kProbeThreads / 64; ++i) s ^= red[i];
    out[blockIdx.x] = s;
  }
}

size_t read_probe_groups(size_t bytes) {
  const size_t per = size_t(kProbeThreads) * kProbeLoads * 16;
  return (bytes + per - 1) / per;
}

std::string launch_read_probe(const void* src, size_t bytes, uint32_t* out, hipStream_t stream) {
  XTG_CHECK(src && out && bytes >= 16 && bytes % 16 == 0, "read probe: %zu bytes (a positive multiple of 16)", bytes);
  XTG_CHECK(reinterpret_cast<uintptr_t>(src) % 16 == 0, "read probe: the buffer must be 16-byte aligned");
  const size_t wgs = read_probe_groups(bytes);
  XTG_CHECK(wgs < (size_t(1) << 31), "read probe: %zu bytes", bytes);
  hipLaunchKernelGGL(read_probe_kernel, dim3(unsigned(wgs)), dim3(kProbeThreads), 0, stream,
                     static_cast<const uint4*>(src), bytes / 16, out);
  HIP_CHECK(hipGetLastError());
  return "read_probe_kernel";
}

}  // namespace xtg::hip
