// Row kernels of the Dory decode step: the fused Q/K producer and the nGPT norms around the projections.
//
// Semantics (FP32 throughout; justnorm(x) = x / sqrt(sum x^2 + 1e-6), engine/src/kernels.cpp:162-175):
//   qk_rope_norm: NeoX RoPE of q and k at positions pos0 + row, then justnorm per head, then q *= qscale (per
//                 dim over all heads); k is not scaled (packs/dory/dory.cpp:482-490). The angle is
//                 FP32(pos) * inv_freq[i] with inv_freq computed on the host as the reference does
//                 (engine/src/kernels.cpp:191-201), so the angles are bit-identical; cos / sin run here.
//   slerp_norm:   x = justnorm(ya + lr * (yb - ya)), ya = justnorm(x), yb = justnorm(o) (kernels.cpp:177-189)
//   swiglu_norm:  g = justnorm(silu(g * sg) * (u * su)) (kernels.cpp:225-234 then justnorm, dory.cpp:474-475)
//   gate_norm:    a = justnorm(a * sigmoid(g * gs)) over all heads (dory.cpp:510-515)
//   add_norm:     out = justnorm(a + b), or justnorm(a) without b (dory.cpp:532-541)
// One work-group per row (per (row, head) for the producer); sums are wave reductions then one LDS step.
#include <cmath>

#include "common.hpp"
#include "rows.hpp"

namespace xtg::hip {

constexpr int kRowThreads = 256;

__device__ inline float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off);
  return v;
}

// Sum over the work-group (kRowThreads threads); every thread gets the total. red holds kRowThreads / 64 floats.
__device__ inline float group_sum(float v, float* red) {
  v = wave_sum(v);
  const int w = threadIdx.x >> 6;
  __syncthreads();   // red may still be read from a previous call
  if ((threadIdx.x & 63) == 0) red[w] = v;
  __syncthreads();
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < kRowThreads / 64; ++i) s += red[i];
  return s;
}

__device__ inline float inv_norm_of(float sumsq) { return 1.f / sqrtf(sumsq + 1e-6f); }

// One wave per (row, head): thread i holds the pair (i, i + d/2); d <= 128.
__global__ void __launch_bounds__(64) qk_rope_norm_kernel(float* __restrict__ q, float* __restrict__ k, int m,
                                                          int heads, int kv_heads, int d, long long pos0,
                                                          const float* __restrict__ inv_freq,
                                                          const float* __restrict__ qscale) {
  const int per_row = heads + kv_heads;
  const int row = blockIdx.x / per_row, hh = blockIdx.x % per_row;
  const bool is_q = hh < heads;
  const int h = is_q ? hh : hh - heads;
  float* v = is_q ? q + (size_t(row) * heads + h) * d : k + (size_t(row) * kv_heads + h) * d;
  const int half = d / 2, i = threadIdx.x;
  float o1 = 0.f, o2 = 0.f;
  if (i < half) {
    const float ang = float(pos0 + row) * inv_freq[i];
    const float c = cosf(ang), s = sinf(ang);
    const float x1 = v[i], x2 = v[i + half];
    o1 = x1 * c - x2 * s;
    o2 = x2 * c + x1 * s;
  }
  const float f = inv_norm_of(wave_sum(o1 * o1 + o2 * o2));
  if (i < half) {
    o1 *= f;
    o2 *= f;
    if (is_q && qscale) {
      o1 *= qscale[h * d + i];
      o2 *= qscale[h * d + i + half];
    }
    v[i] = o1;
    v[i + half] = o2;
  }
}

__global__ void __launch_bounds__(kRowThreads) slerp_norm_kernel(float* __restrict__ x, const float* __restrict__ o,
                                                                  const float* __restrict__ lr, int w) {
  __shared__ float red[kRowThreads / 64];
  float* xr = x + size_t(blockIdx.x) * w;
  const float* orow = o + size_t(blockIdx.x) * w;
  float sa = 0.f, sb = 0.f;
  for (int j = threadIdx.x; j < w; j += kRowThreads) {
    sa += xr[j] * xr[j];
    sb += orow[j] * orow[j];
  }
  const float fa = inv_norm_of(group_sum(sa, red)), fb = inv_norm_of(group_sum(sb, red));
  float s = 0.f;
  for (int j = threadIdx.x; j < w; j += kRowThreads) {
    const float ya = xr[j] * fa, yb = orow[j] * fb, t = ya + lr[j] * (yb - ya);
    xr[j] = t;
    s += t * t;
  }
  const float f = inv_norm_of(group_sum(s, red));
  for (int j = threadIdx.x; j < w; j += kRowThreads) xr[j] *= f;
}

__global__ void __launch_bounds__(kRowThreads) swiglu_norm_kernel(float* __restrict__ g, const float* __restrict__ u,
                                                                   const float* __restrict__ sg,
                                                                   const float* __restrict__ su, int w) {
  __shared__ float red[kRowThreads / 64];
  float* gr = g + size_t(blockIdx.x) * w;
  const float* ur = u + size_t(blockIdx.x) * w;
  float s = 0.f;
  for (int j = threadIdx.x; j < w; j += kRowThreads) {
    const float z = gr[j] * sg[j];
    const float t = z / (1.f + expf(-z)) * (ur[j] * su[j]);
    gr[j] = t;
    s += t * t;
  }
  const float f = inv_norm_of(group_sum(s, red));
  for (int j = threadIdx.x; j < w; j += kRowThreads) gr[j] *= f;
}

__global__ void __launch_bounds__(kRowThreads) gate_norm_kernel(float* __restrict__ a, const float* __restrict__ gate,
                                                                 const float* __restrict__ gs, int w) {
  __shared__ float red[kRowThreads / 64];
  float* ar = a + size_t(blockIdx.x) * w;
  const float* gr = gate + size_t(blockIdx.x) * w;
  float s = 0.f;
  for (int j = threadIdx.x; j < w; j += kRowThreads) {
    const float t = ar[j] * (1.f / (1.f + expf(-gr[j] * gs[j])));
    ar[j] = t;
    s += t * t;
  }
  const float f = inv_norm_of(group_sum(s, red));
  for (int j = threadIdx.x; j < w; j += kRowThreads) ar[j] *= f;
}

__global__ void __launch_bounds__(kRowThreads) add_norm_kernel(const float* __restrict__ a, const float* __restrict__ b,
                                                                float* __restrict__ out, int w) {
  __shared__ float red[kRowThreads / 64];
  const float* ar = a + size_t(blockIdx.x) * w;
  const float* br = b ? b + size_t(blockIdx.x) * w : nullptr;
  float* orow = out + size_t(blockIdx.x) * w;
  float s = 0.f;
  for (int j = threadIdx.x; j < w; j += kRowThreads) {
    const float t = ar[j] + (br ? br[j] : 0.f);
    s += t * t;
  }
  const float f = inv_norm_of(group_sum(s, red));
  for (int j = threadIdx.x; j < w; j += kRowThreads) orow[j] = (ar[j] + (br ? br[j] : 0.f)) * f;
}

std::string launch_qk_rope_norm(float* q, float* k, int m, int heads, int kv_heads, int d, long long pos0,
                                const float* inv_freq, const float* qscale, hipStream_t stream) {
  XTG_CHECK(d % 2 == 0 && d <= 128, "rope: head_dim %d (even, at most 128)", d);
  hipLaunchKernelGGL(qk_rope_norm_kernel, dim3(unsigned(m * (heads + kv_heads))), dim3(64), 0, stream, q, k, m, heads,
                     kv_heads, d, pos0, inv_freq, qscale);
  HIP_CHECK(hipGetLastError());
  return "qk_rope_norm_kernel";
}

std::string launch_slerp_norm(float* x, const float* o, const float* lr, int rows, int w, hipStream_t stream) {
  hipLaunchKernelGGL(slerp_norm_kernel, dim3(unsigned(rows)), dim3(kRowThreads), 0, stream, x, o, lr, w);
  HIP_CHECK(hipGetLastError());
  return "slerp_norm_kernel";
}

std::string launch_swiglu_norm(float* g, const float* u, const float* sg, const float* su, int rows, int w,
                               hipStream_t stream) {
  hipLaunchKernelGGL(swiglu_norm_kernel, dim3(unsigned(rows)), dim3(kRowThreads), 0, stream, g, u, sg, su, w);
  HIP_CHECK(hipGetLastError());
  return "swiglu_norm_kernel";
}

std::string launch_gate_norm(float* a, const float* gate, const float* gs, int rows, int w, hipStream_t stream) {
  hipLaunchKernelGGL(gate_norm_kernel, dim3(unsigned(rows)), dim3(kRowThreads), 0, stream, a, gate, gs, w);
  HIP_CHECK(hipGetLastError());
  return "gate_norm_kernel";
}

std::string launch_add_norm(const float* a, const float* b, float* out, int rows, int w, hipStream_t stream) {
  hipLaunchKernelGGL(add_norm_kernel, dim3(unsigned(rows)), dim3(kRowThreads), 0, stream, a, b, out, w);
  HIP_CHECK(hipGetLastError());
  return "add_norm_kernel";
}

}  // namespace xtg::hip
