// Row kernels of the Dory decode step: the Q/K producer of the reference's host path and the nGPT norms around
// the projections.
//
// Semantics (FP32 throughout; justnorm(x) = x / sqrt(sum x^2 + 1e-6), engine/src/kernels.cpp:162-175):
//   qk_rope_norm: NeoX RoPE of q and k at positions pos0 + row, then justnorm per head, then q *= qscale (per
//                 dim over all heads); k is not scaled (packs/dory/dory.cpp:482-490). The angle is
//                 FP32(pos) * inv_freq[i] with inv_freq computed on the host as the reference does
//                 (engine/src/kernels.cpp:191-201), so the angles are bit-identical; cos / sin run here.
//   slerp_norm:   x = justnorm(ya + lr * (yb - ya)), ya = justnorm(x), yb = justnorm(o) (kernels.cpp:177-189)
//   swiglu_norm:  g = justnorm(silu(g * sg) * (u * su)) (kernels.cpp:225-234 then justnorm, dory.cpp:474-475)
//   gate_norm:    a = justnorm(a * sigmoid(g * gs)) over all heads (dory.cpp:510-515)
//   add_norm:     out = justnorm(a + b), or justnorm(a) without b (dory.cpp:532-541); out may be a or b (each
//                 thread reads its elements before it writes them)
// The norms run one work-group of 512 threads per row with the whole row in registers (one read of each input,
// the sums as block reductions), and can also write the row as the next projection's GEMV operand (the f16
// high / low split prep_x_kernel makes), so no separate operand pass runs between a norm and its projection.
#include <climits>
#include <cmath>

#include "common.hpp"
#include "rowops.hpp"
#include "rows.hpp"

namespace xtg::hip {

constexpr int kNormThreads = 512;
constexpr int kNormRed = 2 * kNormThreads / 64;

// One wave per (row, head): thread t holds the pairs (i, i + d/2) for i = t + 64 u < d/2; d <= 256.
__global__ void __launch_bounds__(64) qk_rope_norm_kernel(float* __restrict__ q, float* __restrict__ k, int m,
                                                          int heads, int kv_heads, int d, long long pos0,
                                                          const float* __restrict__ inv_freq,
                                                          const float* __restrict__ qscale) {
  const int per_row = heads + kv_heads;
  const int row = blockIdx.x / per_row, hh = blockIdx.x % per_row;
  const bool is_q = hh < heads;
  const int h = is_q ? hh : hh - heads;
  float* v = is_q ? q + (size_t(row) * heads + h) * d : k + (size_t(row) * kv_heads + h) * d;
  const int half = d / 2;
  float o1[2] = {0.f, 0.f}, o2[2] = {0.f, 0.f}, ss = 0.f;
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    const int i = int(threadIdx.x) + 64 * u;
    if (i < half) {
      const float ang = float(pos0 + row) * inv_freq[i];
      const float c = cosf(ang), s = sinf(ang);
      const float x1 = v[i], x2 = v[i + half];
      o1[u] = x1 * c - x2 * s;
      o2[u] = x2 * c + x1 * s;
      ss += o1[u] * o1[u] + o2[u] * o2[u];
    }
  }
  const float f = inv_norm_of(wave_sum(ss));
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    const int i = int(threadIdx.x) + 64 * u;
    if (i < half) {
      float a = o1[u] * f, b = o2[u] * f;
      if (is_q && qscale) {
        a *= qscale[h * d + i];
        b *= qscale[h * d + i + half];
      }
      v[i] = a;
      v[i + half] = b;
    }
  }
}

// The normalised row t * f: written to out (if any) and as operand row j (if any). The row's largest magnitude
// rides with the norm's sum: scaling by f > 0 is monotone under rounding, so max |t f| = fl(max |t| * f) exactly,
// and one exchange serves both.
template <int U>
__device__ inline void finish_row(float (&t)[U][8], float sumsq, int w, bool vec, float* out, f16x8* xop, float* xinv,
                                  size_t ostride, float* red) {
  float mx = 0.f;
  if (xop) {
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
      for (int e = 0; e < 8; ++e) mx = fmaxf(mx, fabsf(t[u][e]));
  }
  block_sum_max<kNormThreads>(sumsq, mx, red);
  const float f = inv_norm_of(sumsq);
#pragma unroll
  for (int u = 0; u < U; ++u)
#pragma unroll
    for (int e = 0; e < 8; ++e) t[u][e] *= f;
  if (out) store_row<kNormThreads, U>(out, w, vec, t);
  if (xop) emit_operand_mx<kNormThreads, U>(t, w, int(blockIdx.x), xop, xinv, ostride, mx * f);
}

// A second part of a row split in two along K (GemvCall::ksplit): r += that part, element by element (first part +
// second, the one order).
template <int U>
__device__ inline void add_part(const float* row, int w, int vec, float (&r)[U][8]) {
  float p[U][8];
  load_row<kNormThreads, U>(row, w, vec, p);
#pragma unroll
  for (int u = 0; u < U; ++u)
#pragma unroll
    for (int e = 0; e < 8; ++e) r[u][e] += p[u][e];
}

// PART: o holds two parts of a row split along K (the second at o + part), added as they load; its loads go out with
// the others (a load behind a branch would wait for them).
template <int U, bool PART>
__device__ inline void slerp_norm_row(float* __restrict__ x, const float* __restrict__ o, size_t part,
                                      const float* __restrict__ lr, int w, int vec, f16x8* __restrict__ xop,
                                      float* __restrict__ xinv, size_t ostride) {
  __shared__ float red[kNormRed];
  float* xr = x + size_t(blockIdx.x) * w;
  float a[U][8], b[U][8], l[U][8];
  load_row<kNormThreads, U>(xr, w, vec, a);
  load_row<kNormThreads, U>(o + size_t(blockIdx.x) * w, w, vec, b);
  load_row<kNormThreads, U>(lr, w, vec, l);
  if constexpr (PART) add_part<U>(o + part + size_t(blockIdx.x) * w, w, vec, b);
  float sa = 0.f, sb = 0.f;
#pragma unroll
  for (int u = 0; u < U; ++u)
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      sa += a[u][e] * a[u][e];
      sb += b[u][e] * b[u][e];
    }
  block_sum2<kNormThreads>(sa, sb, red);
  const float fa = inv_norm_of(sa), fb = inv_norm_of(sb);
  float s = 0.f;
#pragma unroll
  for (int u = 0; u < U; ++u)
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float ya = a[u][e] * fa, yb = b[u][e] * fb;
      a[u][e] = ya + l[u][e] * (yb - ya);
      s += a[u][e] * a[u][e];
    }
  finish_row<U>(a, s, w, vec, xr, xop, xinv, ostride, red);
}

template <int U>
__global__ void __launch_bounds__(kNormThreads) slerp_norm_kernel(float* __restrict__ x, const float* __restrict__ o,
                                                                   size_t part, const float* __restrict__ lr, int w,
                                                                   int vec, f16x8* __restrict__ xop,
                                                                   float* __restrict__ xinv, size_t ostride) {
  slerp_norm_row<U, false>(x, o, part, lr, w, vec, xop, xinv, ostride);
}

template <int U>
__global__ void __launch_bounds__(kNormThreads) slerp_norm_part_kernel(float* __restrict__ x,
                                                                        const float* __restrict__ o, size_t part,
                                                                        const float* __restrict__ lr, int w, int vec,
                                                                        f16x8* __restrict__ xop,
                                                                        float* __restrict__ xinv, size_t ostride) {
  slerp_norm_row<U, true>(x, o, part, lr, w, vec, xop, xinv, ostride);
}

// PART: g and u hold two parts of rows split along K (the second at + part), added as they load, with the other loads.
template <int U, bool PART>
__device__ inline void swiglu_norm_row(const float* g, const float* __restrict__ u_, size_t part,
                                       const float* __restrict__ sg, const float* __restrict__ su, int w, int vec,
                                       float* out, f16x8* __restrict__ xop, float* __restrict__ xinv, size_t ostride) {
  __shared__ float red[kNormRed];
  float a[U][8], b[U][8], s1[U][8], s2[U][8];
  load_row<kNormThreads, U>(g + size_t(blockIdx.x) * w, w, vec, a);
  load_row<kNormThreads, U>(u_ + size_t(blockIdx.x) * w, w, vec, b);
  load_row<kNormThreads, U>(sg, w, vec, s1);
  load_row<kNormThreads, U>(su, w, vec, s2);
  if constexpr (PART) {
    add_part<U>(g + part + size_t(blockIdx.x) * w, w, vec, a);
    add_part<U>(u_ + part + size_t(blockIdx.x) * w, w, vec, b);
  }
  float s = 0.f;
#pragma unroll
  for (int u = 0; u < U; ++u)
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float z = a[u][e] * s1[u][e];
      a[u][e] = z / (1.f + expf(-z)) * (b[u][e] * s2[u][e]);
      s += a[u][e] * a[u][e];
    }
  finish_row<U>(a, s, w, vec, out ? out + size_t(blockIdx.x) * w : nullptr, xop, xinv, ostride, red);
}

template <int U>
__global__ void __launch_bounds__(kNormThreads) swiglu_norm_kernel(const float* g, const float* __restrict__ u_,
                                                                    size_t part, const float* __restrict__ sg,
                                                                    const float* __restrict__ su, int w, int vec,
                                                                    float* out, f16x8* __restrict__ xop,
                                                                    float* __restrict__ xinv, size_t ostride) {
  swiglu_norm_row<U, false>(g, u_, part, sg, su, w, vec, out, xop, xinv, ostride);
}

template <int U>
__global__ void __launch_bounds__(kNormThreads) swiglu_norm_part_kernel(const float* g, const float* __restrict__ u_,
                                                                         size_t part, const float* __restrict__ sg,
                                                                         const float* __restrict__ su, int w, int vec,
                                                                         float* out, f16x8* __restrict__ xop,
                                                                         float* __restrict__ xinv, size_t ostride) {
  swiglu_norm_row<U, true>(g, u_, part, sg, su, w, vec, out, xop, xinv, ostride);
}

template <int U>
__global__ void __launch_bounds__(kNormThreads) gate_norm_kernel(const float* a_,
                                                                  const float* __restrict__ gate,
                                                                  const float* __restrict__ gs, int w, int vec,
                                                                  float* out, f16x8* __restrict__ xop,
                                                                  float* __restrict__ xinv, size_t ostride) {
  __shared__ float red[kNormRed];
  float a[U][8], g[U][8], sc[U][8];
  load_row<kNormThreads, U>(a_ + size_t(blockIdx.x) * w, w, vec, a);
  load_row<kNormThreads, U>(gate + size_t(blockIdx.x) * w, w, vec, g);
  load_row<kNormThreads, U>(gs, w, vec, sc);
  float s = 0.f;
#pragma unroll
  for (int u = 0; u < U; ++u)
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      a[u][e] = a[u][e] * (1.f / (1.f + expf(-g[u][e] * sc[u][e])));
      s += a[u][e] * a[u][e];
    }
  finish_row<U>(a, s, w, vec, out ? out + size_t(blockIdx.x) * w : nullptr, xop, xinv, ostride, red);
}

template <int U>
__global__ void __launch_bounds__(kNormThreads) add_norm_kernel(const float* a_, const float* b_, float* out,
                                                                 int w, int vec, f16x8* __restrict__ xop,
                                                                 float* __restrict__ xinv, size_t ostride) {
  __shared__ float red[kNormRed];
  float a[U][8], b[U][8];
  load_row<kNormThreads, U>(a_ + size_t(blockIdx.x) * w, w, vec, a);
  if (b_) {
    load_row<kNormThreads, U>(b_ + size_t(blockIdx.x) * w, w, vec, b);
#pragma unroll
    for (int u = 0; u < U; ++u)
#pragma unroll
      for (int e = 0; e < 8; ++e) a[u][e] += b[u][e];
  }
  float s = 0.f;
#pragma unroll
  for (int u = 0; u < U; ++u)
#pragma unroll
    for (int e = 0; e < 8; ++e) s += a[u][e] * a[u][e];
  finish_row<U>(a, s, w, vec, out + size_t(blockIdx.x) * w, xop, xinv, ostride, red);
}

// xtg::argmax (engine/src/sampler.cpp:8-13) of each row of n logits: the first index of the largest value. A NaN
// never compares greater, so NaNs are passed over, except that a NaN in element 0 is never displaced (answer 0).
// One work-group of 1024 threads per row; (value, index) pairs reduce with "greater, or equal at a smaller index".
constexpr int kArgmaxThreads = 1024;

__device__ inline void argmax_take(float& bv, int& bi, float v, int i) {
  if (v > bv || (v == bv && i < bi)) {
    bv = v;
    bi = i;
  }
}

__global__ void __launch_bounds__(kArgmaxThreads) argmax_kernel(const float* __restrict__ x, int n, int vec,
                                                                 int* __restrict__ out) {
  __shared__ float sv[kArgmaxThreads / 64];
  __shared__ int si[kArgmaxThreads / 64];
  const float* r = x + size_t(blockIdx.x) * size_t(n);
  float bv = -INFINITY;
  int bi = INT_MAX;   // no element yet (an element equal to -inf still takes the place)
  int i0 = 0;
  if (vec) {
    const int n4 = n / 4;
    for (int c = threadIdx.x; c < n4; c += kArgmaxThreads) {
      const float4 t = reinterpret_cast<const float4*>(r)[c];
      argmax_take(bv, bi, t.x, 4 * c);
      argmax_take(bv, bi, t.y, 4 * c + 1);
      argmax_take(bv, bi, t.z, 4 * c + 2);
      argmax_take(bv, bi, t.w, 4 * c + 3);
    }
    i0 = 4 * n4;
  }
  for (int i = i0 + int(threadIdx.x); i < n; i += kArgmaxThreads) argmax_take(bv, bi, r[i], i);
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) {
    const float v = __shfl_xor(bv, off);
    const int i = __shfl_xor(bi, off);
    argmax_take(bv, bi, v, i);
  }
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (lane == 0) {
    sv[wave] = bv;
    si[wave] = bi;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int w = 1; w < kArgmaxThreads / 64; ++w) argmax_take(bv, bi, sv[w], si[w]);
    out[blockIdx.x] = (r[0] != r[0] || bi == INT_MAX) ? 0 : bi;
  }
}

// ------------------------------------------------------------------------------------------------ launchers

namespace {

// Chunks of 8 per thread for a row of w floats: 1, 2, 4 or 8 (rows up to 32768 wide).
int norm_chunks(int w) {
  const int chunks = (w + 7) / 8;
  for (int u : {1, 2, 4, 8})
    if (chunks <= u * kNormThreads) return u;
  fail("row kernels: width %d above %d", w, 8 * 8 * kNormThreads);
}

bool aligned16(const void* p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; }

// vec: whole chunks of every row may be read as float4s
bool rows_vec(int w, std::initializer_list<const void*> ptrs) {
  if (w % 4 != 0) return false;
  for (const void* p : ptrs)
    if (p && !aligned16(p)) return false;
  return true;
}

struct Operand {
  f16x8* xop = nullptr;
  float* xinv = nullptr;
  size_t stride = 0;   // bytes from one 8-row group to the next
};

Operand operand_of(void* op, int rows, int w) {
  if (!op) return {};
  XTG_CHECK(rows <= kMaxOperandRows, "row kernels: %d rows for an operand of at most %d", rows, kMaxOperandRows);
  XTG_CHECK(w % 16 == 0, "row kernels: operand width %d (a multiple of 16)", w);
  XTG_CHECK(aligned16(op), "row kernels: operand at %p is not 16-byte aligned", op);
  return {static_cast<f16x8*>(op), reinterpret_cast<float*>(static_cast<char*>(op) + xop_bytes(w)), op_group_bytes(w)};
}

#define XTG_NORM_DISPATCH(KERNEL, ...)                                                                   \
  do {                                                                                                   \
    const int u_ = norm_chunks(w);                                                                       \
    const dim3 g_{unsigned(rows)}, b_{unsigned(kNormThreads)};                                                     \
    if (u_ == 1) hipLaunchKernelGGL(KERNEL<1>, g_, b_, 0, stream, __VA_ARGS__);                          \
    else if (u_ == 2) hipLaunchKernelGGL(KERNEL<2>, g_, b_, 0, stream, __VA_ARGS__);                     \
    else if (u_ == 4) hipLaunchKernelGGL(KERNEL<4>, g_, b_, 0, stream, __VA_ARGS__);                     \
    else hipLaunchKernelGGL(KERNEL<8>, g_, b_, 0, stream, __VA_ARGS__);                                  \
    HIP_CHECK(hipGetLastError());                                                                        \
    return strf("%s<%d>", #KERNEL, u_);                                                                  \
  } while (0)

}  // namespace

std::string launch_qk_rope_norm(float* q, float* k, int m, int heads, int kv_heads, int d, long long pos0,
                                const float* inv_freq, const float* qscale, hipStream_t stream) {
  XTG_CHECK(d % 2 == 0 && d <= 256, "rope: head_dim %d (even, at most 256)", d);
  hipLaunchKernelGGL(qk_rope_norm_kernel, dim3(unsigned(m * (heads + kv_heads))), dim3(64), 0, stream, q, k, m, heads,
                     kv_heads, d, pos0, inv_freq, qscale);
  HIP_CHECK(hipGetLastError());
  return "qk_rope_norm_kernel";
}

std::string launch_slerp_norm(float* x, const float* o, const float* lr, int rows, int w, void* op,
                              hipStream_t stream, size_t part) {
  const Operand p = operand_of(op, rows, w);
  const int vec = rows_vec(w, {x, o, lr, o + part});
  if (part) XTG_NORM_DISPATCH(slerp_norm_part_kernel, x, o, part, lr, w, vec, p.xop, p.xinv, p.stride);
  XTG_NORM_DISPATCH(slerp_norm_kernel, x, o, part, lr, w, vec, p.xop, p.xinv, p.stride);
}

std::string launch_swiglu_norm(const float* g, const float* u, const float* sg, const float* su, int rows, int w,
                               float* out, void* op, hipStream_t stream, size_t part) {
  XTG_CHECK(!part || (out != g && out != u), "swiglu_norm: a split input is not written in place");
  const Operand p = operand_of(op, rows, w);
  const int vec = rows_vec(w, {g, u, sg, su, out, g + part, u + part});
  if (part) XTG_NORM_DISPATCH(swiglu_norm_part_kernel, g, u, part, sg, su, w, vec, out, p.xop, p.xinv, p.stride);
  XTG_NORM_DISPATCH(swiglu_norm_kernel, g, u, part, sg, su, w, vec, out, p.xop, p.xinv, p.stride);
}

std::string launch_gate_norm(const float* a, const float* gate, const float* gs, int rows, int w, float* out, void* op,
                             hipStream_t stream) {
  const Operand p = operand_of(op, rows, w);
  const int vec = rows_vec(w, {a, gate, gs, out});
  XTG_NORM_DISPATCH(gate_norm_kernel, a, gate, gs, w, vec, out, p.xop, p.xinv, p.stride);
}

std::string launch_add_norm(const float* a, const float* b, float* out, int rows, int w, void* op,
                            hipStream_t stream) {
  const Operand p = operand_of(op, rows, w);
  const int vec = rows_vec(w, {a, b, out});
  XTG_NORM_DISPATCH(add_norm_kernel, a, b, out, w, vec, p.xop, p.xinv, p.stride);
}

std::string launch_argmax(const float* x, int rows, int n, int* out, hipStream_t stream) {
  const int vec = rows_vec(n, {x});
  hipLaunchKernelGGL(argmax_kernel, dim3(unsigned(rows)), dim3(kArgmaxThreads), 0, stream, x, n, vec, out);
  HIP_CHECK(hipGetLastError());
  return "argmax_kernel";
}

}  // namespace xtg::hip
