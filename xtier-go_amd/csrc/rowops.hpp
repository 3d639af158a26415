// Device helpers shared by the row kernels, the attention finish and the GEMV's activation operand:
// block-wide reductions, whole-row register tiles, and the writer of the GEMV's MFMA activation operand.
#pragma once

#include <hip/hip_runtime.h>

#include <cfloat>
#include <cmath>
#include <cstdint>

#include "kernels.hpp"

namespace xtg::hip {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));

// Cross-lane steps of a wave reduction, all on the vector ALUs: DPP within rows of 16 lanes, then the gfx950
// permlane swaps across rows. Each step pairs every lane with a partner and both compute op(a, b) of the same
// two values, so every lane of a reduced group ends with bit-identical results.
template <int CTRL>
__device__ inline float dpp(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}
constexpr int kDppXor1 = 0xB1, kDppXor2 = 0x4E, kDppHalfMirror = 0x141, kDppMirror = 0x140;

// {r[0], r[1]} = {v[l], v[l ^ 16]} (permlane16) or {v[l], v[l ^ 32]} (permlane32) in every lane l
__device__ inline float xor16_sum(float v) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ inline float xor32_sum(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ inline float xor16_max(float v) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ inline float xor32_max(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

__device__ inline float wave_sum(float v) {
  v += dpp<kDppXor1>(v);
  v += dpp<kDppXor2>(v);
  v += dpp<kDppHalfMirror>(v);
  v += dpp<kDppMirror>(v);
  return xor32_sum(xor16_sum(v));
}

__device__ inline float wave_max(float v) {
  v = fmaxf(v, dpp<kDppXor1>(v));
  v = fmaxf(v, dpp<kDppXor2>(v));
  v = fmaxf(v, dpp<kDppHalfMirror>(v));
  v = fmaxf(v, dpp<kDppMirror>(v));
  return xor32_max(xor16_max(v));
}

// Sum (or max) over a work-group of NT threads; every thread gets the result. red holds 2 * NT / 64 floats; a
// call waits until every thread has read the previous call's values before it writes.
template <int NT>
__device__ inline float block_sum(float v, float* red) {
  v = wave_sum(v);
  __syncthreads();   // red may still be read by a previous call
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < NT / 64; ++i) s += red[i];
  return s;
}

template <int NT>
__device__ inline void block_sum2(float& a, float& b, float* red) {
  a = wave_sum(a);
  b = wave_sum(b);
  __syncthreads();
  if ((threadIdx.x & 63) == 0) {
    red[threadIdx.x >> 6] = a;
    red[NT / 64 + (threadIdx.x >> 6)] = b;
  }
  __syncthreads();
  a = 0.f;
  b = 0.f;
#pragma unroll
  for (int i = 0; i < NT / 64; ++i) {
    a += red[i];
    b += red[NT / 64 + i];
  }
}

template <int NT>
__device__ inline float block_max(float v, float* red) {
  v = wave_max(v);
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  float s = red[0];
#pragma unroll
  for (int i = 1; i < NT / 64; ++i) s = fmaxf(s, red[i]);
  return s;
}

// A sum and a max over the work-group in one exchange; every thread gets both.
template <int NT>
__device__ inline void block_sum_max(float& s, float& m, float* red) {
  s = wave_sum(s);
  m = wave_max(m);
  __syncthreads();
  if ((threadIdx.x & 63) == 0) {
    red[threadIdx.x >> 6] = s;
    red[NT / 64 + (threadIdx.x >> 6)] = m;
  }
  __syncthreads();
  s = 0.f;
  m = red[NT / 64];
#pragma unroll
  for (int i = 0; i < NT / 64; ++i) {
    s += red[i];
    m = fmaxf(m, red[NT / 64 + i]);
  }
}

// justnorm's factor: x / sqrt(sum x^2 + 1e-6) as x * (1 / sqrt(...)) (engine/src/kernels.cpp:162-175)
__device__ inline float inv_norm_of(float sumsq) { return 1.f / sqrtf(sumsq + 1e-6f); }

// ------------------------------------------------------------------------------------------- row tiles
//
// A row of w floats held by NT threads in U chunks of 8: thread t's chunk u is elements 8 (t + u NT) .. +8.
// Elements past w read as zero. vec: the row is 16-byte aligned and w % 4 == 0 (whole chunks load as float4s).

template <int NT, int U>
__device__ inline void load_row(const float* __restrict__ p, int w, bool vec, float (&v)[U][8]) {
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int e0 = 8 * (int(threadIdx.x) + u * NT);
    if (vec && e0 + 8 <= w) {
      const float4 a = *reinterpret_cast<const float4*>(p + e0);
      const float4 b = *reinterpret_cast<const float4*>(p + e0 + 4);
      v[u][0] = a.x, v[u][1] = a.y, v[u][2] = a.z, v[u][3] = a.w;
      v[u][4] = b.x, v[u][5] = b.y, v[u][6] = b.z, v[u][7] = b.w;
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) v[u][e] = e0 + e < w ? p[e0 + e] : 0.f;
    }
  }
}

template <int NT, int U>
__device__ inline void store_row(float* __restrict__ p, int w, bool vec, const float (&v)[U][8]) {
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int e0 = 8 * (int(threadIdx.x) + u * NT);
    if (vec && e0 + 8 <= w) {
      *reinterpret_cast<float4*>(p + e0) = make_float4(v[u][0], v[u][1], v[u][2], v[u][3]);
      *reinterpret_cast<float4*>(p + e0 + 4) = make_float4(v[u][4], v[u][5], v[u][6], v[u][7]);
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e)
        if (e0 + e < w) p[e0 + e] = v[u][e];
    }
  }
}

// ---------------------------------------------------------------------------------- activation operand
//
// The GEMV's activation operand (kernels.hpp): [kt][4 steps][64 entries][8 f16]; chunk c (inputs 8c .. 8c + 7)
// of row j goes, as the f16 high and low parts of x * 2^e, to columns 2 j and 2 j + 1 of k-tile c / 16: chunk
// w = 4 g + t of a tile is lane group g's part of MFMA step t, entry 4 * column + g. xinv[j] = 2^-e.

__device__ inline void store_chunk(f16x8* xop, int j, int c, const float v[8], float up) {
  f16x8 hi, lo;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const float s = v[i] * up;
    const _Float16 h = (_Float16)s;
    hi[i] = h;
    lo[i] = (_Float16)(s - (float)h);
  }
  const int w = c & 15, g = w >> 2, t = w & 3;
  const size_t base = (size_t(c >> 4) * 4 + size_t(t)) * 64;
  xop[base + size_t(8 * j + g)] = hi;
  xop[base + size_t(8 * j + 4 + g)] = lo;
}

// The power of two that brings a row's largest magnitude mx to [2^14, 2^15) (1 for a zero or non-finite max),
// clamped to 2^+-120.
__device__ inline int operand_exponent(float mx) {
  int e = 0;
  if (mx > 0.f && mx <= FLT_MAX) e = 14 - ilogbf(mx);
  return e < -120 ? -120 : (e > 120 ? 120 : e);
}

// Row `row` of an operand of consecutive 8-row groups `stride` bytes apart (xop / xinv: group 0's operand and row
// factors), from a row tile (values past w are zero): the work-group's max, then every chunk of the row's
// kt = ceil(w / 128) k-tiles (zero chunks past w included). red: 2 * NT / 64 floats.
// emit_operand with the row's largest magnitude mx already known (no reduction).
template <int NT, int U>
__device__ inline void emit_operand_mx(const float (&v)[U][8], int w, int row, f16x8* xop, float* xinv, size_t stride,
                                       float mx) {
  const size_t off = size_t(row / kMaxRows) * stride;
  xop = reinterpret_cast<f16x8*>(reinterpret_cast<char*>(xop) + off);
  xinv = reinterpret_cast<float*>(reinterpret_cast<char*>(xinv) + off);
  const int j = row % kMaxRows;
  const int ex = operand_exponent(mx);
  const float up = ldexpf(1.f, ex);
  if (threadIdx.x == 0) xinv[j] = ldexpf(1.f, -ex);
  const int chunks = ((w + kTileK - 1) / kTileK) * (kTileK / 8);
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int c = int(threadIdx.x) + u * NT;
    if (c < chunks) store_chunk(xop, j, c, v[u], up);
  }
  const float zero[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  for (int c = int(threadIdx.x) + U * NT; c < chunks; c += NT) store_chunk(xop, j, c, zero, up);
}

template <int NT, int U>
__device__ inline void emit_operand(const float (&v)[U][8], int w, int row, f16x8* xop, float* xinv, size_t stride,
                                    float* red) {
  float mx = 0.f;
#pragma unroll
  for (int u = 0; u < U; ++u)
#pragma unroll
    for (int e = 0; e < 8; ++e) mx = fmaxf(mx, fabsf(v[u][e]));
  emit_operand_mx<NT, U>(v, w, row, xop, xinv, stride, block_max<NT>(mx, red));
}

}  // namespace xtg::hip
