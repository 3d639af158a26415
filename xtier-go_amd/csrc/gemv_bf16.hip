// BF16 GEMV / skinny GEMM for 1..8 activation rows on gfx950 matrix cores (a BF16 checkpoint's LM head).
//
// Semantics: y[i][n] = sum_j bf16(w[n][j]) * x[i][j], FP32 products and sums (engine/src/kernels.cpp:140-155).
//
// Design (MI355X, bandwidth-bound: 2 bytes of weight per multiply-add per row):
//  - Weights are repacked once, at prepare, into tiles of 16 rows x 128 inputs. Each of a tile's four 32-input
//    steps is one wave's 1 KiB MFMA A operand (lane l: row l % 16, inputs 8 (l / 16) .. +8), so BF16 weights go
//    from HBM straight into v_mfma_f32_16x16x32_bf16 with no conversion, one contiguous 16-byte load per lane.
//  - The FP32 activations become three BF16 terms (t0 + t1 + t2 = x to about 24 significant bits, so the
//    products keep FP32-level accuracy). A 16-column B operand holds the terms of 5 rows (column 3 r + t: term t
//    of row 5 cb + r in column block cb); 6..8 rows take a second block, a second MFMA per weight operand.
//  - The launch skeleton is the NVFP4 GEMV's: R row-blocks and T k-tiles per wave, S waves per work-group along
//    k, partials added in LDS in a fixed order; nontemporal weight loads (read once per call).
//  - Output: the three term columns of a row (neighbour lanes) are added, times an optional per-column factor.
#include <algorithm>
#include <cstdlib>
#include <cstring>

#include "common.hpp"
#include "kernels.hpp"

namespace xtg::hip {

namespace {
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
constexpr int kRowsPerBlock = 5;   // activation rows per 16-column block (3 terms each)
}  // namespace

void pack_bf16_tiles(const uint16_t* w, int n, int k, std::vector<uint16_t>& out) {
  const int nb = (n + kTileRows - 1) / kTileRows, kt = (k + kTileK - 1) / kTileK;
  out.assign(size_t(nb) * size_t(kt) * (kBf16TileBytes / 2), 0);
  for (int rb = 0; rb < nb; ++rb)
    for (int t = 0; t < kt; ++t) {
      uint16_t* tile = out.data() + (size_t(rb) * size_t(kt) + size_t(t)) * (kBf16TileBytes / 2);
      for (int s = 0; s < 4; ++s)
        for (int l = 0; l < 64; ++l) {
          const int row = rb * kTileRows + (l & 15);
          const int k0 = t * kTileK + 32 * s + 8 * (l >> 4);
          if (row >= n || k0 >= k) continue;
          std::memcpy(tile + (s * 64 + l) * 8, w + size_t(row) * size_t(k) + size_t(k0),
                      size_t(std::min(8, k - k0)) * 2);
        }
    }
}

// ---------------------------------------------------------------------------------------- activation operand

// One work-group per activation row j: every 8-input chunk of the row (zeros past k) as three BF16 terms into
// column 3 (j % 5) + t of block j / 5, entry 4 column + g of the chunk's step (k-tile c / 16, step (c % 16) / 4,
// g = c % 4), so that lane (g, column) of the GEMV loads it.
constexpr int kPrepThreads = 256;
__global__ void __launch_bounds__(kPrepThreads) prep_x_bf16_kernel(const void* __restrict__ x, int x_dtype, int k,
                                                                   int kt, uint4* __restrict__ xop) {
  const int j = blockIdx.x;
  const int cb = j / kRowsPerBlock, col0 = 3 * (j % kRowsPerBlock);
  for (int c = threadIdx.x; c < kt * 16; c += kPrepThreads) {
    float v[8];
    const int k0 = 8 * c;
    const size_t base = size_t(j) * size_t(k) + size_t(k0);
    if (x_dtype == kXBF16) {
      const uint16_t* xb = static_cast<const uint16_t*>(x);
#pragma unroll
      for (int e = 0; e < 8; ++e) v[e] = k0 + e < k ? __uint_as_float(uint32_t(xb[base + e]) << 16) : 0.f;
    } else {
      const float* xf = static_cast<const float*>(x);
#pragma unroll
      for (int e = 0; e < 8; ++e) v[e] = k0 + e < k ? xf[base + e] : 0.f;
    }
    bf16x8 t0, t1, t2;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const __bf16 a = (__bf16)v[e];   // v_cvt_pk_bf16_f32: round to nearest even
      const float r = v[e] - (float)a;  // exact
      const __bf16 b = (__bf16)r;
      t0[e] = a;
      t1[e] = b;
      t2[e] = (__bf16)(r - (float)b);
    }
    const int tile = c >> 4, step = (c & 15) >> 2, g = c & 3;
    uint4* dst = xop + ((size_t(tile) * 4 + size_t(step)) * 2 + size_t(cb)) * 64;
    dst[4 * (col0 + 0) + g] = __builtin_bit_cast(uint4, t0);
    dst[4 * (col0 + 1) + g] = __builtin_bit_cast(uint4, t1);
    dst[4 * (col0 + 2) + g] = __builtin_bit_cast(uint4, t2);
  }
}

std::string launch_prep_x_bf16(const void* x, int x_dtype, int m, int k, void* xop, hipStream_t stream) {
  XTG_CHECK(m >= 1 && m <= kMaxRows, "prep_x_bf16: %d rows (1..%d)", m, kMaxRows);
  XTG_CHECK(k > 0, "prep_x_bf16: width %d", k);
  const int kt = (k + kTileK - 1) / kTileK;
  hipLaunchKernelGGL(prep_x_bf16_kernel, dim3(unsigned(m)), dim3(kPrepThreads), 0, stream, x, x_dtype, k, kt,
                     static_cast<uint4*>(xop));
  HIP_CHECK(hipGetLastError());
  return "prep_x_bf16_kernel";
}

// ------------------------------------------------------------------------------------------------------ GEMV

namespace {

struct Bf16Args {
  const uint4* tiles;
  const uint4* xop;
  const float* col_scale;
  float* y;
  int n, nb, kt, m;
  int live[2];   // live columns of each block: 3 x its rows
};

// Rows 4 g .. 4 g + 3 of row-block rb for activation row j (terms already added).
__device__ inline void store4(const Bf16Args& a, int rb, int g, int j, f32x4 v) {
  if (j >= a.m) return;
  const int n0 = rb * kTileRows + 4 * g;
  float* yp = a.y + size_t(j) * size_t(a.n);
#pragma unroll
  for (int e = 0; e < 4; ++e)
    if (n0 + e < a.n) yp[n0 + e] = a.col_scale ? v[e] * a.col_scale[n0 + e] : v[e];
}

template <int R, int T, int CB>
__global__ void __launch_bounds__(512) gemv_bf16_kernel(const Bf16Args a) {
  extern __shared__ f32x4 red[];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, S = blockDim.x >> 6;
  const int rb0 = int(blockIdx.x) * R;
  const int col = lane & 15, grp = lane >> 4, entry = 4 * col + grp;
  f32x4 acc[R][CB];
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int cb = 0; cb < CB; ++cb) acc[r][cb] = f32x4{0.f, 0.f, 0.f, 0.f};

  // rounds of T k-tiles per wave (one round when S T covers k); in each, every load first: T k-tiles x 4 steps
  // of activation terms (live columns only) and R x T x 4 weight operands, then the matrix ops
  for (int kt0 = wave * T; kt0 < a.kt; kt0 += S * T) {
    uint4 xb[T][4][CB];
    uint4 wb[T][R][4];
#pragma unroll
    for (int u = 0; u < T; ++u) {
      const int kt = kt0 + u;
      const bool ok = kt < a.kt;
#pragma unroll
      for (int s = 0; s < 4; ++s)
#pragma unroll
        for (int cb = 0; cb < CB; ++cb)
          xb[u][s][cb] = ok && col < a.live[cb]
                             ? a.xop[((size_t(kt) * 4 + size_t(s)) * 2 + size_t(cb)) * 64 + size_t(entry)]
                             : make_uint4(0, 0, 0, 0);
#pragma unroll
      for (int r = 0; r < R; ++r) {
        const bool ok2 = ok && rb0 + r < a.nb;
        const uint4* tile = a.tiles + (size_t(rb0 + r) * size_t(a.kt) + size_t(kt)) * 256;
#pragma unroll
        for (int s = 0; s < 4; ++s) {
          if (ok2) {
            const u32x4 w4 = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(tile + s * 64 + lane));
            wb[u][r][s] = make_uint4(w4[0], w4[1], w4[2], w4[3]);
          } else {
            wb[u][r][s] = make_uint4(0, 0, 0, 0);
          }
        }
      }
    }
#pragma unroll
    for (int u = 0; u < T; ++u)
#pragma unroll
      for (int r = 0; r < R; ++r)
#pragma unroll
        for (int s = 0; s < 4; ++s) {
          const bf16x8 A = __builtin_bit_cast(bf16x8, wb[u][r][s]);
#pragma unroll
          for (int cb = 0; cb < CB; ++cb)
            acc[r][cb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A, __builtin_bit_cast(bf16x8, xb[u][s][cb]),
                                                                 acc[r][cb], 0, 0, 0);
        }
  }

  if (S == 1) {
    // lane (g, 3 q) adds the terms held by lanes (g, 3 q + 1) and (g, 3 q + 2)
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
      for (int cb = 0; cb < CB; ++cb) {
        f32x4 v = acc[r][cb];
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] += __shfl(v[e], lane + 1) + __shfl(v[e], lane + 2);
        if (col % 3 == 0 && col < 15 && rb0 + r < a.nb) store4(a, rb0 + r, grp, cb * kRowsPerBlock + col / 3, v);
      }
    return;
  }
#pragma unroll
  for (int r = 0; r < R; ++r)
#pragma unroll
    for (int cb = 0; cb < CB; ++cb) red[((wave * R + r) * CB + cb) * 64 + lane] = acc[r][cb];
  __syncthreads();
  // one item per (row-block, column block, activation row of the block, lane group)
  for (int item = threadIdx.x; item < R * CB * kRowsPerBlock * 4; item += blockDim.x) {
    const int g = item & 3, q = (item >> 2) % kRowsPerBlock, rc = (item >> 2) / kRowsPerBlock;
    const int r = rc / CB, cb = rc % CB;
    if (rb0 + r >= a.nb) continue;
    const int ln = g * 16 + 3 * q;
    f32x4 sum = f32x4{0.f, 0.f, 0.f, 0.f};
    for (int w = 0; w < S; ++w) {
      const f32x4* p = red + ((w * R + r) * CB + cb) * 64 + ln;
      sum += p[0] + p[1] + p[2];
    }
    store4(a, rb0 + r, g, cb * kRowsPerBlock + q, sum);
  }
}

using Bf16Fn = void (*)(const Bf16Args);

Bf16Fn bf16_fn(int r, int t, int cb) {
#define XTG_CASE(R, T) \
  if (r == R && t == T) return cb == 1 ? gemv_bf16_kernel<R, T, 1> : gemv_bf16_kernel<R, T, 2>;
  XTG_CASE(1, 1) XTG_CASE(1, 2) XTG_CASE(1, 4) XTG_CASE(2, 1) XTG_CASE(2, 2) XTG_CASE(4, 1) XTG_CASE(4, 2)
#undef XTG_CASE
  if (r == 2 && t == 4 && cb == 1) return gemv_bf16_kernel<2, 4, 1>;   // with two column blocks it spills
  return nullptr;
}

}  // namespace

// Work-groups of S <= 8 waves (512 threads: up to 256 VGPRs per lane); a wave takes rounds of T k-tiles until k is
// covered. Measured on MI355X (131072 x 2560 and 32768 x 3072, rotated cold weights): one or two rows want one
// row-block and two k-tiles per wave (88% of HBM peak on the 671 MB head); from three rows on, two row-blocks
// and one k-tile per wave (86% at 5 rows, 83% at 6, 78% at 8), which halves the activation terms each weight
// byte brings in from L2. Few row-blocks keep one row-block per wave, for more work-groups.
GemvShape gemv_bf16_shape(int kt, int nb, int m) {
  const int cb = m > kRowsPerBlock ? 2 : 1;
  if (const char* env = std::getenv("XTG_GEMV_BF16_SHAPE")) {   // "R,T": a fixed shape for experiments
    int r = 0, t = 0;
    if (std::sscanf(env, "%d,%d", &r, &t) == 2 && bf16_fn(r, t, cb))
      return {r, t, std::max(1, std::min(8, (kt + t - 1) / t))};
  }
  const bool wide = nb >= 512 && m >= 3;
  const int r = wide ? 2 : 1, t = wide || kt < 2 ? 1 : 2;
  return {r, t, std::max(1, std::min(8, (kt + t - 1) / t))};
}

std::string launch_gemv_bf16(const PackedBf16& w, const void* xop, int m, float* y, const float* col_scale,
                             hipStream_t stream) {
  XTG_CHECK(m >= 1 && m <= kMaxRows, "gemv_bf16: %d rows (1..%d)", m, kMaxRows);
  const GemvShape sh = gemv_bf16_shape(w.kt, w.nb, m);
  Bf16Args a{};
  a.tiles = reinterpret_cast<const uint4*>(w.tiles);
  a.xop = static_cast<const uint4*>(xop);
  a.col_scale = col_scale;
  a.y = y;
  a.n = w.n;
  a.nb = w.nb;
  a.kt = w.kt;
  a.m = m;
  const int cb = m > kRowsPerBlock ? 2 : 1;
  a.live[0] = 3 * std::min(m, kRowsPerBlock);
  a.live[1] = 3 * std::max(0, m - kRowsPerBlock);
  const int threads = sh.s * 64;
  Bf16Fn fn = bf16_fn(sh.r, sh.t, cb);
  XTG_CHECK(fn != nullptr && threads <= 512, "gemv_bf16: no kernel for R=%d T=%d S=%d", sh.r, sh.t, sh.s);
  const unsigned wgs = unsigned((w.nb + sh.r - 1) / sh.r);
  const size_t lds = sh.s > 1 ? size_t(sh.s) * size_t(sh.r) * size_t(cb) * 64 * sizeof(f32x4) : 0;
  hipLaunchKernelGGL(fn, dim3(wgs), dim3(unsigned(threads)), lds, stream, a);
  HIP_CHECK(hipGetLastError());
  return strf("gemv_bf16_kernel<%d, %d, %d>", sh.r, sh.t, cb);
}

}  // namespace xtg::hip
