// NVFP4 GEMM for prefill chunks (more than 8 activation rows) on gfx950 matrix cores.
//
// Semantics: y[m][n] = global * sum_g e4m3(scale[n][g]) * sum_{j in g} e2m1(code[n][j]) * x[m][j], the prefill
// branch of matmul_nvfp4 (engine/src/kernels.cpp:116-137; the CPU decodes each weight row to FP32 and dots it
// with every input row, so the two differ only in FP32 rounding order).
//
// Design (MI355X; compute-bound once a chunk has tens of rows):
//  - Operands as in the GEMV: weights in the prepared 16 x 128 tiles, dequantised exactly to f16 in registers;
//    activations in 8-row groups of the GEMV's operand (each row as f16 high and low parts, columns 2 r and
//    2 r + 1), so v_mfma_f32_16x16x32_f16 keeps ~22 bits of every activation and accumulates in FP32. With
//    XTG_GEMM_PARTS=1 (or GemvCall::parts = 1) a pair of groups feeds one matrix op with the 16 rows' high parts
//    only: half the matrix ops and operand bytes per output, f16 activations (rel-L2 ~2e-4 against FP32, the
//    precision class of the reference's FP16 GPU prefill GEMM); the default keeps both parts.
//  - A work-group of 4 waves owns 4 RB row-blocks (64 RB output rows) and GB activation groups (8 GB rows).
//    Each k-tile (128 inputs) the work-group stages the groups' operand tile (4 KiB each) in LDS, double-buffered,
//    in lane order (contiguous 16-byte writes and reads); each wave dequantises its RB weight tiles once and runs
//    them against all GB groups: 4 RB GB matrix ops per k-tile per wave. The next k-tile's loads go out into
//    registers before the current one's math and are written to LDS after it, one barrier per k-tile; within a
//    k-tile, each 32-input step's operand fragments are read from LDS during the previous step's matrix ops. (Direct
//    global-to-LDS loads would save those registers, but the compiler then waits for them before every LDS read
//    of the current buffer, serialising the pipeline.)
//  - Tiles are dealt so that work-group i, which runs on XCD i mod 8, gets a contiguous run of tiles: the
//    work-groups of one XCD share weight tiles (consecutive m-tiles of one n-tile) in that XCD's L2.
#include <algorithm>
#include <cstdio>
#include <cstdlib>

#include "common.hpp"
#include "kernels.hpp"
#include "nvfp4.hpp"

namespace xtg::hip {

namespace {
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));
constexpr int kGemmWaves = 4;
}  // namespace

struct GemmArgs {
  const uint8_t* tiles[4];
  int nb[4];
  int n[4];
  float global[4];
  long long y_off[4];
  const float* col_scale[4];
  int tile_end[4];   // cumulative (n-tile x m-tile) counts per weight
  int nw, kt, m, groups, mtiles;
  const char* op;    // group g's operand at op + g * op_stride; its row factors xop_bytes later
  size_t op_stride, xop_bytes;
  float* y;
};

template <int GB>
struct XTile {
  uint4 v[GB];
};
template <int RB>
struct WTile {
  u32x4 c[RB];
  uint32_t s[RB];
};

// A k-tile's activation operand for groups g0 .. g0 + GB - 1: lane L of wave w fetches, for every group, entry
// 4 (L & 15) + (L >> 4) of step w (a permutation within one run of 1 KiB), which it later stores at lane slot L:
// the lane that reads it back as its B operand. Every load is unconditional (a branch around a load makes its
// other path wait for it): a group past the last one reloads the last group, whose results for it are never stored.
template <int GB>
__device__ inline XTile<GB> load_x(const char* op, size_t stride, int groups, int g0, int kt, int wave, int lane) {
  XTile<GB> r;
  const size_t at = (size_t(kt) * 4 + size_t(wave)) * 64 + size_t(4 * (lane & 15) + (lane >> 4));
#pragma unroll
  for (int i = 0; i < GB; ++i) r.v[i] = reinterpret_cast<const uint4*>(op + size_t(min(g0 + i, groups - 1)) * stride)[at];
  return r;
}

// The same for the single-part operand of group pairs p0 .. p0 + GP - 1 (16 rows each): lane L = (kgrp, row) of
// wave w fetches the high part of row (L & 15) of the pair, chunk L >> 4 of step w, from its 8-row group, and stores
// it at lane slot L. The low parts are never read.
template <int GP>
__device__ inline XTile<GP> load_x1(const char* op, size_t stride, int groups, int p0, int kt, int wave, int lane) {
  XTile<GP> r;
  const int row = lane & 15;
  const size_t at = (size_t(kt) * 4 + size_t(wave)) * 64 + size_t(8 * (row & 7) + (lane >> 4));
#pragma unroll
  for (int i = 0; i < GP; ++i)
    r.v[i] = reinterpret_cast<const uint4*>(op + size_t(min(2 * (p0 + i) + (row >> 3), groups - 1)) * stride)[at];
  return r;
}

// Row-blocks rb0 .. rb0 + RB - 1 of k-tile kt (a row-block past the last reloads the last one).
template <int RB>
__device__ inline WTile<RB> load_w(const uint8_t* tiles, int nb, int kt_count, int rb0, int kt, int lane) {
  WTile<RB> w;
#pragma unroll
  for (int r = 0; r < RB; ++r) {
    const uint8_t* tile = tiles + (size_t(min(rb0 + r, nb - 1)) * size_t(kt_count) + size_t(kt)) * kTileBytes;
    w.c[r] = *reinterpret_cast<const u32x4*>(tile + 16 * lane);
    w.s[r] = uint32_t(*reinterpret_cast<const uint16_t*>(tile + 1024 + 2 * lane));
  }
  return w;
}

// RB row-blocks per wave, GB operand blocks per work-group tile, OCC work-groups per CU the registers are
// budgeted for (one: up to 512 VGPRs and AGPRs per lane). PARTS = 2: a block is an 8-row group's high and low f16
// parts (~22 bits of each activation); PARTS = 1: a block is a pair of groups, 16 rows of their high parts only
// (11 bits: the f16 precision of the reference's GPU prefill GEMM, engine/src/opencl.cpp:232-269), half the matrix
// ops and operand bytes per row.
template <int RB, int GB, int OCC, int PARTS>
__global__ void __launch_bounds__(kGemmWaves * 64, OCC) gemm_kernel(const GemmArgs a) {
  constexpr int kTileGroups = GB;
  __shared__ uint4 xs[2][kTileGroups][4][64];   // [buffer][group][step][lane], 8 GB KiB
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int col = lane & 15, grp = lane >> 4;

  // which tile: work-group i runs on XCD i % 8; give each XCD a contiguous run of the tile order
  const int total = a.tile_end[a.nw - 1];
  const int per = total / 8;
  const int id = int(blockIdx.x);
  const int t = id < per * 8 ? (id % 8) * per + id / 8 : id;
  int wi = 0;
  while (wi < a.nw - 1 && t >= a.tile_end[wi]) ++wi;
  const int lt = t - (wi ? a.tile_end[wi - 1] : 0);
  const int ntile = lt / a.mtiles, mtile = lt % a.mtiles;
  const int rb0 = ntile * (kGemmWaves * RB) + wave * RB;
  const int g0 = mtile * kTileGroups;   // PARTS = 1: the first pair
  const int nb = a.nb[wi], KT = a.kt;
  const uint8_t* __restrict__ tiles = a.tiles[wi];

  f32x4 acc[RB][kTileGroups];
#pragma unroll
  for (int r = 0; r < RB; ++r)
#pragma unroll
    for (int g = 0; g < kTileGroups; ++g) acc[r][g] = f32x4{0.f, 0.f, 0.f, 0.f};

  auto xload = [&](int kt) {
    if constexpr (PARTS == 1)
      return load_x1<GB>(a.op, a.op_stride, a.groups, g0, kt, wave, lane);
    else
      return load_x<GB>(a.op, a.op_stride, a.groups, g0, kt, wave, lane);
  };
  WTile<RB> w = load_w<RB>(tiles, nb, KT, rb0, 0, lane);
  {
    const XTile<GB> x0 = xload(0);
#pragma unroll
    for (int i = 0; i < GB; ++i) xs[0][i][wave][lane] = x0.v[i];
  }
  for (int kt = 0; kt < KT; ++kt) {
    __syncthreads();   // buffer kt & 1 is complete, and every wave is done reading the other one
    const int cur = kt & 1;
    const int nxt = min(kt + 1, KT - 1);   // the last k-tile reloads itself: no branch around the loads
    // the next k-tile's loads, in flight during this one's math
    const XTile<GB> xn = xload(nxt);
    const WTile<RB> wn = load_w<RB>(tiles, nb, KT, rb0, nxt, lane);
    __builtin_amdgcn_sched_barrier(0);   // keep them ahead of the math (the scheduler would sink them to their use)
    // step s + 1's operand fragments are read from LDS while step s's matrix ops run (read just before their
    // use, each pair of matrix ops would wait out an LDS round trip)
    f16x8 Bn[kTileGroups];
#pragma unroll
    for (int g = 0; g < kTileGroups; ++g) Bn[g] = __builtin_bit_cast(f16x8, xs[cur][g][0][lane]);
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      f16x8 B[kTileGroups];
#pragma unroll
      for (int g = 0; g < kTileGroups; ++g) B[g] = Bn[g];
      if (s < 3) {
#pragma unroll
        for (int g = 0; g < kTileGroups; ++g) Bn[g] = __builtin_bit_cast(f16x8, xs[cur][g][s + 1][lane]);
      }
      __builtin_amdgcn_sched_barrier(0);
      f16x8 A[RB];
#pragma unroll
      for (int r = 0; r < RB; ++r) A[r] = dequant8(w.c[r][s], scale_pair(w.s[r], s >> 1));
#pragma unroll
      for (int g = 0; g < kTileGroups; ++g)
#pragma unroll
        for (int r = 0; r < RB; ++r)
          acc[r][g] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A[r], B[g], acc[r][g], 0, 0, 0);
    }
#pragma unroll
    for (int i = 0; i < GB; ++i) xs[cur ^ 1][i][wave][lane] = xn.v[i];
    w = wn;
  }

  // lane (grp, col) holds rows 4 grp .. 4 grp + 3 of its row-block for operand column col; PARTS = 2: columns 2 j
  // and 2 j + 1 (neighbour lanes) are row j's high and low parts; PARTS = 1: column col is row col of the pair
  const int n = a.n[wi];
  const float glob = a.global[wi];
  const float* cs = a.col_scale[wi];
  if constexpr (PARTS == 1) {
#pragma unroll
    for (int g = 0; g < kTileGroups; ++g) {
      const int gi = 2 * (g0 + g) + (col >> 3);
      const int mrow = gi * kMaxRows + (col & 7);
      const bool row_ok = gi < a.groups && mrow < a.m;
      const float xinv =
          row_ok ? reinterpret_cast<const float*>(a.op + size_t(gi) * a.op_stride + a.xop_bytes)[col & 7] : 0.f;
#pragma unroll
      for (int r = 0; r < RB; ++r) {
        const f32x4 v = acc[r][g];
        if (row_ok && rb0 + r < nb) {
          const int n0 = (rb0 + r) * kTileRows + 4 * grp;
          float* yp = a.y + a.y_off[wi] + (long long)mrow * n;
          const float f = glob * xinv;
#pragma unroll
          for (int e = 0; e < 4; ++e)
            if (n0 + e < n) yp[n0 + e] = cs ? (v[e] * f) * cs[n0 + e] : v[e] * f;
        }
      }
    }
    return;
  }
#pragma unroll
  for (int g = 0; g < kTileGroups; ++g) {
    const int gi = g0 + g;
    const int mrow = gi * kMaxRows + (col >> 1);
    const bool row_ok = gi < a.groups && mrow < a.m;
    const float xinv = row_ok ? reinterpret_cast<const float*>(a.op + size_t(gi) * a.op_stride + a.xop_bytes)[col >> 1]
                              : 0.f;
#pragma unroll
    for (int r = 0; r < RB; ++r) {
      f32x4 v = acc[r][g];
#pragma unroll
      for (int e = 0; e < 4; ++e) v[e] += dpp<kDppXor1>(v[e]);
      if ((col & 1) == 0 && row_ok && rb0 + r < nb) {
        const int n0 = (rb0 + r) * kTileRows + 4 * grp;
        float* yp = a.y + a.y_off[wi] + (long long)mrow * n;
        const float f = glob * xinv;
#pragma unroll
        for (int e = 0; e < 4; ++e)
          if (n0 + e < n) yp[n0 + e] = cs ? (v[e] * f) * cs[n0 + e] : v[e] * f;
      }
    }
  }
}

using GemmFn = void (*)(const GemmArgs);
static GemmFn gemm_fn(int rb, int gb, int parts) {
#define XTG_GEMM(R, G, O, P) \
  if (rb == R && gb == G && parts == P) return gemm_kernel<R, G, O, P>;
  XTG_GEMM(4, 4, 2, 2) XTG_GEMM(2, 4, 2, 2) XTG_GEMM(1, 4, 2, 2)
  XTG_GEMM(4, 4, 2, 1) XTG_GEMM(2, 4, 2, 1) XTG_GEMM(1, 4, 2, 1) XTG_GEMM(4, 2, 2, 1) XTG_GEMM(2, 2, 2, 1)
  XTG_GEMM(1, 2, 2, 1)
#undef XTG_GEMM
  return nullptr;
}

static std::string run_gemm(const GemvCall& c, int rb, int gb, int parts, hipStream_t stream);

std::string launch_gemm(const GemvCall& c, hipStream_t stream) {
  XTG_CHECK(c.nw >= 1 && c.nw <= 4, "gemm: %d weights (1..4)", c.nw);
  XTG_CHECK(c.m >= 1, "gemm: %d rows", c.m);
  int parts = c.parts;
  if (const char* env = std::getenv("XTG_GEMM_PARTS")) parts = std::atoi(env);
  XTG_CHECK(parts == 1 || parts == 2, "gemm: %d operand parts (1 or 2)", parts);
  const int groups = (c.m + kMaxRows - 1) / kMaxRows;
  const int blocks = parts == 1 ? (groups + 1) / 2 : groups;   // operand blocks: groups, or pairs of them
  // launch shape (XTG_GEMM_SHAPE=RB,GB fixes it, for experiments)
  auto tiles_for = [&](int r, int g) {
    const int mt = (blocks + g - 1) / g;
    long t = 0;
    for (int i = 0; i < c.nw; ++i) t += long((c.w[i]->nb + kGemmWaves * r - 1) / (kGemmWaves * r)) * mt;
    return t;
  };
  // measured on MI355X over the 4B-shaped projections at 64 .. 2048 rows: four groups per tile throughout; two
  // row-blocks per wave (34 % of the dense f16 peak on gate/up at 512 rows), four only with thousands of tiles
  // (2048-row chunks of the wide projections), one with fewer than 512 tiles of two (the 3072-wide o and down
  // projections at 512 rows: 45 and 79 us against 46 and 83 us with two)
  int gb = 4;
  int rb = tiles_for(4, 4) >= 2048 ? 4 : tiles_for(2, 4) >= 512 ? 2 : 1;
  // single part (blocks of 16 rows), measured likewise (512 / 2048 rows): four row-blocks and four pairs on the
  // wide projections at 2048 rows and gate/up at 512 (198 / 319 / 76 us), four and two on o and down at 2048
  // (85 / 152 us), two and two below that (q/k/v/g 62 us, o 35 us, down 61 us at 512 rows); eight pairs were 2-4x
  // slower at every size (the compiler keeps an 8-block XTile in scratch memory; eight two-part groups without
  // that, as two 4-group halves, were still 13-40 % slower than the shapes above)
  if (parts == 1) {
    gb = tiles_for(4, 4) >= 512 ? 4 : 2;
    rb = gb == 4 || tiles_for(4, 2) >= 768 ? 4 : 2;
  }
  if (const char* env = std::getenv("XTG_GEMM_SHAPE")) {
    int r = 0, g = 0;
    if (std::sscanf(env, "%d,%d", &r, &g) == 2 && gemm_fn(r, g, parts) != nullptr)
      return run_gemm(c, r, g, parts, stream);
  }
  return run_gemm(c, rb, gb, parts, stream);
}

static std::string run_gemm(const GemvCall& c, int rb, int gb, int parts, hipStream_t stream) {
  const int kt = c.w[0]->kt;
  const int groups = (c.m + kMaxRows - 1) / kMaxRows;
  const int blocks = parts == 1 ? (groups + 1) / 2 : groups;
  const int mtiles = (blocks + gb - 1) / gb;
  GemmArgs a{};
  int end = 0;
  for (int i = 0; i < c.nw; ++i) {
    XTG_CHECK(c.w[i]->kt == kt, "gemm: input widths differ");
    a.tiles[i] = c.w[i]->tiles;
    a.nb[i] = c.w[i]->nb;
    a.n[i] = c.w[i]->n;
    a.global[i] = c.w[i]->global;
    a.y_off[i] = (long long)c.y_off[i];
    a.col_scale[i] = c.col_scale[i];
    end += ((c.w[i]->nb + kGemmWaves * rb - 1) / (kGemmWaves * rb)) * mtiles;
    a.tile_end[i] = end;
  }
  for (int i = c.nw; i < 4; ++i) a.tile_end[i] = end;
  a.nw = c.nw;
  a.kt = kt;
  a.m = c.m;
  a.groups = groups;
  a.mtiles = mtiles;
  a.op = static_cast<const char*>(c.xop);
  a.op_stride = op_group_bytes(c.w[0]->k);
  a.xop_bytes = xop_bytes(c.w[0]->k);
  a.y = c.y;
  const dim3 grid{unsigned(end)}, block{unsigned(kGemmWaves * 64)};
  const GemmFn fn = gemm_fn(rb, gb, parts);
  XTG_CHECK(fn != nullptr, "gemm: no kernel for RB=%d GB=%d, %d parts", rb, gb, parts);
  hipLaunchKernelGGL(fn, grid, block, 0, stream, a);
  HIP_CHECK(hipGetLastError());
  return parts == 1 ? strf("gemm_kernel<%d, %d, f16>", rb, gb) : strf("gemm_kernel<%d, %d>", rb, gb);
}

}  // namespace xtg::hip
