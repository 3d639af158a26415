// NVFP4 GEMM for prefill chunks (more than 8 activation rows) on gfx950 matrix cores.
//
// Semantics: y[m][n] = global * sum_g e4m3(scale[n][g]) * sum_{j in g} e2m1(code[n][j]) * x[m][j], the prefill
// branch of matmul_nvfp4 (engine/src/kernels.cpp:116-137; the CPU decodes each weight row to FP32 and dots it
// with every input row, so the two differ only in FP32 rounding order).
//
// Design (MI355X; compute-bound once a chunk has tens of rows):
//  - Operands as in the GEMV: weights in the prepared 16 x 128 tiles, dequantised exactly to f16 in registers;
//    activations in 8-row groups of the GEMV's operand (each row as f16 high and low parts, columns 2 r and
//    2 r + 1), so v_mfma_f32_16x16x32_f16 keeps ~22 bits of every activation and accumulates in FP32.
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

// RB row-blocks per wave, GB activation groups per work-group tile, OCC work-groups per CU the registers are
// budgeted for (one: up to 512 VGPRs and AGPRs per lane)
template <int RB, int GB, int OCC>
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
  const int g0 = mtile * kTileGroups;
  const int nb = a.nb[wi], KT = a.kt;
  const uint8_t* __restrict__ tiles = a.tiles[wi];

  f32x4 acc[RB][kTileGroups];
#pragma unroll
  for (int r = 0; r < RB; ++r)
#pragma unroll
    for (int g = 0; g < kTileGroups; ++g) acc[r][g] = f32x4{0.f, 0.f, 0.f, 0.f};

  WTile<RB> w = load_w<RB>(tiles, nb, KT, rb0, 0, lane);
  {
    const XTile<GB> x0 = load_x<GB>(a.op, a.op_stride, a.groups, g0, 0, wave, lane);
#pragma unroll
    for (int i = 0; i < GB; ++i) xs[0][i][wave][lane] = x0.v[i];
  }
  for (int kt = 0; kt < KT; ++kt) {
    __syncthreads();   // buffer kt & 1 is complete, and every wave is done reading the other one
    const int cur = kt & 1;
    const int nxt = min(kt + 1, KT - 1);   // the last k-tile reloads itself: no branch around the loads
    // the next k-tile's loads, in flight during this one's math
    const XTile<GB> xn = load_x<GB>(a.op, a.op_stride, a.groups, g0, nxt, wave, lane);
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

  // lane (grp, col) holds rows 4 grp .. 4 grp + 3 of its row-block for operand column col; columns 2 j and
  // 2 j + 1 (neighbour lanes) are row j's high and low parts
  const int n = a.n[wi];
  const float glob = a.global[wi];
  const float* cs = a.col_scale[wi];
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
static GemmFn gemm_fn(int rb, int gb) {
#define XTG_GEMM(R, G, O) \
  if (rb == R && gb == G) return gemm_kernel<R, G, O>;
  XTG_GEMM(4, 4, 2) XTG_GEMM(2, 4, 2) XTG_GEMM(1, 4, 2)
#undef XTG_GEMM
  return nullptr;
}

static std::string run_gemm(const GemvCall& c, int rb, int gb, hipStream_t stream);

std::string launch_gemm(const GemvCall& c, hipStream_t stream) {
  XTG_CHECK(c.nw >= 1 && c.nw <= 4, "gemm: %d weights (1..4)", c.nw);
  XTG_CHECK(c.m >= 1, "gemm: %d rows", c.m);
  const int groups = (c.m + kMaxRows - 1) / kMaxRows;
  // launch shape (XTG_GEMM_SHAPE=RB,GB fixes it, for experiments)
  auto tiles_for = [&](int r, int g) {
    const int mt = (groups + g - 1) / g;
    long t = 0;
    for (int i = 0; i < c.nw; ++i) t += long((c.w[i]->nb + kGemmWaves * r - 1) / (kGemmWaves * r)) * mt;
    return t;
  };
  // measured on MI355X over the 4B-shaped projections at 64 .. 2048 rows: four groups per tile throughout; two
  // row-blocks per wave (34 % of the dense f16 peak on gate/up at 512 rows), four only with thousands of tiles
  // (2048-row chunks of the wide projections), one with fewer than 512 tiles of two (the 3072-wide o and down
  // projections at 512 rows: 45 and 79 us against 46 and 83 us with two)
  const int gb = 4;
  const int rb = tiles_for(4, 4) >= 2048 ? 4 : tiles_for(2, 4) >= 512 ? 2 : 1;
  if (const char* env = std::getenv("XTG_GEMM_SHAPE")) {
    int r = 0, g = 0;
    if (std::sscanf(env, "%d,%d", &r, &g) == 2 && gemm_fn(r, g) != nullptr)
      return run_gemm(c, r, g, stream);
  }
  return run_gemm(c, rb, gb, stream);
}

static std::string run_gemm(const GemvCall& c, int rb, int gb, hipStream_t stream) {
  const int kt = c.w[0]->kt;
  const int groups = (c.m + kMaxRows - 1) / kMaxRows;
  const int mtiles = (groups + gb - 1) / gb;
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
  const GemmFn fn = gemm_fn(rb, gb);
  XTG_CHECK(fn != nullptr, "gemm: no kernel for RB=%d GB=%d", rb, gb);
  hipLaunchKernelGGL(fn, grid, block, 0, stream, a);
  HIP_CHECK(hipGetLastError());
  return strf("gemm_kernel<%d, %d>", rb, gb);
}

}  // namespace xtg::hip
