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
//    Each k-tile (128 inputs) the work-group copies the groups' operand tile (4 KiB each) into LDS with direct
//    global-to-LDS loads, double-buffered, in lane order (no bank conflicts on the 16-byte reads, no staging
//    registers); each wave dequantises its RB weight tiles once and runs them against all GB groups: 4 RB GB
//    matrix ops per k-tile per wave. The next k-tile's loads are issued before the current one's math, one
//    barrier per k-tile.
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

// 16 bytes per lane from global memory straight into LDS: lane L writes lds_block + 16 L (wave-uniform block).
__device__ inline void copy_to_lds16(const uint4* src, uint4* lds_block) {
  __builtin_amdgcn_global_load_lds(src, lds_block, 16, 0, 0);
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

  // a k-tile's activation operand into LDS buffer buf, straight from global memory (global_load_lds_dwordx4:
  // lane L of a wave writes 16 bytes at the block's base + 16 L). Wave w moves step w of every group; lane L
  // fetches the entry 4 (L & 15) + (L >> 4) that lane L reads back as its B operand. Absent groups (past the
  // last row) are skipped: their stale columns produce outputs that are never stored.
  auto xload = [&](int kt, int buf) {
    const int e = 4 * (lane & 15) + (lane >> 4);
#pragma unroll
    for (int i = 0; i < kTileGroups; ++i)
      if (g0 + i < a.groups) {
        const uint4* src = reinterpret_cast<const uint4*>(a.op + size_t(g0 + i) * a.op_stride) +
                           (size_t(kt) * 4 + size_t(wave)) * 64 + size_t(e);
        copy_to_lds16(src, &xs[buf][i][wave][0]);
      }
  };
  auto wload = [&](int kt, u32x4 (&cw)[RB], uint32_t (&sw)[RB]) {
#pragma unroll
    for (int r = 0; r < RB; ++r) {
      if (rb0 + r < nb) {
        const uint8_t* tile = tiles + (size_t(rb0 + r) * size_t(KT) + size_t(kt)) * kTileBytes;
        cw[r] = *reinterpret_cast<const u32x4*>(tile + 16 * lane);
        sw[r] = uint32_t(*reinterpret_cast<const uint16_t*>(tile + 1024 + 2 * lane));
      } else {
        cw[r] = u32x4{0u, 0u, 0u, 0u};
        sw[r] = 0u;
      }
    }
  };

  f32x4 acc[RB][kTileGroups];
#pragma unroll
  for (int r = 0; r < RB; ++r)
#pragma unroll
    for (int g = 0; g < kTileGroups; ++g) acc[r][g] = f32x4{0.f, 0.f, 0.f, 0.f};

  u32x4 cw[RB];
  uint32_t sw[RB];
  xload(0, 0);
  wload(0, cw, sw);
  for (int kt = 0; kt < KT; ++kt) {
    // this wave's loads of k-tile kt have landed (its LDS copies included); after the barrier every wave's have,
    // and every wave is done reading the other buffer
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
    const int cur = kt & 1;
    const bool more = kt + 1 < KT;
    u32x4 cwn[RB];
    uint32_t swn[RB];
    if (more) {
      xload(kt + 1, cur ^ 1);
      wload(kt + 1, cwn, swn);
    }
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      f16x8 A[RB];
#pragma unroll
      for (int r = 0; r < RB; ++r) A[r] = dequant8(cw[r][s], scale_pair(sw[r], s >> 1));
#pragma unroll
      for (int g = 0; g < kTileGroups; ++g) {
        const f16x8 B = __builtin_bit_cast(f16x8, xs[cur][g][s][lane]);
#pragma unroll
        for (int r = 0; r < RB; ++r) acc[r][g] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A[r], B, acc[r][g], 0, 0, 0);
      }
    }
    if (more) {
#pragma unroll
      for (int r = 0; r < RB; ++r) {
        cw[r] = cwn[r];
        sw[r] = swn[r];
      }
    }
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
  XTG_GEMM(4, 8, 1) XTG_GEMM(2, 8, 2) XTG_GEMM(1, 8, 2) XTG_GEMM(4, 4, 2) XTG_GEMM(2, 4, 2) XTG_GEMM(1, 4, 2)
#undef XTG_GEMM
  return nullptr;
}

std::string launch_gemm(const GemvCall& c, hipStream_t stream) {
  XTG_CHECK(c.nw >= 1 && c.nw <= 4, "gemm: %d weights (1..4)", c.nw);
  XTG_CHECK(c.m >= 1, "gemm: %d rows", c.m);
  const int kt = c.w[0]->kt;
  const int groups = (c.m + kMaxRows - 1) / kMaxRows;
  // launch shape (XTG_GEMM_SHAPE=RB,GB fixes it, for experiments): four row-blocks per wave and eight groups per
  // tile when that still gives a work-group per CU, else smaller tiles
  int rb = 4, gb = 8;
  auto tiles_for = [&](int r, int g) {
    const int mt = (groups + g - 1) / g;
    long t = 0;
    for (int i = 0; i < c.nw; ++i) t += long((c.w[i]->nb + kGemmWaves * r - 1) / (kGemmWaves * r)) * mt;
    return t;
  };
  if (tiles_for(4, 8) < 256) {
    rb = 2;
    if (tiles_for(2, 8) < 256) gb = 4;
  }
  if (const char* env = std::getenv("XTG_GEMM_SHAPE")) {
    int r = 0, g = 0;
    if (std::sscanf(env, "%d,%d", &r, &g) == 2 && (r == 1 || r == 2 || r == 4) && (g == 4 || g == 8)) rb = r, gb = g;
  }
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
